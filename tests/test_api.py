"""The drop-in API surface on the CPU (construction only; nothing here launches a kernel):
compile / WideBuilder argument handling and error texts (reference api.py:36-237), the
registry honoured by TracedWideModel (registry.py:36-157, traced_wide.py:384-387), and the
epilogue-fusion bookkeeping of TracedWideModel."""

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import wide_compiler as wc
from wide_compiler.core.traced_wide import BinaryOp, TracedWideModel


class _MLP(nn.Module):
    def __init__(self):
        super().__init__()
        self.fc1 = nn.Linear(8, 16)
        self.fc2 = nn.Linear(16, 4)

    def forward(self, x):
        return self.fc2(F.relu(self.fc1(x)))


def test_compile_single_model_needs_n():
    with pytest.raises(ValueError, match="n required when passing single model"):
        wc.compile(_MLP(), torch.randn(2, 8))


def test_compile_empty_list_and_missing_sample():
    with pytest.raises(ValueError, match="models list is empty"):
        wc.compile([], torch.randn(2, 8))
    with pytest.raises(ValueError, match="sample_input required for FX tracing"):
        wc.compile([_MLP(), _MLP()])


def test_compile_single_model_with_n_makes_reinitialised_copies():
    torch.manual_seed(0)
    base = _MLP()
    wide = wc.compile(base, torch.randn(2, 8), n=3)
    assert isinstance(wide, TracedWideModel) and wide.n == 3
    fc1 = wide.stages["fc1"]
    # copies are re-initialised (reference _clone_model, api.py:244-252): no two models alike
    assert not torch.equal(fc1.weight[0], fc1.weight[1])
    assert not any(torch.equal(fc1.weight[i], base.fc1.weight) for i in range(3))


def test_compile_list_keeps_each_models_weights():
    models = [_MLP() for _ in range(4)]
    wide = wc.compile(models, torch.randn(2, 8))
    fc2 = wide.stages["fc2"]
    for i, m in enumerate(models):
        assert torch.equal(fc2.weight[i], m.fc2.weight)
        assert torch.equal(fc2.bias[i], m.fc2.bias)


def test_builder_chain():
    models = [_MLP() for _ in range(3)]
    built = (wc.WideBuilder(models).with_sample(torch.randn(2, 8)).with_config(wc.WideConfig.default())
             .validate(False).debug(False).build())
    assert isinstance(built, TracedWideModel) and built.n == 3
    with pytest.raises(ValueError, match="n required when passing single model"):
        wc.WideBuilder(_MLP())
    assert wc.WideBuilder(_MLP(), n=5)._models.__len__() == 5
    with pytest.raises(ValueError, match="sample_input required"):
        wc.WideBuilder(models).build()
    b = wc.WideBuilder(models).compile("default")
    assert b._config.compile is True and b._config.compile_mode == "default"


class _Scale(nn.Module):
    def __init__(self):
        super().__init__()
        self.s = nn.Parameter(torch.randn(4))

    def forward(self, x):
        return x * self.s


class _WideScale(nn.Module):
    """A user primitive: N _Scale modules as one [N, 4] parameter."""

    def __init__(self, n):
        super().__init__()
        self.n = n
        self.s = nn.Parameter(torch.zeros(n, 4))

    @classmethod
    def from_modules(cls, modules):
        w = cls(len(modules))
        with torch.no_grad():
            for i, m in enumerate(modules):
                w.s[i].copy_(m.s)
        return w

    def forward(self, x):            # x [N, B, 4]
        return x * self.s[:, None, :]


class _WithScale(nn.Module):
    def __init__(self):
        super().__init__()
        self.fc = nn.Linear(8, 4)
        self.scale = _Scale()

    def forward(self, x):
        return self.scale(self.fc(x))


def test_registered_primitive_is_used_by_compile():
    models = [_WithScale() for _ in range(3)]
    # unregistered: fx traces through the user module, as in the reference (traced_wide.py:306)
    wide = wc.compile(models, torch.randn(2, 8))
    assert "scale" not in wide.stages and any(isinstance(op, BinaryOp) for op in wide.stages.values())
    try:
        wc.register("_Scale", _WideScale)
        assert "_Scale" in wc.list_registered()
        wide = wc.compile(models, torch.randn(2, 8))
        op = wide.stages["scale"]
        assert isinstance(op, _WideScale)
        for i, m in enumerate(models):
            assert torch.equal(op.s[i], m.scale.s)
        # the builder's register() is the same registry
        wide2 = wc.WideBuilder(models).register("_Scale", _WideScale).with_sample(torch.randn(2, 8)).build()
        assert isinstance(wide2.stages["scale"], _WideScale)
    finally:
        wc.unregister("_Scale")
    assert "_Scale" not in wc.list_registered()


def test_register_requires_from_modules():
    class NoBuilder(nn.Module):
        pass
    with pytest.raises(TypeError, match="must implement classmethod from_modules"):
        wc.register("NoBuilder", NoBuilder)


class _LateAliasResidual(nn.Module):
    """The residual operand's ReLU (folded into c1) comes after c2 in fx order."""

    def __init__(self):
        super().__init__()
        self.c1 = nn.Conv2d(4, 4, 3, padding=1)
        self.c2 = nn.Conv2d(4, 4, 3, padding=1)

    def forward(self, x):
        a = self.c1(x)
        h = self.c2(x)
        return h + torch.relu(a)


def test_residual_is_read_from_the_stage_that_computes_it():
    models = [_LateAliasResidual() for _ in range(2)]
    wide = wc.compile(models, torch.randn(1, 4, 5, 5))
    order = {name: i for i, name in enumerate(wide._execution_order)}
    assert wide._residual_of, "the add should fold into c2's epilogue"
    for conv, res in wide._residual_of.items():
        # the residual's value exists when the conv runs: a real stage, computed before it
        assert res not in wide._aliases
        assert order[res] < order[conv]
    assert wide._residual_of == {"c2": "c1"}
    assert wide.stages["c1"].fused_activation == "relu"


def test_self_attention_fusion_rules():
    """WideAttention routes self-attention to the fused projection kernel only where it applies:
    bf16, head dim 32, 1 <= S <= 512, D <= 768, no mask, 16-byte aligned rows (host logic only)."""
    import torch
    import wide_compiler as wc
    w = wc.WideAttention(2, 64, 2).to(torch.bfloat16)
    params = (w.q_weight, w.kv_weight, w.out_weight, w.q_bias, w.kv_bias, w.out_bias)
    x = torch.zeros(2, 3, 40, 64, dtype=torch.bfloat16)
    assert w._fusable(x, None, params)
    assert not w._fusable(x, torch.zeros(40, 40, dtype=torch.bool), params)
    assert not w._fusable(x.float(), None, params)
    assert not w._fusable(torch.zeros(2, 3, 513, 64, dtype=torch.bfloat16), None, params)
    assert not w._fusable(torch.zeros(2, 3, 0, 64, dtype=torch.bfloat16), None, params)
    assert not w._fusable(torch.zeros(2, 3, 40, 66, dtype=torch.bfloat16)[..., :64], None, params)
    assert w._fusable(torch.zeros(2, 3, 40, 72, dtype=torch.bfloat16)[..., 8:], None, params)
    w.fuse_projections = False
    assert not w._fusable(x, None, params)
    w64 = wc.WideAttention(2, 128, 2).to(torch.bfloat16)          # head dim 64
    assert not w64._fusable(torch.zeros(2, 3, 40, 128, dtype=torch.bfloat16), None,
                            (w64.q_weight, w64.kv_weight, w64.out_weight, w64.q_bias, w64.kv_bias, w64.out_bias))


def test_torch_compile_sees_the_traced_forward_as_one_operator():
    """Under torch.compile the traced forward is one node, torch.ops.wide_compiler.module_call,
    whose fake implementation gives the packed output shape (from a meta-device copy of model
    0) without launching anything; a copy of the model gets a handle of its own."""
    import copy
    from torch._subclasses.fake_tensor import FakeTensorMode
    torch.manual_seed(1)
    wide = TracedWideModel.from_models([_MLP() for _ in range(5)], torch.randn(4, 8))
    h = wide.__dict__["_op_handle"]
    with FakeTensorMode():
        y = torch.ops.wide_compiler.module_call(h, [torch.empty(7, 40)])
    assert tuple(y[0].shape) == (7, 20) and y[0].dtype == torch.float32
    assert copy.deepcopy(wide).__dict__["_op_handle"] != h
    graphs = []

    class _Captured(Exception):
        pass

    def backend(gm, example_inputs):
        graphs.append(gm)

        def run(*args):
            raise _Captured

        return run

    with pytest.raises(_Captured):
        torch.compile(wide, backend=backend)(torch.randn(7, 40))
    ops = [nd.target for nd in graphs[0].graph.nodes if nd.op == "call_function"]
    assert torch.ops.wide_compiler.module_call.default in ops or torch.ops.wide_compiler.module_call in ops
    assert len([o for o in ops if "module_call" in str(o)]) == 1
