"""GPU checks of the drop-in API behaviour: compile_model=True (torch.compile around the wide
model, reference api.py:138-147) in both modes, graph replay of a traced model
(TracedWideModel.use_graphs), parameter writes through ``.data`` seen by
the next forward (the reference reads its parameters on every call), a residual whose ReLU
alias follows the conv it feeds, and WideBatchNorm1d (wide_batchnorm_1d.py:53-73) alone and
folded into a traced Conv1d epilogue."""

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import wide_ref
from tests._util import TOL_F32, gen, rel_err, tol

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _MLP(nn.Module):
    def __init__(self):
        super().__init__()
        self.fc1 = nn.Linear(16, 32)
        self.fc2 = nn.Linear(32, 8)

    def forward(self, x):
        return self.fc2(F.relu(self.fc1(x)))


@pytest.mark.parametrize("mode", ["default", "reduce-overhead"])
def test_compile_model_true_matches_eager(hip, mode):
    import wide_compiler as wc
    torch.manual_seed(300)
    models = [_MLP().to(DEV) for _ in range(5)]
    sample = torch.randn(4, 16, device=DEV)
    eager = wc.compile(models, sample)
    compiled = wc.compile(models, sample, compile_model=True, compile_mode=mode)
    g = gen(301)
    import warnings
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        for _ in range(4):                              # successive calls with new inputs
            x = torch.randn(4, 5 * 16, generator=g).to(DEV)
            with torch.no_grad():
                ref = eager(x).clone()
                got = compiled(x).clone()
            torch.cuda.synchronize()
            assert rel_err(got, ref) <= TOL_F32
    # the forward is one operator in the compiled graph (wide_compiler::module_call), so
    # reduce-overhead mode captures its kernel launches: no empty CUDA graph
    assert not [w for w in caught if "Graph is empty" in str(w.message)], [str(w.message) for w in caught]


def test_builder_compile_chain_runs(hip):
    import wide_compiler as wc
    torch.manual_seed(302)
    models = [_MLP().to(DEV) for _ in range(3)]
    sample = torch.randn(2, 16, device=DEV)
    built = wc.WideBuilder(models).with_sample(sample).validate().compile("default").build()
    x = torch.randn(2, 3 * 16, device=DEV)
    with torch.no_grad():
        y = built(x)
        outs = wc.unpack(y, 3)
        for k in range(3):
            assert rel_err(outs[k], models[k](x[:, 16 * k:16 * (k + 1)])) <= TOL_F32


def test_conv_sees_weight_writes_through_data(hip):
    import wide_compiler as wc
    torch.manual_seed(303)
    convs = [nn.Conv2d(8, 8, 3, padding=1) for _ in range(4)]
    wide = wc.WideConv2d.from_modules(convs).to(DEV)
    x = torch.randn(4, 2, 8, 6, 6, generator=gen(304)).to(DEV)
    with torch.no_grad():
        wide(x)
        wide.grouped_conv.weight.data.mul_(0.5)         # EMA-style write: no version bump
        wide.grouped_conv.bias.data.add_(1.0)
        y = wide(x).cpu()
    w = wide.grouped_conv.weight.detach().cpu().double()
    b = wide.grouped_conv.bias.detach().cpu().double()
    exact = wide_ref.conv2d(x.cpu().double(), w, b, 4, (1, 1), (1, 1), (1, 1))
    assert rel_err(y, exact) <= TOL_F32


def test_attention_sees_weight_writes_through_data(hip):
    import wide_compiler as wc
    torch.manual_seed(305)
    mods = [nn.MultiheadAttention(64, 4, batch_first=True) for _ in range(2)]
    wide = wc.WideAttention.from_modules(mods).to(DEV).eval()
    x = torch.randn(2, 2, 10, 64, generator=gen(306)).to(DEV)
    with torch.no_grad():
        wide(x)
        wide.q_weight.data.mul_(-1.0)
        wide.kv_weight.data[:, :16].zero_()
        y = wide(x).cpu()
    p = [getattr(wide, a).detach().cpu().double() for a in
         ("q_weight", "kv_weight", "out_weight", "q_bias", "kv_bias", "out_bias")]
    xs = x.cpu().double()
    exact = wide_ref.attention(xs, xs, xs, *p, 4)
    assert rel_err(y, exact) <= TOL_F32


class _LateAliasResidual(nn.Module):
    def __init__(self):
        super().__init__()
        self.c1 = nn.Conv2d(8, 8, 3, padding=1)
        self.c2 = nn.Conv2d(8, 8, 3, padding=1)

    def forward(self, x):
        a = self.c1(x)
        h = self.c2(x)
        return h + torch.relu(a)


def test_residual_whose_relu_follows_the_conv(hip):
    import wide_compiler as wc
    torch.manual_seed(307)
    models = [_LateAliasResidual().to(DEV) for _ in range(3)]
    ins = [torch.randn(2, 8, 6, 6, generator=gen(308 + i)).to(DEV) for i in range(3)]
    wide = wc.compile(models, ins[0])
    assert wide._residual_of == {"c2": "c1"}
    with torch.no_grad():
        outs = wc.unpack(wide(wc.pack(ins)), 3)
        for k in range(3):
            assert rel_err(outs[k], models[k](ins[k])) <= TOL_F32


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(5, 3, 12), (4, 2, 12, 9)])
def test_batchnorm1d_eval(hip, dtype, shape):
    import wide_compiler as wc
    torch.manual_seed(309)
    c = shape[2]
    mods = []
    for _ in range(shape[0]):
        m = nn.BatchNorm1d(c).eval()
        with torch.no_grad():
            m.weight.normal_(1.0, 0.2)
            m.bias.normal_(0.0, 0.2)
            m.running_mean.normal_(0.0, 0.5)
            m.running_var.uniform_(0.5, 2.0)
        mods.append(m.to(dtype))
    wide = wc.WideBatchNorm1d.from_modules(mods).to(DEV).eval()
    x = torch.randn(*shape, generator=gen(310)).to(dtype)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
        for k in range(shape[0]):
            ref = mods[k].float()(x[k].float()).double()
            assert rel_err(y[k], ref) <= tol(dtype)


class _ConvBN1d(nn.Module):
    def __init__(self):
        super().__init__()
        self.conv = nn.Conv1d(8, 16, 3, padding=1)
        self.bn = nn.BatchNorm1d(16)

    def forward(self, x):
        return F.relu(self.bn(self.conv(x)))


def test_traced_conv1d_bn1d_relu_folds_and_matches(hip):
    import wide_compiler as wc
    torch.manual_seed(311)
    models = []
    for _ in range(4):
        m = _ConvBN1d()
        with torch.no_grad():
            m.bn.weight.normal_(1.0, 0.2)
            m.bn.bias.normal_(0.0, 0.2)
            m.bn.running_mean.normal_(0.0, 0.3)
            m.bn.running_var.uniform_(0.5, 2.0)
        models.append(m.eval().to(DEV))
    ins = [torch.randn(3, 8, 20, generator=gen(312 + i)).to(DEV) for i in range(4)]
    wide = wc.compile(models, ins[0]).eval()
    s = wide.summary()
    assert s.count("fused into") == 2, s               # bn and relu -> the conv epilogue
    with torch.no_grad():
        outs = wc.unpack(wide(wc.pack(ins)), 4)
        for k in range(4):
            assert rel_err(outs[k], models[k](ins[k])) <= TOL_F32


class _Block(nn.Module):
    """conv3x3-BN-ReLU-conv3x3-BN + identity, ReLU (the ResBlock shape of the conv tests)."""

    def __init__(self, c):
        super().__init__()
        self.conv1 = nn.Conv2d(c, c, 3, padding=1)
        self.bn1 = nn.BatchNorm2d(c)
        self.conv2 = nn.Conv2d(c, c, 3, padding=1)
        self.bn2 = nn.BatchNorm2d(c)

    def forward(self, x):
        out = F.relu(self.bn1(self.conv1(x)))
        return F.relu(self.bn2(self.conv2(out)) + x)


def _graph_models(kind):
    torch.manual_seed(310)
    if kind == "mlp":
        return [_MLP().to(DEV) for _ in range(6)], (4, 16), torch.float32
    mods = []
    for _ in range(3):
        m = _Block(32)
        with torch.no_grad():
            for bn in (m.bn1, m.bn2):
                bn.weight.normal_(1.0, 0.1)
                bn.bias.normal_(0.0, 0.1)
        mods.append(m.to(DEV, torch.bfloat16).eval())
    return mods, (2, 32, 16, 16), torch.bfloat16


@pytest.mark.parametrize("kind", ["mlp", "resblock"])
def test_traced_graph_replay_matches_eager(hip, kind):
    """use_graphs(): the second forward of one input buffer captures, later ones replay, with the
    program's own eager work between replays; every call equals the eager forward bit for bit.
    A second buffer layout gets its own graph, replays reuse one output buffer (documented), and
    inputs at fresh addresses run directly (no capture, no copy)."""
    import wide_compiler as wc
    models, shape, dtype = _graph_models(kind)
    n = len(models)
    sample = torch.randn(*shape, device=DEV).to(dtype)
    eager = wc.compile(models, sample).eval()
    graphed = wc.compile(models, sample).eval().use_graphs()
    graphs = graphed.__dict__["_graphs"]
    g = gen(311)
    packed_shape = (shape[0], n * shape[1], *shape[2:])
    xbuf = torch.empty(packed_shape, device=DEV, dtype=dtype)
    outs = []
    with torch.no_grad():
        for i in range(5):
            xbuf.copy_(torch.randn(*packed_shape, generator=g).to(DEV, dtype))
            ref = eager(xbuf).clone()
            got = graphed(xbuf)
            outs.append(got)
            assert torch.equal(got, ref), (kind, i)
            assert len(graphs) == (0 if i == 0 else 1)
            torch.cuda.synchronize()
            (xbuf * 2).sum().item()                     # eager work between replays
        assert all(o.data_ptr() == outs[1].data_ptr() for o in outs[1:])
        x2 = torch.empty((2 * shape[0], *packed_shape[1:]), device=DEV, dtype=dtype)
        for _ in range(3):
            x2.copy_(torch.randn(*x2.shape, generator=g).to(DEV, dtype))
            assert torch.equal(graphed(x2), eager(x2))
        assert len(graphs) == 2
        for _ in range(3):                              # fresh tensors: direct launches only
            x = torch.randn(*packed_shape, generator=g).to(DEV, dtype)
            assert torch.equal(graphed(x), eager(x))
        assert len(graphs) == 2
        xbuf.copy_(torch.randn(*packed_shape, generator=g).to(DEV, dtype))
        assert torch.equal(graphed(xbuf), eager(xbuf))  # the first buffer's graph again
    graphed.use_graphs(False)
    with torch.no_grad():
        assert torch.equal(graphed(xbuf), eager(xbuf))
