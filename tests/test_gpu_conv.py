"""GPU parity of the implicit-GEMM grouped convolution and the traced ResBlock against the oracle."""

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import wide_ref
from tests._util import TOL_BF16, TOL_F32, gen, rel_err, tol

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16]


def _rand(shape, g, dtype=torch.float32):
    return torch.randn(shape, generator=g).to(dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,b,ci,co,hw,k,stride,pad,dil", [
    (4, 2, 64, 64, (32, 32), 3, 1, 1, 1),
    (3, 2, 3, 16, (17, 13), 3, 1, 1, 1),
    (2, 1, 40, 72, (9, 11), 3, 2, 1, 1),
    (2, 3, 8, 8, (12, 12), 5, 1, 2, 2),
    (5, 1, 16, 130, (6, 7), 1, 1, 0, 1),
    (2, 2, 96, 24, (5, 70), (3, 1), (1, 2), (1, 0), 1),
])
def test_conv2d(hip, dtype, n, b, ci, co, hw, k, stride, pad, dil):
    import wide_compiler as wc
    g = gen(200)
    torch.manual_seed(200)
    mods = [nn.Conv2d(ci, co, k, stride=stride, padding=pad, dilation=dil) for _ in range(n)]
    wide = wc.WideConv2d.from_modules(mods).to(DEV, dtype)
    x = _rand((n, b, ci, *hw), g, dtype)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    cw = wide.grouped_conv.weight.detach().cpu()
    cb = wide.grouped_conv.bias.detach().cpu()
    exact = wide_ref.conv2d(x.double(), cw.double(), cb.double(), n, stride=wide.stride, padding=wide.padding,
                            dilation=wide.dilation)
    assert y.shape == exact.shape
    assert rel_err(y, exact) <= tol(dtype)
    if dtype == torch.bfloat16:
        assert rel_err(y, wide_ref.conv2d(x, cw, cb, n, stride=wide.stride, padding=wide.padding,
                                          dilation=wide.dilation)) <= TOL_BF16


TOL_F16 = 2e-3   # fp16 output rounding (2^-11 relative) over fp32 accumulation


@pytest.mark.parametrize("n,b,ci,co,hw,k,stride,pad,dil", [
    (4, 2, 64, 64, (32, 32), 3, 1, 1, 1),
    (2, 1, 40, 72, (9, 11), 3, 2, 1, 1),
    (2, 3, 8, 8, (12, 12), 5, 1, 2, 2),
    (5, 1, 16, 130, (6, 7), 1, 1, 0, 1),
])
def test_conv2d_fp16(hip, n, b, ci, co, hw, k, stride, pad, dil):
    """fp16 models: packed-weight implicit GEMM on the fp16 MFMA (v_mfma_f32_16x16x32_f16)."""
    import wide_compiler as wc
    g = gen(205)
    torch.manual_seed(205)
    mods = [nn.Conv2d(ci, co, k, stride=stride, padding=pad, dilation=dil) for _ in range(n)]
    wide = wc.WideConv2d.from_modules(mods).to(DEV, torch.float16)
    x = _rand((n, b, ci, *hw), g, torch.float16)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    cw = wide.grouped_conv.weight.detach().cpu()
    cb = wide.grouped_conv.bias.detach().cpu()
    exact = wide_ref.conv2d(x.double(), cw.double(), cb.double(), n, stride=wide.stride, padding=wide.padding,
                            dilation=wide.dilation)
    assert y.dtype == torch.float16
    assert rel_err(y, exact) <= TOL_F16


def test_conv2d_weight_update_invalidates_packing(hip):
    import wide_compiler as wc
    g = gen(201)
    wide = wc.WideConv2d(3, 8, 8, 3, padding=1).to(DEV)
    x = _rand((3, 2, 8, 6, 6), g).to(DEV)
    with torch.no_grad():
        wide(x)
        wide.grouped_conv.weight.mul_(2.0)
        y = wide(x).cpu()
    exact = wide_ref.conv2d(x.cpu().double(), wide.grouped_conv.weight.detach().cpu().double(),
                            wide.grouped_conv.bias.detach().cpu().double(), 3, padding=(1, 1))
    assert rel_err(y, exact) <= TOL_F32


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [4, 12])     # SEQUENTIAL / GROUPED state layouts
@pytest.mark.parametrize("stride,pad,dil", [(1, 1, 1), (2, 1, 2)])
def test_conv1d(hip, dtype, n, stride, pad, dil):
    import wide_compiler as wc
    g = gen(202)
    torch.manual_seed(202)
    mods = [nn.Conv1d(64, 48, 3, stride=stride, padding=pad, dilation=dil) for _ in range(n)]
    wide = wc.WideConv1d.from_modules(mods).to(DEV, dtype)
    x = _rand((n, 8, 64, 256), g, dtype)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    w, bias = wide._filters()
    w = w.detach().cpu().reshape(n * 48, 64, 3)
    exact = wide_ref.conv1d(x.double(), w.double(), bias.detach().cpu().double(), n, stride=stride, padding=pad,
                            dilation=dil)
    assert rel_err(y, exact) <= tol(dtype)


def _bn_modules(n, c, seed):
    torch.manual_seed(seed)
    mods = [nn.BatchNorm2d(c).eval() for _ in range(n)]
    for m in mods:
        with torch.no_grad():
            m.running_mean.normal_(0, 0.2)
            m.running_var.uniform_(0.5, 2.0)
            m.weight.normal_(1.0, 0.1)
            m.bias.normal_(0.0, 0.1)
    return mods


@pytest.mark.parametrize("dtype", DTYPES)
def test_conv_fused_bn_residual_relu(hip, dtype):
    import wide_compiler as wc
    g = gen(203)
    n, b, c = 3, 2, 32
    torch.manual_seed(203)
    conv = wc.WideConv2d.from_modules([nn.Conv2d(c, c, 3, padding=1) for _ in range(n)]).to(DEV, dtype)
    bn = wc.WideBatchNorm2d.from_modules(_bn_modules(n, c, 204)).to(DEV, dtype).eval()
    conv.fused_bn = bn
    conv.fused_activation = "relu"
    x = _rand((n, b, c, 10, 12), g, dtype)
    r = _rand((n, b, c, 10, 12), g, dtype)
    with torch.no_grad():
        y = conv(x.to(DEV), residual=r.to(DEV)).cpu()
    op = bn.op
    d = lambda t: t.detach().cpu().double()  # noqa: E731
    ref = wide_ref.conv2d(x.double(), d(conv.grouped_conv.weight), d(conv.grouped_conv.bias), n, padding=(1, 1))
    ref = wide_ref.batchnorm_eval(ref, d(op.weight), d(op.bias), d(op.running_mean), d(op.running_var), op.eps, n)
    ref = F.relu(ref + r.double())
    assert rel_err(y, ref) <= tol(dtype)


@pytest.mark.parametrize("n,b,ci,co,h,w,fused", [
    (3, 2, 64, 64, 32, 32, False),     # one 64-channel tile, 8-row blocks
    (5, 3, 64, 128, 20, 32, True),     # two channel tiles, partial last row block
    (7, 2, 32, 64, 9, 64, True),       # C_in 32, 4-row blocks
    (100, 3, 64, 64, 16, 16, True),    # more items than workgroups, model changes inside a range
    (2, 1, 32, 64, 32, 32, False),
])
def test_conv2d_resident_weights(hip, n, b, ci, co, h, w, fused):
    """bf16 "same" 3x3 convolutions on the resident-weight kernel, with and without the fused
    BN + residual + ReLU epilogue."""
    import wide_compiler as wc
    g = gen(207)
    torch.manual_seed(207)
    dtype = torch.bfloat16
    conv = wc.WideConv2d.from_modules([nn.Conv2d(ci, co, 3, padding=1) for _ in range(n)]).to(DEV, dtype)
    x = _rand((n, b, ci, h, w), g, dtype)
    d = lambda t: t.detach().cpu().double()  # noqa: E731
    ref = wide_ref.conv2d(x.double(), d(conv.grouped_conv.weight), d(conv.grouped_conv.bias), n, padding=(1, 1))
    kw = {}
    if fused:
        bn = wc.WideBatchNorm2d.from_modules(_bn_modules(n, co, 208)).to(DEV, dtype).eval()
        conv.fused_bn = bn
        conv.fused_activation = "relu"
        r = _rand((n, b, co, h, w), g, dtype)
        kw["residual"] = r.to(DEV)
        op = bn.op
        ref = wide_ref.batchnorm_eval(ref, d(op.weight), d(op.bias), d(op.running_mean), d(op.running_var), op.eps,
                                      n)
        ref = F.relu(ref + r.double())
    with torch.no_grad():
        y = conv(x.to(DEV), **kw).cpu()
    assert rel_err(y, ref) <= TOL_BF16


@pytest.mark.parametrize("kh,n,b,ci,w,h", [
    (3, 40, 4, 64, 32, 32),            # 640 items over 256 workgroups: 2-3 items each, model changes inside
    (3, 100, 6, 64, 16, 16),
    (3, 40, 4, 32, 32, 32),            # C_in 32: fewer staging units than threads in a group
    (3, 30, 4, 32, 64, 20),            # partial last row block
    (1, 100, 8, 64, 256, 1),           # the 1x3 kernel (Conv1d over L = 256)
    (1, 100, 8, 32, 256, 1),
])
def test_resident_kernel_weight_layouts_agree(hip, monkeypatch, kh, n, b, ci, w, h):
    """The resident-weight kernel staging the module's filter bank directly (through a free
    input buffer, whose zero halo columns must survive) and staging the packed copy give
    bit-identical outputs matching the oracle, with several items per workgroup so that both
    groups of a workgroup stage inputs and weights are reloaded at model boundaries."""
    from wide_compiler import _hip
    g = gen(215)
    co = 64
    x = _rand((n, b, ci, h, w), g, torch.bfloat16).to(DEV)
    wt = (_rand((n * co, ci, kh, 3), g) * 0.1).to(torch.bfloat16).to(DEV)
    bias = _rand((n * co,), g).to(DEV)
    packs = []
    real_pack = _hip.conv_pack_weights
    monkeypatch.setattr(_hip, "conv_pack_weights", lambda *a: packs.append(1) or real_pack(*a))
    outs = []
    for packed in (False, True):
        y = torch.full((n, b, co, h, w), float("nan"), dtype=torch.bfloat16, device=DEV)
        _hip.conv2d(x=x, weight=wt, n=n, c_in=ci, c_out=co, kernel=(kh, 3), stride=(1, 1),
                    padding=(kh // 2, 1), dilation=(1, 1), y=y, bias=bias, relu=True, packed=packed)
        outs.append(y.cpu())
    assert len(packs) == 1                              # only the packed=True call packed
    assert torch.equal(outs[0], outs[1])
    ref = F.relu(wide_ref.conv2d(x.cpu().double(), wt.cpu().double(), bias.cpu().double(), n,
                                 padding=(kh // 2, 1)))
    assert rel_err(outs[0], ref) <= TOL_BF16


def test_resident_conv_repeatable_on_fresh_inputs(hip):
    """Regression: the resident-weight kernel's epilogue once exchanged 16-lane rows with a
    cross-lane swap instruction that now and then delivered a stale word (about one launch in
    ten right after new inputs and another instantiation, at pixels 0, 1, 8, 9 of a 16-pixel
    tile).  Fresh inputs, instantiations interleaved, three launches each: all bit-identical."""
    from wide_compiler import _hip
    g = torch.Generator(device=DEV).manual_seed(216)
    cfgs = [(40, 4, 64, 32, 32), (100, 6, 64, 16, 16), (40, 4, 32, 32, 32), (30, 4, 32, 64, 20)]
    for _ in range(12):
        for n, b, ci, w, h in cfgs:
            x = torch.randn((n, b, ci, h, w), device=DEV, generator=g).to(torch.bfloat16)
            wt = (torch.randn((n * 64, ci, 3, 3), device=DEV, generator=g) * 0.1).to(torch.bfloat16)
            bias = torch.randn((n * 64,), device=DEV, generator=g)
            outs = []
            for packed in (False, True, False):
                y = torch.full((n, b, 64, h, w), float("nan"), dtype=torch.bfloat16, device=DEV)
                _hip.conv2d(x=x, weight=wt, n=n, c_in=ci, c_out=64, kernel=(3, 3), stride=(1, 1), padding=(1, 1),
                            dilation=(1, 1), y=y, bias=bias, relu=True, packed=packed)
                outs.append(y)
            assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2]), (n, b, ci, w, h)


def test_conv1d_resident_weights(hip):
    """Conv1d(64 -> 128, k=3, pad 1) over L=256: the 1x3 resident-weight kernel."""
    import wide_compiler as wc
    g = gen(209)
    torch.manual_seed(209)
    n = 6
    mods = [nn.Conv1d(64, 128, 3, padding=1) for _ in range(n)]
    wide = wc.WideConv1d.from_modules(mods).to(DEV, torch.bfloat16)
    x = _rand((n, 4, 64, 256), g, torch.bfloat16)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    w, bias = wide._filters()
    w = w.detach().cpu().reshape(n * 128, 64, 3)
    exact = wide_ref.conv1d(x.double(), w.double(), bias.detach().cpu().double(), n, padding=1)
    assert rel_err(y, exact) <= TOL_BF16


class ResBlock(nn.Module):
    """cli.py:84-97."""

    def __init__(self, channels=64):
        super().__init__()
        self.conv1 = nn.Conv2d(channels, channels, 3, padding=1)
        self.bn1 = nn.BatchNorm2d(channels)
        self.conv2 = nn.Conv2d(channels, channels, 3, padding=1)
        self.bn2 = nn.BatchNorm2d(channels)

    def forward(self, x):
        identity = x
        out = F.relu(self.bn1(self.conv1(x)))
        out = self.bn2(self.conv2(out))
        return F.relu(out + identity)


def _resblocks(n, c, dtype, seed=300):
    mods = []
    for i in range(n):
        torch.manual_seed(seed + i)
        m = ResBlock(c)
        with torch.no_grad():
            for bnm in (m.bn1, m.bn2):
                bnm.weight.normal_(1.0, 0.1)
                bnm.bias.normal_(0.0, 0.1)
        mods.append(m.to(dtype).eval())
    return mods


def _params(mods):
    from tests.test_oracle import resblock_params
    return resblock_params(mods)


@pytest.mark.parametrize("dtype", DTYPES)
def test_traced_resblock_fuses_and_matches(hip, dtype):
    import wide_compiler as wc
    n, b, c, hw = 6, 2, 16, 8
    mods = _resblocks(n, c, dtype)
    g = gen(205)
    ins = [_rand((b, c, hw, hw), g, dtype) for _ in range(n)]
    wide = wc.compile([m.to(DEV) for m in mods], ins[0].to(DEV)).eval()
    s = wide.summary()
    assert s.count("fused into") == 5, s   # bn1, relu, bn2, add, relu -> conv1 / conv2 epilogues
    packed = wide_ref.pack_inputs(ins)
    with torch.no_grad():
        y = wide(packed.to(DEV)).cpu()
    p = {k: (v.double() if torch.is_tensor(v) else v) for k, v in _params([m.cpu() for m in mods]).items()}
    exact = wide_ref.resblock_wide(packed.double(), n, p)
    assert rel_err(y, exact) <= tol(dtype)
    with torch.no_grad():
        outs = wc.unpack(y, n)
        for k in (0, n - 1):
            assert rel_err(outs[k], mods[k](ins[k]).float()) <= tol(dtype)


def test_resblock_config_n100(hip):
    """The ResBlock configuration at full size: N=100, B=8, 64 channels, 32x32, bf16.  Every
    model against the fp32 oracle (one wide evaluation), three spread models against fp64."""
    import wide_compiler as wc
    n, b, c, hw = 100, 8, 64, 32
    mods = _resblocks(n, c, torch.bfloat16)
    g = gen(206)
    x = torch.randn(b, n * c, hw, hw, generator=g).to(torch.bfloat16)
    wide = wc.compile([m.to(DEV) for m in mods], x[:, :c].to(DEV)).eval()
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    assert y.shape == x.shape
    mods = [m.cpu() for m in mods]
    p32 = {kk: (v.float() if torch.is_tensor(v) else v) for kk, v in _params(mods).items()}
    exact32 = wide_ref.resblock_wide(x.float(), n, p32)
    errs = [rel_err(y[:, k * c:(k + 1) * c], exact32[:, k * c:(k + 1) * c]) for k in range(n)]
    assert max(errs) <= TOL_BF16, max(errs)
    for k in (0, 41, 99):
        pk = {kk: (v.double() if torch.is_tensor(v) else v) for kk, v in _params([mods[k]]).items()}
        exact = wide_ref.resblock_wide(x[:, k * c:(k + 1) * c].double(), 1, pk)
        assert rel_err(y[:, k * c:(k + 1) * c], exact) <= TOL_BF16


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,b,ci,co,dhw,k,stride,pad,dil", [
    (4, 2, 8, 16, (6, 10, 12), 3, 1, 1, 1),
    (3, 1, 3, 70, (5, 7, 9), (1, 3, 3), 1, (0, 1, 1), 1),       # 2 output-channel tiles, C_in < 32
    (2, 2, 40, 24, (7, 8, 6), (3, 1, 1), (2, 1, 1), (1, 0, 0), 1),
    (2, 1, 16, 8, (9, 9, 9), 3, 2, 2, 2),                       # depth taps past both ends skipped
    (2, 2, 32, 32, (4, 16, 16), (2, 3, 3), 1, (0, 1, 1), 1),
])
def test_conv3d(hip, dtype, n, b, ci, co, dhw, k, stride, pad, dil):
    import wide_compiler as wc
    torch.manual_seed(500)
    mods = [nn.Conv3d(ci, co, k, stride=stride, padding=pad, dilation=dil).to(dtype) for _ in range(n)]
    wide = wc.WideConv3d.from_modules([m.to(DEV) for m in mods])
    assert set(wide.state_dict()) == {"conv.weight", "conv.bias"}
    x = _rand((n, b, ci) + dhw, gen(501), dtype)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    w, bias = wide.conv.weight.detach().cpu(), wide.conv.bias.detach().cpu()
    c = wide.conv
    exact = wide_ref.conv3d(x.double(), w.double(), bias.double(), n, c.stride, c.padding, c.dilation)
    assert rel_err(y, exact) <= tol(dtype)
    if dtype == torch.bfloat16:    # the reference's own bf16 path (CPU)
        assert rel_err(y, wide_ref.conv3d(x, w, bias, n, c.stride, c.padding, c.dilation)) <= TOL_BF16


def test_conv3d_fp16(hip):
    import wide_compiler as wc
    g = gen(206)
    torch.manual_seed(206)
    n, b, ci, co = 3, 2, 8, 16
    mods = [nn.Conv3d(ci, co, 3, padding=1) for _ in range(n)]
    wide = wc.WideConv3d.from_modules(mods).to(DEV, torch.float16)
    x = _rand((n, b, ci, 6, 7, 8), g, torch.float16)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    ref = torch.stack([F.conv3d(x[i].double(), mods[i].weight.detach().to(torch.float16).double(),
                                mods[i].bias.detach().to(torch.float16).double(), padding=1) for i in range(n)])
    assert y.dtype == torch.float16
    assert rel_err(y, ref) <= TOL_F16


def test_conv3d_sequential_matches_grouped_and_relu(hip):
    import wide_compiler as wc
    torch.manual_seed(502)
    n, ci, co = 3, 6, 10
    mods = [nn.Conv3d(ci, co, 3, padding=1, bias=False).to(DEV) for _ in range(n)]
    grouped = wc.WideConv3d.from_modules(mods)
    seq = wc.WideConv3d.from_modules(mods, strategy="sequential")
    assert seq.strategy.value == "sequential" and len(seq.convs) == n
    x = torch.randn(n, 2, ci, 4, 5, 6, generator=gen(503)).to(DEV)
    with torch.no_grad():
        yg = grouped(x)
        assert torch.equal(yg, seq(x))
        grouped.fused_activation = "relu"
        assert torch.equal(grouped(x), F.relu(yg))
    for i in range(n):
        with torch.no_grad():
            assert rel_err(yg[i].cpu(), mods[i].cpu()(x[i].cpu())) <= TOL_F32
