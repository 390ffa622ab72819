"""
GPU parity of WideGroupNorm / WideInstanceNorm1d / WideInstanceNorm2d (wc_group_norm, and
wc_bn_eval for eval-mode running statistics) against the oracle in float64 on the same
(rounded) inputs: normwise relative error <= TOL_F32 = 1e-5 (fp32), TOL_BF16 = 2e-2 (bf16).
The shapes reach every kernel configuration: one wave per row with 1 / 2 / 4 vectors per lane,
four waves per row with up to 16 vectors per lane, the three-pass long-row kernel, rows whose
spatial size is not a multiple of the vector width (scalar path) and inputs with no spatial dims.
"""

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import wide_ref
from tests._util import TOL_BF16, gen, rel_err, tol

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16]


def _gn_modules(n, groups, c, affine, seed):
    g = gen(seed)
    mods = [nn.GroupNorm(groups, c, affine=affine) for _ in range(n)]
    if affine:
        with torch.no_grad():
            for m in mods:
                m.weight.copy_(torch.randn(c, generator=g) * 0.5 + 1)
                m.bias.copy_(torch.randn(c, generator=g) * 0.5)
    return mods


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,b,c,groups,spatial", [
    (32, 8, 64, 32, (32, 32)),     # 2048-element rows
    (3, 2, 6, 3, (5, 7)),          # spatial 35: scalar path
    (2, 3, 16, 4, (64, 64)),       # 16384-element rows: four waves x 16 (fp32) / 8 (bf16) vectors
    (2, 1, 8, 1, (96, 96)),        # 73728-element rows: three-pass kernel
    (4, 5, 12, 3, ()),             # no spatial dims
    (5, 4, 32, 8, (16,)),          # 1-d spatial, 64-element rows
])
def test_group_norm(hip, dtype, n, b, c, groups, spatial):
    import wide_compiler as wc
    mods = _gn_modules(n, groups, c, True, 300)
    wide = wc.WideGroupNorm.from_modules(mods).to(DEV, dtype)
    assert set(wide.state_dict()) == {"norm.weight", "norm.bias"}
    x = (torch.randn((n, b, c) + spatial, generator=gen(301)) * 2 + 0.7).to(dtype)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    w, bb = wide.norm.weight.detach().cpu(), wide.norm.bias.detach().cpu()
    exact = wide_ref.group_norm(x.double(), w.double(), bb.double(), groups, wide.eps)
    assert rel_err(y, exact) <= tol(dtype)
    if dtype == torch.bfloat16:  # the reference's own bf16 path
        assert rel_err(y, wide_ref.group_norm(x, w, bb, groups, wide.eps)) <= TOL_BF16
    if dtype == torch.float32:
        for i in (0, n - 1):
            assert rel_err(y[i], mods[i](x[i])) <= tol(dtype)


@pytest.mark.parametrize("relu", [False, True])
def test_group_norm_no_affine_sequential_relu(hip, relu):
    import wide_compiler as wc
    n, b, c, groups = 6, 3, 12, 4
    mods = _gn_modules(n, groups, c, False, 302)
    wide = wc.WideGroupNorm.from_modules(mods, strategy="sequential").to(DEV)
    assert wide.strategy.value == "sequential"
    wide.fused_activation = "relu" if relu else None
    x = torch.randn(n, b, c, 9, 4, generator=gen(303))
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    exact = wide_ref.group_norm(x.double(), None, None, groups, 1e-5)
    if relu:
        exact = F.relu(exact)
    assert rel_err(y, exact) <= tol(torch.float32)


def test_group_norm_sequential_affine_matches_fused(hip):
    import wide_compiler as wc
    n, c, groups = 4, 8, 2
    mods = _gn_modules(n, groups, c, True, 304)
    fused = wc.WideGroupNorm.from_modules(mods).to(DEV)
    seq = wc.WideGroupNorm.from_modules(mods, strategy="sequential").to(DEV)
    x = torch.randn(n, 3, c, 6, 6, generator=gen(305)).to(DEV)
    with torch.no_grad():
        assert torch.equal(fused(x), seq(x))


def _in_modules(cls, n, c, affine, track, seed):
    g = gen(seed)
    mods = [cls(c, affine=affine, track_running_stats=track) for _ in range(n)]
    with torch.no_grad():
        for m in mods:
            if affine:
                m.weight.copy_(torch.randn(c, generator=g) * 0.5 + 1)
                m.bias.copy_(torch.randn(c, generator=g) * 0.5)
            if track:
                m.running_mean.copy_(torch.randn(c, generator=g))
                m.running_var.copy_(torch.rand(c, generator=g) + 0.5)
    return mods


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kind,spatial", [("1d", (256,)), ("1d", (37,)), ("2d", (32, 32)), ("2d", (7, 9))])
@pytest.mark.parametrize("affine", [False, True])
def test_instance_norm(hip, dtype, kind, spatial, affine):
    import wide_compiler as wc
    cls, wcls = (nn.InstanceNorm1d, wc.WideInstanceNorm1d) if kind == "1d" else \
        (nn.InstanceNorm2d, wc.WideInstanceNorm2d)
    n, b, c = 8, 4, 16
    mods = _in_modules(cls, n, c, affine, False, 306)
    wide = wcls.from_modules(mods).to(DEV, dtype)
    x = (torch.randn((n, b, c) + spatial, generator=gen(307)) * 1.5 - 0.3).to(dtype)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    w = wide.norm.weight.detach().cpu().double() if affine else None
    bb = wide.norm.bias.detach().cpu().double() if affine else None
    exact = wide_ref.instance_norm(x.double(), w, bb, wide.eps)
    assert rel_err(y, exact) <= tol(dtype)


@pytest.mark.parametrize("kind", ["1d", "2d"])
def test_instance_norm_running_stats_eval(hip, kind):
    import wide_compiler as wc
    cls, wcls, spatial = (nn.InstanceNorm1d, wc.WideInstanceNorm1d, (20,)) if kind == "1d" else \
        (nn.InstanceNorm2d, wc.WideInstanceNorm2d, (6, 5))
    n, b, c = 5, 3, 8
    mods = _in_modules(cls, n, c, True, True, 308)
    # the sequential strategy carries each module's running statistics (load_state_dict)
    wide = wcls.from_modules(mods, strategy="sequential").to(DEV).eval()
    x = torch.randn((n, b, c) + spatial, generator=gen(309))
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    cat = lambda k: torch.cat([getattr(m, k).detach() for m in mods]).double()  # noqa: E731
    exact = wide_ref.instance_norm(x.double(), cat("weight"), cat("bias"), 1e-5, cat("running_mean"),
                                   cat("running_var"))
    assert rel_err(y, exact) <= tol(torch.float32)
    for i in (0, n - 1):
        assert rel_err(y[i], mods[i].eval()(x[i])) <= tol(torch.float32)
    with torch.no_grad(), pytest.raises(RuntimeError, match="eval"):
        wide.train()(x.to(DEV))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [1025, 2047, 4100, 8200, 20000, 65536])
def test_layernorm_long_rows(hip, dtype, d):
    """Rows longer than one wave holds in registers (one workgroup per row, three passes): the
    vector form when 16-byte loads apply, the scalar one otherwise (odd widths), and a strided
    view; against the per-model nn.LayerNorm in fp64 (wide_layernorm.py:41-67)."""
    import wide_compiler as wc
    n, b, t = 3, 2, 3
    torch.manual_seed(d)
    mods = [nn.LayerNorm(d) for _ in range(n)]
    for m in mods:
        nn.init.uniform_(m.weight, 0.5, 1.5)
        nn.init.uniform_(m.bias, -0.5, 0.5)
    wide = wc.WideLayerNorm.from_modules(mods).to(DEV, dtype)
    base = (torch.randn(n, b, t, d + 8, device=DEV) * 2 + 0.5).to(dtype)
    bar = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}[dtype]
    for x in (base[..., :d].contiguous(), base[..., 8:]):
        with torch.no_grad():
            y = wide(x)
            ref = torch.stack([m.to(DEV).double()(x[q].double()) for q, m in enumerate(mods)])
        assert rel_err(y, ref) <= bar, (d, dtype, x.is_contiguous())
