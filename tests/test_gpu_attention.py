"""GPU parity of WideAttention (grouped projections + fused attention kernel) against the oracle."""

import pytest
import torch
import torch.nn as nn

from oracle import wide_ref
from tests._util import TOL_BF16, TOL_F32, gen, rel_err, tol

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16]


def _mha(n, d, h, seed, dtype, random_bias=True):
    mods = []
    for i in range(n):
        torch.manual_seed(seed + i)
        m = nn.MultiheadAttention(d, h, batch_first=True)
        if random_bias:
            with torch.no_grad():
                m.in_proj_bias.normal_(0, 0.1)
                m.out_proj.bias.normal_(0, 0.1)
        mods.append(m.to(dtype).eval())
    return mods


def _oracle(wide, q, k, v, causal, double=True):
    c = (lambda t: None if t is None else t.detach().cpu().double()) if double else \
        (lambda t: None if t is None else t.detach().cpu())
    f = (lambda t: t.double()) if double else (lambda t: t)
    return wide_ref.attention(f(q), f(k), f(v), c(wide.q_weight), c(wide.kv_weight), c(wide.out_weight),
                              c(wide.q_bias), c(wide.kv_bias), c(wide.out_bias), wide.n_heads, is_causal=causal)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,b,t,d,h", [(3, 2, 64, 64, 2), (2, 2, 50, 128, 4), (2, 1, 200, 256, 2),
                                       (4, 3, 17, 32, 1), (2, 2, 130, 256, 8), (2, 1, 300, 128, 2),
                                       (2, 2, 333, 64, 2), (1, 2, 600, 64, 2)])
@pytest.mark.parametrize("causal", [False, True])
def test_self_attention(hip, dtype, n, b, t, d, h, causal):
    import wide_compiler as wc
    g = gen(400)
    wide = wc.WideAttention.from_modules(_mha(n, d, h, 400, torch.float32)).to(DEV, dtype).eval()
    x = torch.randn(n, b, t, d, generator=g).to(dtype)
    with torch.no_grad():
        y = wide(x.to(DEV), is_causal=causal).cpu()
    exact = _oracle(wide, x, x, x, causal)
    assert rel_err(y, exact) <= tol(dtype)
    if dtype == torch.bfloat16:
        assert rel_err(y, _oracle(wide, x, x, x, causal, double=False)) <= TOL_BF16


TOL_F16 = 5e-3   # fp16 Q / K / V / P and outputs (2^-11 relative rounding each)


@pytest.mark.parametrize("n,b,t,d,h", [(3, 2, 64, 64, 2), (2, 2, 130, 256, 8), (2, 1, 200, 256, 2),
                                       (2, 2, 100, 512, 4)])
@pytest.mark.parametrize("causal", [False, True])
def test_self_attention_fp16(hip, n, b, t, d, h, causal):
    """fp16 models: projections on the fp16 MFMA GEMM, attention on the general kernel with
    P rounded to fp16 for the fp16 MFMA (head dims 32, 64, 128)."""
    import wide_compiler as wc
    g = gen(405)
    wide = wc.WideAttention.from_modules(_mha(n, d, h, 405, torch.float32)).to(DEV, torch.float16).eval()
    x = torch.randn(n, b, t, d, generator=g).to(torch.float16)
    with torch.no_grad():
        y = wide(x.to(DEV), is_causal=causal).cpu()
    assert y.dtype == torch.float16
    assert rel_err(y, _oracle(wide, x, x, x, causal)) <= TOL_F16


@pytest.mark.parametrize("dtype", DTYPES)
def test_cross_attention_mha_mode(hip, dtype):
    import wide_compiler as wc
    g = gen(401)
    n, b, tq, tkv, d, h = 3, 2, 40, 77, 64, 4
    wide = wc.WideAttention.from_modules(_mha(n, d, h, 401, torch.float32)).to(DEV, dtype).eval()
    q = torch.randn(n, b, tq, d, generator=g).to(dtype)
    k = torch.randn(n, b, tkv, d, generator=g).to(dtype)
    v = torch.randn(n, b, tkv, d, generator=g).to(dtype)
    with torch.no_grad():
        out, w = wide(q.to(DEV), k.to(DEV), v.to(DEV))
    assert w is None
    assert rel_err(out.cpu(), _oracle(wide, q, k, v, False)) <= tol(dtype)


def test_attention_matches_nn_mha_per_model(hip):
    """Against torch.nn.MultiheadAttention itself (batch_first), the reference's bench model."""
    import wide_compiler as wc
    g = gen(402)
    n, b, t, d, h = 3, 2, 33, 64, 4
    mods = _mha(n, d, h, 402, torch.float32)
    wide = wc.WideAttention.from_modules(mods).to(DEV).eval()
    x = torch.randn(n, b, t, d, generator=g)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
        for k in range(n):
            e, _ = mods[k](x[k], x[k], x[k], need_weights=False)
            assert rel_err(y[k], e) <= TOL_F32


def test_attention_dropout_and_mask_with_causal_raise(hip):
    import wide_compiler as wc
    wide = wc.WideAttention(2, 32, 2, dropout=0.1).to(DEV)
    x = torch.zeros(2, 1, 4, 32, device=DEV)
    with torch.no_grad():
        with pytest.raises(RuntimeError, match="dropout"):
            wide.train()(x)
        with pytest.raises(RuntimeError, match="is_causal"):
            wide.eval()(x, attn_mask=torch.zeros(4, 4, device=DEV), is_causal=True)
        with pytest.raises(RuntimeError, match="broadcast"):
            wide.eval()(x, attn_mask=torch.zeros(3, 4, device=DEV))


def _masks(kind, nb, h, tq, tkv, g):
    """(the mask given to the wide module, the same mask as the oracle's SDPA takes it)"""
    if kind == "bool2d":                     # [Tq, Tkv] boolean, two query rows fully masked
        m = torch.rand(tq, tkv, generator=g) > 0.4
        m[3] = False
        m[tq - 1] = False
        return m, m
    if kind == "add_nb":                     # additive [N*B, 1, Tq, Tkv], some -inf
        m = torch.randn(nb, 1, tq, tkv, generator=g)
        m[torch.rand(nb, 1, tq, tkv, generator=g) > 0.8] = float("-inf")
        return m, m
    m = torch.randn(nb, h, tq, tkv, generator=g) * 2           # additive per head
    return m, m


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kind", ["bool2d", "add_nb", "add_heads"])
@pytest.mark.parametrize("n,b,tq,tkv,d,h", [(2, 2, 37, 37, 64, 2), (3, 1, 20, 70, 128, 4)])
def test_attention_mask(hip, dtype, kind, n, b, tq, tkv, d, h):
    """attn_mask with scaled_dot_product_attention semantics (wide_attention.py:222-228):
    boolean (True = attend) or additive, broadcast over [N*B, heads, Tq, Tkv]; a fully masked
    query row gives zeros, as torch's SDPA does."""
    import wide_compiler as wc
    g = gen(404)
    wide = wc.WideAttention.from_modules(_mha(n, d, h, 404, torch.float32)).to(DEV, dtype).eval()
    q = torch.randn(n, b, tq, d, generator=g).to(dtype)
    kv = q if tq == tkv else torch.randn(n, b, tkv, d, generator=g).to(dtype)
    m, m_ref = _masks(kind, n * b, h, tq, tkv, g)
    with torch.no_grad():
        if tq == tkv:
            y = wide(q.to(DEV), attn_mask=m.to(DEV)).cpu()
        else:
            y, _ = wide(q.to(DEV), kv.to(DEV), kv.to(DEV), attn_mask=m.to(DEV))
            y = y.cpu()
    c = lambda t: None if t is None else t.detach().cpu().double()  # noqa: E731
    exact = wide_ref.attention(q.double(), kv.double(), kv.double(), c(wide.q_weight), c(wide.kv_weight),
                               c(wide.out_weight), c(wide.q_bias), c(wide.kv_bias), c(wide.out_bias), h,
                               attn_mask=m_ref if m_ref.dtype == torch.bool else m_ref.double())
    assert torch.isfinite(y).all()
    assert rel_err(y, exact) <= tol(dtype)


@pytest.mark.parametrize("n,b,t,d,h,bias,strided", [(2, 3, 512, 256, 8, True, False), (3, 2, 257, 96, 3, False, True),
                                                    (2, 2, 1, 64, 2, True, False), (1, 3, 256, 128, 4, True, True),
                                                    (2, 1, 100, 768, 24, True, False), (2, 2, 33, 32, 1, False, False)])
@pytest.mark.parametrize("causal", [False, True])
def test_self_attention_fused_projections(hip, monkeypatch, n, b, t, d, h, bias, strided, causal):
    """bf16 self-attention with head dim 32 runs the Q/K/V projections inside the attention
    kernel (wc_self_attention).  Checked against the fp64 and bf16-input fp32 oracles and against
    the unfused path (projection GEMMs + resident attention kernel) on the same inputs: without
    bias, on a strided input view, one token, 32 tokens + 1, 256 (4-wave tiles) and 512 tokens,
    and a 768-wide model (the largest weight staging)."""
    import wide_compiler as wc
    from wide_compiler import _hip
    g = gen(406)
    torch.manual_seed(406)
    wide = wc.WideAttention(n, d, h, bias=bias)
    if bias:
        with torch.no_grad():
            for p_ in (wide.q_bias, wide.kv_bias, wide.out_bias):
                p_.normal_(0, 0.1)
    wide = wide.to(DEV, torch.bfloat16).eval()
    if strided:
        base = torch.randn(n, b, t, d + 32, generator=g).to(torch.bfloat16)
        xd = base.to(DEV)[..., 16:16 + d]
        x = base[..., 16:16 + d]
    else:
        x = torch.randn(n, b, t, d, generator=g).to(torch.bfloat16)
        xd = x.to(DEV)
    calls = []
    fused = _hip.self_attention
    monkeypatch.setattr(_hip, "self_attention", lambda **kw: (calls.append(1), fused(**kw))[1])
    with torch.no_grad():
        y = wide(xd, is_causal=causal).cpu()
        assert calls, "the fused projection kernel did not run"
        wide.fuse_projections = False
        y_sep = wide(xd, is_causal=causal).cpu()
    assert len(calls) == 1
    assert rel_err(y, _oracle(wide, x, x, x, causal)) <= TOL_BF16
    assert rel_err(y, _oracle(wide, x, x, x, causal, double=False)) <= TOL_BF16
    assert rel_err(y, y_sep) <= TOL_BF16


def test_self_attention_fused_rejects(hip):
    """wc_self_attention refuses what its kernel does not take (nothing is launched)."""
    from wide_compiler import _hip
    n, b, d = 1, 1, 128
    w = torch.zeros(n, d, d, device=DEV, dtype=torch.bfloat16)
    kv = torch.zeros(n, 2 * d, d, device=DEV, dtype=torch.bfloat16)
    for t, heads, dtype in ((513, 4, torch.bfloat16), (64, 2, torch.bfloat16), (64, 4, torch.float32)):
        x = torch.zeros(n, b, t, d, device=DEV, dtype=dtype)
        o = torch.empty_like(x)
        with pytest.raises(RuntimeError, match="wc_self_attention"):
            _hip.self_attention(x=x, q_weight=w.to(dtype), kv_weight=kv.to(dtype), q_bias=None, kv_bias=None, o=o,
                                heads=heads, scale=0.1, causal=False)


def test_attention_config_n16(hip):
    """The attention configuration at full size: N=16 MHA(256, 8 heads), B=8, S=512, bf16.
    Every model against the fp32 oracle, three spread models against fp64."""
    import wide_compiler as wc
    g = gen(403)
    n, b, t, d, h = 16, 8, 512, 256, 8
    wide = wc.WideAttention.from_modules(_mha(n, d, h, 403, torch.float32, random_bias=False)).to(DEV, torch.bfloat16)
    x = torch.randn(n, b, t, d, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        y = wide.eval()(x.to(DEV)).cpu()
    names = ("q_weight", "kv_weight", "out_weight", "q_bias", "kv_bias", "out_bias")
    w32 = [None if getattr(wide, a) is None else getattr(wide, a).detach().cpu().float() for a in names]
    xf = x.float()
    exact32 = wide_ref.attention(xf, xf, xf, *w32, h)
    errs = [rel_err(y[k], exact32[k]) for k in range(n)]
    assert max(errs) <= TOL_BF16, max(errs)
    for k in (0, 7, 15):
        c = lambda w: None if w is None else w.detach().cpu()[k:k + 1].double()  # noqa: E731
        exact = wide_ref.attention(x[k:k + 1].double(), x[k:k + 1].double(), x[k:k + 1].double(),
                                   c(wide.q_weight), c(wide.kv_weight), c(wide.out_weight), c(wide.q_bias),
                                   c(wide.kv_bias), c(wide.out_bias), h)
        assert rel_err(y[k:k + 1], exact) <= TOL_BF16


def test_resident_attention_repeatable_on_fresh_inputs(hip):
    """Guard for the resident-KV kernels' softmax exchange between the wave's lane halves (the
    running max and the row sums; a stale word there would corrupt whole output rows): fresh
    inputs, instantiations interleaved (the fused-projection kernel and the resident kernel,
    causal and not, 4- and 8-wave tiles, head dims 32 and 64), three launches each, all
    bit-identical."""
    from wide_compiler import _hip
    g = torch.Generator(device=DEV).manual_seed(430)
    bf = torch.bfloat16
    cfgs = [(4, 4, 512, 256, 8), (3, 2, 256, 128, 4), (2, 3, 384, 128, 2), (2, 2, 200, 64, 1)]
    for _ in range(6):
        for n, b, s, d, heads in cfgs:
            dh = d // heads
            scale = dh ** -0.5
            for causal in (False, True):
                runs = []
                if dh == 32:
                    x = torch.randn(n, b, s, d, device=DEV, generator=g).to(bf)
                    qw = (torch.randn(n, d, d, device=DEV, generator=g) * d ** -0.5).to(bf)
                    kvw = (torch.randn(n, 2 * d, d, device=DEV, generator=g) * d ** -0.5).to(bf)
                    qb = (torch.randn(n, d, device=DEV, generator=g) * 0.1).to(bf)
                    kvb = (torch.randn(n, 2 * d, device=DEV, generator=g) * 0.1).to(bf)

                    def fused(o, x=x, qw=qw, kvw=kvw, qb=qb, kvb=kvb, causal=causal, heads=heads, scale=scale):
                        _hip.self_attention(x=x, q_weight=qw, kv_weight=kvw, q_bias=qb, kv_bias=kvb, o=o,
                                            heads=heads, scale=scale, causal=causal)
                    runs.append(fused)
                q, k, v = (torch.randn(n * b, s, d, device=DEV, generator=g).to(bf) for _ in range(3))

                def resident(o, q=q, k=k, v=v, causal=causal, heads=heads, dh=dh, scale=scale, s=s, d=d):
                    st = (s * d, d)
                    _hip.attention(q=q, k=k, v=v, o=o.view(n * b, s, d), nb=n * b, heads=heads, sq=s, skv=s,
                                   head_dim=dh, q_strides=st, k_strides=st, v_strides=st, o_strides=st,
                                   scale=scale, causal=causal)
                runs.append(resident)
                for run in runs:
                    outs = []
                    for _ in range(3):
                        o = torch.full((n, b, s, d), float("nan"), dtype=bf, device=DEV)
                        run(o)
                        outs.append(o)
                    assert not torch.isnan(outs[0]).any(), (n, b, s, d, heads, causal, run.__name__)
                    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2]), \
                        (n, b, s, d, heads, causal, run.__name__)
