"""
GPU parity of the HIP kernels against the oracle (the CPU restatement of the reference wide
path) on the same seeded inputs.  Integer / byte work is compared bit-exactly; floating
point by the normwise relative error max|a-b|/max|ref| against TOL_F32 = 1e-5 (fp32) and
TOL_BF16 = 2e-2 (bf16), computed against the oracle run in float64 on the same (rounded)
inputs, and for bf16 additionally against the reference's own bf16 path.
"""

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import bytes_ref, wide_ref
from tests._util import TOL_BF16, TOL_F32, gen, rel_err, tol

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16]


def _rand(shape, g, dtype=torch.float32, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(dtype)


# ----------------------------------------------------------------------------- pack / boundary
@pytest.mark.parametrize("shape,n", [((32, 64), 100), ((8, 64, 4, 4), 10), ((3, 5), 7), ((5,), 3),
                                     ((2, 3, 7), 130)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int64, torch.uint8])
def test_pack_bit_exact(hip, shape, n, dtype):
    import wide_compiler as wc
    g = gen(100)
    ins = [torch.randint(0, 100, shape, generator=g).to(dtype) for _ in range(n)]
    out = wc.pack([t.to(DEV) for t in ins]).cpu()
    assert torch.equal(out, wide_ref.pack_inputs(ins))
    as_np = (lambda t: t.view(torch.int16).numpy()) if dtype == torch.bfloat16 else (lambda t: t.numpy())
    assert np.array_equal(as_np(out), bytes_ref.pack([as_np(t) for t in ins]))


def test_pack_of_unpacked_views_round_trip(hip):
    import wide_compiler as wc
    g = gen(101)
    packed = _rand((4, 12 * 5, 3), g).to(DEV)
    views = wc.unpack(packed, 12)          # strided views, no copy
    again = wc.pack(views)
    assert torch.equal(again, packed)


@pytest.mark.parametrize("n,b,inner,dtype", [(100, 32, 64, torch.float32), (7, 5, 3, torch.bfloat16),
                                             (100, 8, 64 * 16, torch.bfloat16), (3, 2, 1, torch.float32)])
def test_boundary_transpose_bit_exact(hip, n, b, inner, dtype):
    g = gen(102)
    nf = _rand((n, b, inner), g, dtype).to(DEV)
    dst = torch.empty((b, n * inner), dtype=dtype, device=DEV)
    es = nf.element_size()
    hip.swap01(nf, n, b, nf.stride(0) * es, nf.stride(1) * es, inner * es, dst)
    assert torch.equal(dst.cpu(), wide_ref.to_packed(nf.cpu().view(n, b, inner, 1)).view(b, n * inner))


# ----------------------------------------------------------------------------- embedding
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_embedding_shared_bit_exact(hip, dtype):
    import wide_compiler as wc
    g = gen(103)
    torch.manual_seed(103)
    mods = [nn.Embedding(50, 24) for _ in range(6)]
    wide = wc.WideEmbedding.from_modules(mods).to(DEV, dtype)
    ids = torch.randint(0, 50, (3, 9), generator=g)
    with torch.no_grad():
        out = wide(ids.to(DEV)).cpu()
    assert torch.equal(out, wide_ref.embedding(wide.weight.detach().cpu(), ids))


def test_embedding_per_model_bit_exact_and_oob_flag(hip):
    import wide_compiler as wc
    g = gen(104)
    wide = wc.WideEmbedding(5, 33, 16).to(DEV, torch.bfloat16)
    ids = torch.randint(0, 33, (5, 4, 7), generator=g)
    with torch.no_grad():
        out = wide(ids.to(DEV), per_model=True).cpu()
    ref = bytes_ref.embedding_per_model(wide.weight.detach().cpu().float().numpy(), ids.numpy())
    assert np.array_equal(out.float().numpy(), ref)
    wide.index_error()  # no error so far
    bad = ids.clone()
    bad[1, 2, 3] = 33
    with torch.no_grad():
        out = wide(bad.to(DEV), per_model=True).cpu()
    assert torch.count_nonzero(out[1, 2, 3]) == 0
    with pytest.raises(IndexError):
        wide.index_error()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,vocab,d,ids_shape,per_model", [(4, 50, 256, (4, 3, 9), True), (3, 40, 64, (5, 7), False),
                                                           (2, 30, 32, (2, 6), True), (5, 33, 48, (5, 3, 5), True),
                                                           (2, 17, 1024, (2, 4), True), (3, 20, 36, (3, 2), True)])
def test_embedding_layernorm_fused_bit_exact(hip, dtype, n, vocab, d, ids_shape, per_model):
    """forward_layernorm (gather + LayerNorm in one launch) equals the gather followed by the
    LayerNorm bit for bit, against the oracle within the dtype's bar, shared and per-model ids,
    with an out-of-range id (a normalised zero row, the flag set).  Row sizes the fused kernel does
    not take (36 16-bit elements: 72-byte rows) run the two launches."""
    import wide_compiler as wc
    g = gen(107)
    emb = wc.WideEmbedding(n, vocab, d).to(DEV, dtype)
    ln = wc.WideLayerNorm(n, d).to(DEV, dtype)
    with torch.no_grad():
        ln.weight.copy_(torch.randn(n * d, generator=g))
        ln.bias.copy_(torch.randn(n * d, generator=g))
    ids = torch.randint(0, vocab, ids_shape, generator=g)
    with torch.no_grad():
        fused = emb.forward_layernorm(ids.to(DEV), ln, per_model=per_model).cpu()
        two = ln(emb(ids.to(DEV), per_model=per_model)).cpu()
    assert torch.equal(fused, two)
    w = emb.weight.detach().cpu()
    gathered = (torch.stack([w[k][ids[k]] for k in range(n)]) if per_model
                else wide_ref.embedding(w, ids))
    exact = wide_ref.layernorm(gathered.double(), ln.weight.detach().cpu().double(),
                               ln.bias.detach().cpu().double(), n, ln.eps)
    assert rel_err(fused, exact) <= (TOL_F32 if dtype == torch.float32 else TOL_BF16)
    emb.index_error()
    bad = ids.clone()
    bad.view(-1)[3] = vocab
    with torch.no_grad():
        fused = emb.forward_layernorm(bad.to(DEV), ln, per_model=per_model).cpu()
    with pytest.raises(IndexError):
        emb.index_error()
    with torch.no_grad():
        two = ln(emb(bad.to(DEV), per_model=per_model)).cpu()
    assert torch.equal(fused, two)
    with pytest.raises(IndexError):
        emb.index_error()


# ----------------------------------------------------------------------------- norms
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(4, 3, 5, 256), (2, 7, 96), (3, 2, 1000), (64, 16, 8, 256)])
def test_layernorm(hip, dtype, shape):
    import wide_compiler as wc
    g = gen(105)
    n, d = shape[0], shape[-1]
    mod = wc.WideLayerNorm(n, d).to(DEV, dtype)
    with torch.no_grad():
        mod.weight.copy_(torch.randn(n * d, generator=g))
        mod.bias.copy_(torch.randn(n * d, generator=g))
    x = (_rand(shape, g) * 2 + 0.5).to(dtype)
    with torch.no_grad():
        y = mod(x.to(DEV)).cpu()
    w, b = mod.weight.detach().cpu(), mod.bias.detach().cpu()
    exact = wide_ref.layernorm(x.double(), w.double(), b.double(), n, mod.eps)
    assert rel_err(y, exact) <= tol(dtype)
    if dtype == torch.bfloat16:
        assert rel_err(y, wide_ref.layernorm(x, w, b, n, mod.eps)) <= TOL_BF16


def test_layernorm_strided_view(hip):
    import wide_compiler as wc
    g = gen(106)
    n, d = 5, 64
    mod = wc.WideLayerNorm(n, d).to(DEV)
    packed = _rand((6, n * d), g).to(DEV)
    xv = packed.view(6, n, d).movedim(1, 0)    # N-first strided view
    with torch.no_grad():
        y = mod(xv).cpu()
    exact = wide_ref.layernorm(xv.cpu().double(), mod.weight.detach().cpu().double(),
                               mod.bias.detach().cpu().double(), n, mod.eps)
    assert rel_err(y, exact) <= TOL_F32


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("relu", [False, True])
def test_batchnorm2d_eval(hip, dtype, relu):
    import wide_compiler as wc
    g = gen(107)
    n, c = 6, 8
    torch.manual_seed(107)
    mods = [nn.BatchNorm2d(c) for _ in range(n)]
    for m in mods:
        with torch.no_grad():
            m.running_mean.normal_()
            m.running_var.uniform_(0.5, 2)
            m.weight.normal_(1, 0.1)
            m.bias.normal_(0, 0.1)
    wide = wc.WideBatchNorm2d.from_modules(mods).to(DEV, dtype).eval()
    wide.fused_activation = "relu" if relu else None
    x = _rand((n, 3, c, 5, 7), g, dtype)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    op = wide.op
    exact = wide_ref.batchnorm_eval(x.double(), *(t.detach().cpu().double() for t in
                                                  (op.weight, op.bias, op.running_mean, op.running_var)),
                                    op.eps, n)
    if relu:
        exact = F.relu(exact)
    assert rel_err(y, exact) <= tol(dtype)


def test_batchnorm_training_mode_raises(hip):
    import wide_compiler as wc
    wide = wc.WideBatchNorm2d(2, 3).to(DEV).train()
    with torch.no_grad(), pytest.raises(RuntimeError, match="eval"):
        wide(torch.zeros(2, 1, 3, 2, 2, device=DEV))


# ----------------------------------------------------------------------------- grouped GEMM
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,batch,i,o", [(100, (32,), 64, 128), (3, (5, 7), 33, 17), (2, (130,), 256, 200),
                                         (4, (1,), 8, 8), (1, (300,), 512, 96), (8, (2, 3), 1, 5)])
@pytest.mark.parametrize("bias", [True, False])
def test_linear(hip, dtype, n, batch, i, o, bias):
    import wide_compiler as wc
    g = gen(108)
    torch.manual_seed(108)
    mods = [nn.Linear(i, o, bias=bias) for _ in range(n)]
    wide = wc.WideLinear.from_modules(mods).to(DEV, dtype)
    x = _rand((n, *batch, i), g, dtype)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    w = wide.weight.detach().cpu()
    b = wide.bias.detach().cpu() if bias else None
    exact = wide_ref.linear(x.double(), w.double(), None if b is None else b.double())
    assert rel_err(y, exact) <= tol(dtype)
    if dtype == torch.bfloat16:
        assert rel_err(y, wide_ref.linear(x, w, b)) <= TOL_BF16


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("m,o,k", [(300, 300, 264), (256, 260, 64), (257, 255, 72), (512, 256, 512),
                                   (300, 264, 128), (257, 520, 192)])
@pytest.mark.parametrize("rows_inner", [None, 7])
def test_grouped_gemm_large_tiles(hip, out_dtype, m, o, k, rows_inner):
    """bf16 problems big enough (>= 256 tiles of 256 x 256) for the large-tile kernel: ragged
    M / O / K, two-level row addressing, bias + residual + ReLU epilogue, bf16 or fp32 out."""
    from wide_compiler import _hip
    n = 128
    g = gen(113)
    a = _rand((n, m, k), g, torch.bfloat16)
    w = (_rand((n, o, k), g) * k ** -0.5).to(torch.bfloat16)
    bias = _rand((n, o), g, torch.bfloat16)
    res = _rand((n, m, o), g, out_dtype)
    ri = rows_inner or m
    if rows_inner:
        # rows m = outer * ri + inner live at outer * (ri + 3) * k + inner * k: a padded layout
        outer = (m + ri - 1) // ri
        a_store = torch.zeros((n, outer * (ri + 3), k), dtype=torch.bfloat16)
        for r in range(m):
            a_store[:, (r // ri) * (ri + 3) + r % ri] = a[:, r]
        a_so = (ri + 3) * k
    else:
        a_store, a_so = a, 0
    a_d, w_d, b_d, r_d = (t.to(DEV) for t in (a_store, w, bias, res))
    c = torch.empty((n, m, o), dtype=out_dtype, device=DEV)
    _hip.grouped_gemm(n=n, m=m, o=o, k=k, a=a_d, a_sn=a_store.shape[1] * k, a_so=a_so, a_si=k, a_rows_inner=ri,
                      w=w_d, w_sn=o * k, c=c, c_sn=m * o, c_so=0, c_si=o, c_rows_inner=m, bias=b_d, bias_sn=o,
                      residual=r_d, r_sn=m * o, r_so=0, r_si=o, relu=True)
    exact = F.relu(torch.bmm(a.double(), w.double().transpose(1, 2).contiguous()) + bias.double().unsqueeze(1)
                   + res.double())
    assert rel_err(c.cpu(), exact) <= TOL_BF16


@pytest.mark.parametrize("m,o,k,c_ri", [(256, 272, 64, None), (512, 256, 512, None), (272, 512, 128, None),
                                        (272, 512, 128, 48), (2048, 512, 512, 128), (512, 256, 64, None),
                                        (512, 512, 128, 64), (512, 256, 256, None), (544, 320, 512, 32),
                                        (512, 256, 1024, None)])
@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32, None])
@pytest.mark.parametrize("relu", [False, True])
def test_grouped_gemm_large_tiles_plain(hip, m, o, k, c_ri, bias_dtype, relu):
    """The large-tile kernel without residual: one K stage per tile (k = 64), rotated K orders
    over 2-16 stages, bias in bf16, fp32 or absent, with or without ReLU, output rows in one run
    or in groups of c_ri rows two rows apart (two-level output addressing), partial edge tiles
    (m = 544, o = 320)."""
    from wide_compiler import _hip
    n = 128 if m < 1024 else 32
    g = gen(114)
    a = _rand((n, m, k), g, torch.bfloat16)
    w = (_rand((n, o, k), g) * k ** -0.5).to(torch.bfloat16)
    bias = _rand((n, o), g, bias_dtype) if bias_dtype is not None else None
    ri = c_ri or m
    outer = (m + ri - 1) // ri
    pitch = (ri + 2) * o if c_ri else 0
    c = torch.full((n, outer * (ri + 2) if c_ri else m, o), float("nan"), dtype=torch.bfloat16, device=DEV)
    _hip.grouped_gemm(n=n, m=m, o=o, k=k, a=a.to(DEV), a_sn=m * k, a_so=0, a_si=k, a_rows_inner=m,
                      w=w.to(DEV), w_sn=o * k, c=c, c_sn=c.shape[1] * o, c_so=pitch, c_si=o, c_rows_inner=ri,
                      bias=bias.to(DEV) if bias is not None else None, bias_sn=o, relu=relu)
    c = c.cpu()
    rows = [(r // ri) * (ri + 2) + r % ri for r in range(m)] if c_ri else list(range(m))
    got = c[:, rows]
    exact = torch.bmm(a.double(), w.double().transpose(1, 2).contiguous())
    if bias is not None:
        exact = exact + bias.double().unsqueeze(1)
    if relu:
        exact = F.relu(exact)
    assert rel_err(got, exact) <= TOL_BF16
    if c_ri:                                 # the gap rows between groups are never written
        gaps = [r for r in range(c.shape[1]) if r not in set(rows)]
        assert torch.isnan(c[:, gaps]).all()


TOL_F16 = 2e-3   # fp16 output rounding (2^-11 relative) over fp32 accumulation


@pytest.mark.parametrize("m,o,k,n,res", [(64, 48, 40, 4, False), (96, 80, 64, 6, True), (257, 255, 72, 128, True),
                                         (512, 256, 512, 128, False), (512, 256, 256, 128, True)])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("bias_dtype", [torch.float16, torch.float32])
def test_grouped_gemm_fp16(hip, m, o, k, n, res, out_dtype, bias_dtype):
    """fp16 operands on the fp16 MFMA (v_mfma_f32_16x16x32_f16) through every kernel family:
    the small-tile kernel, the 128x64-wave large-tile kernel (k = 72), the two-waves-per-SIMD
    persistent kernel (no residual) and the persistent kernel with a fused residual + ReLU."""
    from wide_compiler import _hip
    g = gen(117)
    a = _rand((n, m, k), g, torch.float16)
    w = (_rand((n, o, k), g) * k ** -0.5).to(torch.float16)
    bias = _rand((n, o), g, bias_dtype)
    r = _rand((n, m, o), g, out_dtype) if res else None
    c = torch.empty((n, m, o), dtype=out_dtype, device=DEV)
    _hip.grouped_gemm(n=n, m=m, o=o, k=k, a=a.to(DEV), a_sn=m * k, a_so=0, a_si=k, a_rows_inner=m, w=w.to(DEV),
                      w_sn=o * k, c=c, c_sn=m * o, c_so=0, c_si=o, c_rows_inner=m, bias=bias.to(DEV), bias_sn=o,
                      residual=None if r is None else r.to(DEV), r_sn=m * o, r_so=0, r_si=o, relu=res)
    exact = torch.bmm(a.double(), w.double().transpose(1, 2).contiguous()) + bias.double().unsqueeze(1)
    if res:
        exact = F.relu(exact + r.double())
    assert rel_err(c.cpu(), exact) <= (TOL_F16 if not res or out_dtype == torch.float32 else 2 * TOL_F16)


def test_linear_fp16_module(hip):
    """WideLinear built from fp16 nn.Linear modules runs on the fp16 MFMA path."""
    import wide_compiler as wc
    g = gen(118)
    torch.manual_seed(118)
    mods = [nn.Linear(96, 64) for _ in range(6)]
    wide = wc.WideLinear.from_modules(mods).to(DEV, torch.float16)
    x = _rand((6, 5, 7, 96), g, torch.float16)
    with torch.no_grad():
        y = wide(x.to(DEV)).cpu()
    exact = wide_ref.linear(x.double(), wide.weight.detach().cpu().double(), wide.bias.detach().cpu().double())
    assert y.dtype == torch.float16
    assert rel_err(y, exact) <= TOL_F16


@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_strided_boundary_view_and_relu(hip, dtype):
    import wide_compiler as wc
    g = gen(109)
    n, b, i, o = 10, 6, 48, 40
    wide = wc.WideLinear(n, i, o).to(DEV, dtype)
    packed = _rand((b, n * i), g, dtype).to(DEV)
    xv = packed.view(b, n, i).movedim(1, 0)
    with torch.no_grad():
        y = wide.forward_into(xv, None, relu=True).cpu()
    exact = F.relu(wide_ref.linear(xv.cpu().double(), wide.weight.detach().cpu().double(),
                                   wide.bias.detach().cpu().double()))
    assert rel_err(y, exact) <= tol(dtype)


def test_linear_forward_only(hip):
    import wide_compiler as wc
    wide = wc.WideLinear(2, 4, 4).to(DEV)
    with pytest.raises(RuntimeError, match="forward-only"):
        wide(torch.zeros(2, 3, 4, device=DEV))


# ----------------------------------------------------------------------------- recurrent
def _rnn_modules(cls, n, i, h, seed, dtype):
    torch.manual_seed(seed)
    return [cls(i, h, batch_first=True).to(dtype) for _ in range(n)]


def _per_step_err(out, exact):
    return [rel_err(out[:, :, t], exact[:, :, t]) for t in range(out.shape[2])]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,b,t,i,h", [(32, 4, 32, 64, 128), (3, 2, 5, 8, 16), (5, 3, 9, 20, 40),
                                       (2, 1, 3, 130, 24), (4, 2, 6, 16, 64),
                                       # fused projection: several 16-step chunks, partial last chunk
                                       (3, 2, 37, 12, 64), (2, 3, 33, 64, 128),
                                       # bf16: partitioned on-chip recurrence (hidden / 128
                                       # workgroups per (model, 16-row chunk)); fp32: streamed
                                       (3, 5, 6, 24, 256), (3, 16, 9, 32, 512), (2, 33, 7, 16, 384),
                                       # 66 x 4 workgroups: two launches of the partitioned kernel
                                       (66, 2, 4, 8, 512),
                                       # streamed (one launch per step): W_hh beyond one workgroup
                                       (2, 20, 4, 8, 288)])
@pytest.mark.parametrize("with_h0", [False, True])
def test_gru(hip, dtype, n, b, t, i, h, with_h0):
    import wide_compiler as wc
    g = gen(110)
    mods = _rnn_modules(nn.GRU, n, i, h, 110, torch.float32)
    wide = wc.WideGRU.from_modules(mods).to(DEV, dtype)
    x = _rand((n, b, t, i), g, dtype)
    h0 = _rand((n, b, h), g, dtype) if with_h0 else None
    with torch.no_grad():
        out, hn = wide(x.to(DEV), None if h0 is None else h0.to(DEV))
    out, hn = out.cpu(), hn.cpu()
    p = [getattr(wide, k).detach().cpu() for k in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
    eo, eh = wide_ref.gru(x.double(), *(q.double() for q in p), h_0=None if h0 is None else h0.double())
    errs = _per_step_err(out, eo)
    # per-timestep bar: TOL at every step t (the error does not compound past it here)
    assert max(errs) <= tol(dtype), errs
    assert rel_err(hn, eh) <= tol(dtype)
    if dtype == torch.bfloat16:
        ro, _ = wide_ref.gru(x, *p, h_0=h0)
        assert max(_per_step_err(out, ro)) <= TOL_BF16


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,b,t,i,h", [(32, 8, 32, 64, 128), (3, 2, 5, 8, 16), (2, 3, 7, 12, 100),
                                       (2, 3, 21, 64, 32),   # fused projection, partial last chunk
                                       # streamed (one launch per step): W_hh beyond one workgroup
                                       (2, 18, 5, 16, 512), (3, 3, 4, 8, 320),
                                       # bf16: partitioned on-chip recurrence (hidden / 128
                                       # workgroups per model); fp32: streamed
                                       (3, 16, 9, 32, 512), (2, 5, 7, 16, 256), (2, 1, 6, 24, 384),
                                       (2, 16, 130, 32, 512),
                                       # batch 33: chunks of 16, 16 and 1 rows; 70 x 4 workgroups:
                                       # two launches of the partitioned kernel
                                       (3, 33, 6, 16, 256), (70, 3, 5, 16, 512)])
@pytest.mark.parametrize("with_state", [False, True])
def test_lstm(hip, dtype, n, b, t, i, h, with_state):
    import wide_compiler as wc
    from wide_compiler import _hip
    g = gen(111)
    mods = _rnn_modules(nn.LSTM, n, i, h, 111, torch.float32)
    wide = wc.WideLSTM.from_modules(mods).to(DEV, dtype)
    x = _rand((n, b, t, i), g, dtype)
    hx = (_rand((n, b, h), g, dtype), _rand((n, b, h), g, dtype)) if with_state else None
    with torch.no_grad():
        out, (hn, cn) = wide(x.to(DEV), None if hx is None else (hx[0].to(DEV), hx[1].to(DEV)))
    _hip.rnn_sync_check(block=True)
    out, hn, cn = out.cpu(), hn.cpu(), cn.cpu()
    p = [getattr(wide, k).detach().cpu() for k in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
    eo, (eh, ec) = wide_ref.lstm(x.double(), *(q.double() for q in p),
                                 hx=None if hx is None else (hx[0].double(), hx[1].double()))
    errs = _per_step_err(out, eo)
    assert max(errs) <= tol(dtype), errs
    assert rel_err(hn, eh) <= tol(dtype)
    assert rel_err(cn, ec) <= tol(dtype)
    if dtype == torch.bfloat16:
        # the reference's own bf16 path (bf16 gates and bf16 cell state, wide_lstm.py:205-229):
        # the same bar at every timestep
        ro, (rh, rc) = wide_ref.lstm(x, *p, hx=hx)
        assert max(_per_step_err(out, ro)) <= TOL_BF16, _per_step_err(out, ro)
        assert rel_err(cn, rc) <= TOL_BF16


@pytest.mark.parametrize("cell,n,b,t,i,h", [("gru", 32, 4, 32, 64, 128), ("gru", 3, 2, 5, 8, 16),
                                             ("lstm", 3, 16, 9, 32, 512), ("lstm", 4, 3, 7, 20, 64),
                                             ("gru", 2, 18, 5, 16, 512), ("lstm", 2, 20, 6, 16, 256),
                                             ("gru", 3, 16, 9, 32, 384), ("lstm", 2, 3, 5, 8, 288)])
def test_rnn_fp16(hip, cell, n, b, t, i, h):
    """fp16 recurrences: fp16 input projection GEMM, the persistent kernel (W_hh in registers,
    fp32 math) for small hidden sizes, the partitioned on-chip kernel (fp16 MFMA) for 256 / 384 /
    512, the streamed kernel (fp16 MFMA per step) otherwise; the per-timestep bar of fp16 at
    every step."""
    import wide_compiler as wc
    g = gen(119)
    cls, wcls, ref = (nn.GRU, wc.WideGRU, wide_ref.gru) if cell == "gru" else (nn.LSTM, wc.WideLSTM, wide_ref.lstm)
    mods = _rnn_modules(cls, n, i, h, 119, torch.float32)
    wide = wcls.from_modules(mods).to(DEV, torch.float16)
    x = _rand((n, b, t, i), g, torch.float16)
    with torch.no_grad():
        out = wide(x.to(DEV))[0].cpu()
    p = [getattr(wide, k).detach().cpu().double() for k in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
    eo = ref(x.double(), *p)[0]
    assert out.dtype == torch.float16
    assert max(_per_step_err(out, eo)) <= 5e-3, _per_step_err(out, eo)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("h", [256, 384, 512])
def test_lstm_nan_crosses_the_exchange(hip, dtype, h):
    """A NaN that starts in one workgroup's units reaches the others through the exchange:
    c0 is NaN at one unit of part 0 (model 1, row 2) and at one unit of the last part (model 2,
    row 17, in the second 16-row chunk).  As in the reference (torch ops throughout), that
    unit's h is NaN at t = 0 and the whole row is NaN from t = 1 on, in every part; every other
    row stays finite and within the bar."""
    import wide_compiler as wc
    from wide_compiler import _hip
    n, b, t, i = 3, 18, 6, 16
    g = gen(131)
    mods = _rnn_modules(nn.LSTM, n, i, h, 131, torch.float32)
    wide = wc.WideLSTM.from_modules(mods).to(DEV, dtype)
    x = _rand((n, b, t, i), g, dtype)
    h0, c0 = _rand((n, b, h), g, dtype), _rand((n, b, h), g, dtype)
    c0[1, 2, 5] = float("nan")
    c0[2, 17, h - 3] = float("nan")
    with torch.no_grad():
        out, (hn, cn) = wide(x.to(DEV), (h0.to(DEV), c0.to(DEV)))
    _hip.rnn_sync_check(block=True)
    out = out.cpu()
    p = [getattr(wide, k).detach().cpu().double() for k in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
    eo, _ = wide_ref.lstm(x.double(), *p, hx=(h0.double(), c0.double()))
    assert torch.equal(out.isnan(), eo.isnan())
    assert out[1, 2, 0].isnan().sum() == 1 and out[1, 2, 1:].isnan().all()
    assert out[2, 17, 0].isnan().sum() == 1 and out[2, 17, 1:].isnan().all()
    fin = ~eo.isnan()
    assert rel_err(out[fin], eo[fin]) <= (tol(dtype) if dtype == torch.bfloat16 else 5e-3)


def test_gru_matches_nn_gru_per_model(hip):
    """The kernel against torch.nn.GRU itself (the reference's validation target)."""
    import wide_compiler as wc
    g = gen(112)
    mods = _rnn_modules(nn.GRU, 4, 10, 32, 112, torch.float32)
    wide = wc.WideGRU.from_modules(mods).to(DEV)
    x = _rand((4, 3, 11, 10), g)
    with torch.no_grad():
        out, _ = wide(x.to(DEV))
        for k in range(4):
            e, _ = mods[k](x[k])
            assert rel_err(out[k].cpu(), e) <= TOL_F32


# ----------------------------------------------------------------------------- traced models
class MLP(nn.Module):
    """cli.py:59-67."""

    def __init__(self, d_in=64, d_hidden=128, d_out=64):
        super().__init__()
        self.fc1 = nn.Linear(d_in, d_hidden)
        self.fc2 = nn.Linear(d_hidden, d_out)

    def forward(self, x):
        return self.fc2(F.relu(self.fc1(x)))


def test_traced_mlp_config(hip):
    """TracedWideModel of N=100 MLP(64,128,64), B=32, fp32 (the CPU-runnable headline model)."""
    import wide_compiler as wc
    n, b = 100, 32
    models = []
    for i in range(n):
        torch.manual_seed(1000 + i)
        models.append(MLP())
    g = gen(113)
    ins = [torch.randn(b, 64, generator=g) for _ in range(n)]
    packed = wide_ref.pack_inputs(ins)
    wide = wc.compile([m.to(DEV) for m in models], ins[0].to(DEV))
    summary = wide.summary()
    assert "fused into fc1" in summary
    with torch.no_grad():
        y = wide(packed.to(DEV)).cpu()
    st = lambda k: torch.stack([getattr(getattr(m, k.split('.')[0]), k.split('.')[1]).detach().cpu().double()
                                for m in models])  # noqa: E731
    exact = wide_ref.mlp_wide(packed.double(), n, st("fc1.weight"), st("fc1.bias"), st("fc2.weight"), st("fc2.bias"))
    assert rel_err(y, exact) <= TOL_F32
    outs = wc.unpack(y, n)
    with torch.no_grad():
        for k in (0, 57, 99):
            assert rel_err(outs[k], models[k].cpu()(ins[k])) <= TOL_F32


class _MLP(nn.Module):
    def __init__(self, d_in, d_hidden, d_out, relu=True):
        super().__init__()
        self.fc1 = nn.Linear(d_in, d_hidden)
        self.fc2 = nn.Linear(d_hidden, d_out)
        self.relu = relu

    def forward(self, x):
        h = self.fc1(x)
        return self.fc2(F.relu(h) if self.relu else h)


class _MLPTap(_MLP):
    """fc1's output feeds fc2 and the model output: the chain must not be fused."""

    def forward(self, x):
        h = self.fc1(x)
        return self.fc2(F.relu(h)) + h.sum(dim=-1, keepdim=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,b,d_in,d_hidden,d_out,relu", [
    (100, 32, 64, 128, 64, True),     # the MLP configuration's shapes
    (7, 37, 32, 64, 16, True),        # rows straddle two 32-row blocks
    (3, 5, 96, 32, 48, False),        # no activation between the layers
    (4, 9, 20, 40, 12, True),         # sizes the fused kernel does not take: two launches
    (5, 100, 64, 96, 128, True),      # fp32: 24-chunk h rows (swizzle over 8), 4 row blocks
    (3, 40, 128, 192, 128, True),     # bf16: 12 hidden column blocks; fp32 exceeds LDS: two launches
    (8, 1040, 64, 128, 48, True),     # 264 workgroups of 32 rows (the others run 16-row ones);
                                      # 3 output column blocks: one wave's tile is unpaired
])
def test_traced_linear_chain(hip, dtype, n, b, d_in, d_hidden, d_out, relu):
    """Linear -> [ReLU] -> Linear runs as one wc_mlp2 launch when the sizes allow it."""
    import wide_compiler as wc
    models = []
    for i in range(n):
        torch.manual_seed(2000 + i)
        models.append(_MLP(d_in, d_hidden, d_out, relu).to(dtype))
    g = gen(114)
    ins = [torch.randn(b, d_in, generator=g).to(dtype) for _ in range(n)]
    packed = wide_ref.pack_inputs(ins)
    wide = wc.compile([m.to(DEV) for m in models], ins[0].to(DEV))
    fused = "one two-layer launch" in wide.summary()
    assert fused == _hip_supported(dtype, d_in, d_hidden, d_out)
    with torch.no_grad():
        y = wide(packed.to(DEV)).cpu()
    st = lambda k: torch.stack([getattr(getattr(m, k.split('.')[0]), k.split('.')[1]).detach().cpu().double()
                                for m in models])  # noqa: E731
    w1, b1, w2, b2 = st("fc1.weight"), st("fc1.bias"), st("fc2.weight"), st("fc2.bias")
    xn = packed.double().view(b, n, d_in).movedim(1, 0)
    h = torch.einsum("nbi,noi->nbo", xn, w1) + b1[:, None]
    h = F.relu(h) if relu else h
    exact = (torch.einsum("nbi,noi->nbo", h, w2) + b2[:, None]).movedim(0, 1).reshape(b, n * d_out)
    assert rel_err(y, exact) <= tol(dtype)
    if dtype == torch.bfloat16:   # the reference's rounding points: bf16 layer outputs
        with torch.no_grad():
            for k in (0, n - 1):
                assert rel_err(y[:, k * d_out:(k + 1) * d_out], models[k].cpu()(ins[k]).float()) <= TOL_BF16


def test_traced_linear_chain_with_tap_is_not_fused(hip):
    import wide_compiler as wc
    n, b = 4, 8
    models = []
    for i in range(n):
        torch.manual_seed(3000 + i)
        models.append(_MLPTap(32, 64, 32))
    g = gen(115)
    ins = [torch.randn(b, 32, generator=g) for _ in range(n)]
    wide = wc.compile([m.to(DEV) for m in models], ins[0].to(DEV))
    assert "one two-layer launch" not in wide.summary()
    with torch.no_grad():
        y = wide(wide_ref.pack_inputs(ins).to(DEV)).cpu()
        for k in range(n):
            assert rel_err(y[:, k * 32:(k + 1) * 32], models[k].cpu()(ins[k])) <= TOL_F32


def _hip_supported(dtype, d_in, d_hidden, d_out):
    from wide_compiler import _hip
    return _hip.mlp2_supported(dtype, d_in, d_hidden, d_out)


def test_compile_validate_true(hip):
    import wide_compiler as wc
    models = [MLP(16, 32, 8).to(DEV) for _ in range(12)]
    wide = wc.compile(models, torch.randn(4, 16, device=DEV), validate=True)
    assert isinstance(wide, wc.TracedWideModel)


def test_cpu_tensors_raise(hip):
    import wide_compiler as wc
    wide = wc.WideLinear(2, 4, 4)
    with torch.no_grad(), pytest.raises(RuntimeError, match="ROCm device"):
        wide(torch.zeros(2, 3, 4))
