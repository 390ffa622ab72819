"""A wide Linear whose per-model input is larger than 2^31 bytes (GPU).

The persistent XL GEMM addresses a model's operands with 32-bit offsets and so declines such
shapes; they run on the 64-bit-addressed kernels instead.  Rows on both sides of the 2^31-byte
offset of every model are checked against torch (fp32 products of the same bf16 values) at the
bf16 bar; the reference computes the same product with einsum (wide_linear.py:150-173)."""

import pytest
import torch
import torch.nn as nn

from tests._util import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_linear_input_beyond_2gib_per_model(hip):
    import wide_compiler as wc
    n, k, o = 2, 8192, 256
    m = (1 << 31) // (k * 2) + 16            # the last 16 rows of each model start past byte 2^31
    torch.manual_seed(0)
    mods = [nn.Linear(k, o) for _ in range(n)]
    wide = wc.WideLinear.from_modules(mods).to(DEV, torch.bfloat16)
    x = torch.randn(n, m, k, device=DEV, dtype=torch.bfloat16)
    assert x[0].numel() * x.element_size() > (1 << 31)
    with torch.no_grad():
        y = wide(x)
    assert tuple(y.shape) == (n, m, o)
    first_past = (1 << 31) // (k * 2)
    for q in range(n):
        w = wide.weight[q].float()
        b = wide.bias[q].float()
        for r0 in (0, m // 2, first_past - 16, first_past):
            rows = slice(r0, r0 + 16)
            ref = x[q, rows].float() @ w.t() + b
            e = rel_err(y[q, rows], ref)
            assert e <= 2e-2, (q, r0, e)
    del x, y
    torch.cuda.empty_cache()


def test_embedding_table_beyond_2gib_per_model(hip):
    """Gather (and gather + LayerNorm in one launch) from a per-model table larger than 2^31 bytes:
    ids past row 2^20 lie beyond the offset.  The gather is bit-exact against torch indexing
    (wide_embedding.py:93-131), and the fused launch bit-identical to gather then LayerNorm."""
    import wide_compiler as wc
    n, d = 2, 1024
    vocab = (1 << 31) // (d * 2) + 64
    torch.manual_seed(1)
    with torch.device("meta"):                  # no 8.6 GB fp32 table on the host
        emb = wc.WideEmbedding(n, vocab, d)
    emb = emb.to_empty(device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        emb.weight.normal_()
    assert emb.weight[0].numel() * emb.weight.element_size() > (1 << 31)
    ln = wc.WideLayerNorm.from_modules([nn.LayerNorm(d) for _ in range(n)]).to(DEV, torch.bfloat16)
    ids = torch.randint(0, vocab, (n, 4, 64), device=DEV)
    ids[:, :, :8] = torch.randint(vocab - 64, vocab, (n, 4, 8), device=DEV)      # past the 2^31-byte row
    with torch.no_grad():
        y = emb(ids, per_model=True)
        ref = torch.stack([emb.weight[q][ids[q]] for q in range(n)])
        assert torch.equal(y, ref)
        y_shared = emb(ids[0])
        assert torch.equal(y_shared, torch.stack([emb.weight[q][ids[0]] for q in range(n)]))
        fused = emb.forward_layernorm(ids, ln, per_model=True)
        assert torch.equal(fused, ln(y))
    del emb, y, ref, y_shared, fused
    torch.cuda.empty_cache()
