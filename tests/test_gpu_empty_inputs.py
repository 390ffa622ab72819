"""Empty inputs through every wide primitive (GPU): a zero batch or zero length gives the empty
output of the shape the per-model torch modules give (stacked on N), without a launch error; a
zero-length sequence into WideGRU / WideLSTM raises RuntimeError, as the reference's per-timestep
`torch.stack` of no timesteps does (wide_gru.py:208, wide_lstm.py:232) and as torch.nn.GRU / LSTM do."""

import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu
DEV = "cuda"
N = 3


def _same_empty(y, ref_shape, dtype):
    assert tuple(y.shape) == tuple(ref_shape), (tuple(y.shape), tuple(ref_shape))
    assert y.numel() == 0 and y.dtype == dtype and y.is_cuda


def test_empty_linear_conv_norms_embedding(hip):
    import wide_compiler as wc
    with torch.no_grad():
        lin = [nn.Linear(8, 5) for _ in range(N)]
        w = wc.WideLinear.from_modules(lin).to(DEV)
        _same_empty(w(torch.randn(N, 0, 8, device=DEV)), (N, 0, 5), torch.float32)
        _same_empty(w(torch.randn(N, 2, 0, 8, device=DEV)), (N, 2, 0, 5), torch.float32)

        conv = [nn.Conv2d(4, 6, 3, padding=1) for _ in range(N)]
        ref = conv[0](torch.randn(0, 4, 8, 8)).shape
        _same_empty(wc.WideConv2d.from_modules(conv).to(DEV)(torch.randn(N, 0, 4, 8, 8, device=DEV)),
                    (N, *ref), torch.float32)
        # the resident-weight kernel's shape (bf16, 3x3 'same', 64 channels)
        cb = wc.WideConv2d.from_modules([nn.Conv2d(64, 64, 3, padding=1) for _ in range(N)]).to(DEV, torch.bfloat16)
        _same_empty(cb(torch.randn(N, 0, 64, 32, 32, device=DEV, dtype=torch.bfloat16)), (N, 0, 64, 32, 32),
                    torch.bfloat16)
        c1 = wc.WideConv1d.from_modules([nn.Conv1d(4, 6, 3, padding=1) for _ in range(N)]).to(DEV)
        _same_empty(c1(torch.randn(N, 0, 4, 10, device=DEV)), (N, 0, 6, 10), torch.float32)

        ln = wc.WideLayerNorm.from_modules([nn.LayerNorm(16) for _ in range(N)]).to(DEV)
        _same_empty(ln(torch.randn(N, 0, 7, 16, device=DEV)), (N, 0, 7, 16), torch.float32)
        _same_empty(ln(torch.randn(N, 2, 0, 16, device=DEV)), (N, 2, 0, 16), torch.float32)
        bn = wc.WideBatchNorm2d.from_modules([nn.BatchNorm2d(4).eval() for _ in range(N)]).to(DEV).eval()
        _same_empty(bn(torch.randn(N, 0, 4, 5, 5, device=DEV)), (N, 0, 4, 5, 5), torch.float32)
        gn = wc.WideGroupNorm.from_modules([nn.GroupNorm(2, 4) for _ in range(N)]).to(DEV)
        _same_empty(gn(torch.randn(N, 0, 4, 5, 5, device=DEV)), (N, 0, 4, 5, 5), torch.float32)

        emb = wc.WideEmbedding.from_modules([nn.Embedding(10, 6) for _ in range(N)]).to(DEV)
        _same_empty(emb(torch.randint(0, 10, (0, 5), device=DEV)), (N, 0, 5, 6), torch.float32)
        _same_empty(emb(torch.randint(0, 10, (2, 0), device=DEV)), (N, 2, 0, 6), torch.float32)
        _same_empty(emb(torch.randint(0, 10, (N, 0, 4), device=DEV), per_model=True), (N, 0, 4, 6), torch.float32)

        packed = wc.pack([torch.randn(0, 8, device=DEV) for _ in range(N)])
        _same_empty(packed, (0, N * 8), torch.float32)
        torch.cuda.synchronize()


def test_empty_attention(hip):
    import wide_compiler as wc
    with torch.no_grad():
        a = wc.WideAttention.from_modules([nn.MultiheadAttention(32, 2, batch_first=True) for _ in range(N)])
        a = a.to(DEV).eval()
        _same_empty(a(torch.randn(N, 0, 7, 32, device=DEV)), (N, 0, 7, 32), torch.float32)
        _same_empty(a(torch.randn(N, 2, 0, 32, device=DEV)), (N, 2, 0, 32), torch.float32)
        # the fused-projection kernel's shape (bf16, head dim 32)
        ab = wc.WideAttention.from_modules([nn.MultiheadAttention(256, 8, batch_first=True) for _ in range(N)])
        ab = ab.to(DEV, torch.bfloat16).eval()
        for shape in ((N, 0, 64, 256), (N, 2, 0, 256)):
            _same_empty(ab(torch.randn(*shape, device=DEV, dtype=torch.bfloat16)), shape, torch.bfloat16)
        torch.cuda.synchronize()


@pytest.mark.parametrize("kind", ["gru", "lstm"])
@pytest.mark.parametrize("hidden, dtype", [(16, torch.float32), (512, torch.bfloat16)])
def test_empty_recurrences(hip, kind, hidden, dtype):
    import wide_compiler as wc
    from wide_compiler import _hip
    cls, wcls = (nn.GRU, wc.WideGRU) if kind == "gru" else (nn.LSTM, wc.WideLSTM)
    with torch.no_grad():
        r = wcls.from_modules([cls(8, hidden, batch_first=True) for _ in range(N)]).to(DEV, dtype)
        out = r(torch.randn(N, 0, 5, 8, device=DEV, dtype=dtype))
        y = out[0]
        _same_empty(y, (N, 0, 5, hidden), dtype)
        h_n = out[1][0] if kind == "lstm" else out[1]
        assert tuple(h_n.shape) == (N, 0, hidden)
        with pytest.raises(RuntimeError):
            r(torch.randn(N, 2, 0, 8, device=DEV, dtype=dtype))
        with pytest.raises(RuntimeError):
            cls(8, hidden, batch_first=True)(torch.randn(2, 0, 8))
        torch.cuda.synchronize()
        _hip.rnn_sync_check(block=True)
