"""Randomized shapes through the wide modules (GPU), against the per-model torch modules in fp64.

A fixed-seed sample of sizes, strides, kernel geometries, head counts, batch sizes, sequence
lengths and dtypes that the fixed-shape tests do not enumerate, so that the host's choice of
kernel path is exercised across shapes as well as the kernels.  Bars (normwise): fp32 1e-5,
fp16 2e-3, bf16 2e-2; the embedding gather is bit-exact.  Reference: for every model i,
torch.nn module i on input i (wide_linear.py, wide_conv2d.py, wide_conv1d.py,
wide_attention.py, wide_lstm.py, wide_gru.py, the norm and embedding primitives are the
reference's restatements of exactly these stacks)."""

import random

import pytest
import torch
import torch.nn as nn

from tests._util import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
BAR = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}
CASES = 30


def _check(got, ref, dt, cfg):
    assert got.shape == ref.shape, cfg
    assert bool(torch.isnan(got).any()) == bool(torch.isnan(ref).any()), cfg
    e = rel_err(got, ref)
    assert e <= BAR[dt], (cfg, e)


def _stack(mods, xs):
    with torch.no_grad():
        return torch.stack([m(x) for m, x in zip(mods, xs)])


def _dt(rng, half=True):
    return rng.choice([torch.float32, torch.bfloat16, torch.float16] if half else [torch.float32, torch.bfloat16])


def test_random_linear(hip):
    import wide_compiler as wc
    rng = random.Random(11)
    torch.manual_seed(11)
    for _ in range(CASES):
        n, b, i, o = rng.randint(1, 40), rng.randint(1, 70), rng.randint(1, 600), rng.randint(1, 600)
        dt, bias, t = _dt(rng), rng.random() < 0.8, rng.choice([None, rng.randint(1, 9)])
        cfg = (n, b, t, i, o, dt, bias)
        mods = [nn.Linear(i, o, bias=bias) for _ in range(n)]
        wide = wc.WideLinear.from_modules(mods).to(DEV, dt)
        x = torch.randn((n, b, i) if t is None else (n, b, t, i)).to(dt)
        with torch.no_grad():
            y = wide(x.to(DEV))
        _check(y, _stack([m.double() for m in mods], [x[k].double() for k in range(n)]), dt, cfg)


def test_random_conv2d_conv1d(hip):
    import wide_compiler as wc
    rng = random.Random(12)
    torch.manual_seed(12)
    for _ in range(CASES):
        two = rng.random() < 0.6
        n, b, dt = rng.randint(1, 8), rng.randint(1, 3), _dt(rng)
        ci, co = rng.choice([1, 3, 8, 16, 32, 40, 64, 96]), rng.choice([1, 4, 16, 32, 64, 72, 128])
        stride, pad, dil = rng.choice([1, 1, 2]), rng.choice([0, 1, 2]), rng.choice([1, 1, 2])
        if two:
            hh, ww, k = rng.randint(1, 40), rng.randint(1, 40), rng.choice([1, 3, 5, (3, 1), (1, 3)])
            kk = k if isinstance(k, tuple) else (k, k)
            if hh + 2 * pad < dil * (kk[0] - 1) + 1 or ww + 2 * pad < dil * (kk[1] - 1) + 1:
                continue
            mods = [nn.Conv2d(ci, co, k, stride=stride, padding=pad, dilation=dil) for _ in range(n)]
            wide = wc.WideConv2d.from_modules(mods).to(DEV, dt)
            x = torch.randn(n, b, ci, hh, ww).to(dt)
        else:
            L, k = rng.randint(1, 90), rng.choice([1, 3, 5, 7])
            if L + 2 * pad < dil * (k - 1) + 1:
                continue
            mods = [nn.Conv1d(ci, co, k, stride=stride, padding=pad, dilation=dil) for _ in range(n)]
            wide = wc.WideConv1d.from_modules(mods).to(DEV, dt)
            x = torch.randn(n, b, ci, L).to(dt)
        cfg = (two, tuple(x.shape), co, k, stride, pad, dil, dt)
        with torch.no_grad():
            y = wide(x.to(DEV))
        _check(y, _stack([m.double() for m in mods], [x[q].double() for q in range(n)]), dt, cfg)


def test_random_attention(hip):
    import wide_compiler as wc
    rng = random.Random(13)
    torch.manual_seed(13)
    for _ in range(CASES):
        n, b, heads = rng.randint(1, 6), rng.randint(1, 4), rng.choice([1, 2, 4, 8])
        d, s, dt = rng.choice([16, 32, 64]) * heads, rng.randint(1, 300), _dt(rng)
        causal = rng.random() < 0.3
        cfg = (n, b, d, heads, s, dt, causal)
        mods = [nn.MultiheadAttention(d, heads, batch_first=True) for _ in range(n)]
        for m in mods:
            nn.init.uniform_(m.in_proj_bias, -0.1, 0.1)
        wide = wc.WideAttention.from_modules(mods).to(DEV, dt).eval()
        x = torch.randn(n, b, s, d).to(dt)
        mask = torch.triu(torch.full((s, s), float("-inf"), dtype=torch.float64), 1) if causal else None
        with torch.no_grad():
            y = wide(x.to(DEV), is_causal=True) if causal else wide(x.to(DEV))
            ref = torch.stack([m.double()(x[q].double(), x[q].double(), x[q].double(), need_weights=False,
                                          attn_mask=mask)[0] for q, m in enumerate(mods)])
        _check(y, ref, dt, cfg)


@pytest.mark.parametrize("kind", ["lstm", "gru"])
def test_random_recurrences(hip, kind):
    import wide_compiler as wc
    from wide_compiler import _hip
    rng = random.Random(14 if kind == "lstm" else 15)
    torch.manual_seed(14)
    for _ in range(CASES):
        n, b, t = rng.randint(1, 6), rng.choice([1, 2, 3, 16, 17, 33]), rng.randint(1, 40)
        i, h = rng.choice([8, 16, 64, 100, 256]), rng.choice([16, 32, 64, 100, 128, 256, 384, 512])
        dt = _dt(rng)
        cfg = (n, b, t, i, h, dt)
        cls, wcls = (nn.LSTM, wc.WideLSTM) if kind == "lstm" else (nn.GRU, wc.WideGRU)
        mods = [cls(i, h, batch_first=True) for _ in range(n)]
        wide = wcls.from_modules(mods).to(DEV, dt)
        x = (torch.randn(n, b, t, i) * 0.5).to(dt)
        with torch.no_grad():
            y = wide(x.to(DEV))[0]
            _hip.rnn_sync_check(block=True)
            ref = torch.stack([m.double()(x[q].double())[0] for q, m in enumerate(mods)])
        _check(y, ref, dt, cfg)


def test_random_norms(hip):
    import wide_compiler as wc
    rng = random.Random(16)
    torch.manual_seed(16)
    for _ in range(CASES):
        kind, n, b, dt = rng.choice(["ln", "bn2", "bn1", "gn", "in2"]), rng.randint(1, 10), rng.randint(1, 5), \
            _dt(rng, half=False)
        if kind == "ln":
            d, t = rng.randint(1, 900), rng.randint(1, 20)
            mods = [nn.LayerNorm(d) for _ in range(n)]
            for m in mods:
                nn.init.uniform_(m.weight, 0.5, 1.5)
                nn.init.uniform_(m.bias, -0.5, 0.5)
            wide = wc.WideLayerNorm.from_modules(mods).to(DEV, dt)
            x = torch.randn(n, b, t, d).to(dt)
        elif kind in ("bn2", "bn1"):
            c = rng.randint(1, 70)
            mods = [(nn.BatchNorm2d if kind == "bn2" else nn.BatchNorm1d)(c).eval() for _ in range(n)]
            for m in mods:
                m.running_mean.uniform_(-1, 1)
                m.running_var.uniform_(0.5, 2)
            wide = (wc.WideBatchNorm2d if kind == "bn2" else wc.WideBatchNorm1d).from_modules(mods).to(DEV, dt).eval()
            x = torch.randn((n, b, c, rng.randint(1, 20), rng.randint(1, 20)) if kind == "bn2"
                            else (n, b, c, rng.randint(1, 30))).to(dt)
        elif kind == "gn":
            g = rng.choice([1, 2, 4, 8])
            c = g * rng.randint(1, 12)
            mods = [nn.GroupNorm(g, c) for _ in range(n)]
            wide = wc.WideGroupNorm.from_modules(mods).to(DEV, dt)
            x = torch.randn(n, b, c, rng.randint(1, 17), rng.randint(1, 17)).to(dt)
        else:
            c = rng.randint(1, 40)
            mods = [nn.InstanceNorm2d(c, affine=True) for _ in range(n)]
            wide = wc.WideInstanceNorm2d.from_modules(mods).to(DEV, dt)
            x = torch.randn(n, b, c, rng.randint(2, 17), rng.randint(2, 17)).to(dt)
        cfg = (kind, tuple(x.shape), dt)
        with torch.no_grad():
            y = wide(x.to(DEV))
        _check(y, _stack([m.double() for m in mods], [x[q].double() for q in range(n)]), dt, cfg)


def test_random_embedding_bit_exact(hip):
    import wide_compiler as wc
    rng = random.Random(17)
    torch.manual_seed(17)
    for _ in range(CASES):
        n, b, t, v, d = rng.randint(1, 10), rng.randint(1, 8), rng.randint(1, 50), rng.randint(1, 5000), \
            rng.randint(1, 700)
        dt, per = _dt(rng), rng.random() < 0.5
        mods = [nn.Embedding(v, d) for _ in range(n)]
        wide = wc.WideEmbedding.from_modules(mods).to(DEV, dt)
        ids = torch.randint(0, v, (n, b, t) if per else (b, t))
        with torch.no_grad():
            y = wide(ids.to(DEV), per_model=per) if per else wide(ids.to(DEV))
            ref = torch.stack([m.to(dt)(ids[q] if per else ids) for q, m in enumerate(mods)])
        assert torch.equal(y.cpu(), ref), (n, b, t, v, d, dt, per)
