"""Randomized shapes through the wide modules (GPU), against the per-model torch modules in fp64.

A fixed-seed sample of sizes, strides, kernel geometries, head counts, batch sizes, sequence
lengths and dtypes that the fixed-shape tests do not enumerate, so that the host's choice of
kernel path is exercised across shapes as well as the kernels.  Bars (normwise): fp32 1e-5,
fp16 2e-3, bf16 2e-2; the embedding gather is bit-exact.  Reference: for every model i,
torch.nn module i on input i (wide_linear.py, wide_conv2d.py, wide_conv1d.py,
wide_attention.py, wide_lstm.py, wide_gru.py, the norm and embedding primitives are the
reference's restatements of exactly these stacks).  Beyond single-input modules: cross-attention
under boolean and additive masks, recurrences from given initial states, strided input views, and
random MLP / CNN stacks through the traced compile path."""

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


def test_random_masked_cross_attention(hip):
    """Separate query / key / value inputs of different lengths, with a boolean mask (the
    scaled_dot_product_attention convention the reference passes through at
    wide_attention.py:222-228: True = attend; nn.MultiheadAttention takes the complement) or an
    additive float mask."""
    import wide_compiler as wc
    rng = random.Random(18)
    torch.manual_seed(18)
    for _ in range(CASES):
        n, b, heads = rng.randint(1, 4), rng.randint(1, 3), rng.choice([1, 2, 4])
        d, sq, skv = rng.choice([16, 32, 64]) * heads, rng.randint(1, 120), rng.randint(1, 120)
        dt, kind = _dt(rng, half=False), rng.choice(["bool", "float", "none"])
        cfg = (n, b, d, heads, sq, skv, dt, kind)
        mods = [nn.MultiheadAttention(d, heads, batch_first=True) for _ in range(n)]
        for m in mods:
            nn.init.uniform_(m.in_proj_bias, -0.1, 0.1)
        wide = wc.WideAttention.from_modules(mods).to(DEV, dt).eval()
        q, k, v = (torch.randn(n, b, s, d).to(dt) for s in (sq, skv, skv))
        mask, ref_mask = None, None
        if kind == "bool":
            mask = torch.rand(sq, skv) > 0.3
            mask[:, 0] = True                     # every query row attends to at least one key
            ref_mask = ~mask
        elif kind == "float":
            mask = torch.randn(sq, skv) * 2
            ref_mask = mask.double()
        with torch.no_grad():
            y, _ = wide(q.to(DEV), k.to(DEV), v.to(DEV), attn_mask=None if mask is None else mask.to(DEV))
            ref = torch.stack([m.double()(q[i].double(), k[i].double(), v[i].double(), need_weights=False,
                                          attn_mask=ref_mask)[0] for i, m in enumerate(mods)])
        _check(y, ref, dt, cfg)


def test_random_head_dims(hip):
    """Any head dim (1-256 in bf16 / fp16, 1-128 in fp32): self-attention (causal or not, with an
    additive mask or none) and cross-attention at random lengths, rows at the odd strides that
    heads * head_dim gives (scaled_dot_product_attention takes any head dim,
    wide_attention.py:212-231)."""
    import wide_compiler as wc
    rng = random.Random(23)
    torch.manual_seed(23)
    for _ in range(CASES):
        dt = _dt(rng)
        dh = rng.randint(1, 128 if dt == torch.float32 else 256)
        n, b, heads = rng.randint(1, 3), rng.randint(1, 3), rng.choice([1, 2, 3])
        d, sq = dh * heads, rng.randint(1, 200)
        kind = rng.choice(["self", "causal", "mask", "cross"])
        skv = rng.randint(1, 200) if kind == "cross" else sq
        cfg = (n, b, d, heads, sq, skv, dt, kind)
        mods = [nn.MultiheadAttention(d, heads, batch_first=True) for _ in range(n)]
        for m in mods:
            nn.init.uniform_(m.in_proj_bias, -0.1, 0.1)
        wide = wc.WideAttention.from_modules(mods).to(DEV, dt).eval()
        q = torch.randn(n, b, sq, d).to(dt)
        k, v = (torch.randn(n, b, skv, d).to(dt) for _ in range(2)) if kind == "cross" else (q, q)
        mask = torch.randn(sq, skv) * 2 if kind == "mask" else None
        ref_mask = mask.double() if mask is not None else (
            torch.triu(torch.full((sq, sq), float("-inf"), dtype=torch.float64), 1) if kind == "causal" else None)
        with torch.no_grad():
            if kind == "cross":
                y, _ = wide(q.to(DEV), k.to(DEV), v.to(DEV))
            else:
                y = wide(q.to(DEV), is_causal=kind == "causal",
                         attn_mask=None if mask is None else mask.to(DEV))
            ref = torch.stack([m.double()(q[i].double(), k[i].double(), v[i].double(), need_weights=False,
                                          attn_mask=ref_mask)[0] for i, m in enumerate(mods)])
        _check(y, ref, dt, cfg)


@pytest.mark.parametrize("kind", ["lstm", "gru"])
def test_random_recurrences_with_initial_state(hip, kind):
    """h0 (and c0) given: the final states as well as the output sequence."""
    import wide_compiler as wc
    from wide_compiler import _hip
    rng = random.Random(19 if kind == "lstm" else 20)
    torch.manual_seed(19)
    for _ in range(CASES // 2):
        n, b, t = rng.randint(1, 5), rng.choice([1, 3, 16, 20]), rng.randint(1, 30)
        i, h, dt = rng.choice([8, 64, 256]), rng.choice([32, 128, 256, 512]), _dt(rng)
        cfg = (n, b, t, i, h, dt)
        cls, wcls = (nn.LSTM, wc.WideLSTM) if kind == "lstm" else (nn.GRU, wc.WideGRU)
        mods = [cls(i, h, batch_first=True) for _ in range(n)]
        wide = wcls.from_modules(mods).to(DEV, dt)
        x = (torch.randn(n, b, t, i) * 0.5).to(dt)
        h0, c0 = ((torch.randn(n, b, h) * 0.5).to(dt) for _ in range(2))
        with torch.no_grad():
            if kind == "lstm":
                y, (hn, cn) = wide(x.to(DEV), (h0.to(DEV), c0.to(DEV)))
                refs = [m.double()(x[q].double(), (h0[q].double()[None], c0[q].double()[None]))
                        for q, m in enumerate(mods)]
                _hip.rnn_sync_check(block=True)
                _check(cn, torch.stack([r[1][1][0] for r in refs]), dt, cfg)
                hn_ref = torch.stack([r[1][0][0] for r in refs])
            else:
                y, hn = wide(x.to(DEV), h0.to(DEV))
                refs = [m.double()(x[q].double(), h0[q].double()[None]) for q, m in enumerate(mods)]
                _hip.rnn_sync_check(block=True)
                hn_ref = torch.stack([r[1][0] for r in refs])
        _check(y, torch.stack([r[0] for r in refs]), dt, cfg)
        _check(hn, hn_ref, dt, cfg)


def test_random_strided_inputs(hip):
    """Inputs that are views with non-unit or padded strides (a sliced feature axis, transposed
    batch / time axes, a cropped image width)."""
    import wide_compiler as wc
    rng = random.Random(21)
    torch.manual_seed(21)
    for _ in range(CASES):
        kind, n, b, dt = rng.choice(["linear", "conv2d", "layernorm"]), rng.randint(1, 6), rng.randint(1, 5), \
            _dt(rng, half=False)
        if kind == "linear":
            i, o, t = rng.randint(1, 200), rng.randint(1, 200), rng.randint(1, 7)
            mods = [nn.Linear(i, o) for _ in range(n)]
            wide = wc.WideLinear.from_modules(mods).to(DEV, dt)
            base = torch.randn(n, t, b, 2 * i).to(dt)
            view = lambda z: z[..., ::2].transpose(1, 2)          # noqa: E731  [n, b, t, i]
        elif kind == "conv2d":
            c, co, hw = rng.choice([3, 8, 16]), rng.choice([4, 16]), rng.randint(3, 16)
            mods = [nn.Conv2d(c, co, 3, padding=1) for _ in range(n)]
            wide = wc.WideConv2d.from_modules(mods).to(DEV, dt)
            base = torch.randn(n, b, c, hw, hw + 3).to(dt)
            view = lambda z, hw=hw: z[..., 1:hw + 1]                # noqa: E731
        else:
            d, t = rng.randint(2, 300), rng.randint(1, 9)
            mods = [nn.LayerNorm(d) for _ in range(n)]
            wide = wc.WideLayerNorm.from_modules(mods).to(DEV, dt)
            base = torch.randn(n, b, t, d + 5).to(dt)
            view = lambda z, d=d: z[..., 2:d + 2]                   # noqa: E731
        x = view(base)
        xd = view(base.to(DEV))
        cfg = (kind, tuple(x.shape), tuple(x.stride()), dt)
        with torch.no_grad():
            y = wide(xd)
        _check(y, _stack([m.double() for m in mods], [x[q].double() for q in range(n)]), dt, cfg)


class _RandMLP(nn.Module):
    def __init__(self, dims, acts):
        super().__init__()
        self.layers = nn.ModuleList([nn.Linear(a, b) for a, b in zip(dims[:-1], dims[1:])])
        self.acts = acts

    def forward(self, x):
        for i, layer in enumerate(self.layers):
            x = layer(x)
            if i + 1 < len(self.layers):
                a = self.acts[i]
                x = torch.relu(x) if a == "relu" else torch.nn.functional.gelu(x) if a == "gelu" else \
                    torch.tanh(x) if a == "tanh" else x
        return x


class _RandCNN(nn.Module):
    def __init__(self, c, depth, res, bn, k):
        super().__init__()
        self.convs = nn.ModuleList([nn.Conv2d(c, c, k, padding=k // 2) for _ in range(depth)])
        self.bns = nn.ModuleList([nn.BatchNorm2d(c) for _ in range(depth)]) if bn else None
        self.res = res

    def forward(self, x):
        for i, conv in enumerate(self.convs):
            y = conv(x)
            if self.bns is not None:
                y = self.bns[i](y)
            x = torch.relu(y + x) if self.res else torch.relu(y)
        return x


def test_random_traced_models(hip):
    """Random MLP and CNN stacks through the public compile / pack / unpack API (the traced
    path: api.py:36 compile, api.py:310-319 pack / unpack, core/traced_wide.py), fp32."""
    import wide_compiler as wc
    rng = random.Random(22)
    torch.manual_seed(22)
    for _ in range(CASES):
        if rng.random() < 0.5:
            n, depth, b = rng.randint(1, 20), rng.randint(1, 4), rng.randint(1, 40)
            dims = [rng.choice([3, 8, 16, 32, 64, 100, 128, 256]) for _ in range(depth + 1)]
            acts = [rng.choice(["relu", "gelu", "tanh", "none"]) for _ in range(depth)]
            cfg = ("mlp", n, dims, acts, b)
            models = [_RandMLP(dims, acts).to(DEV).eval() for _ in range(n)]
            ins = [torch.randn(b, dims[0], device=DEV) for _ in range(n)]
        else:
            n, c, depth = rng.randint(1, 6), rng.choice([4, 8, 16, 32, 64]), rng.randint(1, 3)
            res, bn, k, hw, b = rng.random() < 0.5, rng.random() < 0.6, rng.choice([1, 3]), rng.randint(3, 20), \
                rng.randint(1, 3)
            cfg = ("cnn", n, c, depth, res, bn, k, hw, b)
            models = []
            for _ in range(n):
                m = _RandCNN(c, depth, res, bn, k)
                for q in (m.bns or []):
                    q.running_mean.uniform_(-0.5, 0.5)
                    q.running_var.uniform_(0.5, 2.0)
                models.append(m.to(DEV).eval())
            ins = [torch.randn(b, c, hw, hw, device=DEV) for _ in range(n)]
        wide = wc.compile(models, ins[0]).eval()
        with torch.no_grad():
            outs = wc.unpack(wide(wc.pack(ins)), n)
            for q in range(n):
                _check(outs[q], models[q].double()(ins[q].double()), torch.float32, cfg)
