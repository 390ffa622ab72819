"""
Pins the oracle (CPU restatement of the reference wide path) against independent
implementations: per-model torch.nn modules, float64 brute force and closed forms.  Each
pin is chosen so that a plausible restatement mistake fails it; test_planted_* show that
by planting such mistakes into copies of oracle functions.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import bytes_ref, wide_ref
from tests._util import gen, rel_err

torch.set_num_threads(4)


# ----------------------------------------------------------------------------- byte maps
@pytest.mark.parametrize("shape", [(3, 5), (2, 4, 3, 3), (4,), (2, 3, 7)])
def test_pack_unpack_index_maps(shape):
    n = 5
    ins = [torch.arange(int(np.prod(shape)), dtype=torch.int32).reshape(shape) + 1000 * i for i in range(n)]
    t_packed = wide_ref.pack_inputs(ins)
    np_packed = bytes_ref.pack([t.numpy() for t in ins])
    assert np.array_equal(t_packed.numpy(), np_packed)
    if len(shape) > 1:
        for a, b in zip(wide_ref.unpack_outputs(t_packed, n), bytes_ref.unpack(np_packed, n)):
            assert np.array_equal(a.numpy(), b)
        # closed form: packed[b, i*F + f] = input_i[b, f]
        f = shape[1]
        assert t_packed[1, 3 * f + 2].flatten()[0].item() == ins[3][1, 2].flatten()[0].item()


def test_boundary_maps():
    n, b, c, h = 4, 3, 2, 5
    x = torch.arange(b * n * c * h, dtype=torch.int64).reshape(b, n * c, h)
    nf = wide_ref.to_nfirst(x, n)
    assert np.array_equal(nf.numpy(), bytes_ref.packed_to_nfirst(x.numpy(), n))
    assert nf[2, 1, 1, 3].item() == x[1, 2 * c + 1, 3].item()
    assert np.array_equal(wide_ref.to_packed(nf.contiguous()).numpy(), x.numpy())
    assert np.array_equal(bytes_ref.nfirst_to_packed(nf.numpy()), x.numpy())


def test_embedding_maps():
    g = gen(0)
    w = torch.randn(3, 11, 4, generator=g)
    ids = torch.randint(0, 11, (2, 5), generator=g)
    assert np.array_equal(wide_ref.embedding(w, ids).numpy(), bytes_ref.embedding_shared(w.numpy(), ids.numpy()))
    pm = torch.randint(0, 11, (3, 2, 5), generator=g)
    ref = bytes_ref.embedding_per_model(w.numpy(), pm.numpy())
    assert np.array_equal(wide_ref.embedding_per_model(w, pm).numpy(), ref)
    assert np.array_equal(ref[2, 1, 4], w[2, pm[2, 1, 4]].numpy())


# ----------------------------------------------------------------------------- linear
def test_linear_vs_nn_linear():
    g = gen(1)
    n, b, i, o = 4, 6, 5, 7
    mods = [nn.Linear(i, o).double() for _ in range(n)]
    x = torch.randn(n, b, 3, i, generator=g, dtype=torch.float64)
    w = torch.stack([m.weight for m in mods]).detach()
    bias = torch.stack([m.bias for m in mods]).detach()
    y = wide_ref.linear(x, w, bias)
    for k in range(n):
        assert torch.allclose(y[k], mods[k](x[k]), atol=1e-12)
    # N=1 reduces to F.linear; no bias path
    assert torch.allclose(wide_ref.linear(x[:1], w[:1], None)[0], F.linear(x[0], w[0]), atol=1e-12)


# ----------------------------------------------------------------------------- conv
def _conv2d_brute(x, w, bias, pad):
    b, c, h, wd = x.shape
    co, _, kh, kw = w.shape
    xp = F.pad(x, (pad, pad, pad, pad))
    ho, wo = h + 2 * pad - kh + 1, wd + 2 * pad - kw + 1
    out = torch.zeros(b, co, ho, wo, dtype=x.dtype)
    for bb in range(b):
        for oc in range(co):
            for y in range(ho):
                for xx in range(wo):
                    out[bb, oc, y, xx] = (xp[bb, :, y:y + kh, xx:xx + kw] * w[oc]).sum() + bias[oc]
    return out


def test_conv2d_vs_per_model_and_brute():
    g = gen(2)
    n, b, ci, co = 2, 1, 3, 2
    mods = [nn.Conv2d(ci, co, 3, padding=1).double() for _ in range(n)]
    x = torch.randn(n, b, ci, 4, 4, generator=g, dtype=torch.float64)
    w = torch.cat([m.weight for m in mods]).detach()
    bias = torch.cat([m.bias for m in mods]).detach()
    y = wide_ref.conv2d(x, w, bias, n, padding=(1, 1))
    for k in range(n):
        assert torch.allclose(y[k], mods[k](x[k]), atol=1e-12)
        assert torch.allclose(y[k], _conv2d_brute(x[k], mods[k].weight.detach(), mods[k].bias.detach(), 1),
                              atol=1e-12)


def test_conv1d_vs_per_model():
    g = gen(3)
    n = 3
    mods = [nn.Conv1d(4, 5, 3, stride=2, padding=1, dilation=2).double() for _ in range(n)]
    x = torch.randn(n, 2, 4, 17, generator=g, dtype=torch.float64)
    w = torch.cat([m.weight for m in mods]).detach()
    bias = torch.cat([m.bias for m in mods]).detach()
    y = wide_ref.conv1d(x, w, bias, n, stride=2, padding=1, dilation=2)
    for k in range(n):
        assert torch.allclose(y[k], mods[k](x[k]), atol=1e-12)


# ----------------------------------------------------------------------------- norms
def test_batchnorm_eval_closed_form():
    g = gen(4)
    n, b, c = 3, 2, 4
    x = torch.randn(n, b, c, 3, 3, generator=g, dtype=torch.float64)
    w, bias = torch.randn(n * c, generator=g, dtype=torch.float64), torch.randn(n * c, generator=g, dtype=torch.float64)
    rm, rv = torch.randn(n * c, generator=g, dtype=torch.float64), torch.rand(n * c, generator=g, dtype=torch.float64) + 0.5
    y = wide_ref.batchnorm_eval(x, w, bias, rm, rv, 1e-5, n)
    for i in range(n):
        for ch in range(c):
            k = i * c + ch
            exp = (x[i, :, ch] - rm[k]) / math.sqrt(rv[k] + 1e-5) * w[k] + bias[k]
            assert torch.allclose(y[i, :, ch], exp, atol=1e-12)


def test_layernorm_vs_f_layer_norm():
    g = gen(5)
    n, d = 3, 8
    x = torch.randn(n, 2, 5, d, generator=g, dtype=torch.float64) * 3 + 1
    w = torch.randn(n * d, generator=g, dtype=torch.float64)
    b = torch.randn(n * d, generator=g, dtype=torch.float64)
    y = wide_ref.layernorm(x, w, b, n, 1e-5)
    for i in range(n):
        exp = F.layer_norm(x[i], (d,), w[i * d:(i + 1) * d], b[i * d:(i + 1) * d], 1e-5)
        assert torch.allclose(y[i], exp, atol=1e-12)


def test_conv3d_vs_per_model_and_brute_force():
    g = gen(53)
    n, b, ci, co = 2, 2, 3, 4
    torch.manual_seed(53)
    mods = [nn.Conv3d(ci, co, (2, 3, 2), stride=(1, 2, 1), padding=(1, 1, 0), dilation=(2, 1, 1)).double()
            for _ in range(n)]
    x = torch.randn(n, b, ci, 4, 5, 3, generator=g, dtype=torch.float64)
    w = torch.cat([m.weight for m in mods]).detach()
    bias = torch.cat([m.bias for m in mods]).detach()
    y = wide_ref.conv3d(x, w, bias, n, (1, 2, 1), (1, 1, 0), (2, 1, 1))
    for i in range(n):
        assert torch.allclose(y[i], mods[i](x[i]), atol=1e-12)
    # brute force for model 1, batch 0, output channel 2 at a few positions
    xp = F.pad(x[1, 0], (0, 0, 1, 1, 1, 1))
    wt = mods[1].weight.detach()
    for (od, oh, ow) in [(0, 0, 0), (1, 2, 1), (2, 1, 0)]:
        acc = mods[1].bias[2].item()
        for c in range(ci):
            for t in range(2):
                for r in range(3):
                    for q in range(2):
                        acc += wt[2, c, t, r, q].item() * xp[c, od + 2 * t, oh * 2 + r, ow + q].item()
        assert abs(acc - y[1, 0, 2, od, oh, ow].item()) < 1e-10


def test_group_norm_vs_nn_group_norm():
    g = gen(51)
    n, b, c, groups = 3, 2, 6, 3
    x = torch.randn(n, b, c, 4, 5, generator=g, dtype=torch.float64) * 2 + 0.5
    mods = []
    for i in range(n):
        m = nn.GroupNorm(groups, c).double()
        with torch.no_grad():
            m.weight.copy_(torch.randn(c, generator=g, dtype=torch.float64))
            m.bias.copy_(torch.randn(c, generator=g, dtype=torch.float64))
        mods.append(m)
    w = torch.cat([m.weight for m in mods]).detach()
    bb = torch.cat([m.bias for m in mods]).detach()
    y = wide_ref.group_norm(x, w, bb, groups, 1e-5)
    for i in range(n):
        assert torch.allclose(y[i], mods[i](x[i]), atol=1e-12)
    # groups = 1 is LayerNorm over (C, H, W) without affine; a per-channel grouping would differ
    y1 = wide_ref.group_norm(x, None, None, 1, 1e-5)
    exp = F.layer_norm(x, x.shape[2:], eps=1e-5)
    assert torch.allclose(y1, exp, atol=1e-12)
    assert not torch.allclose(wide_ref.group_norm(x, None, None, c, 1e-5), exp, atol=1e-3)


def test_instance_norm_vs_nn_instance_norm():
    g = gen(52)
    n, b, c = 2, 3, 4
    x1 = torch.randn(n, b, c, 7, generator=g, dtype=torch.float64) * 3 - 1
    x2 = torch.randn(n, b, c, 3, 5, generator=g, dtype=torch.float64)
    for x, cls in ((x1, nn.InstanceNorm1d), (x2, nn.InstanceNorm2d)):
        mods = [cls(c, affine=True).double() for _ in range(n)]
        with torch.no_grad():
            for m in mods:
                m.weight.copy_(torch.randn(c, generator=g, dtype=torch.float64))
                m.bias.copy_(torch.randn(c, generator=g, dtype=torch.float64))
        w = torch.cat([m.weight for m in mods]).detach()
        bb = torch.cat([m.bias for m in mods]).detach()
        y = wide_ref.instance_norm(x, w, bb, 1e-5)
        for i in range(n):
            assert torch.allclose(y[i], mods[i](x[i]), atol=1e-12)
        # eval mode with running statistics
        tracked = [cls(c, affine=True, track_running_stats=True).double().eval() for _ in range(n)]
        with torch.no_grad():
            for m in tracked:
                m.running_mean.copy_(torch.randn(c, generator=g, dtype=torch.float64))
                m.running_var.copy_(torch.rand(c, generator=g, dtype=torch.float64) + 0.5)
                m.weight.copy_(torch.randn(c, generator=g, dtype=torch.float64))
        rm = torch.cat([m.running_mean for m in tracked])
        rv = torch.cat([m.running_var for m in tracked])
        w = torch.cat([m.weight for m in tracked]).detach()
        bb = torch.cat([m.bias for m in tracked]).detach()
        y = wide_ref.instance_norm(x, w, bb, 1e-5, rm, rv)
        for i in range(n):
            assert torch.allclose(y[i], tracked[i](x[i]), atol=1e-12)


# ----------------------------------------------------------------------------- recurrent
def _gru_modules(n, i, h, seed):
    torch.manual_seed(seed)
    return [nn.GRU(i, h, batch_first=True).double() for _ in range(n)]


def _gru_params(mods):
    return [torch.stack([getattr(m, k) for m in mods]).detach()
            for k in ("weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0")]


def test_gru_vs_nn_gru():
    g = gen(6)
    n, b, t, i, h = 3, 2, 5, 4, 6
    mods = _gru_modules(n, i, h, 60)
    x = torch.randn(n, b, t, i, generator=g, dtype=torch.float64)
    h0 = torch.randn(n, b, h, generator=g, dtype=torch.float64)
    out, hn = wide_ref.gru(x, *_gru_params(mods), h_0=h0)
    for k in range(n):
        eo, eh = mods[k](x[k], h0[k].unsqueeze(0))
        assert torch.allclose(out[k], eo, atol=1e-12)
        assert torch.allclose(hn[k], eh[0], atol=1e-12)


def test_gru_single_step_closed_form():
    # T=1, h0=0: h = (1 - z) * n with r, z, n from the textbook equations
    g = gen(7)
    n, b, i, h = 2, 1, 3, 2
    wih = torch.randn(n, 3 * h, i, generator=g, dtype=torch.float64)
    whh = torch.randn(n, 3 * h, h, generator=g, dtype=torch.float64)
    bih = torch.randn(n, 3 * h, generator=g, dtype=torch.float64)
    bhh = torch.randn(n, 3 * h, generator=g, dtype=torch.float64)
    x = torch.randn(n, b, 1, i, generator=g, dtype=torch.float64)
    out, _ = wide_ref.gru(x, wih, whh, bih, bhh)
    for k in range(n):
        gx = wih[k] @ x[k, 0, 0] + bih[k]
        gh = bhh[k]
        r = torch.sigmoid(gx[:h] + gh[:h])
        z = torch.sigmoid(gx[h:2 * h] + gh[h:2 * h])
        nn_ = torch.tanh(gx[2 * h:] + r * gh[2 * h:])
        assert torch.allclose(out[k, 0, 0], (1 - z) * nn_, atol=1e-12)


def test_lstm_vs_nn_lstm():
    g = gen(8)
    n, b, t, i, h = 3, 2, 6, 5, 4
    torch.manual_seed(80)
    mods = [nn.LSTM(i, h, batch_first=True).double() for _ in range(n)]
    p = [torch.stack([getattr(m, k) for m in mods]).detach()
         for k in ("weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0")]
    x = torch.randn(n, b, t, i, generator=g, dtype=torch.float64)
    h0 = torch.randn(n, b, h, generator=g, dtype=torch.float64)
    c0 = torch.randn(n, b, h, generator=g, dtype=torch.float64)
    out, (hn, cn) = wide_ref.lstm(x, *p, hx=(h0, c0))
    for k in range(n):
        eo, (eh, ec) = mods[k](x[k], (h0[k].unsqueeze(0), c0[k].unsqueeze(0)))
        assert torch.allclose(out[k], eo, atol=1e-12)
        assert torch.allclose(hn[k], eh[0], atol=1e-12)
        assert torch.allclose(cn[k], ec[0], atol=1e-12)


# ----------------------------------------------------------------------------- attention
def _mha_params(mods):
    d = mods[0].embed_dim
    qw = torch.stack([m.in_proj_weight[:d] for m in mods]).detach()
    kvw = torch.stack([m.in_proj_weight[d:] for m in mods]).detach()
    qb = torch.stack([m.in_proj_bias[:d] for m in mods]).detach()
    kvb = torch.stack([m.in_proj_bias[d:] for m in mods]).detach()
    ow = torch.stack([m.out_proj.weight for m in mods]).detach()
    ob = torch.stack([m.out_proj.bias for m in mods]).detach()
    return qw, kvw, ow, qb, kvb, ob


@pytest.mark.parametrize("causal", [False, True])
def test_attention_vs_mha(causal):
    g = gen(9)
    n, b, t, d, hh = 2, 2, 5, 8, 2
    torch.manual_seed(90)
    mods = [nn.MultiheadAttention(d, hh, batch_first=True).double().eval() for _ in range(n)]
    for m in mods:  # non-zero biases so a dropped bias term fails
        with torch.no_grad():
            m.in_proj_bias.normal_()
            m.out_proj.bias.normal_()
    x = torch.randn(n, b, t, d, generator=g, dtype=torch.float64)
    qw, kvw, ow, qb, kvb, ob = _mha_params(mods)
    y = wide_ref.attention(x, x, x, qw, kvw, ow, qb, kvb, ob, hh, is_causal=causal)
    mask = torch.triu(torch.ones(t, t, dtype=torch.bool), 1) if causal else None
    for k in range(n):
        e, _ = mods[k](x[k], x[k], x[k], need_weights=False, attn_mask=mask)
        assert torch.allclose(y[k], e, atol=1e-10)


def test_attention_brute_softmax():
    g = gen(10)
    n, b, t, d, hh = 1, 1, 4, 4, 2
    x = torch.randn(n, b, t, d, generator=g, dtype=torch.float64)
    qw = torch.randn(n, d, d, generator=g, dtype=torch.float64)
    kvw = torch.randn(n, 2 * d, d, generator=g, dtype=torch.float64)
    ow = torch.randn(n, d, d, generator=g, dtype=torch.float64)
    y = wide_ref.attention(x, x, x, qw, kvw, ow, None, None, None, hh)
    q = x[0, 0] @ qw[0].T
    k = x[0, 0] @ kvw[0, :d].T
    v = x[0, 0] @ kvw[0, d:].T
    dh = d // hh
    heads = []
    for h in range(hh):
        s = q[:, h * dh:(h + 1) * dh] @ k[:, h * dh:(h + 1) * dh].T / math.sqrt(dh)
        p = torch.exp(s - s.max(dim=1, keepdim=True).values)
        p = p / p.sum(dim=1, keepdim=True)
        heads.append(p @ v[:, h * dh:(h + 1) * dh])
    exp = torch.cat(heads, dim=1) @ ow[0].T
    assert torch.allclose(y[0, 0], exp, atol=1e-10)


# ----------------------------------------------------------------------------- models
class _MLP(nn.Module):
    def __init__(self):
        super().__init__()
        self.fc1 = nn.Linear(6, 10)
        self.fc2 = nn.Linear(10, 4)

    def forward(self, x):
        return self.fc2(F.relu(self.fc1(x)))


def test_mlp_wide_vs_per_model():
    g = gen(11)
    n = 4
    torch.manual_seed(110)
    mods = [_MLP().double() for _ in range(n)]
    ins = [torch.randn(3, 6, generator=g, dtype=torch.float64) for _ in range(n)]
    st = lambda k: torch.stack([getattr(getattr(m, k.split('.')[0]), k.split('.')[1]) for m in mods]).detach()  # noqa
    y = wide_ref.mlp_wide(wide_ref.pack_inputs(ins), n, st("fc1.weight"), st("fc1.bias"), st("fc2.weight"),
                          st("fc2.bias"))
    for k, out in enumerate(wide_ref.unpack_outputs(y, n)):
        assert torch.allclose(out, mods[k](ins[k]), atol=1e-12)


class _ResBlock(nn.Module):
    def __init__(self, c=3):
        super().__init__()
        self.conv1 = nn.Conv2d(c, c, 3, padding=1)
        self.bn1 = nn.BatchNorm2d(c)
        self.conv2 = nn.Conv2d(c, c, 3, padding=1)
        self.bn2 = nn.BatchNorm2d(c)

    def forward(self, x):
        identity = x
        out = F.relu(self.bn1(self.conv1(x)))
        out = self.bn2(self.conv2(out))
        return F.relu(out + identity)


def resblock_params(mods):
    p = {}
    for name in ("conv1", "conv2"):
        p[f"{name}.weight"] = torch.cat([getattr(m, name).weight for m in mods]).detach()
        p[f"{name}.bias"] = torch.cat([getattr(m, name).bias for m in mods]).detach()
    for name in ("bn1", "bn2"):
        for k in ("weight", "bias", "running_mean", "running_var"):
            p[f"{name}.{k}"] = torch.cat([getattr(getattr(m, name), k) for m in mods]).detach()
        p[f"{name}.eps"] = getattr(mods[0], name).eps
    return p


def test_resblock_wide_vs_per_model():
    g = gen(12)
    n = 3
    torch.manual_seed(120)
    mods = [_ResBlock().double().eval() for _ in range(n)]
    for m in mods:
        with torch.no_grad():
            for bn in (m.bn1, m.bn2):
                bn.running_mean.normal_()
                bn.running_var.uniform_(0.5, 2.0)
                bn.weight.normal_(1.0, 0.1)
                bn.bias.normal_(0.0, 0.1)
    ins = [torch.randn(2, 3, 5, 5, generator=g, dtype=torch.float64) for _ in range(n)]
    y = wide_ref.resblock_wide(wide_ref.pack_inputs(ins), n, resblock_params(mods))
    for k, out in enumerate(wide_ref.unpack_outputs(y, n)):
        assert torch.allclose(out, mods[k](ins[k]), atol=1e-12)


# ----------------------------------------------------------------------------- planted mistakes
def test_seq_model_wide_vs_per_model():
    """The composed sequence model (per-model ids) against each torch.nn SeqModel in float64."""
    from wide_compiler.workloads import SeqModel, seq_params
    n, b, t, v, d, h = 3, 2, 5, 40, 16, 24
    mods = []
    for i in range(n):
        torch.manual_seed(400 + i)
        m = SeqModel(v, d, h).double()
        with torch.no_grad():
            m.ln.weight.normal_(1.0, 0.2)
            m.ln.bias.normal_(0.0, 0.2)
        mods.append(m)
    ids = torch.randint(0, v, (n, b, t), generator=gen(401))
    got = wide_ref.seq_model(ids, seq_params(mods))
    with torch.no_grad():
        for i in range(n):
            assert rel_err(got[i], mods[i](ids[i])) <= 1e-12


def test_planted_gru_gate_swap_is_caught():
    """Swapping r and z in a copy of the oracle's GRU must fail the nn.GRU pin."""
    def gru_swapped(x, wih, whh, bih, bhh):
        n, h = wih.shape[0], whh.shape[2]
        perm = torch.cat([torch.arange(h, 2 * h), torch.arange(0, h), torch.arange(2 * h, 3 * h)])
        return wide_ref.gru(x, wih[:, perm], whh[:, perm], bih[:, perm], bhh[:, perm])

    g = gen(13)
    mods = _gru_modules(2, 3, 4, 130)
    x = torch.randn(2, 2, 3, 3, generator=g, dtype=torch.float64)
    out, _ = gru_swapped(x, *_gru_params(mods))
    eo, _ = mods[0](x[0])
    assert not torch.allclose(out[0], eo, atol=1e-6)


def test_planted_layernorm_unbiased_var_is_caught():
    g = gen(14)
    x = torch.randn(1, 2, 6, generator=g, dtype=torch.float64)
    w, b = torch.ones(6, dtype=torch.float64), torch.zeros(6, dtype=torch.float64)
    mean = x.mean(-1, keepdim=True)
    wrong = (x - mean) / torch.sqrt(x.var(-1, unbiased=True, keepdim=True) + 1e-5)
    assert not torch.allclose(wrong[0], F.layer_norm(x[0], (6,), w, b, 1e-5), atol=1e-6)
    assert torch.allclose(wide_ref.layernorm(x, w, b, 1, 1e-5)[0], F.layer_norm(x[0], (6,), w, b, 1e-5))


def test_planted_linear_transpose_is_caught():
    g = gen(15)
    w = torch.randn(2, 4, 4, generator=g, dtype=torch.float64)
    x = torch.randn(2, 3, 4, generator=g, dtype=torch.float64)
    wrong = wide_ref.linear(x, w.transpose(1, 2), None)
    assert not torch.allclose(wrong[1], F.linear(x[1], w[1]), atol=1e-6)
    assert torch.allclose(wide_ref.linear(x, w, None)[1], F.linear(x[1], w[1]), atol=1e-12)
