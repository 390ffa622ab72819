"""Checkpoint compatibility on the CPU (no kernels run): every wide primitive's state_dict has
the reference's keys and shapes (the de-facto on-disk format: wide_linear.py:113-118,
wide_conv2d.py:149-158, wide_conv1d.py:80-105, wide_batchnorm_2d.py:45-51,
wide_layernorm.py:38-39, wide_embedding.py:74, wide_attention.py:96-114, wide_gru.py:99-109,
wide_lstm.py:101-109), a reference-layout dict assembled here from the per-model torch.nn
modules loads with strict=True into a freshly initialised primitive and reproduces the
from_modules parameters, and save -> load round-trips."""

import pytest
import torch
import torch.nn as nn

import wide_compiler as wc
from wide_compiler.core.primitives.wide_conv1d import Conv1dStrategy

N = 3


def _block_diag(blocks):
    rows = sum(b.shape[0] for b in blocks)
    cols = sum(b.shape[1] for b in blocks)
    full = torch.zeros(rows, cols, dtype=blocks[0].dtype)
    r = c = 0
    for b in blocks:
        full[r:r + b.shape[0], c:c + b.shape[1]] = b
        r += b.shape[0]
        c += b.shape[1]
    return full


def _reference_dicts():
    """(wide class, per-model modules, reference-layout state_dict, from_modules kwargs)."""
    torch.manual_seed(7)
    cases = []
    lin = [nn.Linear(5, 6) for _ in range(N)]
    cases.append((wc.WideLinear, lin, {"weight": torch.stack([m.weight for m in lin]),
                                       "bias": torch.stack([m.bias for m in lin])}, {}))
    c2 = [nn.Conv2d(4, 6, 3, padding=1) for _ in range(N)]
    cases.append((wc.WideConv2d, c2, {"grouped_conv.weight": torch.cat([m.weight for m in c2]),
                                      "grouped_conv.bias": torch.cat([m.bias for m in c2])}, {}))
    c1 = [nn.Conv1d(4, 6, 3, padding=1) for _ in range(N)]
    cases.append((wc.WideConv1d, c1, {"weight": torch.stack([m.weight for m in c1]),
                                      "bias": torch.stack([m.bias for m in c1])}, {}))
    cases.append((wc.WideConv1d, c1, {"op.weight": torch.cat([m.weight for m in c1]),
                                      "op.bias": torch.cat([m.bias for m in c1])},
                  {"strategy": Conv1dStrategy.GROUPED}))
    bn = [nn.BatchNorm2d(4).eval() for _ in range(N)]
    for m in bn:
        with torch.no_grad():
            m.weight.normal_()
            m.bias.normal_()
            m.running_mean.normal_()
            m.running_var.uniform_(0.5, 2)
    cases.append((wc.WideBatchNorm2d, bn, {f"op.{k}": torch.cat([getattr(m, k) for m in bn])
                                           for k in ("weight", "bias", "running_mean", "running_var")}
                  | {"op.num_batches_tracked": torch.tensor(0)}, {}))
    ln = [nn.LayerNorm(6) for _ in range(N)]
    for m in ln:
        with torch.no_grad():
            m.weight.normal_()
            m.bias.normal_()
    cases.append((wc.WideLayerNorm, ln, {"weight": torch.cat([m.weight for m in ln]),
                                         "bias": torch.cat([m.bias for m in ln])}, {}))
    emb = [nn.Embedding(10, 6) for _ in range(N)]
    cases.append((wc.WideEmbedding, emb, {"weight": torch.stack([m.weight for m in emb])}, {}))
    mha = [nn.MultiheadAttention(8, 2, batch_first=True) for _ in range(N)]
    for m in mha:
        with torch.no_grad():
            m.in_proj_bias.normal_()
            m.out_proj.bias.normal_()
    d = 8
    cases.append((wc.WideAttention, mha, {
        "q_weight": torch.stack([m.in_proj_weight[:d] for m in mha]),
        "kv_weight": torch.stack([m.in_proj_weight[d:] for m in mha]),
        "out_weight": torch.stack([m.out_proj.weight for m in mha]),
        "q_bias": torch.stack([m.in_proj_bias[:d] for m in mha]),
        "kv_bias": torch.stack([m.in_proj_bias[d:] for m in mha]),
        "out_bias": torch.stack([m.out_proj.bias for m in mha])}, {}))
    gru = [nn.GRU(5, 4, batch_first=True) for _ in range(N)]
    cases.append((wc.WideGRU, gru, {k: torch.stack([getattr(m, k + "_l0") for m in gru])
                                    for k in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")}, {}))
    lstm = [nn.LSTM(5, 4, batch_first=True) for _ in range(N)]
    cases.append((wc.WideLSTM, lstm, {
        "weight_ih": _block_diag([m.weight_ih_l0 for m in lstm]),
        "weight_hh": _block_diag([m.weight_hh_l0 for m in lstm]),
        "bias_ih": torch.cat([m.bias_ih_l0 for m in lstm]),
        "bias_hh": torch.cat([m.bias_hh_l0 for m in lstm])}, {}))
    return [(cls, mods, {k: v.detach().clone() for k, v in sd.items()}, kw) for cls, mods, sd, kw in cases]


CASES = _reference_dicts()
IDS = [f"{c[0].__name__}-{'-'.join(sorted(c[2]))[:20]}" for c in CASES]


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_state_dict_has_reference_keys_and_shapes(case):
    cls, mods, ref_sd, kw = case
    if cls is wc.WideConv1d and "weight" in ref_sd:
        kw = {"strategy": Conv1dStrategy.SEQUENTIAL}
    wide = cls.from_modules(mods, **kw)
    sd = wide.state_dict()
    assert set(sd) == set(ref_sd), (sorted(sd), sorted(ref_sd))
    for k, v in ref_sd.items():
        assert tuple(sd[k].shape) == tuple(v.shape), k
        assert torch.equal(sd[k], v), k


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_reference_layout_dict_loads_and_round_trips(case):
    cls, mods, ref_sd, kw = case
    built = cls.from_modules(mods, **kw)
    fresh = cls.from_modules([type(m)(*_ctor_args(m)) for m in mods], **kw)   # other random init
    fresh.load_state_dict(ref_sd, strict=True)
    for (k1, p1), (k2, p2) in zip(built.named_parameters(), fresh.named_parameters()):
        assert k1 == k2 and torch.equal(p1, p2), k1
    again = cls.from_modules([type(m)(*_ctor_args(m)) for m in mods], **kw)
    again.load_state_dict(fresh.state_dict(), strict=True)
    for k, v in fresh.state_dict().items():
        assert torch.equal(again.state_dict()[k], v), k


def _ctor_args(m):
    if isinstance(m, nn.Linear):
        return (m.in_features, m.out_features)
    if isinstance(m, (nn.Conv1d, nn.Conv2d)):
        return (m.in_channels, m.out_channels, m.kernel_size, m.stride, m.padding)
    if isinstance(m, nn.BatchNorm2d):
        return (m.num_features,)
    if isinstance(m, nn.LayerNorm):
        return (m.normalized_shape,)
    if isinstance(m, nn.Embedding):
        return (m.num_embeddings, m.embedding_dim)
    if isinstance(m, nn.MultiheadAttention):
        return (m.embed_dim, m.num_heads, 0.0, True, False, False, None, None, True)
    if isinstance(m, (nn.GRU, nn.LSTM)):
        return (m.input_size, m.hidden_size, 1, True, True)
    raise TypeError(type(m))


def test_lstm_checkpoint_is_block_diagonal():
    _, mods, ref_sd, _ = next(c for c in CASES if c[0] is wc.WideLSTM)
    sd = wc.WideLSTM.from_modules(mods).state_dict()
    w = sd["weight_hh"]
    g, h = 16, 4
    for i in range(N):
        for j in range(N):
            blk = w[i * g:(i + 1) * g, j * h:(j + 1) * h]
            assert torch.equal(blk, mods[i].weight_hh_l0.detach()) if i == j else not blk.any()


def test_conv1d_checkpoint_crosses_strategies():
    """A checkpoint of either reference strategy loads into either strategy's module."""
    _, mods, _, _ = CASES[2]
    grouped = wc.WideConv1d.from_modules(mods, strategy=Conv1dStrategy.GROUPED)
    seq = wc.WideConv1d.from_modules([nn.Conv1d(4, 6, 3, padding=1) for _ in range(N)],
                                     strategy=Conv1dStrategy.SEQUENTIAL)
    seq.load_state_dict(grouped.state_dict(), strict=True)
    assert torch.equal(seq.weight.reshape(-1), grouped.op.weight.reshape(-1))
    back = wc.WideConv1d.from_modules([nn.Conv1d(4, 6, 3, padding=1) for _ in range(N)],
                                      strategy=Conv1dStrategy.GROUPED)
    back.load_state_dict(seq.state_dict(), strict=True)
    assert torch.equal(back.op.weight, grouped.op.weight) and torch.equal(back.op.bias, grouped.op.bias)
