"""The committed golden fixtures (tests/golden/*.npz, expected outputs from per-model torch.nn
modules in float64) against the oracle on the CPU and against the HIP path on the GPU."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import wide_ref
from tests._util import TOL_F32, rel_err

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DEV = "cuda"


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz")) as z:
        arr = {k: torch.from_numpy(z[k].copy()) for k in z.files if k != "meta"}
        meta = json.loads(str(z["meta"]))
    n = meta["n"]
    sd = [{k[len(f"m{i}."):]: v for k, v in arr.items() if k.startswith(f"m{i}.")} for i in range(n)]
    ins = {k[3:]: v for k, v in arr.items() if k.startswith("in.")}
    outs = {k[4:]: v for k, v in arr.items() if k.startswith("out.")}
    return meta, sd, ins, outs


def st(sd, key):
    return torch.stack([d[key] for d in sd])


def cat(sd, key):
    return torch.cat([d[key] for d in sd])


def modules(cls, sd, *args, **kw):
    mods = []
    for d in sd:
        m = cls(*args, **kw).double()
        m.load_state_dict(d)
        mods.append(m.eval())
    return mods


# ------------------------------------------------------------------------------- oracle (CPU)
EXACT = 1e-10


def test_golden_linear_oracle():
    _, sd, i, o = load("linear")
    assert rel_err(wide_ref.linear(i["x"], st(sd, "weight"), st(sd, "bias")), o["y"]) <= EXACT


def test_golden_conv_oracle():
    m, sd, i, o = load("conv2d")
    y = wide_ref.conv2d(i["x"], cat(sd, "weight"), cat(sd, "bias"), m["n"], stride=(2, 2), padding=(1, 1))
    assert rel_err(y, o["y"]) <= EXACT
    m, sd, i, o = load("conv1d")
    y = wide_ref.conv1d(i["x"], cat(sd, "weight"), cat(sd, "bias"), m["n"], padding=2, dilation=2)
    assert rel_err(y, o["y"]) <= EXACT


def test_golden_norm_oracle():
    m, sd, i, o = load("batchnorm2d")
    y = wide_ref.batchnorm_eval(i["x"], cat(sd, "weight"), cat(sd, "bias"), cat(sd, "running_mean"),
                                cat(sd, "running_var"), 1e-5, m["n"])
    assert rel_err(y, o["y"]) <= EXACT
    m, sd, i, o = load("layernorm")
    y = wide_ref.layernorm(i["x"], cat(sd, "weight"), cat(sd, "bias"), m["n"], 1e-5)
    assert rel_err(y, o["y"]) <= EXACT


def test_golden_embedding_oracle():
    _, sd, i, o = load("embedding")
    w = st(sd, "weight")
    assert torch.equal(wide_ref.embedding(w, i["ids"]), o["shared"])
    assert torch.equal(wide_ref.embedding_per_model(w, i["ids_per_model"]), o["per_model"])


def test_golden_rnn_oracle():
    _, sd, i, o = load("gru")
    p = [st(sd, k) for k in ("weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0")]
    out, hn = wide_ref.gru(i["x"], *p, h_0=i["h0"])
    assert rel_err(out, o["out"]) <= EXACT and rel_err(hn, o["h_n"]) <= EXACT
    _, sd, i, o = load("lstm")
    p = [st(sd, k) for k in ("weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0")]
    out, (hn, cn) = wide_ref.lstm(i["x"], *p, hx=(i["h0"], i["c0"]))
    assert rel_err(out, o["out"]) <= EXACT
    assert rel_err(hn, o["h_n"]) <= EXACT and rel_err(cn, o["c_n"]) <= EXACT


def test_golden_attention_oracle():
    m, sd, i, o = load("attention")
    d = m["embed"]
    w, b = st(sd, "in_proj_weight"), st(sd, "in_proj_bias")
    x = i["x"]
    y = wide_ref.attention(x, x, x, w[:, :d], w[:, d:], st(sd, "out_proj.weight"), b[:, :d], b[:, d:],
                           st(sd, "out_proj.bias"), m["heads"])
    assert rel_err(y, o["y"]) <= EXACT


def test_golden_models_oracle():
    m, sd, i, o = load("mlp")
    y = wide_ref.mlp_wide(i["packed"], m["n"], st(sd, "fc1.weight"), st(sd, "fc1.bias"), st(sd, "fc2.weight"),
                          st(sd, "fc2.bias"))
    assert rel_err(y, o["packed"]) <= EXACT
    m, sd, i, o = load("resblock")
    p = {k: cat(sd, k) for k in sd[0] if "num_batches" not in k}
    p["bn1.eps"] = p["bn2.eps"] = 1e-5
    assert rel_err(wide_ref.resblock_wide(i["packed"], m["n"], p), o["packed"]) <= EXACT
    m, sd, i, o = load("seq_model")
    p = {"emb.weight": st(sd, "emb.weight"), "ln.weight": cat(sd, "ln.weight"), "ln.bias": cat(sd, "ln.bias"),
         "ln.eps": 1e-5, "fc.weight": st(sd, "fc.weight"), "fc.bias": st(sd, "fc.bias")}
    for k in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
        p[f"lstm.{k}"] = st(sd, f"lstm.{k}_l0")
    assert rel_err(wide_ref.seq_model(i["ids"], p), o["logits"]) <= EXACT


# ------------------------------------------------------------------------------- HIP path (GPU)
def _f32(t):
    return t.float().to(DEV)


def _close(got, exp):
    assert rel_err(got.cpu(), exp) <= TOL_F32


@pytest.mark.gpu
def test_golden_primitives_hip(hip):
    import wide_compiler as wc
    with torch.no_grad():
        _, sd, i, o = load("linear")
        wide = wc.WideLinear.from_modules(modules(nn.Linear, sd, 5, 7)).to(DEV, torch.float32)
        _close(wide(_f32(i["x"])), o["y"])

        _, sd, i, o = load("conv2d")
        wide = wc.WideConv2d.from_modules(modules(nn.Conv2d, sd, 3, 4, 3, stride=2, padding=1)).to(DEV,
                                                                                                  torch.float32)
        _close(wide(_f32(i["x"])), o["y"])

        _, sd, i, o = load("conv1d")
        wide = wc.WideConv1d.from_modules(modules(nn.Conv1d, sd, 4, 5, 3, padding=2, dilation=2)).to(
            DEV, torch.float32)
        _close(wide(_f32(i["x"])), o["y"])

        _, sd, i, o = load("batchnorm2d")
        wide = wc.WideBatchNorm2d.from_modules(modules(nn.BatchNorm2d, sd, 4)).to(DEV, torch.float32).eval()
        _close(wide(_f32(i["x"])), o["y"])

        _, sd, i, o = load("layernorm")
        wide = wc.WideLayerNorm.from_modules(modules(nn.LayerNorm, sd, 8)).to(DEV, torch.float32)
        _close(wide(_f32(i["x"])), o["y"])

        _, sd, i, o = load("embedding")
        wide = wc.WideEmbedding.from_modules(modules(nn.Embedding, sd, 11, 6)).to(DEV, torch.float32)
        # a gather commutes with the float64 -> float32 rounding: bit-exact against the fixture
        assert torch.equal(wide(i["ids"].to(DEV)).cpu(), o["shared"].float())
        assert torch.equal(wide(i["ids_per_model"].to(DEV), per_model=True).cpu(), o["per_model"].float())
        wide.index_error()


@pytest.mark.gpu
def test_golden_recurrent_hip(hip):
    import wide_compiler as wc
    with torch.no_grad():
        _, sd, i, o = load("gru")
        wide = wc.WideGRU.from_modules(modules(nn.GRU, sd, 5, 6, batch_first=True)).to(DEV, torch.float32)
        out, hn = wide(_f32(i["x"]), _f32(i["h0"]))
        for t in range(out.shape[2]):
            _close(out[:, :, t], o["out"][:, :, t])
        _close(hn, o["h_n"])
        _, sd, i, o = load("lstm")
        wide = wc.WideLSTM.from_modules(modules(nn.LSTM, sd, 5, 6, batch_first=True)).to(DEV, torch.float32)
        out, (hn, cn) = wide(_f32(i["x"]), (_f32(i["h0"]), _f32(i["c0"])))
        for t in range(out.shape[2]):
            _close(out[:, :, t], o["out"][:, :, t])
        _close(hn, o["h_n"])
        _close(cn, o["c_n"])


@pytest.mark.gpu
def test_golden_attention_hip(hip):
    import wide_compiler as wc
    m, sd, i, o = load("attention")
    mods = modules(nn.MultiheadAttention, sd, m["embed"], m["heads"], batch_first=True)
    wide = wc.WideAttention.from_modules(mods).to(DEV, torch.float32).eval()
    with torch.no_grad():
        _close(wide(_f32(i["x"])), o["y"])


@pytest.mark.gpu
def test_golden_models_hip(hip):
    import wide_compiler as wc
    from wide_compiler.workloads import MLP, ResBlock, SeqModel, WideSeqModel
    with torch.no_grad():
        m, sd, i, o = load("mlp")
        mods = [x.float().to(DEV) for x in modules(MLP, sd)]
        x = _f32(i["packed"])
        wide = wc.compile(mods, x[:, :64]).eval()
        _close(wide(x), o["packed"])

        m, sd, i, o = load("resblock")
        mods = [x.float().to(DEV) for x in modules(ResBlock, sd, 4)]
        x = _f32(i["packed"])
        wide = wc.compile(mods, x[:, :4]).eval()
        _close(wide(x), o["packed"])

        m, sd, i, o = load("seq_model")
        mods = [x.float().to(DEV) for x in modules(SeqModel, sd, 16, 8, 12)]
        wide = WideSeqModel(mods)
        _close(wide(i["ids"].to(DEV)), o["logits"])
