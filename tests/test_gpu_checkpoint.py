"""Reference-layout checkpoints through the HIP forward.

A state_dict in the reference's on-disk format is assembled from per-model torch.nn modules,
loaded with strict=True into a freshly (differently) initialised wide primitive, and the HIP
forward of that primitive is checked against the oracle run on the original modules'
weights:
  * WideLSTM: block-diagonal weight_ih [N*4H, N*I] / weight_hh [N*4H, N*H] and flat biases
    (wide_lstm.py:101-109), bf16 at hidden 512 (the partitioned on-chip kernel's shape);
  * WideConv1d: the grouped strategy's ``op.*`` keys (wide_conv1d.py:84-101), loaded into both
    strategies' modules;
  * WideLinear and WideAttention (wide_linear.py:113-118, wide_attention.py:96-114)."""

import pytest
import torch
import torch.nn as nn

from oracle import wide_ref
from tests._util import TOL_BF16, gen, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _block_diag(blocks):
    return torch.block_diag(*[b.detach() for b in blocks])


def test_lstm_block_diagonal_checkpoint_runs_partitioned_kernel(hip):
    import wide_compiler as wc
    n, b, t, i, h = 6, 16, 24, 64, 512
    torch.manual_seed(700)
    mods = [nn.LSTM(i, h, batch_first=True).to(torch.bfloat16) for _ in range(n)]
    sd = {"weight_ih": _block_diag([m.weight_ih_l0 for m in mods]),
          "weight_hh": _block_diag([m.weight_hh_l0 for m in mods]),
          "bias_ih": torch.cat([m.bias_ih_l0.detach() for m in mods]),
          "bias_hh": torch.cat([m.bias_hh_l0.detach() for m in mods])}
    assert sd["weight_hh"].shape == (n * 4 * h, n * h)
    torch.manual_seed(701)
    fresh = wc.WideLSTM.from_modules([nn.LSTM(i, h, batch_first=True).to(torch.bfloat16) for _ in range(n)])
    fresh.load_state_dict(sd, strict=True)
    fresh = fresh.to(DEV)
    x = torch.randn(n, b, t, i, generator=gen(702)).to(torch.bfloat16)
    with torch.no_grad():
        out, (hn, cn) = fresh(x.to(DEV))
    hip.rnn_sync_check(block=True)
    st = lambda k: torch.stack([getattr(m, k).detach() for m in mods]).double()  # noqa: E731
    eo, (eh, ec) = wide_ref.lstm(x.double(), st("weight_ih_l0"), st("weight_hh_l0"), st("bias_ih_l0"),
                                 st("bias_hh_l0"))
    out = out.cpu()
    errs = [rel_err(out[:, :, s], eo[:, :, s]) for s in range(t)]
    assert max(errs) <= TOL_BF16, errs
    assert rel_err(hn.cpu(), eh) <= TOL_BF16 and rel_err(cn.cpu(), ec) <= TOL_BF16


@pytest.mark.parametrize("into", ["GROUPED", "SEQUENTIAL"])
def test_conv1d_op_checkpoint(hip, into):
    import wide_compiler as wc
    from wide_compiler.core.primitives.wide_conv1d import Conv1dStrategy
    n, b, ci, co, ln = 12, 4, 64, 128, 256
    torch.manual_seed(710)
    mods = [nn.Conv1d(ci, co, 3, padding=1).to(torch.bfloat16) for _ in range(n)]
    sd = {"op.weight": torch.cat([m.weight.detach() for m in mods]),
          "op.bias": torch.cat([m.bias.detach() for m in mods])}
    torch.manual_seed(711)
    fresh = wc.WideConv1d.from_modules([nn.Conv1d(ci, co, 3, padding=1).to(torch.bfloat16) for _ in range(n)],
                                       strategy=Conv1dStrategy.GROUPED)
    fresh.load_state_dict(sd, strict=True)
    if into == "SEQUENTIAL":
        seq = wc.WideConv1d.from_modules([nn.Conv1d(ci, co, 3, padding=1).to(torch.bfloat16) for _ in range(n)],
                                         strategy=Conv1dStrategy.SEQUENTIAL)
        seq.load_state_dict(fresh.state_dict(), strict=True)
        fresh = seq
    fresh = fresh.to(DEV)
    x = torch.randn(n, b, ci, ln, generator=gen(712)).to(torch.bfloat16)
    with torch.no_grad():
        y = fresh(x.to(DEV)).cpu()
    exact = wide_ref.conv1d(x.double(), sd["op.weight"].double(), sd["op.bias"].double(), n, padding=1)
    assert rel_err(y, exact) <= TOL_BF16


def test_linear_and_attention_checkpoints(hip):
    import wide_compiler as wc
    n = 5
    torch.manual_seed(720)
    lin = [nn.Linear(96, 160).to(torch.bfloat16) for _ in range(n)]
    sd = {"weight": torch.stack([m.weight.detach() for m in lin]), "bias": torch.stack([m.bias.detach() for m in lin])}
    fresh = wc.WideLinear.from_modules([nn.Linear(96, 160).to(torch.bfloat16) for _ in range(n)])
    fresh.load_state_dict(sd, strict=True)
    x = torch.randn(n, 33, 96, generator=gen(721)).to(torch.bfloat16)
    with torch.no_grad():
        y = fresh.to(DEV)(x.to(DEV)).cpu()
    assert rel_err(y, wide_ref.linear(x.double(), sd["weight"].double(), sd["bias"].double())) <= TOL_BF16

    d, heads = 256, 8
    mha = [nn.MultiheadAttention(d, heads, batch_first=True) for _ in range(n)]
    for m in mha:
        with torch.no_grad():
            m.in_proj_bias.normal_(0, 0.1)
            m.out_proj.bias.normal_(0, 0.1)
    mha = [m.to(torch.bfloat16).eval() for m in mha]
    sd = {"q_weight": torch.stack([m.in_proj_weight[:d].detach() for m in mha]),
          "kv_weight": torch.stack([m.in_proj_weight[d:].detach() for m in mha]),
          "out_weight": torch.stack([m.out_proj.weight.detach() for m in mha]),
          "q_bias": torch.stack([m.in_proj_bias[:d].detach() for m in mha]),
          "kv_bias": torch.stack([m.in_proj_bias[d:].detach() for m in mha]),
          "out_bias": torch.stack([m.out_proj.bias.detach() for m in mha])}
    fresh = wc.WideAttention.from_modules([nn.MultiheadAttention(d, heads, batch_first=True).to(torch.bfloat16)
                                           for _ in range(n)])
    fresh.load_state_dict(sd, strict=True)
    x = torch.randn(n, 2, 128, d, generator=gen(722)).to(torch.bfloat16)
    with torch.no_grad():
        y = fresh.to(DEV).eval()(x.to(DEV)).cpu()
    c = {k: v.double() for k, v in sd.items()}
    xd = x.double()
    exact = wide_ref.attention(xd, xd, xd, c["q_weight"], c["kv_weight"], c["out_weight"], c["q_bias"],
                               c["kv_bias"], c["out_bias"], heads)
    assert rel_err(y, exact) <= TOL_BF16
