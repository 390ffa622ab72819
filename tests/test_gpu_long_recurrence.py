"""Long sequences through the partitioned on-chip recurrences (GPU): 1024 steps, 8x the sequence
model's 128, so the exchange's step tags, slot parity and step base run through many periods in one
launch.  Reference: every model's torch.nn.LSTM / GRU in fp64 (wide_lstm.py:205-229 and
wide_gru.py:181-205 restate exactly those recurrences per model); bar: the suite's bf16 bar at
every timestep (normwise), and on the final states."""

import pytest
import torch
import torch.nn as nn

from tests._util import TOL_BF16, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("kind,hidden", [("lstm", 512), ("gru", 256), ("gru", 512)])
def test_partitioned_recurrence_1024_steps(hip, kind, hidden):
    import wide_compiler as wc
    from wide_compiler import _hip
    n, b, t, i = 2, 16, 1024, 64
    torch.manual_seed(hidden + (1 if kind == "gru" else 0))
    cls, wcls = (nn.LSTM, wc.WideLSTM) if kind == "lstm" else (nn.GRU, wc.WideGRU)
    mods = [cls(i, hidden, batch_first=True) for _ in range(n)]
    wide = wcls.from_modules(mods).to(DEV, torch.bfloat16)
    x = (torch.randn(n, b, t, i, device=DEV) * 0.5).to(torch.bfloat16)
    with torch.no_grad():
        out, state = wide(x)
        _hip.rnn_sync_check(block=True)
        # the modules' weights as the wide module holds them (bf16), in fp64
        refs = []
        for q, m in enumerate(mods):
            m = m.to(DEV).double()
            for name in ("weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0"):
                getattr(m, name).copy_(getattr(wide, name[:-3])[q].double())
            refs.append(m(x[q].double()))
    ref_out = torch.stack([r[0] for r in refs])
    errs = [rel_err(out[:, :, s], ref_out[:, :, s]) for s in range(t)]
    assert max(errs) <= TOL_BF16, (max(errs), errs.index(max(errs)))
    if kind == "lstm":
        assert rel_err(state[0], torch.stack([r[1][0][0] for r in refs])) <= TOL_BF16
        assert rel_err(state[1], torch.stack([r[1][1][0] for r in refs])) <= TOL_BF16
    else:
        assert rel_err(state, torch.stack([r[1][0] for r in refs])) <= TOL_BF16
