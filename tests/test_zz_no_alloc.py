"""wc_rnn_forward_noalloc (workspace in the library's static per-device scratch) against
wc_rnn_forward (caller-provided workspace), both through the C ABI: the same kernels on the
same inputs, so outputs, h_n and c_n agree bit for bit.  Calls run back to back on one
device, each later one smaller than the one before, so a call that depended on scratch
contents left by the previous one would show here."""

import pytest
import torch
import torch.nn as nn

from tests._util import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(hip, cell, n, b, t, i, h, dtype, seed):
    g = gen(seed)
    torch.manual_seed(seed)
    cls = nn.LSTM if cell == hip.CELL_LSTM else nn.GRU
    mods = [cls(i, h, batch_first=True) for _ in range(n)]
    gates = 4 if cell == hip.CELL_LSTM else 3
    st = lambda k: torch.stack([getattr(m, k).detach() for m in mods]).to(DEV, dtype)  # noqa: E731
    w_ih, w_hh, b_ih, b_hh = st("weight_ih_l0"), st("weight_hh_l0"), st("bias_ih_l0"), st("bias_hh_l0")
    assert w_hh.shape == (n, gates * h, h)
    x = (torch.randn(n, b, t, i, generator=g)).to(DEV, dtype)
    h0 = (torch.randn(n, b, h, generator=g)).to(DEV, dtype)
    c0 = (torch.randn(n, b, h, generator=g)).to(DEV, dtype) if cell == hip.CELL_LSTM else None
    res = []
    for noalloc in (False, True):
        out = torch.full((n, b, t, h), float("nan"), device=DEV, dtype=dtype)
        hn = torch.full((n, b, h), float("nan"), device=DEV, dtype=dtype)
        cn = torch.full((n, b, h), float("nan"), device=DEV, dtype=dtype) if c0 is not None else None
        kw = dict(cell=cell, x=x, w_ih=w_ih, w_hh=w_hh, b_ih=b_ih, b_hh=b_hh, h0=h0, c0=c0, out=out,
                  h_n=hn, c_n=cn)
        (hip.rnn_forward_noalloc if noalloc else hip.rnn_forward)(**kw)
        torch.cuda.synchronize()
        res.append((out.cpu(), hn.cpu(), None if cn is None else cn.cpu()))
    (o0, h0_, c0_), (o1, h1_, c1_) = res
    assert not torch.isnan(o1).any()
    assert torch.equal(o0, o1) and torch.equal(h0_, h1_)
    if c0_ is not None:
        assert torch.equal(c0_, c1_)


def test_noalloc_matches_forward_calls_in_a_row(hip):
    assert hip.lib().wc_rnn_noalloc_scratch_bytes() == 64 << 20
    # partitioned on-chip LSTM (8 x 4 workgroups), then a smaller one (2 x 2), then the
    # register-resident GRU recurrence, then a smaller GRU
    _run(hip, hip.CELL_LSTM, 8, 16, 20, 64, 512, torch.bfloat16, 900)
    _run(hip, hip.CELL_LSTM, 2, 5, 7, 32, 256, torch.bfloat16, 901)
    _run(hip, hip.CELL_GRU, 32, 4, 32, 64, 128, torch.float32, 902)
    _run(hip, hip.CELL_GRU, 3, 2, 5, 8, 16, torch.float32, 903)


def test_noalloc_rejects_sizes_beyond_the_scratch(hip):
    n, b, t, i, h = 64, 16, 128, 256, 512        # the sequence model's LSTM: ~0.5 GB of workspace
    x = torch.empty(n, b, t, i, device=DEV, dtype=torch.bfloat16)
    w_ih = torch.empty(n, 4 * h, i, device=DEV, dtype=torch.bfloat16)
    w_hh = torch.empty(n, 4 * h, h, device=DEV, dtype=torch.bfloat16)
    out = torch.empty(n, b, t, h, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(hip.WideKernelError, match="static scratch"):
        hip.rnn_forward_noalloc(cell=hip.CELL_LSTM, x=x, w_ih=w_ih, w_hh=w_hh, b_ih=None, b_hh=None, h0=None,
                                c0=None, out=out, h_n=None, c_n=None)
