"""The partitioned on-chip LSTM (bf16, hidden 256 / 384 / 512) under graph capture and when its
bounded cross-workgroup waits give up.

A give-up is forced from the host: wc_rnn_set_spin_limit(0) makes every wait give up before
its first poll, so every workgroup records the status word and leaves normally (no kernel is
made to hang).  The verdict must reach the caller in each way the layer runs: an eager call,
replays of a captured graph, and the no-alloc entry point."""

import pytest
import torch
import torch.nn as nn

from oracle import wide_ref
from tests._util import TOL_BF16, gen, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _wide_lstm(n, i, h, seed):
    import wide_compiler as wc
    torch.manual_seed(seed)
    mods = [nn.LSTM(i, h, batch_first=True) for _ in range(n)]
    return wc.WideLSTM.from_modules(mods).to(DEV, torch.bfloat16)


def _x(shape, seed):
    return torch.randn(shape, generator=gen(seed)).to(torch.bfloat16).to(DEV)


def test_captured_lstm_replays_match_eager_bit_for_bit(hip):
    """torch.cuda.graph capture of a partitioned WideLSTM (8 models, hidden 512, bf16): four
    replays on new inputs copied into the captured input buffer, with eager forwards between
    the replays, each equal to the eager forward of the same input bit for bit, and the status
    word clear after every replay."""
    n, b, t, i, h = 8, 16, 40, 64, 512
    wide = _wide_lstm(n, i, h, 611)
    static_x = _x((n, b, t, i), 612)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.no_grad():
        wide(static_x)                                   # warm-up, outside the capture
    torch.cuda.current_stream().wait_stream(s)
    hip.rnn_sync_check(block=True)
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        g_out, (g_hn, g_cn) = wide(static_x)
    for k in range(4):
        xk = _x((n, b, t, i), 620 + k)
        static_x.copy_(xk)
        graph.replay()
        torch.cuda.synchronize()
        hip.rnn_sync_check(block=True)
        with torch.no_grad():
            e_out, (e_hn, e_cn) = wide(xk)
        hip.rnn_sync_check(block=True)
        assert torch.equal(g_out, e_out) and torch.equal(g_hn, e_hn) and torch.equal(g_cn, e_cn), k
    # and the eager result is the LSTM's (per timestep, against the fp64 oracle)
    p = [getattr(wide, a).detach().cpu().double() for a in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
    eo, _ = wide_ref.lstm(xk.cpu().double(), *p)
    assert max(rel_err(e_out.cpu()[:, :, s_], eo[:, :, s_]) for s_ in range(t)) <= TOL_BF16


def test_give_up_is_raised_in_every_mode(hip):
    n, b, t, i, h = 4, 8, 12, 32, 512
    wide = _wide_lstm(n, i, h, 630)
    x = _x((n, b, t, i), 631)
    w = dict(cell=hip.CELL_LSTM, x=x, w_ih=wide.weight_ih.detach(), w_hh=wide.weight_hh.detach(),
             b_ih=wide.bias_ih.detach(), b_hh=wide.bias_hh.detach(), h0=None, c0=None)
    with torch.no_grad():
        ref_out, _ = wide(x)                             # a clean run first
    hip.rnn_sync_check(block=True)
    ref_out = ref_out.clone()
    prev = hip.rnn_set_spin_limit(0)
    try:
        # eager
        with torch.no_grad():
            wide(x)
        with pytest.raises(hip.WideKernelError, match="gave up"):
            hip.rnn_sync_check(block=True)
        hip.rnn_sync_check(block=True)                   # reported once, then cleared
        # graph replays: the capture keeps the spin limit it was captured with
        graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(graph):
            wide(x)
        hip.rnn_set_spin_limit(prev)
        for _ in range(2):
            graph.replay()
            with pytest.raises(hip.WideKernelError, match="gave up"):
                hip.rnn_sync_check(block=True)
        del graph
        # the no-alloc entry point
        hip.rnn_set_spin_limit(0)
        out = torch.empty(n, b, t, h, device=DEV, dtype=torch.bfloat16)
        hip.rnn_forward_noalloc(out=out, h_n=None, c_n=None, **w)
        with pytest.raises(hip.WideKernelError, match="gave up"):
            hip.rnn_sync_check(block=True)
    finally:
        hip.rnn_set_spin_limit(-1)
    assert hip.rnn_set_spin_limit(-1) == 1 << 21
    # with the default limit the layer runs clean again, and equals the first run
    with torch.no_grad():
        again, _ = wide(x)
    hip.rnn_sync_check(block=True)
    assert torch.equal(again, ref_out)
    out = torch.empty(n, b, t, h, device=DEV, dtype=torch.bfloat16)
    hip.rnn_forward_noalloc(out=out, h_n=None, c_n=None, **w)
    hip.rnn_sync_check(block=True)
    assert torch.equal(out, ref_out)


@pytest.mark.parametrize("cell,dtype,n,b,h,part", [
    ("lstm", torch.bfloat16, 64, 16, 512, True), ("lstm", torch.bfloat16, 70, 33, 512, True),
    ("lstm", torch.float16, 3, 20, 256, True), ("gru", torch.bfloat16, 8, 16, 512, True),
    ("gru", torch.float16, 2, 40, 384, True), ("gru", torch.bfloat16, 4, 4, 128, False),
    ("lstm", torch.float32, 2, 4, 512, False), ("gru", torch.bfloat16, 2, 4, 288, False)])
def test_partitioned_plan_is_taken(hip, cell, dtype, n, b, h, part):
    """Which sizes run the partitioned on-chip recurrence (a status word exists only there):
    LSTM and GRU, bf16 and fp16, hidden 256 / 384 / 512, any batch and any number of models."""
    import ctypes
    x = torch.empty(n, b, 3, 8, device=DEV, dtype=dtype)
    g = (4 if cell == "lstm" else 3) * h
    a, _ = hip.rnn_args(cell=hip.CELL_LSTM if cell == "lstm" else hip.CELL_GRU, x=x,
                        w_ih=torch.empty(n, g, 8, device=DEV, dtype=dtype),
                        w_hh=torch.empty(n, g, h, device=DEV, dtype=dtype), b_ih=None, b_hh=None, h0=None,
                        c0=None, out=torch.empty(n, b, 3, h, device=DEV, dtype=dtype), h_n=None, c_n=None,
                        allocate=False)
    assert (hip.lib().wc_rnn_status_offset(ctypes.byref(a)) >= 0) == part


def test_partitioned_lstm_repeated_launches_bit_identical(hip):
    """The partitioned LSTM at the sequence workload's size (64 models x 16 rows = 256
    workgroups, hidden 512, bf16), its recurrence launched four more times on the same gates
    without re-preparing the workspace (the exchange tag base advances across launches, the
    slots keep the previous launch's last values), then a whole forward again: every launch's
    output equals the first forward's bit for bit.  Tolerance tests cannot see a race in the
    h_t exchange that changes a few values; this one does."""
    from wide_compiler import _hip
    n, b, t, i, h = 64, 16, 128, 256, 512
    wide = _wide_lstm(n, i, h, 631)
    x = _x((n, b, t, i), 632)
    with torch.no_grad():
        ref, _ = wide(x)
        _hip.rnn_sync_check(block=True)
        ref = ref.clone()
        out = torch.empty_like(ref)
        a, ws = _hip.rnn_args(cell=_hip.CELL_LSTM, x=x, w_ih=wide.weight_ih, w_hh=wide.weight_hh,
                              b_ih=wide.bias_ih, b_hh=wide.bias_hh, h0=None, c0=None, out=out, h_n=None,
                              c_n=None, status=_hip.rnn_status_word(x.device))
        _hip.rnn_phase(a, "input_projection", x)
        for k in range(4):
            out.fill_(float("nan"))
            _hip.rnn_phase(a, "recurrence", x)
            _hip.rnn_sync_check(block=True)
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"launch {k}"
        again, _ = wide(x)
        _hip.rnn_sync_check(block=True)
    assert torch.equal(again.view(torch.int16), ref.view(torch.int16))
