"""C-ABI checks that need no GPU: the library loads, exports every entry point declared in
include/wc_abi.h, and rejects bad arguments on the host with a negative status + message."""

import ctypes
import os
import re

import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "wc_abi.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wc_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "wc_rnn_forward" in names and "wc_grouped_gemm" in names and "wc_pack_rows" in names


def test_library_exports_every_declared_symbol(hip):
    lib = hip.lib()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares exactly the header's entry points
    assert sorted(hip.SIGNATURES) == _declared()


def test_abi_version(hip):
    assert hip.lib().wc_abi_version() == hip.ABI_VERSION


def test_null_args_rejected_on_host(hip):
    lib = hip.lib()
    assert lib.wc_rnn_forward(None, None) == -1
    assert "null" in hip.last_error()
    assert lib.wc_grouped_gemm(None, None) == -1


def test_bad_dtype_rejected_on_host(hip):
    a = hip._RnnArgs()
    a.cell, a.dtype = hip.CELL_GRU, 7
    a.n, a.batch, a.steps, a.input_size, a.hidden = 1, 1, 1, 1, 1
    assert hip.lib().wc_rnn_forward(ctypes.byref(a), None) == -3
    assert "dtype" in hip.last_error()


def test_rnn_limit_and_workspace_checks(hip):
    a = hip._RnnArgs()
    a.cell, a.dtype = hip.CELL_LSTM, hip.F32
    a.n, a.batch, a.steps, a.input_size, a.hidden = 2, 3, 4, 8, 16
    # fp32 gates_x [n, batch, steps, 4H] + fp32 cell state [n, batch, H]
    assert hip.lib().wc_rnn_workspace_bytes(ctypes.byref(a)) == (2 * 3 * 4 * 64 + 2 * 3 * 16) * 4
    a.x = a.w_ih = a.w_hh = a.out = 16  # never dereferenced: rejected before any launch
    a.workspace, a.workspace_bytes = 16, 8
    assert hip.lib().wc_rnn_forward(ctypes.byref(a), None) == -6
    assert "workspace" in hip.last_error()


def test_gemm_arg_checks(hip):
    g = hip._GemmArgs()
    g.dtype = g.out_dtype = g.bias_dtype = hip.F32
    g.n, g.m, g.o, g.k = 1, 4, 4, 4
    g.a = g.w = g.c = 16
    g.a_rows_inner = 0
    g.c_rows_inner = 4
    assert hip.lib().wc_grouped_gemm(ctypes.byref(g), None) == -6
    g.a_rows_inner = 4
    g.act = 9
    assert hip.lib().wc_grouped_gemm(ctypes.byref(g), None) == -6


def test_oversized_arguments_rejected_without_overflow(hip):
    """Sizes whose products do not fit are rejected, not wrapped (cases the sanitizer probe
    found: tests/test_abi_sanitized.py)."""
    lib = hip.lib()
    big = (1 << 63) - 1
    # packed filter count: -1 for sizes that cannot be counted
    assert lib.wc_conv_packed_weight_elems(1, 64, 64, 3, 3) == 64 * 9 * 64
    assert lib.wc_conv_packed_weight_elems(big, big, 64, 3, 3) == -1
    assert lib.wc_conv_packed_weight_elems(1, 1, (1 << 31) - 1, 1, 1) == -1
    # workspace of a problem with zero steps whose state buffers (n * batch * hidden) overflow
    a = hip._RnnArgs()
    a.cell, a.dtype = hip.CELL_LSTM, hip.F32
    a.n, a.batch, a.steps, a.input_size, a.hidden = 7 * ((1 << 31) - 1), 1, 0, 8, (1 << 31) - 1
    assert lib.wc_rnn_workspace_bytes(ctypes.byref(a)) == -1
    # a rows_inner of 2^32 was truncated to a zero divisor on the host (a SIGFPE)
    g = hip._GemmArgs()
    g.dtype = g.out_dtype = g.bias_dtype = hip.F32
    g.n, g.m, g.o, g.k = 1, 4, 4, 4
    g.a = g.w = g.c = 16
    g.a_rows_inner, g.c_rows_inner = 1 << 32, 4
    assert lib.wc_grouped_gemm(ctypes.byref(g), None) == -5
    assert "rows_inner" in hip.last_error()
    # row counts whose product overflows int64
    assert lib.wc_layernorm(16, 0, 0, 16, 16, 16, 0, 0, 1 << 62, 4, 8, ctypes.c_float(1e-5), hip.F32, hip.F32,
                            None) == -5
    # conv geometry beyond int32 (the output size formula itself would overflow)
    c = hip._ConvArgs()
    c.dtype = c.param_dtype = hip.F32
    c.n, c.batch, c.c_in, c.c_out, c.h, c.w, c.kh, c.kw = 1, 1, 4, 4, 8, 8, 3, 3
    c.stride_h = c.stride_w = c.dil_w = 1
    c.dil_h = big
    c.x = c.y = c.packed_weight = 16
    assert lib.wc_conv2d(ctypes.byref(c), None) == -5


def test_attention_arg_checks(hip):
    """wc_attention's host checks (pointers never dereferenced): head dims past what the kernel
    holds (256 for 16-bit types, 128 for fp32), a row of heads x head dim beyond 32-bit offsets,
    and pointers not aligned to the element size, each rejected before any launch."""
    lib = hip.lib()

    def args(dtype, heads, dh, base=256):
        a = hip._AttnArgs()
        a.dtype, a.nb, a.heads, a.sq, a.skv, a.head_dim, a.scale = dtype, 1, heads, 4, 4, dh, 1.0
        a.q = a.k = a.v = a.o = base
        for f in ("q", "k", "v", "o"):
            setattr(a, f + "_stride_nb", 4 * heads * dh)
            setattr(a, f + "_stride_s", heads * dh)
        return a

    for dtype, dh, limit in ((hip.BF16, 257, "256"), (hip.F16, 300, "256"), (hip.F32, 129, "128")):
        assert lib.wc_attention(ctypes.byref(args(dtype, 1, dh)), None) == -5, (dtype, dh)
        assert f"above {limit}" in hip.last_error()
    assert lib.wc_attention(ctypes.byref(args(hip.BF16, 1 << 24, 128)), None) == -5
    assert "heads x head dim" in hip.last_error()
    assert lib.wc_attention(ctypes.byref(args(hip.BF16, 2, 24, base=257)), None) == -4
    assert "aligned" in hip.last_error()


def test_empty_problems_are_noops(hip):
    lib = hip.lib()
    assert lib.wc_swap01(None, 0, 5, 0, 0, 16, None, None) == 0
    assert lib.wc_pack_rows(None, None, 0, 3, 8, None, None) == 0
    assert lib.wc_layernorm(None, 0, 0, None, None, None, 0, 0, 0, 4, 8, 1e-5, 0, 0, None) == 0


def test_package_never_imports_the_oracle():
    """The product path has no route to the CPU restatement: no package source names it."""
    import pathlib
    pkg = pathlib.Path(__file__).resolve().parents[1] / "pytorch-parallel-compiler_amd" / "wide_compiler"
    offenders = [str(p) for p in pkg.rglob("*.py")
                 if re.search(r"^\s*(from|import)\s+oracle\b", p.read_text(), re.M)]
    assert not offenders, offenders


def test_cpu_tensors_raise_without_touching_a_device():
    """Every primitive refuses CPU tensors (no CPU fallback)."""
    import torch
    import wide_compiler as wc
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        wc.WideLinear(2, 4, 3)(torch.zeros(2, 5, 4))
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        wc.WideLayerNorm(2, 4)(torch.zeros(2, 3, 4))


def test_mlp2_supported_rules(hip):
    s = hip.lib().wc_mlp2_supported
    assert s(hip.F32, 64, 128, 64) == 1
    assert s(hip.BF16, 64, 128, 64) == 1
    assert s(hip.F32, 32, 64, 16) == 1
    assert s(hip.BF16, 32, 64, 16) == 0          # bf16 rows need 64-element multiples
    assert s(hip.F32, 64, 96, 64) == 1 and s(hip.F32, 64, 80, 64) == 0
    assert s(hip.F32, 64, 128, 24) == 0          # out in whole 16-column tiles
    assert s(hip.F32, 64, 288, 64) == 0          # hidden and out at most 256
    assert s(hip.F32, 1024, 256, 256) == 0       # beyond 160 KB of LDS
    assert s(hip.F32, 64, 128, 64) == 1 and s(7, 64, 128, 64) == 0


def test_mlp2_arg_checks(hip):
    a = hip._Mlp2Args()
    a.dtype, a.n, a.m = hip.F32, 1, 4
    a.in_features, a.hidden, a.out_features = 64, 80, 64
    assert hip.lib().wc_mlp2(ctypes.byref(a), None) < 0
    assert "not supported" in hip.last_error()
    a.hidden = 128
    a.x = a.w1 = a.w2 = a.y = 16                 # never dereferenced: rejected before any launch
    a.x_rows_inner, a.y_rows_inner = 0, 4
    assert hip.lib().wc_mlp2(ctypes.byref(a), None) < 0
    assert "rows_inner" in hip.last_error()


def test_self_attention_arg_checks(hip):
    """wc_self_attention validates on the host before any launch (pointers never dereferenced)."""
    lib = hip.lib()
    assert lib.wc_self_attention(None, None) == -1
    a = hip._SelfAttnArgs()
    a.dtype, a.n, a.b, a.s, a.d_model, a.heads = hip.BF16, 2, 3, 64, 256, 8
    a.x = a.q_weight = a.kv_weight = a.o = 16
    a.x_stride_n, a.x_stride_b, a.x_stride_s = 3 * 64 * 256, 64 * 256, 256
    a.o_stride_nb, a.o_stride_s = 64 * 256, 256
    a.q_weight_stride_n, a.kv_weight_stride_n = 256 * 256, 512 * 256
    for field, value, code in (("dtype", hip.F32, -5), ("heads", 4, -5), ("s", 513, -5), ("d_model", 800, -5),
                               ("x", 18, -4), ("x_stride_s", 252, -4), ("x_stride_b", -1, -6)):
        old = getattr(a, field)
        setattr(a, field, value)
        assert lib.wc_self_attention(ctypes.byref(a), None) == code, field
        assert "wc_self_attention" in hip.last_error()
        setattr(a, field, old)
    a.n = 0
    assert lib.wc_self_attention(ctypes.byref(a), None) == 0
