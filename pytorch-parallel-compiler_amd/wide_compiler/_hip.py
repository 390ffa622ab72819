"""
ctypes binding of libwide_hip.so, the gfx950 kernels behind every wide primitive.

The library exposes a plain C ABI (see include/wc_abi.h at the repository root).  This
module loads it once, declares the entry points, and offers thin Python wrappers that

  * check that every tensor lives on a ROCm device, has the dtype / shape / inner
    contiguity the kernel needs, and that no autograd graph is requested (the kernels
    are forward-only);
  * pass raw device pointers, sizes and strides plus torch's current HIP stream;
  * turn a non-zero status into an exception carrying ``wc_last_error()``.

There is no CPU path and no fallback: when the library is missing, or a tensor is on
the CPU, the call raises.
"""

from __future__ import annotations

import ctypes
import os
from typing import Dict, List, Optional, Sequence

import torch
from torch import Tensor

ABI_VERSION = 5

F32, BF16, F16 = 0, 1, 2
ACT_NONE, ACT_RELU = 0, 1
CELL_GRU, CELL_LSTM = 0, 1
ERR_LIMIT = -5                  # WC_ERR_LIMIT: a size or layout the kernel does not take

_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libwide_hip.so")

_lib = None


class WideKernelError(RuntimeError):
    """A libwide_hip.so entry point returned a non-zero status."""


class _RnnArgs(ctypes.Structure):
    _fields_ = [
        ("cell", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("n", ctypes.c_int64), ("batch", ctypes.c_int64), ("steps", ctypes.c_int64),
        ("input_size", ctypes.c_int64), ("hidden", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("x_stride_n", ctypes.c_int64), ("x_stride_b", ctypes.c_int64), ("x_stride_t", ctypes.c_int64),
        ("w_ih", ctypes.c_void_p), ("w_hh", ctypes.c_void_p),
        ("b_ih", ctypes.c_void_p), ("b_hh", ctypes.c_void_p),
        ("h0", ctypes.c_void_p), ("c0", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("h_n", ctypes.c_void_p), ("c_n", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("status", ctypes.c_void_p),
    ]


class _GemmArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("out_dtype", ctypes.c_int32),
        ("bias_dtype", ctypes.c_int32), ("act", ctypes.c_int32),
        ("n", ctypes.c_int64), ("m", ctypes.c_int64), ("o", ctypes.c_int64), ("k", ctypes.c_int64),
        ("a", ctypes.c_void_p),
        ("a_stride_n", ctypes.c_int64), ("a_stride_outer", ctypes.c_int64),
        ("a_stride_inner", ctypes.c_int64), ("a_rows_inner", ctypes.c_int64),
        ("w", ctypes.c_void_p), ("w_stride_n", ctypes.c_int64),
        ("bias", ctypes.c_void_p), ("bias_stride_n", ctypes.c_int64),
        ("residual", ctypes.c_void_p),
        ("r_stride_n", ctypes.c_int64), ("r_stride_outer", ctypes.c_int64), ("r_stride_inner", ctypes.c_int64),
        ("c", ctypes.c_void_p),
        ("c_stride_n", ctypes.c_int64), ("c_stride_outer", ctypes.c_int64),
        ("c_stride_inner", ctypes.c_int64), ("c_rows_inner", ctypes.c_int64),
    ]


class _Mlp2Args(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("act1", ctypes.c_int32), ("act2", ctypes.c_int32),
        ("n", ctypes.c_int64), ("m", ctypes.c_int64), ("in_features", ctypes.c_int64),
        ("hidden", ctypes.c_int64), ("out_features", ctypes.c_int64),
        ("x", ctypes.c_void_p), ("x_stride_n", ctypes.c_int64), ("x_stride_outer", ctypes.c_int64),
        ("x_stride_inner", ctypes.c_int64), ("x_rows_inner", ctypes.c_int64),
        ("w1", ctypes.c_void_p), ("b1", ctypes.c_void_p), ("w2", ctypes.c_void_p), ("b2", ctypes.c_void_p),
        ("y", ctypes.c_void_p), ("y_stride_n", ctypes.c_int64), ("y_stride_outer", ctypes.c_int64),
        ("y_stride_inner", ctypes.c_int64), ("y_rows_inner", ctypes.c_int64),
    ]


class _ConvArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("param_dtype", ctypes.c_int32), ("act", ctypes.c_int32),
        ("n", ctypes.c_int64), ("batch", ctypes.c_int64), ("c_in", ctypes.c_int64), ("c_out", ctypes.c_int64),
        ("h", ctypes.c_int64), ("w", ctypes.c_int64), ("kh", ctypes.c_int64), ("kw", ctypes.c_int64),
        ("stride_h", ctypes.c_int64), ("stride_w", ctypes.c_int64), ("pad_h", ctypes.c_int64),
        ("pad_w", ctypes.c_int64), ("dil_h", ctypes.c_int64), ("dil_w", ctypes.c_int64),
        ("h_out", ctypes.c_int64), ("w_out", ctypes.c_int64),
        ("x", ctypes.c_void_p), ("x_stride_n", ctypes.c_int64), ("x_stride_b", ctypes.c_int64),
        ("packed_weight", ctypes.c_void_p), ("bias", ctypes.c_void_p),
        ("bn_weight", ctypes.c_void_p), ("bn_bias", ctypes.c_void_p), ("bn_mean", ctypes.c_void_p),
        ("bn_var", ctypes.c_void_p), ("bn_eps", ctypes.c_float),
        ("residual", ctypes.c_void_p), ("r_stride_n", ctypes.c_int64), ("r_stride_b", ctypes.c_int64),
        ("y", ctypes.c_void_p), ("y_stride_n", ctypes.c_int64), ("y_stride_b", ctypes.c_int64),
        ("weight", ctypes.c_void_p),
    ]


class _Conv3dArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("param_dtype", ctypes.c_int32), ("act", ctypes.c_int32),
        ("n", ctypes.c_int64), ("batch", ctypes.c_int64), ("c_in", ctypes.c_int64), ("c_out", ctypes.c_int64),
        ("d", ctypes.c_int64), ("h", ctypes.c_int64), ("w", ctypes.c_int64),
        ("kd", ctypes.c_int64), ("kh", ctypes.c_int64), ("kw", ctypes.c_int64),
        ("stride_d", ctypes.c_int64), ("stride_h", ctypes.c_int64), ("stride_w", ctypes.c_int64),
        ("pad_d", ctypes.c_int64), ("pad_h", ctypes.c_int64), ("pad_w", ctypes.c_int64),
        ("dil_d", ctypes.c_int64), ("dil_h", ctypes.c_int64), ("dil_w", ctypes.c_int64),
        ("d_out", ctypes.c_int64), ("h_out", ctypes.c_int64), ("w_out", ctypes.c_int64),
        ("x", ctypes.c_void_p), ("x_stride_n", ctypes.c_int64), ("x_stride_b", ctypes.c_int64),
        ("packed_weight", ctypes.c_void_p), ("bias", ctypes.c_void_p),
        ("y", ctypes.c_void_p), ("y_stride_n", ctypes.c_int64), ("y_stride_b", ctypes.c_int64),
    ]


class _AttnArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32),
        ("nb", ctypes.c_int64), ("heads", ctypes.c_int64), ("sq", ctypes.c_int64), ("skv", ctypes.c_int64),
        ("head_dim", ctypes.c_int64), ("scale", ctypes.c_float),
        ("q", ctypes.c_void_p), ("q_stride_nb", ctypes.c_int64), ("q_stride_s", ctypes.c_int64),
        ("k", ctypes.c_void_p), ("k_stride_nb", ctypes.c_int64), ("k_stride_s", ctypes.c_int64),
        ("v", ctypes.c_void_p), ("v_stride_nb", ctypes.c_int64), ("v_stride_s", ctypes.c_int64),
        ("o", ctypes.c_void_p), ("o_stride_nb", ctypes.c_int64), ("o_stride_s", ctypes.c_int64),
        ("mask", ctypes.c_void_p), ("mask_stride_nb", ctypes.c_int64), ("mask_stride_head", ctypes.c_int64),
        ("mask_stride_q", ctypes.c_int64),
    ]


class _SelfAttnArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32),
        ("n", ctypes.c_int64), ("b", ctypes.c_int64), ("s", ctypes.c_int64), ("d_model", ctypes.c_int64),
        ("heads", ctypes.c_int64), ("scale", ctypes.c_float),
        ("x", ctypes.c_void_p), ("x_stride_n", ctypes.c_int64), ("x_stride_b", ctypes.c_int64),
        ("x_stride_s", ctypes.c_int64),
        ("q_weight", ctypes.c_void_p), ("q_weight_stride_n", ctypes.c_int64),
        ("kv_weight", ctypes.c_void_p), ("kv_weight_stride_n", ctypes.c_int64),
        ("q_bias", ctypes.c_void_p), ("q_bias_stride_n", ctypes.c_int64),
        ("kv_bias", ctypes.c_void_p), ("kv_bias_stride_n", ctypes.c_int64),
        ("o", ctypes.c_void_p), ("o_stride_nb", ctypes.c_int64), ("o_stride_s", ctypes.c_int64),
    ]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float

# name -> (restype, argtypes); the single source of truth for the exported ABI
SIGNATURES = {
    "wc_abi_version": (_I32, []),
    "wc_last_error": (ctypes.c_char_p, []),
    "wc_device_count": (_I32, []),
    "wc_pack_rows": (_I32, [ctypes.POINTER(_P), ctypes.POINTER(_I64), _I64, _I64, _I64, _P, _P]),
    "wc_swap01": (_I32, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "wc_embedding_gather": (_I32, [_P, _I64, _I64, _I64, _I32, _P, _I64, _I32, _P, _P, _P]),
    "wc_layernorm": (_I32, [_P, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I32, _I32, _P]),
    "wc_embedding_layernorm": (_I32, [_P, _I64, _I64, _I64, _P, _I64, _I32, _P, _P, _F, _I32, _I32, _P, _P, _P]),
    "wc_bn_eval": (_I32, [_P, _I64, _I64, _P, _P, _P, _P, _F, _P, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _P]),
    "wc_group_norm": (_I32, [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _F, _I32, _I32, _I32, _P]),
    "wc_rnn_workspace_bytes": (_I64, [ctypes.POINTER(_RnnArgs)]),
    "wc_rnn_status_offset": (_I64, [ctypes.POINTER(_RnnArgs)]),
    "wc_rnn_noalloc_scratch_bytes": (_I64, []),
    "wc_rnn_forward_noalloc": (_I32, [ctypes.POINTER(_RnnArgs), _P]),
    "wc_rnn_forward": (_I32, [ctypes.POINTER(_RnnArgs), _P]),
    "wc_rnn_set_spin_limit": (_I32, [_I32]),
    "wc_rnn_input_projection": (_I32, [ctypes.POINTER(_RnnArgs), _P]),
    "wc_rnn_recurrence": (_I32, [ctypes.POINTER(_RnnArgs), _P]),
    "wc_grouped_gemm": (_I32, [ctypes.POINTER(_GemmArgs), _P]),
    "wc_mlp2_supported": (_I32, [_I32, _I64, _I64, _I64]),
    "wc_mlp2": (_I32, [ctypes.POINTER(_Mlp2Args), _P]),
    "wc_conv_pack_weights": (_I32, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P]),
    "wc_conv_packed_weight_elems": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "wc_conv2d": (_I32, [ctypes.POINTER(_ConvArgs), _P]),
    "wc_conv2d_direct_weights": (_I32, [ctypes.POINTER(_ConvArgs)]),
    "wc_conv3d": (_I32, [ctypes.POINTER(_Conv3dArgs), _P]),
    "wc_attention": (_I32, [ctypes.POINTER(_AttnArgs), _P]),
    "wc_self_attention": (_I32, [ctypes.POINTER(_SelfAttnArgs), _P]),
}


def lib():
    """Load libwide_hip.so (once) after torch's HIP runtime; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"wide_compiler: {LIB_PATH} is not built. Build it with "
            f"`make -C {os.path.dirname(os.path.dirname(LIB_PATH))}` or __graft_entry__.build(); "
            "this build has no fallback path."
        )
    # torch is imported first so its libamdhip64.so.7 is the runtime the library binds to
    handle = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    got = handle.wc_abi_version()
    if got != ABI_VERSION:
        raise ImportError(f"wide_compiler: libwide_hip.so ABI {got} != expected {ABI_VERSION}")
    _lib = handle
    return _lib


def last_error() -> str:
    return lib().wc_last_error().decode(errors="replace")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise WideKernelError(f"{what} failed (status {rc}): {last_error()}")


def dtype_code(t: torch.dtype, what: str) -> int:
    try:
        return _DTYPES[t]
    except KeyError:
        raise TypeError(f"{what}: dtype {t} is not supported (float32, bfloat16, float16)") from None


def require_device(what: str, *tensors: Optional[Tensor]) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"{what}: wide_compiler's MI355X build executes on ROCm device tensors only "
                f"(got a tensor on {t.device}); move the model and inputs to 'cuda'"
            )


def require_forward_only(what: str, *tensors: Optional[Tensor]) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise RuntimeError(
            f"{what}: the HIP wide kernels are forward-only; run under torch.no_grad() or "
            "torch.inference_mode()"
        )


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: Tensor) -> int:
    """The current HIP stream of t's device as an address (what the ABI's void* stream takes).
    torch's raw accessor costs a tenth of building a torch.cuda.Stream object per launch."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------------------
# wrappers
# ---------------------------------------------------------------------------------------

def pack_rows(srcs: Sequence[Tensor], dst: Tensor, rows: int, row_bytes: int,
              row_strides_bytes: Sequence[int]) -> None:
    n = len(srcs)
    arr_p = (_P * n)(*[s.data_ptr() for s in srcs])
    arr_s = (_I64 * n)(*row_strides_bytes)
    _check(lib().wc_pack_rows(arr_p, arr_s, n, rows, row_bytes, dst.data_ptr(), stream_of(dst)),
           "wc_pack_rows")


def swap01(src: Tensor, d0: int, d1: int, s0_bytes: int, s1_bytes: int, inner_bytes: int,
           dst: Tensor) -> None:
    _check(lib().wc_swap01(src.data_ptr(), d0, d1, s0_bytes, s1_bytes, inner_bytes, dst.data_ptr(),
                           stream_of(src)), "wc_swap01")


def embedding_gather(weight: Tensor, ids: Tensor, out: Tensor, shared: bool,
                     err_flag: Optional[Tensor] = None) -> None:
    n, vocab, dim = weight.shape
    rows = ids.numel() if shared else ids.numel() // max(n, 1)
    _check(lib().wc_embedding_gather(weight.data_ptr(), n, vocab, dim, dtype_code(weight.dtype, "embedding"),
                                     ids.data_ptr(), rows, 1 if shared else 0, out.data_ptr(),
                                     ptr(err_flag), stream_of(weight)), "wc_embedding_gather")


def embedding_layernorm(weight: Tensor, ids: Tensor, gamma: Tensor, beta: Optional[Tensor], eps: float,
                        out: Tensor, shared: bool, err_flag: Optional[Tensor] = None) -> bool:
    """Gather + LayerNorm in one launch (wc_embedding_layernorm); False (nothing launched) where
    the fused kernel does not take the row size or alignment."""
    n, vocab, dim = weight.shape
    rows = ids.numel() if shared else ids.numel() // max(n, 1)
    rc = lib().wc_embedding_layernorm(weight.data_ptr(), n, vocab, dim, ids.data_ptr(), rows, 1 if shared else 0,
                                      gamma.data_ptr(), ptr(beta), float(eps), dtype_code(weight.dtype, "embedding"),
                                      dtype_code(gamma.dtype, "layernorm"), out.data_ptr(), ptr(err_flag),
                                      stream_of(weight))
    if rc == ERR_LIMIT:
        return False
    _check(rc, "wc_embedding_layernorm")
    return True


def layernorm(x: Tensor, x_ms: int, x_rs: int, gamma: Tensor, beta: Optional[Tensor], y: Tensor,
              y_ms: int, y_rs: int, n: int, rows_per_model: int, dim: int, eps: float) -> None:
    _check(lib().wc_layernorm(x.data_ptr(), x_ms, x_rs, gamma.data_ptr(), ptr(beta), y.data_ptr(), y_ms, y_rs,
                              n, rows_per_model, dim, float(eps), dtype_code(x.dtype, "layernorm"),
                              dtype_code(gamma.dtype, "layernorm"), stream_of(x)), "wc_layernorm")


def bn_eval(x: Tensor, xsn: int, xsb: int, weight: Optional[Tensor], bias: Optional[Tensor],
            rmean: Tensor, rvar: Tensor, eps: float, y: Tensor, n: int, b: int, c: int, hw: int,
            relu: bool = False) -> None:
    _check(lib().wc_bn_eval(x.data_ptr(), xsn, xsb, ptr(weight), ptr(bias), rmean.data_ptr(), rvar.data_ptr(),
                            float(eps), y.data_ptr(), n, b, c, hw, dtype_code(x.dtype, "batchnorm"),
                            dtype_code(rmean.dtype, "batchnorm"), ACT_RELU if relu else ACT_NONE,
                            stream_of(x)), "wc_bn_eval")


def group_norm(x: Tensor, y: Tensor, n: int, b: int, c: int, s: int, groups: int,
               weight: Optional[Tensor], bias: Optional[Tensor], eps: float, relu: bool = False) -> None:
    """x, y contiguous [n, b, c, s]; statistics per (model, batch row, group of c // groups channels)."""
    pdt = weight.dtype if weight is not None else x.dtype
    _check(lib().wc_group_norm(x.data_ptr(), y.data_ptr(), n, b, c, s, groups, ptr(weight), ptr(bias), float(eps),
                               dtype_code(x.dtype, "group_norm"), dtype_code(pdt, "group_norm"),
                               ACT_RELU if relu else ACT_NONE, stream_of(x)), "wc_group_norm")


def grouped_gemm(*, n: int, m: int, o: int, k: int,
                 a: Tensor, a_sn: int, a_so: int, a_si: int, a_rows_inner: int,
                 w: Tensor, w_sn: int,
                 c: Tensor, c_sn: int, c_so: int, c_si: int, c_rows_inner: int,
                 bias: Optional[Tensor] = None, bias_sn: int = 0,
                 residual: Optional[Tensor] = None, r_sn: int = 0, r_so: int = 0, r_si: int = 0,
                 relu: bool = False) -> None:
    g = _GemmArgs()
    g.dtype = dtype_code(a.dtype, "grouped_gemm")
    g.out_dtype = dtype_code(c.dtype, "grouped_gemm")
    g.bias_dtype = dtype_code(bias.dtype, "grouped_gemm") if bias is not None else g.dtype
    g.act = ACT_RELU if relu else ACT_NONE
    g.n, g.m, g.o, g.k = n, m, o, k
    g.a, g.a_stride_n, g.a_stride_outer, g.a_stride_inner, g.a_rows_inner = a.data_ptr(), a_sn, a_so, a_si, a_rows_inner
    g.w, g.w_stride_n = w.data_ptr(), w_sn
    g.bias, g.bias_stride_n = ptr(bias), bias_sn
    g.residual, g.r_stride_n, g.r_stride_outer, g.r_stride_inner = ptr(residual), r_sn, r_so, r_si
    g.c, g.c_stride_n, g.c_stride_outer, g.c_stride_inner, g.c_rows_inner = c.data_ptr(), c_sn, c_so, c_si, c_rows_inner
    _check(lib().wc_grouped_gemm(ctypes.byref(g), stream_of(a)), "wc_grouped_gemm")


def mlp2_supported(dtype: torch.dtype, in_features: int, hidden: int, out_features: int) -> bool:
    if dtype not in (torch.float32, torch.bfloat16):
        return False
    return bool(lib().wc_mlp2_supported(dtype_code(dtype, "mlp2"), in_features, hidden, out_features))


def mlp2_args(*, n: int, m: int, in_features: int, hidden: int, out_features: int,
              x: Tensor, x_sn: int, x_so: int, x_si: int, x_rows_inner: int,
              w1: Tensor, b1: Optional[Tensor], w2: Tensor, b2: Optional[Tensor],
              y: Tensor, y_sn: int, y_so: int, y_si: int, y_rows_inner: int,
              relu1: bool, relu2: bool) -> "_Mlp2Args":
    """The filled argument block of wc_mlp2 (launch with mlp2_launch; a caller may keep it and
    change only the x / y addresses between launches)."""
    a = _Mlp2Args()
    a.dtype = dtype_code(x.dtype, "mlp2")
    a.act1 = ACT_RELU if relu1 else ACT_NONE
    a.act2 = ACT_RELU if relu2 else ACT_NONE
    a.n, a.m, a.in_features, a.hidden, a.out_features = n, m, in_features, hidden, out_features
    a.x, a.x_stride_n, a.x_stride_outer, a.x_stride_inner, a.x_rows_inner = x.data_ptr(), x_sn, x_so, x_si, x_rows_inner
    a.w1, a.b1, a.w2, a.b2 = w1.data_ptr(), ptr(b1), w2.data_ptr(), ptr(b2)
    a.y, a.y_stride_n, a.y_stride_outer, a.y_stride_inner, a.y_rows_inner = y.data_ptr(), y_sn, y_so, y_si, y_rows_inner
    return a


try:
    # CPython launcher of the entry points (built beside libwide_hip.so): a call through it
    # costs a fraction of a ctypes call, which dominates a small forward's host time
    from . import _wc_launch
except ImportError:     # not built: the ctypes binding of the same entry points
    _wc_launch = None
_entries: Dict[str, int] = {}


def entry_address(name: str) -> int:
    """Address of libwide_hip.so's entry point `name` (looked up once)."""
    a = _entries.get(name)
    if a is None:
        a = _entries[name] = ctypes.cast(getattr(lib(), name), ctypes.c_void_p).value
    return a


def mlp2_launch(a: "_Mlp2Args", stream: int) -> None:
    if _wc_launch is not None:
        rc = _wc_launch.call2(_entries.get("wc_mlp2") or entry_address("wc_mlp2"), ctypes.addressof(a), stream)
    else:
        rc = lib().wc_mlp2(ctypes.byref(a), stream)
    if rc:
        _check(rc, "wc_mlp2")


def mlp2(**kw) -> None:
    """wc_mlp2 with the arguments of mlp2_args, on x's current stream."""
    mlp2_launch(mlp2_args(**kw), stream_of(kw["x"]))


def rnn_args(*, cell: int, x: Tensor, w_ih: Tensor, w_hh: Tensor, b_ih: Optional[Tensor],
             b_hh: Optional[Tensor], h0: Optional[Tensor], c0: Optional[Tensor], out: Tensor,
             h_n: Optional[Tensor], c_n: Optional[Tensor], workspace: Optional[Tensor] = None,
             allocate: bool = True, status: Optional[Tensor] = None):
    """Fill the wc_rnn_args struct; allocates the workspace unless one is given or
    allocate is False (then the struct carries no workspace).  ``status`` is an optional
    int32 device word that a give-up of the partitioned recurrence's bounded waits sets (never
    cleared by the library).  Returns (args, workspace)."""
    n, batch, steps, in_size = x.shape
    hidden = w_hh.shape[-1]
    a = _RnnArgs()
    a.cell = cell
    a.dtype = dtype_code(x.dtype, "rnn")
    a.n, a.batch, a.steps, a.input_size, a.hidden = n, batch, steps, in_size, hidden
    a.x = x.data_ptr()
    a.x_stride_n, a.x_stride_b, a.x_stride_t = x.stride(0), x.stride(1), x.stride(2)
    a.w_ih, a.w_hh, a.b_ih, a.b_hh = w_ih.data_ptr(), w_hh.data_ptr(), ptr(b_ih), ptr(b_hh)
    a.h0, a.c0 = ptr(h0), ptr(c0)
    a.out, a.h_n, a.c_n = out.data_ptr(), ptr(h_n), ptr(c_n)
    if status is not None:
        if status.dtype != torch.int32 or status.device != x.device:
            raise ValueError("rnn status word must be an int32 tensor on the input's device")
        a.status = status.data_ptr()
    if not allocate and workspace is None:
        a.workspace, a.workspace_bytes = None, 0
        return a, None
    need = int(lib().wc_rnn_workspace_bytes(ctypes.byref(a)))
    ws = workspace
    if ws is None or ws.numel() * ws.element_size() < need:
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=x.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * ws.element_size()
    return a, ws


# The partitioned recurrence's bounded cross-workgroup waits report a give-up (its outputs are
# then invalid) in a status word.  Every launch made through rnn_forward /
# rnn_forward_noalloc is given this device's own word, which the library never clears:
# it collects the verdict of every eager launch and of every replay of a captured graph
# until rnn_sync_check reads it, raises, and clears it.  After an eager launch a copy of
# the word is queued to pinned host memory behind an event, so a later check raises
# without blocking the stream; replays of captured launches queue no copy of their own,
# so the next check queues one for every device whose word a capture used.
_status_words: Dict[int, Tensor] = {}
_status_captured: set = set()
_rnn_pending: List = []


def rnn_status_word(device: torch.device) -> Tensor:
    """This device's status word (created, zeroed, at the first recurrent call outside
    graph capture)."""
    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    w = _status_words.get(idx)
    if w is None:
        if torch.cuda.is_current_stream_capturing():
            raise WideKernelError("wide_compiler: run a recurrent layer once outside graph capture before "
                                  "capturing it (its status word is created then)")
        w = _status_words[idx] = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda", idx))
    return w


def _queue_status_copy(word: Tensor) -> None:
    host = torch.empty(1, dtype=torch.int32, pin_memory=True)
    host.copy_(word, non_blocking=True)
    ev = torch.cuda.Event()
    ev.record(torch.cuda.current_stream(word.device))
    _rnn_pending.append((ev, host, word))


def _rnn_watch(word: Tensor) -> None:
    if torch.cuda.is_current_stream_capturing():
        _status_captured.add(word.device.index)
    else:
        _queue_status_copy(word)


def rnn_sync_check(block: bool = False) -> None:
    """Raise WideKernelError if a finished partitioned-recurrence launch or graph replay reported
    a bounded wait that gave up (its outputs are then invalid), and clear the word.
    block=True waits for every launch still in flight; otherwise launches whose status
    has not landed yet are checked by a later call."""
    global _rnn_pending
    if torch.cuda.is_current_stream_capturing():
        return                       # events cannot be queried while a graph is captured
    for idx in _status_captured:
        _queue_status_copy(_status_words[idx])
    if not _rnn_pending:
        return
    keep, failed = [], []
    for ev, host, word in _rnn_pending:
        if block:
            ev.synchronize()
        if ev.query():
            if int(host[0]) != 0 and all(word is not f for f in failed):
                failed.append(word)
        else:
            keep.append((ev, host, word))
    _rnn_pending = keep
    if failed:
        for word in failed:
            word.zero_()
        # copies still in flight may hold the verdict just reported
        _rnn_pending = [e for e in _rnn_pending if all(e[2] is not f for f in failed)]
        raise WideKernelError("wc_rnn_recurrence: a cross-workgroup wait of the partitioned recurrence gave up; "
                              "the outputs of that launch (or graph replay) are invalid")


def rnn_set_spin_limit(polls: int) -> int:
    """Poll rounds after which a partitioned-recurrence wait gives up for launches made from now
    on (0: at the first wait; < 0: the default); returns the previous value."""
    return int(lib().wc_rnn_set_spin_limit(int(polls)))


def _part_status(a: _RnnArgs, x: Tensor) -> Optional[Tensor]:
    """This device's status word, set in ``a``, when these sizes run the partitioned recurrence
    (the one recurrent kernel with cross-workgroup waits); None otherwise."""
    if int(lib().wc_rnn_status_offset(ctypes.byref(a))) < 0:
        return None
    word = rnn_status_word(x.device)
    a.status = word.data_ptr()
    return word


def rnn_forward(**kw) -> None:
    """wc_rnn_forward with a fresh workspace (and, on the partitioned plan, this device's
    status word); a give-up of an earlier launch is raised here (non-blocking), or by
    rnn_sync_check."""
    rnn_sync_check()
    a, ws = rnn_args(**kw)
    word = _part_status(a, kw["x"])
    _check(lib().wc_rnn_forward(ctypes.byref(a), stream_of(kw["x"])), "wc_rnn_forward")
    if word is not None:
        _rnn_watch(word)


def rnn_forward_noalloc(**kw) -> None:
    """wc_rnn_forward_noalloc: the same forward with the workspace in the library's static
    per-device scratch; nothing is allocated for the call (the status word is this
    device's persistent one)."""
    rnn_sync_check()
    a, _ = rnn_args(allocate=False, **kw)
    word = _part_status(a, kw["x"])
    _check(lib().wc_rnn_forward_noalloc(ctypes.byref(a), stream_of(kw["x"])), "wc_rnn_forward_noalloc")
    if word is not None:
        _rnn_watch(word)


def rnn_phase(a: _RnnArgs, phase: str, like: Tensor) -> None:
    """Run one phase ('input_projection' or 'recurrence') of a prepared rnn_args struct."""
    fn = getattr(lib(), f"wc_rnn_{phase}")
    _check(fn(ctypes.byref(a), stream_of(like)), f"wc_rnn_{phase}")


def conv_pack_weights(w: Tensor, n: int, c_out: int, c_in: int, kh: int, kw: int) -> Tensor:
    elems = int(lib().wc_conv_packed_weight_elems(n, c_out, c_in, kh, kw))
    out = torch.empty(max(elems, 8), dtype=w.dtype, device=w.device)
    _check(lib().wc_conv_pack_weights(w.data_ptr(), n, c_out, c_in, kh, kw, dtype_code(w.dtype, "conv"),
                                      out.data_ptr(), stream_of(w)), "wc_conv_pack_weights")
    return out


def conv2d(*, x: Tensor, weight: Tensor, n: int, c_in: int, c_out: int, kernel, stride, padding, dilation,
           y: Tensor, bias: Optional[Tensor] = None, bn=None, residual: Optional[Tensor] = None,
           relu: bool = False, packed: bool = False) -> None:
    """x / y / residual are [n, b, C, H, W] with dense [C, H, W] blocks; ``weight`` is the
    contiguous grouped filter bank [n*C_out, C_in, kh, kw]; bn = (weight, bias, running_mean,
    running_var, eps) or None.  The filters go to the kernel as they are where the library
    reads that layout (wc_conv2d_direct_weights), else (or with ``packed``) through one
    packing pass."""
    a = _ConvArgs()
    a.dtype = dtype_code(x.dtype, "conv")
    params = [t for t in (bias, *(bn[:4] if bn else ())) if t is not None]
    a.param_dtype = dtype_code(params[0].dtype, "conv") if params else a.dtype
    a.act = ACT_RELU if relu else ACT_NONE
    a.n, a.batch, a.c_in, a.c_out = n, x.shape[1], c_in, c_out
    a.h, a.w = x.shape[3], x.shape[4]
    a.kh, a.kw = kernel
    a.stride_h, a.stride_w = stride
    a.pad_h, a.pad_w = padding
    a.dil_h, a.dil_w = dilation
    a.h_out, a.w_out = y.shape[3], y.shape[4]
    a.x, a.x_stride_n, a.x_stride_b = x.data_ptr(), x.stride(0), x.stride(1)
    a.weight = weight.data_ptr()
    a.bias = ptr(bias)
    if bn is not None:
        a.bn_weight, a.bn_bias, a.bn_mean, a.bn_var = ptr(bn[0]), ptr(bn[1]), ptr(bn[2]), ptr(bn[3])
        a.bn_eps = float(bn[4])
    if residual is not None:
        a.residual, a.r_stride_n, a.r_stride_b = residual.data_ptr(), residual.stride(0), residual.stride(1)
    a.y, a.y_stride_n, a.y_stride_b = y.data_ptr(), y.stride(0), y.stride(1)
    if packed or not lib().wc_conv2d_direct_weights(ctypes.byref(a)):
        packed = conv_pack_weights(weight, n, c_out, c_in, a.kh, a.kw)
        a.packed_weight = packed.data_ptr()
    _check(lib().wc_conv2d(ctypes.byref(a), stream_of(x)), "wc_conv2d")


def conv3d(*, x: Tensor, packed_w: Tensor, n: int, c_in: int, c_out: int, kernel, stride, padding, dilation,
           y: Tensor, bias: Optional[Tensor] = None, relu: bool = False) -> None:
    """x / y are [n, b, C, D, H, W] with dense [C, D, H, W] blocks."""
    a = _Conv3dArgs()
    a.dtype = dtype_code(x.dtype, "conv3d")
    a.param_dtype = dtype_code(bias.dtype, "conv3d") if bias is not None else a.dtype
    a.act = ACT_RELU if relu else ACT_NONE
    a.n, a.batch, a.c_in, a.c_out = n, x.shape[1], c_in, c_out
    a.d, a.h, a.w = x.shape[3], x.shape[4], x.shape[5]
    a.kd, a.kh, a.kw = kernel
    a.stride_d, a.stride_h, a.stride_w = stride
    a.pad_d, a.pad_h, a.pad_w = padding
    a.dil_d, a.dil_h, a.dil_w = dilation
    a.d_out, a.h_out, a.w_out = y.shape[3], y.shape[4], y.shape[5]
    a.x, a.x_stride_n, a.x_stride_b = x.data_ptr(), x.stride(0), x.stride(1)
    a.packed_weight = packed_w.data_ptr()
    a.bias = ptr(bias)
    a.y, a.y_stride_n, a.y_stride_b = y.data_ptr(), y.stride(0), y.stride(1)
    _check(lib().wc_conv3d(ctypes.byref(a), stream_of(x)), "wc_conv3d")


def attention(*, q: Tensor, k: Tensor, v: Tensor, o: Tensor, nb: int, heads: int, sq: int, skv: int,
              head_dim: int, q_strides, k_strides, v_strides, o_strides, scale: float, causal: bool,
              mask: Optional[Tensor] = None) -> None:
    """q/k/v/o are base pointers (views) of [nb, S, heads*head_dim]-shaped data with the given
    (stride_nb, stride_s) element strides; ``mask`` is an additive fp32 [nb, heads, sq, skv]
    view with a unit key stride (other strides may be 0)."""
    a = _AttnArgs()
    a.dtype = dtype_code(q.dtype, "attention")
    a.causal = 1 if causal else 0
    a.nb, a.heads, a.sq, a.skv, a.head_dim = nb, heads, sq, skv, head_dim
    a.scale = float(scale)
    a.q, (a.q_stride_nb, a.q_stride_s) = q.data_ptr(), q_strides
    a.k, (a.k_stride_nb, a.k_stride_s) = k.data_ptr(), k_strides
    a.v, (a.v_stride_nb, a.v_stride_s) = v.data_ptr(), v_strides
    a.o, (a.o_stride_nb, a.o_stride_s) = o.data_ptr(), o_strides
    if mask is not None:
        if mask.dtype != torch.float32 or tuple(mask.shape) != (nb, heads, sq, skv) or \
                (skv > 1 and mask.stride(3) != 1) or mask.device != q.device:
            raise ValueError("attention mask must be an fp32 [nb, heads, sq, skv] view with unit key stride "
                             "on the query's device")
        a.mask = mask.data_ptr()
        a.mask_stride_nb, a.mask_stride_head, a.mask_stride_q = mask.stride(0), mask.stride(1), mask.stride(2)
    _check(lib().wc_attention(ctypes.byref(a), stream_of(q)), "wc_attention")


def self_attention(*, x: Tensor, q_weight: Tensor, kv_weight: Tensor, q_bias: Optional[Tensor],
                   kv_bias: Optional[Tensor], o: Tensor, heads: int, scale: float, causal: bool) -> None:
    """Fused self-attention core with the Q and K|V projections inside (wc_self_attention):
    x [N, B, S, D] (unit last stride), q_weight [N, D, D] and kv_weight [N, 2D, D] with
    contiguous rows, biases [N, D] / [N, 2D] or None, o [N, B, S, D] contiguous (the attention
    output before the output projection)."""
    n, b, s, d = x.shape
    a = _SelfAttnArgs()
    a.dtype = dtype_code(x.dtype, "self_attention")
    a.causal = 1 if causal else 0
    a.n, a.b, a.s, a.d_model, a.heads = n, b, s, d, heads
    a.scale = float(scale)
    a.x, a.x_stride_n, a.x_stride_b, a.x_stride_s = x.data_ptr(), x.stride(0), x.stride(1), x.stride(2)
    a.q_weight, a.q_weight_stride_n = q_weight.data_ptr(), q_weight.stride(0)
    a.kv_weight, a.kv_weight_stride_n = kv_weight.data_ptr(), kv_weight.stride(0)
    if q_bias is not None:
        a.q_bias, a.q_bias_stride_n = q_bias.data_ptr(), q_bias.stride(0)
    if kv_bias is not None:
        a.kv_bias, a.kv_bias_stride_n = kv_bias.data_ptr(), kv_bias.stride(0)
    a.o, a.o_stride_nb, a.o_stride_s = o.data_ptr(), o.stride(1), o.stride(2)
    _check(lib().wc_self_attention(ctypes.byref(a), stream_of(x)), "wc_self_attention")


def exported_symbols() -> List[str]:
    return list(SIGNATURES)


# Every entry point that launches kernels is a compile boundary: under torch.compile
# (compile_model=True) dynamo does not trace into the ctypes call and its stream handle,
# but ends the compiled region there and runs the call as is, so inductor never generates
# code for the hot path.
for _name in ("pack_rows", "swap01", "embedding_gather", "layernorm", "bn_eval", "group_norm", "grouped_gemm",
              "mlp2", "mlp2_args", "mlp2_launch", "embedding_layernorm", "rnn_forward", "rnn_forward_noalloc", "rnn_phase", "conv_pack_weights", "conv2d", "conv3d",
              "attention", "self_attention", "rnn_sync_check", "rnn_status_word", "rnn_set_spin_limit"):
    globals()[_name] = torch.compiler.disable(globals()[_name])
del _name
