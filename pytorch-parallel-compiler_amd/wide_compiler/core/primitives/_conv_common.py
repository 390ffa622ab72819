"""
Host side of the implicit-GEMM convolution shared by WideConv1d / WideConv2d.

The filters are read from the module's own parameter on every call, as the reference does:
writes through ``.data`` do not bump a tensor's version counter, so no cache of a derived
layout keyed on it could see them.  The resident-weight kernel stages the filter bank in its
natural [N*C_out, C_in, kh, kw] layout; the other kernels take it packed into a K-contiguous
layout [N, C_out, kh, kw, Ci32] by one small bandwidth kernel per call.  A following eval BatchNorm, residual add and ReLU
are applied in the conv epilogue when TracedWideModel has fused them (``fused_bn`` /
``fused_activation`` / the ``residual`` argument).
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from ... import _hip
from .._layout import inner_block_contiguous


def conv_forward(mod, x: Tensor, one_d: bool = False, residual: Optional[Tensor] = None,
                 out: Optional[Tensor] = None) -> Tensor:
    """x: [N, B, C_in, H, W] (1-D convs pass W = L after an unsqueeze of H = 1).  ``out``, if
    given, is any [N, B, C_out, H', W'] view whose [C_out, H', W'] blocks are dense (e.g. the
    N-first view of a channel-packed tensor)."""
    what = type(mod).__name__
    if one_d:
        w, bias = mod._filters()
        kh, kw = 1, mod.kernel_size
        stride, padding, dilation = (1, mod.stride), (0, mod.padding), (1, mod.dilation)
    else:
        w, bias = mod.grouped_conv.weight, mod.grouped_conv.bias
        kh, kw = mod.kernel_size
        stride, padding, dilation = mod.stride, mod.padding, mod.dilation
    n, ci, co = mod.n, mod.in_channels, mod.out_channels
    if x.shape[0] != n or x.shape[2] != ci:
        raise RuntimeError(f"{what}: expected [N={n}, B, C_in={ci}, ...], got {list(x.shape)}")
    bn = mod.fused_bn
    bn_args = None
    tensors = [x, w, bias, residual]
    if bn is not None:
        op = bn.op
        if op.training or not op.track_running_stats or op.running_mean is None:
            raise RuntimeError(f"{what}: the fused BatchNorm must be in eval mode with running statistics")
        bn_args = (op.weight, op.bias, op.running_mean, op.running_var, op.eps)
        tensors += [op.weight, op.bias, op.running_mean]
    _hip.require_device(what, *tensors)
    _hip.require_forward_only(what, *tensors)
    if x.dtype != w.dtype:
        raise RuntimeError(f"{what}: input dtype {x.dtype} != weight dtype {w.dtype}")
    if not inner_block_contiguous(x, 2):
        x = x.contiguous()
    b, h, wd = x.shape[1], x.shape[3], x.shape[4]
    ho = (h + 2 * padding[0] - dilation[0] * (kh - 1) - 1) // stride[0] + 1
    wo = (wd + 2 * padding[1] - dilation[1] * (kw - 1) - 1) // stride[1] + 1
    if ho <= 0 or wo <= 0:
        raise RuntimeError(f"{what}: input {h}x{wd} is smaller than the kernel")
    if out is not None:
        if tuple(out.shape) != (n, b, co, ho, wo) or out.dtype != x.dtype or not inner_block_contiguous(out, 2):
            raise RuntimeError(f"{what}: output view {list(out.shape)} is not addressable")
        y = out
    else:
        y = torch.empty((n, b, co, ho, wo), dtype=x.dtype, device=x.device)
    if residual is not None:
        if tuple(residual.shape) != tuple(y.shape) or residual.dtype != y.dtype:
            raise RuntimeError(f"{what}: residual {list(residual.shape)} does not match output {list(y.shape)}")
        if not inner_block_contiguous(residual, 2):
            residual = residual.contiguous()
    if y.numel() == 0:
        return y
    if not w.is_contiguous():
        w = w.contiguous()
    _hip.conv2d(x=x, weight=w, n=n, c_in=ci, c_out=co, kernel=(kh, kw), stride=stride, padding=padding,
                dilation=dilation, y=y, bias=bias, bn=bn_args, residual=residual,
                relu=mod.fused_activation == "relu")
    return y
