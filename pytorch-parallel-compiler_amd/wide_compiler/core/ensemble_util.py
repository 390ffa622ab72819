"""
Pack N per-model tensors into the channel-packed wide layout and back
(mirror of wide_compiler/core/ensemble_util.py:20-101).

    pack_inputs([x_0 .. x_{N-1}])  each [B, F, *S]  ->  [B, N*F, *S]
    unpack_outputs(y, n)           [B, N*F, *S]      ->  N views [B, F, *S]

``pack_inputs`` is one pointer-table gather kernel (wc_pack_rows): packed[b, i*F*S + j] =
x_i[b, j], a bit-exact byte copy.  ``unpack_outputs`` returns strided views, exactly as the
reference does, so it launches nothing.
"""

from __future__ import annotations

from typing import List

import torch
from torch import Tensor

from .. import _hip
from ._layout import inner_block_contiguous


def pack_inputs(inputs: List[Tensor]) -> Tensor:
    if not inputs:
        raise ValueError("inputs list is empty")
    first = inputs[0]
    if first.dim() == 0:
        raise ValueError("pack_inputs needs tensors with a batch dimension")
    for i, t in enumerate(inputs):
        if t.shape != first.shape:
            raise RuntimeError(
                f"stack expects each tensor to be equal size, but got {list(first.shape)} at entry 0 "
                f"and {list(t.shape)} at entry {i}"
            )
        if t.dtype != first.dtype or t.device != first.device:
            raise RuntimeError("pack_inputs: all inputs must share dtype and device")
    _hip.require_device("pack_inputs", *inputs)
    n = len(inputs)
    b = first.shape[0]
    rest = tuple(first.shape[1:])
    per_row = 1
    for s in rest:
        per_row *= s
    es = first.element_size()
    srcs = [t if inner_block_contiguous(t, 1) else t.contiguous() for t in inputs]
    if len(rest) == 0:
        out = torch.empty((b, n), dtype=first.dtype, device=first.device)
    else:
        out = torch.empty((b, n * rest[0], *rest[1:]), dtype=first.dtype, device=first.device)
    if out.numel():
        _hip.pack_rows(srcs, out, b, per_row * es, [t.stride(0) * es for t in srcs])
    return out


def unpack_outputs(output: Tensor, n: int) -> List[Tensor]:
    b = output.shape[0]
    rest = output.shape[1:]
    if len(rest) == 0:
        raise ValueError("output must have at least 2 dimensions")
    nf = rest[0]
    if nf % n != 0:
        raise ValueError(f"Cannot split dim 1 ({nf}) into {n} equal parts")
    split = output.view(b, n, nf // n, *rest[1:])
    return [split[:, i] for i in range(n)]


__all__ = ["pack_inputs", "unpack_outputs"]
