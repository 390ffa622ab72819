"""
Stride bookkeeping shared by the primitives.

The kernels address the rows of an N-first operand [N, *batch, F] (F contiguous) as
``n * stride_n + (m // rows_inner) * stride_outer + (m % rows_inner) * stride_inner`` with
m the flattened batch index, so any view whose batch dims collapse into at most two
strided levels is consumed in place -- including the N-first view of a channel-packed
[B, N*F] boundary tensor.  Views that do not collapse are copied once with
``.contiguous()``.
"""

from __future__ import annotations

from typing import NamedTuple, Optional, Sequence, Tuple

from torch import Tensor


class Rows(NamedTuple):
    stride_n: int
    stride_outer: int
    stride_inner: int
    rows_inner: int
    rows: int


def _collapse(sizes: Sequence[int], strides: Sequence[int]) -> Tuple[Tuple[int, int], ...]:
    dims = [(s, st) for s, st in zip(sizes, strides) if s != 1]
    out = []
    for s, st in dims:
        if out and out[-1][1] == st * s:
            ps, _ = out[-1]
            out[-1] = (ps * s, st)
        else:
            out.append((s, st))
    return tuple(out)


def rows_of(x: Tensor) -> Optional[Rows]:
    """Two-level row addressing of x = [N, *batch, F] with unit stride on F, or None."""
    if x.dim() < 2 or (x.shape[-1] > 1 and x.stride(-1) != 1):
        return None
    batch = x.shape[1:-1]
    m = 1
    for s in batch:
        m *= s
    dims = _collapse(batch, x.stride()[1:-1])
    if len(dims) == 0:
        return Rows(x.stride(0), 0, 0, 1, m)
    if len(dims) == 1:
        return Rows(x.stride(0), 0, dims[0][1], dims[0][0], m)
    if len(dims) == 2:
        return Rows(x.stride(0), dims[0][1], dims[1][1], dims[1][0], m)
    return None


def rows_or_contiguous(x: Tensor) -> Tuple[Tensor, Rows]:
    r = rows_of(x)
    if r is None:
        x = x.contiguous()
        r = rows_of(x)
    return x, r


def inner_block_contiguous(t: Tensor, start_dim: int) -> bool:
    """True if dims [start_dim:] of t form one dense row-major block."""
    expected = 1
    for size, stride in reversed(list(zip(t.shape[start_dim:], t.stride()[start_dim:]))):
        if size != 1 and stride != expected:
            return False
        expected *= size
    return True
