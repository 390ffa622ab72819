"""Host-side checks shared by WideGRU and WideLSTM."""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from ... import _hip


def prepare_input(what: str, x: Tensor, n: int, input_size: int, dtype: torch.dtype) -> Tensor:
    if x.dim() != 4 or x.shape[0] != n or x.shape[3] != input_size:
        raise RuntimeError(f"{what}: expected input [N={n}, B, T, {input_size}], got {list(x.shape)}")
    if x.dtype != dtype:
        raise RuntimeError(f"{what}: input dtype {x.dtype} != weight dtype {dtype}")
    if x.shape[2] == 0:
        raise RuntimeError(f"{what}: stack expects a non-empty TensorList (sequence length 0)")
    if x.shape[3] > 1 and x.stride(3) != 1:
        x = x.contiguous()
    return x


def prepare_state(what: str, s: Optional[Tensor], n: int, b: int, h: int, dtype: torch.dtype,
                  name: str) -> Optional[Tensor]:
    if s is None:
        return None
    if tuple(s.shape) != (n, b, h):
        raise RuntimeError(f"{what}: {name} must be [N={n}, B={b}, H={h}], got {list(s.shape)}")
    if s.dtype != dtype:
        raise RuntimeError(f"{what}: {name} dtype {s.dtype} != {dtype}")
    _hip.require_device(what, s)
    return s.contiguous()


def contiguous(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None else (t if t.is_contiguous() else t.contiguous())
