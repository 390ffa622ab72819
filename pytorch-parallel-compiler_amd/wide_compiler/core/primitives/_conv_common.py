"""Host side of the implicit-GEMM convolution shared by WideConv1d / WideConv2d."""

from __future__ import annotations

from torch import Tensor

from ... import _hip


def conv_forward(mod, x: Tensor, one_d: bool = False) -> Tensor:
    raise NotImplementedError(f"{type(mod).__name__}: the convolution kernel is not built yet")
