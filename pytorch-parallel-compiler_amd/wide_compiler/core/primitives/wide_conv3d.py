"""
WideConv3d (construction / state layout of wide_compiler/core/primitives/wide_conv3d.py:
``grouped_conv`` = nn.Conv3d(N*C_in, N*C_out, groups=N)).  Not on the hot path yet.
"""

from __future__ import annotations

from enum import Enum
from typing import List, Union

import torch
from torch import Tensor, nn

from ._unported import not_on_hot_path


class Conv3dStrategy(Enum):
    AUTO = "auto"
    GROUPED = "grouped"
    SEQUENTIAL = "sequential"


def _triple(v):
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v, v)


class WideConv3d(nn.Module):
    def __init__(self, n: int, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0,
                 dilation=1, bias: bool = True, strategy: Union[str, Conv3dStrategy] = "auto"):
        super().__init__()
        self.n = n
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _triple(kernel_size)
        self.stride = _triple(stride)
        self.padding = _triple(padding)
        self.dilation = _triple(dilation)
        if isinstance(strategy, str):
            strategy = Conv3dStrategy(strategy)
        self._strategy = Conv3dStrategy.GROUPED if strategy == Conv3dStrategy.AUTO else strategy
        self.grouped_conv = nn.Conv3d(n * in_channels, n * out_channels, self.kernel_size,
                                      stride=self.stride, padding=self.padding, dilation=self.dilation,
                                      groups=n, bias=bias)

    @property
    def strategy(self) -> Conv3dStrategy:
        return self._strategy

    def forward(self, x: Tensor) -> Tensor:
        not_on_hot_path("WideConv3d")

    @classmethod
    def from_modules(cls, modules: List[nn.Conv3d], strategy="auto") -> "WideConv3d":
        t = modules[0]
        wide = cls(len(modules), t.in_channels, t.out_channels, t.kernel_size, t.stride, t.padding,
                   t.dilation, t.bias is not None, strategy)
        wide = wide.to(device=t.weight.device, dtype=t.weight.dtype)
        co = t.out_channels
        with torch.no_grad():
            for i, m in enumerate(modules):
                wide.grouped_conv.weight[i * co:(i + 1) * co].copy_(m.weight)
                if m.bias is not None:
                    wide.grouped_conv.bias[i * co:(i + 1) * co].copy_(m.bias)
        return wide

    def __repr__(self) -> str:
        return f"WideConv3d({self.n}x[{self.in_channels}->{self.out_channels}], k={self.kernel_size})"


__all__ = ["WideConv3d", "Conv3dStrategy"]
