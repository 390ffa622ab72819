"""
WideConv2d: N independent nn.Conv2d layers
(mirror of wide_compiler/core/primitives/wide_conv2d.py:33-284).

    x [N, B, C_in, H, W] -> [N, B, C_out, H', W']

Parameters keep the reference layout: ``grouped_conv`` = nn.Conv2d(N*C_in, N*C_out,
groups=N) holding model i's filters at output channels [i*C_out, (i+1)*C_out).  Every
strategy ('grouped', 'channels_last', 'sequential', 'auto') is accepted and recorded.
"""

from __future__ import annotations

import warnings
from enum import Enum
from typing import List, Optional, Tuple, Union

import torch
from torch import Tensor, nn

from ._conv_common import conv_forward


class ConvStrategy(Enum):
    AUTO = "auto"
    GROUPED = "grouped"
    CHANNELS_LAST = "channels_last"
    SEQUENTIAL = "sequential"


STRATEGY_THRESHOLDS = {"n_high": 16, "n_crossover": 8, "n_low": 3, "b_low": 16}

_warned = False


def select_strategy(n: int, b: int, c_in: int, c_out: int, h: int = 56, w: int = 56) -> ConvStrategy:
    """The reference's label heuristic (wide_conv2d.py:67-96), including its one-time warning."""
    global _warned
    if not _warned:
        warnings.warn(
            "WideConv2d auto-selection thresholds may need tuning for your GPU. "
            "Run the test suite to verify optimal strategy for your hardware.",
            UserWarning,
        )
        _warned = True
    t = STRATEGY_THRESHOLDS
    if n <= t["n_low"]:
        return ConvStrategy.SEQUENTIAL
    if (n >= t["n_crossover"] and b <= t["b_low"]) or n >= t["n_high"]:
        return ConvStrategy.GROUPED
    return ConvStrategy.SEQUENTIAL


def _pair(v) -> Tuple[int, int]:
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v)


class WideConv2d(nn.Module):
    def __init__(self, n: int, in_channels: int, out_channels: int,
                 kernel_size: Union[int, Tuple[int, int]], stride=1, padding=0, dilation=1,
                 bias: bool = True, strategy: Union[str, ConvStrategy] = "auto"):
        super().__init__()
        self.n = n
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        self.has_bias = bias
        if isinstance(strategy, str):
            strategy = ConvStrategy(strategy)
        if strategy == ConvStrategy.AUTO:
            strategy = select_strategy(n, 8, in_channels, out_channels, 56, 56)
        self._strategy = strategy
        self.grouped_conv = nn.Conv2d(n * in_channels, n * out_channels, self.kernel_size,
                                      stride=self.stride, padding=self.padding,
                                      dilation=self.dilation, groups=n, bias=bias)
        # epilogue fused in by TracedWideModel: a following eval BatchNorm, ReLU, residual add
        self.fused_bn = None
        self.fused_activation = None

    @property
    def strategy(self) -> ConvStrategy:
        return self._strategy

    def forward(self, x: Tensor, residual: Optional[Tensor] = None, out: Optional[Tensor] = None) -> Tensor:
        """x [N, B, C_in, H, W] -> [N, B, C_out, H', W'].  ``residual`` (same shape as the
        output) is added in the epilogue; TracedWideModel passes it when it has fused a
        following ``+``."""
        if x.dim() != 5:
            raise RuntimeError(f"WideConv2d: expected [N, B, C, H, W], got {list(x.shape)}")
        return conv_forward(self, x, residual=residual, out=out)

    @classmethod
    def from_modules(cls, modules: List[nn.Conv2d],
                     strategy: Union[str, ConvStrategy] = "auto") -> "WideConv2d":
        t = modules[0]
        if t.groups != 1:
            raise ValueError("WideConv2d.from_modules supports groups=1 convolutions")
        if isinstance(t.padding, str):
            raise ValueError("WideConv2d.from_modules needs numeric padding")
        if t.padding_mode != "zeros":
            raise ValueError("WideConv2d.from_modules supports padding_mode='zeros'")
        wide = cls(n=len(modules), in_channels=t.in_channels, out_channels=t.out_channels,
                   kernel_size=_pair(t.kernel_size), stride=_pair(t.stride), padding=_pair(t.padding),
                   dilation=_pair(t.dilation), bias=t.bias is not None, strategy=strategy)
        wide = wide.to(device=t.weight.device, dtype=t.weight.dtype)
        co = t.out_channels
        with torch.no_grad():
            for i, m in enumerate(modules):
                wide.grouped_conv.weight[i * co:(i + 1) * co].copy_(m.weight)
                if m.bias is not None:
                    wide.grouped_conv.bias[i * co:(i + 1) * co].copy_(m.bias)
        return wide

    def __repr__(self) -> str:
        return (f"WideConv2d({self.n}x[{self.in_channels}->{self.out_channels}], "
                f"k={self.kernel_size}, strategy={self._strategy.value})")


def create_wide_conv2d(modules: List[nn.Conv2d], strategy: Union[str, ConvStrategy] = "auto") -> WideConv2d:
    return WideConv2d.from_modules(modules, strategy=strategy)


__all__ = ["WideConv2d", "ConvStrategy", "select_strategy", "create_wide_conv2d", "STRATEGY_THRESHOLDS"]
