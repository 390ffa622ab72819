"""
WideConv1d: N independent nn.Conv1d layers
(mirror of wide_compiler/core/primitives/wide_conv1d.py:28-209).

    x [N, B, C_in, L] -> [N, B, C_out, L']

State layout follows the reference and depends on N (wide_conv1d.py:80-105): for N >= 10
(GROUPED) the filters live in ``op`` = nn.Conv1d(N*C_in, N*C_out, groups=N); below that
(SEQUENTIAL) in ``weight`` [N, C_out, C_in, k] and ``bias`` [N, C_out].  Both execute the
same implicit-GEMM kernel as WideConv2d (a 1-D convolution is a 2-D one with H = 1).
"""

from __future__ import annotations

import math
from enum import Enum, auto
from typing import List, Optional

import torch
from torch import Tensor, nn

from ._conv_common import conv_forward

_GROUPED_THRESHOLD = 10


class Conv1dStrategy(Enum):
    GROUPED = auto()
    SEQUENTIAL = auto()


class WideConv1d(nn.Module):
    def __init__(self, n: int, in_channels: int, out_channels: int, kernel_size: int, stride: int = 1,
                 padding: int = 0, dilation: int = 1, bias: bool = True,
                 strategy: Optional[Conv1dStrategy] = None):
        super().__init__()
        self.n = n
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = kernel_size
        self.stride = stride
        self.padding = padding
        self.dilation = dilation
        self.has_bias = bias
        if strategy is None:
            strategy = Conv1dStrategy.GROUPED if n >= _GROUPED_THRESHOLD else Conv1dStrategy.SEQUENTIAL
        self.strategy = strategy
        if strategy == Conv1dStrategy.GROUPED:
            self.op = nn.Conv1d(n * in_channels, n * out_channels, kernel_size, stride=stride,
                                padding=padding, dilation=dilation, groups=n, bias=bias)
        else:
            self.weight = nn.Parameter(torch.empty(n, out_channels, in_channels, kernel_size))
            if bias:
                self.bias = nn.Parameter(torch.empty(n, out_channels))
            else:
                self.register_parameter("bias", None)
            fan_in = in_channels * kernel_size
            bound = 1.0 / math.sqrt(fan_in) if fan_in > 0 else 0.0
            for i in range(n):
                nn.init.kaiming_uniform_(self.weight[i], a=math.sqrt(5))
                if self.bias is not None:
                    nn.init.uniform_(self.bias[i], -bound, bound)
        self.fused_bn = None
        self.fused_activation = None
        self._register_load_state_dict_pre_hook(self._load_any_layout)

    def _load_any_layout(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                         error_msgs):
        """Accept either of the reference's layouts, whichever strategy this module uses: the
        reference picks ``op.*`` (grouped, N >= 10) or ``weight`` / ``bias`` (sequential) from N
        (wide_conv1d.py:80-105), so a checkpoint of one strategy loads into the other here."""
        n, co, ci, k = self.n, self.out_channels, self.in_channels, self.kernel_size
        grouped = self.strategy == Conv1dStrategy.GROUPED
        src, dst = (("weight", "bias"), ("op.weight", "op.bias")) if grouped else \
            (("op.weight", "op.bias"), ("weight", "bias"))
        if prefix + src[0] not in state_dict or prefix + dst[0] in state_dict:
            return
        w = state_dict.pop(prefix + src[0])
        state_dict[prefix + dst[0]] = w.reshape(n * co, ci, k) if grouped else w.reshape(n, co, ci, k)
        if prefix + src[1] in state_dict:
            b = state_dict.pop(prefix + src[1])
            state_dict[prefix + dst[1]] = b.reshape(-1) if grouped else b.reshape(n, co)

    # uniform view of the filters for the kernel: [N*C_out, C_in, 1, k] and [N*C_out]
    def _filters(self):
        if self.strategy == Conv1dStrategy.GROUPED:
            w, b = self.op.weight, self.op.bias
        else:
            w, b = self.weight, self.bias
        w = w.reshape(self.n * self.out_channels, self.in_channels, 1, self.kernel_size)
        return w, (None if b is None else b.reshape(-1))

    def forward(self, x: Tensor, residual: Optional[Tensor] = None) -> Tensor:
        """x [N, B, C_in, L] -> [N, B, C_out, L'] (optional fused residual of the output's shape)."""
        if x.dim() != 4:
            raise RuntimeError(f"WideConv1d: expected [N, B, C, L], got {list(x.shape)}")
        r = None if residual is None else residual.unsqueeze(3)
        return conv_forward(self, x.unsqueeze(3), one_d=True, residual=r).squeeze(3)

    @classmethod
    def from_modules(cls, modules: List[nn.Conv1d], strategy: Optional[Conv1dStrategy] = None) -> "WideConv1d":
        t = modules[0]
        if t.groups != 1:
            raise ValueError("WideConv1d.from_modules supports groups=1 convolutions")
        if isinstance(t.padding, str) or t.padding_mode != "zeros":
            raise ValueError("WideConv1d.from_modules needs numeric zero padding")
        first = lambda v: v[0] if isinstance(v, tuple) else v  # noqa: E731
        wide = cls(n=len(modules), in_channels=t.in_channels, out_channels=t.out_channels,
                   kernel_size=first(t.kernel_size), stride=first(t.stride), padding=first(t.padding),
                   dilation=first(t.dilation), bias=t.bias is not None, strategy=strategy)
        wide = wide.to(device=t.weight.device, dtype=t.weight.dtype)
        co = t.out_channels
        with torch.no_grad():
            for i, m in enumerate(modules):
                if wide.strategy == Conv1dStrategy.GROUPED:
                    wide.op.weight[i * co:(i + 1) * co].copy_(m.weight)
                    if m.bias is not None:
                        wide.op.bias[i * co:(i + 1) * co].copy_(m.bias)
                else:
                    wide.weight[i].copy_(m.weight)
                    if m.bias is not None:
                        wide.bias[i].copy_(m.bias)
        return wide

    def __repr__(self) -> str:
        return (f"WideConv1d({self.n}x[{self.in_channels}->{self.out_channels}], "
                f"k={self.kernel_size}, strategy={self.strategy.name.lower()})")


__all__ = ["WideConv1d", "Conv1dStrategy"]
