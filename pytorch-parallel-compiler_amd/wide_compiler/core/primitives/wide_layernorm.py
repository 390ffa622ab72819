"""
WideLayerNorm: N independent nn.LayerNorm(D) over the last dim
(mirror of wide_compiler/core/primitives/wide_layernorm.py:21-88).

    x [N, *batch, D] -> (x - mean) / sqrt(var + eps) * weight[i] + bias[i]

Parameters keep the reference's flat layout (weight, bias [N*D]).  One wave-reduction
kernel (wc_layernorm) reads each row once and writes it once, statistics in fp32.
"""

from __future__ import annotations

from typing import List

import torch
from torch import Tensor, nn

from ... import _hip
from .._layout import rows_or_contiguous


class WideLayerNorm(nn.Module):
    def __init__(self, n: int, normalized_shape: int, eps: float = 1e-5):
        super().__init__()
        self.n = n
        self.normalized_shape = normalized_shape
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(n * normalized_shape))
        self.bias = nn.Parameter(torch.zeros(n * normalized_shape))

    def forward(self, x: Tensor) -> Tensor:
        what = "WideLayerNorm"
        d = self.normalized_shape
        if x.dim() < 2 or x.shape[0] != self.n or x.shape[-1] != d:
            raise RuntimeError(f"{what}: expected [N={self.n}, ..., {d}], got {list(x.shape)}")
        _hip.require_device(what, x, self.weight, self.bias)
        _hip.require_forward_only(what, x, self.weight, self.bias)
        x, r = rows_or_contiguous(x)
        if r.rows_inner != r.rows and r.rows > 1:
            x = x.contiguous()
            x, r = rows_or_contiguous(x)
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        if out.numel() == 0:
            return out
        row_stride = r.stride_inner if r.rows > 1 else d
        _hip.layernorm(x, r.stride_n, row_stride, self.weight, self.bias, out, r.rows * d, d,
                       self.n, r.rows, d, self.eps)
        return out

    @classmethod
    def from_modules(cls, modules: List[nn.LayerNorm]) -> "WideLayerNorm":
        t = modules[0]
        shape = t.normalized_shape
        if isinstance(shape, (tuple, list)):
            if len(shape) != 1:
                raise ValueError("WideLayerNorm supports a single normalized dimension")
            shape = shape[0]
        wide = cls(len(modules), shape, t.eps)
        wide = wide.to(device=t.weight.device, dtype=t.weight.dtype)
        with torch.no_grad():
            for i, m in enumerate(modules):
                wide.weight[i * shape:(i + 1) * shape].copy_(m.weight)
                wide.bias[i * shape:(i + 1) * shape].copy_(m.bias)
        return wide

    def __repr__(self) -> str:
        return f"WideLayerNorm({self.n}x{self.normalized_shape})"


__all__ = ["WideLayerNorm"]
