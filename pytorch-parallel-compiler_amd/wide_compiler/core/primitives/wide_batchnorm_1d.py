"""
WideBatchNorm1d: N independent eval-mode nn.BatchNorm1d(C) on [N, B, C] or [N, B, C, L]
(mirror of wide_compiler/core/primitives/wide_batchnorm_1d.py:21-107; state layout
``op`` = nn.BatchNorm1d(N*C)).  Same kernel as WideBatchNorm2d (wc_bn_eval).
"""

from __future__ import annotations

from typing import List

from torch import Tensor, nn

from .wide_batchnorm_2d import _bn_forward, _bn_from_modules


class WideBatchNorm1d(nn.Module):
    def __init__(self, n: int, num_features: int, eps: float = 1e-5, momentum: float = 0.1,
                 affine: bool = True, track_running_stats: bool = True):
        super().__init__()
        self.n = n
        self.num_features = num_features
        self.op = nn.BatchNorm1d(n * num_features, eps=eps, momentum=momentum, affine=affine,
                                 track_running_stats=track_running_stats)
        self.fused_activation = None

    def forward(self, x: Tensor) -> Tensor:
        if x.dim() not in (3, 4):
            raise RuntimeError(f"WideBatchNorm1d: expected [N, B, C] or [N, B, C, L], got {list(x.shape)}")
        return _bn_forward("WideBatchNorm1d", self.op, self.n, self.num_features, x,
                           relu=self.fused_activation == "relu")

    @classmethod
    def from_modules(cls, modules: List[nn.BatchNorm1d]) -> "WideBatchNorm1d":
        return _bn_from_modules(cls, modules)

    def __repr__(self) -> str:
        return f"WideBatchNorm1d({self.n}x{self.num_features})"


__all__ = ["WideBatchNorm1d"]
