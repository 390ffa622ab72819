"""
WideGroupNorm (construction / state layout of wide_compiler/core/primitives/wide_groupnorm.py:
``op`` = nn.GroupNorm(N*G, N*C)).  Not on the hot path yet.
"""

from __future__ import annotations

from enum import Enum
from typing import List, Union

import torch
from torch import Tensor, nn

from ._unported import not_on_hot_path


class GroupNormStrategy(Enum):
    AUTO = "auto"
    GROUPED = "grouped"
    SEQUENTIAL = "sequential"


class WideGroupNorm(nn.Module):
    def __init__(self, n: int, num_groups: int, num_channels: int, eps: float = 1e-5, affine: bool = True,
                 strategy: Union[str, GroupNormStrategy] = "auto"):
        super().__init__()
        self.n = n
        self.num_groups = num_groups
        self.num_channels = num_channels
        self.eps = eps
        self.affine = affine
        if isinstance(strategy, str):
            strategy = GroupNormStrategy(strategy)
        self._strategy = GroupNormStrategy.GROUPED if strategy == GroupNormStrategy.AUTO else strategy
        self.op = nn.GroupNorm(n * num_groups, n * num_channels, eps=eps, affine=affine)

    @property
    def strategy(self) -> GroupNormStrategy:
        return self._strategy

    def forward(self, x: Tensor) -> Tensor:
        not_on_hot_path("WideGroupNorm")

    @classmethod
    def from_modules(cls, modules: List[nn.GroupNorm], strategy="auto") -> "WideGroupNorm":
        t = modules[0]
        wide = cls(len(modules), t.num_groups, t.num_channels, t.eps, t.affine, strategy)
        if t.weight is not None:
            wide = wide.to(device=t.weight.device, dtype=t.weight.dtype)
            c = t.num_channels
            with torch.no_grad():
                for i, m in enumerate(modules):
                    wide.op.weight[i * c:(i + 1) * c].copy_(m.weight)
                    wide.op.bias[i * c:(i + 1) * c].copy_(m.bias)
        return wide

    def __repr__(self) -> str:
        return f"WideGroupNorm({self.n}x[{self.num_groups}g, {self.num_channels}c])"


__all__ = ["WideGroupNorm", "GroupNormStrategy"]
