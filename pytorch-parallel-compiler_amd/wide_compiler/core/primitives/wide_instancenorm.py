"""
WideInstanceNorm1d / 2d (construction / state layout of
wide_compiler/core/primitives/wide_instancenorm.py: ``op`` = nn.InstanceNorm*(N*C)).
Not on the hot path yet.
"""

from __future__ import annotations

from enum import Enum
from typing import List, Union

import torch
from torch import Tensor, nn

from ._unported import not_on_hot_path


class InstanceNormStrategy(Enum):
    AUTO = "auto"
    GROUPED = "grouped"
    SEQUENTIAL = "sequential"


class _WideInstanceNorm(nn.Module):
    _norm_cls = None
    _name = ""

    def __init__(self, n: int, num_features: int, eps: float = 1e-5, momentum: float = 0.1,
                 affine: bool = False, track_running_stats: bool = False,
                 strategy: Union[str, InstanceNormStrategy] = "auto"):
        super().__init__()
        self.n = n
        self.num_features = num_features
        if isinstance(strategy, str):
            strategy = InstanceNormStrategy(strategy)
        self._strategy = InstanceNormStrategy.GROUPED if strategy == InstanceNormStrategy.AUTO else strategy
        self.op = self._norm_cls(n * num_features, eps=eps, momentum=momentum, affine=affine,
                                 track_running_stats=track_running_stats)

    @property
    def strategy(self) -> InstanceNormStrategy:
        return self._strategy

    def forward(self, x: Tensor) -> Tensor:
        not_on_hot_path(self._name)

    @classmethod
    def from_modules(cls, modules, strategy="auto"):
        t = modules[0]
        wide = cls(len(modules), t.num_features, t.eps, t.momentum, t.affine, t.track_running_stats, strategy)
        ref = t.weight if t.weight is not None else t.running_mean
        if ref is not None:
            wide = wide.to(device=ref.device, dtype=ref.dtype)
        c = t.num_features
        with torch.no_grad():
            for i, m in enumerate(modules):
                sl = slice(i * c, (i + 1) * c)
                for name in ("weight", "bias", "running_mean", "running_var"):
                    src = getattr(m, name)
                    if src is not None:
                        getattr(wide.op, name)[sl].copy_(src)
        return wide

    def __repr__(self) -> str:
        return f"{self._name}({self.n}x{self.num_features})"


class WideInstanceNorm1d(_WideInstanceNorm):
    _norm_cls = nn.InstanceNorm1d
    _name = "WideInstanceNorm1d"


class WideInstanceNorm2d(_WideInstanceNorm):
    _norm_cls = nn.InstanceNorm2d
    _name = "WideInstanceNorm2d"


__all__ = ["WideInstanceNorm1d", "WideInstanceNorm2d", "InstanceNormStrategy"]
