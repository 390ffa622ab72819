"""
WideInstanceNorm1d / WideInstanceNorm2d: N independent nn.InstanceNorm1d/2d(C) on N-first
[N, B, C, L] / [N, B, C, H, W] (mirror of wide_compiler/core/primitives/wide_instancenorm.py:
21-141, 143-263).

State layout as the reference: strategy 'fused' (the default) holds ``norm`` =
nn.InstanceNorm*(N*C); 'sequential' holds ``norms`` = N nn.InstanceNorm*(C).  The forward
follows nn.InstanceNorm: instance statistics (one wc_group_norm launch with one group per
channel) unless the module tracks running statistics and is in eval mode, where the
running statistics are used (one wc_bn_eval launch).  Training mode with running-statistic
tracking would update buffers and raises (forward-only build).
"""

from __future__ import annotations

from enum import Enum
from typing import Union

import torch
from torch import Tensor, nn

from ... import _hip
from .wide_groupnorm import group_norm_forward, stacked_affine


class InstanceNormStrategy(Enum):
    FUSED = "fused"
    SEQUENTIAL = "sequential"
    AUTO = "auto"


class _WideInstanceNorm(nn.Module):
    _norm_cls = nn.InstanceNorm1d
    _name = "WideInstanceNorm"
    _dims = 4

    def __init__(self, n: int, num_features: int, eps: float = 1e-5, momentum: float = 0.1,
                 affine: bool = False, track_running_stats: bool = False,
                 strategy: Union[str, InstanceNormStrategy] = "auto"):
        super().__init__()
        self.n = n
        self.num_features = num_features
        self.eps = eps
        self.momentum = momentum
        self.affine = affine
        self.track_running_stats = track_running_stats
        if isinstance(strategy, str):
            strategy = InstanceNormStrategy(strategy)
        if strategy == InstanceNormStrategy.AUTO:
            strategy = InstanceNormStrategy.FUSED
        self._strategy = strategy
        self._use_fused = strategy == InstanceNormStrategy.FUSED
        kw = dict(eps=eps, momentum=momentum, affine=affine, track_running_stats=track_running_stats)
        if self._use_fused:
            self.norm = self._norm_cls(n * num_features, **kw)
        else:
            self.norms = nn.ModuleList([self._norm_cls(num_features, **kw) for _ in range(n)])
        self.fused_activation = None

    @property
    def strategy(self) -> InstanceNormStrategy:
        return self._strategy

    def forward(self, x: Tensor) -> Tensor:
        what = self._name
        if x.dim() != self._dims:
            raise RuntimeError(f"{what}: expected a {self._dims}-d N-first input, got {list(x.shape)}")
        n, c = self.n, self.num_features
        relu = self.fused_activation == "relu"
        mods = [self.norm] if self._use_fused else list(self.norms)
        if self._use_fused:
            w, b = self.norm.weight, self.norm.bias
        else:
            w, b = stacked_affine(self.norms)
        if self.track_running_stats:
            if any(m.training for m in mods):
                raise RuntimeError(f"{what}: training mode with running statistics updates buffers; this "
                                   "forward-only build supports eval mode (call .eval())")
            if self._use_fused:
                rm, rv = self.norm.running_mean, self.norm.running_var
            else:
                rm = torch.cat([m.running_mean for m in self.norms])
                rv = torch.cat([m.running_var for m in self.norms])
            if x.shape[0] != n or x.shape[2] != c:
                raise RuntimeError(f"{what}: expected [N={n}, B, C={c}, ...], got {list(x.shape)}")
            _hip.require_device(what, x, rm)
            _hip.require_forward_only(what, x, w, b)
            x = x.contiguous()
            hw = 1
            for d in x.shape[3:]:
                hw *= d
            out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
            if out.numel():
                _hip.bn_eval(x, x.stride(0), x.stride(1), w, b, rm, rv, self.eps, out, n, x.shape[1], c, hw,
                             relu=relu)
            return out
        return group_norm_forward(what, x, n, c, c, w, b, self.eps, relu=relu)

    @classmethod
    def from_modules(cls, modules, strategy: Union[str, InstanceNormStrategy] = "auto"):
        t = modules[0]
        wide = cls(n=len(modules), num_features=t.num_features, eps=t.eps, momentum=t.momentum,
                   affine=t.affine, track_running_stats=t.track_running_stats, strategy=strategy)
        if t.affine:
            wide = wide.to(device=t.weight.device, dtype=t.weight.dtype)
            with torch.no_grad():
                if wide._use_fused:
                    wide.norm.weight.copy_(torch.cat([m.weight for m in modules], dim=0))
                    wide.norm.bias.copy_(torch.cat([m.bias for m in modules], dim=0))
                else:
                    for i, m in enumerate(modules):
                        wide.norms[i].load_state_dict(m.state_dict())
        return wide

    def __repr__(self) -> str:
        return f"{self._name}({self.n}x[{self.num_features}], strategy={self._strategy.value})"


class WideInstanceNorm1d(_WideInstanceNorm):
    _norm_cls = nn.InstanceNorm1d
    _name = "WideInstanceNorm1d"
    _dims = 4


class WideInstanceNorm2d(_WideInstanceNorm):
    _norm_cls = nn.InstanceNorm2d
    _name = "WideInstanceNorm2d"
    _dims = 5


__all__ = ["WideInstanceNorm1d", "WideInstanceNorm2d", "InstanceNormStrategy"]
