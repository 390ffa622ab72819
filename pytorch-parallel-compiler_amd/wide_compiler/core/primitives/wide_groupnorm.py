"""
WideGroupNorm: N independent nn.GroupNorm(G, C) on N-first [N, B, C, *spatial]
(mirror of wide_compiler/core/primitives/wide_groupnorm.py:29-181).

State layout as the reference: strategy 'fused' (the default) holds ``norm`` =
nn.GroupNorm(N*G, N*C), whose weight / bias hold model i's channel c at index i*C + c;
'sequential' holds ``norms`` = N nn.GroupNorm(G, C).  Either way the forward is one
wc_group_norm launch on the N-first tensor (a per-(model, batch row, group) row of
(C / G) * spatial contiguous elements): no permute copies.
"""

from __future__ import annotations

from enum import Enum
from typing import List, Optional, Tuple, Union

import torch
from torch import Tensor, nn

from ... import _hip


class GroupNormStrategy(Enum):
    FUSED = "fused"
    SEQUENTIAL = "sequential"
    AUTO = "auto"


def group_norm_forward(what: str, x: Tensor, n: int, c: int, groups: int, weight: Optional[Tensor],
                       bias: Optional[Tensor], eps: float, relu: bool = False) -> Tensor:
    """x [n, B, c, *spatial] -> normalised copy (contiguous), statistics per (model, batch row, group)."""
    if x.dim() < 3 or x.shape[0] != n or x.shape[2] != c:
        raise RuntimeError(f"{what}: expected [N={n}, B, C={c}, ...], got {list(x.shape)}")
    _hip.require_device(what, x, weight, bias)
    _hip.require_forward_only(what, x, weight, bias)
    x = x.contiguous()
    s = 1
    for d in x.shape[3:]:
        s *= d
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if out.numel():
        _hip.group_norm(x, out, n, x.shape[1], c, s, groups, weight, bias, eps, relu=relu)
    return out


def stacked_affine(norms) -> Tuple[Optional[Tensor], Optional[Tensor]]:
    """weight / bias of N separate norm modules as [N*C] tensors (None when not affine)."""
    if norms[0].weight is None:
        return None, None
    return torch.cat([m.weight for m in norms]), torch.cat([m.bias for m in norms])


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
        if strategy == GroupNormStrategy.AUTO:
            strategy = GroupNormStrategy.FUSED
        self._strategy = strategy
        self._use_fused = strategy == GroupNormStrategy.FUSED
        if self._use_fused:
            self.norm = nn.GroupNorm(n * num_groups, n * num_channels, eps=eps, affine=affine)
        else:
            self.norms = nn.ModuleList([nn.GroupNorm(num_groups, num_channels, eps=eps, affine=affine)
                                        for _ in range(n)])
        self.fused_activation = None

    @property
    def strategy(self) -> GroupNormStrategy:
        return self._strategy

    def forward(self, x: Tensor) -> Tensor:
        if self._use_fused:
            w, b = self.norm.weight, self.norm.bias
        else:
            w, b = stacked_affine(self.norms)
        return group_norm_forward("WideGroupNorm", x, self.n, self.num_channels, self.num_groups, w, b, self.eps,
                                  relu=self.fused_activation == "relu")

    @classmethod
    def from_modules(cls, modules: List[nn.GroupNorm],
                     strategy: Union[str, GroupNormStrategy] = "auto") -> "WideGroupNorm":
        t = modules[0]
        wide = cls(n=len(modules), num_groups=t.num_groups, num_channels=t.num_channels, eps=t.eps,
                   affine=t.affine, strategy=strategy)
        if t.affine:
            device, dtype = t.weight.device, t.weight.dtype
        else:
            device, dtype = torch.device("cpu"), torch.float32
        wide = wide.to(device=device, dtype=dtype)
        with torch.no_grad():
            if wide._use_fused and wide.affine:
                wide.norm.weight.copy_(torch.cat([m.weight for m in modules], dim=0))
                wide.norm.bias.copy_(torch.cat([m.bias for m in modules], dim=0))
            elif not wide._use_fused and wide.affine:
                for i, m in enumerate(modules):
                    wide.norms[i].load_state_dict(m.state_dict())
        return wide

    def __repr__(self) -> str:
        return (f"WideGroupNorm({self.n}x[groups={self.num_groups}, channels={self.num_channels}], "
                f"strategy={self._strategy.value})")


__all__ = ["WideGroupNorm", "GroupNormStrategy", "group_norm_forward", "stacked_affine"]
