"""
WideBatchNorm2d: N independent eval-mode nn.BatchNorm2d(C)
(mirror of wide_compiler/core/primitives/wide_batchnorm_2d.py:21-107).

Parameters and buffers keep the reference layout: ``op`` is an nn.BatchNorm2d(N*C) whose
weight / bias / running_mean / running_var hold model i's channel c at index i*C + c.
The forward is one HBM-bound kernel (wc_bn_eval) on the N-first tensor -- no permute
copies.  Only inference is supported: training-mode statistics raise (forward-only build).
"""

from __future__ import annotations

from typing import List

import torch
from torch import Tensor, nn

from ... import _hip
from .._layout import inner_block_contiguous


def _bn_forward(what: str, op: nn.modules.batchnorm._BatchNorm, n: int, c: int, x: Tensor,
                relu: bool = False) -> Tensor:
    if op.training or not op.track_running_stats or op.running_mean is None:
        raise RuntimeError(
            f"{what}: only eval-mode BatchNorm with running statistics is supported by the "
            "forward-only HIP kernels; call .eval()"
        )
    if x.dim() < 3 or x.shape[0] != n or x.shape[2] != c:
        raise RuntimeError(f"{what}: expected [N={n}, B, C={c}, ...], got {list(x.shape)}")
    _hip.require_device(what, x, op.running_mean)
    _hip.require_forward_only(what, x, op.weight, op.bias)
    if not inner_block_contiguous(x, 2):
        x = x.contiguous()
    b = x.shape[1]
    hw = 1
    for s in x.shape[3:]:
        hw *= s
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if out.numel():
        _hip.bn_eval(x, x.stride(0), x.stride(1), op.weight, op.bias, op.running_mean, op.running_var,
                     op.eps, out, n, b, c, hw, relu=relu)
    return out


class WideBatchNorm2d(nn.Module):
    def __init__(self, n: int, num_features: int, eps: float = 1e-5, momentum: float = 0.1,
                 affine: bool = True, track_running_stats: bool = True):
        super().__init__()
        self.n = n
        self.num_features = num_features
        self.op = nn.BatchNorm2d(n * num_features, eps=eps, momentum=momentum, affine=affine,
                                 track_running_stats=track_running_stats)
        self.fused_activation = None

    def forward(self, x: Tensor) -> Tensor:
        if x.dim() != 5:
            raise RuntimeError(f"WideBatchNorm2d: expected [N, B, C, H, W], got {list(x.shape)}")
        return _bn_forward("WideBatchNorm2d", self.op, self.n, self.num_features, x,
                           relu=self.fused_activation == "relu")

    @classmethod
    def from_modules(cls, modules: List[nn.BatchNorm2d]) -> "WideBatchNorm2d":
        return _bn_from_modules(cls, modules)

    def __repr__(self) -> str:
        return f"WideBatchNorm2d({self.n}x{self.num_features})"


def _bn_from_modules(cls, modules):
    t = modules[0]
    wide = cls(n=len(modules), num_features=t.num_features, eps=t.eps, momentum=t.momentum,
               affine=t.affine, track_running_stats=t.track_running_stats)
    ref = t.weight if t.weight is not None else t.running_mean
    wide = wide.to(device=ref.device if ref is not None else "cpu",
                   dtype=ref.dtype if ref is not None else torch.float32)
    c = t.num_features
    with torch.no_grad():
        for i, m in enumerate(modules):
            sl = slice(i * c, (i + 1) * c)
            if m.weight is not None:
                wide.op.weight[sl].copy_(m.weight)
            if m.bias is not None:
                wide.op.bias[sl].copy_(m.bias)
            if m.running_mean is not None:
                wide.op.running_mean[sl].copy_(m.running_mean)
            if m.running_var is not None:
                wide.op.running_var[sl].copy_(m.running_var)
    wide.train(t.training)
    return wide


__all__ = ["WideBatchNorm2d"]
