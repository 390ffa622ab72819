"""Shared helpers of the test-suite."""

from __future__ import annotations

import torch

# parity bars (normwise: max |a - b| / max |b|)
TOL_F32 = 1e-5
TOL_BF16 = 2e-2


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.abs().max().item()
    num = (a - b).abs().max().item()
    return num / den if den > 0 else num


def tol(dtype: torch.dtype) -> float:
    return TOL_F32 if dtype == torch.float32 else TOL_BF16


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g
