"""
Seeded synthetic workloads of the benchmark configurations (synthetic data, random init).

Model i of a configuration is built under ``torch.manual_seed(SEED + i)`` with the
torch.nn default initialisation; inputs come from a separate ``torch.Generator`` seeded
with ``SEED``.  Each builder returns CPU modules and CPU inputs so that the same objects
feed both the HIP path (after ``.to('cuda')``) and the CPU oracle.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List

import torch
import torch.nn as nn
import torch.nn.functional as F

SEED = 20260101


class MLP(nn.Module):
    """Linear(64,128) - ReLU - Linear(128,64): the reference CLI's sample MLP (cli.py:59-67)."""

    def __init__(self, d_in: int = 64, d_hidden: int = 128, d_out: int = 64):
        super().__init__()
        self.fc1 = nn.Linear(d_in, d_hidden)
        self.fc2 = nn.Linear(d_hidden, d_out)

    def forward(self, x):
        return self.fc2(F.relu(self.fc1(x)))


@dataclass
class Workload:
    name: str
    n: int
    batch: int
    models: List[nn.Module]
    inputs: Dict[str, torch.Tensor]


def _gen(seed: int = SEED) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def mlp_n100(n: int = 100, batch: int = 32) -> Workload:
    """N=100 MLPs, fp32; 100 inputs [32, 64] ~ N(0, 1) channel-packed to [32, 6400]."""
    models = []
    for i in range(n):
        torch.manual_seed(SEED + i)
        models.append(MLP())
    g = _gen()
    xs = [torch.randn(batch, 64, generator=g) for _ in range(n)]
    return Workload("TracedWideModel MLP(64-128-64) N=100 B=32 fp32", n, batch, models, {"per_model": xs})


def gru_n32(n: int = 32, batch: int = 4, steps: int = 32, in_size: int = 64, hidden: int = 128) -> Workload:
    """N=32 nn.GRU(64, 128, batch_first); x [32, 4, 32, 64] ~ N(0, 1) fp32, h0 = 0."""
    models = []
    for i in range(n):
        torch.manual_seed(SEED + i)
        models.append(nn.GRU(in_size, hidden, batch_first=True))
    x = torch.randn(n, batch, steps, in_size, generator=_gen())
    return Workload(f"WideGRU N={n} B={batch} T={steps} {in_size}->{hidden} fp32", n, batch, models, {"x": x})


class ResBlock(nn.Module):
    """conv3x3 - BN - ReLU - conv3x3 - BN - (+x) - ReLU: the reference CLI's ResBlock (cli.py:84-97)."""

    def __init__(self, channels: int = 64):
        super().__init__()
        self.conv1 = nn.Conv2d(channels, channels, 3, padding=1)
        self.bn1 = nn.BatchNorm2d(channels)
        self.conv2 = nn.Conv2d(channels, channels, 3, padding=1)
        self.bn2 = nn.BatchNorm2d(channels)

    def forward(self, x):
        identity = x
        out = F.relu(self.bn1(self.conv1(x)))
        out = self.bn2(self.conv2(out))
        return F.relu(out + identity)


def resblock_n100(n: int = 100, batch: int = 8, channels: int = 64, hw: int = 32) -> Workload:
    """N=100 ResBlock(64) in eval mode, everything bf16.  BatchNorm running mean 0 / var 1 (the
    nn defaults), affine weight ~ N(1, 0.1) and bias ~ N(0, 0.1) (the configuration text gives
    both as "~N(1, 0.1)"; a zero-centred shift keeps the residual path balanced, recorded as a
    choice of this build).  Input [8, 6400, 32, 32] ~ N(0, 1), channel-packed."""
    models = []
    for i in range(n):
        torch.manual_seed(SEED + i)
        m = ResBlock(channels)
        with torch.no_grad():
            for bn in (m.bn1, m.bn2):
                bn.weight.normal_(1.0, 0.1)
                bn.bias.normal_(0.0, 0.1)
        models.append(m.to(torch.bfloat16).eval())
    x = torch.randn(batch, n * channels, hw, hw, generator=_gen()).to(torch.bfloat16)
    return Workload(f"TracedWideModel ResBlock(64) N={n} B={batch} 32x32 bf16", n, batch, models, {"packed": x})


def resblock_params(models: List[nn.Module], dtype: torch.dtype) -> Dict[str, object]:
    """The reference wide layout of a list of ResBlocks (grouped conv filters, flat BN params)."""
    p: Dict[str, object] = {}
    for name in ("conv1", "conv2"):
        p[f"{name}.weight"] = torch.cat([getattr(m, name).weight.detach().cpu() for m in models]).to(dtype)
        p[f"{name}.bias"] = torch.cat([getattr(m, name).bias.detach().cpu() for m in models]).to(dtype)
    for name in ("bn1", "bn2"):
        for k in ("weight", "bias", "running_mean", "running_var"):
            p[f"{name}.{k}"] = torch.cat([getattr(getattr(m, name), k).detach().cpu() for m in models]).to(dtype)
        p[f"{name}.eps"] = getattr(models[0], name).eps
    return p
