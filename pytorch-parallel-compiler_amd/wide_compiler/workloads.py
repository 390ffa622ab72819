"""
Seeded synthetic workloads of the benchmark configurations (synthetic data, random init).

Model i of a configuration is built under ``torch.manual_seed(SEED + i)`` with the
torch.nn default initialisation; inputs come from a separate ``torch.Generator`` seeded
with ``SEED``.  Each builder returns CPU modules and CPU inputs so that the same objects
feed both the HIP path (after ``.to('cuda')``) and the CPU oracle.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

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


def attention_n16(n: int = 16, batch: int = 8, seq: int = 512, embed: int = 256, heads: int = 8) -> Workload:
    """N=16 nn.MultiheadAttention(256, 8 heads, batch_first; xavier-uniform in-projection, the nn
    default), bf16; self-attention input x [16, 8, 512, 256] ~ N(0, 1), no mask."""
    models = []
    for i in range(n):
        torch.manual_seed(SEED + i)
        models.append(nn.MultiheadAttention(embed, heads, batch_first=True).to(torch.bfloat16).eval())
    x = torch.randn(n, batch, seq, embed, generator=_gen()).to(torch.bfloat16)
    return Workload(f"WideAttention MHA(256, 8 heads) N={n} B={batch} S={seq} bf16", n, batch, models, {"x": x})


class SeqModel(nn.Module):
    """Embedding(8192, 256) - LayerNorm(256) - LSTM(256 -> 512, batch_first) - Linear(512 -> 8192):
    one small token model; ids [B, T] -> logits [B, T, 8192]."""

    def __init__(self, vocab: int = 8192, dim: int = 256, hidden: int = 512):
        super().__init__()
        self.emb = nn.Embedding(vocab, dim)          # init ~ N(0, 1) (the nn default)
        self.ln = nn.LayerNorm(dim)
        self.lstm = nn.LSTM(dim, hidden, batch_first=True)
        self.fc = nn.Linear(hidden, vocab)

    def forward(self, ids):
        h, _ = self.lstm(self.ln(self.emb(ids)))
        return self.fc(h)


class WideSeqModel(nn.Module):
    """N SeqModels fused primitive by primitive: per-model embedding gather (each model reads
    its own ids) with the N-first LayerNorm applied as the rows are gathered, WideLSTM,
    WideLinear over the vocabulary.  The wide
    primitives are the reference's (wide_embedding.py, wide_layernorm.py, wide_lstm.py,
    wide_linear.py); the composition is not traced because the LSTM returns a tuple."""

    def __init__(self, models: List[SeqModel]):
        super().__init__()
        from .core.primitives import WideEmbedding, WideLayerNorm, WideLinear, WideLSTM
        self.n = len(models)
        self.emb = WideEmbedding.from_modules([m.emb for m in models])
        self.ln = WideLayerNorm.from_modules([m.ln for m in models])
        self.lstm = WideLSTM.from_modules([m.lstm for m in models])
        self.fc = WideLinear.from_modules([m.fc for m in models])

    def forward(self, ids: torch.Tensor, out: Optional[torch.Tensor] = None, return_state: bool = False):
        """ids [N, B, T] (model i uses row i) -> logits [N, B, T, V]; with ``return_state``
        (logits, lstm_out [N, B, T, H], (h_n, c_n)) from the same launches.  The launches
        are asynchronous: a bounded wait of the LSTM recurrence that gave up is raised by
        ``wide_compiler._hip.rnn_sync_check(block=True)`` (or the next recurrent call)."""
        x = self.emb.forward_layernorm(ids, self.ln, per_model=True)   # = self.ln(self.emb(ids, ...))
        h, state = self.lstm(x)
        y = self.fc.forward_into(h, out)
        return (y, h, state) if return_state else y


def seq_n64(n: int = 64, batch: int = 16, steps: int = 128, vocab: int = 8192, dim: int = 256,
            hidden: int = 512) -> Workload:
    """N=64 SeqModels, weights bf16 (fp32 accumulate, fp32 cell state in the kernels);
    ids [64, 16, 128] uniform int64 in [0, 8192)."""
    models = []
    for i in range(n):
        torch.manual_seed(SEED + i)
        models.append(SeqModel(vocab, dim, hidden).to(torch.bfloat16).eval())
    ids = torch.randint(0, vocab, (n, batch, steps), generator=_gen(), dtype=torch.int64)
    return Workload(f"Emb-LN-LSTM-Linear N={n} B={batch} T={steps} V={vocab} {dim}->{hidden} bf16",
                    n, batch, models, {"ids": ids})


def seq_params(models: List[SeqModel]) -> Dict[str, object]:
    """The wide parameter layout of a list of SeqModels, as the oracle's seq_model takes it
    (LSTM weights in the compact per-model form [N, 4H, I] / [N, 4H, H])."""
    st = lambda ts: torch.stack([t.detach().cpu() for t in ts])  # noqa: E731
    return {
        "emb.weight": st([m.emb.weight for m in models]),
        "ln.weight": torch.cat([m.ln.weight.detach().cpu() for m in models]),
        "ln.bias": torch.cat([m.ln.bias.detach().cpu() for m in models]),
        "ln.eps": models[0].ln.eps,
        "lstm.weight_ih": st([m.lstm.weight_ih_l0 for m in models]),
        "lstm.weight_hh": st([m.lstm.weight_hh_l0 for m in models]),
        "lstm.bias_ih": st([m.lstm.bias_ih_l0 for m in models]),
        "lstm.bias_hh": st([m.lstm.bias_hh_l0 for m in models]),
        "fc.weight": st([m.fc.weight for m in models]),
        "fc.bias": st([m.fc.bias for m in models]),
    }
