"""
WideAttention: N independent nn.MultiheadAttention modules
(mirror of wide_compiler/core/primitives/wide_attention.py:25-356).

    attn(x)            x [N, B, T, D] self-attention          -> Tensor [N, B, T, D]
    attn(q, k, v)      [N, B, Tq, D], [N, B, Tkv, D] (MHA)    -> (Tensor [N, B, Tq, D], None)

Parameters keep the reference layout: q_weight [N, D, D], kv_weight [N, 2D, D],
out_weight [N, D, D], q_bias [N, D], kv_bias [N, 2D], out_bias [N, D].
"""

from __future__ import annotations

from enum import Enum
from typing import List, Optional, Tuple, Union

import torch
from torch import Tensor, nn

from ... import _hip


class AttentionStrategy(Enum):
    FUSED = "fused"
    SEQUENTIAL = "sequential"
    AUTO = "auto"


class WideAttention(nn.Module):
    def __init__(self, n: int, d_model: int, n_heads: int, dropout: float = 0.0, bias: bool = True,
                 strategy: Union[str, AttentionStrategy] = "auto"):
        super().__init__()
        assert d_model % n_heads == 0, f"d_model ({d_model}) must be divisible by n_heads ({n_heads})"
        self.n = n
        self.d_model = d_model
        self.n_heads = n_heads
        self.d_head = d_model // n_heads
        self.dropout = dropout
        self.has_bias = bias
        if isinstance(strategy, str):
            strategy = AttentionStrategy(strategy)
        if strategy == AttentionStrategy.AUTO:
            strategy = AttentionStrategy.FUSED
        self._strategy = strategy
        self.q_weight = nn.Parameter(torch.empty(n, d_model, d_model))
        self.kv_weight = nn.Parameter(torch.empty(n, 2 * d_model, d_model))
        if bias:
            self.q_bias = nn.Parameter(torch.empty(n, d_model))
            self.kv_bias = nn.Parameter(torch.empty(n, 2 * d_model))
        else:
            self.register_parameter("q_bias", None)
            self.register_parameter("kv_bias", None)
        self.out_weight = nn.Parameter(torch.empty(n, d_model, d_model))
        if bias:
            self.out_bias = nn.Parameter(torch.empty(n, d_model))
        else:
            self.register_parameter("out_bias", None)
        self._reset_parameters()

    @property
    def strategy(self) -> AttentionStrategy:
        return self._strategy

    def _reset_parameters(self) -> None:
        d = self.d_model
        for i in range(self.n):
            nn.init.xavier_uniform_(self.q_weight[i])
            nn.init.xavier_uniform_(self.kv_weight[i].view(2, d, d))
            nn.init.xavier_uniform_(self.out_weight[i])
            for b in (self.q_bias, self.kv_bias, self.out_bias):
                if b is not None:
                    nn.init.zeros_(b[i])

    def forward(self, query: Tensor, key: Optional[Tensor] = None, value: Optional[Tensor] = None,
                attn_mask: Optional[Tensor] = None, is_causal: bool = False,
                need_weights: bool = False) -> Union[Tensor, Tuple[Tensor, None]]:
        raise NotImplementedError("WideAttention: the attention kernel is not built yet")

    @classmethod
    def from_modules(cls, modules: List[nn.MultiheadAttention],
                     strategy: Union[str, AttentionStrategy] = "auto") -> "WideAttention":
        t = modules[0]
        if not t._qkv_same_embed_dim:
            raise ValueError("WideAttention.from_modules needs kdim == vdim == embed_dim")
        if t.bias_k is not None or t.add_zero_attn:
            raise ValueError("WideAttention.from_modules does not support add_bias_kv / add_zero_attn")
        wide = cls(n=len(modules), d_model=t.embed_dim, n_heads=t.num_heads, dropout=t.dropout,
                   bias=t.in_proj_bias is not None, strategy=strategy)
        wide = wide.to(device=t.in_proj_weight.device, dtype=t.in_proj_weight.dtype)
        d = t.embed_dim
        with torch.no_grad():
            for i, m in enumerate(modules):
                w = m.in_proj_weight
                wide.q_weight[i].copy_(w[:d])
                wide.kv_weight[i].copy_(w[d:])
                if m.in_proj_bias is not None:
                    wide.q_bias[i].copy_(m.in_proj_bias[:d])
                    wide.kv_bias[i].copy_(m.in_proj_bias[d:])
                wide.out_weight[i].copy_(m.out_proj.weight)
                if m.out_proj.bias is not None and wide.out_bias is not None:
                    wide.out_bias[i].copy_(m.out_proj.bias)
        return wide

    def __repr__(self) -> str:
        return (f"WideAttention({self.n}x[d={self.d_model}, h={self.n_heads}], "
                f"strategy={self._strategy.value})")


__all__ = ["WideAttention", "AttentionStrategy"]
