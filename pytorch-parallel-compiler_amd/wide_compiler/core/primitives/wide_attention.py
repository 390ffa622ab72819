"""
WideAttention: N independent nn.MultiheadAttention modules
(mirror of wide_compiler/core/primitives/wide_attention.py:25-356).

    attn(x)            x [N, B, T, D] self-attention          -> Tensor [N, B, T, D]
    attn(q, k, v)      [N, B, Tq, D], [N, B, Tkv, D] (MHA)    -> (Tensor [N, B, Tq, D], None)

Parameters keep the reference layout: q_weight [N, D, D], kv_weight [N, 2D, D],
out_weight [N, D, D], q_bias [N, D], kv_bias [N, 2D], out_bias [N, D].

Execution (every strategy): bf16 self-attention with head dim 32, at most 512 tokens and no
explicit mask runs the Q, K and V projections inside the attention kernel (wc_self_attention:
each (model, batch row, head) workgroup projects its head from x and keeps K and V in LDS).
Otherwise the Q and K/V projections are grouped MFMA GEMMs with the bias in the epilogue (one
K|V GEMM over kv_weight when key is value) and the attention core is the fused flash-style
kernel wc_attention reading Q/K/V in place in the projections' [N*B, S, heads*Dh] layout.  The
output projection is a grouped GEMM in both cases.  Inference only:
dropout in training mode raises.  ``attn_mask`` follows scaled_dot_product_attention over the
[N*B, heads, Tq, Tkv] scores (wide_attention.py:222-228): boolean (True = attend) or additive,
broadcastable to that shape, not together with ``is_causal``; a query whose keys are all masked
gets zeros, as torch's SDPA gives.
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
        # projections inside the attention kernel where it applies (False: always separate GEMMs)
        self.fuse_projections = True
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
        mha_mode = key is not None
        if key is None:
            key = query
        if value is None:
            value = key
        out = self._attend(query, key, value, attn_mask, is_causal)
        return (out, None) if mha_mode else out

    def _project(self, x: Tensor, w: Tensor, w_sn: int, bias: Optional[Tensor], b_sn: int, o: int,
                 out: Optional[Tensor] = None, col0: int = 0) -> Tensor:
        """[N, B, T, D] @ W[n]^T + b -> [N, B, T, o] via the grouped GEMM (x read in place), or into
        columns [col0, col0 + o) of ``out`` [N, B, T, C] when given."""
        from .._layout import rows_or_contiguous
        x, r = rows_or_contiguous(x)
        m = r.rows
        if out is None:
            out = torch.empty((*x.shape[:-1], o), dtype=x.dtype, device=x.device)
        width = out.shape[-1]
        _hip.grouped_gemm(n=self.n, m=m, o=o, k=self.d_model, a=x, a_sn=r.stride_n, a_so=r.stride_outer,
                          a_si=r.stride_inner, a_rows_inner=r.rows_inner, w=w, w_sn=w_sn, c=out[..., col0:],
                          c_sn=m * width, c_so=0, c_si=width, c_rows_inner=max(m, 1), bias=bias, bias_sn=b_sn)
        return out

    @staticmethod
    def _mask(attn_mask: Tensor, is_causal: bool, nb: int, hh: int, tq: int, tkv: int, dev) -> Tensor:
        """attn_mask (SDPA semantics over [N*B, heads, Tq, Tkv]) as the kernel's additive fp32 view:
        broadcast dimensions keep stride 0, so a [Tq, Tkv] mask is read, not copied N*B*heads times."""
        what = "WideAttention"
        if is_causal:
            raise RuntimeError(f"{what}: attn_mask and is_causal cannot both be set (as in "
                               "scaled_dot_product_attention)")
        if attn_mask.device != dev:
            raise RuntimeError(f"{what}: attn_mask is on {attn_mask.device}, the inputs on {dev}")
        if attn_mask.dim() > 4:
            raise RuntimeError(f"{what}: attn_mask must have at most 4 dims, got {list(attn_mask.shape)}")
        if attn_mask.dtype == torch.bool:
            m = torch.zeros(attn_mask.shape, dtype=torch.float32, device=dev).masked_fill_(~attn_mask, float("-inf"))
        elif attn_mask.is_floating_point():
            m = attn_mask.float()
        else:
            raise RuntimeError(f"{what}: attn_mask must be bool or floating point, got {attn_mask.dtype}")
        if m.dim() > 0 and m.shape[-1] > 1 and m.stride(-1) != 1:
            m = m.contiguous()
        m = m.reshape((1,) * (4 - m.dim()) + tuple(m.shape))
        try:
            return m.expand(nb, hh, tq, tkv)
        except RuntimeError:
            raise RuntimeError(f"{what}: attn_mask {list(attn_mask.shape)} does not broadcast to "
                               f"[N*B={nb}, heads={hh}, Tq={tq}, Tkv={tkv}]") from None

    def _attend(self, query: Tensor, key: Tensor, value: Tensor, attn_mask: Optional[Tensor],
                is_causal: bool) -> Tensor:
        what = "WideAttention"
        n, d, hh, dh = self.n, self.d_model, self.n_heads, self.d_head
        params = (self.q_weight, self.kv_weight, self.out_weight, self.q_bias, self.kv_bias, self.out_bias)
        _hip.require_device(what, query, key, value, *params)
        _hip.require_forward_only(what, query, key, value, *params)
        if self.training and self.dropout > 0:
            raise RuntimeError(f"{what}: attention dropout in training mode is not supported (forward-only "
                               "inference kernels); call .eval()")
        for name, t in (("query", query), ("key", key), ("value", value)):
            if t.dim() != 4 or t.shape[0] != n or t.shape[3] != d:
                raise RuntimeError(f"{what}: {name} must be [N={n}, B, T, {d}], got {list(t.shape)}")
            if t.dtype != self.q_weight.dtype:
                raise RuntimeError(f"{what}: {name} dtype {t.dtype} != weight dtype {self.q_weight.dtype}")
        b, tq, tkv = query.shape[1], query.shape[2], key.shape[2]
        if key.shape[1] != b or value.shape[1] != b or value.shape[2] != tkv:
            raise RuntimeError(f"{what}: key/value must be [N, B={b}, Tkv, D] with matching Tkv")
        mask = self._mask(attn_mask, is_causal, n * b, hh, tq, tkv, query.device) if attn_mask is not None else None
        kvw = self.kv_weight if self.kv_weight.is_contiguous() else self.kv_weight.contiguous()
        qw = self.q_weight if self.q_weight.is_contiguous() else self.q_weight.contiguous()
        ow = self.out_weight if self.out_weight.is_contiguous() else self.out_weight.contiguous()
        kvb = self.kv_bias
        if query is key and key is value and self._fusable(query, mask, params):
            attn = torch.empty((n, b, tq, d), dtype=query.dtype, device=query.device)
            _hip.self_attention(x=query, q_weight=qw, kv_weight=kvw, q_bias=self.q_bias, kv_bias=kvb, o=attn,
                                heads=hh, scale=dh ** -0.5, causal=is_causal)
            return self._project(attn, ow, d * d, self.out_bias, d, d)
        if query is key and key is value:
            # self-attention: the Q and K|V GEMMs write columns [0, D) and [D, 3D) of one
            # [N, B, T, 3D] = Q | K | V buffer, which the attention kernel reads in place; the
            # parameters are read as they are on every call (no concatenated copy to go stale)
            qkv = torch.empty((n, b, tq, 3 * d), dtype=query.dtype, device=query.device)
            self._project(query, qw, d * d, self.q_bias, d, d, out=qkv, col0=0)
            self._project(query, kvw, 2 * d * d, kvb, 2 * d, 2 * d, out=qkv, col0=d)
            q, k_t, v_t = qkv, qkv[..., d:], qkv[..., 2 * d:]
            q_strides = k_strides = v_strides = (tq * 3 * d, 3 * d)
            attn = torch.empty((n, b, tq, d), dtype=query.dtype, device=query.device)
            if tq > 0:
                _hip.attention(q=q, k=k_t, v=v_t, o=attn, nb=n * b, heads=hh, sq=tq, skv=tkv, head_dim=dh,
                               q_strides=q_strides, k_strides=k_strides, v_strides=v_strides,
                               o_strides=(tq * d, d), scale=dh ** -0.5, causal=is_causal, mask=mask)
            return self._project(attn, ow, d * d, self.out_bias, d, d)
        q = self._project(query, qw, d * d, self.q_bias, d, d)
        if key is value:
            kv = self._project(key, kvw, 2 * d * d, kvb, 2 * d, 2 * d)       # [N, B, Tkv, 2D]: K | V
            k_t, v_t = kv, kv[..., d:]
            k_strides = (tkv * 2 * d, 2 * d)
            v_strides = k_strides
        else:
            k_t = self._project(key, kvw, 2 * d * d, kvb, 2 * d, d)
            v_t = self._project(value, kvw[:, d:], 2 * d * d, None if kvb is None else kvb[:, d:], 2 * d, d)
            k_strides = (tkv * d, d)
            v_strides = (tkv * d, d)
        attn = torch.empty((n, b, tq, d), dtype=query.dtype, device=query.device)
        if tq > 0 and tkv > 0:
            _hip.attention(q=q, k=k_t, v=v_t, o=attn, nb=n * b, heads=hh, sq=tq, skv=tkv, head_dim=dh,
                           q_strides=(tq * d, d), k_strides=k_strides, v_strides=v_strides, o_strides=(tq * d, d),
                           scale=dh ** -0.5, causal=is_causal, mask=mask)
        return self._project(attn, ow, d * d, self.out_bias, d, d)

    def _fusable(self, x: Tensor, mask: Optional[Tensor], params) -> bool:
        """The conditions of wc_self_attention: bf16, head dim 32, 1 <= S <= 512, D <= 768, no
        explicit mask, x rows and strides 16-byte aligned, biases with contiguous rows."""
        if not self.fuse_projections or mask is not None or x.dtype != torch.bfloat16 or self.d_head != 32:
            return False
        if not (1 <= x.shape[2] <= 512 and self.d_model <= 768 and x.shape[1] > 0):
            return False
        if x.stride(3) != 1 or x.data_ptr() % 16 or any(st % 8 for st in x.stride()[:3]):
            return False
        return all(t is None or (t.is_contiguous() and t.data_ptr() % 16 == 0) for t in params)

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
