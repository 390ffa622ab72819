"""
WideGRU: N independent single-layer nn.GRU(batch_first=True)
(mirror of wide_compiler/core/primitives/wide_gru.py:41-307).

    x [N, B, T, I], h_0 [N, B, H] (optional)  ->  (output [N, B, T, H], h_n [N, B, H])

Parameters keep the reference layout: weight_ih [N, 3H, I], weight_hh [N, 3H, H],
bias_ih / bias_hh [N, 3H], gate order (r, z, n).  The forward is wc_rnn_forward: one
grouped MFMA GEMM for the input projection of all T steps, then one persistent recurrence
that keeps W_hh on-chip for all T steps (no per-step launches, no per-step HBM traffic for
W_hh): for small hidden sizes each workgroup carries one (model, batch row) with its W_hh
slice in registers; for bf16 / fp16 at hidden 256 / 384 / 512, hidden / 128 workgroups
share a (model, 16-row chunk) and exchange h_t each step.  The launches are asynchronous; a
bounded wait of the shared recurrence that gave up is raised by
``wide_compiler._hip.rnn_sync_check(block=True)`` or by the next recurrent call.
"""

from __future__ import annotations

import math
from enum import Enum
from typing import List, Optional, Tuple, Union

import torch
from torch import Tensor, nn

from ... import _hip
from ._rnn_common import contiguous, prepare_input, prepare_state


class GRUStrategy(Enum):
    FUSED = "fused"
    SEQUENTIAL = "sequential"
    AUTO = "auto"


class WideGRU(nn.Module):
    def __init__(self, n: int, input_size: int, hidden_size: int, num_layers: int = 1,
                 bias: bool = True, batch_first: bool = True, dropout: float = 0.0,
                 bidirectional: bool = False, strategy: Union[str, GRUStrategy] = "auto"):
        super().__init__()
        if num_layers != 1:
            raise NotImplementedError("WideGRU only supports num_layers=1 for fused strategy")
        if bidirectional:
            raise NotImplementedError("WideGRU only supports unidirectional for fused strategy")
        self.n = n
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.num_layers = num_layers
        self.has_bias = bias
        self.batch_first = batch_first
        self.dropout = dropout
        self.bidirectional = bidirectional
        if isinstance(strategy, str):
            strategy = GRUStrategy(strategy)
        if strategy == GRUStrategy.AUTO:
            strategy = GRUStrategy.FUSED
        self._strategy = strategy
        g = 3 * hidden_size
        self.weight_ih = nn.Parameter(torch.empty(n, g, input_size))
        self.weight_hh = nn.Parameter(torch.empty(n, g, hidden_size))
        if bias:
            self.bias_ih = nn.Parameter(torch.empty(n, g))
            self.bias_hh = nn.Parameter(torch.empty(n, g))
        else:
            self.register_parameter("bias_ih", None)
            self.register_parameter("bias_hh", None)
        self._reset_parameters()

    @property
    def strategy(self) -> GRUStrategy:
        return self._strategy

    def _reset_parameters(self) -> None:
        k = 1.0 / math.sqrt(self.hidden_size)
        for p in (self.weight_ih, self.weight_hh, self.bias_ih, self.bias_hh):
            if p is not None:
                nn.init.uniform_(p, -k, k)

    def forward(self, x: Tensor, h_0: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
        what = "WideGRU"
        params = (self.weight_ih, self.weight_hh, self.bias_ih, self.bias_hh)
        _hip.require_device(what, x, *params)
        _hip.require_forward_only(what, x, h_0, *params)
        x = prepare_input(what, x, self.n, self.input_size, self.weight_ih.dtype)
        n, b, t, _ = x.shape
        h = self.hidden_size
        h_0 = prepare_state(what, h_0, n, b, h, x.dtype, "h_0")
        out = torch.empty((n, b, t, h), dtype=x.dtype, device=x.device)
        h_n = torch.empty((n, b, h), dtype=x.dtype, device=x.device)
        if out.numel() == 0:
            return out, (h_0.clone() if h_0 is not None else h_n.zero_())
        _hip.rnn_forward(cell=_hip.CELL_GRU, x=x, w_ih=contiguous(self.weight_ih),
                         w_hh=contiguous(self.weight_hh), b_ih=contiguous(self.bias_ih),
                         b_hh=contiguous(self.bias_hh), h0=h_0, c0=None, out=out, h_n=h_n, c_n=None)
        return out, h_n

    @classmethod
    def from_modules(cls, modules: List[nn.GRU],
                     strategy: Union[str, GRUStrategy] = "auto") -> "WideGRU":
        ref = modules[0]
        if ref.num_layers != 1:
            raise ValueError("WideGRU.from_modules only supports single-layer GRUs")
        if ref.bidirectional:
            raise ValueError("WideGRU.from_modules only supports unidirectional GRUs")
        wide = cls(n=len(modules), input_size=ref.input_size, hidden_size=ref.hidden_size,
                   num_layers=ref.num_layers, bias=ref.bias, batch_first=ref.batch_first,
                   dropout=ref.dropout, bidirectional=ref.bidirectional, strategy=strategy)
        p0 = next(ref.parameters())
        wide = wide.to(device=p0.device, dtype=p0.dtype)
        with torch.no_grad():
            for i, m in enumerate(modules):
                wide.weight_ih[i].copy_(m.weight_ih_l0)
                wide.weight_hh[i].copy_(m.weight_hh_l0)
                if ref.bias:
                    wide.bias_ih[i].copy_(m.bias_ih_l0)
                    wide.bias_hh[i].copy_(m.bias_hh_l0)
        return wide

    def __repr__(self) -> str:
        return (f"WideGRU({self.n}x[{self.input_size}->{self.hidden_size}], "
                f"strategy={self._strategy.value})")


__all__ = ["WideGRU", "GRUStrategy"]
