"""
WideLSTM: N independent single-layer nn.LSTM(batch_first=True)
(mirror of wide_compiler/core/primitives/wide_lstm.py:40-348).

    x [N, B, T, I], hx = (h_0, c_0) [N, B, H] (optional)
        ->  (output [N, B, T, H], (h_n, c_n))

Storage.  The reference keeps O(N^2) block-diagonal parameters (weight_ih [N*4H, N*I],
weight_hh [N*4H, N*H], biases [N*4H]) and re-extracts the N diagonal blocks on every call
(wide_lstm.py:184-199).  Only those blocks are ever read, so this module stores them
compactly (weight_ih [N, 4H, I], weight_hh [N, 4H, H], bias_* [N, 4H]) and translates at
the checkpoint boundary: ``state_dict()`` emits the reference's block-diagonal tensors and
``load_state_dict`` accepts either layout.  Gate order (i, f, g, o); the cell state is
carried in fp32 inside the kernel.

Initialisation follows the reference (wide_lstm.py:113-131): weights U(+-1/sqrt(H)),
biases zero.
"""

from __future__ import annotations

from enum import Enum
from typing import List, Optional, Tuple, Union

import torch
from torch import Tensor, nn

from ... import _hip
from ._rnn_common import contiguous, prepare_input, prepare_state


class LSTMStrategy(Enum):
    FUSED = "fused"
    SEQUENTIAL = "sequential"
    AUTO = "auto"


def _to_block_diag(compact: Tensor) -> Tensor:
    n, g, k = compact.shape
    full = compact.new_zeros(n * g, n * k)
    for i in range(n):
        full[i * g:(i + 1) * g, i * k:(i + 1) * k] = compact[i]
    return full


def _from_block_diag(full: Tensor, n: int, g: int, k: int) -> Tensor:
    return torch.stack([full[i * g:(i + 1) * g, i * k:(i + 1) * k] for i in range(n)], dim=0)


class WideLSTM(nn.Module):
    def __init__(self, n: int, input_size: int, hidden_size: int, num_layers: int = 1,
                 bias: bool = True, batch_first: bool = True, dropout: float = 0.0,
                 bidirectional: bool = False, strategy: Union[str, LSTMStrategy] = "auto"):
        super().__init__()
        if num_layers != 1:
            raise NotImplementedError("WideLSTM currently only supports num_layers=1")
        if bidirectional:
            raise NotImplementedError("WideLSTM currently only supports bidirectional=False")
        if not batch_first:
            raise NotImplementedError("WideLSTM currently only supports batch_first=True")
        self.n = n
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.num_layers = num_layers
        self.bias = bias
        self.batch_first = batch_first
        self.dropout = dropout
        self.bidirectional = bidirectional
        if isinstance(strategy, str):
            strategy = LSTMStrategy(strategy)
        if strategy == LSTMStrategy.AUTO:
            strategy = LSTMStrategy.FUSED
        self._strategy = strategy
        g = 4 * hidden_size
        self.weight_ih = nn.Parameter(torch.empty(n, g, input_size))
        self.weight_hh = nn.Parameter(torch.empty(n, g, hidden_size))
        if bias:
            self.bias_ih = nn.Parameter(torch.zeros(n, g))
            self.bias_hh = nn.Parameter(torch.zeros(n, g))
        else:
            self.register_parameter("bias_ih", None)
            self.register_parameter("bias_hh", None)
        k = 1.0 / (hidden_size ** 0.5)
        with torch.no_grad():
            self.weight_ih.uniform_(-k, k)
            self.weight_hh.uniform_(-k, k)
        self._register_state_dict_hook(WideLSTM._save_block_diag)
        self._register_load_state_dict_pre_hook(self._load_any_layout)

    @property
    def strategy(self) -> LSTMStrategy:
        return self._strategy

    # ---- checkpoint layout translation -------------------------------------------------
    @staticmethod
    def _save_block_diag(module, state_dict, prefix, local_metadata):
        for name in ("weight_ih", "weight_hh"):
            key = prefix + name
            if key in state_dict and state_dict[key].dim() == 3:
                state_dict[key] = _to_block_diag(state_dict[key])
        for name in ("bias_ih", "bias_hh"):
            key = prefix + name
            if key in state_dict and state_dict[key].dim() == 2:
                state_dict[key] = state_dict[key].reshape(-1)
        return state_dict

    def _load_any_layout(self, state_dict, prefix, local_metadata, strict, missing_keys,
                         unexpected_keys, error_msgs):
        n, h, i = self.n, self.hidden_size, self.input_size
        for name, k in (("weight_ih", i), ("weight_hh", h)):
            key = prefix + name
            if key in state_dict and state_dict[key].dim() == 2 and \
                    tuple(state_dict[key].shape) == (n * 4 * h, n * k):
                state_dict[key] = _from_block_diag(state_dict[key], n, 4 * h, k)
        for name in ("bias_ih", "bias_hh"):
            key = prefix + name
            if key in state_dict and state_dict[key].dim() == 1 and state_dict[key].numel() == n * 4 * h:
                state_dict[key] = state_dict[key].reshape(n, 4 * h)

    # ---- forward ------------------------------------------------------------------------
    def forward(self, x: Tensor, hx: Optional[Tuple[Tensor, Tensor]] = None
                ) -> Tuple[Tensor, Tuple[Tensor, Tensor]]:
        """x [N, B, T, I] -> (out [N, B, T, H], (h_n, c_n)), as wide_lstm.py:137-156.

        The launch is asynchronous.  On the partitioned on-chip plan (bf16 or fp16, hidden
        256 / 384 / 512) the recurrence's cross-workgroup waits are bounded; a wait that gives up
        leaves the outputs invalid and is raised by the next recurrent call or by
        ``wide_compiler._hip.rnn_sync_check(block=True)``, which a caller that must trust
        these outputs (or a graph replay of this forward) calls before reading them."""
        what = "WideLSTM"
        params = (self.weight_ih, self.weight_hh, self.bias_ih, self.bias_hh)
        _hip.require_device(what, x, *params)
        h_0, c_0 = (None, None) if hx is None else hx
        _hip.require_forward_only(what, x, h_0, c_0, *params)
        x = prepare_input(what, x, self.n, self.input_size, self.weight_ih.dtype)
        n, b, t, _ = x.shape
        h = self.hidden_size
        h_0 = prepare_state(what, h_0, n, b, h, x.dtype, "h_0")
        c_0 = prepare_state(what, c_0, n, b, h, x.dtype, "c_0")
        out = torch.empty((n, b, t, h), dtype=x.dtype, device=x.device)
        h_n = torch.empty((n, b, h), dtype=x.dtype, device=x.device)
        c_n = torch.empty((n, b, h), dtype=x.dtype, device=x.device)
        if out.numel() == 0:
            return out, (h_n.zero_() if h_0 is None else h_0.clone(),
                         c_n.zero_() if c_0 is None else c_0.clone())
        _hip.rnn_forward(cell=_hip.CELL_LSTM, x=x, w_ih=contiguous(self.weight_ih),
                         w_hh=contiguous(self.weight_hh), b_ih=contiguous(self.bias_ih),
                         b_hh=contiguous(self.bias_hh), h0=h_0, c0=c_0, out=out, h_n=h_n, c_n=c_n)
        return out, (h_n, c_n)

    @classmethod
    def from_modules(cls, modules: List[nn.LSTM],
                     strategy: Union[str, LSTMStrategy] = "auto") -> "WideLSTM":
        ref = modules[0]
        for m in modules:
            if m.input_size != ref.input_size or m.hidden_size != ref.hidden_size:
                raise AssertionError("all LSTMs must share input_size and hidden_size")
            if m.num_layers != 1:
                raise AssertionError("Only single-layer LSTM supported")
            if m.bidirectional:
                raise AssertionError("Bidirectional not supported")
            if m.batch_first != ref.batch_first:
                raise AssertionError("all LSTMs must share batch_first")
            if getattr(m, "proj_size", 0):
                raise AssertionError("LSTM projections (proj_size) are not supported")
        wide = cls(n=len(modules), input_size=ref.input_size, hidden_size=ref.hidden_size,
                   num_layers=1, bias=ref.bias, batch_first=True, dropout=ref.dropout,
                   bidirectional=False, strategy=strategy)
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
        return (f"WideLSTM({self.n}x[{self.input_size}->{self.hidden_size}], "
                f"strategy={self._strategy.value})")


__all__ = ["WideLSTM", "LSTMStrategy"]
