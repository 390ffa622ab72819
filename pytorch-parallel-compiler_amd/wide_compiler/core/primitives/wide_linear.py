"""
WideLinear: N independent nn.Linear layers as one grouped MFMA GEMM
(mirror of wide_compiler/core/primitives/wide_linear.py:35-229).

    x [N, *batch, I]  ->  y [N, *batch, O],   y[i] = x[i] @ weight[i].T + bias[i]

Parameters keep the reference layout (weight [N, O, I], bias [N, O]).  Every strategy
('einsum', 'sequential', 'auto') is accepted and recorded, and all of them execute the
same kernel, wc_grouped_gemm (fp32 accumulation; bias and an optional fused ReLU in the
epilogue).  N-first inputs are read through their strides, so the channel-packed boundary
view [B, N*I] -> [N, B, I] costs no copy.
"""

from __future__ import annotations

import math
from enum import Enum
from typing import List, Optional, Union

import torch
from torch import Tensor, nn

from ... import _hip
from .._layout import rows_of, rows_or_contiguous


class LinearStrategy(Enum):
    EINSUM = "einsum"
    SEQUENTIAL = "sequential"
    AUTO = "auto"


# Thresholds of the reference's heuristic (wide_linear.py:42-47); they only decide the
# recorded strategy label here.
LINEAR_THRESHOLDS = {
    "n_min_einsum": 8,
    "b_max_for_low_n": 64,
    "expansion_max": 8.0,
    "vocab_size": 10000,
}


def select_linear_strategy(n: int, b: int, in_features: int, out_features: int) -> LinearStrategy:
    """The reference's label heuristic (wide_linear.py:50-69)."""
    t = LINEAR_THRESHOLDS
    if n < t["n_min_einsum"] and b > t["b_max_for_low_n"]:
        return LinearStrategy.SEQUENTIAL
    if out_features >= t["vocab_size"]:
        return LinearStrategy.SEQUENTIAL
    return LinearStrategy.EINSUM


class WideLinear(nn.Module):
    def __init__(self, n: int, in_features: int, out_features: int, bias: bool = True,
                 strategy: Union[str, LinearStrategy] = "auto"):
        super().__init__()
        self.n = n
        self.in_features = in_features
        self.out_features = out_features
        self.has_bias = bias
        if isinstance(strategy, str):
            strategy = LinearStrategy(strategy)
        if strategy == LinearStrategy.AUTO:
            strategy = select_linear_strategy(n, 32, in_features, out_features)
        self._strategy = strategy
        self.weight = nn.Parameter(torch.empty(n, out_features, in_features))
        if bias:
            self.bias = nn.Parameter(torch.empty(n, out_features))
        else:
            self.register_parameter("bias", None)
        # epilogue activation fused in by TracedWideModel ("relu" or None)
        self.fused_activation: Optional[str] = None
        self._reset_parameters()

    @property
    def strategy(self) -> LinearStrategy:
        return self._strategy

    def _reset_parameters(self) -> None:
        bound = 1.0 / math.sqrt(self.in_features) if self.in_features > 0 else 0.0
        for i in range(self.n):
            nn.init.kaiming_uniform_(self.weight[i], a=math.sqrt(5))
            if self.bias is not None:
                nn.init.uniform_(self.bias[i], -bound, bound)

    def forward(self, x: Tensor) -> Tensor:
        return self.forward_into(x, None, relu=self.fused_activation == "relu")

    def forward_into(self, x: Tensor, out: Optional[Tensor], relu: bool = False) -> Tensor:
        """Run the GEMM, writing into ``out`` (any view with unit inner stride) if given."""
        what = "WideLinear"
        if x.dim() < 2 or x.shape[0] != self.n or x.shape[-1] != self.in_features:
            raise RuntimeError(
                f"{what}: expected input [N={self.n}, ..., {self.in_features}], got {list(x.shape)}"
            )
        w = self.weight
        b = self.bias
        _hip.require_device(what, x, w, b)
        _hip.require_forward_only(what, x, w, b)
        if x.dtype != w.dtype:
            raise RuntimeError(f"{what}: input dtype {x.dtype} != weight dtype {w.dtype}")
        x, r = rows_or_contiguous(x)
        batch = tuple(x.shape[1:-1])
        if out is None:
            out = torch.empty((self.n, *batch, self.out_features), dtype=x.dtype, device=x.device)
        cr = rows_of(out)
        if cr is None or tuple(out.shape) != (self.n, *batch, self.out_features):
            raise RuntimeError(f"{what}: output view {list(out.shape)} is not addressable")
        if r.rows == 0 or self.out_features == 0:
            return out
        w = w if w.is_contiguous() else w.contiguous()
        _hip.grouped_gemm(
            n=self.n, m=r.rows, o=self.out_features, k=self.in_features,
            a=x, a_sn=r.stride_n, a_so=r.stride_outer, a_si=r.stride_inner, a_rows_inner=r.rows_inner,
            w=w, w_sn=self.out_features * self.in_features,
            c=out, c_sn=cr.stride_n, c_so=cr.stride_outer, c_si=cr.stride_inner, c_rows_inner=cr.rows_inner,
            bias=b, bias_sn=self.out_features, relu=relu,
        )
        return out

    @classmethod
    def from_modules(cls, modules: List[nn.Linear],
                     strategy: Union[str, LinearStrategy] = "auto") -> "WideLinear":
        t = modules[0]
        wide = cls(n=len(modules), in_features=t.in_features, out_features=t.out_features,
                   bias=t.bias is not None, strategy=strategy)
        wide = wide.to(device=t.weight.device, dtype=t.weight.dtype)
        with torch.no_grad():
            for i, m in enumerate(modules):
                wide.weight[i].copy_(m.weight)
                if m.bias is not None:
                    wide.bias[i].copy_(m.bias)
        return wide

    def __repr__(self) -> str:
        act = ", +relu" if self.fused_activation == "relu" else ""
        return (f"WideLinear({self.n}x[{self.in_features}->{self.out_features}], "
                f"strategy={self._strategy.value}{act})")


class WideMLP2(nn.Module):
    """Two chained WideLinear stages (the first optionally followed by ReLU) run as one
    wc_mlp2 launch; TracedWideModel builds it when it finds a Linear -> [ReLU] -> Linear
    chain whose intermediate has no other consumer.  The hidden activations never reach
    memory; they are rounded to the parameter dtype as the first stage would store them.
    Parameters stay in the two WideLinear modules (state_dict keys unchanged)."""

    def __init__(self, first: WideLinear, second: WideLinear, relu1: bool):
        super().__init__()
        self.first = first
        self.second = second
        self.relu1 = relu1
        self.n = first.n
        self.in_features = first.in_features
        self.hidden = first.out_features
        self.out_features = second.out_features
        self.fused_activation: Optional[str] = None

    @staticmethod
    def supported(first: WideLinear, second: WideLinear) -> bool:
        return (first.n == second.n and first.out_features == second.in_features and
                first.weight.dtype == second.weight.dtype and
                _hip.mlp2_supported(first.weight.dtype, first.in_features, first.out_features,
                                    second.out_features))

    def forward(self, x: Tensor) -> Tensor:
        return self.forward_into(x, None, relu=self.fused_activation == "relu")

    def _params(self):
        p1, p2 = self.first._parameters, self.second._parameters
        return p1["weight"], p1.get("bias"), p2["weight"], p2.get("bias")

    def plan_key(self, x: Tensor, out: Optional[Tensor], relu: bool, params) -> tuple:
        return (x.shape, x.stride(), x.dtype, x.device, None if out is None else (out.shape, out.stride()),
                relu, tuple(0 if t is None else t.data_ptr() for t in params))

    def launch_with(self, args, param_ptrs: tuple, x: Tensor, y: Tensor) -> bool:
        """Launch kept arguments `args` (built for parameter addresses param_ptrs) on x / y of the
        form they were built for; False (nothing launched) if a parameter moved or autograd
        would need the result."""
        params = self._params()
        if tuple(0 if t is None else t.data_ptr() for t in params) != param_ptrs or (
                torch.is_grad_enabled() and (x.requires_grad or any(t is not None and t.requires_grad
                                                                    for t in params))):
            return False
        args.x = x.data_ptr()
        args.y = y.data_ptr()
        _hip.mlp2_launch(args, _hip.stream_of(x))
        return True

    def forward_into(self, x: Tensor, out: Optional[Tensor], relu: bool = False) -> Tensor:
        """One wc_mlp2 launch.  The launch arguments of a (shapes, strides, dtype, device,
        parameter addresses) combination are built once and kept: a call that matches only
        sets the x / y addresses, so the host cost of a small wide MLP stays below its GPU time.
        The parameters are still read in place on every call."""
        params = self._params()
        key = self.plan_key(x, out, relu, params)
        plan = self.__dict__.get("_plan")
        if plan is not None and plan[0] == key and not (
                torch.is_grad_enabled() and (x.requires_grad or any(t is not None and t.requires_grad
                                                                    for t in params))):
            _, args, out_shape = plan
            if out is None:
                out = torch.empty(out_shape, dtype=x.dtype, device=x.device)
            args.x = x.data_ptr()
            args.y = out.data_ptr()
            _hip.mlp2_launch(args, _hip.stream_of(x))
            return out
        out = self._forward_checked(x, out, relu, params)
        return out

    def _forward_checked(self, x: Tensor, out: Optional[Tensor], relu: bool, params) -> Tensor:
        what = "WideMLP2"
        if x.dim() < 2 or x.shape[0] != self.n or x.shape[-1] != self.in_features:
            raise RuntimeError(f"{what}: expected input [N={self.n}, ..., {self.in_features}], got {list(x.shape)}")
        key_x, key_out = x, out
        _hip.require_device(what, x, *params)
        _hip.require_forward_only(what, x, *params)
        if x.dtype != params[0].dtype:
            raise RuntimeError(f"{what}: input dtype {x.dtype} != weight dtype {params[0].dtype}")
        x, r = rows_or_contiguous(x)
        batch = tuple(x.shape[1:-1])
        if out is None:
            out = torch.empty((self.n, *batch, self.out_features), dtype=x.dtype, device=x.device)
        cr = rows_of(out)
        if cr is None or tuple(out.shape) != (self.n, *batch, self.out_features):
            raise RuntimeError(f"{what}: output view {list(out.shape)} is not addressable")
        if r.rows == 0:
            return out
        contiguous = all(t is None or t.is_contiguous() for t in params)
        c = lambda t: None if t is None else (t if t.is_contiguous() else t.contiguous())  # noqa: E731
        w1, b1, w2, b2 = (c(t) for t in params)
        args = _hip.mlp2_args(n=self.n, m=r.rows, in_features=self.in_features, hidden=self.hidden,
                              out_features=self.out_features,
                              x=x, x_sn=r.stride_n, x_so=r.stride_outer, x_si=r.stride_inner,
                              x_rows_inner=r.rows_inner, w1=w1, b1=b1, w2=w2, b2=b2,
                              y=out, y_sn=cr.stride_n, y_so=cr.stride_outer, y_si=cr.stride_inner,
                              y_rows_inner=cr.rows_inner, relu1=self.relu1, relu2=relu)
        _hip.mlp2_launch(args, _hip.stream_of(x))
        # keep the arguments for calls of the same form: x read in place (no copy made), the
        # parameters contiguous (their addresses are in the key), the output allocated here
        # or a view of the same shape and strides
        if x is key_x and contiguous:
            self.__dict__["_plan"] = (self.plan_key(key_x, key_out, relu, params), args, tuple(out.shape))
        return out

    def __repr__(self) -> str:
        mid = " -> relu" if self.relu1 else ""
        return f"WideMLP2({self.n}x[{self.in_features} -> {self.hidden}{mid} -> {self.out_features}])"


__all__ = ["WideLinear", "LinearStrategy", "select_linear_strategy", "LINEAR_THRESHOLDS", "WideMLP2"]
