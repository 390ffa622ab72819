"""
WideConv3d: N independent nn.Conv3d on N-first [N, B, C_in, D, H, W]
(mirror of wide_compiler/core/primitives/wide_conv3d.py:28-176).

State layout as the reference: strategy 'grouped' (the default) holds ``conv`` =
nn.Conv3d(N*C_in, N*C_out, groups=N), model i's filters at rows [i*C_out, (i+1)*C_out);
'sequential' holds ``convs`` = N nn.Conv3d.  The forward is one wc_conv3d launch: the
implicit-GEMM convolution kernel with an outer loop over depth taps (each tap stages the
input depth slice it reads), on filters packed once as [N, C_out, kd*kh, kw, Ci32] and
cached until the filter tensors change.
"""

from __future__ import annotations

from enum import Enum
from typing import List, Tuple, Union

import torch
from torch import Tensor, nn

from ... import _hip
from .._layout import inner_block_contiguous


class Conv3dStrategy(Enum):
    GROUPED = "grouped"
    SEQUENTIAL = "sequential"
    AUTO = "auto"


def _padding3(conv: nn.Conv3d) -> Tuple[int, int, int]:
    """Symmetric per-dimension padding of an nn.Conv3d (int / tuple / 'valid' / symmetric 'same')."""
    pad = conv.padding
    if isinstance(pad, str):
        if pad == "valid":
            return (0, 0, 0)
        out = []
        for k, d in zip(conv.kernel_size, conv.dilation):
            total = d * (k - 1)
            if total % 2:
                raise NotImplementedError("WideConv3d: asymmetric 'same' padding is not supported by the kernel")
            out.append(total // 2)
        return tuple(out)
    return tuple(pad)


class WideConv3d(nn.Module):
    def __init__(self, n: int, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0,
                 dilation=1, bias: bool = True, strategy: Union[str, Conv3dStrategy] = "auto"):
        super().__init__()
        self.n = n
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = kernel_size
        self.stride = stride
        self.padding = padding
        self.dilation = dilation
        self.has_bias = bias
        if isinstance(strategy, str):
            strategy = Conv3dStrategy(strategy)
        if strategy == Conv3dStrategy.AUTO:
            strategy = Conv3dStrategy.GROUPED
        self._strategy = strategy
        self._use_grouped = strategy == Conv3dStrategy.GROUPED
        kw = dict(kernel_size=kernel_size, stride=stride, padding=padding, dilation=dilation, bias=bias)
        if self._use_grouped:
            self.conv = nn.Conv3d(n * in_channels, n * out_channels, groups=n, **kw)
        else:
            self.convs = nn.ModuleList([nn.Conv3d(in_channels, out_channels, **kw) for _ in range(n)])
        self.fused_activation = None

    @property
    def strategy(self) -> Conv3dStrategy:
        return self._strategy

    def _filters(self):
        if self._use_grouped:
            return self.conv, self.conv.weight, self.conv.bias
        w = torch.cat([c.weight for c in self.convs], dim=0)
        b = torch.cat([c.bias for c in self.convs], dim=0) if self.has_bias else None
        return self.convs[0], w, b

    def _packed(self, w: Tensor, kd: int, kh: int, kw: int) -> Tensor:
        """The filters in the kernel's layout, packed on every call (no cache: writes through
        ``.data`` do not bump the version counter a cache could key on)."""
        wc = w if w.is_contiguous() else w.contiguous()
        return _hip.conv_pack_weights(wc, self.n, self.out_channels, self.in_channels, kd * kh, kw)

    def forward(self, x: Tensor) -> Tensor:
        what = "WideConv3d"
        ref, w, bias = self._filters()
        n, ci, co = self.n, self.in_channels, self.out_channels
        if x.dim() != 6 or x.shape[0] != n or x.shape[2] != ci:
            raise RuntimeError(f"{what}: expected [N={n}, B, C_in={ci}, D, H, W], got {list(x.shape)}")
        _hip.require_device(what, x, w, bias)
        _hip.require_forward_only(what, x, w, bias)
        if x.dtype != w.dtype:
            raise RuntimeError(f"{what}: input dtype {x.dtype} != weight dtype {w.dtype}")
        if ref.padding_mode != "zeros":
            raise NotImplementedError(f"{what}: padding_mode {ref.padding_mode!r} is not supported")
        kd, kh, kw = ref.kernel_size
        stride, dilation, padding = tuple(ref.stride), tuple(ref.dilation), _padding3(ref)
        if not inner_block_contiguous(x, 2):
            x = x.contiguous()
        dims = x.shape[3:]
        out_dims = [(dims[i] + 2 * padding[i] - dilation[i] * ((kd, kh, kw)[i] - 1) - 1) // stride[i] + 1
                    for i in range(3)]
        if min(out_dims) <= 0:
            raise RuntimeError(f"{what}: input {list(dims)} is smaller than the kernel")
        y = torch.empty((n, x.shape[1], co, *out_dims), dtype=x.dtype, device=x.device)
        if y.numel():
            _hip.conv3d(x=x, packed_w=self._packed(w, kd, kh, kw), n=n, c_in=ci, c_out=co, kernel=(kd, kh, kw),
                        stride=stride, padding=padding, dilation=dilation, y=y, bias=bias,
                        relu=self.fused_activation == "relu")
        return y

    @classmethod
    def from_modules(cls, modules: List[nn.Conv3d], strategy: Union[str, Conv3dStrategy] = "auto") -> "WideConv3d":
        t = modules[0]
        wide = cls(n=len(modules), in_channels=t.in_channels, out_channels=t.out_channels,
                   kernel_size=t.kernel_size, stride=t.stride, padding=t.padding, dilation=t.dilation,
                   bias=t.bias is not None, strategy=strategy)
        wide = wide.to(device=t.weight.device, dtype=t.weight.dtype)
        with torch.no_grad():
            if wide._use_grouped:
                wide.conv.weight.copy_(torch.cat([m.weight for m in modules], dim=0))
                if wide.has_bias:
                    wide.conv.bias.copy_(torch.cat([m.bias for m in modules], dim=0))
            else:
                for i, m in enumerate(modules):
                    wide.convs[i].load_state_dict(m.state_dict())
        return wide

    def __repr__(self) -> str:
        return (f"WideConv3d({self.n}x[{self.in_channels}→{self.out_channels}, k={self.kernel_size}], "
                f"strategy={self._strategy.value})")


__all__ = ["WideConv3d", "Conv3dStrategy"]
