"""
wide_compiler -- N structurally identical models fused into one "wide" model, executed on
AMD Instinct MI355X (gfx950) by hand-written HIP kernels behind a C ABI (libwide_hip.so).

The public surface mirrors the reference WideCompiler (wide_compiler/__init__.py:43-234):

    import wide_compiler
    wide = wide_compiler.compile(models, sample_input)        # TracedWideModel
    packed = wide_compiler.pack(inputs); outs = wide_compiler.unpack(wide(packed), n)
"""

from .api import WideBuilder, compile, pack, unpack  # noqa: A004
from .core.config import WideConfig, get_default_config, set_default_config
from .core.registry import get_registry, list_registered, register, unregister
from .core.traced_wide import BinaryOp, FunctionalOp, TracedWideModel, print_trace
from .core.ensemble_util import pack_inputs, unpack_outputs
from .core.primitives import (
    WideAttention, WideBatchNorm1d, WideBatchNorm2d, WideConv1d, WideConv2d, WideConv3d, WideEmbedding,
    WideGRU, WideGroupNorm, WideInstanceNorm1d, WideInstanceNorm2d, WideLayerNorm, WideLinear, WideLSTM,
)
from .api import benchmark_custom, benchmark_primitive

# the reference's optional benchmark harness is not part of this build
benchmark_multi = None
benchmark_all = None
list_benchmark_primitives = None
BenchmarkResult = None
SweepParams = None

__version__ = "0.6.0+mi355x"

__all__ = [
    "compile", "WideBuilder", "pack", "unpack",
    "WideConfig", "get_default_config", "set_default_config",
    "register", "unregister", "get_registry", "list_registered",
    "TracedWideModel", "FunctionalOp", "BinaryOp", "print_trace", "pack_inputs", "unpack_outputs",
    "WideLinear", "WideConv1d", "WideConv2d", "WideConv3d", "WideBatchNorm1d", "WideBatchNorm2d",
    "WideLayerNorm", "WideGroupNorm", "WideInstanceNorm1d", "WideInstanceNorm2d", "WideEmbedding",
    "WideAttention", "WideGRU", "WideLSTM",
    "benchmark_primitive", "benchmark_multi", "benchmark_all", "benchmark_custom",
    "list_benchmark_primitives", "BenchmarkResult", "SweepParams",
]
