"""Core components: traced wide model, pack/unpack, registry, config, primitives."""

from .primitives import (
    WideBatchNorm1d, WideBatchNorm2d, WideConv1d, WideConv2d, WideEmbedding, WideLayerNorm, WideLinear,
)
from .config import WideConfig, get_default_config, set_default_config
from .registry import (
    WideRegistry, build_wide, get_builder, get_registry, list_registered, register, unregister,
)
from .ensemble_util import pack_inputs, unpack_outputs
from .traced_wide import BinaryOp, FunctionalOp, TracedWideModel, print_trace

__all__ = [
    "TracedWideModel", "FunctionalOp", "BinaryOp", "print_trace",
    "pack_inputs", "unpack_outputs",
    "WideRegistry", "get_registry", "register", "unregister", "get_builder", "build_wide", "list_registered",
    "WideConfig", "get_default_config", "set_default_config",
    "WideLinear", "WideConv2d", "WideConv1d", "WideBatchNorm2d", "WideBatchNorm1d", "WideLayerNorm",
    "WideEmbedding",
]
