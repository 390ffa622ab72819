"""
Build configuration of a wide model (mirror of wide_compiler/core/config.py:16-128).

Only ``validate``, ``validate_rtol``, ``debug`` and the ``compile*`` fields change what this
build does.  With ``compile=True`` the result is wrapped in ``torch.compile`` exactly as the
reference does (api.py:138-147).  The HIP primitives are ctypes calls that dynamo does not
trace into: each one ends a compiled region (a graph break) and runs as is, so inductor
generates code only for the torch operations between them, never for the hot path.
``precision``/``allow_tf32``/``validate_atol``/``fallback_passthrough``/``strict_architecture``/
``profile``/``n`` are carried but unused, as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, Literal, Optional

_COMPILE_MODES = ("default", "reduce-overhead", "max-autotune")
_PRECISIONS = ("fp32", "fp16", "bf16")


@dataclass
class WideConfig:
    n: Optional[int] = None

    compile: bool = False
    compile_mode: Literal["default", "reduce-overhead", "max-autotune"] = "reduce-overhead"
    compile_backend: str = "inductor"
    compile_options: Dict[str, Any] = field(default_factory=dict)

    precision: Literal["fp32", "fp16", "bf16"] = "fp32"
    allow_tf32: bool = True

    validate: bool = False
    validate_rtol: float = 1e-3
    validate_atol: float = 1e-5

    fallback_passthrough: bool = True
    strict_architecture: bool = True

    debug: bool = False
    profile: bool = False

    def __post_init__(self):
        if self.compile_mode not in _COMPILE_MODES:
            raise ValueError(f"compile_mode must be one of {_COMPILE_MODES}")
        if self.precision not in _PRECISIONS:
            raise ValueError(f"precision must be one of {_PRECISIONS}")

    @classmethod
    def default(cls) -> "WideConfig":
        return cls()

    @classmethod
    def fast(cls) -> "WideConfig":
        return cls(compile=True, compile_mode="reduce-overhead", allow_tf32=True, validate=False)

    @classmethod
    def safe(cls) -> "WideConfig":
        return cls(compile=False, validate=True, strict_architecture=True)


def _debug_preset(cls) -> WideConfig:
    return cls(compile=False, validate=True, debug=True, fallback_passthrough=False)


# ``WideConfig.debug()`` is the debugging preset while ``cfg.debug`` is the bool field.
# Installed after the dataclass is built so the field keeps its False default; in the
# reference (config.py:51,94-102) the classmethod replaces the field default, which makes
# every default instance's ``debug`` a truthy bound method.
WideConfig.debug = classmethod(_debug_preset)


_default_config: Optional[WideConfig] = None


def get_default_config() -> WideConfig:
    global _default_config
    if _default_config is None:
        _default_config = WideConfig.default()
    return _default_config


def set_default_config(config: WideConfig) -> None:
    global _default_config
    _default_config = config


__all__ = ["WideConfig", "get_default_config", "set_default_config"]
