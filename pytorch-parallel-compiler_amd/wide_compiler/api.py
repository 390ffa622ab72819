"""
Public API (mirror of wide_compiler/api.py:36-325): ``compile``, ``WideBuilder``, ``pack``,
``unpack``.
"""

from __future__ import annotations

import copy
import dataclasses
from typing import List, Optional, Union

import torch
import torch.nn as nn
from torch import Tensor

from .core.config import WideConfig, get_default_config
from .core.registry import get_registry


def compile(  # noqa: A001 - public name of the reference API
    models: Union[nn.Module, List[nn.Module]],
    sample_input: Optional[Tensor] = None,
    *,
    n: Optional[int] = None,
    config: Optional[WideConfig] = None,
    compile_model: Optional[bool] = None,
    compile_mode: Optional[str] = None,
    validate: Optional[bool] = None,
    debug: Optional[bool] = None,
) -> nn.Module:
    """Fuse N models (or N re-initialised copies of one) into a TracedWideModel."""
    from .core.traced_wide import TracedWideModel

    cfg = config or get_default_config()
    for field, value in (("compile", compile_model), ("compile_mode", compile_mode),
                         ("validate", validate), ("debug", debug)):
        if value is not None:
            cfg = _with_override(cfg, field, value)

    if isinstance(models, nn.Module):
        if n is None:
            raise ValueError("n required when passing single model")
        models = [_clone_model(models) for _ in range(n)]
    if not models:
        raise ValueError("models list is empty")

    if cfg.debug:
        print(f"[WideCompiler] Compiling {len(models)} models")
        print(f"[WideCompiler] Registry: {get_registry()}")
    if sample_input is None:
        raise ValueError(
            "sample_input required for FX tracing. "
            "Provide a sample input tensor with the expected shape."
        )

    wide = TracedWideModel.from_models(models, sample_input)
    if cfg.debug:
        print(f"[WideCompiler] Built model:\n{wide.summary()}")
    if cfg.validate:
        _validate_model(wide, models, sample_input, cfg)
    if cfg.compile:
        if cfg.debug:
            print(f"[WideCompiler] Compiling with mode={cfg.compile_mode}")
        wide = _compiled(wide, cfg)
    return wide


def _compiled(wide: nn.Module, cfg: WideConfig) -> nn.Module:
    """compile_model=True (api.py:137-147): torch.compile around the model.  The traced forward
    is one operator of the compiled graph (torch.ops.wide_compiler.module_call, whose fake
    implementation gives its output shape), so mode="reduce-overhead" captures the kernels'
    launches into its CUDA graph and replays them; other torch code around the model compiles
    as usual.  (TracedWideModel.use_graphs() captures the launches without torch.compile.)"""
    return torch.compile(wide, mode=cfg.compile_mode, backend=cfg.compile_backend, **cfg.compile_options)


class WideBuilder:
    """Fluent construction: WideBuilder(models).with_sample(x).validate().compile().build()."""

    def __init__(self, models: Union[nn.Module, List[nn.Module]], n: Optional[int] = None):
        if isinstance(models, nn.Module):
            if n is None:
                raise ValueError("n required when passing single model")
            self._models = [_clone_model(models) for _ in range(n)]
        else:
            self._models = list(models)
        self._sample_input: Optional[Tensor] = None
        self._config = WideConfig.default()

    def with_sample(self, sample_input: Tensor) -> "WideBuilder":
        self._sample_input = sample_input
        return self

    def with_config(self, config: WideConfig) -> "WideBuilder":
        self._config = config
        return self

    def validate(self, enable: bool = True) -> "WideBuilder":
        self._config = _with_override(self._config, "validate", enable)
        return self

    def compile(self, mode: str = "reduce-overhead") -> "WideBuilder":
        self._config = _with_override(self._config, "compile", True)
        self._config = _with_override(self._config, "compile_mode", mode)
        return self

    def debug(self, enable: bool = True) -> "WideBuilder":
        self._config = _with_override(self._config, "debug", enable)
        return self

    def register(self, module_type: str, wide_class: type) -> "WideBuilder":
        get_registry().register(module_type, wide_class)
        return self

    def build(self) -> nn.Module:
        from .core.traced_wide import TracedWideModel

        if self._sample_input is None:
            raise ValueError("sample_input required - call .with_sample()")
        if self._config.debug:
            print(f"[WideBuilder] Building from {len(self._models)} models")
        wide = TracedWideModel.from_models(self._models, self._sample_input)
        if self._config.validate:
            _validate_model(wide, self._models, self._sample_input, self._config)
        if self._config.compile:
            wide = _compiled(wide, self._config)
        return wide


def _clone_model(model: nn.Module) -> nn.Module:
    """Deep copy with freshly initialised parameters (api.py:244-252)."""
    clone = copy.deepcopy(model)
    for m in clone.modules():
        if hasattr(m, "reset_parameters"):
            m.reset_parameters()
    return clone


def _with_override(config: WideConfig, field: str, value) -> WideConfig:
    return dataclasses.replace(config, **{field: value})


def _validate_model(wide: nn.Module, models: List[nn.Module], sample_input: Tensor, config: WideConfig) -> None:
    """Wide forward vs the N per-model forwards on copies of the sample (api.py:261-303)."""
    from .core.ensemble_util import pack_inputs, unpack_outputs

    n = len(models)
    inputs = [sample_input.clone() for _ in range(n)]
    packed = pack_inputs(inputs)
    wide.eval()
    for m in models:
        m.eval()
    with torch.no_grad():
        expected = [models[i](inputs[i]) for i in range(n)]
        actual = unpack_outputs(wide(packed), n)
    max_diff = max((expected[i] - actual[i]).abs().max().item() for i in range(n))
    if config.debug:
        print(f"[WideCompiler] Validation max_diff: {max_diff:.8f}")
    if max_diff > config.validate_rtol:
        raise ValueError(
            f"Validation failed: max_diff={max_diff:.8f} > rtol={config.validate_rtol}. "
            "Wide model output differs from individual models."
        )


def pack(inputs: List[Tensor]) -> Tensor:
    from .core.ensemble_util import pack_inputs
    return pack_inputs(inputs)


def unpack(output: Tensor, n: int) -> List[Tensor]:
    from .core.ensemble_util import unpack_outputs
    return unpack_outputs(output, n)


def benchmark_primitive(name: str, preset: str = "full", device: str = "cuda", verbose: bool = True, **overrides):
    raise NotImplementedError(
        "the strategy-sweep benchmark harness of the reference is not part of this build; "
        "bench.py at the repository root measures the wide forward on MI355X"
    )


def benchmark_custom(model_class, input_shape, n_values, name: str = "custom", device: str = "cuda",
                     **model_kwargs):
    raise NotImplementedError(
        "the strategy-sweep benchmark harness of the reference is not part of this build; "
        "bench.py at the repository root measures the wide forward on MI355X"
    )


__all__ = ["compile", "WideBuilder", "pack", "unpack", "benchmark_primitive", "benchmark_custom"]
