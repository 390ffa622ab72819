"""
Module-type -> wide-primitive registry (mirror of wide_compiler/core/registry.py:20-157).

Unlike the reference, whose TracedWideModel consults only its private WIDE_BUILDERS dict
(traced_wide.py:384-385), this build's TracedWideModel looks a module type up here first,
so a primitive registered with ``register('MyModule', WideMyModule)`` is used by
``wide_compiler.compile`` -- a strict superset of the reference behaviour.
"""

from __future__ import annotations

from typing import Callable, Dict, List, Optional, Type

import torch.nn as nn

Builder = Callable[[List[nn.Module]], nn.Module]


class WideRegistry:
    """Maps ``type(module).__name__`` to a wide class exposing ``from_modules(modules)``."""

    def __init__(self):
        self._builders: Dict[str, Builder] = {}
        self._classes: Dict[str, Type[nn.Module]] = {}

    def register(self, module_type: str, wide_class: Optional[Type[nn.Module]] = None):
        """``register('Linear', WideLinear)`` or ``@register('Linear')`` as a class decorator."""

        def _add(cls):
            if not hasattr(cls, "from_modules"):
                raise TypeError(
                    f"{cls.__name__} must implement classmethod from_modules(modules: List[nn.Module])"
                )
            self._classes[module_type] = cls
            self._builders[module_type] = cls.from_modules
            return cls

        if wide_class is not None:
            return _add(wide_class)
        return _add

    def unregister(self, module_type: str) -> None:
        self._builders.pop(module_type, None)
        self._classes.pop(module_type, None)

    def get_builder(self, module_type: str) -> Optional[Builder]:
        return self._builders.get(module_type)

    def get_class(self, module_type: str) -> Optional[Type[nn.Module]]:
        return self._classes.get(module_type)

    def has(self, module_type: str) -> bool:
        return module_type in self._builders

    def build(self, modules: List[nn.Module]) -> Optional[nn.Module]:
        if not modules:
            return None
        builder = self.get_builder(type(modules[0]).__name__)
        return None if builder is None else builder(modules)

    def list_registered(self) -> List[str]:
        return list(self._builders)

    def __contains__(self, module_type: str) -> bool:
        return self.has(module_type)

    def __repr__(self) -> str:
        return f"WideRegistry([{', '.join(sorted(self._builders))}])"


_global_registry = WideRegistry()


def get_registry() -> WideRegistry:
    return _global_registry


def register(module_type: str, wide_class: Optional[Type[nn.Module]] = None):
    return _global_registry.register(module_type, wide_class)


def unregister(module_type: str) -> None:
    _global_registry.unregister(module_type)


def get_builder(module_type: str) -> Optional[Builder]:
    return _global_registry.get_builder(module_type)


def build_wide(modules: List[nn.Module]) -> Optional[nn.Module]:
    return _global_registry.build(modules)


def list_registered() -> List[str]:
    return _global_registry.list_registered()


BUILTIN_TYPES = (
    ("Linear", "WideLinear"),
    ("Conv1d", "WideConv1d"),
    ("Conv2d", "WideConv2d"),
    ("Conv3d", "WideConv3d"),
    ("BatchNorm1d", "WideBatchNorm1d"),
    ("BatchNorm2d", "WideBatchNorm2d"),
    ("LayerNorm", "WideLayerNorm"),
    ("GroupNorm", "WideGroupNorm"),
    ("InstanceNorm1d", "WideInstanceNorm1d"),
    ("InstanceNorm2d", "WideInstanceNorm2d"),
    ("Embedding", "WideEmbedding"),
    ("MultiheadAttention", "WideAttention"),
    ("GRU", "WideGRU"),
    ("LSTM", "WideLSTM"),
)


def auto_register_primitives() -> None:
    """Register the 14 built-in primitives (called on import)."""
    from . import primitives

    for module_type, cls_name in BUILTIN_TYPES:
        _global_registry.register(module_type, getattr(primitives, cls_name))


auto_register_primitives()

__all__ = [
    "WideRegistry", "get_registry", "register", "unregister", "get_builder", "build_wide",
    "list_registered", "auto_register_primitives",
]
