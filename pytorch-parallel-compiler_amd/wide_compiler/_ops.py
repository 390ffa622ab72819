"""
A traced wide model's forward as one PyTorch operator, for torch.compile.

``compile(..., compile_model=True)`` wraps the wide model in ``torch.compile`` (reference
api.py:137-147).  The kernels are reached through ctypes, which dynamo cannot trace, so
without an operator every forward would end the compiled region at the first launch and
``mode="reduce-overhead"`` would capture an empty CUDA graph.  Registering the forward as
``torch.ops.wide_compiler.module_call`` (``torch.library.custom_op``) makes it one opaque
node of the compiled graph: dynamo records it with the output shapes of its fake
implementation, inductor calls it as an external kernel, and in reduce-overhead mode the
cudagraph trees capture the launches it makes on the current stream (every kernel of the
forward) into their graph.

A module is named in the graph by an integer handle (the operator's first argument); the
handle maps to the module through a table of weak references, so the operator reads the
module's parameters at their current addresses, as the eager forward does.
"""

from __future__ import annotations

import itertools
import weakref
from typing import Dict, List

import torch
from torch import Tensor

_modules: Dict[int, "weakref.ReferenceType"] = {}
_counter = itertools.count(1)


def register(module) -> int:
    """A new handle for ``module`` (kept as a weak reference)."""
    handle = next(_counter)
    _modules[handle] = weakref.ref(module)
    return handle


def _module(handle: int):
    ref = _modules.get(handle)
    mod = ref() if ref is not None else None
    if mod is None:
        raise RuntimeError(f"wide_compiler::module_call: no live module with handle {handle}")
    return mod


@torch.library.custom_op("wide_compiler::module_call", mutates_args=())
def module_call(handle: int, inputs: List[Tensor]) -> List[Tensor]:
    """The module's forward launches on the current stream; outputs that share storage with
    an input (a forward that returns a view of its input) are copied, as an operator's
    outputs may not alias its inputs."""
    outs = _module(handle).op_forward(*inputs)
    in_ptrs = {t.untyped_storage().data_ptr() for t in inputs}
    return [o.clone() if o.untyped_storage().data_ptr() in in_ptrs else o for o in outs]


@module_call.register_fake
def _module_call_fake(handle: int, inputs: List[Tensor]) -> List[Tensor]:
    return _module(handle).op_fake(*inputs)
