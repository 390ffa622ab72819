"""
WideEmbedding: N independent embedding tables
(mirror of wide_compiler/core/primitives/wide_embedding.py:26-157).

    forward(ids)                   ids [*S] shared by all models      -> [N, *S, D]
    forward(ids, per_model=True)   ids [N, *S], row i used by model i -> [N, *S, D]

The first form is the reference's ``weight[:, ids]`` (wide_embedding.py:93-102) for any
strategy; the second is the per-model lookup a stack of independent sequence models needs
(each model embeds its own tokens), which ``weight[:, ids]`` cannot express.  Both are the
same bit-exact row-gather kernel (wc_embedding_gather).  An out-of-range id reads nothing:
its output row is zero and the module's device-side error flag is raised; call
``index_error()`` (synchronises) to turn that into an IndexError.  With ``strict_ids = True``
every forward does that check itself (one host synchronisation per call, skipped under graph
capture) and raises as the reference's ``weight[:, ids]`` does.
"""

from __future__ import annotations

from enum import Enum
from typing import List, Union

import torch
from torch import Tensor, nn

from ... import _hip


class EmbeddingStrategy(Enum):
    INDEXED = "indexed"
    GATHER = "gather"
    SEQUENTIAL = "sequential"
    AUTO = "auto"


class WideEmbedding(nn.Module):
    def __init__(self, n: int, num_embeddings: int, embedding_dim: int,
                 strategy: Union[str, EmbeddingStrategy] = "auto"):
        super().__init__()
        self.n = n
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        if isinstance(strategy, str):
            strategy = EmbeddingStrategy(strategy)
        if strategy == EmbeddingStrategy.AUTO:
            strategy = EmbeddingStrategy.INDEXED
        self._strategy = strategy
        self.weight = nn.Parameter(torch.empty(n, num_embeddings, embedding_dim))
        nn.init.normal_(self.weight)
        self._err = None
        self.strict_ids = False

    @property
    def strategy(self) -> EmbeddingStrategy:
        return self._strategy

    def _flag(self, device) -> Tensor:
        if self._err is None or self._err.device != device:
            self._err = torch.zeros(1, dtype=torch.int32, device=device)
        return self._err

    def forward(self, x: Tensor, per_model: bool = False) -> Tensor:
        what = "WideEmbedding"
        w = self.weight
        _hip.require_device(what, x, w)
        _hip.require_forward_only(what, w)
        if x.dtype not in (torch.int64, torch.int32, torch.int16, torch.int8, torch.uint8):
            raise IndexError(f"{what}: indices must be an integer tensor, got {x.dtype}")
        ids = x.to(torch.int64).contiguous()
        w = w if w.is_contiguous() else w.contiguous()
        if per_model:
            if x.dim() < 1 or x.shape[0] != self.n:
                raise RuntimeError(f"{what}: per-model ids must be [N={self.n}, ...], got {list(x.shape)}")
            out = torch.empty((*x.shape, self.embedding_dim), dtype=w.dtype, device=w.device)
        else:
            out = torch.empty((self.n, *x.shape, self.embedding_dim), dtype=w.dtype, device=w.device)
        if out.numel():
            _hip.embedding_gather(w, ids, out, shared=not per_model, err_flag=self._flag(w.device))
            if self.strict_ids and not torch.cuda.is_current_stream_capturing():
                self.index_error()
        return out

    def forward_layernorm(self, x: Tensor, ln: "WideLayerNorm", per_model: bool = False) -> Tensor:
        """``ln(self(x, per_model))`` with the LayerNorm applied while the rows are gathered (one
        launch, the gathered rows never written): the same values bit for bit, and the same
        out-of-range id behaviour (a zero row is normalised and the flag is set).  Shapes or
        alignments the fused kernel does not take run the two launches."""
        what = "WideEmbedding"
        w = self.weight
        d = self.embedding_dim
        if ln.n != self.n or ln.normalized_shape != d:
            raise RuntimeError(f"{what}: LayerNorm {ln} does not match {self}")
        _hip.require_device(what, x, w, ln.weight, ln.bias)
        _hip.require_forward_only(what, w, ln.weight, ln.bias)
        if x.dtype not in (torch.int64, torch.int32, torch.int16, torch.int8, torch.uint8):
            raise IndexError(f"{what}: indices must be an integer tensor, got {x.dtype}")
        if per_model and (x.dim() < 1 or x.shape[0] != self.n):
            raise RuntimeError(f"{what}: per-model ids must be [N={self.n}, ...], got {list(x.shape)}")
        ids = x.to(torch.int64).contiguous()
        w = w if w.is_contiguous() else w.contiguous()
        shape = (*x.shape, d) if per_model else (self.n, *x.shape, d)
        out = torch.empty(shape, dtype=w.dtype, device=w.device)
        if out.numel() == 0:
            return out
        if not _hip.embedding_layernorm(w, ids, ln.weight, ln.bias, ln.eps, out, shared=not per_model,
                                        err_flag=self._flag(w.device)):
            return ln(self.forward(x, per_model=per_model))
        if self.strict_ids and not torch.cuda.is_current_stream_capturing():
            self.index_error()
        return out

    def index_error(self) -> None:
        """Raise IndexError if any lookup since the last call used an out-of-range id."""
        if self._err is not None and int(self._err.item()) != 0:
            self._err.zero_()
            raise IndexError(f"WideEmbedding: index out of range [0, {self.num_embeddings})")

    @classmethod
    def from_modules(cls, modules: List[nn.Embedding],
                     strategy: Union[str, EmbeddingStrategy] = "auto") -> "WideEmbedding":
        t = modules[0]
        wide = cls(n=len(modules), num_embeddings=t.num_embeddings, embedding_dim=t.embedding_dim,
                   strategy=strategy)
        wide = wide.to(device=t.weight.device, dtype=t.weight.dtype)
        with torch.no_grad():
            for i, m in enumerate(modules):
                wide.weight[i].copy_(m.weight)
        return wide

    def __repr__(self) -> str:
        return (f"WideEmbedding({self.n}x[{self.num_embeddings}, {self.embedding_dim}], "
                f"strategy={self._strategy.value})")


__all__ = ["WideEmbedding", "EmbeddingStrategy"]
