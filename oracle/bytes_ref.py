"""
Byte / index maps of the wide path as closed-form numpy index arithmetic (test infrastructure).

Pins: the maps are written as explicit integer index formulas over flat arrays, not with
torch.stack / movedim, so they check the reference's stack+view semantics independently
(tests/test_oracle.py compares them with the torch restatement in wide_ref on arange inputs,
where any swapped index shows up as a mismatch).
"""

from __future__ import annotations

from typing import List, Sequence

import numpy as np


def pack(inputs: Sequence[np.ndarray]) -> np.ndarray:
    """ensemble_util.py:44-60: packed[b, i*F + f, *s] = inputs[i][b, f, *s]."""
    n = len(inputs)
    x0 = inputs[0]
    b = x0.shape[0]
    inner = int(np.prod(x0.shape[1:], dtype=np.int64)) if x0.ndim > 1 else 1
    flat = np.empty(b * n * inner, dtype=x0.dtype)
    for i, x in enumerate(inputs):
        src = x.reshape(b, inner)
        for r in range(b):
            base = (r * n + i) * inner
            flat[base:base + inner] = src[r]
    if x0.ndim == 1:
        return flat.reshape(b, n)
    return flat.reshape((b, n * x0.shape[1]) + tuple(x0.shape[2:]))


def unpack(packed: np.ndarray, n: int) -> List[np.ndarray]:
    """ensemble_util.py:83-101: out[i][b, f, *s] = packed[b, i*F + f, *s]."""
    b, nf = packed.shape[0], packed.shape[1]
    f = nf // n
    rest = tuple(packed.shape[2:])
    inner = f * int(np.prod(rest, dtype=np.int64))
    flat = packed.reshape(-1)
    outs = []
    for i in range(n):
        o = np.empty(b * inner, dtype=packed.dtype)
        for r in range(b):
            base = (r * n + i) * inner
            o[r * inner:(r + 1) * inner] = flat[base:base + inner]
        outs.append(o.reshape((b, f) + rest))
    return outs


def packed_to_nfirst(packed: np.ndarray, n: int) -> np.ndarray:
    """traced_wide.py:463-469: nfirst[i, b, c, *s] = packed[b, i*C + c, *s]."""
    return np.stack(unpack(packed, n), axis=0)


def nfirst_to_packed(nfirst: np.ndarray) -> np.ndarray:
    """traced_wide.py:527-532: packed[b, i*C + c, *s] = nfirst[i, b, c, *s]."""
    return pack([nfirst[i] for i in range(nfirst.shape[0])])


def embedding_shared(weight: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """wide_embedding.py:100-102 (weight[:, ids]): out[i, *idx] = weight[i, ids[*idx]]."""
    n, v, d = weight.shape
    flat = ids.reshape(-1)
    out = np.empty((n, flat.size, d), dtype=weight.dtype)
    for i in range(n):
        for r, t in enumerate(flat):
            out[i, r] = weight[i, int(t)]
    return out.reshape((n,) + ids.shape + (d,))


def embedding_per_model(weight: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """Per-model lookup (the sequential strategy's F.embedding per model, wide_embedding.py:130,
    fed model i's own ids): out[i, *idx] = weight[i, ids[i, *idx]]."""
    n, v, d = weight.shape
    flat = ids.reshape(n, -1)
    out = np.empty((n, flat.shape[1], d), dtype=weight.dtype)
    for i in range(n):
        for r in range(flat.shape[1]):
            out[i, r] = weight[i, int(flat[i, r])]
    return out.reshape(ids.shape + (d,))
