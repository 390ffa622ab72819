"""Primitives outside the MI355X hot path of this build (construction and state layout only)."""

from __future__ import annotations


def not_on_hot_path(name: str):
    raise NotImplementedError(
        f"{name}: this primitive is outside the N-first hot path built for MI355X so far; its "
        "construction, from_modules and state_dict layout match the reference, but it has no "
        "HIP kernel yet and this build has no CPU fallback"
    )
