"""Small helpers shared across the package."""

from __future__ import annotations

from typing import Optional


def _version_or_none(t) -> Optional[int]:
    """t._version, or None for inference tensors, which do not track one.

    Cache keys use it as a best-effort mutation check; tensor identity carries
    correctness (reference optimized/util.py:8-21).
    """
    try:
        return t._version
    except RuntimeError:
        return None
