"""The harness's accuracy rule, restated (torch_transformer_benchmark.py:557-624).

Per element: finite (both sides) AND (|opt - ref| <= atol OR |opt - ref| <= rtol * |ref|).
Deliberately not torch.isclose, whose atol + rtol*|ref| is more permissive (:577-583).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import numpy as np

ATOL = 2e-3
RTOL = 0.02


@dataclass
class AccuracyResult:
    """Field names follow the harness's AccuracyResult (:543-554)."""

    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    failed_feature_dims: List[int]
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float


def gate_ratio(reference, optimized, rtol: float = RTOL, atol: float = ATOL) -> float:
    """How much of the rule's allowance the worst element uses: the maximum
    over elements of min(err / atol, err / (rtol |ref|)). An element passes
    iff its ratio is <= 1, so 1 - gate_ratio is the margin left. Non-finite
    elements count as infinite. Not in the harness (its rule is pass/fail);
    the parity tests use it to catch margin loss that max_abs would hide (an
    element far above atol can pass on the relative arm)."""
    ref = np.asarray(reference, dtype=np.float64)
    opt = np.asarray(optimized, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        err = np.abs(opt - ref)
        ratio = np.minimum(err / atol, err / (rtol * np.abs(ref)))
    ratio = np.where(np.isfinite(ref) & np.isfinite(opt), ratio, np.inf)
    return float(np.nanmax(ratio))


def element_ok(reference, optimized, rtol: float = RTOL, atol: float = ATOL) -> np.ndarray:
    """Boolean array: which elements pass the rule."""
    ref = np.asarray(reference, dtype=np.float64)
    opt = np.asarray(optimized, dtype=np.float64)
    finite = np.isfinite(ref) & np.isfinite(opt)
    with np.errstate(invalid="ignore"):
        err = np.abs(opt - ref)
        return finite & ((err <= atol) | (err <= rtol * np.abs(ref)))


def compare_outputs(reference, optimized, rtol: float = RTOL,
                    atol: float = ATOL) -> AccuracyResult:
    """compare_outputs (:557-624) on numpy-convertible arrays.

    The error arithmetic runs in float32, as the harness's `.float()` does, so
    a borderline element is judged the way the harness would judge it.
    """
    ref = np.asarray(reference, dtype=np.float32)
    opt = np.asarray(optimized, dtype=np.float32)
    if ref.shape != opt.shape:
        raise AssertionError(f"shape mismatch: baseline={ref.shape}, optimized={opt.shape}")

    finite = np.isfinite(ref) & np.isfinite(opt)
    with np.errstate(invalid="ignore", over="ignore"):
        abs_err = np.abs(opt - ref)
        passed = finite & ((abs_err <= np.float32(atol)) |
                           (abs_err <= np.float32(rtol) * np.abs(ref)))
    failed = ~passed
    n_failed = int(failed.sum())

    flat = abs_err.reshape(-1)
    worst_flat = int(np.nanargmax(flat)) if flat.size and not np.all(np.isnan(flat)) else 0
    worst = tuple(int(i) for i in np.unravel_index(worst_flat, ref.shape)) if ref.ndim else ()
    denom = np.maximum(np.abs(ref), np.float32(1e-12))
    with np.errstate(invalid="ignore", over="ignore"):
        rel = abs_err / denom
    if ref.ndim == 0:
        dims = [0] if n_failed else []
    elif ref.ndim == 1:
        dims = np.nonzero(failed)[0].tolist()
    else:
        dims = np.nonzero(failed.reshape(-1, ref.shape[-1]).any(axis=0))[0].tolist()
    return AccuracyResult(
        passed=n_failed == 0,
        total_elements=int(ref.size),
        failed_elements=n_failed,
        max_abs_error=float(np.nanmax(abs_err)) if abs_err.size else 0.0,
        max_relative_error=float(np.nanmax(rel)) if rel.size else 0.0,
        mean_abs_error=float(np.nanmean(abs_err)) if abs_err.size else 0.0,
        failed_feature_dims=dims,
        worst_index=worst,
        reference_at_worst=float(ref[worst]) if ref.size else 0.0,
        optimized_at_worst=float(opt[worst]) if opt.size else 0.0,
    )
