"""Shared numeric helpers for the parity tests (bf16 emulation and tolerances)."""

from __future__ import annotations

import numpy as np

# Tolerances stated by the build contract: indices bit-exact, fp32 1e-5 relative,
# bf16 2e-2 relative (measured as a Frobenius-norm relative error).
BF16_RTOL = 2e-2
FP32_RTOL = 1e-5


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest even), returned as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, out)


def rel_err(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def assert_rel(a, b, tol: float, what: str = "") -> None:
    e = rel_err(a, b)
    assert e <= tol, f"{what}: relative error {e:.3e} > {tol:.1e}"
