"""Shared checks of the parity tests."""
from __future__ import annotations

import numpy as np


def max_rel_over_rms(got, ref) -> float:
    """The reference's parity measure (runner/cuda/README.md:113-117): the largest elementwise relative difference over
    the elements at least as large as the rms of the reference."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    big = np.abs(ref) >= rms
    if not big.any():
        return 0.0
    return float(np.max(np.abs(got[big] - ref[big]) / np.abs(ref[big])))


def rel_rms(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.sqrt(np.mean((got - ref) ** 2) / max(np.mean(ref * ref), 1e-300)))


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and a.tobytes() == b.tobytes()


def bf16_inputs(rng, shape, outlier_frac: float = 0.0, scale: float = 1.0):
    """float32 values that are exact bfloat16 (~N(0, scale^2), a fraction of channels x20 before rounding)."""
    from oracle import orc
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    if outlier_frac > 0:
        k = shape[-1]
        hot = rng.choice(k, size=max(1, int(round(k * outlier_frac))), replace=False)
        x[..., hot] *= np.float32(20.0)
    return orc.bf16_round(x)
