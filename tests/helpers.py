"""Shared test utilities: seeded synthetic inputs (numpy PCG64) and error metrics."""
from __future__ import annotations

import numpy as np


def to_bf16(x) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from_bf16(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def randn_bf16(rng, shape, scale=1.0):
    return to_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))


def mx_weights(rng, N, K, smin=119, smax=125):
    """Packed e2m1 codes [N, K/2] (every nibble uniform over the 16 codes) + e8m0 scales [N, K/32] uniform in
    [smin, smax] (2^-8 .. 2^-2 by default)."""
    w = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    s = rng.integers(smin, smax + 1, size=(N, K // 32), dtype=np.uint8)
    return w, s


def max_rel(y, r, floor_frac=2.0 ** -8):
    """max |y - r| / max(|r|, floor_frac * rms(r))."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    rms = np.sqrt(np.mean(r * r)) if r.size else 0.0
    den = np.maximum(np.abs(r), floor_frac * rms)
    den = np.where(den == 0, 1.0, den)
    return float(np.max(np.abs(y - r) / den)) if r.size else 0.0


def max_abs_rms(y, r):
    """max |y - r| / rms(r): the largest error as a fraction of the output scale."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    rms = np.sqrt(np.mean(r * r)) if r.size else 0.0
    return float(np.max(np.abs(y - r)) / rms) if rms else float(np.max(np.abs(y - r), initial=0.0))


def rel_l2(y, r):
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    n = np.linalg.norm(r)
    return float(np.linalg.norm(y - r) / (n if n else 1.0))
