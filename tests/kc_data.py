"""Synthetic inputs in the BASELINE configurations' distributions (numpy).

INT4: weight bytes uniform 0..255 (two uniform nibbles, read through the
reference's sign extension), per-group fp32 scales uniform [0.005, 0.02],
zero-point bytes uniform 0..255 (two uniform nibbles).  The zero buffer is
rows * ceil(G/2) bytes, what the reference's tests allocate; the kernels and
the oracle index it with the reference's floor(G/2) row stride.
"""
from __future__ import annotations

import numpy as np


def make_int4(rows: int, cols: int, gs: int, seed: int):
    rng = np.random.default_rng(seed)
    G = cols // gs
    packed = rng.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
    scales = rng.uniform(0.005, 0.02, size=(rows, G)).astype(np.float32)
    zeros = rng.integers(0, 256, size=(rows, (G + 1) // 2), dtype=np.uint8)
    return packed, scales, zeros


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def normal_bf16(shape, seed: int, std: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return f32_to_bf16_bits((rng.standard_normal(shape) * std).astype(np.float32))


def outlier_activations(rows: int, cols: int, frac: float, factor: float, seed: int):
    """x ~ N(0,1) fp32 with a seeded choice of `frac` of the channels scaled."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    n_out = max(1, int(round(frac * cols)))
    ch = rng.choice(cols, size=n_out, replace=False)
    x[:, ch] *= np.float32(factor)
    return x, np.sort(ch)


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
