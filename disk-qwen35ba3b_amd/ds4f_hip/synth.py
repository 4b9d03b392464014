"""Deterministic synthetic inputs for the hybrid-attention workloads.

Every tensor of a workload is one splitmix64 stream (Steele, Lea & Flood,
"Fast splittable pseudorandom number generators", OOPSLA 2014).  The add
and finaliser constants are the ones the reference's own hash uses
(src/router.c:11-16, ``ds4f_mix64``), so the streams are the reference
project's family.  Stream for tensor id ``tid`` under seed ``S``:

    s_0 = S xor (tid * 0xD1B54A32D192ED03)            (mod 2**64)
    s_i = s_{i-1} + 0x9E3779B97F4A7C15,  draw_i = fmix64(s_i),  i >= 1

A uniform is ``(draw >> 11) * 2**-53``; a normal uses two consecutive
uniforms (Box-Muller, cosine branch): ``sqrt(-2 ln(1-u1)) * cos(2 pi u2)``.
Values are formed in double, cast to float32, and bf16 tensors are then
rounded to nearest-even.  The device generator in the HIP library computes
the same streams; both are checked against each other.
"""
from __future__ import annotations

import numpy as np

GOLDEN = 0x9E3779B97F4A7C15
TID_MUL = 0xD1B54A32D192ED03
MASK64 = (1 << 64) - 1

# Tensor ids.  A per-layer / per-step tensor uses tid(base, layer, step).
GQA_QGATE, GQA_K, GQA_V, GQA_QNW, GQA_KNW, GQA_KCACHE, GQA_VCACHE = 1, 2, 3, 4, 5, 6, 7
LIN_QKV, LIN_Z, LIN_A, LIN_B, LIN_CONVW, LIN_ALOG, LIN_DTB = 16, 17, 18, 19, 20, 21, 22
LIN_NORMW, LIN_STATE, LIN_CONVSTATE = 23, 24, 25
MLX4_Q, MLX4_SCALE, MLX4_BIAS, MLX4_X = 32, 33, 34, 35
BLK_STATE, BLK_INNORM = 36, 37


def tid(base: int, layer: int = 0, step: int = 0) -> int:
    """Tensor id of ``base`` for a given layer and decode step."""
    return (base + (layer << 8) + (step << 20)) & MASK64


def _fmix64(z: np.ndarray) -> np.ndarray:
    z = z ^ (z >> np.uint64(30))
    z = z * np.uint64(0xBF58476D1CE4E5B9)
    z = z ^ (z >> np.uint64(27))
    z = z * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def draws(seed: int, t: int, start: int, n: int) -> np.ndarray:
    """Raw 64-bit draws ``start .. start+n-1`` (0-based) of stream ``t``."""
    s0 = (seed ^ ((t * TID_MUL) & MASK64)) & MASK64
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        s = idx * np.uint64(GOLDEN) + np.uint64(s0)
    return _fmix64(s)


def uniform(seed: int, t: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    u = (draws(seed, t, 0, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    return (lo + (hi - lo) * u).astype(np.float32)


def normal64(seed: int, t: int, n: int) -> np.ndarray:
    """Standard normals in double (before scaling and casting)."""
    x = draws(seed, t, 0, 2 * n)
    u = (x >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    u1, u2 = u[0::2], u[1::2]
    return np.sqrt(-2.0 * np.log(1.0 - u1)) * np.cos(2.0 * np.pi * u2)


def normal(seed: int, t: int, n: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    return (mean + sigma * normal64(seed, t, n)).astype(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> float32 holding the nearest-even bf16 value."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16))
    return (r << np.uint64(16)).astype(np.uint32).view(np.float32).reshape(np.shape(x))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bits (nearest-even)."""
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
