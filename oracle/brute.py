"""Float64 numpy brute force of the projection arithmetic (pins the oracle).

Written without torch: bf16 values travel as uint16 bit patterns, products
and sums are exact-enough float64, and rounding to bf16 is done by hand
(round to nearest, ties to even).  Test infrastructure only.
"""

from __future__ import annotations

import numpy as np


def bf16_bits_to_f64(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float64 (exact)."""
    u32 = bits.astype(np.uint32) << np.uint32(16)
    return u32.view(np.float32).astype(np.float64)


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.asarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    bias = np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))
    return ((u + bias) >> np.uint64(16)).astype(np.uint16)


def round_bf16(values: np.ndarray) -> np.ndarray:
    """float64 -> nearest bf16 value (via float32), as float64."""
    return bf16_bits_to_f64(f32_to_bf16_bits(np.asarray(values, dtype=np.float64).astype(np.float32)))


def bf16_ulp(values: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |values| (8 significant bits)."""
    mag = np.maximum(np.abs(np.asarray(values, dtype=np.float64)), np.finfo(np.float32).tiny)
    return np.exp2(np.floor(np.log2(mag)) - 7.0)


def linear64(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """y[m, n] = sum_k x[m, k] * w[n, k] in float64 (x [M, K], w [N, K] bf16 bits)."""
    x = bf16_bits_to_f64(x_bits)
    w = bf16_bits_to_f64(w_bits)
    return x @ w.T


def abs_dot64(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """sum_k |x[m, k] * w[n, k]| -- scale of the fp32 accumulation error."""
    return np.abs(bf16_bits_to_f64(x_bits)) @ np.abs(bf16_bits_to_f64(w_bits)).T


def fp32_sum_bound(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """Worst-case error of any fp32 summation order of K exact products:
    gamma_K * sum|x w| with gamma_K = K u / (1 - K u), u = 2^-24."""
    k = x_bits.shape[-1]
    u = 2.0 ** -24
    gamma = k * u / (1.0 - k * u)
    return gamma * abs_dot64(x_bits, w_bits)


def silu64(g: np.ndarray) -> np.ndarray:
    return g / (1.0 + np.exp(-g))


def silu_mul_chain(gate64: np.ndarray, up64: np.ndarray) -> np.ndarray:
    """The reference's bf16 rounding chain for SiLU(gate)*up: gate_up rounded
    to bf16, silu rounded to bf16, product rounded to bf16."""
    g = round_bf16(gate64)
    u = round_bf16(up64)
    s = round_bf16(silu64(g))
    return round_bf16(s * u)


def argmax_first(scores: np.ndarray) -> np.ndarray:
    """Index of the first maximum along the last axis."""
    return np.argmax(scores, axis=-1)
