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


# ---------------------------------------------------------------- compositions
#
# Float64 restatements of the decoder-layer compositions, with a bf16 rounding
# wherever the reference's torch code produces a bf16 tensor (each projection,
# each RMSNorm, each elementwise op); inputs and outputs are float64 arrays
# holding bf16 values.  They pin the oracle's composite functions, whose
# order of operations (which tensor is normalised, where each residual joins)
# is what the checks are about.


def proj64(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """bf16(x . W^T): a projection of float64 rows x [.., K] by W [N, K]."""
    return round_bf16(x @ w.T)


def rmsnorm64(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """RMSNorm over the last axis rounded once to bf16: x * r * w with
    r = 1 / sqrt(mean(x^2) + eps)."""
    r = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return round_bf16(x * r * w)


def silu_mul64(gate_up: np.ndarray, gate_dim: int) -> np.ndarray:
    """The bf16 chain of SiLU(gate) * up over a [.., gate | up] array whose
    values are already bf16."""
    return silu_mul_chain(gate_up[..., :gate_dim], gate_up[..., gate_dim:])


def rope64(t: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE over the last axis of t with a bf16 rounding after
    each product and each sum: (a, b) -> (a c - b s, b c + a s)."""
    h = t.shape[-1] // 2
    a, b = t[..., :h], t[..., h:]
    first = round_bf16(round_bf16(a * cos) - round_bf16(b * sin))
    second = round_bf16(round_bf16(b * cos) + round_bf16(a * sin))
    return np.concatenate((first, second), axis=-1)


def qk_heads64(qkv: np.ndarray, n_q: int, n_kv: int, d: int, q_norm_w: np.ndarray, k_norm_w: np.ndarray,
               eps: float, cos: np.ndarray, sin: np.ndarray):
    """Split a [q | k | v] row into heads, RMSNorm each q head with q_norm_w
    and each k head with k_norm_w, then RoPE: q [n_q, d], k, v [n_kv, d]."""
    q = qkv[: n_q * d].reshape(n_q, d)
    k = qkv[n_q * d : (n_q + n_kv) * d].reshape(n_kv, d)
    v = qkv[(n_q + n_kv) * d :].reshape(n_kv, d)
    return rope64(rmsnorm64(q, q_norm_w, eps), cos, sin), rope64(rmsnorm64(k, k_norm_w, eps), cos, sin), v


def attention64(q: np.ndarray, keys: np.ndarray, values: np.ndarray, scale: float) -> np.ndarray:
    """softmax(q K^T scale) V per q head, q head h reading kv head
    h // (n_q / n_kv); q [n_q, d], keys / values [n_kv, S, d]; bf16 output."""
    group = q.shape[0] // keys.shape[0]
    out = np.empty_like(q)
    for h in range(q.shape[0]):
        s = keys[h // group] @ q[h] * scale
        p = np.exp(s - s.max())
        out[h] = p @ values[h // group] / p.sum()
    return round_bf16(out)


def mlp_forward64(hidden, gate_up_w, gate_dim, down_w):
    """down(SiLU(gate) * up) of gate_up(hidden)."""
    return proj64(silu_mul64(proj64(hidden, gate_up_w), gate_dim), down_w)


def post_attention_mlp64(attn, residual, o_w, post_ln_w, gate_up_w, gate_dim, down_w, eps):
    """h = residual + o(attn); h + MLP(rmsnorm(h))."""
    h = round_bf16(residual + proj64(attn, o_w))
    return round_bf16(h + mlp_forward64(rmsnorm64(h, post_ln_w, eps), gate_up_w, gate_dim, down_w))


def decode_layer64(hidden, input_ln_w, qkv_w, n_q, n_kv, d, q_norm_w, k_norm_w, cos, sin, k_cache, v_cache, pos,
                   scale, o_w, post_ln_w, gate_up_w, gate_dim, down_w, eps):
    """One decode token through a layer: input RMSNorm, QKV, q/k heads,
    append at row pos, attention over rows 0..pos, o_proj + residual, then
    the MLP block with its RMSNorm and residual.  Returns (out [H], k_cache,
    v_cache) with the new row written."""
    qkv = proj64(rmsnorm64(hidden, input_ln_w, eps), qkv_w)
    q, k, v = qk_heads64(qkv, n_q, n_kv, d, q_norm_w, k_norm_w, eps, cos, sin)
    k_cache = k_cache.copy()
    v_cache = v_cache.copy()
    k_cache[:, pos] = k
    v_cache[:, pos] = v
    attn = attention64(q, k_cache[:, : pos + 1], v_cache[:, : pos + 1], scale).reshape(-1)
    h = round_bf16(hidden + proj64(attn, o_w))
    out = round_bf16(h + mlp_forward64(rmsnorm64(h, post_ln_w, eps), gate_up_w, gate_dim, down_w))
    return out, k_cache, v_cache
