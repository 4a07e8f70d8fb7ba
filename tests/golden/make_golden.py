"""Write the golden vectors of the projection path (tests/golden/*.npz).

The reference holds no golden vectors for this path (its tests pin only
shapes, tests/test_hot_kernel_cases.py:22-26), so these are computed here,
independently of torch: seeded numpy inputs rounded to bf16 (stored as uint16
bit patterns) and float64 expectations from oracle/brute.py.  Each case
follows a reference function:
  linear_m1     torch.mv(W, x)                qwen_explicit.py:787, :913
  linear_m5     F.linear(x, W)                qwen_explicit.py:748, :819
  silu_mul      F.silu(gate) * up of x.W^T    qwen_explicit.py:828-830, :942-948
  residual      residual + F.linear(x, W)     qwen_explicit.py:819-820, :830-831
  lm_head       argmax of fp32 scores         cutile_logits.py:17-31, :67-69
  pack          the packed tile layout        include/leanstack_amd.h

Run: python tests/golden/make_golden.py   (rewrites the .npz files)
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import brute, packing  # noqa: E402


def normal_bits(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    return brute.f32_to_bf16_bits((rng.standard_normal(shape) * std).astype(np.float32))


def linear_case(seed: int, n: int, k: int, m: int) -> dict:
    rng = np.random.default_rng(seed)
    w = normal_bits(rng, (n, k), 0.02)
    x = normal_bits(rng, (m, k), 1.0)
    return {"x": x, "w": w, "y64": brute.linear64(x, w), "bound": brute.fp32_sum_bound(x, w)}


def silu_case(seed: int, inter: int, k: int, m: int) -> dict:
    rng = np.random.default_rng(seed)
    w = normal_bits(rng, (2 * inter, k), 0.02)
    x = normal_bits(rng, (m, k), 1.0)
    gu = brute.linear64(x, w)
    gate, up = gu[:, :inter], gu[:, inter:]
    return {"x": x, "w": w, "gate64": gate, "up64": up, "out64": brute.silu_mul_chain(gate, up),
            "bound": brute.fp32_sum_bound(x, w)}


def residual_case(seed: int, n: int, k: int, m: int) -> dict:
    rng = np.random.default_rng(seed)
    w = normal_bits(rng, (n, k), 0.02)
    x = normal_bits(rng, (m, k), 1.0)
    r = normal_bits(rng, (m, n), 1.0)
    y = brute.linear64(x, w)
    return {"x": x, "w": w, "r": r, "y64": y, "out64": brute.round_bf16(brute.bf16_bits_to_f64(r) + brute.round_bf16(y)),
            "bound": brute.fp32_sum_bound(x, w)}


def lm_head_case(seed: int, v: int, k: int, m: int) -> dict:
    """Random head with a planted winner per row (row m wins at index idx[m]),
    and for the last row two identical winning rows (the lower index wins)."""
    rng = np.random.default_rng(seed)
    w = normal_bits(rng, (v, k), 0.02)
    x = normal_bits(rng, (m, k), 1.0)
    xf = brute.bf16_bits_to_f64(x)
    planted = rng.choice(v, size=m + 1, replace=False)
    for i in range(m):
        hot = np.sign(xf[i]) * 0.125
        w[planted[i]] = brute.f32_to_bf16_bits(hot.astype(np.float32))
    # last row: duplicate its planted row at a higher index -> tie, lowest index wins
    lo, hi = sorted((planted[m - 1], planted[m]))
    w[lo] = w[planted[m - 1]]
    w[hi] = w[planted[m - 1]]
    scores = brute.linear64(x, w)
    expect = brute.argmax_first(scores)
    top = np.sort(scores, axis=-1)[:, -2:]
    return {"x": x, "w": w, "scores64": scores, "expect": expect.astype(np.int64),
            "margin64": top[:, 1] - top[:, 0], "tie_low": np.int64(lo), "tie_high": np.int64(hi)}


def pack_case(seed: int) -> dict:
    rng = np.random.default_rng(seed)
    w = normal_bits(rng, (64, 96), 0.02)
    return {"w": w, "packed": packing.pack(w, packing.LAYOUT_MFMA16X32),
            "packed_gateup": packing.pack(w, packing.LAYOUT_MFMA16X32_GATEUP)}


CASES = {
    "linear_m1": lambda: linear_case(101, 64, 256, 1),
    "linear_m5": lambda: linear_case(102, 96, 128, 5),
    "silu_mul": lambda: silu_case(103, 64, 256, 3),
    "residual": lambda: residual_case(104, 64, 128, 2),
    "lm_head": lambda: lm_head_case(105, 1024, 256, 4),
    "pack": lambda: pack_case(106),
}


def main() -> None:
    for name, make in CASES.items():
        np.savez_compressed(HERE / f"{name}.npz", **make())
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
