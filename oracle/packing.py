"""Pure-numpy restatement of the packed tile layout (pins the packers).

Element W[n, k] of a row-major [N, K] matrix lands at flat element index
    ((rb * (K/32) + kt) * 64 + g * 16 + r) * 8 + e
with rb = p // 16, r = p % 16 (p = packed row), kt = k // 32, g = (k % 32) // 8,
e = k % 8.  For the interleaved gate/up layout, packed row p holds source row
gate[16*(p//32) + p%16] if p % 32 < 16, else up[16*(p//32) + p%16 - 16]
(up rows start at N/2).  Test infrastructure only.
"""

from __future__ import annotations

import numpy as np

LAYOUT_MFMA16X32 = 1
LAYOUT_MFMA16X32_GATEUP = 2


def packed_row_of_source(n_rows: int, layout: int) -> np.ndarray:
    """src_row -> packed row permutation (array indexed by source row)."""
    src = np.arange(n_rows)
    if layout == LAYOUT_MFMA16X32:
        return src
    half = n_rows // 2
    is_up = src >= half
    j = np.where(is_up, src - half, src)
    return (j // 16) * 32 + np.where(is_up, 16, 0) + j % 16


def flat_index(n_rows: int, k_cols: int, layout: int) -> np.ndarray:
    """[N, K] array of destination flat indices for every source element."""
    p = packed_row_of_source(n_rows, layout)[:, None]
    k = np.arange(k_cols)[None, :]
    rb, r = p // 16, p % 16
    kt, g, e = k // 32, (k % 32) // 8, k % 8
    return ((rb * (k_cols // 32) + kt) * 64 + g * 16 + r) * 8 + e


def pack(w: np.ndarray, layout: int = LAYOUT_MFMA16X32) -> np.ndarray:
    """Row-major [N, K] (any dtype) -> flat packed array."""
    n_rows, k_cols = w.shape
    out = np.empty(n_rows * k_cols, dtype=w.dtype)
    out[flat_index(n_rows, k_cols, layout)] = w
    return out


def unpack(packed: np.ndarray, n_rows: int, k_cols: int, layout: int = LAYOUT_MFMA16X32) -> np.ndarray:
    return packed[flat_index(n_rows, k_cols, layout)]
