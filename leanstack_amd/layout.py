"""Packed weight layout of the MI355X path (layout ids of include/leanstack_amd.h).

LAYOUT_MFMA16X32: W[N, K] bf16 becomes N/16 row-blocks x K/32 tiles of 1 KB;
inside a tile lane l of a 64-wide wavefront owns the 16 bytes
W[16*rb + l%16, 32*kt + 8*(l//16) : +8] -- one v_mfma_f32_16x16x32_bf16
A operand per 16-byte load.  In torch terms:

    packed = W.view(N/16, 16, K/32, 4, 8).permute(0, 2, 3, 1, 4)

LAYOUT_MFMA16X32_GATEUP: the fused [gate; up] matrix (gate rows first, as
leanstack's packer concatenates it, src/leanstack/pack.py:281-284) with its
16-row blocks interleaved gate, up, gate, up, ... before tiling.

The reference keeps these weights row-major (pack.py:269-286) and splits the
fused tensors into row views at load (src/leanstack/leanserve.py:429-438).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib

TILE_ROWS = 16
TILE_K = 32
TILE_BYTES = TILE_ROWS * TILE_K * 2

LAYOUT_NAMES = {
    _lib.LAYOUT_MFMA16X32: "mfma16x32",
    _lib.LAYOUT_MFMA16X32_GATEUP: "mfma16x32_gateup",
}
LAYOUT_IDS = {name: layout for layout, name in LAYOUT_NAMES.items()}


def check_shape(n: int, k: int, layout: int) -> None:
    if layout not in LAYOUT_NAMES:
        raise ValueError(f"unsupported packed layout id {layout}")
    if n <= 0 or k <= 0 or n % TILE_ROWS or k % TILE_K:
        raise ValueError(f"packed layout needs N % {TILE_ROWS} == 0 and K % {TILE_K} == 0, got N={n}, K={k}")
    if layout == _lib.LAYOUT_MFMA16X32_GATEUP and n % (2 * TILE_ROWS):
        raise ValueError(f"fused gate_up N={n} must be divisible by {2 * TILE_ROWS}")


def _interleave_gate_up(w: torch.Tensor) -> torch.Tensor:
    n, k = w.shape
    half = n // 2
    gate = w[:half].reshape(half // TILE_ROWS, TILE_ROWS, k)
    up = w[half:].reshape(half // TILE_ROWS, TILE_ROWS, k)
    return torch.stack((gate, up), dim=1).reshape(n, k)


def _deinterleave_gate_up(w: torch.Tensor) -> torch.Tensor:
    n, k = w.shape
    half = n // 2
    pairs = w.reshape(half // TILE_ROWS, 2, TILE_ROWS, k)
    return torch.cat((pairs[:, 0].reshape(half, k), pairs[:, 1].reshape(half, k)), dim=0)


def pack_tensor(w: torch.Tensor, layout: int = _lib.LAYOUT_MFMA16X32) -> torch.Tensor:
    """Re-tile row-major W[N, K] (bf16, any device) into a flat packed tensor."""
    if w.dtype != torch.bfloat16 or w.ndim != 2:
        raise ValueError(f"expected a 2-D bfloat16 weight, got {tuple(w.shape)} {w.dtype}")
    n, k = w.shape
    check_shape(n, k, layout)
    src = w.contiguous()
    if layout == _lib.LAYOUT_MFMA16X32_GATEUP:
        src = _interleave_gate_up(src)
    tiles = src.view(n // TILE_ROWS, TILE_ROWS, k // TILE_K, 4, 8).permute(0, 2, 3, 1, 4)
    return tiles.contiguous().view(-1)


def unpack_tensor(packed: torch.Tensor, n: int, k: int, layout: int = _lib.LAYOUT_MFMA16X32) -> torch.Tensor:
    """Inverse of pack_tensor: row-major W[N, K]."""
    check_shape(n, k, layout)
    if packed.numel() != n * k or packed.dtype != torch.bfloat16:
        raise ValueError(f"packed tensor has {packed.numel()} {packed.dtype} elements, expected {n * k} bf16")
    tiles = packed.reshape(n // TILE_ROWS, k // TILE_K, 4, TILE_ROWS, 8).permute(0, 3, 1, 2, 4)
    w = tiles.contiguous().view(n, k)
    if layout == _lib.LAYOUT_MFMA16X32_GATEUP:
        w = _deinterleave_gate_up(w)
    return w


@dataclass(frozen=True)
class PackedWeight:
    """A resident weight in a packed layout: the tensor the projection entry
    points receive in place of the reference's row-major nn weights."""

    data: torch.Tensor  # flat bf16, N*K elements, 16-byte aligned
    n: int
    k: int
    layout: int = _lib.LAYOUT_MFMA16X32

    def __post_init__(self) -> None:
        check_shape(self.n, self.k, self.layout)
        if self.data.dtype != torch.bfloat16 or self.data.numel() != self.n * self.k:
            raise ValueError("packed data must hold N*K bfloat16 elements")
        if not self.data.is_contiguous():
            raise ValueError("packed data must be contiguous")

    @property
    def shape(self) -> tuple[int, int]:
        """Logical [N, K] shape (as the reference's row-major weight had)."""
        return (self.n, self.k)

    @property
    def device(self) -> torch.device:
        return self.data.device

    @property
    def nbytes(self) -> int:
        return self.n * self.k * 2

    @property
    def out_features(self) -> int:
        return self.n // 2 if self.layout == _lib.LAYOUT_MFMA16X32_GATEUP else self.n

    def unpack(self) -> torch.Tensor:
        return unpack_tensor(self.data, self.n, self.k, self.layout)

    @classmethod
    def from_rowmajor(cls, w: torch.Tensor, layout: int = _lib.LAYOUT_MFMA16X32,
                      out: torch.Tensor | None = None) -> "PackedWeight":
        packed = pack_tensor(w, layout)
        if out is not None:
            if out.numel() != packed.numel() or out.dtype != torch.bfloat16:
                raise ValueError("destination view has the wrong size or dtype")
            out.copy_(packed)
            packed = out
        n, k = w.shape
        return cls(packed, n, k, layout)
