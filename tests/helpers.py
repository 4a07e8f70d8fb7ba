"""Shared input generation and parity metrics for the tests."""

from __future__ import annotations

import numpy as np
import torch

# Parity bar for bf16 outputs with fp32 accumulation.
COS_MIN = 0.9999
REL_MAX = 1e-2


def seeded_normal(shape, std: float, seed: int) -> torch.Tensor:
    """N(0, std^2) drawn in fp32 on the CPU from a seeded generator, rounded to bf16."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * std).to(torch.bfloat16)


def weight(n: int, k: int, seed: int = 0) -> torch.Tensor:
    return seeded_normal((n, k), 0.02, seed)


def activations(m: int, k: int, seed: int = 1) -> torch.Tensor:
    return seeded_normal((m, k), 1.0, seed)


def parity(y: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    """(cosine similarity, normwise max relative error max|y-ref| / max|ref|)."""
    a = y.detach().float().cpu().reshape(-1).double()
    b = ref.detach().float().cpu().reshape(-1).double()
    cos = float(torch.dot(a, b) / (a.norm() * b.norm()).clamp_min(1e-300))
    rel = float((a - b).abs().max() / b.abs().max().clamp_min(1e-300))
    return cos, rel


def assert_parity(y: torch.Tensor, ref: torch.Tensor, what: str = "") -> tuple[float, float]:
    assert y.shape == ref.shape, f"{what}: shape {tuple(y.shape)} != {tuple(ref.shape)}"
    cos, rel = parity(y, ref)
    assert cos >= COS_MIN and rel <= REL_MAX, f"{what}: cos={cos:.6f} rel={rel:.3e}"
    return cos, rel


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 numpy bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)
