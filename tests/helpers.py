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


def assert_greedy_rows(idx: torch.Tensor, ref_scores: torch.Tensor, got_scores: torch.Tensor, what: str = "") -> None:
    """Greedy tokens against the oracle's scores, unconditionally.

    delta = the largest |kernel score - oracle score| over the vocab (the
    kernel's own scores, read back).  Where the oracle's top-1 margin exceeds
    2*delta no score perturbation of that size can change the argmax, so the
    token must equal the oracle's; otherwise it must be one of the oracle's
    near-maximal tokens (within 2*delta of the top score), of which the
    oracle's top-2 are the usual pair."""
    ref_scores = ref_scores.float().reshape(-1, ref_scores.shape[-1])
    got_scores = got_scores.float().reshape(ref_scores.shape)
    idx = idx.reshape(-1)
    for row in range(ref_scores.shape[0]):
        s = ref_scores[row]
        delta = float((got_scores[row] - s).abs().max())
        top = torch.topk(s, 2)
        margin = float(top.values[0] - top.values[1])
        token = int(idx[row])
        print(f"{what} row {row}: token {token}, oracle {int(top.indices[0])}, margin {margin:.4g}, delta {delta:.3g}")
        if margin > 2 * delta:
            assert token == int(top.indices[0]), f"{what} row {row}: {token} != {int(top.indices[0])}"
        else:
            near = torch.nonzero(s >= top.values[0] - 2 * delta).view(-1).tolist()
            assert token in near, f"{what} row {row}: {token} not among the near-maximal {near[:8]}"
