"""GPU parity of the fused RMSNorm projection (lsk_rmsnorm_linear_bf16) against
the CPU oracle: F.rms_norm over the hidden dimension, then the projection.

Bar: cosine >= 0.9999 and normwise max relative error <= 1e-2 (the
projection bar), plus two sharper checks:
  - rows of powers of two, whose sums of squares are exact in fp32 in any
    order, give a normalised activation equal to the oracle's bit for bit, so
    the fused kernel's output equals the unfused kernel's on the
    oracle-normalised rows bit for bit (same tiles, same fp32 accumulation
    order);
  - on random rows the two differ on at most 2% of the outputs (a normalised
    value that lands next to a bf16 rounding boundary may round the other way
    when r or the product order differs in the last fp32 bit).
Rows carry different scales (0.05 .. 400) so that a per-row factor applied to
the wrong row, a dropped eps or a wrong mean fails the relative bound.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from leanstack_amd import _lib, kernels
from leanstack_amd.geometry import QWEN3_4B as G
from leanstack_amd.layout import PackedWeight
from oracle import projections as ref
from tests.helpers import assert_parity, seeded_normal, weight

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
EPS = G.rms_norm_eps
SCALES = (0.05, 1.0, 3.0, 400.0, 0.5, 20.0, 1.5, 0.2)


def _rows(m: int, k: int, seed: int) -> torch.Tensor:
    x = seeded_normal((m, k), 1.0, seed).float()
    s = torch.tensor([SCALES[i % len(SCALES)] for i in range(m)]).view(m, 1)
    return (x * s).to(torch.bfloat16)


def _norm_weight(k: int, seed: int) -> torch.Tensor:
    return (1.0 + seeded_normal((k,), 0.3, seed).float()).to(torch.bfloat16)


def _expect(x, nw, w, epilogue, residual, eps=EPS):
    y = ref.linear(ref.rmsnorm(x, nw, eps), w)
    if epilogue == _lib.EPI_SILU_MUL:
        return ref.silu_mul(y, w.shape[0] // 2)
    if epilogue == _lib.EPI_RESIDUAL_ADD:
        return residual + y
    return y


def _fused(x, nw, pw, epilogue=_lib.EPI_NONE, residual=None, eps=EPS):
    res = residual.to(DEV) if residual is not None else None
    y = kernels.rmsnorm_linear(x.to(DEV), nw.to(DEV), eps, pw, epilogue=epilogue, residual=res)
    torch.cuda.synchronize()
    return y.cpu()


def _unfused(xn, pw, epilogue=_lib.EPI_NONE, residual=None):
    res = residual.to(DEV) if residual is not None else None
    y = kernels.linear(xn.to(DEV), pw, epilogue=epilogue, residual=res)
    torch.cuda.synchronize()
    return y.cpu()


# (N, K, layout, epilogue): the two Qwen3-4B uses (QKV after input_layernorm,
# gate_up after post_attention_layernorm), the residual epilogue, and K values
# that take the round-based kernel (K/32 = 32, 128, 304).
CASES = {
    "qkv": (G.qkv_dim, G.hidden_size, _lib.LAYOUT_MFMA16X32, _lib.EPI_NONE),
    "gate_up": (2 * G.intermediate_size, G.hidden_size, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL),
    "residual": (G.hidden_size, G.hidden_size, _lib.LAYOUT_MFMA16X32, _lib.EPI_RESIDUAL_ADD),
    "k1024": (512, 1024, _lib.LAYOUT_MFMA16X32, _lib.EPI_NONE),
    "k4096_silu": (1024, 4096, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL),
    "k9728": (256, 9728, _lib.LAYOUT_MFMA16X32, _lib.EPI_NONE),
}
M_VALUES = {
    "qkv": [1, 2, 5, 8, 16],
    "gate_up": [1, 3, 16],
    "residual": [1, 4],
    "k1024": [1, 7, 16],
    "k4096_silu": [1, 9],
    "k9728": [2, 16],
}
PARAMS = [(name, m) for name in CASES for m in M_VALUES[name]]


@pytest.mark.parametrize("name,m", PARAMS, ids=[f"{n}-m{m}" for n, m in PARAMS])
def test_rmsnorm_linear_matches_oracle(gpu, name, m):
    n, k, layout, epi = CASES[name]
    seed = 7000 + 37 * m + n % 97
    w = weight(n, k, seed=seed)
    x = _rows(m, k, seed + 1)
    nw = _norm_weight(k, seed + 2)
    residual = seeded_normal((m, n), 1.0, seed + 3) if epi == _lib.EPI_RESIDUAL_ADD else None
    pw = PackedWeight.from_rowmajor(w.to(DEV), layout)
    y = _fused(x, nw, pw, epi, residual)
    assert_parity(y, _expect(x, nw, w, epi, residual), f"{name} M={m}")
    # Against the unfused kernel on the oracle-normalised rows: only the rare
    # element whose normalised value rounds differently may differ.
    xn = ref.rmsnorm(x, nw, EPS)
    y_unfused = _unfused(xn, pw, epi, residual)
    diff = (y != y_unfused).float().mean().item()
    assert diff <= 0.02, f"{name} M={m}: {diff:.4f} of the outputs differ from the unfused path"


def _random_norm_cases(count: int, seed: int) -> list[tuple[int, int, int, int]]:
    """(M, N, K, epilogue) with M = 1..16, N a multiple of 32 up to 8192 and K a
    multiple of 32 up to 12288: every activation-chunk and prologue form."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 17)), 32 * int(rng.integers(1, 257)), 32 * int(rng.integers(1, 385)),
             int(rng.integers(0, 3))) for _ in range(count)]


@pytest.mark.parametrize("m,n,k,epi", _random_norm_cases(16, 4242))
def test_rmsnorm_linear_random_shapes(gpu, m, n, k, epi):
    layout = _lib.LAYOUT_MFMA16X32_GATEUP if epi == _lib.EPI_SILU_MUL else _lib.LAYOUT_MFMA16X32
    seed = m * 131 + n + k
    w = weight(n, k, seed=seed)
    x = _rows(m, k, seed + 1)
    nw = _norm_weight(k, seed + 2)
    residual = seeded_normal((m, n), 1.0, seed + 3) if epi == _lib.EPI_RESIDUAL_ADD else None
    pw = PackedWeight.from_rowmajor(w.to(DEV), layout)
    y = _fused(x, nw, pw, epi, residual)
    assert_parity(y, _expect(x, nw, w, epi, residual), f"M={m} N={n} K={k} epi={epi}")


@pytest.mark.parametrize("name,m", [("qkv", 1), ("qkv", 16), ("gate_up", 4), ("k4096_silu", 3)])
def test_rmsnorm_linear_exact_sum_rows(gpu, name, m):
    """x in {+-1/4, +-1/2, +-1, +-2}: every partial sum of squares is a multiple
    of 1/16 far below 2^20, so r is the same in any summation order; and every
    x is a power of two, so x * r and x * nw are exact and the kernel's order
    (x * nw) * r rounds to the same value as the oracle's (x * r) * nw.  The
    weight rows are one-hot, so each projection output is one normalised value
    (a single-term sum, the same in any accumulation order or kernel shape):
    the fused output then equals the unfused kernel on the oracle's rows bit
    for bit."""
    n, k, layout, epi = CASES[name]
    gen = torch.Generator().manual_seed(8000 + m)
    mag = torch.tensor([0.25, 0.5, 1.0, 2.0])[torch.randint(0, 4, (m, k), generator=gen)]
    sign = torch.randint(0, 2, (m, k), generator=gen).float() * 2 - 1
    x = (mag * sign).to(torch.bfloat16)
    nw = _norm_weight(k, 8100 + m)
    w = torch.zeros((n, k), dtype=torch.bfloat16)
    w[torch.arange(n), (torch.arange(n) * 7 + m) % k] = 1.0
    pw = PackedWeight.from_rowmajor(w.to(DEV), layout)
    y = _fused(x, nw, pw, epi)
    xn = ref.rmsnorm(x, nw, EPS)
    assert torch.equal(y, _unfused(xn, pw, epi)), f"{name} M={m}"
    assert_parity(y, _expect(x, nw, w, epi, None), f"{name} M={m} exact rows")


def test_rmsnorm_linear_eps_and_zero_row(gpu):
    """A large eps is honoured (it rescales every row), and an all-zero row
    gives an all-zero output instead of NaN (r = 1/sqrt(eps) times 0)."""
    n, k = G.qkv_dim, G.hidden_size
    w = weight(n, k, seed=8300)
    x = _rows(3, k, 8301)
    x[1] = 0
    nw = _norm_weight(k, 8302)
    pw = PackedWeight.from_rowmajor(w.to(DEV), _lib.LAYOUT_MFMA16X32)
    y = _fused(x, nw, pw, eps=0.5)
    assert torch.all(y[1] == 0)
    keep = [0, 2]
    assert_parity(y[keep], _expect(x, nw, w, _lib.EPI_NONE, None, eps=0.5)[keep], "eps=0.5")


def test_rmsnorm_linear_strided_rows_and_repeat(gpu):
    """Rows at a stride > K (a view into a wider buffer) and two calls in a row
    give the same result as contiguous rows."""
    n, k = 2 * G.intermediate_size, G.hidden_size
    w = weight(n, k, seed=8400)
    wide = _rows(5, k + 64, 8401)
    x = wide[:, :k]
    nw = _norm_weight(k, 8402)
    pw = PackedWeight.from_rowmajor(w.to(DEV), _lib.LAYOUT_MFMA16X32_GATEUP)
    xd = wide.to(DEV)[:, :k]
    nwd = nw.to(DEV)
    y1 = kernels.rmsnorm_linear(xd, nwd, EPS, pw, epilogue=_lib.EPI_SILU_MUL)
    y2 = kernels.rmsnorm_linear(xd.contiguous(), nwd, EPS, pw, epilogue=_lib.EPI_SILU_MUL)
    torch.cuda.synchronize()
    assert torch.equal(y1.cpu(), y2.cpu())
    assert_parity(y1.cpu(), _expect(x, nw, w, _lib.EPI_SILU_MUL, None), "strided rows")


def test_decode_step_with_norms_fused_matches_separate(gpu):
    """DecodeLinearStack.launch_with_norms: the step with its RMSNorms fused
    into QKV / gate_up gives the same outputs as F.rms_norm launches ahead of
    unfused projections (to the projection bar), at M = 1 and 8."""
    from leanstack_amd.stack import DecodeLinearStack, LayerProjections

    gen = torch.Generator(device=DEV).manual_seed(8500)

    def pw(n, k, layout=_lib.LAYOUT_MFMA16X32):
        return PackedWeight.from_rowmajor((torch.randn((n, k), generator=gen, device=DEV) * 0.02)
                                          .to(torch.bfloat16), layout)

    layers = [LayerProjections(pw(G.qkv_dim, G.hidden_size), pw(G.hidden_size, G.q_dim),
                               pw(2 * G.intermediate_size, G.hidden_size, _lib.LAYOUT_MFMA16X32_GATEUP),
                               pw(G.hidden_size, G.intermediate_size)) for _ in range(2)]
    stack = DecodeLinearStack(layers, G, max_rows=8, device=torch.device(DEV))
    for m in (1, 8):
        stack.launch_with_norms(m, fused=True)
        torch.cuda.synchronize()
        fused = (stack.y_qkv[:m].cpu(), stack.act[:m].cpu(), stack.y_down[:m].cpu())
        stack.launch_with_norms(m, fused=False)
        torch.cuda.synchronize()
        separate = (stack.y_qkv[:m].cpu(), stack.act[:m].cpu(), stack.y_down[:m].cpu())
        for what, a, b in zip(("qkv", "act", "down"), fused, separate):
            assert_parity(a, b, f"step with norms M={m} {what}")
