"""Projections of 17..128 rows (verify batches, short prefills, the
reference's M = 64 hot-kernel cases): the skinny kernel, with and without the
split of every row-block's K range, against the oracle's F.linear."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle.projections as ref
from leanstack_amd import _lib, kernels
from leanstack_amd.geometry import QWEN3_4B as G
from leanstack_amd.layout import PackedWeight
from tests.helpers import activations, assert_parity, weight

pytestmark = pytest.mark.gpu


def _plan(m: int, n: int, k: int, ws_bytes: int) -> list[int]:
    plan = (ctypes.c_int * 4)()
    assert _lib.load().lsk_linear_plan(m, n, k, ws_bytes, plan) == _lib.OK, _lib.last_error()
    return list(plan)


def _run(m, n, k, epi, split, seed):
    layout = _lib.LAYOUT_MFMA16X32_GATEUP if epi == _lib.EPI_SILU_MUL else _lib.LAYOUT_MFMA16X32
    w = weight(n, k, seed=seed)
    x = activations(m, k, seed=seed + 1)
    r = activations(m, n, seed=seed + 2) if epi == _lib.EPI_RESIDUAL_ADD else None
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(w.to(dev), layout)
    ws = kernels.prefill_workspace(dev, m, n, k) if split else None
    xd, rd = x.to(dev), (r.to(dev) if r is not None else None)
    print(f"case M={m} N={n} K={k} epi={epi} split={split} plan={_plan(m, n, k, 0 if ws is None else ws.numel())}",
          flush=True)
    y1 = kernels.linear(xd, pw, epilogue=epi, residual=rd, workspace=ws)
    y2 = kernels.linear(xd, pw, epilogue=epi, residual=rd, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16)), "not bitwise repeatable"
    if ws is not None:
        assert int(ws.view(torch.int32)[64:2048].abs().sum()) == 0, "arrival counters not zero after the call"
    yl = ref.linear(x, w)
    expect = ref.silu_mul(yl, n // 2) if epi == _lib.EPI_SILU_MUL else (r + yl if r is not None else yl)
    return y1.cpu(), expect


# every token-group count (2..8 groups of 16; 5 and 7 run as 6 and 8), part-full last groups
TOKEN_COUNTS = [17, 31, 32, 33, 48, 64, 65, 80, 96, 100, 112, 113, 127, 128]


@pytest.mark.parametrize("m", TOKEN_COUNTS)
@pytest.mark.parametrize("split", [False, True])
def test_skinny_o_proj(gpu, m, split):
    """o_proj (160 row-blocks, two per workgroup; with the workspace K split
    three ways) at every token-group count, plain epilogue."""
    y, expect = _run(m, G.hidden_size, G.q_dim, _lib.EPI_NONE, split, seed=1000 + m)
    assert_parity(y, expect, f"o_proj M={m} split={split}")


@pytest.mark.parametrize("m", [17, 64, 100, 128])
@pytest.mark.parametrize("split", [False, True])
def test_skinny_down_residual(gpu, m, split):
    """down_proj + residual (K = 9728) through the split combine's epilogue."""
    y, expect = _run(m, G.hidden_size, G.intermediate_size, _lib.EPI_RESIDUAL_ADD, split, seed=1100 + m)
    assert_parity(y, expect, f"down+residual M={m} split={split}")


@pytest.mark.parametrize("m", [17, 64, 128])
@pytest.mark.parametrize("split", [False, True])
def test_skinny_gate_up_silu(gpu, m, split):
    """The fused gate_up with SiLU*up: 608 gate/up pairs fill the chip, so
    the workspace changes nothing (and at 128 rows the 128 x 128 GEMM takes
    it); a narrow gate_up (64 pairs) splits."""
    y, expect = _run(m, 2 * G.intermediate_size, G.hidden_size, _lib.EPI_SILU_MUL, split, seed=1200 + m)
    assert_parity(y, expect, f"gate_up+silu M={m} split={split}")
    y, expect = _run(m, 2048, G.hidden_size, _lib.EPI_SILU_MUL, split, seed=1250 + m)
    assert_parity(y, expect, f"gate_up(2048)+silu M={m} split={split}")


@pytest.mark.parametrize("m", [24, 64, 128])
def test_skinny_qkv_and_kv(gpu, m):
    """Fused QKV (384 row-blocks, no split) and the kv slice (64 row-blocks,
    split four ways on 256 CUs)."""
    y, expect = _run(m, G.qkv_dim, G.hidden_size, _lib.EPI_NONE, True, seed=1300 + m)
    assert_parity(y, expect, f"qkv M={m}")
    y, expect = _run(m, 1024, G.hidden_size, _lib.EPI_NONE, True, seed=1350 + m)
    assert_parity(y, expect, f"kv M={m}")


def test_skinny_plans(gpu):
    """The plan lsk_linear_plan reports for the skinny kernel, and a
    workspace too small for the split refused before launch."""
    lib = _lib.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    ws_of = lambda m, n, k: lib.lsk_workspace_bytes(_lib.OP_LINEAR, m, n, k)  # noqa: E731
    for (m, n, k) in ((64, 1024, 2560), (64, 2560, 4096), (64, 2560, 9728), (64, 4096, 2560), (128, 6144, 2560),
                      (64, 9728, 2560), (17, 4096, 2560)):
        ws = ws_of(m, n, k)
        p = _plan(m, n, k, ws)
        assert p[0] in (16, 32, 64) and p[1] == n // p[0], p
        groups = p[1]
        assert p[0] < 64 or m <= 64  # 4 row-blocks per workgroup only up to 4 token groups
        if p[3] == 1:
            assert p[2] == 0
        else:
            assert p[2] == groups and ws > 0
            assert abs(groups * p[3] - cus) <= groups  # the split brings the grid to about one per CU
            plan = (ctypes.c_int * 4)()
            # (the reported size covers the SiLU*up split too)
            assert lib.lsk_linear_plan(m, n, k, 8192, plan) == _lib.ERR_WORKSPACE
        nows = _plan(m, n, k, 0)
        assert nows[2] == 0 and nows[3] == 1
    # 65..128 rows of a wide projection take the 128 x 128 GEMM (no plan, no workspace)
    assert _plan(128, 9728, 2560, ws_of(128, 9728, 2560)) == [0, 0, 0, 1] and ws_of(128, 9728, 2560) == 0
    if cus == 256:
        assert _plan(64, 1024, 2560, ws_of(64, 1024, 2560)) == [16, 64, 64, 4]     # kv: narrow, one row-block
        assert _plan(64, 2560, 9728, ws_of(64, 2560, 9728)) == [32, 80, 80, 3]     # down: pairs, 3 splits
        assert _plan(64, 2560, 9728, 0) == [32, 80, 0, 1]                          # down without a workspace
        assert _plan(128, 2560, 9728, ws_of(128, 2560, 9728)) == [32, 80, 80, 3]
        assert _plan(64, 4096, 2560, ws_of(64, 4096, 2560)) == [32, 128, 128, 2]   # q
        assert _plan(64, 9728, 2560, ws_of(64, 9728, 2560)) == [64, 152, 0, 1]     # gate_up half: 4 row-blocks
        assert _plan(17, 4096, 2560, ws_of(17, 4096, 2560)) == [16, 256, 0, 1]     # q at 17 rows: one per CU


def test_skinny_refuses_small_workspace(gpu):
    """A workspace below the split's need is refused with ERR_WORKSPACE and
    nothing is written."""
    m, n, k = 64, 1024, 2560
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(weight(n, k, seed=5).to(dev))
    small = torch.zeros(16384, device=dev, dtype=torch.uint8)  # the split's flags fit, its partials do not
    out = torch.full((m, n), 7.0, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="workspace"):
        kernels.linear(activations(m, k, seed=6).to(dev), pw, out=out, workspace=small)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


@pytest.mark.parametrize("split", [False, True])
def test_skinny_strides(gpu, split):
    """Activations with a row stride past K, outputs and residual at the
    narrowest strides the ABI accepts (ldy = N + 4, ldr = N + 1): nothing
    between rows is written."""
    m, n, k = 72, 1024, 2560
    dev = torch.device("cuda:0")
    w = weight(n, k, seed=7)
    x = activations(m, k, seed=8)
    r = activations(m, n, seed=9)
    pw = PackedWeight.from_rowmajor(w.to(dev))
    xb = torch.zeros((m, k + 40), device=dev, dtype=torch.bfloat16)
    xb[:, :k] = x.to(dev)
    yb = torch.full((m, n + 4), -3.0, device=dev, dtype=torch.bfloat16)
    rb = torch.zeros((m, n + 1), device=dev, dtype=torch.bfloat16)
    rb[:, :n] = r.to(dev)
    lib = _lib.load()
    ws = kernels.prefill_workspace(dev, m, n, k) if split else None
    ws_ptr, ws_bytes = (None, 0) if ws is None else (ws.data_ptr(), ws.numel())
    st = lib.lsk_linear_bf16(pw.data.data_ptr(), pw.layout, n, k, xb.data_ptr(), m, k + 40, yb.data_ptr(), n + 4,
                             _lib.EPI_RESIDUAL_ADD, rb.data_ptr(), n + 1, ws_ptr, ws_bytes,
                             torch.cuda.current_stream().cuda_stream)
    assert st == _lib.OK, _lib.last_error()
    torch.cuda.synchronize()
    assert bool((yb[:, n:] == -3.0).all()), "wrote between output rows"
    assert_parity(yb[:, :n].cpu(), r + ref.linear(x, w), f"strided skinny split={split}")


def _skinny_shapes(count: int, seed: int) -> list[tuple[int, int, int, int]]:
    """Seeded (M, N, K, epilogue) with M = 17..128 and N, K any multiple of
    32 up to 4096 (off every GEMM tile grid too)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        m = int(rng.integers(17, 129))
        n = 32 * int(rng.integers(1, 129))
        k = 32 * int(rng.integers(2, 129))
        out.append((m, n, k, int(rng.integers(0, 3))))
    return out


@pytest.mark.parametrize("m,n,k,epi", _skinny_shapes(12, 77))
def test_skinny_random_shapes(gpu, m, n, k, epi):
    """Seeded random shapes through the auto workspace, every row against the
    oracle."""
    y, expect = _run(m, n, k, epi, True, seed=m + n + k)
    assert_parity(y, expect, f"M={m} N={n} K={k} epi={epi}")
