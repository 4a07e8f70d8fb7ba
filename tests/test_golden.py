"""The CPU oracle against the committed golden vectors (tests/golden/*.npz)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import brute, packing
from oracle import projections as ref
from tests.helpers import from_bits

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def within(got, y64, bound):
    slack = 0.5 * np.maximum(brute.bf16_ulp(y64), brute.bf16_ulp(got)) + bound + 1e-30
    return np.all(np.abs(got - y64) <= slack)


@pytest.mark.parametrize("name", ["linear_m1", "linear_m5"])
def test_linear_golden(name):
    g = load(name)
    x, w = from_bits(g["x"]), from_bits(g["w"])
    got = ref.linear(x, w).double().numpy()
    assert within(got, g["y64"], g["bound"])
    if x.shape[0] == 1:
        assert within(ref.mv(w, x[0]).double().numpy()[None], g["y64"], g["bound"])


def test_silu_mul_golden():
    g = load("silu_mul")
    inter = g["gate64"].shape[1]
    got = ref.silu_mul(ref.linear(from_bits(g["x"]), from_bits(g["w"])), inter).double().numpy()
    # The gate/up products round to bf16 before SiLU; near a rounding boundary
    # the fp32 sum may round the other way, moving the result by an ulp of
    # the gate.  Bound: one bf16 ulp of the output plus the propagated error.
    slack = brute.bf16_ulp(g["out64"]) * 2 + 4 * g["bound"].max()
    assert np.all(np.abs(got - g["out64"]) <= slack)
    assert np.mean(got == g["out64"]) > 0.98


def test_residual_golden():
    g = load("residual")
    got = (from_bits(g["r"]) + ref.linear(from_bits(g["x"]), from_bits(g["w"]))).double().numpy()
    assert np.all(np.abs(got - g["out64"]) <= brute.bf16_ulp(g["out64"]) + 2 * g["bound"])


def test_lm_head_golden():
    g = load("lm_head")
    x, w = from_bits(g["x"]), from_bits(g["w"])
    got = ref.logits_argmax(x, w).view(-1).numpy()
    assert np.array_equal(got, g["expect"])
    assert g["expect"][-1] == g["tie_low"] and g["margin64"][-1] == 0.0


def test_pack_golden():
    g = load("pack")
    assert np.array_equal(packing.pack(g["w"], packing.LAYOUT_MFMA16X32), g["packed"])
    assert np.array_equal(packing.pack(g["w"], packing.LAYOUT_MFMA16X32_GATEUP), g["packed_gateup"])
    n, k = g["w"].shape
    assert np.array_equal(packing.unpack(g["packed"], n, k, packing.LAYOUT_MFMA16X32), g["w"])
