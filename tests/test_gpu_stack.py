"""GPU tests of the persistent stack kernel (lsk_stack_prepare / lsk_stack_run)."""

from __future__ import annotations

import pytest
import torch

from leanstack_amd import _lib, kernels
from leanstack_amd.geometry import QWEN3_4B as G
from leanstack_amd.layout import PackedWeight
from oracle import projections as ref
from tests.helpers import activations, assert_parity, weight

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _layer_weights(seed: int):
    h, q, i, qkv = G.hidden_size, G.q_dim, G.intermediate_size, G.qkv_dim
    return {
        "qkv": weight(qkv, h, seed=seed),
        "o": weight(h, q, seed=seed + 1),
        "gate_up": weight(2 * i, h, seed=seed + 2),
        "down": weight(h, i, seed=seed + 3),
    }


def _packed(ws):
    return {
        "qkv": PackedWeight.from_rowmajor(ws["qkv"].to(DEV)),
        "o": PackedWeight.from_rowmajor(ws["o"].to(DEV)),
        "gate_up": PackedWeight.from_rowmajor(ws["gate_up"].to(DEV), _lib.LAYOUT_MFMA16X32_GATEUP),
        "down": PackedWeight.from_rowmajor(ws["down"].to(DEV)),
    }


def _chain_specs(pws, x0, m, layers):
    """A real dependency chain: qkv(x) -> o(q part) + residual -> gate_up ->
    down + residual -> next layer's qkv ...  Output buffers start as NaN."""
    nan = float("nan")
    specs, bufs = [], []
    x = x0
    for l in range(layers):
        p = pws[l]
        qkv = torch.full((m, G.qkv_dim), nan, device=DEV, dtype=torch.bfloat16)
        h1 = torch.full((m, G.hidden_size), nan, device=DEV, dtype=torch.bfloat16)
        act = torch.full((m, G.intermediate_size), nan, device=DEV, dtype=torch.bfloat16)
        h2 = torch.full((m, G.hidden_size), nan, device=DEV, dtype=torch.bfloat16)
        i0 = len(specs)
        specs.append({"x": x, "weight": p["qkv"], "out": qkv, "depends_on": i0 - 1})
        specs.append({"x": qkv[:, : G.q_dim], "weight": p["o"], "out": h1, "epilogue": _lib.EPI_RESIDUAL_ADD,
                      "residual": x, "depends_on": i0})
        specs.append({"x": h1, "weight": p["gate_up"], "out": act, "epilogue": _lib.EPI_SILU_MUL,
                      "depends_on": i0 + 1})
        specs.append({"x": act, "weight": p["down"], "out": h2, "epilogue": _lib.EPI_RESIDUAL_ADD,
                      "residual": h1, "depends_on": i0 + 2})
        bufs.append((qkv, h1, act, h2))
        x = h2
    return specs, bufs


def _oracle_chain(ws_rows, x0_cpu, layers):
    x = x0_cpu
    outs = []
    for l in range(layers):
        w = ws_rows[l]
        qkv = ref.linear(x, w["qkv"])
        h1 = x + ref.linear(qkv[:, : G.q_dim], w["o"])
        act = ref.silu_mul(ref.linear(h1, w["gate_up"]), G.intermediate_size)
        h2 = h1 + ref.linear(act, w["down"])
        outs.append((qkv, h1, act, h2))
        x = h2
    return outs


@pytest.mark.parametrize("m", [1, 4, 8, 16])
def test_stack_dependency_chain_matches_oracle(gpu, m):
    layers = 2
    ws_rows = [_layer_weights(100 * l + 7) for l in range(layers)]
    pws = [_packed(w) for w in ws_rows]
    x0 = activations(m, G.hidden_size, seed=11 + m)
    specs, bufs = _chain_specs(pws, x0.to(DEV), m, layers)
    step = kernels.StackStep(specs, m, DEV)
    step.launch()
    assert step.error() == 0
    expect = _oracle_chain(ws_rows, x0, layers)
    for l in range(layers):
        for name, got, want in zip(("qkv", "h1", "act", "h2"), bufs[l], expect[l]):
            assert not torch.isnan(got).any(), f"layer {l} {name}: NaN (read before its producer finished?)"
            assert_parity(got.cpu(), want, f"stack chain M={m} layer {l} {name}")


def test_stack_independent_projections_and_determinism(gpu):
    """Independent projections (no dependencies) match the oracle, and two
    launches of one program give bitwise-identical outputs (fixed summation
    order: compute waves, then workgroups in index order)."""
    m = 3
    w = _layer_weights(5)
    p = _packed(w)
    xs = [activations(m, k, seed=20 + i) for i, k in enumerate((G.hidden_size, G.q_dim, G.hidden_size))]
    outs = [torch.full((m, n), float("nan"), device=DEV, dtype=torch.bfloat16)
            for n in (G.qkv_dim, G.hidden_size, G.intermediate_size)]
    specs = [
        {"x": xs[0].to(DEV), "weight": p["qkv"], "out": outs[0]},
        {"x": xs[1].to(DEV), "weight": p["o"], "out": outs[1]},
        {"x": xs[2].to(DEV), "weight": p["gate_up"], "out": outs[2], "epilogue": _lib.EPI_SILU_MUL},
    ]
    step = kernels.StackStep(specs, m, DEV)
    step.launch()
    assert step.error() == 0
    first = [o.clone() for o in outs]
    assert_parity(outs[0].cpu(), ref.linear(xs[0], w["qkv"]), "stack qkv")
    assert_parity(outs[1].cpu(), ref.linear(xs[1], w["o"]), "stack o")
    assert_parity(outs[2].cpu(), ref.silu_mul(ref.linear(xs[2], w["gate_up"]), G.intermediate_size), "stack gate_up")
    for o in outs:
        o.fill_(float("nan"))
    step.launch()
    assert step.error() == 0
    for a, b in zip(outs, first):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_stack_graph_replays(gpu):
    """Captured once, replayed several times with eager work in between: every
    replay gives the eager result and the workspace comes back clean."""
    m, layers = 2, 2
    ws_rows = [_layer_weights(300 + 10 * l) for l in range(layers)]
    pws = [_packed(w) for w in ws_rows]
    x0 = activations(m, G.hidden_size, seed=31).to(DEV)
    specs, bufs = _chain_specs(pws, x0, m, layers)
    step = kernels.StackStep(specs, m, DEV)
    step.launch()
    torch.cuda.synchronize()
    eager = [t.clone() for t in bufs[-1]]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step.launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        step.launch()
    for replay in range(4):
        for t in bufs[-1]:
            t.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(bufs[-1], eager):
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {replay} differs"
    assert step.error() == 0
    assert _sync_words_clear(step)


def _sync_words_clear(step) -> bool:
    """Exit counter and per-workgroup progress words are back to zero
    (workspace words 1 and 64 .. 64+G)."""
    grid = torch.cuda.get_device_properties(0).multi_processor_count
    words = step.workspace.view(torch.int32)
    return int(words[1]) == 0 and int(words[64:64 + grid].abs().sum()) == 0


def test_stack_rejects_bad_programs(gpu):
    w = _packed(_layer_weights(9))
    x = activations(1, G.hidden_size, seed=1).to(DEV)
    y = torch.empty((1, G.qkv_dim), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError):  # dependency on itself
        kernels.StackStep([{"x": x, "weight": w["qkv"], "out": y, "depends_on": 0}], 1, DEV)
    with pytest.raises(ValueError):  # M above 16
        kernels.StackStep([{"x": torch.zeros((17, G.hidden_size), device=DEV, dtype=torch.bfloat16),
                            "weight": w["qkv"], "out": torch.empty((17, G.qkv_dim), device=DEV,
                                                                   dtype=torch.bfloat16)}], 17, DEV)
    small = PackedWeight.from_rowmajor(weight(64, 128, seed=3).to(DEV))  # K = 128, not a multiple of 512
    with pytest.raises(ValueError):
        kernels.StackStep([{"x": torch.zeros((1, 128), device=DEV, dtype=torch.bfloat16), "weight": small,
                            "out": torch.empty((1, 64), device=DEV, dtype=torch.bfloat16)}], 1, DEV)
    # Tensors the program could only use through a copy: the program holds
    # addresses, so a copy would cut a producer -> consumer chain silently.
    wide = torch.zeros((2, G.hidden_size + 1), device=DEV, dtype=torch.bfloat16)
    y2 = torch.empty((2, G.qkv_dim), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="in place"):  # row stride not a multiple of 8
        kernels.StackStep([{"x": wide[:, : G.hidden_size], "weight": w["qkv"], "out": y2}], 2, DEV)
    with pytest.raises(ValueError, match="in place"):  # output columns not contiguous
        kernels.StackStep([{"x": torch.zeros((2, G.hidden_size), device=DEV, dtype=torch.bfloat16),
                            "weight": w["qkv"],
                            "out": torch.empty((G.qkv_dim, 2), device=DEV, dtype=torch.bfloat16).t()}], 2, DEV)
    with pytest.raises(ValueError):  # out of the wrong size
        kernels.StackStep([{"x": x, "weight": w["qkv"], "out": torch.empty((2, G.qkv_dim), device=DEV,
                                                                        dtype=torch.bfloat16)}], 1, DEV)


def test_stack_reused_buffer_across_layers(gpu):
    """gate_up(l) -> act -> down(l) with ONE act buffer for every layer (the
    decode step reuses its scratch): each layer's down must read its own
    layer's act, never a stale copy left by the previous layer in some
    XCD's cache.  Each down writes its own output so every layer is checked."""
    m, layers = 2, 8
    gen = torch.Generator(device=DEV).manual_seed(5)
    h, i = G.hidden_size, G.intermediate_size
    act = torch.full((m, i), float("nan"), device=DEV, dtype=torch.bfloat16)
    specs, outs, expect = [], [], []
    for l in range(layers):
        w_gu = (torch.randn((2 * i, h), generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
        w_d = (torch.randn((h, i), generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
        x = torch.randn((m, h), generator=gen, device=DEV).to(torch.bfloat16)
        gu = PackedWeight.from_rowmajor(w_gu, _lib.LAYOUT_MFMA16X32_GATEUP)
        dn = PackedWeight.from_rowmajor(w_d)
        y = torch.full((m, h), float("nan"), device=DEV, dtype=torch.bfloat16)
        base = len(specs)
        specs.append({"x": x, "weight": gu, "out": act, "epilogue": _lib.EPI_SILU_MUL, "depends_on": base - 1})
        specs.append({"x": act, "weight": dn, "out": y, "depends_on": base})
        outs.append(y)
        a = kernels.linear(x, gu, epilogue=_lib.EPI_SILU_MUL)
        expect.append(kernels.linear(a, dn))
    torch.cuda.synchronize()
    step = kernels.StackStep(specs, m, DEV)
    for _ in range(3):
        for y in outs:
            y.fill_(float("nan"))
        step.launch()
        torch.cuda.synchronize()
        assert step.error() == 0
        for l, (y, e) in enumerate(zip(outs, expect)):
            assert_parity(y.cpu(), e.cpu(), f"layer {l} down after shared act")
