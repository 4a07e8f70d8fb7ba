"""GPU parity of the HIP projections against the CPU oracle (same seeded inputs).

Bar: cosine >= 0.9999 and normwise max relative error <= 1e-2 for bf16
outputs with fp32 accumulation; exact argmax for the lm_head.  Every case
calls the C ABI through leanstack_amd.kernels.
"""

from __future__ import annotations

import ctypes
import numpy as np
import pytest
import torch

from leanstack_amd import _lib, kernels
from leanstack_amd.geometry import QWEN3_4B as G
from leanstack_amd.layout import PackedWeight
from oracle import brute
from oracle import projections as ref
from tests.helpers import activations, assert_greedy_rows, assert_parity, bits, weight

pytestmark = pytest.mark.gpu

PROJ = {
    "qkv_proj": (G.qkv_dim, G.hidden_size),
    "o_proj": (G.hidden_size, G.q_dim),
    "down_proj": (G.hidden_size, G.intermediate_size),
}


def _gpu_linear(x, w, layout=_lib.LAYOUT_MFMA16X32, epilogue=_lib.EPI_NONE, residual=None, workspace="auto"):
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(w.to(dev), layout)
    res = residual.to(dev) if residual is not None else None
    y = kernels.linear(x.to(dev), pw, epilogue=epilogue, residual=res, workspace=workspace)
    torch.cuda.synchronize()
    return y.cpu()


# The reference's hot-kernel GEMM cases (src/leanstack/hot_kernels.py:79-166):
# key -> (M, N, K).  gate_up there is one half of the fused projection (no
# SiLU); q_proj and kv_proj are the row slices of the fused QKV.
HOT_KERNEL_CASES = {
    "q_proj_prefill64": (64, 4096, 2560),
    "q_proj_prefill1024": (1024, 4096, 2560),
    "kv_proj_prefill64": (64, 1024, 2560),
    "o_proj_prefill64": (64, 2560, 4096),
    "gate_up_proj_prefill64": (64, 9728, 2560),
    "down_proj_prefill64": (64, 2560, 9728),
}


@pytest.mark.parametrize("case", sorted(HOT_KERNEL_CASES))
def test_reference_hot_kernel_cases(gpu, case):
    """Every GEMM case of the reference's hot-kernel table at its own M
    (64, and 1024 for q_proj) against the oracle's F.linear."""
    m, n, k = HOT_KERNEL_CASES[case]
    w = weight(n, k, seed=70 + n % 97)
    x = activations(m, k, seed=71)
    assert_parity(_gpu_linear(x, w), ref.linear(x, w), case)


def test_dispatch_timing_times_each_kernel(gpu):
    """lsk_dispatch_timing_begin/end bind an event pair to each dispatch:
    one positive duration per kernel launched, in order, results unchanged;
    launches past the limit run untimed; no nested or unmatched timing."""
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(weight(2560, 4096, seed=3).to(dev))
    xd = activations(1, 4096, seed=4).to(dev)
    plain = kernels.linear(xd, pw)
    torch.cuda.synchronize()
    outs = []
    durs = kernels.kernel_durations_us(lambda: outs.extend(kernels.linear(xd, pw) for _ in range(5)), max_dispatches=8)
    assert len(durs) == 5 and all(0.0 < d < 1e4 for d in durs), durs
    for o in outs:
        assert torch.equal(o.view(torch.int16), plain.view(torch.int16))
    assert len(kernels.kernel_durations_us(lambda: [kernels.linear(xd, pw) for _ in range(3)], max_dispatches=2)) == 2
    lib = _lib.load()
    n = ctypes.c_int(-1)
    assert lib.lsk_dispatch_timing_begin(4) == _lib.OK
    assert lib.lsk_dispatch_timing_begin(4) == _lib.ERR_INVALID
    assert lib.lsk_dispatch_timing_end(None, 0, ctypes.byref(n)) == _lib.OK and n.value == 0
    assert lib.lsk_dispatch_timing_end(None, 0, ctypes.byref(n)) == _lib.ERR_INVALID
    assert lib.lsk_dispatch_timing_begin(0) == _lib.ERR_INVALID


def test_auto_workspaces_are_per_stream(gpu):
    """workspace="auto" keeps one split-K workspace per (device, stream):
    calls on another stream never share the arrival flags and partial slots
    of a call that may overlap them."""
    dev = torch.device("cuda:0")
    a = kernels.prefill_workspace(dev, 2048, 2560, 4096)
    other = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(other):
        b = kernels.prefill_workspace(dev, 2048, 2560, 4096)
    assert a is not None and b is not None
    assert a.data_ptr() != b.data_ptr()
    assert kernels.prefill_workspace(dev, 2048, 2560, 4096).data_ptr() == a.data_ptr()


def test_o_proj_gemv_2560x4096(gpu):
    """x[1,4096] ~ N(0,1), W[2560,4096] ~ N(0,0.02): elementwise within bf16
    rounding + the fp32 summation bound of the float64 brute force."""
    w = weight(2560, 4096, seed=0)
    x = activations(1, 4096, seed=1)
    y = _gpu_linear(x, w)
    assert_parity(y.view(-1), ref.mv(w, x.view(-1)), "o_proj M=1 vs torch.mv")
    y64 = brute.linear64(bits(x), bits(w))
    bound = brute.fp32_sum_bound(bits(x), bits(w))
    got = y.double().numpy()
    slack = 0.5 * np.maximum(brute.bf16_ulp(y64), brute.bf16_ulp(got)) + bound
    assert np.all(np.abs(got - y64) <= slack)


@pytest.mark.parametrize("name", sorted(PROJ))
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 15, 16])
def test_decode_projection(gpu, name, m):
    """Every M of the decode forms: the staged-activation kernels switch their
    chunks per lane with M (QKV 1..5 up to M = 8, o_proj 1..8 up to M = 8,
    down 2..6 up to M = 5, then two phases of 4 or 5 at M = 6..8), then
    fragment loads per tile; M = 9..15 leave part of the 16 MFMA columns
    unused."""
    n, k = PROJ[name]
    w = weight(n, k, seed=10 + m)
    x = activations(m, k, seed=100 + m)
    y = _gpu_linear(x, w)
    expect = ref.mv(w, x.view(-1)).view(1, -1) if m == 1 else ref.linear(x, w)
    assert_parity(y, expect, f"{name} M={m}")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 15, 16])
def test_decode_gate_up_silu(gpu, m):
    """Every M of the gate_up decode forms (4 waves x 10 pairs up to M = 2,
    then 8 x 5 with 1..5 staged chunks per lane, and the 16-row kernel)."""
    n, k = 2 * G.intermediate_size, G.hidden_size
    w = weight(n, k, seed=20 + m)
    x = activations(m, k, seed=200 + m)
    y = _gpu_linear(x, w, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL)
    expect = ref.silu_mul(ref.linear(x, w), G.intermediate_size)
    assert_parity(y, expect, f"gate_up+silu M={m}")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 12])
def test_decode_down_residual(gpu, m):
    n, k = G.hidden_size, G.intermediate_size
    w = weight(n, k, seed=30 + m)
    x = activations(m, k, seed=300 + m)
    r = activations(m, n, seed=301 + m)
    y = _gpu_linear(x, w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=r)
    assert_parity(y, r + ref.linear(x, w), f"down+residual M={m}")


@pytest.mark.parametrize("m", [1, 5, 6, 12])
def test_decode_o_residual(gpu, m):
    """o_proj with the residual epilogue (values read before the weight stream)."""
    n, k = G.hidden_size, G.q_dim
    w = weight(n, k, seed=40 + m)
    x = activations(m, k, seed=400 + m)
    r = activations(m, n, seed=401 + m)
    y = _gpu_linear(x, w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=r)
    assert_parity(y, r + ref.linear(x, w), f"o+residual M={m}")


@pytest.mark.parametrize("name", sorted(PROJ))
@pytest.mark.parametrize("m", [17, 128, 300])
def test_prefill_projection(gpu, name, m):
    n, k = PROJ[name]
    w = weight(n, k, seed=40 + m)
    x = activations(m, k, seed=400 + m)
    y = _gpu_linear(x, w)
    assert_parity(y, ref.linear(x, w), f"{name} prefill M={m}")


@pytest.mark.parametrize("m", [64, 257])
def test_prefill_gate_up_silu(gpu, m):
    n, k = 2 * G.intermediate_size, G.hidden_size
    w = weight(n, k, seed=50 + m)
    x = activations(m, k, seed=500 + m)
    y = _gpu_linear(x, w, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL)
    expect = ref.silu_mul(ref.linear(x, w), G.intermediate_size)
    assert_parity(y, expect, f"gate_up+silu prefill M={m}")


def _every_bf16_gate(rows: int, cols: int) -> torch.Tensor:
    """[rows, cols] bf16 holding each of the 65536 bit patterns once, the
    non-finite ones (exponent 0xFF) replaced by 0."""
    pat = np.arange(rows * cols, dtype=np.uint32).astype(np.uint16)
    pat[(pat & 0x7F80) == 0x7F80] = 0
    return torch.from_numpy(pat.reshape(rows, cols).view(np.int16)).view(torch.bfloat16)


def _assert_silu_elementwise(got: torch.Tensor, expect: torch.Tensor, what: str) -> None:
    """Within one bf16 ulp everywhere, identical in at least 99.9 % of the
    elements: the kernel's float32 SiLU differs from the oracle's by far less
    than the bf16 half-ulp, so the roundings part only next to a boundary."""
    g = got.double().numpy()
    e = expect.double().numpy()
    ulp = brute.bf16_ulp(np.maximum(np.abs(g), np.abs(e)))
    bad = np.abs(g - e) > ulp
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off by more than one ulp, first {np.argwhere(bad)[:4]}"
    same = float(np.mean(g == e))
    assert same >= 0.999, f"{what}: only {same:.5f} identical"


def test_prefill_silu_every_bf16_gate(gpu):
    """One-hot activations make gate and up exact weight entries, so the
    SiLU*up epilogue of the prefill kernel meets every finite bf16 gate value
    (M = 2048 tokens cycling over K = 128 columns of 512 gate rows)."""
    inter, k, m = 512, 128, 2048
    gen = torch.Generator(device="cpu").manual_seed(70)
    up = (torch.rand((inter, k), generator=gen) * 2 - 1).to(torch.bfloat16)
    w = torch.cat((_every_bf16_gate(inter, k), up))
    x = torch.eye(k, dtype=torch.bfloat16).repeat(m // k, 1)
    y = _gpu_linear(x, w, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL)
    # gate_up[t] = w[:, t % k] exactly (the CPU bf16 matmul would flush the
    # subnormal entries, which the MFMA keeps).
    gate_up = w.t().repeat(m // k, 1)
    _assert_silu_elementwise(y, ref.silu_mul(gate_up, inter), "prefill SiLU over every bf16 gate")


def test_decode_silu_every_bf16_gate(gpu):
    """The decode kernels' SiLU*up epilogue over every finite bf16 gate value:
    M = 8 one-hot tokens read columns 0..7 of 8192 gate rows."""
    inter, k, m = 8192, G.hidden_size, 8
    gen = torch.Generator(device="cpu").manual_seed(71)
    w = torch.zeros((2 * inter, k), dtype=torch.bfloat16)
    w[:inter, :m] = _every_bf16_gate(inter, m)
    w[inter:, :m] = (torch.rand((inter, m), generator=gen) * 2 - 1).to(torch.bfloat16)
    x = torch.eye(m, k, dtype=torch.bfloat16)
    y = _gpu_linear(x, w, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL)
    _assert_silu_elementwise(y, ref.silu_mul(w[:, :m].t().contiguous(), inter), "decode SiLU over every bf16 gate")


def _linear_plan(m: int, n: int, k: int) -> list[int]:
    """The prefill GEMM's plan with the auto workspace: [block rows, blocks,
    split blocks, chunks per split block]."""
    lib = _lib.load()
    plan = (ctypes.c_int * 4)()
    ws = lib.lsk_workspace_bytes(_lib.OP_LINEAR, m, n, k)
    assert lib.lsk_linear_plan(m, n, k, ws, plan) == _lib.OK
    return list(plan)


# (M, N, K, epilogue) and the plan each gives on a 256-CU MI355X: the split
# counts S = 2, 3, 4, 8 and 16 of the last round, 128- and 256-row blocks,
# each epilogue through the split combine.
SPLIT_CASES = {
    "s2": (512, 6144, 2560, _lib.EPI_NONE, [128, 96, 96, 2]),
    "s3": (1024, 2560, 2560, _lib.EPI_NONE, [128, 80, 80, 3]),
    "s3_silu": (1024, 2560, 2560, _lib.EPI_SILU_MUL, [128, 80, 80, 3]),
    "s3_256": (2048, 2560, 4096, _lib.EPI_RESIDUAL_ADD, [256, 80, 80, 3]),
    "s4": (300, 2560, 9728, _lib.EPI_NONE, [128, 40, 40, 4]),
    "s8": (200, 2560, 4096, _lib.EPI_RESIDUAL_ADD, [128, 20, 20, 8]),
    "s16": (200, 1024, 8192, _lib.EPI_NONE, [128, 8, 8, 16]),
}


@pytest.mark.parametrize("case", sorted(SPLIT_CASES))
def test_prefill_every_split_count(gpu, case):
    """Every split count of the partial last round against the oracle, twice
    (bitwise equal), with the workspace left zeroed and its error word clear."""
    m, n, k, epi, plan = SPLIT_CASES[case]
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert _linear_plan(m, n, k) == plan
    layout = _lib.LAYOUT_MFMA16X32_GATEUP if epi == _lib.EPI_SILU_MUL else _lib.LAYOUT_MFMA16X32
    w = weight(n, k, seed=80 + k % 97)
    x = activations(m, k, seed=800 + m)
    r = activations(m, n, seed=801 + m) if epi == _lib.EPI_RESIDUAL_ADD else None
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(w.to(dev), layout)
    ws = kernels.prefill_workspace(dev, m, n, k)
    xd, rd = x.to(dev), (r.to(dev) if r is not None else None)
    y1 = kernels.linear(xd, pw, epilogue=epi, residual=rd, workspace=ws)
    y2 = kernels.linear(xd, pw, epilogue=epi, residual=rd, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert kernels.linear_error(ws) == 0
    assert int(ws.view(torch.int32)[64:2048].abs().sum()) == 0  # arrival/departure words zero again
    yl = ref.linear(x, w)
    expect = ref.silu_mul(yl, n // 2) if epi == _lib.EPI_SILU_MUL else (r + yl if r is not None else yl)
    assert_parity(y1.cpu(), expect, f"split-K {case} M={m} N={n} K={k}")


@pytest.mark.parametrize("m", [1500, 2047])
@pytest.mark.parametrize("proj", ["qkv", "down_residual"])
def test_prefill_ragged_token_count(gpu, m, proj):
    """Token counts that leave the last 256-token block part-full (220 and
    255 rows), in full against the oracle: QKV on 192-row blocks in one round,
    down + residual on split blocks (2 chunks at 1500 tokens, 3 at 2047)."""
    if proj == "qkv":
        n, k, epi = G.qkv_dim, G.hidden_size, _lib.EPI_NONE
    else:
        n, k, epi = G.hidden_size, G.intermediate_size, _lib.EPI_RESIDUAL_ADD
    w = weight(n, k, seed=90 + m % 7)
    x = activations(m, k, seed=900 + m)
    r = activations(m, n, seed=901 + m) if epi == _lib.EPI_RESIDUAL_ADD else None
    y = _gpu_linear(x, w, epilogue=epi, residual=r)
    expect = ref.linear(x, w) if r is None else r + ref.linear(x, w)
    assert_parity(y, expect, f"{proj} prefill M={m}")


def test_prefill_residual(gpu):
    m, n, k = 200, G.hidden_size, G.q_dim
    w = weight(n, k, seed=60)
    x = activations(m, k, seed=600)
    r = activations(m, n, seed=601)
    y = _gpu_linear(x, w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=r)
    assert_parity(y, r + ref.linear(x, w), "o_proj+residual prefill")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16])
def test_lm_head_argmax_fp32(gpu, m):
    """Tied lm_head E[151936, 2560]: GPU argmax == CPU fp32-score argmax, for
    every M the head serves up to its limit of 16 rows."""
    e = weight(G.vocab_size, G.hidden_size, seed=70)
    h = activations(m, G.hidden_size, seed=700 + m)
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(e.to(dev))
    logits = torch.empty((m, G.vocab_size), device=dev, dtype=torch.float32)
    idx = kernels.lm_head_argmax(h.to(dev), pw, logits_out=logits).cpu()
    scores = ref.logits_scores_fp32(h, e)
    assert_greedy_rows(idx, scores, logits.cpu(), f"lm_head fp32 M={m}")
    assert_parity(logits.cpu(), scores, "lm_head fp32 logits")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
def test_rmsnorm_lm_head_argmax(gpu, m):
    """The final RMSNorm inside the lm_head kernel: argmax of
    rms_norm(h) . E^T against the oracle's norm and fp32 scores (a near tie
    may go either way), logits at the parity bar."""
    e = weight(G.vocab_size, G.hidden_size, seed=71)
    h = activations(m, G.hidden_size, seed=710 + m) * 3
    gen = torch.Generator().manual_seed(720 + m)
    nw = (1 + 0.2 * torch.randn(G.hidden_size, generator=gen)).to(torch.bfloat16)
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(e.to(dev))
    logits = torch.empty((m, G.vocab_size), device=dev, dtype=torch.float32)
    idx = kernels.lm_head_argmax(h.to(dev), pw, logits_out=logits, norm_weight=nw.to(dev), eps=1e-6).cpu()
    scores = ref.logits_scores_fp32(ref.rmsnorm(h, nw, 1e-6), e)
    assert_greedy_rows(idx, scores, logits.cpu(), f"rmsnorm lm_head M={m}")
    assert_parity(logits.cpu(), scores, f"rmsnorm lm_head M={m} logits")


def test_lm_head_argmax_bf16_mode(gpu):
    """bf16-rounded logits: matches torch.mv(W, h).argmax (first maximum)."""
    e = weight(G.vocab_size, G.hidden_size, seed=71)
    h = activations(1, G.hidden_size, seed=710)
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(e.to(dev))
    logits = torch.empty((1, G.vocab_size), device=dev, dtype=torch.float32)
    idx = kernels.lm_head_argmax(h.to(dev), pw, logits_mode=_lib.LOGITS_BF16, logits_out=logits).cpu()
    expect = ref.bf16_logits_argmax(h, e)
    bf = torch.mv(e, h.view(-1)).float()
    top = torch.topk(bf, 2).values
    print(f"idx={idx.tolist()} expect={expect.tolist()} top2={top.tolist()}")
    assert torch.equal(idx, expect)


def test_lm_head_workspace_left_zero_across_calls(gpu):
    """One workspace through calls of M = 16, 1, 8, 3, 16 in a row, eager and
    replayed from a graph: each call's argmax meets the oracle, and after each
    call the whole workspace (status word and every partial) is zero again,
    which is the state the next call starts from."""
    e = weight(G.vocab_size, G.hidden_size, seed=73)
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(e.to(dev))
    ws = kernels.LmHeadWorkspace(16, G.vocab_size, G.hidden_size, dev)
    for i, m in enumerate((16, 1, 8, 3, 16)):
        h = activations(m, G.hidden_size, seed=730 + i)
        logits = torch.empty((m, G.vocab_size), device=dev, dtype=torch.float32)
        idx = kernels.lm_head_argmax(h.to(dev), pw, logits_out=logits, workspace=ws).cpu()
        assert_greedy_rows(idx, ref.logits_scores_fp32(h, e), logits.cpu(), f"call {i} M={m}")
        assert int(torch.count_nonzero(ws.buffer)) == 0, f"workspace not zero after call {i} (M={m})"
    # replays of one captured call with new inputs copied in between
    m = 4
    h_dev = torch.empty((m, G.hidden_size), device=dev, dtype=torch.bfloat16)
    out = torch.empty((m,), device=dev, dtype=torch.long)
    logits = torch.empty((m, G.vocab_size), device=dev, dtype=torch.float32)
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        kernels.lm_head_argmax(h_dev, pw, workspace=ws, out=out, logits_out=logits)
    for i in range(3):
        h = activations(m, G.hidden_size, seed=740 + i)
        h_dev.copy_(h.to(dev))
        out.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        assert_greedy_rows(out.cpu(), ref.logits_scores_fp32(h, e), logits.cpu(), f"replay {i}")
        assert int(torch.count_nonzero(ws.buffer)) == 0, f"workspace not zero after replay {i}"
    assert ws.give_ups() == 0


def test_lm_head_ties_pick_lowest_index(gpu):
    """Two identical maximal vocab rows: the lower index wins, in both modes."""
    v, k = 4096, 256
    e = weight(v, k, seed=72)
    h = activations(1, k, seed=720)
    hot = torch.sign(h.float()).to(torch.bfloat16) * 0.5
    e[1234] = hot
    e[3001] = hot
    e[17] = -hot
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(e.to(dev))
    for mode in (_lib.LOGITS_FP32, _lib.LOGITS_BF16):
        idx = kernels.lm_head_argmax(h.to(dev), pw, logits_mode=mode).cpu()
        assert idx.tolist() == [1234]


@pytest.mark.parametrize("v", [16 * 101, 16 * 512, 16 * 513, 16 * 514, 16 * 1187, 16 * 2048])
def test_lm_head_tail_workgroups(gpu, v):
    """The scoring grid takes two 16-row vocab blocks per workgroup, then a
    tail of 512 one-block workgroups (513 when the count past 512 is odd; all
    one-block up to 512 blocks): at 101, 512, 513, 514, 1187 (the vocab shard
    of 8-way tensor parallelism) and 2048 blocks every row's fp32 score equals
    the CPU's (each row scored once, in its own place), and a maximum planted
    in the first and last pair, the first and last tail block and the last
    row is found."""
    k = 256
    dev = torch.device("cuda:0")
    h = activations(1, k, seed=740)
    hot = torch.sign(h.float()).to(torch.bfloat16) * 0.5
    nb = v // 16
    pairs = (nb - 512) // 2 if nb > 512 else 0
    tail0 = 32 * pairs  # first vocab row of the tail
    rows = sorted({0, 31, max(tail0 - 1, 0), tail0, tail0 + 16, v - 17, v - 1})
    for row in rows:
        e = weight(v, k, seed=741)
        e[row] = hot
        pw = PackedWeight.from_rowmajor(e.to(dev))
        logits = torch.empty((1, v), device=dev, dtype=torch.float32)
        idx = kernels.lm_head_argmax(h.to(dev), pw, logits_out=logits).cpu()
        assert idx.tolist() == [row], (v, row, idx.tolist())
        if row == rows[0]:
            expect = ref.logits_scores_fp32(h, e)
            got = logits.cpu()
            assert_parity(got, expect, f"lm_head logits V={v}")
            # elementwise: fp32 sums of 256 products in another order, far below one misplaced row
            err = (got - expect).abs().max()
            assert float(err) <= 1e-4 * float(expect.abs().max()) + 1e-5, (v, float(err))


def test_device_pack_matches_host_packer(gpu):
    """torch-permute packing on the GPU equals the C host packer, byte for byte."""
    w = weight(2 * 256, 512, seed=80)
    lib = _lib.load()
    for layout in (_lib.LAYOUT_MFMA16X32, _lib.LAYOUT_MFMA16X32_GATEUP):
        dev_packed = PackedWeight.from_rowmajor(w.to("cuda:0"), layout).data.cpu()
        host = torch.empty_like(w).view(-1)
        status = lib.lsk_pack_bf16(w.data_ptr(), w.shape[0], w.shape[1], layout, host.data_ptr())
        _lib.check(status, "pack")
        assert torch.equal(dev_packed.view(torch.int16), host.view(torch.int16))


def test_strided_activations(gpu):
    """x rows at a stride larger than K (a column slice of a wider buffer)."""
    n, k, m = 2560, 4096, 4
    w = weight(n, k, seed=90)
    wide = activations(m, k + 64, seed=900)
    x = wide[:, 32 : 32 + k]
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(w.to(dev))
    y = kernels.linear(wide.to(dev)[:, 32 : 32 + k], pw).cpu()
    assert_parity(y, ref.linear(x, w), "strided x")


@pytest.mark.parametrize("m", [5, 300])
def test_largest_activation_stride(gpu, m):
    """x rows at the largest stride the ABI accepts, 2^22 - 8 elements: a
    256-row block of them spans 2^31 - 4096 bytes, the prefill kernel's
    32-bit activation descriptor at its limit (M = 300: two token blocks,
    the second part-full; M = 5: the decode kernel).  One step wider, the
    ABI refuses the stride and the wrapper reads the rows through a copy."""
    n, k = 2560, 4096
    ld = _lib.MAX_ACTIVATION_STRIDE
    assert ld == (1 << 22) - 8
    w = weight(n, k, seed=91)
    x = activations(m, k, seed=910 + m)
    expect = ref.linear(x, w)
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(w.to(dev))
    for stride in (ld, ld + 8):
        wide = torch.empty((m, stride), device=dev, dtype=torch.bfloat16)
        wide[:, :k] = x.to(dev)
        y = kernels.linear(wide[:, :k], pw)
        if stride > ld:
            status = _lib.load().lsk_linear_bf16(pw.data.data_ptr(), pw.layout, n, k, wide.data_ptr(), m, stride,
                                                 y.data_ptr(), n, 0, None, 0, None, 0, None)
            assert status == _lib.ERR_INVALID, _lib.last_error()
        torch.cuda.synchronize()
        del wide
        assert_parity(y.cpu(), expect, f"x at stride {stride}, M={m}")


def test_zero_rows_give_empty_results(gpu):
    """No rows in, no rows out, nothing launched: the empty results F.linear
    and torch.argmax give for a [0, K] input."""
    dev = torch.device("cuda:0")
    n, k = 2560, 4096
    pw = PackedWeight.from_rowmajor(weight(n, k, seed=92).to(dev))
    x = torch.empty((0, k), device=dev, dtype=torch.bfloat16)
    y = kernels.linear(x, pw)
    assert y.shape == (0, n) and y.dtype == torch.bfloat16
    y = kernels.linear(x, pw, epilogue=_lib.EPI_RESIDUAL_ADD, residual=torch.empty((0, n), device=dev,
                                                                                   dtype=torch.bfloat16))
    assert y.shape == (0, n)
    y = kernels.rmsnorm_linear(x, torch.ones(k, device=dev, dtype=torch.bfloat16), 1e-6, pw)
    assert y.shape == (0, n)
    head = PackedWeight.from_rowmajor(weight(64, k, seed=93).to(dev))
    idx = kernels.lm_head_argmax(x, head)
    assert idx.shape == (0,) and idx.dtype == torch.long
    torch.cuda.synchronize()


def test_rejects_bad_shapes_before_launch(gpu):
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(weight(64, 64, seed=1).to(dev))
    with pytest.raises(ValueError):
        kernels.linear(activations(1, 32, seed=2).to(dev), pw)
    with pytest.raises(ValueError):
        kernels.linear(activations(1, 64, seed=2).to(dev), pw, epilogue=_lib.EPI_SILU_MUL)
    with pytest.raises(ValueError):
        kernels.lm_head_argmax(activations(17, 64, seed=2).to(dev), pw)


@pytest.mark.parametrize("name", sorted(PROJ) + ["gate_up_proj"])
def test_prefill_m2048_full_shapes(gpu, name):
    """M=2048 at every projection shape (the large-tile MFMA kernel), against the oracle."""
    m = 2048
    if name == "gate_up_proj":
        n, k = 2 * G.intermediate_size, G.hidden_size
        w = weight(n, k, seed=81)
        x = activations(m, k, seed=810)
        y = _gpu_linear(x, w, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL)
        expect = ref.silu_mul(ref.linear(x, w), G.intermediate_size)
    else:
        n, k = PROJ[name]
        w = weight(n, k, seed=82)
        x = activations(m, k, seed=820)
        y = _gpu_linear(x, w)
        expect = ref.linear(x, w)
    assert_parity(y, expect, f"{name} prefill M=2048")


@pytest.mark.parametrize("name", sorted(PROJ) + ["gate_up_proj"])
@pytest.mark.parametrize("m", [300, 2048])
def test_prefill_one_block_per_workgroup(gpu, name, m):
    """The data-parallel prefill kernel (no workspace) at every projection shape."""
    if name == "gate_up_proj":
        n, k = 2 * G.intermediate_size, G.hidden_size
        w = weight(n, k, seed=83)
        x = activations(m, k, seed=830)
        y = _gpu_linear(x, w, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL, workspace=None)
        expect = ref.silu_mul(ref.linear(x, w), G.intermediate_size)
    else:
        n, k = PROJ[name]
        w = weight(n, k, seed=84)
        x = activations(m, k, seed=840)
        y = _gpu_linear(x, w, workspace=None)
        expect = ref.linear(x, w)
    assert_parity(y, expect, f"{name} data-parallel M={m}")


def test_split_k_workspace_contract(gpu):
    """Split-K: residual epilogue through split blocks, flags left zero,
    error word clear, and two calls on one workspace give identical bits."""
    dev = torch.device("cuda:0")
    m, n, k = 2048, G.hidden_size, G.intermediate_size  # 80 blocks, each split in 3 K chunks
    w = weight(n, k, seed=85)
    x = activations(m, k, seed=850)
    r = activations(m, n, seed=851)
    pw = PackedWeight.from_rowmajor(w.to(dev))
    nbytes = _lib.load().lsk_workspace_bytes(_lib.OP_LINEAR, m, n, k)
    assert nbytes > 0
    ws = torch.zeros(nbytes, device=dev, dtype=torch.uint8)
    y1 = kernels.linear(x.to(dev), pw, epilogue=_lib.EPI_RESIDUAL_ADD, residual=r.to(dev), workspace=ws)
    y2 = kernels.linear(x.to(dev), pw, epilogue=_lib.EPI_RESIDUAL_ADD, residual=r.to(dev), workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    assert_parity(y1.cpu(), r + ref.linear(x, w), "down+residual split-K M=2048")
    flags = ws[256:8192].view(torch.int32)
    assert int(flags.abs().sum().item()) == 0
    assert kernels.linear_error(ws) == 0
    with pytest.raises(ValueError):
        kernels.linear(x.to(dev), pw, workspace=ws[: nbytes // 2])
    # The plan refuses the workspace the launch refuses, and plans the split
    # round only with a whole one.
    lib = _lib.load()
    plan = (ctypes.c_int * 4)(9, 9, 9, 9)
    assert lib.lsk_linear_plan(m, n, k, nbytes - 1, plan) == _lib.ERR_WORKSPACE
    assert lib.lsk_linear_plan(m, n, k, nbytes, plan) == _lib.OK and plan[2] > 0 and plan[3] > 1
    assert lib.lsk_linear_plan(m, n, k, 0, plan) == _lib.OK and plan[2] == 0 and plan[3] == 1


def _prefill_case(name, m, seed):
    if name == "gate_up_proj":
        n, k = 2 * G.intermediate_size, G.hidden_size
        return weight(n, k, seed=seed), activations(m, k, seed=seed + 1), _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL
    n, k = PROJ[name]
    return weight(n, k, seed=seed), activations(m, k, seed=seed + 1), _lib.LAYOUT_MFMA16X32, _lib.EPI_NONE


def _oracle(x, w, epilogue):
    y = ref.linear(x, w)
    return ref.silu_mul(y, G.intermediate_size) if epilogue == _lib.EPI_SILU_MUL else y


@pytest.mark.parametrize("name", sorted(PROJ) + ["gate_up_proj"])
def test_prefill_m512_full_shapes(gpu, name):
    """M=512 (the smallest prefill bucket of the benchmark) at every projection shape."""
    w, x, layout, epi = _prefill_case(name, 512, seed=91)
    y = _gpu_linear(x, w, layout, epi)
    assert_parity(y, _oracle(x, w, epi), f"{name} prefill M=512")


@pytest.mark.parametrize("name", sorted(PROJ) + ["gate_up_proj"])
def test_prefill_m8192_sampled_rows(gpu, name):
    """M=8192 at every projection shape: the whole GEMM runs on the GPU; output
    rows depend only on their own activation row, so the oracle checks a
    sample of rows (block edges, the last row, and random rows)."""
    m = 8192
    w, x, layout, epi = _prefill_case(name, m, seed=93)
    y = _gpu_linear(x, w, layout, epi)
    gen = torch.Generator().manual_seed(94)
    rows = torch.cat([torch.tensor([0, 1, 255, 256, 4095, 4096, 8190, 8191]),
                      torch.randint(0, m, (56,), generator=gen)]).unique()
    assert_parity(y[rows], _oracle(x[rows], w, epi), f"{name} prefill M=8192 (rows sampled)")


def _random_shapes(count: int, seed: int) -> list[tuple[int, int, int, int]]:
    """(M, N, K, epilogue) drawn over every routing class of lsk_linear_bf16:
    decode (M <= 16), the skinny kernel (M = 17..128), decode slices (N or K
    off the block GEMM's grid, M > 128), the 128-row GEMM, and the block GEMM
    with and without a split last round."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        cls = i % 4
        m = int(rng.integers(1, 17)) if cls == 0 else int(rng.integers(17, 3000))
        if cls == 1:  # off the block grid: N a multiple of 32 only, or K of 32 only
            n = 32 * int(rng.integers(1, 160))
            k = 32 * int(rng.integers(2, 200))
        else:
            n = 128 * int(rng.integers(1, 80))
            k = 128 * int(rng.integers(1, 96))
        epi = int(rng.integers(0, 3))
        out.append((m, n, k, epi))
    return out


@pytest.mark.parametrize("m,n,k,epi", _random_shapes(24, 2026))
def test_linear_random_shapes(gpu, m, n, k, epi):
    """Seeded random shapes against the oracle on sampled rows (the first,
    last, block-edge and random rows; every row when M <= 64), with the
    auto workspace; the plan the block GEMM takes is printed with the case."""
    layout = _lib.LAYOUT_MFMA16X32_GATEUP if epi == _lib.EPI_SILU_MUL else _lib.LAYOUT_MFMA16X32
    w = weight(n, k, seed=m + n + k)
    x = activations(m, k, seed=m * 7 + k)
    r = activations(m, n, seed=m * 11 + n) if epi == _lib.EPI_RESIDUAL_ADD else None
    print(f"case M={m} N={n} K={k} epi={epi} plan={_linear_plan(m, n, k)}", flush=True)
    y = _gpu_linear(x, w, layout, epi, residual=r)
    if m <= 64:
        rows = torch.arange(m)
    else:
        gen = torch.Generator().manual_seed(m)
        edges = torch.tensor([0, 1, 127, 128, 255, 256, m - 2, m - 1])
        rows = torch.cat([edges[edges < m], torch.randint(0, m, (40,), generator=gen)]).unique()
    yl = ref.linear(x[rows], w)
    if epi == _lib.EPI_SILU_MUL:
        expect = ref.silu_mul(yl, n // 2)
    elif epi == _lib.EPI_RESIDUAL_ADD:
        expect = r[rows] + yl
    else:
        expect = yl
    assert_parity(y[rows], expect, f"M={m} N={n} K={k} epi={epi}")


def test_lm_head_argmax_follows_torch_on_nan_and_inf(gpu):
    """Scores that are NaN, +inf or all -inf: the kernel's token is what
    torch.argmax returns on the same scores (the first NaN wins, +inf beats
    any finite score, an all -inf row gives index 0), in both logit modes --
    never an index outside the vocab."""
    v, k = 4096, 256
    dev = torch.device("cuda:0")
    h = activations(1, k, seed=730).abs() + 0.5  # positive, so a row's sign fixes its score's sign
    cases = {}
    e = weight(v, k, seed=731)
    e[3000] = float("nan")
    e[1500] = float("nan")
    e[200] = float("inf")
    cases["nan rows"] = e
    e = weight(v, k, seed=732)
    e[2222] = float("inf")
    e[3333] = float("inf")
    cases["inf rows"] = e
    cases["all -inf"] = torch.full((v, k), float("-inf"), dtype=torch.bfloat16)
    for what, e in cases.items():
        expect = int(ref.logits_scores_fp32(h, e).argmax(dim=-1))
        pw = PackedWeight.from_rowmajor(e.to(dev))
        for mode in (_lib.LOGITS_FP32, _lib.LOGITS_BF16):
            idx = kernels.lm_head_argmax(h.to(dev), pw, logits_mode=mode).cpu()
            assert idx.tolist() == [expect], (what, mode, idx.tolist(), expect)
    assert [int(ref.logits_scores_fp32(h, e).argmax(dim=-1)) for e in cases.values()] == [1500, 2222, 0]


def test_split_k_lost_wait_is_reported_and_poisons(gpu):
    """A split-K workgroup whose bounded wait gives up (forced from the host
    with a wait limit of 0 polls: every chunk that is not the last to arrive
    stops waiting at once) sets the workspace's error word and writes NaN to
    its share of the block instead of a partial sum; tiles of chunks that did
    complete match the oracle, and the flags are left clear.  With the limit
    restored the next call is whole again."""
    dev = torch.device("cuda:0")
    m, n, k = 2048, G.hidden_size, G.intermediate_size  # 80 blocks, each split in 3 K chunks
    w = weight(n, k, seed=86)
    x = activations(m, k, seed=860)
    pw = PackedWeight.from_rowmajor(w.to(dev))
    ws = torch.zeros(_lib.load().lsk_workspace_bytes(_lib.OP_LINEAR, m, n, k), device=dev, dtype=torch.uint8)
    expect = ref.linear(x, w)
    try:
        kernels.set_linear_wait_limit(0)
        y = kernels.linear(x.to(dev), pw, workspace=ws)
        torch.cuda.synchronize()
    finally:
        kernels.set_linear_wait_limit(kernels.LINEAR_WAIT_LIMIT_DEFAULT)
    assert kernels.linear_error(ws) != 0
    y = y.cpu()
    bad = torch.isnan(y.float())
    print(f"NaN outputs after forced give-ups: {int(bad.sum())} of {y.numel()}")
    assert bad.any()
    assert_parity(y[~bad], expect[~bad], "split-K tiles that completed")
    assert int(ws[256:8192].view(torch.int32).abs().sum().item()) == 0
    y2 = kernels.linear(x.to(dev), pw, workspace=ws)
    torch.cuda.synchronize()
    assert kernels.linear_error(ws) == 0
    assert_parity(y2.cpu(), expect, "split-K after the limit is restored")


@pytest.mark.parametrize("m", [1024, 2048])
def test_prefill_192_row_blocks_with_epilogues(gpu, m):
    """Shapes whose weight rows split into 192-row blocks (N % 192 == 0 with
    fewer block-rows per CU than 256-row blocks): the residual epilogue on a
    QKV-shaped weight, and SiLU*up on a fused gate_up of 2 x 1536 rows, with
    the split-K workspace (M = 1024: 128 blocks split in two) and without."""
    n, k = G.qkv_dim, G.hidden_size
    w = weight(n, k, seed=95)
    x = activations(m, k, seed=950)
    r = activations(m, n, seed=951)
    for ws in ("auto", None):
        y = _gpu_linear(x, w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=r, workspace=ws)
        assert_parity(y, r + ref.linear(x, w), f"qkv-shaped + residual M={m} workspace={ws}")
    inter = 1536
    wg = weight(2 * inter, k, seed=96)
    y = _gpu_linear(x, wg, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL)
    assert_parity(y, ref.silu_mul(ref.linear(x, wg), inter), f"gate_up 2x{inter} + silu M={m}")


@pytest.mark.parametrize("case", ["plain_2x8", "residual_2x8", "residual_3x4", "silu_3x4", "silu_2x8"])
@pytest.mark.parametrize("narrow", [False, True])
def test_prefill_whole_block_epilogue_strides(gpu, case, narrow):
    """The whole-block prefill epilogue (no workspace: one workgroup per
    output block) through the C ABI, at contiguous 16-byte-aligned output and
    residual rows and at the narrowest the ABI accepts: y 8-byte aligned with
    ldy % 8 == 4, the residual 2-byte aligned with ldr % 8 == 2.  Elements
    between the rows stay as they were.  M = 300 leaves a partial token block;
    the 2x8 cases run 256-row weight blocks, the 3x4 cases 192-row ones."""
    dev = torch.device("cuda:0")
    m, k = 300, G.hidden_size
    if case.startswith("silu"):
        inter = 1536 if case.endswith("3x4") else 2048
        n, layout, epi = 2 * inter, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL
        n_out = inter
    else:
        n = G.qkv_dim if case.endswith("3x4") else G.hidden_size
        layout, n_out = _lib.LAYOUT_MFMA16X32, n
        epi = _lib.EPI_RESIDUAL_ADD if case.startswith("residual") else _lib.EPI_NONE
    w = weight(n, k, seed=97)
    x = activations(m, k, seed=970)
    pw = PackedWeight.from_rowmajor(w.to(dev), layout)
    xd = x.to(dev)
    ldy, y_off = (n_out + 4, 4) if narrow else (n_out, 0)
    y_buf = torch.full((m * ldy + 8,), -7.0, device=dev, dtype=torch.bfloat16)
    res_ptr, ldr, r = None, 0, None
    if epi == _lib.EPI_RESIDUAL_ADD:
        r = activations(m, n, seed=971)
        ldr, r_off = (n + 2, 1) if narrow else (n, 0)
        r_buf = torch.zeros((m * ldr + 8,), device=dev, dtype=torch.bfloat16)
        r_buf[r_off:r_off + m * ldr].view(m, ldr)[:, :n] = r.to(dev)
        res_ptr = r_buf.data_ptr() + 2 * r_off
    lib = _lib.load()
    status = lib.lsk_linear_bf16(pw.data.data_ptr(), layout, n, k, xd.data_ptr(), m, k,
                                 y_buf.data_ptr() + 2 * y_off, ldy, epi, res_ptr, ldr, None, 0,
                                 torch.cuda.current_stream().cuda_stream)
    _lib.check(status, "lsk_linear_bf16")
    torch.cuda.synchronize()
    rows = y_buf[y_off:y_off + m * ldy].view(m, ldy).cpu()
    y = rows[:, :n_out]
    if epi == _lib.EPI_SILU_MUL:
        expect = ref.silu_mul(ref.linear(x, w), n_out)
    elif epi == _lib.EPI_RESIDUAL_ADD:
        expect = r + ref.linear(x, w)
    else:
        expect = ref.linear(x, w)
    assert_parity(y, expect, f"{case} narrow={narrow}")
    untouched = torch.cat([y_buf[:y_off].cpu(), rows[:, n_out:].reshape(-1), y_buf[y_off + m * ldy:].cpu()])
    assert bool((untouched == -7.0).all()), "the epilogue wrote outside the output rows"


@pytest.mark.parametrize("m", [1, 3, 12])
@pytest.mark.parametrize("case", ["o_residual", "down_residual", "qkv", "gate_up_silu"])
def test_decode_narrowest_strides(gpu, case, m):
    """The decode kernels through the C ABI at the narrowest rows the ABI
    accepts: x 16-byte aligned at ldx = K + 8, y 8-byte aligned with
    ldy % 8 == 4, the residual 2-byte aligned with ldr % 8 == 2.  Elements
    between the rows stay as they were."""
    dev = torch.device("cuda:0")
    if case == "gate_up_silu":
        n, k, layout, epi = 2 * G.intermediate_size, G.hidden_size, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL
        n_out = G.intermediate_size
    else:
        n, k = {"o_residual": PROJ["o_proj"], "down_residual": PROJ["down_proj"], "qkv": PROJ["qkv_proj"]}[case]
        layout, n_out = _lib.LAYOUT_MFMA16X32, n
        epi = _lib.EPI_RESIDUAL_ADD if case.endswith("residual") else _lib.EPI_NONE
    w = weight(n, k, seed=98 + m)
    x = activations(m, k, seed=980 + m)
    pw = PackedWeight.from_rowmajor(w.to(dev), layout)
    ldx = k + 8
    x_buf = torch.zeros((m, ldx), device=dev, dtype=torch.bfloat16)
    x_buf[:, :k] = x.to(dev)
    ldy, y_off = n_out + 4, 4
    y_buf = torch.full((m * ldy + 8,), -7.0, device=dev, dtype=torch.bfloat16)
    res_ptr, ldr, r = None, 0, None
    if epi == _lib.EPI_RESIDUAL_ADD:
        r = activations(m, n, seed=981 + m)
        ldr, r_off = n + 2, 1
        r_buf = torch.zeros((m * ldr + 8,), device=dev, dtype=torch.bfloat16)
        r_buf[r_off:r_off + m * ldr].view(m, ldr)[:, :n] = r.to(dev)
        res_ptr = r_buf.data_ptr() + 2 * r_off
    status = _lib.load().lsk_linear_bf16(pw.data.data_ptr(), layout, n, k, x_buf.data_ptr(), m, ldx,
                                         y_buf.data_ptr() + 2 * y_off, ldy, epi, res_ptr, ldr, None, 0,
                                         torch.cuda.current_stream().cuda_stream)
    _lib.check(status, "lsk_linear_bf16")
    torch.cuda.synchronize()
    rows = y_buf[y_off:y_off + m * ldy].view(m, ldy).cpu()
    y = rows[:, :n_out]
    if epi == _lib.EPI_SILU_MUL:
        expect = ref.silu_mul(ref.linear(x, w), n_out)
    elif epi == _lib.EPI_RESIDUAL_ADD:
        expect = r + ref.linear(x, w)
    else:
        expect = ref.linear(x, w)
    assert_parity(y, expect, f"decode {case} M={m} narrow rows")
    untouched = torch.cat([y_buf[:y_off].cpu(), rows[:, n_out:].reshape(-1), y_buf[y_off + m * ldy:].cpu()])
    assert bool((untouched == -7.0).all()), "the kernel wrote outside the output rows"


@pytest.mark.parametrize("m", [1, 3, 12])
def test_lm_head_strided_hidden_rows(gpu, m):
    """Hidden rows at a stride above K (a view into a wider buffer, read in
    place): the same indices and bit-identical fp32 logits as contiguous
    rows, with and without the fused final RMSNorm (M <= 8)."""
    dev = torch.device("cuda:0")
    e = weight(G.vocab_size, G.hidden_size, seed=72)
    h = activations(m, G.hidden_size, seed=720 + m).to(dev)
    pw = PackedWeight.from_rowmajor(e.to(dev))
    wide = torch.zeros((m, G.hidden_size + 64), device=dev, dtype=torch.bfloat16)
    wide[:, 32:32 + G.hidden_size] = h
    view = wide[:, 32:32 + G.hidden_size]
    assert view.stride(0) == G.hidden_size + 64 and view.data_ptr() % 16 == 0
    norms = [None] + ([torch.ones(G.hidden_size, device=dev, dtype=torch.bfloat16) * 1.5] if m <= 8 else [])
    for nw in norms:
        la = torch.empty((m, G.vocab_size), device=dev, dtype=torch.float32)
        lb = torch.empty_like(la)
        ia = kernels.lm_head_argmax(h, pw, logits_out=la, norm_weight=nw)
        ib = kernels.lm_head_argmax(view, pw, logits_out=lb, norm_weight=nw)
        torch.cuda.synchronize()
        assert torch.equal(ia, ib) and torch.equal(la.view(torch.int32), lb.view(torch.int32)), f"norm={nw is not None}"
