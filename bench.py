"""Benchmark of the MI355X BF16 projection path (one JSON line on stdout).

Headline workload (`value`): one decode step of the 36-layer Qwen3-4B-shaped
projection stack at M = 1 -- fused QKV [6144x2560], o_proj [2560x4096], fused
gate_up [19456x2560] with the SiLU(gate)*up epilogue and down_proj
[2560x9728] per layer, 36 distinct random N(0, 0.02) layers (7.27 GB, far
above the 256 MB MALL), fresh N(0, 1) activations per layer, RMSNorm /
attention between projections stubbed.  The step is captured as one HIP
graph and replayed; `value` is algorithmic HBM bytes per step (weights +
activations read + outputs written) / step time, in GB/s.

Also reported (under "detail"): the verify sweep M = 1, 2, 4, 8 over the same
stack, the step with the two RMSNorms of each layer (fused into the QKV and
gate_up kernels, or as separate F.rms_norm launches), a whole decode token with
attention over 320 and 4095 cached rows (every layer HIP), a greedy decode loop in
the reference's decode_64_256 shape (256 tokens after 64 cached rows, one graph
replay per token, per-step events), each projection kind's
per-launch time, the tied lm_head + argmax at M = 1..8, the prefill GEMMs
at M = 512, 2048, 8192 in TFLOP/s, and one GPU's share of 8-way tensor
parallelism at the real shard shapes (its M = 1 step, lm_head and prefill
layer; the all-reduces between shards are not run).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
import types
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

METRIC = "HBM GB/s + µs/step, Qwen3-4B BF16 decode linears M=1..8; prefill TFLOPS"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def settle(torch, graph, seconds: float = 0.3) -> None:
    """Replay `graph` untimed for `seconds` so the GPU leaves its idle clocks
    before the first timed run: the first configuration measured after the
    set-up (arena load, captures) ran 8% slow with only W = 5 warmup replays
    and not after 100.  W warmup replays and K timed replays still follow."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            graph.replay()
        torch.cuda.synchronize()


def time_graph(torch, graph, steps: int, warmup: int) -> float:
    """Milliseconds per replay: W untimed replays, then K replays bracketed by
    synchronize + HIP events on the replay stream."""
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def prefill_profile() -> dict:
    """The committed prefill counter profile (profiles/prefill_counters.json),
    or {} when absent."""
    path = REPO / "profiles" / "prefill_counters.json"
    return json.loads(path.read_text()) if path.exists() else {}


def profiled_mfma_util() -> float | None:
    """Time-weighted MfmaUtil of the four prefill projections at M = 2048 as
    the committed counter profile measured it, or None."""
    return prefill_profile().get("mfma_util_pct_m2048")


def measured_traffic(kernel_label: str):
    """HBM bytes per launch of the roofline kernel, as the committed counter
    profile measured it (profiles/hbm_traffic.json), or None."""
    path = REPO / "profiles" / "hbm_traffic.json"
    if not path.exists():
        return None
    kernels = json.loads(path.read_text()).get("kernels", {})
    for name, rec in kernels.items():
        if kernel_label.startswith(name.split("<")[0]) and name.split("<")[1].split(">")[0].replace(" ", "") in \
                kernel_label.replace(" ", ""):
            return rec["traffic_bytes"]
    return None


def cpu_model() -> str:
    """The host CPU's model name, CPU family and model numbers (/proc/cpuinfo;
    a virtual machine may report only a generic name, e.g. "AMD EPYC", whose
    family / model then tell the generation) and whether a hypervisor runs it,
    or the platform's description."""
    try:
        fields = {}
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, value = line.partition(":")
            key = key.strip()
            if key in ("model name", "cpu family", "model", "flags") and key not in fields:
                fields[key] = value.strip()
        if "model name" in fields:
            text = fields["model name"]
            if "cpu family" in fields and "model" in fields:
                text += f" (family {fields['cpu family']}, model {fields['model']})"
            if "hypervisor" in fields.get("flags", "").split():
                text += ", virtualised"
            return text
    except OSError:
        pass
    return platform.processor() or platform.machine()


CPU_LAYERS = 4  # 808 MB of distinct weights: larger than any host L3, so the sample streams DRAM


def cpu_baseline(g, seconds: float) -> dict:
    """The reference's CPU torch path (torch.mv in bf16 + F.silu*mul, via the
    oracle) on this host's cores, over a bounded sample: CPU_LAYERS distinct
    random Qwen3-4B layers cycled in order, M = 1, for about `seconds`."""
    import torch

    from oracle import projections as ref

    threads = torch.get_num_threads()
    gen = torch.Generator(device="cpu").manual_seed(0)
    layers = []
    for _ in range(CPU_LAYERS):
        layers.append({
            name: (torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16)
            for name, (n, k) in g.projections().items()
        })
    xs = {name: torch.randn(k, generator=gen).to(torch.bfloat16) for name, (n, k) in g.projections().items()}

    def one_layer(w):
        ref.mv(w["qkv_proj"], xs["qkv_proj"])
        ref.mv(w["o_proj"], xs["o_proj"])
        act = ref.silu_mul(ref.mv(w["gate_up_proj"], xs["gate_up_proj"]), g.intermediate_size)
        ref.mv(w["down_proj"], act)

    one_layer(layers[0])  # warm
    done = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        one_layer(layers[done % CPU_LAYERS])
        done += 1
    elapsed = time.perf_counter() - t0
    gbs = done * g.layer_bytes(1) / elapsed / 1e9
    return {
        "value": round(gbs, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{done} Qwen3-4B decode layers at M=1 (torch.mv bf16 qkv/o/gate_up/down + F.silu*mul, "
                   f"{CPU_LAYERS} distinct random layers = {CPU_LAYERS * g.layer_bytes(1) / 1e6:.0f} MB cycled) in "
                   f"{elapsed:.1f} s; {elapsed / done * 1e6:.0f} us/layer; cpu={cpu_model()}, "
                   f"os.cpu_count={os.cpu_count()}, torch threads={threads}"),
    }


def cpu_o_proj_gemv(seconds: float) -> dict:
    """The o_proj GEMV x[1,4096] . W[2560,4096]^T alone on the CPU torch
    path (torch.mv in bf16, qwen_explicit.py:913 via the oracle), W ~
    N(0,0.02), x ~ N(0,1), seeded, timed for about `seconds` on this host's
    cores.  W is 21 MB, so on a host with a large L3 the repeated calls may
    read it from cache; that is the workload as stated."""
    import torch

    from oracle import projections as ref

    gen = torch.Generator(device="cpu").manual_seed(0)
    w = (torch.randn(2560, 4096, generator=gen) * 0.02).to(torch.bfloat16)
    x = torch.randn(4096, generator=gen).to(torch.bfloat16)
    ref.mv(w, x)  # warm
    done = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        ref.mv(w, x)
        done += 1
    elapsed = time.perf_counter() - t0
    nbytes = 2560 * 4096 * 2 + 4096 * 2 + 2560 * 2
    us = elapsed / done * 1e6
    return {"us": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 2), "cores": torch.get_num_threads(),
            "bytes": nbytes, "calls": done,
            "sample": f"{done} calls of torch.mv(W[2560,4096] bf16, x[4096] bf16) in {elapsed:.1f} s, one W "
                      f"(21 MB) reused"}


# The reference's hot-kernel GEMM cases (src/leanstack/hot_kernels.py:79-166):
# key -> (M, N, K); its published per-kernel figures are for these shapes
# (docs/REMOTE_VALIDATION.md:193-197).
HOT_KERNEL_CASES = {
    "q_proj_prefill64": (64, 4096, 2560),
    "q_proj_prefill1024": (1024, 4096, 2560),
    "kv_proj_prefill64": (64, 1024, 2560),
    "o_proj_prefill64": (64, 2560, 4096),
    "gate_up_proj_prefill64": (64, 9728, 2560),
    "down_proj_prefill64": (64, 2560, 9728),
}


ROOF_KERNEL = "decode_half_kernel<4,2,1,10,-3> (gate_up 19456x2560 + silu*up, M=1)"
PREFILL_ROOF_KERNEL = "gemm_wdx_kernel (qkv, o, gate_up + silu*up, down at 2048 tokens)"
PREFILL_REPS = 8  # launches per graph replay: back to back, as the layers of a prefill run


def prefill_graph_times(torch, kernels, lib, stack, layer, m: int, steps: int, gen, dev) -> dict[str, float]:
    """Microseconds per launch of each prefill projection at m tokens (split-K
    workspace): PREFILL_REPS launches per graph replay, so the graph's own
    launch cost is not counted against one GEMM; HIP events on the replay
    stream around max(3, steps // 2) replays after 2 warm-ups."""
    weights = {"qkv_proj": layer.qkv, "o_proj": layer.o, "gate_up_proj": layer.gate_up, "down_proj": layer.down}
    out = {}
    for name, pw in weights.items():
        x = torch.randn((m, pw.k), generator=gen, device=dev).to(torch.bfloat16)
        epi = lib.EPI_SILU_MUL if name == "gate_up_proj" else lib.EPI_NONE
        y = torch.empty((m, pw.out_features), device=dev, dtype=torch.bfloat16)
        graph = stack.capture(lambda x=x, pw=pw, epi=epi, y=y: [
            kernels.linear(x, pw, epilogue=epi, out=y) for _ in range(PREFILL_REPS)])
        out[name] = time_graph(torch, graph, max(3, steps // 2), 2) * 1e3 / PREFILL_REPS
        del graph, x, y
    return out


TP_DEGREE = 8


def tp_shard(torch, kernels, lib, stack, g, steps: int, warmup: int, gen, dev, prefill_tokens: int | None) -> dict:
    """One GPU's share of TP_DEGREE-way tensor parallelism at the real shard
    shapes: QKV split by output rows (4 q heads + 1 kv head, 768 x 2560),
    o_proj by its K (2560 x 512), gate_up by output rows keeping the gate/up
    pairing (2 x 1216 x 2560, SiLU*up), down by its K (2560 x 1216), the tied
    lm_head by vocab (18992 x 2560).  Timed: the shard's 36-layer M = 1 step
    (144 launches in one graph over 36 distinct shard layers), each shard
    projection over 36 launches, the shard's greedy head (4 calls per
    replay), and its prefill layer at `prefill_tokens` tokens (None: not
    timed).  The all-reduces that would join the shards are not run."""
    from leanstack_amd.layout import PackedWeight

    tp, h, inter, n_l = TP_DEGREE, g.hidden_size, g.intermediate_size, g.num_hidden_layers
    shapes = {"qkv_proj": (g.qkv_dim // tp, h), "o_proj": (h, g.q_dim // tp),
              "gate_up_proj": (2 * inter // tp, h), "down_proj": (h, inter // tp)}

    def pack(name):
        n, k = shapes[name]
        w = (torch.randn((n, k), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        return PackedWeight.from_rowmajor(
            w, lib.LAYOUT_MFMA16X32_GATEUP if name == "gate_up_proj" else lib.LAYOUT_MFMA16X32)

    def call_bytes(name, m):
        n, k = shapes[name]
        return n * k * 2 + m * k * 2 + m * (n // 2 if name == "gate_up_proj" else n) * 2

    layers = [{name: pack(name) for name in shapes} for _ in range(n_l)]
    x = {name: torch.randn((n_l, 1, shapes[name][1]), generator=gen, device=dev).to(torch.bfloat16)
         for name in ("qkv_proj", "o_proj", "gate_up_proj")}
    y = {"qkv_proj": torch.empty((1, shapes["qkv_proj"][0]), device=dev, dtype=torch.bfloat16),
         "o_proj": torch.empty((1, h), device=dev, dtype=torch.bfloat16),
         "gate_up_proj": torch.empty((1, inter // tp), device=dev, dtype=torch.bfloat16),
         "down_proj": torch.empty((1, h), device=dev, dtype=torch.bfloat16)}

    def launch(name, l):
        if name == "down_proj":  # reads the activation gate_up wrote, as in the full step
            kernels.linear(y["gate_up_proj"], layers[l][name], out=y[name])
        else:
            epi = lib.EPI_SILU_MUL if name == "gate_up_proj" else lib.EPI_NONE
            kernels.linear(x[name][l], layers[l][name], epilogue=epi, out=y[name])

    graph = stack.capture(lambda: [launch(name, l) for l in range(n_l) for name in shapes])
    settle(torch, graph, 0.1)
    ms = time_graph(torch, graph, steps, warmup)
    del graph
    step_bytes = n_l * sum(call_bytes(name, 1) for name in shapes)
    res = {
        "tp": tp,
        "shapes": {name: list(s) for name, s in shapes.items()},
        "decode_step_m1": {"us": round(ms * 1e3, 1), "launches": 4 * n_l, "bytes": step_bytes,
                           "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                           "frac_of_hbm_peak": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "floor_us_at_hbm_peak": round(step_bytes / (HBM_PEAK_GBS * 1e9) * 1e6, 1)},
        "per_projection_m1": {},
        "not_run": "the two all-reduces of [M, 2560] per layer and the head's (max, index) exchange (one GPU)",
    }
    log(f"tp{tp} shard step M=1: {ms * 1e3:.1f} us ({res['decode_step_m1']['GB/s']} GB/s, floor "
        f"{res['decode_step_m1']['floor_us_at_hbm_peak']} us)")
    for name in shapes:
        graph = stack.capture(lambda name=name: [launch(name, l) for l in range(n_l)])
        us = time_graph(torch, graph, steps, warmup) * 1e3 / n_l
        del graph
        res["per_projection_m1"][name] = {"us_per_launch": round(us, 2),
                                          "GB/s": round(call_bytes(name, 1) / (us * 1e-6) / 1e9, 1)}
        log(f"tp{tp} shard {name} {shapes[name][0]}x{shapes[name][1]} M=1: {us:.2f} us/launch")
    del layers, x, y

    v = g.vocab_size // tp
    e = PackedWeight.from_rowmajor((torch.randn((v, h), generator=gen, device=dev) * 0.02).to(torch.bfloat16))
    hidden = torch.randn((1, h), generator=gen, device=dev).to(torch.bfloat16)
    ws = kernels.LmHeadWorkspace(1, v, h, dev)
    tok = torch.empty((1,), device=dev, dtype=torch.long)
    reps = 4
    graph = stack.capture(lambda: [kernels.lm_head_argmax(hidden, e, workspace=ws, out=tok) for _ in range(reps)])
    us = time_graph(torch, graph, steps, warmup) * 1e3 / reps
    del graph
    head_bytes = v * h * 2 + h * 2
    res["lm_head_m1"] = {"vocab_rows": v, "us": round(us, 2), "GB/s": round(head_bytes / (us * 1e-6) / 1e9, 1)}
    log(f"tp{tp} shard lm_head {v}x{h} M=1: {us:.2f} us")
    del e

    if prefill_tokens is not None:
        m = prefill_tokens
        p0 = {name: pack(name) for name in shapes}
        layer = types.SimpleNamespace(qkv=p0["qkv_proj"], o=p0["o_proj"], gate_up=p0["gate_up_proj"],
                                      down=p0["down_proj"])
        times = prefill_graph_times(torch, kernels, lib, stack, layer, m, steps, gen, dev)
        flops = {name: 2 * m * shapes[name][0] * shapes[name][1] for name in shapes}
        layer_us = sum(times.values())
        res["prefill"] = {
            "tokens": m,
            "layer_us": round(layer_us, 1),
            "layer_TFLOP/s": round(sum(flops.values()) / (layer_us * 1e-6) / 1e12, 1),
            "per_projection": {name: {"us": round(us, 1), "TFLOP/s": round(flops[name] / (us * 1e-6) / 1e12, 1)}
                               for name, us in times.items()},
        }
        log(f"tp{tp} shard prefill M={m}: layer {res['prefill']['layer_us']} us, "
            f"{res['prefill']['layer_TFLOP/s']} TFLOP/s")
    return res


def step_kernel_durations(kernels, stack, g, reps: int) -> dict[str, list[float]]:
    """Each dispatch's own duration (us) over `reps` eager launches of the
    36-layer M = 1 step, by projection (the step launches qkv, o, gate_up,
    down per layer, in that order).  The events are bound to the dispatches
    themselves (lsk_dispatch_timing_begin/end), so these are the kernels'
    execution times with the GPU idle between launches."""
    durs = kernels.kernel_durations_us(lambda: [stack.launch(1) for _ in range(reps)],
                                       max_dispatches=4 * g.num_hidden_layers * reps)
    return {name: durs[i::4] for i, name in enumerate(g.projections())}


def probe_step_floor(torch, steps: int, warmup: int) -> dict:
    """What a decode step's launch structure can reach, measured with
    lsk_probe_stream_step on the step's exact weight bytes (36 layers x
    {qkv, o, gate_up, down}, each CU streaming an equal share of each
    projection, every tile multiplied, nothing else computed): one
    persistent launch with no dependency between projections, with a flat
    grid barrier before each, with the two-level barrier, with tag words;
    the same dependency forms on 144 segments of 12 KB per CU (the
    boundary's own latency); and a HIP graph of 144 single-projection
    launches of the same kernel (the structure of the product step).  Each
    launch timed with events on its stream, median of `steps` after
    `warmup`."""
    import ctypes

    from leanstack_amd import _lib
    from leanstack_amd.geometry import QWEN3_4B as G

    lib = _lib.load()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    per_layer = [n * k // 512 for n, k in G.projections().values()]  # 1 KB tiles (512 bf16 values)
    seg = per_layer * G.num_hidden_layers
    if any(t % cus for t in seg):
        raise SystemExit(f"projection tile counts {per_layer} are not multiples of the {cus} CUs")
    total = sum(seg) * 1024
    weights = torch.empty(total, dtype=torch.uint8, device=dev)
    weights.view(torch.int16).random_(-2000, 2000)  # small finite bf16 values
    ws = torch.zeros(lib.lsk_probe_workspace_bytes(), dtype=torch.uint8, device=dev)
    arr = (ctypes.c_longlong * len(seg))(*seg)

    def launch(mode, ring, segs=arr, count=len(seg), base=weights.data_ptr(), nbytes=total):
        st = lib.lsk_probe_stream_step(base, nbytes, segs, count, mode, ring, ws.data_ptr(), ws.numel(),
                                       torch.cuda.current_stream().cuda_stream)
        _lib.check(st, "lsk_probe_stream_step")

    def timed(fn) -> float:
        for _ in range(warmup):
            fn()
        out = []
        for _ in range(steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            out.append(a.elapsed_time(b) * 1e3)
        return statistics.median(out)

    res = {"bytes": total, "projections": len(seg), "cus": cus}
    forms = [("one_launch_no_dependency_ring4", 0, 4), ("one_launch_no_dependency_ring16", 0, 16),
             ("one_launch_flat_barrier_ring4", 1, 4), ("one_launch_two_level_barrier_ring4", 2, 4),
             ("one_launch_two_level_barrier_ring16", 2, 16)]
    if cus <= 256:  # the tag-word form holds one word per CU for at most 256 CUs
        forms.append(("one_launch_tag_words_ring4", 3, 4))
    for name, mode, ring in forms:
        us = timed(lambda: launch(mode, ring))
        torch.cuda.synchronize()
        if int(ws[:4].view(torch.int32).item()) != 0:
            raise SystemExit(f"probe {name}: a bounded wait gave up")
        res[name] = {"us": round(us, 1), "GB/s": round(total / (us * 1e-6) / 1e9, 1)}
        log(f"probe {name}: {us:.1f} us, {total / (us * 1e-6) / 1e9:.0f} GB/s")
    # The boundary's own latency: 144 segments of one tile per compute wave
    # (12 KB per CU), so each segment streams in well under a microsecond and
    # the launch is almost all boundaries.
    small = [cus * 12] * len(seg)
    small_arr = (ctypes.c_longlong * len(small))(*small)
    lat = {}
    for name, mode in (("no_dependency", 0), ("two_level_barrier", 2), ("tag_words", 3)):
        if mode == 3 and cus > 256:
            continue
        us = timed(lambda: launch(mode, 4, segs=small_arr, count=len(small), nbytes=sum(small) * 1024))
        torch.cuda.synchronize()
        if int(ws[:4].view(torch.int32).item()) != 0:
            raise SystemExit(f"probe {name} on 12 KB segments: a bounded wait gave up")
        lat[name] = {"us": round(us, 1)}
        log(f"probe {name} on 12 KB segments: {us:.1f} us")
    for name in lat:
        if name != "no_dependency":
            lat[name]["us_per_boundary"] = round((lat[name]["us"] - lat["no_dependency"]["us"]) / (len(small) - 1), 2)
    res["segments_of_12_tiles_per_cu"] = lat
    # 144 dependent launches, one projection each, captured as one graph
    offsets, off = [], 0
    singles = []
    for t in seg:
        singles.append((ctypes.c_longlong * 1)(t))
        offsets.append(off)
        off += t * 1024

    def graph_step():
        for t, o, one in zip(seg, offsets, singles):
            launch(0, 4, segs=one, count=1, base=weights.data_ptr() + o, nbytes=t * 1024)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        graph_step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        graph_step()
    us = timed(graph.replay)
    res["graph_of_144_launches_ring4"] = {"us": round(us, 1), "GB/s": round(total / (us * 1e-6) / 1e9, 1)}
    log(f"probe graph of 144 launches: {us:.1f} us, {total / (us * 1e-6) / 1e9:.0f} GB/s")
    base = res["one_launch_no_dependency_ring4"]["us"]
    for name in ("one_launch_flat_barrier_ring4", "one_launch_two_level_barrier_ring4",
                 "one_launch_two_level_barrier_ring16", "one_launch_tag_words_ring4", "graph_of_144_launches_ring4"):
        if name in res:
            res[name]["us_per_boundary_over_no_dependency"] = round((res[name]["us"] - base) / (len(seg) - 1), 2)
    return res


def probe_mfma(torch, steps: int, warmup: int) -> dict:
    """The dense BF16 MFMA rate with no memory traffic (lsk_probe_mfma_rate):
    4 waves per workgroup, 16 accumulator tiles of v_mfma_f32_32x32x16_bf16
    each (the prefill GEMM's instruction and accumulators), on every CU (one
    workgroup per CU; launches of about 3.5 and 35 ms) and on 32 CUs;
    TFLOP/s = 32768 FLOP x 64 MFMAs x iterations x waves / time (HIP events,
    median of `steps`)."""
    from leanstack_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    res = {"cus": cus, "mfma": "v_mfma_f32_32x32x16_bf16", "flop_per_mfma": 32768}
    for wgs, iterations in ((cus, 4000), (32, 4000), (cus, 40000)):
        def run():
            _lib.check(lib.lsk_probe_mfma_rate(wgs, iterations, sink.data_ptr(), torch.cuda.current_stream().cuda_stream),
                       "lsk_probe_mfma_rate")
        for _ in range(warmup):
            run()
        times = []
        for _ in range(steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            run()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) * 1e3)
        us = statistics.median(times)
        flops = 32768.0 * 64 * iterations * 4 * wgs
        key = f"workgroups_{wgs}_iterations_{iterations}"
        res[key] = {"us": round(us, 1), "TFLOP/s": round(flops / (us * 1e-6) / 1e12, 1),
                    "frac_of_2.5PF_scaled_to_CUs": round(flops / (us * 1e-6) / 1e12 / (BF16_PEAK_TFLOPS * wgs / cus), 4)}
        log(f"probe mfma on {wgs} workgroups x {iterations} iterations: {us:.1f} us, {res[key]['TFLOP/s']} TFLOP/s")
    return res


def mean(values: list[float]) -> float:
    return sum(values) / len(values)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="skip the prefill sweep and the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--pmc", action="store_true",
                    help="short run for hardware-counter profiling: a 1 GiB copy of known size, then each "
                         "projection kind once per layer, the QKV and gate_up kernels with the RMSNorm prologue "
                         "once per layer, and the lm_head once, no graphs")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the two roofline measurements of the default run (the gate_up decode kernel over "
                         "36-launch graph replays, the four prefill GEMMs at M = 2048 over 8-launch replays), for "
                         "profiling with rocprofv3 --kernel-trace --stats: the trace then holds exactly their "
                         "dispatches")
    ap.add_argument("--probe-step-floor", action="store_true",
                    help="only the launch-structure probe (lsk_probe_stream_step): the step's weight bytes streamed "
                         "by one persistent launch with and without a grid barrier per projection, and by a graph "
                         "of 144 single-projection launches")
    ap.add_argument("--probe-mfma", action="store_true",
                    help="only the MFMA-rate probe (lsk_probe_mfma_rate): dense BF16 MFMAs with no memory traffic, "
                         "on every CU and on 32")
    ap.add_argument("--tp-shard-only", action="store_true",
                    help="only the tensor-parallel shard measurements (one GPU's share of 8-way TP at the real "
                         "shard shapes: the 36-layer M = 1 step, the lm_head, the prefill layer at 2048 tokens)")
    ap.add_argument("--pmc-prefill", action="store_true",
                    help="short run for hardware-counter profiling of the prefill GEMMs: each projection at "
                         "M = 512, 2048 and 8192, three launches each, no graphs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}), flush=True)
        return 2

    import torch

    from leanstack_amd import _lib, kernels
    from leanstack_amd.build import LIBRARY, build_library
    from leanstack_amd.geometry import QWEN3_4B as G
    from leanstack_amd.leanserve import ResidentArena, build_resident_buffer_plan, layer_entry_names
    from leanstack_amd.stack import DecodeLinearStack, DecodeStep, LayerProjections

    if not LIBRARY.exists():
        build_library()
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    steps, warmup = args.steps, args.warmup

    if args.probe_mfma:
        print(json.dumps({"probe_mfma": probe_mfma(torch, max(steps, 5), max(warmup, 2))}), flush=True)
        return 0
    if args.probe_step_floor:
        print(json.dumps({"probe_step_floor": probe_step_floor(torch, max(steps, 5), max(warmup, 2))}), flush=True)
        return 0

    # --- resident weights: 36 layers + lm_head in one arena ------------------
    t0 = time.perf_counter()
    plan = build_resident_buffer_plan(G, max_rows=16, include_embedding=False, buckets=())
    arena = ResidentArena(plan, dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    layers = []
    for l in range(G.num_hidden_layers):
        names = layer_entry_names(l)
        for proj, (n, k) in G.projections().items():
            w = (torch.randn((n, k), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
            arena.store_rowmajor(names[proj], w)
            del w
        layers.append(LayerProjections(arena.packed(names["qkv_proj"]), arena.packed(names["o_proj"]),
                                       arena.packed(names["gate_up_proj"]), arena.packed(names["down_proj"])))
    e = (torch.randn((G.vocab_size, G.hidden_size), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    arena.store_rowmajor("lm_head.weight", e)
    lm_head = arena.packed("lm_head.weight")
    torch.cuda.synchronize()
    log(f"arena {plan.arena_bytes / 1e9:.2f} GB resident in {time.perf_counter() - t0:.1f} s")

    stack = DecodeLinearStack(layers, G, max_rows=16, device=dev)

    if args.roofline_only:
        # The default run's two roofline measurements and nothing else, so a
        # kernel trace of this command holds exactly their dispatches.
        graph = stack.capture(lambda: stack.launch_projection("gate_up_proj", 1))
        settle(torch, graph)
        ms = time_graph(torch, graph, steps, warmup)
        del graph
        us = ms * 1e3 / G.num_hidden_layers
        bytes_gu = G.projection_bytes("gate_up_proj", 1)
        pre = prefill_graph_times(torch, kernels, _lib, stack, layers[0], 2048, steps, gen, dev)
        layer_us = sum(pre.values())
        print(json.dumps({
            "roofline_only": True,
            "roofline": {"kernel": ROOF_KERNEL, "us_per_launch": round(us, 3),
                         "launches": G.num_hidden_layers * (steps + warmup),
                         "achieved": round(bytes_gu / (us * 1e-6) / 1e9, 1),
                         "frac": round(bytes_gu / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
            "roofline_prefill": {"kernel": PREFILL_ROOF_KERNEL, "layer_us": round(layer_us, 2),
                                 "us_per_launch": {n: round(v, 3) for n, v in pre.items()},
                                 "frac": round(G.layer_flops(2048) / (layer_us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS,
                                               4)},
        }), flush=True)
        return 0

    if args.pmc:
        # Calibration: a plain device copy of exactly 1 GiB (read 1 GiB, write 1 GiB).
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        for name in G.projections():
            stack.launch_projection(name, 1)
        # the QKV and gate_up kernels with the RMSNorm prologue, once per layer each
        for l, p in enumerate(layers):
            kernels.rmsnorm_linear(stack.x_qkv[l, :1], stack.norm_w[l, 0], stack.eps, p.qkv, out=stack.y_qkv[:1])
        for l, p in enumerate(layers):
            kernels.rmsnorm_linear(stack.x_gu[l, :1], stack.norm_w[l, 1], stack.eps, p.gate_up,
                                   epilogue=_lib.EPI_SILU_MUL, out=stack.act[:1])
        hidden = torch.randn((1, G.hidden_size), generator=gen, device=dev).to(torch.bfloat16)
        kernels.lm_head_argmax(hidden, lm_head)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_run": True, "copy_bytes": 2 * src.numel(),
                          "bytes_per_launch": {n: G.projection_bytes(n, 1) for n in G.projections()}}), flush=True)
        return 0

    if args.tp_shard_only:
        shard = tp_shard(torch, kernels, _lib, stack, G, steps, warmup, gen, dev, 2048)
        print(json.dumps({"tp_shard": shard}), flush=True)
        return 0

    if args.pmc_prefill:
        p0 = layers[0]
        weights = {"qkv_proj": p0.qkv, "o_proj": p0.o, "gate_up_proj": p0.gate_up, "down_proj": p0.down}
        for m in (512, 2048, 8192):
            for name, pw in weights.items():
                x = torch.randn((m, pw.k), generator=gen, device=dev).to(torch.bfloat16)
                epi = _lib.EPI_SILU_MUL if name == "gate_up_proj" else _lib.EPI_NONE
                for _ in range(3):
                    kernels.linear(x, pw, epilogue=epi)
                torch.cuda.synchronize()
                log(f"prefill {name} M={m}: 3 launches, {G.projection_flops(name, m) / 1e9:.1f} GFLOP each")
        print(json.dumps({"pmc_prefill_run": True}), flush=True)
        return 0

    # --- headline: 36-layer decode step, verify sweep -----------------------
    # (a) 144 projection launches captured in one HIP graph;
    # (b) the persistent stack kernel: one launch per step, every projection
    #     waiting for all earlier ones (the decode step's dependency chain).
    sweep_launches, sweep = {}, {}
    stack_errors = 0
    for m in (1, 2, 4, 8):
        graph = stack.capture(lambda m=m: stack.launch(m))
        if m == 1:
            settle(torch, graph)
        ms = time_graph(torch, graph, steps, warmup)
        sweep_launches[m] = ms
        log(f"stack (144 launches) M={m}: {ms * 1e3:.1f} us/step, {G.stack_bytes(m) / ms / 1e6:.0f} GB/s")
        del graph
        if m not in (1, 8):
            continue  # the persistent form is the slower one; timed at both ends of the sweep only
        prog = stack.persistent_step(m, chain=True)
        graph = stack.capture(prog.launch)
        ms = time_graph(torch, graph, steps, warmup)
        stack_errors += prog.error()
        sweep[m] = ms
        log(f"stack (persistent) M={m}: {ms * 1e3:.1f} us/step, {G.stack_bytes(m) / ms / 1e6:.0f} GB/s")
        del graph, prog
    if stack_errors:
        raise SystemExit(f"persistent stack kernel reported {stack_errors} failed waits")
    # The headline step path is whichever product path is faster at M = 1
    # (the persistent form is timed at M = 1 and 8 only; if it ever wins it
    # must be timed at every M).
    persistent_is_faster = sweep[1] < sweep_launches[1]
    if persistent_is_faster:
        raise SystemExit("the persistent step is faster at M = 1: time it over the whole verify sweep")
    headline = sweep_launches
    ms_step = headline[1]
    value = G.stack_bytes(1) / (ms_step * 1e-3) / 1e9

    # --- the step with its RMSNorms: fused into QKV / gate_up, or separate ---
    norm_steps = {}
    for m in (1, 8):
        row = {}
        for fused in (True, False):
            graph = stack.capture(lambda m=m, fused=fused: stack.launch_with_norms(m, fused))
            ms = time_graph(torch, graph, steps, warmup)
            row["fused" if fused else "separate_rms_norm"] = round(ms * 1e3, 1)
            del graph
        row["projections_only"] = round(sweep_launches[m] * 1e3, 1)
        norm_steps[m] = row
        log(f"step with RMSNorms M={m}: fused {row['fused']} us, separate {row['separate_rms_norm']} us, "
            f"projections only {row['projections_only']} us")

    # --- a whole decode token with attention, every layer HIP ----------------
    # input norm + QKV, attention (q/k norms, RoPE, cache append, GQA over the
    # cached rows), o_proj + residual, post norm + gate_up, down + residual,
    # then the final norm and the lm_head argmax; cache rows random.
    token_steps = {}
    n_l, n_kv, hd = G.num_hidden_layers, G.num_key_value_heads, G.head_dim
    kv_rows = 4096
    k_cache = torch.randn((n_l, n_kv, kv_rows, hd), generator=gen, device=dev).to(torch.bfloat16)
    v_cache = torch.randn((n_l, n_kv, kv_rows, hd), generator=gen, device=dev).to(torch.bfloat16)
    norms = (1 + 0.1 * torch.randn((n_l, 2, G.hidden_size), generator=gen, device=dev)).to(torch.bfloat16)
    qk_norms = (1 + 0.1 * torch.randn((n_l, 2, hd), generator=gen, device=dev)).to(torch.bfloat16)
    final_norm = (1 + 0.1 * torch.randn((G.hidden_size,), generator=gen, device=dev)).to(torch.bfloat16)
    token_step = DecodeStep(layers, norms, qk_norms, final_norm, lm_head, G, k_cache, v_cache, dev)
    token_step.hidden[0].copy_(torch.randn((1, G.hidden_size), generator=gen, device=dev).to(torch.bfloat16))
    # One graph for every position: the attention kernels read the position
    # from token_step.pos_dev, written before the replays.
    token_step.set_position(0)
    graph = stack.capture(lambda: token_step.launch())
    for pos in (320, kv_rows - 1):
        token_step.set_position(pos)
        ms = time_graph(torch, graph, steps, warmup)
        token_steps[pos] = {"us": round(ms * 1e3, 1), "tokens_per_s": round(1e3 / ms, 1)}
        log(f"decode token with attention over {pos} cached rows: {ms * 1e3:.1f} us ({1e3 / ms:.0f} tokens/s)")
    del graph

    # --- a greedy decode loop: each token the argmax of the one before -------
    # The reference's decode loop (qwen_explicit_runtime_loop.py:331-385) with
    # its per-step events, in the shape of its decode_64_256 benchmark (a
    # 64-token prompt, 256 generated tokens): the cache rows below position
    # 64 stand for the prompt.  One graph of DecodeStep.launch_next (embedding
    # row of the last token, the 36 layers, the head, token record, position
    # advance) is replayed once per token, with a pair of events around each
    # replay and one pair around the loop. The loop runs twice from the same
    # start (same first token, position and cache rows below it): the second
    # run must emit the same tokens.
    loop_tokens, loop_start = 256, 64
    embedding = (0.02 * torch.randn((G.vocab_size, G.hidden_size), generator=gen, device=dev)).to(torch.bfloat16)
    emitted = torch.full((kv_rows,), -1, device=dev, dtype=torch.long)
    graph = stack.capture(lambda: token_step.launch_next(embedding, emitted))
    runs = []
    for _ in range(2):
        token_step.token.fill_(1)
        token_step.set_position(loop_start)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(loop_tokens)]
        loop_ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        loop_ev[0].record()
        for a, b in ev:
            a.record()
            graph.replay()
            b.record()
        loop_ev[1].record()
        torch.cuda.synchronize()
        step_us = sorted(a.elapsed_time(b) * 1e3 for a, b in ev)
        runs.append((loop_ev[0].elapsed_time(loop_ev[1]) * 1e3, step_us,
                     emitted[loop_start:loop_start + loop_tokens].cpu()))
    del graph, embedding, token_step, k_cache, v_cache
    loop_us, step_us, toks = runs[1]
    if not torch.equal(runs[0][2], toks) or int(toks.min()) < 0:
        raise SystemExit("greedy decode loop: the two runs from the same start emitted different tokens")
    greedy_loop = {
        "workload": "decode_64_256 shape: 64 cached prompt rows, 256 greedy tokens (prefill not timed)",
        "tokens": loop_tokens, "first_position": loop_start, "loop_us": round(loop_us, 1),
        "tokens_per_s": round(loop_tokens / (loop_us * 1e-6), 1),
        "step_us_median": round(step_us[len(step_us) // 2], 1), "step_us_p10": round(step_us[len(step_us) // 10], 1),
        "step_us_p90": round(step_us[len(step_us) * 9 // 10], 1), "distinct_tokens": int(toks.unique().numel()),
        "repeatable": True,
    }
    log(f"greedy decode loop, {loop_tokens} tokens from position {loop_start}: {loop_us / loop_tokens:.1f} us/token "
        f"({greedy_loop['tokens_per_s']} tokens/s), step median {greedy_loop['step_us_median']} us, "
        f"{greedy_loop['distinct_tokens']} distinct tokens, same tokens on a second run")

    # --- per projection kind: 36 launches of one kind per replay ------------
    per_kernel = {}
    for name in G.projections():
        graph = stack.capture(lambda name=name: stack.launch_projection(name, 1))
        ms = time_graph(torch, graph, steps, warmup)
        us = ms * 1e3 / G.num_hidden_layers
        per_kernel[name] = {
            "us_per_launch": round(us, 2),
            "GB/s": round(G.projection_bytes(name, 1) / (us * 1e-6) / 1e9, 1),
            "bytes_per_launch": G.projection_bytes(name, 1),
        }
        log(f"{name} M=1: {us:.2f} us/launch, {per_kernel[name]['GB/s']} GB/s")
        del graph
    # Dominant kernel of the step: the fused gate_up + SiLU*up decode kernel
    # (49% of the step's bytes), per launch over 36 back-to-back launches.
    roof_kernel = ROOF_KERNEL
    roof_bytes = G.projection_bytes("gate_up_proj", 1)
    roof_us = per_kernel["gate_up_proj"]["us_per_launch"]
    achieved = roof_bytes / (roof_us * 1e-6) / 1e9
    # The same kernels launched eagerly, one dispatch at a time, each timed
    # by events bound to the dispatch itself: their own durations with the
    # GPU idle between launches (slower than back to back in a graph).
    step_durs = step_kernel_durations(kernels, stack, G, 2)
    for name, v in step_durs.items():
        per_kernel[name]["eager_kernel_us"] = round(mean(v), 3)
        log(f"{name} M=1 eager dispatch: {mean(v):.3f} us kernel time")

    # --- lm_head + argmax ------------------------------------------------------
    head = {}
    hidden = torch.randn((16, G.hidden_size), generator=gen, device=dev).to(torch.bfloat16)
    logits = torch.empty((16, G.vocab_size), device=dev, dtype=torch.float32)
    ws = kernels.LmHeadWorkspace(16, G.vocab_size, G.hidden_size, dev)
    tokens = torch.empty((16,), device=dev, dtype=torch.long)
    # The greedy head as the reference's cuTile head runs it (fp32 scores,
    # tile maxima, argmax; no logits written: cutile_logits.py:17-31, :67-69),
    # 4 calls per graph replay (as the prefill GEMMs run 8), so that one
    # replay's own launch cost is not charged to one call.  Beside it: one
    # call per replay, and the same head also writing the fp32 logits.
    head_reps = 4
    for m in (1, 2, 4, 8):
        def head_fn(m=m, reps=head_reps, with_logits=False):
            for _ in range(reps):
                kernels.lm_head_argmax(hidden[:m], lm_head, logits_out=logits[:m] if with_logits else None,
                                       workspace=ws, out=tokens[:m])
        row = {}
        for key, fn, reps in (("us", head_fn, head_reps), ("us_one_call_per_replay", lambda m=m: head_fn(m, 1), 1),
                              ("us_with_fp32_logits", lambda m=m: head_fn(m, head_reps, True), head_reps)):
            graph = stack.capture(fn)
            settle(torch, graph, 0.05)
            row[key] = round(time_graph(torch, graph, steps, warmup) / reps * 1e3, 2)
            del graph
        row["GB/s"] = round(G.lm_head_call_bytes(m, logits=False) / (row["us"] * 1e-6) / 1e9, 1)
        head[m] = row
        log(f"lm_head M={m}: {row['us']} us ({row['us_one_call_per_replay']} us as one call per replay, "
            f"{row['us_with_fp32_logits']} us also writing fp32 logits), {row['GB/s']} GB/s")

    # --- prefill GEMMs ---------------------------------------------------------
    prefill = {}
    if not args.quick:
        for m in (512, 2048, 8192):
            times = prefill_graph_times(torch, kernels, _lib, stack, layers[0], m, steps, gen, dev)
            row = {name: {"us": round(us, 1), "TFLOP/s": round(G.projection_flops(name, m) / (us * 1e-6) / 1e12, 1)}
                   for name, us in times.items()}
            layer_us = sum(times.values())
            row["layer_us"] = round(layer_us, 1)
            row["layer_TFLOP/s"] = round(G.layer_flops(m) / (layer_us * 1e-6) / 1e12, 1)
            prefill[m] = row
            log(f"prefill M={m}: layer {row['layer_us']} us, {row['layer_TFLOP/s']} TFLOP/s")

    # --- the reference's hot-kernel GEMM cases --------------------------------
    hot = {}
    if not args.quick:
        from leanstack_amd.layout import PackedWeight

        for case, (m, n, k) in HOT_KERNEL_CASES.items():
            w = (torch.randn((n, k), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
            pw = PackedWeight.from_rowmajor(w)
            x = torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
            y = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
            reps = 8
            graph = stack.capture(lambda x=x, pw=pw, y=y, r=reps: [kernels.linear(x, pw, out=y) for _ in range(r)])
            ms = time_graph(torch, graph, max(3, steps // 2), 2) / reps
            hot[case] = {"m": m, "n": n, "k": k, "us": round(ms * 1e3, 2),
                         "TFLOP/s": round(2 * m * n * k / (ms * 1e-3) / 1e12, 1)}
            log(f"hot-kernel case {case}: {hot[case]['us']} us, {hot[case]['TFLOP/s']} TFLOP/s")
            del graph, w, pw, x, y

    # Prefill roofline at 2048 tokens: the layer's four GEMMs against dense
    # BF16 MFMA peak (2.5 PFLOP/s), TFLOP/s = 2 M N K / time.
    prefill_roofline = None
    if 2048 in prefill:
        row = prefill[2048]
        achieved_tf = row["layer_TFLOP/s"]
        prefill_roofline = {
            "bound": "mfma",
            "kernel": PREFILL_ROOF_KERNEL,
            "flops_per_layer": G.layer_flops(2048),
            "achieved": achieved_tf,
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved_tf / BF16_PEAK_TFLOPS, 4),
            "layer_us": row["layer_us"],
            "us_per_launch": {n: row[n]["us"] for n in G.projections()},
            "per_projection_TFLOP/s": {n: row[n]["TFLOP/s"] for n in G.projections()},
            "mfma_util_pct": profiled_mfma_util(),
            "mfma_util_source": "profiles/prefill_gemm_counters.md (rocprofv3 --pmc MfmaUtil, bench.py --pmc-prefill)",
        }

    # --- one GPU's share of 8-way tensor parallelism ---------------------------
    shard = tp_shard(torch, kernels, _lib, stack, G, steps, warmup, gen, dev, None if args.quick else 2048)

    cpu = None
    if not args.quick:
        cpu = cpu_baseline(G, args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads")
        cpu["o_proj_gemv_2560x4096"] = cpu_o_proj_gemv(min(3.0, args.cpu_seconds))
        log(f"cpu baseline, o_proj GEMV 2560x4096 at M=1 alone: {cpu['o_proj_gemv_2560x4096']['us']} us, "
            f"{cpu['o_proj_gemv_2560x4096']['GB/s']} GB/s")

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations, generated on the GPU)",
        "config": {
            "workload": "qwen3-4b decode projection stack: 36 layers x (qkv 6144x2560, o 2560x4096, "
                        "gate_up 19456x2560 + silu*up, down 2560x9728), M=1, each projection after the previous one",
            "layers": G.num_hidden_layers,
            "m": 1,
            "bytes_per_step": G.stack_bytes(1),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": roof_kernel,
            "bytes_per_launch": roof_bytes,
            "us_per_launch": round(roof_us, 3),
            "us_per_launch_source": (f"HIP events on the replay stream around {steps} replays of a graph of "
                                     f"{G.num_hidden_layers} back-to-back launches (one per layer), after {warmup} "
                                     f"warm-up replays"),
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(roof_kernel),
            "traffic_source": "profiles/decode_projections_hbm_traffic.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                              "scaled by a 1 GiB copy in the same run)",
        },
        "roofline_prefill": prefill_roofline,
        "cpu_baseline": cpu,
        "detail": {
            "stack_frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
            "step_path": "HIP graph of 144 projection launches",
            "verify_sweep_us_per_step": {str(m): round(v * 1e3, 1) for m, v in headline.items()},
            "verify_ratio_vs_m1": {str(m): round(v / headline[1], 4) for m, v in headline.items()},
            # one layer = the step over 36 distinct layers (7.27 GB, no MALL reuse) / 36
            "one_layer_us": {str(m): round(v * 1e3 / G.num_hidden_layers, 2) for m, v in headline.items()},
            "launches_sweep_us_per_step": {str(m): round(v * 1e3, 1) for m, v in sweep_launches.items()},
            "persistent_us_per_step": {str(m): round(v * 1e3, 1) for m, v in sweep.items()},
            "step_with_rmsnorms_us": {str(m): v for m, v in norm_steps.items()},
            "decode_token_with_attention": {str(p): v for p, v in token_steps.items()},
            "greedy_decode_loop": greedy_loop,
            "per_projection_m1": per_kernel,
            "lm_head_argmax": {str(m): v for m, v in head.items()},
            "prefill": {str(m): v for m, v in prefill.items()},
            "hot_kernel_cases": hot,
            "tp8_shard": shard,
            "device": torch.cuda.get_device_name(0),
        },
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
