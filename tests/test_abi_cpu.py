"""The C ABI without a GPU: the library loads, exports every declared symbol,
and rejects bad arguments before anything touches the device."""

from __future__ import annotations

import ctypes
import json
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from leanstack_amd import _lib

REPO = Path(__file__).resolve().parent.parent


def test_library_exports_every_header_function():
    lib = _lib.load()
    names = _lib.header_functions()
    assert {"lsk_linear_bf16", "lsk_lm_head_argmax_bf16", "lsk_pack_bf16", "lsk_stack_run"} <= set(names)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing
    assert set(names) == set(_lib._SIGNATURES)  # every export has declared ctypes types
    assert lib.lsk_abi_version() == _lib.ABI_VERSION


def test_projection_struct_layout():
    # struct lsk_projection on x86-64 (natural alignment, 8-byte pointers)
    assert ctypes.sizeof(_lib.Projection) == 72
    assert _lib.Projection.x.offset == 24 and _lib.Projection.y.offset == 40
    assert _lib.Projection.residual.offset == 56 and _lib.Projection.depends_on.offset == 68


FAKE = 0x10000  # a 64 KiB-aligned non-null address: never dereferenced, calls fail validation first


@pytest.mark.parametrize("kwargs,code", [
    (dict(layout=9), _lib.ERR_LAYOUT),
    (dict(n=2568), _lib.ERR_INVALID),        # N not a multiple of 16
    (dict(k=2576), _lib.ERR_INVALID),        # K not a multiple of 32
    (dict(m=0), _lib.ERR_INVALID),
    (dict(ldx=2552), _lib.ERR_INVALID),      # ldx < K
    (dict(ldx=2564), _lib.ERR_INVALID),      # ldx not a multiple of 8
    (dict(ldx=1 << 22), _lib.ERR_INVALID),   # 256 rows x ldx x 2 bytes would reach 2^31
    (dict(epi=1), _lib.ERR_INVALID),         # SiLU needs the gate_up layout
    (dict(epi=5), _lib.ERR_INVALID),
    (dict(epi=2), _lib.ERR_INVALID),         # residual-add without a residual
    (dict(x=0), _lib.ERR_INVALID),
    (dict(x=FAKE + 2), _lib.ERR_INVALID),    # x misaligned
    (dict(ldy=6142), _lib.ERR_INVALID),      # ldy < N
])
def test_linear_rejects_before_launch(kwargs, code):
    a = dict(w=FAKE, layout=1, n=6144, k=2560, x=FAKE, m=1, ldx=2560, y=FAKE, ldy=6144, epi=0, res=None, ldr=0)
    a.update(kwargs)
    lib = _lib.load()
    status = lib.lsk_linear_bf16(a["w"], a["layout"], a["n"], a["k"], a["x"] or None, a["m"], a["ldx"], a["y"],
                                 a["ldy"], a["epi"], a["res"], a["ldr"], None, 0, None)
    assert status == code, _lib.last_error()
    assert _lib.last_error()
    with pytest.raises(ValueError):
        _lib.check(status, "lsk_linear_bf16")


@pytest.mark.parametrize("kwargs,code", [
    (dict(layout=9), _lib.ERR_LAYOUT),
    (dict(k=2576), _lib.ERR_INVALID),        # K not a multiple of 32
    (dict(m=0), _lib.ERR_INVALID),
    (dict(m=17), _lib.ERR_INVALID),          # decode / verify rows only
    (dict(nw=0), _lib.ERR_INVALID),          # no norm weight
    (dict(nw=FAKE + 8), _lib.ERR_INVALID),   # norm weight misaligned
    (dict(eps=-1e-6), _lib.ERR_INVALID),
    (dict(eps=float("nan")), _lib.ERR_INVALID),
    (dict(eps=float("inf")), _lib.ERR_INVALID),
    (dict(epi=1), _lib.ERR_INVALID),         # SiLU needs the gate_up layout
    (dict(layout=2), _lib.ERR_INVALID),      # gate_up layout needs the SiLU epilogue
    (dict(x=FAKE + 2), _lib.ERR_INVALID),
    (dict(ldy=6140), _lib.ERR_INVALID),
])
def test_rmsnorm_linear_rejects_before_launch(kwargs, code):
    a = dict(w=FAKE, layout=1, n=6144, k=2560, x=FAKE, m=1, ldx=2560, nw=FAKE, eps=1e-6, y=FAKE, ldy=6144, epi=0)
    a.update(kwargs)
    lib = _lib.load()
    status = lib.lsk_rmsnorm_linear_bf16(a["w"], a["layout"], a["n"], a["k"], a["x"], a["m"], a["ldx"],
                                         a["nw"] or None, a["eps"], a["y"], a["ldy"], a["epi"], None, 0, None)
    assert status == code, _lib.last_error()
    assert _lib.last_error()


@pytest.mark.parametrize("kwargs,code", [
    (dict(d=64), _lib.ERR_INVALID),            # head_dim other than 128
    (dict(n_q=24), _lib.ERR_INVALID),          # 3 q heads per kv head
    (dict(n_q=7), _lib.ERR_INVALID),           # not a multiple of n_kv
    (dict(n_kv=0), _lib.ERR_INVALID),
    (dict(pos=4096), _lib.ERR_INVALID),        # pos == max_seq_len
    (dict(pos=-1), _lib.ERR_INVALID),
    (dict(s=20000, pos=10), _lib.ERR_INVALID),   # caches longer than 16384 rows
    (dict(n_q=128, n_kv=128), _lib.ERR_INVALID),  # more than 64 kv heads
    (dict(pos=128, ws=0), _lib.ERR_WORKSPACE),   # more than 128 rows need the workspace
    (dict(pos=600, nbytes=1024), _lib.ERR_WORKSPACE),
    (dict(kc=FAKE + 8), _lib.ERR_INVALID),     # cache misaligned
    (dict(qkv=0), _lib.ERR_INVALID),
    (dict(eps=-1.0), _lib.ERR_INVALID),
    (dict(scale=float("inf")), _lib.ERR_INVALID),
])
def test_decode_attention_rejects_before_launch(kwargs, code):
    a = dict(qkv=FAKE, n_q=32, n_kv=8, d=128, kc=FAKE, s=4096, pos=10, eps=1e-6, scale=128 ** -0.5, ws=FAKE,
             nbytes=1 << 30)
    a.update(kwargs)
    lib = _lib.load()
    status = lib.lsk_decode_attention_bf16(a["qkv"] or None, a["n_q"], a["n_kv"], a["d"], FAKE, FAKE, a["eps"], FAKE,
                                           FAKE, a["kc"], FAKE, a["s"], a["pos"], a["scale"], FAKE, a["ws"] or None,
                                           a["nbytes"], None)
    assert status == code, _lib.last_error()
    assert _lib.last_error()


@pytest.mark.parametrize("kwargs,code", [
    (dict(pos_ptr=0), _lib.ERR_INVALID),         # no device position
    (dict(pos_ptr=FAKE + 2), _lib.ERR_INVALID),  # not 4-byte aligned
    (dict(ws=0), _lib.ERR_WORKSPACE),            # the launch shape covers max_seq_len rows
    (dict(s=20000), _lib.ERR_INVALID),
    (dict(d=64), _lib.ERR_INVALID),
    (dict(eps=float("nan")), _lib.ERR_INVALID),
])
def test_decode_attention_at_rejects_before_launch(kwargs, code):
    a = dict(pos_ptr=FAKE, s=4096, d=128, eps=1e-6, ws=FAKE)
    a.update(kwargs)
    lib = _lib.load()
    status = lib.lsk_decode_attention_at_bf16(FAKE, 32, 8, a["d"], FAKE, FAKE, a["eps"], FAKE, FAKE, FAKE, FAKE,
                                              a["s"], a["pos_ptr"] or None, 128 ** -0.5, FAKE, a["ws"] or None,
                                              1 << 30, None)
    assert status == code, _lib.last_error()
    assert _lib.last_error()


def test_attention_workspace_bytes():
    """Counters for 64 kv heads, then one (m, l, acc) slot of 4 * (2G + 128G)
    bytes per (kv head, chunk) for the most chunks a position below
    max_seq_len needs: 1 up to 128 rows, 64-row chunks up to 512 rows (at
    most 8), then chunks of a multiple of 128 rows (at most 32)."""
    lib = _lib.load()
    slot = 4 * (2 * 4 + 128 * 4)
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 4096) == 256 + 8 * 32 * slot
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 16384) == 256 + 8 * 32 * slot
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 1000) == 256 + 8 * 8 * slot
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 100) == 256 + 8 * 1 * slot
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 128) == 256 + 8 * 1 * slot
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 129) == 256 + 8 * 3 * slot   # 3 chunks of 64 rows
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 300) == 256 + 8 * 5 * slot
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 512) == 256 + 8 * 8 * slot
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 600) == 256 + 8 * 8 * slot   # 512 rows need 8
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 1500) == 256 + 8 * 12 * slot
    assert lib.lsk_attention_workspace_bytes(32, 8, 64, 4096) == 0      # head_dim
    assert lib.lsk_attention_workspace_bytes(24, 8, 128, 4096) == 0     # 3 q heads per kv head
    assert lib.lsk_attention_workspace_bytes(32, 8, 128, 16385) == 0    # too many rows


def test_lm_head_rejects_before_launch():
    lib = _lib.load()
    ok = dict(V=151936, K=2560, M=1)
    ws = lib.lsk_workspace_bytes(_lib.OP_LM_HEAD_ARGMAX, 1, 151936, 2560)
    # status header + one partial per scoring workgroup: 4492 of two 16-row
    # vocab blocks, then a tail of 512 single blocks (151936 / 16 = 9496 = 2 * 4492 + 512)
    assert ws == 64 + (4492 + 512) * 8
    # an odd count of row-blocks (the vocab shard of 8-way tensor parallelism,
    # 151936 / 8 = 18992 = 16 * 1187): 337 pairs, then a tail of 513 single blocks
    assert lib.lsk_workspace_bytes(_lib.OP_LM_HEAD_ARGMAX, 1, 18992, 2560) == 64 + (337 + 513) * 8
    # up to 512 row-blocks, one workgroup each
    assert lib.lsk_workspace_bytes(_lib.OP_LM_HEAD_ARGMAX, 2, 16 * 101, 2560) == 64 + 2 * 101 * 8
    assert lib.lsk_workspace_bytes(_lib.OP_LM_HEAD_ARGMAX, 1, 151928, 2560) == 0  # V % 16 != 0
    cases = [
        (dict(M=17), _lib.ERR_INVALID),
        (dict(V=151928), _lib.ERR_INVALID),   # V % 16 != 0: not whole row-blocks
        (dict(mode=3), _lib.ERR_INVALID),
        (dict(ws=ws - 8), _lib.ERR_WORKSPACE),
        (dict(layout=2), _lib.ERR_LAYOUT),
    ]
    for over, code in cases:
        a = dict(ok, mode=0, ws=ws, layout=1)
        a.update(over)
        st = lib.lsk_lm_head_argmax_bf16(FAKE, a["layout"], a["V"], a["K"], FAKE, a["M"], 2560, None, a["mode"], FAKE,
                                         FAKE, a["ws"], None)
        assert st == code, (over, _lib.last_error())


def test_rmsnorm_lm_head_rejects_before_launch():
    lib = _lib.load()
    ws = lib.lsk_workspace_bytes(_lib.OP_LM_HEAD_ARGMAX, 8, 151936, 2560)
    cases = [
        (dict(K=4096), _lib.ERR_INVALID),       # the fused norm serves K = 2560
        (dict(M=9), _lib.ERR_INVALID),          # and up to 8 rows
        (dict(nw=0), _lib.ERR_INVALID),         # no norm weight
        (dict(nw=FAKE + 8), _lib.ERR_INVALID),  # misaligned norm weight
        (dict(eps=-1.0), _lib.ERR_INVALID),
        (dict(layout=2), _lib.ERR_LAYOUT),
        (dict(ws=8), _lib.ERR_WORKSPACE),
    ]
    for over, code in cases:
        a = dict(V=151936, K=2560, M=1, nw=FAKE, eps=1e-6, layout=1, ws=ws)
        a.update(over)
        st = lib.lsk_rmsnorm_lm_head_argmax_bf16(FAKE, a["layout"], a["V"], a["K"], FAKE, a["M"], a["K"],
                                                 a["nw"] or None, a["eps"], None, 0, FAKE, FAKE, a["ws"], None)
        assert st == code, (over, _lib.last_error())


def test_stack_prepare_rejects_bad_programs():
    lib = _lib.load()
    good = _lib.Projection(FAKE, 1, 6144, 2560, FAKE, 2560, FAKE, 6144, 0, None, 0, -1)
    prog_bytes = lib.lsk_stack_program_bytes(2)
    assert lib.lsk_stack_workspace_bytes(144) % 256 == 0

    def prepare(*projs, m=1, nbytes=prog_bytes):
        arr = (_lib.Projection * len(projs))(*projs)
        return lib.lsk_stack_prepare(arr, len(projs), m, FAKE, nbytes)

    self_dep = _lib.Projection(FAKE, 1, 6144, 2560, FAKE, 2560, FAKE, 6144, 0, None, 0, 1)
    assert prepare(good, self_dep) == _lib.ERR_INVALID
    assert prepare(good, good, m=17) == _lib.ERR_INVALID
    assert prepare(good, good, nbytes=prog_bytes - 1) == _lib.ERR_INVALID
    k_small = _lib.Projection(FAKE, 1, 64, 128, FAKE, 128, FAKE, 64, 0, None, 0, -1)
    assert prepare(good, k_small) == _lib.ERR_INVALID  # K/32 = 4 < 8 waves
    assert "projection 1" in _lib.last_error()
    assert lib.lsk_stack_run(FAKE, 2, FAKE, 16, None) == _lib.ERR_WORKSPACE


def test_bench_refuses_more_than_one_gpu():
    out = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 2
    assert "one GPU" in json.loads(out.stdout.strip().splitlines()[-1])["error"]


def test_product_package_does_not_import_the_oracle():
    for path in (REPO / "leanstack_amd").rglob("*.py"):
        text = path.read_text(encoding="utf-8")
        assert "import oracle" not in text and "from oracle" not in text, path


def test_wrappers_refuse_outputs_of_the_wrong_size():
    """A caller's `out` must hold exactly what the kernel writes: the C layer
    sees only a pointer, so x[5, K] with out[1, N] would write 4 rows past the
    allocation.  The wrappers check sizes before anything reaches the device
    (CPU tensors here: the size check comes first)."""
    from leanstack_amd import kernels
    from leanstack_amd.layout import PackedWeight

    w = PackedWeight(torch.zeros(64 * 64, dtype=torch.bfloat16), 64, 64, _lib.LAYOUT_MFMA16X32)
    x = torch.zeros((5, 64), dtype=torch.bfloat16)
    for bad in (torch.empty((1, 64), dtype=torch.bfloat16), torch.empty((5, 64), dtype=torch.float32),
                torch.empty((5, 128), dtype=torch.bfloat16)[:, :64], torch.empty((6, 64), dtype=torch.bfloat16)):
        with pytest.raises(ValueError, match="out must be"):
            kernels.linear(x, w, out=bad)
        with pytest.raises(ValueError, match="out must be"):
            kernels.rmsnorm_linear(x, torch.ones(64, dtype=torch.bfloat16), 1e-6, w, out=bad)
    for bad in (torch.empty(4, dtype=torch.long), torch.empty(5, dtype=torch.int32),
                torch.empty((5, 2), dtype=torch.long)[:, 0]):
        with pytest.raises(ValueError, match="out must be"):
            kernels.lm_head_argmax(x, w, out=bad)
    with pytest.raises(ValueError, match="residual has"):
        kernels.linear(x, w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=torch.zeros((4, 64), dtype=torch.bfloat16))
    # right sizes pass the size checks and stop at the device check
    with pytest.raises(ValueError, match="GPU tensor"):
        kernels.linear(x, w, out=torch.empty((5, 64), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="GPU tensor"):
        kernels.lm_head_argmax(x, w, out=torch.empty(8, dtype=torch.long))


def test_wrappers_refuse_tensors_on_another_device():
    """Every tensor of a call must live on the first one's device: the C layer
    launches on one device and would take another device's pointers as its
    own.  (Meta tensors stand in for a second device here.)"""
    from leanstack_amd import kernels

    a = torch.zeros(4)
    assert kernels._one_device(a, (torch.zeros(2), "w"), (None, "residual")) == a.device
    with pytest.raises(ValueError, match="residual is on meta"):
        kernels._one_device(a, (torch.zeros(2), "w"), (torch.zeros(2, device="meta"), "residual"))


def test_launch_next_refuses_a_bad_token_buffer():
    """DecodeStep.launch_next's token buffer: 1-D int64 on the step's device."""
    from leanstack_amd.stack import DecodeStep

    step = DecodeStep.__new__(DecodeStep)
    step.g = type("G", (), {"hidden_size": 64})()
    step.pos_dev = torch.zeros(1, dtype=torch.int32)
    emb = torch.zeros((16, 64), dtype=torch.bfloat16)
    for bad in (torch.zeros(4, dtype=torch.int32), torch.zeros((2, 2), dtype=torch.long),
                torch.zeros(0, dtype=torch.long)):
        with pytest.raises(ValueError, match="tokens_out"):
            step.launch_next(emb, bad)


def test_noalloc_lm_head_rejects_before_launch():
    """The allocation-free head refuses calls whose workspace exceeds its
    static scratch (64 + M * P * 8 bytes > 1 MiB, P the scoring workgroups)
    and the usual bad arguments, before touching the GPU."""
    lib = _lib.load()

    def call(**over):
        a = dict(w=FAKE, layout=1, v=151936, k=2560, x=FAKE, m=1, ldx=2560, logits=None, mode=0, out=FAKE)
        a.update(over)
        return lib.lsk_lm_head_argmax_noalloc_bf16(a["w"], a["layout"], a["v"], a["k"], a["x"], a["m"], a["ldx"],
                                                   a["logits"], a["mode"], a["out"], None)

    st = call(m=16, v=1 << 19)  # 16 rows x 16640 partials x 8 B = 2.03 MiB
    assert st == _lib.ERR_INVALID and "static scratch" in _lib.last_error()
    st = call(m=16, v=253952)  # P = 8192: the partials fill exactly 1 MiB, the status header is 64 bytes over
    assert st == _lib.ERR_INVALID and "static scratch" in _lib.last_error()
    assert call(m=17) == _lib.ERR_INVALID
    assert call(layout=2) == _lib.ERR_LAYOUT
    assert call(mode=7) == _lib.ERR_INVALID
    assert call(out=FAKE + 4) == _lib.ERR_INVALID


def test_linear_plan_rejects_and_routes_without_a_device():
    """lsk_linear_plan validates before any HIP call; decode-routed shapes
    (M <= 16, or off the block GEMM's tile grid) answer {0, 0, 0, 1} on the
    host alone."""
    lib = _lib.load()
    plan = (ctypes.c_int * 4)(9, 9, 9, 9)
    assert lib.lsk_linear_plan(2048, 2560, 4096, 0, None) == _lib.ERR_INVALID
    assert lib.lsk_linear_plan(0, 2560, 4096, 0, plan) == _lib.ERR_INVALID
    assert lib.lsk_linear_plan(64, 2560, -1, 0, plan) == _lib.ERR_INVALID
    for m, n, k in [(1, 2560, 4096), (16, 19456, 2560), (300, 2560 + 16, 4096), (300, 2560, 4096 + 32)]:
        plan = (ctypes.c_int * 4)(9, 9, 9, 9)
        assert lib.lsk_linear_plan(m, n, k, 1 << 26, plan) == _lib.OK
        assert list(plan) == [0, 0, 0, 1], (m, n, k, list(plan))


def test_probe_rejects_before_launch():
    """The launch-structure probe refuses bad arguments before touching the
    GPU: no segments, an unknown mode or ring depth, a small workspace."""
    lib = _lib.load()
    need = lib.lsk_probe_workspace_bytes()
    assert need >= 4 * (256 + 256 + 8 * 256)
    segs = (ctypes.c_longlong * 2)(256 * 12, 256 * 12)
    fake = 1 << 20  # never dereferenced: every case fails validation first

    def call(count=2, mode=0, ring=4, ws_bytes=need, weights=fake):
        return lib.lsk_probe_stream_step(weights, 1 << 30, segs, count, mode, ring, fake, ws_bytes, None)

    assert call(count=0) == _lib.ERR_INVALID
    assert call(count=257) == _lib.ERR_INVALID
    assert call(mode=4) == _lib.ERR_INVALID
    assert call(mode=-1) == _lib.ERR_INVALID
    assert call(ring=8) == _lib.ERR_INVALID
    assert call(weights=fake + 8) == _lib.ERR_INVALID
    assert call(ws_bytes=need - 4) == _lib.ERR_WORKSPACE
