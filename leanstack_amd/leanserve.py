"""leanserve for the MI355X path: a resident arena planner that allocates.

The reference's planner is descriptive only: it sums file sizes, sizes the KV
cache per bucket and estimates scratch with bf16 logits, and never allocates
(src/leanstack/leanserve.py:331-377).  Here the plan is the allocation: one
device buffer (one hipMalloc through torch) holds every packed projection
weight of all layers, the norms, the row-major embedding, a packed copy of
the tied lm_head, the activation scratch for the largest row count a call
may carry, fp32 logits, the argmax workspace and the KV cache of the largest
bucket.  Every entry is a fixed, aligned view; nothing is allocated after
start-up.  With 288 GB of HBM the whole Qwen3-4B stack (about 8.8 GB) is
resident with room to spare.
"""

from __future__ import annotations

import json
import struct
from dataclasses import dataclass, field
from pathlib import Path
from math import ceil
from typing import Iterable

import torch

from . import _lib
from .geometry import QWEN3_4B, QwenGeometry
from .layout import PackedWeight

ARENA_ALIGNMENT = 4096

_DTYPE_BYTES = {torch.bfloat16: 2, torch.float32: 4, torch.int64: 8, torch.uint8: 1}
_DTYPE_NAMES = {torch.bfloat16: "bfloat16", torch.float32: "float32", torch.int64: "int64", torch.uint8: "uint8"}


@dataclass(frozen=True)
class ArenaEntry:
    name: str
    role: str
    offset: int
    nbytes: int
    dtype: str
    shape: tuple[int, ...]
    layout: int | None = None  # packed layout id for projection weights

    @property
    def end(self) -> int:
        return self.offset + self.nbytes


@dataclass(frozen=True)
class ScratchPlan:
    """Activation scratch for `rows` rows (the reference sizes one row and bf16
    logits, src/leanstack/leanserve.py:341-347; here logits are fp32, the
    precision the greedy head compares in)."""

    rows: int
    hidden_state_bytes: int
    residual_bytes: int
    qkv_projection_bytes: int
    attention_output_bytes: int
    mlp_activation_bytes: int
    logits_bytes: int
    argmax_workspace_bytes: int
    token_bytes: int

    @property
    def total_bytes(self) -> int:
        return (
            self.hidden_state_bytes + self.residual_bytes + self.qkv_projection_bytes
            + self.attention_output_bytes + self.mlp_activation_bytes + self.logits_bytes
            + self.argmax_workspace_bytes + self.token_bytes
        )


@dataclass(frozen=True)
class BucketSpec:
    key: str
    prompt_tokens: int
    max_new_tokens: int


@dataclass(frozen=True)
class ResidentBucketPlan:
    key: str
    prompt_tokens: int
    max_new_tokens: int
    max_seq_len: int
    kv_tokens_capacity: int
    kv_cache_bytes: int


@dataclass(frozen=True)
class ResidentBufferPlan:
    geometry: QwenGeometry
    layers: int
    weights_bytes: int
    page_size: int
    batch_size: int
    scratch: ScratchPlan
    buckets: tuple[ResidentBucketPlan, ...]
    entries: tuple[ArenaEntry, ...] = field(default_factory=tuple)
    alignment: int = ARENA_ALIGNMENT

    @property
    def max_kv_cache_bytes(self) -> int:
        return max((b.kv_cache_bytes for b in self.buckets), default=0)

    @property
    def resident_bytes(self) -> int:
        """Payload bytes (before alignment padding), as the reference reports."""
        return self.weights_bytes + self.max_kv_cache_bytes + self.scratch.total_bytes

    @property
    def arena_bytes(self) -> int:
        return max((e.end for e in self.entries), default=0)

    def entry(self, name: str) -> ArenaEntry:
        for e in self.entries:
            if e.name == name:
                return e
        raise KeyError(name)


# The reference's benchmark buckets (src/leanstack/benchmark.py:59-93).
DEFAULT_BUCKETS = (
    BucketSpec("decode_64_256", 64, 256),
    BucketSpec("decode_64_512", 64, 512),
    BucketSpec("prefill_1024_64", 1024, 64),
)


class _Planner:
    def __init__(self, alignment: int) -> None:
        self.alignment = alignment
        self.offset = 0
        self.entries: list[ArenaEntry] = []

    def add(self, name: str, role: str, dtype: torch.dtype, shape: tuple[int, ...], layout: int | None = None) -> None:
        nbytes = _DTYPE_BYTES[dtype]
        for d in shape:
            nbytes *= d
        self.offset = ceil(self.offset / self.alignment) * self.alignment
        self.entries.append(ArenaEntry(name, role, self.offset, nbytes, _DTYPE_NAMES[dtype], tuple(shape), layout))
        self.offset += nbytes


def layer_entry_names(layer: int) -> dict[str, str]:
    p = f"layers.{layer}."
    return {
        "input_layernorm": p + "input_layernorm.weight",
        "qkv_proj": p + "attention.qkv_proj.weight",
        "o_proj": p + "attention.o_proj.weight",
        "q_norm": p + "attention.q_norm.weight",
        "k_norm": p + "attention.k_norm.weight",
        "post_attention_layernorm": p + "post_attention_layernorm.weight",
        "gate_up_proj": p + "mlp.gate_up_proj.weight",
        "down_proj": p + "mlp.down_proj.weight",
    }


def build_resident_buffer_plan(
    geometry: QwenGeometry = QWEN3_4B,
    *,
    layers: int | None = None,
    buckets: Iterable[BucketSpec] = DEFAULT_BUCKETS,
    page_size: int = 16,
    batch_size: int = 1,
    max_rows: int = 16,
    include_embedding: bool = True,
    include_lm_head: bool = True,
    alignment: int = ARENA_ALIGNMENT,
) -> ResidentBufferPlan:
    """Lay out every resident tensor in one arena (offsets aligned to `alignment`).

    `max_rows` is the largest M any projection call carries (16 covers decode
    and speculative verify; a prefill bucket raises it to the prompt length)."""
    g = geometry
    n_layers = g.num_hidden_layers if layers is None else layers
    pl = _Planner(alignment)
    bf16 = torch.bfloat16
    weights = 0
    if include_embedding:
        pl.add("model.embed_tokens.weight", "embedding", bf16, (g.vocab_size, g.hidden_size))
    for layer in range(n_layers):
        names = layer_entry_names(layer)
        proj = g.projections()
        pl.add(names["input_layernorm"], "input_layernorm", bf16, (g.hidden_size,))
        pl.add(names["qkv_proj"], "attention_qkv_fused", bf16, proj["qkv_proj"], _lib.LAYOUT_MFMA16X32)
        pl.add(names["o_proj"], "attention_output_projection", bf16, proj["o_proj"], _lib.LAYOUT_MFMA16X32)
        pl.add(names["q_norm"], "attention_q_norm", bf16, (g.head_dim,))
        pl.add(names["k_norm"], "attention_k_norm", bf16, (g.head_dim,))
        pl.add(names["post_attention_layernorm"], "post_attention_layernorm", bf16, (g.hidden_size,))
        pl.add(names["gate_up_proj"], "mlp_gate_up_fused", bf16, proj["gate_up_proj"], _lib.LAYOUT_MFMA16X32_GATEUP)
        pl.add(names["down_proj"], "mlp_down_projection", bf16, proj["down_proj"], _lib.LAYOUT_MFMA16X32)
    pl.add("model.norm.weight", "final_norm", bf16, (g.hidden_size,))
    if include_lm_head:
        pl.add("lm_head.weight", "lm_head", bf16, (g.vocab_size, g.hidden_size), _lib.LAYOUT_MFMA16X32)
    weights = sum(e.nbytes for e in pl.entries)

    head_rows = min(max_rows, 16)
    lib = _lib.load()
    ws = lib.lsk_workspace_bytes(_lib.OP_LM_HEAD_ARGMAX, head_rows, g.vocab_size, g.hidden_size) if include_lm_head else 0
    scratch = ScratchPlan(
        rows=max_rows,
        hidden_state_bytes=max_rows * g.hidden_size * 2,
        residual_bytes=max_rows * g.hidden_size * 2,
        qkv_projection_bytes=max_rows * g.qkv_dim * 2,
        attention_output_bytes=max_rows * g.q_dim * 2,
        mlp_activation_bytes=max_rows * g.intermediate_size * 2,
        logits_bytes=head_rows * g.vocab_size * 4 if include_lm_head else 0,
        argmax_workspace_bytes=ws,
        token_bytes=head_rows * 8,
    )
    pl.add("scratch.hidden", "scratch", bf16, (max_rows, g.hidden_size))
    pl.add("scratch.residual", "scratch", bf16, (max_rows, g.hidden_size))
    pl.add("scratch.qkv", "scratch", bf16, (max_rows, g.qkv_dim))
    pl.add("scratch.attn", "scratch", bf16, (max_rows, g.q_dim))
    pl.add("scratch.mlp_act", "scratch", bf16, (max_rows, g.intermediate_size))
    if include_lm_head:
        pl.add("scratch.logits", "scratch", torch.float32, (head_rows, g.vocab_size))
        pl.add("scratch.argmax_workspace", "scratch", torch.uint8, (ws,))
    pl.add("scratch.tokens", "scratch", torch.int64, (head_rows,))

    bucket_plans = []
    for b in buckets:
        max_seq = int(b.prompt_tokens) + int(b.max_new_tokens)
        cap = ceil(max_seq / page_size) * page_size
        kv = batch_size * n_layers * 2 * g.num_key_value_heads * g.head_dim * cap * 2
        bucket_plans.append(ResidentBucketPlan(b.key, b.prompt_tokens, b.max_new_tokens, max_seq, cap, kv))
    if bucket_plans:
        cap = max(b.kv_tokens_capacity for b in bucket_plans)
        pl.add("kv_cache", "kv_cache", bf16, (n_layers, 2, batch_size, g.num_key_value_heads, cap, g.head_dim))

    return ResidentBufferPlan(
        geometry=g, layers=n_layers, weights_bytes=weights, page_size=page_size, batch_size=batch_size,
        scratch=scratch, buckets=tuple(bucket_plans), entries=tuple(pl.entries), alignment=alignment,
    )


_TORCH_DTYPES = {v: k for k, v in _DTYPE_NAMES.items()}


class ResidentArena:
    """The allocation behind a ResidentBufferPlan: one device buffer, typed views."""

    def __init__(self, plan: ResidentBufferPlan, device: torch.device | str) -> None:
        self.plan = plan
        self.device = torch.device(device)
        raw = torch.empty(plan.arena_bytes + 256, dtype=torch.uint8, device=self.device)
        skew = (-raw.data_ptr()) % 256  # device allocations are aligned already; host ones may not be
        self.buffer = raw[skew : skew + plan.arena_bytes]
        self._index = {e.name: e for e in plan.entries}
        self.load_stats: dict[str, int] | None = None  # set by the pack loader
        if "scratch.argmax_workspace" in self._index:
            # the greedy head's workspace must start zeroed (each call leaves
            # it so)
            self.view("scratch.argmax_workspace").zero_()

    def weight_names(self) -> set[str]:
        """Entries a pack must fill: everything but scratch and the KV cache."""
        return {e.name for e in self.plan.entries if e.role not in ("scratch", "kv_cache")}

    def view(self, name: str) -> torch.Tensor:
        e = self._index[name]
        raw = self.buffer[e.offset : e.end]
        return raw.view(_TORCH_DTYPES[e.dtype]).view(e.shape)

    def packed(self, name: str) -> PackedWeight:
        e = self._index[name]
        if e.layout is None:
            raise ValueError(f"{name} is not a packed projection weight")
        flat = self.buffer[e.offset : e.end].view(torch.bfloat16)
        n, k = e.shape
        return PackedWeight(flat, n, k, e.layout)

    def store_rowmajor(self, name: str, w: torch.Tensor) -> None:
        """Copy a row-major weight into its entry, packing projection weights."""
        e = self._index[name]
        if tuple(w.shape) != e.shape:
            raise ValueError(f"{name}: shape {tuple(w.shape)} != planned {e.shape}")
        if e.layout is None:
            self.view(name).copy_(w)
        else:
            PackedWeight.from_rowmajor(w.to(self.device, torch.bfloat16), e.layout,
                                       out=self.buffer[e.offset : e.end].view(torch.bfloat16))

    def store_packed(self, name: str, packed: torch.Tensor) -> None:
        e = self._index[name]
        if e.layout is None or packed.dtype != torch.bfloat16 or packed.numel() * 2 != e.nbytes:
            raise ValueError(f"{name}: not a bfloat16 packed entry of {e.nbytes} bytes")
        self.buffer[e.offset : e.end].view(torch.bfloat16).copy_(packed.reshape(-1))


# ----------------------------------------------------------------- loading


def _check_entry_layout(entry: ArenaEntry, layout_name: str, logical_shape) -> None:
    """A pack tensor may fill a planned entry only in the entry's own layout
    and logical shape (a gate_up stored as plain mfma16x32, or a row-major
    tensor where a packed one is planned, is refused)."""
    from .layout import LAYOUT_IDS

    expect = "rowmajor" if entry.layout is None else next(n for n, i in LAYOUT_IDS.items() if i == entry.layout)
    if layout_name != expect:
        raise ValueError(f"{entry.name}: the pack stores layout {layout_name!r}, the plan needs {expect!r}")
    if tuple(logical_shape) != tuple(entry.shape):
        raise ValueError(f"{entry.name}: the pack's shape {list(logical_shape)} != planned {list(entry.shape)}")


# Bytes per read + host-to-device copy when a file region is staged.
LOAD_CHUNK_BYTES = 256 << 20


class _RegionReader:
    """Reads byte ranges of pack files into arena ranges: straight into the
    buffer for a host arena, through two pinned staging buffers (read one
    while the other is copied) for a device arena."""

    def __init__(self, arena: "ResidentArena", largest: int) -> None:
        self.dst = arena.buffer
        self.device = self.dst.device.type == "cuda"
        self.stage, self.done = [], [None, None]
        if self.device:
            size = min(LOAD_CHUNK_BYTES, max(largest, 1))
            self.stage = [torch.empty(size, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        self.reads = 0
        self.copies = 0

    def read(self, path: Path, file_offset: int, nbytes: int, arena_offset: int) -> None:
        with open(path, "rb", buffering=0) as f:
            f.seek(file_offset)
            if not self.device:
                got = f.readinto(memoryview(self.dst[arena_offset : arena_offset + nbytes].numpy()))
                if got != nbytes:
                    raise ValueError(f"{path}: {got} of {nbytes} bytes at offset {file_offset} (truncated file)")
                self.reads += 1
                self.copies += 1
                return
            done, i = 0, 0
            while done < nbytes:
                n = min(len(self.stage[0]), nbytes - done)
                slot = i % 2
                if self.done[slot] is not None:
                    self.done[slot].synchronize()
                got = f.readinto(memoryview(self.stage[slot].numpy())[:n])
                if got != n:
                    raise ValueError(f"{path}: {done + got} of {nbytes} bytes at offset {file_offset} (truncated file)")
                # The copy and its event on the arena device's stream, so the
                # event covers the copy whichever device is current.
                stream = torch.cuda.current_stream(self.dst.device)
                with torch.cuda.stream(stream):
                    self.dst[arena_offset + done : arena_offset + done + n].copy_(self.stage[slot][:n],
                                                                                  non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(stream)
                self.done[slot] = ev
                done += n
                i += 1
                self.copies += 1
            self.reads += 1

    def finish(self) -> None:
        for ev in self.done:
            if ev is not None:
                ev.synchronize()


def _safetensors_data_offsets(path: Path) -> dict[str, tuple[int, int]]:
    """Absolute byte range of every tensor in a safetensors file, read from
    its header (8-byte little-endian header length, JSON header whose
    `data_offsets` are relative to the data region that follows it)."""
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise ValueError(f"{path}: truncated (no safetensors header)")
        (hlen,) = struct.unpack("<Q", head)
        raw = f.read(hlen)
    if len(raw) != hlen:
        raise ValueError(f"{path}: truncated safetensors header")
    header = json.loads(raw)
    base = 8 + hlen
    return {name: (base + int(v["data_offsets"][0]), base + int(v["data_offsets"][1]))
            for name, v in header.items() if name != "__metadata__"}


def load_pack_into_arena(root: Path, manifest, arena: "ResidentArena") -> dict[str, int]:
    """Fill every planned weight of `arena` from the pack at `root` by
    direct file offsets.  A file whose tensors sit at the same relative
    offsets as their arena entries (the layout the packer writes) is one
    read and one copy of its whole data region; any other file is one read
    of its region with a copy per tensor.  Refuses a pack that misses a
    planned weight or stores one in another layout or size.  Returns load
    statistics: files, bulk (files loaded as one image), per_tensor (tensors
    copied one by one), bytes."""
    plan = arena.plan
    planned = arena.weight_names()
    by_file: dict[str, list] = {}
    for t in manifest.tensors:
        if t.name in planned:
            e = plan.entry(t.name)
            _check_entry_layout(e, t.layout, t.logical_shape)
            if t.size_bytes != e.nbytes:
                raise ValueError(f"{t.name}: the pack stores {t.size_bytes} bytes, the plan needs {e.nbytes}")
            by_file.setdefault(t.file, []).append(t)
    missing = sorted(planned - {t.name for ts in by_file.values() for t in ts})
    if missing:
        raise ValueError(f"{root}: the pack has no tensor for {len(missing)} planned weights, e.g. {missing[:3]}")
    # The manifest's offsets must name the bytes the safetensors header
    # itself gives each tensor: a wrong offset would load another tensor's
    # bytes (or the header) with every size check still passing.
    for file_name, ts in by_file.items():
        ranges = _safetensors_data_offsets(root / file_name)
        for t in ts:
            if t.name not in ranges:
                raise ValueError(f"{root / file_name}: no tensor {t.name} in the safetensors header")
            lo, hi = ranges[t.name]
            if (lo, hi - lo) != (t.file_offset_bytes, t.size_bytes):
                raise ValueError(f"{t.name}: the manifest places it at file offset {t.file_offset_bytes} "
                                 f"({t.size_bytes} bytes), the safetensors header at {lo} ({hi - lo} bytes)")
    largest = max(ts[-1].file_offset_bytes + ts[-1].size_bytes - ts[0].file_offset_bytes
                  for ts in (sorted(v, key=lambda t: t.file_offset_bytes) for v in by_file.values()))
    reader = _RegionReader(arena, largest)
    stats = {"files": 0, "bulk": 0, "per_tensor": 0, "bytes": 0}
    for file_name, ts in by_file.items():
        ts = sorted(ts, key=lambda t: t.file_offset_bytes)
        f0, a0 = ts[0].file_offset_bytes, plan.entry(ts[0].name).offset
        span = ts[-1].file_offset_bytes + ts[-1].size_bytes - f0
        inside = {e.name for e in plan.entries if e.offset < a0 + span and e.end > a0}
        image = inside == {t.name for t in ts} and all(
            t.file_offset_bytes - f0 == plan.entry(t.name).offset - a0 for t in ts)
        if image:
            reader.read(root / file_name, f0, span, a0)
            stats["bulk"] += 1
        else:
            for t in ts:
                reader.read(root / file_name, t.file_offset_bytes, t.size_bytes, plan.entry(t.name).offset)
            stats["per_tensor"] += len(ts)
        stats["files"] += 1
        stats["bytes"] += sum(t.size_bytes for t in ts)
    reader.finish()
    return stats


def materialize_qwen_semantic_stack_from_leanpack(
    pack_dir: str | Path,
    *,
    device: str | torch.device = "cuda:0",
    include_output_head: bool = True,
    max_rows: int = 16,
    buckets: Iterable[BucketSpec] | None = None,
):
    """Load a leanpack/v1 artifact into one resident arena and build the
    runtime (replaces src/leanstack/leanserve.py:470-530, which copies each
    tensor to its own allocation).  The KV cache is sized for the manifest's
    buckets (as the reference's planner reads them, leanserve.py:199-202,
    :331-377) unless `buckets` is given.  Returns (runtime, arena); the
    arena's `load_stats` records how the files were read."""
    from .pack import geometry_from_manifest, load_packed_artifact_manifest
    from .runtime import (
        QwenSemanticAttentionRuntime,
        QwenSemanticLayerRuntime,
        QwenSemanticMlpRuntime,
        QwenSemanticStackRuntime,
        QwenServeConfig,
        split_rows,
    )

    root = Path(pack_dir)
    manifest = load_packed_artifact_manifest(root)
    g = geometry_from_manifest(manifest)
    if buckets is None:
        buckets = [BucketSpec(b.key, b.prompt_tokens, b.max_new_tokens) for b in manifest.buckets]
    plan = build_resident_buffer_plan(g, buckets=buckets, max_rows=max_rows, include_lm_head=include_output_head)
    arena = ResidentArena(plan, device)
    arena.load_stats = load_pack_into_arena(root, manifest, arena)

    cfg = QwenServeConfig(
        vocab_size=g.vocab_size, hidden_size=g.hidden_size, intermediate_size=g.intermediate_size,
        num_hidden_layers=g.num_hidden_layers, num_attention_heads=g.num_attention_heads,
        num_key_value_heads=g.num_key_value_heads, max_position_embeddings=g.max_position_embeddings,
        head_dim=g.head_dim, rms_norm_eps=g.rms_norm_eps, rope_parameters={"rope_theta": g.rope_theta},
    )
    layers = []
    for layer in range(g.num_hidden_layers):
        n = layer_entry_names(layer)
        qkv = arena.packed(n["qkv_proj"])
        q, k, v = split_rows(qkv, (g.q_dim, g.kv_dim, g.kv_dim))
        attention = QwenSemanticAttentionRuntime(
            layer_idx=layer, q_proj_weight=q, k_proj_weight=k, v_proj_weight=v, qkv_proj_weight=qkv,
            q_proj_out_dim=g.q_dim, k_proj_out_dim=g.kv_dim, num_attention_heads=g.num_attention_heads,
            num_key_value_heads=g.num_key_value_heads,
            num_key_value_groups=g.num_attention_heads // g.num_key_value_heads, head_dim=g.head_dim,
            attention_scale=g.head_dim ** -0.5, o_proj_weight=arena.packed(n["o_proj"]),
            q_norm_weight=arena.view(n["q_norm"]), k_norm_weight=arena.view(n["k_norm"]),
        )
        mlp = QwenSemanticMlpRuntime(gate_up_proj_weight=arena.packed(n["gate_up_proj"]),
                                     gate_proj_out_dim=g.intermediate_size,
                                     down_proj_weight=arena.packed(n["down_proj"]))
        layers.append(QwenSemanticLayerRuntime(
            layer_idx=layer, input_layernorm_weight=arena.view(n["input_layernorm"]), attention=attention,
            post_attention_layernorm_weight=arena.view(n["post_attention_layernorm"]), mlp=mlp))
    dev = torch.device(device)
    inv_freq = 1.0 / (g.rope_theta ** (torch.arange(0, g.head_dim, 2, device=dev, dtype=torch.float32) / g.head_dim))
    runtime = QwenSemanticStackRuntime(
        model_path=root, config=cfg, layer_indices=tuple(range(g.num_hidden_layers)),
        embed_tokens_weight=arena.view("model.embed_tokens.weight"), layers=tuple(layers),
        rope_inv_freq=inv_freq, attention_scaling=1.0,
        final_norm_weight=arena.view("model.norm.weight") if include_output_head else None,
        lm_head_weight=arena.packed("lm_head.weight") if include_output_head else None,
        device=dev, dtype=torch.bfloat16,
    )
    return runtime, arena
