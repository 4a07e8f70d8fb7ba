"""leanpack/v1: the offline packed artifact in the MI355X tile layout.

The reference's packer (src/leanstack/pack.py:226-375, format leanpack/v0)
writes row-major fused tensors per layer -- qkv_proj = cat(q, k, v) and
gate_up_proj = cat(gate, up) (:269-286) -- plus a separate lm_head copy
(:318-323) and a manifest.  leanpack/v1 keeps the same file split and
manifest fields (so the reference's manifest readers still find geometry,
buckets, files and tensors) and changes three things:

  - Projection tensors are stored as the flat 1-D bf16 tensor of their packed
    layout (include/leanstack_amd.h), with the logical [N, K] shape and the
    layout name recorded per tensor.  The lm_head copy is stored packed too:
    the row-major embedding serves the token gather, the packed copy the
    greedy head, so the reference's duplicate becomes a useful one.
  - Direct offset loading (the format doc's missing "mmap-style offset
    loading", docs/LEANPACK_FORMAT.md:73-78): every file is still a valid
    safetensors file, but each tensor's data starts at a 4096-byte aligned
    file offset, recorded in the manifest (`file_offset_bytes`), and the
    tensors of a file follow the resident arena's order and alignment, so a
    file's data region is a byte image of a contiguous arena range.  The
    loader reads it once and copies it to the device once, straight into the
    arena; gaps are filled by zero `__pad__` tensors, which keeps the
    safetensors byte buffer free of holes.
  - A manifest `layout` section names the tile geometry and the target GPU;
    loaders refuse an unknown format or layout.
"""

from __future__ import annotations

import json
import struct
from dataclasses import asdict, dataclass, field
from datetime import datetime, timezone
from pathlib import Path
from typing import Any, Mapping

import torch

from . import _lib
from .geometry import QWEN3_4B, QwenGeometry
from .layout import LAYOUT_NAMES, TILE_BYTES, TILE_K, TILE_ROWS, pack_tensor

FORMAT_VERSION = "leanpack/v1"
TARGET_GPU = "MI355X / gfx950"

LAYOUT_SECTION = {
    "tile_rows": TILE_ROWS,
    "tile_k": TILE_K,
    "tile_bytes": TILE_BYTES,
    "lane_order": "lane l of tile (rb, kt) holds W[16*rb + l%16, 32*kt + 8*(l//16) : +8]",
    "gate_up_interleave_rows": TILE_ROWS,
    "layouts": {name: layout for layout, name in LAYOUT_NAMES.items()},
    "target_gpu": TARGET_GPU,
}


# Alignment of every tensor's data in a pack file: the resident arena's entry
# alignment (leanserve.ARENA_ALIGNMENT), so that a file's data region and its
# arena range have the same layout.
FILE_ALIGNMENT = 4096


@dataclass(frozen=True)
class PackedTensorEntry:
    name: str
    role: str
    file: str
    dtype: str
    shape: list[int]            # stored shape (1-D for packed projections)
    logical_shape: list[int]    # [N, K] of the weight as the model uses it
    layout: str                 # "rowmajor" or a packed layout name
    numel: int
    logical_offset_bytes: int   # offset inside the file's data region (aligned)
    size_bytes: int
    source_tensors: list[str]
    file_offset_bytes: int      # absolute byte offset of the data in the file (FILE_ALIGNMENT aligned)


@dataclass(frozen=True)
class PackedFileEntry:
    file: str
    tensor_count: int
    size_bytes: int
    data_offset_bytes: int = 0  # where the (aligned) data region starts in the file
    data_bytes: int = 0         # length of the data region, padding included


# Manifest metadata of the reference's leanpack (src/leanstack/pack.py:64-100).
@dataclass(frozen=True)
class BucketEntry:
    key: str
    prompt_tokens: int
    max_new_tokens: int


@dataclass(frozen=True)
class SpeculativeModeEntry:
    key: str
    draft_layer_count: int
    proposal_len: int


@dataclass(frozen=True)
class DraftHeadEntry:
    key: str
    draft_layer_count: int
    file: str
    tensor_name: str
    input_size: int
    output_size: int
    fit_samples: int
    ridge_lambda: float


# The Qwen3-4B contract's exact prompt buckets and the benchmark buckets built
# on them (src/leanstack/model_registry.py:37, src/leanstack/benchmark.py:
# 59-93), and the speculative modes the reference records (pack.py:178-193:
# a 12-layer draft proposing 4 or 2 tokens).
QWEN_EXACT_PROMPT_BUCKETS = (64, 512, 1024)
QWEN_BUCKETS = (
    BucketEntry("decode_64_256", 64, 256),
    BucketEntry("decode_64_512", 64, 512),
    BucketEntry("prefill_1024_64", 1024, 64),
)

# The kernels a runtime on this pack needs: the C-ABI entry points of
# libleanstack_amd.so that the dispatch calls.
REQUIRED_KERNELS = (
    "lsk_linear_bf16",
    "lsk_rmsnorm_linear_bf16",
    "lsk_decode_attention_at_bf16",
    "lsk_lm_head_argmax_bf16",
    "lsk_rmsnorm_lm_head_argmax_bf16",
)
BACKEND_POLICY = (
    "Every projection, the decode attention step and the greedy head run on hand-written HIP kernels for gfx950 "
    "behind the C ABI of libleanstack_amd.so.",
    "No torch.compile, Triton or library GEMM on the hot path; a missing library or a rejected argument raises "
    "instead of falling back.",
    "Weights stay resident in one device arena in the packed mfma16x32 layouts recorded per tensor.",
)


def speculative_modes(num_hidden_layers: int) -> list[SpeculativeModeEntry]:
    draft = min(12, max(num_hidden_layers - 1, 1))
    return [SpeculativeModeEntry("draft12_k4", draft, 4), SpeculativeModeEntry("draft12_k2", draft, 2)]


@dataclass(frozen=True)
class PackedArtifactManifest:
    format_version: str
    created_at_utc: str
    model_key: str
    semantic_model_id: str | None
    source_model_path: str
    target_gpu: str
    dtype: str
    geometry: dict[str, int]
    model_hparams: dict[str, Any]
    layout: dict[str, Any]
    exact_prompt_buckets: list[int] = field(default_factory=list)
    buckets: list[BucketEntry] = field(default_factory=list)
    speculative_modes: list[SpeculativeModeEntry] = field(default_factory=list)
    draft_heads: list[DraftHeadEntry] = field(default_factory=list)
    required_kernels: list[str] = field(default_factory=list)
    backend_policy: list[str] = field(default_factory=list)
    files: list[PackedFileEntry] = field(default_factory=list)
    tensors: list[PackedTensorEntry] = field(default_factory=list)

    def as_payload(self) -> dict[str, Any]:
        payload = asdict(self)
        return payload

    @classmethod
    def from_payload(cls, payload: dict[str, Any]) -> "PackedArtifactManifest":
        return cls(
            format_version=payload["format_version"],
            created_at_utc=payload["created_at_utc"],
            model_key=payload["model_key"],
            semantic_model_id=payload.get("semantic_model_id"),
            source_model_path=payload.get("source_model_path", ""),
            target_gpu=payload.get("target_gpu", ""),
            dtype=payload["dtype"],
            geometry=dict(payload.get("geometry", {})),
            model_hparams=dict(payload.get("model_hparams", {})),
            layout=dict(payload.get("layout", {})),
            exact_prompt_buckets=[int(b) for b in payload.get("exact_prompt_buckets", [])],
            buckets=[BucketEntry(**b) for b in payload.get("buckets", [])],
            speculative_modes=[SpeculativeModeEntry(**m) for m in payload.get("speculative_modes", [])],
            draft_heads=[DraftHeadEntry(**h) for h in payload.get("draft_heads", [])],
            required_kernels=list(payload.get("required_kernels", [])),
            backend_policy=list(payload.get("backend_policy", [])),
            files=[PackedFileEntry(**f) for f in payload.get("files", [])],
            tensors=[PackedTensorEntry(**t) for t in payload.get("tensors", [])],
        )

    def tensor(self, name: str) -> PackedTensorEntry:
        for t in self.tensors:
            if t.name == name:
                return t
        raise KeyError(name)


def load_packed_artifact_manifest(path_or_dir: str | Path) -> PackedArtifactManifest:
    """Read and validate a leanpack/v1 manifest (ValueError on a v0 or unknown
    format, or on a layout this library does not implement)."""
    path = Path(path_or_dir)
    if path.is_dir():
        path = path / "manifest.json"
    payload = json.loads(path.read_text(encoding="utf-8"))
    fmt = payload.get("format_version")
    if fmt != FORMAT_VERSION:
        raise ValueError(f"{path}: format {fmt!r} is not {FORMAT_VERSION} (repack the checkpoint with this packer)")
    for t in payload.get("tensors", []):
        # An early leanpack/v1 writer left this field out; the loader reads
        # every tensor at this offset, so a manifest without it is refused.
        if not isinstance(t.get("file_offset_bytes"), int) or t["file_offset_bytes"] < 0:
            raise ValueError(f"{path}: tensor {t.get('name')!r} has no file_offset_bytes "
                             f"(written by an older packer; repack the checkpoint with this packer)")
    manifest = PackedArtifactManifest.from_payload(payload)
    known = set(LAYOUT_NAMES.values()) | {"rowmajor"}
    for t in manifest.tensors:
        if t.layout not in known:
            raise ValueError(f"{path}: tensor {t.name} uses unknown layout {t.layout!r}")
    if manifest.layout.get("tile_rows") != TILE_ROWS or manifest.layout.get("tile_k") != TILE_K:
        raise ValueError(f"{path}: tile geometry {manifest.layout} does not match {TILE_ROWS}x{TILE_K}")
    return manifest


def geometry_from_manifest(manifest: PackedArtifactManifest) -> QwenGeometry:
    g = manifest.geometry
    h = manifest.model_hparams
    return QwenGeometry(
        num_hidden_layers=int(g["num_hidden_layers"]), hidden_size=int(g["hidden_size"]),
        intermediate_size=int(g["intermediate_size"]), num_attention_heads=int(g["num_attention_heads"]),
        num_key_value_heads=int(g["num_key_value_heads"]), head_dim=int(g["head_dim"]),
        vocab_size=int(g["vocab_size"]), max_position_embeddings=int(g.get("max_position_embeddings", 32768)),
        rms_norm_eps=float(h.get("rms_norm_eps", 1e-6)), rope_theta=float(h.get("rope_theta", 1_000_000.0)),
    )


def hf_layer_names(layer: int) -> dict[str, str]:
    p = f"model.layers.{layer}."
    return {
        "input_layernorm": p + "input_layernorm.weight",
        "q_proj": p + "self_attn.q_proj.weight",
        "k_proj": p + "self_attn.k_proj.weight",
        "v_proj": p + "self_attn.v_proj.weight",
        "o_proj": p + "self_attn.o_proj.weight",
        "q_norm": p + "self_attn.q_norm.weight",
        "k_norm": p + "self_attn.k_norm.weight",
        "post_attention_layernorm": p + "post_attention_layernorm.weight",
        "gate_proj": p + "mlp.gate_proj.weight",
        "up_proj": p + "mlp.up_proj.weight",
        "down_proj": p + "mlp.down_proj.weight",
    }


def synthetic_qwen_checkpoint(geometry: QwenGeometry = QWEN3_4B, *, seed: int = 0,
                              std: float = 0.02) -> dict[str, torch.Tensor]:
    """A random checkpoint with the Hugging Face tensor names of a Qwen3
    model (no network or real weights here): projections N(0, std^2), norms
    1 + N(0, 0.01).  CPU bf16 tensors."""
    g = geometry
    gen = torch.Generator(device="cpu").manual_seed(seed)

    def w(n, k):
        return (torch.randn(n, k, generator=gen) * std).to(torch.bfloat16)

    def norm(n):
        return (1 + 0.01 * torch.randn(n, generator=gen)).to(torch.bfloat16)

    out = {"model.embed_tokens.weight": w(g.vocab_size, g.hidden_size), "model.norm.weight": norm(g.hidden_size)}
    for layer in range(g.num_hidden_layers):
        n = hf_layer_names(layer)
        out[n["input_layernorm"]] = norm(g.hidden_size)
        out[n["q_proj"]] = w(g.q_dim, g.hidden_size)
        out[n["k_proj"]] = w(g.kv_dim, g.hidden_size)
        out[n["v_proj"]] = w(g.kv_dim, g.hidden_size)
        out[n["o_proj"]] = w(g.hidden_size, g.q_dim)
        out[n["q_norm"]] = norm(g.head_dim)
        out[n["k_norm"]] = norm(g.head_dim)
        out[n["post_attention_layernorm"]] = norm(g.hidden_size)
        out[n["gate_proj"]] = w(g.intermediate_size, g.hidden_size)
        out[n["up_proj"]] = w(g.intermediate_size, g.hidden_size)
        out[n["down_proj"]] = w(g.hidden_size, g.intermediate_size)
    return out


_ST_DTYPES = {torch.bfloat16: "BF16", torch.float32: "F32", torch.uint8: "U8"}


def _align(n: int) -> int:
    return -(-n // FILE_ALIGNMENT) * FILE_ALIGNMENT


def write_aligned_safetensors(path: Path, tensors: dict[str, torch.Tensor]) -> tuple[int, int, dict[str, int]]:
    """Write `tensors` (in this order) as a safetensors file whose data
    region starts at a FILE_ALIGNMENT boundary and in which every tensor's
    data starts at a FILE_ALIGNMENT offset from it, the gaps filled by zero
    `__pad__.<i>` uint8 tensors (the format requires a byte buffer without
    holes).  The header is padded with spaces, which the format allows.
    Returns (data_offset, data_bytes, {name: offset inside the data region})."""
    header: dict[str, Any] = {"__metadata__": {"format": "pt", "layout": FORMAT_VERSION}}
    offsets: dict[str, int] = {}
    pads: list[tuple[int, int]] = []
    pos = 0
    for i, (name, t) in enumerate(tensors.items()):
        if t.dtype not in _ST_DTYPES:
            raise ValueError(f"{name}: dtype {t.dtype} is not stored by leanpack")
        start = _align(pos)
        if start > pos:
            header[f"__pad__.{i}"] = {"dtype": "U8", "shape": [start - pos], "data_offsets": [pos, start]}
            pads.append((pos, start))
        size = t.numel() * t.element_size()
        header[name] = {"dtype": _ST_DTYPES[t.dtype], "shape": list(t.shape), "data_offsets": [start, start + size]}
        offsets[name] = start
        pos = start + size
    raw = json.dumps(header, separators=(",", ":")).encode("utf-8")
    data_offset = _align(8 + len(raw))
    raw += b" " * (data_offset - 8 - len(raw))
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        end = 0
        for name, t in tensors.items():
            start = offsets[name]
            if start > end:
                f.write(bytes(start - end))
            f.write(t.detach().contiguous().cpu().view(torch.uint8).numpy().tobytes())
            end = start + t.numel() * t.element_size()
    return data_offset, pos, offsets


def _entries(file_name: str, tensors: dict[str, torch.Tensor], meta: dict[str, tuple], data_offset: int,
             offsets: dict[str, int]) -> list[PackedTensorEntry]:
    entries = []
    for name, t in tensors.items():
        role, logical, layout, sources = meta[name]
        entries.append(PackedTensorEntry(
            name=name, role=role, file=file_name, dtype=str(t.dtype).removeprefix("torch."), shape=list(t.shape),
            logical_shape=list(logical), layout=layout, numel=t.numel(), logical_offset_bytes=offsets[name],
            size_bytes=t.numel() * t.element_size(), source_tensors=list(sources),
            file_offset_bytes=data_offset + offsets[name]))
    return entries


def build_qwen_leanpack(tensors: Mapping[str, torch.Tensor], output_dir: str | Path, *,
                        geometry: QwenGeometry = QWEN3_4B, model_key: str = "qwen",
                        semantic_model_id: str | None = "Qwen/Qwen3-4B-Base", source_model_path: str = "",
                        overwrite: bool = False, exact_prompt_buckets=QWEN_EXACT_PROMPT_BUCKETS,
                        buckets=QWEN_BUCKETS) -> PackedArtifactManifest:
    """Pack a Qwen3 checkpoint (Hugging Face tensor names, row-major) into
    leanpack/v1 at output_dir.  `buckets` are recorded in the manifest and
    size the loader's KV cache (BucketEntry list)."""
    g = geometry
    root = Path(output_dir)
    if root.exists() and any(root.iterdir()) and not overwrite:
        raise FileExistsError(f"output_dir already exists: {root}")
    root.mkdir(parents=True, exist_ok=True)
    files: list[PackedFileEntry] = []
    entries: list[PackedTensorEntry] = []
    rowmajor, mfma, gateup = "rowmajor", LAYOUT_NAMES[_lib.LAYOUT_MFMA16X32], LAYOUT_NAMES[_lib.LAYOUT_MFMA16X32_GATEUP]

    def write(file_name: str, group: dict[str, torch.Tensor], meta: dict[str, tuple]) -> None:
        group = {k: v.contiguous() for k, v in group.items()}
        data_offset, data_bytes, offsets = write_aligned_safetensors(root / file_name, group)
        files.append(PackedFileEntry(file_name, len(group), (root / file_name).stat().st_size, data_offset,
                                     data_bytes))
        entries.extend(_entries(file_name, group, meta, data_offset, offsets))

    embed = tensors["model.embed_tokens.weight"].to(torch.bfloat16)
    write("embeddings.safetensors", {"model.embed_tokens.weight": embed},
          {"model.embed_tokens.weight": ("embedding", embed.shape, rowmajor, ["model.embed_tokens.weight"])})

    for layer in range(g.num_hidden_layers):
        n = hf_layer_names(layer)
        p = f"layers.{layer}."
        qkv = torch.cat((tensors[n["q_proj"]], tensors[n["k_proj"]], tensors[n["v_proj"]]), dim=0).to(torch.bfloat16)
        gate_up = torch.cat((tensors[n["gate_proj"]], tensors[n["up_proj"]]), dim=0).to(torch.bfloat16)
        o = tensors[n["o_proj"]].to(torch.bfloat16)
        down = tensors[n["down_proj"]].to(torch.bfloat16)
        group = {
            p + "input_layernorm.weight": tensors[n["input_layernorm"]].to(torch.bfloat16),
            p + "attention.qkv_proj.weight": pack_tensor(qkv, _lib.LAYOUT_MFMA16X32),
            p + "attention.o_proj.weight": pack_tensor(o, _lib.LAYOUT_MFMA16X32),
            p + "attention.q_norm.weight": tensors[n["q_norm"]].to(torch.bfloat16),
            p + "attention.k_norm.weight": tensors[n["k_norm"]].to(torch.bfloat16),
            p + "post_attention_layernorm.weight": tensors[n["post_attention_layernorm"]].to(torch.bfloat16),
            p + "mlp.gate_up_proj.weight": pack_tensor(gate_up, _lib.LAYOUT_MFMA16X32_GATEUP),
            p + "mlp.down_proj.weight": pack_tensor(down, _lib.LAYOUT_MFMA16X32),
        }
        meta = {
            p + "input_layernorm.weight": ("input_layernorm", [g.hidden_size], rowmajor, [n["input_layernorm"]]),
            p + "attention.qkv_proj.weight": ("attention_qkv_fused", qkv.shape, mfma,
                                              [n["q_proj"], n["k_proj"], n["v_proj"]]),
            p + "attention.o_proj.weight": ("attention_output_projection", o.shape, mfma, [n["o_proj"]]),
            p + "attention.q_norm.weight": ("attention_q_norm", [g.head_dim], rowmajor, [n["q_norm"]]),
            p + "attention.k_norm.weight": ("attention_k_norm", [g.head_dim], rowmajor, [n["k_norm"]]),
            p + "post_attention_layernorm.weight": ("post_attention_layernorm", [g.hidden_size], rowmajor,
                                                    [n["post_attention_layernorm"]]),
            p + "mlp.gate_up_proj.weight": ("mlp_gate_up_fused", gate_up.shape, gateup,
                                            [n["gate_proj"], n["up_proj"]]),
            p + "mlp.down_proj.weight": ("mlp_down_projection", down.shape, mfma, [n["down_proj"]]),
        }
        write(f"layer-{layer:03d}.safetensors", group, meta)

    head_src = "lm_head.weight" if "lm_head.weight" in tensors else "model.embed_tokens.weight"
    head = tensors[head_src].to(torch.bfloat16)
    write("output.safetensors",
          {"model.norm.weight": tensors["model.norm.weight"].to(torch.bfloat16),
           "lm_head.weight": pack_tensor(head, _lib.LAYOUT_MFMA16X32)},
          {"model.norm.weight": ("final_norm", [g.hidden_size], rowmajor, ["model.norm.weight"]),
           "lm_head.weight": ("lm_head", head.shape, mfma, [head_src])})

    manifest = PackedArtifactManifest(
        format_version=FORMAT_VERSION,
        created_at_utc=datetime.now(timezone.utc).isoformat(),
        model_key=model_key,
        semantic_model_id=semantic_model_id,
        source_model_path=source_model_path,
        target_gpu=TARGET_GPU,
        dtype="bfloat16",
        geometry={
            "num_hidden_layers": g.num_hidden_layers, "hidden_size": g.hidden_size,
            "intermediate_size": g.intermediate_size, "num_attention_heads": g.num_attention_heads,
            "num_key_value_heads": g.num_key_value_heads, "head_dim": g.head_dim, "vocab_size": g.vocab_size,
            "max_position_embeddings": g.max_position_embeddings,
        },
        model_hparams={"rms_norm_eps": g.rms_norm_eps, "rope_theta": g.rope_theta},
        layout=dict(LAYOUT_SECTION),
        exact_prompt_buckets=list(exact_prompt_buckets),
        buckets=list(buckets),
        speculative_modes=speculative_modes(g.num_hidden_layers),
        draft_heads=[],
        required_kernels=list(REQUIRED_KERNELS),
        backend_policy=list(BACKEND_POLICY),
        files=files,
        tensors=entries,
    )
    (root / "manifest.json").write_text(json.dumps(manifest.as_payload(), indent=2) + "\n", encoding="utf-8")
    return manifest
