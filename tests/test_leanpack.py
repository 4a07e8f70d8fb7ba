"""leanpack/v1: pack a synthetic Qwen3 checkpoint, validate the manifest, and
materialize it into the resident arena (CPU here; the GPU variant runs the
dispatch entry points on a real-shape layer)."""

from __future__ import annotations

import json

import pytest
import torch

from leanstack_amd import _lib
from leanstack_amd.geometry import QwenGeometry
from leanstack_amd.leanserve import materialize_qwen_semantic_stack_from_leanpack
from leanstack_amd.pack import (
    FORMAT_VERSION,
    build_qwen_leanpack,
    hf_layer_names,
    load_packed_artifact_manifest,
    synthetic_qwen_checkpoint,
)

TINY = QwenGeometry(num_hidden_layers=2, hidden_size=256, intermediate_size=512, num_attention_heads=4,
                    num_key_value_heads=2, head_dim=64, vocab_size=1024)


@pytest.fixture(scope="module")
def tiny_pack(tmp_path_factory):
    ckpt = synthetic_qwen_checkpoint(TINY, seed=3)
    out = tmp_path_factory.mktemp("pack")
    manifest = build_qwen_leanpack(ckpt, out, geometry=TINY)
    return ckpt, out, manifest


def test_manifest_layout_and_geometry(tiny_pack):
    _, out, manifest = tiny_pack
    assert manifest.format_version == FORMAT_VERSION
    assert manifest.layout["tile_rows"] == 16 and manifest.layout["tile_k"] == 32
    assert manifest.layout["target_gpu"].startswith("MI355X")
    assert manifest.geometry["num_hidden_layers"] == 2
    assert [f.file for f in manifest.files] == ["embeddings.safetensors", "layer-000.safetensors",
                                                "layer-001.safetensors", "output.safetensors"]
    t = manifest.tensor("layers.1.attention.qkv_proj.weight")
    assert t.layout == "mfma16x32" and t.logical_shape == [512, 256] and t.shape == [512 * 256]
    assert t.source_tensors == ["model.layers.1.self_attn.q_proj.weight", "model.layers.1.self_attn.k_proj.weight",
                                "model.layers.1.self_attn.v_proj.weight"]
    assert manifest.tensor("layers.0.mlp.gate_up_proj.weight").layout == "mfma16x32_gateup"
    assert manifest.tensor("lm_head.weight").source_tensors == ["model.embed_tokens.weight"]  # tied head
    reread = load_packed_artifact_manifest(out)
    assert reread.tensors == manifest.tensors


def test_loader_refuses_other_formats(tiny_pack, tmp_path):
    _, out, _ = tiny_pack
    payload = json.loads((out / "manifest.json").read_text())
    bad = tmp_path / "v0"
    bad.mkdir()
    (bad / "manifest.json").write_text(json.dumps(dict(payload, format_version="leanpack/v0")))
    with pytest.raises(ValueError):
        load_packed_artifact_manifest(bad)
    payload["tensors"][1]["layout"] = "tiles64x64"
    (bad / "manifest.json").write_text(json.dumps(payload))
    with pytest.raises(ValueError):
        load_packed_artifact_manifest(bad)


def test_materialize_round_trips_every_tensor(tiny_pack):
    ckpt, out, _ = tiny_pack
    runtime, arena = materialize_qwen_semantic_stack_from_leanpack(out, device="cpu", buckets=())
    assert torch.equal(runtime.embed_tokens_weight, ckpt["model.embed_tokens.weight"])
    assert torch.equal(runtime.lm_head_weight.unpack(), ckpt["model.embed_tokens.weight"])
    for layer, lr in enumerate(runtime.layers):
        n = hf_layer_names(layer)
        att, mlp = lr.attention, lr.mlp
        assert torch.equal(att.q_proj_weight.unpack(), ckpt[n["q_proj"]])
        assert torch.equal(att.k_proj_weight.unpack(), ckpt[n["k_proj"]])
        assert torch.equal(att.v_proj_weight.unpack(), ckpt[n["v_proj"]])
        assert torch.equal(att.o_proj_weight.unpack(), ckpt[n["o_proj"]])
        fused = torch.cat((ckpt[n["gate_proj"]], ckpt[n["up_proj"]]))
        assert torch.equal(mlp.gate_up_proj_weight.unpack(), fused)
        assert mlp.gate_up_proj_weight.layout == _lib.LAYOUT_MFMA16X32_GATEUP
        assert torch.equal(mlp.down_proj_weight.unpack(), ckpt[n["down_proj"]])
        assert torch.equal(lr.input_layernorm_weight, ckpt[n["input_layernorm"]])
        assert torch.equal(att.k_norm_weight, ckpt[n["k_norm"]])
        # views share the arena: one allocation holds everything
        assert att.qkv_proj_weight.data.untyped_storage().data_ptr() == arena.buffer.untyped_storage().data_ptr()
    assert runtime.config.num_key_value_heads == 2 and runtime.layers[0].attention.num_key_value_groups == 2


def test_files_are_aligned_safetensors(tiny_pack):
    """Every file opens with safetensors and holds the packed tensors; each
    tensor's data starts at a 4096-byte file offset that the manifest
    records, and reading those bytes at that offset gives the tensor."""
    from safetensors import safe_open

    from leanstack_amd.layout import pack_tensor

    ckpt, out, manifest = tiny_pack
    expect = {"model.embed_tokens.weight": ckpt["model.embed_tokens.weight"],
              "layers.1.attention.o_proj.weight": pack_tensor(ckpt[hf_layer_names(1)["o_proj"]], _lib.LAYOUT_MFMA16X32),
              "layers.0.input_layernorm.weight": ckpt[hf_layer_names(0)["input_layernorm"]]}
    for t in manifest.tensors:
        assert t.file_offset_bytes % 4096 == 0 and t.logical_offset_bytes % 4096 == 0
        with safe_open(str(out / t.file), framework="pt") as f:
            stored = f.get_tensor(t.name)
        assert list(stored.shape) == t.shape and stored.numel() * 2 == t.size_bytes
        raw = (out / t.file).read_bytes()[t.file_offset_bytes : t.file_offset_bytes + t.size_bytes]
        assert raw == stored.contiguous().view(torch.uint8).numpy().tobytes()
        if t.name in expect:
            assert torch.equal(stored.view(torch.int16), expect[t.name].reshape(stored.shape).view(torch.int16))
    for fe in manifest.files:
        assert fe.data_offset_bytes % 4096 == 0 and fe.size_bytes == (out / fe.file).stat().st_size


def test_manifest_carries_the_reference_metadata(tiny_pack):
    """Buckets, speculative modes, required kernels and backend policy, the
    leanpack/v0 fields the reference's loader and planner read
    (src/leanstack/pack.py:95-100, leanserve.py:199-202)."""
    _, out, manifest = tiny_pack
    assert manifest.exact_prompt_buckets == [64, 512, 1024]
    assert [(b.key, b.prompt_tokens, b.max_new_tokens) for b in manifest.buckets] == [
        ("decode_64_256", 64, 256), ("decode_64_512", 64, 512), ("prefill_1024_64", 1024, 64)]
    assert [m.key for m in manifest.speculative_modes] == ["draft12_k4", "draft12_k2"]
    assert manifest.speculative_modes[0].draft_layer_count == 1  # 2-layer model: min(12, L - 1)
    assert "lsk_linear_bf16" in manifest.required_kernels and manifest.backend_policy
    assert load_packed_artifact_manifest(out).buckets == manifest.buckets


def test_loader_reads_each_file_as_one_arena_image(tiny_pack):
    """Every file's data region is a byte image of its arena range: one read
    and one copy per file, no per-tensor reads; the KV cache is sized from
    the manifest's buckets (1088 tokens -> 1088 rows in pages of 16)."""
    _, out, manifest = tiny_pack
    runtime, arena = materialize_qwen_semantic_stack_from_leanpack(out, device="cpu")
    assert arena.load_stats == {"files": len(manifest.files), "bulk": len(manifest.files), "per_tensor": 0,
                                "bytes": sum(t.size_bytes for t in manifest.tensors)}
    kv = arena.plan.entry("kv_cache")
    assert kv.shape[4] == 1088 and [b.key for b in arena.plan.buckets] == [b.key for b in manifest.buckets]


def test_loader_places_tensors_one_by_one_when_offsets_differ(tiny_pack):
    """With an arena of another alignment the files are no longer images of
    arena ranges: the loader copies each tensor to its entry, same result."""
    from leanstack_amd.leanserve import ResidentArena, build_resident_buffer_plan, load_pack_into_arena
    from leanstack_amd.pack import geometry_from_manifest

    ckpt, out, manifest = tiny_pack
    plan = build_resident_buffer_plan(geometry_from_manifest(manifest), buckets=(), alignment=8192)
    arena = ResidentArena(plan, "cpu")
    stats = load_pack_into_arena(out, manifest, arena)
    assert stats["bulk"] < stats["files"] and stats["per_tensor"] > 0
    assert torch.equal(arena.view("model.embed_tokens.weight"), ckpt["model.embed_tokens.weight"])
    assert torch.equal(arena.packed("layers.1.mlp.down_proj.weight").unpack(), ckpt[hf_layer_names(1)["down_proj"]])


def test_loader_refuses_a_truncated_file(tiny_pack, tmp_path):
    import shutil

    _, out, _ = tiny_pack
    bad = tmp_path / "short"
    shutil.copytree(out, bad)
    data = (bad / "layer-001.safetensors").read_bytes()
    (bad / "layer-001.safetensors").write_bytes(data[: len(data) - 4096])
    with pytest.raises(ValueError, match="truncated"):
        materialize_qwen_semantic_stack_from_leanpack(bad, device="cpu", buckets=())


def _copy_pack(src, dst, edit):
    """A copy of the pack at dst whose manifest payload went through edit()."""
    import shutil

    shutil.copytree(src, dst)
    payload = json.loads((dst / "manifest.json").read_text())
    edit(payload)
    (dst / "manifest.json").write_text(json.dumps(payload))
    return dst


def test_loader_refuses_a_pack_missing_a_planned_weight(tiny_pack, tmp_path):
    """A planned weight with no tensor in the pack would leave uninitialised
    arena bytes under the runtime: the loader raises instead."""
    _, out, _ = tiny_pack

    def drop(payload):
        payload["tensors"] = [t for t in payload["tensors"] if t["name"] != "layers.1.mlp.down_proj.weight"]

    bad = _copy_pack(out, tmp_path / "truncated", drop)
    with pytest.raises(ValueError, match="no tensor for 1 planned"):
        materialize_qwen_semantic_stack_from_leanpack(bad, device="cpu", buckets=())


def test_loader_refuses_a_mislabelled_layout(tiny_pack, tmp_path):
    """A gate_up stored as plain mfma16x32 (or a packed weight labelled
    row-major) has the right byte count but the wrong tile order."""
    _, out, _ = tiny_pack

    def relabel(name, layout):
        def edit(payload):
            for t in payload["tensors"]:
                if t["name"] == name:
                    t["layout"] = layout
        return edit

    bad = _copy_pack(out, tmp_path / "gateup", relabel("layers.0.mlp.gate_up_proj.weight", "mfma16x32"))
    with pytest.raises(ValueError, match="plan needs 'mfma16x32_gateup'"):
        materialize_qwen_semantic_stack_from_leanpack(bad, device="cpu", buckets=())
    bad = _copy_pack(out, tmp_path / "rowmajor", relabel("layers.0.attention.o_proj.weight", "rowmajor"))
    with pytest.raises(ValueError, match="plan needs 'mfma16x32'"):
        materialize_qwen_semantic_stack_from_leanpack(bad, device="cpu", buckets=())


def test_loader_refuses_a_manifest_without_file_offsets(tiny_pack, tmp_path):
    """An early leanpack/v1 manifest had no file_offset_bytes; reading each
    tensor at offset 0 would load the safetensors header as weights with
    every size check passing, so such a manifest is refused."""
    _, out, _ = tiny_pack

    def strip(payload):
        for t in payload["tensors"]:
            t.pop("file_offset_bytes", None)

    bad = _copy_pack(out, tmp_path / "nooffsets", strip)
    with pytest.raises(ValueError, match="no file_offset_bytes"):
        materialize_qwen_semantic_stack_from_leanpack(bad, device="cpu", buckets=())


def test_loader_refuses_an_offset_the_header_contradicts(tiny_pack, tmp_path):
    """An offset that points at another tensor's (aligned, same-sized)
    bytes passes the layout and size checks; the safetensors header names
    the true range, and the loader holds the manifest to it."""
    _, out, _ = tiny_pack

    def shift(payload):
        for t in payload["tensors"]:
            if t["name"] == "layers.0.attention.o_proj.weight":
                t["file_offset_bytes"] += 4096

    bad = _copy_pack(out, tmp_path / "shifted", shift)
    with pytest.raises(ValueError, match="the safetensors header at"):
        materialize_qwen_semantic_stack_from_leanpack(bad, device="cpu", buckets=())


@pytest.mark.gpu
def test_real_shape_layer_from_pack_runs_the_dispatch_path(gpu, tmp_path):
    from leanstack_amd import dispatch
    from oracle import projections as ref
    from tests.helpers import activations, assert_parity

    g = QwenGeometry(num_hidden_layers=1, vocab_size=4096)
    ckpt = synthetic_qwen_checkpoint(g, seed=9)
    build_qwen_leanpack(ckpt, tmp_path / "pack", geometry=g)
    runtime, _ = materialize_qwen_semantic_stack_from_leanpack(tmp_path / "pack", device="cuda:0", buckets=())
    lr = runtime.layers[0]
    n = hf_layer_names(0)
    h = activations(1, g.hidden_size, seed=4).view(-1)
    y = dispatch._semantic_mlp_epilogue_vector(h.cuda(), lr.post_attention_layernorm_weight, lr.mlp.gate_up_proj_weight,
                                               lr.mlp.gate_proj_out_dim, lr.mlp.down_proj_weight, g.rms_norm_eps)
    gu = torch.cat((ckpt[n["gate_proj"]], ckpt[n["up_proj"]]))
    expect = ref.mlp_epilogue_vector(h, ckpt[n["post_attention_layernorm"]], gu, g.intermediate_size,
                                     ckpt[n["down_proj"]], g.rms_norm_eps)
    assert_parity(y.cpu(), expect, "mlp from leanpack")
    tok = dispatch.select_semantic_greedy_token(runtime, h.view(1, 1, -1).cuda())
    normed = ref.rmsnorm(h.view(1, -1), ckpt["model.norm.weight"], g.rms_norm_eps).view(-1)
    assert tok.item() == ref.logits_argmax(normed, ckpt["model.embed_tokens.weight"]).item()


@pytest.mark.gpu
@pytest.mark.parametrize("per_tensor", [False, True])
def test_device_arena_matches_host_arena_through_small_chunks(gpu, tiny_pack, monkeypatch, per_tensor):
    """The device loader stages file regions through two pinned buffers,
    reading one while the other is copied; with 4 KB chunks every region takes
    many turns of both.  The device arena's weight bytes equal the host
    arena's, read straight from the files (whole-file images, or one tensor at
    a time with another alignment)."""
    from leanstack_amd import leanserve
    from leanstack_amd.leanserve import ResidentArena, build_resident_buffer_plan, load_pack_into_arena
    from leanstack_amd.pack import geometry_from_manifest

    _, out, manifest = tiny_pack
    monkeypatch.setattr(leanserve, "LOAD_CHUNK_BYTES", 4096)
    extra = {"alignment": 8192} if per_tensor else {}
    plan = build_resident_buffer_plan(geometry_from_manifest(manifest), buckets=(), **extra)
    host, dev = ResidentArena(plan, "cpu"), ResidentArena(plan, "cuda:0")
    s_host = load_pack_into_arena(out, manifest, host)
    s_dev = load_pack_into_arena(out, manifest, dev)
    assert s_host == s_dev and (s_dev["per_tensor"] > 0) == per_tensor
    got = dev.buffer.cpu()
    for e in plan.entries:
        if e.name in host.weight_names():
            assert torch.equal(got[e.offset : e.end], host.buffer[e.offset : e.end]), e.name
