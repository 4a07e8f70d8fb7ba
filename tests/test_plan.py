"""The resident arena planner: closed-form byte counts, alignment, no overlaps.

Byte counts follow the reference's accounting (src/leanstack/leanserve.py:
331-377, KV per bucket = L * 2 * n_kv * d * ceil(S/16)*16 * 2) with two
deliberate changes: logits are sized fp32 and scratch is sized for M rows.
"""

from __future__ import annotations

from math import ceil

import pytest

from leanstack_amd import _lib
from leanstack_amd.geometry import QWEN3_4B as G
from leanstack_amd.leanserve import (
    ARENA_ALIGNMENT,
    DEFAULT_BUCKETS,
    BucketSpec,
    build_resident_buffer_plan,
    layer_entry_names,
)


def test_geometry_matches_the_reference_registry():
    # src/leanstack/model_registry.py:16-23 and tests/test_active_contract.py:16-21
    assert (G.num_hidden_layers, G.hidden_size, G.intermediate_size) == (36, 2560, 9728)
    assert (G.num_attention_heads, G.num_key_value_heads, G.head_dim, G.vocab_size) == (32, 8, 128, 151936)
    # fused shapes of the packer (src/leanstack/pack.py:269-286); the unfused
    # (K, N) pairs of tests/test_hot_kernel_cases.py:22-26 are their pieces
    p = G.projections()
    assert p["qkv_proj"] == (4096 + 1024 + 1024, 2560)
    assert p["o_proj"] == (2560, 4096)
    assert p["gate_up_proj"] == (2 * 9728, 2560)
    assert p["down_proj"] == (2560, 9728)


def test_per_step_byte_accounting():
    assert G.layer_weight_bytes() == 201_850_880
    assert G.num_hidden_layers * G.layer_weight_bytes() == 7_266_631_680
    assert G.layer_bytes(1) == 201_930_752
    assert G.layer_bytes(4) == 202_170_368
    assert G.stack_bytes(1) == 7_269_507_072
    assert G.stack_bytes(8) == 7_289_634_816
    assert G.lm_head_bytes() == 777_912_320
    assert G.lm_head_call_bytes(1) == 777_912_320 + 5_120 + 607_744
    assert G.lm_head_call_bytes(1, logits=False) == 777_912_320 + 5_120
    assert G.layer_flops(2048) == 2 * 2048 * G.layer_params()
    assert round(G.layer_flops(2048) / 1e9, 2) == 413.39


def test_plan_entries_are_aligned_and_disjoint():
    plan = build_resident_buffer_plan(G, layers=3, buckets=DEFAULT_BUCKETS)
    entries = sorted(plan.entries, key=lambda e: e.offset)
    for a, b in zip(entries, entries[1:]):
        assert a.end <= b.offset
    assert all(e.offset % ARENA_ALIGNMENT == 0 for e in entries)
    assert plan.arena_bytes >= plan.resident_bytes


def test_plan_weight_bytes_closed_form():
    plan = build_resident_buffer_plan(G, buckets=())
    per_layer = G.layer_weight_bytes() + 2 * G.hidden_size * 2 + 2 * G.head_dim * 2
    embed = G.vocab_size * G.hidden_size * 2
    expect = G.num_hidden_layers * per_layer + embed + G.hidden_size * 2 + G.lm_head_bytes()
    assert plan.weights_bytes == expect
    names = layer_entry_names(7)
    assert plan.entry(names["gate_up_proj"]).layout == _lib.LAYOUT_MFMA16X32_GATEUP
    assert plan.entry(names["qkv_proj"]).layout == _lib.LAYOUT_MFMA16X32
    assert plan.entry("lm_head.weight").layout == _lib.LAYOUT_MFMA16X32
    assert plan.entry("model.embed_tokens.weight").layout is None  # row-major for the gather


def test_kv_and_scratch_closed_forms():
    buckets = (BucketSpec("decode_64_256", 64, 256), BucketSpec("prefill_1024_64", 1024, 64))
    plan = build_resident_buffer_plan(G, buckets=buckets, max_rows=16)
    for b, bp in zip(buckets, plan.buckets):
        cap = ceil((b.prompt_tokens + b.max_new_tokens) / 16) * 16
        assert bp.kv_tokens_capacity == cap
        assert bp.kv_cache_bytes == 36 * 2 * 8 * 128 * cap * 2
    assert plan.buckets[0].kv_cache_bytes == 47_185_920  # 64+256 tokens -> 320-token cache
    s = plan.scratch
    assert s.logits_bytes == 16 * G.vocab_size * 4  # fp32 logits, 16 rows
    assert s.mlp_activation_bytes == 16 * G.intermediate_size * 2
    assert s.argmax_workspace_bytes == _lib.load().lsk_workspace_bytes(_lib.OP_LM_HEAD_ARGMAX, 16, G.vocab_size,
                                                                      G.hidden_size)
    kv = plan.entry("kv_cache")
    assert kv.nbytes == plan.max_kv_cache_bytes


def test_plan_fits_one_mi355x_with_room():
    plan = build_resident_buffer_plan(G, buckets=DEFAULT_BUCKETS)
    assert plan.arena_bytes < 10e9  # ~8.9 GB of 288 GB HBM


@pytest.mark.parametrize("rows", [1, 8, 2048])
def test_scratch_scales_with_rows(rows):
    plan = build_resident_buffer_plan(G, buckets=(), max_rows=rows, include_embedding=False)
    assert plan.entry("scratch.qkv").shape == (rows, G.qkv_dim)
    assert plan.entry("scratch.logits").shape == (min(rows, 16), G.vocab_size)
