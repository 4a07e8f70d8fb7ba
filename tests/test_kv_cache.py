"""The static KV cache manager on the CPU (leanstack_amd/kv_cache.py): the
reference's StaticKVBlockManager contract (src/leanstack/runtime/kv_cache.py:
207-330) and the two additions the decode attention kernel relies on
(`layer_tensors`, `advance`)."""

from __future__ import annotations

import pytest
import torch

from leanstack_amd.kv_cache import KVPageLayout, StaticKVBlockManager


def _layout(**over):
    kw = dict(num_layers=3, num_key_value_heads=2, head_dim=8, page_size=4, max_seq_len=10, batch_size=1,
              dtype=torch.bfloat16, device=torch.device("cpu"))
    kw.update(over)
    return KVPageLayout(**kw)


def _states(t, seed, b=1, h=2, d=8):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn((b, h, t, d), generator=g).to(torch.bfloat16),
            torch.randn((b, h, t, d), generator=g).to(torch.bfloat16))


def test_layout_rejects_bad_geometry():
    for over in (dict(page_size=0), dict(max_seq_len=0), dict(batch_size=0)):
        with pytest.raises(ValueError):
            _layout(**over)


def test_append_get_and_lengths():
    cache = StaticKVBlockManager(_layout())
    k1, v1 = _states(3, 1)
    k, v = cache.append_and_get(1, k1, v1)
    assert torch.equal(k, k1) and torch.equal(v, v1)
    k2, v2 = _states(2, 2)
    cache.append(1, k2, v2)
    k, v = cache.get(1)
    assert torch.equal(k, torch.cat((k1, k2), dim=2)) and torch.equal(v, torch.cat((v1, v2), dim=2))
    assert cache.get_layer_seq_length(1) == 5 and cache.get_layer_seq_length(0) == 0
    assert cache.get_seq_length() == 5
    assert cache.page_table(1) == (0, 1)  # 5 rows in pages of 4
    assert cache.get(0)[0].shape == (1, 2, 0, 8)


def test_append_rejects_mismatched_states_and_overflow():
    cache = StaticKVBlockManager(_layout())
    k, v = _states(3, 3)
    with pytest.raises(ValueError):
        cache.append(0, k, v[:, :, :2])
    with pytest.raises(ValueError):
        cache.append(0, *_states(3, 4, h=3))
    with pytest.raises(ValueError):
        cache.append(0, *_states(3, 5, d=4))
    with pytest.raises(ValueError):
        cache.append(0, *_states(3, 6, b=2))
    cache.append(0, *_states(9, 7))
    with pytest.raises(ValueError, match="overflow"):
        cache.append(0, *_states(2, 8))
    assert cache.get_layer_seq_length(0) == 9  # a refused append moves nothing
    with pytest.raises(ValueError, match="overflow"):
        cache.advance(0, 2)
    cache.advance(0, 1)
    assert cache.get_layer_seq_length(0) == 10


def test_snapshot_restore_rolls_back_the_cursor():
    """The speculative verify rollback (qwen_explicit_runtime_loop.py:822-847):
    rows written after the snapshot are forgotten, earlier ones kept."""
    cache = StaticKVBlockManager(_layout())
    k1, v1 = _states(2, 9)
    for layer in range(3):
        cache.append(layer, k1, v1)
    snap = cache.snapshot_cursor()
    for layer in range(3):
        cache.append(layer, *_states(4, 10 + layer))
    assert cache.get_seq_length() == 6
    cache.restore_cursor(snap)
    assert [cache.get_layer_seq_length(i) for i in range(3)] == [2, 2, 2] and cache.get_seq_length() == 2
    assert torch.equal(cache.get(2)[0], k1)
    k3, v3 = _states(1, 20)
    cache.append(2, k3, v3)  # overwrites row 2 of layer 2
    assert torch.equal(cache.get(2)[1], torch.cat((v1, v3), dim=2))


def test_storage_views_of_an_arena_entry():
    """Key / value caches are views of one [L, 2, B, n_kv, S, d] tensor: a
    write through the manager lands in the storage, and layer_tensors gives
    the contiguous [n_kv, S, d] block the attention kernel addresses."""
    layout = _layout()
    storage = torch.zeros((3, 2, 1, 2, 10, 8), dtype=torch.bfloat16)
    cache = StaticKVBlockManager(layout, storage)
    k, v = _states(3, 30)
    cache.append(2, k, v)
    assert torch.equal(storage[2, 0, 0, :, :3], k[0]) and torch.equal(storage[2, 1, 0, :, :3], v[0])
    kl, vl = cache.layer_tensors(2)
    assert kl.shape == (2, 10, 8) and kl.is_contiguous() and vl.is_contiguous()
    assert kl.data_ptr() == storage[2, 0, 0].data_ptr() and vl.data_ptr() == storage[2, 1, 0].data_ptr()
    kl[:, 3] = 1.0  # what the kernel's append does, then the cursor moves
    cache.advance(2, 1)
    assert torch.equal(cache.get(2)[0][0, :, 3], torch.ones(2, 8, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        StaticKVBlockManager(layout, torch.zeros((3, 2, 1, 2, 9, 8), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        StaticKVBlockManager(layout, torch.zeros((3, 2, 1, 2, 10, 8), dtype=torch.float32))


def test_layer_tensors_serve_batch_one_only():
    cache = StaticKVBlockManager(_layout(batch_size=2))
    with pytest.raises(ValueError, match="batch 1"):
        cache.layer_tensors(0)
