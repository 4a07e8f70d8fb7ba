"""The arena KV cache on the CPU (leanstack_amd/kv_cache.py): what the decode
dispatch reads from it (layer_seq_lens, layer_tensors, advance), the rows
the torch glue writes, and the speculative rollback."""

from __future__ import annotations

import pytest
import torch

from leanstack_amd import dispatch
from leanstack_amd.kv_cache import ArenaKVCache


def _rows(t, seed, h=2, d=8):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn((h, t, d), generator=g).to(torch.bfloat16),
            torch.randn((h, t, d), generator=g).to(torch.bfloat16))


def _cache(**over):
    kw = dict(num_layers=3, num_key_value_heads=2, head_dim=8, capacity=10)
    kw.update(over)
    return ArenaKVCache(**kw)


def test_rejects_empty_dimensions():
    for over in (dict(num_layers=0), dict(num_key_value_heads=0), dict(head_dim=0), dict(capacity=0)):
        with pytest.raises(ValueError):
            _cache(**over)


def test_write_rows_and_cursors():
    cache = _cache()
    k1, v1 = _rows(3, 1)
    cache.write_rows(1, k1, v1)
    k2, v2 = _rows(2, 2)
    cache.write_rows(1, k2[None], v2[None])  # a batch axis of 1 is accepted
    k, v = cache.attended(1)
    assert k.shape == (1, 2, 5, 8)
    assert torch.equal(k[0], torch.cat((k1, k2), dim=1)) and torch.equal(v[0], torch.cat((v1, v2), dim=1))
    assert cache.rows(1) == 5 and cache.rows(0) == 0 and cache.max_layer_seq_len == 5
    assert cache.attended(0)[0].shape == (1, 2, 0, 8)


def test_refuses_rows_that_do_not_fit():
    cache = _cache()
    k, v = _rows(3, 3)
    with pytest.raises(ValueError):
        cache.write_rows(0, k, v[:, :2])
    with pytest.raises(ValueError):
        cache.write_rows(0, *_rows(3, 4, h=3))
    with pytest.raises(ValueError):
        cache.write_rows(0, *_rows(3, 5, d=4))
    cache.write_rows(0, *_rows(9, 7))
    before = cache.storage.clone()
    with pytest.raises(ValueError, match="does not fit"):
        cache.write_rows(0, *_rows(2, 8))
    assert cache.rows(0) == 9 and torch.equal(cache.storage, before)  # a refused write moves nothing
    with pytest.raises(ValueError, match="does not fit"):
        cache.advance(0, 2)
    with pytest.raises(ValueError):
        cache.advance(0, -1)
    cache.advance(0, 1)
    assert cache.rows(0) == 10


def test_mark_and_rewind():
    """Rows written after a mark are dropped by rewind and overwritten by the
    next write; earlier rows stay."""
    cache = _cache()
    k1, v1 = _rows(2, 9)
    for layer in range(3):
        cache.write_rows(layer, k1, v1)
    mark = cache.mark()
    for layer in range(3):
        cache.write_rows(layer, *_rows(4, 10 + layer))
    assert cache.max_layer_seq_len == 6
    cache.rewind(mark)
    assert [cache.rows(i) for i in range(3)] == [2, 2, 2]
    assert torch.equal(cache.attended(2)[0][0], k1)
    k3, v3 = _rows(1, 20)
    cache.write_rows(2, k3, v3)
    assert torch.equal(cache.attended(2)[1][0], torch.cat((v1, v3), dim=1))
    with pytest.raises(ValueError):
        cache.rewind((5, 5, 5))  # not an earlier state
    with pytest.raises(ValueError):
        cache.rewind((1, 1))


def test_works_in_place_on_an_arena_region():
    """The cache over a [L, 2, 1, n_kv, S, d] arena entry: writes land in the
    region, layer_tensors are its contiguous [n_kv, S, d] blocks, and the
    reference-shaped key_cache / value_cache views see the same memory."""
    region = torch.zeros((3, 2, 1, 2, 10, 8), dtype=torch.bfloat16)
    cache = ArenaKVCache(3, 2, 8, 10, storage=region)
    k, v = _rows(3, 30)
    cache.write_rows(2, k, v)
    assert torch.equal(region[2, 0, 0, :, :3], k) and torch.equal(region[2, 1, 0, :, :3], v)
    kl, vl = cache.layer_tensors(2)
    assert kl.shape == (2, 10, 8) and kl.is_contiguous() and vl.is_contiguous()
    assert kl.data_ptr() == region[2, 0, 0].data_ptr() and vl.data_ptr() == region[2, 1, 0].data_ptr()
    assert cache.key_cache.shape == (3, 1, 2, 10, 8) and cache.key_cache.data_ptr() == region.data_ptr()
    kl[:, 3] = 1.0  # what the decode kernel's append does; then the cursor moves
    cache.advance(2, 1)
    assert torch.equal(cache.attended(2)[0][0, :, 3], torch.ones(2, 8, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        ArenaKVCache(3, 2, 8, 10, storage=torch.zeros((3, 2, 1, 2, 9, 8), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        ArenaKVCache(3, 2, 8, 10, storage=torch.zeros((3, 2, 2, 2, 10, 8), dtype=torch.bfloat16))


def test_dispatch_reads_the_cache_it_advances():
    """dispatch's cache accessors on this cache: the layer blocks and the
    cursor, then one row counted."""
    cache = _cache()
    cache.write_rows(1, *_rows(4, 40))
    k, v, pos = dispatch._static_cache_layer(cache, 1)
    assert pos == 4 and k.data_ptr() == cache.layer_tensors(1)[0].data_ptr()
    dispatch._advance_cache(cache, 1)
    assert cache.rows(1) == 5
