"""The packed layout: three independent packers agree, round trips are exact,
and the layout places each element where the MFMA operand order needs it."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from leanstack_amd import _lib
from leanstack_amd.layout import PackedWeight, pack_tensor, unpack_tensor
from oracle import packing

LAYOUTS = [_lib.LAYOUT_MFMA16X32, _lib.LAYOUT_MFMA16X32_GATEUP]


def _w(n, k, seed=0):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(n, k, generator=gen).to(torch.bfloat16)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("n,k", [(32, 32), (64, 96), (256, 2560)])
def test_torch_c_and_numpy_packers_agree(layout, n, k):
    w = _w(n, k, seed=n + k)
    by_torch = pack_tensor(w, layout).view(torch.int16).numpy()
    by_numpy = packing.pack(w.view(torch.int16).numpy(), layout)
    host = torch.empty(n * k, dtype=torch.bfloat16)
    _lib.check(_lib.load().lsk_pack_bf16(w.data_ptr(), n, k, layout, host.data_ptr()), "pack")
    assert np.array_equal(by_torch, by_numpy)
    assert np.array_equal(by_torch, host.view(torch.int16).numpy())


@pytest.mark.parametrize("layout", LAYOUTS)
def test_round_trips_are_exact(layout):
    w = _w(128, 320, seed=1)
    packed = pack_tensor(w, layout)
    assert torch.equal(unpack_tensor(packed, 128, 320, layout).view(torch.int16), w.view(torch.int16))
    back = torch.empty_like(w)
    _lib.check(_lib.load().lsk_unpack_bf16(packed.data_ptr(), 128, 320, layout, back.data_ptr()), "unpack")
    assert torch.equal(back.view(torch.int16), w.view(torch.int16))
    assert torch.equal(PackedWeight(packed, 128, 320, layout).unpack().view(torch.int16), w.view(torch.int16))


def test_tile_lane_order_matches_the_mfma_operand():
    """Tile (rb, kt) lane l holds W[16 rb + l%16, 32 kt + 8 (l/16) + e]."""
    n, k = 32, 64
    w = torch.arange(n * k, dtype=torch.float32).view(n, k)  # unique values, exact in fp32
    idx = torch.arange(n * k, dtype=torch.int64).view(n, k)
    # pack the index map through the packer's permutation by packing bf16 bit patterns
    packed = pack_tensor(idx.to(torch.int16).view(torch.bfloat16), _lib.LAYOUT_MFMA16X32).view(torch.int16)
    kt_count = k // 32
    for rb in range(n // 16):
        for kt in range(kt_count):
            tile = packed[(rb * kt_count + kt) * 512 : (rb * kt_count + kt + 1) * 512].view(64, 8)
            for lane in (0, 5, 16, 37, 63):
                row = 16 * rb + lane % 16
                col = 32 * kt + 8 * (lane // 16)
                assert tile[lane].tolist() == idx[row, col : col + 8].to(torch.int16).tolist()
    del w


def test_gate_up_interleave_pairs_blocks():
    """Packed row-block 2j = gate rows 16j..16j+15, 2j+1 = up rows 16j..16j+15."""
    inter, k = 48, 32
    rows = torch.arange(2 * inter, dtype=torch.int16).view(-1, 1).repeat(1, k)
    packed = pack_tensor(rows.view(torch.bfloat16), _lib.LAYOUT_MFMA16X32_GATEUP).view(torch.int16)
    tiles = packed.view(2 * inter // 16, 1, 64, 8)  # one k-tile per row-block
    for pr_block in range(2 * inter // 16):
        pair, is_up = divmod(pr_block, 2)
        lane_rows = tiles[pr_block, 0, :16, 0].tolist()  # lanes 0..15 = rows of the block
        base = (inter if is_up else 0) + 16 * pair
        assert lane_rows == list(range(base, base + 16))


@pytest.mark.parametrize("n,k,layout", [(15, 32, 1), (16, 40, 1), (48, 32, 2), (16, 32, 7)])
def test_rejects_unpackable_shapes(n, k, layout):
    lib = _lib.load()
    assert lib.lsk_packed_bytes(layout, n, k) == 0
    buf = torch.empty(max(n * k, 1), dtype=torch.bfloat16)
    assert lib.lsk_pack_bf16(buf.data_ptr(), n, k, layout, buf.data_ptr()) < 0
    assert _lib.last_error()
    with pytest.raises(ValueError):
        pack_tensor(torch.zeros(n, k, dtype=torch.bfloat16), layout)


def test_packed_bytes_of_the_qwen_projections():
    lib = _lib.load()
    assert lib.lsk_packed_bytes(1, 6144, 2560) == 31_457_280
    assert lib.lsk_packed_bytes(1, 2560, 4096) == 20_971_520
    assert lib.lsk_packed_bytes(2, 19456, 2560) == 99_614_720
    assert lib.lsk_packed_bytes(1, 2560, 9728) == 49_807_360
    assert lib.lsk_packed_bytes(1, 151936, 2560) == 777_912_320
