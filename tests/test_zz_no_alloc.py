"""The allocation-free lm_head (lsk_lm_head_argmax_noalloc_bf16) against the
workspace entry point it varies (lsk_lm_head_argmax_bf16), through the C ABI:
two calls in a row on the same device -- the second smaller, so it runs over
the first call's leftover scratch contents -- each giving the same token ids
and the same fp32 scores, bit for bit, as the workspace call on the same
inputs (identical kernels, so identical arithmetic).  Ordered last in the
suite because every call on a device shares the one static scratch."""

from __future__ import annotations

import pytest
import torch

from leanstack_amd import _lib, kernels
from leanstack_amd.layout import PackedWeight
from tests.helpers import activations, weight

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _both(e: PackedWeight, h: torch.Tensor, mode: int):
    lib = _lib.load()
    m, v, k = h.shape[0], e.n, e.k
    stream = kernels.stream_handle()
    ws = torch.zeros(lib.lsk_workspace_bytes(_lib.OP_LM_HEAD_ARGMAX, m, v, k), dtype=torch.uint8, device=DEV)
    idx_ws = torch.full((m,), -1, dtype=torch.long, device=DEV)
    scores_ws = torch.empty((m, v), dtype=torch.float32, device=DEV)
    _lib.check(lib.lsk_lm_head_argmax_bf16(e.data.data_ptr(), e.layout, v, k, h.data_ptr(), m, k,
                                           scores_ws.data_ptr(), mode, idx_ws.data_ptr(), ws.data_ptr(), ws.numel(),
                                           stream), "workspace head")
    idx_na = torch.full((m,), -1, dtype=torch.long, device=DEV)
    scores_na = torch.empty((m, v), dtype=torch.float32, device=DEV)
    _lib.check(lib.lsk_lm_head_argmax_noalloc_bf16(e.data.data_ptr(), e.layout, v, k, h.data_ptr(), m, k,
                                                   scores_na.data_ptr(), mode, idx_na.data_ptr(), stream),
               "allocation-free head")
    torch.cuda.synchronize()
    return idx_ws.cpu(), scores_ws.cpu(), idx_na.cpu(), scores_na.cpu()


def test_noalloc_head_matches_the_workspace_head_twice(gpu):
    big = PackedWeight.from_rowmajor(weight(151936, 2560, seed=501).to(DEV))
    small = PackedWeight.from_rowmajor(weight(65536, 2560, seed=502).to(DEV))
    cases = [(big, activations(8, 2560, seed=503).to(DEV), _lib.LOGITS_FP32),
             (small, activations(3, 2560, seed=504).to(DEV), _lib.LOGITS_BF16)]
    for call, (e, h, mode) in enumerate(cases):
        idx_ws, s_ws, idx_na, s_na = _both(e, h, mode)
        print(f"call {call}: M={h.shape[0]} V={e.n} tokens {idx_na.tolist()}")
        assert idx_na.tolist() == idx_ws.tolist(), f"call {call}"
        assert torch.equal(s_na.view(torch.int32), s_ws.view(torch.int32)), f"call {call}"
        assert all(0 <= t < e.n for t in idx_na.tolist())
