"""The launch-structure probe (lsk_probe_stream_step, bench.py
--probe-step-floor) runs to completion in every mode, its bounded waits never
give up, and it leaves its workspace zero for the next launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from leanstack_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("ring", [4, 16])
def test_probe_modes_complete(gpu, mode, ring):
    lib = _lib.load()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    seg = [cus * 12, cus * 40, cus * 13, cus * 12] * 3
    weights = torch.zeros(sum(seg) * 1024, dtype=torch.uint8, device=dev)
    ws = torch.zeros(lib.lsk_probe_workspace_bytes(), dtype=torch.uint8, device=dev)
    arr = (ctypes.c_longlong * len(seg))(*seg)
    print(f"case mode={mode} ring={ring} segments={len(seg)}", flush=True)
    for _ in range(3):
        st = lib.lsk_probe_stream_step(weights.data_ptr(), weights.numel(), arr, len(seg), mode, ring, ws.data_ptr(),
                                       ws.numel(), torch.cuda.current_stream().cuda_stream)
        assert st == _lib.OK, _lib.last_error()
        torch.cuda.synchronize()
        assert int(ws.view(torch.int32)[0].item()) == 0, "a bounded wait gave up"
        assert int(ws.view(torch.int32)[1:].abs().sum().item()) == 0, "workspace not left zero"
    short = (ctypes.c_longlong * 1)(cus * 11)
    assert lib.lsk_probe_stream_step(weights.data_ptr(), weights.numel(), short, 1, mode, ring, ws.data_ptr(),
                                     ws.numel(), None) == _lib.ERR_INVALID


def test_probe_mfma_runs(gpu):
    """The MFMA-rate probe completes, leaves its sink alone, and refuses bad
    arguments before launch."""
    lib = _lib.load()
    sink = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda:0"))
    assert lib.lsk_probe_mfma_rate(8, 10, sink.data_ptr(), torch.cuda.current_stream().cuda_stream) == _lib.OK
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    assert lib.lsk_probe_mfma_rate(0, 10, sink.data_ptr(), None) == _lib.ERR_INVALID
    assert lib.lsk_probe_mfma_rate(8, 0, sink.data_ptr(), None) == _lib.ERR_INVALID
