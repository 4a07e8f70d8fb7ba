"""Torch-tensor wrappers of the C ABI: projections and the greedy lm_head.

Tensors are device memory that torch owns; the kernels run on torch's current
HIP stream (``torch.cuda.current_stream().cuda_stream`` is a hipStream_t on
ROCm), as the cuTile head launches on the current stream
(src/leanstack/runtime/cutile_logits.py:59).  Nothing here falls back to
another implementation: a missing library or a rejected argument raises.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .layout import PackedWeight


def _require_device(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{what} must be a GPU tensor, got device {t.device}")


def _one_device(first: torch.Tensor, *named: tuple[torch.Tensor | None, str]) -> torch.device:
    """The device of `first`, after checking that every other tensor given
    (None skipped) lives on it: the C layer launches on one device and sees
    only pointers."""
    dev = first.device
    for t, what in named:
        if t is not None and t.device != dev:
            raise ValueError(f"{what} is on {t.device}, the call's tensors are on {dev}")
    return dev


def _rows(x: torch.Tensor, k: int, what: str) -> tuple[torch.Tensor, int, int]:
    """View x as [M, k] rows with unit column stride; returns (x2d, M, ld).
    Rows the kernels cannot read in place (column stride, row stride not a
    multiple of 8 or above the library's largest, misalignment) are copied."""
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{what} must be bfloat16, got {x.dtype}")
    if x.shape[-1] != k:
        raise ValueError(f"{what} last dim {x.shape[-1]} != K={k}")
    x2 = x.reshape(-1, k)
    if (x2.stride(-1) != 1 or (x2.shape[0] > 1 and (x2.stride(0) % 8 or x2.stride(0) > _lib.MAX_ACTIVATION_STRIDE))
            or x2.data_ptr() % 16):
        x2 = x2.contiguous()
    ld = x2.stride(0) if x2.shape[0] > 1 else k
    return x2, x2.shape[0], ld


def stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check_out(out: torch.Tensor, m: int, n_out: int, dtype: torch.dtype, what: str = "out") -> None:
    """A caller-supplied output must hold exactly the m x n_out values the
    kernel writes, contiguously: the C layer sees only a pointer."""
    if out.dtype != dtype or out.shape[-1:] != (n_out,) or out.numel() != m * n_out or not out.is_contiguous():
        raise ValueError(f"{what} must be a contiguous {dtype} tensor of {m} x {n_out} values "
                         f"(got {out.dtype} {tuple(out.shape)})")


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _device_workspace(cache: dict[tuple[int, int], torch.Tensor], device: torch.device, nbytes: int,
                      what: str) -> torch.Tensor:
    """The zero-filled workspace of `cache` for `device` and the current
    stream, grown to `nbytes`.  One per (device, stream): the split blocks of
    a call count arrivals in the workspace's flag words and read each other's
    partial slots, so two calls that overlap must not share one, and calls on
    one stream are ordered.  It is never allocated while the stream is being
    captured, so a captured graph never replays a workspace's allocation or
    zero fill (run the same launch once on the capture stream before the
    capture); a graph keeps using the workspace of the stream it was captured
    on, so eager calls on that stream must not overlap its replays."""
    key = (_device_index(device), torch.cuda.current_stream(device).cuda_stream)
    ws = cache.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"the {what} workspace must be allocated before graph capture: run the same "
                               f"launch once on the capture stream, outside the capture, first")
        ws = torch.zeros(nbytes, device=device, dtype=torch.uint8)
        cache[key] = ws
    return ws


_prefill_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def prefill_workspace(device: torch.device, m: int, n: int, k: int) -> torch.Tensor | None:
    """The split-K workspace of the prefill GEMM on `device` for the current
    stream (zero-filled once, left zero-filled by every call), or None when
    the shape does not use one."""
    nbytes = _lib.load().lsk_workspace_bytes(_lib.OP_LINEAR, m, n, k)
    if nbytes == 0:
        return None
    return _device_workspace(_prefill_workspaces, device, nbytes, "prefill")


def set_linear_wait_limit(polls: int) -> None:
    """Polls of a split-K arrival word before a prefill workgroup gives up
    (then the workspace's error word is set and its tiles are NaN)."""
    _lib.load().lsk_set_linear_wait_limit(int(polls))


LINEAR_WAIT_LIMIT_DEFAULT = 1 << 22


def kernel_durations_us(fn, max_dispatches: int = 4096) -> list[float]:
    """Run fn() (eager launches of this library's kernels on the current
    stream) with every dispatch timed by events bound to the dispatch itself
    (lsk_dispatch_timing_begin/end), and return each kernel's own duration in
    microseconds, in launch order.  Waits for the timed kernels."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("dispatch timing cannot run inside a graph capture")
    lib = _lib.load()
    _lib.check(lib.lsk_dispatch_timing_begin(int(max_dispatches)), "lsk_dispatch_timing_begin")
    durations = (ctypes.c_float * int(max_dispatches))()
    count = ctypes.c_int(0)
    try:
        fn()
    finally:
        status = lib.lsk_dispatch_timing_end(durations, int(max_dispatches), ctypes.byref(count))
    _lib.check(status, "lsk_dispatch_timing_end")
    return [float(durations[i]) for i in range(min(count.value, int(max_dispatches)))]


def linear_error(workspace: torch.Tensor) -> int:
    """Read and clear the error word of a prefill workspace (0 = no bounded
    wait gave up since the last read).  Synchronous."""
    err = ctypes.c_int(0)
    _lib.check(_lib.load().lsk_linear_error(workspace.data_ptr(), ctypes.byref(err)), "lsk_linear_error")
    return err.value


def linear(x: torch.Tensor, weight: PackedWeight, *, epilogue: int = _lib.EPI_NONE,
           residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
           workspace: torch.Tensor | None | str = "auto") -> torch.Tensor:
    """out[..., N'] = epilogue(x[..., K] . W^T) on the GPU.

    epilogue EPI_NONE (N' = N), EPI_SILU_MUL (gate_up layout, N' = N/2,
    SiLU(gate)*up), EPI_RESIDUAL_ADD (N' = N, residual + projection).
    workspace: "auto" uses the split-K workspace of the device and current
    stream for prefill shapes (prefill_workspace), None runs one
    workgroup per output block with no waits (the form for prefill calls
    that may run concurrently with other kernels on the device), a uint8
    device tensor is used as given.  A split-K workgroup whose bounded wait
    gives up (possible only when another kernel holds CUs the split needs)
    sets the workspace's error word (linear_error) and writes NaN to its
    tiles."""
    if not isinstance(weight, PackedWeight):
        raise ValueError("weight must be a PackedWeight (pack it with leanstack_amd.layout / leanserve)")
    lib = _lib.load()
    x2, m, ldx = _rows(x, weight.k, "x")
    n_out = weight.n // 2 if epilogue == _lib.EPI_SILU_MUL else weight.n
    if out is not None:
        _check_out(out, m, n_out, torch.bfloat16)
    r2 = None
    if residual is not None:
        r2, rm, ldr = _rows(residual, weight.n, "residual")
        if rm != m:
            raise ValueError(f"residual has {rm} rows, x has {m}")
    _require_device(x, "x")
    _require_device(weight.data, "weight")
    if out is None:
        out = torch.empty((*x.shape[:-1], n_out), device=x.device, dtype=torch.bfloat16)
    _require_device(out, "out")
    res_ptr, ldr = (None, 0) if r2 is None else (r2.data_ptr(), ldr)
    if r2 is not None:
        _require_device(r2, "residual")
    if m == 0:
        return out  # no rows: nothing to launch (F.linear returns the empty result too)
    if isinstance(workspace, str):
        if workspace != "auto":
            raise ValueError(f"workspace must be 'auto', None or a tensor, not {workspace!r}")
        workspace = prefill_workspace(x.device, m, weight.n, weight.k) if m > _lib.DECODE_MAX_M else None
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        _require_device(workspace, "workspace")
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    dev = _one_device(x, (weight.data, "weight"), (out, "out"), (r2, "residual"), (workspace, "workspace"))
    with torch.cuda.device(dev):
        status = lib.lsk_linear_bf16(
            weight.data.data_ptr(), weight.layout, weight.n, weight.k,
            x2.data_ptr(), m, ldx,
            out.data_ptr(), n_out,
            epilogue, res_ptr, ldr,
            ws_ptr, ws_bytes, stream_handle(),
        )
    _lib.check(status, "lsk_linear_bf16")
    return out


def rmsnorm_linear(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, weight: PackedWeight, *,
                   epilogue: int = _lib.EPI_NONE, residual: torch.Tensor | None = None,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """out[..., N'] = epilogue(rms_norm(x) . W^T) for 1..16 rows of x, the
    RMSNorm (F.rms_norm over the last dim with `norm_weight` and `eps`, one
    bf16 rounding) computed inside the projection kernel."""
    if not isinstance(weight, PackedWeight):
        raise ValueError("weight must be a PackedWeight (pack it with leanstack_amd.layout / leanserve)")
    lib = _lib.load()
    x2, m, ldx = _rows(x, weight.k, "x")
    nw = norm_weight.reshape(-1)
    if nw.dtype != torch.bfloat16 or nw.numel() != weight.k:
        raise ValueError(f"norm_weight must be a bfloat16 [{weight.k}] tensor, got {nw.dtype} {tuple(norm_weight.shape)}")
    n_out = weight.n // 2 if epilogue == _lib.EPI_SILU_MUL else weight.n
    if out is not None:
        _check_out(out, m, n_out, torch.bfloat16)
    r2 = None
    if residual is not None:
        r2, rm, ldr = _rows(residual, weight.n, "residual")
        if rm != m:
            raise ValueError(f"residual has {rm} rows, x has {m}")
    _require_device(x, "x")
    _require_device(weight.data, "weight")
    _require_device(norm_weight, "norm_weight")
    if nw.stride(0) != 1 or nw.data_ptr() % 16:
        nw = nw.contiguous() if nw.stride(0) != 1 else nw.clone()
    if out is None:
        out = torch.empty((*x.shape[:-1], n_out), device=x.device, dtype=torch.bfloat16)
    _require_device(out, "out")
    res_ptr, ldr = (None, 0) if r2 is None else (r2.data_ptr(), ldr)
    if r2 is not None:
        _require_device(r2, "residual")
    if m == 0:
        return out
    dev = _one_device(x, (weight.data, "weight"), (nw, "norm_weight"), (out, "out"), (r2, "residual"))
    with torch.cuda.device(dev):
        status = lib.lsk_rmsnorm_linear_bf16(
            weight.data.data_ptr(), weight.layout, weight.n, weight.k,
            x2.data_ptr(), m, ldx,
            nw.data_ptr(), float(eps),
            out.data_ptr(), n_out,
            epilogue, res_ptr, ldr, stream_handle(),
        )
    _lib.check(status, "lsk_rmsnorm_linear_bf16")
    return out


_attention_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def attention_workspace(device: torch.device, n_q: int, n_kv: int, head_dim: int,
                        max_seq_len: int) -> torch.Tensor:
    """The decode attention workspace of `device` for the current stream
    (zero-filled once, left zero-filled by every call), large enough for this
    geometry.  Calls on other streams get their own."""
    nbytes = _lib.load().lsk_attention_workspace_bytes(n_q, n_kv, head_dim, max_seq_len)
    if nbytes == 0:
        raise ValueError(f"no attention workspace for n_q={n_q}, n_kv={n_kv}, head_dim={head_dim}, "
                         f"max_seq_len={max_seq_len}")
    return _device_workspace(_attention_workspaces, device, nbytes, "attention")


def decode_attention(qkv: torch.Tensor, q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, eps: float,
                     cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     pos: int | torch.Tensor, scale: float, *, num_attention_heads: int, num_key_value_heads: int,
                     out: torch.Tensor | None = None, workspace: torch.Tensor | str = "auto") -> torch.Tensor:
    """One decode token of one layer between QKV and o_proj: per-head q/k
    RMSNorm and RoPE of the raw QKV row, k and v written to row `pos` of the
    layer's caches ([n_kv, max_seq_len, d] bf16, batch 1), and GQA attention
    over rows 0..pos.  Returns out [n_q * d] bf16.  The caller advances its
    cache cursor.  workspace: "auto" (attention_workspace), or a zero-filled
    uint8 device tensor of lsk_attention_workspace_bytes() bytes.

    pos: an int (cos / sin are this position's rows, d/2 values each), or a
    one-element int32 device tensor read by the kernel (cos / sin are then the
    whole [max_seq_len, d/2] tables): one launch for any position, so a
    captured HIP graph can be replayed token after token with the caller
    writing the next position into that tensor.  Out-of-range device
    positions change nothing."""
    lib = _lib.load()
    n_q, n_kv = num_attention_heads, num_key_value_heads
    on_device = isinstance(pos, torch.Tensor)
    for t, what in ((qkv, "qkv"), (q_norm_weight, "q_norm_weight"), (k_norm_weight, "k_norm_weight"), (cos, "cos"),
                    (sin, "sin"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _require_device(t, what)
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{what} must be bfloat16, got {t.dtype}")
    if k_cache.dim() != 3 or k_cache.shape != v_cache.shape or k_cache.shape[0] != n_kv:
        raise ValueError(f"k_cache / v_cache must be [n_kv={n_kv}, max_seq_len, head_dim], got "
                         f"{tuple(k_cache.shape)} / {tuple(v_cache.shape)}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache / v_cache must be contiguous")
    d, s_max = k_cache.shape[2], k_cache.shape[1]
    if qkv.numel() != (n_q + 2 * n_kv) * d:
        raise ValueError(f"qkv has {qkv.numel()} values, expected {(n_q + 2 * n_kv) * d}")
    rope_len = s_max * (d // 2) if on_device else d // 2
    if q_norm_weight.numel() != d or k_norm_weight.numel() != d or cos.numel() != rope_len or sin.numel() != rope_len:
        where = f"the whole [{s_max}, {d // 2}] tables" if on_device else "this position's row"
        raise ValueError(f"norm weights must hold {d} values and cos / sin {rope_len} ({where})")
    if on_device:
        _require_device(pos, "pos")
        if pos.dtype != torch.int32 or pos.numel() != 1:
            raise ValueError("a device pos must be a one-element int32 tensor")
    flat = [t.reshape(-1).contiguous() for t in (qkv, q_norm_weight, k_norm_weight, cos, sin)]
    if out is None:
        out = torch.empty((n_q * d,), device=qkv.device, dtype=torch.bfloat16)
    if out.dtype != torch.bfloat16 or out.numel() != n_q * d or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous bfloat16 tensor of {n_q * d} values")
    if isinstance(workspace, str):
        if workspace != "auto":
            raise ValueError(f"workspace must be 'auto' or a tensor, not {workspace!r}")
        workspace = attention_workspace(qkv.device, n_q, n_kv, d, s_max)
    _require_device(workspace, "workspace")
    dev = _one_device(qkv, (q_norm_weight, "q_norm_weight"), (k_norm_weight, "k_norm_weight"), (cos, "cos"),
                      (sin, "sin"), (k_cache, "k_cache"), (v_cache, "v_cache"), (out, "out"),
                      (workspace, "workspace"), (pos if on_device else None, "pos"))
    common = (flat[0].data_ptr(), n_q, n_kv, d, flat[1].data_ptr(), flat[2].data_ptr(), float(eps),
              flat[3].data_ptr(), flat[4].data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), s_max)
    tail = (float(scale), out.data_ptr(), workspace.data_ptr(), workspace.numel() * workspace.element_size())
    with torch.cuda.device(dev):
        tail += (stream_handle(),)
        if on_device:
            status = lib.lsk_decode_attention_at_bf16(*common, pos.data_ptr(), *tail)
        else:
            status = lib.lsk_decode_attention_bf16(*common, int(pos), *tail)
    _lib.check(status, "lsk_decode_attention_at_bf16" if on_device else "lsk_decode_attention_bf16")
    return out


class LmHeadWorkspace:
    """Device workspace of the greedy head, sized once per (M, V, K): a status
    word and the per-workgroup argmax partials.  Zero-filled here; every call
    leaves the partials zero again, so it is never cleared between calls.
    Calls that share one must be stream-ordered."""

    def __init__(self, m: int, v: int, k: int, device: torch.device | str) -> None:
        nbytes = _lib.load().lsk_workspace_bytes(_lib.OP_LM_HEAD_ARGMAX, m, v, k)
        if nbytes == 0:
            raise ValueError(f"no lm_head workspace for M={m}, V={v}, K={k}")
        self.m, self.v, self.k = m, v, k
        self.buffer = torch.zeros(nbytes, device=device, dtype=torch.uint8)

    def give_ups(self) -> int:
        """Argmax stages (rows) that gave up waiting for a partial since the
        workspace was made (their out_idx was -1); 0 while every grid runs to
        its end.  Synchronizes with the device."""
        return int(self.buffer[:4].view(torch.int32).item())


def lm_head_argmax(hidden: torch.Tensor, weight: PackedWeight, *, logits_mode: int = _lib.LOGITS_FP32,
                   logits_out: torch.Tensor | None = None, workspace: LmHeadWorkspace | None = None,
                   out: torch.Tensor | None = None, norm_weight: torch.Tensor | None = None,
                   eps: float = 1e-6) -> torch.Tensor:
    """Greedy token per row: int64 [M] = argmax over the vocab of hidden . W^T.

    logits_mode LOGITS_FP32 compares fp32 scores (cuTile head); LOGITS_BF16
    compares bf16-rounded logits (torch.mv head).  Lowest index wins ties.
    norm_weight: the final RMSNorm ([K] bf16, with eps) applied to hidden in
    the kernel (K = 2560, M <= 8)."""
    if not isinstance(weight, PackedWeight) or weight.layout != _lib.LAYOUT_MFMA16X32:
        raise ValueError("lm_head weight must be a PackedWeight in the mfma16x32 layout")
    lib = _lib.load()
    h2, m, ldx = _rows(hidden, weight.k, "hidden")
    v = weight.n
    if out is not None and (out.dtype != torch.long or out.numel() < m or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous int64 tensor of at least {m} values "
                         f"(got {out.dtype} {tuple(out.shape)})")
    if logits_out is not None:
        if logits_out.dtype != torch.float32 or logits_out.numel() != m * v or not logits_out.is_contiguous():
            raise ValueError(f"logits_out must be a contiguous float32 tensor of {m}x{v}")
    if norm_weight is not None and (norm_weight.dtype != torch.bfloat16 or norm_weight.numel() != weight.k):
        raise ValueError(f"norm_weight must be a bfloat16 tensor of {weight.k} values")
    _require_device(hidden, "hidden")
    _require_device(weight.data, "weight")
    if m == 0:  # no rows: an empty index tensor, as torch.argmax over [0, V] scores gives
        return out if out is not None else torch.empty((0,), device=hidden.device, dtype=torch.long)
    if workspace is None or workspace.m < m or workspace.v != v or workspace.k != weight.k:
        workspace = LmHeadWorkspace(m, v, weight.k, hidden.device)
    if out is None:
        out = torch.empty((m,), device=hidden.device, dtype=torch.long)
    _require_device(out, "out")
    logits_ptr = None
    if logits_out is not None:
        _require_device(logits_out, "logits_out")
        logits_ptr = logits_out.data_ptr()
    dev = _one_device(hidden, (weight.data, "weight"), (out, "out"), (logits_out, "logits_out"),
                      (norm_weight, "norm_weight"), (workspace.buffer, "workspace"))
    if norm_weight is not None:
        _require_device(norm_weight, "norm_weight")
        nw = norm_weight.reshape(-1).contiguous()
        with torch.cuda.device(dev):
            status = lib.lsk_rmsnorm_lm_head_argmax_bf16(
                weight.data.data_ptr(), weight.layout, v, weight.k, h2.data_ptr(), m, ldx, nw.data_ptr(), float(eps),
                logits_ptr, logits_mode, out.data_ptr(), workspace.buffer.data_ptr(), workspace.buffer.numel(),
                stream_handle(),
            )
        _lib.check(status, "lsk_rmsnorm_lm_head_argmax_bf16")
        return out
    with torch.cuda.device(dev):
        status = lib.lsk_lm_head_argmax_bf16(
            weight.data.data_ptr(), weight.layout, v, weight.k,
            h2.data_ptr(), m, ldx,
            logits_ptr, logits_mode,
            out.data_ptr(),
            workspace.buffer.data_ptr(), workspace.buffer.numel(), stream_handle(),
        )
    _lib.check(status, "lsk_lm_head_argmax_bf16")
    return out


def lm_head_argmax_noalloc(hidden: torch.Tensor, weight: PackedWeight, out: torch.Tensor, *,
                           logits_mode: int = _lib.LOGITS_FP32, logits_out: torch.Tensor | None = None) -> torch.Tensor:
    """lm_head_argmax with no allocation anywhere on the call: the argmax
    partials use the library's static device scratch
    (lsk_lm_head_argmax_noalloc_bf16), `out` (int64, at least M values) is
    the caller's, and `hidden` must already be contiguous [M, K] bf16 rows.
    Usable under HIP graph capture; calls on one device that are not
    stream-ordered with each other race on the scratch."""
    if not isinstance(weight, PackedWeight) or weight.layout != _lib.LAYOUT_MFMA16X32:
        raise ValueError("lm_head weight must be a PackedWeight in the mfma16x32 layout")
    if hidden.dtype != torch.bfloat16 or hidden.shape[-1] != weight.k or not hidden.is_contiguous():
        raise ValueError(f"hidden must be contiguous bfloat16 [M, {weight.k}] rows")
    m = hidden.numel() // weight.k
    if out.dtype != torch.long or out.numel() < m or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous int64 tensor of at least {m} values")
    if logits_out is not None and (logits_out.dtype != torch.float32 or logits_out.numel() != m * weight.n
                                   or not logits_out.is_contiguous()):
        raise ValueError(f"logits_out must be a contiguous float32 tensor of {m}x{weight.n}")
    for t, what in ((hidden, "hidden"), (weight.data, "weight"), (out, "out")):
        _require_device(t, what)
    if m == 0:
        return out
    dev = _one_device(hidden, (weight.data, "weight"), (out, "out"), (logits_out, "logits_out"))
    with torch.cuda.device(dev):
        status = _lib.load().lsk_lm_head_argmax_noalloc_bf16(
            weight.data.data_ptr(), weight.layout, weight.n, weight.k, hidden.data_ptr(), m, weight.k,
            logits_out.data_ptr() if logits_out is not None else None, logits_mode, out.data_ptr(), stream_handle())
    _lib.check(status, "lsk_lm_head_argmax_noalloc_bf16")
    return out


class StackStep:
    """A prepared stack program: many projections at the same M in one
    persistent launch (lsk_stack_prepare / lsk_stack_run).

    `projections` is a list of dicts with keys x, weight (PackedWeight), out,
    and optionally epilogue, residual, depends_on (index of an earlier entry:
    every entry up to it finishes before this one reads its inputs).  The
    program holds the tensors' addresses, so x, out and residual are used in
    place (rows of unit column stride, row strides a multiple of 8 elements,
    16-byte aligned): one entry's out can be a later entry's x.  A tensor
    that would need a copy is refused."""

    def __init__(self, projections: list[dict], m: int, device: torch.device | str) -> None:
        lib = _lib.load()
        device = torch.device(device)
        count = len(projections)
        arr = (_lib.Projection * count)()
        self._keep = []  # tensors whose pointers the program holds

        def in_place(t: torch.Tensor, t2: torch.Tensor, what: str) -> None:
            if t2.data_ptr() != t.data_ptr() or t2.stride(-1) != 1:
                raise ValueError(f"{what} must be usable in place (unit column stride, row stride a multiple "
                                 f"of 8, 16-byte aligned): the program holds its address")
            if t.device.type != "cuda" or t.device.index != (device.index if device.index is not None
                                                             else torch.cuda.current_device()):
                raise ValueError(f"{what} is on {t.device}, the program on {device}")

        for i, spec in enumerate(projections):
            w = spec["weight"]
            if not isinstance(w, PackedWeight):
                raise ValueError(f"projection {i}: weight must be a PackedWeight")
            x, out = spec["x"], spec["out"]
            epi = spec.get("epilogue", _lib.EPI_NONE)
            x2, xm, ldx = _rows(x, w.k, f"projection {i} x")
            if xm != m:
                raise ValueError(f"projection {i}: x has {xm} rows, the step runs M={m}")
            in_place(x, x2, f"projection {i} x")
            in_place(w.data, w.data, f"projection {i} weight")
            n_out = w.n // 2 if epi == _lib.EPI_SILU_MUL else w.n
            if out.dtype != torch.bfloat16 or out.shape[-1] != n_out or out.numel() != m * n_out:
                raise ValueError(f"projection {i}: out must be bfloat16 [{m}, {n_out}]")
            o2 = out.reshape(-1, n_out)
            in_place(out, o2, f"projection {i} out")
            ldy = o2.stride(0) if m > 1 else n_out
            res = spec.get("residual")
            res_ptr, ldr = None, 0
            if res is not None:
                r2, rm, ldr = _rows(res, w.n, f"projection {i} residual")
                if rm != m:
                    raise ValueError(f"projection {i}: residual has {rm} rows, the step runs M={m}")
                in_place(res, r2, f"projection {i} residual")
                res_ptr = r2.data_ptr()
                self._keep.append(r2)
            self._keep += [x2, o2, w.data]
            arr[i] = _lib.Projection(w.data.data_ptr(), w.layout, w.n, w.k, x2.data_ptr(), ldx, o2.data_ptr(), ldy,
                                     epi, res_ptr, ldr, int(spec.get("depends_on", -1)))
        self.count = count
        self.m = m
        with torch.cuda.device(device):
            self.program = torch.empty(lib.lsk_stack_program_bytes(count), dtype=torch.uint8, device=device)
            self.workspace = torch.zeros(lib.lsk_stack_workspace_bytes(count), dtype=torch.uint8, device=device)
            status = lib.lsk_stack_prepare(arr, count, m, self.program.data_ptr(), self.program.numel())
        _lib.check(status, "lsk_stack_prepare")

    def launch(self) -> None:
        lib = _lib.load()
        with torch.cuda.device(self.program.device):
            status = lib.lsk_stack_run(self.program.data_ptr(), self.count, self.workspace.data_ptr(),
                                       self.workspace.numel(), stream_handle())
        _lib.check(status, "lsk_stack_run")

    def error(self) -> int:
        """Read and clear the error word (synchronises): 0 if every wait completed."""
        lib = _lib.load()
        torch.cuda.synchronize(self.workspace.device)
        out = ctypes.c_int(0)
        _lib.check(lib.lsk_stack_error(self.workspace.data_ptr(), ctypes.byref(out)), "lsk_stack_error")
        return out.value
