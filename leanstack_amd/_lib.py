"""ctypes binding of libleanstack_amd.so (include/leanstack_amd.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already loaded (same SONAME).  There is no fallback: if the
library is missing or cannot be loaded, every projection entry point raises.
"""

from __future__ import annotations

import ctypes
import re
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded first: the library shares its HIP runtime)

LIBRARY_PATH = Path(__file__).resolve().parent / "libleanstack_amd.so"
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "leanstack_amd.h"

ABI_VERSION = 3

# enum lsk_layout / lsk_epilogue / lsk_op / lsk_logits_mode / lsk_status
LAYOUT_ROWMAJOR = 0
LAYOUT_MFMA16X32 = 1
LAYOUT_MFMA16X32_GATEUP = 2
EPI_NONE = 0
EPI_SILU_MUL = 1
EPI_RESIDUAL_ADD = 2
OP_LINEAR = 0
OP_LM_HEAD_ARGMAX = 1
LOGITS_FP32 = 0
LOGITS_BF16 = 1
OK = 0
ERR_INVALID = -1
ERR_LAYOUT = -2
ERR_HIP = -3
ERR_WORKSPACE = -4

# Largest M served by the decode/verify kernel (kDecodeMaxM in the library).
DECODE_MAX_M = 16
# Largest activation row stride in elements (kMaxActivationStride).
MAX_ACTIVATION_STRIDE = (1 << 22) - 8

_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_c_void = ctypes.c_void_p

# Argument/return types of every exported function, in header order.
_SIGNATURES: dict[str, tuple[type | None, list]] = {
    "lsk_abi_version": (_c_int, []),
    "lsk_last_error": (ctypes.c_char_p, []),
    "lsk_packed_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "lsk_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "lsk_pack_bf16": (_c_int, [_c_void, _c_int, _c_int, _c_int, _c_void]),
    "lsk_unpack_bf16": (_c_int, [_c_void, _c_int, _c_int, _c_int, _c_void]),
    "lsk_linear_plan": (_c_int, [_c_int, _c_int, _c_int, _c_size, ctypes.POINTER(_c_int)]),
    "lsk_linear_bf16": (
        _c_int,
        [_c_void, _c_int, _c_int, _c_int, _c_void, _c_int, _c_int, _c_void, _c_int, _c_int, _c_void, _c_int,
         _c_void, _c_size, _c_void],
    ),
    "lsk_rmsnorm_linear_bf16": (
        _c_int,
        [_c_void, _c_int, _c_int, _c_int, _c_void, _c_int, _c_int, _c_void, ctypes.c_float, _c_void, _c_int, _c_int,
         _c_void, _c_int, _c_void],
    ),
    "lsk_attention_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "lsk_decode_attention_bf16": (
        _c_int,
        [_c_void, _c_int, _c_int, _c_int, _c_void, _c_void, ctypes.c_float, _c_void, _c_void, _c_void, _c_void, _c_int,
         _c_int, ctypes.c_float, _c_void, _c_void, _c_size, _c_void],
    ),
    "lsk_decode_attention_at_bf16": (
        _c_int,
        [_c_void, _c_int, _c_int, _c_int, _c_void, _c_void, ctypes.c_float, _c_void, _c_void, _c_void, _c_void, _c_int,
         _c_void, ctypes.c_float, _c_void, _c_void, _c_size, _c_void],
    ),
    "lsk_lm_head_argmax_bf16": (
        _c_int,
        [_c_void, _c_int, _c_int, _c_int, _c_void, _c_int, _c_int, _c_void, _c_int, _c_void, _c_void, _c_size,
         _c_void],
    ),
    "lsk_rmsnorm_lm_head_argmax_bf16": (
        _c_int,
        [_c_void, _c_int, _c_int, _c_int, _c_void, _c_int, _c_int, _c_void, ctypes.c_float, _c_void, _c_int, _c_void,
         _c_void, _c_size, _c_void],
    ),
    "lsk_lm_head_argmax_noalloc_bf16": (
        _c_int,
        [_c_void, _c_int, _c_int, _c_int, _c_void, _c_int, _c_int, _c_void, _c_int, _c_void, _c_void],
    ),
}

class Projection(ctypes.Structure):
    """struct lsk_projection (include/leanstack_amd.h)."""

    _fields_ = [
        ("w_packed", _c_void),
        ("layout_id", _c_int),
        ("N", _c_int),
        ("K", _c_int),
        ("x", _c_void),
        ("ldx", _c_int),
        ("y", _c_void),
        ("ldy", _c_int),
        ("epilogue", _c_int),
        ("residual", _c_void),
        ("ldr", _c_int),
        ("depends_on", _c_int),
    ]


_SIGNATURES.update({
    "lsk_stack_program_bytes": (_c_size, [_c_int]),
    "lsk_stack_workspace_bytes": (_c_size, [_c_int]),
    "lsk_stack_prepare": (_c_int, [ctypes.POINTER(Projection), _c_int, _c_int, _c_void, _c_size]),
    "lsk_stack_run": (_c_int, [_c_void, _c_int, _c_void, _c_size, _c_void]),
    "lsk_stack_error": (_c_int, [_c_void, ctypes.POINTER(_c_int)]),
    "lsk_linear_error": (_c_int, [_c_void, ctypes.POINTER(_c_int)]),
    "lsk_set_linear_wait_limit": (None, [ctypes.c_uint]),
    "lsk_dispatch_timing_begin": (_c_int, [_c_int]),
    "lsk_dispatch_timing_end": (_c_int, [ctypes.POINTER(ctypes.c_float), _c_int, ctypes.POINTER(_c_int)]),
    "lsk_probe_workspace_bytes": (_c_size, []),
    "lsk_probe_mfma_rate": (_c_int, [_c_int, _c_int, _c_void, _c_void]),
    "lsk_probe_stream_step": (
        _c_int, [_c_void, _c_size, ctypes.POINTER(ctypes.c_longlong), _c_int, _c_int, _c_int, _c_void, _c_size, _c_void]),
})

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class LibraryMissingError(RuntimeError):
    """The gfx950 library is not built or cannot be loaded."""


def header_functions(header: Path = HEADER_PATH) -> list[str]:
    """Names of the functions include/leanstack_amd.h declares."""
    text = header.read_text(encoding="utf-8")
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(lsk_[a-z0-9_]+)\s*\(", text)


def load() -> ctypes.CDLL:
    """Load (once) and return the library, with argument types declared."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.exists():
            raise LibraryMissingError(
                f"{LIBRARY_PATH} is not built; run `python -m leanstack_amd.build` (hipcc, gfx950)"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as exc:
            raise LibraryMissingError(f"cannot load {LIBRARY_PATH}: {exc}") from exc
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.lsk_abi_version()
        if version != ABI_VERSION:
            raise LibraryMissingError(f"library ABI {version} != expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def last_error() -> str:
    raw = load().lsk_last_error()
    return raw.decode("utf-8", "replace") if raw else ""


def check(status: int, what: str) -> None:
    """Raise for a negative lsk_status: ValueError for argument/layout/workspace
    errors (rejected before launch), RuntimeError for HIP failures."""
    if status == OK:
        return
    message = f"{what}: {last_error()}"
    if status in (ERR_INVALID, ERR_LAYOUT, ERR_WORKSPACE):
        raise ValueError(message)
    raise RuntimeError(message)
