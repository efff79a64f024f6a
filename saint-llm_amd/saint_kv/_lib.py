"""ctypes binding of ``libsaintkv.so`` (the C ABI declared in ``include/saintkv.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch
already mapped (both resolve the soname ``libamdhip64.so.7``); streams handed
over from ``torch.cuda.current_stream()`` are therefore valid in the library.

There is no fallback: if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library is mapped)

LIB_PATH = Path(__file__).resolve().parent / "libsaintkv.so"

# Status codes (include/saintkv.h).
SKV_OK = 0
SKV_EINVAL = -1
SKV_EOVERFLOW = -2
SKV_ENOSPC = -3
SKV_EHIP = -4
SKV_ESTATE = -5

SKV_STATUS_MAX_PAGES = 1
SKV_STATUS_NOSPC = 2
SKV_STATUS_BADARG = 4
SKV_STATUS_STACK = 8
SKV_STATUS_UNITS = 16

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float

# name -> argtypes; every function returns int (except skv_last_error).
SIGNATURES: dict[str, list] = {
    "skv_abi_version": [],
    "skv_free_stack_init": [_P, _P, _P, _I64, _P],
    "skv_reserve": [_P, _P, _I64, _P, _I64, _I64, _P, _P, _I32, _I64, _I64, _P, _P],
    "skv_paged_append": [
        _P, _I64, _I64, _I64, _P, _I64, _P, _P, _I32, _P, _I64, _I64, _I64, _I64, _P,
    ],
    "skv_paged_gather": [_P, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P],
    "skv_append_gather": [
        _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _I32, _P, _I64, _I64, _I64,
        _I64, _P,
    ],
    "skv_decode_append_gather": [
        _P, _P, _I64, _P, _I64, _P, _P, _I32, _P, _P, _P, _I64, _I64, _P, _I64, _I64, _P, _I64,
        _I64, _I64, _P, _I64, _I64, _P,
    ],
    "skv_decode_append_gather_noalloc": [
        _P, _P, _I64, _P, _I64, _P, _P, _I32, _P, _P, _P, _I64, _I64, _P, _I64, _I64, _P, _I64,
        _I64, _I64, _I64, _I64, _P,
    ],
    "skv_plan_units": [_P, _P, _I64, _P, _I64, _P, _P, _I32, _P, _P, _I64, _I64, _P, _I64, _I64, _P],
    "skv_copy_slices": [_P, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _P],
    "skv_ring_append": [_P, _I64, _I64, _P, _P, _I32, _P, _I64, _I64, _I64, _I64, _P],
    "skv_ring_read": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P],
    "skv_compress_append": [
        _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I32, _I64, _I64,
        _I32, _I64, _P,
    ],
    "skv_fp8_quant_append": [
        _P, _I64, _I64, _I64, _P, _I64, _P, _P, _I32, _P, _I64, _I64, _I64, _I64, _I64, _P,
    ],
    "skv_fp8_encode_host": [_P, _P, _I64],
    "skv_fp8_decode_host": [_P, _P, _I64],
    "skv_topk_select": [_P, _I64, _I64, _P, _P, _I32, _I64, _P, _I64, _P, _P],
    "skv_topk_select_decode": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _P],
    "skv_indexer_scores": [_P, _P, _P, _I64, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "skv_topk_workspace_words": [],
    "skv_topk_gather": [
        _P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _P, _I64, _I32, _P,
    ],
    "skv_release": [_P, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _P, _P],
    "skv_decode_step": [_P, _P, _P],
    "skv_decode_step_launches": [_P],
    "skv_decode_desc_sizes": [_P],
    "skv_attention_workspace": [_P],
    "skv_decode_attention": [_P, _P, _I64, _P],
    "skv_decode_step_attend_workspace": [_P, _P],
    "skv_decode_step_attend": [_P, _P, _P, _P, _I64, _P],
    "skv_attention_desc_size": [],
    "skv_compact": [ctypes.c_void_p, _I32, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P],
}

# Entry formats and the FP8 entry layout (include/saintkv.h).
SKV_FMT_BF16 = 0
SKV_FMT_FP8 = 1
SKV_FMT_F32 = 2  # fp32 entries from fp32 c/z rows (skv_compress_append only)
SKV_FMT_IN_F32 = 0x100  # skv_compress_append: fp32 c/z rows into bf16 or fp8 entries
SKV_FP8_ROPE_DIMS = 64


def fp8_entry_bytes(channels: int) -> int:
    main = channels - SKV_FP8_ROPE_DIMS
    return main + main // 128 * 4 + 2 * SKV_FP8_ROPE_DIMS


class PoolRef(ctypes.Structure):
    """skv_pool_ref: one pool sharing a block table."""

    _fields_ = [("base", ctypes.c_void_p), ("page_bytes", ctypes.c_int64)]

# entry points returning a size rather than a status code
INT64_RESULTS = {"skv_topk_workspace_words", "skv_attention_workspace", "skv_attention_desc_size",
                 "skv_decode_step_attend_workspace"}

_lib: ctypes.CDLL | None = None


class SaintKVLibraryMissing(RuntimeError):
    """Raised when the HIP library has not been built."""


def load() -> ctypes.CDLL:
    """Load and type the library once; raise if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise SaintKVLibraryMissing(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            " (hipcc --offload-arch=gfx950). There is no CPU fallback.",
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int64 if name in INT64_RESULTS else ctypes.c_int
    lib.skv_last_error.argtypes = []
    lib.skv_last_error.restype = ctypes.c_char_p
    abi = lib.skv_abi_version()
    if abi != 1:
        raise SaintKVLibraryMissing(f"libsaintkv ABI version {abi} != 1 expected by saint_kv")
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().skv_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Map a negative status code onto the reference's exception types."""
    if rc == SKV_OK:
        return
    msg = last_error() or f"{what} failed with code {rc}"
    if rc == SKV_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    fn = getattr(load(), name)
    check(fn(*args), name)


def stream_handle(device: torch.device | None = None) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def topk_workspace_words() -> int:
    return int(load().skv_topk_workspace_words())
