"""Typed torch-tensor wrappers over the C ABI (one function per entry point).

Each wrapper validates devices, dtypes and shapes on the host, then passes raw
pointers, byte strides and torch's current HIP stream to ``libsaintkv.so``.
Nothing here computes on the CPU; the wrappers only describe memory.
"""

from __future__ import annotations

import math

import torch

from saint_kv import _lib

INT32 = torch.int32


def _require_gpu(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{name} is on {t.device}; saint_kv runs only on a ROCm GPU (no CPU fallback)",
        )


def _require_i32(t: torch.Tensor, name: str, shape: tuple[int, ...] | None = None) -> None:
    _require_gpu(t, name)
    if t.dtype != INT32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 tensor; got {t.dtype}")
    if shape is not None and tuple(t.shape) != shape:
        raise ValueError(f"{name} must have shape {shape}; got {tuple(t.shape)}")


def row_bytes_of(pool: torch.Tensor) -> int:
    """Bytes of one row of a pool shaped [n_pages, block_size, *row]."""
    if pool.dim() < 3:
        raise ValueError(f"pool must be [n_pages, block_size, *row]; got {tuple(pool.shape)}")
    return math.prod(pool.shape[2:]) * pool.element_size()


def _check_pool(pool: torch.Tensor) -> tuple[int, int, int]:
    _require_gpu(pool, "pool")
    if not pool.is_contiguous():
        raise ValueError("pool must be contiguous")
    rb = row_bytes_of(pool)
    if rb % 16:
        raise ValueError(f"pool row must be a multiple of 16 bytes; got {rb}")
    return pool.shape[0], pool.shape[1], rb


def _row_view_strides(t: torch.Tensor, row_bytes: int, name: str) -> tuple[int, int]:
    """(seq stride, row stride) in bytes of a [B, T, *row] tensor with dense rows."""
    if t.dim() < 3:
        raise ValueError(f"{name} must be 3D or more (B, T, *row); got {tuple(t.shape)}")
    es = t.element_size()
    if math.prod(t.shape[2:]) * es != row_bytes:
        raise ValueError(
            f"{name} rows hold {math.prod(t.shape[2:]) * es} bytes; the pool row holds {row_bytes}",
        )
    inner = t[0, 0] if t.shape[0] and t.shape[1] else None
    if inner is not None and not inner.is_contiguous():
        raise ValueError(f"{name} rows must be contiguous")
    return t.stride(0) * es, t.stride(1) * es


def _n_new_args(n_new: int | torch.Tensor, batch: int) -> tuple[int | None, int]:
    if isinstance(n_new, torch.Tensor):
        _require_i32(n_new, "n_new", (batch,))
        return n_new.data_ptr(), 0
    if int(n_new) < 0:
        raise ValueError(f"n_new must be >= 0; got {n_new}")
    return None, int(n_new)


def free_stack_init(free_stack: torch.Tensor, free_top: torch.Tensor,
                    order: torch.Tensor | None = None) -> None:
    """Fill the free stack so pops return ``order`` (default 0, 1, 2, ...)."""
    n = free_stack.numel()
    _require_i32(free_stack, "free_stack")
    _require_i32(free_top, "free_top", (1,))
    if order is not None:
        _require_i32(order, "order", (n,))
    _lib.call("skv_free_stack_init", free_stack.data_ptr(), free_top.data_ptr(),
              _lib.ptr(order), n, _lib.stream_handle(free_stack.device))


def reserve(free_stack: torch.Tensor, free_top: torch.Tensor, block_table: torch.Tensor,
            seq_lens: torch.Tensor, n_new: int | torch.Tensor, block_size: int,
            status: torch.Tensor | None = None, max_pages: int | None = None) -> None:
    """Pop pages for the next ``n_new`` rows of every sequence and advance ``seq_lens``."""
    _require_i32(free_stack, "free_stack")
    _require_i32(free_top, "free_top", (1,))
    _require_i32(block_table, "block_table")
    if block_table.dim() != 2:
        raise ValueError("block_table must be 2D [batch, max_pages]")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    if status is not None:
        _require_i32(status, "status", (1,))
    n_ptr, n_uni = _n_new_args(n_new, batch)
    _lib.call("skv_reserve", free_stack.data_ptr(), free_top.data_ptr(), free_stack.numel(),
              block_table.data_ptr(),
              bt_stride, bt_stride if max_pages is None else max_pages, seq_lens.data_ptr(),
              n_ptr, n_uni, batch, block_size, _lib.ptr(status),
              _lib.stream_handle(block_table.device))


def paged_append(pool: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                 src: torch.Tensor, n_new: int | torch.Tensor) -> None:
    """Write rows ``[seq_lens-n_new, seq_lens)`` of each sequence from ``src`` (B, T, *row)."""
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    _require_gpu(src, "src")
    if src.shape[0] != batch:
        raise ValueError(f"src batch {src.shape[0]} != block_table batch {batch}")
    s_seq, s_row = _row_view_strides(src, rb, "src")
    n_ptr, n_uni = _n_new_args(n_new, batch)
    if n_ptr is None and n_uni > src.shape[1]:
        raise ValueError(f"n_new={n_uni} exceeds src length {src.shape[1]}")
    _lib.call("skv_paged_append", pool.data_ptr(), rb, bs, n_pages, block_table.data_ptr(),
              bt_stride, seq_lens.data_ptr(), n_ptr, n_uni, src.data_ptr(), s_seq, s_row,
              src.shape[1], batch, _lib.stream_handle(pool.device))


def _capacity_rows(t: torch.Tensor, rb: int) -> int:
    """Rows of ``rb`` bytes between t's first element and the end of its storage."""
    avail = t.untyped_storage().nbytes() - t.storage_offset() * t.element_size()
    return max(avail, 0) // rb


def _dst_args(out: torch.Tensor, rb: int, batch: int,
              row_offsets: torch.Tensor | None) -> tuple[int | None, int, int]:
    _require_gpu(out, "out")
    es = out.element_size()
    cap = _capacity_rows(out, rb)
    if row_offsets is not None:
        if row_offsets.dtype != torch.int64 or tuple(row_offsets.shape) != (batch,):
            raise ValueError("row_offsets must be int64 [batch]")
        _require_gpu(row_offsets, "row_offsets")
        if not out.is_contiguous():
            raise ValueError("packed out must be contiguous")
        return row_offsets.data_ptr(), 0, cap
    if out.dim() < 3 or out.shape[0] != batch:
        raise ValueError(f"out must be [batch={batch}, rows, *row]; got {tuple(out.shape)}")
    if math.prod(out.shape[2:]) * es != rb or (batch and not out[0].is_contiguous()):
        raise ValueError("out rows must be dense and match the pool row size")
    seq_stride_bytes = out.stride(0) * es
    if seq_stride_bytes % rb:
        raise ValueError("out sequence stride must be a whole number of rows")
    return None, seq_stride_bytes // rb, cap


def paged_gather(pool: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                 out: torch.Tensor, row_offsets: torch.Tensor | None = None) -> torch.Tensor:
    """Copy rows ``[0, seq_lens[b])`` of every sequence, in order, into ``out``."""
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    off_ptr, seq_rows, cap = _dst_args(out, rb, batch, row_offsets)
    _lib.call("skv_paged_gather", out.data_ptr(), off_ptr, seq_rows, cap, pool.data_ptr(), rb, bs,
              n_pages, block_table.data_ptr(), bt_stride, seq_lens.data_ptr(), batch,
              _lib.stream_handle(pool.device))
    return out


def append_gather(pool: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                  src: torch.Tensor, n_new: int | torch.Tensor, out: torch.Tensor,
                  row_offsets: torch.Tensor | None = None) -> torch.Tensor:
    """Fused decode step: append ``src`` rows to the pool and gather every sequence into ``out``."""
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    _require_gpu(src, "src")
    if src.shape[0] != batch:
        raise ValueError(f"src batch {src.shape[0]} != block_table batch {batch}")
    s_seq, s_row = _row_view_strides(src, rb, "src")
    n_ptr, n_uni = _n_new_args(n_new, batch)
    off_ptr, seq_rows, cap = _dst_args(out, rb, batch, row_offsets)
    _lib.call("skv_append_gather", out.data_ptr(), off_ptr, seq_rows, cap, pool.data_ptr(), rb,
              bs, n_pages, block_table.data_ptr(), bt_stride, seq_lens.data_ptr(), n_ptr, n_uni,
              src.data_ptr(), s_seq, s_row, src.shape[1], batch, _lib.stream_handle(pool.device))
    return out
