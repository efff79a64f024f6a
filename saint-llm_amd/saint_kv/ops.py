"""Typed torch-tensor wrappers over the C ABI (one function per entry point).

Each wrapper validates devices, dtypes and shapes on the host, then passes raw
pointers, byte strides and torch's current HIP stream to ``libsaintkv.so``.
Nothing here computes on the CPU; the wrappers only describe memory.
"""

from __future__ import annotations

import ctypes
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


def _from_page(block_table: torch.Tensor, seq_lens: torch.Tensor, out: torch.Tensor, bs: int,
               first_page: int, row_offsets: torch.Tensor | None) -> tuple[int, torch.Tensor, torch.Tensor]:
    """(table pointer, lengths, out view) that make a gather start at page
    ``first_page`` of every sequence: the table row from that page on, the
    lengths less its first row, and out from that row on."""
    if first_page == 0:
        return block_table.data_ptr(), seq_lens, out
    if row_offsets is not None:
        raise ValueError("first_page needs out as [batch, rows, *row], not packed rows")
    if not 0 < first_page < block_table.shape[1]:
        raise ValueError(f"first_page must be in [0, {block_table.shape[1]}); got {first_page}")
    # the shifted table row holds bt_stride - first_page pages: clamp there, so
    # that no length reaches past it into the next sequence's row
    lens = torch.clamp(seq_lens - first_page * bs, min=0,
                       max=(block_table.shape[1] - first_page) * bs).to(torch.int32)
    return block_table.data_ptr() + first_page * block_table.element_size(), lens, out[:, first_page * bs:]


def paged_gather(pool: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                 out: torch.Tensor, row_offsets: torch.Tensor | None = None,
                 first_page: int = 0) -> torch.Tensor:
    """Copy rows ``[0, seq_lens[b])`` of every sequence, in order, into ``out``.

    With ``first_page`` > 0 only rows ``[first_page * block_size, seq_lens[b])``
    are copied (to the same rows of ``out``); the rows before are left as they
    are.  A caller that keeps ``out`` as a running copy of the cache refreshes
    it this way in O(new rows) instead of O(length)."""
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    bt_ptr, lens, out_v = _from_page(block_table, seq_lens, out, bs, first_page, row_offsets)
    off_ptr, seq_rows, cap = _dst_args(out_v, rb, batch, row_offsets)
    _lib.call("skv_paged_gather", out_v.data_ptr(), off_ptr, seq_rows, cap, pool.data_ptr(), rb, bs,
              n_pages, bt_ptr, bt_stride, lens.data_ptr(), batch, _lib.stream_handle(pool.device))
    return out


def append_gather(pool: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                  src: torch.Tensor, n_new: int | torch.Tensor, out: torch.Tensor,
                  row_offsets: torch.Tensor | None = None, first_page: int = 0) -> torch.Tensor:
    """Fused decode step: append ``src`` rows to the pool and gather every sequence into ``out``
    (from page ``first_page`` on, as in ``paged_gather``; the appended rows must lie there)."""
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    _require_gpu(src, "src")
    if src.shape[0] != batch:
        raise ValueError(f"src batch {src.shape[0]} != block_table batch {batch}")
    s_seq, s_row = _row_view_strides(src, rb, "src")
    n_ptr, n_uni = _n_new_args(n_new, batch)
    bt_ptr, lens, out_v = _from_page(block_table, seq_lens, out, bs, first_page, row_offsets)
    off_ptr, seq_rows, cap = _dst_args(out_v, rb, batch, row_offsets)
    _lib.call("skv_append_gather", out_v.data_ptr(), off_ptr, seq_rows, cap, pool.data_ptr(), rb,
              bs, n_pages, bt_ptr, bt_stride, lens.data_ptr(), n_ptr, n_uni,
              src.data_ptr(), s_seq, s_row, src.shape[1], batch, _lib.stream_handle(pool.device))
    return out


def unit_table(max_units: int, device: torch.device) -> torch.Tensor:
    """Workspace of skv_decode_append_gather for up to ``max_units`` page units."""
    return torch.zeros(8 + 8 * max_units, dtype=torch.int32, device=device)


def plan_units(free_stack: torch.Tensor, free_top: torch.Tensor, block_table: torch.Tensor,
               seq_lens: torch.Tensor, n_new: int | torch.Tensor, block_size: int,
               out: torch.Tensor, row_bytes: int, units: torch.Tensor, max_units: int,
               row_offsets: torch.Tensor | None = None, status: torch.Tensor | None = None) -> None:
    """First launch of decode_append_gather: reserve pages + page-unit table."""
    _require_i32(free_stack, "free_stack")
    _require_i32(free_top, "free_top", (1,))
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    n_ptr, n_uni = _n_new_args(n_new, batch)
    off_ptr, seq_rows, _ = _dst_args(out, row_bytes, batch, row_offsets)
    _require_i32(units, "units")
    if units.numel() < 8 + 8 * max_units:
        raise ValueError(f"unit table of {units.numel()} words is smaller than 8 + 8*{max_units}")
    _lib.call("skv_plan_units", free_stack.data_ptr(), free_top.data_ptr(), free_stack.numel(),
              block_table.data_ptr(), bt_stride, seq_lens.data_ptr(), n_ptr, n_uni,
              _lib.ptr(status), off_ptr, seq_rows, block_size, units.data_ptr(), max_units, batch,
              _lib.stream_handle(block_table.device))


def copy_slices(pool: torch.Tensor, src: torch.Tensor, out: torch.Tensor, units: torch.Tensor,
                max_units: int) -> None:
    """Second launch of decode_append_gather: the copy over 4 KB page-unit slices."""
    n_pages, bs, rb = _check_pool(pool)
    _require_gpu(src, "src")
    s_seq, s_row = _row_view_strides(src, rb, "src")
    _require_gpu(out, "out")
    _require_i32(units, "units")
    if units.numel() < 8 + 8 * max_units:
        raise ValueError(f"unit table of {units.numel()} words is smaller than 8 + 8*{max_units}")
    _lib.call("skv_copy_slices", out.data_ptr(), _capacity_rows(out, rb), pool.data_ptr(), rb, bs,
              n_pages, src.data_ptr(), s_seq, s_row, src.shape[1], units.data_ptr(), max_units,
              _lib.stream_handle(pool.device))


def decode_append_gather(free_stack: torch.Tensor, free_top: torch.Tensor, block_table: torch.Tensor,
                         seq_lens: torch.Tensor, pool: torch.Tensor, src: torch.Tensor,
                         n_new: int | torch.Tensor, out: torch.Tensor, units: torch.Tensor,
                         max_units: int, row_offsets: torch.Tensor | None = None,
                         status: torch.Tensor | None = None) -> torch.Tensor:
    """Reserve pages for ``n_new`` rows per sequence, append ``src`` and gather
    every sequence into ``out`` (two launches; see skv_decode_append_gather)."""
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(free_stack, "free_stack", (n_pages,))
    _require_i32(free_top, "free_top", (1,))
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    _require_gpu(src, "src")
    if src.shape[0] != batch:
        raise ValueError(f"src batch {src.shape[0]} != block_table batch {batch}")
    s_seq, s_row = _row_view_strides(src, rb, "src")
    n_ptr, n_uni = _n_new_args(n_new, batch)
    off_ptr, seq_rows, cap = _dst_args(out, rb, batch, row_offsets)
    _require_i32(units, "units")
    if units.numel() < 8 + 8 * max_units:
        raise ValueError(f"unit table of {units.numel()} words is smaller than 8 + 8*{max_units}")
    if status is not None:
        _require_i32(status, "status", (1,))
    _lib.call("skv_decode_append_gather", free_stack.data_ptr(), free_top.data_ptr(), n_pages,
              block_table.data_ptr(), bt_stride, seq_lens.data_ptr(), n_ptr, n_uni,
              _lib.ptr(status), out.data_ptr(), off_ptr, seq_rows, cap, pool.data_ptr(), rb, bs,
              src.data_ptr(), s_seq, s_row, src.shape[1], units.data_ptr(), max_units, batch,
              _lib.stream_handle(pool.device))
    return out


NOALLOC_MAX_UNITS = 65536  # SKV_NOALLOC_MAX_UNITS


def decode_append_gather_noalloc(free_stack: torch.Tensor, free_top: torch.Tensor,
                                 block_table: torch.Tensor, seq_lens: torch.Tensor, pool: torch.Tensor,
                                 src: torch.Tensor, n_new: int | torch.Tensor, out: torch.Tensor,
                                 max_units: int, row_offsets: torch.Tensor | None = None,
                                 status: torch.Tensor | None = None) -> torch.Tensor:
    """decode_append_gather with the library's static page-unit table
    (skv_decode_append_gather_noalloc): no workspace, no device allocation;
    ``max_units`` <= NOALLOC_MAX_UNITS.  Calls that overlap on one GPU race."""
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(free_stack, "free_stack", (n_pages,))
    _require_i32(free_top, "free_top", (1,))
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    _require_gpu(src, "src")
    if src.shape[0] != batch:
        raise ValueError(f"src batch {src.shape[0]} != block_table batch {batch}")
    s_seq, s_row = _row_view_strides(src, rb, "src")
    n_ptr, n_uni = _n_new_args(n_new, batch)
    off_ptr, seq_rows, cap = _dst_args(out, rb, batch, row_offsets)
    if status is not None:
        _require_i32(status, "status", (1,))
    _lib.call("skv_decode_append_gather_noalloc", free_stack.data_ptr(), free_top.data_ptr(), n_pages,
              block_table.data_ptr(), bt_stride, seq_lens.data_ptr(), n_ptr, n_uni,
              _lib.ptr(status), out.data_ptr(), off_ptr, seq_rows, cap, pool.data_ptr(), rb, bs,
              src.data_ptr(), s_seq, s_row, src.shape[1], max_units, batch,
              _lib.stream_handle(pool.device))
    return out


# ---------------------------------------------------------------------------
# SWA ring
# ---------------------------------------------------------------------------
def _check_ring(ring: torch.Tensor) -> tuple[int, int, int]:
    _require_gpu(ring, "ring")
    if ring.dim() < 3 or not ring.is_contiguous():
        raise ValueError(f"ring must be a contiguous [batch, window, *row]; got {tuple(ring.shape)}")
    rb = math.prod(ring.shape[2:]) * ring.element_size()
    return ring.shape[0], ring.shape[1], rb


def ring_append(ring: torch.Tensor, seq_lens: torch.Tensor, src: torch.Tensor,
                n_new: int | torch.Tensor) -> None:
    """Write the newest ``n_new`` tokens (``seq_lens`` already counts them) into the ring."""
    batch, window, rb = _check_ring(ring)
    _require_i32(seq_lens, "seq_lens", (batch,))
    _require_gpu(src, "src")
    if src.shape[0] != batch:
        raise ValueError(f"src batch {src.shape[0]} != ring batch {batch}")
    s_seq, s_row = _row_view_strides(src, rb, "src")
    n_ptr, n_uni = _n_new_args(n_new, batch)
    _lib.call("skv_ring_append", ring.data_ptr(), window, rb, seq_lens.data_ptr(), n_ptr, n_uni,
              src.data_ptr(), s_seq, s_row, src.shape[1], batch, _lib.stream_handle(ring.device))


def ring_read(ring: torch.Tensor, seq_lens: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[b, r] = token at position L-n+r, n = min(window, L), in position order."""
    batch, window, rb = _check_ring(ring)
    _require_i32(seq_lens, "seq_lens", (batch,))
    _, seq_rows, cap = _dst_args(out, rb, batch, None)
    _lib.call("skv_ring_read", out.data_ptr(), seq_rows, cap, ring.data_ptr(), window, rb,
              seq_lens.data_ptr(), batch, _lib.stream_handle(ring.device))
    return out


# ---------------------------------------------------------------------------
# Compression pooling into a paged compressed cache
# ---------------------------------------------------------------------------
def _entry_format(pool: torch.Tensor, channels: int) -> int:
    rb = row_bytes_of(pool)
    if pool.dtype == torch.bfloat16 and rb == 2 * channels:
        return _lib.SKV_FMT_BF16
    if pool.dtype == torch.uint8 and rb == _lib.fp8_entry_bytes(channels):
        return _lib.SKV_FMT_FP8
    raise ValueError(
        f"pool rows of {rb} bytes ({pool.dtype}) match neither bf16 entries of {channels} "
        f"channels nor fp8 entries of {_lib.fp8_entry_bytes(channels)} bytes",
    )


def compress_append(pool: torch.Tensor, block_table: torch.Tensor, tail_state: torch.Tensor,
                    c_new: torch.Tensor, z_new: torch.Tensor, bias: torch.Tensor,
                    seq_lens: torch.Tensor, n_new: int | torch.Tensor) -> int:
    """Pool every block of m tokens completed by this append into the paged cache.

    ``pool`` is bf16 [n_pages, bs, C] (bf16 entries), uint8 [n_pages, bs, E]
    (fp8 entries) or fp32 [n_pages, bs, C] (fp32 entries, unrounded);
    ``tail_state`` fp32 [B, 3, C] carries the incomplete block;
    ``c_new``/``z_new`` [B, T, C] with identical strides, bf16 or fp32 (fp32
    for an fp32 pool; fp32 rows into a bf16 or fp8 pool are pooled unrounded
    and the entry is rounded once); ``bias`` fp32 [m, C] (m = compression
    rate).  Returns the entry format used.
    """
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    channels = c_new.shape[-1]
    if pool.dtype == torch.float32 and rb == 4 * channels:
        fmt = _lib.SKV_FMT_F32
    else:
        fmt = _entry_format(pool, channels)
    in_dtype = torch.float32 if fmt == _lib.SKV_FMT_F32 else c_new.dtype
    if in_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"c_new/z_new must be bf16 or fp32; got {c_new.dtype}")
    in_flag = _lib.SKV_FMT_IN_F32 if (in_dtype == torch.float32 and fmt != _lib.SKV_FMT_F32) else 0
    _require_gpu(tail_state, "tail_state")
    if (tail_state.dtype != torch.float32 or tuple(tail_state.shape) != (batch, 3, channels)
            or not tail_state.is_contiguous()):
        raise ValueError(f"tail_state must be contiguous fp32 [{batch}, 3, {channels}]")
    for name, t in (("c_new", c_new), ("z_new", z_new)):
        _require_gpu(t, name)
        if t.dtype != in_dtype or t.dim() != 3 or t.shape[0] != batch or t.stride(-1) != 1:
            raise ValueError(f"{name} must be {in_dtype} [batch, T, channels] with dense rows")
    if c_new.shape != z_new.shape or c_new.stride() != z_new.stride():
        raise ValueError("c_new and z_new must have the same shape and strides")
    _require_gpu(bias, "bias")
    if bias.dtype != torch.float32 or bias.dim() != 2 or bias.shape[1] != channels \
            or not bias.is_contiguous():
        raise ValueError(f"bias must be contiguous fp32 [m, {channels}]")
    m = bias.shape[0]
    n_ptr, n_uni = _n_new_args(n_new, batch)
    es = c_new.element_size()
    _lib.call("skv_compress_append", pool.data_ptr(), rb, bs, n_pages, block_table.data_ptr(),
              bt_stride, tail_state.data_ptr(), c_new.data_ptr(), z_new.data_ptr(),
              c_new.stride(0) * es, c_new.stride(1) * es, c_new.shape[1], bias.data_ptr(),
              seq_lens.data_ptr(), n_ptr, n_uni, m, channels, fmt | in_flag, batch,
              _lib.stream_handle(pool.device))
    return fmt


def fp8_quant_append(pool: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                     src: torch.Tensor, n_new: int | torch.Tensor) -> None:
    """Quantize bf16 rows [B, T, C] into fp8 entries (uint8 pool [n_pages, bs, E])."""
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    _require_gpu(src, "src")
    if src.dtype != torch.bfloat16 or src.dim() != 3 or src.shape[0] != batch or src.stride(-1) != 1:
        raise ValueError("src must be bf16 [batch, T, channels] with dense rows")
    channels = src.shape[-1]
    if pool.dtype != torch.uint8 or rb != _lib.fp8_entry_bytes(channels):
        raise ValueError(f"fp8 pool rows must be {_lib.fp8_entry_bytes(channels)} uint8")
    n_ptr, n_uni = _n_new_args(n_new, batch)
    es = src.element_size()
    _lib.call("skv_fp8_quant_append", pool.data_ptr(), rb, bs, n_pages, block_table.data_ptr(),
              bt_stride, seq_lens.data_ptr(), n_ptr, n_uni, src.data_ptr(), src.stride(0) * es,
              src.stride(1) * es, src.shape[1], channels, batch, _lib.stream_handle(pool.device))


def fp8_encode_host(x: torch.Tensor) -> torch.Tensor:
    """e4m3fn codes of fp32 CPU values through the library's own codec (no GPU)."""
    if x.device.type != "cpu" or x.dtype != torch.float32:
        raise ValueError("fp8_encode_host takes a CPU float32 tensor")
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.uint8)
    _lib.call("skv_fp8_encode_host", x.data_ptr(), out.data_ptr(), x.numel())
    return out


def fp8_decode_host(codes: torch.Tensor) -> torch.Tensor:
    if codes.device.type != "cpu" or codes.dtype != torch.uint8:
        raise ValueError("fp8_decode_host takes a CPU uint8 tensor")
    codes = codes.contiguous()
    out = torch.empty(codes.shape, dtype=torch.float32)
    _lib.call("skv_fp8_decode_host", codes.data_ptr(), out.data_ptr(), codes.numel())
    return out


# ---------------------------------------------------------------------------
# Top-k selection and gather
# ---------------------------------------------------------------------------
def _check_scores(scores: torch.Tensor, rows: int) -> None:
    _require_gpu(scores, "scores")
    if scores.dtype != torch.float32 or scores.dim() != 2 or scores.stride(1) != 1:
        raise ValueError("scores must be fp32 [rows, n] with unit column stride")
    if scores.shape[0] != rows:
        raise ValueError(f"scores has {scores.shape[0]} rows, expected {rows}")


def _check_idx_out(out: torch.Tensor, rows: int, k: int) -> None:
    _require_gpu(out, "out")
    if out.dtype != torch.int32 or out.dim() != 2 or out.shape[0] != rows or out.shape[1] < k:
        raise ValueError(f"out must be int32 [{rows}, >={k}]")
    if out.stride(1) != 1:
        raise ValueError("out must have unit column stride")


def topk_workspace(rows: int, device: torch.device) -> torch.Tensor:
    """Zeroed workspace for the multi-workgroup top-k of ``rows`` rows."""
    return torch.zeros(rows * _lib.topk_workspace_words(), dtype=torch.int32, device=device)


def _ws_ptr(workspace: torch.Tensor | None, rows: int) -> int | None:
    if workspace is None:
        return None
    _require_i32(workspace, "workspace")
    if workspace.numel() < rows * _lib.topk_workspace_words():
        raise ValueError("top-k workspace too small: need rows * skv_topk_workspace_words() int32")
    return workspace.data_ptr()


def topk_select(scores: torch.Tensor, n_valid: torch.Tensor, n_cols: int | torch.Tensor, k: int,
                out: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Per row: the min(k, n_cols, n_valid) best valid columns, -1 padded to k.

    With ``workspace`` (see topk_workspace) each row is spread over several
    workgroups; without it one workgroup handles a row.
    """
    rows = n_valid.shape[0]
    _require_i32(n_valid, "n_valid", (rows,))
    _check_scores(scores, rows)
    _check_idx_out(out, rows, k)
    if isinstance(n_cols, torch.Tensor):
        _require_i32(n_cols, "n_cols", (rows,))
        nc_ptr, nc_uni = n_cols.data_ptr(), 0
    else:
        nc_ptr, nc_uni = None, int(n_cols)
        if nc_uni > scores.shape[1]:
            raise ValueError(f"n_cols={nc_uni} exceeds the score row length {scores.shape[1]}")
    _lib.call("skv_topk_select", scores.data_ptr(), scores.stride(0), rows, n_valid.data_ptr(),
              nc_ptr, nc_uni, k, out.data_ptr(), out.stride(0), _ws_ptr(workspace, rows),
              _lib.stream_handle(scores.device))
    return out


def topk_select_decode(scores: torch.Tensor, seq_lens: torch.Tensor, m: int, k: int,
                       out: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Decode query at position L-1 of each sequence: causal block mask from seq_lens."""
    batch = seq_lens.shape[0]
    _require_i32(seq_lens, "seq_lens", (batch,))
    _check_scores(scores, batch)
    _check_idx_out(out, batch, k)
    _lib.call("skv_topk_select_decode", scores.data_ptr(), scores.stride(0), batch,
              seq_lens.data_ptr(), m, k, out.data_ptr(), out.stride(0), _ws_ptr(workspace, batch),
              _lib.stream_handle(scores.device))
    return out


def topk_gather(pool: torch.Tensor, block_table: torch.Tensor, n_entries: torch.Tensor,
                idx: torch.Tensor, out: torch.Tensor, channels: int,
                row_seq: torch.Tensor | None = None) -> torch.Tensor:
    """out[r, j] = entry max(idx[r, j], 0) of the row's sequence (fp8 entries dequantized)."""
    n_pages, bs, rb = _check_pool(pool)
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(n_entries, "n_entries", (batch,))
    _require_gpu(idx, "idx")
    if idx.dtype != torch.int32 or idx.dim() != 2 or idx.stride(1) != 1:
        raise ValueError("idx must be int32 [rows, k] with unit column stride")
    rows, k = idx.shape
    if row_seq is None:
        if rows != batch:
            raise ValueError("without row_seq, idx must have one row per sequence")
    else:
        _require_i32(row_seq, "row_seq", (rows,))
    fmt = _entry_format(pool, channels)
    out_row = rb if fmt == _lib.SKV_FMT_BF16 else 2 * channels
    _require_gpu(out, "out")
    if not out.is_contiguous() or out.numel() * out.element_size() != rows * k * out_row:
        raise ValueError(f"out must be contiguous with {rows}x{k} rows of {out_row} bytes")
    _lib.call("skv_topk_gather", out.data_ptr(), pool.data_ptr(), rb, bs, n_pages,
              block_table.data_ptr(), bt_stride, n_entries.data_ptr(), idx.data_ptr(),
              idx.stride(0), k, rows, _lib.ptr(row_seq), channels, fmt,
              _lib.stream_handle(pool.device))
    return out


def indexer_scores(q: torch.Tensor, w: torch.Tensor, idx_pool: torch.Tensor, block_table: torch.Tensor,
                   n_entries: torch.Tensor, out: torch.Tensor, max_entries: int | None = None) -> torch.Tensor:
    """Lightning-indexer scores over the paged compressed indexer keys.

    out[b, t, s] = sum_h w[b, t, h] * relu(q[b, t, h, :] . k[b, s, :]) for
    s < min(n_entries[b], max_entries) (default max_entries: out's last dim);
    unmasked, -inf for unmapped pages, other columns untouched.
    q: bf16 [B, T, H, c]; w: fp32 [B, T, H]; idx_pool: bf16 [n_pages,
    block_size, c]; out: fp32 [B, T, n] with rows of unit stride.
    """
    _require_gpu(q, "q")
    if q.dtype != torch.bfloat16 or q.dim() != 4 or not q.is_contiguous():
        raise ValueError("q must be a contiguous bf16 [B, T, H, c] tensor")
    batch, t, heads, c = q.shape
    _require_gpu(w, "w")
    if w.dtype != torch.float32 or tuple(w.shape) != (batch, t, heads) or not w.is_contiguous():
        raise ValueError(f"w must be a contiguous fp32 [{batch}, {t}, {heads}] tensor")
    _require_gpu(idx_pool, "idx_pool")
    if idx_pool.dtype != torch.bfloat16 or idx_pool.dim() != 3 or idx_pool.shape[2] != c or \
            not idx_pool.is_contiguous():
        raise ValueError(f"idx_pool must be a contiguous bf16 [n_pages, block_size, {c}] tensor")
    n_pages, bs = idx_pool.shape[0], idx_pool.shape[1]
    _require_i32(block_table, "block_table")
    if block_table.dim() != 2 or block_table.shape[0] != batch:
        raise ValueError(f"block_table must be int32 [{batch}, max_pages]")
    _require_i32(n_entries, "n_entries", (batch,))
    _require_gpu(out, "out")
    if out.dtype != torch.float32 or out.dim() != 3 or tuple(out.shape[:2]) != (batch, t) or out.stride(2) != 1 \
            or out.stride(0) != t * out.stride(1):
        raise ValueError(f"out must be fp32 [{batch}, {t}, n] with unit column stride and dense rows")
    n = out.shape[2] if max_entries is None else int(max_entries)
    if n > out.shape[2]:
        raise ValueError(f"max_entries={n} exceeds out's {out.shape[2]} columns")
    _lib.call("skv_indexer_scores", q.data_ptr(), w.data_ptr(), idx_pool.data_ptr(), bs, n_pages,
              block_table.data_ptr(), block_table.shape[1], n_entries.data_ptr(), out.data_ptr(),
              out.stride(1), batch, t, heads, c, n, _lib.stream_handle(q.device))
    return out


# ---------------------------------------------------------------------------
# Eviction and compaction
# ---------------------------------------------------------------------------
def release(free_stack: torch.Tensor, free_top: torch.Tensor, block_table: torch.Tensor,
            seq_lens: torch.Tensor, mask: torch.Tensor, block_size: int,
            status: torch.Tensor | None = None) -> None:
    """Return every page of the sequences with mask[b] to the free stack."""
    _require_i32(free_stack, "free_stack")
    _require_i32(free_top, "free_top", (1,))
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    _require_gpu(mask, "mask")
    if mask.dtype not in (torch.uint8, torch.bool) or tuple(mask.shape) != (batch,):
        raise ValueError("mask must be uint8/bool [batch]")
    if status is not None:
        _require_i32(status, "status", (1,))
    _lib.call("skv_release", free_stack.data_ptr(), free_top.data_ptr(), free_stack.numel(),
              block_table.data_ptr(), bt_stride, seq_lens.data_ptr(), mask.contiguous().data_ptr(),
              batch, block_size, _lib.ptr(status), _lib.stream_handle(block_table.device))


def compact(pools: list[torch.Tensor], block_table: torch.Tensor, seq_lens: torch.Tensor,
            block_size: int, free_stack: torch.Tensor, free_top: torch.Tensor,
            workspace: torch.Tensor, info: torch.Tensor) -> None:
    """Defragment ``pools`` (sharing ``block_table``) so live pages occupy [0, n_live).

    ``workspace`` (int32 [3 * n_pages]): its first n_pages words must be zero
    before the first call; every call leaves them zero (the rest is scratch).
    """
    n_pages = free_stack.numel()
    refs = (_lib.PoolRef * len(pools))()
    for i, p in enumerate(pools):
        pn, pbs, rb = _check_pool(p)
        if pn != n_pages or pbs != block_size:
            raise ValueError("every pool must have n_pages pages of block_size rows")
        refs[i].base = p.data_ptr()
        refs[i].page_bytes = pbs * rb
    _require_i32(block_table, "block_table")
    batch, bt_stride = block_table.shape
    _require_i32(seq_lens, "seq_lens", (batch,))
    _require_i32(free_stack, "free_stack")
    _require_i32(free_top, "free_top", (1,))
    _require_i32(workspace, "workspace", (3 * n_pages,))
    _require_i32(info, "info", (2,))
    _lib.call("skv_compact", ctypes.cast(refs, ctypes.c_void_p), len(pools), block_table.data_ptr(), bt_stride,
              seq_lens.data_ptr(), batch, block_size, n_pages, free_stack.data_ptr(),
              free_top.data_ptr(), workspace.data_ptr(), info.data_ptr(),
              _lib.stream_handle(block_table.device))
