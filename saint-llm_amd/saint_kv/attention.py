"""Decode attention over the paged cache (``skv_decode_attention``).

One query token per sequence, MQA (one K/V head, H query heads).  The
reference computes it in three consumers of the cache:

* ``CSA.forward`` (csa.py:324-373): softmax over ``k_norm`` of the top-k picked
  compressed entries (K = V, no sink) plus the sliding-window branch;
* ``HCA.forward`` (hca.py:126-169): softmax over ``k_norm`` of every visible
  compressed entry (``s*m + m-1 < q_pos``, K = V, the layer's sink) plus the
  window branch;
* ``SWAttention.forward`` (swa.py:115-137): the window branch alone,

each branch through ``scaled_dot_product`` / ``softmax_with_sink``
(common.py:77-124).  Here the picked or visible entries are read straight from
the paged pool (bf16 or fp8), so the gathered copy of csa.py:329-331 is never
formed.
"""

from __future__ import annotations

import ctypes

import torch

from saint_kv import _lib
from saint_kv.ops import _require_gpu, _require_i32

KIND = {"swa": 0, "hca": 1, "csa": 2}  # SKV_LAYER_*
_P = ctypes.c_void_p
_I64 = ctypes.c_int64


class AttentionDesc(ctypes.Structure):
    """Mirror of skv_attention_desc (include/saintkv.h)."""

    _fields_ = [
        ("kind", ctypes.c_int32), ("format", ctypes.c_int32),
        ("batch", _I64), ("n_heads", _I64), ("head_dim", _I64),
        ("q", _P), ("out", _P), ("lens", _P),
        ("pool", _P), ("entry_bytes", _I64), ("block_size", _I64), ("n_pages", _I64),
        ("block_table", _P), ("bt_stride", _I64), ("n_entries", _P),
        ("m", _I64), ("max_entries", _I64),
        ("picks", _P), ("pick_stride", _I64), ("top_k", _I64),
        ("knorm_w", _P), ("eps", ctypes.c_float), ("softcap", ctypes.c_float), ("sink", _P),
        ("win_k", _P), ("win_v", _P), ("window", _I64), ("splits", _I64),
    ]


def _check_layout() -> None:
    size = _lib.load().skv_attention_desc_size()
    if size != ctypes.sizeof(AttentionDesc):
        raise RuntimeError(f"skv_attention_desc layout mismatch: library {size} vs ctypes "
                           f"{ctypes.sizeof(AttentionDesc)}")


def _bf16_rows(t: torch.Tensor, name: str, shape: tuple[int, ...]) -> None:
    _require_gpu(t, name)
    if t.dtype != torch.bfloat16 or tuple(t.shape) != shape or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous bf16 tensor of shape {shape}; got "
                         f"{t.dtype} {tuple(t.shape)}")


def _f32_vec(t: torch.Tensor, name: str, n: int) -> None:
    _require_gpu(t, name)
    if t.dtype != torch.float32 or tuple(t.shape) != (n,) or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous fp32 [{n}] tensor")


def decode_attention(q: torch.Tensor, kind: str, lens: torch.Tensor, win_k: torch.Tensor,
                     win_v: torch.Tensor, *, pool: torch.Tensor | None = None, fp8: bool = False,
                     block_table: torch.Tensor | None = None, n_entries: torch.Tensor | None = None,
                     m: int = 1, max_entries: int = 0, picks: torch.Tensor | None = None,
                     knorm_w: torch.Tensor | None = None, eps: float = 1.0e-6,
                     sink: torch.Tensor | None = None, softcap: float | None = None,
                     out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                     splits: int = 0) -> torch.Tensor:
    """One layer's attention output (before the output projection), fp32 [B, H, D].

    q: bf16 [B, H, D] (roped, q_norm applied); lens: int32 [B] tokens after the
    step's append; win_k / win_v: bf16 [B, W, D] rings (slot pos % W; may be
    the same tensor).  Compressed branch ("csa" / "hca"): pool [n_pages,
    block_size, D] bf16, or [n_pages, block_size, entry_bytes] uint8 fp8
    entries with ``fp8=True``; block_table int32 [B, max_pages]; n_entries
    int32 [B]; knorm_w fp32 [D]; "csa": picks int32 [B, k] (the top-k row,
    -1 padded); "hca": the compression rate m (max_entries bounds the entries
    per sequence for the split; 0 = the table's capacity).  sink: fp32 [H] or
    None; softcap: the window branch's c*tanh(s/c), or None.
    """
    _check_layout()
    if kind not in KIND:
        raise ValueError(f"kind must be one of {sorted(KIND)}; got {kind!r}")
    _require_gpu(q, "q")
    if q.dtype != torch.bfloat16 or q.dim() != 3 or not q.is_contiguous():
        raise ValueError("q must be a contiguous bf16 [B, H, D] tensor")
    batch, heads, dim = q.shape
    _require_i32(lens, "lens", (batch,))
    if win_k.dim() != 3:
        raise ValueError("win_k must be bf16 [B, W, D]")
    window = win_k.shape[1]
    _bf16_rows(win_k, "win_k", (batch, window, dim))
    _bf16_rows(win_v, "win_v", (batch, window, dim))
    d = AttentionDesc()
    d.kind = KIND[kind]
    d.format = _lib.SKV_FMT_FP8 if fp8 else _lib.SKV_FMT_BF16
    d.batch, d.n_heads, d.head_dim = batch, heads, dim
    d.q = q.data_ptr()
    d.lens = lens.data_ptr()
    d.win_k, d.win_v, d.window = win_k.data_ptr(), win_v.data_ptr(), window
    d.eps = eps
    d.softcap = 0.0 if softcap is None else float(softcap)
    if softcap is not None and softcap <= 0:
        raise ValueError("softcap must be positive (or None)")
    if sink is not None:
        _f32_vec(sink, "sink", heads)
        d.sink = sink.data_ptr()
    d.splits = int(splits)
    if kind != "swa":
        if pool is None or block_table is None or n_entries is None or knorm_w is None:
            raise ValueError(f"{kind} attention needs pool, block_table, n_entries and knorm_w")
        _require_gpu(pool, "pool")
        if pool.dim() != 3 or not pool.is_contiguous():
            raise ValueError("pool must be a contiguous [n_pages, block_size, row] tensor")
        if fp8:
            if pool.dtype != torch.uint8 or pool.shape[2] != _lib.fp8_entry_bytes(dim):
                raise ValueError(f"fp8 pool must be uint8 [n_pages, block_size, {_lib.fp8_entry_bytes(dim)}]")
            d.entry_bytes = pool.shape[2]
        else:
            if pool.dtype != torch.bfloat16 or pool.shape[2] != dim:
                raise ValueError(f"pool must be bf16 [n_pages, block_size, {dim}]")
            d.entry_bytes = 2 * dim
        d.pool, d.n_pages, d.block_size = pool.data_ptr(), pool.shape[0], pool.shape[1]
        _require_i32(block_table, "block_table")
        if block_table.dim() != 2 or block_table.shape[0] != batch:
            raise ValueError(f"block_table must be int32 [{batch}, max_pages]")
        d.block_table, d.bt_stride = block_table.data_ptr(), block_table.shape[1]
        _require_i32(n_entries, "n_entries", (batch,))
        d.n_entries = n_entries.data_ptr()
        _f32_vec(knorm_w, "knorm_w", dim)
        d.knorm_w = knorm_w.data_ptr()
        if kind == "csa":
            if picks is None:
                raise ValueError("csa attention needs picks")
            _require_i32(picks, "picks")
            if picks.dim() != 2 or picks.shape[0] != batch:
                raise ValueError(f"picks must be int32 [{batch}, k]")
            d.picks, d.pick_stride, d.top_k = picks.data_ptr(), picks.shape[1], picks.shape[1]
        else:
            d.m, d.max_entries = int(m), int(max_entries)
    if out is None:
        out = torch.empty(batch, heads, dim, dtype=torch.float32, device=q.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (batch, heads, dim) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous fp32 [{batch}, {heads}, {dim}] tensor")
    d.out = out.data_ptr()
    need = int(_lib.load().skv_attention_workspace(ctypes.byref(d)))
    if need < 0:
        _lib.check(-1, "skv_attention_workspace")
    global _LAST_WS
    if workspace is None:
        workspace = torch.empty(max(need, 4) // 4 + 1, dtype=torch.float32, device=q.device)
    elif workspace.device != q.device or workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace must hold {need} bytes on {q.device}")
    elif not workspace.is_contiguous() or workspace.data_ptr() % 16:
        raise ValueError("workspace must be a contiguous tensor whose data is 16-byte aligned")
    _lib.call("skv_decode_attention", ctypes.byref(d), workspace.data_ptr(),
              workspace.numel() * workspace.element_size(), _lib.stream_handle(q.device))
    _LAST_WS = workspace
    return out


_LAST_WS: torch.Tensor | None = None


def step_attention_desc(q: torch.Tensor, kind: str, window: int, *, knorm_w: torch.Tensor | None = None,
                        eps: float = 1.0e-6, sink: torch.Tensor | None = None, softcap: float | None = None,
                        win_v: torch.Tensor | None = None, out: torch.Tensor | None = None,
                        max_entries: int = 0, splits: int = 0) -> tuple[AttentionDesc, torch.Tensor]:
    """The caller's fields of skv_decode_step_attend's attention descriptor:
    q (bf16 [B, H, D]), out (fp32 [B, H, D], allocated when None), knorm_w
    (fp32 [D], "csa"/"hca"), eps, sink (fp32 [H] or None), softcap, win_v
    (bf16 [B, window, D] value ring, or None for the layer's own ring: K = V)
    and the split bounds.  The cache's fields come from the step's descriptor.
    Returns (descriptor, out)."""
    _check_layout()
    if kind not in KIND:
        raise ValueError(f"kind must be one of {sorted(KIND)}; got {kind!r}")
    _require_gpu(q, "q")
    if q.dtype != torch.bfloat16 or q.dim() != 3 or not q.is_contiguous():
        raise ValueError("q must be a contiguous bf16 [B, H, D] tensor")
    batch, heads, dim = q.shape
    d = AttentionDesc()
    d.kind = KIND[kind]
    d.batch, d.n_heads, d.head_dim = batch, heads, dim
    d.q = q.data_ptr()
    d.eps = eps
    if softcap is not None and softcap <= 0:
        raise ValueError("softcap must be positive (or None)")
    d.softcap = 0.0 if softcap is None else float(softcap)
    if sink is not None:
        _f32_vec(sink, "sink", heads)
        d.sink = sink.data_ptr()
    if win_v is not None:
        _bf16_rows(win_v, "win_v", (batch, window, dim))
        d.win_v = win_v.data_ptr()
    if kind != "swa":
        if knorm_w is None:
            raise ValueError(f"{kind} attention needs knorm_w")
        _f32_vec(knorm_w, "knorm_w", dim)
        d.knorm_w = knorm_w.data_ptr()
    d.max_entries, d.splits = int(max_entries), int(splits)
    if out is None:
        out = torch.empty(batch, heads, dim, dtype=torch.float32, device=q.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (batch, heads, dim) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous fp32 [{batch}, {heads}, {dim}] tensor")
    d.out = out.data_ptr()
    return d, out


def last_workspace() -> torch.Tensor | None:
    """The workspace the last decode_attention call used (allocated by it when
    none was passed), for callers that keep it for later calls."""
    return _LAST_WS
