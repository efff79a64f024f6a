"""Decode attention over the paged cache (``skv_decode_attention``).

T >= 1 query tokens per sequence (the last T tokens of the cache, as the
cached forward of csa.py:276-281 / hca.py:127-131 sees them), MQA (one K/V
head, H query heads).  The reference computes it in three consumers of the
cache:

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
        ("n_queries", _I64), ("ring", _I64), ("win_stride", _I64),
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


def _window_slots(win_k: torch.Tensor, win_v: torch.Tensor, shape: tuple[int, ...]) -> int:
    """Bytes between window slots of win_k / win_v: bf16 [B, R, D] with unit
    last stride and whole sequences of R slots, e.g. the K and V halves of a
    [B, R, 2, D] cache (kv_cache.py's rows)."""
    for t, name in ((win_k, "win_k"), (win_v, "win_v")):
        _require_gpu(t, name)
        if t.dtype != torch.bfloat16 or tuple(t.shape) != shape:
            raise ValueError(f"{name} must be bf16 of shape {shape}; got {t.dtype} {tuple(t.shape)}")
    st = win_k.stride()
    if win_v.stride() != st or st[2] != 1 or st[0] != shape[1] * st[1] or st[1] < shape[2]:
        raise ValueError("win_k / win_v must share strides (R * S, S, 1) with S >= D")
    if (st[1] * 2) % 16 or win_k.data_ptr() % 16 or win_v.data_ptr() % 16:
        raise ValueError("window slots must start at 16-byte boundaries")
    return st[1] * 2


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
                     splits: int = 0, window: int | None = None) -> torch.Tensor:
    """One layer's attention output (before the output projection), fp32
    [B, H, D], or [B, T, H, D] for T query tokens per sequence.

    q: bf16 [B, H, D] or [B, T, H, D] (roped, q_norm applied): query token t
    of sequence b is the cache's position lens[b] - T + t; lens: int32 [B]
    tokens after the append of the T tokens; win_k / win_v: bf16 [B, R, D]
    rings (slot pos % R; may be the same tensor, or strided views such as
    the K and V halves of [B, R, 2, D] rows) that hold the last min(window +
    T - 1, lens[b]) positions: R >= window + T - 1, or a contiguous cache of
    the sequence's whole capacity (R = max_len, slot pos = pos); window: the
    sliding window W <= R (None: R).  Compressed
    branch ("csa" / "hca"): pool [n_pages, block_size, D] bf16, or [n_pages,
    block_size, entry_bytes] uint8 fp8 entries with ``fp8=True``;
    block_table int32 [B, max_pages]; n_entries int32 [B]; knorm_w fp32 [D];
    "csa": picks int32 [B, k] or [B, T, k] (each query's top-k row, -1
    padded); "hca": the compression rate m (max_entries bounds the entries
    per sequence for the split; 0 = the table's capacity).  sink: fp32 [H] or
    None; softcap: the window branch's c*tanh(s/c), or None.
    """
    _check_layout()
    if kind not in KIND:
        raise ValueError(f"kind must be one of {sorted(KIND)}; got {kind!r}")
    _require_gpu(q, "q")
    if q.dtype != torch.bfloat16 or q.dim() not in (3, 4) or not q.is_contiguous():
        raise ValueError("q must be a contiguous bf16 [B, H, D] or [B, T, H, D] tensor")
    lead = tuple(q.shape[:-2])  # (B,) or (B, T)
    batch, n_q = lead[0], (lead[1] if len(lead) == 2 else 1)
    heads, dim = q.shape[-2:]
    _require_i32(lens, "lens", (batch,))
    if win_k.dim() != 3:
        raise ValueError("win_k must be bf16 [B, R, D]")
    ring = win_k.shape[1]
    win_stride = _window_slots(win_k, win_v, (batch, ring, dim))
    window = ring if window is None else int(window)
    if not 1 <= window <= ring:
        raise ValueError(f"window must be in [1, {ring}] (the rings' slots); got {window}")
    d = AttentionDesc()
    d.kind = KIND[kind]
    d.format = _lib.SKV_FMT_FP8 if fp8 else _lib.SKV_FMT_BF16
    d.batch, d.n_heads, d.head_dim = batch, heads, dim
    d.n_queries, d.ring = n_q, ring
    d.q = q.data_ptr()
    d.lens = lens.data_ptr()
    d.win_k, d.win_v, d.window = win_k.data_ptr(), win_v.data_ptr(), window
    d.win_stride = 0 if win_stride == 2 * dim else win_stride
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
            if tuple(picks.shape[:-1]) != lead or not picks.is_contiguous():
                raise ValueError(f"picks must be a contiguous int32 [{', '.join(map(str, lead))}, k] tensor")
            d.picks, d.pick_stride, d.top_k = picks.data_ptr(), picks.shape[-1], picks.shape[-1]
        else:
            d.m, d.max_entries = int(m), int(max_entries)
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    elif out.dtype != torch.float32 or out.shape != q.shape or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous fp32 {list(q.shape)} tensor")
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


def cached_attention(layer, q: torch.Tensor, *, window: int, top_idx: torch.Tensor | None = None,
                     knorm_w: torch.Tensor | None = None, eps: float = 1.0e-6,
                     sink: torch.Tensor | None = None, softcap: float | None = None,
                     workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The attention of a cached forward over a drop-in cache layer
    (``saint_kv.kv_cache``) for the t_new tokens its last ``append`` added, on
    the reference's tensors, read in place from the layer's pages:

    * ``CSAKVCacheLayer``: ``sparse_attn_out + sw_attn_out`` of CSA.forward
      (csa.py:324-371) for ``top_idx`` (B, t_new, top_k) from
      ``_indexer_topk_cached`` (csa.py:377-422; -1 padded, any integer dtype);
    * ``HCAKVCacheLayer``: ``compressed_attn_out + sw_attn_out`` of HCA.forward
      (hca.py:123-167), entries visible per query (s*m + m-1 < q_pos);
    * ``SWAKVCacheLayer``: the window branch of SWAttention.forward
      (swa.py:115-136),

    before the output projection.  q: bf16 (B, n_heads, t_new, head_dim) as
    those forwards hold it (roped, q_norm applied); window: the attention's
    sliding_window_size; knorm_w / eps: its ``k_norm`` (RMSNorm) weight and
    eps (CSA/HCA); sink: its ``sink_logit`` ([n_heads]) or None; softcap: its
    ``logit_softcap`` or None.  The layer must be a bf16 cache.  Returns
    fp32 (B, n_heads, t_new, head_dim) (a view of a [B, t_new, n_heads,
    head_dim] tensor)."""
    from saint_kv import kv_cache as kvc

    if isinstance(layer, kvc.CSAKVCacheLayer):
        kind = "csa"
    elif isinstance(layer, kvc.HCAKVCacheLayer):
        kind = "hca"
    elif isinstance(layer, kvc.SWAKVCacheLayer):
        kind = "swa"
    else:
        raise TypeError(f"layer must be a saint_kv.kv_cache layer; got {type(layer).__name__}")
    if layer.dtype != torch.bfloat16:
        raise ValueError(f"cached_attention needs a bf16 cache; this layer holds {layer.dtype}")
    if q.dim() != 4 or q.shape[0] != layer.batch_size or q.shape[3] != layer.head_dim:
        raise ValueError(f"q must be (B={layer.batch_size}, n_heads, t_new, {layer.head_dim})")
    t_new = q.shape[2]
    if not 1 <= t_new <= layer.length:
        raise ValueError(f"t_new must be in [1, {layer.length}] (the layer's length); got {t_new}")
    sw = layer._rows if kind == "swa" else layer._sw
    rows = sw.out  # (B, max_seq_len, 2, D): [K | V] per position, slot = position
    qt = q.to(torch.bfloat16).transpose(1, 2).contiguous()  # [B, t_new, H, D]

    def f32(t):  # module parameters in any float dtype
        return None if t is None else t.detach().to(device=q.device, dtype=torch.float32).contiguous()

    knorm_w, sink = f32(knorm_w), f32(sink)
    args = dict(window=min(int(window), rows.shape[1]), sink=sink, softcap=softcap,
                workspace=workspace, eps=eps)
    if kind != "swa":
        stream = layer._streams[0]
        args.update(pool=stream.pool, block_table=stream.block_table, n_entries=stream.lens,
                    knorm_w=knorm_w)
        if kind == "csa":
            if top_idx is None or tuple(top_idx.shape[:2]) != (layer.batch_size, t_new):
                raise ValueError(f"csa needs top_idx (B={layer.batch_size}, t_new={t_new}, top_k)")
            args["picks"] = top_idx.to(device=q.device, dtype=torch.int32).contiguous()
        else:
            args["m"] = layer.compression_rate
            args["max_entries"] = max(layer.n_blocks, 1)
    out = decode_attention(qt, kind, sw.lens, rows[:, :, 0], rows[:, :, 1], **args)
    return out.transpose(1, 2)
