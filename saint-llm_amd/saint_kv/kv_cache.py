"""Drop-in heterogeneous KV cache layers backed by paged HIP storage.

Same names, constructor signatures, attributes, return values and error
types/messages as the reference classes in
packages/inference/src/saint_llm_inference/kv_cache.py:

* ``SWAKVCacheLayer``  (kv_cache.py:32-87)
* ``HCAKVCacheLayer``  (kv_cache.py:90-207)
* ``CSAKVCacheLayer``  (kv_cache.py:210-327)
* ``KVCacheBundle``    (kv_cache.py:333-427)

Differences in mechanism (not in results):

* K/V rows and compressed entries live in fixed-size pages of a per-layer page
  pool reached through an int32 block table; ``append`` writes the new rows
  with ``skv_append_gather`` / ``skv_paged_append`` and returns contiguous
  tensors gathered from the pages (the values the reference's slice views
  hold).  The returned tensors are views of per-layer gather buffers that the
  next ``append`` refreshes, as the reference's views alias its storage.
* Caches live on a ROCm GPU only: ``device=None`` means the current GPU, and a
  CPU device raises.  There is no CPU code path.
* ``compressor`` callables are invoked exactly as the reference does (on the
  m-aligned prefix of ``cat(h_buffer, h_new)``); their output is copied into
  the paged compressed cache.  Fast path: when every compressor of a bf16
  cache is a ``TokenLevelCompressor``-shaped module (``w_b_kv``, ``w_b_z``,
  ``bias_b``, ``m``, ``c``; csa.py:59-64), only the two projections its
  forward pools with are run (torch), and the per-channel softmax pooling
  and entry emission run in ``skv_compress_append`` straight into the pages,
  token by token, through a carried fp32 pooling state (csa.py:79-87), so
  no block is replayed from ``h_buffer``.  ``h_buffer`` / ``h_buf_count``
  keep the reference's contents either way.
"""

from __future__ import annotations

from collections.abc import Callable

import numpy as np
import torch
from torch import Tensor

from saint_kv import ops

DEFAULT_BLOCK_SIZE = 16


def _device(device: torch.device | str | None) -> torch.device:
    if device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("saint_kv caches need a ROCm GPU; none is visible (no CPU fallback)")
        return torch.device("cuda", torch.cuda.current_device())
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(f"saint_kv caches run only on a ROCm GPU, not {dev} (no CPU fallback)")
    return dev


class _PagedRows:
    """Rows of ``row_shape`` for ``batch`` lock-step sequences in a private page pool.

    The pool holds exactly the pages ``max_rows`` rows need, so it never runs
    out; page ids are handed out by the device free stack (skv_reserve).  Rows
    whose size is not a multiple of 16 bytes are stored with the last dim
    zero-padded (the kernels move 16-byte chunks); views hide the padding.

    The gather buffer is a running copy of the pages: an append refreshes it
    from the page that holds the first new row on (at most block_size - 1
    earlier rows plus the new ones), so an append costs O(new rows), not
    O(length), as the reference's slice views cost nothing per append.
    """

    def __init__(self, batch: int, max_rows: int, row_shape: tuple[int, ...], dtype: torch.dtype,
                 device: torch.device, block_size: int) -> None:
        es = torch.empty((), dtype=dtype).element_size()
        lead, d = int(np.prod(row_shape[:-1])), row_shape[-1]
        d_pad = d
        while (lead * d_pad * es) % 16:
            d_pad += 1
        self.d, self.d_pad = d, d_pad
        store_shape = (*row_shape[:-1], d_pad)
        self.batch, self.max_rows, self.block_size = batch, max_rows, block_size
        self.max_pages = max(1, -(-max_rows // block_size))
        n_pages = batch * self.max_pages
        self.pool = torch.zeros(n_pages, block_size, *store_shape, dtype=dtype, device=device)
        self.free_stack = torch.empty(n_pages, dtype=torch.int32, device=device)
        self.free_top = torch.empty(1, dtype=torch.int32, device=device)
        self.block_table = torch.full((batch, self.max_pages), -1, dtype=torch.int32, device=device)
        self.lens = torch.zeros(batch, dtype=torch.int32, device=device)
        self.status = torch.zeros(1, dtype=torch.int32, device=device)
        self._out = torch.zeros(batch, max_rows, *store_shape, dtype=dtype, device=device)
        ops.free_stack_init(self.free_stack, self.free_top)
        self.length = 0

    @property
    def out(self) -> Tensor:
        """(B, max_rows, *row_shape) gather buffer; rows [0, length) are current."""
        return self._out if self.d == self.d_pad else self._out[..., : self.d]

    def append(self, rows: Tensor) -> Tensor:
        """Append rows (B, n, *row) and return the gathered (B, length, *row)."""
        n = rows.shape[1]
        if n:
            if self.d_pad != self.d:
                rows = torch.nn.functional.pad(rows, (0, self.d_pad - self.d))
            ops.reserve(self.free_stack, self.free_top, self.block_table, self.lens, n,
                        self.block_size, self.status)
            ops.append_gather(self.pool, self.block_table, self.lens, rows, n, self._out,
                              first_page=self.length // self.block_size)
            self.length += n
        return self.out[:, : self.length]

    def reset(self) -> None:
        if self.length:
            mask = torch.ones(self.batch, dtype=torch.uint8, device=self.pool.device)
            ops.release(self.free_stack, self.free_top, self.block_table, self.lens, mask,
                        self.block_size, self.status)
        self.length = 0


def _reference_forward(comp: object) -> bool:
    """Whether calling ``comp`` runs TokenLevelCompressor.forward itself
    (csa.py:66-88) and nothing around it: a torch module whose class has a
    ``TokenLevelCompressor`` on its MRO whose ``forward`` is the one the
    module resolves (no subclass overrides it, e.g. with the overlapping a/b
    pooling that csa.py:78-79 leaves for later), with no forward hooks or
    pre-hooks of its own or global ones."""
    if not isinstance(comp, torch.nn.Module):
        return False
    cls = next((k for k in type(comp).__mro__ if k.__name__ == "TokenLevelCompressor"), None)
    if cls is None or "forward" not in vars(cls) or type(comp).forward is not vars(cls)["forward"]:
        return False
    if comp._forward_hooks or comp._forward_pre_hooks:
        return False
    from torch.nn.modules import module as _module

    return not (_module._global_forward_hooks or _module._global_forward_pre_hooks)


def _fast_compressor(comp: object, m: int, c: int) -> tuple | None:
    """(w_b_kv, w_b_z, bias_b) of a TokenLevelCompressor module with this
    cache's compression rate and channels (csa.py:59-64) whose forward is the
    reference's own (_reference_forward): the b-branch projections and
    positional bias that forward pools with (csa.py:73-87; the a-branch is
    computed there but unused).  None for any other callable, which is then
    called as the reference calls it."""
    if not _reference_forward(comp):
        return None
    w_kv, w_z, bias = (getattr(comp, n, None) for n in ("w_b_kv", "w_b_z", "bias_b"))
    if not (callable(w_kv) and callable(w_z) and isinstance(bias, Tensor)):
        return None
    if getattr(comp, "m", None) != m or getattr(comp, "c", None) != c or tuple(bias.shape) != (m, c):
        return None
    return w_kv, w_z, bias


def _check_3d(what: str, *ts: Tensor) -> None:
    if any(t.dim() != 3 for t in ts):
        shapes = ", ".join(str(tuple(t.shape)) for t in ts)
        raise ValueError(f"{what} must all be 3D (B, T, *); got {shapes}")


class SWAKVCacheLayer:
    """Append-only KV cache for ``SWAttention`` on paged storage (kv_cache.py:32-87).

    K and V of a token share one page row ([K | V]); ``append`` returns the
    contiguous (B, length, head_dim) K and V.
    """

    def __init__(self, max_seq_len: int, head_dim: int, *, batch_size: int = 1,
                 device: torch.device | str | None = None, dtype: torch.dtype = torch.float32,
                 block_size: int = DEFAULT_BLOCK_SIZE) -> None:
        if max_seq_len <= 0:
            raise ValueError(f"max_seq_len must be positive; got {max_seq_len}")
        self.max_seq_len = max_seq_len
        self.head_dim = head_dim
        self.batch_size = batch_size
        self.dtype = dtype
        self._rows = _PagedRows(batch_size, max_seq_len, (2, head_dim), dtype, _device(device),
                                block_size)

    @property
    def length(self) -> int:
        return self._rows.length

    @property
    def k(self) -> Tensor:
        """(B, max_seq_len, head_dim): rows [0, length) hold the cached keys."""
        return self._rows.out[:, :, 0]

    @property
    def v(self) -> Tensor:
        return self._rows.out[:, :, 1]

    def append(self, k_new: Tensor, v_new: Tensor) -> tuple[Tensor, Tensor]:
        """Append new K/V entries; return the full cache up to the current length."""
        if k_new.dim() != 3 or v_new.dim() != 3:
            raise ValueError(
                f"k_new/v_new must be 3D (B, T, head_dim); got {tuple(k_new.shape)}, "
                f"{tuple(v_new.shape)}",
            )
        n = k_new.shape[1]
        if self.length + n > self.max_seq_len:
            raise RuntimeError(
                f"SWAKVCacheLayer overflow: tried to append {n} tokens at "
                f"length {self.length} into max_seq_len={self.max_seq_len}",
            )
        rows = torch.stack([k_new.to(self.dtype), v_new.to(self.dtype)], dim=2)
        full = self._rows.append(rows)
        return full[:, :, 0], full[:, :, 1]

    def reset(self) -> None:
        """Drop all cached entries; ready for a fresh prompt."""
        self._rows.reset()


class _CompressedLayer:
    """Shared HCA/CSA machinery: SW branch rows, h-buffer, compressed streams."""

    kind = "compressed"

    def __init__(self, max_seq_len: int, hidden_dim: int, head_dims: list[int],
                 compression_rate: int, *, batch_size: int, device, dtype: torch.dtype,
                 block_size: int) -> None:
        if max_seq_len <= 0:
            raise ValueError(f"max_seq_len must be positive; got {max_seq_len}")
        if compression_rate <= 0:
            raise ValueError(f"compression_rate must be positive; got {compression_rate}")
        dev = _device(device)
        self.max_seq_len = max_seq_len
        self.hidden_dim = hidden_dim
        self.head_dim = head_dims[0]
        self.compression_rate = compression_rate
        self.batch_size = batch_size
        self.dtype = dtype
        max_blocks = max_seq_len // compression_rate
        self._max_blocks = max_blocks
        self._sw = _PagedRows(batch_size, max_seq_len, (2, head_dims[0]), dtype, dev, block_size)
        self._streams = [_PagedRows(batch_size, max(max_blocks, 1), (d,), dtype, dev, block_size)
                         for d in head_dims]
        self.h_buffer = torch.zeros(batch_size, compression_rate, hidden_dim, device=dev, dtype=dtype)
        self.h_buf_count = 0
        # fast path: per stream the online-softmax state of the block being
        # filled; _tail_folded says whether it holds the buffered tokens
        self._tails = [torch.zeros(batch_size, 3, d, dtype=torch.float32, device=dev) for d in head_dims]
        self._tail_folded = True
        self.fast_appends = 0  # appends that took the fast path

    @property
    def length(self) -> int:
        return self._sw.length

    @property
    def n_blocks(self) -> int:
        return self._streams[0].length

    @property
    def sw_k(self) -> Tensor:
        return self._sw.out[:, :, 0]

    @property
    def sw_v(self) -> Tensor:
        return self._sw.out[:, :, 1]

    def _append(self, name: str, h_new: Tensor, sw_k_new: Tensor, sw_v_new: Tensor,
                compressors: list[Callable[[Tensor], Tensor]]) -> list[Tensor]:
        _check_3d("h_new, sw_k_new, sw_v_new", h_new, sw_k_new, sw_v_new)
        n = sw_k_new.shape[1]
        if self.length + n > self.max_seq_len:
            raise RuntimeError(
                f"{name} overflow: tried to append {n} tokens at "
                f"length {self.length} into max_seq_len={self.max_seq_len}",
            )
        # 1) SW branch K/V (kv_cache.py:167-168)
        rows = torch.stack([sw_k_new.to(self.dtype), sw_v_new.to(self.dtype)], dim=2)
        sw = self._sw.append(rows)
        # 2) combine the buffered h with the new chunk (kv_cache.py:171-179;
        # torch.cat promotes the cache-dtype buffer and h_new as there)
        if self.h_buf_count > 0:
            combined = torch.cat([self.h_buffer[:, : self.h_buf_count], h_new], dim=1)
        else:
            combined = h_new
        total = self.h_buf_count + n
        n_complete = total // self.compression_rate
        n_consumed = n_complete * self.compression_rate
        fast = self._fast_path(compressors)
        if fast is not None:
            # 3') fold the tokens into the pooling state, emit completed blocks
            if n_complete > 0 and self.n_blocks + n_complete > self._max_blocks:
                raise RuntimeError(
                    f"{name} overflow: {self.n_blocks + n_complete} compressed blocks exceed "
                    f"{self._max_blocks}",
                )
            # the tokens the state has not folded yet: the new ones, or the
            # buffered ones too after a compressor call left them out
            h_fold, n_fold = (h_new, n) if self._tail_folded else (combined, total)
            # the reference hands a token to its compressor from h_new when the
            # token's block completes in the same call, else from h_buffer,
            # i.e. rounded to the cache dtype: fold the leftover tokens so
            leftover = total - n_consumed
            if leftover > 0 and h_fold.dtype != self.dtype:
                k = min(leftover, n_fold)
                h_fold = torch.cat([h_fold[:, : n_fold - k], h_fold[:, n_fold - k:].to(self.dtype).to(h_fold.dtype)],
                                   dim=1)
            self._fold(fast, h_fold, n_fold, n_complete, self.n_blocks * self.compression_rate + total)
            self.fast_appends += 1
        # 3) emit complete blocks through the caller's compressors (kv_cache.py:182-189)
        elif n_complete > 0:
            tail = combined[:, :n_consumed]
            outs = [c(tail) for c in compressors]
            if any(o.shape[1] != n_complete for o in outs):
                got = " / ".join(str(o.shape[1]) for o in outs)
                raise RuntimeError(f"compressor returned {got} blocks, expected {n_complete}")
            if self.n_blocks + n_complete > self._max_blocks:
                raise RuntimeError(
                    f"{name} overflow: {self.n_blocks + n_complete} compressed blocks exceed "
                    f"{self._max_blocks}",
                )
            for stream, o in zip(self._streams, outs, strict=True):
                stream.append(o.to(self.dtype).contiguous())
        # 4) stash the leftover tail (kv_cache.py:192-195)
        leftover = total - n_consumed
        if leftover > 0:
            self.h_buffer[:, :leftover] = combined[:, n_consumed:]
        self.h_buf_count = leftover
        # a compressor call leaves the buffered tokens out of the fold state
        self._tail_folded = fast is not None or leftover == 0
        compressed = [s.out[:, : s.length] for s in self._streams]
        return [*compressed, sw[:, :, 0], sw[:, :, 1]]

    def _fast_path(self, compressors: list) -> list | None:
        """The streams' (w_kv, w_z, bias) when every compressor takes the fast path
        (bf16 caches keep bf16 entries; fp32 caches, the reference's default,
        keep unrounded fp32 entries)."""
        if self.dtype not in (torch.bfloat16, torch.float32):
            return None
        out = []
        for comp, stream in zip(compressors, self._streams, strict=True):
            if stream.d % 8 or stream.d > 2048:
                return None
            f = _fast_compressor(comp, self.compression_rate, stream.d)
            if f is None:
                return None
            out.append(f)
        return out

    def _fold(self, fast: list, h: Tensor, n_fold: int, n_complete: int, tok_after: int) -> None:
        """Fold the last n_fold tokens of the compressor token stream, whose
        hidden states are h (the first at a block start or right after the
        tokens already folded), into each stream's pooling state; tok_after is
        the stream's token count after them.  Completed blocks go to the
        stream's pages (skv_compress_append) and its gather buffer."""
        lens = torch.full((self.batch_size,), tok_after, dtype=torch.int32, device=self.h_buffer.device)
        for stream, state, (w_kv, w_z, bias) in zip(self._streams, self._tails, fast, strict=True):
            if n_complete > 0:
                ops.reserve(stream.free_stack, stream.free_top, stream.block_table, stream.lens, n_complete,
                            stream.block_size, stream.status)
            if n_fold > 0:
                hh = h.to(bias.dtype)  # the module's own dtype, as its forward sees it
                with torch.no_grad():  # the kernel consumes raw buffers; no autograd graph
                    # the projections as the module computes them: a bf16
                    # module's bf16 values, otherwise fp32 (pooled unrounded
                    # into a bf16 cache's entries, which round once)
                    pdt = torch.bfloat16 if (bias.dtype == torch.bfloat16 and self.dtype == torch.bfloat16) \
                        else torch.float32
                    c = w_kv(hh).to(pdt).contiguous()
                    z = w_z(hh).to(pdt).contiguous()
                ops.compress_append(stream.pool, stream.block_table, state, c, z,
                                    bias.detach().to(torch.float32).contiguous(), lens, n_fold)
            if n_complete > 0:
                first_page = stream.length // stream.block_size  # the page of the first new entry
                stream.length += n_complete
                ops.paged_gather(stream.pool, stream.block_table, stream.lens, stream._out,
                                 first_page=first_page)

    def reset(self) -> None:
        self._sw.reset()
        for s in self._streams:
            s.reset()
        self.h_buf_count = 0
        self._tail_folded = True


class HCAKVCacheLayer(_CompressedLayer):
    """Append-only KV cache for ``HCA`` on paged storage (kv_cache.py:90-207)."""

    def __init__(self, max_seq_len: int, hidden_dim: int, head_dim: int, compression_rate: int, *,
                 batch_size: int = 1, device: torch.device | str | None = None,
                 dtype: torch.dtype = torch.float32, block_size: int = DEFAULT_BLOCK_SIZE) -> None:
        super().__init__(max_seq_len, hidden_dim, [head_dim], compression_rate,
                         batch_size=batch_size, device=device, dtype=dtype, block_size=block_size)

    @property
    def compressed(self) -> Tensor:
        """(B, max_blocks, head_dim): rows [0, n_blocks) hold the compressed entries."""
        return self._streams[0].out

    def append(self, h_new: Tensor, sw_k_new: Tensor, sw_v_new: Tensor, *,
               compressor: Callable[[Tensor], Tensor]) -> tuple[Tensor, Tensor, Tensor]:
        """Append T_new tokens; return (compressed_view, sw_k_view, sw_v_view)."""
        out = self._append("HCAKVCacheLayer", h_new, sw_k_new, sw_v_new, [compressor])
        return out[0], out[1], out[2]


class CSAKVCacheLayer(_CompressedLayer):
    """Append-only KV cache for ``CSA`` on paged storage (kv_cache.py:210-327).

    The main (``compressed_kv``) and indexer (``indexer_kv``) streams advance in
    lockstep on m-aligned boundaries.
    """

    def __init__(self, max_seq_len: int, hidden_dim: int, head_dim: int, c_indexer: int,
                 compression_rate: int, *, batch_size: int = 1,
                 device: torch.device | str | None = None, dtype: torch.dtype = torch.float32,
                 block_size: int = DEFAULT_BLOCK_SIZE) -> None:
        super().__init__(max_seq_len, hidden_dim, [head_dim, c_indexer], compression_rate,
                         batch_size=batch_size, device=device, dtype=dtype, block_size=block_size)
        self.c_indexer = c_indexer

    @property
    def compressed_kv(self) -> Tensor:
        return self._streams[0].out

    @property
    def indexer_kv(self) -> Tensor:
        return self._streams[1].out

    def append(self, h_new: Tensor, sw_k_new: Tensor, sw_v_new: Tensor, *,
               compressor: Callable[[Tensor], Tensor],
               indexer_compressor: Callable[[Tensor], Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor]:
        """Append T_new tokens. Returns (compressed_kv, indexer_kv, sw_k, sw_v) views."""
        out = self._append("CSAKVCacheLayer", h_new, sw_k_new, sw_v_new,
                           [compressor, indexer_compressor])
        return out[0], out[1], out[2], out[3]


_CacheLayer = SWAKVCacheLayer | HCAKVCacheLayer | CSAKVCacheLayer | None


def _attention_kind(attention: object) -> str | None:
    """"SWAttention", "HCA" or "CSA" if one of those class names is on the
    module's MRO, tried in that order (the isinstance chain of
    kv_cache.py:395-426); None otherwise."""
    names = {c.__name__ for c in type(attention).__mro__}
    for kind in ("SWAttention", "HCA", "CSA"):
        if kind in names:
            return kind
    return None


class KVCacheBundle:
    """Per-layer KV cache container indexed by transformer block index (kv_cache.py:333-427)."""

    def __init__(self, layers: list[_CacheLayer]) -> None:
        self._layers = list(layers)

    def __len__(self) -> int:
        return len(self._layers)

    def for_layer(self, idx: int) -> _CacheLayer:
        """Return the cache for block ``idx`` or ``None`` if uncached."""
        return self._layers[idx]

    @property
    def length(self) -> int:
        """Decoded positions cached in the first populated entry (all advance in lockstep)."""
        for layer in self._layers:
            if layer is not None:
                return layer.length
        return 0

    def reset(self) -> None:
        for layer in self._layers:
            if layer is not None:
                layer.reset()

    @classmethod
    def for_model(cls, model: object, *, max_seq_len: int, batch_size: int = 1,
                  device: torch.device | str | None = None,
                  dtype: torch.dtype = torch.float32) -> KVCacheBundle:
        """Build a bundle by walking ``model.blocks`` (kv_cache.py:369-427).

        Attention modules are recognised by the class names along their MRO
        (``SWAttention``, ``HCA``, ``CSA``, checked in the reference's
        isinstance order), so subclasses map as they do in the reference and
        the bundle needs no import of the model package.
        """
        cfg = model.cfg  # type: ignore[attr-defined]
        head_dim = cfg.attention.head_dim
        hidden_dim = cfg.hidden_dim
        layers: list[_CacheLayer] = []
        for block in model.blocks:  # type: ignore[attr-defined]
            kind = _attention_kind(block.attention)
            if kind == "SWAttention":
                layers.append(SWAKVCacheLayer(max_seq_len=max_seq_len, head_dim=head_dim,
                                              batch_size=batch_size, device=device, dtype=dtype))
            elif kind == "HCA":
                layers.append(HCAKVCacheLayer(max_seq_len=max_seq_len, hidden_dim=hidden_dim,
                                              head_dim=head_dim,
                                              compression_rate=cfg.hca.compression_rate,
                                              batch_size=batch_size, device=device, dtype=dtype))
            elif kind == "CSA":
                layers.append(CSAKVCacheLayer(max_seq_len=max_seq_len, hidden_dim=hidden_dim,
                                              head_dim=head_dim,
                                              c_indexer=cfg.csa.indexer_head_dim,
                                              compression_rate=cfg.csa.compression_rate,
                                              batch_size=batch_size, device=device, dtype=dtype))
            else:
                layers.append(None)
        return cls(layers)
