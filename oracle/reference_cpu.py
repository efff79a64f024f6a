"""CPU oracle for the heterogeneous KV-cache path — TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU with torch-eager and numpy, what the reference
(iZonex/saint-llm, ``packages/inference`` and the cache-consuming slices of
``packages/core`` / ``packages/kernels``) computes on this path, extended to the
paged / ragged form the HIP library implements.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only to verify results or as the timed CPU baseline — never as a
product code path.  The HIP library never calls into it.

Pinning (what fixes each function independently of this file):
  * contiguous caches      — restate kv_cache.py:32-327 line for line in
                             behaviour; pinned by the reference test behaviours
                             (tests/test_oracle_paged.py, test_oracle_compute.py).
  * paged append / gather  — closed form: the gather of a paged sequence equals
                             the concatenation of everything appended to it
                             (tests/test_oracle_paged.py, brute force).
  * reserve / release /
    compact                — documented allocation policy; pinned by invariants
                             (no double ownership, free ∪ used = pool, pop order)
                             and hand-worked small cases.
  * SWA ring               — closed form: last min(W, L) positions in order.
  * compression pooling    — textbook per-channel softmax over the m tokens;
                             pinned by uniform-weight, one-hot and m=1 cases and
                             a pure-Python math.exp brute force.
  * indexer scores         — einsum + clamp(min=0) + weighted head sum of
                             kernels/attention.py:33-50 in fp64; pinned by a
                             pure-Python loop, the reference test's invariant
                             (positive weights give non-negative scores) and
                             ReLU-before-weighting / orthogonal special cases.
  * top-k select           — torch.topk (the reference's library routine) on
                             distinct scores, causal-mask geometry of
                             kernels/attention.py:53-57, -1 padding.
  * sparse gather          — torch.gather formula of csa.py:326-331 on the
                             contiguous restatement plus brute force.
  * FP8 e4m3fn             — torch's float8_e4m3fn cast (the call site of
                             quant/reference.py:109-110) on 1x128 blocks;
                             fmax, zero-block, saturation special cases.
  * decode attention       — scaled_dot_product / softmax_with_sink /
                             RMSNorm of common.py in fp64; pinned by torch's
                             scaled_dot_product_attention and rms_norm
                             (library routines), the sink's closed form
                             (equal logits give 1/(n+1)), one-key and
                             all-masked special cases, the HCA visibility
                             rule by brute force, and a pure-Python loop.
No function here is "parity unpinned".
"""

from __future__ import annotations

from collections.abc import Callable
import numpy as np
import torch
from torch import Tensor

FLT_MIN = float(np.finfo(np.float32).tiny)
E4M3_MAX = 448.0

# Packed FP8 compressed-entry layout: 512 e4m3 codes, 4 fp32 scales (one per
# 1x128 block of the main dims), 64 bf16 rope dims = 656 bytes.
FP8_MAIN = 512
FP8_BLOCK = 128
FP8_ROPE = 64
FP8_ENTRY_BYTES = FP8_MAIN + 4 * (FP8_MAIN // FP8_BLOCK) + 2 * FP8_ROPE


# ===========================================================================
# Contiguous caches: the reference semantics (kv_cache.py)
# ===========================================================================
class ContiguousSWA:
    """SWAKVCacheLayer semantics (kv_cache.py:32-87): one cursor, contiguous rows."""

    def __init__(self, max_seq_len: int, head_dim: int, *, batch_size: int = 1,
                 dtype: torch.dtype = torch.float32) -> None:
        if max_seq_len <= 0:  # kv_cache.py:54-55
            raise ValueError(f"max_seq_len must be positive; got {max_seq_len}")
        self.max_seq_len = max_seq_len
        self.head_dim = head_dim
        self.batch_size = batch_size
        self.k = torch.zeros(batch_size, max_seq_len, head_dim, dtype=dtype)
        self.v = torch.zeros(batch_size, max_seq_len, head_dim, dtype=dtype)
        self.length = 0

    def append(self, k_new: Tensor, v_new: Tensor) -> tuple[Tensor, Tensor]:
        if k_new.dim() != 3 or v_new.dim() != 3:  # kv_cache.py:69-73
            raise ValueError("k_new/v_new must be 3D (B, T, head_dim)")
        n = k_new.shape[1]
        if self.length + n > self.max_seq_len:  # kv_cache.py:75-79
            raise RuntimeError("SWAKVCacheLayer overflow")
        self.k[:, self.length:self.length + n] = k_new  # kv_cache.py:80-81
        self.v[:, self.length:self.length + n] = v_new
        self.length += n
        return self.k[:, :self.length], self.v[:, :self.length]  # kv_cache.py:83

    def reset(self) -> None:
        self.length = 0


class ContiguousCompressed:
    """HCA/CSA block-emission state machine (kv_cache.py:138-202, 266-322).

    ``n_streams`` compressors advance in lockstep (1 for HCA, 2 for CSA).
    """

    def __init__(self, max_seq_len: int, hidden_dim: int, head_dims: list[int],
                 compression_rate: int, *, batch_size: int = 1,
                 dtype: torch.dtype = torch.float32) -> None:
        if max_seq_len <= 0:
            raise ValueError(f"max_seq_len must be positive; got {max_seq_len}")
        if compression_rate <= 0:
            raise ValueError(f"compression_rate must be positive; got {compression_rate}")
        self.max_seq_len = max_seq_len
        self.m = compression_rate
        max_blocks = max_seq_len // compression_rate  # kv_cache.py:127
        self.compressed = [torch.zeros(batch_size, max_blocks, d, dtype=dtype) for d in head_dims]
        self.h_buffer = torch.zeros(batch_size, compression_rate, hidden_dim, dtype=dtype)
        self.h_buf_count = 0
        self.n_blocks = 0
        sw_dim = head_dims[0]
        self.sw_k = torch.zeros(batch_size, max_seq_len, sw_dim, dtype=dtype)
        self.sw_v = torch.zeros(batch_size, max_seq_len, sw_dim, dtype=dtype)
        self.length = 0

    def append(self, h_new: Tensor, sw_k_new: Tensor, sw_v_new: Tensor,
               compressors: list[Callable[[Tensor], Tensor]]) -> tuple[Tensor, ...]:
        n = sw_k_new.shape[1]
        if self.length + n > self.max_seq_len:  # kv_cache.py:160-164
            raise RuntimeError("overflow")
        self.sw_k[:, self.length:self.length + n] = sw_k_new  # :167-168
        self.sw_v[:, self.length:self.length + n] = sw_v_new
        if self.h_buf_count > 0:  # :171-176
            combined = torch.cat([self.h_buffer[:, :self.h_buf_count], h_new], dim=1)
        else:
            combined = h_new
        total = self.h_buf_count + n  # :177-179
        n_complete = total // self.m
        n_consumed = n_complete * self.m
        if n_complete > 0:  # :182-189
            tail = combined[:, :n_consumed]
            outs = [c(tail) for c in compressors]
            for o in outs:
                if o.shape[1] != n_complete:
                    raise RuntimeError(f"compressor returned {o.shape[1]} blocks, expected {n_complete}")
            for buf, o in zip(self.compressed, outs, strict=True):
                buf[:, self.n_blocks:self.n_blocks + n_complete] = o
            self.n_blocks += n_complete
        leftover = total - n_consumed  # :192-195
        if leftover > 0:
            self.h_buffer[:, :leftover] = combined[:, n_consumed:]
        self.h_buf_count = leftover
        self.length += n
        return (*(c[:, :self.n_blocks] for c in self.compressed),
                self.sw_k[:, :self.length], self.sw_v[:, :self.length])


# ===========================================================================
# Page allocation policy (no reference counterpart; planned in
# saint_llm_inference/__init__.py:5-9).  The stack is a LIFO of page ids;
# a pop returns stack[top-1].
# ===========================================================================
STATUS_MAX_PAGES = 1
STATUS_NOSPC = 2
STATUS_BADARG = 4
STATUS_STACK = 8


def free_stack_init(n_pages: int, order: np.ndarray | None = None) -> tuple[np.ndarray, int]:
    """Stack whose successive pops return ``order`` (default 0, 1, 2, ...)."""
    pop_order = np.arange(n_pages, dtype=np.int32) if order is None else np.asarray(order, np.int32)
    return pop_order[::-1].copy(), n_pages


def _ceil_div(a: np.ndarray | int, b: int) -> np.ndarray | int:
    return -(-a // b)


def reserve(stack: np.ndarray, top: int, block_table: np.ndarray, seq_lens: np.ndarray,
            n_new: np.ndarray | int, block_size: int, max_pages: int | None = None) -> tuple[int, int]:
    """Pop pages for rows [L, L+n) of every sequence; advance seq_lens.

    Order: ascending sequence index, then logical page.  All-or-nothing.
    Returns (status bits, new top).  Mutates block_table / seq_lens in place.
    """
    batch = block_table.shape[0]
    max_pages = block_table.shape[1] if max_pages is None else max_pages
    n = np.broadcast_to(np.asarray(n_new, dtype=np.int64), (batch,))
    lens = seq_lens.astype(np.int64)
    status = 0
    if (n < 0).any() or (lens < 0).any():
        status |= STATUS_BADARG
    p0 = _ceil_div(lens, block_size)
    p1 = _ceil_div(lens + np.maximum(n, 0), block_size)
    if (p1 > max_pages).any():
        status |= STATUS_MAX_PAGES
    need = np.where(n >= 0, p1 - p0, 0)
    total = int(need.sum())
    if total > top:
        status |= STATUS_NOSPC
    if status:
        return status, top
    t = 0
    for b in range(batch):
        for j in range(int(need[b])):
            block_table[b, p0[b] + j] = stack[top - 1 - t]
            t += 1
    seq_lens[:] = (lens + n).astype(seq_lens.dtype)
    return 0, top - total


def release(stack: np.ndarray, top: int, block_table: np.ndarray, seq_lens: np.ndarray,
            mask: np.ndarray, block_size: int) -> tuple[int, int]:
    """Push the pages of every sequence with mask[b] back on the stack.

    Push order: ascending b; within b from the last logical page to the first,
    so the next pops return the last released sequence's pages in logical order.
    Released rows of the block table become -1 and their lengths 0.
    Returns (status bits, new top).
    """
    n_pages_total = stack.shape[0]
    batch = block_table.shape[0]
    counts = np.where(mask.astype(bool), _ceil_div(seq_lens.astype(np.int64), block_size), 0)
    if top + int(counts.sum()) > n_pages_total:
        return STATUS_STACK, top
    t = top
    for b in range(batch):
        c = int(counts[b])
        for j in range(c - 1, -1, -1):
            stack[t] = block_table[b, j]
            t += 1
        if mask[b]:
            block_table[b, :c] = -1
            seq_lens[b] = 0
    return 0, t


def live_pages(block_table: np.ndarray, seq_lens: np.ndarray, block_size: int) -> np.ndarray:
    """Physical ids referenced by live rows, in (sequence, logical page) order."""
    out = []
    for b in range(block_table.shape[0]):
        out.extend(block_table[b, : int(_ceil_div(int(seq_lens[b]), block_size))].tolist())
    return np.asarray(out, dtype=np.int64)


def compact_plan(block_table: np.ndarray, seq_lens: np.ndarray, block_size: int,
                 n_pages: int) -> tuple[np.ndarray, np.ndarray, int]:
    """Hole-filling compaction plan.

    n_live = number of live pages.  Live pages with id >= n_live ("movers"),
    ascending, move into the free ids < n_live ("holes"), ascending; pages
    already below n_live keep their id.  Returns (movers, holes, n_live).
    """
    live = np.zeros(n_pages, dtype=bool)
    live[live_pages(block_table, seq_lens, block_size)] = True
    n_live = int(live.sum())
    ids = np.arange(n_pages)
    movers = ids[(ids >= n_live) & live]
    holes = ids[(ids < n_live) & ~live]
    assert movers.shape == holes.shape
    return movers, holes, n_live


def compact(pools: list[Tensor], block_table: np.ndarray, seq_lens: np.ndarray,
            block_size: int) -> tuple[np.ndarray, int, int]:
    """Apply the compaction plan: copy pages, rewrite tables, rebuild the stack.

    Returns (stack, top, n_moved).  After it, live pages are exactly
    [0, n_live) and pops return n_live, n_live+1, ...
    """
    n_pages = pools[0].shape[0]
    movers, holes, n_live = compact_plan(block_table, seq_lens, block_size, n_pages)
    remap = np.arange(n_pages)
    remap[movers] = holes
    for p in pools:
        if len(movers):
            p[torch.from_numpy(holes)] = p[torch.from_numpy(movers)]
    for b in range(block_table.shape[0]):
        c = int(_ceil_div(int(seq_lens[b]), block_size))
        block_table[b, :c] = remap[block_table[b, :c]]
    stack, _ = free_stack_init(n_pages - n_live, np.arange(n_live, n_pages, dtype=np.int32))
    full = np.zeros(n_pages, dtype=np.int32)
    full[: n_pages - n_live] = stack
    return full, n_pages - n_live, len(movers)


# ===========================================================================
# Paged append / gather (kv_cache.py:80-83 on paged storage)
# ===========================================================================
def paged_append(pool: Tensor, block_table: np.ndarray, seq_lens: np.ndarray,
                 src: Tensor, n_new: np.ndarray | int) -> None:
    """Write rows [L-n, L) (seq_lens already advanced) of each sequence."""
    bs = pool.shape[1]
    n = np.broadcast_to(np.asarray(n_new), (block_table.shape[0],))
    for b in range(block_table.shape[0]):
        L = int(seq_lens[b])
        for i in range(int(n[b])):
            pos = L - int(n[b]) + i
            pool[int(block_table[b, pos // bs]), pos % bs] = src[b, i]


def paged_gather(pool: Tensor, block_table: np.ndarray, seq_lens: np.ndarray,
                 out: Tensor) -> Tensor:
    """out[b, :L_b] = rows 0..L_b-1 of sequence b, in order."""
    bs = pool.shape[1]
    for b in range(block_table.shape[0]):
        L = int(seq_lens[b])
        if L == 0:
            continue
        pages = torch.from_numpy(block_table[b, : int(_ceil_div(L, bs))].astype(np.int64))
        rows = pool[pages].reshape(-1, *pool.shape[2:])[:L]
        out[b, :L] = rows
    return out


# ===========================================================================
# SWA ring (swa.py:115-125, csa.py:352-360: visible = last min(W, L) keys)
# ===========================================================================
def ring_append(ring: Tensor, seq_lens_before: np.ndarray, src: Tensor,
                n_new: np.ndarray | int) -> None:
    """ring[b, pos % W] = token at absolute position pos; later writes win."""
    w = ring.shape[1]
    n = np.broadcast_to(np.asarray(n_new), (ring.shape[0],))
    for b in range(ring.shape[0]):
        for i in range(int(n[b])):
            ring[b, (int(seq_lens_before[b]) + i) % w] = src[b, i]


def ring_read(ring: Tensor, seq_lens: np.ndarray, out: Tensor) -> Tensor:
    """out[b, r] = token at position L-n+r, n = min(W, L), r < n (positional order)."""
    w = ring.shape[1]
    for b in range(ring.shape[0]):
        L = int(seq_lens[b])
        n = min(w, L)
        for r in range(n):
            out[b, r] = ring[b, (L - n + r) % w]
    return out


def swa_window_positions(L: int, window: int) -> list[int]:
    """Key positions visible to a decode query at L-1 (swa.py:119-125)."""
    q = L - 1
    return [k for k in range(L) if k <= q and q - k < window]


# ===========================================================================
# Compression pooling (TokenLevelCompressor, csa.py:79-87)
# ===========================================================================
def compress_pool(c: Tensor, z: Tensor, bias: Tensor) -> Tensor:
    """out[..., j] = sum_i softmax_i(z[..., i, j] + bias[i, j]) * c[..., i, j].

    c, z: (..., m, C); bias (m, C).  fp32 arithmetic, fp32 result.
    """
    w = torch.softmax(z.float() + bias.float(), dim=-2)  # csa.py:82, 86
    return (w * c.float()).sum(dim=-2)  # csa.py:87


# Pooling parity: 1e-2 relative to the entry, plus a cancellation term.  A
# GPU entry is the same fp32 softmax-weighted sum in another order (online
# softmax, hardware exp), rounded once to bf16 (2^-9 relative, inside the
# 1e-2).  Each weight and product carries a few fp32 ulps of relative error,
# so the absolute error of the sum scales with sum_i w_i |c_i|, not with the
# result, which is near zero when the terms cancel; 1e-4 of that sum covers
# m=128 terms of ~1e-7 relative error each with a margin of about 8.
POOL_REL = 1.0e-2
POOL_CANCEL = 1.0e-4


def pooling_bound(c: Tensor, z: Tensor, bias: Tensor) -> Tensor:
    """Per-channel tolerance of a pooled entry against compress_pool:
    POOL_REL * |out| + POOL_CANCEL * sum_i w_i |c_i| (fp32, shape of the output)."""
    w = torch.softmax(z.float() + bias.float(), dim=-2)
    out = (w * c.float()).sum(dim=-2)
    return POOL_REL * out.abs() + POOL_CANCEL * (w * c.float().abs()).sum(dim=-2)


BF16_ULP = 2.0 ** -8  # one unit in the last place of bf16, relative (round to nearest: half of it)


def pooling_bound_rounded_inputs(c: Tensor, z: Tensor, bias: Tensor, u: float = BF16_ULP) -> Tensor:
    """pooling_bound widened for projections c, z that the pooled side holds
    rounded to a format of relative precision u (bf16 GEMM outputs), while
    c, z here are the exact (fp32) projections.  With w = softmax(z + bias)
    and out = sum_i w_i c_i, the first-order change of out is
    d out = sum_i w_i dc_i + sum_i w_i (c_i - out) dz_i, so |dc_i| <= u |c_i|
    and |dz_i| <= u |z_i| move out by at most
    u * (sum_i w_i |c_i| + sum_i w_i |c_i - out| |z_i|); twice that is added
    for the second-order terms."""
    w = torch.softmax(z.float() + bias.float(), dim=-2)
    cf = c.float()
    out = (w * cf).sum(dim=-2, keepdim=True)
    drift = (w * cf.abs()).sum(dim=-2) + (w * (cf - out).abs() * z.float().abs()).sum(dim=-2)
    return pooling_bound(c, z, bias) + 2.0 * u * drift


def compress_append(pool: Tensor, block_table: np.ndarray, tail_c: Tensor, tail_z: Tensor,
                    c_new: Tensor, z_new: Tensor, bias: Tensor, seq_lens: np.ndarray,
                    n_new: np.ndarray | int, fp8: bool = False,
                    bound_pool: Tensor | None = None) -> list[tuple[int, int, Tensor]]:
    """Emission state machine of kv_cache.py:170-195 / 291-315 on paged entries.

    seq_lens are token counts after the append.  Every block of m tokens
    completed by the n_new tokens is pooled (compress_pool, rounded to bf16)
    into entry floor(p/m); the incomplete block's new tokens go to the tails
    (slot p % m).  With bound_pool (fp32, the pool's pages and slots), the
    entry's pooling_bound goes to the same slot.  Returns [(b, entry, bf16
    value)] of the emitted entries.
    """
    m = tail_c.shape[1]
    bs = pool.shape[1]
    n = np.broadcast_to(np.asarray(n_new), (block_table.shape[0],))
    emitted = []
    for b in range(block_table.shape[0]):
        L, k = int(seq_lens[b]), int(n[b])
        if k <= 0:
            continue
        first_new = L - k

        def row(t: Tensor, tail: Tensor, p: int) -> Tensor:
            return tail[b, p % m] if p < first_new else t[b, p - first_new]

        for e in range(first_new // m, L // m):
            cs = torch.stack([row(c_new, tail_c, e * m + i) for i in range(m)])
            zs = torch.stack([row(z_new, tail_z, e * m + i) for i in range(m)])
            val = compress_pool(cs, zs, bias).to(torch.bfloat16)
            page, slot = int(block_table[b, e // bs]), e % bs
            pool[page, slot] = fp8_pack_entries(val.unsqueeze(0))[0] if fp8 else val
            if bound_pool is not None:
                bound_pool[page, slot] = pooling_bound(cs, zs, bias)
            emitted.append((b, e, val))
        for p in range(max(first_new, (L // m) * m), L):
            tail_c[b, p % m] = c_new[b, p - first_new]
            tail_z[b, p % m] = z_new[b, p - first_new]
    return emitted


class TokenLevelCompressor(torch.nn.Module):
    """csa.py:41-88 restated: two branches of projections (a, b) and
    positional biases; the forward pools every m hidden states with the
    b-branch only (softmax over the m tokens per channel, weighted sum of the
    b-branch values); the a-branch is computed and unused, as there.  Plain
    nn.Linear projections without bias (the default linear factory)."""

    def __init__(self, hidden_dim: int, c: int, m: int) -> None:
        super().__init__()
        self.c, self.m = c, m
        self.w_a_kv = torch.nn.Linear(hidden_dim, c, bias=False)
        self.w_b_kv = torch.nn.Linear(hidden_dim, c, bias=False)
        self.w_a_z = torch.nn.Linear(hidden_dim, c, bias=False)
        self.w_b_z = torch.nn.Linear(hidden_dim, c, bias=False)
        self.bias_a = torch.nn.Parameter(torch.zeros(m, c))
        self.bias_b = torch.nn.Parameter(torch.zeros(m, c))

    def forward(self, h: Tensor) -> Tensor:
        b, t, _ = h.shape
        usable = (t // self.m) * self.m  # csa.py:67-70
        if usable == 0:
            return h.new_zeros(b, 0, self.c)
        h_use = h[:, :usable]
        n = usable // self.m
        _ = self.w_a_kv(h_use), self.w_a_z(h_use)  # computed, unused (csa.py:73-76, 84-85)
        c_b = self.w_b_kv(h_use).view(b, n, self.m, self.c)
        z_b = self.w_b_z(h_use).view(b, n, self.m, self.c) + self.bias_b  # csa.py:82
        return (torch.softmax(z_b, dim=-2) * c_b).sum(dim=-2)  # csa.py:86-87


def compress_pool_bf16_module(c: Tensor, z: Tensor, bias: Tensor) -> Tensor:
    """The same pooling with the rounding a bf16 module applies at every op
    (z + bias, softmax and the product each rounded to bf16; csa.py:82-87)."""
    zb = (z.to(torch.bfloat16) + bias.to(torch.bfloat16))
    w = torch.softmax(zb, dim=-2)
    return (w * c.to(torch.bfloat16)).sum(dim=-2)


# ===========================================================================
# Lightning-indexer scores (kernels/attention.py:33-50; csa.py:405-409)
# ===========================================================================
def indexer_scores(q: np.ndarray, k: np.ndarray, w: np.ndarray) -> np.ndarray:
    """scores[b, t, s] = sum_h w[b, t, h] * max(0, q[b, t, h, :] . k[b, s, :]),
    unmasked, in fp64: the einsum "bthc,bnc->bthn", clamp(min=0) and weighted
    sum over heads of lightning_indexer_scores_reference (attention.py:47-50;
    the cached path, csa.py:405-409).  q (B, T, H, c), k (B, S, c), w (B, T, H)."""
    hs = np.einsum("bthc,bsc->bths", np.asarray(q, np.float64), np.asarray(k, np.float64))
    return (np.asarray(w, np.float64)[..., None] * np.maximum(hs, 0.0)).sum(axis=2)


def indexer_scores_bound(q: np.ndarray, k: np.ndarray, w: np.ndarray) -> np.ndarray:
    """sum_h |w| * sum_c |q k| per score: the magnitude that fp32 accumulation
    errors of indexer_scores scale with."""
    aq = np.abs(np.asarray(q, np.float64))
    ak = np.abs(np.asarray(k, np.float64))
    return (np.abs(np.asarray(w, np.float64))[..., None] * np.einsum("bthc,bsc->bths", aq, ak)).sum(axis=2)


# ===========================================================================
# Top-k selection (csa.py:405-422; kernels/attention.py:53-89)
# ===========================================================================
def order_key(scores: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 key of fp32 scores (-0.0 folded onto +0.0, NaN
    above +inf as torch.topk ranks it)."""
    s = np.asarray(scores, dtype=np.float32)
    s = np.where(s == 0.0, np.float32(0.0), s)
    u = s.view(np.uint32)
    key = np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint32)
    return np.where(np.isnan(s), np.uint32(0xFFFFFFFF), key)


def n_valid_blocks(q_pos: int, m: int) -> int:
    """#blocks s with s*m + m - 1 < q_pos (kernels/attention.py:53-57)."""
    return max(0, q_pos // m)


def topk_select(scores: np.ndarray, n_valid: np.ndarray, k: int, n_blocks: int) -> np.ndarray:
    """Rows of fp32 scores -> (R, k_eff) int64 indices, k_eff = min(k, n_blocks).

    Entries s >= n_valid[r] are masked to -inf (causal mask, csa.py:411-415);
    the order is descending score, ties by ascending index; picks whose score
    is not finite (NaN, +inf or -inf) become -1 (isfinite, csa.py:420-422).
    """
    scores = np.asarray(scores, dtype=np.float32)[:, :n_blocks]
    rows = scores.shape[0]
    k_eff = min(k, n_blocks)
    out = np.full((rows, k_eff), -1, dtype=np.int64)
    if k_eff == 0:
        return out
    for r in range(rows):
        s = scores[r].copy()
        s[int(n_valid[r]):] = -np.inf
        key = order_key(s)
        idx = np.arange(n_blocks)
        order = np.lexsort((idx, ~key))[:k_eff]
        picks = np.where(~np.isfinite(s[order]), -1, order)
        out[r] = picks
    return out


def topk_select_torch(scores: Tensor, n_valid: np.ndarray, k: int, n_blocks: int) -> Tensor:
    """The reference's own formulation (csa.py:411-422) for cross-checking."""
    s = scores[:, :n_blocks].clone()
    ar = torch.arange(n_blocks).unsqueeze(0)
    s = s.masked_fill(ar >= torch.as_tensor(n_valid).unsqueeze(-1), float("-inf"))
    k_eff = min(k, n_blocks)
    if k_eff == 0:
        return torch.full((s.shape[0], 0), -1, dtype=torch.long)
    top_scores, top_idx = s.topk(k_eff, dim=-1)
    return torch.where(torch.isfinite(top_scores), top_idx, top_idx.new_full((), -1))


# ===========================================================================
# Sparse top-k gather (csa.py:326-331) on paged storage
# ===========================================================================
def topk_gather(pool: Tensor, block_table: np.ndarray, seq_of_row: np.ndarray,
                idx: np.ndarray, out: Tensor) -> Tensor:
    """out[r, j] = entry max(idx[r, j], 0) of sequence seq_of_row[r]; a -1 pick
    copies entry 0, as clamp(min=0) + torch.gather do in csa.py:328-331."""
    bs = pool.shape[1]
    for r in range(idx.shape[0]):
        b = int(seq_of_row[r])
        for j in range(idx.shape[1]):
            e = max(int(idx[r, j]), 0)
            out[r, j] = pool[int(block_table[b, e // bs]), e % bs]
    return out


def contiguous_sparse_gather(compressed: Tensor, idx: Tensor) -> Tensor:
    """csa.py:328-331 verbatim in behaviour: (B, nb, D) x (B, t, k) -> (B, t, k, D)."""
    b, t, _ = idx.shape
    nb, d = compressed.shape[1], compressed.shape[2]
    gi = idx.clamp(min=0).unsqueeze(-1).expand(-1, -1, -1, d)
    return torch.gather(compressed.unsqueeze(1).expand(b, t, nb, d), 2, gi)


# ===========================================================================
# FP8 e4m3fn 1x128 blocks (quant/reference.py:75-116)
# ===========================================================================
def fp8_quantize_blocks(x: Tensor, block: int = FP8_BLOCK) -> tuple[Tensor, Tensor]:
    """cast_to_fp8(x.reshape(-1, block), axis=0): per-row-of-128 absmax scale.

    Returns (codes uint8 (..., n), scales fp32 (..., n/block)).
    """
    shp = x.shape
    xb = x.reshape(-1, block)
    amax = xb.detach().abs().to(torch.float32).amax(dim=1, keepdim=True)  # :76-78
    scale = (amax / E4M3_MAX).clamp(min=FLT_MIN)  # :79
    q = (xb.to(torch.float32) / scale).clamp(-E4M3_MAX, E4M3_MAX)  # :109
    fp8 = q.to(torch.float8_e4m3fn)  # :110
    return fp8.view(torch.uint8).reshape(shp), scale.reshape(*shp[:-1], shp[-1] // block)


def fp8_dequantize_blocks(codes: Tensor, scales: Tensor, block: int = FP8_BLOCK) -> Tensor:
    """dequant_from_fp8 (:114-116) then RNE to bf16."""
    shp = codes.shape
    f = codes.reshape(-1, block).view(torch.float8_e4m3fn).to(torch.float32)
    return (f * scales.reshape(-1, 1)).to(torch.bfloat16).reshape(shp)


def fp8_pack_entries(x: Tensor) -> Tensor:
    """(N, 576) bf16 -> (N, 656) uint8 entries: codes | scales | rope (bf16 kept)."""
    assert x.dtype == torch.bfloat16 and x.shape[-1] == FP8_MAIN + FP8_ROPE
    codes, scales = fp8_quantize_blocks(x[..., :FP8_MAIN])
    rope = x[..., FP8_MAIN:].contiguous().view(torch.uint8)
    return torch.cat([codes, scales.contiguous().view(torch.uint8), rope], dim=-1)


def fp8_unpack_entries(e: Tensor) -> Tensor:
    """(N, 656) uint8 -> (N, 576) bf16: dequantized main dims + verbatim rope."""
    codes = e[..., :FP8_MAIN].contiguous()
    scales = e[..., FP8_MAIN:FP8_MAIN + 16].contiguous().view(torch.float32)
    rope = e[..., FP8_MAIN + 16:].contiguous().view(torch.bfloat16)
    return torch.cat([fp8_dequantize_blocks(codes, scales), rope], dim=-1)


# ===========================================================================
# Decode attention over the cache (csa.py:324-373, hca.py:126-169,
# swa.py:115-137, common.py:12-20 and 77-124), one query token per sequence
# ===========================================================================
def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float = 1.0e-6) -> np.ndarray:
    """RMSNorm.forward (common.py:18-20) in fp64: weight * x / sqrt(mean(x^2) + eps)."""
    x = np.asarray(x, np.float64)
    var = (x * x).mean(axis=-1, keepdims=True)
    return np.asarray(weight, np.float64) * x / np.sqrt(var + eps)


def attention_row(q: np.ndarray, k: np.ndarray, v: np.ndarray, valid: np.ndarray,
                  sink: np.ndarray | None = None, softcap: float | None = None) -> np.ndarray:
    """scaled_dot_product (common.py:92-124) for one query row in fp64.

    q (H, D), k and v (N, D), valid (N,) bool.  scores = q k^T / sqrt(D)
    (:117), softcap c * tanh(s / c) (:120-121), masked keys -inf (:122-123),
    softmax with the per-head sink logit in the denominator (:77-89), then
    probs @ v (:124).  A row without a valid key gives 0: the reference's
    outcome with a sink (all mass on the sink) and its row_has_pick /
    row_has_block zeroing without one (csa.py:344-348, hca.py:137-141).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    valid = np.asarray(valid, bool)
    h, d = q.shape
    if not valid.any():
        return np.zeros((h, v.shape[-1]))
    s = q @ k[valid].T / np.sqrt(d)
    if softcap is not None:
        s = softcap * np.tanh(s / softcap)
    mx = s.max(axis=-1, keepdims=True)
    if sink is not None:
        mx = np.maximum(mx, np.asarray(sink, np.float64)[:, None])
    e = np.exp(s - mx)
    den = e.sum(axis=-1, keepdims=True)
    if sink is not None:
        den = den + np.exp(np.asarray(sink, np.float64)[:, None] - mx)
    return (e @ v[valid]) / den


def csa_sparse_attention(q: np.ndarray, entries: np.ndarray, picks: np.ndarray,
                         knorm_w: np.ndarray, eps: float = 1.0e-6) -> np.ndarray:
    """The sparse branch of CSA.forward (csa.py:324-350) for one query row:
    entries[picks.clamp(0)] through k_norm, K = V, no sink and no softcap; a
    -1 pick is masked.  q (H, D), entries (n_entries, D), picks (k,)."""
    picks = np.asarray(picks, np.int64)
    if not (picks >= 0).any():
        return np.zeros(np.asarray(q).shape)
    keys = rms_norm(np.asarray(entries, np.float64)[np.maximum(picks, 0)], knorm_w, eps)
    return attention_row(q, keys, keys, picks >= 0)


def hca_compressed_attention(q: np.ndarray, entries: np.ndarray, q_pos: int, m: int,
                             knorm_w: np.ndarray, eps: float = 1.0e-6,
                             sink: np.ndarray | None = None) -> np.ndarray:
    """The compressed branch of HCA.forward (hca.py:126-141) for one query
    row at position q_pos: every entry through k_norm, K = V, entry s visible
    when s*m + m - 1 < q_pos (:128-131), the layer's sink, no softcap."""
    entries = np.asarray(entries, np.float64)
    n = entries.shape[0]
    valid = np.arange(n) * m + (m - 1) < q_pos
    keys = rms_norm(entries, knorm_w, eps) if n else entries
    return attention_row(q, keys, keys, valid, sink)


def window_attention(q: np.ndarray, win_k: np.ndarray, win_v: np.ndarray,
                     sink: np.ndarray | None = None, softcap: float | None = None) -> np.ndarray:
    """The sliding-window branch (swa.py:115-136, csa.py:352-371,
    hca.py:143-167) of a decode query: the keys and values of the last
    min(W, L) positions (the mask k_pos <= q_pos and q_pos - k_pos < W of
    swa.py:121-124 keeps exactly those), as cached (k already normed and
    roped by the caller), with the sink and the softcap."""
    n = np.asarray(win_k).shape[0]
    return attention_row(q, win_k, win_v, np.ones(n, bool), sink, softcap)


def decode_attention(q: np.ndarray, kind: str, L: int, *, entries: np.ndarray | None = None,
                     picks: np.ndarray | None = None, m: int = 1,
                     knorm_w: np.ndarray | None = None, eps: float = 1.0e-6,
                     sink: np.ndarray | None = None, softcap: float | None = None,
                     win_k: np.ndarray | None = None, win_v: np.ndarray | None = None) -> np.ndarray:
    """One layer's attention output before the output projection for the
    query of a sequence whose length after the step's append is L:
    compressed branch + window branch (csa.py:373, hca.py:169), window only
    for "swa" (swa.py:137).  CSA's sparse branch takes no sink (csa.py:337-345),
    HCA's compressed branch takes the layer's sink; the softcap applies to the
    window branch only (csa.py:367-371, hca.py:163-167)."""
    out = window_attention(q, win_k, win_v, sink, softcap)
    if kind == "csa":
        out = out + csa_sparse_attention(q, entries, picks, knorm_w, eps)
    elif kind == "hca":
        out = out + hca_compressed_attention(q, entries, L - 1, m, knorm_w, eps, sink)
    else:
        assert kind == "swa", kind
    return out
