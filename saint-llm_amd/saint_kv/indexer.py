"""Lightning-indexer scores and the cached top-k on the GPU, in the reference's call shapes.

``lightning_indexer_scores(q_indexer, k_compressed, head_weights)`` mirrors
``lightning_indexer_scores_reference`` (kernels/attention.py:33-50) for
contiguous compressed keys; ``ops.indexer_scores`` takes the paged cache
(``DecodeCache.idx_pool``).  Both run ``skv_indexer_scores`` (bf16 inputs,
fp32 accumulation, fp32 scores).  The visual bias is not supported: the
cached decode path does not use it (csa.py:396-399).

``indexer_topk`` is ``CSA._indexer_topk_cached`` (csa.py:377-422) after the
indexer's projections: scores over the cached compressed indexer keys, the
causal block mask of every query token at its absolute position, top-k and
-1 for non-finite picks, one score row per (sequence, query token), so any
``t_new >= 1`` works.  ``indexer_topk_cached`` has the method's own
signature (it runs the ``self.indexer`` projections of csa.py:401-404 in
torch) for a caller that swaps the method in.
"""

from __future__ import annotations

import torch

from saint_kv import ops


def lightning_indexer_scores(q_indexer: torch.Tensor, k_compressed: torch.Tensor, head_weights: torch.Tensor,
                             visual_bias: torch.Tensor | None = None) -> torch.Tensor:
    """(B, T, n_blocks) unmasked scores: sum_h w[b,t,h] * relu(q[b,t,h,:] . k[b,s,:]).

    q_indexer (B, T, H, c), k_compressed (B, n_blocks, c) and head_weights
    (B, T, H) are cast to bf16 / bf16 / fp32 on their device.
    """
    if visual_bias is not None:
        raise NotImplementedError("visual_bias is not supported (the cached decode path ignores it)")
    if q_indexer.dim() != 4 or k_compressed.dim() != 3 or head_weights.dim() != 3:
        raise ValueError("q_indexer must be (B, T, H, c), k_compressed (B, n_blocks, c), head_weights (B, T, H)")
    b, t, h, c = q_indexer.shape
    n_blocks = k_compressed.shape[1]
    if k_compressed.shape[0] != b or k_compressed.shape[2] != c or tuple(head_weights.shape) != (b, t, h):
        raise ValueError("q_indexer, k_compressed and head_weights disagree on B, T, H or c")
    dev = q_indexer.device
    out = torch.empty(b, t, n_blocks, dtype=torch.float32, device=dev)
    if n_blocks == 0 or b == 0 or t == 0:
        return out
    # one page per sequence: page b holds that sequence's n_blocks keys
    pool = k_compressed.to(torch.bfloat16).contiguous()
    table = torch.arange(b, dtype=torch.int32, device=dev).unsqueeze(1)
    n_ent = torch.full((b,), n_blocks, dtype=torch.int32, device=dev)
    return ops.indexer_scores(q_indexer.to(torch.bfloat16).contiguous(), head_weights.float().contiguous(), pool,
                              table, n_ent, out)


def indexer_topk(q_indexer: torch.Tensor, head_weights: torch.Tensor, k_indexer_comp: torch.Tensor, *,
                 cache_offset: int, total_len: int, n_blocks: int, m: int, top_k: int) -> torch.Tensor:
    """(B, t_new, min(top_k, n_blocks)) int64 picks of csa.py:405-422.

    q_indexer (B, t_new, H, c) and head_weights (B, t_new, H) are the
    indexer's query and head weights of the t_new new tokens at positions
    cache_offset .. total_len - 1; k_indexer_comp (B, >= n_blocks, c) holds
    the cached compressed indexer keys.  Entry s is visible to the query at
    position q iff s * m + m - 1 < q (csa.py:411-415); a row's picks are its
    visible entries by descending score (ties: lower entry first), and a pick
    whose score is not finite (a masked entry, NaN, +-inf) is -1
    (csa.py:420-422).  The scores come from skv_indexer_scores, the picks from
    skv_topk_select (one row per query token).
    """
    if q_indexer.dim() != 4 or head_weights.dim() != 3 or k_indexer_comp.dim() != 3:
        raise ValueError("q_indexer must be (B, t_new, H, c), head_weights (B, t_new, H), "
                         "k_indexer_comp (B, n_blocks, c)")
    b, t_new, _, c = q_indexer.shape
    if total_len - cache_offset != t_new or cache_offset < 0:
        raise ValueError(f"total_len - cache_offset must equal t_new={t_new}; got {cache_offset}..{total_len}")
    if m <= 0 or top_k < 0 or n_blocks < 0 or n_blocks > k_indexer_comp.shape[1]:
        raise ValueError(f"need m > 0, top_k >= 0 and 0 <= n_blocks <= {k_indexer_comp.shape[1]}")
    dev = q_indexer.device
    k_eff = min(top_k, n_blocks)
    if k_eff == 0 or b == 0 or t_new == 0:
        return torch.full((b, t_new, k_eff), -1, dtype=torch.long, device=dev)
    scores = lightning_indexer_scores(q_indexer, k_indexer_comp[:, :n_blocks], head_weights)  # (B, t_new, n)
    # visible entries of the query at position q: s < floor(q / m) (s * m + m - 1 < q)
    q_pos = torch.arange(cache_offset, total_len, device=dev, dtype=torch.int64)
    n_valid = torch.clamp(q_pos // m, max=n_blocks).to(torch.int32).repeat(b)
    rows = b * t_new
    out = torch.empty(rows, k_eff, dtype=torch.int32, device=dev)
    # long rows are spread over several workgroups through a zeroed workspace
    ws = ops.topk_workspace(rows, dev) if n_blocks > 4096 else None
    ops.topk_select(scores.view(rows, n_blocks), n_valid, n_blocks, k_eff, out, ws)
    return out.view(b, t_new, k_eff).long()


def indexer_topk_cached(self, h: torch.Tensor, k_indexer_comp: torch.Tensor, *, cache_offset: int,
                        total_len: int, n_blocks: int, m: int,
                        is_visual: torch.Tensor | None = None) -> torch.Tensor:
    """``CSA._indexer_topk_cached`` (csa.py:377-422) with the HIP scores and
    top-k: ``self.indexer``'s projections (w_dq, w_iuq, w_w; csa.py:401-404)
    run in torch as there, then ``indexer_topk``.  ``is_visual`` is ignored,
    as the reference ignores it on the cached path (csa.py:396-399)."""
    del is_visual
    b, t_new, _ = h.shape
    idx = self.indexer
    with torch.no_grad():
        q = idx.w_iuq(idx.w_dq(h)).view(b, t_new, idx.n_heads, idx.c_indexer)
        w = idx.w_w(h)
    return indexer_topk(q, w, k_indexer_comp, cache_offset=cache_offset, total_len=total_len,
                        n_blocks=n_blocks, m=m, top_k=idx.top_k)
