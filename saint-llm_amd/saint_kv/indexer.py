"""Lightning-indexer scores on the GPU, in the reference's call shape.

``lightning_indexer_scores(q_indexer, k_compressed, head_weights)`` mirrors
``lightning_indexer_scores_reference`` (kernels/attention.py:33-50) for
contiguous compressed keys; ``ops.indexer_scores`` takes the paged cache
(``DecodeCache.idx_pool``).  Both run ``skv_indexer_scores`` (bf16 inputs,
fp32 accumulation, fp32 scores).  The visual bias is not supported: the
cached decode path does not use it (csa.py:396-399).
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
