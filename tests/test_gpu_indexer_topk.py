"""The cached indexer top-k in the reference's call shape (csa.py:377-422).

``saint_kv.indexer.indexer_topk`` takes what ``CSA._indexer_topk_cached``
computes from its projections (the indexer query and head weights of t_new
query tokens, the cached compressed indexer keys, cache_offset, total_len,
n_blocks, m, top_k) and returns its (B, t_new, min(top_k, n_blocks)) int64
picks with -1 padding, through skv_indexer_scores and skv_topk_select.

* integer-valued inputs, whose scores are exact in fp32: the picks equal the
  oracle's ``topk_select`` over the oracle's fp64 ``indexer_scores``, with
  the causal mask of every query token at its own position, bit for bit
  (many equal scores: ties go to the lower entry);
* N(0,1) inputs: the picks equal the oracle's select over the GPU's scores,
  which are within 1e-5 of the fp32-accumulation bound of the oracle's;
* the method-shaped ``indexer_topk_cached`` runs a stand-in indexer's
  projections (w_dq, w_iuq, w_w) as csa.py:401-404 does and gives the same
  picks as ``indexer_topk`` on them;
* empty results: n_blocks = 0 or top_k = 0 give (B, t_new, 0).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu


def _want(scores: np.ndarray, cache_offset: int, total_len: int, n_blocks: int, m: int, top_k: int) -> np.ndarray:
    """The oracle's picks: one row per (sequence, query token) at its position."""
    b, t, _ = scores.shape
    q_pos = np.arange(cache_offset, total_len)
    n_valid = np.array([ref.n_valid_blocks(int(q), m) for q in q_pos])
    out = np.stack([ref.topk_select(scores[i], np.minimum(n_valid, n_blocks), top_k, n_blocks) for i in range(b)])
    return out.reshape(b, t, -1)


@pytest.mark.parametrize("t_new,n_blocks,top_k,m", [(1, 300, 64, 4), (4, 300, 512, 4), (3, 5000, 512, 4),
                                                     (2, 700, 48, 128), (5, 17, 2048, 2)])
def test_indexer_topk_exact_scores_match_oracle(dev, t_new, n_blocks, top_k, m) -> None:
    from saint_kv.indexer import indexer_topk

    g = torch.Generator().manual_seed(n_blocks + t_new)
    B, H, C = 3, 16, 64
    # small integers: every dot product and weighted sum is exact in fp32
    q = torch.randint(-2, 3, (B, t_new, H, C), generator=g).float()
    k = torch.randint(-2, 3, (B, n_blocks + 5, C), generator=g).float()
    w = torch.randint(-2, 3, (B, t_new, H), generator=g).float() * 0.5
    total_len = n_blocks * m + 2  # the last query tokens see every entry, the first fewer
    cache_offset = total_len - t_new
    got = indexer_topk(q.to(dev), w.to(dev), k.to(dev), cache_offset=cache_offset, total_len=total_len,
                       n_blocks=n_blocks, m=m, top_k=top_k)
    assert got.dtype == torch.long and tuple(got.shape) == (B, t_new, min(top_k, n_blocks))
    scores = ref.indexer_scores(q.numpy(), k[:, :n_blocks].numpy(), w.numpy())
    assert np.array_equal(got.cpu().numpy(), _want(scores, cache_offset, total_len, n_blocks, m, top_k))


def test_indexer_topk_partial_visibility_and_padding(dev) -> None:
    """Query tokens early in a long block: a row whose visible entries are
    fewer than top_k is padded with -1, and each query token of the same
    call sees its own prefix (t_new = 6 tokens spanning two blocks of m = 4)."""
    from saint_kv.indexer import indexer_topk

    g = torch.Generator().manual_seed(7)
    B, H, C, m, n_blocks, top_k = 2, 8, 32, 4, 40, 16
    q = torch.randn(B, 6, H, C, generator=g)
    k = torch.randn(B, n_blocks, C, generator=g)
    w = torch.randn(B, 6, H, generator=g)
    for cache_offset in (0, 3, 30, 62):
        total_len = cache_offset + 6
        got = indexer_topk(q.to(dev), w.to(dev), k.to(dev), cache_offset=cache_offset, total_len=total_len,
                           n_blocks=n_blocks, m=m, top_k=top_k).cpu().numpy()
        from saint_kv.indexer import lightning_indexer_scores

        sc = lightning_indexer_scores(q.to(dev), k.to(dev), w.to(dev)).cpu().numpy()
        want = _want(sc, cache_offset, total_len, n_blocks, m, top_k)
        assert np.array_equal(got, want), cache_offset
        for t in range(6):
            nv = min((cache_offset + t) // m, n_blocks)
            assert (got[:, t, min(nv, top_k):] == -1).all() and (got[:, t, :min(nv, top_k)] >= 0).all()


def test_indexer_topk_normal_scores_against_oracle(dev) -> None:
    from saint_kv.indexer import indexer_topk, lightning_indexer_scores

    g = torch.Generator().manual_seed(3)
    B, t_new, H, C, m, n_blocks, top_k = 4, 3, 64, 128, 4, 9000, 512
    q = torch.randn(B, t_new, H, C, generator=g).to(torch.bfloat16)
    k = torch.randn(B, n_blocks, C, generator=g).to(torch.bfloat16)
    w = torch.randn(B, t_new, H, generator=g)
    total_len = n_blocks * m - 7
    cache_offset = total_len - t_new
    got = indexer_topk(q.to(dev), w.to(dev), k.to(dev), cache_offset=cache_offset, total_len=total_len,
                       n_blocks=n_blocks, m=m, top_k=top_k).cpu().numpy()
    sc = lightning_indexer_scores(q.to(dev), k.to(dev), w.to(dev)).cpu()
    exact = ref.indexer_scores(q.float().numpy(), k.float().numpy(), w.numpy())
    bound = ref.indexer_scores_bound(q.float().numpy(), k.float().numpy(), w.numpy())
    assert (np.abs(sc.numpy() - exact) <= 1e-5 * bound).all()  # fp32 accumulation of bf16 products
    assert np.array_equal(got, _want(sc.numpy(), cache_offset, total_len, n_blocks, m, top_k))
    # the reference's own formulation picks the same sets (csa.py:411-422)
    for b in range(B):
        nv = np.array([min((cache_offset + t) // m, n_blocks) for t in range(t_new)])
        tr = ref.topk_select_torch(sc[b], nv, top_k, n_blocks).numpy()
        for t in range(t_new):
            assert set(tr[t].tolist()) == set(got[b, t].tolist())


def test_indexer_topk_cached_method_shape(dev) -> None:
    from types import SimpleNamespace

    from saint_kv.indexer import indexer_topk, indexer_topk_cached

    g = torch.Generator().manual_seed(9)
    B, t_new, D, H, C, m, n_blocks = 2, 2, 96, 8, 32, 4, 200
    lin = lambda i, o: torch.nn.Linear(i, o, bias=False).to(dev)  # noqa: E731
    torch.manual_seed(9)
    indexer = SimpleNamespace(w_dq=lin(D, 48), w_iuq=lin(48, H * C), w_w=lin(D, H), n_heads=H, c_indexer=C,
                              top_k=32)
    csa = SimpleNamespace(indexer=indexer)
    h = torch.randn(B, t_new, D, generator=g).to(dev)
    k = torch.randn(B, n_blocks, C, generator=g).to(dev)
    total_len = n_blocks * m
    got = indexer_topk_cached(csa, h, k, cache_offset=total_len - t_new, total_len=total_len,
                              n_blocks=n_blocks, m=m, is_visual=None)
    with torch.no_grad():
        q = indexer.w_iuq(indexer.w_dq(h)).view(B, t_new, H, C)
        w = indexer.w_w(h)
    want = indexer_topk(q, w, k, cache_offset=total_len - t_new, total_len=total_len, n_blocks=n_blocks, m=m,
                        top_k=32)
    assert torch.equal(got, want)


def test_indexer_topk_empty(dev) -> None:
    from saint_kv.indexer import indexer_topk

    q = torch.randn(2, 3, 4, 16, device=dev)
    w = torch.randn(2, 3, 4, device=dev)
    k = torch.randn(2, 10, 16, device=dev)
    for n_blocks, top_k in ((0, 8), (10, 0)):
        got = indexer_topk(q, w, k, cache_offset=5, total_len=8, n_blocks=n_blocks, m=4, top_k=top_k)
        assert tuple(got.shape) == (2, 3, 0) and got.dtype == torch.long
    with pytest.raises(ValueError, match="t_new"):
        indexer_topk(q, w, k, cache_offset=5, total_len=9, n_blocks=10, m=4, top_k=4)
