"""Pin the oracle's paged storage, allocation policy and SWA ring (CPU only).

Each check is independent of the oracle's own formula: concatenation of what
was appended, hand-worked pop orders, set invariants, window closed forms.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref


def _fresh(batch: int, n_pages: int, max_pages: int, order=None):
    stack, top = ref.free_stack_init(n_pages, order)
    bt = np.full((batch, max_pages), -1, dtype=np.int32)
    lens = np.zeros(batch, dtype=np.int32)
    return stack, top, bt, lens


def test_free_stack_pops_ascending_by_default() -> None:
    stack, top = ref.free_stack_init(5)
    assert [int(stack[top - 1 - i]) for i in range(5)] == [0, 1, 2, 3, 4]


def test_free_stack_custom_order() -> None:
    order = np.array([3, 0, 4, 1, 2], dtype=np.int32)
    stack, top = ref.free_stack_init(5, order)
    assert [int(stack[top - 1 - i]) for i in range(5)] == order.tolist()


def test_reserve_hand_worked() -> None:
    # bs=4; seq0 grows 0->5 (2 pages), seq1 0->0, seq2 0->9 (3 pages)
    stack, top, bt, lens = _fresh(3, 10, 4)
    st, top = ref.reserve(stack, top, bt, lens, np.array([5, 0, 9]), 4)
    assert st == 0 and top == 5
    assert bt[0, :2].tolist() == [0, 1] and bt[2, :3].tolist() == [2, 3, 4]
    assert (bt[1] == -1).all() and lens.tolist() == [5, 0, 9]
    # seq0 5->8 stays in page 1; seq2 9->13 needs page 3 (logical) -> id 5
    st, top = ref.reserve(stack, top, bt, lens, np.array([3, 0, 4]), 4)
    assert st == 0 and top == 4 and bt[2, 3] == 5 and lens.tolist() == [8, 0, 13]


def test_reserve_all_or_nothing() -> None:
    stack, top, bt, lens = _fresh(2, 3, 8)
    st, top2 = ref.reserve(stack, top, bt, lens, np.array([8, 8]), 4)  # needs 4 > 3
    assert st == ref.STATUS_NOSPC and top2 == top
    assert (bt == -1).all() and (lens == 0).all()
    stack, top, bt, lens = _fresh(1, 100, 2)
    st, _ = ref.reserve(stack, top, bt, lens, 9, 4)  # 3 pages > max 2
    assert st == ref.STATUS_MAX_PAGES and lens[0] == 0


def test_paged_append_gather_equals_concatenation() -> None:
    g = torch.Generator().manual_seed(0)
    batch, bs, d, n_pages = 3, 4, 8, 64
    order = np.random.default_rng(0).permutation(n_pages).astype(np.int32)
    stack, top, bt, lens = _fresh(batch, n_pages, 16, order)
    pool = torch.zeros(n_pages, bs, d)
    history = [[] for _ in range(batch)]
    for step in range(6):
        n = np.array([step % 3, 5, 1 + step], dtype=np.int32)
        src = torch.randn(batch, int(n.max()), d, generator=g)
        st, top = ref.reserve(stack, top, bt, lens, n, bs)
        assert st == 0
        ref.paged_append(pool, bt, lens, src, n)
        for b in range(batch):
            history[b].append(src[b, : n[b]])
    out = torch.full((batch, int(lens.max()), d), float("nan"))
    ref.paged_gather(pool, bt, lens, out)
    for b in range(batch):
        expect = torch.cat(history[b])
        assert torch.equal(out[b, : lens[b]], expect)
    # every page referenced once; free + used = pool
    used = ref.live_pages(bt, lens, bs)
    assert len(set(used.tolist())) == len(used)
    assert sorted(used.tolist() + stack[:top].tolist()) == list(range(n_pages))


def test_paged_matches_contiguous_reference_semantics() -> None:
    """Lock-step appends reproduce SWAKVCacheLayer's contiguous views (kv_cache.py:80-83)."""
    g = torch.Generator().manual_seed(1)
    cont = ref.ContiguousSWA(max_seq_len=20, head_dim=8, batch_size=2)
    stack, top, bt, lens = _fresh(2, 10, 5, np.random.default_rng(1).permutation(10))
    pool_k = torch.zeros(10, 4, 8)
    for n in (3, 1, 7, 2):
        k = torch.randn(2, n, 8, generator=g)
        full_k, _ = cont.append(k, k)
        st, top = ref.reserve(stack, top, bt, lens, n, 4)
        ref.paged_append(pool_k, bt, lens, k, n)
        out = torch.zeros(2, cont.length, 8)
        ref.paged_gather(pool_k, bt, lens, out)
        assert torch.equal(out, full_k)


def test_contiguous_error_contract() -> None:
    with pytest.raises(ValueError, match="max_seq_len"):
        ref.ContiguousSWA(max_seq_len=0, head_dim=8)
    c = ref.ContiguousSWA(max_seq_len=4, head_dim=8)
    with pytest.raises(RuntimeError, match="overflow"):
        c.append(torch.randn(1, 5, 8), torch.randn(1, 5, 8))
    with pytest.raises(ValueError, match="must be 3D"):
        c.append(torch.randn(1, 8), torch.randn(1, 8))


def test_contiguous_block_emission_state_machine() -> None:
    """3 then 6 tokens at m=4: 2 blocks + 1 leftover (test_kv_cache.py:339-367)."""
    calls = []

    def stub(h):
        calls.append(h.shape[1])
        return torch.full((h.shape[0], h.shape[1] // 4, 4), float(len(calls)))

    c = ref.ContiguousCompressed(16, 8, [4], 4)
    c.append(torch.randn(1, 3, 8), torch.randn(1, 3, 4), torch.randn(1, 3, 4), [stub])
    assert (c.h_buf_count, c.n_blocks) == (3, 0)
    c.append(torch.randn(1, 6, 8), torch.randn(1, 6, 4), torch.randn(1, 6, 4), [stub])
    assert (c.n_blocks, c.h_buf_count, c.length) == (2, 1, 9)
    assert calls == [8]


def test_release_push_order_and_tables() -> None:
    stack, top, bt, lens = _fresh(3, 12, 4)
    st, top = ref.reserve(stack, top, bt, lens, np.array([5, 3, 9]), 4)  # pages [0,1],[2],[3,4,5]
    assert st == 0 and top == 6
    st, top = ref.release(stack, top, bt, lens, np.array([1, 0, 1]), 4)
    assert st == 0 and top == 11
    # pops now return seq2's pages in logical order, then seq0's
    pops = [int(stack[top - 1 - i]) for i in range(5)]
    assert pops == [3, 4, 5, 0, 1]
    assert (bt[0] == -1).all() and (bt[2] == -1).all() and lens.tolist() == [0, 3, 0]
    # releasing more pages than the stack can hold is refused
    st, _ = ref.release(stack, 12, bt, np.array([0, 4, 0], dtype=np.int32), np.array([0, 1, 0]), 4)
    assert st == ref.STATUS_STACK


def test_compaction_fills_holes_and_preserves_content() -> None:
    g = torch.Generator().manual_seed(2)
    rng = np.random.default_rng(2)
    batch, bs, n_pages = 6, 4, 40
    stack, top, bt, lens = _fresh(batch, n_pages, 10, rng.permutation(n_pages))
    pool = torch.randn(n_pages, bs, 3, generator=g)
    n = rng.integers(1, 30, size=batch).astype(np.int32)
    st, top = ref.reserve(stack, top, bt, lens, n, bs)
    before = torch.zeros(batch, int(lens.max()), 3)
    ref.paged_gather(pool, bt, lens, before)
    mask = np.array([1, 0, 0, 1, 0, 1])
    st, top = ref.release(stack, top, bt, lens, mask, bs)
    live_before = ref.live_pages(bt, lens, bs)
    movers, holes, n_live = ref.compact_plan(bt, lens, bs, n_pages)
    assert n_live == len(live_before)
    assert (movers >= n_live).all() and (holes < n_live).all()
    stack, top, moved = ref.compact([pool], bt, lens, bs)
    assert moved == len(movers)
    live = ref.live_pages(bt, lens, bs)
    assert sorted(live.tolist()) == list(range(n_live))
    assert [int(stack[top - 1 - i]) for i in range(top)] == list(range(n_live, n_pages))
    after = torch.zeros_like(before)
    ref.paged_gather(pool, bt, lens, after)
    for b in range(batch):
        if not mask[b]:
            assert torch.equal(after[b, : lens[b]], before[b, : lens[b]])


def test_ring_is_last_window_in_order() -> None:
    g = torch.Generator().manual_seed(3)
    w, batch = 8, 2
    ring = torch.zeros(batch, w, 4)
    lens = np.zeros(batch, dtype=np.int32)
    hist = [[] for _ in range(batch)]
    for n in (3, 9, 1, 5, 0, 12):
        ns = np.array([n, max(n - 1, 0)])
        src = torch.randn(batch, max(n, 1), 4, generator=g)
        ref.ring_append(ring, lens, src, ns)
        for b in range(batch):
            hist[b].extend(src[b, i] for i in range(ns[b]))
        lens = lens + ns
        out = torch.zeros(batch, w, 4)
        ref.ring_read(ring, lens, out)
        for b in range(batch):
            L = int(lens[b])
            vis = ref.swa_window_positions(L, w)
            assert vis == list(range(max(0, L - w), L))
            for r, pos in enumerate(vis):
                assert torch.equal(out[b, r], hist[b][pos])
