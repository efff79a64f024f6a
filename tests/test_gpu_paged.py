"""GPU parity of paged storage: free stack, reserve, append, gather (bit-exact).

The HIP library is called through the C ABI (saint_kv.ops) and compared with
the CPU oracle on the same seeded inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


class _State:
    """Device + oracle copies of one paged cache."""

    def __init__(self, dev, batch, n_pages, max_pages, bs, row_shape, dtype, order=None, seed=0):
        from saint_kv import ops

        self.ops = ops
        self.bs = bs
        self.stack = torch.empty(n_pages, dtype=torch.int32, device=dev)
        self.top = torch.empty(1, dtype=torch.int32, device=dev)
        self.bt = torch.full((batch, max_pages), -1, dtype=torch.int32, device=dev)
        self.lens = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.status = torch.full((1,), -7, dtype=torch.int32, device=dev)
        order_t = None if order is None else torch.as_tensor(order, dtype=torch.int32, device=dev)
        ops.free_stack_init(self.stack, self.top, order_t)
        self.pool = torch.zeros(n_pages, bs, *row_shape, dtype=dtype, device=dev)
        self.r_stack, self.r_top = ref.free_stack_init(n_pages, order)
        self.r_bt = np.full((batch, max_pages), -1, dtype=np.int32)
        self.r_lens = np.zeros(batch, dtype=np.int32)

    def reserve(self, n_new):
        n_dev = n_new if isinstance(n_new, int) else torch.as_tensor(n_new, dtype=torch.int32,
                                                                      device=self.bt.device)
        self.ops.reserve(self.stack, self.top, self.bt, self.lens, n_dev, self.bs, self.status)
        st, self.r_top = ref.reserve(self.r_stack, self.r_top, self.r_bt, self.r_lens, n_new, self.bs)
        return st

    def check_tables(self):
        torch.cuda.synchronize()
        assert int(self.top.item()) == self.r_top
        assert np.array_equal(_np(self.bt), self.r_bt)
        assert np.array_equal(_np(self.lens), self.r_lens)
        assert np.array_equal(_np(self.stack)[: self.r_top], self.r_stack[: self.r_top])


def test_free_stack_init_default_and_permuted(dev) -> None:
    from saint_kv import ops

    for order in (None, np.random.default_rng(5).permutation(1000).astype(np.int32)):
        stack = torch.empty(1000, dtype=torch.int32, device=dev)
        top = torch.empty(1, dtype=torch.int32, device=dev)
        ops.free_stack_init(stack, top, None if order is None else torch.as_tensor(order, device=dev))
        r_stack, r_top = ref.free_stack_init(1000, order)
        assert int(top.item()) == r_top and np.array_equal(_np(stack), r_stack)


def test_reserve_matches_policy_ragged(dev) -> None:
    rng = np.random.default_rng(11)
    s = _State(dev, 37, 4096, 64, 16, (16,), torch.bfloat16, rng.permutation(4096).astype(np.int32))
    for _ in range(20):
        n = rng.integers(0, 50, size=37).astype(np.int32)
        n[rng.integers(0, 37, size=5)] = 0
        assert s.reserve(n) == 0
        assert int(s.status.item()) == 0
        s.check_tables()
    s.reserve(3)  # uniform count path
    s.check_tables()


def test_reserve_refusals_write_nothing(dev) -> None:
    s = _State(dev, 4, 10, 4, 8, (8,), torch.bfloat16)
    assert s.reserve(np.array([8, 8, 8, 8], dtype=np.int32)) == 0
    s.check_tables()
    # 7 more pages needed, 6 free -> NOSPC, nothing changes
    st = s.reserve(np.array([16, 16, 16, 8], dtype=np.int32))
    assert st == ref.STATUS_NOSPC
    torch.cuda.synchronize()
    assert int(s.status.item()) == ref.STATUS_NOSPC
    s.check_tables()
    # a sequence past max_pages (4 pages of 8 = 32 rows) -> MAX_PAGES
    st = s.reserve(np.array([25, 0, 0, 0], dtype=np.int32))
    assert st == ref.STATUS_MAX_PAGES
    torch.cuda.synchronize()
    assert int(s.status.item()) == ref.STATUS_MAX_PAGES
    s.check_tables()


@pytest.mark.parametrize("l0", [(512, 300)])
def test_append_gather_small_kv_config(dev, l0) -> None:
    """B=2, K|V bf16 1x128 each (256 B rows), bs=16, shuffled pages, 32 decode steps."""
    g = torch.Generator().manual_seed(0)
    batch, bs, n_pages, max_pages = 2, 16, 128, 40
    order = np.random.default_rng(0).permutation(n_pages).astype(np.int32)
    s = _State(dev, batch, n_pages, max_pages, bs, (2, 128), torch.bfloat16, order)
    r_pool = torch.zeros(n_pages, bs, 2, 128, dtype=torch.bfloat16)
    # prefill with ragged lengths
    pre = torch.randn(batch, max(l0), 2, 128, generator=g).to(torch.bfloat16)
    n0 = np.array(l0, dtype=np.int32)
    assert s.reserve(n0) == 0
    s.ops.paged_append(s.pool, s.bt, s.lens, pre.to(dev), torch.as_tensor(n0, device=dev))
    ref.paged_append(r_pool, s.r_bt, s.r_lens, pre, n0)
    out = torch.zeros(batch, max(l0) + 32, 2, 128, dtype=torch.bfloat16, device=dev)
    r_out = torch.zeros(batch, max(l0) + 32, 2, 128, dtype=torch.bfloat16)
    for _ in range(32):
        tok = torch.randn(batch, 1, 2, 128, generator=g).to(torch.bfloat16)
        assert s.reserve(1) == 0
        s.ops.append_gather(s.pool, s.bt, s.lens, tok.to(dev), 1, out)
        ref.paged_append(r_pool, s.r_bt, s.r_lens, tok, 1)
        ref.paged_gather(r_pool, s.r_bt, s.r_lens, r_out)
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), r_out)
    s.check_tables()
    assert torch.equal(s.pool.cpu(), r_pool)


def test_gather_into_packed_rows(dev) -> None:
    g = torch.Generator().manual_seed(3)
    rng = np.random.default_rng(3)
    batch, bs, n_pages = 9, 64, 300
    s = _State(dev, batch, n_pages, 32, bs, (576,), torch.bfloat16, rng.permutation(n_pages).astype(np.int32))
    n = rng.integers(0, 1500, size=batch).astype(np.int32)
    n[2] = 0
    src = torch.randn(batch, int(n.max()), 576, generator=g).to(torch.bfloat16)
    assert s.reserve(n) == 0
    s.ops.paged_append(s.pool, s.bt, s.lens, src.to(dev), torch.as_tensor(n, device=dev))
    offs = np.concatenate([[0], np.cumsum(n)[:-1]]).astype(np.int64)
    out = torch.zeros(int(n.sum()), 576, dtype=torch.bfloat16, device=dev)
    s.ops.paged_gather(s.pool, s.bt, s.lens, out, torch.as_tensor(offs, device=dev))
    torch.cuda.synchronize()
    expect = torch.cat([src[b, : n[b]] for b in range(batch)])
    assert torch.equal(out.cpu(), expect)


def test_append_spanning_pages_and_strided_source(dev) -> None:
    """Multi-row appends that cross page boundaries from a non-contiguous source."""
    g = torch.Generator().manual_seed(4)
    batch, bs, n_pages = 5, 8, 200
    s = _State(dev, batch, n_pages, 40, bs, (64,), torch.float32,
               np.random.default_rng(4).permutation(n_pages).astype(np.int32))
    r_pool = torch.zeros(n_pages, bs, 64)
    hist = [[] for _ in range(batch)]
    for step in range(7):
        n = np.array([(3 * step + b) % 19 for b in range(batch)], dtype=np.int32)
        big = torch.randn(batch, 40, 2, 64, generator=g)
        src = big[:, : int(n.max()) or 1, 1]  # strided rows: every other 256-byte block
        assert s.reserve(n) == 0
        s.ops.paged_append(s.pool, s.bt, s.lens, big.to(dev)[:, : src.shape[1], 1],
                           torch.as_tensor(n, device=dev))
        ref.paged_append(r_pool, s.r_bt, s.r_lens, src, n)
        for b in range(batch):
            hist[b].append(src[b, : n[b]])
    s.check_tables()
    assert torch.equal(s.pool.cpu(), r_pool)
    out = torch.zeros(batch, int(s.r_lens.max()), 64, device=dev)
    s.ops.paged_gather(s.pool, s.bt, s.lens, out)
    torch.cuda.synchronize()
    for b in range(batch):
        assert torch.equal(out[b, : s.r_lens[b]].cpu(), torch.cat(hist[b]))


def test_gather_from_page(dev) -> None:
    """paged_gather / append_gather with first_page: rows from page first_page
    on equal the full gather's (oracle), rows before it are left untouched, and
    the appended rows reach the pool as with a full gather.  Ragged lengths,
    one sequence shorter than the first page's first row."""
    g = torch.Generator().manual_seed(5)
    rng = np.random.default_rng(5)
    batch, bs, n_pages, max_pages = 4, 16, 64, 12
    s = _State(dev, batch, n_pages, max_pages, bs, (64,), torch.bfloat16,
               rng.permutation(n_pages).astype(np.int32))
    r_pool = torch.zeros(n_pages, bs, 64, dtype=torch.bfloat16)
    n0 = np.array([70, 33, 100, 40], dtype=np.int32)
    src = torch.randn(batch, int(n0.max()), 64, generator=g).to(torch.bfloat16)
    assert s.reserve(n0) == 0
    s.ops.paged_append(s.pool, s.bt, s.lens, src.to(dev), torch.as_tensor(n0, device=dev))
    ref.paged_append(r_pool, s.r_bt, s.r_lens, src, n0)
    for first_page in (0, 1, 2, 6):
        out = torch.full((batch, max_pages * bs, 64), 7.0, dtype=torch.bfloat16, device=dev)
        s.ops.paged_gather(s.pool, s.bt, s.lens, out, first_page=first_page)
        want = ref.paged_gather(r_pool, s.r_bt, s.r_lens, torch.zeros(batch, max_pages * bs, 64,
                                                                       dtype=torch.bfloat16))
        got = out.cpu()
        lo = first_page * bs
        for b in range(batch):
            L = int(s.r_lens[b])
            assert (got[b, :lo] == 7.0).all(), (first_page, b)
            assert torch.equal(got[b, lo:L], want[b, lo:L]), (first_page, b)
            assert (got[b, max(L, lo):] == 7.0).all(), (first_page, b)
    # append 3 rows and refresh from the page of the first new row
    new = torch.randn(batch, 3, 64, generator=g).to(torch.bfloat16)
    out = torch.zeros(batch, max_pages * bs, 64, dtype=torch.bfloat16, device=dev)
    s.ops.paged_gather(s.pool, s.bt, s.lens, out)
    first_page = int(s.r_lens.min()) // bs
    assert s.reserve(3) == 0
    s.ops.append_gather(s.pool, s.bt, s.lens, new.to(dev), 3, out, first_page=first_page)
    ref.paged_append(r_pool, s.r_bt, s.r_lens, new, 3)
    s.check_tables()
    assert torch.equal(s.pool.cpu(), r_pool)
    want = ref.paged_gather(r_pool, s.r_bt, s.r_lens, torch.zeros(batch, max_pages * bs, 64, dtype=torch.bfloat16))
    got = out.cpu()
    for b in range(batch):
        L = int(s.r_lens[b])
        assert torch.equal(got[b, :L], want[b, :L]), b
    with pytest.raises(ValueError, match="first_page"):
        s.ops.paged_gather(s.pool, s.bt, s.lens, out, first_page=max_pages)


def test_empty_batch_and_zero_lengths(dev) -> None:
    from saint_kv import ops

    s = _State(dev, 3, 16, 4, 4, (8,), torch.float32)
    out = torch.full((3, 4, 8), 7.0, device=dev)
    ops.paged_gather(s.pool, s.bt, s.lens, out)  # all lengths 0: nothing written
    torch.cuda.synchronize()
    assert (out == 7.0).all()
    assert s.reserve(0) == 0
    s.check_tables()
    empty_bt = torch.empty(0, 4, dtype=torch.int32, device=dev)
    empty_lens = torch.empty(0, dtype=torch.int32, device=dev)
    ops.paged_gather(s.pool, empty_bt, empty_lens, torch.empty(0, 4, 8, device=dev))


def test_full_size_decode_gather_config(dev) -> None:
    """B=64, D=576 bf16, L~U[1k,32k], bs=64, pool of 200k pages (random permutation):
    after a one-token decode step (skv_append_gather), then a second through the
    headline path (skv_decode_append_gather: planner + 4 KB slices), the gather
    of every sequence equals what was appended and the tables equal the
    oracle's (size-independent check at full size)."""
    torch.manual_seed(0)
    rng = np.random.default_rng(0)
    from saint_kv import ops

    batch, bs, n_pages, d = 64, 64, 200_000, 576
    lens0 = rng.integers(1024, 32769, size=batch).astype(np.int32)
    max_pages = int((lens0.max() + 1 + bs - 1) // bs)
    s = _State(dev, batch, n_pages, max_pages, bs, (d,), torch.bfloat16,
               rng.permutation(n_pages).astype(np.int32))
    total = int(lens0.sum())
    src = torch.randn(total + batch, d, device=dev, dtype=torch.bfloat16)
    offs = np.concatenate([[0], np.cumsum(lens0)[:-1]]).astype(np.int64)
    assert s.reserve(lens0) == 0
    src_b = torch.zeros(batch, int(lens0.max()), d, dtype=torch.bfloat16, device=dev)
    for b in range(batch):
        src_b[b, : lens0[b]] = src[offs[b]: offs[b] + lens0[b]]
    ops.paged_append(s.pool, s.bt, s.lens, src_b, torch.as_tensor(lens0, device=dev))
    del src_b
    tok = src[total:].view(batch, 1, d)
    assert s.reserve(1) == 0
    out_offs = torch.as_tensor(offs + np.arange(batch), device=dev)
    out = torch.empty(total + batch, d, dtype=torch.bfloat16, device=dev)
    ops.append_gather(s.pool, s.bt, s.lens, tok, 1, out, out_offs)
    torch.cuda.synchronize()
    s.check_tables()
    for b in range(batch):
        o = int(offs[b]) + b
        assert torch.equal(out[o: o + lens0[b]], src[offs[b]: offs[b] + lens0[b]])
        assert torch.equal(out[o + lens0[b]], tok[b, 0])
    del out
    # a second step through the headline path: k_plan_units (reserve + unit
    # table) and k_copy_slices (4 KB slices), at the same full size
    tok2 = torch.randn(batch, 1, d, device=dev, dtype=torch.bfloat16)
    units_n = int((-(-(lens0.astype(np.int64) + 2) // bs)).sum())
    units = ops.unit_table(units_n, dev)
    out_offs2 = torch.as_tensor(offs + 2 * np.arange(batch), device=dev)
    out2 = torch.empty(total + 2 * batch, d, dtype=torch.bfloat16, device=dev)
    ops.decode_append_gather(s.stack, s.top, s.bt, s.lens, s.pool, tok2, 1, out2, units, units_n,
                             out_offs2, s.status)
    st, s.r_top = ref.reserve(s.r_stack, s.r_top, s.r_bt, s.r_lens, 1, bs)
    assert st == 0
    s.check_tables()
    assert int(s.status.item()) == 0
    for b in range(batch):
        o = int(offs[b]) + 2 * b
        assert torch.equal(out2[o: o + lens0[b]], src[offs[b]: offs[b] + lens0[b]])
        assert torch.equal(out2[o + lens0[b]], tok[b, 0])
        assert torch.equal(out2[o + lens0[b] + 1], tok2[b, 0])


def test_decode_append_gather_matches_two_call_path(dev) -> None:
    """skv_decode_append_gather (planner + 4 KB slices) == skv_reserve + skv_append_gather."""
    from saint_kv import ops

    rng = np.random.default_rng(7)
    g = torch.Generator().manual_seed(7)
    batch, bs, n_pages, d = 9, 64, 3000, 576
    order = rng.permutation(n_pages).astype(np.int32)
    a = _State(dev, batch, n_pages, 80, bs, (d,), torch.bfloat16, order)
    b = _State(dev, batch, n_pages, 80, bs, (d,), torch.bfloat16, order)
    lens0 = rng.integers(0, 4000, size=batch).astype(np.int32)
    lens0[3] = 0
    pre = torch.randn(batch, int(lens0.max()), d, generator=g).to(torch.bfloat16).to(dev)
    for s in (a, b):
        s.reserve(lens0)
        s.ops.paged_append(s.pool, s.bt, s.lens, pre, torch.as_tensor(lens0, device=dev))
    cap = lens0.astype(np.int64) + 2 * 20  # up to 2 new tokens per step
    offs = torch.as_tensor(np.concatenate([[0], np.cumsum(cap)[:-1]]), device=dev)
    out_a = torch.zeros(int(cap.sum()), d, dtype=torch.bfloat16, device=dev)
    out_b = torch.zeros_like(out_a)
    units = ops.unit_table(batch * 80, dev)
    lens = lens0.astype(np.int64)
    for step in range(20):
        n = 1 if step % 3 else int(rng.integers(0, 3))
        tok = torch.randn(batch, max(n, 1), d, generator=g).to(torch.bfloat16).to(dev)
        max_units = int((-(-(lens + n) // bs)).sum())
        ops.decode_append_gather(a.stack, a.top, a.bt, a.lens, a.pool, tok, n, out_a, units,
                                 max_units, offs, a.status)
        b.reserve(n)
        ops.append_gather(b.pool, b.bt, b.lens, tok, n, out_b, offs)
        lens += n
        torch.cuda.synchronize()
        assert int(a.status.item()) == 0
        assert torch.equal(a.bt, b.bt) and torch.equal(a.lens, b.lens) and torch.equal(a.top, b.top)
        assert torch.equal(out_a, out_b), step
    assert torch.equal(a.pool, b.pool)
    # a unit table that is too small is refused: nothing changes, nothing copied
    before = (a.bt.clone(), a.lens.clone(), a.top.clone(), out_a.clone())
    ops.decode_append_gather(a.stack, a.top, a.bt, a.lens, a.pool, tok, 1, out_a, units, 3, offs,
                             a.status)
    torch.cuda.synchronize()
    assert int(a.status.item()) == 16  # SKV_STATUS_UNITS
    assert torch.equal(a.bt, before[0]) and torch.equal(a.lens, before[1])
    assert torch.equal(a.top, before[2]) and torch.equal(out_a, before[3])


def test_pipelined_planner_matches_sequential(dev) -> None:
    """The planner of step i+1 on a second stream, into the other of two unit
    tables, overlapping step i's copy (the headline bench loop): every step's
    output, the tables and the pool equal the sequential two-call path."""
    from saint_kv import ops

    rng = np.random.default_rng(8)
    g = torch.Generator().manual_seed(8)
    batch, bs, n_pages, d, steps = 9, 64, 3000, 576, 12
    order = rng.permutation(n_pages).astype(np.int32)
    a = _State(dev, batch, n_pages, 80, bs, (d,), torch.bfloat16, order)
    b = _State(dev, batch, n_pages, 80, bs, (d,), torch.bfloat16, order)
    lens0 = rng.integers(0, 4000, size=batch).astype(np.int32)
    lens0[2] = 63  # crosses a page boundary on the first step
    pre = torch.randn(batch, int(lens0.max()), d, generator=g).to(torch.bfloat16).to(dev)
    for s in (a, b):
        s.reserve(lens0)
        s.ops.paged_append(s.pool, s.bt, s.lens, pre, torch.as_tensor(lens0, device=dev))
    cap = lens0.astype(np.int64) + steps
    offs = torch.as_tensor(np.concatenate([[0], np.cumsum(cap)[:-1]]), device=dev)
    outs_a = [torch.zeros(int(cap.sum()), d, dtype=torch.bfloat16, device=dev) for _ in range(steps)]
    out_b = torch.zeros_like(outs_a[0])
    toks = [torch.randn(batch, 1, d, generator=g).to(torch.bfloat16).to(dev) for _ in range(steps)]
    units = [ops.unit_table(batch * 80, dev) for _ in range(2)]
    ps = torch.cuda.Stream(device=dev)
    plan_done = [torch.cuda.Event() for _ in range(2)]
    copy_done = [torch.cuda.Event() for _ in range(2)]
    main = torch.cuda.current_stream(dev)
    ps.wait_stream(main)
    lens = lens0.astype(np.int64)
    for step in range(steps):
        k = step % 2
        max_units = int((-(-(lens + 1) // bs)).sum())
        ps.wait_event(copy_done[k])  # the copy two steps back has read units[k]
        with torch.cuda.stream(ps):
            ops.plan_units(a.stack, a.top, a.bt, a.lens, 1, bs, outs_a[step], 2 * d, units[k], max_units,
                           offs, a.status)
        plan_done[k].record(ps)
        main.wait_event(plan_done[k])
        ops.copy_slices(a.pool, toks[step], outs_a[step], units[k], max_units)
        copy_done[k].record(main)
        lens += 1
    torch.cuda.synchronize()
    assert int(a.status.item()) == 0
    for step in range(steps):
        b.reserve(1)
        ops.append_gather(b.pool, b.bt, b.lens, toks[step], 1, out_b, offs)
        torch.cuda.synchronize()
        assert torch.equal(outs_a[step], out_b), step
    assert torch.equal(a.bt, b.bt) and torch.equal(a.lens, b.lens) and torch.equal(a.top, b.top)
    assert torch.equal(a.pool, b.pool)
