"""GPU parity of the fused decode step (skv_decode_step) against the oracle.

A stack of CSA (bf16 and fp8, m=4), HCA (m=128) and SWA layers is prefilled
through the kernels, then stepped token by token; after every step the tables,
rings, top-k indices and gathered outputs are compared with the oracle
composition of reserve / ring / pooling / top-k / gather.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


class _Oracle:
    def __init__(self, cache, specs, order_seed):
        self.specs = specs
        self.bs = cache.block_size
        self.m_groups = [g.m for g in cache.groups]
        rng = np.random.default_rng(order_seed)
        self.stack, self.top, self.bt, self.ent = [], [], [], []
        for g in cache.groups:  # same permutation draws as DecodeCache
            st, top = ref.free_stack_init(g.n_pages, rng.permutation(g.n_pages).astype(np.int32))
            self.stack.append(st)
            self.top.append(top)
            self.bt.append(np.full(tuple(g.block_table.shape), -1, dtype=np.int32))
            self.ent.append(np.zeros(cache.batch, dtype=np.int32))
        B, C, CI, W = cache.batch, cache.latent, cache.c_indexer, cache.window
        self.ring = [torch.zeros(B, W, C, dtype=torch.bfloat16) for _ in specs]
        self.pool, self.ipool, self.tails = [], [], []
        self.bound, self.ibound = [], []
        for i, s in enumerate(specs):
            if s.kind == "swa":
                self.pool.append(None)
                self.ipool.append(None)
                self.bound.append(None)
                self.ibound.append(None)
                self.tails.append(None)
                continue
            n_pages = cache.groups[cache.group_of_rate[s.m]].n_pages
            self.pool.append(torch.zeros(n_pages, self.bs, C, dtype=torch.bfloat16))
            self.ipool.append(torch.zeros(n_pages, self.bs, CI, dtype=torch.bfloat16) if s.kind == "csa" else None)
            self.bound.append(torch.zeros(n_pages, self.bs, C, dtype=torch.float32))
            self.ibound.append(torch.zeros(n_pages, self.bs, CI, dtype=torch.float32) if s.kind == "csa" else None)
            self.tails.append([torch.zeros(B, s.m, C, dtype=torch.bfloat16), torch.zeros(B, s.m, C, dtype=torch.bfloat16),
                               torch.zeros(B, s.m, CI, dtype=torch.bfloat16), torch.zeros(B, s.m, CI, dtype=torch.bfloat16)])
        self.lens = np.zeros(B, dtype=np.int32)

    def append(self, n, data, bias, ibias):
        """n new tokens per sequence (data: per layer dict of CPU bf16 [B, T, *])."""
        n = np.asarray(n, dtype=np.int32)
        before = self.lens.copy()
        self.lens = self.lens + n
        for gi, m in enumerate(self.m_groups):
            st, self.top[gi] = ref.reserve(self.stack[gi], self.top[gi], self.bt[gi], self.ent[gi],
                                           self.lens // m - self.ent[gi], self.bs)
            assert st == 0
        for i, s in enumerate(self.specs):
            ref.ring_append(self.ring[i], before, data[i]["kv"], n)
            if s.kind == "swa":
                continue
            gi = self.m_groups.index(s.m)
            t = self.tails[i]
            ref.compress_append(self.pool[i], self.bt[gi], t[0], t[1], data[i]["c"], data[i]["z"],
                                bias[i], self.lens, n, bound_pool=self.bound[i])
            if s.kind == "csa":
                ref.compress_append(self.ipool[i], self.bt[gi], t[2], t[3], data[i]["ci"],
                                    data[i]["zi"], ibias[i], self.lens, n, bound_pool=self.ibound[i])


def _rand_data(g, specs, B, T, C, CI):
    out = []
    for s in specs:
        d = {"kv": torch.randn(B, T, C, generator=g).to(torch.bfloat16)}
        if s.kind != "swa":
            d["c"] = torch.randn(B, T, C, generator=g).to(torch.bfloat16)
            d["z"] = torch.randn(B, T, C, generator=g).to(torch.bfloat16)
        if s.kind == "csa":
            d["ci"] = torch.randn(B, T, CI, generator=g).to(torch.bfloat16)
            d["zi"] = torch.randn(B, T, CI, generator=g).to(torch.bfloat16)
        out.append(d)
    return out


# score_cols: default width, or a wider buffer whose extra columns are NaN
# (the step must read only the first L // m columns of a row); rows wider
# than 16 chunks of 2048 scores span 17 or more histogram chunks
@pytest.mark.parametrize("score_cols", [None, 17412, 40000])
def test_decode_step_matches_oracle(dev, score_cols) -> None:
    from saint_kv.decode import LayerSpec

    _decode_oracle_steps(dev, [LayerSpec("csa", m=4, top_k=64, fp8=True), LayerSpec("csa", m=4, top_k=64),
                               LayerSpec("hca", m=128), LayerSpec("swa")], score_cols)


# a batch that is a multiple of 8: each sequence's blocks of every launch of
# the step run on one XCD
def test_decode_step_matches_oracle_batch_of_8(dev) -> None:
    from saint_kv.decode import LayerSpec

    _decode_oracle_steps(dev, [LayerSpec("csa", m=4, top_k=64, fp8=True), LayerSpec("csa", m=4, top_k=64),
                               LayerSpec("hca", m=128), LayerSpec("swa")], None,
                         lens0=[0, 1, 130, 511, 1300, 64, 900, 2000])


# steps without a CSA layer: no top-k launches, gather launch of dense tiles
# only; the SWA-only stack has no page group at all
@pytest.mark.parametrize("kinds", [("hca-fp8", "swa"), ("swa", "swa"), ("hca",)])
def test_decode_step_without_csa_layers(dev, kinds) -> None:
    from saint_kv.decode import LayerSpec

    specs = [LayerSpec("hca", m=128, fp8=k.endswith("fp8")) if k.startswith("hca") else LayerSpec("swa")
             for k in kinds]
    _decode_oracle_steps(dev, specs, None)


def _decode_oracle_steps(dev, specs, score_cols, lens0=(0, 1, 130, 511, 1300)) -> None:
    from saint_kv.decode import DecodeCache

    B, max_len, bs, W, C, CI = len(lens0), 2048, 16, 32, 576, 128
    seed = 3
    cache = DecodeCache(specs, B, max_len, block_size=bs, window=W, device=dev, page_order_seed=seed,
                        score_cols=score_cols)
    for sc in cache.scores:
        if sc is not None:
            sc.fill_(float("nan"))  # columns past max_len // m must never be read
    orc = _Oracle(cache, specs, seed)
    g = torch.Generator().manual_seed(seed)
    bias = [None if s.kind == "swa" else torch.randn(s.m, C, generator=g) for s in specs]
    ibias = [torch.randn(s.m, CI, generator=g) if s.kind == "csa" else None for s in specs]
    for i, s in enumerate(specs):
        if bias[i] is not None:
            cache.bias[i].copy_(bias[i])
        if ibias[i] is not None:
            cache.idx_bias[i].copy_(ibias[i])
    lens0 = np.array(lens0, dtype=np.int64)
    pre = _rand_data(g, specs, B, int(lens0.max()), C, CI)
    cache.prefill(lens0, data=[{k: v.to(dev) for k, v in d.items()} for d in pre])
    orc.append(lens0, pre, bias, ibias)
    for step in range(40):
        data = _rand_data(g, specs, B, 1, C, CI)
        scores = [torch.randn(B, max_len // s.m, generator=g) if s.kind == "csa" else None for s in specs]
        if scores[0] is not None:
            scores[0][1, :3] = float("nan")
        if step == 5 and len(scores) > 1 and scores[1] is not None:
            scores[1][:, :] = 0.0  # ties everywhere
        for i, s in enumerate(specs):
            for k, v in data[i].items():
                cache.inputs[i][k].copy_(v[:, 0])
            if scores[i] is not None:
                cache.scores[i][:, :scores[i].shape[1]].copy_(scores[i])
        cache.step()
        orc.append(np.ones(B, dtype=np.int32), data, bias, ibias)
        torch.cuda.synchronize()
        cache.check_status()
        assert np.array_equal(_np(cache.tok_lens), orc.lens)
        for gi, grp in enumerate(cache.groups):
            assert np.array_equal(_np(grp.block_table), orc.bt[gi])
            assert np.array_equal(_np(grp.n_entries), orc.ent[gi])
            assert int(grp.free_top.item()) == orc.top[gi]
        for i, s in enumerate(specs):
            assert torch.equal(cache.ring[i].cpu(), orc.ring[i]), (step, i)
            win = ref.ring_read(orc.ring[i], orc.lens, torch.zeros(B, W, C, dtype=torch.bfloat16))
            ow = cache.out_window[i].cpu()
            for b in range(B):
                n = min(W, int(orc.lens[b]))
                assert torch.equal(ow[b, :n], win[b, :n]), (step, i, b)
            if s.kind == "swa":
                continue
            gi = cache.group_of_rate[s.m]
            gpu_pool = cache.pool[i].cpu()
            src = ref.fp8_unpack_entries(gpu_pool.reshape(-1, 656)).reshape(*gpu_pool.shape[:2], C) \
                if s.fp8 else gpu_pool
            if s.kind == "csa":
                q = orc.lens - 1
                n_valid = np.array([ref.n_valid_blocks(int(x), s.m) for x in q])
                idx = _np(cache.topk_idx[i])
                for b in range(B):
                    n_cols = int(orc.lens[b]) // s.m
                    exp = ref.topk_select(scores[i][b:b + 1].numpy(), n_valid[b:b + 1], s.top_k, n_cols)[0]
                    assert np.array_equal(idx[b, : len(exp)], exp), (step, i, b)
                    assert (idx[b, len(exp):] == -1).all()
                out = cache.out_entries[i].cpu()
                exp_out = torch.zeros_like(out)
                ref.topk_gather(src, orc.bt[gi], np.arange(B), idx, exp_out)
                for b in range(B):
                    if orc.ent[gi][b] == 0:
                        exp_out[b] = 0
                assert torch.equal(out, exp_out), (step, i)
            else:
                out = cache.out_entries[i].cpu()
                dense = ref.paged_gather(src, orc.bt[gi], orc.ent[gi], torch.zeros_like(out))
                for b in range(B):
                    e = int(orc.ent[gi][b])
                    assert torch.equal(out[b, :e], dense[b, :e]), (step, i, b)
    # pooled values: GPU entries within the pooling tolerance of the oracle's,
    # and the fp8 layer's codes equal the quantization of the bf16 layer's
    # entries (same inputs, same block table)
    torch.cuda.synchronize()
    for i, s in enumerate(specs):
        if s.kind == "swa" or s.fp8:
            continue
        gi = cache.group_of_rate[s.m]
        live = ref.live_pages(orc.bt[gi], orc.ent[gi], bs)
        for b in range(B):
            e = int(orc.ent[gi][b])
            got = ref.paged_gather(cache.pool[i].cpu(), orc.bt[gi][b:b + 1], orc.ent[gi][b:b + 1],
                                   torch.zeros(1, max(e, 1), C, dtype=torch.bfloat16))
            exp = ref.paged_gather(orc.pool[i], orc.bt[gi][b:b + 1], orc.ent[gi][b:b + 1],
                                   torch.zeros(1, max(e, 1), C, dtype=torch.bfloat16))
            bound = ref.paged_gather(orc.bound[i], orc.bt[gi][b:b + 1], orc.ent[gi][b:b + 1],
                                     torch.zeros(1, max(e, 1), C, dtype=torch.float32))
            assert ((got.float() - exp.float()).abs() <= bound).all(), (i, b)
        if s.kind == "csa":
            gi_pool = cache.idx_pool[i].cpu()
            err = (gi_pool[live].float() - orc.ipool[i][live].float()).abs()
            assert (err <= orc.ibound[i][live]).all(), i
        del live
    # layers 0 (fp8) and 1 (bf16) saw the same data? no: inputs differ per layer,
    # so fp8 exactness is covered by test_compress_ragged_chunks_fp8.


def test_decode_release_and_compact(dev) -> None:
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=32, fp8=True), LayerSpec("hca", m=128)]
    B, max_len = 8, 8192
    cache = DecodeCache(specs, B, max_len, block_size=16, window=16, device=dev, page_order_seed=9)
    gen = torch.Generator(device=dev).manual_seed(9)
    lens0 = np.random.default_rng(9).integers(100, 6000, size=B)
    cache.prefill(lens0, generator=gen)
    for i, s in enumerate(specs):
        for v in cache.inputs[i].values():
            v.normal_(generator=gen)
        if cache.scores[i] is not None:
            cache.scores[i].normal_(generator=gen)
    for _ in range(3):
        cache.step()
    cache.check_status()
    # dense view of every live sequence before
    csa_g = cache.groups[cache.group_of_rate[4]]
    before = []
    for b in range(B):
        e = int(csa_g.n_entries[b])
        out = torch.zeros(1, e, 576, dtype=torch.bfloat16, device=dev)
        idx = torch.arange(e, dtype=torch.int32, device=dev).view(1, e)
        from saint_kv import ops
        ops.topk_gather(cache.pool[0], csa_g.block_table[b:b + 1], csa_g.n_entries[b:b + 1], idx, out, 576)
        before.append(out)
    mask = np.zeros(B, dtype=bool)
    mask[[1, 4, 6]] = True
    cache.release(mask)
    with pytest.raises(RuntimeError, match="double free"):
        cache.release(mask)
    info = cache.compact()
    torch.cuda.synchronize()
    for gi, g in enumerate(cache.groups):
        n_live, moved = info[gi]
        bt = _np(g.block_table)
        ent = _np(g.n_entries)
        live = ref.live_pages(bt, ent, 16)
        assert sorted(live.tolist()) == list(range(n_live))
        assert int(g.free_top.item()) == g.n_pages - n_live
    from saint_kv import ops
    for b in range(B):
        if mask[b]:
            continue
        e = int(csa_g.n_entries[b])
        out = torch.zeros(1, e, 576, dtype=torch.bfloat16, device=dev)
        idx = torch.arange(e, dtype=torch.int32, device=dev).view(1, e)
        ops.topk_gather(cache.pool[0], csa_g.block_table[b:b + 1], csa_g.n_entries[b:b + 1], idx, out, 576)
        assert torch.equal(out, before[b])
    cache.step()  # decode continues after compaction
    cache.check_status()


def _check_csa_outputs(cache, i, scores, ctx):
    """topk_idx and out_entries of CSA layer i against the oracle select and
    gather over the cache's own pool and block table."""
    s = cache.layers[i]
    g = cache.groups[cache.group_of_rate[s.m]]
    lens = _np(cache.tok_lens).astype(np.int64)
    bt, ent = _np(g.block_table), _np(g.n_entries)
    idx = _np(cache.topk_idx[i])
    exp_idx = np.full_like(idx, -1)
    for b in range(cache.batch):
        n_cols = int(lens[b]) // s.m
        nv = np.array([ref.n_valid_blocks(int(lens[b]) - 1, s.m)])
        e = ref.topk_select(scores[b:b + 1].numpy(), nv, s.top_k, n_cols)[0]
        exp_idx[b, :len(e)] = e
    assert np.array_equal(idx, exp_idx), ctx
    pool = cache.pool[i].cpu()
    src = ref.fp8_unpack_entries(pool.reshape(-1, pool.shape[-1])).reshape(*pool.shape[:2], -1) \
        if s.fp8 else pool
    exp_out = torch.zeros(cache.batch, s.top_k, cache.latent, dtype=torch.bfloat16)
    ref.topk_gather(src, bt, np.arange(cache.batch), exp_idx, exp_out)
    exp_out[ent == 0] = 0
    assert torch.equal(cache.out_entries[i].cpu(), exp_out), ctx


def test_decode_compactions_with_groups_of_growing_size(dev) -> None:
    """Two page groups, the first compacted (m=4) smaller than the second
    (m=128, given a larger pool), and two release + compaction rounds: each
    group compacts in its own slice of the workspace, so the larger group never
    reads the smaller one's scratch as marks or block counts.  Tables, free
    stacks and entries equal the oracle's replay of release / compact on the
    same tables."""
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("hca", m=128), LayerSpec("csa", m=4, top_k=16)]
    B, max_len, bs = 6, 8192, 16
    cache = DecodeCache(specs, B, max_len, block_size=bs, window=16, device=dev, page_order_seed=4,
                        pages_per_group={128: 2000})
    assert cache.groups[0].n_pages < cache.groups[1].n_pages
    pool_of = {cache.group_of_rate[sp.m]: cache.pool[i] for i, sp in enumerate(specs)}
    gen = torch.Generator(device=dev).manual_seed(4)
    rng = np.random.default_rng(4)
    cache.prefill(rng.integers(500, 8000, size=B), generator=gen)
    views = {}

    def entries(g, b):
        e = int(g.n_entries[b])
        return ref.paged_gather(pool_of[cache.groups.index(g)].cpu(), _np(g.block_table)[b:b + 1],
                                _np(g.n_entries)[b:b + 1], torch.zeros(1, max(e, 1), 576, dtype=torch.bfloat16))[0, :e]

    for rnd, fin in enumerate(([0, 3], [2])):
        mask = np.zeros(B, dtype=bool)
        mask[fin] = True
        r_tabs = []
        for g in cache.groups:
            r_bt, r_ent = _np(g.block_table).copy(), _np(g.n_entries).copy()
            r_stack, r_top = _np(g.free_stack).copy(), int(g.free_top.item())
            st, r_top = ref.release(r_stack, r_top, r_bt, r_ent, mask.astype(np.uint8), bs)
            assert st == 0
            r_tabs.append((r_bt, r_ent))
        for b in range(B):
            if not mask[b] and cache.host_lens[b]:
                views[b] = [entries(g, b) for g in cache.groups]
        cache.release(mask)
        info = cache.compact()
        for gi, g in enumerate(cache.groups):
            r_bt, r_ent = r_tabs[gi]
            pools = [torch.zeros(g.n_pages, 1, 1, dtype=torch.uint8)]
            r_stack2, r_top2, moved = ref.compact(pools, r_bt, r_ent, bs)
            assert info[gi][1] == moved, (rnd, gi)
            assert np.array_equal(_np(g.block_table), r_bt), (rnd, gi)
            assert int(g.free_top.item()) == r_top2
            assert np.array_equal(_np(g.free_stack)[:r_top2], r_stack2[:r_top2])
        for b, vs in views.items():
            if mask[b] or not cache.host_lens[b]:
                continue
            for g, v in zip(cache.groups, vs):
                assert torch.equal(entries(g, b), v), (rnd, b)
        off = 0
        for g in cache.groups:  # the marks of every group's slice are zero again
            assert not _np(cache._compact_ws[off: off + g.n_pages]).any()
            off += 3 * g.n_pages
        views = {}
        cache.step()
        cache.check_status()


def test_decode_scores_from_cached_indexer_keys(dev) -> None:
    """The indexer scores of each step computed on the GPU from the cache's own
    paged indexer keys (ops.indexer_scores) match the oracle, and the step
    selects and gathers on exactly those scores (csa.py:403-422 end to end,
    after the projections)."""
    from saint_kv import ops
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=32)]
    B, H = 3, 64
    cache = DecodeCache(specs, B, 4096, block_size=16, window=16, device=dev, page_order_seed=7)
    gen = torch.Generator(device=dev).manual_seed(7)
    for v in cache.inputs[0].values():
        v.normal_(generator=gen)
    cache.bias[0].normal_(generator=gen)
    cache.idx_bias[0].normal_(generator=gen)
    cache.prefill(np.array([1000, 37, 2900]), generator=gen)
    grp = cache.groups[cache.group_of_rate[4]]
    g = torch.Generator().manual_seed(7)
    for step in range(6):
        for v in cache.inputs[0].values():
            v.normal_(generator=gen)
        q = torch.randn(B, 1, H, cache.c_indexer, generator=g).to(torch.bfloat16)
        w = torch.randn(B, 1, H, generator=g)
        cache.scores[0].fill_(float("nan"))
        ops.indexer_scores(q.to(dev), w.to(dev), cache.idx_pool[0], grp.block_table, grp.n_entries,
                           cache.scores[0].view(B, 1, -1))
        torch.cuda.synchronize()
        got = cache.scores[0].cpu()
        ent, bt = _np(grp.n_entries), _np(grp.block_table)
        ipool = cache.idx_pool[0].float().cpu().numpy()
        for b in range(B):
            n = int(ent[b])
            keys = np.stack([ipool[bt[b, e // 16], e % 16] for e in range(n)])[None]
            qn, wn = q[b:b + 1].float().numpy(), w[b:b + 1].numpy()
            exp = ref.indexer_scores(qn, keys, wn)[0, 0]
            bound = ref.indexer_scores_bound(qn, keys, wn)[0, 0]
            assert (np.abs(got[b, :n].numpy() - exp) <= 1e-5 * bound + 1e-30).all(), (step, b)
        cache.step()
        torch.cuda.synchronize()
        cache.check_status()
        _check_csa_outputs(cache, 0, got.nan_to_num(nan=float("-inf")), step)


@pytest.mark.parametrize("max_len", [20480, 70000])
def test_decode_topk_rank_cases(dev, max_len) -> None:
    """Sparse selection of the decode step over score patterns that exercise
    every path of the rank step: sure and tie candidates, exact duplicates,
    sel < top_k fills across several parts, an empty row, non-finite scores,
    candidate lists longer than the launch's LDS holds (ranked from global
    memory) and tie bins over the list capacity (the full-select fallback),
    at score rows of 5120 and 17500 columns."""
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=300), LayerSpec("csa", m=4, top_k=50, fp8=True)]
    B = 4
    cache = DecodeCache(specs, B, max_len, block_size=64, window=16, device=dev, page_order_seed=5)
    gen = torch.Generator(device=dev).manual_seed(5)
    cache.prefill(np.array([2, 900, 17000, max_len - 480]), generator=gen)
    g = torch.Generator().manual_seed(5)
    patterns = ["normal", "const", "dup", "sparse", "nonfinite", "const_neg", "wide", "normal"]
    for step, pat in enumerate(patterns):
        for i in range(len(specs)):
            for v in cache.inputs[i].values():
                v.normal_(generator=gen)
        scores = []
        for s in specs:
            shape = (B, max_len // s.m)
            if pat == "normal":
                sc = torch.randn(*shape, generator=g)
            elif pat == "const":
                sc = torch.full(shape, 0.5)  # one tie bin holding every score
            elif pat == "const_neg":
                sc = torch.full(shape, -3.0)
                sc[:, ::97] = 1.0
            elif pat == "dup":
                sc = torch.randint(0, 8, shape, generator=g).float()
            elif pat == "sparse":
                sc = torch.relu(torch.randn(*shape, generator=g) - 1.3)
            elif pat == "wide":  # 250 sure keys over one tie bin of 3900
                sc = torch.full(shape, -1.0)
                sc[:, :3900] = 0.5 + 0.1 * torch.rand(B, 3900, generator=g)
                sc[:, 3900:4150] = 10.0 + torch.rand(B, 250, generator=g)
            else:
                sc = torch.randn(*shape, generator=g)
                sc[:, 5:40:3] = float("nan")
                sc[:, 7:60:5] = float("inf")
                sc[:, 9:90:4] = float("-inf")
                sc[2, :] = float("-inf")
            scores.append(sc)
            cache.scores[len(scores) - 1][:, :sc.shape[1]].copy_(sc)
        cache.step()
        torch.cuda.synchronize()
        cache.check_status()
        for i in range(len(specs)):
            _check_csa_outputs(cache, i, scores[i], (step, pat, i))


def test_decode_refused_step_changes_nothing(dev) -> None:
    """A step whose page reservation is refused (pool exhausted) sets the
    status bit and leaves every buffer of the cache as it was."""
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=8), LayerSpec("hca", m=128), LayerSpec("swa")]
    B, bs = 2, 16
    cache = DecodeCache(specs, B, 1024, block_size=bs, window=8, device=dev, page_order_seed=1,
                        pages_per_group={4: 2})
    gen = torch.Generator(device=dev).manual_seed(1)
    cache.prefill(np.array([64, 10]), generator=gen)  # 16 + 2 CSA entries: both pages taken

    def fill():
        for i in range(len(specs)):
            for v in cache.inputs[i].values():
                v.normal_(generator=gen)
            if cache.scores[i] is not None:
                cache.scores[i].normal_(generator=gen)

    for _ in range(3):  # lens 65..67: still 16 entries in one page
        fill()
        cache.step()
    cache.check_status()

    def snapshot():
        bufs = [cache.tok_lens]
        for grp in cache.groups:
            bufs += [grp.block_table, grp.n_entries, grp.free_top, grp.free_stack]
        # (topk_ws is scratch: the step leaves its histogram and counters ready
        # for the next step, whatever they held before)
        for lst in (cache.ring, cache.pool, cache.state, cache.idx_pool, cache.idx_state,
                    cache.topk_idx, cache.out_entries, cache.out_window):
            bufs += [t for t in lst if t is not None]
        return [t.clone() for t in bufs]

    fill()
    torch.cuda.synchronize()
    before = snapshot()
    cache.step()  # length 68 of sequence 0 needs a 17th entry, i.e. a second page
    torch.cuda.synchronize()
    assert int(cache.status.item()) == 2  # SKV_STATUS_NOSPC
    after = snapshot()
    for j, (x, y) in enumerate(zip(before, after)):
        assert torch.equal(x, y), j
    with pytest.raises(RuntimeError, match="refused"):
        cache.check_status()
    assert cache.host_lens.tolist() == [67, 13]
    # a sequence that needs no page can still step once the other one finishes
    cache.release(np.array([True, False]))
    fill()
    cache.step()
    cache.check_status()
    assert cache.tok_lens.tolist() == [1, 14]


# the step computes its own scores (LayerSpec.idx_heads): the scores it writes
# equal skv_indexer_scores over the entries before the step, bit for bit, and
# its top-k and gathered entries equal the oracle's on those scores; a batch
# of 8 places every sequence's blocks on one XCD, a batch of 5 spreads them
@pytest.mark.parametrize("lens0", [[0, 3, 4, 2051, 3000], [0, 3, 4, 2051, 3000, 17, 1024, 4000]])
def test_decode_step_computes_scores(dev, lens0) -> None:
    from saint_kv import ops
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=64, idx_heads=64), LayerSpec("hca", m=128),
             LayerSpec("csa", m=4, top_k=24, fp8=True, idx_heads=20)]
    B, max_len, bs, C = len(lens0), 4096, 16, 576
    cache = DecodeCache(specs, B, max_len, block_size=bs, window=32, device=dev, page_order_seed=7)
    gen = torch.Generator(device=dev).manual_seed(7)
    for i in range(len(specs)):
        for t in (cache.bias[i], cache.idx_bias[i]):
            if t is not None:
                t.normal_(generator=gen)
    cache.prefill(np.array(lens0), generator=gen)
    for step in range(9):
        for i in range(len(specs)):
            for v in cache.inputs[i].values():
                v.normal_(generator=gen)
        if step == 4:
            cache.inputs[0]["iw"].zero_()  # every score 0: one tie bin
        exp = [None] * len(specs)
        for i, s in enumerate(specs):
            if s.kind == "csa":
                g = cache.groups[cache.group_of_rate[s.m]]
                exp[i] = torch.full_like(cache.scores[i], float("nan"))
                ops.indexer_scores(cache.inputs[i]["iq"].unsqueeze(1), cache.inputs[i]["iw"].unsqueeze(1),
                                   cache.idx_pool[i], g.block_table, g.n_entries, exp[i].unsqueeze(1))
        before = cache.host_lens.copy()
        cache.step()
        torch.cuda.synchronize()
        cache.check_status()
        for i, s in enumerate(specs):
            if exp[i] is None:
                continue
            gi = cache.group_of_rate[s.m]
            got, want = cache.scores[i].cpu(), exp[i].cpu()
            idx = _np(cache.topk_idx[i])
            for b in range(B):
                n = int(before[b]) // s.m
                assert ref.n_valid_blocks(int(before[b]), s.m) == n
                assert torch.equal(got[b, :n], want[b, :n]), (step, i, b)
                sel = ref.topk_select(want[b:b + 1].numpy(), np.array([n]), s.top_k, (int(before[b]) + 1) // s.m)[0]
                assert np.array_equal(idx[b, :len(sel)], sel), (step, i, b)
                assert (idx[b, len(sel):] == -1).all(), (step, i, b)
            pool = cache.pool[i].cpu()
            src = ref.fp8_unpack_entries(pool.reshape(-1, 656)).reshape(*pool.shape[:2], C) if s.fp8 else pool
            out = cache.out_entries[i].cpu()
            exp_out = torch.zeros_like(out)
            ref.topk_gather(src, _np(cache.groups[gi].block_table), np.arange(B), idx, exp_out)
            ent = _np(cache.groups[gi].n_entries)
            for b in range(B):
                if ent[b] == 0:
                    exp_out[b] = 0
            assert torch.equal(out, exp_out), (step, i)


def test_decode_step_scores_all_or_none(dev) -> None:
    from saint_kv.decode import DecodeCache, LayerSpec

    with pytest.raises(ValueError, match="every CSA layer"):
        DecodeCache([LayerSpec("csa", idx_heads=8), LayerSpec("csa")], 2, 256, device=dev)
    with pytest.raises(ValueError, match="indexer stream"):
        DecodeCache([LayerSpec("csa", indexer=False, idx_heads=8)], 2, 256, device=dev)


# the same steps two ways, replayed from HIP graphs three times with eager
# input fills between the replays: scores computed in the step (idx_heads)
# and a caller's skv_indexer_scores launch recorded before each step
# (capture's before_step); every table, score, pick and gathered row agrees
def test_step_scores_fused_equals_separate_launch_in_graphs(dev) -> None:
    from saint_kv import ops
    from saint_kv.decode import DecodeCache, LayerSpec

    B, IH, lens0 = 3, 16, np.array([5, 700, 1999])

    def make(fused):
        specs = [LayerSpec("csa", m=4, top_k=32, idx_heads=IH if fused else 0), LayerSpec("hca", m=16)]
        c = DecodeCache(specs, B, 4096, block_size=16, window=32, device=dev, page_order_seed=9)
        gen = torch.Generator(device=dev).manual_seed(9)
        for i in range(len(specs)):
            for t in (c.bias[i], c.idx_bias[i]):
                if t is not None:
                    t.normal_(generator=gen)
        c.prefill(lens0, generator=gen)
        return c

    fused, sep = make(True), make(False)
    iq = torch.empty(B, 1, IH, 128, dtype=torch.bfloat16, device=dev)
    iw = torch.empty(B, 1, IH, dtype=torch.float32, device=dev)
    g0 = sep.groups[sep.group_of_rate[4]]

    def scores_launch():
        ops.indexer_scores(iq, iw, sep.idx_pool[0], g0.block_table, g0.n_entries, sep.scores[0].unsqueeze(1))

    graph_f, graph_s = fused.capture(2), sep.capture(2, scores_launch)
    gen = torch.Generator(device=dev).manual_seed(10)
    for rep in range(3):
        for i in range(2):
            for k, v in fused.inputs[i].items():
                v.normal_(generator=gen)
                if k == "iq":
                    iq.copy_(v.unsqueeze(1))
                elif k == "iw":
                    iw.copy_(v.unsqueeze(1))
                else:
                    sep.inputs[i][k].copy_(v)
        torch.cuda.synchronize()
        graph_f.replay()
        graph_s.replay()
        torch.cuda.synchronize()
        fused.check_status()
        sep.check_status()
        assert torch.equal(fused.tok_lens, sep.tok_lens)
        for a, b in zip(fused.groups, sep.groups):
            assert torch.equal(a.block_table, b.block_table) and torch.equal(a.n_entries, b.n_entries)
        for b in range(B):
            n = int(sep.host_lens[b] - 1) // 4
            assert torch.equal(fused.scores[0][b, :n], sep.scores[0][b, :n]), (rep, b)
        for i in range(2):
            assert torch.equal(fused.out_entries[i], sep.out_entries[i]), (rep, i)
            assert torch.equal(fused.out_window[i], sep.out_window[i]), (rep, i)
            assert torch.equal(fused.pool[i], sep.pool[i]), (rep, i)
        assert torch.equal(fused.topk_idx[0], sep.topk_idx[0]), rep


def test_step_without_copies_equals_materialized_step(dev) -> None:
    """DecodeCache(materialize=False): the step skips the gathered copies
    (CSA picks' entries, HCA entries, windows) and writes everything else
    exactly as the materializing step does: indices, pools, states, rings,
    tables, lengths; the attention over either cache gives the same output."""
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=64, fp8=True), LayerSpec("hca", m=128), LayerSpec("csa", m=4, top_k=48),
             LayerSpec("swa")]
    B, max_len = 6, 4096
    caches = [DecodeCache(specs, B, max_len, block_size=16, window=32, device=dev, page_order_seed=4,
                          materialize=mat) for mat in (True, False)]
    assert caches[1].out_window[0] is None and caches[1].out_entries[0] is None
    lens0 = np.array([0, 3, 127, 500, 1300, 2047])
    for c in caches:
        for i in range(len(specs)):
            g0 = torch.Generator(device=dev).manual_seed(40 + i)
            if c.bias[i] is not None:
                c.bias[i].normal_(generator=g0)
            if c.idx_bias[i] is not None:
                c.idx_bias[i].normal_(generator=g0)
        c.prefill(lens0, generator=torch.Generator(device=dev).manual_seed(41))
    g = torch.Generator().manual_seed(42)
    q = torch.randn(B, 16, 576, generator=g).to(torch.bfloat16).to(dev)
    knorm = torch.rand(576, generator=g).to(dev) + 0.5
    for step in range(10):
        for i in range(len(specs)):
            vals = {k: torch.randn(v.shape, generator=g).to(v.dtype) for k, v in caches[0].inputs[i].items()}
            sc = torch.randn(caches[0].scores[i].shape, generator=g) if caches[0].scores[i] is not None else None
            for c in caches:
                for k, v in vals.items():
                    c.inputs[i][k].copy_(v)
                if sc is not None:
                    c.scores[i].copy_(sc)
        for c in caches:
            c.step()
        torch.cuda.synchronize()
        for c in caches:
            c.check_status()
        a, b = caches
        assert torch.equal(a.tok_lens, b.tok_lens)
        for ga, gb in zip(a.groups, b.groups):
            assert torch.equal(ga.block_table, gb.block_table) and torch.equal(ga.n_entries, gb.n_entries)
            assert torch.equal(ga.free_top, gb.free_top)
        for i, s in enumerate(specs):
            assert torch.equal(a.ring[i], b.ring[i])
            if s.kind == "swa":
                continue
            assert torch.equal(a.pool[i], b.pool[i]) and torch.equal(a.state[i], b.state[i])
            if s.kind == "csa":
                assert torch.equal(a.topk_idx[i], b.topk_idx[i]), (step, i)
                assert torch.equal(a.idx_pool[i], b.idx_pool[i])
    for i, s in enumerate(specs):
        kw = {} if s.kind == "swa" else {"knorm_w": knorm}
        oa = caches[0].attention(i, q, **kw)
        ob = caches[1].attention(i, q, **kw)
        torch.cuda.synchronize()
        assert torch.equal(oa, ob), i
