"""Full-size parity of the fused decode step (skv_decode_step) at the workload
configurations, against the oracle.

The caches are prefilled synthetically on the GPU (N(0,1) entries and ring
rows; fp8 pools quantize N(0,1) rows with 1% x20 outliers), because an oracle
prefill of 64k-1M tokens per sequence would not finish in seconds.  What the
step reads and writes is then checked exactly:

* block tables, entry counts, free-stack tops and the free stacks: the oracle's
  reserve / release / compact replayed from the same page permutation;
* SWA rings and the window copies: the GPU ring read back once after the
  prefill, then advanced by the oracle's ring_append, and ring_read;
* top-k indices: the oracle's topk_select on the step's scores (bit-exact);
* gathered CSA picks and dense HCA rows: the closed form "row (b, e) is pool
  row block_table[b, e // bs] * bs + e % bs" evaluated with torch indexing on
  the GPU pool (fp8 rows dequantized by the oracle), bit-exact;
* emitted entries: the oracle's compress_pool of the block's tokens (the
  incomplete blocks of the prefill are folded from known tail tokens), within
  1e-2 relative plus a cancellation term (pooling_bound), fp8 within the
  e4m3 rounding on top.

Configurations: one CSA layer at B=16, L=65,536, m=4, top-k 512, W=128;
eight layers alternating CSA (m=4, top-k 512) and HCA (m=128), B=32,
L~U[32k,128k], W=128; one FP8 CSA layer, B=4, L~U[256k,1M], top-k 1024,
W=128, then 30% of the sequences released and the pool compacted.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

C, CI, W, BS = 576, 128, 128, 64


def _np(t):
    return t.detach().cpu().numpy()


class _Streams:
    """Tokens of the incomplete block of every (layer, stream, sequence)."""

    def __init__(self, B, m, ch, tail_c, tail_z, lens0):
        self.m = m
        self.c = torch.zeros(B, m, ch, dtype=torch.bfloat16)
        self.z = torch.zeros(B, m, ch, dtype=torch.bfloat16)
        for b in range(B):
            t = int(lens0[b]) % m
            self.c[b, :t] = tail_c[b, :t]
            self.z[b, :t] = tail_z[b, :t]

    def push(self, pos: np.ndarray, c, z) -> list[int]:
        """Token at position pos[b] of every sequence; returns the sequences
        whose block it completes."""
        done = []
        for b in range(len(pos)):
            slot = int(pos[b]) % self.m
            self.c[b, slot] = c[b]
            self.z[b, slot] = z[b]
            if slot == self.m - 1:
                done.append(b)
        return done


def _rows(bt: np.ndarray, b: int, e: np.ndarray) -> np.ndarray:
    """Pool rows (flat page * bs + slot) of entries e of sequence b."""
    e = np.maximum(np.asarray(e, np.int64), 0)
    return bt[b, e // BS].astype(np.int64) * BS + e % BS


def _pool_rows(pool: torch.Tensor, rows: np.ndarray, fp8: bool) -> torch.Tensor:
    flat = pool.view(pool.shape[0] * pool.shape[1], -1)
    got = flat.index_select(0, torch.as_tensor(rows, device=pool.device)).cpu()
    return ref.fp8_unpack_entries(got) if fp8 else got


class _Run:
    def __init__(self, dev, specs, lens0, steps, seed, outlier_frac=0.0):
        from saint_kv.decode import DecodeCache

        self.dev, self.specs = dev, specs
        self.B = B = len(lens0)
        self.lens = np.asarray(lens0, np.int64).copy()
        max_len = int(self.lens.max()) + steps + 8
        self.cache = cache = DecodeCache(specs, B, max_len, window=W, block_size=BS, device=dev,
                                         page_order_seed=seed)
        self.g = g = torch.Generator().manual_seed(seed)
        self.bias, self.ibias, tails = [], [], []
        for i, s in enumerate(specs):
            if s.kind == "swa":
                self.bias.append(None)
                self.ibias.append(None)
                tails.append(None)
                continue
            self.bias.append(torch.randn(s.m, C, generator=g))
            cache.bias[i].copy_(self.bias[i])
            t = {"c": torch.randn(B, s.m, C, generator=g).to(torch.bfloat16),
                 "z": torch.randn(B, s.m, C, generator=g).to(torch.bfloat16)}
            if s.kind == "csa":
                self.ibias.append(torch.randn(s.m, CI, generator=g))
                cache.idx_bias[i].copy_(self.ibias[i])
                t["ci"] = torch.randn(B, s.m, CI, generator=g).to(torch.bfloat16)
                t["zi"] = torch.randn(B, s.m, CI, generator=g).to(torch.bfloat16)
            else:
                self.ibias.append(None)
            tails.append(t)
        gen = torch.Generator(device=dev).manual_seed(seed)
        cache.prefill(self.lens, generator=gen, outlier_frac=outlier_frac,
                      tails=[None if t is None else {k: v.to(dev) for k, v in t.items()} for t in tails])
        # oracle tables: the same permutation draws as DecodeCache, the prefill's reserve
        rng = np.random.default_rng(seed)
        self.stack, self.top, self.bt, self.ent = [], [], [], []
        for grp in cache.groups:
            st, top = ref.free_stack_init(grp.n_pages, rng.permutation(grp.n_pages).astype(np.int32))
            bt = np.full(tuple(grp.block_table.shape), -1, dtype=np.int32)
            ent = np.zeros(B, dtype=np.int32)
            status, top = ref.reserve(st, top, bt, ent, self.lens // grp.m, BS)
            assert status == 0
            self.stack.append(st)
            self.top.append(top)
            self.bt.append(bt)
            self.ent.append(ent)
        self.check_tables()
        self.ring = [r.cpu() for r in cache.ring]
        self.blocks = []
        for i, s in enumerate(specs):
            if s.kind == "swa":
                self.blocks.append(None)
                continue
            st = [_Streams(B, s.m, C, tails[i]["c"], tails[i]["z"], self.lens)]
            if s.kind == "csa":
                st.append(_Streams(B, s.m, CI, tails[i]["ci"], tails[i]["zi"], self.lens))
            self.blocks.append(st)

    def check_tables(self):
        torch.cuda.synchronize()
        for gi, grp in enumerate(self.cache.groups):
            assert np.array_equal(_np(grp.block_table), self.bt[gi])
            assert np.array_equal(_np(grp.n_entries), self.ent[gi])
            top = int(grp.free_top.item())
            assert top == self.top[gi]
            assert np.array_equal(_np(grp.free_stack[:top]), self.stack[gi][:top])
        assert np.array_equal(_np(self.cache.tok_lens), self.lens)

    def step(self, step: int) -> None:
        cache, B, g = self.cache, self.B, self.g
        data, scores = [], []
        for i, s in enumerate(self.specs):
            d = {"kv": torch.randn(B, C, generator=g).to(torch.bfloat16)}
            if s.kind != "swa":
                d["c"] = torch.randn(B, C, generator=g).to(torch.bfloat16)
                d["z"] = torch.randn(B, C, generator=g).to(torch.bfloat16)
            if s.kind == "csa":
                d["ci"] = torch.randn(B, CI, generator=g).to(torch.bfloat16)
                d["zi"] = torch.randn(B, CI, generator=g).to(torch.bfloat16)
            for k, v in d.items():
                cache.inputs[i][k].copy_(v)
            sc = None
            if s.kind == "csa":
                sc = torch.randn(B, cache.scores[i].shape[1], generator=g)
                cache.scores[i].copy_(sc)
            data.append(d)
            scores.append(sc)
        cache.step()
        torch.cuda.synchronize()
        cache.check_status()
        pos = self.lens.copy()  # position of the new token
        self.lens += 1
        for gi, grp in enumerate(cache.groups):
            status, self.top[gi] = ref.reserve(self.stack[gi], self.top[gi], self.bt[gi], self.ent[gi],
                                               self.lens // grp.m - self.ent[gi], BS)
            assert status == 0
        self.check_tables()
        for i, s in enumerate(self.specs):
            ref.ring_append(self.ring[i], pos, data[i]["kv"].unsqueeze(1), 1)
            assert torch.equal(cache.ring[i].cpu(), self.ring[i]), (step, i)
            win = ref.ring_read(self.ring[i], self.lens, torch.zeros(B, W, C, dtype=torch.bfloat16))
            ow = cache.out_window[i].cpu()
            for b in range(B):
                n = min(W, int(self.lens[b]))
                assert torch.equal(ow[b, :n], win[b, :n]), (step, i, b)
            if s.kind == "swa":
                continue
            gi = cache.group_of_rate[s.m]
            bt = self.bt[gi]
            self._check_emitted(i, s, gi, pos, data[i])
            if s.kind == "csa":
                n_valid = (self.lens - 1) // s.m
                idx = _np(cache.topk_idx[i])
                for b in range(B):
                    exp = ref.topk_select(scores[i][b:b + 1].numpy(), n_valid[b:b + 1], s.top_k,
                                          int(self.lens[b]) // s.m)[0]
                    assert np.array_equal(idx[b, :len(exp)], exp), (step, i, b)
                    assert (idx[b, len(exp):] == -1).all()
                # a -1 pick reads entry 0; a sequence without entries gets zero rows
                have = [b for b in range(B) if self.ent[gi][b] > 0]
                out = cache.out_entries[i].cpu()
                if have:
                    rows = np.concatenate([_rows(bt, b, idx[b]) for b in have])
                    want = _pool_rows(cache.pool[i], rows, s.fp8).view(len(have), s.top_k, C)
                    assert torch.equal(out[have], want), (step, i)
                for b in range(B):
                    if self.ent[gi][b] == 0:
                        assert not out[b].any(), (step, i, b)
            else:
                out = cache.out_entries[i].cpu()
                for b in range(B):
                    e = int(self.ent[gi][b])
                    want = _pool_rows(cache.pool[i], _rows(bt, b, np.arange(e)), s.fp8)
                    assert torch.equal(out[b, :e], want), (step, i, b)

    def _check_emitted(self, i, s, gi, pos, d) -> None:
        pools = [(self.cache.pool[i], s.fp8, self.bias[i], "c", "z")]
        if s.kind == "csa":
            pools.append((self.cache.idx_pool[i], False, self.ibias[i], "ci", "zi"))
        for (pool, fp8, bias, kc, kz), blk in zip(pools, self.blocks[i]):
            for b in blk.push(pos, d[kc], d[kz]):
                e = int(pos[b]) // s.m
                want = ref.compress_pool(blk.c[b], blk.z[b], bias)
                bound = ref.pooling_bound(blk.c[b], blk.z[b], bias)
                got = _pool_rows(pool, _rows(self.bt[gi], b, [e]), fp8)[0].float()
                tol = bound + (0.0625 * want.abs() if fp8 else 0.0)
                assert ((got - want).abs() <= tol).all(), (i, kc, b, e, float((got - want).abs().max()))


def test_fullsize_csa_64k(dev) -> None:
    """One CSA layer (m=4, top-k 512, W=128), B=16, L=65,536; two blocks complete."""
    from saint_kv.decode import LayerSpec

    run = _Run(dev, [LayerSpec("csa", m=4, top_k=512)], np.full(16, 65536), steps=8, seed=31)
    for step in range(8):
        run.step(step)


def test_fullsize_mixed_8layer(dev) -> None:
    """Eight layers alternating CSA (m=4, top-k 512) and HCA (m=128), W=128,
    B=32, L~U[32k,128k]; a few sequences sit just before an HCA block end."""
    from saint_kv.decode import LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=512) if i % 2 == 0 else LayerSpec("hca", m=128) for i in range(8)]
    lens0 = np.random.default_rng(32).integers(32 * 1024, 128 * 1024 + 1, size=32)
    lens0[:4] = lens0[:4] // 128 * 128 + np.array([125, 126, 127, 0])
    run = _Run(dev, specs, lens0, steps=5, seed=32)
    for step in range(5):
        run.step(step)


def test_fullsize_fp8_1m_release_compact(dev) -> None:
    """One FP8 CSA layer (m=4, top-k 1024, W=128), B=4, L~U[256k,1M] with 1%
    x20 outliers; 30% of the sequences finish, release and compaction are
    checked against the oracle (tables, stack, page contents), and the cache
    keeps stepping afterwards."""
    from saint_kv.decode import LayerSpec

    lens0 = np.random.default_rng(33).integers(256 * 1024, 1024 * 1024 + 1, size=4)
    run = _Run(dev, [LayerSpec("csa", m=4, top_k=1024, fp8=True)], lens0, steps=10, seed=33,
               outlier_frac=0.01)
    for step in range(6):
        run.step(step)
    cache = run.cache
    grp = cache.groups[0]
    pools = [cache.pool[0], cache.idx_pool[0]]
    before = [p.clone() for p in pools]
    mask = np.zeros(4, dtype=bool)
    mask[np.random.default_rng(34).choice(4, size=round(0.3 * 4), replace=False)] = True
    cache.release(mask)
    status, run.top[0] = ref.release(run.stack[0], run.top[0], run.bt[0], run.ent[0], mask, BS)
    assert status == 0
    run.lens[mask] = 0
    run.check_tables()
    info = cache.compact()
    n_pages = grp.n_pages
    movers, holes, n_live = ref.compact_plan(run.bt[0], run.ent[0], BS, n_pages)
    stack, run.top[0], moved = ref.compact([torch.zeros(n_pages, 1, 1, dtype=torch.uint8)], run.bt[0],
                                           run.ent[0], BS)
    run.stack[0] = stack
    assert info == [(n_live, moved)] and moved == len(movers) > 0
    run.check_tables()
    for p, b4 in zip(pools, before):
        want = b4.clone()
        want[torch.as_tensor(holes, device=dev)] = b4[torch.as_tensor(movers, device=dev)]
        assert torch.equal(p, want)
    del before
    # the finished sequences are empty; the others keep stepping on the rewritten tables
    for blk in run.blocks[0]:
        blk.c[torch.as_tensor(mask)] = 0
        blk.z[torch.as_tensor(mask)] = 0
    run.ring[0][torch.as_tensor(mask)] = cache.ring[0][torch.as_tensor(mask, device=dev)].cpu()
    for step in range(6, 9):
        run.step(step)
