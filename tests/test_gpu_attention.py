"""GPU parity of the decode attention over the paged cache (skv_decode_attention)
against the fp64 oracle (csa.py:324-373, hca.py:126-169, swa.py:115-137).

Tolerance: the kernel rounds q*w and the softmax weights to bf16 for its MFMAs
and each split's partial output to bf16 (relative 2^-9 each), and accumulates
in fp32, so every output element is held
to |got - want| <= ATT_TOL * max|want| of its (sequence, head) row plus 1e-4,
and the mean error to a tenth of that.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

ATT_TOL = 1e-2


def _i32(a, dev) -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, dtype=np.int32), device=dev)


class Case:
    """A paged compressed cache, window rings and queries on the GPU, with
    their CPU copies for the oracle."""

    def __init__(self, dev, seed, batch, heads, dim, n_ent, lens, window=128, bs=64, fp8=False):
        g = torch.Generator().manual_seed(seed)
        rng = np.random.default_rng(seed)
        self.dev, self.batch, self.heads, self.dim, self.window = dev, batch, heads, dim, window
        self.n_ent = np.asarray(n_ent, np.int32)
        self.lens = np.asarray(lens, np.int32)
        self.bs = bs
        bt_stride = max(1, -(-int(self.n_ent.max()) // bs)) + 1
        n_pages = batch * bt_stride + 5
        perm = rng.permutation(n_pages)
        table = np.full((batch, bt_stride), -1, np.int32)
        self.entries = []
        row_bytes = ref.FP8_ENTRY_BYTES if fp8 else None
        pool = torch.zeros(n_pages, bs, row_bytes if fp8 else dim,
                           dtype=torch.uint8 if fp8 else torch.bfloat16)
        k = 0
        for b in range(batch):
            n = int(self.n_ent[b])
            x = torch.randn(n, dim, generator=g).to(torch.bfloat16)
            if fp8:
                packed = ref.fp8_pack_entries(x) if n else torch.zeros(0, row_bytes, dtype=torch.uint8)
                x = ref.fp8_unpack_entries(packed) if n else x
            for p in range(-(-n // bs)):
                table[b, p] = perm[k]
                rows = slice(p * bs, min(n, (p + 1) * bs))
                pool[perm[k], : rows.stop - rows.start] = packed[rows] if fp8 else x[rows]
                k += 1
            self.entries.append(x.float().numpy().astype(np.float64))
        self.table = table
        self.pool = pool.to(dev)
        self.q = torch.randn(batch, heads, dim, generator=g).to(torch.bfloat16)
        self.win_k = torch.randn(batch, window, dim, generator=g).to(torch.bfloat16)
        self.win_v = torch.randn(batch, window, dim, generator=g).to(torch.bfloat16)
        self.knorm_w = torch.rand(dim, generator=g) + 0.5
        self.sink = torch.randn(heads, generator=g)

    def picks(self, top_k, seed):
        """Top-k rows as the selector emits them: distinct valid entries in
        some order, -1 past the valid ones."""
        rng = np.random.default_rng(seed)
        out = np.full((self.batch, top_k), -1, np.int32)
        for b in range(self.batch):
            n = int(self.n_ent[b])
            k = min(top_k, n)
            out[b, :k] = rng.choice(n, size=k, replace=False) if k else []
        return out

    def window_rows(self, b):
        L = int(self.lens[b])
        cnt = min(L, self.window)
        slots = [(p % self.window) for p in range(L - cnt, L)]
        return (self.win_k[b, slots].float().numpy().astype(np.float64),
                self.win_v[b, slots].float().numpy().astype(np.float64))

    def run(self, kind, picks=None, m=1, sink=True, softcap=None, splits=0, fp8=False, max_entries=0):
        from saint_kv import decode_attention

        d = self.dev
        kw = {}
        if kind != "swa":
            kw = dict(pool=self.pool, fp8=fp8, block_table=_i32(self.table, d),
                      n_entries=_i32(self.n_ent, d), knorm_w=self.knorm_w.to(d), m=m,
                      max_entries=max_entries)
            if kind == "csa":
                kw["picks"] = _i32(picks, d)
        out = decode_attention(self.q.to(d), kind, _i32(self.lens, d), self.win_k.to(d), self.win_v.to(d),
                               sink=self.sink.to(d) if sink else None, softcap=softcap, splits=splits, **kw)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def want(self, kind, picks=None, m=1, sink=True, softcap=None):
        out = np.zeros((self.batch, self.heads, self.dim))
        for b in range(self.batch):
            wk, wv = self.window_rows(b)
            out[b] = ref.decode_attention(
                self.q[b].float().numpy(), kind, int(self.lens[b]), entries=self.entries[b],
                picks=None if picks is None else picks[b], m=m, knorm_w=self.knorm_w.numpy(), eps=1e-6,
                sink=self.sink.numpy() if sink else None, softcap=softcap, win_k=wk, win_v=wv)
        return out


def _assert_close(got, want, label=""):
    assert np.isfinite(got).all(), label
    scale = np.abs(want).max(axis=-1, keepdims=True)
    err = np.abs(got - want)
    bad = err > ATT_TOL * scale + 1e-4
    assert not bad.any(), (label, float(err.max()), np.argwhere(bad)[:5].tolist())
    assert err.mean() <= 0.1 * ATT_TOL * scale.mean() + 1e-5, (label, float(err.mean()))


@pytest.mark.parametrize("heads,dim", [(64, 576), (40, 512), (128, 128)])
def test_attention_csa_matches_oracle(dev, heads, dim) -> None:
    c = Case(dev, heads + dim, 4, heads, dim, n_ent=[300, 1000, 64, 17], lens=[1203, 4003, 259, 70])
    picks = c.picks(96, 1)
    for softcap in (None, 3.0):
        got = c.run("csa", picks, softcap=softcap)
        _assert_close(got, c.want("csa", picks, softcap=softcap), f"csa softcap={softcap}")


@pytest.mark.parametrize("m", [4, 128])
def test_attention_hca_matches_oracle(dev, m) -> None:
    lens = [m * 300 + 1, m * 41, 5, m * 7 + 3, 1]
    n_ent = [(L // m) for L in lens]
    c = Case(dev, 10 + m, 5, 64, 576, n_ent=n_ent, lens=lens, bs=16)
    for sink in (True, False):
        got = c.run("hca", m=m, sink=sink)
        _assert_close(got, c.want("hca", m=m, sink=sink), f"hca m={m} sink={sink}")


def test_attention_swa_only(dev) -> None:
    c = Case(dev, 3, 6, 64, 576, n_ent=[0] * 6, lens=[1, 2, 127, 128, 129, 100000])
    for softcap in (None, 1.5):
        got = c.run("swa", softcap=softcap)
        _assert_close(got, c.want("swa", softcap=softcap), f"swa softcap={softcap}")


def test_attention_fp8_pool(dev) -> None:
    c = Case(dev, 4, 3, 64, 576, n_ent=[700, 40, 300], lens=[2801, 163, 1200], fp8=True)
    picks = c.picks(256, 2)
    got = c.run("csa", picks, fp8=True)
    _assert_close(got, c.want("csa", picks), "csa fp8")
    got = c.run("hca", m=4, fp8=True)
    _assert_close(got, c.want("hca", m=4), "hca fp8")


def test_attention_splits_agree(dev) -> None:
    """Every split of the keys over workgroups gives the same result."""
    c = Case(dev, 5, 3, 64, 576, n_ent=[2000, 513, 3], lens=[8001, 2055, 13])
    picks = c.picks(512, 3)
    want = c.want("csa", picks)
    outs = [c.run("csa", picks, splits=s) for s in (1, 2, 5, 16, 64)]
    for s, got in zip((1, 2, 5, 16, 64), outs):
        _assert_close(got, want, f"splits={s}")
    # one unit over 2000 entries: several runs of resolved rows
    got = c.run("hca", m=4, splits=1)
    _assert_close(got, c.want("hca", m=4), "hca one unit")


def test_attention_edge_rows(dev) -> None:
    """No valid pick, unmapped pages, picks past the entry count, a single
    window token."""
    c = Case(dev, 6, 4, 64, 576, n_ent=[50, 50, 50, 0], lens=[200, 1, 200, 1])
    picks = c.picks(64, 4)
    picks[0, :] = -1                 # no valid pick: the sparse branch adds 0
    picks[2, 5] = 60                 # past the entry count: masked
    c.table[1, 0] = -1               # unmapped page: its picks are masked
    want_picks = picks.copy()
    want_picks[2, 5] = -1
    want_picks[1, :] = -1
    got = c.run("csa", picks)
    _assert_close(got, c.want("csa", want_picks), "edge")


def test_attention_bad_arguments(dev) -> None:
    from saint_kv import decode_attention

    q = torch.zeros(2, 64, 576, dtype=torch.bfloat16, device=dev)
    ring = torch.zeros(2, 128, 576, dtype=torch.bfloat16, device=dev)
    lens = _i32([1, 1], dev)
    with pytest.raises(ValueError):
        decode_attention(q, "csa", lens, ring, ring)  # no pool
    with pytest.raises(ValueError):
        decode_attention(q[:, :, :100].contiguous(), "swa", lens, ring[:, :, :100].contiguous(),
                         ring[:, :, :100].contiguous())  # head_dim not a multiple of 32
    with pytest.raises(ValueError):  # more than 256 heads
        decode_attention(torch.zeros(2, 300, 576, dtype=torch.bfloat16, device=dev), "swa", lens, ring, ring)
    assert math.isfinite(decode_attention(q, "swa", lens, ring, ring).sum().item())
    # a workspace view off the 16-byte grid is refused, by the wrapper and by the library
    from saint_kv import attention

    ws = attention.last_workspace()
    buf = torch.empty(ws.numel() + 8, dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="aligned"):
        decode_attention(q, "swa", lens, ring, ring, workspace=buf[1:])
    decode_attention(q, "swa", lens, ring, ring, workspace=buf[4:])  # 16-byte offset: accepted


def test_attention_after_decode_step(dev) -> None:
    """The attention of each layer of a DecodeCache right after its fused
    step, over the cache's own pools, block tables, picks and rings, against
    the oracle over the step's gathered outputs (out_entries / out_window)."""
    from saint_kv import decode_attention
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=128), LayerSpec("csa", m=4, top_k=64, fp8=True),
             LayerSpec("hca", m=16), LayerSpec("swa")]
    B, W, H, D = 3, 32, 64, 576
    cache = DecodeCache(specs, B, 8192, window=W, block_size=16, device=dev, page_order_seed=3)
    gen = torch.Generator(device=dev).manual_seed(11)
    cache.prefill(np.array([900, 2047, 37]), generator=gen)
    g = torch.Generator().manual_seed(11)
    for i, s in enumerate(specs):
        for v in cache.inputs[i].values():
            v.normal_(generator=gen)
        if s.kind == "csa":
            cache.scores[i].copy_(torch.randn(*cache.scores[i].shape, generator=g))
    cache.step()
    torch.cuda.synchronize()
    cache.check_status()
    lens = cache.tok_lens.cpu().numpy().astype(np.int64)
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    knw = torch.rand(D, generator=g) + 0.5
    sink = torch.randn(H, generator=g)
    for i, s in enumerate(specs):
        kw = {}
        if s.kind != "swa":
            grp = cache.groups[cache.group_of_rate[s.m]]
            kw = dict(pool=cache.pool[i], fp8=s.fp8, block_table=grp.block_table, n_entries=grp.n_entries,
                      m=s.m, knorm_w=knw.to(dev))
            if s.kind == "csa":
                kw["picks"] = cache.topk_idx[i]
        got = decode_attention(q.to(dev), s.kind, cache.tok_lens, cache.ring[i], cache.ring[i],
                               sink=sink.to(dev), **kw).cpu().numpy()
        # the cache's own entry point (workspace kept per layer), twice
        for _ in range(2):
            mine = cache.attention(i, q.to(dev), knw.to(dev) if s.kind != "swa" else None, sink=sink.to(dev))
            assert np.array_equal(mine.cpu().numpy(), got), (i, s.kind)
        want = np.zeros((B, H, D))
        for b in range(B):
            L = int(lens[b])
            win = cache.out_window[i][b, :min(W, L)].float().cpu().numpy().astype(np.float64)
            ent = picks = None
            if s.kind == "csa":
                ent = cache.out_entries[i][b].float().cpu().numpy().astype(np.float64)
                idx = cache.topk_idx[i][b].cpu().numpy()
                picks = np.where(idx >= 0, np.arange(len(idx)), -1)
            elif s.kind == "hca":
                ent = cache.out_entries[i][b, :L // s.m].float().cpu().numpy().astype(np.float64)
            want[b] = ref.decode_attention(q[b].float().numpy(), s.kind, L, entries=ent, picks=picks, m=s.m,
                                           knorm_w=knw.numpy(), sink=sink.numpy(), win_k=win, win_v=win)
        _assert_close(got, want, f"layer {i} {s.kind}")
