"""Several query tokens per sequence (t_new >= 1, the cached forward of
csa.py:276-281 / hca.py:127-131 / swa.py:115-125) through skv_decode_attention
and through ``cached_attention`` over the drop-in cache layers, against the
fp64 oracle row by row.

Query token t of a sequence whose cache holds L tokens after the append is
position q_pos = L - T + t (cache_offset = L - T): its window is the positions
k_pos <= q_pos with q_pos - k_pos < W (swa.py:121-124), an HCA entry s is
visible when s*m + m-1 < q_pos (hca.py:128-130), and a CSA query attends over
its own top-k row.  The oracle takes each (sequence, token) row with its own
L_t = q_pos + 1.  The drop-in test also restates the reference's masked form
(every cached position under the mask, csa.py:352-371) in fp64 torch, which
checks the per-row window selection.  Tolerance as in test_gpu_attention.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

ATT_TOL = 1e-2


def _i32(a, dev) -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, dtype=np.int32), device=dev)


def _assert_close(got, want, label=""):
    assert np.isfinite(got).all(), label
    scale = np.abs(want).max(axis=-1, keepdims=True)
    err = np.abs(got - want)
    bad = err > ATT_TOL * scale + 1e-4
    assert not bad.any(), (label, float(err.max()), np.argwhere(bad)[:5].tolist())
    assert err.mean() <= 0.1 * ATT_TOL * scale.mean() + 1e-5, (label, float(err.mean()))


def _f64(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy().astype(np.float64)


class MultiCase:
    """A paged compressed cache (bf16 or fp8 entries), window rings of R slots
    (or [K | V] rows of a contiguous cache) and T queries per sequence."""

    def __init__(self, dev, seed, batch, heads, dim, T, lens, m, window, ring, bs=16, fp8=False, kv_rows=False):
        g = torch.Generator().manual_seed(seed)
        rng = np.random.default_rng(seed)
        self.dev, self.batch, self.heads, self.dim = dev, batch, heads, dim
        self.T, self.m, self.window, self.ring = T, m, window, ring
        self.lens = np.asarray(lens, np.int32)
        self.n_ent = self.lens // m
        bt_stride = max(1, -(-int(self.n_ent.max()) // bs)) + 1
        n_pages = batch * bt_stride + 3
        perm = rng.permutation(n_pages)
        table = np.full((batch, bt_stride), -1, np.int32)
        row = ref.FP8_ENTRY_BYTES if fp8 else dim
        pool = torch.zeros(n_pages, bs, row, dtype=torch.uint8 if fp8 else torch.bfloat16)
        self.entries = []
        k = 0
        for b in range(batch):
            n = int(self.n_ent[b])
            x = torch.randn(n, dim, generator=g).to(torch.bfloat16)
            packed = ref.fp8_pack_entries(x) if fp8 and n else None
            if fp8 and n:
                x = ref.fp8_unpack_entries(packed)
            for p in range(-(-n // bs)):
                table[b, p] = perm[k]
                rows = slice(p * bs, min(n, (p + 1) * bs))
                pool[perm[k], : rows.stop - rows.start] = packed[rows] if fp8 else x[rows]
                k += 1
            self.entries.append(_f64(x))
        self.fp8, self.table, self.pool = fp8, table, pool.to(dev)
        # window rows: position p of sequence b in slot p % ring
        kv = torch.randn(batch, ring, 2, dim, generator=g).to(torch.bfloat16)
        if kv_rows:
            self.kv = kv.to(dev)
            self.win_k, self.win_v = self.kv[:, :, 0], self.kv[:, :, 1]
        else:
            self.win_k, self.win_v = kv[:, :, 0].contiguous().to(dev), kv[:, :, 1].contiguous().to(dev)
        self.cpu_k, self.cpu_v = _f64(kv[:, :, 0]), _f64(kv[:, :, 1])
        self.q = torch.randn(batch, T, heads, dim, generator=g).to(torch.bfloat16)
        self.knorm_w = torch.rand(dim, generator=g) + 0.5
        self.sink = torch.randn(heads, generator=g)
        # each query's top-k row: distinct entries it may see, -1 padded
        top_k = 24
        self.picks = np.full((batch, T, top_k), -1, np.int32)
        for b in range(batch):
            for t in range(T):
                n_valid = min(ref.n_valid_blocks(self.q_pos(b, t), m), int(self.n_ent[b]))
                kk = min(top_k - 3, n_valid)
                if kk:
                    self.picks[b, t, :kk] = rng.choice(n_valid, size=kk, replace=False)

    def q_pos(self, b, t):
        return int(self.lens[b]) - self.T + t

    def run(self, kind, softcap=None, splits=0, q=None, picks=None):
        from saint_kv import decode_attention

        d = self.dev
        kw = {}
        if kind != "swa":
            kw = dict(pool=self.pool, fp8=self.fp8, block_table=_i32(self.table, d),
                      n_entries=_i32(self.n_ent, d), knorm_w=self.knorm_w.to(d), m=self.m)
            if kind == "csa":
                kw["picks"] = _i32(self.picks if picks is None else picks, d)
        out = decode_attention((self.q if q is None else q).to(d), kind, _i32(self.lens, d), self.win_k,
                               self.win_v, sink=self.sink.to(d), softcap=softcap, splits=splits,
                               window=self.window, **kw)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def want(self, kind, softcap=None):
        out = np.zeros((self.batch, self.T, self.heads, self.dim))
        for b in range(self.batch):
            for t in range(self.T):
                L_t = self.q_pos(b, t) + 1
                pos = ref.swa_window_positions(L_t, self.window)
                slots = [p % self.ring for p in pos]
                out[b, t] = ref.decode_attention(
                    self.q[b, t].float().numpy(), kind, L_t, entries=self.entries[b], picks=self.picks[b, t],
                    m=self.m, knorm_w=self.knorm_w.numpy(), eps=1e-6, sink=self.sink.numpy(), softcap=softcap,
                    win_k=self.cpu_k[b, slots], win_v=self.cpu_v[b, slots])
        return out


@pytest.mark.parametrize("kind", ["csa", "hca", "swa"])
@pytest.mark.parametrize("heads,dim,T", [(64, 576, 5), (40, 512, 3), (16, 128, 9)])
def test_multi_query_matches_oracle(dev, kind, heads, dim, T) -> None:
    """T tokens per sequence over a ring of exactly W + T - 1 slots, the
    positions wrapped around it; HCA m=8, CSA m=4."""
    m = 4 if kind == "csa" else 8
    W = 32
    c = MultiCase(dev, heads + T, 3, heads, dim, T, lens=[203, 1001, T + 2], m=m, window=W, ring=W + T - 1)
    for softcap in (None, 3.0):
        for splits in (0, 3):
            _assert_close(c.run(kind, softcap, splits), c.want(kind, softcap), f"{kind} softcap={softcap} s={splits}")


def test_multi_query_fp8_and_kv_rows(dev) -> None:
    """fp8 entries, and window slots that are the K and V halves of [B, R, 2,
    D] rows of a contiguous cache (R >= every length: slot = position)."""
    c = MultiCase(dev, 7, 2, 64, 576, 4, lens=[150, 97], m=4, window=64, ring=160, fp8=True, kv_rows=True)
    for kind in ("csa", "hca", "swa"):
        _assert_close(c.run(kind), c.want(kind), kind)


def test_one_query_rows_agree(dev) -> None:
    """T = 1 as [B, 1, H, D] gives the [B, H, D] call's output bit for bit."""
    c = MultiCase(dev, 11, 3, 64, 576, 1, lens=[300, 70, 9], m=4, window=32, ring=32)
    for kind in ("csa", "hca", "swa"):
        four = c.run(kind)
        three = c.run(kind, q=c.q[:, 0], picks=c.picks[:, 0])
        assert np.array_equal(four[:, 0], three), kind


def _masked_reference(q, ent, picks, sw_k, sw_v, q_pos, W, m, kind, knorm_w, sink, softcap):
    """The reference's cached-forward arithmetic in fp64 torch over every
    cached position under its masks: CSA's sparse branch as clamp + gather +
    k_norm + mask + row_has_pick (csa.py:324-350), HCA's compressed branch
    under s*m + m-1 < q_pos with the sink (hca.py:126-141), the window branch
    under k_pos <= q_pos and q_pos - k_pos < W with the sink and the softcap
    (csa.py:352-371, common.py:77-124).  q (H, T, D), picks (T, k), q_pos (T,)."""
    def sdpa(qq, k, v, mask, sink_logit, cap):
        s = qq @ k.transpose(-1, -2) / k.shape[-1] ** 0.5
        if cap is not None:
            s = cap * torch.tanh(s / cap)
        s = s.masked_fill(~mask, float("-inf"))
        if sink_logit is not None:
            sl = sink_logit.view(-1, 1, 1).expand(-1, s.shape[1], 1)
            p = torch.softmax(torch.cat([s, sl], dim=-1), dim=-1)[..., :-1]
        else:
            p = torch.softmax(s, dim=-1)
        p = torch.nan_to_num(p, nan=0.0)
        return p @ v

    def k_norm(x):
        return knorm_w * x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6)

    H, T, D = q.shape
    k_pos = torch.arange(sw_k.shape[0]).view(1, -1)
    qp = q_pos.view(-1, 1)
    sw_mask = (k_pos <= qp) & ((qp - k_pos) < W)
    out = sdpa(q, sw_k, sw_v, sw_mask.unsqueeze(0), sink, softcap)
    if kind == "csa":
        valid = picks >= 0
        kv = k_norm(ent[picks.clamp(min=0)])  # (T, k, D)
        s = torch.einsum("htd,tkd->htk", q, kv) / D ** 0.5
        s = s.masked_fill(~valid.unsqueeze(0), float("-inf"))
        has = valid.any(-1).view(1, T, 1)
        s = torch.where(has, s, torch.zeros_like(s))
        mixed = torch.einsum("htk,tkd->htd", torch.softmax(s, dim=-1), kv)
        out = out + torch.where(has, mixed, torch.zeros_like(mixed))
    elif kind == "hca" and ent.shape[0]:
        block_end = torch.arange(ent.shape[0]).view(1, -1) * m + (m - 1)
        valid = block_end < qp
        ck = k_norm(ent)
        comp = sdpa(q, ck, ck, valid.unsqueeze(0), sink, None)
        out = out + comp
    return out


@pytest.mark.parametrize("kind", ["csa", "hca", "swa"])
def test_cached_attention_over_drop_in_layers(dev, kind) -> None:
    """The drop-in layers (bf16) after a prefill of 37 tokens, a 6-token
    append and a 1-token append: cached_attention for each call's new tokens
    against the oracle row by row and against the reference's masked form."""
    from saint_kv import kv_cache as kvc
    from saint_kv.attention import cached_attention

    B, H, D, hidden, W = 2, 16, 128, 64, 16
    m = 4 if kind == "csa" else 8
    g = torch.Generator().manual_seed(5)
    w_c = torch.randn(hidden, D, generator=g) / hidden ** 0.5
    w_i = torch.randn(hidden, 32, generator=g) / hidden ** 0.5

    def comp(w):
        return lambda x: (x.float().view(B, -1, m, hidden).mean(2) @ w.to(x.device)).to(x.dtype)

    if kind == "csa":
        layer = kvc.CSAKVCacheLayer(96, hidden, D, 32, m, batch_size=B, device=dev, dtype=torch.bfloat16)
    elif kind == "hca":
        layer = kvc.HCAKVCacheLayer(96, hidden, D, m, batch_size=B, device=dev, dtype=torch.bfloat16)
    else:
        layer = kvc.SWAKVCacheLayer(96, D, batch_size=B, device=dev, dtype=torch.bfloat16)
    knorm_w = (torch.rand(D, generator=g) + 0.5).to(dev)
    sink = torch.randn(H, generator=g).to(dev)
    rng = np.random.default_rng(3)
    for t_new in (37, 6, 1):
        h = torch.randn(B, t_new, hidden, generator=g).to(torch.bfloat16).to(dev)
        k_new = torch.randn(B, t_new, D, generator=g).to(torch.bfloat16).to(dev)
        v_new = torch.randn(B, t_new, D, generator=g).to(torch.bfloat16).to(dev)
        if kind == "csa":
            ent_view, _, sw_k, sw_v = layer.append(h, k_new, v_new, compressor=comp(w_c), indexer_compressor=comp(w_i))
        elif kind == "hca":
            ent_view, sw_k, sw_v = layer.append(h, k_new, v_new, compressor=comp(w_c))
        else:
            sw_k, sw_v = layer.append(k_new, v_new)
            ent_view = torch.zeros(B, 0, D)
        L = layer.length
        q_pos = torch.arange(L - t_new, L)
        picks = np.full((B, t_new, 8), -1, np.int64)
        for b in range(B):
            for t in range(t_new):
                n_valid = min(ref.n_valid_blocks(int(q_pos[t]), m), ent_view.shape[1])
                kk = min(6, n_valid)
                if kk:
                    picks[b, t, :kk] = rng.choice(n_valid, size=kk, replace=False)
        q = torch.randn(B, H, t_new, D, generator=g).to(torch.bfloat16)
        got = cached_attention(layer, q.to(dev), window=W, top_idx=torch.as_tensor(picks).to(dev),
                               knorm_w=knorm_w, sink=sink, softcap=2.5)
        torch.cuda.synchronize()
        got = got.cpu().numpy()
        assert got.shape == (B, H, t_new, D)
        ent64 = [_f64(ent_view[b]) for b in range(B)]
        k64, v64 = _f64(sw_k), _f64(sw_v)
        want = np.zeros_like(got, dtype=np.float64)
        masked = np.zeros_like(want)
        for b in range(B):
            for t in range(t_new):
                L_t = int(q_pos[t]) + 1
                pos = ref.swa_window_positions(L_t, W)
                want[b, :, t] = ref.decode_attention(
                    _f64(q[b, :, t]), kind, L_t, entries=ent64[b], picks=picks[b, t], m=m,
                    knorm_w=_f64(knorm_w), eps=1e-6, sink=_f64(sink), softcap=2.5, win_k=k64[b, pos],
                    win_v=v64[b, pos])
            masked[b] = _masked_reference(
                torch.from_numpy(_f64(q[b])), torch.from_numpy(ent64[b]), torch.as_tensor(picks[b]),
                torch.from_numpy(k64[b]), torch.from_numpy(v64[b]), q_pos, W, m, kind,
                torch.from_numpy(_f64(knorm_w)), torch.from_numpy(_f64(sink)), 2.5).numpy()
        np.testing.assert_allclose(masked, want, rtol=1e-9, atol=1e-9)
        _assert_close(got.transpose(0, 2, 1, 3), want.transpose(0, 2, 1, 3), f"{kind} t_new={t_new}")
