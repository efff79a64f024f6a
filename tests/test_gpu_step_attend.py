"""GPU parity of the decode step with the attention fused in
(skv_decode_step_attend, DecodeCache.step_attend) against the two calls it
replaces, skv_decode_step followed by skv_decode_attention, and against the
fp64 oracle (csa.py:299-373, hca.py:110-169, swa.py:107-137), and from run
to run (two identically seeded fused caches give the same output bits).

Two caches are built from the same seeds and fed the same inputs, one stepped
with step() + attention(), the other with step_attend().  Bit for bit: the
top-k rows, lengths, entry counts, block tables, free-stack tops, rings,
pools and pooling states.  The attention outputs differ only in how the picks
are split over units (each unit's partial output is rounded to bf16), so they
are held to the attention's oracle tolerance (test_gpu_attention.py): within
1e-2 of each (sequence, head) row's largest value.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

ATT_TOL = 1e-2


def _assert_close(got, want, label=""):
    assert np.isfinite(got).all(), label
    scale = np.abs(want).max(axis=-1, keepdims=True)
    err = np.abs(got - want)
    bad = err > ATT_TOL * scale + 1e-4
    assert not bad.any(), (label, float(err.max()), np.argwhere(bad)[:5].tolist())
    assert err.mean() <= 0.1 * ATT_TOL * scale.mean() + 1e-5, (label, float(err.mean()))


def _pair(specs, B, max_len, lens, dev, *, window=32, block_size=16, seed=3, pages=None):
    from saint_kv.decode import DecodeCache

    caches = []
    for _ in range(2):
        c = DecodeCache(specs, B, max_len, window=window, block_size=block_size, device=dev,
                        page_order_seed=seed, materialize=False, pages_per_group=pages)
        gen = torch.Generator(device=dev).manual_seed(seed)
        if c.bias[0] is not None:
            c.bias[0].normal_(generator=gen)
        if c.idx_bias[0] is not None:
            c.idx_bias[0].normal_(generator=gen)
        c.prefill(np.asarray(lens), generator=gen)
        caches.append(c)
    torch.cuda.synchronize()
    return caches


def _feed(caches, g, scores=None):
    """The same new-token rows and scores into both caches."""
    a = caches[0]
    for name, t in a.inputs[0].items():
        v = torch.randn(t.shape, generator=g).to(t.dtype)
        for c in caches:
            c.inputs[0][name].copy_(v)
    if a.scores[0] is not None:
        v = torch.randn(a.scores[0].shape, generator=g) if scores is None else scores
        for c in caches:
            c.scores[0].copy_(v)


def _state(c):
    out = {"tok_lens": c.tok_lens, "ring": c.ring[0]}
    for gi, g in enumerate(c.groups):
        out[f"bt{gi}"], out[f"ne{gi}"], out[f"top{gi}"] = g.block_table, g.n_entries, g.free_top
    if c.pool[0] is not None:
        out["pool"], out["state"] = c.pool[0], c.state[0]
    if c.topk_idx[0] is not None:
        out["topk_idx"] = c.topk_idx[0]
    return {k: v.cpu().contiguous().view(torch.uint8).numpy().copy() for k, v in out.items()}  # the bits


def _oracle(c, q, knw, sink, spec, W):
    """fp64 oracle of the layer's attention over c's cache (bf16 pools)."""
    B, H, D = q.shape
    lens = c.tok_lens.cpu().numpy()
    ring = c.ring[0].float().cpu().numpy().astype(np.float64)
    want = np.zeros((B, H, D))
    if spec.kind != "swa":
        g = c.groups[c.group_of_rate[spec.m]]
        bt = g.block_table.cpu().numpy()
        pool = c.pool[0].float().cpu().numpy().astype(np.float64)
        bs = pool.shape[1]
    for b in range(B):
        L = int(lens[b])
        n_w = min(W, L)
        win = np.stack([ring[b, pos % W] for pos in range(L - n_w, L)]) if n_w else np.zeros((0, D))
        ent = picks = None
        if spec.kind == "csa":  # the picked entries only
            idx = c.topk_idx[0][b].cpu().numpy().astype(np.int64)
            e = np.maximum(idx, 0)
            ent = np.where((idx >= 0)[:, None], pool[bt[b, e // bs], e % bs], 0.0)
            picks = np.where(idx >= 0, np.arange(len(idx)), -1)
        elif spec.kind != "swa":
            n = L // spec.m
            ent = np.stack([pool[bt[b, e // bs], e % bs] for e in range(n)]) if n else np.zeros((0, D))
        want[b] = ref.decode_attention(q[b].float().cpu().numpy(), spec.kind, L, entries=ent, picks=picks, m=spec.m,
                                       knorm_w=None if knw is None else knw.cpu().numpy(),
                                       sink=None if sink is None else sink.cpu().numpy(), win_k=win, win_v=win)
    return want


def _run_pair(caches, spec, steps, dev, g, H=64, W=32, oracle=True, scores=None):
    sep, fus = caches
    D = sep.latent
    for s in range(steps):
        _feed(caches, g, scores)
        q = torch.randn(sep.batch, H, D, generator=g).to(torch.bfloat16).to(dev)
        knw = (torch.rand(D, generator=g) + 0.5).to(dev) if spec.kind != "swa" else None
        sink = torch.randn(H, generator=g).to(dev)
        sep.step()
        want = sep.attention(0, q, knw, sink=sink).cpu().numpy()
        got = fus.step_attend(q, knw, sink=sink).cpu().numpy()
        torch.cuda.synchronize()
        sep.check_status()
        fus.check_status()
        a, b = _state(sep), _state(fus)
        for k in a:
            assert np.array_equal(a[k], b[k]), (spec.kind, s, k)
        _assert_close(got, want, f"{spec.kind} step {s}")
        if oracle and not spec.fp8:
            _assert_close(got, _oracle(fus, q, knw, sink, spec, W), f"{spec.kind} step {s} oracle")


@pytest.mark.parametrize("kind,fp8", [("csa", False), ("csa", True), ("hca", False), ("swa", False)])
def test_step_attend_matches_step_then_attention(dev, kind, fp8) -> None:
    from saint_kv.decode import LayerSpec

    spec = LayerSpec(kind, m=16 if kind == "hca" else 4, top_k=128 if not fp8 else 64, fp8=fp8)
    caches = _pair([spec], 3, 8192, [900, 2047, 37], dev)
    _run_pair(caches, spec, 6, dev, torch.Generator().manual_seed(5))


def test_step_attend_xcd_batch_many_heads(dev) -> None:
    """A batch of 8 (every launch places sequence b on XCD b % 8) and 128
    heads (two head groups: the second group's units rank again but leave the
    top-k row to the first)."""
    from saint_kv.decode import LayerSpec

    spec = LayerSpec("csa", m=4, top_k=256)
    lens = [4096, 333, 7000, 129, 5, 2048, 6001, 1024]
    caches = _pair([spec], 8, 8192, lens, dev, seed=7)
    _run_pair(caches, spec, 3, dev, torch.Generator().manual_seed(8), H=128)


def test_step_attend_partial_head_group_latent_512(dev) -> None:
    """40 heads (a partial head group) over a 512-channel latent."""
    from saint_kv.decode import DecodeCache, LayerSpec

    spec = LayerSpec("csa", m=4, top_k=96)
    caches = []
    for _ in range(2):
        c = DecodeCache([spec], 3, 4096, latent=512, window=32, block_size=16, device=dev, page_order_seed=5,
                        materialize=False)
        gen = torch.Generator(device=dev).manual_seed(5)
        c.bias[0].normal_(generator=gen)
        c.idx_bias[0].normal_(generator=gen)
        c.prefill(np.array([1500, 77, 3001]), generator=gen)
        caches.append(c)
    _run_pair(caches, spec, 3, dev, torch.Generator().manual_seed(6), H=40)


def test_step_attend_tie_overflow_full_select(dev) -> None:
    """Equal scores over 5,000 entries put every entry in one tie bin, past
    the candidate lists' capacity: the units fall back to the full select."""
    from saint_kv.decode import LayerSpec

    spec = LayerSpec("csa", m=4, top_k=512)
    caches = _pair([spec], 2, 24000, [20000, 20480], dev)
    zeros = torch.zeros(caches[0].scores[0].shape)
    _run_pair(caches, spec, 2, dev, torch.Generator().manual_seed(9), scores=zeros)
    idx = caches[1].topk_idx[0].cpu().numpy()
    lens = caches[1].tok_lens.cpu().numpy()
    for b in range(2):  # ties go to the lower index
        n_valid = (int(lens[b]) - 1) // 4
        assert np.array_equal(idx[b], np.arange(min(512, n_valid)))


def test_step_attend_rows_past_the_run_table(dev) -> None:
    """One launch over a row of 135,000 entries (66 filter chunks, more than
    the run table holds: its units rank every candidate, by entry index mod
    the unit count, and write every position) and a row of 75,000 entries
    (37 chunks: its units rank their ties and the window units write the sure
    candidates' positions).  Two steps; the top-k rows bit for bit against
    the separate path."""
    from saint_kv.decode import LayerSpec

    spec = LayerSpec("csa", m=4, top_k=512)
    caches = _pair([spec], 2, 540064, [540000, 300000], dev, window=128, block_size=64)
    assert caches[0].scores[0].shape[1] > 64 * 2048  # past the run table
    _run_pair(caches, spec, 2, dev, torch.Generator().manual_seed(13), W=128, oracle=False)


def test_step_attend_long_lists_rank_from_global(dev) -> None:
    """top-k 2048 over 2,000 sure candidates and a 3,000-key tie bin: 5,000
    candidates, more than a unit holds in LDS, so the units rank from the
    lists in global memory."""
    from saint_kv.decode import LayerSpec

    spec = LayerSpec("csa", m=4, top_k=2048)
    caches = _pair([spec], 2, 24064, [24000, 24000], dev)
    cols = caches[0].scores[0].shape[1]
    g = torch.Generator().manual_seed(12)
    row = -torch.rand(cols, generator=g)  # below the ties
    row[:2000] = 10.0 + torch.rand(2000, generator=g)  # sure
    row[2000:5000] = 1.0  # one tie bin
    scores = torch.stack([row, row.flip(0).roll(5000)])
    _run_pair(caches, spec, 1, dev, g, scores=scores)
    idx = caches[1].topk_idx[0].cpu().numpy()
    assert set(idx[0][:2000]) == set(range(2000)) and np.array_equal(idx[0][2000:], np.arange(2000, 2048))


def test_step_attend_config3_shape(dev) -> None:
    """B=16 at 64k context, CSA m=4, top-k 512, W=128, block size 64 (the
    64k decode workload), two steps, against the separate path and the fp64
    oracle."""
    from saint_kv.decode import LayerSpec

    spec = LayerSpec("csa", m=4, top_k=512)
    caches = _pair([spec], 16, 65536 + 16, np.full(16, 65536), dev, window=128, block_size=64)
    _run_pair(caches, spec, 2, dev, torch.Generator().manual_seed(10), W=128)


@pytest.mark.parametrize("fp8", [False, True])
def test_step_attend_bit_reproducible(dev, fp8) -> None:
    """Two caches built from the same seeds and stepped with the same inputs
    give bit-identical attention outputs: a CSA unit attends over the picks
    whose entry index is its own residue, so its partial output does not
    depend on the order in which the filter chunks (several per score row,
    rows of 7,000-16,000 columns) appended to the candidate lists.  The
    outputs stay within the oracle tolerance."""
    from saint_kv.decode import LayerSpec

    spec = LayerSpec("csa", m=4, top_k=512, fp8=fp8)
    lens = [65000, 28000, 41000, 60000, 33333, 52000, 47000, 64000]
    caches = _pair([spec], 8, 65536, lens, dev, window=128, block_size=64, seed=21)
    g = torch.Generator().manual_seed(22)
    D = caches[0].latent
    for s in range(3):
        _feed(caches, g)
        q = torch.randn(8, 64, D, generator=g).to(torch.bfloat16).to(dev)
        knw = (torch.rand(D, generator=g) + 0.5).to(dev)
        sink = torch.randn(64, generator=g).to(dev)
        outs = [c.step_attend(q, knw, sink=sink).cpu().numpy() for c in caches]
        torch.cuda.synchronize()
        for c in caches:
            c.check_status()
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), s
        a, b = _state(caches[0]), _state(caches[1])
        for k in a:
            assert np.array_equal(a[k], b[k]), (s, k)
        if not fp8:
            _assert_close(outs[0], _oracle(caches[0], q, knw, sink, spec, 128), f"step {s} oracle")


def test_step_attend_refused_step(dev) -> None:
    """A step whose pages run out is refused as skv_decode_step refuses it:
    check_status raises and nothing is committed."""
    from saint_kv.decode import LayerSpec

    spec = LayerSpec("csa", m=4, top_k=32)
    # 2 sequences of 64 entries (bs 16 -> 4 full pages each) in a pool of 8
    # pages: the entry the next token completes (L = 260) needs a fifth page
    c = _pair([spec], 2, 4096, [259, 259], dev, pages={4: 8})[1]
    before = _state(c)
    g = torch.Generator().manual_seed(2)
    _feed([c], g)
    q = torch.randn(2, 64, c.latent, generator=g).to(torch.bfloat16).to(dev)
    c.step_attend(q, (torch.rand(c.latent, generator=g) + 0.5).to(dev))
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError):
        c.check_status()
    after = _state(c)
    for k in ("tok_lens", "bt0", "ne0", "top0"):
        assert np.array_equal(before[k], after[k]), k


def test_step_attend_rejects_bad_use(dev) -> None:
    from saint_kv.decode import DecodeCache, LayerSpec

    c = DecodeCache([LayerSpec("csa", m=4, top_k=32)], 2, 1024, window=32, block_size=16, device=dev)
    q = torch.zeros(2, 64, 576, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="materialize"):
        c.step_attend(q, torch.ones(576, device=dev))
    c2 = DecodeCache([LayerSpec("csa", m=4, top_k=32), LayerSpec("swa")], 2, 1024, window=32, block_size=16,
                     device=dev, materialize=False)
    with pytest.raises(ValueError, match="one-layer"):
        c2.step_attend(q, torch.ones(576, device=dev))
    c3 = DecodeCache([LayerSpec("csa", m=4, top_k=32)], 2, 1024, window=32, block_size=16, device=dev,
                     materialize=False)
    with pytest.raises(ValueError, match="knorm_w"):
        c3.step_attend(q)
