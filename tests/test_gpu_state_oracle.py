"""Snapshot files written from the GPU cache, read and checked by the oracle.

A DecodeCache runs a ragged prefill and decode steps beside the oracle's
cache (reference_cpu: paged pools through the same page policy, the ring,
the buffered tokens of every incomplete block).  Every sequence is then saved
with every SWA strategy and the file is read by oracle.state_file, which
does not use saint_kv.  Each section must hold what the oracle's cache holds:

* header: length, layout, kept SWA rows by the full / periodic / zero closed
  forms;
* ``swa``: the ring rows of the kept positions, bit for bit;
* ``entries``: the oracle's pooled entries within the pooling bound (bf16
  streams), or, for an fp8 layer fed the same tokens as a bf16 layer, the
  e4m3fn quantization of that layer's entries bit for bit;
* ``state``: for an incomplete block of r tokens, the running maximum bit for
  bit, the softmax denominator within 1e-5 relative, and numerator /
  denominator (the block pooled so far) within the pooling bound.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref
from oracle import state_file as sf
from test_gpu_decode import _Oracle, _rand_data

pytestmark = pytest.mark.gpu

B, MAX_LEN, BS, W, C, CI = 3, 2048, 16, 32, 576, 128
STRATEGIES = [("full", None), ("periodic", 7), ("periodic", 8), ("zero", None)]


def _specs():
    from saint_kv.decode import LayerSpec

    # layer 1 is layer 0's fp8 twin: same tokens, bias and page group
    return [LayerSpec("csa", m=4, top_k=16), LayerSpec("csa", m=4, top_k=16, fp8=True, indexer=False),
            LayerSpec("hca", m=16), LayerSpec("swa")]


def _twin(data):
    data[1] = {k: v.clone() for k, v in data[0].items()}
    return data


def _run(dev):
    from saint_kv.decode import DecodeCache

    specs = _specs()
    seed = 11
    cache = DecodeCache(specs, B, MAX_LEN, block_size=BS, window=W, device=dev, page_order_seed=seed)
    orc = _Oracle(cache, specs, seed)
    g = torch.Generator().manual_seed(seed)
    bias = [None if s.kind == "swa" else torch.randn(s.m, C, generator=g) for s in specs]
    ibias = [torch.randn(s.m, CI, generator=g) if s.kind == "csa" else None for s in specs]
    bias[1], ibias[1] = bias[0], ibias[0]
    for i, s in enumerate(specs):
        if bias[i] is not None:
            cache.bias[i].copy_(bias[i])
        if s.kind == "csa" and s.indexer:
            cache.idx_bias[i].copy_(ibias[i])
    lens0 = np.array([2, 37, 301], dtype=np.int64)
    pre = _twin(_rand_data(g, specs, B, int(lens0.max()), C, CI))
    cache.prefill(lens0, data=[{k: v.to(dev) for k, v in d.items()} for d in pre])
    orc.append(lens0, pre, bias, ibias)
    for _ in range(6):
        data = _twin(_rand_data(g, specs, B, 1, C, CI))
        for i, s in enumerate(specs):
            for k, v in cache.inputs[i].items():
                v.copy_(data[i][k][:, 0])
            if cache.scores[i] is not None:
                cache.scores[i].normal_()
        cache.step()
        orc.append(np.ones(B, dtype=np.int32), data, bias, ibias)
    torch.cuda.synchronize()
    cache.check_status()
    assert np.array_equal(cache.tok_lens.cpu().numpy(), orc.lens)
    return specs, cache, orc, bias, ibias


def _streams(i, s, orc, bias, ibias):
    """(suffix, oracle pool, bound pool, tail c, tail z, bias) per stream."""
    t = orc.tails[i]
    out = [("", orc.pool[i], orc.bound[i], t[0], t[1], bias[i])]
    if s.kind == "csa" and s.indexer:
        out.append(("_idx", orc.ipool[i], orc.ibound[i], t[2], t[3], ibias[i]))
    return out


def test_snapshot_sections_match_oracle(dev, tmp_path) -> None:
    specs, cache, orc, bias, ibias = _run(dev)
    lens = orc.lens.tolist()
    assert lens == [8, 43, 307]  # r = 0 and r > 0 blocks, L < W and L > W
    checked_states = 0
    for b in range(B):
        L = int(lens[b])
        for strategy, period in STRATEGIES:
            path = tmp_path / f"s{b}_{strategy}{period}.skv"
            cache.save(b, path, strategy, period)
            hdr, sec = sf.read_state(path)
            ctx = (b, strategy, period)
            assert hdr["length"] == L, ctx
            assert hdr["layout"]["layers"] == [{"kind": s.kind, "m": s.m, "top_k": s.top_k, "fp8": s.fp8,
                                                "indexer": s.indexer} for s in specs]
            lo, hi = sf.kept_rows(L, W, strategy, period)
            assert hdr["swa_rows"] == [lo, hi], ctx
            expected_names = set()
            for i, s in enumerate(specs):
                if hi > lo:
                    expected_names.add(("swa", i))
                    want = torch.stack([orc.ring[i][b, p % W] for p in range(lo, hi)])
                    assert torch.equal(sec[("swa", i)], want), (ctx, i)
                if s.kind == "swa":
                    continue
                gi = orc.m_groups.index(s.m)
                n_ent = L // s.m
                r = L % s.m
                for sfx, pool, bound, tc, tz, bi in _streams(i, s, orc, bias, ibias):
                    expected_names |= {("entries" + sfx, i), ("state" + sfx, i)}
                    ent = sec[("entries" + sfx, i)]
                    assert ent.shape[0] == n_ent, (ctx, i, sfx)
                    ch = pool.shape[-1]
                    if s.fp8:
                        assert torch.equal(ent, ref.fp8_pack_entries(sec[("entries", 0)])), (ctx, i)
                    elif n_ent:
                        one = (orc.bt[gi][b:b + 1], np.array([n_ent], dtype=np.int32))
                        want = ref.paged_gather(pool, *one, torch.zeros(1, n_ent, ch, dtype=torch.bfloat16))[0]
                        tol = ref.paged_gather(bound, *one, torch.zeros(1, n_ent, ch))[0]
                        assert ((ent.float() - want.float()).abs() <= tol).all(), (ctx, i, sfx)
                    st = sec[("state" + sfx, i)]
                    assert st.shape == (3, ch)
                    if s.fp8:  # the twin folds the same tokens
                        if r:
                            assert torch.equal(st, sec[("state", 0)]), (ctx, i)
                        continue
                    if r == 0:
                        continue  # no incomplete block: the state is unspecified
                    cs, zs, bs_ = tc[b, :r], tz[b, :r], bi[:r]
                    want = sf.tail_state(cs, zs, bs_)
                    assert torch.equal(st[0], want[0]), (ctx, i, sfx)
                    assert ((st[1] - want[1]).abs() <= 1e-5 * want[1]).all(), (ctx, i, sfx)
                    pooled = st[2] / st[1]
                    exact = ref.compress_pool(cs, zs, bs_)
                    assert ((pooled - exact).abs() <= ref.pooling_bound(cs, zs, bs_)).all(), (ctx, i, sfx)
                    checked_states += 1
            assert set(sec) == expected_names, ctx
    assert checked_states >= 10


def test_snapshot_of_empty_sequence(dev, tmp_path) -> None:
    from saint_kv.decode import DecodeCache

    cache = DecodeCache(_specs(), 2, 256, block_size=BS, window=W, device=dev)
    cache.prefill(np.array([0, 9]), generator=torch.Generator(device=dev).manual_seed(2))
    path = tmp_path / "empty.skv"
    cache.save(0, path)
    hdr, sec = sf.read_state(path)
    assert hdr["length"] == 0 and hdr["swa_rows"] == [0, 0]
    for (name, i), t in sec.items():
        assert name.startswith(("entries", "state")), name
        if name.startswith("entries"):
            assert t.shape[0] == 0
