"""GPU round trip of the per-request snapshot (saint_kv.state): a sequence
saved from one cache and loaded into an empty slot of another, with different
physical pages and neighbours, continues bit-exactly: the same top-k indices,
gathered entries and windows step after step, for every SWA strategy."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from saint_kv import ops

pytestmark = pytest.mark.gpu

SPECS = None


def _specs():
    from saint_kv.decode import LayerSpec

    return [LayerSpec("csa", m=4, top_k=32), LayerSpec("csa", m=4, top_k=16, fp8=True, indexer=False),
            LayerSpec("hca", m=16), LayerSpec("swa")]


def _feed(cache, gen, b_rows, inputs=None, scores=None):
    """Random inputs and scores; rows b_rows copied from the given ones."""
    ins, scs = [], []
    for i, s in enumerate(cache.layers):
        step_in = {}
        for k, v in cache.inputs[i].items():
            v.normal_(generator=gen)
            if inputs is not None:
                v[b_rows] = inputs[i][k][b_rows]
            step_in[k] = v.clone()
        ins.append(step_in)
        sc = None
        if s.kind == "csa":
            cache.scores[i].normal_(generator=gen)
            if scores is not None:
                cache.scores[i][b_rows] = scores[i][b_rows]
            sc = cache.scores[i].clone()
        scs.append(sc)
    return ins, scs


def _outputs(cache, b):
    out = []
    L = int(cache.host_lens[b])
    for i, s in enumerate(cache.layers):
        out.append(("window", cache.out_window[i][b].clone()))
        if s.kind == "csa":
            out.append(("topk", cache.topk_idx[i][b].clone()))
            out.append(("entries", cache.out_entries[i][b].clone()))
        elif s.kind == "hca":
            out.append(("entries", cache.out_entries[i][b, :L // s.m].clone()))
    return out


@pytest.mark.parametrize("swa,period", [("full", None), ("periodic", 7), ("periodic", 8), ("zero", None)])
def test_snapshot_resumes_bit_exact(dev, tmp_path, swa, period) -> None:
    from saint_kv.decode import DecodeCache

    specs = _specs()
    W = 16
    a = DecodeCache(specs, 3, 2048, window=W, block_size=16, device=dev, page_order_seed=1)
    gen = torch.Generator(device=dev).manual_seed(3)
    a.prefill(np.array([300, 517, 64]), generator=gen)
    for _ in range(3):
        _feed(a, gen, [1])
        a.step()
    a.check_status()
    L = int(a.host_lens[1])  # 520
    path = tmp_path / "seq1.skv"
    hdr = a.save(1, path, swa, period)
    assert hdr["length"] == L
    # the SWA rows a caller would recompute: the oracle of the ring (the last W rows)
    lens1 = torch.tensor([L], dtype=torch.int32, device=dev)
    rings = []
    for i in range(len(specs)):
        r = torch.empty(1, W, a.latent, dtype=torch.bfloat16, device=dev)
        ops.ring_read(a.ring[i][1:2], lens1, r)
        rings.append(r)
    b = DecodeCache(specs, 3, 2048, window=W, block_size=16, device=dev, page_order_seed=7)
    b.prefill(np.array([100, 0, 50]), generator=gen)
    lo, hi = b.load(1, path)
    if swa == "full" or (swa == "periodic" and L % period == 0):
        assert (lo, hi) == (L, L)
    else:
        assert hi == L and lo < L
        for i in range(len(specs)):  # the caller appends the missing rows
            src = rings[i][:, W - (hi - lo):]
            ops.ring_append(b.ring[i][1:2], lens1, src.contiguous(), hi - lo)
    for step in range(3):
        ins, scs = _feed(a, gen, [1])
        _feed(b, gen, [1], ins, scs)
        a.step()
        b.step()
        a.check_status()
        b.check_status()
        for (name, x), (_, y) in zip(_outputs(a, 1), _outputs(b, 1)):
            assert torch.equal(x, y), (swa, period, step, name)


def test_snapshot_refuses_mismatch(dev, tmp_path) -> None:
    from saint_kv.decode import DecodeCache, LayerSpec

    a = DecodeCache(_specs(), 2, 1024, window=16, block_size=16, device=dev)
    a.prefill(np.array([40, 70]), generator=torch.Generator(device=dev).manual_seed(1))
    path = tmp_path / "s.skv"
    a.save(0, path)
    with pytest.raises(RuntimeError, match="not empty"):
        a.load(1, path)
    other = DecodeCache([LayerSpec("csa", m=4, top_k=32)], 2, 1024, window=16, block_size=16, device=dev)
    with pytest.raises(ValueError, match="layout"):
        other.load(0, path)
    a.release(np.array([False, True]))
    assert a.load(1, path) == (40, 40)
