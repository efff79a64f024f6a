"""Refused page reservations across page groups.

Every page group of a DecodeCache reserves with its own all-or-nothing
``skv_reserve``.  When one group's pool is too small, prefill and
load_sequence must raise and leave the sequences empty: the groups that did
reserve give their pages back, so every free list holds the same page ids as
before and a later reservation that fits succeeds.  Both orders are covered:
the refusing group first (a later group's success must not hide it) and last
(the earlier groups' pages must be returned).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _free_sets(cache):
    out = []
    for g in cache.groups:
        top = int(g.free_top.item())
        out.append((top, sorted(g.free_stack[:top].cpu().tolist())))
    return out


def _assert_empty(cache, rows) -> None:
    for g in cache.groups:
        assert (g.block_table[rows] == -1).all()
        assert (g.n_entries[rows] == 0).all()
    assert (cache.tok_lens[rows] == 0).all()
    assert (cache.host_lens[rows] == 0).all()


def _specs():
    from saint_kv.decode import LayerSpec

    return [LayerSpec("csa", m=4, top_k=16), LayerSpec("hca", m=128)]


# the m=4 group is group 0 and the m=128 group is group 1
@pytest.mark.parametrize("small", [{4: 20}, {128: 2}], ids=["first-group-refuses", "last-group-refuses"])
def test_prefill_refused_by_one_group(dev, small) -> None:
    from saint_kv.decode import DecodeCache

    cache = DecodeCache(_specs(), 3, 8192, block_size=16, window=32, device=dev, pages_per_group=small)
    before = _free_sets(cache)
    # m=4: 1000+750+1250 entries = 63+47+79 pages; m=128: 31+23+39 entries = 2+2+3 pages
    with pytest.raises(RuntimeError, match="refused"):
        cache.prefill(np.array([4000, 3000, 5000]))
    assert _free_sets(cache) == before
    _assert_empty(cache, slice(None))
    assert int(cache.status.item()) == 0
    # the free lists are whole: a prefill that fits succeeds afterwards
    cache.prefill(np.array([256, 0, 300]))
    assert cache.host_lens.tolist() == [256, 0, 300]
    for g in cache.groups:
        assert g.n_entries.cpu().tolist() == [256 // g.m, 0, 300 // g.m]


@pytest.mark.parametrize("small", [{4: 10}, {128: 1}], ids=["first-group-refuses", "last-group-refuses"])
def test_load_refused_by_one_group(dev, tmp_path, small) -> None:
    from saint_kv.decode import DecodeCache

    gen = torch.Generator(device=dev).manual_seed(5)
    a = DecodeCache(_specs(), 2, 8192, block_size=16, window=32, device=dev)
    a.prefill(np.array([3000, 200]), generator=gen)
    path = tmp_path / "seq0.skv"
    a.save(0, path)

    b = DecodeCache(_specs(), 2, 8192, block_size=16, window=32, device=dev, pages_per_group=small)
    b.prefill(np.array([0, 70]), generator=gen)
    before = _free_sets(b)
    bt_before = [g.block_table.clone() for g in b.groups]
    # seq 0 needs 750 entries = 47 pages (m=4) and 23 entries = 2 pages (m=128)
    with pytest.raises(RuntimeError, match="refused"):
        b.load(0, path)
    assert _free_sets(b) == before
    _assert_empty(b, slice(0, 1))
    for g, bt in zip(b.groups, bt_before):  # the neighbour keeps its pages
        assert torch.equal(g.block_table, bt)
    assert b.host_lens.tolist() == [0, 70]
    # the same file loads into a cache whose pools fit
    c = DecodeCache(_specs(), 2, 8192, block_size=16, window=32, device=dev)
    c.load(1, path)
    assert c.host_lens.tolist() == [0, 3000]
