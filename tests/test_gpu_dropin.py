"""The drop-in cache classes reproduce the reference behaviours of
packages/inference/tests/test_kv_cache.py on paged HIP storage (GPU), and
their outputs equal the contiguous restatement of kv_cache.py (the oracle)."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu


def _kv():
    from saint_kv import kv_cache

    return kv_cache


# ---------- SWAKVCacheLayer (test_kv_cache.py:30-86) ----------
def test_swa_initial_state_and_append(dev) -> None:
    kv = _kv()
    cache = kv.SWAKVCacheLayer(max_seq_len=16, head_dim=32)
    assert cache.length == 0 and cache.k.shape == (1, 16, 32) and cache.v.shape == (1, 16, 32)
    cache = kv.SWAKVCacheLayer(max_seq_len=16, head_dim=8)
    k, v = torch.randn(1, 4, 8, device=dev), torch.randn(1, 4, 8, device=dev)
    full_k, full_v = cache.append(k, v)
    assert cache.length == 4 and full_k.shape == (1, 4, 8)
    assert torch.equal(full_k, k) and torch.equal(full_v, v)


def test_swa_multiple_appends_concatenate(dev) -> None:
    cache = _kv().SWAKVCacheLayer(max_seq_len=16, head_dim=8)
    a_k, a_v = torch.randn(1, 2, 8, device=dev), torch.randn(1, 2, 8, device=dev)
    b_k, b_v = torch.randn(1, 3, 8, device=dev), torch.randn(1, 3, 8, device=dev)
    cache.append(a_k, a_v)
    full_k, full_v = cache.append(b_k, b_v)
    assert cache.length == 5
    assert torch.equal(full_k[:, :2], a_k) and torch.equal(full_k[:, 2:5], b_k)
    assert torch.equal(full_v[:, :2], a_v) and torch.equal(full_v[:, 2:5], b_v)


def test_swa_errors_and_reset(dev) -> None:
    kv = _kv()
    cache = kv.SWAKVCacheLayer(max_seq_len=4, head_dim=8)
    with pytest.raises(RuntimeError, match="overflow"):
        cache.append(torch.randn(1, 5, 8, device=dev), torch.randn(1, 5, 8, device=dev))
    with pytest.raises(ValueError, match="must be 3D"):
        cache.append(torch.randn(1, 8, device=dev), torch.randn(1, 8, device=dev))
    cache = kv.SWAKVCacheLayer(max_seq_len=16, head_dim=8)
    cache.append(torch.randn(1, 4, 8, device=dev), torch.randn(1, 4, 8, device=dev))
    cache.reset()
    assert cache.length == 0
    k = torch.randn(1, 16, 8, device=dev)
    full_k, _ = cache.append(k, k)  # every page is reusable after reset
    assert torch.equal(full_k, k)


def test_swa_matches_contiguous_reference_batched_bf16(dev) -> None:
    kv = _kv()
    g = torch.Generator().manual_seed(0)
    cont = ref.ContiguousSWA(300, 128, batch_size=3, dtype=torch.bfloat16)
    cache = kv.SWAKVCacheLayer(300, 128, batch_size=3, dtype=torch.bfloat16)
    for n in (17, 1, 1, 64, 3, 100, 1):
        k = torch.randn(3, n, 128, generator=g).to(torch.bfloat16)
        v = torch.randn(3, n, 128, generator=g).to(torch.bfloat16)
        ek, ev = cont.append(k, v)
        gk, gv = cache.append(k.to(dev), v.to(dev))
        assert torch.equal(gk.cpu(), ek) and torch.equal(gv.cpu(), ev)


# ---------- HCA / CSA (test_kv_cache.py:307-490) ----------
class _Compressor(torch.nn.Module):
    """TokenLevelCompressor-shaped pooling (csa.py:66-88) with random weights."""

    def __init__(self, hidden, c, m, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.m, self.c = m, c
        self.w_kv = torch.randn(hidden, c, generator=g)
        self.w_z = torch.randn(hidden, c, generator=g)
        self.bias = torch.randn(m, c, generator=g)

    def forward(self, h):
        b, t, _ = h.shape
        nb = t // self.m
        cz = (h @ self.w_kv.to(h.device)).view(b, nb, self.m, self.c)
        zz = (h @ self.w_z.to(h.device)).view(b, nb, self.m, self.c) + self.bias.to(h.device)
        return (torch.softmax(zz, dim=-2) * cz).sum(dim=-2)


def test_hca_state_machine_and_errors(dev) -> None:
    kv = _kv()
    cache = kv.HCAKVCacheLayer(max_seq_len=32, hidden_dim=128, head_dim=32, compression_rate=8)
    assert (cache.length, cache.n_blocks, cache.h_buf_count) == (0, 0, 0)
    with pytest.raises(ValueError, match="max_seq_len"):
        kv.HCAKVCacheLayer(max_seq_len=0, hidden_dim=8, head_dim=4, compression_rate=2)
    with pytest.raises(ValueError, match="compression_rate"):
        kv.HCAKVCacheLayer(max_seq_len=8, hidden_dim=8, head_dim=4, compression_rate=0)
    cache = kv.HCAKVCacheLayer(max_seq_len=4, hidden_dim=8, head_dim=4, compression_rate=2)
    with pytest.raises(RuntimeError, match="overflow"):
        cache.append(torch.randn(1, 5, 8, device=dev), torch.randn(1, 5, 4, device=dev),
                     torch.randn(1, 5, 4, device=dev), compressor=lambda x: x.new_zeros(1, 0, 4))
    cache = kv.HCAKVCacheLayer(max_seq_len=16, hidden_dim=8, head_dim=4, compression_rate=4)
    counter = [0]

    def stub(h):
        counter[0] += 1
        return torch.full((h.shape[0], h.shape[1] // 4, 4), float(counter[0]), device=h.device)

    cache.append(torch.randn(1, 3, 8, device=dev), torch.randn(1, 3, 4, device=dev),
                 torch.randn(1, 3, 4, device=dev), compressor=stub)
    assert cache.h_buf_count == 3 and cache.n_blocks == 0
    comp, sk, sv = cache.append(torch.randn(1, 6, 8, device=dev), torch.randn(1, 6, 4, device=dev),
                                torch.randn(1, 6, 4, device=dev), compressor=stub)
    assert (cache.n_blocks, cache.h_buf_count, cache.length) == (2, 1, 9)
    assert comp.shape == (1, 2, 4) and (comp == 1.0).all()
    with pytest.raises(RuntimeError, match="compressor returned 3 blocks, expected 1"):
        cache.append(torch.randn(1, 3, 8, device=dev), torch.randn(1, 3, 4, device=dev),
                     torch.randn(1, 3, 4, device=dev),
                     compressor=lambda h: torch.zeros(1, 3, 4, device=h.device))


@pytest.mark.parametrize("kind", ["hca", "csa"])
def test_compressed_layers_match_contiguous_reference(dev, kind) -> None:
    kv = _kv()
    g = torch.Generator().manual_seed(1)
    B, H, D, CI, m, T = 2, 64, 32, 16, 4, 60
    comp = _Compressor(H, D, m, 2)
    icomp = _Compressor(H, CI, m, 3)
    dims = [D] if kind == "hca" else [D, CI]
    cont = ref.ContiguousCompressed(T, H, dims, m, batch_size=B)
    if kind == "hca":
        cache = kv.HCAKVCacheLayer(T, H, D, m, batch_size=B)
    else:
        cache = kv.CSAKVCacheLayer(T, H, D, CI, m, batch_size=B)
    calls = []
    for n in (3, 6, 1, 5, 4, 9, 1, 1, 1, 1, 28):
        h = torch.randn(B, n, H, generator=g)
        sk, sv = torch.randn(B, n, D, generator=g), torch.randn(B, n, D, generator=g)
        exp = cont.append(h, sk, sv, [comp] if kind == "hca" else [comp, icomp])
        # the compressors run on the CPU in both paths, so the cache's copies
        # of their outputs must match bit for bit
        def kv_c(x):
            calls.append("kv")
            return comp(x.cpu()).to(dev)

        def ix_c(x):
            calls.append("idx")
            return icomp(x.cpu()).to(dev)

        if kind == "hca":
            got = cache.append(h.to(dev), sk.to(dev), sv.to(dev), compressor=kv_c)
        else:

            got = cache.append(h.to(dev), sk.to(dev), sv.to(dev), compressor=kv_c,
                               indexer_compressor=ix_c)
        assert len(got) == len(exp)
        for a, b in zip(got, exp, strict=True):
            assert a.shape == b.shape
            assert torch.equal(a.cpu(), b)
        assert cache.length == cont.length and cache.n_blocks == cont.n_blocks
        assert cache.h_buf_count == cont.h_buf_count
        assert torch.equal(cache.h_buffer[:, : cache.h_buf_count].cpu(), cont.h_buffer[:, : cont.h_buf_count])
    if kind == "csa":
        assert calls[0::2] == ["kv"] * (len(calls) // 2) and calls[1::2] == ["idx"] * (len(calls) // 2)
    else:
        assert set(calls) == {"kv"}
    cache.reset()
    assert (cache.length, cache.n_blocks, cache.h_buf_count) == (0, 0, 0)


def test_compressed_copy_is_exact(dev) -> None:
    """The compressed views hold exactly the compressor's output (no arithmetic)."""
    kv = _kv()
    cache = kv.CSAKVCacheLayer(max_seq_len=8, hidden_dim=8, head_dim=4, c_indexer=2, compression_rate=4)
    out_kv = torch.randn(1, 2, 4, device=dev)
    out_ix = torch.randn(1, 2, 2, device=dev)
    ckv, cix, sk, sv = cache.append(torch.randn(1, 8, 8, device=dev), torch.randn(1, 8, 4, device=dev),
                                    torch.randn(1, 8, 4, device=dev), compressor=lambda h: out_kv,
                                    indexer_compressor=lambda h: out_ix)
    assert torch.equal(ckv, out_kv) and torch.equal(cix, out_ix) and cache.n_blocks == 2


# ---------- KVCacheBundle (test_kv_cache.py:158-260) ----------
def test_bundle_plumbing(dev) -> None:
    kv = _kv()
    cache = kv.SWAKVCacheLayer(max_seq_len=16, head_dim=8)
    cache.append(torch.randn(1, 3, 8, device=dev), torch.randn(1, 3, 8, device=dev))
    bundle = kv.KVCacheBundle([None, cache, None])
    assert bundle.length == 3 and len(bundle) == 3
    assert bundle.for_layer(1) is cache and bundle.for_layer(0) is None
    assert kv.KVCacheBundle([None, None]).length == 0
    bundle.reset()
    assert bundle.length == 0


def test_bundle_for_model(dev) -> None:
    kv = _kv()

    def att(name):
        return SimpleNamespace(attention=type(name, (), {})())

    cfg = SimpleNamespace(hidden_dim=64, attention=SimpleNamespace(head_dim=32),
                          hca=SimpleNamespace(compression_rate=8),
                          csa=SimpleNamespace(compression_rate=4, indexer_head_dim=16))
    model = SimpleNamespace(cfg=cfg, blocks=[att("SWAttention"), att("SWAttention"), att("CSA"),
                                             att("HCA"), att("CSA"), att("MLPOnly")])
    bundle = kv.KVCacheBundle.for_model(model, max_seq_len=8)
    kinds = [type(bundle.for_layer(i)).__name__ if bundle.for_layer(i) is not None else None
             for i in range(len(bundle))]
    assert kinds == ["SWAKVCacheLayer", "SWAKVCacheLayer", "CSAKVCacheLayer", "HCAKVCacheLayer",
                     "CSAKVCacheLayer", None]
    csa = bundle.for_layer(2)
    assert csa.c_indexer == 16 and csa.compression_rate == 4 and bundle.for_layer(3).compression_rate == 8
