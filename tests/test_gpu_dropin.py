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


def _exact_compressor(hidden: int, c: int, m: int, g: torch.Generator):
    """A TokenLevelCompressor whose projections of integer hidden states in
    [-2, 2] are exact in any summation order (weights in {0, +-1/2, +-1}, at
    most 8 nonzero per output), so that projecting tokens in one call or in
    several gives the same bf16 values."""
    comp = ref.TokenLevelCompressor(hidden, c, m)
    for lin in (comp.w_a_kv, comp.w_b_kv, comp.w_a_z, comp.w_b_z):
        w = torch.zeros(c, hidden)
        for o in range(c):
            cols = torch.randperm(hidden, generator=g)[:8]
            w[o, cols] = torch.tensor([-1.0, -0.5, 0.5, 1.0])[torch.randint(0, 4, (8,), generator=g)]
        lin.weight.data = w
    comp.bias_a.data = torch.randn(m, c, generator=g).to(torch.bfloat16).float()
    comp.bias_b.data = torch.randn(m, c, generator=g).to(torch.bfloat16).float()
    return comp


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_compressor_fast_path_matches_reference_formula(dev, dtype) -> None:
    """A CSA/HCA drop-in layer given TokenLevelCompressor modules runs the
    fast path (two projections + skv_compress_append into the pages): the
    block counts, h-buffer and SW views match the reference state machine,
    and every compressed entry equals the reference pooling formula
    (csa.py:79-87) on the module's own b-branch projections within the
    pooling bound, and the module's forward within 1e-2 in norm (bf16 cache:
    bf16 entries).  An fp32 cache, the reference's default, keeps unrounded
    fp32 entries: within a hundredth of the pooling bound and 1e-5 in norm
    of the module's fp32 forward.  A plain callable mid-block switches that
    append to the reference's call-and-copy path; the next fast append folds
    the buffered tokens first."""
    import copy

    from saint_kv.kv_cache import CSAKVCacheLayer, HCAKVCacheLayer

    g = torch.Generator().manual_seed(0)
    H, D, CI, B = 64, 64, 32, 3
    bf = dtype
    fp32 = dtype == torch.float32
    for m, layer_cls in ((4, CSAKVCacheLayer), (16, HCAKVCacheLayer)):
        kw = {"c_indexer": CI} if layer_cls is CSAKVCacheLayer else {}
        n_streams = 2 if kw else 1
        cpu_comps = [_exact_compressor(H, d, m, g) for d in [D, CI][:n_streams]]
        comps = [copy.deepcopy(c).to(dev, bf) for c in cpu_comps]
        layer = layer_cls(max_seq_len=200, hidden_dim=H, head_dim=D, compression_rate=m, batch_size=B,
                          device=dev, dtype=bf, **kw)
        cont = ref.ContiguousCompressed(200, H, [D, CI][:n_streams], m, batch_size=B, dtype=bf)
        hist_h = []
        for step, n in enumerate((3, 6, 1, 5, 4, 9, 1, 1, 2, 17, 1)):
            h = torch.randint(-2, 3, (B, n, H), generator=g).to(bf).to(dev)
            sk = torch.randn(B, n, D, generator=g).to(bf).to(dev)
            sv = torch.randn(B, n, D, generator=g).to(bf).to(dev)
            hist_h.append(h)
            plain = step == 6  # a plain callable: the reference path for this append
            use = [(lambda x, c=c: c(x)) if plain else c for c in comps]
            args = {"compressor": use[0]}
            if kw:
                args["indexer_compressor"] = use[1]
            out = layer.append(h, sk, sv, **args)
            with torch.no_grad():
                want = cont.append(h.cpu(), sk.cpu(), sv.cpu(),
                                   [lambda x, c=c: c(x.float()).to(dtype) for c in cpu_comps])
            assert layer.n_blocks == cont.n_blocks and layer.h_buf_count == cont.h_buf_count
            assert layer.length == cont.length
            assert torch.equal(out[-2].cpu(), want[-2]) and torch.equal(out[-1].cpu(), want[-1])
            assert torch.equal(layer.h_buffer[:, :layer.h_buf_count].cpu(), cont.h_buffer[:, :cont.h_buf_count])
        assert layer.fast_appends == 10
        allh = torch.cat(hist_h, dim=1).cpu().float()
        nb = layer.n_blocks
        for si, c in enumerate(cpu_comps):
            got = out[si].float().cpu()
            hh = allh[:, : nb * m]
            with torch.no_grad():
                cz = c.w_b_kv(hh).view(B, nb, m, -1)  # exact, and exact in bf16
                zz = c.w_b_z(hh).view(B, nb, m, -1)
            want_f = ref.compress_pool(cz, zz, c.bias_b)
            bound = ref.pooling_bound(cz, zz, c.bias_b) / (100 if fp32 else 1)
            assert ((got - want_f).abs() <= bound).all(), (m, si, float((got - want_f).abs().max()))
            # the module's bf16 forward rounds at every op: within 1e-2 in norm
            with torch.no_grad():
                mod = comps[si](hh.to(bf).to(dev)).float().cpu()
            assert float((got - mod).norm() / mod.norm()) < (1e-5 if fp32 else 1e-2)


def test_compressor_fast_path_only_for_the_reference_forward(dev) -> None:
    """The fast path runs only when calling the module would run
    TokenLevelCompressor.forward and nothing else: a subclass that overrides
    forward, or a module with a forward hook, is called as the reference
    calls it (kv_cache.py:182-189), and its own outputs become the entries."""
    from saint_kv.kv_cache import HCAKVCacheLayer

    class Doubled(ref.TokenLevelCompressor):
        def forward(self, h):
            return 2.0 * super().forward(h)

    g = torch.Generator().manual_seed(4)
    H, D, m, B = 32, 16, 4, 2
    plain = ref.TokenLevelCompressor(H, D, m)
    hooked = ref.TokenLevelCompressor(H, D, m)
    hooked.register_forward_hook(lambda mod, args, out: out + 1.0)
    for comp, scale, shift in ((Doubled(H, D, m), 2.0, 0.0), (hooked, 1.0, 1.0)):
        comp.load_state_dict(plain.state_dict())
        comp = comp.to(dev)
        layer = HCAKVCacheLayer(max_seq_len=64, hidden_dim=H, head_dim=D, compression_rate=m, batch_size=B,
                                device=dev)
        h = torch.randn(B, 12, H, generator=g)
        out, _, _ = layer.append(h.to(dev), torch.zeros(B, 12, D, device=dev), torch.zeros(B, 12, D, device=dev),
                                 compressor=comp)
        assert layer.fast_appends == 0
        with torch.no_grad():
            want = scale * plain(h) + shift
        torch.testing.assert_close(out.cpu(), want, rtol=1e-5, atol=1e-5)


def test_compressor_fast_path_fp32_module_into_bf16_cache(dev) -> None:
    """An fp32 TokenLevelCompressor feeding a bf16 cache, one token per append
    (every block spans appends): the reference pools in fp32, sees buffered
    tokens rounded to bf16 (its h_buffer) and rounds the entry once when it
    copies it into its cache.  The fast path pools the fp32 projections of
    the same token values: every entry within the pooling bound of the
    oracle's pooling of those projections, elementwise."""
    from saint_kv.kv_cache import HCAKVCacheLayer

    g = torch.Generator().manual_seed(6)
    H, D, m, B, T = 48, 32, 4, 3, 22
    comp = ref.TokenLevelCompressor(H, D, m)
    with torch.no_grad():
        comp.bias_b.copy_(torch.randn(m, D, generator=g))
    layer = HCAKVCacheLayer(max_seq_len=64, hidden_dim=H, head_dim=D, compression_rate=m, batch_size=B,
                            device=dev, dtype=torch.bfloat16)
    mod = comp.to(dev)
    h = torch.randn(B, T, H, generator=g)
    for i in range(T):
        out, _, _ = layer.append(h[:, i:i + 1].to(dev), torch.zeros(B, 1, D, device=dev),
                                 torch.zeros(B, 1, D, device=dev), compressor=mod)
    assert layer.fast_appends == T
    nb = T // m
    # the token values the reference's compressor sees: every token but the
    # last of its block was buffered (bf16), the last came in h_new (fp32)
    seen = h[:, : nb * m].clone().view(B, nb, m, H)
    seen[:, :, : m - 1] = seen[:, :, : m - 1].to(torch.bfloat16).float()
    with torch.no_grad():
        cz, zz = comp.cpu().w_b_kv(seen), comp.w_b_z(seen)
        want = ref.compress_pool(cz, zz, comp.bias_b)
        bound = ref.pooling_bound(cz, zz, comp.bias_b)
    got = out[:, :nb].float().cpu()
    assert ((got - want).abs() <= bound).all(), float((got - want).abs().max())
