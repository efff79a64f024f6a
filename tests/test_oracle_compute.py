"""Pin the oracle's pooling, top-k, sparse gather and FP8 codec (CPU only).

Every check fixes the oracle by something other than its own formula: closed
forms, brute force, the reference's torch formulation (topk / gather / cast),
and the special cases the reference's own tests assert.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref


# ---------------------------------------------------------------- pooling ----
def test_pool_uniform_weights_is_token_mean() -> None:
    g = torch.Generator().manual_seed(0)
    c = torch.randn(5, 4, 16, generator=g)
    # z varies across channels but not across the m tokens -> softmax over
    # tokens is uniform; a softmax over the wrong axis would not give the mean
    z = torch.randn(5, 1, 16, generator=g).expand(5, 4, 16)
    out = ref.compress_pool(c, z, torch.zeros(4, 16))
    assert torch.allclose(out, c.mean(dim=1), atol=1e-6)


def test_pool_one_hot_selects_token() -> None:
    g = torch.Generator().manual_seed(1)
    c = torch.randn(3, 8, 32, generator=g)
    pick = torch.randint(0, 8, (3, 32), generator=g)
    z = torch.zeros(3, 8, 32)
    z.scatter_(1, pick.unsqueeze(1), 120.0)
    out = ref.compress_pool(c, z, torch.zeros(8, 32))
    assert torch.allclose(out, torch.gather(c, 1, pick.unsqueeze(1)).squeeze(1), atol=1e-6)


def test_pool_bias_is_per_token_and_channel() -> None:
    g = torch.Generator().manual_seed(2)
    c = torch.randn(2, 4, 8, generator=g)
    bias = torch.full((4, 8), -1e4)
    bias[2] = 0.0  # only token 2 survives
    out = ref.compress_pool(c, torch.zeros(2, 4, 8), bias)
    assert torch.allclose(out, c[:, 2], atol=1e-6)


def test_pool_m1_is_identity() -> None:
    c = torch.randn(4, 1, 8)
    assert torch.equal(ref.compress_pool(c, torch.randn(4, 1, 8), torch.randn(1, 8)), c[:, 0])


def test_pool_brute_force() -> None:
    rng = np.random.default_rng(3)
    m, ch = 4, 6
    c = rng.standard_normal((m, ch))
    z = rng.standard_normal((m, ch))
    bias = rng.standard_normal((m, ch))
    expect = np.zeros(ch)
    for j in range(ch):
        e = [math.exp(z[i, j] + bias[i, j]) for i in range(m)]
        expect[j] = sum(e[i] / sum(e) * c[i, j] for i in range(m))
    got = ref.compress_pool(torch.tensor(c), torch.tensor(z), torch.tensor(bias))
    assert np.allclose(got.numpy(), expect, rtol=1e-6, atol=1e-7)


def test_pool_bf16_module_rounding_within_tolerance() -> None:
    """The reference's all-bf16 op sequence (every op rounded to bf16) stays within
    1e-2 relative of the fp32 pooling in norm; single channels whose weighted terms
    cancel can be off by a few bf16 ulps of the largest term, which bounds the
    elementwise gap at 3e-2."""
    g = torch.Generator().manual_seed(4)
    for m in (4, 128):
        c = torch.randn(64, m, 576, generator=g).to(torch.bfloat16)
        z = torch.randn(64, m, 576, generator=g).to(torch.bfloat16)
        bias = torch.randn(m, 576, generator=g)
        fp32 = ref.compress_pool(c, z, bias)
        mod = ref.compress_pool_bf16_module(c, z, bias).float()
        assert ((mod - fp32).norm() / fp32.norm()) < 1e-2
        assert (mod - fp32).abs().max() < 3e-2


def test_paged_compression_matches_contiguous_state_machine() -> None:
    """Per-token (c, z) staging + paged emission == the reference's h-buffer +
    compressor replay (kv_cache.py:170-195), chunk sizes 3, 6, 1, 5, 4, 9."""
    g = torch.Generator().manual_seed(5)
    B, H, C, m, bs = 2, 16, 8, 4, 4
    wc, wz = torch.randn(H, C, generator=g), torch.randn(H, C, generator=g)
    bias = torch.randn(m, C, generator=g)

    def compressor(h):  # TokenLevelCompressor shape: (B, n*m, H) -> (B, n, C)
        b, t, _ = h.shape
        cz = (h @ wc).view(b, t // m, m, C), (h @ wz).view(b, t // m, m, C)
        return ref.compress_pool(cz[0], cz[1], bias)

    cont = ref.ContiguousCompressed(64, H, [C], m, batch_size=B)
    stack, top = ref.free_stack_init(32, np.random.default_rng(5).permutation(32))
    bt = np.full((B, 8), -1, dtype=np.int32)
    n_ent = np.zeros(B, dtype=np.int32)
    pool = torch.zeros(32, bs, C, dtype=torch.bfloat16)
    tail_c = torch.zeros(B, m, C, dtype=torch.bfloat16)
    tail_z = torch.zeros(B, m, C, dtype=torch.bfloat16)
    L = 0
    for n in (3, 6, 1, 5, 4, 9):
        h = torch.randn(B, n, H, generator=g)
        comp, _, _ = cont.append(h, h[..., :C], h[..., :C], [compressor])
        new_entries = (L + n) // m - L // m
        st, top = ref.reserve(stack, top, bt, n_ent, new_entries, bs)
        assert st == 0
        L += n
        ref.compress_append(pool, bt, tail_c, tail_z, (h @ wc).to(torch.bfloat16),
                            (h @ wz).to(torch.bfloat16), bias,
                            np.full(B, L, dtype=np.int32), n)
        assert cont.n_blocks == L // m and int(n_ent[0]) == L // m
        got = torch.zeros(B, L // m, C, dtype=torch.bfloat16)
        ref.paged_gather(pool, bt, n_ent, got)
        # c, z rounded to bf16 before pooling + bf16 output: within the 1e-2 budget
        torch.testing.assert_close(got.float(), comp, rtol=2e-2, atol=2e-2)


# --------------------------------------------------------- indexer scores ----
def _indexer_inputs(b=2, t=3, h=4, c=16, n=5, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((b, t, h, c)), rng.standard_normal((b, n, c)), rng.standard_normal((b, t, h)))


def test_indexer_scores_brute_force() -> None:
    """attention.py:47-50 written out as plain loops."""
    q, k, w = _indexer_inputs()
    got = ref.indexer_scores(q, k, w)
    b, t, h, c = q.shape
    n = k.shape[1]
    assert got.shape == (b, t, n)
    for bi in range(b):
        for ti in range(t):
            for s in range(n):
                tot = 0.0
                for hi in range(h):
                    dot = sum(float(q[bi, ti, hi, ci]) * float(k[bi, s, ci]) for ci in range(c))
                    tot += float(w[bi, ti, hi]) * max(dot, 0.0)
                assert math.isclose(got[bi, ti, s], tot, rel_tol=1e-12, abs_tol=1e-12)


def test_indexer_scores_non_negative_with_positive_weights() -> None:
    """test_lightning_indexer.py:37-43: ReLU before weighting, so all-positive
    head weights give non-negative scores; negative weights may not."""
    q, k, _ = _indexer_inputs(seed=1)
    assert (ref.indexer_scores(q, k, np.ones(q.shape[:3])) >= 0).all()
    assert (ref.indexer_scores(q, k, -np.ones(q.shape[:3])) <= 0).all()


def test_indexer_scores_special_cases() -> None:
    """One head: w * relu(q.k); negative dots contribute nothing whatever the
    weight; orthogonal keys score 0; the weights are linear."""
    q = np.zeros((1, 1, 2, 4))
    q[0, 0, 0] = [1, 2, 0, 0]
    q[0, 0, 1] = [0, 0, 3, 0]
    k = np.array([[[1, 1, 0, 0], [-1, -1, 0, 0], [0, 0, 0, 5], [0, 0, 2, 0]]], dtype=np.float64)
    w = np.array([[[2.0, -0.5]]])
    got = ref.indexer_scores(q, k, w)[0, 0]
    # entry 0: head0 dot 3 -> 6, head1 dot 0; entry 1: head0 dot -3 -> 0;
    # entry 2: orthogonal to both; entry 3: head1 dot 6 * -0.5
    assert got.tolist() == [6.0, 0.0, 0.0, -3.0]
    q2, k2, w2 = _indexer_inputs(seed=2)
    np.testing.assert_allclose(ref.indexer_scores(q2, k2, 3.0 * w2), 3.0 * ref.indexer_scores(q2, k2, w2),
                               rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ top-k ----
def test_topk_equals_torch_topk_on_distinct_scores() -> None:
    rng = np.random.default_rng(6)
    for n, k in ((64, 16), (1000, 512), (37, 100)):
        s = rng.standard_normal((9, n)).astype(np.float32)
        nv = rng.integers(0, n + 1, size=9)
        got = ref.topk_select(s, nv, k, n)
        exp = ref.topk_select_torch(torch.from_numpy(s), nv, k, n).numpy()
        assert np.array_equal(got, exp)


def test_topk_causal_geometry() -> None:
    """kernels/attention.py:53-57 with t=8, n_blocks=4, m=2 (test_lightning_indexer.py:68-78)."""
    mask = np.array([[s < ref.n_valid_blocks(q, 2) for s in range(4)] for q in range(8)])
    assert not mask[0].any()
    assert mask[2, 0] and not mask[2, 1]
    assert mask[7, :3].all() and not mask[7, 3]
    for q in range(40):
        for s in range(20):
            assert (s < ref.n_valid_blocks(q, 4)) == (s * 4 + 3 < q)


def test_topk_picks_are_causal_and_padded() -> None:
    """test_lightning_indexer.py:96-130 behaviours at every query position."""
    rng = np.random.default_rng(7)
    n_blocks, m, k = 8, 4, 5
    for q in range(32):
        s = rng.standard_normal((1, n_blocks)).astype(np.float32)
        nv = np.array([ref.n_valid_blocks(q, m)])
        out = ref.topk_select(s, nv, k, n_blocks)[0]
        picks = [i for i in out.tolist() if i >= 0]
        assert len(picks) == min(k, int(nv[0]))
        assert all(p * m + m - 1 < q for p in picks)
        assert (out[len(picks):] == -1).all()
    assert ref.topk_select(np.zeros((2, 0), np.float32), np.array([0, 0]), 4, 0).shape == (2, 0)
    assert ref.topk_select(np.zeros((2, 3), np.float32), np.array([3, 3]), 5, 2).shape == (2, 2)


def test_topk_ties_and_non_finite() -> None:
    s = np.zeros((1, 10), dtype=np.float32)
    assert ref.topk_select(s, np.array([10]), 4, 10)[0].tolist() == [0, 1, 2, 3]
    s = np.array([[1.0, np.nan, 3.0, np.inf, -np.inf, 2.0, -0.0, 0.0]], dtype=np.float32)
    out = ref.topk_select(s, np.array([8]), 8, 8)[0].tolist()
    # NaN ranks first, then +inf; both are non-finite -> -1 (isfinite, csa.py:421)
    assert out == [-1, -1, 2, 5, 0, 6, 7, -1]
    exp = ref.topk_select_torch(torch.from_numpy(s), np.array([8]), 8, 8)[0].tolist()
    assert sorted(out) == sorted(exp)


def test_sparse_gather_matches_reference_formula() -> None:
    g = torch.Generator().manual_seed(8)
    rng = np.random.default_rng(8)
    B, nb, d, bs = 3, 40, 16, 8
    comp = torch.randn(B, nb, d, generator=g)
    stack, top = ref.free_stack_init(64, rng.permutation(64))
    bt = np.full((B, 8), -1, dtype=np.int32)
    lens = np.zeros(B, dtype=np.int32)
    ref.reserve(stack, top, bt, lens, nb, bs)
    pool = torch.zeros(64, bs, d)
    ref.paged_append(pool, bt, lens, comp, nb)
    idx = torch.from_numpy(rng.integers(-1, nb, size=(B, 1, 12)))
    expect = ref.contiguous_sparse_gather(comp, idx)[:, 0]
    got = torch.zeros(B, 12, d)
    ref.topk_gather(pool, bt, np.arange(B), idx[:, 0].numpy(), got)
    assert torch.equal(got, expect)
    assert torch.equal(got[idx[:, 0] == -1], comp[:, 0].unsqueeze(1).expand(B, 12, d)[idx[:, 0] == -1])


# -------------------------------------------------------------------- FP8 ----
def test_fp8_format_constants() -> None:
    assert torch.finfo(torch.float8_e4m3fn).max == ref.E4M3_MAX == 448.0
    assert ref.FP8_ENTRY_BYTES == 656


def test_fp8_zero_block_and_saturation() -> None:
    codes, scales = ref.fp8_quantize_blocks(torch.zeros(2, 128))
    assert (codes == 0).all() and (scales == ref.FLT_MIN).all()
    assert (ref.fp8_dequantize_blocks(codes, scales) == 0).all()
    x = torch.zeros(1, 128)
    x[0, :5] = torch.tensor([0.0, 100.0, 1000.0, 1e6, -1e6])
    codes, scales = ref.fp8_quantize_blocks(x)
    assert codes[0, 3] == 0x7E and codes[0, 4] == 0xFE  # +-448
    assert torch.isfinite(ref.fp8_dequantize_blocks(codes, scales).float()).all()


def test_fp8_roundtrip_budget_and_scale_axis() -> None:
    g = torch.Generator().manual_seed(9)
    x = torch.randn(64, 512, generator=g) * 3.0
    codes, scales = ref.fp8_quantize_blocks(x)
    assert scales.shape == (64, 4)
    deq = ref.fp8_dequantize_blocks(codes, scales).float()
    err = (deq - x).abs() / x.abs().clamp(min=1e-3)
    assert err.median() < 0.20  # test_quant_fp8.py:26-41
    # per-block scale = amax/448 of exactly that block of 128
    assert torch.equal(scales[:, 1], (x[:, 128:256].abs().amax(1) / 448.0).clamp(min=ref.FLT_MIN))


def test_fp8_entry_pack_layout() -> None:
    g = torch.Generator().manual_seed(10)
    x = torch.randn(7, 576, generator=g).to(torch.bfloat16)
    e = ref.fp8_pack_entries(x)
    assert e.shape == (7, 656) and e.dtype == torch.uint8
    assert torch.equal(e[:, 528:].contiguous().view(torch.bfloat16), x[:, 512:])
    back = ref.fp8_unpack_entries(e)
    assert torch.equal(back[:, 512:], x[:, 512:])
    assert ((back[:, :512].float() - x[:, :512].float()).abs() <= x[:, :512].float().abs() * 0.07 + 1e-2).all()


def _e4m3_all_values() -> torch.Tensor:
    return torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()


def test_library_codec_decode_matches_torch_on_all_codes() -> None:
    from saint_kv import ops

    codes = torch.arange(256, dtype=torch.uint8)
    got = ops.fp8_decode_host(codes)
    exp = _e4m3_all_values()
    nan = torch.isnan(exp)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan], exp[~nan])


def test_library_codec_encode_matches_torch_exhaustively() -> None:
    """All 65536 bf16 patterns (clamped as the quantiser does), every e4m3 value,
    every midpoint between neighbours and its fp32 neighbours, 2M random floats."""
    from saint_kv import ops

    bf = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    bf = bf[torch.isfinite(bf)].clamp(-448.0, 448.0)
    vals = _e4m3_all_values()
    pos = torch.unique(vals[torch.isfinite(vals) & (vals >= 0)])
    mids = (pos[1:] + pos[:-1]) / 2
    up = torch.nextafter(mids, torch.full_like(mids, 1e9))
    dn = torch.nextafter(mids, torch.full_like(mids, -1e9))
    g = torch.Generator().manual_seed(11)
    rnd = (torch.rand(2_000_000, generator=g) * 2 - 1) * torch.exp2(torch.randint(-14, 10, (2_000_000,), generator=g).float())
    x = torch.cat([bf, pos, -pos, mids, -mids, up, -up, dn, -dn, rnd.clamp(-448, 448)])
    got = ops.fp8_encode_host(x)
    exp = x.to(torch.float8_e4m3fn).view(torch.uint8)
    bad = (got != exp).nonzero()
    assert bad.numel() == 0, [(float(x[i]), int(got[i]), int(exp[i])) for i in bad[:5, 0]]


def test_pooling_bound_covers_reordering_and_catches_a_dropped_term() -> None:
    """ref.pooling_bound holds the fp32 pooling of another summation order and
    exp (fp64 reference, reversed fp32 order) and is violated by a planted
    mistake: one token's term dropped, or the bias ignored."""
    g = torch.Generator().manual_seed(4)
    for m in (4, 128):
        c = torch.randn(64, m, 576, generator=g).to(torch.bfloat16)
        z = torch.randn(64, m, 576, generator=g).to(torch.bfloat16)
        bias = torch.randn(m, 576, generator=g)
        want = ref.compress_pool(c, z, bias)
        bound = ref.pooling_bound(c, z, bias)
        w64 = torch.softmax(z.double() + bias.double(), dim=-2)
        exact = (w64 * c.double()).sum(dim=-2)
        rev = (torch.softmax(z.float().flip(-2) + bias.flip(-2), dim=-2) * c.float().flip(-2)).sum(dim=-2)
        for got in (exact.float(), rev, rev.to(torch.bfloat16).float()):
            assert ((got - want).abs() <= bound).all()
        dropped = (w64[:, 1:] * c.double()[:, 1:]).sum(dim=-2).float()
        no_bias = ref.compress_pool(c, z, torch.zeros_like(bias))
        for bad in (dropped, no_bias):
            assert ((bad - want).abs() > bound).float().mean() > 0.5


def test_pooling_bound_rounded_inputs_covers_bf16_projections() -> None:
    """ref.pooling_bound_rounded_inputs holds the pooling of projections
    rounded to bf16 (and of ones pushed a whole bf16 ulp either way, as a
    GEMM that sums in another order may round them), measured against the
    pooling of the exact fp32 projections, elementwise; a planted mistake (the
    bias ignored; at m <= 8 a dropped token, which at m = 128 moves an entry
    by about a 128th of a term) still violates it on most channels."""
    g = torch.Generator().manual_seed(5)
    for m in (2, 8, 128):
        c = torch.randn(32, m, 64, generator=g) * 3
        z = torch.randn(32, m, 64, generator=g)
        bias = torch.randn(m, 64, generator=g).to(torch.bfloat16).float()
        want = ref.compress_pool(c, z, bias)
        bound = ref.pooling_bound_rounded_inputs(c, z, bias)
        cb, zb = c.to(torch.bfloat16).float(), z.to(torch.bfloat16).float()
        ulp = lambda t: t.abs() * ref.BF16_ULP  # noqa: E731
        sign = lambda: torch.randint(0, 2, c.shape, generator=g).float() * 2 - 1  # noqa: E731
        for cc, zz in ((cb, zb), (cb + sign() * ulp(cb), zb + sign() * ulp(zb))):
            got = ref.compress_pool(cc, zz, bias).to(torch.bfloat16).float()
            assert ((got - want).abs() <= bound).all(), m
        w = torch.softmax(z + bias, dim=-2)
        dropped = (w[:, 1:] * c[:, 1:]).sum(dim=-2)
        no_bias = ref.compress_pool(c, z, torch.zeros_like(bias))
        for bad in ((dropped, no_bias) if m <= 8 else (no_bias,)):
            assert ((bad - want).abs() > bound).float().mean() > 0.5, m


def test_token_level_compressor_restatement_pools_its_b_branch() -> None:
    """The oracle TokenLevelCompressor equals compress_pool of its own b-branch
    projections (the formula the fast path of the drop-in uses), ignores its
    a-branch, drops an incomplete trailing block and returns no block for
    fewer than m tokens."""
    g = torch.Generator().manual_seed(9)
    comp = ref.TokenLevelCompressor(24, 16, 4)
    for p in comp.parameters():
        p.data = torch.randn(p.shape, generator=g)
    h = torch.randn(2, 11, 24, generator=g)
    out = comp(h)
    assert out.shape == (2, 2, 16)
    c = comp.w_b_kv(h[:, :8]).view(2, 2, 4, 16)
    z = comp.w_b_z(h[:, :8]).view(2, 2, 4, 16)
    torch.testing.assert_close(out, ref.compress_pool(c, z, comp.bias_b), rtol=1e-6, atol=1e-6)
    comp.w_a_kv.weight.data.zero_()
    comp.bias_a.data.fill_(5.0)
    torch.testing.assert_close(comp(h), out)
    assert comp(h[:, :3]).shape == (2, 0, 16)
