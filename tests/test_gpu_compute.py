"""GPU parity of the SWA ring, compression pooling, FP8 codec, indexer scores,
top-k select, top-k gather, release and compaction against the CPU oracle.

Bit-exact for indices, tables, copies and FP8 codes; pooled values (bf16)
within 1e-2 relative of the fp32 oracle plus the oracle's cancellation term
(ref.pooling_bound: 1e-4 of the sum of the weighted magnitudes).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu



def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def _i32(a, dev) -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, dtype=np.int32), device=dev)


# ------------------------------------------------------------------- ring ----
def test_ring_append_read_ragged(dev) -> None:
    from saint_kv import ops

    g = torch.Generator().manual_seed(0)
    batch, w, d = 5, 128, 576
    ring = torch.zeros(batch, w, d, dtype=torch.bfloat16, device=dev)
    r_ring = torch.zeros(batch, w, d, dtype=torch.bfloat16)
    lens = np.zeros(batch, dtype=np.int32)
    for n_step in ([3, 0, 130, 1, 64], [1, 1, 1, 1, 1], [300, 7, 0, 128, 2], [1, 0, 1, 0, 1]):
        n = np.array(n_step, dtype=np.int32)
        src = torch.randn(batch, int(n.max()), d, generator=g).to(torch.bfloat16)
        before = lens.copy()
        lens = lens + n
        ops.ring_append(ring, _i32(lens, dev), src.to(dev), _i32(n, dev))
        ref.ring_append(r_ring, before, src, n)
        out = torch.zeros(batch, w, d, dtype=torch.bfloat16, device=dev)
        ops.ring_read(ring, _i32(lens, dev), out)
        r_out = ref.ring_read(r_ring, lens, torch.zeros(batch, w, d, dtype=torch.bfloat16))
        torch.cuda.synchronize()
        assert torch.equal(ring.cpu(), r_ring)
        assert torch.equal(out.cpu(), r_out)


# ---------------------------------------------------------------- pooling ----
def _compress_case(dev, batch, m, channels, chunks, fp8, seed):
    from saint_kv import ops

    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    bs, n_pages, max_pages = 16, 256, 64
    order = rng.permutation(n_pages).astype(np.int32)
    stack = torch.empty(n_pages, dtype=torch.int32, device=dev)
    top = torch.empty(1, dtype=torch.int32, device=dev)
    ops.free_stack_init(stack, top, _i32(order, dev))
    bt = torch.full((batch, max_pages), -1, dtype=torch.int32, device=dev)
    n_ent = torch.zeros(batch, dtype=torch.int32, device=dev)
    r_stack, r_top = ref.free_stack_init(n_pages, order)
    r_bt = np.full((batch, max_pages), -1, dtype=np.int32)
    r_ent = np.zeros(batch, dtype=np.int32)
    row = ref.FP8_ENTRY_BYTES if fp8 else channels
    dt = torch.uint8 if fp8 else torch.bfloat16
    pool = torch.zeros(n_pages, bs, row, dtype=dt, device=dev)
    pool_bf = torch.zeros(n_pages, bs, channels, dtype=torch.bfloat16, device=dev)
    r_pool = torch.zeros(n_pages, bs, channels, dtype=torch.bfloat16)
    r_bound = torch.zeros(n_pages, bs, channels, dtype=torch.float32)
    state = [torch.zeros(batch, 3, channels, dtype=torch.float32, device=dev) for _ in range(2)]
    r_tc = torch.zeros(batch, m, channels, dtype=torch.bfloat16)
    r_tz = torch.zeros(batch, m, channels, dtype=torch.bfloat16)
    bias = torch.randn(m, channels, generator=g)
    lens = np.zeros(batch, dtype=np.int32)
    for n_step in chunks:
        n = np.asarray(n_step, dtype=np.int32)
        t = max(int(n.max()), 1)
        c = torch.randn(batch, t, channels, generator=g).to(torch.bfloat16)
        z = torch.randn(batch, t, channels, generator=g).to(torch.bfloat16)
        new_ent = (lens + n) // m - lens // m
        lens = lens + n
        ops.reserve(stack, top, bt, n_ent, _i32(new_ent, dev), bs)
        r_status, r_top = ref.reserve(r_stack, r_top, r_bt, r_ent, new_ent, bs)
        assert r_status == 0
        # same staging, two formats: the fp8 run must quantize the bf16 run's values
        ops.compress_append(pool_bf, bt, state[0], c.to(dev), z.to(dev), bias.to(dev),
                            _i32(lens, dev), _i32(n, dev))
        ops.compress_append(pool, bt, state[1], c.to(dev), z.to(dev), bias.to(dev),
                            _i32(lens, dev), _i32(n, dev))
        ref.compress_append(r_pool, r_bt, r_tc, r_tz, c, z, bias, lens, n, bound_pool=r_bound)
    torch.cuda.synchronize()
    assert np.array_equal(_np(bt), r_bt) and np.array_equal(_np(n_ent), r_ent)
    # the carried state of each incomplete block pools (acc / sum) to the
    # oracle's pooling of that block's buffered tokens
    assert torch.equal(state[0].cpu(), state[1].cpu())
    for b in range(batch):
        r = int(lens[b]) % m
        if r:
            part = ref.compress_pool(r_tc[b, :r], r_tz[b, :r], bias[:r])
            st = state[0][b].cpu()
            torch.testing.assert_close(st[2] / st[1], part, rtol=1e-4, atol=1e-4)
    got = torch.zeros(batch, int(r_ent.max()), channels, dtype=torch.bfloat16, device=dev)
    ops.paged_gather(pool_bf, bt, n_ent, got)
    exp = ref.paged_gather(r_pool, r_bt, r_ent, torch.zeros(got.shape, dtype=torch.bfloat16))
    bound = ref.paged_gather(r_bound, r_bt, r_ent, torch.zeros(got.shape, dtype=torch.float32))
    err = (got.cpu().float() - exp.float()).abs()
    assert (err <= bound).all(), float((err - bound).max())
    if fp8:
        live = ref.live_pages(r_bt, r_ent, bs)
        q_exp = ref.fp8_pack_entries(pool_bf.cpu()[live].reshape(-1, channels))
        # only filled slots of each live page are compared
        filled = torch.zeros(len(live), bs, dtype=torch.bool)
        k = 0
        for b in range(batch):
            for j in range(int(-(-r_ent[b] // bs))):
                filled[k, : min(bs, int(r_ent[b]) - j * bs)] = True
                k += 1
        assert torch.equal(pool.cpu()[live].reshape(-1, row)[filled.reshape(-1)],
                           q_exp[filled.reshape(-1)])
    return r_ent


@pytest.mark.parametrize("m,channels", [(4, 128), (4, 576), (128, 576)])
def test_compress_decode_steps(dev, m, channels) -> None:
    steps = [[1] * 3] * (3 * m + 5)
    ent = _compress_case(dev, 3, m, channels, steps, fp8=False, seed=m + channels)
    assert ent.tolist() == [(3 * m + 5) // m] * 3


def test_compress_ragged_chunks_fp8(dev) -> None:
    chunks = [[3, 0, 9], [6, 4, 1], [1, 13, 0], [5, 4, 4], [0, 1, 2], [9, 9, 9]]
    _compress_case(dev, 3, 4, 576, chunks, fp8=True, seed=7)


def test_compress_long_prefill_hca(dev) -> None:
    _compress_case(dev, 2, 128, 576, [[700, 333], [1, 1], [200, 5]], fp8=True, seed=8)


# -------------------------------------------------------------------- FP8 ----
def test_fp8_quant_append_bit_exact(dev) -> None:
    from saint_kv import ops

    g = torch.Generator().manual_seed(12)
    batch, bs, n_pages, n = 4, 8, 64, 37
    x = torch.randn(batch, n, 576, generator=g)
    outl = torch.rand(batch, n, 576, generator=g) < 0.01
    x = torch.where(outl, x * 20, x)
    x[0, 0, :128] = 0.0                      # zero block -> scale FLT_MIN, codes 0
    x[1, 2, 128:256] *= 1e-30                # subnormal-range codes
    x[2, 3, 256:384] = 3e38                  # huge but finite
    x = x.to(torch.bfloat16)
    stack = torch.empty(n_pages, dtype=torch.int32, device=dev)
    top = torch.empty(1, dtype=torch.int32, device=dev)
    ops.free_stack_init(stack, top)
    bt = torch.full((batch, 8), -1, dtype=torch.int32, device=dev)
    lens = torch.zeros(batch, dtype=torch.int32, device=dev)
    ops.reserve(stack, top, bt, lens, n, bs)
    pool = torch.zeros(n_pages, bs, 656, dtype=torch.uint8, device=dev)
    ops.fp8_quant_append(pool, bt, lens, x.to(dev), n)
    torch.cuda.synchronize()
    got = torch.zeros(batch, n, 656, dtype=torch.uint8, device=dev)
    ops.paged_gather(pool, bt, lens, got)
    exp = ref.fp8_pack_entries(x.reshape(-1, 576)).reshape(batch, n, 656)
    assert torch.equal(got.cpu(), exp)


def _bf16_in_range(lim: float = 448.0) -> torch.Tensor:
    """Every finite bf16 value x with |x| <= lim (both zeros included)."""
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    f = bits.float()
    return bits[torch.isfinite(f) & (f.abs() <= lim)]


def test_fp8_encode_all_bf16_inputs(dev) -> None:
    """The GPU quantizer over every bf16 value in [-448, 448]: each 128-dim
    block holds a 448 anchor, so its scale is exactly 1 and every other code
    is the encoder's direct output (compared with torch's e4m3fn cast)."""
    from saint_kv import ops

    vals = _bf16_in_range()
    per_block = 127
    n_blocks = -(-vals.numel() // per_block)
    pad = n_blocks * per_block - vals.numel()
    vals = torch.cat([vals, torch.zeros(pad, dtype=torch.bfloat16)]).view(n_blocks, per_block)
    blocks = torch.cat([torch.full((n_blocks, 1), 448.0, dtype=torch.bfloat16), vals], dim=1)
    n_rows = -(-n_blocks // 4)
    blocks = torch.cat([blocks, torch.zeros(n_rows * 4 - n_blocks, 128, dtype=torch.bfloat16)])
    x = torch.cat([blocks.view(n_rows, 512), torch.zeros(n_rows, 64, dtype=torch.bfloat16)], dim=1)
    x = x.view(1, n_rows, 576)
    bs = 8
    n_pages = -(-n_rows // bs)
    stack = torch.empty(n_pages, dtype=torch.int32, device=dev)
    top = torch.empty(1, dtype=torch.int32, device=dev)
    ops.free_stack_init(stack, top)
    bt = torch.full((1, n_pages), -1, dtype=torch.int32, device=dev)
    lens = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.reserve(stack, top, bt, lens, n_rows, bs)
    pool = torch.zeros(n_pages, bs, 656, dtype=torch.uint8, device=dev)
    ops.fp8_quant_append(pool, bt, lens, x.to(dev), n_rows)
    got = torch.zeros(1, n_rows, 656, dtype=torch.uint8, device=dev)
    ops.paged_gather(pool, bt, lens, got)
    exp = ref.fp8_pack_entries(x.reshape(-1, 576)).reshape(1, n_rows, 656)
    assert torch.equal(got.cpu(), exp)


def test_fp8_decode_all_codes(dev) -> None:
    """The GPU dequantizing gather over all 256 e4m3fn codes, at scale 1 and
    at a scale that exercises the product's rounding to bf16 (NaN codes:
    NaN out, payload aside)."""
    from saint_kv import ops

    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    main = torch.cat([codes, codes.flip(0)])  # 512 codes: 4 blocks of 128
    entries = []
    for scale in (1.0, 0.3719):
        sc = torch.full((4,), scale, dtype=torch.float32)
        rope = torch.randn(64, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
        entries.append(torch.cat([main, sc.view(torch.uint8), rope.view(torch.uint8)]))
    pool = torch.stack(entries).view(1, 2, 656).to(dev)
    bt = torch.zeros(1, 1, dtype=torch.int32, device=dev)
    n_ent = torch.full((1,), 2, dtype=torch.int32, device=dev)
    idx = torch.tensor([[0, 1]], dtype=torch.int32, device=dev)
    out = torch.zeros(1, 2, 576, dtype=torch.bfloat16, device=dev)
    ops.topk_gather(pool, bt, n_ent, idx, out, 576)
    exp = ref.fp8_unpack_entries(torch.stack(entries))
    got = out.cpu()[0]
    nan = torch.isnan(exp)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan].view(torch.int16), exp[~nan].view(torch.int16))


# ------------------------------------------------------------------ top-k ----
@pytest.mark.parametrize("multi", [False, True])
@pytest.mark.parametrize("n,k", [(64, 16), (16384, 512), (20000, 1024), (100_000, 1024), (5000, 2048)])
def test_topk_select_distinct(dev, n, k, multi) -> None:
    from saint_kv import ops

    rng = np.random.default_rng(n + k)
    rows = 6
    ws = ops.topk_workspace(rows, dev) if multi else None
    if multi:  # a first call on other data: the workspace must come back clean
        warm = torch.randn(rows, n, device=dev)
        ops.topk_select(warm, _i32(np.full(rows, n), dev), n, k,
                        torch.empty(rows, k, dtype=torch.int32, device=dev), ws)
    s = rng.standard_normal((rows, n)).astype(np.float32)
    n_valid = rng.integers(0, n + 1, size=rows).astype(np.int32)
    n_valid[0], n_valid[1] = n, min(k // 2, n)
    out = torch.full((rows, k), -7, dtype=torch.int32, device=dev)
    ops.topk_select(torch.from_numpy(s).to(dev), _i32(n_valid, dev), n, k, out, ws)
    exp = ref.topk_select(s, n_valid, k, n)
    torch.cuda.synchronize()
    if multi:
        # each row's histogram (2048 words) and list counters (next 4) are back to zero
        wsv = ws.view(rows, -1).cpu()
        assert (wsv[:, :2052] == 0).all()
    got = _np(out)[:, : exp.shape[1]]
    assert np.array_equal(got, exp)
    assert (_np(out)[:, exp.shape[1]:] == -1).all()
    # torch.topk (the reference's routine) picks the same score at every rank;
    # only the order among equal fp32 samples (which occur at this n) may differ
    exp_t = ref.topk_select_torch(torch.from_numpy(s), n_valid, k, n).numpy()
    assert np.array_equal(got == -1, exp_t == -1)
    rows_i = np.arange(rows)[:, None]
    assert np.array_equal(np.where(got >= 0, s[rows_i, np.maximum(got, 0)], 0),
                          np.where(exp_t >= 0, s[rows_i, np.maximum(exp_t, 0)], 0))


@pytest.mark.parametrize("multi", [False, True])
def test_topk_select_ties_nonfinite_ragged_cols(dev, multi) -> None:
    from saint_kv import ops

    rng = np.random.default_rng(13)
    rows, n, k = 5, 40000, 512
    s = rng.standard_normal((rows, n)).astype(np.float32)
    s[0] = 0.0                                              # all ties
    s[1, ::3] = 1.5                                         # many ties at the threshold
    s[2, :10] = [np.nan, np.inf, -np.inf, 0.0, -0.0, np.nan, 5.0, np.inf, -np.inf, 7.0]
    s[3] = np.round(s[3] * 4) / 4                           # heavy ties, in LDS range below
    n_cols = np.array([n, n, 30000, 20000, 100], dtype=np.int32)
    n_valid = np.array([n, 39000, 30000, 20000, 50], dtype=np.int32)
    out = torch.full((rows, k), -7, dtype=torch.int32, device=dev)
    ws = ops.topk_workspace(rows, dev) if multi else None
    ops.topk_select(torch.from_numpy(s).to(dev), _i32(n_valid, dev), _i32(n_cols, dev), k, out, ws)
    torch.cuda.synchronize()
    for r in range(rows):
        exp = ref.topk_select(s[r:r + 1], n_valid[r:r + 1], k, int(n_cols[r]))[0]
        assert np.array_equal(_np(out)[r, : len(exp)], exp), r
        assert (_np(out)[r, len(exp):] == -1).all()


def test_topk_select_multi_threshold_ties(dev) -> None:
    """Duplicates straddling the threshold, few enough for the multi path's tie list."""
    from saint_kv import ops

    rng = np.random.default_rng(21)
    rows, n, k = 4, 30000, 700
    s = rng.standard_normal((rows, n)).astype(np.float32)
    s = np.round(s * 2048) / 2048  # ~1e-3 resolution: many equal keys near the threshold
    ws = ops.topk_workspace(rows, dev)
    out = torch.full((rows, k), -7, dtype=torch.int32, device=dev)
    n_valid = np.array([n, n - 5, 12345, 701], dtype=np.int32)
    ops.topk_select(torch.from_numpy(s).to(dev), _i32(n_valid, dev), n, k, out, ws)
    torch.cuda.synchronize()
    exp = ref.topk_select(s, n_valid, k, n)
    assert np.array_equal(_np(out), exp)


@pytest.mark.parametrize("multi", [False, True])
def test_topk_select_decode_masks(dev, multi) -> None:
    from saint_kv import ops

    rng = np.random.default_rng(14)
    m, k = 4, 512
    lens = np.array([0, 1, 4, 5, 8, 2049, 65536, 12345], dtype=np.int32)
    n = int(lens.max() // m)
    s = rng.standard_normal((len(lens), n)).astype(np.float32)
    out = torch.full((len(lens), k), -7, dtype=torch.int32, device=dev)
    ws = ops.topk_workspace(len(lens), dev) if multi else None
    ops.topk_select_decode(torch.from_numpy(s).to(dev), _i32(lens, dev), m, k, out, ws)
    torch.cuda.synchronize()
    for b, L in enumerate(lens):
        n_cols = int(L) // m
        exp = ref.topk_select(s[b:b + 1], np.array([ref.n_valid_blocks(int(L) - 1, m)]), k, n_cols)[0]
        assert np.array_equal(_np(out)[b, : len(exp)], exp), b
        assert (_np(out)[b, len(exp):] == -1).all()


# ----------------------------------------------------------- top-k gather ----
# --------------------------------------------------------- indexer scores ----
# bf16 products accumulate in fp32: each score is within IDX_RTOL of
# sum_h |w| * sum_c |q k| (the oracle's bound) of the fp64 oracle on the same
# bf16-rounded inputs
IDX_RTOL = 1e-5


@pytest.mark.parametrize("t,h,c", [(1, 64, 128), (1, 4, 16), (3, 20, 40), (2, 17, 128)])
def test_indexer_scores_paged(dev, t, h, c) -> None:
    from saint_kv import ops

    g = torch.Generator().manual_seed(h * 1000 + c)
    batch, bs, n_max = 5, 16, 600
    n_ent = np.array([600, 0, 1, 257, 33], dtype=np.int32)
    bt_stride = -(-n_max // bs)
    n_pages = batch * bt_stride + 3
    perm = np.random.default_rng(h).permutation(n_pages)[:batch * bt_stride].reshape(batch, bt_stride)
    table = perm.astype(np.int32)
    table[3, 5] = -1  # an unmapped page: entries 80..95 of sequence 3 score -inf
    pool = torch.randn(n_pages, bs, c, generator=g).to(torch.bfloat16)
    q = torch.randn(batch, t, h, c, generator=g).to(torch.bfloat16)
    w = torch.randn(batch, t, h, generator=g)
    out = torch.full((batch, t, n_max + 7), float("nan"), device=dev)
    ops.indexer_scores(q.to(dev), w.to(dev), pool.to(dev), _i32(table, dev), _i32(n_ent, dev), out,
                       max_entries=n_max)
    got = _np(out)
    k_seq = np.zeros((batch, n_max, c))
    for b in range(batch):
        for e in range(n_max):
            pg = table[b, e // bs]
            if pg >= 0:
                k_seq[b, e] = pool[pg, e % bs].float().numpy()
    exp = ref.indexer_scores(q.float().numpy(), k_seq, w.numpy())
    bound = ref.indexer_scores_bound(q.float().numpy(), k_seq, w.numpy())
    for b in range(batch):
        n = int(n_ent[b])
        live = np.ones(n, dtype=bool)
        if b == 3:
            live[80:96] = False
            assert (got[b, :, 80:96] == -np.inf).all()
        err = np.abs(got[b, :, :n][:, live] - exp[b, :, :n][:, live])
        assert (err <= IDX_RTOL * bound[b, :, :n][:, live] + 1e-30).all(), (b, float(err.max()))
        assert np.isnan(got[b, :, n:]).all()  # columns past the entry count are untouched


def test_indexer_scores_reference_shape(dev) -> None:
    """lightning_indexer_scores in the reference's call shape (contiguous keys)
    on test_lightning_indexer.py's default sizes, and its positive-weight invariant."""
    from saint_kv.indexer import lightning_indexer_scores

    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 32, 4, 16, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 4, 16, generator=g).to(torch.bfloat16)
    w = torch.randn(2, 32, 4, generator=g)
    got = _np(lightning_indexer_scores(q.to(dev), k.to(dev), w.to(dev)))
    assert got.shape == (2, 32, 4)
    qn, kn, wn = q.float().numpy(), k.float().numpy(), w.numpy()
    err = np.abs(got - ref.indexer_scores(qn, kn, wn))
    assert (err <= IDX_RTOL * ref.indexer_scores_bound(qn, kn, wn) + 1e-30).all()
    pos = _np(lightning_indexer_scores(q.to(dev), k.to(dev), torch.ones(2, 32, 4, device=dev)))
    assert (pos >= 0).all()


@pytest.mark.parametrize("fp8", [False, True])
def test_topk_gather_paged(dev, fp8) -> None:
    from saint_kv import ops

    g = torch.Generator().manual_seed(15)
    rng = np.random.default_rng(15)
    batch, bs, n_pages, k = 4, 64, 400, 96
    ent = np.array([5000, 0, 1, 777], dtype=np.int32)
    stack = torch.empty(n_pages, dtype=torch.int32, device=dev)
    top = torch.empty(1, dtype=torch.int32, device=dev)
    order = rng.permutation(n_pages).astype(np.int32)
    ops.free_stack_init(stack, top, _i32(order, dev))
    bt = torch.full((batch, 100), -1, dtype=torch.int32, device=dev)
    n_ent = torch.zeros(batch, dtype=torch.int32, device=dev)
    ops.reserve(stack, top, bt, n_ent, _i32(ent, dev), bs)
    x = torch.randn(batch, int(ent.max()), 576, generator=g).to(torch.bfloat16)
    if fp8:
        pool = torch.zeros(n_pages, bs, 656, dtype=torch.uint8, device=dev)
        ops.fp8_quant_append(pool, bt, n_ent, x.to(dev), _i32(ent, dev))
    else:
        pool = torch.zeros(n_pages, bs, 576, dtype=torch.bfloat16, device=dev)
        ops.paged_append(pool, bt, n_ent, x.to(dev), _i32(ent, dev))
    idx = np.stack([rng.integers(-1, max(int(e), 1), size=k) for e in ent]).astype(np.int32)
    idx[0, :5] = [-1, 0, 4999, 4998, -1]
    out = torch.full((batch, k, 576), 9.0, dtype=torch.bfloat16, device=dev)
    ops.topk_gather(pool, bt, n_ent, _i32(idx, dev), out, 576)
    torch.cuda.synchronize()
    src = ref.fp8_unpack_entries(ref.fp8_pack_entries(x.reshape(-1, 576))).reshape(x.shape) if fp8 else x
    for b in range(batch):
        for j in range(k):
            e = max(int(idx[b, j]), 0)
            exp = src[b, e] if e < ent[b] else torch.zeros(576, dtype=torch.bfloat16)
            assert torch.equal(out[b, j].cpu(), exp), (b, j)


# ------------------------------------------------------ release / compact ----
def test_release_and_compact(dev) -> None:
    from saint_kv import ops

    g = torch.Generator().manual_seed(16)
    rng = np.random.default_rng(16)
    batch, bs, n_pages = 10, 16, 600
    order = rng.permutation(n_pages).astype(np.int32)
    stack = torch.empty(n_pages, dtype=torch.int32, device=dev)
    top = torch.empty(1, dtype=torch.int32, device=dev)
    ops.free_stack_init(stack, top, _i32(order, dev))
    bt = torch.full((batch, 60), -1, dtype=torch.int32, device=dev)
    lens = torch.zeros(batch, dtype=torch.int32, device=dev)
    r_stack, r_top = ref.free_stack_init(n_pages, order)
    r_bt = np.full((batch, 60), -1, dtype=np.int32)
    r_lens = np.zeros(batch, dtype=np.int32)
    n = rng.integers(1, 900, size=batch).astype(np.int32)
    ops.reserve(stack, top, bt, lens, _i32(n, dev), bs)
    _, r_top = ref.reserve(r_stack, r_top, r_bt, r_lens, n, bs)
    pool_a = torch.randn(n_pages, bs, 128, generator=g).to(torch.bfloat16).to(dev)
    pool_b = torch.randint(0, 255, (n_pages, bs, 656), generator=g, dtype=torch.uint8).to(dev)
    r_pools = [pool_a.cpu(), pool_b.cpu()]
    before = ref.paged_gather(r_pools[0], r_bt, r_lens, torch.zeros(batch, int(n.max()), 128, dtype=torch.bfloat16))
    mask = np.zeros(batch, dtype=np.uint8)
    mask[rng.choice(batch, size=3, replace=False)] = 1
    status = torch.full((1,), -7, dtype=torch.int32, device=dev)
    ops.release(stack, top, bt, lens, torch.as_tensor(mask, device=dev), bs, status)
    st, r_top = ref.release(r_stack, r_top, r_bt, r_lens, mask, bs)
    torch.cuda.synchronize()
    assert st == 0 and int(status.item()) == 0
    assert int(top.item()) == r_top and np.array_equal(_np(stack)[:r_top], r_stack[:r_top])
    assert np.array_equal(_np(bt), r_bt) and np.array_equal(_np(lens), r_lens)
    ws = torch.zeros(3 * n_pages, dtype=torch.int32, device=dev)  # marks zero before the first call
    ws[n_pages:] = -5  # the rest is scratch
    info = torch.zeros(2, dtype=torch.int32, device=dev)
    ops.compact([pool_a, pool_b], bt, lens, bs, stack, top, ws, info)
    r_stack, r_top, moved = ref.compact(r_pools, r_bt, r_lens, bs)
    torch.cuda.synchronize()
    assert np.array_equal(_np(bt), r_bt)
    assert int(top.item()) == r_top and np.array_equal(_np(stack)[:r_top], r_stack[:r_top])
    assert _np(info).tolist() == [len(ref.live_pages(r_bt, r_lens, bs)), moved]
    live = ref.live_pages(r_bt, r_lens, bs)
    assert torch.equal(pool_a.cpu()[live], r_pools[0][live])
    assert torch.equal(pool_b.cpu()[live], r_pools[1][live])
    assert not _np(ws)[:n_pages].any()  # the marks are left zero for the next call
    # a second compaction of the now dense pools moves nothing and changes nothing
    bt_before, top_before = bt.clone(), int(top.item())
    ops.compact([pool_a, pool_b], bt, lens, bs, stack, top, ws, info)
    torch.cuda.synchronize()
    assert _np(info).tolist() == [len(live), 0]
    assert torch.equal(bt, bt_before) and int(top.item()) == top_before
    assert not _np(ws)[:n_pages].any()
    after = torch.zeros_like(before, device=dev)
    ops.paged_gather(pool_a, bt, lens, after)
    for b in range(batch):
        if not mask[b]:
            assert torch.equal(after[b, : n[b]].cpu(), before[b, : n[b]])
    # a double release is refused without touching anything
    ops.release(stack, top, bt, torch.full_like(lens, 10 * n_pages), torch.ones(batch, dtype=torch.uint8, device=dev), bs, status)
    torch.cuda.synchronize()
    assert int(status.item()) in (ref.STATUS_STACK, ref.STATUS_BADARG)
    assert int(top.item()) == r_top


def test_release_and_compact_multi_pass_plan(dev) -> None:
    """Compaction of a 40,000-page pool: ten plan workgroups of 4096 page ids
    each rank their block's holes and movers from the live-page counts of the
    blocks before theirs; n_live is not a multiple of 16 and lies inside a
    block, and the movers and holes span many blocks.  Tables, stack, counts
    and page contents equal the oracle's, and the workspace's marks are zero
    again afterwards."""
    from saint_kv import ops

    rng = np.random.default_rng(40)
    g = torch.Generator().manual_seed(40)
    batch, bs, n_pages, bt_stride = 96, 4, 40_000, 1024
    order = rng.permutation(n_pages).astype(np.int32)
    stack = torch.empty(n_pages, dtype=torch.int32, device=dev)
    top = torch.empty(1, dtype=torch.int32, device=dev)
    ops.free_stack_init(stack, top, _i32(order, dev))
    bt = torch.full((batch, bt_stride), -1, dtype=torch.int32, device=dev)
    lens = torch.zeros(batch, dtype=torch.int32, device=dev)
    r_stack, r_top = ref.free_stack_init(n_pages, order)
    r_bt = np.full((batch, bt_stride), -1, dtype=np.int32)
    r_lens = np.zeros(batch, dtype=np.int32)
    n = rng.integers(1, 4 * bt_stride, size=batch).astype(np.int32)
    while int((-(-n // bs)).sum()) > n_pages - 7:
        n = n * 9 // 10 + 1
    ops.reserve(stack, top, bt, lens, _i32(n, dev), bs)
    st, r_top = ref.reserve(r_stack, r_top, r_bt, r_lens, n, bs)
    assert st == 0
    pool_a = torch.randint(0, 255, (n_pages, bs, 16), generator=g, dtype=torch.uint8)
    pool_b = torch.randn(n_pages, bs, 8, generator=g).to(torch.bfloat16)
    r_pools = [pool_a.clone(), pool_b.clone()]
    pools = [pool_a.to(dev), pool_b.to(dev)]
    mask = np.zeros(batch, dtype=np.uint8)
    mask[rng.choice(batch, size=41, replace=False)] = 1
    status = torch.full((1,), -7, dtype=torch.int32, device=dev)
    ops.release(stack, top, bt, lens, torch.as_tensor(mask, device=dev), bs, status)
    st, r_top = ref.release(r_stack, r_top, r_bt, r_lens, mask, bs)
    assert st == 0
    movers, holes, n_live = ref.compact_plan(r_bt, r_lens, bs, n_pages)
    # the plan's passes: n_live is not a multiple of 16, and movers and holes
    # reach into every 16,384-id pass
    assert n_live % 16 and n_live > 16384
    assert movers.max() >= 32768 and holes.min() < 16384 and holes.max() >= 16384
    assert n_live % 4096  # inside a plan block
    ws = torch.zeros(3 * n_pages, dtype=torch.int32, device=dev)
    info = torch.zeros(2, dtype=torch.int32, device=dev)
    ops.compact(pools, bt, lens, bs, stack, top, ws, info)
    r_stack, r_top, moved = ref.compact(r_pools, r_bt, r_lens, bs)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert not _np(ws)[:n_pages].any()
    assert _np(info).tolist() == [n_live, moved] and moved == len(movers)
    assert np.array_equal(_np(bt), r_bt) and np.array_equal(_np(lens), r_lens)
    assert int(top.item()) == r_top and np.array_equal(_np(stack)[:r_top], r_stack[:r_top])
    for p, rp in zip(pools, r_pools):
        assert torch.equal(p.cpu(), rp)
    assert not _np(ws)[:n_pages].any()
