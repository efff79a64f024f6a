"""Pin the oracle's decode attention (CPU only).

The oracle restates scaled_dot_product / softmax_with_sink / RMSNorm of
common.py:12-124 and the three consumers (csa.py:324-373, hca.py:126-169,
swa.py:115-137).  Each check below fixes it by something other than its own
formula: torch's scaled_dot_product_attention and rms_norm (library routines),
closed forms of the sink and the softcap, one-key and all-masked cases, the
HCA visibility rule by brute force, and a pure-Python loop.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import reference_cpu as ref


def _rand(rng: np.random.Generator, *shape: int) -> np.ndarray:
    return rng.standard_normal(shape)


def test_attention_row_matches_torch_sdpa() -> None:
    rng = np.random.default_rng(0)
    h, n, d = 8, 37, 64
    q, k, v = _rand(rng, h, d), _rand(rng, n, d), _rand(rng, n, d)
    valid = rng.random(n) < 0.7
    valid[3] = True
    got = ref.attention_row(q, k, v, valid)
    want = F.scaled_dot_product_attention(
        torch.from_numpy(q)[:, None], torch.from_numpy(k)[None].expand(h, n, d),
        torch.from_numpy(v)[None].expand(h, n, d),
        attn_mask=torch.from_numpy(valid)[None, None].expand(h, 1, n))[:, 0]
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-12, atol=1e-12)


def test_sink_closed_form() -> None:
    # q = 0: every score is 0, so each key gets 1 / (n + e^sink) and the
    # output is sum(v) / (n + e^sink), per head
    rng = np.random.default_rng(1)
    h, n, d = 4, 9, 16
    v = _rand(rng, n, d)
    sink = np.array([-3.0, 0.0, 1.5, 40.0])
    got = ref.attention_row(np.zeros((h, d)), _rand(rng, n, d), v, np.ones(n, bool), sink)
    want = v.sum(0)[None, :] / (n + np.exp(sink))[:, None]
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-15)


def test_sink_matches_concatenated_softmax() -> None:
    # softmax_with_sink's own construction (common.py:84-89): append the sink
    # column, softmax, drop it; here through torch
    rng = np.random.default_rng(2)
    h, n, d = 6, 20, 32
    q, k, v = _rand(rng, h, d), _rand(rng, n, d), _rand(rng, n, d)
    valid = rng.random(n) < 0.5
    valid[0] = True
    sink = rng.standard_normal(h) * 3
    s = torch.from_numpy(q @ k.T / math.sqrt(d)).masked_fill(~torch.from_numpy(valid), float("-inf"))
    probs = torch.softmax(torch.cat([s, torch.from_numpy(sink)[:, None]], dim=-1), dim=-1)[:, :-1]
    want = (probs @ torch.from_numpy(v)).numpy()
    np.testing.assert_allclose(ref.attention_row(q, k, v, valid, sink), want, rtol=1e-12, atol=1e-14)
    # a sink far below every score is no sink
    np.testing.assert_allclose(ref.attention_row(q, k, v, valid, np.full(h, -1e4)),
                               ref.attention_row(q, k, v, valid), rtol=1e-12)


def test_scale_and_softcap_closed_form() -> None:
    # q = e0 and k_j = 2 s_j e0 in D = 4 make the scaled score exactly s_j;
    # one-hot values read the probabilities back
    s = np.array([3.0, -1.0, 0.5, 7.0])
    d = 4
    q = np.zeros((1, d))
    q[0, 0] = 1.0
    k = np.zeros((4, d))
    k[:, 0] = 2.0 * s
    v = np.eye(4)
    for cap in (None, 2.5, 50.0):
        z = s if cap is None else cap * np.tanh(s / cap)
        want = np.exp(z - z.max()) / np.exp(z - z.max()).sum()
        got = ref.attention_row(q, k, v, np.ones(4, bool), None, cap)[0]
        np.testing.assert_allclose(got, want, rtol=1e-12)


def test_rms_norm_matches_torch() -> None:
    rng = np.random.default_rng(3)
    x, w = _rand(rng, 11, 576), rng.random(576) + 0.5
    want = F.rms_norm(torch.from_numpy(x), (576,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(ref.rms_norm(x, w, 1e-6), want, rtol=1e-12)


def test_csa_single_pick_and_no_pick() -> None:
    rng = np.random.default_rng(4)
    h, d = 5, 64
    q, e, w = _rand(rng, h, d), _rand(rng, 30, d), rng.random(d) + 0.5
    # one valid pick: softmax over one key is 1, the output is the normed entry
    out = ref.csa_sparse_attention(q, e, np.array([-1, 17, -1, -1]), w)
    np.testing.assert_allclose(out, np.broadcast_to(ref.rms_norm(e[17], w), (h, d)), rtol=1e-12)
    # no valid pick: zeros (csa.py:344-348)
    assert not ref.csa_sparse_attention(q, e, np.full(6, -1), w).any()
    # the order of the picks does not matter; -1 picks add nothing
    picks = np.array([3, 9, 28, 0, 14])
    a = ref.csa_sparse_attention(q, e, picks, w)
    b = ref.csa_sparse_attention(q, e, np.concatenate([picks[::-1], [-1, -1]]), w)
    np.testing.assert_allclose(a, b, rtol=1e-12)


def test_hca_visibility_brute_force() -> None:
    rng = np.random.default_rng(5)
    h, d, m = 3, 32, 4
    e, w = _rand(rng, 9, d), rng.random(d) + 0.5
    q = _rand(rng, h, d)
    sink = rng.standard_normal(h)
    for q_pos in range(0, 40):
        vis = [s for s in range(9) if s * m + m - 1 < q_pos]
        assert len(vis) == min(9, ref.n_valid_blocks(q_pos, m))
        got = ref.hca_compressed_attention(q, e, q_pos, m, w, 1e-6, sink)
        if not vis:
            assert not got.any()
            continue
        keys = ref.rms_norm(e[vis], w)
        want = ref.attention_row(q, keys, keys, np.ones(len(vis), bool), sink)
        np.testing.assert_allclose(got, want, rtol=1e-12)


def test_decode_attention_pure_python() -> None:
    rng = np.random.default_rng(6)
    h, d, m, L = 2, 4, 2, 9
    q = rng.standard_normal((h, d)).tolist()
    ent = rng.standard_normal((5, d)).tolist()
    wk = rng.standard_normal((3, d)).tolist()
    wv = rng.standard_normal((3, d)).tolist()
    knw = (rng.random(d) + 0.5).tolist()
    sink = [0.3, -0.7]
    cap = 1.7

    def norm(x):
        r = 1.0 / math.sqrt(sum(t * t for t in x) / len(x) + 1e-6)
        return [knw[i] * x[i] * r for i in range(len(x))]

    def attend(qh, keys, vals, s_h, capped):
        sc = [sum(a * b for a, b in zip(qh, kk)) / math.sqrt(d) for kk in keys]
        if capped:
            sc = [cap * math.tanh(t / cap) for t in sc]
        mx = max(sc + ([s_h] if s_h is not None else []))
        ex = [math.exp(t - mx) for t in sc]
        den = sum(ex) + (math.exp(s_h - mx) if s_h is not None else 0.0)
        return [sum(ex[j] * vals[j][c] for j in range(len(keys))) / den for c in range(d)]

    vis = [s for s in range(5) if s * m + m - 1 < L - 1]
    ck = [norm(ent[s]) for s in vis]
    want = []
    for hh in range(h):
        a = attend(q[hh], wk, wv, sink[hh], True)
        b = attend(q[hh], ck, ck, sink[hh], False)
        want.append([x + y for x, y in zip(a, b)])
    got = ref.decode_attention(np.array(q), "hca", L, entries=np.array(ent), m=m,
                               knorm_w=np.array(knw), sink=np.array(sink), softcap=cap,
                               win_k=np.array(wk), win_v=np.array(wv))
    np.testing.assert_allclose(got, np.array(want), rtol=1e-12)
    # CSA: no sink on the sparse branch
    picks = [4, -1, 1]
    ck = [norm(ent[p]) for p in picks if p >= 0]
    want = []
    for hh in range(h):
        a = attend(q[hh], wk, wv, sink[hh], True)
        b = attend(q[hh], ck, ck, None, False)
        want.append([x + y for x, y in zip(a, b)])
    got = ref.decode_attention(np.array(q), "csa", L, entries=np.array(ent), picks=np.array(picks),
                               knorm_w=np.array(knw), sink=np.array(sink), softcap=cap,
                               win_k=np.array(wk), win_v=np.array(wv))
    np.testing.assert_allclose(got, np.array(want), rtol=1e-12)
