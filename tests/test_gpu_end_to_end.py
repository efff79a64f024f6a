"""A three-layer decode loop (CSA with its indexer, HCA, SWA) through the
cache, token by token, against an uncached recompute.

The property is the one of the reference's cached-vs-uncached layer tests
(test_kv_cache.py:370-415: a layer run token by token over its cache equals
the full pass): here every step goes through the kernels (prefill through the
compressor kernels, then the fused decode step computing the CSA scores from
the indexer query, then each layer's attention over the cache), and the
recompute rebuilds, from every token's inputs so far, the compressed entries
(oracle pooling, rounded to bf16 as the compressor emits them), the indexer
scores, the top-k, the window and each layer's attention.

The model around the cache is a stand-in (the reference's modules do not run
here): the per-layer inputs (latent row, compressor and indexer projections,
queries) are random linear maps of a hidden vector, and the next hidden vector
is tanh of a random projection of the summed layer outputs.  The loop is
teacher-forced: the cached path's outputs feed the next token of both paths.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

TOL = 1e-2  # relative to each output row's largest magnitude (bf16 operands, fp32 accumulation)


def _close(got: np.ndarray, want: np.ndarray, label: str) -> None:
    assert np.isfinite(got).all(), label
    scale = np.abs(want).max(axis=-1, keepdims=True)
    err = np.abs(got - want)
    assert (err <= TOL * scale + 1e-4).all(), (label, float(err.max()))


def test_decode_loop_matches_uncached(dev) -> None:
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=16, idx_heads=8), LayerSpec("hca", m=16), LayerSpec("swa")]
    B, Hd, C, CI, W, H, IH = 2, 64, 576, 128, 32, 16, 8
    lens0 = np.array([37, 130])
    steps = 12
    cache = DecodeCache(specs, B, 512, window=W, block_size=16, device=dev, page_order_seed=5)
    g = torch.Generator().manual_seed(5)

    def lin(n_in, n_out, scale=1.0):
        return torch.randn(n_in, n_out, generator=g) * (scale / n_in ** 0.5)

    widths = {"kv": C, "c": C, "z": C, "ci": CI, "zi": CI}
    proj = []
    for s in specs:
        names = ["kv"] + (["c", "z"] if s.kind != "swa" else []) + (["ci", "zi"] if s.kind == "csa" else [])
        p = {k: lin(Hd, widths[k]) for k in names}
        p["q"] = lin(Hd, H * C)
        if s.kind == "csa":
            p["iq"] = lin(Hd, IH * CI)
            p["iw"] = lin(Hd, IH)
        proj.append(p)
    w_out = [lin(H * C, Hd, 4.0) for _ in specs]
    bias = [torch.randn(s.m, C, generator=g) if s.kind != "swa" else None for s in specs]
    ibias = [torch.randn(s.m, CI, generator=g) if s.kind == "csa" else None for s in specs]
    for i in range(len(specs)):
        if bias[i] is not None:
            cache.bias[i].copy_(bias[i])
        if ibias[i] is not None:
            cache.idx_bias[i].copy_(ibias[i])
    knorm_w = torch.rand(C, generator=g) + 0.5
    sink = torch.randn(H, generator=g)

    def layer_inputs(x):  # x: [B, T, Hd] fp32 -> per layer bf16 rows
        return [{k: (x @ w).to(torch.bfloat16) for k, w in p.items() if k not in ("q", "iq", "iw")}
                for p in proj]

    # prefill through the compressor kernels; the history keeps every token's rows
    x0 = torch.randn(B, int(lens0.max()), Hd, generator=g)
    pre = layer_inputs(x0)
    cache.prefill(lens0, data=[{k: v.to(dev) for k, v in d.items()} for d in pre])
    hist = [[{k: v[b, :lens0[b]] for k, v in pre[i].items()} for b in range(B)] for i in range(len(specs))]
    x = torch.randn(B, Hd, generator=g)
    for step in range(steps):
        rows = layer_inputs(x.unsqueeze(1))
        qs, iqs, iws = [], [], []
        for i, s in enumerate(specs):
            for k, v in rows[i].items():
                cache.inputs[i][k].copy_(v[:, 0])
                for b in range(B):
                    hist[i][b][k] = torch.cat([hist[i][b][k], v[b]])
            qs.append((x @ proj[i]["q"]).to(torch.bfloat16).view(B, H, C))
            if s.kind == "csa":
                iqs.append((x @ proj[i]["iq"]).to(torch.bfloat16).view(B, IH, CI))
                iws.append((x @ proj[i]["iw"]).float())
                cache.inputs[i]["iq"].copy_(iqs[-1])
                cache.inputs[i]["iw"].copy_(iws[-1])
            else:
                iqs.append(None)
                iws.append(None)
        cache.step()
        outs = []
        for i, s in enumerate(specs):
            outs.append(cache.attention(i, qs[i].to(dev), knorm_w.to(dev) if s.kind != "swa" else None,
                                        sink=sink.to(dev)).cpu())
        torch.cuda.synchronize()
        cache.check_status()
        # the uncached recompute of every layer of every sequence
        for i, s in enumerate(specs):
            for b in range(B):
                h = hist[i][b]
                L = h["kv"].shape[0]
                win = h["kv"][L - min(W, L):].double().numpy()
                kw = {}
                if s.kind != "swa":
                    n = L // s.m
                    ent = ref.compress_pool(h["c"][:n * s.m].view(n, s.m, C), h["z"][:n * s.m].view(n, s.m, C),
                                            bias[i]).to(torch.bfloat16).double().numpy()
                    kw = dict(entries=ent, m=s.m, knorm_w=knorm_w.double().numpy())
                    if s.kind == "csa":
                        ient = ref.compress_pool(h["ci"][:n * s.m].view(n, s.m, CI),
                                                 h["zi"][:n * s.m].view(n, s.m, CI), ibias[i]).to(torch.bfloat16)
                        n_valid = ref.n_valid_blocks(L - 1, s.m)
                        sc = ref.indexer_scores(iqs[i][b][None, None].float().numpy(), ient[None].float().numpy(),
                                                iws[i][b][None, None].numpy())[0]
                        picks = ref.topk_select(sc, np.array([n_valid]), s.top_k, n)[0]
                        got_picks = cache.topk_idx[i][b, :len(picks)].cpu().numpy()
                        assert np.array_equal(got_picks, picks), (step, b)
                        kw["picks"] = picks
                want = ref.decode_attention(qs[i][b].double().numpy(), s.kind, L, sink=sink.double().numpy(),
                                            win_k=win, win_v=win, **kw)
                _close(outs[i][b].numpy(), want, f"step {step} layer {i} ({s.kind}) seq {b}")
        # the next token's hidden vector, from the cached path
        y = sum(outs[i].reshape(B, -1) @ w_out[i] for i in range(len(specs)))
        x = torch.tanh(y)


def test_layer_sequential_decode_loop_matches_uncached(dev) -> None:
    """The same property with the layers in sequence, as a model runs them:
    each layer has its own cache, stepped without gathered copies
    (materialize=False: the attention reads the picks and the window in place),
    and layer i's inputs are linear maps of x_i, where x_{i+1} = tanh(x_i +
    out_i W_i) takes layer i's attention output.  Every layer's picks and
    attention output match the uncached recompute at every token."""
    from saint_kv.decode import DecodeCache, LayerSpec

    specs = [LayerSpec("csa", m=4, top_k=16, idx_heads=8), LayerSpec("hca", m=16), LayerSpec("swa"),
             LayerSpec("csa", m=4, top_k=8, idx_heads=8)]
    B, Hd, C, CI, W, H, IH = 2, 64, 576, 128, 32, 16, 8
    lens0 = np.array([29, 75])
    steps = 10
    caches = [DecodeCache([s], B, 512, window=W, block_size=16, device=dev, page_order_seed=11 + i,
                          materialize=False) for i, s in enumerate(specs)]
    assert all(c.out_entries[0] is None and c.out_window[0] is None for c in caches)
    g = torch.Generator().manual_seed(6)

    def lin(n_in, n_out, scale=1.0):
        return torch.randn(n_in, n_out, generator=g) * (scale / n_in ** 0.5)

    widths = {"kv": C, "c": C, "z": C, "ci": CI, "zi": CI}
    proj = []
    for s in specs:
        names = ["kv"] + (["c", "z"] if s.kind != "swa" else []) + (["ci", "zi"] if s.kind == "csa" else [])
        p = {k: lin(Hd, widths[k]) for k in names}
        p["q"] = lin(Hd, H * C)
        if s.kind == "csa":
            p["iq"] = lin(Hd, IH * CI)
            p["iw"] = lin(Hd, IH)
        proj.append(p)
    w_out = [lin(H * C, Hd, 4.0) for _ in specs]
    bias = [torch.randn(s.m, C, generator=g) if s.kind != "swa" else None for s in specs]
    ibias = [torch.randn(s.m, CI, generator=g) if s.kind == "csa" else None for s in specs]
    for c, b_, ib in zip(caches, bias, ibias):
        if b_ is not None:
            c.bias[0].copy_(b_)
        if ib is not None:
            c.idx_bias[0].copy_(ib)
    knorm_w = torch.rand(C, generator=g) + 0.5
    sink = torch.randn(H, generator=g)

    def rows_of(i, x):  # x: [B, T, Hd] fp32 -> layer i's bf16 rows
        return {k: (x @ w).to(torch.bfloat16) for k, w in proj[i].items() if k not in ("q", "iq", "iw")}

    # prefill: each layer's prompt rows from its own random hidden states
    hist = []
    for i, c in enumerate(caches):
        pre = rows_of(i, torch.randn(B, int(lens0.max()), Hd, generator=g))
        c.prefill(lens0, data=[{k: v.to(dev) for k, v in pre.items()}])
        hist.append([{k: v[b, :lens0[b]] for k, v in pre.items()} for b in range(B)])
    x = torch.randn(B, Hd, generator=g)
    for step in range(steps):
        xi = x
        for i, (s, c) in enumerate(zip(specs, caches)):
            rows = rows_of(i, xi.unsqueeze(1))
            for k, v in rows.items():
                c.inputs[0][k].copy_(v[:, 0])
                for b in range(B):
                    hist[i][b][k] = torch.cat([hist[i][b][k], v[b]])
            q = (xi @ proj[i]["q"]).to(torch.bfloat16).view(B, H, C)
            if s.kind == "csa":
                iq = (xi @ proj[i]["iq"]).to(torch.bfloat16).view(B, IH, CI)
                iw = (xi @ proj[i]["iw"]).float()
                c.inputs[0]["iq"].copy_(iq)
                c.inputs[0]["iw"].copy_(iw)
            c.step()
            out = c.attention(0, q.to(dev), knorm_w.to(dev) if s.kind != "swa" else None, sink=sink.to(dev)).cpu()
            torch.cuda.synchronize()
            c.check_status()
            for b in range(B):
                h = hist[i][b]
                L = h["kv"].shape[0]
                win = h["kv"][L - min(W, L):].double().numpy()
                kw = {}
                if s.kind != "swa":
                    n = L // s.m
                    ent = ref.compress_pool(h["c"][:n * s.m].view(n, s.m, C), h["z"][:n * s.m].view(n, s.m, C),
                                            bias[i]).to(torch.bfloat16).double().numpy()
                    kw = dict(entries=ent, m=s.m, knorm_w=knorm_w.double().numpy())
                    if s.kind == "csa":
                        ient = ref.compress_pool(h["ci"][:n * s.m].view(n, s.m, CI),
                                                 h["zi"][:n * s.m].view(n, s.m, CI), ibias[i]).to(torch.bfloat16)
                        sc = ref.indexer_scores(iq[b][None, None].float().numpy(), ient[None].float().numpy(),
                                                iw[b][None, None].numpy())[0]
                        picks = ref.topk_select(sc, np.array([ref.n_valid_blocks(L - 1, s.m)]), s.top_k, n)[0]
                        assert np.array_equal(c.topk_idx[0][b, :len(picks)].cpu().numpy(), picks), (step, i, b)
                        kw["picks"] = picks
                want = ref.decode_attention(q[b].double().numpy(), s.kind, L, sink=sink.double().numpy(),
                                            win_k=win, win_v=win, **kw)
                _close(out[b].numpy(), want, f"step {step} layer {i} ({s.kind}) seq {b}")
            xi = torch.tanh(xi + out.reshape(B, -1) @ w_out[i])  # the next layer's hidden vector
        x = xi
