"""The oracle against the reference's real cached decode loop (CPU).

tests/golden/decode_tiny.* were written from the reference itself (see
tests/golden/make_decode_fixtures.py): every cache ``append`` of a seeded
``ModelConfig.tiny()`` model decoding two prompts with
``greedy_decode_cached``, with compressor inputs/outputs and weights.

* ContiguousSWA / ContiguousCompressed (the kv_cache.py state machine),
  replayed with the recorded compressor outputs, return the recorded views
  bit for bit, and hand their compressors the recorded inputs: the buffered
  tokens are joined in the reference's order.
* TokenLevelCompressor with the recorded b-branch weights maps every
  recorded compressor input to the recorded output (fp32, within 1e-6
  relative), and compress_pool of its projections gives the same: the
  pooling formula is the reference module's.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

from oracle import reference_cpu as ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load():
    from safetensors.torch import load_file

    return (json.loads((GOLDEN / "decode_tiny.json").read_text()),
            load_file(str(GOLDEN / "decode_tiny.safetensors")))


def test_fixture_covers_every_layer_kind() -> None:
    meta, t = _load()
    kinds = {c["type"] for c in meta["calls"]}
    assert kinds == {"SWAKVCacheLayer", "CSAKVCacheLayer", "HCAKVCacheLayer"}
    # prefill of 11 tokens then 6 single-token steps (the 7th token needs no cache)
    assert len(meta["calls"]) == 4 * 7
    assert t["tokens"].shape == (2, 11 + meta["max_new_tokens"])
    assert torch.equal(t["tokens"][:, :11], t["prompt"])
    # some step completes a block (compressor called) and some does not
    n_calls = [len(v) for c in meta["calls"] for v in c["compressor_calls"].values()]
    assert 0 in n_calls and 1 in n_calls


def test_oracle_cache_replays_reference_appends() -> None:
    meta, t = _load()
    caches = []
    for rec in meta["layers"]:
        if rec["type"] == "SWAKVCacheLayer":
            caches.append(ref.ContiguousSWA(rec["max_seq_len"], rec["head_dim"], batch_size=rec["batch_size"]))
        else:
            dims = [rec["head_dim"]] + ([rec["c_indexer"]] if "c_indexer" in rec else [])
            caches.append(ref.ContiguousCompressed(rec["max_seq_len"], rec["hidden_dim"], dims,
                                                   rec["compression_rate"], batch_size=rec["batch_size"]))
    for c in meta["calls"]:
        args = [t[n] for n in c["args"]]
        if c["type"] == "SWAKVCacheLayer":
            got = caches[c["layer"]].append(*args)
        else:
            def stub(rec):
                it = iter(rec)

                def fn(x):
                    x_name, y_name = next(it)
                    assert torch.equal(x, t[x_name]), (c["n"], x_name)
                    return t[y_name]
                return fn

            comps = [stub(c["compressor_calls"][k]) for k in ("compressor", "indexer_compressor")
                     if k in c["compressor_calls"]]
            got = caches[c["layer"]].append(*args, comps)
        assert len(got) == len(c["out"])
        for g, name in zip(got, c["out"]):
            assert torch.equal(g, t[name]), (c["n"], name)


def test_oracle_compressor_matches_reference_module() -> None:
    meta, t = _load()
    hidden = meta["config"]["hidden_dim"]
    n_checked = 0
    for name, dims in meta["compressors"].items():
        mod = ref.TokenLevelCompressor(hidden, dims["c"], dims["m"])
        with torch.no_grad():
            mod.w_b_kv.weight.copy_(t[f"{name}.w_b_kv"])
            mod.w_b_z.weight.copy_(t[f"{name}.w_b_z"])
            mod.bias_b.copy_(t[f"{name}.bias_b"])
        layer, key = name.split(".")
        for c in meta["calls"]:
            if f"l{c['layer']}" != layer:
                continue
            for x_name, y_name in c["compressor_calls"].get(key, []):
                x, want = t[x_name], t[y_name]
                with torch.no_grad():
                    got = mod(x)
                    b, n_tok, _ = x.shape
                    n = n_tok // dims["m"]
                    cb = (x @ t[f"{name}.w_b_kv"].T).view(b, n, dims["m"], dims["c"])
                    zb = (x @ t[f"{name}.w_b_z"].T).view(b, n, dims["m"], dims["c"])
                    pooled = ref.compress_pool(cb, zb, t[f"{name}.bias_b"])
                for y in (got, pooled):
                    assert y.shape == want.shape
                    torch.testing.assert_close(y, want, rtol=1e-6, atol=1e-6)
                n_checked += 1
    assert n_checked >= 10
