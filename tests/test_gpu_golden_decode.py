"""Replay of the reference's real cached decode loop through the drop-in.

The fixtures (tests/golden/decode_tiny.*) were written by
tests/golden/make_decode_fixtures.py from the reference itself: a seeded
``ModelConfig.tiny()`` ``SaintLLM`` decoding two prompts with
``greedy_decode_cached`` (generate.py:67-127), its bundle built by
``KVCacheBundle.for_model`` (kv_cache.py:369-427).  They hold the layer types
and sizes for_model chose and every cache ``append`` in call order: inputs,
compressor inputs and outputs, returned views.

* for_model over a stand-in model with the same config and attention class
  names builds the same layers (type, max_seq_len, head_dim, batch, m,
  hidden_dim, c_indexer).
* fp32 replay: every append, with compressors that check their input against
  the recorded one and return the recorded output, returns the recorded
  views bit for bit (SW rows, compressed entries, indexer entries).
* fast-path replay: the compressors are TokenLevelCompressor modules with
  the recorded b-branch weights, so the drop-in runs its projections and the
  HIP pooling.  Every compressed entry is held elementwise to the pooling of
  the recorded compressor inputs (csa.py:79-87): fp32 bundle (the reference
  decode loop's own dtype) within ref.pooling_bound of the recorded inputs'
  projections and of the reference's recorded entry; bf16 bundle (bf16
  inputs, weights and entries) within ref.pooling_bound_rounded_inputs of
  the projections of the bf16-rounded inputs (the bf16 GEMMs round each
  projection once).  The views are also within 1e-4 (fp32) / 1e-2 (bf16) of
  the recorded ones in norm, and the SW views are the recorded ones (bf16:
  rounded to bf16).
"""

from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load():
    from safetensors.torch import load_file

    meta = json.loads((GOLDEN / "decode_tiny.json").read_text())
    return meta, load_file(str(GOLDEN / "decode_tiny.safetensors"))


def _stand_in_model(meta):
    cfg = meta["config"]
    conf = SimpleNamespace(
        hidden_dim=cfg["hidden_dim"], attention=SimpleNamespace(head_dim=cfg["head_dim"]),
        csa=SimpleNamespace(compression_rate=cfg["csa_m"], indexer_head_dim=cfg["c_indexer"]),
        hca=SimpleNamespace(compression_rate=cfg["hca_m"]))
    classes = {n: type(n, (), {}) for n in set(meta["attention_types"])}
    return SimpleNamespace(cfg=conf, blocks=[SimpleNamespace(attention=classes[n]()) for n in meta["attention_types"]])


def _bundle(meta, dev, dtype):
    from saint_kv.kv_cache import KVCacheBundle

    kw = meta["for_model_kwargs"]
    return KVCacheBundle.for_model(_stand_in_model(meta), max_seq_len=kw["max_seq_len"],
                                   batch_size=kw["batch_size"], device=dev, dtype=dtype)


def test_for_model_builds_the_reference_layers(dev) -> None:
    meta, _ = _load()
    bundle = _bundle(meta, dev, torch.float32)
    assert len(bundle) == len(meta["layers"])
    for i, rec in enumerate(meta["layers"]):
        layer = bundle.for_layer(i)
        assert type(layer).__name__ == rec["type"]
        for key in ("max_seq_len", "head_dim", "batch_size", "compression_rate", "hidden_dim", "c_indexer"):
            if key in rec:
                assert getattr(layer, key) == rec[key], (i, key)


def _replay(meta, t, dev, dtype, compressor_for):
    bundle = _bundle(meta, dev, dtype)
    outs = []
    for c in meta["calls"]:
        layer = bundle.for_layer(c["layer"])
        args = [t[n].to(dev, dtype) for n in c["args"]]
        # the keyword compressors the reference passed (called or not)
        kw = {key: compressor_for(c, key) for key in c["compressor_calls"]}
        got = layer.append(*args, **kw)
        outs.append((c, [g.cpu() for g in got], layer))  # the views as they were after this call
    return bundle, outs


def test_replay_reference_appends_bit_exact(dev) -> None:
    meta, t = _load()

    def compressor_for(c, key):
        rec = c["compressor_calls"].get(key, [])

        it = iter(rec)

        def fn(x):
            x_name, y_name = next(it)
            assert torch.equal(x.cpu(), t[x_name]), (c["n"], key)  # the reference's compressor input
            return t[y_name].to(x.device)

        return fn

    _, outs = _replay(meta, t, dev, torch.float32, compressor_for)
    for c, got, _ in outs:
        assert len(got) == len(c["out"])
        for g, name in zip(got, c["out"]):
            assert torch.equal(g, t[name]), (c["n"], name)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_replay_fast_path_against_reference(dev, dtype) -> None:
    meta, t = _load()
    bf = dtype
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    modules = {}
    for name, dims in meta["compressors"].items():
        mod = ref.TokenLevelCompressor(meta["config"]["hidden_dim"], dims["c"], dims["m"])
        with torch.no_grad():
            mod.w_b_kv.weight.copy_(t[f"{name}.w_b_kv"])
            mod.w_b_z.weight.copy_(t[f"{name}.w_b_z"])
            mod.bias_b.copy_(t[f"{name}.bias_b"])
        modules[name] = mod.to(dev, bf)

    bundle, outs = _replay(meta, t, dev, bf, lambda c, key: modules[f"l{c['layer']}.{key}"])
    # every entry of every compressed stream, elementwise: the recorded
    # compressor inputs of the stream in call order hold its entries' tokens
    n_checked = 0
    for name, dims in meta["compressors"].items():
        li, key = int(name.split(".")[0][1:]), name.split(".", 1)[1]
        m, ch = dims["m"], dims["c"]
        xs = [t[x] for c in meta["calls"] if c["layer"] == li for x, _ in c["compressor_calls"].get(key, [])]
        ys = [t[y] for c in meta["calls"] if c["layer"] == li for _, y in c["compressor_calls"].get(key, [])]
        if not xs:
            continue
        x = torch.cat([v.view(v.shape[0], -1, m, v.shape[-1]) for v in xs], dim=1).float()  # (B, n, m, hidden)
        rec = torch.cat(ys, dim=1).float()  # the reference's entries
        wkv, wz, bias = (t[f"{name}.{w}"].float() for w in ("w_b_kv", "w_b_z", "bias_b"))
        if bf == torch.bfloat16:  # what the bf16 module and the drop-in see
            x, wkv, wz, bias = (v.to(torch.bfloat16).float() for v in (x, wkv, wz, bias))
        cz, zz = x @ wkv.T, x @ wz.T
        want = ref.compress_pool(cz, zz, bias)
        if bf == torch.bfloat16:
            bound = ref.pooling_bound_rounded_inputs(cz, zz, bias)
        else:
            bound = ref.pooling_bound(cz, zz, bias)
            assert ((rec - want).abs() <= bound).all(), name  # the reference's own entries
        layer = bundle.for_layer(li)
        view = (layer.compressed if key == "compressor" and not hasattr(layer, "compressed_kv")
                else layer.compressed_kv if key == "compressor" else layer.indexer_kv)
        got = view[:, : want.shape[1]].float().cpu()
        assert got.shape == want.shape, name
        err = (got - want).abs()
        assert (err <= bound).all(), (name, float((err / bound.clamp(min=1e-30)).max()))
        if bf == torch.float32:
            assert ((got - rec).abs() <= bound).all(), name
        n_checked += want.numel()
    assert n_checked > 0
    fast = set()
    for c, got, layer in outs:
        for j, (g, name) in enumerate(zip(got, c["out"])):
            want = t[name]
            if c["type"] == "SWAKVCacheLayer" or j >= len(got) - 2:  # SW rows: copies of bf16 inputs
                assert torch.equal(g, want.to(bf)), (c["n"], name)
            elif want.numel():
                err = float((g.float() - want).norm() / want.norm())
                assert err < tol, (c["n"], name, err)
            else:
                assert g.shape == want.shape
        if c["type"] != "SWAKVCacheLayer":
            fast.add(c["layer"])
            assert layer.fast_appends > 0
    assert fast == {1, 2, 3}
