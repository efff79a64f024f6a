"""Write the decode fixtures of the reference's real cached decode loop.

Run in the build container only, where the reference source tree is present
(it is imported from its source directories on sys.path, not installed):

    python tests/golden/make_decode_fixtures.py [reference_root]

A seeded ``ModelConfig.tiny()`` ``SaintLLM`` (fp32, CPU) decodes a batch of
prompts with ``greedy_decode_cached`` (generate.py:67-127), whose bundle comes
from ``KVCacheBundle.for_model`` (kv_cache.py:369-427).  Every cache layer's
``append`` is recorded in call order: its inputs, each compressor's input
and output, and the views it returns; also the layer types and dimensions
``for_model`` chose, the b-branch weights of every compressor, and the
decoded tokens.  Output: ``decode_tiny.safetensors`` (tensors) and
``decode_tiny.json`` (call order, names, shapes) beside this script.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent


def main(ref_root: Path) -> None:
    sys.dont_write_bytecode = True  # nothing may be written into the reference tree
    for pkg in ("core", "inference", "kernels", "data"):
        sys.path.insert(0, str(ref_root / "packages" / pkg / "src"))
    from saint_llm_core.config import ModelConfig
    from saint_llm_core.model import SaintLLM
    from saint_llm_inference import kv_cache as kvc
    from saint_llm_inference.generate import greedy_decode_cached

    torch.manual_seed(1234)
    cfg = ModelConfig.tiny()
    model = SaintLLM(cfg).eval()
    prompt = torch.randint(0, cfg.vocab_size, (2, 11), generator=torch.Generator().manual_seed(7))
    max_new = 7

    tensors: dict[str, torch.Tensor] = {}
    calls: list[dict] = []
    meta: dict = {"prompt_shape": list(prompt.shape), "max_new_tokens": max_new}

    def put(name: str, t: torch.Tensor) -> str:
        tensors[name] = t.detach().contiguous().clone()
        return name

    orig_for_model = kvc.KVCacheBundle.for_model.__func__

    def for_model(cls, model_, **kw):
        bundle = orig_for_model(cls, model_, **kw)
        meta["for_model_kwargs"] = {k: (str(v) if k in ("device", "dtype") else v) for k, v in kw.items()}
        layers = []
        for i, layer in enumerate(bundle._layers):
            if layer is None:
                layers.append(None)
                continue
            rec = {"type": type(layer).__name__, "max_seq_len": layer.max_seq_len, "head_dim": layer.head_dim,
                   "batch_size": layer.batch_size}
            if hasattr(layer, "compression_rate"):
                rec.update(compression_rate=layer.compression_rate, hidden_dim=layer.hidden_dim)
            if hasattr(layer, "c_indexer"):
                rec["c_indexer"] = layer.c_indexer
            layers.append(rec)
            _wrap(i, layer)
        meta["layers"] = layers
        meta["attention_types"] = [type(b.attention).__name__ for b in model_.blocks]
        return bundle

    def _wrap(i: int, layer) -> None:
        orig = layer.append

        def append(*args, **kw):
            c = {"layer": i, "type": type(layer).__name__, "n": len(calls)}
            pfx = f"c{len(calls)}"
            c["args"] = [put(f"{pfx}.arg{j}", a) for j, a in enumerate(args)]
            comps = {}
            for key in ("compressor", "indexer_compressor"):
                if key in kw:
                    fn = kw[key]
                    seen = []

                    def rec(x, fn=fn, seen=seen, key=key):
                        y = fn(x)
                        seen.append((put(f"{pfx}.{key}.in{len(seen)}", x), put(f"{pfx}.{key}.out{len(seen)}", y)))
                        return y

                    kw[key] = rec
                    comps[key] = (fn, seen)
                    if not any(w.startswith(f"l{i}.{key}.") for w in tensors):
                        for wn in ("w_b_kv", "w_b_z"):
                            put(f"l{i}.{key}.{wn}", getattr(fn, wn).weight)
                        put(f"l{i}.{key}.bias_b", fn.bias_b)
                        meta.setdefault("compressors", {})[f"l{i}.{key}"] = {"m": fn.m, "c": fn.c}
            out = orig(*args, **kw)
            c["compressor_calls"] = {k: [list(p) for p in v[1]] for k, v in comps.items()}
            c["out"] = [put(f"{pfx}.out{j}", o) for j, o in enumerate(out)]
            calls.append(c)
            return out

        layer.append = append

    kvc.KVCacheBundle.for_model = classmethod(for_model)
    tokens = greedy_decode_cached(model, prompt, max_new_tokens=max_new)
    put("tokens", tokens)
    put("prompt", prompt)
    meta["calls"] = calls
    meta["config"] = {"hidden_dim": cfg.hidden_dim, "head_dim": cfg.attention.head_dim,
                      "csa_m": cfg.csa.compression_rate, "c_indexer": cfg.csa.indexer_head_dim,
                      "hca_m": cfg.hca.compression_rate, "n_layers": cfg.n_layers}
    save_file(tensors, str(HERE / "decode_tiny.safetensors"))
    (HERE / "decode_tiny.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print(f"{len(calls)} append calls, {len(tensors)} tensors, tokens {tokens.tolist()}")


if __name__ == "__main__":
    main(Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference"))
