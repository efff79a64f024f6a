"""The snapshot-file oracle (oracle.state_file) pinned on the CPU.

* tail_state: one token gives (z + bias, 1, c) exactly; a whole block's
  numerator / denominator is compress_pool (the softmax pooling, csa.py:86-87);
  two partial states merged by the online-softmax rule give the state of
  their union; the maximum is the elementwise maximum.
* kept_rows: brute force over the positions (the ring holds the last W;
  periodic keeps those before the last multiple of p), and agreement with
  saint_kv.state.swa_rows_kept on a sweep.
* read_state: a file assembled here byte by byte reads back section by
  section; bad magic, version and misaligned offsets are refused.
"""

from __future__ import annotations

import json
import struct

import pytest
import torch

from oracle import reference_cpu as ref
from oracle import state_file as sf


def test_tail_state_single_token_and_full_block() -> None:
    g = torch.Generator().manual_seed(0)
    c = torch.randn(4, 64, generator=g).to(torch.bfloat16)
    z = torch.randn(4, 64, generator=g).to(torch.bfloat16)
    bias = torch.randn(4, 64, generator=g)
    one = sf.tail_state(c[:1], z[:1], bias[:1])
    assert torch.equal(one[0], z[0].float() + bias[0])
    assert torch.equal(one[1], torch.ones(64))
    assert torch.equal(one[2], c[0].float())
    full = sf.tail_state(c, z, bias)
    torch.testing.assert_close(full[2] / full[1], ref.compress_pool(c, z, bias), rtol=1e-6, atol=1e-6)
    assert torch.equal(full[0], (z.float() + bias).max(dim=0).values)
    assert (full[1] >= 1).all()  # the maximum's own term is exp(0)


def test_tail_state_merge_is_union() -> None:
    g = torch.Generator().manual_seed(1)
    c, z, bias = (torch.randn(7, 32, generator=g) for _ in range(3))
    a, b = sf.tail_state(c[:3], z[:3], bias[:3]), sf.tail_state(c[3:], z[3:], bias[3:])
    mx = torch.maximum(a[0], b[0])
    sa, sb = torch.exp(a[0] - mx), torch.exp(b[0] - mx)
    merged = torch.stack([mx, a[1] * sa + b[1] * sb, a[2] * sa + b[2] * sb])
    torch.testing.assert_close(merged, sf.tail_state(c, z, bias), rtol=1e-6, atol=1e-6)


def test_kept_rows_brute_force() -> None:
    from saint_kv import state

    for L in range(0, 70):
        for W in (1, 8, 16):
            in_ring = [p for p in range(L) if p >= L - W]
            assert sf.kept_rows(L, W, "full") == ((in_ring[0], L) if in_ring else (0, 0))
            assert sf.kept_rows(L, W, "zero")[0] == sf.kept_rows(L, W, "zero")[1]
            for p in (1, 5, 8, 64):
                lo, hi = sf.kept_rows(L, W, "periodic", p)
                kept = [q for q in in_ring if q < (L // p) * p]
                assert list(range(lo, hi)) == kept, (L, W, p)
                assert state.swa_rows_kept(L, W, "periodic", p) == (lo, hi)
            for strat in ("full", "zero"):
                assert state.swa_rows_kept(L, W, strat, None) == sf.kept_rows(L, W, strat)


def _file(sections: list[tuple[dict, bytes]], version: int = 1, magic: bytes = b"SKVSTATE") -> bytes:
    hdr = {"length": 3, "sections": [s for s, _ in sections]}
    raw = json.dumps(hdr).encode()
    head = magic + struct.pack("<II", version, len(raw)) + raw
    head += b"\0" * ((-len(head)) % 16)
    body = bytearray()
    for s, data in sections:
        assert len(body) == s["offset"]
        body += data + b"\0" * ((-len(data)) % 16)
    return head + bytes(body)


def test_read_state_sections_and_refusals(tmp_path) -> None:
    a = torch.arange(6, dtype=torch.float32).reshape(2, 3)
    bb = torch.tensor([1.5, -2.0, 3.25], dtype=torch.bfloat16)
    secs = [({"name": "state", "layer": 2, "dtype": "float32", "shape": [2, 3], "offset": 0, "nbytes": 24},
             a.numpy().tobytes()),
            ({"name": "swa", "layer": 0, "dtype": "bfloat16", "shape": [3], "offset": 32, "nbytes": 6},
             bb.view(torch.uint8).numpy().tobytes())]
    p = tmp_path / "ok.skv"
    p.write_bytes(_file(secs))
    hdr, got = sf.read_state(p)
    assert hdr["length"] == 3
    assert torch.equal(got[("state", 2)], a) and torch.equal(got[("swa", 0)], bb)
    for bad, match in ((_file(secs, magic=b"XXXXXXXX"), "snapshot"), (_file(secs, version=2), "version")):
        p.write_bytes(bad)
        with pytest.raises(ValueError, match=match):
            sf.read_state(p)
    # a section whose offset is not a multiple of 16
    hdr2 = {"length": 3, "sections": [dict(secs[0][0], offset=8)]}
    enc = json.dumps(hdr2).encode()
    head = b"SKVSTATE" + struct.pack("<II", 1, len(enc)) + enc
    p.write_bytes(head + b"\0" * ((-len(head)) % 16) + bytes(8) + secs[0][1])
    with pytest.raises(ValueError, match="aligned"):
        sf.read_state(p)
