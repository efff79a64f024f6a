"""The snapshot file format and the SWA strategies' row ranges (host only)."""

from __future__ import annotations

import json
import struct

import pytest

from saint_kv import state


def test_swa_rows_kept() -> None:
    # full: the last min(W, L) rows; zero: none; periodic: up to the last multiple of p
    assert state.swa_rows_kept(520, 16, "full", None) == (504, 520)
    assert state.swa_rows_kept(10, 16, "full", None) == (0, 10)
    assert state.swa_rows_kept(520, 16, "zero", None) == (504, 504)
    assert state.swa_rows_kept(520, 16, "periodic", 8) == (504, 520)
    assert state.swa_rows_kept(520, 16, "periodic", 7) == (504, 518)
    assert state.swa_rows_kept(520, 16, "periodic", 100) == (504, 504)  # checkpoint 500 left the ring
    with pytest.raises(ValueError):
        state.swa_rows_kept(520, 16, "periodic", None)


def test_header_roundtrip_and_errors(tmp_path) -> None:
    hdr = {"layout": {"latent": 576}, "length": 5, "sections": []}
    raw = json.dumps(hdr).encode()
    p = tmp_path / "ok.skv"
    p.write_bytes(state.MAGIC + struct.pack("<II", state.VERSION, len(raw)) + raw + b"\0" * ((-(16 + len(raw))) % 16))
    got, base = state.read_header(p)
    assert got == hdr and base % 16 == 0 and base >= 16 + len(raw)
    bad = tmp_path / "bad.skv"
    bad.write_bytes(b"NOTSTATE" + bytes(8))
    with pytest.raises(ValueError, match="not a saint_kv"):
        state.read_header(bad)
    old = tmp_path / "old.skv"
    old.write_bytes(state.MAGIC + struct.pack("<II", 99, 2) + b"{}")
    with pytest.raises(ValueError, match="version"):
        state.read_header(old)
    cut = tmp_path / "cut.skv"
    cut.write_bytes(state.MAGIC + struct.pack("<II", state.VERSION, 100) + b"{}")
    with pytest.raises(ValueError, match="truncated"):
        state.read_header(cut)
