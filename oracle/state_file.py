"""Oracle of the per-request snapshot file (test infrastructure only).

Only tests may import this module; the product never does.  It reads the
``SKVSTATE`` file that saint_kv writes for one request without using
saint_kv, and states what each section must hold in terms of the oracle's own
cache (reference_cpu: the paged pools, the ring, the buffered tokens of the
incomplete block).

The reference plans the state cache without implementing it
(``saint_llm_inference/__init__.py:6-7``: "State cache for SWA + uncompressed
CSA/HCA tail tokens"; "Three SWA strategies (Full / Periodic / Zero)").  What
the oracle fixes:

* layout: the 8 magic bytes ``SKVSTATE``, uint32 version 1, uint32 header
  length, the JSON header, sections at 16-byte aligned offsets after it, each
  ``{name, layer, dtype, shape, offset, nbytes}``;
* ``swa`` rows kept per strategy at length L and window W (``kept_rows``):
  full keeps positions [L - min(W, L), L), periodic with period p the ones of
  those below the last multiple of p, zero none; row j of the section is
  the ring row of position lo + j (``reference_cpu.ring_read``);
* ``entries`` / ``entries_idx``: the L // m compressed entries of the stream
  in order, as the pool stores them (bf16 values, or fp8 656-byte entries);
* ``state`` / ``state_idx``: fp32 [3, C] online-softmax state of the
  incomplete block when L % m = r > 0 (``tail_state`` of its r buffered
  tokens): row 0 the running maximum of z + bias, row 1 the sum of
  exp(z + bias - max), row 2 the same weighted sum of c.  With r = 0 the
  state is not part of the request (the next token starts a new block) and
  its bytes are unspecified.
"""

from __future__ import annotations

import json
import struct
from pathlib import Path

import torch
from torch import Tensor

MAGIC = b"SKVSTATE"
VERSION = 1
_DTYPES = {"bfloat16": torch.bfloat16, "uint8": torch.uint8, "float32": torch.float32}


def read_state(path: str | Path) -> tuple[dict, dict[tuple[str, int], Tensor]]:
    """(header, {(section name, layer): CPU tensor}) of a snapshot file."""
    raw = Path(path).read_bytes()
    if raw[:8] != MAGIC:
        raise ValueError("not a snapshot")
    version, n = struct.unpack_from("<II", raw, 8)
    if version != VERSION:
        raise ValueError(f"version {version}")
    header = json.loads(raw[16:16 + n])
    base = 16 + n + (-(16 + n)) % 16
    out = {}
    for s in header["sections"]:
        if s["offset"] % 16:
            raise ValueError(f"section {s['name']}/{s['layer']} not 16-byte aligned")
        lo = base + s["offset"]
        buf = bytearray(raw[lo:lo + s["nbytes"]])
        if len(buf) != s["nbytes"]:
            raise ValueError("truncated section")
        t = torch.frombuffer(buf, dtype=torch.uint8) if buf else torch.zeros(0, dtype=torch.uint8)
        out[(s["name"], s["layer"])] = t.view(_DTYPES[s["dtype"]]).reshape(s["shape"])
    return header, out


def kept_rows(L: int, window: int, strategy: str, period: int | None = None) -> tuple[int, int]:
    """Positions [lo, hi) of the SWA rows a snapshot at length L keeps."""
    lo = max(0, L - window)
    if strategy == "full":
        return lo, L
    if strategy == "zero":
        return lo, lo
    assert strategy == "periodic" and period and period > 0
    last_checkpoint = (L // period) * period
    return lo, max(lo, last_checkpoint)


def tail_state(c: Tensor, z: Tensor, bias: Tensor) -> Tensor:
    """fp32 [3, C] pooling state of r >= 1 buffered tokens: c, z (r, C), bias
    (r, C) the rows of the block's first r positions (csa.py:82, 86-87)."""
    v = z.float() + bias.float()
    mx = v.max(dim=0).values
    w = torch.exp(v - mx)
    return torch.stack([mx, w.sum(dim=0), (w * c.float()).sum(dim=0)])
