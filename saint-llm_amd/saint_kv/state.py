"""Per-request persistence of a DecodeCache sequence: the state cache and the
compressed KV of one request, on disk.

The reference plans this module and its layout without implementing it
(``saint_llm_inference/__init__.py:6-7``: "kv_cache.state — State cache for
SWA + uncompressed CSA/HCA tail tokens", "kv_cache.on_disk — Three SWA
strategies (Full / Periodic / Zero)"; the layout figure
``docs/img/Screenshot 2026-04-25 at 12.08.35.png``: per request, the SWA KV of
every layer and the uncompressed tail state of every CSA/HCA layer; per block,
the CSA main and indexer entries and the HCA entries).  A snapshot of sequence
b at length L holds:

* every compressed entry of every CSA/HCA layer (main and indexer streams,
  bf16 or fp8 bytes as stored), gathered from the pages by ``skv_paged_gather``;
* the tail state of every CSA/HCA stream (the online-softmax state of the
  incomplete block, fp32 [3, channels]), the "uncompressed KV state";
* the SWA rows of every layer, by strategy:
  - ``"full"``: the last min(W, L) rows: the request resumes exactly;
  - ``"periodic"`` (period p): the rows up to the last multiple of p the ring
    still holds; the caller recomputes the rest;
  - ``"zero"``: none; the caller recomputes the last min(W, L) rows.

``load_sequence`` writes a snapshot into an empty slot of a cache with the same
layout: it pops pages from the free lists (``skv_reserve``), writes the
entries into them (``skv_paged_append``), the tail states, and the stored SWA
rows (``skv_ring_append``), and returns the positions whose SWA rows the
caller must append (``ops.ring_append``) before the next step.

File layout (little-endian): the 8 magic bytes ``SKVSTATE``, a uint32
format version, a uint32 header length, the UTF-8 JSON header, then the
sections in header order, each padded to 16 bytes.
"""

from __future__ import annotations

import json
import struct
from pathlib import Path

import torch

from saint_kv import ops

MAGIC = b"SKVSTATE"
VERSION = 1
STRATEGIES = ("full", "periodic", "zero")
_DTYPES = {"bfloat16": torch.bfloat16, "uint8": torch.uint8, "float32": torch.float32}


def _layout(cache) -> dict:
    return {
        "latent": cache.latent, "c_indexer": cache.c_indexer, "window": cache.window,
        "block_size": cache.block_size,
        "layers": [{"kind": s.kind, "m": s.m, "top_k": s.top_k, "fp8": s.fp8, "indexer": s.indexer}
                   for s in cache.layers],
    }


def swa_rows_kept(L: int, window: int, swa: str, period: int | None) -> tuple[int, int]:
    """Positions [lo, hi) of the SWA rows a snapshot at length L keeps."""
    lo = L - min(window, L)
    if swa == "full":
        return lo, L
    if swa == "zero":
        return lo, lo
    if period is None or period <= 0:
        raise ValueError("the periodic strategy needs a positive period")
    return lo, max(lo, L - L % period)


def _streams(cache, i: int):
    """(section suffix, pool, state, channels) of layer i's compressed streams."""
    s = cache.layers[i]
    out = [("", cache.pool[i], cache.state[i], cache.latent)]
    if s.kind == "csa" and s.indexer:
        out.append(("_idx", cache.idx_pool[i], cache.idx_state[i], cache.c_indexer))
    return out


def save_sequence(cache, b: int, path: str | Path, swa: str = "full", period: int | None = None) -> dict:
    """Write sequence b's snapshot to ``path``; returns the header."""
    if swa not in STRATEGIES:
        raise ValueError(f"swa must be one of {STRATEGIES}; got {swa!r}")
    if not 0 <= b < cache.batch:
        raise ValueError(f"sequence {b} out of range")
    L = int(cache.host_lens[b])
    dev = cache.device
    lo, hi = swa_rows_kept(L, cache.window, swa, period)
    tensors: list[tuple[str, int, torch.Tensor]] = []
    lens_b = torch.tensor([L], dtype=torch.int32, device=dev)
    for i, spec in enumerate(cache.layers):
        if hi > lo:
            rows = torch.empty(1, L - lo, cache.latent, dtype=torch.bfloat16, device=dev)
            ops.ring_read(cache.ring[i][b:b + 1], lens_b, rows)
            tensors.append(("swa", i, rows[0, :hi - lo]))
        if spec.kind == "swa":
            continue
        g = cache.groups[cache.group_of_rate[spec.m]]
        n_ent = L // spec.m
        n_t = torch.tensor([n_ent], dtype=torch.int32, device=dev)
        for suffix, pool, state, _ in _streams(cache, i):
            ent = torch.empty(1, max(n_ent, 1), *pool.shape[2:], dtype=pool.dtype, device=dev)
            ops.paged_gather(pool, g.block_table[b:b + 1], n_t, ent)
            tensors.append(("entries" + suffix, i, ent[0, :n_ent]))
            tensors.append(("state" + suffix, i, state[b]))
    # one pinned host buffer, filled by asynchronous copies, one synchronisation
    sections, off = [], 0
    for name, layer, t in tensors:
        nbytes = t.numel() * t.element_size()
        sections.append({"name": name, "layer": layer, "dtype": str(t.dtype).replace("torch.", ""),
                         "shape": list(t.shape), "offset": off, "nbytes": nbytes})
        off += nbytes + (-nbytes) % 16
    host = torch.zeros(max(off, 16), dtype=torch.uint8, pin_memory=True)
    for sec, (_, _, t) in zip(sections, tensors):
        if sec["nbytes"]:
            host[sec["offset"]:sec["offset"] + sec["nbytes"]].copy_(
                t.contiguous().view(-1).view(torch.uint8), non_blocking=True)
    torch.cuda.current_stream(dev).synchronize()
    header = {"layout": _layout(cache), "length": L, "swa": swa, "period": period, "swa_rows": [lo, hi],
              "sections": sections}
    hdr = json.dumps(header, sort_keys=True).encode()
    with open(path, "wb") as f:
        f.write(MAGIC + struct.pack("<II", VERSION, len(hdr)) + hdr)
        f.write(b"\0" * ((-(16 + len(hdr))) % 16))
        f.write(memoryview(host.numpy())[:off])
    return header


def read_header(path: str | Path) -> tuple[dict, int]:
    """The header of a snapshot and the file offset of its first section."""
    with open(path, "rb") as f:
        head = f.read(16)
        if len(head) < 16 or head[:8] != MAGIC:
            raise ValueError(f"{path}: not a saint_kv state snapshot")
        version, n = struct.unpack("<II", head[8:])
        if version != VERSION:
            raise ValueError(f"{path}: snapshot format version {version}, expected {VERSION}")
        hdr = f.read(n)
        if len(hdr) != n:
            raise ValueError(f"{path}: truncated header")
    return json.loads(hdr), 16 + n + (-(16 + n)) % 16


def load_sequence(cache, b: int, path: str | Path) -> tuple[int, int]:
    """Write a snapshot into the empty slot b; returns the positions [lo, hi)
    whose SWA rows the caller must append (``ops.ring_append`` of every
    layer's ring) before the next step, empty for a full snapshot."""
    header, base = read_header(path)
    if header["layout"] != _layout(cache):
        raise ValueError("snapshot layout (channels, window, block size, layer specs) differs from the cache's")
    if not 0 <= b < cache.batch:
        raise ValueError(f"sequence {b} out of range")
    if cache.host_lens[b] != 0:
        raise RuntimeError(f"sequence {b} is not empty; release it first")
    L = int(header["length"])
    if L > cache.max_len:
        raise ValueError(f"snapshot length {L} exceeds max_len={cache.max_len}")
    dev = cache.device
    sec = {(s["name"], s["layer"]): s for s in header["sections"]}
    # the sections into one pinned buffer, then one device buffer
    end = max([s["offset"] + s["nbytes"] for s in header["sections"]] + [0])
    host = torch.empty(max(end, 16), dtype=torch.uint8, pin_memory=True)
    with open(path, "rb") as f:
        f.seek(base)
        if f.readinto(memoryview(host.numpy())[:end]) < end:
            raise ValueError(f"{path}: truncated sections")
    blob = host.to(dev, non_blocking=True)

    def tensor(name: str, layer: int) -> torch.Tensor:
        s = sec[(name, layer)]
        t = blob[s["offset"]: s["offset"] + s["nbytes"]]
        return t.view(_DTYPES[s["dtype"]]).reshape(s["shape"])

    # pages for the entries, from each page group's free list; on a refusal
    # the slot is left empty and every group's free list as it was
    cache.reserve_entries(slice(b, b + 1), [L // g.m for g in cache.groups])
    lo, hi = header["swa_rows"]
    for i, spec in enumerate(cache.layers):
        if hi > lo:
            rows = tensor("swa", i)
            ops.ring_append(cache.ring[i][b:b + 1], torch.tensor([hi], dtype=torch.int32, device=dev),
                            rows.unsqueeze(0), hi - lo)
        if spec.kind == "swa":
            continue
        g = cache.groups[cache.group_of_rate[spec.m]]
        n_ent = L // spec.m
        for suffix, pool, state, _ in _streams(cache, i):
            if n_ent:
                ops.paged_append(pool, g.block_table[b:b + 1], g.n_entries[b:b + 1],
                                 tensor("entries" + suffix, i).unsqueeze(0), n_ent)
            state[b].copy_(tensor("state" + suffix, i))
    cache.tok_lens[b] = L
    cache.host_lens[b] = L
    torch.cuda.current_stream(dev).synchronize()  # the pinned buffer is read until here
    return (hi, L) if hi < L else (L, L)
