"""skv_decode_append_gather_noalloc: the allocation-free decode step.

The entry point keeps its page-unit table in the library's static device
array instead of a caller workspace.  Its results must equal those of
skv_decode_append_gather (the workspace form) bit for bit: output rows, pool,
block tables, lengths, free stack and status, on two calls in a row, the
second smaller than the first (the static table still holds the first call's
units), and on a refusal.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

ROW = 576  # bf16 channels of a latent row (1152 bytes)


def _state(dev, lens: np.ndarray, n_pages: int, bs: int, seed: int) -> dict:
    from saint_kv import ops

    g = torch.Generator(device=dev).manual_seed(seed)
    batch = len(lens)
    bt_stride = int(-(-(lens.max() + 8) // bs))
    st = {
        "stack": torch.empty(n_pages, dtype=torch.int32, device=dev),
        "top": torch.empty(1, dtype=torch.int32, device=dev),
        "bt": torch.full((batch, bt_stride), -1, dtype=torch.int32, device=dev),
        "lens": torch.zeros(batch, dtype=torch.int32, device=dev),
        "pool": torch.empty(n_pages, bs, ROW, dtype=torch.bfloat16, device=dev).normal_(generator=g),
        "status": torch.full((1,), -7, dtype=torch.int32, device=dev),
    }
    order = torch.as_tensor(np.random.default_rng(seed).permutation(n_pages).astype(np.int32), device=dev)
    ops.free_stack_init(st["stack"], st["top"], order)
    n0 = torch.as_tensor(lens.astype(np.int32), device=dev)
    ops.reserve(st["stack"], st["top"], st["bt"], st["lens"], n0, bs)
    src = torch.empty(batch, int(lens.max()), ROW, dtype=torch.bfloat16, device=dev).normal_(generator=g)
    ops.paged_append(st["pool"], st["bt"], st["lens"], src, n0)
    return st


def _clone(st: dict) -> dict:
    return {k: v.clone() for k, v in st.items()}


def _step(dev, st: dict, noalloc: bool, tok: torch.Tensor, max_units: int, out_rows: int) -> torch.Tensor:
    from saint_kv import ops

    out = torch.zeros(st["bt"].shape[0], out_rows, ROW, dtype=torch.bfloat16, device=dev)
    args = (st["stack"], st["top"], st["bt"], st["lens"], st["pool"], tok, 1, out)
    if noalloc:
        ops.decode_append_gather_noalloc(*args, max_units, status=st["status"])
    else:
        units = ops.unit_table(max_units, dev)
        ops.decode_append_gather(*args, units, max_units, status=st["status"])
    return out


def _assert_same(a: dict, b: dict, out_a: torch.Tensor, out_b: torch.Tensor, what: str) -> None:
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b), f"{what}: gathered rows differ"
    for k in ("stack", "top", "bt", "lens", "pool", "status"):
        assert torch.equal(a[k], b[k]), f"{what}: {k} differs"


@pytest.mark.gpu
def test_noalloc_matches_workspace_form(dev) -> None:
    from saint_kv import ops

    rng = np.random.default_rng(11)
    bs = 64
    # call 1: 24 sequences of up to 3000 rows (about 700 page units)
    lens1 = rng.integers(100, 3000, size=24)
    lens1[3] = 64 * 20  # a full last page: the new row opens a page
    a = _state(dev, lens1, 2048, bs, seed=1)
    n = _clone(a)
    tok1 = torch.randn(24, 1, ROW, device=dev).to(torch.bfloat16)
    units1 = int((-(-(lens1 + 1) // bs)).sum())
    big = units1 + 64
    out_a = _step(dev, a, False, tok1, big, int(lens1.max()) + 1)
    out_n = _step(dev, n, True, tok1, big, int(lens1.max()) + 1)
    _assert_same(a, n, out_a, out_n, "call 1")
    assert int(n["status"].item()) == 0
    assert torch.equal(n["lens"].cpu(), torch.as_tensor(lens1 + 1, dtype=torch.int32))

    # call 2: a smaller batch and shorter sequences; the launch still covers
    # `big` units, so the static table's stale units of call 1 past the new
    # count must not be copied
    lens2 = rng.integers(1, 300, size=5)
    a2 = _state(dev, lens2, 64, bs, seed=2)
    n2 = _clone(a2)
    tok2 = torch.randn(5, 1, ROW, device=dev).to(torch.bfloat16)
    out_a2 = _step(dev, a2, False, tok2, big, int(lens2.max()) + 1)
    out_n2 = _step(dev, n2, True, tok2, big, int(lens2.max()) + 1)
    _assert_same(a2, n2, out_a2, out_n2, "call 2")
    assert int(n2["status"].item()) == 0

    # call 3: a unit bound below the step's units is refused (SKV_STATUS_UNITS):
    # nothing changes and nothing is copied, in both forms
    a3, n3 = _clone(a2), _clone(a2)
    out_a3 = _step(dev, a3, False, tok2, 2, int(lens2.max()) + 2)
    out_n3 = _step(dev, n3, True, tok2, 2, int(lens2.max()) + 2)
    _assert_same(a3, n3, out_a3, out_n3, "refused call")
    assert int(n3["status"].item()) == 16  # SKV_STATUS_UNITS
    assert torch.equal(n3["lens"], a2["lens"]) and torch.equal(n3["bt"], a2["bt"])
    assert not out_n3.any()


def test_noalloc_refuses_oversized_unit_bound() -> None:
    """max_units past the static table is refused before any device work."""
    from saint_kv import _lib

    lib = _lib.load()
    fake = ctypes.c_void_p(16)
    rc = lib.skv_decode_append_gather_noalloc(
        fake, fake, 8, fake, 4, fake, None, 1, None, fake, None, 4, 64, fake, 1152, 64, fake, 1152, 1152,
        1, 65537, 2, None)
    assert rc == _lib.SKV_EINVAL and "max_units" in _lib.last_error()
    rc = lib.skv_decode_append_gather_noalloc(
        fake, fake, 8, fake, 4, fake, None, 1, None, fake, None, 4, 64, fake, 1152, 64, fake, 1152, 1152,
        1, -1, 2, None)
    assert rc == _lib.SKV_EINVAL
