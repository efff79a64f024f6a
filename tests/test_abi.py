"""The C-ABI library loads on a CPU-only host and exports what the header declares.

No compute call is made here (no GPU needed).
"""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared() -> set[str]:
    names: set[str] = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(skv_\w+)\s*\(", text, flags=re.M))
    return names


def test_header_declares_entry_points() -> None:
    names = _declared()
    assert "skv_abi_version" in names and "skv_last_error" in names
    assert len(names) >= 7


def test_library_exports_every_declared_symbol() -> None:
    from saint_kv import _lib

    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (skv_\w+)", out))
    assert _declared() <= exported
    # every exported skv_ symbol is declared in a header (no hidden ABI)
    assert exported <= _declared()


def test_python_signatures_cover_the_header() -> None:
    from saint_kv import _lib

    assert set(_lib.SIGNATURES) | {"skv_last_error"} == _declared()


def test_abi_version_and_error_text() -> None:
    from saint_kv import _lib

    lib = _lib.load()
    assert lib.skv_abi_version() == 1
    # an argument error is reported without touching the GPU
    rc = lib.skv_free_stack_init(None, None, None, 0, None)
    assert rc == _lib.SKV_EINVAL
    assert "n_pages" in _lib.last_error()
    with pytest.raises(ValueError, match="n_pages"):
        _lib.check(rc, "skv_free_stack_init")


def test_argument_errors_map_to_value_error() -> None:
    from saint_kv import _lib

    lib = _lib.load()
    rc = lib.skv_paged_gather(None, None, 0, 0, None, 24, 16, 1, None, 1, None, 1, None)
    assert rc == _lib.SKV_EINVAL and "row_bytes" in _lib.last_error()
    rc = lib.skv_reserve(None, None, 8, None, 4, 8, None, None, 1, 1, 16, None, None)
    assert rc == _lib.SKV_EINVAL and "max_pages" in _lib.last_error()
    fake = 16  # never dereferenced: the sizes are refused first
    rc = lib.skv_indexer_scores(fake, fake, fake, 16, 8, fake, 4, fake, fake, 64, 2, 1, 65, 128, 64, None)
    assert rc == _lib.SKV_EINVAL and "n_heads" in _lib.last_error()
    rc = lib.skv_indexer_scores(fake, fake, fake, 16, 8, fake, 4, fake, fake, 64, 2, 1, 64, 100, 64, None)
    assert rc == _lib.SKV_EINVAL and "channels" in _lib.last_error()


def test_attention_descriptor_and_workspace() -> None:
    """skv_attention_desc layout and the host-only workspace query: its size
    formula and the argument checks that precede any device work."""
    import ctypes

    from saint_kv import _lib
    from saint_kv.attention import KIND, AttentionDesc

    lib = _lib.load()
    assert lib.skv_attention_desc_size() == ctypes.sizeof(AttentionDesc)
    d = AttentionDesc()
    d.kind, d.format = KIND["csa"], _lib.SKV_FMT_BF16
    d.batch, d.n_heads, d.head_dim = 16, 64, 576
    d.entry_bytes, d.block_size, d.n_pages, d.bt_stride = 1152, 64, 4096, 256
    d.pick_stride = d.top_k = 512
    d.window = 128
    ws = lib.skv_attention_workspace(ctypes.byref(d))
    # units x 64 heads x ((max, sum) fp32 + head_dim bf16), units a multiple of the batch
    per_unit = 64 * (8 + 2 * 576)
    assert ws > 0 and ws % (16 * per_unit) == 0 and ws // per_unit <= 16 * 64
    d.splits = 3
    assert lib.skv_attention_workspace(ctypes.byref(d)) % per_unit == 0
    for field, value, msg in (("head_dim", 100, "head_dim"), ("n_heads", 300, "n_heads"),
                              ("window", 0, "window"), ("top_k", 600, "top_k")):
        bad = AttentionDesc.from_buffer_copy(d)
        setattr(bad, field, value)
        assert lib.skv_attention_workspace(ctypes.byref(bad)) == -1
        assert msg in _lib.last_error()
    bad = AttentionDesc.from_buffer_copy(d)
    bad.format, bad.head_dim, bad.entry_bytes = _lib.SKV_FMT_FP8, 320, _lib.fp8_entry_bytes(320)
    assert lib.skv_attention_workspace(ctypes.byref(bad)) == -1 and "fp8" in _lib.last_error()
    bad = AttentionDesc.from_buffer_copy(d)
    bad.kind, bad.m = KIND["hca"], 0
    assert lib.skv_attention_workspace(ctypes.byref(bad)) == -1 and "m >= 1" in _lib.last_error()
    # T query tokens per sequence: units per query row (a multiple of the 64
    # rows), and the window's ring and slot stride
    multi = AttentionDesc.from_buffer_copy(d)
    multi.n_queries, multi.ring, multi.win_stride = 4, 131, 4 * 576
    ws_multi = lib.skv_attention_workspace(ctypes.byref(multi))
    assert ws_multi > 0 and ws_multi % (64 * per_unit) == 0
    for field, value, msg in (("n_queries", -1, "n_queries"), ("n_queries", 5000, "n_queries"),
                              ("ring", 100, "ring"), ("win_stride", 1000, "win_stride"),
                              ("win_stride", 1160, "win_stride")):
        bad = AttentionDesc.from_buffer_copy(multi)
        setattr(bad, field, value)
        assert lib.skv_attention_workspace(ctypes.byref(bad)) == -1
        assert msg in _lib.last_error()


def test_single_hip_runtime_mapped() -> None:
    """The library binds to the HIP runtime torch already mapped (one libamdhip64)."""
    import torch  # noqa: F401

    from saint_kv import _lib

    _lib.load()
    maps = Path("/proc/self/maps").read_text()
    libs = {ln.split()[-1] for ln in maps.splitlines() if "libamdhip64" in ln}
    assert len(libs) == 1, libs


def test_decode_step_score_fields_checked_on_host() -> None:
    """skv_decode_step refuses, before any device work, a step whose CSA
    layers disagree on computing their scores (idx_q), or whose step scores
    lack the indexer stream or exceed 64 heads.  The pointers are never
    dereferenced on these paths (placeholders)."""
    import ctypes

    from saint_kv import _lib
    from saint_kv.decode import DecodeDescC

    lib = _lib.load()
    fake = 0x1000  # placeholder address: the checks fail before any use
    d = DecodeDescC()
    d.batch, d.n_layers, d.n_groups = 2, 2, 1
    d.latent, d.c_indexer, d.window = 576, 128, 128
    d.tok_lens = d.status = d.step_lens = d.step_top = fake
    G = d.groups[0]
    G.free_stack = G.free_top = G.block_table = G.n_entries = fake
    G.n_pages, G.bt_stride, G.m, G.block_size = 64, 8, 4, 64
    for i in range(2):
        Ly = d.layers[i]
        Ly.kind, Ly.group, Ly.format, Ly.top_k = 2, 0, _lib.SKV_FMT_BF16, 16  # CSA
        Ly.ring = Ly.kv_new = Ly.out_window = Ly.pool = Ly.state = Ly.bias = fake
        Ly.c_new = Ly.z_new = Ly.out_entries = Ly.scores = Ly.topk_idx = Ly.topk_ws = fake
        Ly.entry_bytes, Ly.score_stride = 1152, 128
        Ly.idx_pool = Ly.idx_state = Ly.idx_bias = Ly.ci_new = Ly.zi_new = fake

    def step(desc):
        return lib.skv_decode_step(ctypes.byref(desc), ctypes.c_void_p(fake), None)

    one = DecodeDescC.from_buffer_copy(d)
    one.layers[0].idx_q, one.layers[0].idx_w, one.layers[0].idx_heads = fake, fake, 8
    assert step(one) == _lib.SKV_EINVAL and "every CSA layer" in _lib.last_error()
    many = DecodeDescC.from_buffer_copy(one)
    many.layers[1].idx_q, many.layers[1].idx_w, many.layers[1].idx_heads = fake, fake, 65
    assert step(many) == _lib.SKV_EINVAL and "idx_heads" in _lib.last_error()
    no_stream = DecodeDescC.from_buffer_copy(one)
    no_stream.layers[1].idx_q, no_stream.layers[1].idx_w, no_stream.layers[1].idx_heads = fake, fake, 8
    no_stream.layers[1].idx_pool = None
    assert step(no_stream) == _lib.SKV_EINVAL


def test_step_attend_checked_on_host() -> None:
    """skv_decode_step_attend's workspace query and argument checks run on the
    host before any device work: one layer, no gathered copies, head_dim equal
    to the latent, the batch of the step, a workspace large enough.  Pointers
    are placeholders, never dereferenced on these paths."""
    import ctypes

    from saint_kv import _lib
    from saint_kv.attention import KIND, AttentionDesc
    from saint_kv.decode import DecodeDescC

    lib = _lib.load()
    fake = 0x1000
    d = DecodeDescC()
    d.batch, d.n_layers, d.n_groups = 16, 1, 1
    d.latent, d.c_indexer, d.window = 576, 128, 128
    d.tok_lens = d.status = d.step_lens = d.step_top = fake
    G = d.groups[0]
    G.free_stack = G.free_top = G.block_table = G.n_entries = fake
    G.n_pages, G.bt_stride, G.m, G.block_size = 4096, 256, 4, 64
    Ly = d.layers[0]
    Ly.kind, Ly.group, Ly.format, Ly.top_k = KIND["csa"], 0, _lib.SKV_FMT_BF16, 512
    Ly.ring = Ly.kv_new = Ly.pool = Ly.state = Ly.bias = fake
    Ly.c_new = Ly.z_new = Ly.scores = Ly.topk_idx = Ly.topk_ws = fake
    Ly.entry_bytes, Ly.score_stride = 1152, 16384
    Ly.idx_pool = Ly.idx_state = Ly.idx_bias = Ly.ci_new = Ly.zi_new = fake
    a = AttentionDesc()
    a.batch, a.n_heads, a.head_dim = 16, 64, 576
    a.q = a.out = a.knorm_w = fake
    ws = lib.skv_decode_step_attend_workspace(ctypes.byref(d), ctypes.byref(a))
    # the same units as skv_decode_attention over the layer: a multiple of the batch
    per_unit = 64 * (8 + 2 * 576)
    assert ws > 0 and ws % (16 * per_unit) == 0

    def call(desc, attn, ws_bytes=ws):
        return lib.skv_decode_step_attend(ctypes.byref(desc), ctypes.c_void_p(fake), ctypes.byref(attn),
                                          ctypes.c_void_p(fake), ws_bytes, None)

    assert call(d, a, ws - 16) == _lib.SKV_EINVAL and "workspace" in _lib.last_error()
    two = DecodeDescC.from_buffer_copy(d)
    two.n_layers = 2
    two.layers[1] = d.layers[0]
    assert call(two, a) == _lib.SKV_EINVAL and "one layer" in _lib.last_error()
    assert lib.skv_decode_step_attend_workspace(ctypes.byref(two), ctypes.byref(a)) == -1
    copies = DecodeDescC.from_buffer_copy(d)
    copies.layers[0].out_window = fake
    assert call(copies, a) == _lib.SKV_EINVAL and "gathered copies" in _lib.last_error()
    for field, value in (("head_dim", 512), ("batch", 8)):
        bad = AttentionDesc.from_buffer_copy(a)
        setattr(bad, field, value)
        assert call(d, bad) == _lib.SKV_EINVAL and "head_dim" in _lib.last_error()
    no_q = AttentionDesc.from_buffer_copy(a)
    no_q.q = None
    assert call(d, no_q) == _lib.SKV_EINVAL
    assert lib.skv_decode_step_attend(ctypes.byref(d), ctypes.c_void_p(fake), None, None, 0, None) == _lib.SKV_EINVAL
