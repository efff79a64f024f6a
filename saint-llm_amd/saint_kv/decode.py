"""Heterogeneous paged KV cache for batched decode (ragged sequences).

``DecodeCache`` holds, for a stack of CSA / HCA / SWA layers:

* per layer an SWA ring of the last ``window`` latent rows (bf16);
* per CSA/HCA layer a paged compressed cache (bf16 or FP8 entries) whose page
  ids come from the free stack of the layer's page group (one group per
  compression rate; layers of a group share the block table, as their entry
  counts advance in lockstep), plus the fp32 running pooling state of the
  block being filled;
* per CSA layer the indexer stream (bf16 entries, same pages).

``step()`` runs one decode step for every sequence through the fused C-ABI
entry point ``skv_decode_step`` (three launches).  The per-step inputs live in
fixed device buffers (``inputs``), so a sequence of steps can be captured in a
HIP graph and replayed.

Reference: the per-layer caches of kv_cache.py:32-327 composed as
KVCacheBundle (kv_cache.py:333-427) and driven by the cached decode loop
(generate.py:113-126, model.py:294-315).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from saint_kv import _lib, ops

KIND = {"swa": 0, "hca": 1, "csa": 2}
MAX_LAYERS = 16
MAX_GROUPS = 4
MAX_BATCH = 1024

_P = ctypes.c_void_p


class PageGroupC(ctypes.Structure):
    _fields_ = [
        ("free_stack", _P), ("free_top", _P), ("n_pages", ctypes.c_int64),
        ("block_table", _P), ("bt_stride", ctypes.c_int64), ("n_entries", _P),
        ("m", ctypes.c_int32), ("block_size", ctypes.c_int32),
    ]


class DecodeLayerC(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32), ("group", ctypes.c_int32), ("format", ctypes.c_int32),
        ("top_k", ctypes.c_int32), ("ring", _P), ("pool", _P), ("entry_bytes", ctypes.c_int64),
        ("state", _P), ("bias", _P), ("idx_pool", _P), ("idx_state", _P), ("idx_bias", _P),
        ("kv_new", _P), ("c_new", _P), ("z_new", _P), ("ci_new", _P), ("zi_new", _P),
        ("scores", _P), ("score_stride", ctypes.c_int64), ("topk_idx", _P), ("topk_ws", _P),
        ("out_entries", _P), ("out_rows", ctypes.c_int64), ("out_window", _P),
        ("idx_q", _P), ("idx_w", _P), ("idx_heads", ctypes.c_int32), ("idx_pad_", ctypes.c_int32),
    ]


class DecodeDescC(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("n_layers", ctypes.c_int32), ("n_groups", ctypes.c_int32),
        ("latent", ctypes.c_int32), ("c_indexer", ctypes.c_int32), ("window", ctypes.c_int32),
        ("tok_lens", _P), ("status", _P), ("step_lens", _P), ("step_top", _P),
        ("groups", PageGroupC * MAX_GROUPS), ("layers", DecodeLayerC * MAX_LAYERS),
    ]


def check_struct_layout() -> None:
    """Raise if the ctypes mirrors disagree with the library's struct sizes."""
    sizes = (ctypes.c_int64 * 3)()
    _lib.call("skv_decode_desc_sizes", ctypes.cast(sizes, ctypes.c_void_p))
    mine = (ctypes.sizeof(DecodeDescC), ctypes.sizeof(DecodeLayerC), ctypes.sizeof(PageGroupC))
    if tuple(sizes) != mine:
        raise RuntimeError(f"decode descriptor layout mismatch: library {tuple(sizes)} vs ctypes {mine}")


@dataclass(frozen=True)
class LayerSpec:
    """One attention layer's cache: kind "csa" | "hca" | "swa"."""

    kind: str
    m: int = 4
    top_k: int = 512
    fp8: bool = False
    indexer: bool = True
    # CSA with an indexer: > 0 makes the step compute the layer's scores from
    # inputs["iq"] (bf16 [batch, idx_heads, c_indexer]) and inputs["iw"]
    # (fp32 [batch, idx_heads]) instead of reading them from ``scores``
    idx_heads: int = 0


@dataclass
class _Group:
    m: int
    n_pages: int
    free_stack: torch.Tensor
    free_top: torch.Tensor
    block_table: torch.Tensor
    n_entries: torch.Tensor


class DecodeCache:
    """Paged heterogeneous cache of ``batch`` ragged sequences on one GPU.

    ``score_cols`` sets the width of each CSA layer's indexer-score buffer
    (default ``max_len // m`` rounded up to a multiple of 4); the step reads
    only the first ``L // m`` columns of a row.

    ``input_sets`` > 1 allocates that many sets of per-step input buffers
    (``inputs_by_set[k]``: the new tokens' rows; ``scores_by_set[k]``: the CSA
    scores), each with its own descriptor: ``step(k)`` reads set k, and a
    captured sequence of steps cycles through the sets, so that a caller can
    stage the next steps' inputs while earlier ones run.  ``inputs`` and
    ``scores`` are set 0.

    ``materialize=False`` drops the gathered copies (``out_entries`` of
    CSA/HCA layers and ``out_window``): the step then writes the top-k
    indices, pools, states, rings and lengths only, which is all a consumer
    reading the cache in place (``attention``) needs.
    """

    def __init__(self, layers: list[LayerSpec], batch: int, max_len: int, *,
                 latent: int = 576, c_indexer: int = 128, window: int = 128,
                 block_size: int = 64, device: torch.device | str | None = None,
                 page_order_seed: int | None = 0, pages_per_group: dict[int, int] | None = None,
                 hca_out_rows: int | None = None, score_cols: int | None = None,
                 input_sets: int = 1, materialize: bool = True) -> None:
        if not 0 < len(layers) <= MAX_LAYERS:
            raise ValueError(f"1..{MAX_LAYERS} layers supported; got {len(layers)}")
        scored = [s.idx_heads > 0 for s in layers if s.kind == "csa"]
        if any(scored) and not all(scored):
            raise ValueError("either every CSA layer computes its scores in the step (idx_heads > 0) or none does")
        if any(not 0 <= s.idx_heads <= 64 for s in layers):
            raise ValueError("idx_heads must be in [0, 64]")
        if not 0 < batch <= MAX_BATCH:
            raise ValueError(f"batch must be in [1, {MAX_BATCH}]; got {batch}")
        if max_len <= 0:
            raise ValueError(f"max_len must be positive; got {max_len}")
        if input_sets < 1:
            raise ValueError(f"input_sets must be positive; got {input_sets}")
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError("DecodeCache runs only on a ROCm GPU (no CPU fallback)")
        _lib.load()
        check_struct_layout()
        self.device = dev
        self.layers = list(layers)
        self.batch, self.max_len = batch, max_len
        self.latent, self.c_indexer, self.window, self.block_size = latent, c_indexer, window, block_size
        self.tok_lens = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)

        self.step_lens = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.step_top = torch.zeros(MAX_GROUPS, dtype=torch.int32, device=dev)
        # one status word per page group for the host-driven reserve / release
        # calls (a later group's success must not hide an earlier refusal)
        self.group_status = torch.zeros(MAX_GROUPS, dtype=torch.int32, device=dev)
        self.host_lens = np.zeros(batch, dtype=np.int64)
        self._attn_ws: dict[int | str, torch.Tensor] = {}  # per layer, and "step" for step_attend

        # page groups: one per compression rate
        rates = sorted({s.m for s in layers if s.kind in ("csa", "hca")})
        if len(rates) > MAX_GROUPS:
            raise ValueError(f"at most {MAX_GROUPS} distinct compression rates")
        self.groups: list[_Group] = []
        self.group_of_rate = {}
        rng = np.random.default_rng(page_order_seed) if page_order_seed is not None else None
        for m in rates:
            max_entries = max_len // m
            bt_stride = max(1, -(-max_entries // block_size))
            n_pages = (pages_per_group or {}).get(m, batch * bt_stride)
            stack = torch.empty(n_pages, dtype=torch.int32, device=dev)
            top = torch.empty(1, dtype=torch.int32, device=dev)
            order = None if rng is None else torch.as_tensor(
                rng.permutation(n_pages).astype(np.int32), device=dev)
            ops.free_stack_init(stack, top, order)
            self.group_of_rate[m] = len(self.groups)
            self.groups.append(_Group(
                m=m, n_pages=n_pages, free_stack=stack, free_top=top,
                block_table=torch.full((batch, bt_stride), -1, dtype=torch.int32, device=dev),
                n_entries=torch.zeros(batch, dtype=torch.int32, device=dev)))
        # compaction buffers: zeroed once; each page group has its own slice of
        # the workspace, whose page marks the compaction leaves zero
        self._compact_info = torch.zeros(max(len(self.groups), 1), 2, dtype=torch.int32, device=dev)
        self._compact_ws = torch.zeros(max(self.compact_workspace_words(), 1), dtype=torch.int32, device=dev)

        bf = torch.bfloat16
        self.ring, self.pool, self.state, self.bias = [], [], [], []
        self.idx_pool, self.idx_state, self.idx_bias = [], [], []
        self.inputs_by_set: list[list[dict[str, torch.Tensor]]] = [[] for _ in range(input_sets)]
        self.scores_by_set: list[list[torch.Tensor | None]] = [[] for _ in range(input_sets)]
        self.topk_idx, self.out_entries, self.out_window = [], [], []
        self.topk_ws = []
        for spec in layers:
            if spec.kind not in KIND:
                raise ValueError(f"unknown layer kind {spec.kind!r}")
            self.ring.append(torch.zeros(batch, window, latent, dtype=bf, device=dev))
            self.out_window.append(torch.zeros(batch, window, latent, dtype=bf, device=dev) if materialize else None)
            inp = {"kv": (batch, latent)}  # shapes; one tensor per input set below
            pool = state = bias = ipool = istate = ibias = sc = tk = oe = ws = None
            if spec.kind in ("csa", "hca"):
                g = self.groups[self.group_of_rate[spec.m]]
                if spec.fp8:
                    pool = torch.zeros(g.n_pages, block_size, _lib.fp8_entry_bytes(latent),
                                       dtype=torch.uint8, device=dev)
                else:
                    pool = torch.zeros(g.n_pages, block_size, latent, dtype=bf, device=dev)
                state = torch.zeros(batch, 3, latent, dtype=torch.float32, device=dev)
                bias = torch.zeros(spec.m, latent, dtype=torch.float32, device=dev)
                inp["c"] = inp["z"] = (batch, latent)
                if spec.kind == "csa":
                    if spec.indexer:
                        ipool = torch.zeros(g.n_pages, block_size, c_indexer, dtype=bf, device=dev)
                        istate = torch.zeros(batch, 3, c_indexer, dtype=torch.float32, device=dev)
                        ibias = torch.zeros(spec.m, c_indexer, dtype=torch.float32, device=dev)
                        inp["ci"] = inp["zi"] = (batch, c_indexer)
                        if spec.idx_heads > 0:
                            inp["iq"] = (batch, spec.idx_heads, c_indexer)
                            inp["iw"] = (batch, spec.idx_heads)
                    elif spec.idx_heads > 0:
                        raise ValueError("idx_heads needs the layer's indexer stream (indexer=True)")
                    # default width rounded up to 4 columns (16-byte rows)
                    cols = -(-max(1, max_len // spec.m) // 4) * 4 if score_cols is None else int(score_cols)
                    if cols < max_len // spec.m:
                        raise ValueError(f"score_cols must be >= max_len // m = {max_len // spec.m}")
                    sc = (batch, cols)
                    tk = torch.full((batch, spec.top_k), -1, dtype=torch.int32, device=dev)
                    ws = ops.topk_workspace(batch, dev)
                    oe = torch.zeros(batch, spec.top_k, latent, dtype=bf, device=dev) if materialize else None
                elif materialize:
                    rows = hca_out_rows or max(1, max_len // spec.m)
                    oe = torch.zeros(batch, rows, latent, dtype=bf, device=dev)
            self.pool.append(pool)
            self.state.append(state)
            self.bias.append(bias)
            self.idx_pool.append(ipool)
            self.idx_state.append(istate)
            self.idx_bias.append(ibias)
            for k in range(input_sets):
                self.inputs_by_set[k].append({
                    n: torch.zeros(shp, dtype=torch.float32 if n == "iw" else bf, device=dev)
                    for n, shp in inp.items()})
                self.scores_by_set[k].append(
                    None if sc is None else torch.zeros(sc, dtype=torch.float32, device=dev))
            self.topk_idx.append(tk)
            self.topk_ws.append(ws)
            self.out_entries.append(oe)
        self.inputs = self.inputs_by_set[0]
        self.scores = self.scores_by_set[0]
        self._descs = [self._build_desc(k) for k in range(input_sets)]
        self._desc, self._desc_dev = self._descs[0]

    @property
    def n_input_sets(self) -> int:
        return len(self.inputs_by_set)

    def step_launches(self) -> int:
        """Kernel launches of one step, as skv_decode_step_launches reports them."""
        n = int(_lib.load().skv_decode_step_launches(ctypes.addressof(self._desc)))
        _lib.check(min(n, 0), "skv_decode_step_launches")
        return n

    # ----------------------------------------------------------- descriptor --
    def _build_desc(self, k: int) -> tuple[DecodeDescC, torch.Tensor]:
        """Host and device descriptors of the step reading input set k."""
        inputs, scores = self.inputs_by_set[k], self.scores_by_set[k]
        d = DecodeDescC()
        d.batch, d.n_layers, d.n_groups = self.batch, len(self.layers), len(self.groups)
        d.latent, d.c_indexer, d.window = self.latent, self.c_indexer, self.window
        d.tok_lens, d.status = self.tok_lens.data_ptr(), self.status.data_ptr()
        d.step_lens, d.step_top = self.step_lens.data_ptr(), self.step_top.data_ptr()
        for i, g in enumerate(self.groups):
            G = d.groups[i]
            G.free_stack, G.free_top, G.n_pages = g.free_stack.data_ptr(), g.free_top.data_ptr(), g.n_pages
            G.block_table, G.bt_stride = g.block_table.data_ptr(), g.block_table.shape[1]
            G.n_entries, G.m, G.block_size = g.n_entries.data_ptr(), g.m, self.block_size
        p = _lib.ptr
        for i, spec in enumerate(self.layers):
            Ly = d.layers[i]
            Ly.kind = KIND[spec.kind]
            Ly.ring, Ly.out_window = p(self.ring[i]), p(self.out_window[i])
            Ly.kv_new = p(inputs[i]["kv"])
            if spec.kind in ("csa", "hca"):
                Ly.group = self.group_of_rate[spec.m]
                Ly.format = _lib.SKV_FMT_FP8 if spec.fp8 else _lib.SKV_FMT_BF16
                Ly.pool, Ly.entry_bytes = p(self.pool[i]), ops.row_bytes_of(self.pool[i])
                Ly.state, Ly.bias = p(self.state[i]), p(self.bias[i])
                Ly.c_new, Ly.z_new = p(inputs[i]["c"]), p(inputs[i]["z"])
                Ly.out_entries = p(self.out_entries[i])  # None: not copied
                if spec.kind == "csa":
                    Ly.top_k = spec.top_k
                    Ly.scores, Ly.score_stride = p(scores[i]), scores[i].shape[1]
                    Ly.topk_idx = p(self.topk_idx[i])
                    Ly.topk_ws = p(self.topk_ws[i])
                    if spec.indexer:
                        Ly.idx_pool, Ly.idx_state = p(self.idx_pool[i]), p(self.idx_state[i])
                        Ly.idx_bias = p(self.idx_bias[i])
                        Ly.ci_new, Ly.zi_new = p(inputs[i]["ci"]), p(inputs[i]["zi"])
                        if spec.idx_heads > 0:
                            Ly.idx_q, Ly.idx_w = p(inputs[i]["iq"]), p(inputs[i]["iw"])
                            Ly.idx_heads = spec.idx_heads
                elif self.out_entries[i] is not None:
                    Ly.out_rows = self.out_entries[i].shape[1]
        raw = bytes(memoryview(d))
        return d, torch.tensor(list(raw), dtype=torch.uint8, device=self.device)

    # ------------------------------------------------------------------ step --
    def step(self, input_set: int = 0) -> None:
        """One decode step of every sequence from input set ``input_set`` (default
        ``inputs`` and ``scores``; for layers with ``idx_heads``, from ``inputs["iq"]`` /
        ``inputs["iw"]``: the step writes the set's ``scores`` itself)."""
        if (self.host_lens + 1 > self.max_len).any():
            raise RuntimeError(f"DecodeCache overflow: a sequence would exceed max_len={self.max_len}")
        self._launch_step(input_set)
        self.host_lens += 1

    def _launch_step(self, input_set: int) -> None:
        d, d_dev = self._descs[input_set]
        _lib.call("skv_decode_step", ctypes.addressof(d), d_dev.data_ptr(), _lib.stream_handle(self.device))

    def step_attend(self, q: torch.Tensor, knorm_w: torch.Tensor | None = None,
                    sink: torch.Tensor | None = None, softcap: float | None = None,
                    v_ring: torch.Tensor | None = None, eps: float = 1.0e-6,
                    out: torch.Tensor | None = None, input_set: int = 0) -> torch.Tensor:
        """One decode step of this one-layer cache followed by the layer's
        attention for the new token's query q (bf16 [batch, H, latent]), as
        ``step(input_set)`` then ``attention(0, q, ...)`` give them, in one
        call of skv_decode_step_attend: the attention launch ranks the top-k
        picks itself (writing ``topk_idx``) and takes the place of the step's
        gather launch.  Needs ``materialize=False`` (no gathered copies).
        Returns the fp32 [batch, H, latent] output (``out`` when given).  After
        a refused step (``check_status`` raises) the output is undefined."""
        if (self.host_lens + 1 > self.max_len).any():
            raise RuntimeError(f"DecodeCache overflow: a sequence would exceed max_len={self.max_len}")
        out = self._launch_step_attend(input_set, q, knorm_w, sink, softcap, v_ring, eps, out)
        self.host_lens += 1
        return out

    def _launch_step_attend(self, input_set: int, q: torch.Tensor, knorm_w: torch.Tensor | None,
                            sink: torch.Tensor | None, softcap: float | None, v_ring: torch.Tensor | None,
                            eps: float, out: torch.Tensor | None) -> torch.Tensor:
        from saint_kv.attention import step_attention_desc

        if len(self.layers) != 1:
            raise ValueError("step_attend needs a one-layer cache")
        if self.out_window[0] is not None or self.out_entries[0] is not None:
            raise ValueError("step_attend needs a cache built with materialize=False")
        spec = self.layers[0]
        if q.shape[0] != self.batch or q.dim() != 3 or q.shape[2] != self.latent:
            raise ValueError(f"q must be bf16 [{self.batch}, H, {self.latent}]")
        ad, out = step_attention_desc(q, spec.kind, self.window, knorm_w=knorm_w, eps=eps, sink=sink,
                                      softcap=softcap, win_v=v_ring, out=out)
        d, d_dev = self._descs[input_set]
        lib = _lib.load()
        need = int(lib.skv_decode_step_attend_workspace(ctypes.addressof(d), ctypes.byref(ad)))
        if need < 0:
            _lib.check(-1, "skv_decode_step_attend_workspace")
        ws = self._attn_ws.get("step")
        if ws is None or ws.numel() * 4 < need:  # allocated once (not while a graph is captured)
            ws = torch.empty(max(need, 4) // 4 + 1, dtype=torch.float32, device=self.device)
            self._attn_ws["step"] = ws
        _lib.call("skv_decode_step_attend", ctypes.addressof(d), d_dev.data_ptr(), ctypes.byref(ad),
                  ws.data_ptr(), ws.numel() * 4, _lib.stream_handle(self.device))
        return out

    def capture(self, steps: int, before_step=None) -> "CapturedSteps":
        """Capture ``steps`` decode steps in one HIP graph (see CapturedSteps);
        step s reads input set s % input_sets.  ``before_step()`` (optional)
        records the caller's own launches ahead of each step, e.g. its
        indexer-score launch."""
        return CapturedSteps(self, steps, before_step)

    def check_status(self) -> None:
        """Synchronise and raise if a page reservation was refused.

        A refused step changes nothing on the device (every later step of a
        captured sequence is refused the same way), so the host-side lengths
        are re-read from ``tok_lens`` before raising."""
        st = int(self.status.item())
        if st:
            self.host_lens = self.tok_lens.cpu().numpy().astype(np.int64)
            raise RuntimeError(f"DecodeCache page reservation refused (status bits {st})")

    # ------------------------------------------------------------ page plans --
    def reserve_entries(self, rows: slice, n_new: list) -> None:
        """Pop pages for ``n_new[gi]`` more entries (an int or an int32 tensor
        over ``rows``) of every sequence in ``rows``, in every page group.

        Each group's ``skv_reserve`` is all-or-nothing and reports into its own
        status word.  If any group refuses, the groups that did reserve give
        their pages of ``rows`` back (``skv_release``), so every sequence in
        ``rows`` is left empty and the free lists hold what they held before,
        and RuntimeError is raised.  ``rows`` must hold sequences without
        entries."""
        if not self.groups:
            return
        gst = self.group_status
        gst.zero_()
        for gi, g in enumerate(self.groups):
            ops.reserve(g.free_stack, g.free_top, g.block_table[rows], g.n_entries[rows], n_new[gi],
                        self.block_size, gst[gi:gi + 1])
        bad = gst[: len(self.groups)].cpu().tolist()
        if not any(bad):
            return
        n_rows = g.n_entries[rows].numel()
        ones = torch.ones(n_rows, dtype=torch.uint8, device=self.device)
        for gi, g in enumerate(self.groups):
            if bad[gi] == 0:
                ops.release(g.free_stack, g.free_top, g.block_table[rows], g.n_entries[rows], ones,
                            self.block_size, gst[gi:gi + 1])
        undo = gst[: len(self.groups)].cpu().tolist()
        failed = [f"group m={g.m}: status bits {b}" for g, b in zip(self.groups, bad) if b]
        if any(u for u, b in zip(undo, bad) if b == 0):
            raise RuntimeError("DecodeCache page reservation refused (" + "; ".join(failed) +
                               ") and the undo of the other groups failed")
        raise RuntimeError("DecodeCache page reservation refused (" + "; ".join(failed) + ")")

    # --------------------------------------------------------------- prefill --
    def prefill(self, lens: np.ndarray, generator: torch.Generator | None = None,
                data: dict | None = None, outlier_frac: float = 0.0,
                outlier_scale: float = 20.0, tails: list | None = None) -> None:
        """Bring every sequence from empty to ``lens[b]`` tokens.

        With ``data`` (per layer dicts of bf16 [B, T, ...] tensors "kv", "c", "z",
        "ci", "zi") the caches are built through the kernels exactly as decode
        would build them.  Without it the compressed entries and rings are
        filled with N(0,1) values (synthetic contexts for benchmarking; fp8
        pools quantize N(0,1) rows in which a fraction ``outlier_frac`` of the
        values is multiplied by ``outlier_scale``) and the incomplete blocks'
        states are folded from N(0,1) tokens, or, with ``tails`` (per layer a
        dict of bf16 [B, T >= max(lens % m), ch] tensors "c", "z", "ci", "zi";
        None for SWA layers), from the first ``lens[b] % m`` rows of those.
        """
        lens = np.asarray(lens, dtype=np.int64)
        if lens.shape != (self.batch,) or (lens < 0).any() or (lens > self.max_len).any():
            raise ValueError("lens must be [batch] in [0, max_len]")
        if (self.host_lens != 0).any():
            raise RuntimeError("prefill needs empty sequences")
        dev = self.device
        lens_t = torch.as_tensor(lens.astype(np.int32), device=dev)
        self.reserve_entries(slice(None), [torch.as_tensor((lens // g.m).astype(np.int32), device=dev)
                                           for g in self.groups])
        for i, spec in enumerate(self.layers):
            if data is not None:
                src = data[i]["kv"]
                ops.ring_append(self.ring[i], lens_t, src, lens_t)
            else:
                self.ring[i].normal_(generator=generator)
            if spec.kind == "swa":
                continue
            g = self.groups[self.group_of_rate[spec.m]]
            streams = [(self.pool[i], self.state[i], self.bias[i], "c", "z", self.latent)]
            if spec.kind == "csa" and spec.indexer:
                streams.append((self.idx_pool[i], self.idx_state[i], self.idx_bias[i], "ci", "zi",
                                self.c_indexer))
            for pool, state, bias, kc, kz, ch in streams:
                if data is not None:
                    ops.compress_append(pool, g.block_table, state, data[i][kc], data[i][kz], bias,
                                        lens_t, lens_t)
                    continue
                self._fill_entries(pool, g, lens // spec.m, ch, generator, outlier_frac,
                                   outlier_scale)
                tail = lens % spec.m
                if tail.max() > 0:
                    t = int(tail.max())
                    if tails is not None:
                        c, z = tails[i][kc][:, :t], tails[i][kz][:, :t]
                    else:
                        c = torch.randn(self.batch, t, ch, generator=generator, device=dev).to(torch.bfloat16)
                        z = torch.randn(self.batch, t, ch, generator=generator, device=dev).to(torch.bfloat16)
                    ops.compress_append(pool, g.block_table, state, c, z, bias, lens_t,
                                        torch.as_tensor(tail.astype(np.int32), device=dev))
        self.tok_lens.copy_(lens_t)
        self.host_lens = lens.copy()

    def _fill_entries(self, pool: torch.Tensor, g: _Group, n_ent: np.ndarray, ch: int,
                      generator: torch.Generator | None, outlier_frac: float,
                      outlier_scale: float) -> None:
        if pool.dtype == torch.bfloat16:
            for chunk in pool.split(4096):
                chunk.normal_(generator=generator)
            return
        # fp8 pools: quantize N(0,1) rows so every entry is a valid code/scale set
        step = 16384
        done = np.zeros_like(n_ent)
        tmp_lens = torch.zeros(self.batch, dtype=torch.int32, device=self.device)
        while (done < n_ent).any():
            n = np.minimum(n_ent - done, step).astype(np.int32)
            x = torch.randn(self.batch, int(n.max()), ch, generator=generator, device=self.device)
            if outlier_frac > 0:
                hit = torch.rand(x.shape, generator=generator, device=self.device) < outlier_frac
                x = torch.where(hit, x * outlier_scale, x)
            x = x.to(torch.bfloat16)
            tmp_lens.copy_(torch.as_tensor((done + n).astype(np.int32)))
            ops.fp8_quant_append(pool, g.block_table, tmp_lens, x, torch.as_tensor(n, device=self.device))
            done += n

    # -------------------------------------------------------------- attention --
    def attention(self, i: int, q: torch.Tensor, knorm_w: torch.Tensor | None = None,
                  sink: torch.Tensor | None = None, softcap: float | None = None,
                  v_ring: torch.Tensor | None = None, eps: float = 1.0e-6,
                  out: torch.Tensor | None = None) -> torch.Tensor:
        """Layer i's attention for the query of every sequence after the last
        step (saint_kv.attention.decode_attention over this cache's pool, block
        table, picks and ring).  ``v_ring``: the window's values, a [batch,
        window, latent] ring kept by the caller (default: the K ring, K = V).
        The workspace is kept per layer between calls."""
        from saint_kv.attention import decode_attention

        spec = self.layers[i]
        kw = {}
        if spec.kind != "swa":
            if knorm_w is None:
                raise ValueError(f"layer {i} ({spec.kind}) needs knorm_w")
            g = self.groups[self.group_of_rate[spec.m]]
            kw = dict(pool=self.pool[i], fp8=spec.fp8, block_table=g.block_table, n_entries=g.n_entries,
                      m=spec.m, knorm_w=knorm_w)
            if spec.kind == "csa":
                kw["picks"] = self.topk_idx[i]
        ws = self._attn_ws.get(i)
        out = decode_attention(q, spec.kind, self.tok_lens, self.ring[i],
                               self.ring[i] if v_ring is None else v_ring, sink=sink, softcap=softcap,
                               eps=eps, out=out, workspace=ws, **kw)
        if ws is None:  # keep the workspace decode_attention sized for this layer
            from saint_kv.attention import last_workspace

            self._attn_ws[i] = last_workspace()
        return out

    # ------------------------------------------------------------ persistence --
    def save(self, b: int, path, swa: str = "full", period: int | None = None) -> dict:
        """Write sequence b's snapshot (compressed entries, tail states, SWA rows
        by strategy "full" / "periodic" / "zero"); see saint_kv.state."""
        from saint_kv import state

        return state.save_sequence(self, b, path, swa, period)

    def load(self, b: int, path) -> tuple[int, int]:
        """Restore a snapshot into the empty slot b; returns the positions whose
        SWA rows the caller appends before the next step; see saint_kv.state."""
        from saint_kv import state

        return state.load_sequence(self, b, path)

    # -------------------------------------------------- eviction / compaction --
    def release(self, mask: np.ndarray, mask_dev: torch.Tensor | None = None, check: bool = True) -> None:
        """Finish the sequences with mask[b]: their pages return to the free lists.

        ``mask_dev`` (optional): the same mask already on the device as uint8,
        so that the call issues no host-to-device copy.  Each group's release
        reports into its own status word; ``check`` synchronises and raises
        RuntimeError if any group refused (a free stack that would overflow or
        an invalid page id: the pool's bookkeeping is already corrupt).  With
        ``check=False`` nothing waits; ``check_release()`` reads the words
        later."""
        mask = np.asarray(mask, dtype=bool)
        if mask.shape != (self.batch,):
            raise ValueError("mask must be [batch]")
        if (mask & (self.host_lens == 0)).any():
            raise RuntimeError("release of a sequence that holds no tokens (double free)")
        m_dev = torch.as_tensor(mask.astype(np.uint8), device=self.device) if mask_dev is None else mask_dev
        for gi, g in enumerate(self.groups):
            ops.release(g.free_stack, g.free_top, g.block_table, g.n_entries, m_dev,
                        self.block_size, self.group_status[gi:gi + 1])
        self.tok_lens.masked_fill_(m_dev.view(torch.bool), 0)  # 0/1 bytes read as bool, no conversion
        self.host_lens[mask] = 0
        if check:
            self.check_release()

    def check_release(self) -> None:
        """Synchronise and raise if the last release() was refused by any page group."""
        bad = self.group_status[: len(self.groups)].cpu().tolist()
        if any(bad):
            raise RuntimeError("DecodeCache release refused (" + "; ".join(
                f"group m={g.m}: status bits {b}" for g, b in zip(self.groups, bad) if b) + ")")

    def compact_workspace_words(self) -> int:
        """int32 words of the compaction workspace: 3 * n_pages per page group."""
        return sum(3 * g.n_pages for g in self.groups)

    def compact(self, workspace: torch.Tensor | None = None, sync: bool = True):
        """Defragment every page group; returns [(n_live, n_moved)] per group.

        With ``sync=False`` nothing waits for the device: the result is an
        int32 device tensor [n_groups, 2] holding the same pairs (reused by the
        next call).  A caller's ``workspace`` must hold
        ``compact_workspace_words()`` int32, zero before its first use; group g
        uses its own slice (3 * n_pages words), whose first n_pages words (the
        page marks) every compaction leaves zero."""
        info = self._compact_info
        ws_all = workspace if workspace is not None else self._compact_ws
        if ws_all.numel() < self.compact_workspace_words():
            raise ValueError(f"compaction workspace needs {self.compact_workspace_words()} int32")
        ws_off = 0
        for gi, g in enumerate(self.groups):
            pools = []
            for i, spec in enumerate(self.layers):
                if spec.kind in ("csa", "hca") and self.group_of_rate[spec.m] == gi:
                    pools.append(self.pool[i])
                    if self.idx_pool[i] is not None:
                        pools.append(self.idx_pool[i])
            ws = ws_all[ws_off: ws_off + 3 * g.n_pages]
            ws_off += 3 * g.n_pages
            ops.compact(pools, g.block_table, g.n_entries, self.block_size, g.free_stack,
                        g.free_top, ws, info[gi])
        if not sync:
            return info
        return [tuple(int(v) for v in row) for row in info.cpu()]


class CapturedSteps:
    """``steps`` decode steps of a DecodeCache recorded in one HIP graph.

    Every replay runs those steps on the device state as it is at replay time
    (token counts, pages and states live in device memory), with the inputs
    and scores the buffers hold then.  The host-side token counts advance by
    ``steps`` per replay; call ``cache.check_status()`` after replays to
    surface a refused page reservation.
    """

    def __init__(self, cache: DecodeCache, steps: int, before_step=None) -> None:
        if steps <= 0:
            raise ValueError("steps must be positive")
        self.cache, self.steps = cache, steps
        self.graph = torch.cuda.CUDAGraph()
        lens_before = cache.host_lens.copy()
        with torch.cuda.graph(self.graph):
            for s in range(steps):
                if before_step is not None:
                    before_step()
                cache._launch_step(s % cache.n_input_sets)
        cache.host_lens = lens_before  # capture records, it does not run

    def replay(self) -> None:
        if (self.cache.host_lens + self.steps > self.cache.max_len).any():
            raise RuntimeError(
                f"DecodeCache overflow: {self.steps} more steps exceed max_len={self.cache.max_len}")
        self.graph.replay()
        self.cache.host_lens += self.steps
