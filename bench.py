"""Benchmark of the paged KV-cache decode step on one MI355X.

Workload (the headline configuration): paged decode append + full block-table
gather, bf16 MLA-style latent rows of 512 + 64 dims (1152 B per token), one
layer, batch 64, context lengths uniform in [1024, 32768], block size 64,
physical pages a random permutation of a 200k-page pool (14.7 GB), one new
token per sequence per step, values N(0,1).  Each step = reserve (page
allocation) + fused append+gather of every sequence into a packed buffer.

Prints one JSON line (see the keys below).  Progress goes to stderr.

A step is the two launches of skv_decode_append_gather (ops.plan_units +
ops.copy_slices): a one-workgroup planner (page reservation + page-unit table)
and the fused append + gather over 4 KB slices.  The planner of step i+1 runs
on a second stream into a second unit table while step i's copy runs.

Algorithmic bytes per step (read + write of every gathered row, the appended
row read + written, one int32 block-table entry per page):
    2 * sum(L) * 1152 + B * 2 * 1152 + sum(ceil(L / 64)) * 4
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "saint-llm_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak, 8 TB/s
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_k_copy_slices_b64_L1k-32k.json"
DECODE_TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_decode_legs.json"
ATTN_TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_attention_layer_seq.json"
INDEXER_TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_indexer_scores.json"


def committed_traffic(path: Path, key: str | None, alg_bytes: float) -> tuple[int | None, str | None]:
    """(HBM bytes, source label) for this run's algorithmic bytes: the ratio of
    counted FETCH_SIZE + WRITE_SIZE bytes to algorithmic bytes that the
    committed profile holds (rocprofv3 counter passes, calibrated on a plain
    copy), times this run's bytes.  Not a counter reading of this run."""
    try:
        d = json.loads(path.read_text())
        rec = d if key is None else d["legs"][key]
        ratio = rec["traffic_over_alg"]
    except (OSError, KeyError, ValueError, TypeError):
        return None, None
    return int(round(ratio * alg_bytes)), (
        f"committed counter ratio x this run's bytes: {path.relative_to(ROOT)}"
        + ("" if key is None else f" [{key}]") + f", ratio {ratio}")
ROW = 576  # 512 latent + 64 rope, bf16
ROW_BYTES = ROW * 2


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def alg_bytes_append_gather(lens: np.ndarray, bs: int) -> int:
    L = lens.astype(np.int64)
    return int(2 * L.sum() * ROW_BYTES + len(L) * 2 * ROW_BYTES + (-(-L // bs)).sum() * 4)


def copy_bandwidth(dev: torch.device, nbytes: int = 2 << 30, iters: int = 20) -> float:
    """Read+write GB/s of torch's device copy over nbytes (the plain-copy yardstick)."""
    a = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).normal_()
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    del a, b
    return 2 * nbytes / (ms * 1e-3) / 1e9


class PagedDecode:
    """Device state of the paged-append+gather workload."""

    def __init__(self, dev: torch.device, batch: int, lmin: int, lmax: int, bs: int,
                 n_pages: int, steps_total: int, seed: int = 0) -> None:
        from saint_kv import ops

        self.ops = ops
        rng = np.random.default_rng(seed)
        self.bs = bs
        self.batch = batch
        self.lens0 = rng.integers(lmin, lmax + 1, size=batch).astype(np.int32)
        max_pages = int(-(-(int(self.lens0.max()) + steps_total) // bs))
        order = rng.permutation(n_pages).astype(np.int32)
        self.stack = torch.empty(n_pages, dtype=torch.int32, device=dev)
        self.top = torch.empty(1, dtype=torch.int32, device=dev)
        ops.free_stack_init(self.stack, self.top, torch.as_tensor(order, device=dev))
        self.bt = torch.full((batch, max_pages), -1, dtype=torch.int32, device=dev)
        self.lens = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        gen = torch.Generator(device=dev).manual_seed(seed)
        self.pool = torch.empty(n_pages, bs, ROW, dtype=torch.bfloat16, device=dev)
        for chunk in self.pool.split(8192):
            chunk.normal_(generator=gen)
        # prefill: map pages for the initial contexts (content is the N(0,1) pool)
        ops.reserve(self.stack, self.top, self.bt, self.lens,
                    torch.as_tensor(self.lens0, device=dev), bs, self.status)
        cap = self.lens0.astype(np.int64) + steps_total
        self.offsets = torch.as_tensor(np.concatenate([[0], np.cumsum(cap)[:-1]]), device=dev)
        self.out = torch.empty(int(cap.sum()), ROW, dtype=torch.bfloat16, device=dev)
        self.tokens = torch.empty(steps_total, batch, 1, ROW, dtype=torch.bfloat16, device=dev)
        self.tokens.normal_(generator=gen)
        # two page-unit tables: step i+1's planner (on its own stream, default
        # priority) fills one while step i's copy reads the other; the copy reads
        # only its unit table, the pool, the new tokens and the output
        self.units = [ops.unit_table(batch * max_pages, dev) for _ in range(2)]
        self.plan_stream = torch.cuda.Stream(device=dev)
        self.plan_done = [torch.cuda.Event() for _ in range(2)]
        self.copy_done = [torch.cuda.Event() for _ in range(2)]
        self.step_idx = 0
        torch.cuda.synchronize()
        if int(self.status.item()) != 0:
            raise RuntimeError(f"prefill reserve refused: status {int(self.status.item())}")

    def host_lens(self) -> np.ndarray:
        return self.lens0 + self.step_idx

    def start(self) -> None:
        """Order the planner stream after everything issued so far on the current stream."""
        self.plan_stream.wait_stream(torch.cuda.current_stream())

    def step(self, ev: tuple | None = None) -> None:
        """skv_decode_append_gather: planner (reserve + page-unit table) + 4 KB-slice copy.

        The planner runs on its own stream and overlaps the previous step's copy."""
        max_units = int((-(-(self.host_lens() + 1) // self.bs)).sum())
        k = self.step_idx % 2
        main = torch.cuda.current_stream()
        ps = self.plan_stream
        ps.wait_event(self.copy_done[k])  # the copy two steps back has read units[k]
        with torch.cuda.stream(ps):
            self.ops.plan_units(self.stack, self.top, self.bt, self.lens, 1, self.bs, self.out,
                                ROW_BYTES, self.units[k], max_units, self.offsets, self.status)
        self.plan_done[k].record(ps)
        main.wait_event(self.plan_done[k])
        if ev is not None:
            ev[0].record()
        self.ops.copy_slices(self.pool, self.tokens[self.step_idx], self.out, self.units[k], max_units)
        if ev is not None:
            ev[1].record()
        self.copy_done[k].record(main)
        self.step_idx += 1


def cpu_baseline(seconds: float = 10.0, seed: int = 0) -> dict:
    """The oracle's paged append+gather on host cores, on a bounded sample."""
    from oracle import reference_cpu as ref

    rng = np.random.default_rng(seed)
    threads = torch.get_num_threads()
    bs, n_seq = 64, 8
    lens = rng.integers(1024, 32769, size=n_seq).astype(np.int32)
    pages_needed = int((-(-(lens.astype(np.int64) + 64) // bs)).sum())
    n_pages = pages_needed + 16
    stack, top = ref.free_stack_init(n_pages, rng.permutation(n_pages).astype(np.int32))
    bt = np.full((n_seq, int(-(-(int(lens.max()) + 64) // bs))), -1, dtype=np.int32)
    cur = np.zeros(n_seq, dtype=np.int32)
    _, top = ref.reserve(stack, top, bt, cur, lens, bs)
    pool = torch.randn(n_pages, bs, ROW).to(torch.bfloat16)
    out = torch.empty(n_seq, int(lens.max()) + 64, ROW, dtype=torch.bfloat16)
    tok = torch.randn(n_seq, 1, ROW).to(torch.bfloat16)
    start = (stack.copy(), top, bt.copy(), cur.copy())
    done_bytes, t0, steps = 0, time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        # rounds of 64 decode steps from the prefilled state (the buffers hold 64 extra rows)
        stack, top, bt, cur = start[0].copy(), start[1], start[2].copy(), start[3].copy()
        for _ in range(64):
            _, top = ref.reserve(stack, top, bt, cur, 1, bs)
            ref.paged_append(pool, bt, cur, tok, 1)
            ref.paged_gather(pool, bt, cur, out)
            done_bytes += alg_bytes_append_gather(cur, bs)
            steps += 1
            if time.perf_counter() - t0 >= seconds:
                break
    dt = time.perf_counter() - t0
    return {
        "value": round(done_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{steps} decode steps of 8 sequences (L~U[1k,32k], sum L={int(lens.sum())}) "
                  f"of the same append+gather, torch-eager CPU oracle, {dt:.1f} s",
    }


# ---------------------------------------------------------------------------
# Decode-step legs: heterogeneous compressed cache (CSA / HCA / SWA layers)
# ---------------------------------------------------------------------------
def decode_step_bytes(specs, lens_after: np.ndarray, window: int, latent: int = 576,
                      c_indexer: int = 128, bs: int = 64, copies: bool = True) -> int:
    """Compulsory HBM bytes of one fused decode step, for the sequences'
    token counts after the step: reads + writes of every row, entry, state,
    score and index the step touches (the formula is stated in the design notes).
    ``copies=False``: a step that writes no gathered copies (the picks' and
    window's rows are then the attention's reads, not the step's)."""
    L = lens_after.astype(np.int64)
    p = L - 1
    E = latent * 2
    total = 0
    for s in specs:
        cnt = np.minimum(L, window) if copies else np.zeros_like(L)
        total += int((2 * E + 2 * cnt * E).sum())  # token in + ring write; window read + write
        if s.kind == "swa":
            continue
        ent_bytes = (latent - 64) + (latent - 64) // 128 * 4 + 128 if s.fp8 else E
        streams = [(latent, ent_bytes)]
        if s.kind == "csa" and s.indexer:
            streams.append((c_indexer, c_indexer * 2))
        for ch, eb in streams:
            st = 3 * ch * 4
            emit = ((p + 1) % s.m == 0)
            total += int((2 * ch * 2 + ch * 4  # c, z rows + bias row
                          + np.where(p % s.m != 0, st, 0)  # state read
                          + np.where(emit, eb, st)).sum())  # entry or state write
        n_ent = L // s.m
        if s.kind == "csa":
            n_valid = np.maximum(p, 0) // s.m
            k_eff = np.minimum(s.top_k, n_ent)
            total += int((n_valid * 4 + s.top_k * 4).sum())  # scores read, indices written
            if s.idx_heads:  # scores computed in the step: indexer keys, query and weights read, scores written
                total += int((n_valid * (c_indexer * 2 + 4) + s.idx_heads * (c_indexer * 2 + 4)).sum())
            if copies:
                total += int((k_eff * (ent_bytes + E + 8) + (s.top_k - k_eff) * E).sum())
        elif copies:
            total += int((n_ent * (ent_bytes + E) + (-(-n_ent // bs)) * 4).sum())
    return total


def decode_kv_tokens(specs, lens_after: np.ndarray, window: int) -> int:
    """KV rows delivered to attention per step: top-k picks + window (CSA),
    all entries + window (HCA), window (SWA)."""
    L = lens_after.astype(np.int64)
    tot = 0
    for s in specs:
        tot += int(np.minimum(L, window).sum())
        if s.kind == "csa":
            tot += int(np.minimum(s.top_k, L // s.m).sum())
        elif s.kind == "hca":
            tot += int((L // s.m).sum())
    return tot


def run_decode_leg(dev, name: str, specs, batch: int, lens0: np.ndarray, steps: int,
                   per_graph: int = 20, window: int = 128, seed: int = 0,
                   outlier_frac: float = 0.0, evict_frac: float | None = None,
                   separate_scores: int = 0, input_sets: int = 20) -> dict:
    """Decode steps of a DecodeCache replayed from HIP graphs of ``per_graph``
    steps.  The steps cycle through ``input_sets`` sets of new-token rows and
    N(0,1) scores (one per step of a graph by default), so every step gathers
    other picks than the step before: a pick is reused only ``input_sets``
    steps later, after hundreds of MB of other traffic."""
    from saint_kv.decode import DecodeCache

    max_len = int(lens0.max()) + steps + 2 * per_graph + 8
    t0 = time.perf_counter()
    n_sets = 1 if separate_scores else input_sets
    cache = DecodeCache(specs, batch, max_len, window=window, device=dev, page_order_seed=seed,
                        hca_out_rows=max(1, max_len // 128), input_sets=n_sets)
    gen = torch.Generator(device=dev).manual_seed(seed)
    for i, s in enumerate(specs):
        if cache.bias[i] is not None:
            cache.bias[i].normal_(generator=gen)
        if cache.idx_bias[i] is not None:
            cache.idx_bias[i].normal_(generator=gen)
        for k in range(n_sets):
            for v in cache.inputs_by_set[k][i].values():
                v.normal_(generator=gen)
            if cache.scores_by_set[k][i] is not None:
                cache.scores_by_set[k][i].normal_(generator=gen)
    cache.prefill(lens0, generator=gen, outlier_frac=outlier_frac)
    torch.cuda.synchronize()
    log(f"{name}: prefilled {batch} x mean {int(lens0.mean())} tokens in {time.perf_counter() - t0:.1f} s")
    before = None
    if separate_scores:
        # the caller's own indexer-score launch before each step (skv_indexer_scores
        # over the entries before the step), in place of the step computing them
        from saint_kv import ops

        iq = torch.empty(batch, 1, separate_scores, cache.c_indexer, dtype=torch.bfloat16, device=dev)
        iw = torch.empty(batch, 1, separate_scores, dtype=torch.float32, device=dev)
        iq.normal_(generator=gen)
        iw.normal_(generator=gen)
        score_layers = [i for i, s in enumerate(specs) if s.kind == "csa"]

        def before():
            for i in score_layers:
                g = cache.groups[cache.group_of_rate[specs[i].m]]
                ops.indexer_scores(iq, iw, cache.idx_pool[i], g.block_table, g.n_entries,
                                   cache.scores[i].unsqueeze(1))
    graph = cache.capture(per_graph, before)
    graph.replay()  # warm-up replay
    torch.cuda.synchronize()
    cache.check_status()
    reps = max(1, steps // per_graph)
    lens_start = cache.host_lens.copy()
    stream = torch.cuda.current_stream(dev)  # the graphs replay on it
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    cache.check_status()
    n_steps = reps * per_graph
    ms = e0.elapsed_time(e1) / n_steps
    if separate_scores:  # the same bytes as the step that computes its own scores
        import dataclasses

        specs = [dataclasses.replace(s, idx_heads=separate_scores) if s.kind == "csa" else s for s in specs]
    alg = sum(decode_step_bytes(specs, lens_start + i + 1, window) for i in range(n_steps)) / n_steps
    toks = sum(decode_kv_tokens(specs, lens_start + i + 1, window) for i in range(n_steps)) / n_steps
    gbs = alg / (ms * 1e-3) / 1e9
    rec = {
        "batch": batch, "layers": [f"{s.kind}{'-fp8' if s.fp8 else ''}(m={s.m},k={s.top_k})" if s.kind != "swa" else "swa" for s in specs],
        "mean_ctx": int(lens0.mean()), "steps": n_steps, "us_per_step": round(ms * 1e3, 2),
        "alg_bytes_per_step": int(alg), "gbs": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "kv_tokens_per_step": int(toks), "kv_tokens_per_s": round(toks / (ms * 1e-3), 1),
        "launches_per_step": cache.step_launches() + (sum(s.kind == "csa" for s in specs) if separate_scores else 0),
        "hip_graph_steps": per_graph,
        "input_sets": n_sets,
        "scores": ("computed in the step" if any(s.idx_heads for s in specs) and not separate_scores
                   else "skv_indexer_scores launch before each step" if separate_scores else "input"),
    }
    traffic, source = committed_traffic(DECODE_TRAFFIC_FILE, name, alg)
    rec["roofline"] = {
        "bound": "hbm",
        "kernel": f"skv_decode_step ({cache.step_launches()} launch(es) per step; the step as the unit)",
        "achieved": rec["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(rec["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": source,
        "alg_bytes_per_launch": int(alg), "avg_launch_us": rec["us_per_step"],
    }
    log(f"{name}: {rec['us_per_step']} us/step, {rec['gbs']} GB/s ({rec['pct_hbm_peak']}%), "
        f"{rec['kv_tokens_per_s'] / 1e6:.1f} M KV tok/s")
    if evict_frac is not None:
        rng = np.random.default_rng(seed + 1)
        n_fin = int(round(evict_frac * batch))
        mask = np.zeros(batch, dtype=bool)
        mask[rng.choice(batch, size=n_fin, replace=False)] = True
        # the release/compaction kernels' first launches in the process load
        # their code; a small throwaway cache takes that cost outside the timing
        warm = DecodeCache(specs, 2, 4096, window=window, device=dev, page_order_seed=seed)
        warm.prefill(np.array([3000, 2000]), generator=gen)
        warm.release(np.array([True, False]))
        warm.compact()
        del warm
        ws = torch.zeros(cache.compact_workspace_words(), dtype=torch.int32, device=dev)
        m_dev = torch.as_tensor(mask.astype(np.uint8), device=dev)
        torch.cuda.synchronize()
        # the release and compaction launches recorded in one HIP graph and
        # replayed once: the interval holds their kernels, not their host calls
        g_ev = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_ev):
            cache.release(mask, m_dev, check=False)
            info_dev = cache.compact(ws, sync=False)
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        g_ev.replay()
        c1.record(stream)
        torch.cuda.synchronize()
        cache.check_release()
        info = [tuple(int(v) for v in row) for row in info_dev.cpu()]
        page_bytes = 0
        for i, s in enumerate(specs):
            if cache.pool[i] is not None:
                page_bytes += ops_row_bytes(cache.pool[i]) * cache.block_size
            if cache.idx_pool[i] is not None:
                page_bytes += ops_row_bytes(cache.idx_pool[i]) * cache.block_size
        moved = sum(m for _, m in info)
        cms = c0.elapsed_time(c1)
        rec["evict_compact"] = {
            "finished": n_fin, "pages_live": [n for n, _ in info], "pages_moved": moved,
            "bytes_moved_rw": 2 * moved * page_bytes, "ms": round(cms, 3),
            "gbs": round(2 * moved * page_bytes / (cms * 1e-3) / 1e9, 1) if cms > 0 else None,
        }
        cache.step()  # decoding continues on the compacted pools
        torch.cuda.synchronize()
        cache.check_status()
        log(f"{name}: release {n_fin} + compaction moved {moved} pages in {cms:.3f} ms")
    del cache, graph
    torch.cuda.empty_cache()
    return rec


def ops_row_bytes(pool: torch.Tensor) -> int:
    from saint_kv import ops

    return ops.row_bytes_of(pool)


def cpu_baseline_decode(seconds: float = 5.0, seed: int = 0) -> dict:
    """The oracle's CSA decode read path (top-k select + block-table gather +
    window read) on host cores for 2 sequences at 64k context."""
    from oracle import reference_cpu as ref

    rng = np.random.default_rng(seed)
    n_seq, m, k, L, bs, w = 2, 4, 512, 65536, 64, 128
    n_ent = L // m
    pages = n_seq * (n_ent // bs)
    pool = torch.randn(pages, bs, ROW).to(torch.bfloat16)
    bt = rng.permutation(pages).astype(np.int32).reshape(n_seq, n_ent // bs)
    ring = torch.randn(n_seq, w, ROW).to(torch.bfloat16)
    scores = rng.standard_normal((n_seq, n_ent)).astype(np.float32)
    out = torch.empty(n_seq, k, ROW, dtype=torch.bfloat16)
    win = torch.empty(n_seq, w, ROW, dtype=torch.bfloat16)
    lens = np.full(n_seq, L, dtype=np.int64)
    t0, steps = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        idx = ref.topk_select(scores, np.full(n_seq, (L - 1) // m), k, n_ent)
        ref.topk_gather(pool, bt, np.arange(n_seq), idx, out)
        ref.ring_read(ring, lens, win)
        steps += 1
    dt = time.perf_counter() - t0
    per_step = n_seq * (n_ent * 4 + k * 4 + k * (2 * ROW * 2 + 8) + w * 2 * ROW * 2)
    return {"value": round(steps * per_step / dt / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{steps} CSA read steps (top-512 of 16384 scores + gather + 128-row window) "
                      f"for 2 sequences at 64k context, torch/numpy CPU oracle, {dt:.1f} s"}


def run_layer_seq_leg(dev, n_layers: int = 8, batch: int = 16, L: int = 65536, steps: int = 100,
                      per_graph: int = 10, heads: int = 64, window: int = 128, seed: int = 8,
                      mode: str = "fused", kinds: list | None = None, lens: np.ndarray | None = None,
                      name: str = "layer_seq_64k") -> dict:
    """What a model's decode step sees at 64k context: n_layers CSA layers
    (m=4, top-k 512, W=128), one after another, each layer's cache step
    followed by its decode attention over the step's picks and window (the
    next layer's inputs come from that attention, so the layers cannot be
    stepped together).  Each layer has its own cache and input sets; the
    sequence of layers is replayed from HIP graphs of ``per_graph`` model
    steps.  ``mode``: "fused", one skv_decode_step_attend per layer (the
    attention launch ranks the picks itself, in place of the step's gather
    launch); "separate", skv_decode_step then skv_decode_attention;
    "materialize", the same with the step's gathered copies written.  The
    attention reads the picks' entries and the window rows in place.
    ``kinds`` (default all "csa") alternates CSA (m=4, top-k 512) and HCA
    (m=128) layers; ``lens`` gives ragged lengths (default L each)."""
    from saint_kv.decode import DecodeCache, LayerSpec

    kinds = kinds or ["csa"] * n_layers
    n_layers = len(kinds)
    lens = np.full(batch, L, dtype=np.int64) if lens is None else np.asarray(lens, dtype=np.int64)
    specs = [LayerSpec("csa", m=4, top_k=512) if kd == "csa" else LayerSpec("hca", m=128) for kd in kinds]
    max_len = int(lens.max()) + steps + 2 * per_graph + 8
    gen = torch.Generator(device=dev).manual_seed(seed)
    caches, qs, knorm, outs = [], [], [], []
    for li, spec in enumerate(specs):
        c = DecodeCache([spec], batch, max_len, window=window, device=dev, page_order_seed=seed + li,
                        input_sets=per_graph, materialize=mode == "materialize")
        c.bias[0].normal_(generator=gen)
        if c.idx_bias[0] is not None:
            c.idx_bias[0].normal_(generator=gen)
        for k in range(per_graph):
            for v in c.inputs_by_set[k][0].values():
                v.normal_(generator=gen)
            if c.scores_by_set[k][0] is not None:
                c.scores_by_set[k][0].normal_(generator=gen)
        c.prefill(lens, generator=gen)
        caches.append(c)
        qs.append(torch.empty(batch, heads, 576, dtype=torch.bfloat16, device=dev).normal_(generator=gen))
        knorm.append(torch.empty(576, dtype=torch.float32, device=dev).uniform_(0.5, 1.5, generator=gen))
        outs.append(torch.empty(batch, heads, 576, dtype=torch.float32, device=dev))
    def layer(li, c, s):
        if mode == "fused":
            c._launch_step_attend(s % c.n_input_sets, qs[li], knorm[li], None, None, None, 1.0e-6, outs[li])
        else:
            c._launch_step(s % c.n_input_sets)
            c.attention(0, qs[li], knorm[li], out=outs[li])

    for li, c in enumerate(caches):  # warm-up: kernel loads and each layer's attention workspace
        layer(li, c, 0)
        c.host_lens += 1
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for s in range(per_graph):
            for li, c in enumerate(caches):
                layer(li, c, s)
    graph.replay()  # warm-up replay
    for c in caches:
        c.host_lens += per_graph
    torch.cuda.synchronize()
    reps = max(1, steps // per_graph)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    for c in caches:
        c.host_lens += reps * per_graph
        c.check_status()
    us = e0.elapsed_time(e1) * 1e3 / (reps * per_graph)
    # bytes of the layers: their steps (gathered copies only when
    # materialized) and their attention's reads of the picked or visible
    # entries, the K/V window, the query, the pick rows and block-table
    # slots, and its output
    lens_after = lens + 1
    cnt = np.minimum(lens_after, window)
    model_bytes = 0
    for spec in specs:
        if spec.kind == "csa":
            keys = np.minimum(lens_after // spec.m, spec.top_k)
            meta = batch * spec.top_k * 4 + int(keys.sum()) * 4
        else:
            keys = (lens_after - 1) // spec.m
            meta = int((-(-keys // 64)).sum()) * 4
        model_bytes += (int(keys.sum()) * 576 * 2 + int(cnt.sum()) * 576 * 4 + batch * heads * 576 * 6
                        + meta + batch * 8)
        model_bytes += decode_step_bytes([spec], lens_after, window, copies=mode == "materialize")
    layer_bytes = model_bytes / n_layers
    gbs = model_bytes / (us * 1e-6) / 1e9
    what = (f"{n_layers} CSA layers (m=4, top-k 512, W=128)" if all(kd == "csa" for kd in kinds) else
            f"{n_layers} layers alternating CSA (m=4, top-k 512) and HCA (m=128), each with W=128")
    rec = {
        "workload": f"{what} in sequence, B={batch}, L in [{int(lens.min())}, {int(lens.max())}]: per layer "
                    f"one decode step, then its decode attention ({heads} heads x 576) over its picks or entries",
        "model_steps": reps * per_graph, "us_per_model_step": round(us, 2),
        "us_per_layer": round(us / n_layers, 2),
        "mode": mode,
        "launches_per_layer": caches[0].step_launches() + (1 if mode == "fused" else 2),
        "gathered_copies": mode == "materialize",
        "kv_tokens_per_s": round(sum(decode_kv_tokens([sp], lens_after, window) for sp in specs) / (us * 1e-6), 1),
        "alg_bytes_per_layer": int(layer_bytes), "gbs": round(gbs, 1),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
    }
    traffic, source = committed_traffic(ATTN_TRAFFIC_FILE, f"{name}_{mode}", layer_bytes)
    rec["roofline"] = {
        "bound": "hbm",
        "kernel": f"one layer: decode step + attention ({rec['launches_per_layer']} launches; the layer as the unit)",
        "achieved": rec["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(rec["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": source,
        "alg_bytes_per_launch": int(layer_bytes), "avg_launch_us": rec["us_per_layer"],
    }
    log(f"{name} ({mode}): {rec['us_per_model_step']} us per {n_layers}-layer model step, "
        f"{rec['us_per_layer']} us per layer (step + attention), {rec['gbs']} GB/s ({rec['pct_hbm_peak']}%)")
    del caches
    torch.cuda.empty_cache()
    return rec


def run_indexer_leg(dev, batch: int, n_ent: int, heads: int, channels: int, launches: int,
                    bs: int = 64, n_pools: int = 16, seed: int = 6) -> dict:
    """Lightning-indexer scores of one decode query per sequence over the paged
    compressed indexer keys (skv_indexer_scores).  The launches rotate over
    n_pools distinct pools and queries (> 1 GB in all), so every launch reads
    its keys from HBM, not from the 256 MB Infinity Cache."""
    from saint_kv import ops

    g = torch.Generator(device=dev).manual_seed(seed)
    pages_per_seq = -(-n_ent // bs)
    n_pages = batch * pages_per_seq
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    table = perm.view(batch, pages_per_seq).to(dev)
    n_entries = torch.full((batch,), n_ent, dtype=torch.int32, device=dev)
    pools = [torch.empty(n_pages, bs, channels, dtype=torch.bfloat16, device=dev).normal_(generator=g)
             for _ in range(n_pools)]
    qs = [torch.empty(batch, 1, heads, channels, dtype=torch.bfloat16, device=dev).normal_(generator=g)
          for _ in range(n_pools)]
    ws = [torch.empty(batch, 1, heads, dtype=torch.float32, device=dev).normal_(generator=g)
          for _ in range(n_pools)]
    out = torch.empty(batch, 1, n_ent, dtype=torch.float32, device=dev)
    for i in range(2 * n_pools):  # warm-up (kernel load, first touch)
        ops.indexer_scores(qs[i % n_pools], ws[i % n_pools], pools[i % n_pools], table, n_entries, out)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(launches):
        ops.indexer_scores(qs[i % n_pools], ws[i % n_pools], pools[i % n_pools], table, n_entries, out)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / launches
    alg = batch * n_ent * channels * 2 + batch * heads * (channels * 2 + 4) + batch * n_ent * 4 + \
        batch * pages_per_seq * 4
    flops = 2.0 * batch * heads * channels * n_ent
    gbs = alg / (us * 1e-6) / 1e9
    rec = {
        "workload": f"B={batch}, {n_ent} compressed entries/seq (64k ctx, m=4), {heads} heads x {channels} bf16, "
                    f"bs={bs}, paged, {n_pools} rotating pools",
        "launches": launches, "us_per_launch": round(us, 2), "alg_bytes_per_launch": int(alg),
        "gbs": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "mfma_tflops": round(flops / (us * 1e-6) / 1e12, 1),
    }
    traffic, source = committed_traffic(INDEXER_TRAFFIC_FILE, "indexer_64k", alg)
    rec["roofline"] = {
        "bound": "hbm",
        "kernel": "k_indexer_scores (skv_indexer_scores)",
        "achieved": rec["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(rec["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": source,
        "alg_bytes_per_launch": int(alg), "avg_launch_us": rec["us_per_launch"],
    }
    log(f"indexer_64k: {rec['us_per_launch']} us/launch, {rec['gbs']} GB/s ({rec['pct_hbm_peak']}%), "
        f"{rec['mfma_tflops']} TFLOP/s bf16")
    del pools, qs, ws
    torch.cuda.empty_cache()
    return rec


def run_attention_leg(dev, name: str, kind: str, batch: int, lens: np.ndarray, launches: int,
                      heads: int = 64, dim: int = 576, m: int = 4, top_k: int = 512, window: int = 128,
                      bs: int = 64, n_sets: int = 8, seed: int = 7) -> dict:
    """Decode attention of one layer (skv_decode_attention: per-split partial
    softmax, then the merge) over the paged compressed entries and the K/V
    window rings.  The launches rotate over n_sets distinct pools, rings,
    queries and pick rows, so the keys come from HBM, not from the 256 MB
    Infinity Cache."""
    from saint_kv import decode_attention

    g = torch.Generator(device=dev).manual_seed(seed)
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    n_ent = lens // m
    pages = -(-n_ent // bs)
    bt_stride = int(pages.max())
    n_pages = int(pages.sum())
    perm = rng.permutation(n_pages)
    table = np.full((batch, bt_stride), -1, dtype=np.int32)
    k = 0
    for b in range(batch):
        table[b, :pages[b]] = perm[k:k + pages[b]]
        k += int(pages[b])
    table_d = torch.as_tensor(table, device=dev)
    n_ent_d = torch.as_tensor(n_ent.astype(np.int32), device=dev)
    lens_d = torch.as_tensor(lens.astype(np.int32), device=dev)
    knorm_w = (torch.rand(dim, generator=g, device=dev) + 0.5)
    sink = torch.randn(heads, generator=g, device=dev)
    sets = []
    for _ in range(n_sets):
        pool = torch.empty(n_pages, bs, dim, dtype=torch.bfloat16, device=dev).normal_(generator=g)
        q = torch.empty(batch, heads, dim, dtype=torch.bfloat16, device=dev).normal_(generator=g)
        wk = torch.empty(batch, window, dim, dtype=torch.bfloat16, device=dev).normal_(generator=g)
        wv = torch.empty(batch, window, dim, dtype=torch.bfloat16, device=dev).normal_(generator=g)
        picks = None
        if kind == "csa":
            pk = np.full((batch, top_k), -1, dtype=np.int32)
            for b in range(batch):
                kk = min(top_k, int(n_ent[b]))
                pk[b, :kk] = rng.choice(int(n_ent[b]), size=kk, replace=False)
            picks = torch.as_tensor(pk, device=dev)
        sets.append((pool, q, wk, wv, picks))
    out = torch.empty(batch, heads, dim, dtype=torch.float32, device=dev)

    def launch(i):
        pool, q, wk, wv, picks = sets[i % n_sets]
        return decode_attention(q, kind, lens_d, wk, wv, pool=pool, block_table=table_d, n_entries=n_ent_d,
                                m=m, picks=picks, knorm_w=knorm_w, sink=sink, out=out, workspace=ws)

    ws = torch.empty(64 << 20, dtype=torch.float32, device=dev)  # 256 MB: more than any split needs here
    for i in range(2 * n_sets):
        launch(i)
    torch.cuda.synchronize()
    # one HIP graph of 2 x n_sets layer calls, replayed: the host's per-call
    # argument checks stay out of the timed region
    per_graph = 2 * n_sets
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(per_graph):
            launch(i)
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, launches // per_graph)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    launches = reps * per_graph
    us = e0.elapsed_time(e1) * 1e3 / launches
    if kind == "csa":
        keys = np.minimum(n_ent, top_k)
        meta = batch * top_k * 4 + int(keys.sum()) * 4  # pick rows, block-table slots
    else:
        keys = np.maximum(lens - 1, 0) // m
        meta = int(pages.sum()) * 4
    cnt = np.minimum(lens, window)
    alg = int(keys.sum()) * dim * 2 + int(cnt.sum()) * dim * 4 + batch * heads * dim * (2 + 4) + meta + batch * 8
    flops = 4.0 * heads * dim * float(keys.sum() + cnt.sum())
    gbs = alg / (us * 1e-6) / 1e9
    rec = {
        "workload": f"{kind.upper()} layer: B={batch}, {heads} heads x {dim} bf16, "
                    + (f"top-k {top_k} of L/{m} entries" if kind == "csa" else f"all L/{m} entries")
                    + f", W={window} K/V window, bs={bs}, L in [{int(lens.min())}, {int(lens.max())}], "
                    f"{n_sets} rotating sets",
        "launches": launches, "us_per_launch": round(us, 2), "alg_bytes_per_launch": alg,
        "gbs": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "mfma_tflops": round(flops / (us * 1e-6) / 1e12, 1),
    }
    traffic, source = committed_traffic(ATTN_TRAFFIC_FILE, name, alg)
    rec["roofline"] = {
        "bound": "hbm",
        "kernel": "skv_decode_attention (k_attn_part, then the merge; the layer call as the unit)",
        "achieved": rec["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(rec["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": source,
        "alg_bytes_per_launch": alg, "avg_launch_us": rec["us_per_launch"],
    }
    log(f"{name}: {rec['us_per_launch']} us/launch, {rec['gbs']} GB/s ({rec['pct_hbm_peak']}%), "
        f"{rec['mfma_tflops']} TFLOP/s bf16")
    del sets, ws, graph
    torch.cuda.empty_cache()
    return rec


def run_state_leg(dev, seed: int = 9) -> dict:
    """Save and restore of one 64k-token request of a CSA layer (m=4, with the
    indexer stream, W=128): its 16,384 compressed entries (main and indexer),
    tail states and SWA rows, through a file (saint_kv.state).  Host-side IO:
    device-to-host and host-to-device copies plus the file system."""
    import tempfile

    from saint_kv.decode import DecodeCache, LayerSpec

    L = 65536
    cache = DecodeCache([LayerSpec("csa", m=4, top_k=512)], 2, L + 64, device=dev, page_order_seed=seed)
    cache.prefill(np.array([L, 0]), generator=torch.Generator(device=dev).manual_seed(seed))
    torch.cuda.synchronize()
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "req.skv")
        cache.save(0, path)  # warm-up (allocations, file creation)
        t0 = time.perf_counter()
        cache.save(0, path)
        t1 = time.perf_counter()
        nbytes = os.path.getsize(path)
        cache.load(1, path)
        torch.cuda.synchronize()
        cache.release(np.array([False, True]))
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        cache.load(1, path)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
    rec = {"workload": "one 64k-token CSA request (m=4, indexer stream, W=128): save to and load from a file",
           "bytes": nbytes, "save_ms": round((t1 - t0) * 1e3, 2), "load_ms": round((t3 - t2) * 1e3, 2),
           "save_gbs": round(nbytes / (t1 - t0) / 1e9, 2), "load_gbs": round(nbytes / (t3 - t2) / 1e9, 2)}
    log(f"state_64k: {nbytes / 1e6:.1f} MB, save {rec['save_ms']} ms ({rec['save_gbs']} GB/s), "
        f"load {rec['load_ms']} ms ({rec['load_gbs']} GB/s)")
    del cache
    torch.cuda.empty_cache()
    return rec


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--legs", default="csa_64k,csa_64k_b256,csa_64k_idx,mixed_8layer,fp8_1m,layer_seq_64k,"
                    "layer_seq_mixed",
                    help="comma list of decode-step legs to run after the headline ('' for none)")
    ap.add_argument("--leg-steps", type=int, default=200)
    ap.add_argument("--layer-steps", type=int, default=100, help="timed model steps of the layer-sequential legs")
    ap.add_argument("--layer-modes", default="fused,separate,materialize",
                    help="comma list of the layer-sequential legs' modes to run")
    ap.add_argument("--no-indexer", action="store_true", help="skip the indexer-score leg")
    ap.add_argument("--no-attention", action="store_true", help="skip the decode-attention legs")
    ap.add_argument("--no-state", action="store_true", help="skip the request save/load leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the cache shards by "
              "sequence with no per-step exchange, so N GPUs run N independent copies.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    from saint_kv import _lib

    _lib.load()
    log(f"device {torch.cuda.get_device_name(dev)}")
    copy_gbs = copy_bandwidth(dev)
    log(f"torch copy_ yardstick {copy_gbs:.0f} GB/s")

    batch, bs, n_pages = 64, 64, 200_000
    total_steps = args.warmup + 2 * args.steps  # a timed pass, then a pass with per-launch events
    w = PagedDecode(dev, batch, 1024, 32768, bs, n_pages, total_steps)
    log(f"prefilled {batch} sequences, sum L = {int(w.lens0.sum())}")
    for _ in range(args.warmup):
        w.step()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # timed pass: the steps back to back, events only around the whole pass
    alg_total = 0
    lens_steps = []
    for i in range(args.steps):
        lens_steps.append(w.host_lens() + i + 1)
    torch.cuda.synchronize()
    t_start.record(stream)
    w.start()  # the first planner after t_start
    for i in range(args.steps):
        w.step()
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    for L in lens_steps:
        alg_total += alg_bytes_append_gather(L, bs)
    ms_per_step = total_ms / args.steps
    value = alg_total / (total_ms * 1e-3) / 1e9
    # kernel pass: HIP events around every copy launch, on its stream
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    alg_kern = 0
    for i in range(args.steps):
        alg_kern += alg_bytes_append_gather(w.host_lens() + i + 1, bs)
    torch.cuda.synchronize()
    w.start()
    for i in range(args.steps):
        w.step(evs[i])
    torch.cuda.synchronize()
    kern_ms = np.array([a.elapsed_time(b) for a, b in evs])
    alg_per_launch = alg_kern / args.steps
    kern_avg_ms = float(kern_ms.mean())
    achieved = alg_per_launch / (kern_avg_ms * 1e-3) / 1e9
    tokens_per_step = float(np.mean([L.sum() for L in lens_steps]))
    log(f"step {ms_per_step * 1e3:.1f} us, kernel {kern_avg_ms * 1e3:.1f} us, "
        f"{value:.0f} GB/s, kernel {achieved:.0f} GB/s")

    head_traffic, head_traffic_source = committed_traffic(TRAFFIC_FILE, None, alg_per_launch)
    del w
    torch.cuda.empty_cache()
    legs = {}
    from saint_kv.decode import LayerSpec

    rng = np.random.default_rng(1)
    wanted = [x for x in args.legs.split(",") if x]
    if "csa_64k" in wanted:
        legs["csa_64k"] = run_decode_leg(
            dev, "csa_64k", [LayerSpec("csa", m=4, top_k=512)], 16,
            np.full(16, 65536, dtype=np.int64), args.leg_steps, seed=3)
    if "csa_64k_b256" in wanted:
        legs["csa_64k_b256"] = run_decode_leg(
            dev, "csa_64k_b256", [LayerSpec("csa", m=4, top_k=512)], 256,
            np.full(256, 65536, dtype=np.int64), args.leg_steps, seed=6)
    if "csa_64k_idx" in wanted:
        legs["csa_64k_idx"] = run_decode_leg(
            dev, "csa_64k_idx", [LayerSpec("csa", m=4, top_k=512, idx_heads=64)], 16,
            np.full(16, 65536, dtype=np.int64), args.leg_steps, seed=3)
    if "csa_64k_idx_sep" in wanted:
        legs["csa_64k_idx_sep"] = run_decode_leg(
            dev, "csa_64k_idx_sep", [LayerSpec("csa", m=4, top_k=512)], 16,
            np.full(16, 65536, dtype=np.int64), args.leg_steps, seed=3, separate_scores=64)
    if "mixed_8layer" in wanted:
        specs = [LayerSpec("csa", m=4, top_k=512) if i % 2 == 0 else LayerSpec("hca", m=128)
                 for i in range(8)]
        legs["mixed_8layer"] = run_decode_leg(
            dev, "mixed_8layer", specs, 32, rng.integers(32768, 131073, size=32), args.leg_steps, seed=4)
    if "fp8_1m" in wanted:
        legs["fp8_1m"] = run_decode_leg(
            dev, "fp8_1m", [LayerSpec("csa", m=4, top_k=1024, fp8=True)], 4,
            rng.integers(262144, 1048577, size=4), args.leg_steps, seed=5, outlier_frac=0.01,
            evict_frac=0.3)

    layer_modes = [x for x in args.layer_modes.split(",") if x]

    def layer_seq_modes(modes, **kw):
        """The fused mode's record with the other modes' records under their keys."""
        rec = {}
        for mode, key in (("fused", None), ("separate", "separate"), ("materialize", "with_gathered_copies")):
            if mode in modes and mode in layer_modes:
                r = run_layer_seq_leg(dev, mode=mode, steps=args.layer_steps, **kw)
                if key is None:
                    rec.update(r)
                else:
                    rec[key] = r
        return rec or None

    layer_seq = None
    if "layer_seq_64k" in wanted:
        layer_seq = layer_seq_modes(("fused", "separate", "materialize"))
    layer_seq_mixed = None
    if "layer_seq_mixed" in wanted:
        # the 8-layer CSA/HCA stack of mixed_8layer (B=32, L~U[32k,128k]) as a model steps it
        mixed_lens = np.random.default_rng(4).integers(32768, 131073, size=32)
        layer_seq_mixed = layer_seq_modes(("fused", "separate"), batch=32, kinds=["csa", "hca"] * 4,
                                          lens=mixed_lens, name="layer_seq_mixed")
    indexer = None if args.no_indexer else run_indexer_leg(dev, 16, 16384, 64, 128, 200)
    state_io = None if args.no_state else run_state_leg(dev)
    attention = {}
    if not args.no_attention:
        attention["attn_csa_64k"] = run_attention_leg(dev, "attn_csa_64k", "csa", 16, np.full(16, 65536), 200)
        attention["attn_hca_mixed"] = run_attention_leg(
            dev, "attn_hca_mixed", "hca", 32, np.random.default_rng(4).integers(32768, 131073, size=32), 200,
            m=128)

    cpu = None
    cpu_dec = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle baseline")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads")
        if "csa_64k" in legs:
            cpu_dec = cpu_baseline_decode(min(args.cpu_seconds, 5.0))
            legs["csa_64k"]["cpu_baseline"] = cpu_dec
            log(f"cpu baseline (64k CSA read path) {cpu_dec['value']} GB/s")

    rec = {
        "metric": "KV append+gather GB/s (% of HBM peak) and decode-step KV tokens/s at 64k ctx",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) KV rows, seeded; random-permutation page pool",
        "config": {
            "workload": "paged decode append + full block-table gather (B=64, L~U[1k,32k], "
                        "latent 512+64 bf16, bs=64, 200k-page pool, 1 token/seq/step; each step's "
                        "planner overlaps the previous step's copy on a second stream)",
            "batch": batch,
            "block_size": bs,
            "row_bytes": ROW_BYTES,
            "pool_pages": n_pages,
            "parallelism": "single GPU",
        },
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "kv_tokens_per_s": round(tokens_per_step / (ms_per_step * 1e-3), 1),
        "copy_yardstick_gbs": round(copy_gbs, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": "k_copy_slices (fused append + gather of skv_decode_append_gather)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": head_traffic,
            "traffic_source": head_traffic_source,
            "alg_bytes_per_launch": int(alg_per_launch),
            "avg_launch_us": round(kern_avg_ms * 1e3, 2),
        },
        "cpu_baseline": cpu,
        "decode_kv_tokens_per_s_64k": legs.get("csa_64k", {}).get("kv_tokens_per_s"),
        "decode_legs": legs,
        "layer_seq_64k": layer_seq,
        "layer_seq_mixed": layer_seq_mixed,
        "indexer_64k": indexer,
        "attention": attention or None,
        "state_64k": state_io,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
