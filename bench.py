#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X.

Workload (one "step"): the SwiftKV decode-attention stage of a full decode step
of Llama-2-7B geometry -- 32 layers x 32 heads x head_dim 128, MHA -- for a
batch of 64 independent sequences at position 4095 (context 4096).  Per layer
one call of swiftkv_attention_f32: FP32 q/k/v -> Q15.17, RoPE, INT8/G32
quantize + append of token 4095, attention over the 4096-token INT8 cache.
Inputs (q/k/v for all 32 layers) and the 77 GB cache are resident in HBM
before timing; the cache is filled on the device through the append rule from
seeded N(0,1) rows.

    python bench.py [--steps K] [--warmup W] [--batch 64] [--context 4096]

Prints ONE JSON line.  value = algorithmic bytes of the step / step time
(GB/s), where per (sequence, layer) at position p the step moves
9216*p + 9216 + 65536 bytes (288 B per cached token-head + the appended row +
FP32 q/k/v/out).  Also reported: us/layer, tokens/s, % of 8 TB/s, the batch-1
figures (1% of K channels x20), the step kernel's roofline (hipEvents around
the timed region over the step-kernel launches in it), the integer-compatibility entry's time on the same workload, the
reference emulator's attention stage timed on this host (cpu_baseline), and
the secondary configurations under "configs": batch 1 at position 127 (one
layer), batch 1 at position 2047 (32 layers), batch 64 with attended lengths
drawn from U{256..4096} (one layer, and 32 layers), batch 16 decoding 512 steps from
position 32256 to 32767 on Student-t(3) data (one layer), and the batch-64
call with host-memory inputs and outputs (PCIe included; never `value`).
The batch-64 and batch-1 workloads are also timed through the entry that
takes the Q/K/V projection's split-K FP32 partials (--parts, default 4), and
the batch sizes between them (2 to 32) at position 4095 over 32 layers.
On the host: the reference emulator's attention stage at position 4095 (one
thread as shipped, and with its OpenMP pragmas), the FP32 tolerance oracle
(reported apart from the reference), and the reference's attention loop at
position 32256 extrapolated to the batch-16 512-step run.
"""
import argparse
import gc
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBPS = 8000.0
# Timer slots of the per-step event pairs (the library holds 64 slots; bench
# uses 0..9 for its regions).
STEP_SLOT0, STEP_SLOTS = 16, 48
MIN_STEP_SAMPLES = 20
METRIC = "decode-attn µs/layer + achieved HBM GB/s (% of peak), ctx 4096, batch 1/64"
TOKEN_HEAD_BYTES = 288
# Untimed warm-up of the main workload, in seconds, when its cache is large
# (above SETTLE_MIN_BYTES): the stream runs slower for a second or more after
# gigabytes have been allocated and filled (see Cache; a 4.8 GB cache of 16
# sequences at context 32768 timed right after its fill measured 714 us per
# launch against 693 settled).
SETTLE_S = 1.5
SETTLE_MIN_BYTES = 4 << 30


def step_bytes(position: int, parts: int = 1) -> int:
    """Algorithmic bytes of one (sequence, layer) step at `position`; with
    split-K partial inputs q/k/v each arrive as `parts` FP32 rows."""
    return 32 * (position * TOKEN_HEAD_BYTES + TOKEN_HEAD_BYTES + (3 * parts + 1) * 128 * 4)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


PROFILE_KEYS = ("traffic_bytes_per_launch", "algorithmic_bytes_per_launch", "trace_avg_us", "fetch_ratio",
                "lds_bank_conflict_cycles_per_launch", "lds_instructions_per_launch", "achieved_waves_per_simd",
                "achieved_occupancy_frac", "vgprs", "bench_ms_per_step", "commit")


def profile_summary(batch: int, context: int, ragged: bool = False):
    """The committed rocprofv3 summary of the step kernel on this workload:
    HBM bytes per launch (FETCH_SIZE and WRITE_SIZE, each scaled by the
    copy-kernel calibration), their ratio to the algorithmic bytes, LDS bank
    conflicts, achieved occupancy, and the commit and bench ms/step of the run
    it came from.  ({}, None) when no summary covers the workload."""
    path = os.path.join(REPO, "profiles", f"step_kernel_batch{batch}{'_ragged' if ragged else ''}_ctx{context}.md")
    if not os.path.exists(path):
        return {}, None
    vals = {}
    for line in open(path):
        key, sep, rest = line.partition(":")
        if sep and key.strip() in PROFILE_KEYS:
            text = rest.strip()
            if key.strip() == "commit":
                vals["commit"] = text
                continue
            try:
                vals[key.strip()] = float(text) if "." in text or "e" in text else int(text)
            except ValueError:
                vals[key.strip()] = text
    return vals, os.path.relpath(path, REPO)


def profile_counters(vals):
    """The counter evidence carried in a bench line's roofline."""
    keys = ("fetch_ratio", "lds_bank_conflict_cycles_per_launch", "lds_instructions_per_launch",
            "achieved_waves_per_simd", "achieved_occupancy_frac", "vgprs", "trace_avg_us", "commit",
            "bench_ms_per_step")
    return {k: vals[k] for k in keys if k in vals} or None


class Cache:
    """A KV cache and RoPE table filled on the device once, before any timed
    region, and kept until the end of the run: a workload of `batch`
    sequences uses slots 0 .. batch-1 and layers 0 .. layers-1.  Large
    allocations and frees between timed workloads are avoided on purpose: on
    MI355X the device streams about 4% slower for a second or more after
    tens of GB are allocated or freed (batch 4: 26.9 us/layer settled, 28.1
    right after a 77 GB cache was allocated and filled or freed, with no
    attention kernel in between)."""

    def __init__(self, skv, ctx, batch, layers, cap, seed, ntok=None, dist=0, outliers=False):
        self.batch, self.layers, self.cap = batch, layers, cap
        self.lut = skv.RopeLut.generate(ctx, max(cap, 4096))
        self.kv = skv.KVCache(ctx, layers=layers, max_batch=batch, max_seq_len=cap)
        t0 = time.time()
        ntok = cap - 1 if ntok is None else ntok
        self.kv.fill_synthetic(self.lut, ntok=ntok, seed=seed, dist=dist, k_outliers=outliers)
        ctx.synchronize()
        log(f"[bench] filled {self.kv.nbytes / 1e9:.1f} GB cache ({layers} layers x {batch} seq x {ntok} tokens) "
            f"in {time.time() - t0:.1f} s")

    def close(self):
        self.kv.close()
        self.lut.close()


def run_gpu(*args, **kwargs):
    """_run_gpu with Python's cyclic garbage collector paused: at batch 1 the
    host enqueues a call in about 6.5 us against a 10.5 us layer on the GPU, so
    a collection inside a timed region would leave the GPU idle."""
    enabled = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        return _run_gpu(*args, **kwargs)
    finally:
        if enabled:
            gc.enable()


def _run_gpu(skv, ctx, cache, positions, layers, steps, warmup, seed, outliers=False, dist=0, exact_steps=0,
             graph=True, advance=False, parts=0, settle_s=0.0, graph_steps=1):
    """Time `steps` decode steps of `layers` calls each over sequences at `positions`.

    `cache` (a Cache) holds the sequences' rows up to max(positions) (its
    fill); q/k/v for every layer are resident before timing (with outliers,
    1% of k's channels scaled x20, as in the cache's own rows).  With
    advance=True step s runs at positions + s (a decode run whose appends feed
    the next step); otherwise every step repeats the same positions (the
    appended row is rewritten with the same bits).  The untimed warm-up runs
    `warmup` steps and, with settle_s, goes on until that much time has
    passed.  The graph replay records `graph_steps` steps in one graph (for a
    one-layer step, a graph of one call would time hipGraphLaunch itself).
    """
    positions = np.asarray(positions, np.int32)
    batch = positions.size
    last = int(positions.max()) + (steps if advance else 1)   # last written position + 1
    assert batch <= cache.batch and layers <= cache.layers and last <= cache.cap, "workload outside its cache"
    kv, lut = cache.kv, cache.lut
    n_in = layers * batch * 4096
    qkv = [ctx.alloc(n_in * 4) for _ in range(3)]
    for i, buf in enumerate(qkv):
        ctx.fill_synthetic(buf, n_in, seed + 1, 1000 + i, dist=dist, outliers=(outliers and i == 1))
    out = ctx.alloc(batch * 4096 * 4)
    aq = ctx.alloc(batch * 128 * 56)
    asc = ctx.alloc(batch * 128)
    layer_stride = batch * 4096 * 4

    def one_step(pos):
        for layer in range(layers):
            off = layer * layer_stride
            skv.swiftkv_attention(ctx, qkv[0].ptr + off, qkv[1].ptr + off, qkv[2].ptr + off, kv, lut, aq, asc,
                                  layer, pos, out)

    for _ in range(0 if advance else warmup):
        one_step(positions)
    ctx.synchronize()
    t_settle = time.time()
    while not advance and time.time() - t_settle < settle_s:
        one_step(positions)
        ctx.synchronize()
    ctx.timer_record(0)
    for s in range(steps):
        one_step(positions + s if advance else positions)
    ctx.timer_record(1)
    ms = ctx.timer_elapsed_ms(0, 1)
    # The same steps again, each one bracketed by events (slot i before step
    # i, all on the stream, no host wait between steps): the median step.
    samples = []
    if not advance and layers >= 8:   # one launch per step would time the event pair itself
        n_each = max(MIN_STEP_SAMPLES, min(steps, STEP_SLOTS - 1))
        for s in range(n_each):
            ctx.timer_record(STEP_SLOT0 + s)
            one_step(positions)
        ctx.timer_record(STEP_SLOT0 + n_each)
        samples = [ctx.timer_elapsed_ms(STEP_SLOT0 + s, STEP_SLOT0 + s + 1) for s in range(n_each)]
    # The same steps again with an event pair around every launch, for the
    # step kernel's average duration (the roofline).  The event records add
    # small gaps on the stream, so `value` comes from the pass above.
    ctx.profile(True)
    for s in range(steps):
        one_step(positions + s if advance else positions)
    ctx.synchronize()
    counts, kms = ctx.profile_collect()
    ctx.profile(False)
    ms_graph = None
    if graph:
        # The same step recorded once into a HIP graph and replayed: the
        # GPU-side time of the per-layer calls without host launch overhead.
        ctx.capture_begin()
        for _ in range(graph_steps):
            one_step(positions)
        g = ctx.capture_end()
        for _ in range(warmup):
            g.launch()
        replays = max(1, steps // graph_steps)
        ctx.timer_record(2)
        for _ in range(replays):
            g.launch()
        ctx.timer_record(3)
        ms_graph = ctx.timer_elapsed_ms(2, 3) * steps / (replays * graph_steps)
        g.close()
    o = out.download(np.float32, (batch, 4096))
    assert np.isfinite(o).all(), "non-finite attention output"
    exact = None
    if exact_steps:
        # The integer-compatibility entry on the same workload (sequential
        # recurrence per head; reported beside the fast path, not as `value`).
        out_i = ctx.alloc(batch * 4096 * 4)

        def exact_step():
            for layer in range(layers):
                off = layer * layer_stride
                skv.swiftkv_attention_exact(ctx, qkv[0].ptr + off, qkv[1].ptr + off, qkv[2].ptr + off, kv, lut,
                                            aq, asc, layer, positions, out_i)
        exact_step()
        ctx.timer_record(4)
        for _ in range(exact_steps):
            exact_step()
        ctx.timer_record(5)
        ms_exact = ctx.timer_elapsed_ms(4, 5)
        oi = out_i.download(np.int32, (batch, 4096))
        out_i.free()
        err = float(np.abs(oi * 2.0 ** -17 - o.astype(np.float64)).max())
        exact = {"us_per_layer": 1000.0 * ms_exact / exact_steps / layers,
                 "gbps": exact_steps * layers * sum(step_bytes(int(p)) for p in positions) / (ms_exact / 1e3) / 1e9,
                 "max_abs_diff_vs_fp32_path": err}
    partials = None
    if parts:
        # The same steps fed by `parts`-way split-K FP32 partials through
        # swiftkv_attention_partials: the upstream linear stage's reduction and
        # finalize run inside the step's input loads.  Layout [part][layer][batch][4096].
        pbuf = [ctx.alloc(parts * n_in * 4) for _ in range(3)]
        for i, buf in enumerate(pbuf):
            ctx.fill_synthetic(buf, parts * n_in, seed + 2, 2000 + i, dist=dist)

        def parts_step():
            for layer in range(layers):
                off = layer * layer_stride
                skv.swiftkv_attention_partials(ctx, pbuf[0].ptr + off, pbuf[1].ptr + off, pbuf[2].ptr + off, parts,
                                               kv, lut, aq, asc, layer, positions, out, part_stride=n_in)
        for _ in range(warmup):
            parts_step()
        ctx.timer_record(6)
        for _ in range(steps):
            parts_step()
        ctx.timer_record(7)
        ms_parts = ctx.timer_elapsed_ms(6, 7)
        assert np.isfinite(out.download(np.float32, (batch, 4096))).all(), "non-finite output (partials)"
        for b in pbuf:
            b.free()
        pbytes = steps * layers * sum(step_bytes(int(p), parts) for p in positions)
        partials = {"parts": parts, "us_per_layer": 1000.0 * ms_parts / steps / layers,
                    "gbps": pbytes / (ms_parts / 1e3) / 1e9}
    for b in qkv + [out, aq, asc]:
        b.free()
    step_total = [sum(step_bytes(int(p) + (s if advance else 0)) for p in positions) for s in range(steps)]
    total_bytes = layers * sum(step_total)
    ms_step = ms / steps
    res = {
        "ms_per_step": ms_step,
        "ms_per_step_median": float(np.median(samples)) if samples else None,
        "step_samples": len(samples),
        "us_per_layer": 1000.0 * ms_step / layers,
        "gbps": total_bytes / (ms / 1e3) / 1e9,
        "tokens_per_s": batch * steps / (ms / 1e3),
        "kernel_launches": dict(zip(["append", "step"], counts)),
        "kernel_avg_us": {k: (1000.0 * t / c if c else None) for k, t, c in zip(["append", "step"], kms, counts)},
        "exact": exact,
        "partials": partials,
        "sum_attended": int(sum(int(p) + 1 for p in positions)),
    }
    res["pct_of_peak"] = 100.0 * res["gbps"] / HBM_PEAK_GBPS
    if ms_graph is not None:
        res["graph"] = {"us_per_layer": 1000.0 * ms_graph / steps / layers,
                        "gbps": total_bytes / (ms_graph / 1e3) / 1e9,
                        "tokens_per_s": batch * steps / (ms_graph / 1e3)}
        res["graph"]["pct_of_peak"] = 100.0 * res["graph"]["gbps"] / HBM_PEAK_GBPS
    # Dominant kernel: the step kernel moves the whole step's algorithmic bytes
    # (cached tokens, appended row, q/k/v in, output out) and is the only
    # kernel in the timed region (the profiled pass of the same calls counts
    # its launches), so the region's event-timed duration over its launch
    # count is the kernel's average launch duration.  An event pair around
    # every launch (kernel_avg_us) adds the records' own cost to each launch.
    assert counts[0] == 0, "the timed calls launched a kernel other than the step kernel"
    launches_per_call = counts[1] / (steps * layers)
    res["step_launches"] = counts[1]
    res["step_avg_us"] = 1000.0 * ms / (steps * layers * launches_per_call)
    res["dominant_bytes_per_launch"] = int(sum(step_total) / steps / launches_per_call)
    res["step_kernel_gbps"] = res["dominant_bytes_per_launch"] / (res["step_avg_us"] / 1e6) / 1e9
    return res


def run_prefill(skv, ctx, tokens, layers, reps, seed, modes=("own", "shared")):
    """swiftkv_append_tokens: the append rule (conversion, RoPE of k at its own
    position, G32 quantization) over a `tokens`-long prompt of one sequence,
    every layer; bytes = FP32 k and v read plus the 288-B rows written.  Each
    layer reads its own k and v, as a model's layers do, so the inputs come
    from HBM; the same prompt with one k/v pair for every layer (256 MB or
    less stays in the MALL) is reported beside it."""
    lut = skv.RopeLut.generate(ctx, max(tokens, 4096))
    kv = skv.KVCache(ctx, layers=layers, max_batch=1, max_seq_len=tokens)
    n = tokens * 4096
    ks, vs = [ctx.alloc(n * 4) for _ in range(layers)], [ctx.alloc(n * 4) for _ in range(layers)]
    for layer in range(layers):
        ctx.fill_synthetic(ks[layer], n, seed, 2 * layer)
        ctx.fill_synthetic(vs[layer], n, seed, 2 * layer + 1)
    per_layer_s = {}
    for mode in modes:
        def prompt():
            for layer in range(layers):
                i = layer if mode == "own" else 0
                skv.swiftkv_append_tokens(ctx, ks[i], vs[i], kv, lut, layer, 0, 0, tokens)
        prompt()                              # warm-up pass
        ctx.synchronize()
        t0 = time.time()                      # and untimed prompts while the fresh allocations settle (see Cache)
        while time.time() - t0 < SETTLE_S:
            prompt()
            ctx.synchronize()
        ctx.timer_record(8)
        for _ in range(reps):
            prompt()
        ctx.timer_record(9)
        per_layer_s[mode] = ctx.timer_elapsed_ms(8, 9) / 1e3 / reps / layers
    for b in ks + vs:
        b.free()
    kv.close()
    lut.close()
    bytes_per_layer = tokens * 32 * (2 * 128 * 4 + TOKEN_HEAD_BYTES)
    res = {}
    if "own" in per_layer_s:
        t = per_layer_s["own"]
        res = {"us_per_layer": round(t * 1e6, 2), "gbps": round(bytes_per_layer / t / 1e9, 1),
               "tokens_per_s": round(tokens / t / layers, 1)}
    if "shared" in per_layer_s:
        t = per_layer_s["shared"]
        res["one_kv_for_all_layers"] = {"us_per_layer": round(t * 1e6, 2), "gbps": round(bytes_per_layer / t / 1e9, 1)}
    res["bytes_per_layer"] = bytes_per_layer
    res["sample"] = f"{reps} prompts of {tokens} tokens x {layers} layers, one sequence, each layer its own k/v"
    return res


def run_host_io(skv, ctx, cache, context, reps, seed):
    """The per-layer call with host-memory q/k/v/out/A14 (pageable numpy
    arrays): copies in, step, copies out, wait -- the PCIe-inclusive rate,
    on layer 0 of every sequence of `cache`."""
    pos = context - 1
    batch, kv, lut = cache.batch, cache.kv, cache.lut
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((batch, 4096)).astype(np.float32) for _ in range(3))
    out = np.empty((batch, 4096), np.float32)
    aq, asc = np.empty((batch, 128, 56), np.uint8), np.empty((batch, 128), np.uint8)
    positions = np.full(batch, pos, np.int32)
    ctx.set_host_io(True)
    times = []
    try:
        for i in range(reps + 2):
            t0 = time.perf_counter()
            skv.swiftkv_attention(ctx, q, k, v, kv, lut, aq, asc, 0, positions, out)
            if i >= 2:
                times.append(time.perf_counter() - t0)
    finally:
        ctx.set_host_io(False)
    assert np.isfinite(out).all()
    t = float(np.median(times))
    return {"us_per_layer": round(t * 1e6, 1), "gbps": round(batch * step_bytes(pos) / t / 1e9, 1),
            "host_bytes_per_layer": int(q.nbytes * 3 + out.nbytes + aq.nbytes + asc.nbytes),
            "sample": f"median of {reps} synchronous calls, one layer, pageable host arrays"}


def summary(res, graph=True):
    """The figures reported for a secondary configuration."""
    d = {"us_per_layer": round(res["us_per_layer"], 3), "gbps": round(res["gbps"], 1),
         "pct_of_peak": round(res["pct_of_peak"], 2), "tokens_per_s": round(res["tokens_per_s"], 1),
         "step_kernel_avg_us": round(res["step_avg_us"], 2),
         "step_kernel_gbps": round(res["step_kernel_gbps"], 1)}
    if res.get("ms_per_step_median"):
        layers = res["ms_per_step"] / res["us_per_layer"] * 1000.0
        d["us_per_layer_median_step"] = round(1000.0 * res["ms_per_step_median"] / layers, 3)
    if graph and "graph" in res:
        d["graph_replay"] = {k: round(v, 3) for k, v in res["graph"].items()}
    return d


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


_CPU_CACHES = {}


def _cpu_cache(position: int):
    """The oracle's host cache of one sequence filled to `position` tokens by
    the append rule from seeded N(0,1) rows, with that step's q/k/v; built
    once and shared by the CPU timings."""
    if position not in _CPU_CACHES:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        sys.path.insert(0, os.path.join(REPO, "tests"))
        import oracle as O
        from helpers import f32_normal
        cos, sin = O.rope_values(position + 1)
        sc = O.SequenceCache(32, position + 1)
        sc.fill_q17(O.f2q17(f32_normal(7, (position, 4096))), O.f2q17(f32_normal(8, (position, 4096))), 0, cos,
                    sin)
        qkv = [O.f2q17(f32_normal(9 + i, (4096,))) for i in range(3)]
        _CPU_CACHES[position] = (cos, sin, sc, qkv)
    return _CPU_CACHES[position]


def cpu_baseline(target_seconds: float, position: int, omp: bool):
    """The reference emulator's attention stage (oracle/_ref, compiled from the
    reference source) on this host: one sequence x 32 heads per call at
    `position`, cache pre-filled through the oracle's append rule."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import oracle as O
    if not O.Reference.available(omp):
        return None
    R = O.Reference(omp=omp)
    cos, sin, sc, (q, k, v) = _cpu_cache(position)
    R.set_rope(cos, sin)
    rc = R.cache(position + 1)
    rc.load_from(sc, position)
    qr, kr = R.apply_rope(q, position), R.apply_rope(k, position)
    rc.attention(qr, kr, v, position)          # warm-up call
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < target_seconds or len(times) < 3:
        t0 = time.perf_counter()
        rc.attention(qr, kr, v, position)
        times.append(time.perf_counter() - t0)
    per_call = float(np.median(times))
    return {
        "value": step_bytes(position) / per_call / 1e9,
        "unit": "GB/s",
        "us_per_layer_batch1": per_call * 1e6,
        "us_per_layer_batch64": per_call * 64 * 1e6,
        "cores": R.L.ref_omp_threads(),
        "cpu_model": cpu_model(),
        "nproc": os.cpu_count(),
        "kind": "reference",
        "sample": (f"{len(times)} calls of the reference emulator's swiftkv_attention_4pe (32 heads, one "
                   f"sequence, one layer, position {position}), median; batch-64 figure = 64 x per-call"),
    }


def cpu_fp32_oracle(target_seconds: float, position: int):
    """The FP32 tolerance oracle (oracle/swiftkv_oracle.c: the append rule,
    then the FP32 softmax formula with double accumulation) on this host, one
    thread, one sequence x 32 heads per call at `position`.  Timed separately
    from the reference: it is the oracle, not the reference."""
    cos, sin, sc, (q, k, v) = _cpu_cache(position)
    sc.step_q17(q, k, v, position, cos[position], sin[position], fp=True)   # warm-up call
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < target_seconds or len(times) < 3:
        t0 = time.perf_counter()
        sc.step_q17(q, k, v, position, cos[position], sin[position], fp=True)
        times.append(time.perf_counter() - t0)
    per_call = float(np.median(times))
    return {"us_per_sequence_layer": round(per_call * 1e6, 1), "gbps": round(step_bytes(position) / per_call / 1e9, 3),
            "cores": 1, "kind": "oracle (FP32 formula, double accumulation)",
            "sample": f"{len(times)} calls at position {position}, one sequence x 32 heads, median"}


def cpu_reference_long_context(calls: int, position: int, batch: int, steps: int):
    """The reference emulator's attention loop (oracle/_ref, one thread) at a
    position beyond its own 4096-token limit, for the batch-16 32K decode run:
    `calls` calls of one sequence at `position` (q/k rotated by the oracle's
    extended table, cache rows random codes -- the loop's cost does not depend
    on their values), scaled to batch x steps calls at the run's mean position."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    if not O.Reference.available(False):
        return None
    R = O.Reference(omp=False)
    rng = np.random.default_rng(11)
    sc = O.SequenceCache(32, position + 1)
    sc.kc[:] = rng.integers(-127, 128, sc.kc.shape, dtype=np.int8)
    sc.vc[:] = rng.integers(-127, 128, sc.vc.shape, dtype=np.int8)
    sc.ks[:] = rng.integers(0, 8, sc.ks.shape, dtype=np.uint8)
    sc.vs[:] = rng.integers(0, 8, sc.vs.shape, dtype=np.uint8)
    rc = R.cache(position + 1)
    rc.load_from(sc, position)
    del sc
    q, k, v = (rng.integers(-(1 << 18), 1 << 18, 4096, dtype=np.int32) for _ in range(3))
    times = []
    for _ in range(calls):
        t0 = time.perf_counter()
        rc.attention(q, k, v, position)
        times.append(time.perf_counter() - t0)
    per_call = float(np.median(times))
    mean_pos = position + (steps - 1) / 2.0
    total_s = per_call * (mean_pos + 1) / (position + 1) * batch * steps
    return {"us_per_sequence_step": round(per_call * 1e6, 1), "extrapolated_total_s": round(total_s, 1),
            "cores": 1, "kind": "reference",
            "sample": (f"{calls} calls of the reference emulator's swiftkv_attention_4pe at position {position} "
                       f"(one sequence, 32 heads), median; extrapolated to {batch} sequences x {steps} steps "
                       f"at the mean position")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--split", type=int, default=0, help="tokens per split (0 = heuristic)")
    ap.add_argument("--ragged", action="store_true",
                    help="main workload with attended lengths drawn from U{256..context} (seed 4), the ragged "
                         "configuration, instead of every sequence at position context - 1")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batch1", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the secondary configurations (position 127, 2047, ragged, 32K)")
    ap.add_argument("--exact-steps", type=int, default=1,
                    help="steps of the integer-compatibility entry to time (0 = skip)")
    ap.add_argument("--parts", type=int, default=4,
                    help="also time the step fed by this many split-K FP32 partials (0 = skip)")
    ap.add_argument("--prefill", type=int, default=0, metavar="TOKENS",
                    help="only time swiftkv_append_tokens over a prompt of TOKENS tokens, --layers layers, "
                         "--steps prompts, each layer reading its own k/v (--prefill-shared: one k/v for all)")
    ap.add_argument("--prefill-shared", action="store_true")
    ap.add_argument("--calibrate", action="store_true",
                    help="only run the FP32->Q15.17 conversion kernel over 256 Mi elements (a copy of known "
                         "size: 1 GiB read, 1 GiB written per launch) to scale HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; --gpus must be 1 (the path shards by "
                                   "head/sequence across GPUs by design only)"}))
        sys.exit(2)

    import importlib
    skv = importlib.import_module("4pe_u250_amd")
    ctx = skv.Context(0)
    if args.calibrate:
        n = 256 << 20
        src, dst = ctx.alloc(4 * n), ctx.alloc(4 * n)
        ctx.fill_synthetic(src, n, 1, 1)
        for _ in range(3):
            ctx.convert_f32_q17(src, dst, n)
        ctx.synchronize()
        print(json.dumps({"calibration": "convert_kernel", "elements": n, "read_bytes": 4 * n,
                          "write_bytes": 4 * n, "launches": 3}), flush=True)
        ctx.close()
        return
    if args.prefill:
        r = run_prefill(skv, ctx, args.prefill, args.layers, args.steps, seed=2034,
                        modes=("shared",) if args.prefill_shared else ("own",))
        print(json.dumps({"prefill_tokens": args.prefill, "layers": args.layers, "prompts": args.steps,
                          "inputs": "one k/v for every layer" if args.prefill_shared else "each layer its own k/v",
                          **r}), flush=True)
        ctx.close()
        return
    ctx.set_split_tokens(args.split)
    log(f"[bench] {skv.version()}")
    if args.ragged:
        main_positions = np.random.default_rng(4).integers(256, args.context + 1, args.batch) - 1
    else:
        main_positions = np.full(args.batch, args.context - 1)
    # The prefill allocates and frees its own cache and inputs, so it runs
    # before the decode caches exist.
    prefill = run_prefill(skv, ctx, 4096, 32, 5, seed=2034) if not args.no_configs else None
    # Every decode cache of the run is allocated and filled here, before the
    # first timed decode region, and freed at the end (see Cache).  The main
    # cache also serves the secondary workloads of up to its batch and context.
    main = Cache(skv, ctx, args.batch, args.layers, args.context, seed=2026, ntok=int(main_positions.max()))
    b1_cache = (Cache(skv, ctx, 1, args.layers, args.context, seed=2027, outliers=True)
                if not args.no_batch1 else None)
    long_cache = (Cache(skv, ctx, 16, 1, 32768, seed=2031, ntok=32256, dist=skv.DIST_STUDENT_T3)
                  if not args.no_configs else None)
    main_res = run_gpu(skv, ctx, main, main_positions, args.layers, args.steps, args.warmup,
                       seed=2026, exact_steps=args.exact_steps, parts=args.parts,
                       settle_s=SETTLE_S if main.kv.nbytes + (long_cache.kv.nbytes if long_cache else 0) > SETTLE_MIN_BYTES
                       else 0.0)
    log(f"[bench] batch {args.batch}: {main_res['us_per_layer']:.1f} us/layer, {main_res['gbps']:.0f} GB/s "
        f"(graph replay {main_res['graph']['us_per_layer']:.1f} us/layer)")
    if main_res["partials"]:
        log(f"[bench] batch {args.batch}, {args.parts} split-K partials: "
            f"{main_res['partials']['us_per_layer']:.1f} us/layer")
    b1 = None
    extra = {}
    if not args.no_batch1:
        # batch-1 headline: 1% of K channels x20
        b1 = run_gpu(skv, ctx, b1_cache, [args.context - 1], args.layers, max(args.steps, 20), args.warmup,
                     seed=2027, outliers=True, parts=args.parts, exact_steps=min(args.exact_steps, 1) * 5)
        log(f"[bench] batch 1: {b1['us_per_layer']:.2f} us/layer, {b1['gbps']:.0f} GB/s "
            f"(graph replay {b1['graph']['us_per_layer']:.2f} us/layer)")
        if b1["partials"]:
            log(f"[bench] batch 1, {args.parts} split-K partials: {b1['partials']['us_per_layer']:.2f} us/layer")
    if not args.no_configs:
        # The secondary workloads run on the main cache's slots 0 .. batch-1
        # (every one fits its 64 sequences x 32 layers x 4096 tokens).
        assert not args.ragged and args.batch >= 64 and args.layers >= 32 and args.context >= 4096, \
            "the secondary workloads use the default main cache"
        # One launch per step: a graph of a single node would time hipGraphLaunch, not the kernel.
        # One layer per step, so eager steps are timed at the host's call rate when that is slower than the
        # GPU; the graph replay (50 recorded calls per graph) is the GPU's own time per call.
        r = run_gpu(skv, ctx, main, [127], 1, 200, args.warmup, seed=2028, graph_steps=50)
        extra["batch1_position127_1layer"] = summary(r)
        r = run_gpu(skv, ctx, main, [2047], 32, 20, args.warmup, seed=2029)
        extra["batch1_position2047_32layers"] = summary(r)
        # One layer repeated: its 37.8 MB stay resident in the 256 MB MALL, so
        # this is the cache-resident figure, reported apart from the sweep.
        r = run_gpu(skv, ctx, main, [4095], 1, 200, args.warmup, seed=2033, graph_steps=50)
        extra["batch1_position4095_1layer_repeated_mall_resident"] = summary(r)
        rng = np.random.default_rng(4)
        lengths = rng.integers(256, 4097, 64)
        r = run_gpu(skv, ctx, main, lengths - 1, 32, args.steps, args.warmup, seed=2030)
        extra["batch64_ragged_32layers"] = dict(summary(r), length_seed=4, sum_attended=r["sum_attended"],
                                                lengths="U{256..4096}")
        # the same lengths, one layer timed on its own (its 1.3 GB exceeds the 256 MB MALL)
        r = run_gpu(skv, ctx, main, lengths - 1, 1, 100, args.warmup, seed=2030, graph=False)
        extra["batch64_ragged_1layer"] = dict(summary(r, graph=False), length_seed=4, lengths="U{256..4096}")
        sweep = {}
        # The batch sizes between the two headline ones, 32 layers at context 4096.  Three warm-up steps: the
        # first steps after a workload of another batch size run 0.1-0.4 us/layer slower.
        for b in (2, 4, 8, 16, 32):
            r = run_gpu(skv, ctx, main, np.full(b, args.context - 1), 32, 20, 3, seed=2040 + b, graph=False)
            sweep[str(b)] = {"us_per_layer": round(r["us_per_layer"], 2), "gbps": round(r["gbps"], 1),
                             "pct_of_peak": round(r["pct_of_peak"], 2)}
        extra["batch_sweep_position4095_32layers"] = sweep
        log("[bench] batch sweep: " + ", ".join(f"{b}: {v['us_per_layer']:.1f} us" for b, v in sweep.items()))
        r = run_gpu(skv, ctx, long_cache, np.full(16, 32256), 1, 512, 0, seed=2031, dist=skv.DIST_STUDENT_T3,
                    graph=False, advance=True)
        extra["batch16_positions32256to32767_1layer_t3"] = dict(summary(r, graph=False),
                                                                 steps=512, ms_total=round(r["ms_per_step"] * 512, 2))
        for k, v in extra.items():
            if "us_per_layer" in v:
                log(f"[bench] {k}: {v['us_per_layer']:.2f} us/layer, {v['gbps']:.0f} GB/s")
        extra["batch64_position4095_host_io"] = run_host_io(skv, ctx, main, args.context, 20, seed=2032)
    for c in (main, b1_cache, long_cache):
        if c is not None:
            c.close()
    if not args.no_configs:
        extra["prefill_append_4096tokens_32layers"] = prefill
        log(f"[bench] prefill append, 4096 tokens: {prefill['us_per_layer']:.1f} us/layer, {prefill['gbps']:.0f} GB/s")
        log(f"[bench] host-memory I/O, batch {args.batch}: "
            f"{extra['batch64_position4095_host_io']['us_per_layer']:.1f} us/layer")
    ctx.close()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds, args.context - 1, omp=False)
        if cpu:
            log(f"[bench] cpu reference: {cpu['us_per_layer_batch1']:.0f} us per sequence-layer")
            omp = cpu_baseline(max(2.0, args.cpu_seconds / 4), args.context - 1, omp=True)
            if omp:
                cpu["openmp"] = {"value": omp["value"], "cores": omp["cores"],
                                 "us_per_layer_batch1": omp["us_per_layer_batch1"]}
        oracle_fp = cpu_fp32_oracle(max(2.0, args.cpu_seconds / 4), args.context - 1)
        log(f"[bench] cpu FP32 oracle: {oracle_fp['us_per_sequence_layer']:.0f} us per sequence-layer")
        if extra:
            long_ref = cpu_reference_long_context(2, 32256, 16, 512)
            if long_ref:
                extra["batch16_positions32256to32767_1layer_t3"]["cpu_reference"] = long_ref
                log(f"[bench] cpu reference at position 32256: {long_ref['us_per_sequence_step']:.0f} us per "
                    f"sequence-step")

    att = main_res["step_avg_us"]
    prof, traffic_src = profile_summary(args.batch, args.context, ragged=args.ragged)
    traffic = prof.get("traffic_bytes_per_launch")
    line = {
        "metric": METRIC,
        "value": round(main_res["gbps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["ms_per_step"], 4),
        "ms_per_step_median": (round(main_res["ms_per_step_median"], 4) if main_res["ms_per_step_median"]
                               else None),
        "step_timing": (f"ms_per_step: hipEvents around the {args.steps} timed steps / {args.steps}; "
                        + (f"ms_per_step_median: median of {main_res['step_samples']} further steps, each between "
                           "its own pair of events on the stream" if main_res["step_samples"] else
                           "no per-step median: a step of fewer than 8 launches would time its own event pair")),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded N(0,1) q/k/v and cache rows, cache built on device by the append rule)",
        "config": {"workload": (f"decode-attention step: {args.layers} layers x batch {args.batch} x "
                                + (f"attended lengths U{{256..{args.context}}} (seed 4)" if args.ragged else
                                   f"position {args.context - 1} (ctx {args.context})")
                                + ", 32 heads x 128, MHA, INT8/G32 KV cache"),
                   "batch": args.batch, "context": args.context, "layers": args.layers, "heads": 32,
                   "head_dim": 128, "kv_dtype": "int8+fp32 G32 scales"},
        "us_per_layer": round(main_res["us_per_layer"], 2),
        "us_per_layer_median_step": (round(1000.0 * main_res["ms_per_step_median"] / args.layers, 2)
                                     if main_res["ms_per_step_median"] else None),
        "tokens_per_s": round(main_res["tokens_per_s"], 1),
        "pct_of_peak": round(main_res["pct_of_peak"], 2),
        "kernel_avg_us_event_pairs": {k: (round(v, 2) if v else v) for k, v in main_res["kernel_avg_us"].items()},
        "graph_replay": {k: round(v, 2) for k, v in main_res["graph"].items()},
        "roofline": {"bound": "hbm", "achieved": round(main_res["step_kernel_gbps"], 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(main_res["step_kernel_gbps"] / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "traffic_source": traffic_src, "kernel": "step_kernel",
                     "bytes_per_launch": main_res["dominant_bytes_per_launch"],
                     "avg_launch_us": round(att, 2),
                     "launches": main_res["step_launches"],
                     "timing": "hipEvents around the timed region on the context stream / step-kernel launches in "
                               "it (the only kernel there)",
                     "profile_counters": profile_counters(prof)},
        "cpu_baseline": cpu,
    }
    if not args.no_cpu:
        line["cpu_fp32_oracle"] = oracle_fp
    if main_res["exact"]:
        e = main_res["exact"]
        line["integer_exact_path"] = {"us_per_layer": round(e["us_per_layer"], 1), "gbps": round(e["gbps"], 1),
                                      "max_abs_diff_vs_fp32_path": e["max_abs_diff_vs_fp32_path"]}
    if main_res["partials"]:
        p = main_res["partials"]
        line["split_k_partials_input"] = {
            "parts": p["parts"], "us_per_layer": round(p["us_per_layer"], 2), "gbps": round(p["gbps"], 1),
            "note": "same workload through swiftkv_attention_partials; bytes count the parts x FP32 q/k/v rows"}
    if b1:
        line["batch1"] = dict(summary(b1), workload="32 layers x batch 1 x position 4095, 1% of K channels x20")
        if b1["exact"]:
            line["batch1"]["integer_exact_path"] = {"us_per_layer": round(b1["exact"]["us_per_layer"], 1),
                                                    "max_abs_diff_vs_fp32_path":
                                                        b1["exact"]["max_abs_diff_vs_fp32_path"]}
        if b1["partials"]:
            line["batch1"]["split_k_partials_input"] = {"parts": b1["partials"]["parts"],
                                                        "us_per_layer": round(b1["partials"]["us_per_layer"], 3),
                                                        "gbps": round(b1["partials"]["gbps"], 1)}
        prof1, t1_src = profile_summary(1, args.context)
        line["batch1"]["us_per_layer_median_step"] = round(1000.0 * b1["ms_per_step_median"] / args.layers, 3)
        line["batch1"]["roofline"] = {"bound": "hbm (latency-bound at this size)",
                                      "achieved": round(b1["step_kernel_gbps"], 1), "peak": HBM_PEAK_GBPS,
                                      "unit": "GB/s", "frac": round(b1["step_kernel_gbps"] / HBM_PEAK_GBPS, 4),
                                      "traffic": prof1.get("traffic_bytes_per_launch"), "traffic_source": t1_src,
                                      "bytes_per_launch": b1["dominant_bytes_per_launch"],
                                      "avg_launch_us": round(b1["step_avg_us"], 2),
                                      "profile_counters": profile_counters(prof1)}
    if extra:
        line["configs"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
