"""Phase breakdown of the decode-attention step kernel on the GPU.

    python 4pe_u250_amd/phase_stamps.py [--batches 1,2,4] [--position 4095] [--layers 32] [--reps 10]
                                        [--parts 4] [--raw DIR]

Runs 32-layer decode steps through the instrumented build libswiftkv_stamps.so
(built by build.py: the product sources with SWIFTKV_PHASE_STAMPS, whose step
kernel records s_memrealtime, a 100 MHz clock, at its phase boundaries) and
prints, per batch size, the phases of the last layer's launch in microseconds
from the first workgroup's start, medians over the repetitions:
  - start:       workgroup entry (spread of the dispatch);
  - first loads: wave 0's first block and row loads all arrived (the build
                 waits for them there, about 0.2 us later than the product);
  - stream:      every wave's first-block arrival (p50, max);
  - scan:        every wave's scan end (p50, max) and the scan time after its
                 first block arrived;
  - LDS merge:   the workgroup's waves merged;
  - arrival:     a split workgroup's count taken (split heads only);
  - merge:       the last split's fetch and log-sum-exp merge;
  - epilogue:    FP32 row and A14/E8M0 words written;
  - launch:      the event-timed time per layer minus the span from the first
                 workgroup's start to the last one's end (dispatch, completion
                 and the gap to the next launch);
  - per XCD:     workgroups, their median span from entry to end, and the
                 XCD's last workgroup end;
  - per wave:    each wave slot's mean first-block arrival and scan end, and
                 the median first-block spread inside a workgroup;
  - merges:      split heads' mergers, and how many sit on odd XCDs;
  - dispatch:    the XCD of grid index i is (i + offset) mod 8 when one offset
                 holds for the whole launch.
With --parts N (2 or 4) the steps go through swiftkv_attention_partials, fed
N split-K FP32 partials of q, k and v.
Diagnostics only: nothing here is the product path, and the product library
compiles every stamp away.
"""
import argparse
import ctypes as C
import importlib
import json
import os
import sys
import time

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(PKG))
STAMPS_LIB = os.path.join(PKG, "libswiftkv_stamps.so")
WGS, SLOTS = 8192, 8
TICK_US = 0.01   # s_memrealtime runs at 100 MHz


def pct(x, q):
    x = np.asarray(x, np.float64)
    x = x[np.isfinite(x)]
    return float(np.percentile(x, q)) if x.size else float("nan")


def launch_phases(ph, wv, nwg, index=None):
    """Phase times (us) of one launch from its stamps; `index`: the live
    workgroups' linear grid indices (for the dispatch order)."""
    ph = ph[:nwg].astype(np.int64)
    wv = wv[:nwg].astype(np.int64)
    t0 = ph[:, 0].min()
    rel = lambda x: np.where(x > 0, (x - t0) * TICK_US, np.nan)
    split = (ph[:, 6] & 2) != 0
    merger = (ph[:, 6] & 1) != 0
    entry, first, lds, arrive, merged, done = (rel(ph[:, i]) for i in range(6))
    wd, we = rel(wv[:, :, 0]), rel(wv[:, :, 1])
    end = np.fmax(np.where(np.isnan(done), -np.inf, done), np.where(np.isnan(arrive), -np.inf, arrive))
    d = {"start_max": pct(entry, 100), "first_loads_p50": pct(first, 50), "first_loads_max": pct(first, 100),
         "stream_p50": pct(wd, 50), "stream_max": pct(wd, 100),
         "scan_end_p50": pct(we, 50), "scan_end_max": pct(we, 100), "scan_after_data_p50": pct(we - wd, 50),
         "lds_merge_p50": pct(lds, 50), "lds_merge_max": pct(lds, 100), "span": float(np.max(end))}
    if merger.any():
        d.update({"arrival_p50": pct(arrive[split] - lds[split], 50),
                  "merge_p50": pct(merged[merger] - arrive[merger], 50),
                  "epilogue_p50": pct(done[merger] - merged[merger], 50),
                  "last_lds_to_end": float(np.max(end) - np.nanmax(lds))})
    else:
        d.update({"epilogue_p50": pct(done - lds, 50), "last_lds_to_end": float(np.max(end) - np.nanmax(lds))})
    # Per XCD (slot 7's low half): workgroups, their mean span from entry to
    # end, and the XCD's last workgroup end.
    xcd = ph[:, 7] & 0xFFFFFFFF
    d["xcd_workgroups"] = [int((xcd == x).sum()) for x in range(8)]
    d["xcd_workgroup_us_p50"] = [pct((end - entry)[xcd == x], 50) if (xcd == x).any() else float("nan")
                                  for x in range(8)]
    d["xcd_done"] = [float(np.max(end[xcd == x])) if (xcd == x).any() else float("nan") for x in range(8)]
    # Per wave slot (waves that stamped): mean first-block arrival and scan
    # end, and the median spread of first-block arrivals inside a workgroup.
    waves = int(np.max(np.sum(wv[:, :, 0] > 0, axis=1)))
    d["wave_first_block_mean"] = [float(np.nanmean(wd[:, w])) for w in range(waves)]
    d["wave_scan_end_mean"] = [float(np.nanmean(we[:, w])) for w in range(waves)]
    d["first_block_spread_p50"] = pct(np.nanmax(wd[:, :waves], axis=1) - np.nanmin(wd[:, :waves], axis=1), 50)
    # The split that counted last and merged: how many sit on odd XCDs.
    d["mergers"] = int(merger.sum())
    d["mergers_on_odd_xcd"] = int((merger & (xcd % 2 == 1)).sum())
    # Dispatch order: XCD minus linear grid index, mod 8, when one value
    # holds for every workgroup of the launch (-1 otherwise).
    if index is not None:
        offs = np.unique((xcd - np.asarray(index, np.int64)) % 8)
        d["dispatch_xcd_offset"] = int(offs[0]) if offs.size == 1 else -1
    return d


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--batches", default="1,2,4")
    ap.add_argument("--position", type=int, default=4095)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--json", default=None, help="also write the medians here")
    ap.add_argument("--parts", type=int, default=0, help="feed N split-K FP32 partials (swiftkv_attention_partials)")
    ap.add_argument("--raw", default=None, metavar="DIR",
                    help="also save each repetition's stamps of the last launch (live workgroups, with their "
                         "grid index) as DIR/stamps_batch<B>.npz")
    args = ap.parse_args()
    if not os.path.exists(STAMPS_LIB):
        raise SystemExit(f"{STAMPS_LIB} is missing: python 4pe_u250_amd/build.py")
    skv = importlib.import_module("4pe_u250_amd")
    skv.LIB_PATH = STAMPS_LIB
    L = skv.lib()
    L.swiftkv_debug_phase_stamps.argtypes = [C.c_void_p, C.c_void_p]
    ctx = skv.Context(0)
    out = {}
    for batch in (int(x) for x in args.batches.split(",")):
        layers, pos = args.layers, args.position
        lut = skv.RopeLut.generate(ctx, max(pos + 1, 4096))
        kv = skv.KVCache(ctx, layers=layers, max_batch=batch, max_seq_len=pos + 1)
        kv.fill_synthetic(lut, ntok=pos, seed=5)
        parts = args.parts
        per_layer = batch * 4096 * max(parts, 1)          # elements of one layer's q (all its parts)
        n = layers * per_layer
        qkv = [ctx.alloc(n * 4) for _ in range(3)]
        for i, b in enumerate(qkv):
            ctx.fill_synthetic(b, n, 9, 100 + i)
        o, aq, asc = ctx.alloc(batch * 4096 * 4), ctx.alloc(batch * 128 * 56), ctx.alloc(batch * 128)
        positions = np.full(batch, pos, np.int32)
        stride = per_layer * 4

        def step():
            for layer in range(layers):
                q, k, v = (buf.ptr + layer * stride for buf in qkv)
                if parts:
                    skv.swiftkv_attention_partials(ctx, q, k, v, parts, kv, lut, aq, asc, layer, positions, o)
                else:
                    skv.swiftkv_attention(ctx, q, k, v, kv, lut, aq, asc, layer, positions, o)

        # Warm up for 1.5 s: right after gigabytes are allocated and filled
        # the device streams slower for a second or more.
        t_warm = time.time()
        while time.time() - t_warm < 1.5:
            step()
            ctx.synchronize()
        rows, raw = [], []
        ph = np.zeros((WGS, SLOTS), np.uint64)
        wv = np.zeros((WGS, 16, 2), np.uint64)
        for _ in range(args.reps):
            ph[:] = 0
            wv[:] = 0
            ctx.timer_record(0)
            step()
            ctx.timer_record(1)
            us_layer = 1000.0 * ctx.timer_elapsed_ms(0, 1) / layers
            if L.swiftkv_debug_phase_stamps(ph.ctypes.data, wv.ctypes.data) != 0:
                raise SystemExit("reading the stamps failed")
            # workgroups of the last launch: stamps left by an earlier, larger
            # launch are milliseconds older
            live = (ph[:, 0] > 0) & (ph[:, 0] >= ph[:, 0].max() - np.uint64(100000))
            nwg = int(live.sum())
            if args.raw:
                raw.append((np.flatnonzero(live), ph[live].copy(), wv[live].copy()))
            d = launch_phases(ph[live], wv[live], nwg, index=np.flatnonzero(live))
            d["us_per_layer"] = us_layer
            d["launch"] = us_layer - d["span"]
            d["workgroups"] = nwg
            rows.append(d)
        med = {k: (np.round(np.median([r[k] for r in rows], axis=0), 3).tolist() if isinstance(rows[0][k], list)
                   else round(float(np.median([r[k] for r in rows])), 3)) for k in rows[0]}
        tag = f", {parts} partials" if parts else ""
        out[f"batch{batch}_position{pos}" + (f"_parts{parts}" if parts else "")] = med
        print(f"batch {batch}, position {pos}, {layers} layers{tag}: " + json.dumps(med), flush=True)
        if args.raw:
            os.makedirs(args.raw, exist_ok=True)
            split, grid, waves, block, order = skv.step_plan(positions)
            np.savez_compressed(os.path.join(args.raw, f"stamps_batch{batch}.npz"),
                                index=np.stack([r[0] for r in raw]), phase=np.stack([r[1] for r in raw]),
                                wave=np.stack([r[2] for r in raw]), grid=np.array([grid, 32, batch]),
                                split_tokens=split, waves=waves, position=pos)
        for b in qkv + [o, aq, asc]:
            b.free()
        kv.close()
        lut.close()
    ctx.close()
    if args.json:
        with open(args.json, "w") as f:
            json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
