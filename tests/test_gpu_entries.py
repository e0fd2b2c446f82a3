"""Every step entry on the same seeded workload, through the C ABI.

One cache per case, filled on the device through the append rule; the same
step then runs through swiftkv_attention_f32 (the reference entry), the
Q15.17-input entry, the allocation-free entry and the split-K partials entry
(2 or 4 parts whose reduction in the reference's order is the FP32 input).
A step never reads the row it appends (the new token is forwarded), so the
entries can share the cache.  Required:
- bit-identical FP32 outputs, A14 words, E8M0 codes and appended rows across
  the four entries (the allocation-free entry may instead refuse a plan that
  splits a head more than 8 ways, with SWIFTKV_ERANGE);
- on sampled sequences, the oracle: every cached and appended row bit-exact,
  the FP32 output within max-abs 2e-5 + rel 1e-4 of the FP32 formula, the A14
  rule bit-exact on the output;
- for positions below 4096, the integer-compatibility entry bit-exact against
  the oracle's integer recurrence (state, A14 words, E8M0 codes).
Cases are seeded random draws of batch (1-257), uniform or ragged positions,
cache capacity, layer, forced split and step shape, data distribution and K
outlier channels."""
import sys

import numpy as np
import pytest

import oracle as O
from gpu_cases import H, assert_close, assert_rows_equal, oracle_cache_synthetic

pytestmark = pytest.mark.gpu


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lut4096(skv, ctx):
    lut = skv.RopeLut.generate(ctx, 4096)
    yield lut
    lut.close()


def _draw(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.choice([1, 1, 2, 3, 4, 5, 8, 12, 16, 24, 33, 64, 100, 257]))
    uniform = rng.random() < 0.5
    hi = 4096 if B <= 64 else 1600
    positions = [int(rng.integers(0, hi))] * B if uniform else [int(p) for p in rng.integers(0, hi, B)]
    mp = max(positions)
    return dict(
        rng=rng, B=B, positions=positions, uniform=uniform,
        cap=min(4096, mp + 1 + int(rng.choice([0, 0, 1, 63, 64, 700]))),
        layers=int(rng.integers(1, 4)))


def _step(skv, ctx, entry, B, q, k, v, kv, lut, layer, positions, parts=0, stride=None):
    out, aq, asc = ctx.alloc(B * 4096 * 4), ctx.alloc(B * 128 * 56), ctx.alloc(B * 128)
    try:
        if entry == "f32":
            skv.swiftkv_attention(ctx, q, k, v, kv, lut, aq, asc, layer, positions, out)
        elif entry == "q17":
            skv.swiftkv_attention(ctx, q, k, v, kv, lut, aq, asc, layer, positions, out, q17=True)
        elif entry == "noalloc":
            skv.swiftkv_attention_noalloc(ctx, q, k, v, kv, lut, aq, asc, layer, positions, out)
        elif entry == "parts":
            skv.swiftkv_attention_partials(ctx, q, k, v, parts, kv, lut, aq, asc, layer, positions, out,
                                           part_stride=stride)
        else:
            skv.swiftkv_attention_exact(ctx, q, k, v, kv, lut, aq, asc, layer, positions, out)
        ctx.synchronize()
        return (out.download(np.uint32, (B, 4096)), aq.download(np.uint8, (B, 128, 56)),
                asc.download(np.uint8, (B, 128)))
    finally:
        for x in (out, aq, asc):
            x.free()


def _new_rows(kv, positions, layer, seqs):
    return [kv.read(b, layer, h, positions[b], 1) for b in seqs for h in (0, 7, 31)]


@pytest.mark.parametrize("case", range(24))
def test_every_entry_on_one_workload(skv, ctx, lut4096, rope_tables, case):
    cos, sin = rope_tables
    seed = 64000 + case
    d = _draw(seed)
    rng, B, positions, cap, layers = d["rng"], d["B"], d["positions"], d["cap"], d["layers"]
    layer = int(rng.integers(0, layers))
    split = 256 * int(rng.integers(1, 17)) if rng.random() < 0.4 else 0
    shape = [None, None, (4, 64), (8, 32), (8, 64)][int(rng.integers(0, 5))]
    dist, kout = int(rng.integers(0, 2)), bool(rng.random() < 0.4)
    parts = int(rng.choice([2, 4]))
    mp = max(positions)
    _note(f"case {case}: batch {B} {'uniform' if d['uniform'] else 'ragged'}, positions up to {mp}, cap {cap}, "
          f"layer {layer} of {layers}, split {split}, shape {shape}, dist {dist}, K outliers {kout}, {parts} parts")
    kv = skv.KVCache(ctx, layers=layers, max_batch=B, max_seq_len=cap)
    bufs = []
    try:
        kv.fill_synthetic(lut4096, ntok=mp, seed=seed, layer0=layer, nlayers=1, dist=dist, k_outliers=kout)
        ctx.set_split_tokens(split)
        ctx.debug_set_step_shape(*(shape or (0, 0)))
        # q/k/v as split-K partials and as their reduction in the reference's order
        pq, pk, pv = (np.stack([np.random.default_rng(seed * 10 + 3 * i + j).standard_normal((B, 4096))
                                .astype(np.float32) for j in range(parts)]) for i in range(3))
        if kout:
            pk[:, :, ::97] *= np.float32(20.0)
        red = [O.reduce_partials(x) for x in (pq, pk, pv)]
        stride = B * 4096 + int(rng.choice([0, 64, 4096]))
        dparts = []
        for x in (pq, pk, pv):
            flat = np.zeros((parts - 1) * stride + B * 4096, np.float32)
            for p in range(parts):
                flat[p * stride:p * stride + B * 4096] = x[p].reshape(-1)
            dparts.append(ctx.to_device(flat))
        dred = [ctx.to_device(x) for x in red]
        dq17 = [ctx.to_device(O.f2q17(x)) for x in red]
        bufs = dparts + dred + dq17
        sample = sorted({0, B - 1, int(rng.integers(0, B))})

        ref = _step(skv, ctx, "f32", B, *dred, kv, lut4096, layer, positions)
        ref_rows = _new_rows(kv, positions, layer, sample)
        for entry, args, extra in (("q17", dq17, {}), ("noalloc", dred, {}),
                                   ("parts", dparts, {"parts": parts, "stride": stride})):
            try:
                got = _step(skv, ctx, entry, B, *args, kv, lut4096, layer, positions, **extra)
            except skv.SwiftKVError as e:
                splits = (mp + split) // split if split else 0
                assert entry == "noalloc" and e.code == skv.ERANGE and splits > 8, f"{entry}: {e}"
                _note(f"  the allocation-free entry refused {splits} splits per head")
                continue
            for a, b_, what in zip(got, ref, ("FP32 output", "A14 words", "E8M0 codes")):
                bad = np.argwhere(a != b_)
                assert bad.size == 0, f"{entry}: {what} differ from the f32 entry at {bad[:3].tolist()}"
            for x, y in zip(_new_rows(kv, positions, layer, sample), ref_rows):
                for u, w in zip(x, y):
                    assert (u.view(np.uint8) == w.view(np.uint8)).all(), f"{entry}: appended row differs"

        exact = mp < 4096
        ex = _step(skv, ctx, "exact", B, *dred, kv, lut4096, layer, positions) if exact else None
        qq, kq, vq = (O.f2q17(x) for x in red)
        out = ref[0].view(np.float32)
        for b in sample:
            p = positions[b]
            sc = oracle_cache_synthetic(skv, ctx, cos, sin, seed, b, layer, p, p + 1, dist=dist, k_outliers=kout)
            res = sc.step_q17(qq[b], kq[b], vq[b], p, cos[p], sin[p], fp=True, integer=exact)
            assert_rows_equal(kv, sc, b, layer, 0, p + 1)
            assert_close(out[b].reshape(H, 128), res["fp"], f"seq {b} position {p}")
            q14, e8 = O.a14(out[b].reshape(128, 32))
            assert (ref[2][b] == e8).all() and (ref[1][b] == O.pack_a14(q14)).all(), f"seq {b}: A14 rule"
            if exact:
                iref = res["int"].reshape(4096)
                diff = np.flatnonzero(ex[0][b].view(np.int32) != iref)
                assert diff.size == 0, f"integer entry, seq {b} position {p}: {diff.size} Q15.17 values differ"
                q14, e8 = O.a14_q17(iref.reshape(128, 32))
                assert (ex[2][b] == e8).all() and (ex[1][b] == O.pack_a14(q14)).all(), f"integer entry, seq {b}: A14"
    finally:
        for x in bufs:
            x.free()
        ctx.set_split_tokens(0)
        ctx.debug_set_step_shape(0, 0)
        kv.close()


@pytest.mark.parametrize("layers,layer,batch,positions_hi,cap", [
    (64, 63, 3, 300, 320),        # the most layers a cache holds, its last layer
    (1, 0, 4096, 63, 64),         # the most sequences a cache holds, one call: 16 launches, slots up to 4095
])
def test_extreme_cache_geometry(skv, ctx, lut4096, rope_tables, layers, layer, batch, positions_hi, cap):
    """The step at the cache's limits: pages addressed through every layer of a
    64-layer cache, and a 4096-sequence call whose later launches start at
    high cache slots (page offsets past 2^31 bytes).  Sampled sequences against
    the oracle: every cached and appended row bit-exact, the FP32 output
    within tolerance."""
    cos, sin = rope_tables
    seed = 65000 + batch + layers
    rng = np.random.default_rng(seed)
    positions = [int(p) for p in rng.integers(0, positions_hi + 1, batch)]
    positions[-1] = positions_hi
    _note(f"case: {layers} layers (layer {layer}), batch {batch}, positions up to {positions_hi}, cap {cap}")
    kv = skv.KVCache(ctx, layers=layers, max_batch=batch, max_seq_len=cap)
    bufs = []
    try:
        kv.fill_synthetic(lut4096, ntok=positions_hi, seed=seed, layer0=layer, nlayers=1)
        q, k, v = (np.random.default_rng(seed + i).standard_normal((batch, 4096)).astype(np.float32) for i in range(3))
        bufs = [ctx.to_device(x) for x in (q, k, v)]
        out = _step(skv, ctx, "f32", batch, *bufs, kv, lut4096, layer, positions)[0].view(np.float32)
        qq, kq, vq = O.f2q17(q), O.f2q17(k), O.f2q17(v)
        for b in sorted({0, batch // 2, batch - 1}):
            p = positions[b]
            sc = oracle_cache_synthetic(skv, ctx, cos, sin, seed, b, layer, p, p + 1)
            res = sc.step_q17(qq[b], kq[b], vq[b], p, cos[p], sin[p], fp=True)
            assert_rows_equal(kv, sc, b, layer, 0, p + 1)
            assert_close(out[b].reshape(H, 128), res["fp"], f"seq {b} position {p}")
    finally:
        for x in bufs:
            x.free()
        kv.close()


def test_long_context_entries_agree(skv, ctx, rope_tables):
    """Contexts of 20001 and 32768 tokens (4 splits of 8192 per head): the
    FP32, Q15.17, allocation-free and 4-part split-K entries give the same
    bits (outputs, A14/E8M0 words, appended rows).  The FP32 entry at these
    lengths is checked against the oracle by the long-context decode test."""
    _note("case: batch 2 at positions 32767 and 20000, cap 32768, every fast entry")
    lut = skv.RopeLut.generate(ctx, 32768)
    kv = skv.KVCache(ctx, layers=1, max_batch=2, max_seq_len=32768)
    positions = [32767, 20000]
    bufs = []
    try:
        kv.fill_synthetic(lut, ntok=32767, seed=66001, dist=skv.DIST_STUDENT_T3)
        parts = np.stack([np.random.default_rng(66002 + j).standard_normal((3, 2, 4096)).astype(np.float32)
                          for j in range(4)], axis=1)   # [tensor][part][batch][4096]
        red = [O.reduce_partials(parts[i]) for i in range(3)]
        dparts = [ctx.to_device(parts[i].reshape(-1)) for i in range(3)]
        dred = [ctx.to_device(x) for x in red]
        dq17 = [ctx.to_device(O.f2q17(x)) for x in red]
        bufs = dparts + dred + dq17
        ref = _step(skv, ctx, "f32", 2, *dred, kv, lut, 0, positions)
        ref_rows = _new_rows(kv, positions, 0, [0, 1])
        for entry, args, extra in (("q17", dq17, {}), ("noalloc", dred, {}),
                                   ("parts", dparts, {"parts": 4, "stride": 2 * 4096})):
            got = _step(skv, ctx, entry, 2, *args, kv, lut, 0, positions, **extra)
            for a, b_, what in zip(got, ref, ("FP32 output", "A14 words", "E8M0 codes")):
                assert (a == b_).all(), f"{entry}: {what} differ from the f32 entry"
            for x, y in zip(_new_rows(kv, positions, 0, [0, 1]), ref_rows):
                for u, w in zip(x, y):
                    assert (u.view(np.uint8) == w.view(np.uint8)).all(), f"{entry}: appended row differs"
        assert np.isfinite(ref[0].view(np.float32)).all()
    finally:
        for x in bufs:
            x.free()
        kv.close()
        lut.close()
