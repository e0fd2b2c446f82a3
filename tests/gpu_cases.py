"""Scenario builder shared by the GPU tests: the same seeded inputs go through
the HIP path (C ABI) and the oracle."""
import numpy as np

import oracle as O
from helpers import f32_normal, splitmix64

H = 32


def student_t3(seed: int, shape) -> np.ndarray:
    """Student-t(nu=3) scaled to unit variance: N / sqrt(chi2_3 / 3) / sqrt(3)."""
    n = f32_normal(seed, shape).astype(np.float64)
    c = sum(f32_normal(seed + 7919 * (i + 1), shape).astype(np.float64) ** 2 for i in range(3))
    return (n / np.sqrt(c / 3.0) / np.sqrt(3.0)).astype(np.float32)


def wide_values(seed: int, shape) -> np.ndarray:
    """N(0,1) rows, each scaled by 2^e with e uniform in [-8, 15], and 2% of the entries set to +-20000 (past
    the Q15.17 range, so they saturate): G32 shifts from small to 25, including the code 64 at shift 25 whose
    dequantized value wraps."""
    x = f32_normal(seed, shape).astype(np.float64)
    rows, total = shape[0], int(np.prod(shape))
    z = splitmix64(seed + 3, rows + total)
    e = (z[:rows] % np.uint64(24)).astype(np.int64) - 8
    x *= np.ldexp(1.0, e).reshape((rows,) + (1,) * (len(shape) - 1))
    zz = z[rows:].reshape(shape)
    sign = np.where((zz >> np.uint64(32)) & np.uint64(1), 1.0, -1.0)
    return np.where(zz % np.uint64(50) == 0, 20000.0 * sign, x).astype(np.float32)


RISING_CHANNELS = np.array([h * 128 + c for h in range(H) for c in range(120, 128)])


def rising_keys(tokens) -> np.ndarray:
    """Keys on the slowest-rotating channel pairs (j = 60..63) of every head,
    growing with the token index: against a query on the same channels
    (rising_query) the scores rise, so most tokens set a new running maximum."""
    t = np.asarray(tokens, dtype=np.float64)
    k = np.zeros((t.size, 4096), np.float32)
    k[:, RISING_CHANNELS] = (0.25 * (1.0 + t / 64.0))[:, None].astype(np.float32)
    return k


def rising_query(batch: int) -> np.ndarray:
    q = np.zeros((batch, 4096), np.float32)
    q[:, RISING_CHANNELS] = 1.0
    return q


def outlier_channels(seed: int, count: int = 41) -> np.ndarray:
    z = splitmix64(seed, 4 * count)
    return np.unique((z % np.uint64(4096)).astype(np.int64))[:count]


def history(seed: int, n: int, dist: str = "normal", outliers=None):
    if dist == "t3":
        k, v = student_t3(seed, (n, 4096)), student_t3(seed + 1, (n, 4096))
    elif dist == "wide":
        k, v = f32_normal(seed, (n, 4096)), wide_values(seed + 1, (n, 4096))
    elif dist == "rising":
        k, v = rising_keys(np.arange(n)), f32_normal(seed + 1, (n, 4096))
    else:
        k, v = f32_normal(seed, (n, 4096)), f32_normal(seed + 1, (n, 4096))
    if outliers is not None:
        k[:, outliers] *= np.float32(20.0)
    return k, v


def prefill(skv, ctx, kv, lut, layer, seq, k_hist, v_hist, chunk=1024):
    """Bulk-append a FP32 history [n][4096] at positions [0, n)."""
    n = k_hist.shape[0]
    for t0 in range(0, n, chunk):
        t1 = min(n, t0 + chunk)
        dk = ctx.to_device(k_hist[t0:t1])
        dv = ctx.to_device(v_hist[t0:t1])
        skv.swiftkv_append_tokens(ctx, dk, dv, kv, lut, layer, seq, t0, t1 - t0)
        ctx.synchronize()
        dk.free()
        dv.free()


def run_step(skv, ctx, kv, lut, layer, positions, q, k, v, q17=False, a14=True):
    """One step through the C ABI; returns (out [B,4096], act_q [B,128,56], act_scale [B,128])."""
    B = len(positions)
    dq, dk, dv = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
    out = ctx.alloc(B * 4096 * 4)
    aq = ctx.alloc(B * 128 * 56) if a14 else None
    asc = ctx.alloc(B * 128) if a14 else None
    skv.swiftkv_attention(ctx, dq, dk, dv, kv, lut, aq, asc, layer, positions, out, q17=q17)
    ctx.synchronize()
    res = (out.download(np.float32, (B, 4096)),
           aq.download(np.uint8, (B, 128, 56)) if a14 else None,
           asc.download(np.uint8, (B, 128)) if a14 else None)
    for b in (dq, dk, dv, out, aq, asc):
        if b is not None:
            b.free()
    return res


def oracle_sequence(cos, sin, k_hist, v_hist, cap):
    sc = O.SequenceCache(H, cap)
    if k_hist.shape[0]:
        sc.fill_q17(O.f2q17(k_hist), O.f2q17(v_hist), 0, cos, sin)
    return sc


def assert_rows_equal(kv, sc, seq, layer, tok0, n, heads=range(H)):
    for h in heads:
        kc, vc, ks, vs = kv.read(seq, layer, h, tok0, n)
        assert (kc == sc.kc[h, tok0:tok0 + n]).all(), f"seq {seq} head {h}: K codes differ"
        assert (vc == sc.vc[h, tok0:tok0 + n]).all(), f"seq {seq} head {h}: V codes differ"
        assert (ks.view(np.uint32) == O.shift_scale_bits(sc.ks[h, tok0:tok0 + n])).all(), f"seq {seq} head {h}: K scales"
        assert (vs.view(np.uint32) == O.shift_scale_bits(sc.vs[h, tok0:tok0 + n])).all(), f"seq {seq} head {h}: V scales"


RTOL, ATOL = 1e-4, 2e-5   # tolerance vs the FP32 formula (double-precision oracle)


def assert_close(got, ref, what=""):
    err = np.abs(got.astype(np.float64) - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), (f"{what}: {int(bad.sum())} values outside atol {ATOL} + rtol {RTOL}; "
                           f"max abs err {err.max():.3g}")
    return float(err.max())


def synthetic_rows(ctx, seed, slot, layer, t0, n, dist=0, k_outliers=False):
    """FP32 K/V rows [t0, t0+n) that the device cache filler used for (slot,
    layer): streams 2*(64*slot + layer) (K) and that + 1 (V)."""
    sid = 2 * (slot * 64 + layer)
    buf = ctx.alloc(n * 4096 * 4)
    ctx.fill_synthetic(buf, n * 4096, seed, sid, dist, k_outliers, first=t0 * 4096)
    k = buf.download(np.float32, (n, 4096))
    ctx.fill_synthetic(buf, n * 4096, seed, sid + 1, dist, False, first=t0 * 4096)
    v = buf.download(np.float32, (n, 4096))
    buf.free()
    return k, v


def oracle_cache_synthetic(skv, ctx, cos, sin, seed, slot, layer, ntok, cap, dist=0, k_outliers=False, chunk=4096):
    """The oracle's cache of (slot, layer) rebuilt from the filler's FP32 rows
    [0, ntok) through the append rule."""
    sc = O.SequenceCache(H, cap)
    for t0 in range(0, ntok, chunk):
        n = min(chunk, ntok - t0)
        k, v = synthetic_rows(ctx, seed, slot, layer, t0, n, dist, k_outliers)
        sc.fill_q17(O.f2q17(k), O.f2q17(v), t0, cos, sin)
    return sc
