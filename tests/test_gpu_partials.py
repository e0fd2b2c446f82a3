"""GPU parity of split-K partial inputs: the step fed by the Q/K/V projection's
FP32 partial sums (swiftkv_attention_partials) and the standalone finalize
(swiftkv_convert_partials_q17), against the oracle's reduction in the linear
stage's order (int4_linear_controller.cpp:1039-1054, 1655-1667, 1100-1118).

Bar: bit-exact.  The fused step must equal the FP32 step fed with the
oracle-reduced inputs in every output bit (cache rows, FP32 output, A14/E8M0),
and its FP32 output must be within max-abs 2e-5 + rel 1e-4 of the oracle's
FP32 formula on the finalized inputs."""
import sys

import numpy as np
import pytest

import oracle as O
from gpu_cases import H, assert_close, assert_rows_equal, history, oracle_sequence, prefill
from helpers import f32_normal, splitmix64

pytestmark = pytest.mark.gpu


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lut4096(skv, ctx):
    lut = skv.RopeLut.generate(ctx, 4096)
    yield lut
    lut.close()


def cancelling_partials(seed: int, parts: int, shape) -> np.ndarray:
    """[parts][*shape] FP32 partials of mixed magnitude (2^0..2^12 times
    N(0,1)), so partial sums cancel and every FP32 add rounds at or above the
    Q15.17 resolution: a wrong order or an exact sum changes the result."""
    z = splitmix64(seed + 77, parts * int(np.prod(shape)))
    e = (z % np.uint64(13)).astype(np.int32).reshape((parts,) + tuple(shape))
    base = f32_normal(seed, (parts,) + tuple(shape))
    return np.ldexp(base, e).astype(np.float32)


def edge_partials(parts: int) -> np.ndarray:
    """Columns of hand-picked partial tuples: ties of the FP32 adds, ties of
    the Q15.17 rounding, saturation, signed zeros, subnormals, inf and NaN."""
    f = np.float32
    nan_pos = np.uint32(0x7fc00000).view(f)
    nan_neg = np.uint32(0xffc00000).view(f)
    cols = [
        [2.0 ** 13, 2.0 ** -11, 2.0 ** -11, -(2.0 ** 13)],
        [2.0 ** 13, 2.0 ** -11, -(2.0 ** 13), 2.0 ** -11],
        [2.0 ** 13 + 2.0 ** -10, 2.0 ** -11, 0.0, 0.0],
        [2.0 ** -18, 2.0 ** -19, 2.0 ** -19, 0.0],
        [1.5 * 2.0 ** -17, 0.0, 0.0, 0.0],
        [2.0 ** 14, -(2.0 ** -10), 0.0, 0.0],
        [-(2.0 ** 14), 2.0 ** -9, 0.0, 0.0],
        [3.0e38, 3.0e38, 1.0, 1.0],
        [-3.0e38, -3.0e38, 1.0, 1.0],
        [-0.0, -0.0, -0.0, -0.0],
        [1e-45, 1e-45, -1e-45, 1e-40],
        [np.inf, 1.0, 2.0, 3.0],
        [-np.inf, 1.0, 2.0, 3.0],
        [np.inf, -np.inf, 1.0, 1.0],
        [1.0, 2.0, np.inf, -np.inf],
        [nan_pos, 1.0, 1.0, 1.0],
        [nan_neg, 1.0, 1.0, 1.0],
        [1.0, nan_neg, 2.0, 3.0],
        [1.0, 2.0, 3.0, nan_neg],
        [np.inf, 1.0, nan_neg, 1.0],
    ]
    a = np.array(cols, dtype=f).T          # [4][ncols]
    return np.ascontiguousarray(a[:parts])


def _upload_parts(ctx, parts_arr: np.ndarray, stride: int):
    """Device buffer holding part p at element offset p * stride."""
    P = parts_arr.shape[0]
    n = parts_arr[0].size
    host = np.zeros((P - 1) * stride + n, np.float32)
    for p in range(P):
        host[p * stride:p * stride + n] = parts_arr[p].reshape(-1)
    return ctx.to_device(host)


@pytest.mark.parametrize("parts", [1, 2, 4])
def test_convert_partials_bit_exact(skv, ctx, parts):
    _note(f"convert_partials_q17 parts={parts}")
    rnd = cancelling_partials(4100 + parts, parts, (1 << 18,))
    edge = edge_partials(parts)
    arr = np.concatenate([edge, rnd], axis=1)
    n = arr.shape[1]
    stride = n + 37 if parts > 1 else n
    src = _upload_parts(ctx, arr, stride)
    dst = ctx.alloc(n * 4)
    ctx.convert_partials_q17(src, dst, n, parts, stride)
    ctx.synchronize()
    got = dst.download(np.int32, (n,))
    want = O.finalize_partials(arr)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (f"{bad.size} of {n} differ; first at {bad[0]}: parts {arr[:, bad[0]]}, "
                           f"got {got[bad[0]]}, want {want[bad[0]]}")
    src.free()
    dst.free()


def _two_caches(skv, ctx, lut, positions, seed, cap):
    """Two caches holding the same prefilled histories, and the oracle's copy."""
    B = len(positions)
    kvs = [skv.KVCache(ctx, layers=1, max_batch=B, max_seq_len=cap) for _ in range(2)]
    hists = []
    for b, p in enumerate(positions):
        kh, vh = history(seed + 10 * b, p)
        for kv in kvs:
            prefill(skv, ctx, kv, lut, 0, b, kh, vh)
        hists.append((kh, vh))
    return kvs, hists


def _step(skv, ctx, kv, lut, positions, dq, dk, dv, parts=None, stride=None):
    B = len(positions)
    out, aq, asc = ctx.alloc(B * 4096 * 4), ctx.alloc(B * 128 * 56), ctx.alloc(B * 128)
    if parts is None:
        skv.swiftkv_attention(ctx, dq, dk, dv, kv, lut, aq, asc, 0, positions, out)
    else:
        skv.swiftkv_attention_partials(ctx, dq, dk, dv, parts, kv, lut, aq, asc, 0, positions, out,
                                       part_stride=stride)
    ctx.synchronize()
    res = (out.download(np.float32, (B, 4096)), aq.download(np.uint8, (B, 128, 56)),
           asc.download(np.uint8, (B, 128)))
    for x in (out, aq, asc):
        x.free()
    return res


CASES = [
    # (positions, parts, extra stride, split tokens, seed)
    ([0, 1000, 4095], 4, 0, 0, 11),
    ([4095], 4, 0, 0, 12),           # eight splits of one head, in-launch merge
    ([2047, 300], 2, 64, 256, 13),   # forced small splits, padded part stride
    ([17] * 300, 4, 4096, 0, 14),    # more sequences than one launch carries
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_partials_step_equals_reduced_f32_step(skv, ctx, lut4096, rope_tables, case):
    positions, parts, extra, split, seed = CASES[case]
    B = len(positions)
    _note(f"attention_partials case {case}: batch {B} parts {parts} positions {sorted(set(positions))[:4]} "
          f"extra stride {extra} split {split}")
    cos, sin = rope_tables
    cap = max(positions) + 1
    ctx.set_split_tokens(split)
    kvs, hists = _two_caches(skv, ctx, lut4096, positions, 900 + seed, cap)
    stride = B * 4096 + extra
    pq, pk, pv = (cancelling_partials(seed * 10 + i, parts, (B, 4096)) for i in range(3))
    rq, rk, rv = (O.reduce_partials(x) for x in (pq, pk, pv))
    d = [_upload_parts(ctx, x, stride) for x in (pq, pk, pv)]
    got = _step(skv, ctx, kvs[0], lut4096, positions, *d, parts=parts, stride=stride)
    for x in d:
        x.free()
    d = [ctx.to_device(x) for x in (rq, rk, rv)]
    ref = _step(skv, ctx, kvs[1], lut4096, positions, *d)
    for x in d:
        x.free()
    assert (got[0].view(np.uint32) == ref[0].view(np.uint32)).all(), "FP32 output bits differ"
    assert (got[1] == ref[1]).all() and (got[2] == ref[2]).all(), "A14/E8M0 differ"
    # the appended rows and the output against the oracle on the finalized inputs
    fq, fk, fv = (O.finalize_partials(x) for x in (pq, pk, pv))
    for b, p in list(enumerate(positions))[:4]:
        kh, vh = hists[b]
        sc = oracle_sequence(cos, sin, kh, vh, p + 1)
        res = sc.step_q17(fq[b], fk[b], fv[b], p, cos[p], sin[p], fp=True)
        assert_rows_equal(kvs[0], sc, b, 0, 0, p + 1)
        assert_close(got[0][b].reshape(H, 128), res["fp"], f"seq {b} position {p}")
    ctx.set_split_tokens(0)
    for kv in kvs:
        kv.close()


def test_partials_host_memory_io(skv, ctx, lut4096):
    positions = [600, 95]
    B, parts = len(positions), 4
    _note("attention_partials in host-memory I/O mode")
    kvs, _ = _two_caches(skv, ctx, lut4096, positions, 950, 640)
    stride = B * 4096 + 8
    host = []
    for i in range(3):
        arr = cancelling_partials(700 + i, parts, (B, 4096))
        flat = np.zeros((parts - 1) * stride + B * 4096, np.float32)
        for p in range(parts):
            flat[p * stride:p * stride + B * 4096] = arr[p].reshape(-1)
        host.append(flat)
    d = [ctx.to_device(x) for x in host]
    dev = _step(skv, ctx, kvs[0], lut4096, positions, *d, parts=parts, stride=stride)
    for x in d:
        x.free()
    out = np.zeros((B, 4096), np.float32)
    aq = np.zeros((B, 128, 56), np.uint8)
    asc = np.zeros((B, 128), np.uint8)
    ctx.set_host_io(True)
    try:
        skv.swiftkv_attention_partials(ctx, *host, parts, kvs[1], lut4096, aq, asc, 0, positions, out,
                                       part_stride=stride)
    finally:
        ctx.set_host_io(False)
    assert (out.view(np.uint32) == dev[0].view(np.uint32)).all()
    assert (aq == dev[1]).all() and (asc == dev[2]).all()
    for kv in kvs:
        kv.close()


def test_partials_error_codes(skv, ctx, lut4096):
    _note("attention_partials / convert_partials_q17 argument checks")
    kv = skv.KVCache(ctx, layers=1, max_batch=2, max_seq_len=64)
    buf = ctx.alloc(4 * 2 * 4096 * 4)
    out = ctx.alloc(2 * 4096 * 4)
    for parts, stride in [(3, 8192), (0, 8192), (4, 8191), (2, -1), (4, (1 << 40) + 1)]:
        with pytest.raises(skv.SwiftKVError) as ei:
            skv.swiftkv_attention_partials(ctx, buf, buf, buf, parts, kv, lut4096, None, None, 0, [5, 6], out,
                                           part_stride=stride)
        assert ei.value.code == -1, (parts, stride)
    with pytest.raises(skv.SwiftKVError):
        ctx.convert_partials_q17(buf, out, 100, 3, 100)
    with pytest.raises(skv.SwiftKVError):
        ctx.convert_partials_q17(buf, out, 100, 2, 99)
    with pytest.raises(skv.SwiftKVError):
        ctx.convert_partials_q17(buf, out, 100, 4, (1 << 40) + 1)
    buf.free()
    out.free()
    kv.close()


def test_partials_graph_replay_matches_eager(skv, ctx, lut4096):
    """The partial-input step recorded into a HIP graph (batch 1, eight splits
    merged inside the launch) and replayed three times, with eager work and
    synchronizations between the replays: every replay equals the eager call
    bit for bit."""
    _note("attention_partials: HIP graph replay vs eager")
    positions = [2000]
    kv = skv.KVCache(ctx, layers=1, max_batch=1, max_seq_len=2048)
    kh, vh = history(960, 2000)
    prefill(skv, ctx, kv, lut4096, 0, 0, kh, vh)
    stride = 4096 + 32
    d = [_upload_parts(ctx, cancelling_partials(970 + i, 4, (1, 4096)), stride) for i in range(3)]
    out, aq, asc = ctx.alloc(4096 * 4), ctx.alloc(128 * 56), ctx.alloc(128)

    def step():
        skv.swiftkv_attention_partials(ctx, *d, 4, kv, lut4096, aq, asc, 0, positions, out, part_stride=stride)

    def snapshot():
        ctx.synchronize()
        return (out.download(np.float32, (4096,)), aq.download(np.uint8, (128, 56)), asc.download(np.uint8, (128,)))

    step()
    eager = snapshot()
    ctx.capture_begin()
    step()
    g = ctx.capture_end()
    scratch = ctx.alloc(4096 * 4)
    for rep in range(3):
        out.zero()
        g.launch()
        ctx.convert_partials_q17(d[0], scratch, 4096, 4, stride)   # eager work between replays
        got = snapshot()
        assert (got[0].view(np.uint32) == eager[0].view(np.uint32)).all(), f"replay {rep}: output differs"
        assert (got[1] == eager[1]).all() and (got[2] == eager[2]).all(), f"replay {rep}: A14/E8M0 differ"
    g.close()
    for x in d + [out, aq, asc, scratch]:
        x.free()
    kv.close()
