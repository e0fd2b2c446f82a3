"""GPU parity of the integer-compatibility step (swiftkv_attention_exact),
bit for bit:
  - the reference's own known-answer test (tb_attention_pe0_kv_rtl.cpp:79-110):
    PE0's 32 A14 words and E8M0 codes hash to the two published values;
  - the reference emulator's decode outputs (golden.json, made from the
    emulator's attention stage): A14 codes and scales of every step, chained;
  - the oracle's integer recurrence on FP32 histories with heavy tails,
    outlier channels and positions on both sides of the kernel's 256-token
    chunk boundaries, and at position 4095, the reference's last -- normalized
    Q15.17 state, A14 words and E8M0 codes;
  - the reference's bound: positions at or past 4096 are refused.

The kernel runs one of three launch shapes by batch size: four workgroups per
(sequence, head) for batches 1-2, two for batches 3-8, one from batch 9.  The
large-query, rescale-chain and saturation cases run in each shape."""
import sys

import numpy as np
import pytest

import oracle as O
from gpu_cases import (H, assert_rows_equal, history, oracle_cache_synthetic, oracle_sequence, outlier_channels,
                       prefill, rising_keys, rising_query)
from helpers import f32_normal, kat_vector

pytestmark = pytest.mark.gpu

_FNV_OFFSET, _FNV_PRIME, _M64 = 1469598103934665603, 1099511628211, (1 << 64) - 1


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lut4096(skv, ctx):
    lut = skv.RopeLut.generate(ctx, 4096)
    yield lut
    lut.close()


def exact_step(skv, ctx, kv, lut, layer, positions, q, k, v, q17):
    """One integer-compatibility step; returns (out_q17 [B,4096] int32, act_q [B,128,56], act_scale [B,128])."""
    B = len(positions)
    dq, dk, dv = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
    out = ctx.alloc(B * 4096 * 4)
    aq = ctx.alloc(B * 128 * 56)
    asc = ctx.alloc(B * 128)
    skv.swiftkv_attention_exact(ctx, dq, dk, dv, kv, lut, aq, asc, layer, positions, out, q17=q17)
    ctx.synchronize()
    res = (out.download(np.int32, (B, 4096)), aq.download(np.uint8, (B, 128, 56)),
           asc.download(np.uint8, (B, 128)))
    for buf in (dq, dk, dv, out, aq, asc):
        buf.free()
    return res


def kat_hash(words: np.ndarray, codes: np.ndarray) -> int:
    """FNV-1a style hash of 32 groups: 7 little-endian u64 of each 56-byte word, then its code
    (tb_attention_pe0_kv_rtl.cpp:33-58)."""
    h = _FNV_OFFSET
    for g in range(32):
        for c in range(7):
            h ^= int.from_bytes(words[g, 8 * c:8 * c + 8].tobytes(), "little")
            h = (h * _FNV_PRIME) & _M64
        h ^= int(codes[g])
        h = (h * _FNV_PRIME) & _M64
    return h


def test_exact_reproduces_reference_kat(skv, ctx, lut4096, golden):
    _note("case: reference KAT, PE0 heads 0..7, positions 0 and 1")
    kv = skv.KVCache(ctx, layers=1, max_batch=1, max_seq_len=64)
    kv.zero()
    for pos, seeds in enumerate(golden["kat"]["seeds"]):
        q, k, v = (np.zeros((1, 4096), np.int32) for _ in range(3))
        q[0, :1024], k[0, :1024], v[0, :1024] = (kat_vector(s) for s in seeds)
        _, aq, asc = exact_step(skv, ctx, kv, lut4096, 0, [pos], q, k, v, q17=True)
        assert hex(kat_hash(aq[0, :32], asc[0, :32])) == golden["kat"][f"pos{pos}"], f"position {pos}"
    kv.close()


@pytest.mark.parametrize("case", [0, 1, 2])
def test_exact_matches_reference_decode(skv, ctx, lut4096, golden, case):
    from golden.make_golden import fnv_chain, step_inputs
    g = golden["decode"][case]
    last = g["last_position"]
    _note(f"case: reference decode chain {case}, seed {g['seed']}, positions 0..{last}, span {g['span_bits']}")
    kv = skv.KVCache(ctx, layers=1, max_batch=1, max_seq_len=last + 1)
    h = _FNV_OFFSET
    for pos in range(last + 1):
        q, k, v = step_inputs(g["seed"], pos, g["span_bits"])
        _, aq, asc = exact_step(skv, ctx, kv, lut4096, 0, [pos], q[None], k[None], v[None], q17=True)
        codes = skv.unpack_a14(aq[0]).reshape(4096).astype(np.int16)
        scale = np.where(asc[0] == 0, 0.0, np.ldexp(1.0, asc[0].astype(np.int32) - 140)).astype(np.float32)
        h = fnv_chain(h, codes.tobytes() + scale.tobytes())
    assert (codes == np.array(g["a14_last"], np.int16)).all()
    assert (scale == np.array(g["scale_last"], np.float32)).all()
    assert hex(h) == g["chain_hash"]
    kv.close()


@pytest.mark.parametrize("positions,dist,q17,big_query", [
    ([0, 1, 255, 256], "normal", False, False),
    ([257, 511, 512, 1030], "t3", False, False),
    ([1500, 77], "t3", True, False),
    ([300, 700], "wide", False, False),
    ([300, 700, 5, 257, 256, 511, 1, 0, 64], "wide", False, False),
    ([300, 1030, 1], "normal", False, True),   # two workgroups per head
    ([700], "t3", False, True),                # four workgroups per head
    ([300, 1030, 1, 700, 5, 257, 256, 511, 64], "normal", False, True),   # one workgroup per head
])
def test_exact_matches_oracle_integer_recurrence(skv, ctx, lut4096, rope_tables, positions, dist, q17, big_query):
    """big_query: queries past 64.0 in some heads (and saturated channels in
    one), so the query's upper byte limbs are nonzero and the score dot
    products take all five limbs; the other heads keep the three-limb form."""
    _note(f"case: exact vs oracle, positions {positions}, {dist}, q17={q17}, big query={big_query}")
    cos, sin = rope_tables
    seed = 500 + positions[0]
    outl = outlier_channels(seed)
    B = len(positions)
    kv = skv.KVCache(ctx, layers=2, max_batch=B, max_seq_len=max(positions) + 1)
    layer = 1
    scs = []
    for b, p in enumerate(positions):
        kh, vh = history(seed + 10 * b, p, dist, outl)
        prefill(skv, ctx, kv, lut4096, layer, b, kh, vh)
        scs.append(oracle_sequence(cos, sin, kh, vh, p + 1))
    q = f32_normal(seed + 1000, (B, 4096))
    k = f32_normal(seed + 1001, (B, 4096))
    v = f32_normal(seed + 1002, (B, 4096))
    k[:, outl] *= np.float32(20.0)
    if big_query:
        q[:, 0:16 * 128] *= np.float32(300.0)                        # heads 0-15 beyond 64.0
        q[:, 5 * 128:5 * 128 + 8] = np.float32([3e4, -3e4, 1e9, -1e9, 2e4, -2e4, 17000.0, -16384.0])
    qq, kq, vq = O.f2q17(q), O.f2q17(k), O.f2q17(v)
    if big_query:
        assert (np.abs(qq[:, :16 * 128].astype(np.int64)) >= 1 << 23).any() and (qq == np.iinfo(np.int32).min).any()
    if q17:
        out, aq, asc = exact_step(skv, ctx, kv, lut4096, layer, positions, qq, kq, vq, q17=True)
    else:
        out, aq, asc = exact_step(skv, ctx, kv, lut4096, layer, positions, q, k, v, q17=False)
    for b, p in enumerate(positions):
        res = scs[b].step_q17(qq[b], kq[b], vq[b], p, cos[p], sin[p], fp=False, integer=True)
        assert_rows_equal(kv, scs[b], b, layer, 0, p + 1)
        ref = res["int"].reshape(4096)
        diff = np.flatnonzero(out[b] != ref)
        assert diff.size == 0, f"seq {b} position {p}: {diff.size} Q15.17 values differ (first {diff[:4]})"
        q14, e8 = O.a14_q17(ref.reshape(128, 32))
        assert (asc[b] == e8).all(), f"seq {b}: E8M0 codes"
        assert (aq[b] == O.pack_a14(q14)).all(), f"seq {b}: A14 words"
    kv.close()


@pytest.mark.parametrize("batch", [1, 3, 9])   # four, two and one workgroups per head
def test_exact_every_token_a_new_maximum(skv, ctx, lut4096, rope_tables, batch):
    """Keys that grow along the query's direction make most tokens a new
    running maximum (578 of 700: INT8 quantization makes some neighbours tie,
    and a tie is no new maximum), so each chunk's ordered part holds almost
    all of it and takes the rescale branch token after token.  Query and keys
    live on the slowest-rotating channel pairs (j = 60..63), so the rotation
    cannot undo the growth."""
    _note(f"case: exact, rising keys, batch {batch}, position 700")
    cos, sin = rope_tables
    p = 700
    kv = skv.KVCache(ctx, layers=1, max_batch=batch, max_seq_len=p + 1)
    scs = []
    for b in range(batch):
        kh, vh = history(8100 + 10 * b, p, "rising")
        prefill(skv, ctx, kv, lut4096, 0, b, kh, vh)
        scs.append(oracle_sequence(cos, sin, kh, vh, p + 1))
    q, k = rising_query(batch), rising_keys([p] * batch)
    v = f32_normal(8200, (batch, 4096))
    qq, kq, vq = O.f2q17(q), O.f2q17(k), O.f2q17(v)
    out, aq, asc = exact_step(skv, ctx, kv, lut4096, 0, [p] * batch, qq, kq, vq, q17=True)
    for b in range(batch):
        res = scs[b].step_q17(qq[b], kq[b], vq[b], p, cos[p], sin[p], fp=False, integer=True)
        ref = res["int"].reshape(4096)
        diff = np.flatnonzero(out[b] != ref)
        assert diff.size == 0, f"seq {b}: {diff.size} Q15.17 values differ (first {diff[:4]})"
        q14, e8 = O.a14_q17(ref.reshape(128, 32))
        assert (asc[b] == e8).all() and (aq[b] == O.pack_a14(q14)).all(), f"seq {b}: A14"
    kv.close()


def saturating_history(n, mag, lead, flip):
    """Keys zero, so every score is 0 and every coefficient exp(0) = 1.0 (no
    token after the first is a new maximum), and V = +-mag on alternate
    channels: -sign before token `lead`, +sign up to `flip`, -sign after, so
    Y (Q15.17, 2^31 = 16384.0) climbs from -lead mag to either end of the
    int32 range, stays there, and comes back.  mag 31.0 quantizes to shift 15
    and mag 40.0 to shift 16."""
    t = np.arange(n)
    run = np.where((t >= lead) & (t < flip), 1.0, -1.0)
    sign = np.where(np.arange(4096) % 2 == 0, 1.0, -1.0)
    return np.zeros((n, 4096), np.float32), (mag * run[:, None] * sign[None, :]).astype(np.float32)


def saturation_cases(mag, batch):
    """(position, lead, flip) per sequence: Y first saturates after 16384 / mag
    tokens (lead 0), or at token 968, 200 tokens into its 256-token chunk (the
    composed part there), with lead = (968 - 16384 / mag) / 2."""
    late = int(round((968 - 16384 / mag) / 2))
    cases = [(1300, 0, 1000), (1250, late, 1100), (1100, 0, 900)]
    return [cases[b % len(cases)] for b in range(batch)]


# batch 1: four workgroups per head; 3: two; 9: one
@pytest.mark.parametrize("mag,batch", [(31.0, 1), (31.0, 3), (31.0, 9), (40.0, 1), (40.0, 3), (40.0, 9)])
def test_exact_y_saturates(skv, ctx, lut4096, rope_tables, mag, batch):
    """Y reaches INT32_MAX and INT32_MIN (alternate channels) early in a chunk
    (its ordered part) or late in one (its composed part), stays, and comes
    back: the saturating adds, the batch sums taken at once away from the
    ends of the range, and the composed clamp-add maps, against the oracle's
    integer recurrence bit for bit.  Shift 15 takes the fused-multiply-add
    term form, shift 16 the rint form."""
    _note(f"case: exact, saturating Y, |V| = {mag}, batch {batch}")
    cos, sin = rope_tables
    cases = saturation_cases(mag, batch)
    positions = [c[0] for c in cases]
    kv = skv.KVCache(ctx, layers=1, max_batch=batch, max_seq_len=max(positions) + 1)
    scs = []
    for b, (p, lead, flip) in enumerate(cases):
        kh, vh = saturating_history(p, mag, lead, flip)
        prefill(skv, ctx, kv, lut4096, 0, b, kh, vh)
        scs.append(oracle_sequence(cos, sin, kh, vh, p + 1))
        assert (scs[-1].vs[:, :p] == (15 if mag < 32 else 16)).all()
    q = f32_normal(9100, (batch, 4096))
    k = np.zeros((batch, 4096), np.float32)
    v = (-mag * np.where(np.arange(4096) % 2 == 0, 1.0, -1.0)).astype(np.float32)[None].repeat(batch, 0)
    qq, kq, vq = O.f2q17(q), O.f2q17(k), O.f2q17(v)
    out, aq, asc = exact_step(skv, ctx, kv, lut4096, 0, positions, qq, kq, vq, q17=True)
    for b, p in enumerate(positions):
        res = scs[b].step_q17(qq[b], kq[b], vq[b], p, cos[p], sin[p], fp=True, integer=True)
        ref = res["int"].reshape(4096)
        # saturation changed the result: the unsaturated mean is far away
        assert np.abs(ref * 2.0 ** -17 - res["fp"].reshape(4096)).min() > 1.0
        diff = np.flatnonzero(out[b] != ref)
        assert diff.size == 0, f"seq {b} position {p}: {diff.size} Q15.17 values differ (first {diff[:4]})"
        q14, e8 = O.a14_q17(ref.reshape(128, 32))
        assert (asc[b] == e8).all() and (aq[b] == O.pack_a14(q14)).all(), f"seq {b}: A14"
    kv.close()


@pytest.mark.parametrize("seed,batch", [(99001, 1), (99004, 3), (99009, 9)])
def test_exact_y_saturates_mixed_shifts(skv, ctx, lut4096, rope_tables, seed, batch):
    """Y saturates while the V shifts change from token to token (magnitudes
    15 to 130 per token and 1024-channel block: shifts 14 to 18), so batches
    and composed runs switch between the fused-multiply-add, rint and integer
    term forms around the saturation points; keys zero except a few tokens
    that set new maxima.  Bit for bit against the oracle's recurrence."""
    _note(f"case: exact, saturating Y with mixed shifts, seed {seed}, batch {batch}")
    cos, sin = rope_tables
    rng = np.random.default_rng(seed)
    positions = [int(p) for p in rng.integers(500, 1400, batch)]
    kv = skv.KVCache(ctx, layers=1, max_batch=batch, max_seq_len=max(positions) + 1)
    scs = []
    chan_sign = np.where(np.arange(4096) % 2 == 0, 1.0, -1.0)
    for b, p in enumerate(positions):
        k = np.zeros((p, 4096), np.float32)
        k[rng.integers(0, p, 6), :] = f32_normal(seed + 10 * b, (6, 4096)) * np.float32(0.05)
        mags = np.repeat(rng.choice([15.0, 31.0, 40.0, 60.0, 100.0, 130.0], size=(p, 4)), 1024, axis=1)
        sign_t = np.where((np.arange(p) // int(rng.integers(200, 700))) % 2 == 0, 1.0, -1.0)
        v = (mags * sign_t[:, None] * chan_sign[None, :]).astype(np.float32)
        prefill(skv, ctx, kv, lut4096, 0, b, k, v)
        scs.append(oracle_sequence(cos, sin, k, v, p + 1))
        shifts = set(np.unique(scs[-1].vs[:, :p]).tolist())
        assert {15, 16, 17}.issubset(shifts), shifts
    q = f32_normal(seed + 1000, (batch, 4096))
    k = np.zeros((batch, 4096), np.float32)
    v = (31.0 * chan_sign).astype(np.float32)[None].repeat(batch, 0)
    qq, kq, vq = O.f2q17(q), O.f2q17(k), O.f2q17(v)
    out, aq, asc = exact_step(skv, ctx, kv, lut4096, 0, positions, qq, kq, vq, q17=True)
    saturated = 0
    for b, p in enumerate(positions):
        res = scs[b].step_q17(qq[b], kq[b], vq[b], p, cos[p], sin[p], fp=True, integer=True)
        ref = res["int"].reshape(4096)
        saturated += int(np.abs(ref * 2.0 ** -17 - res["fp"].reshape(4096)).max() > 1.0)
        diff = np.flatnonzero(out[b] != ref)
        assert diff.size == 0, f"seq {b} position {p}: {diff.size} Q15.17 values differ (first {diff[:4]})"
        q14, e8 = O.a14_q17(ref.reshape(128, 32))
        assert (asc[b] == e8).all() and (aq[b] == O.pack_a14(q14)).all(), f"seq {b}: A14"
    assert saturated > 0
    kv.close()


def test_exact_batch_over_one_launch(skv, ctx, lut4096, rope_tables):
    """The exact entry over 260 sequences (two launches), against the oracle's
    integer recurrence on a sample of sequences from both launches."""
    _note("case: exact, batch 260, positions 0..40")
    cos, sin = rope_tables
    positions = [int(p) for p in np.random.default_rng(260).integers(0, 41, 260)]
    B = len(positions)
    kv = skv.KVCache(ctx, layers=1, max_batch=B, max_seq_len=64)
    hist = [history(7000 + 10 * b, p) for b, p in enumerate(positions)]
    for b, (kh, vh) in enumerate(hist):
        prefill(skv, ctx, kv, lut4096, 0, b, kh, vh)
    q, k, v = (O.f2q17(f32_normal(7001 + i, (B, 4096))) for i in range(3))
    out, aq, asc = exact_step(skv, ctx, kv, lut4096, 0, positions, q, k, v, q17=True)
    for b in (0, 1, 128, 255, 256, 257, 259):
        p = positions[b]
        sc = oracle_sequence(cos, sin, hist[b][0], hist[b][1], p + 1)
        res = sc.step_q17(q[b], k[b], v[b], p, cos[p], sin[p], fp=False, integer=True)
        assert (out[b] == res["int"].reshape(4096)).all(), f"seq {b} position {p}"
        q14, e8 = O.a14_q17(res["int"].reshape(128, 32))
        assert (asc[b] == e8).all() and (aq[b] == O.pack_a14(q14)).all(), f"seq {b}: A14"
    kv.close()


@pytest.mark.parametrize("batch,dist,outliers,q17", [(1, 0, True, False), (4, 1, False, True), (12, 0, False, False)],
                         ids=["batch1_four_workgroups", "batch4_two_workgroups_t3", "batch12_one_workgroup"])
def test_exact_position4095_matches_oracle(skv, ctx, lut4096, rope_tables, batch, dist, outliers, q17):
    """The integer-compatibility entry at the reference's last position, 4095
    (16 chunks of 256 tokens per head), in each launch shape: four workgroups
    per head (batch 1, K with 1% of channels x20), two (batch 4, Student-t(3),
    Q15.17 inputs) and one (batch 12).  The device fills the cache from
    synthetic streams through the append rule; the oracle rebuilds two sampled
    sequences from the same streams and runs the integer recurrence over all
    32 heads: every cached row, the appended row, the Q15.17 state, the A14
    words and the E8M0 codes bit for bit."""
    cos, sin = rope_tables
    p = 4095
    seed = 4700 + batch
    _note(f"case: exact at position {p}, batch {batch}, dist {dist}, K outliers {outliers}, q17={q17}")
    kv = skv.KVCache(ctx, layers=1, max_batch=batch, max_seq_len=p + 1)
    kv.fill_synthetic(lut4096, ntok=p, seed=seed, dist=dist, k_outliers=outliers)
    host = []
    for i in range(3):
        buf = ctx.alloc(batch * 4096 * 4)
        ctx.fill_synthetic(buf, batch * 4096, seed + 1, 9300 + i, dist, outliers and i == 1)
        host.append(buf.download(np.float32, (batch, 4096)))
        buf.free()
    q, k, v = host
    qq, kq, vq = O.f2q17(q), O.f2q17(k), O.f2q17(v)
    out, aq, asc = exact_step(skv, ctx, kv, lut4096, 0, [p] * batch, *((qq, kq, vq) if q17 else (q, k, v)), q17=q17)
    for b in sorted({0, batch - 1}):
        _note(f"  oracle check of slot {b}")
        sc = oracle_cache_synthetic(skv, ctx, cos, sin, seed, b, 0, p, p + 1, dist=dist, k_outliers=outliers)
        res = sc.step_q17(qq[b], kq[b], vq[b], p, cos[p], sin[p], fp=False, integer=True)
        assert_rows_equal(kv, sc, b, 0, 0, p + 1)
        ref = res["int"].reshape(4096)
        diff = np.flatnonzero(out[b] != ref)
        assert diff.size == 0, f"seq {b}: {diff.size} Q15.17 values differ (first {diff[:4]})"
        q14, e8 = O.a14_q17(ref.reshape(128, 32))
        assert (asc[b] == e8).all(), f"seq {b}: E8M0 codes"
        assert (aq[b] == O.pack_a14(q14)).all(), f"seq {b}: A14 words"
    kv.close()


def test_exact_refuses_positions_past_the_reference_bound(skv, ctx):
    """The integer-compatibility entry keeps the reference's bound (position
    ap_uint<12>, SWIFTKV_MAX_SEQ_LEN = 4096): a call with any position at or
    past 4096 returns SWIFTKV_ERANGE and enqueues nothing -- the output and
    activation buffers keep their bytes and no row is appended, not even for a
    sequence whose position is in range -- on a cache and RoPE table that hold
    those positions, where the FP32 step accepts them; in host-memory I/O mode
    too.  Position 4095 is accepted."""
    _note("case: exact entry refuses positions >= 4096")
    n = 4160
    lut = skv.RopeLut.generate(ctx, n)
    kv = skv.KVCache(ctx, layers=1, max_batch=2, max_seq_len=n)
    kv.zero()
    q, k, v = (f32_normal(4400 + i, (2, 4096)) for i in range(3))
    dq, dk, dv = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
    sentinel = [np.full(2 * 4096, 0x5A5A5A5A, np.uint32).view(np.int32), np.full(2 * 128 * 56, 0x5A, np.uint8),
                np.full(2 * 128, 0x5A, np.uint8)]
    out, aq, asc = (ctx.to_device(x) for x in sentinel)
    for positions in ([100, 4096], [4096, 4096], [3, 4100], [n - 1, n - 1]):
        with pytest.raises(skv.SwiftKVError) as ei:
            skv.swiftkv_attention_exact(ctx, dq, dk, dv, kv, lut, aq, asc, 0, positions, out)
        assert ei.value.code == skv.ERANGE and "4096" in str(ei.value), str(ei.value)
    hout = sentinel[0].copy()
    ctx.set_host_io(True)
    try:
        with pytest.raises(skv.SwiftKVError) as ei:
            skv.swiftkv_attention_exact(ctx, q, k, v, kv, lut, None, None, 0, [4096, 7], hout)
        assert ei.value.code == skv.ERANGE
    finally:
        ctx.set_host_io(False)
    ctx.synchronize()
    assert (hout == sentinel[0]).all()
    assert (out.download(np.int32, (2 * 4096,)) == sentinel[0]).all()
    assert (aq.download(np.uint8, (2 * 128 * 56,)) == sentinel[1]).all()
    assert (asc.download(np.uint8, (2 * 128,)) == sentinel[2]).all()
    for seq in (0, 1):
        for h in range(H):
            kc, vc, ks, vs = kv.read(seq, 0, h, 0, n)
            assert not kc.any() and not vc.any() and not ks.any() and not vs.any(), f"seq {seq} head {h}"
    # the bound is the entry's own: the FP32 step accepts the same positions
    fout = ctx.alloc(2 * 4096 * 4)
    skv.swiftkv_attention(ctx, dq, dk, dv, kv, lut, None, None, 0, [4096, n - 1], fout)
    ctx.synchronize()
    assert kv.read(0, 0, 0, 4096, 1)[0].any() and kv.read(1, 0, 0, n - 1, 1)[0].any()
    # and the exact entry accepts the last position below it
    skv.swiftkv_attention_exact(ctx, dq, dk, dv, kv, lut, aq, asc, 0, [4095, 100], out)
    ctx.synchronize()
    assert kv.read(0, 0, 0, 4095, 1)[0].any() and kv.read(1, 0, 0, 100, 1)[0].any()
    for buf in (dq, dk, dv, out, aq, asc, fout):
        buf.free()
    kv.close()
    lut.close()


def test_exact_and_fast_path_agree(skv, ctx, lut4096, rope_tables):
    """Same cache, same inputs: the integer recurrence (LUT exp, 18-bit
    reciprocal) and the FP32 path land within the integer path's own error."""
    _note("case: exact vs FP32 step, position 700")
    cos, sin = rope_tables
    p = 700
    kv = skv.KVCache(ctx, layers=1, max_batch=1, max_seq_len=p + 1)
    kh, vh = history(31, p)
    prefill(skv, ctx, kv, lut4096, 0, 0, kh, vh)
    q, k, v = (f32_normal(31 + i, (1, 4096)) for i in (1000, 1001, 1002))
    out_i, _, _ = exact_step(skv, ctx, kv, lut4096, 0, [p], q, k, v, q17=False)
    dq, dk, dv = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
    out = ctx.alloc(4096 * 4)
    skv.swiftkv_attention(ctx, dq, dk, dv, kv, lut4096, None, None, 0, [p], out)
    ctx.synchronize()
    out_f = out.download(np.float32, (1, 4096))
    for buf in (dq, dk, dv, out):
        buf.free()
    kv.close()
    err = np.abs(out_i[0] * 2.0 ** -17 - out_f[0].astype(np.float64))
    assert err.max() < 2e-3 * max(1.0, np.abs(out_f).max()), err.max()


@pytest.mark.parametrize("positions", [
    [5, 300, 64],
    [int(p) for p in np.random.default_rng(37).integers(0, 301, 37)],
])
def test_host_io_mode_matches_device_mode(skv, ctx, lut4096, positions):
    """Host-memory I/O stages through the device and returns the same bits as
    the device-pointer call, for the FP32, Q15.17 and exact entries and the
    bulk append."""
    B = len(positions)
    _note(f"case: host-memory I/O vs device pointers, batch {B}")
    kv = skv.KVCache(ctx, layers=1, max_batch=B, max_seq_len=301)
    kvh = skv.KVCache(ctx, layers=1, max_batch=B, max_seq_len=301)
    for b, p in enumerate(positions):
        kh, vh = history(70 + b, p)
        prefill(skv, ctx, kv, lut4096, 0, b, kh, vh)
        ctx.set_host_io(True)
        try:
            skv.swiftkv_append_tokens(ctx, np.ascontiguousarray(kh), np.ascontiguousarray(vh), kvh, lut4096, 0,
                                      b, 0, p)
        finally:
            ctx.set_host_io(False)
    q, k, v = (f32_normal(80 + i, (B, 4096)) for i in range(3))
    ref = []
    for fn, args, odt in ((skv.swiftkv_attention, (q, k, v), np.float32),
                          (skv.swiftkv_attention, tuple(O.f2q17(x) for x in (q, k, v)), np.float32),
                          (skv.swiftkv_attention_exact, (q, k, v), np.int32)):
        q17 = args[0].dtype == np.int32
        dq, dk, dv = (ctx.to_device(x) for x in args)
        out, aq, asc = ctx.alloc(B * 4096 * 4), ctx.alloc(B * 128 * 56), ctx.alloc(B * 128)
        fn(ctx, dq, dk, dv, kv, lut4096, aq, asc, 0, positions, out, q17=q17)
        ctx.synchronize()
        ref = (out.download(odt, (B, 4096)), aq.download(np.uint8, (B, 128, 56)), asc.download(np.uint8, (B, 128)))
        for buf in (dq, dk, dv, out, aq, asc):
            buf.free()
        hout, haq, hasc = np.zeros((B, 4096), odt), np.zeros((B, 128, 56), np.uint8), np.zeros((B, 128), np.uint8)
        ctx.set_host_io(True)
        try:
            fn(ctx, *(np.ascontiguousarray(x) for x in args), kvh, lut4096, haq, hasc, 0, positions, hout, q17=q17)
            with pytest.raises(skv.SwiftKVError):
                ctx.capture_begin()
        finally:
            ctx.set_host_io(False)
        assert (hout == ref[0]).all() and (haq == ref[1]).all() and (hasc == ref[2]).all(), fn.__name__
    for b, p in enumerate(positions):
        for h in (0, 17, 31):
            got, want = kvh.read(b, 0, h, 0, p + 1), kv.read(b, 0, h, 0, p + 1)
            assert all((x == y).all() for x, y in zip(got, want)), f"seq {b} head {h}"
    kv.close()
    kvh.close()
