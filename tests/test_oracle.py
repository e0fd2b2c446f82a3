"""CPU tests that pin the oracle (oracle/swiftkv_oracle.c) before it is trusted.

Each check is chosen so a plausible mistake (dropped term, wrong sign, wrong
index, transposed operand) fails it:
  - the reference's own known-answer test hashes (integer path, positions 0/1);
  - the reference rope_lut.bin (sha256 + decoded entries);
  - the reference emulator's outputs on decode sequences (golden.json);
  - the compiled reference emulator (oracle/_ref) where it is built;
  - closed forms / invariants for the FP32 formula.
"""
import hashlib
import threading

import numpy as np
import pytest

from helpers import kat_vector, q17_uniform


# ----------------------------------------------------------------- RoPE table
def test_rope_closed_form_matches_reference_file_hash(oracle, rope_tables, golden):
    cos, sin = rope_tables
    image = oracle.rope_pack(cos, sin)
    assert image.size == golden["rope"]["bytes"]
    assert hashlib.sha256(image.tobytes()).hexdigest() == golden["rope"]["sha256"]


def test_rope_closed_form_matches_reference_entries(rope_tables, golden):
    cos, sin = rope_tables
    for pos, pair, c, s in golden["rope"]["entries"]:
        assert cos[pos, pair] == c and sin[pos, pair] == s, (pos, pair)


def test_rope_pack_unpack_roundtrip(oracle, rope_tables):
    cos, sin = rope_tables
    c2, s2 = oracle.rope_unpack(oracle.rope_pack(cos[:64], sin[:64]))
    assert (c2 == cos[:64]).all() and (s2 == sin[:64]).all()


def test_rope_extension_beyond_4096(oracle, rope_tables):
    cos, sin = rope_tables
    c2, s2 = oracle.rope_values(8, pos0=4090)
    assert (c2[:6] == cos[4090:4096]).all() and (s2[:6] == sin[4090:4096]).all()
    c3, s3 = oracle.rope_values(2, pos0=32766)
    assert np.all(np.abs(c3) <= 131072) and np.all(np.abs(s3) <= 131072)
    # cos^2 + sin^2 = 1 within Q1.17 rounding
    r2 = (c3.astype(np.float64) ** 2 + s3.astype(np.float64) ** 2) / 131072.0 ** 2
    assert np.all(np.abs(r2 - 1.0) < 4.0 / 131072.0)


# ----------------------------------------------------------------- conversion
def _f2q17_rint(bits: np.ndarray) -> np.ndarray:
    """Independent formula: RNE(x * 2^17) in float64, saturated; NaN by sign."""
    with np.errstate(invalid="ignore", over="ignore"):
        x = bits.view(np.float32).astype(np.float64)
        r = np.rint(x * 131072.0)
    r = np.where(np.isnan(r), np.where((bits >> np.uint32(31)) != 0, -2.0 ** 31, 2.0 ** 31), r)
    return np.clip(r, -2.0 ** 31, 2.0 ** 31 - 1).astype(np.int64).astype(np.int32)


def test_f2q17_against_rint_formula(oracle):
    # every exponent, sign, 2^12 fractions each, plus halfway fractions
    e = np.arange(256, dtype=np.uint32)
    frac = np.concatenate([np.arange(4096, dtype=np.uint32) * np.uint32(2048 + 1) % np.uint32(1 << 23),
                           np.array([0, 1, (1 << 22), (1 << 22) + 1, (1 << 22) - 1, (1 << 23) - 1], np.uint32)])
    bits = ((e[:, None, None] << np.uint32(23)) | frac[None, None, :] |
            (np.array([0, 1], np.uint32)[None, :, None] << np.uint32(31))).reshape(-1)
    got = oracle.f2q17(bits.view(np.float32))
    assert (got == _f2q17_rint(bits)).all()
    # halfway cases at every shift: sig = odd/even * 2^(sh-1) patterns
    for ex in range(109, 133):
        sh = 133 - ex
        for q in (0, 1, 2, 3, (1 << (24 - sh)) - 1):
            sig = (1 << 23) | 0
            for low in ((q << sh) | (1 << (sh - 1)),):
                b = np.uint32((ex << 23) | (low & 0x7fffff))
                assert oracle.f2q17(np.array([b], np.uint32).view(np.float32))[0] == \
                    _f2q17_rint(np.array([b], np.uint32))[0]
            del sig


def test_f2q17_exhaustive_digest_matches_rint(oracle):
    """All 2^32 bit patterns: compare the oracle's order-independent digest with
    the digest of the independent formula, computed in numpy over 2^26 blocks in
    8 threads (ctypes and numpy release the GIL)."""
    pytest.importorskip("numpy")
    span = 1 << 32
    chunk = 1 << 26
    starts = list(range(0, span, chunk))
    results = {}

    def mix64(z):
        with np.errstate(over="ignore"):
            z = z + np.uint64(0x9E3779B97F4A7C15)
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            return z ^ (z >> np.uint64(31))

    def work(lo):
        bits = np.arange(lo, lo + chunk, dtype=np.uint64).astype(np.uint32)
        q = _f2q17_rint(bits).view(np.uint32).astype(np.uint64)
        with np.errstate(over="ignore"):
            d = int(mix64((bits.astype(np.uint64) << np.uint64(32)) ^ q).sum(dtype=np.uint64))
        results[("np", lo)] = d
        results[("c", lo)] = oracle.f2q17_digest(lo, lo + chunk)

    threads = []
    for i in range(0, len(starts), 8):
        ts = [threading.Thread(target=work, args=(lo,)) for lo in starts[i:i + 8]]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        threads += ts
    mask = (1 << 64) - 1
    np_total = sum(results[("np", lo)] for lo in starts) & mask
    c_total = sum(results[("c", lo)] for lo in starts) & mask
    assert np_total == c_total


# ----------------------------------------------------- split-K partial finalize
# The Q/K/V linear stage adds its four PE partials as (p0 + p1) + (p2 + p3) in
# FP32, then converts (int4_linear_controller.cpp:1039-1054, 1655-1667,
# 1100-1118).  No golden vectors exist for that stage, so the oracle is pinned
# by known answers derived by hand from IEEE-754 round-to-nearest-even; each
# one names the alternative it excludes.
_A, _H = 2.0 ** 13, 2.0 ** -11     # ulp(2^13) = 2^-10, so 2^13 + 2^-11 is a tie


def _fin(oracle, *parts):
    return int(oracle.finalize_partials(np.array([[x] for x in parts], np.float32))[0])


def test_partials_known_answers(oracle):
    # fl(2^13 + 2^-11) ties to the even 2^13; fl(2^-11 - 2^13) = -(2^13 - 2^-11)
    # exactly (ulp below 2^13 is 2^-11), so the tree gives 2^-11 = 64 in Q15.17.
    # Left to right: 2^13, 2^13 (second tie), 0.  Right to left: 2^-10.  Pairs
    # (0,3)+(1,2): 0 + 2^-10.  Exact sum: 2^-10.
    assert _fin(oracle, _A, _H, _H, -_A) == 64
    # Tree: 2^13 (tie) + (-(2^13 - 2^-11)) = 2^-11 -> 64.  Pairs (0,2)+(1,3):
    # 0 + 2^-10 -> 128.
    assert _fin(oracle, _A, _H, -_A, _H) == 64
    # Two parts: 2^13 + 2^-10 has an odd significand, so adding 2^-11 ties up
    # to 2^13 + 2^-9 -> 2^30 + 256.  An exact (or double) sum would give
    # 2^30 + 192.
    assert _fin(oracle, _A + 2.0 ** -10, _H) == 2 ** 30 + 256
    # One part is the plain conversion.
    assert _fin(oracle, 1.5 * 2.0 ** -17) == 2
    # The alternatives really do give the values excluded above.
    f = np.float32
    a, h = f(_A), f(_H)
    assert float(((a + h) + h) + (-a)) == 0.0                  # left to right
    assert float(((-a + h) + h) + a) == 2.0 ** -10             # right to left
    assert float((a + -a) + (h + h)) == 2.0 ** -10             # pairs (0,3)+(1,2)
    assert float((a + -a) + (h + h)) != float((a + h) + (-a + h))


def test_partials_tree_symmetries(oracle):
    """Swapping within a pair, or the two pairs, cannot change an IEEE sum;
    swapping across pairs generally does (so the checks see the pairing)."""
    rng = np.random.default_rng(5)
    p = (rng.standard_normal((4, 200000)) * np.exp2(rng.integers(0, 13, (4, 200000)))).astype(np.float32)
    base = oracle.finalize_partials(p)
    assert (oracle.finalize_partials(p[[1, 0, 3, 2]]) == base).all()
    assert (oracle.finalize_partials(p[[2, 3, 0, 1]]) == base).all()
    assert (oracle.finalize_partials(p[[0, 2, 1, 3]]) != base).any()
    assert (oracle.finalize_partials(p[:1]) == oracle.f2q17(p[0])).all()
    two = oracle.reduce_partials(p[:2])
    assert (two.view(np.uint32) == (p[0] + p[1]).view(np.uint32)).all()


def test_partials_nan_rule_matches_host_arithmetic(oracle):
    """A NaN operand propagates with its sign; inf - inf gives the negative
    default NaN -- what the host's own FP32 adds (x86 SSE, the reference C
    model's platform) do.  The conversion then saturates by that sign."""
    f = np.float32
    nan_p, nan_n = np.uint32(0x7fc00000).view(f), np.uint32(0xffc00000).view(f)
    pairs = [(np.inf, -np.inf), (-np.inf, np.inf), (nan_p, f(1)), (f(1), nan_p), (nan_n, f(1)), (f(1), nan_n),
             (nan_n, np.inf), (np.inf, nan_n)]
    with np.errstate(invalid="ignore"):
        for a, b in pairs:
            got = oracle.reduce_partials(np.array([[a], [b]], f))[0]
            host = np.array([a], f) + np.array([b], f)
            assert np.isnan(got) and np.signbit(got) == np.signbit(host[0]), (a, b)
    assert _fin(oracle, np.inf, -np.inf) == -2 ** 31
    assert _fin(oracle, 1.0, nan_p) == 2 ** 31 - 1
    assert _fin(oracle, 1.0, 2.0, 3.0, nan_n) == -2 ** 31


# ----------------------------------------------------------------- quantizer
def test_g32_quantize_invariants_and_bruteforce(oracle):
    rng = np.random.default_rng(5)
    rows = [rng.integers(-2 ** 31, 2 ** 31, 128, dtype=np.int64).astype(np.int32),
            (rng.standard_normal(128) * 131072).astype(np.int32),
            np.zeros(128, np.int32),
            np.full(128, np.iinfo(np.int32).min, np.int32),
            np.concatenate([np.full(64, np.iinfo(np.int32).max, np.int32), np.full(64, -1, np.int32)]),
            np.arange(-64, 64, dtype=np.int32)]
    for x in rows:
        codes, shifts = oracle.quantize_rows(x)
        for g in range(4):
            grp = x[32 * g:32 * g + 32].astype(np.int64)
            m = int(np.abs(grp).max())
            s = int(shifts[g])
            # brute force: the smallest shift with round(m / 2^s) representable in 7 bits + 1
            exp_s = 0 if m == 0 else max(m.bit_length() - 1 - 6, 0)
            assert s == exp_s
            assert s <= 25
            c = codes[32 * g:32 * g + 32].astype(np.int64)
            assert np.all(np.abs(c) <= 127)
            recon = c * (1 << s)
            err = np.abs(recon - grp)
            clamped = np.abs(c) == 127
            assert np.all(err[~clamped] <= (1 << s) // 2 if s else err[~clamped] == 0)
            # code is the RNE-free "round half away from zero" of |r| / 2^s
            expect = np.sign(grp) * np.minimum(127, (np.abs(grp) + ((1 << s) >> 1)) >> s)
            assert (c == expect).all()


def test_record_pack_layout(oracle):
    rng = np.random.default_rng(3)
    kc = rng.integers(-127, 128, 128).astype(np.int8)
    vc = rng.integers(-127, 128, 128).astype(np.int8)
    ks = np.array([0, 5, 25, 31], np.uint8)
    vs = np.array([1, 2, 3, 17], np.uint8)
    rec = oracle.pack_record(kc, ks, vc, vs)
    meta = int.from_bytes(rec[:64].tobytes(), "little")
    for g in range(4):
        assert (meta >> (5 * g)) & 31 == ks[g]
        assert (meta >> (20 + 5 * g)) & 31 == vs[g]
    assert meta >> 40 == 0
    assert (rec[64:192].view(np.int8) == kc).all() and (rec[192:320].view(np.int8) == vc).all()
    k2, ks2, v2, vs2 = oracle.unpack_record(rec)
    assert (k2 == kc).all() and (ks2 == ks).all() and (v2 == vc).all() and (vs2 == vs).all()


# ----------------------------------------------------------------- RoPE rotate
def test_rope_rotate_position0_identity_and_norm(oracle, rope_tables):
    cos, sin = rope_tables
    x = q17_uniform(9, (32, 128), 20)
    assert (oracle.rope_rotate(x, cos[0], sin[0]) == x).all()
    y = oracle.rope_rotate(x, cos[1234], sin[1234]).astype(np.float64)
    n0 = np.linalg.norm(x.astype(np.float64).reshape(-1, 64, 2), axis=-1)
    n1 = np.linalg.norm(y.reshape(-1, 64, 2), axis=-1)
    assert np.all(np.abs(n1 - n0) <= 2.0 + n0 * 3.0 / 131072.0)
    # rotation by +theta then by the table entry of the same angle negated = identity within rounding
    back = oracle.rope_rotate(y.astype(np.int32), cos[1234], -sin[1234]).astype(np.float64)
    assert np.all(np.abs(back - x) <= 4.0 + np.abs(x) * 4.0 / 131072.0)


# ----------------------------------------------------------------- KAT
def test_reference_kat_hashes(oracle, rope_tables, golden):
    cos, sin = rope_tables
    h0, h1 = oracle.kat_pe0(cos, sin)
    assert hex(h0) == golden["kat"]["pos0"]
    assert hex(h1) == golden["kat"]["pos1"]


def test_kat_generator_matches_oracle_kat(oracle, rope_tables, golden):
    """The Python KAT generator (used for GPU runs) matches the oracle's."""
    v = kat_vector(3)
    assert v[0] == (3 * 101) % 458753 - 229376
    assert v[1023] == (1023 * 40 + 303) % 458753 - 229376


# ----------------------------------------------------------------- exp LUT
def test_exp_lut_closed_form_table_and_points(oracle):
    assert oracle.exp_neg_q17(0) == 1 << 17
    assert oracle.exp_neg_q17(5) == 1 << 17
    assert oracle.exp_neg_q17(-(32 << 17)) == 0
    # exp(x) within the chord error of a 32-segment linear interpolation of
    # 2^f (h^2/8 * ln2^2 ~ 5.9e-5 relative) plus the Q1.17 output LSB
    for x in np.linspace(-31.9, -0.001, 997):
        raw = int(round(x * 131072))
        got = oracle.exp_neg_q17(raw) / 131072.0
        true = np.exp(raw / 131072.0)
        assert abs(got - true) <= 6.0e-5 * true + 1.0 / 131072.0


# ----------------------------------------------------------------- decode golden
def _a14_q17(oracle, int_out):
    q = np.empty(4096, np.int16)
    scale = np.empty(128, np.float32)
    flat = int_out.reshape(-1)
    for g in range(128):
        qq = np.empty(32, np.int16)
        ee = np.empty(1, np.uint8)
        oracle.lib().oracle_a14_group_q17(np.ascontiguousarray(flat[32 * g:32 * g + 32]), qq, ee)
        q[32 * g:32 * g + 32] = qq
        scale[g] = 0.0 if ee[0] == 0 else np.ldexp(1.0, int(ee[0]) - 127 - 13)
    return q, scale


@pytest.mark.parametrize("case", [0, 1, 2])
def test_integer_path_matches_reference_decode(oracle, rope_tables, golden, case):
    from golden.make_golden import fnv_chain, step_inputs
    cos, sin = rope_tables
    g = golden["decode"][case]
    last = g["last_position"]
    sc = oracle.SequenceCache(32, last + 1)
    h = 1469598103934665603
    for pos in range(last + 1):
        q, k, v = step_inputs(g["seed"], pos, g["span_bits"])
        res = sc.step_q17(q, k, v, pos, cos[pos], sin[pos], fp=False, integer=True)
        aq, asc = _a14_q17(oracle, res["int"])
        h = fnv_chain(h, aq.tobytes() + asc.tobytes())
    assert (aq == np.array(g["a14_last"], np.int16)).all()
    assert (asc == np.array(g["scale_last"], np.float32)).all()
    assert hex(h) == g["chain_hash"]


# ----------------------------------------------------------------- FP32 formula
def _rand_cache(oracle, rope_tables, n, seed, heads=1):
    cos, sin = rope_tables
    k = q17_uniform(seed, (n, heads * 128), 18)
    v = q17_uniform(seed + 1, (n, heads * 128), 18)
    sc = oracle.SequenceCache(heads, n)
    sc.fill_q17(k, v, 0, cos, sin)
    return sc


def _deq(codes, shifts):
    return codes.astype(np.float64) * np.ldexp(1.0, shifts.astype(np.int64) - 17).repeat(32, axis=-1)


def test_fp_single_token_is_v(oracle, rope_tables):
    sc = _rand_cache(oracle, rope_tables, 1, 21)
    q = q17_uniform(99, (128,), 18)
    out = oracle.attend_head_fp(q, sc.kc[0, :1], sc.ks[0, :1], sc.vc[0, :1], sc.vs[0, :1])
    assert np.array_equal(out, _deq(sc.vc[0, 0], sc.vs[0, 0]))


def test_fp_identical_keys_give_mean_v(oracle, rope_tables):
    sc = _rand_cache(oracle, rope_tables, 50, 23)
    kc = np.repeat(sc.kc[0, :1], 50, axis=0)
    ks = np.repeat(sc.ks[0, :1], 50, axis=0)
    q = q17_uniform(98, (128,), 18)
    out = oracle.attend_head_fp(q, kc, ks, sc.vc[0, :50], sc.vs[0, :50])
    mean = np.mean([_deq(sc.vc[0, t], sc.vs[0, t]) for t in range(50)], axis=0)
    assert np.allclose(out, mean, rtol=1e-12, atol=1e-12)


def test_fp_dominant_score_selects_its_value(oracle, rope_tables):
    sc = _rand_cache(oracle, rope_tables, 20, 25)
    kc = np.zeros((20, 128), np.int8)
    ks = np.zeros((20, 4), np.uint8)
    kc[7] = 127
    ks[7] = 17                            # k^ = 127 on every channel
    q = np.full(128, 1 << 17, np.int32)   # q^ = 1: score 16256/sqrt(128) ~ 1437, others 0
    out = oracle.attend_head_fp(q, kc, ks, sc.vc[0, :20], sc.vs[0, :20])
    assert np.array_equal(out, _deq(sc.vc[0, 7], sc.vs[0, 7]))


def test_fp_matches_brute_force_numpy(oracle, rope_tables):
    """Independent numpy restatement of the softmax formula (two-pass, float64)."""
    sc = _rand_cache(oracle, rope_tables, 77, 27)
    q = q17_uniform(97, (128,), 18)
    K = _deq(sc.kc[0, :77], sc.ks[0, :77])
    V = _deq(sc.vc[0, :77], sc.vs[0, :77])
    s = (K @ (q.astype(np.float64) / 131072.0)) * float(np.float32(1.0) / np.sqrt(np.float32(128.0)))
    p = np.exp(s - s.max())
    p /= p.sum()
    assert np.allclose(oracle.attend_head_fp(q, sc.kc[0, :77], sc.ks[0, :77], sc.vc[0, :77], sc.vs[0, :77]),
                       p @ V, rtol=1e-12, atol=1e-15)


def test_fp_and_integer_paths_agree(oracle, rope_tables):
    sc = _rand_cache(oracle, rope_tables, 300, 29)
    q = q17_uniform(96, (128,), 18)
    fp = oracle.attend_head_fp(q, sc.kc[0, :300], sc.ks[0, :300], sc.vc[0, :300], sc.vs[0, :300])
    it = oracle.attend_head_int(q, sc.kc[0, :300], sc.ks[0, :300], sc.vc[0, :300], sc.vs[0, :300])
    assert np.max(np.abs(fp - it / 131072.0)) < 1e-3


# ----------------------------------------------------------------- A14 epilogue
def test_a14_float_rule_equals_the_integer_rule_on_q17_values(oracle):
    """The float A14 rule (applied to the FP32 path's output) and the integer
    path's rule (pinned by the reference KAT hashes, the emulator decode
    goldens and the reference build) must agree on every value the integer
    path can produce, raw * 2^-17: same lanes, same E8M0 code.  Spans from
    2^1 to 2^31 raw cover group exponents -15 to 15."""
    rng = np.random.default_rng(8)
    for span in range(1, 32):
        raw = rng.integers(-(1 << span) + 1, 1 << span, (64, 32), dtype=np.int64).astype(np.int32)
        raw[0] = 0
        raw[1, 5] = (1 << span) - 1
        raw[2, :] = np.where(np.arange(32) % 2, 1, -1) << (span - 1)   # ties at the top octave
        x = (raw.astype(np.float32) * np.float32(2.0 ** -17))
        qf, ef = oracle.a14(x)
        qi, ei = oracle.a14_q17(raw)
        assert (qf == qi).all() and (ef == ei).all(), f"span 2^{span}"
        assert ef[0] == 0 and (qf[0] == 0).all()


def test_a14_scale_invariance_down_to_the_exponent_floor(oracle):
    """Scaling a group by 2^-k leaves its lanes unchanged and lowers its code
    by k while the group exponent stays >= -127 (the reference's floor,
    swiftkv_attention.cpp:1722-1724).  Below the floor the code stays 0 and
    the lanes still decode, lane * 2^-140, to within half a step of the
    value: the scaling must stay finite where 2^(13-e) overflows (e < -114)."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((8, 32)).astype(np.float32)
    x[1, 3] = 0.0
    q0, e0 = oracle.a14(x)
    top = np.frexp(np.abs(x).max(axis=1))[1]
    assert (e0 == top + 127).all()
    assert (np.abs(q0).max(axis=1) >= 4096).all()     # the largest lane lands in the top octave
    for k in range(1, 150):
        xs = np.ldexp(x, -k).astype(np.float32)
        q, e = oracle.a14(xs)
        for r in range(8):
            if top[r] - k >= -100:           # every lane still a normal float: exact invariance
                assert e[r] == e0[r] - k and (q[r] == q0[r]).all(), (k, r)
            elif top[r] - k >= -127:         # small lanes become subnormal and lose low bits
                assert e[r] == e0[r] - k and (np.abs(q[r].astype(int) - q0[r]) <= 1).all(), (k, r)
            else:
                assert e[r] == 0
                step = 2.0 ** -140
                assert (np.abs(q[r] * step - xs[r].astype(np.float64)) <= 0.5 * step + 2.0 ** -151).all(), (k, r)


def test_a14_packing(oracle, skv):
    rng = np.random.default_rng(10)
    q = rng.integers(-8191, 8192, (16, 32)).astype(np.int16)
    words = oracle.pack_a14(q)
    assert (skv.unpack_a14(words) == q).all()


# ----------------------------------------------------------------- reference build (oracle/_ref)
ref_available = pytest.mark.skipif(not __import__("oracle").Reference.available(),
                                   reason="oracle/_ref not built (reference sources absent)")


@ref_available
def test_oracle_primitives_match_reference_build(oracle, rope_tables):
    R = oracle.Reference()
    cos, sin = rope_tables
    R.set_rope(cos, sin)
    rng = np.random.default_rng(17)
    bits = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    assert (R.f2q17(f) == oracle.f2q17(f)).all()
    for pos in (0, 1, 77, 2048, 4095):
        x = q17_uniform(pos + 5, (4096,), 30)
        mine = oracle.rope_rotate(x.reshape(32, 128), cos[pos], sin[pos]).reshape(-1)
        assert (R.apply_rope(x, pos) == mine).all()
    for xv in list(range(-(32 << 17) - 3, -(32 << 17) + 3)) + list(rng.integers(-(33 << 17), 10, 20000)):
        assert R.L.ref_exp_negative_q17(int(xv)) == oracle.exp_neg_q17(int(xv))
    for span in (8, 18, 24, 31):
        x = q17_uniform(span, (64, 32), min(span, 30))
        if span == 31:
            x[0, 0] = np.iinfo(np.int32).min
            x[1, 0] = np.iinfo(np.int32).max
        for row in x:
            s = R.L.ref_shift_for_group(np.ascontiguousarray(row))
            assert s == oracle.lib().oracle_g32_shift(np.ascontiguousarray(row))
            for val in row[:8]:
                assert R.L.ref_quantize_raw(int(val), s) == oracle.lib().oracle_g32_code(int(val), s)


@ref_available
def test_oracle_step_matches_reference_build_long_context(oracle, rope_tables):
    cos, sin = rope_tables
    R = oracle.Reference()
    R.set_rope(cos, sin)
    pos = 1500
    k = q17_uniform(31, (pos, 4096), 18)
    v = q17_uniform(32, (pos, 4096), 18)
    sc = oracle.SequenceCache(32, pos + 1)
    sc.fill_q17(k, v, 0, cos, sin)
    rc = R.cache(pos + 1)
    rc.load_from(sc, pos)
    q, kn, vn = (q17_uniform(33 + i, (4096,), 18) for i in range(3))
    aq, asc = rc.attention(R.apply_rope(q, pos), R.apply_rope(kn, pos), vn, pos)
    res = sc.step_q17(q, kn, vn, pos, cos[pos], sin[pos], fp=False, integer=True)
    mq, ms = _a14_q17(oracle, res["int"])
    assert (mq == aq).all() and (ms == asc).all()
    for h in (0, 13, 31):
        kc, ks, vc, vs = rc.row(h, pos)
        assert (kc == sc.kc[h, pos]).all() and (ks == sc.ks[h, pos]).all()
        assert (vc == sc.vc[h, pos]).all() and (vs == sc.vs[h, pos]).all()
