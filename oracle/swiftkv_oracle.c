/*
 * swiftkv_oracle.c -- CPU restatement of the SwiftKV decode-attention arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the oracle for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and
 * only to compare against or to time as a baseline.  The product library
 * (4pe_u250_amd/csrc) never links or calls it.
 *
 * Every function names the reference lines it restates (paths relative to the
 * reference repository).  Integer semantics follow the HLS types:
 *   int4_fxp32_t           = ap_fixed<32,15,AP_RND_CONV,AP_SAT>   (Q15.17)
 *   swiftkv_dot_t          = ap_fixed<44,20,AP_RND_CONV,AP_WRAP>  (Q20.24)
 *   swiftkv_normalization_t= ap_ufixed<30,13,AP_RND_CONV,AP_WRAP> (Q13.17)
 *   swiftkv_coefficient_t  = ap_ufixed<18,1,AP_RND_CONV,AP_SAT>   (Q1.17)
 * AP_RND_CONV is round-half-to-even; because ties-to-even is symmetric it is
 * the same on the two's-complement value and on sign/magnitude.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   f2q17            exhaustive 2^32 sweep against an independent rint()-based
 *                    formula, and against the compiled reference emulator.
 *   reduce_partials  known answers derived by hand from IEEE-754 rounding
 *                    that tell the pair tree apart from left-to-right,
 *                    right-to-left and the other pairings and from an exact
 *                    sum; the NaN rule against the host's own FP32 adds.
 *   rope_lut_*       sha256 of the packed 4096-position table equals the
 *                    reference rope_lut.bin; per-entry check against the
 *                    reference emulator's decode of that file.
 *   rope_rotate      identity at position 0, norm preservation, and the
 *                    compiled reference emulator on random inputs.
 *   g32 quantize     invariants (|q|<=127, reconstruction error bound) and
 *                    brute force over all shifts, and the reference emulator.
 *   integer attention the reference's own known-answer test (two FNV hashes
 *                    from tb_attention_pe0_kv_rtl.cpp:109-110), the compiled
 *                    reference emulator at long contexts.
 *   fp attention     closed forms: one token => v, identical keys => mean(v),
 *                    one dominant score => that v; and agreement with the
 *                    integer recurrence within its LUT error.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HD 128          /* head_dim (swiftkv_attention.hpp:5-6) */
#define PAIRS 64        /* RoPE pairs per head (hpp:55-56) */
#define G32 32          /* KV quantization group (hpp:11) */
#define NGROUPS 4       /* groups per head (hpp:12-13) */

/* ------------------------------------------------------------------------ */
/* small integer helpers                                                      */
/* ------------------------------------------------------------------------ */

static int32_t sat32(int64_t x) {
    if (x > INT32_MAX) return INT32_MAX;
    if (x < INT32_MIN) return INT32_MIN;
    return (int32_t)x;
}

/* Round-half-even of x / 2^s on the magnitude (emulator:507-517). */
int64_t oracle_rne_shift(int64_t x, unsigned s) {
    if (s == 0) return x;
    int neg = x < 0;
    uint64_t mag = neg ? (uint64_t)(-(x + 1)) + 1u : (uint64_t)x;
    uint64_t q = mag >> s;
    uint64_t rem = mag & ((1ull << s) - 1u);
    uint64_t half = 1ull << (s - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return neg ? -(int64_t)q : (int64_t)q;
}

/* Two's-complement truncation to `bits` bits (emulator:519-524). */
int64_t oracle_wrap(int64_t x, unsigned bits) {
    uint64_t mask = (bits >= 64) ? ~0ull : ((1ull << bits) - 1u);
    uint64_t r = (uint64_t)x & mask;
    if (bits < 64 && (r >> (bits - 1)) & 1u) r |= ~mask;
    return (int64_t)r;
}

/* ------------------------------------------------------------------------ */
/* a1: FP32 -> Q15.17 (int4_linear_controller.cpp:38-83, emulator:481-505)    */
/* ------------------------------------------------------------------------ */
int32_t oracle_f2q17(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    uint32_t sign = b >> 31, e = (b >> 23) & 0xffu, frac = b & 0x7fffffu;
    if (e < 109u) return 0;                 /* |x| < 2^-18 (also zero/denormal) */
    if (e >= 141u) return sign ? INT32_MIN : INT32_MAX;   /* |x| >= 2^14, inf, nan */
    uint64_t sig = (1u << 23) | frac, mag;
    if (e >= 133u) {
        mag = sig << (e - 133u);
    } else {
        unsigned sh = 133u - e;             /* 1..24 */
        uint64_t q = sig >> sh, rem = sig & ((1ull << sh) - 1u), half = 1ull << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        mag = q;
    }
    if (!sign) return mag > (uint64_t)INT32_MAX ? INT32_MAX : (int32_t)mag;
    return mag >= (1ull << 31) ? INT32_MIN : -(int32_t)mag;
}

void oracle_f2q17_array(const float* in, int32_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f2q17(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Q/K/V linear-stage partial reduction and finalize                          */
/* (int4_linear_controller.cpp:1039-1054 adds two FP32 lanes; :1655-1660      */
/* reduces partials 0+1 and 2+3 into pair sums; :1100-1118 adds the two pair  */
/* sums and converts to Q15.17, for the Q/K/V modes only, :129-132).          */
/* ------------------------------------------------------------------------ */
/* One FP32 add with the NaN sign fixed: x86 SSE (the platform of the
 * reference's C model) returns a NaN operand as the result, and the negative
 * default NaN for inf - inf; when both operands are NaN the C source leaves
 * the choice to the compiler, and this picks the first. */
static float add_partials(float a, float b) {
    const float s = a + b;
    if (!isnan(s)) return s;
    if (isnan(a)) return a;
    if (isnan(b)) return b;
    uint32_t bits = 0xffc00000u;
    float nan_neg;
    memcpy(&nan_neg, &bits, 4);
    return nan_neg;
}

/* parts = 1, 2 or 4; part p of element i at in[i + p * part_stride].
 * Two parts: fl(p0 + p1).  Four: fl(fl(p0 + p1) + fl(p2 + p3)). */
void oracle_reduce_partials(const float* in, int parts, int64_t part_stride, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float x = in[i];
        if (parts >= 2) x = add_partials(in[i], in[i + part_stride]);
        if (parts == 4) x = add_partials(x, add_partials(in[i + 2 * part_stride], in[i + 3 * part_stride]));
        out[i] = x;
    }
}

void oracle_finalize_partials(const float* in, int parts, int64_t part_stride, int32_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float x;
        oracle_reduce_partials(in + i, parts, part_stride, &x, 1);
        out[i] = oracle_f2q17(x);
    }
}

/* Order-independent digest of f2q17 over the bit patterns [lo, hi):
 * sum over i of mix(i, f2q17(bits=i)).  Summed over all 2^32 patterns it is
 * compared with the same digest of an independent float64 rint() formula. */
static uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
uint64_t oracle_f2q17_digest(uint64_t lo, uint64_t hi) {
    uint64_t acc = 0;
    for (uint64_t i = lo; i < hi; ++i) {
        uint32_t bits = (uint32_t)i;
        float f;
        memcpy(&f, &bits, 4);
        acc += mix64(((uint64_t)bits << 32) ^ (uint32_t)oracle_f2q17(f));
    }
    return acc;
}

/* ------------------------------------------------------------------------ */
/* a2: RoPE LUT (scripts/generate_rope_lut.py:67-150, hpp:55-81)              */
/* ------------------------------------------------------------------------ */

/* cos/sin of pos * theta^(-j/64) as signed Q1.17 (19-bit saturated), RNE. */
void oracle_rope_values(int pos0, int npos, double theta, int32_t* cosv, int32_t* sinv) {
    for (int p = 0; p < npos; ++p) {
        for (int j = 0; j < PAIRS; ++j) {
            double freq = 1.0 / pow(theta, (double)j / (double)PAIRS);
            double ang = (double)(pos0 + p) * freq;
            double c = nearbyint(cos(ang) * 131072.0), s = nearbyint(sin(ang) * 131072.0);
            if (c > 262143.0) c = 262143.0;
            if (c < -262144.0) c = -262144.0;
            if (s > 262143.0) s = 262143.0;
            if (s < -262144.0) s = -262144.0;
            cosv[(size_t)p * PAIRS + j] = (int32_t)c;
            sinv[(size_t)p * PAIRS + j] = (int32_t)s;
        }
    }
}

static void put_bits(uint8_t* base, int bit, int width, uint32_t value) {
    for (int b = 0; b < width; ++b) {
        int dst = bit + b;
        if ((value >> b) & 1u) base[dst >> 3] |= (uint8_t)(1u << (dst & 7));
    }
}
static uint32_t get_bits(const uint8_t* base, int bit, int width) {
    uint32_t v = 0;
    for (int b = 0; b < width; ++b) {
        int src = bit + b;
        v |= (uint32_t)((base[src >> 3] >> (src & 7)) & 1u) << b;
    }
    return v;
}

/* File layout: position p, LUT word w (pairs 16w..16w+15) at byte (p*4+w)*128;
 * pair lane i: cos at bits [38i, 38i+18], sin at [38i+19, 38i+37] of the
 * little-endian 608-bit word; bytes 76..127 of each 128-byte slot are zero. */
void oracle_rope_pack(int npos, const int32_t* cosv, const int32_t* sinv, uint8_t* out) {
    memset(out, 0, (size_t)npos * 512);
    for (int p = 0; p < npos; ++p)
        for (int j = 0; j < PAIRS; ++j) {
            uint8_t* slot = out + ((size_t)p * 4 + (size_t)(j / 16)) * 128;
            int lane = j % 16;
            put_bits(slot, 38 * lane, 19, (uint32_t)cosv[(size_t)p * PAIRS + j] & 0x7ffffu);
            put_bits(slot, 38 * lane + 19, 19, (uint32_t)sinv[(size_t)p * PAIRS + j] & 0x7ffffu);
        }
}

static int32_t sext19(uint32_t r) { return (r & 0x40000u) ? (int32_t)(r | 0xfff80000u) : (int32_t)r; }

void oracle_rope_unpack(int npos, const uint8_t* in, int32_t* cosv, int32_t* sinv) {
    for (int p = 0; p < npos; ++p)
        for (int j = 0; j < PAIRS; ++j) {
            const uint8_t* slot = in + ((size_t)p * 4 + (size_t)(j / 16)) * 128;
            int lane = j % 16;
            cosv[(size_t)p * PAIRS + j] = sext19(get_bits(slot, 38 * lane, 19));
            sinv[(size_t)p * PAIRS + j] = sext19(get_bits(slot, 38 * lane + 19, 19));
        }
}

/* ------------------------------------------------------------------------ */
/* a3: adjacent-pair integer rotation (swiftkv_attention.cpp:20-95,          */
/*     emulator:526-541).  x'[2j]=sat32((a c - b s)>>17), x'[2j+1]=          */
/*     sat32((a s + b c)>>17), floor shift on the 52-bit sum.                 */
/* ------------------------------------------------------------------------ */
void oracle_rope_rotate(int32_t* x, const int32_t* cos64, const int32_t* sin64) {
    for (int j = 0; j < PAIRS; ++j) {
        int64_t a = x[2 * j], b = x[2 * j + 1], c = cos64[j], s = sin64[j];
        x[2 * j] = sat32((a * c - b * s) >> 17);
        x[2 * j + 1] = sat32((a * s + b * c) >> 17);
    }
}

/* Rows [nrows][128], each rotated with its own table row cos/sin [nrows][64]. */
void oracle_rope_rotate_rows(int32_t* x, int64_t nrows, const int32_t* cos_rows, const int32_t* sin_rows) {
    for (int64_t r = 0; r < nrows; ++r) oracle_rope_rotate(x + r * HD, cos_rows + r * PAIRS, sin_rows + r * PAIRS);
}

/* ------------------------------------------------------------------------ */
/* a4: G32 power-of-two quantization (cpp:348-414, emulator:543-564)          */
/* ------------------------------------------------------------------------ */
uint8_t oracle_g32_shift(const int32_t* r) {
    uint32_t m = 0;
    for (int i = 0; i < G32; ++i) {
        uint32_t a = r[i] < 0 ? (uint32_t)(-(int64_t)r[i]) : (uint32_t)r[i];
        if (a > m) m = a;
    }
    if (m == 0) return 0;
    int msb = 31;
    while (!((m >> msb) & 1u)) --msb;
    return (uint8_t)(msb > 6 ? msb - 6 : 0);
}

int8_t oracle_g32_code(int32_t r, uint8_t s) {
    uint64_t mag = r < 0 ? (uint64_t)(-(int64_t)r) : (uint64_t)r;
    if (s) mag += 1ull << (s - 1);
    mag >>= s;
    if (mag > 127u) mag = 127u;
    return r < 0 ? (int8_t)(-(int)mag) : (int8_t)mag;
}

/* One head row (128 channels) -> 128 codes + 4 shifts. */
void oracle_quantize_row(const int32_t* x, int8_t* codes, uint8_t* shifts) {
    for (int g = 0; g < NGROUPS; ++g) {
        uint8_t s = oracle_g32_shift(x + g * G32);
        shifts[g] = s;
        for (int i = 0; i < G32; ++i) codes[g * G32 + i] = oracle_g32_code(x[g * G32 + i], s);
    }
}

/* Many rows at once: x [nrows][128] -> codes [nrows][128], shifts [nrows][4]. */
void oracle_quantize_rows(const int32_t* x, int64_t nrows, int8_t* codes, uint8_t* shifts) {
    for (int64_t r = 0; r < nrows; ++r) oracle_quantize_row(x + r * HD, codes + r * HD, shifts + r * NGROUPS);
}

/* FP32 value of a G32 scale: 2^(s-17), exactly representable. */
float oracle_shift_scale(uint8_t s) { return ldexpf(1.0f, (int)s - 17); }

/* ------------------------------------------------------------------------ */
/* a5: reference DDR record [meta, K0, K1, V0, V1] (hpp:94-110,               */
/*     cpp:427-582).  meta bits [5g,5g+4] = K shift g, [20+5g..] = V shift g; */
/*     K codes bytes 64..191 (channel i at byte 64+i), V codes 192..319.      */
/* ------------------------------------------------------------------------ */
void oracle_pack_record(const int8_t* kc, const uint8_t* ks, const int8_t* vc, const uint8_t* vs,
                        uint8_t* rec320) {
    memset(rec320, 0, 320);
    for (int g = 0; g < NGROUPS; ++g) {
        put_bits(rec320, 5 * g, 5, ks[g] & 31u);
        put_bits(rec320, 20 + 5 * g, 5, vs[g] & 31u);
    }
    memcpy(rec320 + 64, kc, HD);
    memcpy(rec320 + 192, vc, HD);
}

void oracle_unpack_record(const uint8_t* rec320, int8_t* kc, uint8_t* ks, int8_t* vc, uint8_t* vs) {
    for (int g = 0; g < NGROUPS; ++g) {
        ks[g] = (uint8_t)get_bits(rec320, 5 * g, 5);
        vs[g] = (uint8_t)get_bits(rec320, 20 + 5 * g, 5);
    }
    memcpy(kc, rec320 + 64, HD);
    memcpy(vc, rec320 + 192, HD);
}

/* ------------------------------------------------------------------------ */
/* a9: LUT exp for x <= 0 (cpp:185-260, emulator:566-595)                     */
/* ------------------------------------------------------------------------ */
static uint32_t exp2_q30(int i) {
    /* RNE(2^(30 + i/32)); i = 0..32 (the table at cpp:185-195). */
    return (uint32_t)nearbyint(ldexp(pow(2.0, (double)i / 32.0), 30));
}

uint32_t oracle_exp_neg_q17(int32_t x) {
    if (x >= 0) return 1u << 17;
    if (x <= -(32 << 17)) return 0;
    /* log2(e) as ap_fixed<24,3> = RNE(1.4426950408889634 * 2^21) */
    const int64_t log2e_q21 = (int64_t)nearbyint(1.4426950408889634 * 2097152.0);
    int64_t l = oracle_wrap(oracle_rne_shift((int64_t)x * log2e_q21, 21), 24);
    int64_t ex = l >> 17;                      /* floor */
    uint32_t f = (uint32_t)(l - (ex << 17));   /* 17-bit fraction */
    uint32_t idx = f >> 12, rm = f & 0xfffu;
    uint32_t base = exp2_q30((int)idx), next = exp2_q30((int)idx + 1);
    uint32_t interp = base + (uint32_t)(((uint64_t)(next - base) * rm + (1u << 11)) >> 12);
    int sh = 13 - (int)ex;
    uint64_t out = 0;
    if (sh <= 0) out = (uint64_t)interp << (-sh);
    else if (sh < 32) out = ((uint64_t)interp + (1ull << (sh - 1))) >> sh;
    return (uint32_t)out & 0x3ffffu;
}

/* Q15.17 x unsigned multiplier, RNE >> 17, wrap to 32 (cpp:1530-1550). */
static int32_t mulq17_wrap(int32_t a, uint32_t b) {
    return (int32_t)oracle_wrap(oracle_rne_shift((int64_t)a * (int64_t)b, 17), 32);
}

/* ------------------------------------------------------------------------ */
/* a6-a11: integer single-pass recurrence for one head (cpp:934-1880,        */
/* emulator:633-689).  Inputs: rotated query (Q15.17), the cached codes and   */
/* shifts for tokens 0..ntok-1.  Output: normalized Q15.17 state [128].       */
/* ------------------------------------------------------------------------ */
void oracle_attend_head_int(const int32_t* q, const int8_t* kc, const uint8_t* ks,
                            const int8_t* vc, const uint8_t* vs, int ntok, int32_t* out) {
    const int64_t score_scale = 11585;  /* RNE(2^17 / sqrt(128)) (cpp:1101-1102) */
    int32_t run_max = 0;
    uint32_t z = 0;
    int32_t y[HD];
    memset(y, 0, sizeof(y));
    for (int t = 0; t < ntok; ++t) {
        const int8_t* k = kc + (size_t)t * HD;
        const uint8_t* kss = ks + (size_t)t * NGROUPS;
        int64_t dot = 0;
        for (int g = 0; g < NGROUPS; ++g) {
            int64_t half[2];
            for (int h = 0; h < 2; ++h) {
                int64_t s = 0;
                for (int i = 0; i < 16; ++i) {
                    int c = g * 32 + h * 16 + i;
                    s += (int64_t)q[c] * k[c];
                }
                int sh = kss[g];
                half[h] = oracle_wrap(sh >= 10 ? (int64_t)((uint64_t)s << (sh - 10)) : (s >> (10 - sh)), 44);
            }
            int64_t gd = oracle_wrap(half[0] + half[1], 44);
            dot = g == 0 ? gd : oracle_wrap(dot + gd, 44);
        }
        int32_t score = sat32(oracle_rne_shift(dot * score_scale, 24));
        uint32_t coef = 1u << 17;
        int rescale = 0;
        if (t == 0) {
            run_max = score;
            z = 1u << 17;
        } else if (score <= run_max) {
            coef = oracle_exp_neg_q17(sat32((int64_t)score - run_max));
            z = (z + coef) & ((1u << 30) - 1u);
        } else {
            coef = oracle_exp_neg_q17(sat32((int64_t)run_max - score));
            z = (uint32_t)oracle_rne_shift((int64_t)z * coef, 17) & ((1u << 30) - 1u);
            z = (z + (1u << 17)) & ((1u << 30) - 1u);
            run_max = score;
            rescale = 1;
        }
        const int8_t* v = vc + (size_t)t * HD;
        const uint8_t* vss = vs + (size_t)t * NGROUPS;
        for (int d = 0; d < HD; ++d) {
            int32_t val = (int32_t)((uint32_t)(int32_t)v[d] << vss[d / G32]);
            if (t == 0) y[d] = val;
            else if (rescale) y[d] = sat32((int64_t)mulq17_wrap(y[d], coef) + val);
            else y[d] = sat32((int64_t)y[d] + mulq17_wrap(val, coef));
        }
    }
    /* 18-bit quotient floor((2^34 + z/2) / z) (cpp:271-300). */
    uint32_t inv = 0;
    if (z != 0) {
        uint64_t qt = ((1ull << 34) + (z >> 1)) / z;
        inv = (uint32_t)(qt & 0x3ffffu);
    } else {
        inv = 0x3ffffu;
    }
    for (int d = 0; d < HD; ++d) out[d] = mulq17_wrap(y[d], inv);
}

/* ------------------------------------------------------------------------ */
/* A14 / E8M0 epilogue (cpp:1715-1771, 2656-2682; emulator:690-711).          */
/* Values are float; int path passes raw*2^-17.  Per 32 values:               */
/* e = frexp exponent of max|x|, at least -127;                               */
/* q = trunc(clamp(x*2^(13-e) +- 0.5, +-8191));                               */
/* code = e + 127, or 0 when the group is all zero.                           */
/* ------------------------------------------------------------------------ */
void oracle_a14_group(const float* x, int16_t* q14, uint8_t* code) {
    float mx = 0.0f;
    for (int i = 0; i < G32; ++i) {
        float a = fabsf(x[i]);
        if (a > mx) mx = a;
    }
    if (mx == 0.0f) {
        for (int i = 0; i < G32; ++i) q14[i] = 0;
        *code = 0;
        return;
    }
    int e;
    frexpf(mx, &e);
    if (e < -127) e = -127; /* cpp:1722-1724 */
    for (int i = 0; i < G32; ++i) {
        /* x * 2^(13-e) as ldexpf: the same value as the product with the
         * power of two wherever that power is finite, and finite for a group
         * max below 2^-115, where 2^(13-e) itself overflows. */
        volatile float r = ldexpf(x[i], 13 - e);
        volatile float rr = r >= 0.0f ? r + 0.5f : r - 0.5f;
        float c = rr;
        if (c > 8191.0f) c = 8191.0f;
        if (c < -8191.0f) c = -8191.0f;
        q14[i] = (int16_t)c;
    }
    *code = (uint8_t)(e + 127);
}

/* Integer-path variant: group max on raw magnitudes (INT32_MIN -> INT32_MAX),
 * converted once to float (emulator:690-700, cpp:1694-1705). */
void oracle_a14_group_q17(const int32_t* raw, int16_t* q14, uint8_t* code) {
    int32_t mraw = 0;
    for (int i = 0; i < G32; ++i) {
        int32_t a = raw[i] == INT32_MIN ? INT32_MAX : (raw[i] < 0 ? -raw[i] : raw[i]);
        if (a > mraw) mraw = a;
    }
    float mx = (float)mraw * (1.0f / 131072.0f);
    if (mx == 0.0f) {
        for (int i = 0; i < G32; ++i) q14[i] = 0;
        *code = 0;
        return;
    }
    int e;
    frexpf(mx, &e);
    float inv = ldexpf(1.0f, 13 - e);
    for (int i = 0; i < G32; ++i) {
        volatile float v = (float)raw[i] * (1.0f / 131072.0f);
        volatile float r = v * inv;
        volatile float rr = r >= 0.0f ? r + 0.5f : r - 0.5f;
        float c = rr;
        if (c > 8191.0f) c = 8191.0f;
        if (c < -8191.0f) c = -8191.0f;
        q14[i] = (int16_t)c;
    }
    *code = (uint8_t)(e + 127);
}

/* Pack 32 int14 lanes into the 448-bit activation word, lane 0 at bits
 * [13:0] (cpp:1761-1768), as 56 little-endian bytes. */
void oracle_pack_a14(const int16_t* q14, uint8_t* word56) {
    memset(word56, 0, 56);
    for (int i = 0; i < G32; ++i) put_bits(word56, 14 * i, 14, (uint32_t)(uint16_t)q14[i] & 0x3fffu);
}

/* ------------------------------------------------------------------------ */
/* a14: the FP32 formula the GPU path implements (emulator:1164-1194,        */
/* run_autoround.cpp:232-270), evaluated in double over the dequantized       */
/* cache: q^ = q_raw*2^-17, k^ = code*2^(s-17), score = (q^.k^)/sqrtf(128),   */
/* two-pass softmax, out = sum p v^.                                         */
/* ------------------------------------------------------------------------ */
void oracle_attend_head_fp(const int32_t* q, const int8_t* kc, const uint8_t* ks,
                           const int8_t* vc, const uint8_t* vs, int ntok, double* out) {
    const double scale = (double)(1.0f / sqrtf(128.0f));
    double qf[HD];
    for (int d = 0; d < HD; ++d) qf[d] = (double)q[d] * (1.0 / 131072.0);
    double* sc = (double*)malloc(sizeof(double) * (size_t)(ntok > 0 ? ntok : 1));
    double mx = -INFINITY;
    for (int t = 0; t < ntok; ++t) {
        const int8_t* k = kc + (size_t)t * HD;
        const uint8_t* kss = ks + (size_t)t * NGROUPS;
        double dot = 0.0;
        for (int g = 0; g < NGROUPS; ++g) {
            double part = 0.0;
            for (int i = 0; i < G32; ++i) part += qf[g * G32 + i] * (double)k[g * G32 + i];
            dot += part * ldexp(1.0, (int)kss[g] - 17);
        }
        sc[t] = dot * scale;
        if (sc[t] > mx) mx = sc[t];
    }
    double sum = 0.0;
    for (int t = 0; t < ntok; ++t) {
        sc[t] = exp(sc[t] - mx);
        sum += sc[t];
    }
    for (int d = 0; d < HD; ++d) out[d] = 0.0;
    for (int t = 0; t < ntok; ++t) {
        const int8_t* v = vc + (size_t)t * HD;
        const uint8_t* vss = vs + (size_t)t * NGROUPS;
        double p = sc[t] / sum;
        for (int d = 0; d < HD; ++d) out[d] += p * (double)v[d] * ldexp(1.0, (int)vss[d / G32] - 17);
    }
    free(sc);
}

/* ------------------------------------------------------------------------ */
/* Whole step for one sequence, all heads (emulator:602-714 with the        */
/* conversion and RoPE of emulator:753-760 in front).  Inputs are Q15.17    */
/* q/k/v [heads*128]; the cache arrays are per head [heads][cap][128] codes */
/* and [heads][cap][4] shifts and are updated in place at `pos`.            */
/* fp_out (nullable) gets the double FP32-path result, int_out (nullable)   */
/* the integer recurrence result.                                           */
/* ------------------------------------------------------------------------ */
void oracle_step_q17(int heads, int cap, const int32_t* q, const int32_t* k, const int32_t* v,
                     const int32_t* cos64, const int32_t* sin64, int pos,
                     int8_t* kcache, uint8_t* kshift, int8_t* vcache, uint8_t* vshift,
                     int32_t* qrot_out, double* fp_out, int32_t* int_out) {
    for (int h = 0; h < heads; ++h) {
        int32_t qr[HD], kr[HD];
        memcpy(qr, q + (size_t)h * HD, sizeof(qr));
        memcpy(kr, k + (size_t)h * HD, sizeof(kr));
        oracle_rope_rotate(qr, cos64, sin64);
        oracle_rope_rotate(kr, cos64, sin64);
        if (qrot_out) memcpy(qrot_out + (size_t)h * HD, qr, sizeof(qr));
        size_t row = (size_t)h * cap + (size_t)pos;
        oracle_quantize_row(kr, kcache + row * HD, kshift + row * NGROUPS);
        oracle_quantize_row(v + (size_t)h * HD, vcache + row * HD, vshift + row * NGROUPS);
        const int8_t* kc = kcache + (size_t)h * cap * HD;
        const int8_t* vc = vcache + (size_t)h * cap * HD;
        const uint8_t* ks = kshift + (size_t)h * cap * NGROUPS;
        const uint8_t* vs = vshift + (size_t)h * cap * NGROUPS;
        if (fp_out) oracle_attend_head_fp(qr, kc, ks, vc, vs, pos + 1, fp_out + (size_t)h * HD);
        if (int_out) oracle_attend_head_int(qr, kc, ks, vc, vs, pos + 1, int_out + (size_t)h * HD);
    }
}

/* Prefill: apply the append rule (RoPE of k at each position, G32 quantize)
 * for tokens [pos0, pos0+n) of one sequence.  k/v are Q15.17 [n][heads*128]. */
void oracle_fill_q17(int heads, int cap, int n, int pos0, const int32_t* k, const int32_t* v,
                     const int32_t* cos_tab, const int32_t* sin_tab,
                     int8_t* kcache, uint8_t* kshift, int8_t* vcache, uint8_t* vshift) {
    for (int t = 0; t < n; ++t) {
        int pos = pos0 + t;
        for (int h = 0; h < heads; ++h) {
            int32_t kr[HD];
            memcpy(kr, k + ((size_t)t * heads + h) * HD, sizeof(kr));
            oracle_rope_rotate(kr, cos_tab + (size_t)pos * PAIRS, sin_tab + (size_t)pos * PAIRS);
            size_t row = (size_t)h * cap + (size_t)pos;
            oracle_quantize_row(kr, kcache + row * HD, kshift + row * NGROUPS);
            oracle_quantize_row(v + ((size_t)t * heads + h) * HD, vcache + row * HD, vshift + row * NGROUPS);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* The reference's known-answer test (_rtl_check/linear_4pe_reduction_cosim/ */
/* tb_attention_pe0_kv_rtl.cpp:21-58, 79-110): PE0 = heads 0..7, layer 0,    */
/* q/k/v from the deterministic generator, positions 0 then 1 on the same    */
/* cache, output = FNV-style hash over the 32 packed A14 words and E8M0       */
/* bytes.  cos_tab/sin_tab hold at least positions 0 and 1.                  */
/* ------------------------------------------------------------------------ */
static void kat_vector(unsigned seed, int32_t* out1024) {
    for (int i = 0; i < 1024; ++i) {
        uint32_t raw = ((uint32_t)i * (37u + seed) + seed * 101u) % 458753u;
        out1024[i] = (int32_t)raw - 229376;
    }
}

static uint64_t kat_hash(const uint8_t* words /*32 x 56*/, const uint8_t* codes /*32*/) {
    uint64_t h = 1469598103934665603ull;
    for (int g = 0; g < 32; ++g) {
        for (int c = 0; c < 7; ++c) {
            uint64_t bits;
            memcpy(&bits, words + g * 56 + c * 8, 8);
            h ^= bits;
            h *= 1099511628211ull;
        }
        h ^= codes[g];
        h *= 1099511628211ull;
    }
    return h;
}

void oracle_kat_pe0(const int32_t* cos_tab, const int32_t* sin_tab, uint64_t* hash0, uint64_t* hash1) {
    const int heads = 8, cap = 2;
    int8_t kc[8 * 2 * HD], vc[8 * 2 * HD];
    uint8_t ks[8 * 2 * NGROUPS], vs[8 * 2 * NGROUPS];
    memset(kc, 0, sizeof(kc));
    memset(vc, 0, sizeof(vc));
    memset(ks, 0, sizeof(ks));
    memset(vs, 0, sizeof(vs));
    static const unsigned seeds[2][3] = {{3, 11, 29}, {43, 61, 79}};
    for (int pos = 0; pos < 2; ++pos) {
        int32_t q[1024], k[1024], v[1024], o[1024];
        kat_vector(seeds[pos][0], q);
        kat_vector(seeds[pos][1], k);
        kat_vector(seeds[pos][2], v);
        oracle_step_q17(heads, cap, q, k, v, cos_tab + pos * PAIRS, sin_tab + pos * PAIRS, pos,
                        kc, ks, vc, vs, NULL, NULL, o);
        uint8_t words[32 * 56], codes[32];
        for (int g = 0; g < 32; ++g) {
            int16_t q14[32];
            oracle_a14_group_q17(o + g * 32, q14, &codes[g]);
            oracle_pack_a14(q14, words + g * 56);
        }
        uint64_t hv = kat_hash(words, codes);
        if (pos == 0) *hash0 = hv;
        else *hash1 = hv;
    }
}
