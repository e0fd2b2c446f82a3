// swiftkv_exact.hip -- integer-compatibility step: the reference's Q15.17
// single-pass recurrence evaluated exactly on the GPU, so the A14 words and
// E8M0 codes equal the reference's bit for bit (swiftkv_attention.cpp:934-1880;
// llama2_decoder_sw_emulator.cpp:633-711).  Slow by construction -- the
// (max, Z, Y) recurrence is sequential per head -- and meant for bit-level
// comparison with the FPGA / C model; the sequential chains bound it, not HBM.
//
// Grid (32 heads x SLICES, batch rows), 256 threads per (sequence, head,
// slice of 128 / SLICES channels); SLICES is 4 for the smallest batches, 2
// up to batch 8 and 1 otherwise.  Wave 0 first appends the new row like the fast step; then
// tokens [0, position] are processed in chunks of kChunk:
//   - the 4 waves issue all of the chunk's loads at once through one buffer
//     resource (K codes and scales into registers, V codes straight into
//     LDS), then compute the integer
//     scores (lane = 16-channel half-group c of token row r; the per-half
//     shift and the 44-bit wraps are associative modulo 2^44, so the octet
//     sum may run in any order), the exact 64-bit dot taken as signed-byte
//     dot products over five limbs of the query;
//   - one thread per token turns its score and the exclusive prefix maximum
//     into a coefficient word (exp LUT, rescale flag), and the same pass lays
//     out, per group, the product of the coefficient and the V scale (exact
//     in FP32), the per-wave coefficient sums and ballots for Z and Y;
//   - Y, one channel per thread: the first kCh threads run the chunk's
//     first part in token order, adding independently formed terms, while
//     the rest of the threads compose the remaining tokens (no first or
//     rescaling token among them) into clamp-add maps applied after the
//     barrier; a term is one fused multiply-add of the code and the product
//     when the shift is at most 15, an exact FP32 product and rint at 16,
//     32-bit integer operations above; wave 3 also advances Z by prefix-sum
//     differences and steps only at first and rescaling tokens;
// then Y * 1/Z and the integer-path A14/E8M0 epilogue.
#include <type_traits>

#include "swiftkv_device.hpp"

namespace swiftkv {
namespace {

using namespace dev;

constexpr int kChunk = 256;                   // cached tokens per chunk (V codes staged in LDS)
constexpr int kBatch = 8;                     // tokens whose LDS reads go out together in the Y pass
static_assert(kChunk % kBatch == 0, "batches tile a chunk");
static_assert(kBatch % 4 == 0 && 64 % kBatch == 0, "a batch is whole 16-byte reads inside one 64-token ballot");
constexpr int kPasses = kChunk / 32;          // score passes per chunk: 4 waves x 8 token rows each
// Largest batch whose launch splits each head's Y over 4 workgroups (32
// channels each): at context 4096 this took batch 1 and 2 from 175 to 147-150
// us, was even at batch 4 and slower from batch 8 on, where one workgroup per
// head already fills the machine and the 4x score work shows.
constexpr int kExactSlicedMaxBatch = 2;
// Largest batch whose launch splits each head's Y over 2 workgroups (64
// channels each): batch 3 and 4 ran 16-21% faster than with one workgroup
// per head (whose 128 workgroups leave half the CUs idle), batch 6 and 8 up
// to 6%; from batch 12 on the doubled score work made it slower.
constexpr int kExactHalfSlicedMaxBatch = 8;
constexpr int64_t kScoreScaleQ17 = 11585;     // RNE(2^17 / sqrt(128)) (swiftkv_attention.cpp:1101-1102)
constexpr int64_t kLog2eQ21 = 3025551;        // RNE(log2(e) * 2^21) (cpp:207-208)

__device__ __forceinline__ int64_t wrap_bits(int64_t x, int bits) {
    const uint64_t mask = (1ull << bits) - 1u;
    uint64_t r = static_cast<uint64_t>(x) & mask;
    if ((r >> (bits - 1)) & 1u) r |= ~mask;
    return static_cast<int64_t>(r);
}

// Round-half-even of x / 2^s (AP_RND_CONV), 1 <= s <= 31.  With q =
// floor(x / 2^s) and r = x - q 2^s: r < 2^(s-1) gives q, r > 2^(s-1) gives
// q + 1, and the tie gives q + (q & 1) -- all three are floor((x + 2^(s-1) - 1
// + (q & 1)) / 2^s), for either sign of x.  RNE of the exact quotient is odd-
// symmetric, so this equals rounding the magnitude and restoring the sign.
__device__ __forceinline__ int64_t rne_shift(int64_t x, int s) {
    return (x + ((int64_t{1} << (s - 1)) - 1) + ((x >> s) & 1)) >> s;
}

// Q15.17 x unsigned Q1.17 multiplier, RNE >> 17, wrapped to 32 bits.
__device__ __forceinline__ int32_t mulq17_wrap(int32_t a, uint32_t b) {
    return static_cast<int32_t>(static_cast<uint32_t>(
        rne_shift(static_cast<int64_t>(a) * static_cast<int64_t>(b), 17)));   // low 32 bits = the wrap
}

// exp(x) for x <= 0 in Q1.17 through the 33-entry Q30 exp2 table with 12-bit
// linear interpolation (swiftkv_attention.cpp:185-260).
__device__ __forceinline__ uint32_t exp_neg_q17(int32_t x, const uint32_t* lut) {
    if (x >= 0) return 1u << 17;
    if (x <= -(32 << 17)) return 0u;
    const int64_t l = wrap_bits(rne_shift(static_cast<int64_t>(x) * kLog2eQ21, 21), 24);
    const int64_t ex = l >> 17;
    const uint32_t f = static_cast<uint32_t>(l - (ex << 17));
    const uint32_t idx = f >> 12, rm = f & 0xfffu;
    const uint32_t base = lut[idx], next = lut[idx + 1];
    const uint32_t interp = base + static_cast<uint32_t>((static_cast<uint64_t>(next - base) * rm + (1u << 11)) >> 12);
    const int sh = 13 - static_cast<int>(ex);
    uint64_t out = 0;
    if (sh <= 0) out = static_cast<uint64_t>(interp) << (-sh);
    else if (sh < 32) out = (static_cast<uint64_t>(interp) + (1ull << (sh - 1))) >> sh;
    return static_cast<uint32_t>(out) & 0x3ffffu;
}

// The 16 rotated query channels of one half-group as five planes of signed
// bytes, four channels per word: q = l0 + l1 2^8 + l2 2^16 + l3 2^24 + l4 2^32,
// each limb the signed low byte of what the limbs below it leave, so every
// limb lies in [-128, 127] and the top one in {-1, 0, 1} for any int32 q.
struct QueryLimbs {
    int32_t w[5][4];
};

__device__ __forceinline__ QueryLimbs split_query(const int32_t* q) {
    QueryLimbs L;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t packed[5] = {0u, 0u, 0u, 0u, 0u};
#pragma unroll
        for (int byte = 0; byte < 4; ++byte) {
            int64_t rest = q[4 * j + byte];
#pragma unroll
            for (int k = 0; k < 5; ++k) {
                const int32_t limb = static_cast<int8_t>(static_cast<uint8_t>(rest));
                packed[k] |= static_cast<uint32_t>(static_cast<uint8_t>(limb)) << (8 * byte);
                rest = (rest - limb) >> 8;
            }
        }
#pragma unroll
        for (int k = 0; k < 5; ++k) L.w[k][j] = static_cast<int32_t>(packed[k]);
    }
    return L;
}

// 44-bit token dot contribution of one 16-channel half-group: the 16 int8
// codes times the int32 rotated query, scaled by 2^(shift-10) (cpp:934-995).
// The exact sum is taken limb by limb: four signed-byte dot products per limb
// (each limb's sum stays within 16 * 128 * 128 = 2^18), then combined in 64
// bits, so it equals the sum of the 16 full products.
// NL = 3 when the wave's query limbs 3 and 4 are all zero (|q| below about
// 2^23, i.e. |q| < 64.0, the common case): those limbs add nothing.
template <int NL>
__device__ __forceinline__ int64_t half_dot(const QueryLimbs& L, int4 w, uint32_t shift) {
    const int32_t d[4] = {w.x, w.y, w.z, w.w};
    int64_t s = 0;
#pragma unroll
    for (int k = NL - 1; k >= 0; --k) {
        int32_t acc = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_sdot4(L.w[k][j], d[j], acc, false);
        s = s * 256 + acc;
    }
    const int64_t p = shift >= 10 ? static_cast<int64_t>(static_cast<uint64_t>(s) << (shift - 10))
                                  : (s >> (10 - shift));
    return wrap_bits(p, 44);
}

__device__ __forceinline__ int32_t score_of(int64_t token_dot) {
    return sat32(rne_shift(wrap_bits(token_dot, 44) * kScoreScaleQ17, 24));
}

__device__ __forceinline__ uint32_t shift_of(float scale) { return (__float_as_uint(scale) >> 23) - 110u; }

// The single-pass recurrence (cpp:1276-1335, 1463-1558) in three parts.
// The running maximum before token i is the prefix maximum of the scores
// (the reference raises it only on a strictly larger score, and a maximum
// does not depend on order), so every token's coefficient and rescale flag
// follow from its score and that prefix maximum, for all tokens of a chunk at
// once.  What stays sequential is Z at first and rescaling tokens, and Y.
constexpr uint32_t kInit = 1u << 31;      // first token of the sequence: Y = v, Z = 1
constexpr uint32_t kRescale = 1u << 30;   // new maximum: Y = Y * coef + v, Z = Z * coef + 1
constexpr uint32_t kCoefMask = (1u << 18) - 1u;
constexpr uint32_t kMask30 = (1u << 30) - 1u;

// Coefficient word of a token with score s and prefix maximum `before`.
__device__ __forceinline__ uint32_t coef_word(int32_t s, int32_t before, const uint32_t* lut) {
    if (s <= before) return exp_neg_q17(sat32(static_cast<int64_t>(s) - before), lut);
    return exp_neg_q17(sat32(static_cast<int64_t>(before) - s), lut) | kRescale;
}

// Z in Q13.17, wrapped to 30 bits.
__device__ __forceinline__ uint32_t z_step(uint32_t z, uint32_t word) {
    if (word & kInit) return 1u << 17;
    const uint32_t coef = word & kCoefMask;
    if (word & kRescale)
        return ((static_cast<uint32_t>(rne_shift(static_cast<int64_t>(z) * coef, 17)) & kMask30) + (1u << 17)) &
               kMask30;
    return (z + coef) & kMask30;
}

// Y per token and channel (cpp:1463-1558):
//   first token  Y = v
//   no rescale   Y = sat32(Y + wrap32(RNE(v c >> 17)))
//   rescale      Y = sat32(wrap32(RNE(Y c >> 17)) + v)
// with v = code << shift as the reference's ap_int<32> (it wraps for code 64,
// shift 25).  The no-rescale term does not depend on Y, so the terms of a
// batch of tokens are formed independently and only the saturating adds run
// in series.  The term in 32-bit operations, c < 2^18 and |code| <= 128:
//   shift >= 17: v is a multiple of 2^17, so the quotient is exact and equals
//                (v >> 17) c, with |v >> 17| <= 2^14 -- the low 32 bits of a
//                24-bit product are the wrap;
//   shift < 17:  v c = (code c) 2^shift exactly, |code c| < 2^25, so the term
//                is RNE((code c) / 2^k) for k = 17 - shift in 1..17, in the
//                floor((x + 2^(k-1) - 1 + bit k of x) >> k) form of rne_shift.
__device__ __forceinline__ int32_t dequant_raw(int32_t code, uint32_t shift) {
    return static_cast<int32_t>(static_cast<uint32_t>(code) << shift);
}

// Both cases in one form: x = v >> min(shift, 17) is the code itself below
// 17 and v >> 17 above, m = x c, and the rounding shift k = 17 - shift
// clamps to 0 above 17, where the rounding terms (2^(16-shift) - 1 and a
// zero-width bit field) vanish and the term is m.
__device__ __forceinline__ int32_t value_term(int32_t code, uint32_t shift, uint32_t coef) {
    const int32_t m = __mul24(dequant_raw(code, shift) >> min(shift, 17u), static_cast<int32_t>(coef));
    const uint32_t k = __builtin_elementwise_sub_sat(17u, shift);
    const int32_t bit = static_cast<int32_t>(__builtin_amdgcn_ubfe(static_cast<uint32_t>(m), k, min(k, 1u)));
    return (m + static_cast<int32_t>(0xffffu >> shift) + bit) >> k;
}

__device__ __forceinline__ int32_t value_step(int32_t y, uint32_t word, int32_t code, uint32_t shift, int32_t term) {
    if (word & kInit) return dequant_raw(code, shift);
    if (word & kRescale) return __builtin_elementwise_add_sat(mulq17_wrap(y, word & kCoefMask), dequant_raw(code, shift));
    return __builtin_elementwise_add_sat(y, term);
}


// Sum over the 8 lanes of an aligned octet of a 64-bit integer (DPP moves of
// both halves, integer adds, so exact in any order); every lane gets it.
template <int Ctrl>
__device__ __forceinline__ int64_t dpp64(int64_t x) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), Ctrl, 0xF, 0xF, true));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x >> 32), Ctrl, 0xF, 0xF, true));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ int64_t octet_sum64(int64_t x) {
    x += dpp64<kDppQuadXor1>(x);
    x += dpp64<kDppQuadXor2>(x);
    return x + dpp64<kDppHalfMirror>(x);
}

// Inclusive wave scans with DPP (GFX9): row shifts by 1, 2, 4, 8 scan each
// 16-lane row, then row 0's last lane is broadcast into row 1 and row 2's
// into row 3, then lane 31 into rows 2 and 3.  Lanes a move cannot reach, and
// rows outside its row mask, take the identity.
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143, kDppWaveShr1 = 0x138;

template <int Ctrl, int RowMask>
__device__ __forceinline__ int32_t dpp_shifted(int32_t identity, int32_t x) {
    return __builtin_amdgcn_update_dpp(identity, x, Ctrl, RowMask, 0xF, false);
}

__device__ __forceinline__ int32_t wave_scan_max(int32_t x) {
    x = max(x, dpp_shifted<kDppRowShr1, 0xF>(INT32_MIN, x));
    x = max(x, dpp_shifted<kDppRowShr2, 0xF>(INT32_MIN, x));
    x = max(x, dpp_shifted<kDppRowShr4, 0xF>(INT32_MIN, x));
    x = max(x, dpp_shifted<kDppRowShr8, 0xF>(INT32_MIN, x));
    x = max(x, dpp_shifted<kDppRowBcast15, 0xA>(INT32_MIN, x));
    return max(x, dpp_shifted<kDppRowBcast31, 0xC>(INT32_MIN, x));
}

__device__ __forceinline__ uint32_t wave_scan_add(uint32_t v) {
    int32_t x = static_cast<int32_t>(v);
    x += dpp_shifted<kDppRowShr1, 0xF>(0, x);
    x += dpp_shifted<kDppRowShr2, 0xF>(0, x);
    x += dpp_shifted<kDppRowShr4, 0xF>(0, x);
    x += dpp_shifted<kDppRowShr8, 0xF>(0, x);
    x += dpp_shifted<kDppRowBcast15, 0xA>(0, x);
    return static_cast<uint32_t>(x + dpp_shifted<kDppRowBcast31, 0xC>(0, x));
}

// A wave-uniform 64-bit value read by every lane, moved to scalar registers.
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    return (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32))))
            << 32) |
           static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

// The Y pass reads, per token and G32 group, the product p = c 2^(s-17) of
// the token's coefficient c (an integer, at most 2^17) and the group's V
// scale 2^(s-17); the FP32 product is exact.  The no-rescale term is then
// RNE(code p), since v c 2^-17 = (code 2^s) c 2^-17 for a shift below 17.
//
// Shift at most 15 (V groups below 32.0, the common case): |code p| <= 128
// 2^15 = 2^22, so code p + 1.5 2^23 lies in [2^23, 2^24), where the floats
// are the integers.  One fused multiply-add rounds the exact sum once, to
// nearest even, and 1.5 2^23 is an even integer, so the result is 1.5 2^23 +
// RNE(code p) and its bit pattern is 0x4b400000 + RNE(code p).
constexpr float kRoundMagic = 12582912.0f;   // 1.5 * 2^23
constexpr uint32_t kRoundMagicBits = 0x4b400000u;
__device__ __forceinline__ uint32_t term_bits(int32_t code, float p) {
    return __float_as_uint(__builtin_fmaf(static_cast<float>(code), p, kRoundMagic));
}
// A term of that form is at most 2^22 in magnitude.
constexpr int64_t kFastTermBound = int64_t{1} << 22;

// The codes and Y terms of tokens [i0, i0 + kBatch) for channel ch, for any
// shift: the coefficient words come from 16-byte reads, the products p of the
// channel's group from 16-byte reads, the codes from one byte read per token.
// A first or rescaling token's p is its V scale alone (its term is not used).
// wide17: some token of the batch has a shift of 17 or more.  Otherwise every
// |code c| <= 2^24 is exact in FP32, so code p is exact and rint gives RNE
// (the short form, returns true); else the shift is recovered from the
// exponents of p and c and the 32-bit integer form runs (returns false).
__device__ __forceinline__ bool slow_terms(const uint32_t* s_words, const float* s_p_g,
                                           const int8_t (*s_vc)[kHeadDim], int i0, int ch, bool wide17,
                                           int32_t* code, float* p, int32_t* term) {
    uint32_t coef[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch / 4; ++q) {
        const uint4 cq = *reinterpret_cast<const uint4*>(&s_words[i0 + 4 * q]);
        const float4 pq = *reinterpret_cast<const float4*>(&s_p_g[i0 + 4 * q]);
        coef[4 * q] = cq.x & kCoefMask;
        coef[4 * q + 1] = cq.y & kCoefMask;
        coef[4 * q + 2] = cq.z & kCoefMask;
        coef[4 * q + 3] = cq.w & kCoefMask;
        p[4 * q] = pq.x;
        p[4 * q + 1] = pq.y;
        p[4 * q + 2] = pq.z;
        p[4 * q + 3] = pq.w;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) code[j] = s_vc[i0 + j][ch];
    if (!wide17) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) term[j] = static_cast<int32_t>(__builtin_rintf(static_cast<float>(code[j]) * p[j]));
        return true;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
        // p = c 2^(s-17) exactly, so s = 17 + exponent(p) - exponent(c); a
        // zero coefficient gives a zero term for any shift.
        const uint32_t sh = coef[j] == 0u ? 0u
                                          : min(17u + shift_of(p[j]) - shift_of(static_cast<float>(coef[j])), 25u);
        term[j] = value_term(code[j], sh, coef[j]);
    }
    return false;
}
// A short-form term is at most 128 2^16 = 2^23 in magnitude.
constexpr int64_t kShortTermBound = int64_t{1} << 23;

// What the fused-multiply-add terms of tokens [i0, i0 + kBatch) for channel
// ch read: the products p of the channel's group and the codes.
struct FastBatch {
    float p[kBatch];
    int32_t code[kBatch];
};
__device__ __forceinline__ FastBatch load_fast(const float* s_p_g, const int8_t (*s_vc)[kHeadDim], int i0, int ch) {
    FastBatch f;
#pragma unroll
    for (int q = 0; q < kBatch / 4; ++q) {
        const float4 pq = *reinterpret_cast<const float4*>(&s_p_g[i0 + 4 * q]);
        f.p[4 * q] = pq.x;
        f.p[4 * q + 1] = pq.y;
        f.p[4 * q + 2] = pq.z;
        f.p[4 * q + 3] = pq.w;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) f.code[j] = s_vc[i0 + j][ch];
    return f;
}
// The term bits 0x4b400000 + term of such a batch, every shift at most 15.
__device__ __forceinline__ void fast_term_bits(const FastBatch& f, uint32_t* tb) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) tb[j] = term_bits(f.code[j], f.p[j]);
}
constexpr uint64_t kBatchMask = (uint64_t{1} << kBatch) - 1u;
// No partial sum of a batch of fused-multiply-add terms exceeds this.
constexpr uint32_t kSatMargin = static_cast<uint32_t>(kBatch * kFastTermBound);

// The per-group products p of a chunk and the query's LDS bytes: shared
// with one workgroup per head (where LDS bounds the residency: four
// workgroups per CU), separate with four (three per CU by registers).
template <int G, int CH>
union ProductsOrQuery {
    float p[G][kChunk];
    int32_t q[kHeadDim];
    int16_t q14[CH];
};
template <int G, int CH>
struct ProductsAndQuery {
    float p[G][kChunk];
    int32_t q[kHeadDim];
    int16_t q14[CH];
};

struct ExactArgs {
    StepArgs step;
    uint32_t exp_lut[33];     // RNE(2^(30 + i/32)), i = 0..32 (cpp:185-195)
};

// SLICES workgroups share a (sequence, head): each runs the whole token loop
// (scores, coefficients, Z) but Y for kHeadDim / SLICES channels only, so a
// small batch spreads over more CUs.  All of them append the new row; they
// write the same bytes.
template <bool Q17, int SLICES>
__global__ __launch_bounds__(256) void exact_kernel(ExactArgs ea) {
    static_assert(SLICES == 1 || SLICES == 2 || SLICES == 4, "128, 64 or 32 channels per workgroup");
    // Y roles: threads [0, kCh) run the ordered part (one channel each),
    // threads [kSeqLanes, 256) compose kCompParts parts of kCh channels,
    // threads in between (wave 0's upper half when kCh = 32) idle.
    constexpr int kCh = kHeadDim / SLICES;
    constexpr int kSeqLanes = kCh < 64 ? 64 : kCh;
    constexpr int kCompParts = (256 - kSeqLanes) / kCh;
    constexpr int kGroups = kCh / 32;   // G32 groups of this workgroup's channels
    constexpr bool kPrefetchY = SLICES == 4;   // the Y pass reads a batch ahead (registers allow it)
    // The ordered part's share of a chunk, measured: 8/16 with one composed
    // part (9/16 and 10/16 ran up to 3% slower at batch 16), 2/16 with six
    // (3/16 ran 7% slower at batch 1; the composed runs round up to whole
    // batches).
    constexpr int kSeqShare16 = kCompParts == 1 ? 8 : kCompParts == 3 ? 4 : 2;
    // The longest composed run (the rest of a chunk after the ordered share,
    // split into kCompParts runs of whole batches): its short-form terms, and
    // its prefix sums of fused-multiply-add terms, stay within int32.
    constexpr int kMaxRun =
        ((kChunk * (16 - kSeqShare16) / 16 + kCompParts - 1) / kCompParts + kBatch - 1) / kBatch * kBatch;
    static_assert(kMaxRun * kShortTermBound < (int64_t(1) << 31), "short-form sums of a run fit in 32 bits");
    static_assert(2 * kMaxRun * kFastTermBound < (int64_t(1) << 31), "a run's prefix-sum range fits in 32 bits");
    const StepArgs& a = ea.step;
    const uint32_t row = a.rows[blockIdx.y];
    const int h = blockIdx.x / SLICES, slice = blockIdx.x % SLICES, b = static_cast<int>(row & 0xffu);
    const int pos = static_cast<int>(row >> 8);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int c = lane & 7, r = lane >> 3;
    const int d = threadIdx.x;                  // token of the chunk (coefficients), channel (Y, d < 128)
    int8_t* page = page_ptr(a.kv, a.slot0 + b, a.layer, h);
    const int64_t cap = a.kv.seq_cap;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        page, static_cast<short>(0), static_cast<int32_t>(cap * kTokenBytes), kBufferWord3);

    // Per token of the chunk: the score, then (each thread rewrites its own
    // token after reading it) the coefficient word, zero past n.
    __shared__ __align__(16) uint32_t s_tok[kChunk];
    __shared__ int8_t s_vc[kChunk][kHeadDim];            // V codes of the chunk
    // Per group of this workgroup's channels and token of the chunk: the V
    // scale (the score pass), then the product p = c 2^(s-17) for ordinary
    // tokens (the coefficient pass).  The rotated query before the token loop
    // and the A14 codes after it use the same bytes.
    __shared__ __align__(16) std::conditional_t<SLICES == 1, ProductsOrQuery<kGroups, kCh>, ProductsAndQuery<kGroups, kCh>>
        s_u;
    __shared__ int32_t s_wave_max[kChunk / 64];
    __shared__ uint32_t s_wave_sum[kChunk / 64];
    // Per-wave ballots: first and rescaling tokens; those and tokens with a V
    // shift of 16 or more in this workgroup's groups (the slow form); tokens
    // with a shift of 17 or more.
    __shared__ uint64_t s_special[kChunk / 64];
    __shared__ uint64_t s_slow[kChunk / 64];
    __shared__ uint64_t s_wide17[kChunk / 64];
    __shared__ int64_t s_map_sum[kCompParts * kCh];      // the composed maps of the parts after split
    __shared__ int32_t s_map_lo[kCompParts * kCh];
    __shared__ int32_t s_map_hi[kCompParts * kCh];
    __shared__ uint32_t s_lut[33];
    __shared__ uint32_t s_inv;
    int32_t* const s_q = s_u.q;
    int16_t* const s_q14 = s_u.q14;
    if (threadIdx.x < 33) s_lut[threadIdx.x] = ea.exp_lut[threadIdx.x];

    // Wave 0 rotates the query into LDS and appends the new row; the barrier
    // makes the row visible to the workgroup (its waves share one CU), so the
    // token loop below reads tokens [0, pos] uniformly from the cache.
    if (wave == 0) {
        const size_t row_elem = static_cast<size_t>(b) * kModelDim + h * kHeadDim + 2 * lane;
        const int2 cs = a.lut[static_cast<size_t>(pos) * kRopePairs + lane];
        const int2 qi = load_pair<Q17>(a.q, row_elem);
        const int2 ki = load_pair<Q17>(a.k, row_elem);
        const int2 vi = load_pair<Q17>(a.v, row_elem);
        int32_t q0, q1, k0, k1;
        rope_pair(qi.x, qi.y, cs, q0, q1);
        rope_pair(ki.x, ki.y, cs, k0, k1);
        (void)append_row_codes(page, a.kv.seq_cap, pos, lane, k0, k1, vi.x, vi.y);
        s_q[2 * lane] = q0;
        s_q[2 * lane + 1] = q1;
    }
    __syncthreads();
    QueryLimbs ql;
    {
        int32_t qc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) qc[j] = s_q[16 * c + j];
        ql = split_query(qc);
    }
    if constexpr (SLICES == 1) __syncthreads();   // the score pass below writes the query's bytes (s_u)
    // Limbs 3 and 4 zero in every lane of the wave: three-limb dot products.
    // (With four workgroups per head, at batch 1 and 2, the branch measured
    // 1% slower, so those launches keep five.)
    const bool q3 = SLICES == 1 &&
                    __builtin_amdgcn_ballot_w64((ql.w[3][0] | ql.w[3][1] | ql.w[3][2] | ql.w[3][3] | ql.w[4][0] |
                                                 ql.w[4][1] | ql.w[4][2] | ql.w[4][3]) != 0) == 0;

    const int len = pos + 1;
    int32_t run_max = INT32_MIN;   // prefix maximum before the chunk (every thread)
    uint32_t z = 0;                // Z (wave 3, uniform)
    int32_t y = 0;                 // Y of channel slice * kCh + d (threads d < kCh)
    // A chunk's loads, 4 waves x 8 token rows per pass: per lane the K codes
    // and scale pair into registers, and the V codes straight into LDS (lane
    // l of a wave writes bytes [16 l, 16 l + 16) of its 8 rows, which is
    // channel chunk c of row r), all passes at once.  Rows past the chunk's
    // end load its last token (inside the page) and are not used.  The page
    // is read through one buffer resource: per-lane 32-bit offsets within the
    // chunk, the chunk's own offset in an SGPR.
    v4i kq[kPasses];
    v2u scl[kPasses];
    auto issue = [&](int tc, bool with_k, bool with_v) {   // flags are compile-time at every call
        const int nc = min(kChunk, len - tc);
        const int32_t k_chunk = tc * kCodeBytes, v_chunk = static_cast<int32_t>(cap + tc) * kCodeBytes;
        const int32_t s_chunk = static_cast<int32_t>(cap * 2 * kCodeBytes) + tc * kScaleBytes;
#pragma unroll
        for (int ps = 0; ps < kPasses; ++ps) {
            const int32_t tr = min(wave * 8 + r + 32 * ps, nc - 1);
            if (with_k) {
                scl[ps] = __builtin_amdgcn_raw_buffer_load_b64(rsrc, tr * kScaleBytes + (c >> 1) * 8, s_chunk, 0);
                kq[ps] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, tr * kCodeBytes + c * 16, k_chunk, 0);
            }
            if (with_v)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rsrc, (__attribute__((address_space(3))) void*)&s_vc[wave * 8 + 32 * ps][0], 16,
                    tr * kCodeBytes + c * 16, v_chunk, 0, 0);
        }
    };
    // With SLICES = 4 (the smallest batches, where each chunk's load latency
    // is exposed) the next chunk's K codes and scales are loaded while this
    // chunk's coefficient and Y passes run; its V codes, which go to LDS,
    // follow at the top of its own iteration (the barrier after the scores
    // waits for every write into LDS, so they cannot be outstanding there).
    constexpr bool kPrefetch = SLICES > 1;
    if constexpr (kPrefetch) issue(0, true, false);
    for (int t0 = 0; t0 < len; t0 += kChunk) {
        const int n = min(kChunk, len - t0);
        issue(t0, !kPrefetch, true);
        // Scores of tokens [t0, t0+n).  Every lane of an octet ends a pass
        // with its token's sum; lane c keeps pass c's, so each lane scales,
        // rounds and saturates one sum per chunk.
        static_assert(kPasses == 8, "one pass per lane of an octet");
        int64_t own = 0;
#pragma unroll
        for (int ps = 0; ps < kPasses; ++ps) {
            const int i = wave * 8 + r + 32 * ps;
            const int4 kw = make_int4(kq[ps].x, kq[ps].y, kq[ps].z, kq[ps].w);
            // the token's sum of its 8 half-groups (lanes 8r .. 8r+7), exact
            const uint32_t ksh = shift_of(__uint_as_float(scl[ps].x));
            const int64_t p = octet_sum64(q3 ? half_dot<3>(ql, kw, ksh) : half_dot<5>(ql, kw, ksh));
            if (c == ps) own = p;
            // the V scale of group c / 2, its exponent alone (the stored
            // scales are powers of two); slots past n take the scale of shift
            // 0 and are read by the Y pass with a zero coefficient
            if ((c & 1) == 0 && (c >> 1) / kGroups == slice)
                s_u.p[(c >> 1) % kGroups][i] =
                    __uint_as_float(i < n ? scl[ps].y & 0x7f800000u : 110u << 23);
        }
        {
            const int i = wave * 8 + r + 32 * c;   // the token of pass c
            if (i < n) s_tok[i] = static_cast<uint32_t>(score_of(own));
        }
        __builtin_amdgcn_s_waitcnt(0);   // the V codes are in LDS before the barrier
        if constexpr (kPrefetch)
            if (t0 + kChunk < len) issue(t0 + kChunk, true, false);
        __syncthreads();

        // Coefficient words, one token per thread: the exclusive prefix
        // maximum (wave scan, then the maxima of the waves before) gives each
        // token's running maximum.  The same pass lays out what Y and Z read:
        // the coefficient words, the products p of the coefficient and each
        // group's V scale (the scale alone for first and rescaling tokens),
        // the per-wave sums of the coefficients of ordinary tokens, and the
        // per-wave ballots.
        const int32_t sv = d < n ? static_cast<int32_t>(s_tok[d]) : INT32_MIN;
        float sc[kGroups];   // the token's V scales, read with its score
#pragma unroll
        for (int gl = 0; gl < kGroups; ++gl) sc[gl] = s_u.p[gl][d];
        const int32_t incl = wave_scan_max(sv);
        if (lane == 63) s_wave_max[wave] = incl;
        int32_t excl = dpp_shifted<kDppWaveShr1, 0xF>(INT32_MIN, incl);
        __syncthreads();
        int32_t before = run_max;
        for (int w = 0; w < wave; ++w) before = max(before, s_wave_max[w]);
        excl = lane == 0 ? before : max(before, excl);
        const uint32_t word = d >= n ? 0u : (t0 == 0 && d == 0) ? kInit : coef_word(sv, excl, s_lut);
        const bool special = (word & (kInit | kRescale)) != 0u;
        const uint32_t psum = wave_scan_add(special ? 0u : (word & kCoefMask));
        const uint64_t special_mask = __ballot(special);
        const float cf = static_cast<float>(word & kCoefMask);
        bool wide16 = false, wide17 = false;   // a V shift of 16 (scale 2^-1) or more, of 17 (2^0) or more
#pragma unroll
        for (int gl = 0; gl < kGroups; ++gl) {
            wide16 |= sc[gl] >= 0.5f;
            wide17 |= sc[gl] >= 1.0f;
            s_u.p[gl][d] = special ? sc[gl] : cf * sc[gl];   // exact: an integer below 2^18 times a power of two
        }
        const uint64_t slow_mask = __ballot(special || wide16), wide17_mask = __ballot(wide17);
        s_tok[d] = word;
        if (lane == 63) s_wave_sum[wave] = psum;
        if (lane == 0) {
            s_special[wave] = special_mask;
            s_slow[wave] = slow_mask;
            s_wide17[wave] = wide17_mask;
        }
#pragma unroll
        for (int w = 0; w < kChunk / 64; ++w) run_max = max(run_max, s_wave_max[w]);
        __syncthreads();

        // Y in parts at once.  Threads [0, kCh) (one channel each) run
        // tokens [0, split) in order; the composing threads split [split, n)
        // into kCompParts runs of q tokens and compose each run into one map
        // Y -> clamp(Y + A, L, H) (every ordinary token is Y -> sat32(Y + t),
        // and such maps compose: A adds t, L and H take sat32(. + t)), which
        // the ordered threads apply in order after the barrier.  A batch or
        // run with a first or rescaling token, or a shift of 16 or more,
        // takes the slow form (the ballots say which).  split is
        // about kSeqShare16/16 of n, past the chunk's last first or rescaling
        // token, and a multiple of kBatch, and so is q.  Slots past n have a
        // zero coefficient, so a zero term.
        const int split0 = min(n, ((n * kSeqShare16) / 16 + kBatch - 1) & ~(kBatch - 1));
        int last_special = -1;
#pragma unroll
        for (int w = 0; w < kChunk / 64; ++w) {
            const int lo = split0 - 64 * w;
            if (lo < 64) {
                uint64_t m = uniform64(s_special[w]);
                if (lo > 0) m &= ~0ull << lo;
                if (m != 0u) last_special = 64 * w + 63 - __builtin_clzll(m);
            }
        }
        const int split = last_special < 0 ? split0 : (last_special + kBatch) & ~(kBatch - 1);
        const int rest = n - split;
        const int q = rest > 0 ? ((rest + kCompParts - 1) / kCompParts + kBatch - 1) & ~(kBatch - 1) : 0;
        const int cp = d < kSeqLanes ? 0 : (d - kSeqLanes) / kCh;   // composed part of a composing thread
        const int cl = d < kSeqLanes ? d % kCh : (d - kSeqLanes) % kCh;
        const int ch = slice * kCh + cl;
        const float* s_p_g = s_u.p[cl >> 5];   // this channel's group
        if (d < kCh) {
            // With four workgroups per head a CU holds one of them, so the
            // ordered part's LDS latency is exposed: the next batch's reads go
            // out while this one's terms are formed.
            FastBatch next;
            if constexpr (kPrefetchY)
                if (split > 0) next = load_fast(s_p_g, s_vc, 0, ch);
            for (int span = 0; span < split; span += 64) {
                const uint64_t spans = uniform64(s_special[span >> 6]);
                const uint64_t slows = uniform64(s_slow[span >> 6]);
                const uint64_t wides = uniform64(s_wide17[span >> 6]);
                const int end = min(span + 64, split);
                for (int i0 = span; i0 < end; i0 += kBatch) {
                    const int at = i0 - span;
                    FastBatch cur;
                    if constexpr (kPrefetchY) {
                        cur = next;
                        if (i0 + kBatch < split) next = load_fast(s_p_g, s_vc, i0 + kBatch, ch);
                    }
                    if (((slows >> at) & kBatchMask) == 0u) {
                        // No first or rescaling token and every shift at most
                        // 15: fused-multiply-add terms.  Where no Y of the
                        // wave lies within kBatch 2^22 of either end of the
                        // int32 range no partial sum saturates, and the batch
                        // adds its terms at once (modulo 2^32, then exact).
                        if constexpr (!kPrefetchY) cur = load_fast(s_p_g, s_vc, i0, ch);
                        uint32_t tb[kBatch];
                        fast_term_bits(cur, tb);
                        const bool safe = static_cast<uint32_t>(y) + (0x80000000u - kSatMargin) <= ~(2u * kSatMargin);
                        if (__builtin_amdgcn_ballot_w64(!safe) == 0u) {
                            uint32_t acc = static_cast<uint32_t>(y) - kBatch * kRoundMagicBits;
#pragma unroll
                            for (int j = 0; j < kBatch; ++j) acc += tb[j];
                            y = static_cast<int32_t>(acc);
                        } else {
#pragma unroll
                            for (int j = 0; j < kBatch; ++j)
                                y = __builtin_elementwise_add_sat(y, static_cast<int32_t>(tb[j] - kRoundMagicBits));
                        }
                    } else {
                        int32_t code[kBatch], term[kBatch];
                        float pv[kBatch];
                        slow_terms(s_tok, s_p_g, s_vc, i0, ch, ((wides >> at) & kBatchMask) != 0u, code, pv, term);
                        if (((spans >> at) & kBatchMask) == 0u) {
#pragma unroll
                            for (int j = 0; j < kBatch; ++j) y = __builtin_elementwise_add_sat(y, term[j]);
                        } else {
                            // A first or rescaling token's p is its V scale.
#pragma unroll
                            for (int j = 0; j < kBatch; ++j) {
                                const uint32_t w = static_cast<uint32_t>(
                                    __builtin_amdgcn_readfirstlane(static_cast<int>(s_tok[i0 + j])));
                                y = value_step(y, w, code[j], shift_of(pv[j]), term[j]);
                            }
                        }
                    }
                }
            }
        } else if (d >= kSeqLanes) {
            if (wave == 3) {
                // Z: ordinary tokens add their coefficients modulo 2^30, so
                // between two first or rescaling tokens Z advances by a
                // difference of prefix sums, and only those tokens step in
                // order.  The prefix sums of a 64-token span that holds such
                // a token come from a wave scan of its coefficient words.
                uint32_t done = 0u, offset = 0u;   // prefix sum already added; sum of the spans before
#pragma unroll
                for (int w = 0; w < kChunk / 64; ++w) {
                    uint64_t m = uniform64(s_special[w]);
                    if (m != 0u) {
                        const uint32_t wd = s_tok[64 * w + lane];
                        const uint32_t incl = wave_scan_add((wd & (kInit | kRescale)) != 0u ? 0u : (wd & kCoefMask));
                        while (m != 0u) {
                            const int i = __builtin_ctzll(m);
                            // the sum of the ordinary tokens before i (i itself counts zero)
                            const uint32_t upto =
                                offset + static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), i));
                            z = (z + (upto - done)) & kMask30;
                            done = upto;
                            z = z_step(z, static_cast<uint32_t>(
                                              __builtin_amdgcn_readfirstlane(static_cast<int>(s_tok[64 * w + i]))));
                            m &= m - 1u;
                        }
                    }
                    offset += s_wave_sum[w];
                }
                z = (z + (offset - done)) & kMask30;
            }
            // A composing thread's run [begin, end) holds no first or
            // rescaling token.  With kCh = 32 a wave holds two parts, so what
            // depends on the run is read per lane.
            const int begin = split + cp * q, end = min(n, begin + q);
            if (begin < n) {
                // Slow-form tokens in [split, n) (wave-uniform), then, with
                // two parts per wave, in this lane's run.
                bool slow_run = false;
#pragma unroll
                for (int w = 0; w < kChunk / 64; ++w) {
                    const int lo_t = max(split - 64 * w, 0), hi_t = min(n - 64 * w, 64);
                    if (lo_t < hi_t)
                        slow_run |= (uniform64(s_slow[w]) & (~0ull >> (64 - (hi_t - lo_t))) << lo_t) != 0u;
                }
                if (kCompParts > 1 && slow_run) {
                    slow_run = false;
#pragma unroll
                    for (int w = 0; w < kChunk / 64; ++w) {
                        const int lo_t = max(begin - 64 * w, 0), hi_t = min(end - 64 * w, 64);
                        if (lo_t < hi_t)
                            slow_run |= (s_slow[w] & (~0ull >> (64 - (hi_t - lo_t))) << lo_t) != 0u;
                    }
                }
                if (!slow_run) {
                    // Fused-multiply-add terms.  With prefix sums P_k (P_0 =
                    // 0) the map is A = P_n, L = INT32_MIN + P_n - min P_k,
                    // H = INT32_MAX + P_n - max P_k: the sat32 recursion of L
                    // and H in closed form, exact while neither reaches the
                    // far end of the int32 range (|P_k| < 2^30, see kMaxRun).
                    int32_t pk = 0, pmin = 0, pmax = 0;
                    FastBatch next;
                    if constexpr (kPrefetchY) next = load_fast(s_p_g, s_vc, begin, ch);
                    for (int i0 = begin; i0 < end; i0 += kBatch) {
                        FastBatch cur;
                        if constexpr (kPrefetchY) {
                            cur = next;
                            if (i0 + kBatch < end) next = load_fast(s_p_g, s_vc, i0 + kBatch, ch);
                        } else {
                            cur = load_fast(s_p_g, s_vc, i0, ch);
                        }
                        uint32_t tb[kBatch];
                        fast_term_bits(cur, tb);
#pragma unroll
                        for (int j = 0; j < kBatch; j += 2) {
                            const int32_t p1 = pk + static_cast<int32_t>(tb[j] - kRoundMagicBits);
                            const int32_t p2 = p1 + static_cast<int32_t>(tb[j + 1] - kRoundMagicBits);
                            pmin = min(pmin, min(p1, p2));
                            pmax = max(pmax, max(p1, p2));
                            pk = p2;
                        }
                    }
                    s_map_sum[cp * kCh + cl] = pk;
                    s_map_lo[cp * kCh + cl] = INT32_MIN + (pk - pmin);
                    s_map_hi[cp * kCh + cl] = INT32_MAX + (pk - pmax);
                } else {
                    int64_t sum = 0;
                    int32_t sum_short = 0;   // the short-form batches' terms (see kMaxRun)
                    int32_t lo = INT32_MIN, hi = INT32_MAX;
                    for (int i0 = begin; i0 < end; i0 += kBatch) {
                        int32_t code[kBatch], term[kBatch];
                        float pv[kBatch];
                        const bool wide = ((s_wide17[i0 >> 6] >> (i0 & 63)) & kBatchMask) != 0u;
                        if (slow_terms(s_tok, s_p_g, s_vc, i0, ch, wide, code, pv, term)) {
#pragma unroll
                            for (int j = 0; j < kBatch; ++j) {
                                sum_short += term[j];
                                lo = __builtin_elementwise_add_sat(lo, term[j]);
                                hi = __builtin_elementwise_add_sat(hi, term[j]);
                            }
                        } else {
#pragma unroll
                            for (int j = 0; j < kBatch; ++j) {
                                sum += term[j];
                                lo = __builtin_elementwise_add_sat(lo, term[j]);
                                hi = __builtin_elementwise_add_sat(hi, term[j]);
                            }
                        }
                    }
                    sum += sum_short;
                    s_map_sum[cp * kCh + cl] = sum;
                    s_map_lo[cp * kCh + cl] = lo;
                    s_map_hi[cp * kCh + cl] = hi;
                }
            }
        }
        __syncthreads();
        if (d < kCh) {
#pragma unroll
            for (int p = 0; p < kCompParts; ++p) {
                if (split + p * q >= n) break;
                const int k = p * kCh + cl;
                y = static_cast<int32_t>(min(max(static_cast<int64_t>(y) + s_map_sum[k], static_cast<int64_t>(s_map_lo[k])),
                                             static_cast<int64_t>(s_map_hi[k])));
            }
        }
    }
    // The normalizer 1/Z: the 18-bit quotient floor((2^34 + Z/2) / Z) (cpp:271-300).
    if (wave == 3 && lane == 0)
        s_inv = z ? static_cast<uint32_t>(((1ull << 34) + (z >> 1)) / z) & 0x3ffffu : 0x3ffffu;
    __syncthreads();

    // Y * inv with RNE and a 32-bit wrap (cpp:1666-1710),
    // and the integer-path A14/E8M0 (cpp:1694-1771, 2656-2682): group max of
    // |raw| (INT32_MIN counts as INT32_MAX), one float conversion, frexp
    // exponent e, q = trunc(clamp(raw*2^-17 * 2^(13-e) +- 0.5, +-8191)),
    // code = e + 127.  Threads d < kCh own channel slice * kCh + d; a group
    // is 32 lanes of one wave.
    const size_t grp0 = static_cast<size_t>(b) * (kHeads * kGroupsPerHead) + h * kGroupsPerHead + slice * kGroups;
    if (d < kCh) {
        const int32_t o = mulq17_wrap(y, s_inv);
        reinterpret_cast<int32_t*>(a.out)[static_cast<size_t>(b) * kModelDim + h * kHeadDim + slice * kCh + d] = o;
        int32_t m = o == INT32_MIN ? INT32_MAX : (o < 0 ? -o : o);
#pragma unroll
        for (int s = 1; s < 32; s <<= 1) m = max(m, __shfl_xor(m, s));
        const float mx = static_cast<float>(m) * 0x1p-17f;
        int16_t q14 = 0;
        uint8_t code = 0;
        if (mx != 0.0f) {
            int e = 0;
            (void)frexpf(mx, &e);
            const float x = __fmul_rn(static_cast<float>(o) * 0x1p-17f, ldexpf(1.0f, 13 - e));
            float rr = x >= 0.0f ? __fadd_rn(x, 0.5f) : __fsub_rn(x, 0.5f);
            rr = fminf(fmaxf(rr, -8191.0f), 8191.0f);
            q14 = static_cast<int16_t>(static_cast<int>(rr));
            code = static_cast<uint8_t>(e + 127);
        }
        s_q14[d] = q14;
        if (a.act_scale != nullptr && (d & 31) == 0) a.act_scale[grp0 + (d >> 5)] = code;
    }
    __syncthreads();
    if (a.act_q != nullptr && d < kGroups * 14) {
        const int gi = d / 14, w = d % 14;
        uint32_t word = 0;
        const int bit0 = 32 * w;
        for (int i = bit0 / 14; i <= (bit0 + 31) / 14 && i < 32; ++i) {
            const uint32_t val = static_cast<uint32_t>(static_cast<uint16_t>(s_q14[gi * 32 + i])) & 0x3fffu;
            const int sh = 14 * i - bit0;
            word |= sh >= 0 ? (val << sh) : (val >> -sh);
        }
        reinterpret_cast<uint32_t*>(a.act_q + (grp0 + gi) * 56)[w] = word;
    }
}

}  // namespace

hipError_t launch_exact(const StepArgs& a, const uint32_t* exp_lut, bool q17, hipStream_t s) {
    ExactArgs ea;
    ea.step = a;
    for (int i = 0; i < 33; ++i) ea.exp_lut[i] = exp_lut[i];
    if (a.batch <= kExactSlicedMaxBatch) {
        const dim3 grid(kHeads * 4, a.batch);
        if (q17) exact_kernel<true, 4><<<grid, 256, 0, s>>>(ea);
        else exact_kernel<false, 4><<<grid, 256, 0, s>>>(ea);
    } else if (a.batch <= kExactHalfSlicedMaxBatch) {
        const dim3 grid(kHeads * 2, a.batch);
        if (q17) exact_kernel<true, 2><<<grid, 256, 0, s>>>(ea);
        else exact_kernel<false, 2><<<grid, 256, 0, s>>>(ea);
    } else {
        const dim3 grid(kHeads, a.batch);
        if (q17) exact_kernel<true, 1><<<grid, 256, 0, s>>>(ea);
        else exact_kernel<false, 1><<<grid, 256, 0, s>>>(ea);
    }
    return hipGetLastError();
}

}  // namespace swiftkv
