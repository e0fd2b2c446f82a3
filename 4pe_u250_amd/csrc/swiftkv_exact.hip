// swiftkv_exact.hip -- integer-compatibility step: the reference's Q15.17
// single-pass recurrence evaluated exactly on the GPU, so the A14 words and
// E8M0 codes equal the reference's bit for bit (swiftkv_attention.cpp:934-1880;
// llama2_decoder_sw_emulator.cpp:633-711).  Slow by construction -- the
// (max, Z, Y) recurrence is sequential per head -- and meant for bit-level
// comparison with the FPGA / C model; the sequential chains bound it, not HBM.
//
// Grid (32 heads, batch rows), 256 threads per (sequence, head).  Wave 0
// first appends the new row like the fast step; then tokens [0, position]
// are processed in chunks of kChunk:
//   - the 4 waves compute the chunk's integer scores (lane = 16-channel
//     half-group c of token row r; the per-half shift and the 44-bit wraps are
//     associative modulo 2^44, so the octet sum may run in any order) and
//     stage its V codes in LDS;
//   - one thread per token turns its score and the exclusive prefix maximum
//     into a coefficient word (exp LUT, rescale flag);
//   - threads 0..127 run Y, one channel each, and wave 2 runs Z, both in
//     token order;
// then Y * 1/Z and the integer-path A14/E8M0 epilogue.
#include "swiftkv_device.hpp"

namespace swiftkv {
namespace {

using namespace dev;

constexpr int kChunk = 256;                   // cached tokens per chunk (V codes staged in LDS)
constexpr int kBatch = 8;                     // tokens whose LDS reads go out together in the Y and Z passes
static_assert(kChunk % kBatch == 0, "batches tile a chunk");
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

// 44-bit token dot contribution of one 16-channel half-group: the 16 int8
// codes times the int32 rotated query, scaled by 2^(shift-10) (cpp:934-995).
__device__ __forceinline__ int64_t half_dot(const int32_t* q, int4 w, uint32_t shift) {
    const int32_t d[4] = {w.x, w.y, w.z, w.w};
    int64_t s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int byte = 0; byte < 4; ++byte)
            s += static_cast<int64_t>(q[4 * j + byte]) * static_cast<int8_t>(d[j] >> (8 * byte));
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
// once.  What stays sequential is Z (one wave, a few operations per token)
// and Y (one lane per channel).
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

// One token of Y for one channel: no rescale  Y = sat32(Y + wrap32(RNE(v c >> 17))),
// rescale  Y = sat32(wrap32(RNE(Y c >> 17)) + v); one multiply either way.
__device__ __forceinline__ int32_t value_step(int32_t y, uint32_t word, int32_t val) {
    if (word & kInit) return val;
    const bool rescale = (word & kRescale) != 0u;
    const int32_t m = mulq17_wrap(rescale ? y : val, word & kCoefMask);
    return __builtin_elementwise_add_sat(rescale ? val : y, m);
}

// code << shift as the reference's ap_int<32> (wraps for code 64, shift 25).
__device__ __forceinline__ int32_t dequant_raw(uint32_t code_byte, uint32_t shift) {
    return static_cast<int32_t>(static_cast<uint32_t>(static_cast<int32_t>(static_cast<int8_t>(code_byte))) << shift);
}

struct ExactArgs {
    StepArgs step;
    uint32_t exp_lut[33];     // RNE(2^(30 + i/32)), i = 0..32 (cpp:185-195)
};

template <bool Q17>
__global__ __launch_bounds__(256) void exact_kernel(ExactArgs ea) {
    const StepArgs& a = ea.step;
    const uint32_t row = a.rows[blockIdx.y];
    const int h = blockIdx.x, b = static_cast<int>(row & 0xffu);
    const int pos = static_cast<int>(row >> 8);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int c = lane & 7, r = lane >> 3;
    const int d = threadIdx.x;                  // token of the chunk (coefficients), channel (Y, d < 128)
    int8_t* page = page_ptr(a.kv, a.slot0 + b, a.layer, h);
    const int64_t cap = a.kv.seq_cap;
    const float* scales = reinterpret_cast<const float*>(page + cap * (2 * kCodeBytes));

    __shared__ int32_t s_q[kHeadDim];
    __shared__ int32_t s_score[kChunk];
    __shared__ uint32_t s_word[kChunk];                  // coefficient words of the chunk
    __shared__ int8_t s_vc[kChunk][kHeadDim];            // V codes of the chunk
    __shared__ uint8_t s_vs[kChunk][kGroupsPerHead];     // V shifts of the chunk
    __shared__ int32_t s_wave_max[kChunk / 64];
    __shared__ uint32_t s_lut[33];
    __shared__ uint32_t s_inv;
    __shared__ int16_t s_q14[kHeadDim];
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
    int32_t qc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) qc[j] = s_q[16 * c + j];

    const int len = pos + 1;
    int32_t run_max = INT32_MIN;   // prefix maximum before the chunk (every thread)
    uint32_t z = 0;                // Z (wave 2, uniform)
    int32_t y = 0;                 // Y of channel d (threads d < 128)
    for (int t0 = 0; t0 < len; t0 += kChunk) {
        const int n = min(kChunk, len - t0);
        // Scores of tokens [t0, t0+n), 4 waves x 8 token rows per pass; the
        // same passes stage the chunk's V codes and shifts in LDS.
        for (int i = wave * 8 + r; i < kChunk; i += 32) {
            const int64_t t = t0 + i;
            int64_t p = 0;
            if (i < n) {
                const float2 sc = *reinterpret_cast<const float2*>(scales + t * 8 + (c >> 1) * 2);
                p = half_dot(qc, *reinterpret_cast<const int4*>(page + t * kCodeBytes + c * 16), shift_of(sc.x));
                reinterpret_cast<int4*>(&s_vc[i][0])[c] =
                    *reinterpret_cast<const int4*>(page + cap * kCodeBytes + t * kCodeBytes + c * 16);
                if ((c & 1) == 0) s_vs[i][c >> 1] = static_cast<uint8_t>(shift_of(sc.y));
            }
            // sum of the token's 8 half-groups (lanes 8r .. 8r+7), modulo 2^44
            p += __shfl_xor(p, 1);
            p += __shfl_xor(p, 2);
            p += __shfl_xor(p, 4);
            if (c == 0 && i < n) s_score[i] = score_of(p);
        }
        __syncthreads();

        // Coefficient words, one token per thread: the exclusive prefix
        // maximum (wave scan, then the maxima of the waves before) gives each
        // token's running maximum.
        const int32_t sv = d < n ? s_score[d] : INT32_MIN;
        int32_t incl = sv;
#pragma unroll
        for (int k = 1; k < 64; k <<= 1) {
            const int32_t o = __shfl_up(incl, k);
            if (lane >= k) incl = max(incl, o);
        }
        if (lane == 63) s_wave_max[wave] = incl;
        int32_t excl = __shfl_up(incl, 1);
        __syncthreads();
        int32_t before = run_max;
        for (int w = 0; w < wave; ++w) before = max(before, s_wave_max[w]);
        excl = lane == 0 ? before : max(before, excl);
        if (d < n) s_word[d] = (t0 == 0 && d == 0) ? kInit : coef_word(sv, excl, s_lut);
#pragma unroll
        for (int w = 0; w < kChunk / 64; ++w) run_max = max(run_max, s_wave_max[w]);
        __syncthreads();

        // Y (threads 0..127, one channel each) and Z (wave 2), in token order.
        // The LDS reads of kBatch tokens go out before their updates, so one
        // read latency covers the batch (indices stay below kChunk: kChunk is
        // a multiple of kBatch; entries past n are read and not used).
        if (d < kHeadDim) {
            const int g = d >> 5;
            for (int i0 = 0; i0 < n; i0 += kBatch) {
                uint32_t w[kBatch];
                int32_t v[kBatch];
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {
                    w[j] = s_word[i0 + j];
                    v[j] = dequant_raw(static_cast<uint8_t>(s_vc[i0 + j][d]), s_vs[i0 + j][g]);
                }
#pragma unroll
                for (int j = 0; j < kBatch; ++j)
                    if (i0 + j < n) y = value_step(y, w[j], v[j]);
            }
        } else if (wave == 2) {
            for (int i0 = 0; i0 < n; i0 += kBatch) {
                uint32_t w[kBatch];
#pragma unroll
                for (int j = 0; j < kBatch; ++j) w[j] = s_word[i0 + j];
#pragma unroll
                for (int j = 0; j < kBatch; ++j)
                    if (i0 + j < n) z = z_step(z, __builtin_amdgcn_readfirstlane(w[j]));
            }
        }
        __syncthreads();
    }
    // The normalizer 1/Z: the 18-bit quotient floor((2^34 + Z/2) / Z) (cpp:271-300).
    if (wave == 2 && lane == 0)
        s_inv = z ? static_cast<uint32_t>(((1ull << 34) + (z >> 1)) / z) & 0x3ffffu : 0x3ffffu;
    __syncthreads();

    // Y * inv with RNE and a 32-bit wrap (cpp:1666-1710),
    // and the integer-path A14/E8M0 (cpp:1694-1771, 2656-2682): group max of
    // |raw| (INT32_MIN counts as INT32_MAX), one float conversion, frexp
    // exponent e, q = trunc(clamp(raw*2^-17 * 2^(13-e) +- 0.5, +-8191)),
    // code = e + 127.  Threads d < 128 own channel d; a group is 32 lanes of
    // one wave.
    const size_t grp0 = static_cast<size_t>(b) * (kHeads * kGroupsPerHead) + h * kGroupsPerHead;
    if (d < kHeadDim) {
        const int32_t o = mulq17_wrap(y, s_inv);
        reinterpret_cast<int32_t*>(a.out)[static_cast<size_t>(b) * kModelDim + h * kHeadDim + d] = o;
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
    if (a.act_q != nullptr && d < kGroupsPerHead * 14) {
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
    const dim3 grid(kHeads, a.batch);
    if (q17) exact_kernel<true><<<grid, 256, 0, s>>>(ea);
    else exact_kernel<false><<<grid, 256, 0, s>>>(ea);
    return hipGetLastError();
}

}  // namespace swiftkv
