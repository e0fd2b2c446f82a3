// swiftkv_exact.hip -- integer-compatibility step: the reference's Q15.17
// single-pass recurrence evaluated exactly on the GPU, so the A14 words and
// E8M0 codes equal the reference's bit for bit (swiftkv_attention.cpp:934-1880;
// llama2_decoder_sw_emulator.cpp:633-711).  Slow by construction -- the
// (max, Z, Y) recurrence is sequential per head -- and meant for bit-level
// comparison with the FPGA / C model, not for throughput.
//
// Grid (32 heads, batch), 256 threads per (sequence, head):
//   - cached tokens are processed in chunks of kChunk: the 4 waves compute the
//     chunk's integer scores in parallel (lane = 16-channel half-group c of
//     token row r; the per-half shift and the 44-bit wraps are associative
//     modulo 2^44, so the octet sum may run in any order), then wave 0 runs
//     the recurrence over the chunk in token order;
//   - the new row (converted, rotated, quantized, appended like the fast step)
//     is the last token of the recurrence, taken from registers;
//   - finally Y * 1/Z and the integer-path A14/E8M0 epilogue.
#include "swiftkv_device.hpp"

namespace swiftkv {
namespace {

using namespace dev;

constexpr int kChunk = 256;                   // cached tokens per chunk (V codes staged in LDS)
constexpr int64_t kScoreScaleQ17 = 11585;     // RNE(2^17 / sqrt(128)) (swiftkv_attention.cpp:1101-1102)
constexpr int64_t kLog2eQ21 = 3025551;        // RNE(log2(e) * 2^21) (cpp:207-208)

__device__ __forceinline__ int64_t wrap_bits(int64_t x, int bits) {
    const uint64_t mask = (1ull << bits) - 1u;
    uint64_t r = static_cast<uint64_t>(x) & mask;
    if ((r >> (bits - 1)) & 1u) r |= ~mask;
    return static_cast<int64_t>(r);
}

// Round-half-even of x / 2^s on the magnitude (AP_RND_CONV).
__device__ __forceinline__ int64_t rne_shift(int64_t x, int s) {
    const bool neg = x < 0;
    const uint64_t mag = neg ? static_cast<uint64_t>(-(x + 1)) + 1u : static_cast<uint64_t>(x);
    uint64_t q = mag >> s;
    const uint64_t rem = mag & ((1ull << s) - 1u);
    const uint64_t half = 1ull << (s - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return neg ? -static_cast<int64_t>(q) : static_cast<int64_t>(q);
}

// Q15.17 x unsigned Q1.17 multiplier, RNE >> 17, wrapped to 32 bits.
__device__ __forceinline__ int32_t mulq17_wrap(int32_t a, uint32_t b) {
    return static_cast<int32_t>(wrap_bits(rne_shift(static_cast<int64_t>(a) * static_cast<int64_t>(b), 17), 32));
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
__device__ __forceinline__ int64_t half_dot(const int32_t* q, const int8_t* row16, uint32_t shift) {
    const int4 w = *reinterpret_cast<const int4*>(row16);
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

// One token of the (max, Z, Y) recurrence (cpp:1276-1335, 1463-1558).
// Lane l owns channels 2l, 2l+1; vals are the token's dequantized codes.
struct Recurrence {
    int32_t run_max;
    uint32_t z;
    int32_t y0, y1;
    bool started;
};

__device__ __forceinline__ void recur(Recurrence& st, int32_t score, int32_t val0, int32_t val1, const uint32_t* lut) {
    if (!st.started) {
        st.run_max = score;
        st.z = 1u << 17;
        st.y0 = val0;
        st.y1 = val1;
        st.started = true;
        return;
    }
    constexpr uint32_t kMask30 = (1u << 30) - 1u;
    if (score <= st.run_max) {
        const uint32_t coef = exp_neg_q17(sat32(static_cast<int64_t>(score) - st.run_max), lut);
        st.z = (st.z + coef) & kMask30;
        st.y0 = sat32(static_cast<int64_t>(st.y0) + mulq17_wrap(val0, coef));
        st.y1 = sat32(static_cast<int64_t>(st.y1) + mulq17_wrap(val1, coef));
    } else {
        const uint32_t coef = exp_neg_q17(sat32(static_cast<int64_t>(st.run_max) - score), lut);
        st.z = static_cast<uint32_t>(rne_shift(static_cast<int64_t>(st.z) * coef, 17)) & kMask30;
        st.z = (st.z + (1u << 17)) & kMask30;
        st.run_max = score;
        st.y0 = sat32(static_cast<int64_t>(mulq17_wrap(st.y0, coef)) + val0);
        st.y1 = sat32(static_cast<int64_t>(mulq17_wrap(st.y1, coef)) + val1);
    }
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
    int8_t* page = page_ptr(a.kv, a.slot0 + b, a.layer, h);
    const int64_t cap = a.kv.seq_cap;
    const float* scales = reinterpret_cast<const float*>(page + cap * (2 * kCodeBytes));

    __shared__ int32_t s_q[kHeadDim];
    __shared__ int32_t s_score[kChunk];
    __shared__ uint16_t s_v[kChunk][kHeadDim / 2];      // V code pairs of the chunk
    __shared__ uint8_t s_vs[kChunk][kGroupsPerHead];    // V shifts of the chunk
    __shared__ uint32_t s_lut[33];
    __shared__ int16_t s_q14[kHeadDim];
    if (threadIdx.x < 33) s_lut[threadIdx.x] = ea.exp_lut[threadIdx.x];

    // Rotated query (shared through LDS) and, in wave 0, the new row, appended
    // to the cache and kept in registers for the last recurrence step.
    const size_t elem = static_cast<size_t>(b) * kModelDim + h * kHeadDim + 2 * lane;
    const int2 cs = a.lut[static_cast<size_t>(pos) * kRopePairs + lane];
    int32_t q0 = 0, q1 = 0;
    RowCodes rc{};
    if (wave == 0) {
        const int2 qi = load_pair<Q17>(a.q, elem);
        const int2 ki = load_pair<Q17>(a.k, elem);
        const int2 vi = load_pair<Q17>(a.v, elem);
        int32_t k0, k1;
        rope_pair(qi.x, qi.y, cs, q0, q1);
        rope_pair(ki.x, ki.y, cs, k0, k1);
        rc = append_row_codes(page, a.kv.seq_cap, pos, lane, k0, k1, vi.x, vi.y);
        s_q[2 * lane] = q0;
        s_q[2 * lane + 1] = q1;
    }
    __syncthreads();
    int32_t qc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) qc[j] = s_q[16 * c + j];

    Recurrence st{0, 0u, 0, 0, false};
    for (int t0 = 0; t0 < pos; t0 += kChunk) {
        const int n = min(kChunk, pos - t0);
        // Scores of tokens [t0, t0+n), 4 waves x 8 token rows per pass; the
        // same passes stage the chunk's V codes and shifts in LDS.
        for (int i = wave * 8 + r; i < kChunk; i += 32) {
            const int64_t t = t0 + i;
            int64_t p = 0;
            if (i < n) {
                const float2 sc = *reinterpret_cast<const float2*>(scales + t * 8 + (c >> 1) * 2);
                p = half_dot(qc, page + t * kCodeBytes + c * 16, shift_of(sc.x));
                const int4 vw = *reinterpret_cast<const int4*>(page + cap * kCodeBytes + t * kCodeBytes + c * 16);
                reinterpret_cast<int4*>(&s_v[i][0])[c] = vw;
                if ((c & 1) == 0) s_vs[i][c >> 1] = static_cast<uint8_t>(shift_of(sc.y));
            }
            // sum of the token's 8 half-groups (lanes 8r .. 8r+7), modulo 2^44
            p += __shfl_xor(p, 1);
            p += __shfl_xor(p, 2);
            p += __shfl_xor(p, 4);
            if (c == 0 && i < n) s_score[i] = score_of(p);
        }
        __syncthreads();
        if (wave == 0) {
            const int g = lane >> 4;
            for (int i = 0; i < n; ++i) {
                const uint32_t vs = s_vs[i][g];
                const uint16_t vc = s_v[i][lane];
                recur(st, s_score[i], dequant_raw(vc & 0xffu, vs), dequant_raw(vc >> 8, vs), s_lut);
            }
        }
        __syncthreads();
    }
    if (wave != 0) return;

    // The new token: its dot from registers (half-group = 8 lanes, then the 8
    // half-groups), then the last recurrence step.
    int64_t part = static_cast<int64_t>(q0) * static_cast<int8_t>(rc.k0) +
                   static_cast<int64_t>(q1) * static_cast<int8_t>(rc.k1);
    part += __shfl_xor(part, 1);
    part += __shfl_xor(part, 2);
    part += __shfl_xor(part, 4);
    int64_t p = wrap_bits(rc.sk >= 10 ? static_cast<int64_t>(static_cast<uint64_t>(part) << (rc.sk - 10))
                                      : (part >> (10 - rc.sk)), 44);
    p += __shfl_xor(p, 8);
    p += __shfl_xor(p, 16);
    p += __shfl_xor(p, 32);
    recur(st, score_of(p), dequant_raw(rc.v0, rc.sv), dequant_raw(rc.v1, rc.sv), s_lut);

    // Normalize: 18-bit quotient floor((2^34 + Z/2) / Z) (cpp:271-300), then
    // Y * inv with RNE and a 32-bit wrap (cpp:1666-1710).
    const uint32_t inv = st.z ? static_cast<uint32_t>(((1ull << 34) + (st.z >> 1)) / st.z) & 0x3ffffu : 0x3ffffu;
    const int32_t o0 = mulq17_wrap(st.y0, inv), o1 = mulq17_wrap(st.y1, inv);
    reinterpret_cast<int2*>(a.out)[elem >> 1] = make_int2(o0, o1);   // Q15.17 state
    if (a.act_q == nullptr) return;

    // Integer-path A14/E8M0 (cpp:1694-1771, 2656-2682): group max of |raw|
    // (INT32_MIN counts as INT32_MAX), one float conversion, frexp exponent e,
    // q = trunc(clamp(raw*2^-17 * 2^(13-e) +- 0.5, +-8191)), code = e + 127.
    auto mag = [](int32_t x) { return x == INT32_MIN ? INT32_MAX : (x < 0 ? -x : x); };
    int32_t m = max(mag(o0), mag(o1));
#pragma unroll
    for (int s = 1; s < 16; s <<= 1) m = max(m, __shfl_xor(m, s));
    const float mx = static_cast<float>(m) * 0x1p-17f;
    int16_t c0 = 0, c1 = 0;
    uint8_t code = 0;
    if (mx != 0.0f) {
        int e = 0;
        (void)frexpf(mx, &e);
        const float inv_scale = ldexpf(1.0f, 13 - e);
        auto quant = [&](int32_t raw) {
            const float x = __fmul_rn(static_cast<float>(raw) * 0x1p-17f, inv_scale);
            float rr = x >= 0.0f ? __fadd_rn(x, 0.5f) : __fsub_rn(x, 0.5f);
            rr = fminf(fmaxf(rr, -8191.0f), 8191.0f);
            return static_cast<int16_t>(static_cast<int>(rr));
        };
        c0 = quant(o0);
        c1 = quant(o1);
        code = static_cast<uint8_t>(e + 127);
    }
    s_q14[2 * lane] = c0;
    s_q14[2 * lane + 1] = c1;
    const size_t grp0 = static_cast<size_t>(b) * (kHeads * kGroupsPerHead) + h * kGroupsPerHead;
    if ((lane & 15) == 0) a.act_scale[grp0 + (lane >> 4)] = code;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (lane < kGroupsPerHead * 14) {
        const int gi = lane / 14, w = lane % 14;
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
