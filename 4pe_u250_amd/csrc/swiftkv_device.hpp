// swiftkv_device.hpp -- device-side arithmetic shared by the kernels:
// FP32 -> Q15.17, integer RoPE, G32 quantization, the append of one row, and
// the DPP cross-lane helpers.  Included by swiftkv_kernels.hip and
// swiftkv_synth.hip only.
#pragma once

#include "swiftkv_common.hpp"

namespace swiftkv {
namespace dev {

// Vector register types of the buffer-load and -store builtins.
typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v2i __attribute__((ext_vector_type(2)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int32_t kBufferWord3 = 0x00020000;   // raw buffer resource, gfx9 data format

// ---------------------------------------------------------------- numerics

// FP32 -> Q15.17 with round-half-even and saturation.  The reference states
// it on the bit pattern (int4_linear_controller.cpp:38-83): exponent < 109
// (|x| < 2^-18) -> 0, exponent >= 141 (|x| >= 2^14, inf, nan) -> saturate by
// sign, otherwise RNE of sig >> (133 - e) or sig << (e - 133).  The same
// value, branch-free: x * 2^17 is exact (a power-of-two scaling; it overflows
// to inf only where the rule saturates anyway), v_rndne_f32 rounds it
// half-even to an integer exactly, and v_cvt_i32_f32 clamps out-of-range
// values to INT32_MIN/INT32_MAX.  Every |x| < 2^-18 rounds to 0 and every
// |x| >= 2^14 clamps, so only NaN (which the conversion maps to 0) needs
// its sign-saturated value: a NaN is replaced by the infinity of its sign
// before the conversion.
__device__ __forceinline__ int32_t f32_to_q17(float x) {
    const float inf = __uint_as_float((__float_as_uint(x) & 0x80000000u) | 0x7f800000u);
    const float r = __builtin_isnan(x) ? inf : __builtin_rintf(x * 131072.0f);
    int32_t v;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(v) : "v"(r));
    return v;
}

__device__ __forceinline__ int32_t sat32(int64_t x) {
    return x > INT32_MAX ? INT32_MAX : (x < INT32_MIN ? INT32_MIN : static_cast<int32_t>(x));
}

// Adjacent-pair rotation with a Q1.17 (cos, sin): floor shift of the 52-bit
// sum, saturated to int32 (swiftkv_attention.cpp:20-51).
__device__ __forceinline__ void rope_pair(int32_t a, int32_t b, int2 cs, int32_t& x0, int32_t& x1) {
    const int64_t c = cs.x, s = cs.y;
    x0 = sat32((static_cast<int64_t>(a) * c - static_cast<int64_t>(b) * s) >> 17);
    x1 = sat32((static_cast<int64_t>(a) * s + static_cast<int64_t>(b) * c) >> 17);
}

__device__ __forceinline__ uint32_t magnitude(int32_t r) {
    return r < 0 ? 0u - static_cast<uint32_t>(r) : static_cast<uint32_t>(r);
}

// G32 shift: msb(max|r|) - 6, floored at 0 (swiftkv_attention.cpp:374-399).
__device__ __forceinline__ uint32_t g32_shift(uint32_t m) {
    if (m == 0u) return 0u;
    const uint32_t msb = 31u - static_cast<uint32_t>(__clz(m));
    return msb > 6u ? msb - 6u : 0u;
}

// Code = sign * min(127, (|r| + 2^(s-1)) >> s) (swiftkv_attention.cpp:401-418).
__device__ __forceinline__ uint32_t g32_code_byte(int32_t r, uint32_t s) {
    const uint32_t rnd = s ? (1u << (s - 1u)) : 0u;
    uint32_t q = (magnitude(r) + rnd) >> s;      // |r| <= 2^31, rnd <= 2^24: no wrap
    q = q > 127u ? 127u : q;
    const int32_t c = r < 0 ? -static_cast<int32_t>(q) : static_cast<int32_t>(q);
    return static_cast<uint32_t>(c) & 0xffu;
}

// FP32 bit pattern of 2^(s-17) (s <= 25: always a normal float).
__device__ __forceinline__ float shift_scale(uint32_t s) { return __uint_as_float((s + 110u) << 23); }

// ---------------------------------------------------------------- cross-lane
// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i within 8 lanes
constexpr int kDppRowRor8 = 0x128;     // rotate by 8 within 16 lanes

template <int Ctrl>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), Ctrl, 0xF, 0xF, true));
}

template <int Ctrl>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), Ctrl, 0xF, 0xF, true));
}

// Max over the 16 lanes of an aligned DPP row (one G32 group of a row when
// lane l holds channels 2l and 2l+1); every lane gets it.
__device__ __forceinline__ uint32_t row16_max(uint32_t x) {
    x = max(x, dpp_u<kDppQuadXor1>(x));
    x = max(x, dpp_u<kDppQuadXor2>(x));
    x = max(x, dpp_u<kDppHalfMirror>(x));
    return max(x, dpp_u<kDppRowRor8>(x));
}

// Sum over the 8 lanes of an aligned octet; every lane gets the same bits
// (each step adds a value and its partner in commutative order).
__device__ __forceinline__ float octet_sum(float x) {
    x += dpp_f<kDppQuadXor1>(x);
    x += dpp_f<kDppQuadXor2>(x);
    x += dpp_f<kDppHalfMirror>(x);
    return x;
}

// Max / sum across the 8 octets of a wave (lanes l, l^8, l^16, ...).
__device__ __forceinline__ float across_octets_max(float x) {
    x = fmaxf(x, dpp_f<kDppRowRor8>(x));
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}
__device__ __forceinline__ float across_octets_sum(float x) {
    x += dpp_f<kDppRowRor8>(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- append

template <bool Q17>
__device__ __forceinline__ int2 load_pair(const void* base, size_t elem) {
    if constexpr (Q17) {
        return *reinterpret_cast<const int2*>(static_cast<const int32_t*>(base) + elem);
    } else {
        const float2 f = *reinterpret_cast<const float2*>(static_cast<const float*>(base) + elem);
        return make_int2(f32_to_q17(f.x), f32_to_q17(f.y));
    }
}

// Split-K partial reduction of the upstream linear stage, in its fixed order:
// the pair sums fl(p0 + p1) and fl(p2 + p3), then their sum
// (int4_linear_controller.cpp:1039-1054 adds two FP32 lanes; :1655-1660 pairs
// partials 0+1 and 2+3; :1100-1118 adds the two pair sums, then converts).
// IEEE round-to-nearest-even adds, never reassociated or contracted.  The
// conversion that follows saturates a NaN by its sign bit, so a NaN sum takes
// a defined sign: that of a NaN operand (the first, if both are NaN), or, for
// inf - inf, the negative default NaN that x86 SSE arithmetic (the platform of
// the reference's C model) produces.  Selects, not branches: a branch here
// splits the step's prologue into blocks at whose join the compiler waits for
// every load in flight, the first cache block included.
__device__ __forceinline__ float add_partials(float a, float b) {
    const float s = __fadd_rn(a, b);
    const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b), us = __float_as_uint(s);
    const uint32_t nan_sum = (ua << 1) > 0xff000000u ? ua : ((ub << 1) > 0xff000000u ? ub : 0xffc00000u);
    return __uint_as_float((us << 1) > 0xff000000u ? nan_sum : us);
}

template <int NP>
__device__ __forceinline__ float reduce_parts(const float* p) {
    static_assert(NP == 2 || NP == 4, "the reference reduces pairs, then pairs of pairs");
    if constexpr (NP == 2) return add_partials(p[0], p[1]);
    else return add_partials(add_partials(p[0], p[1]), add_partials(p[2], p[3]));
}

// Raw input bits of channels (elem, elem+1) -- FP32 or Q15.17, or the NP
// split-K FP32 partials -- and their later conversion to Q15.17, so the loads
// can be issued well before the values are needed.
template <int IN>
struct InPair {
    int2 p[IN >= 2 ? IN : 1];
};

template <int IN>
__device__ __forceinline__ InPair<IN> load_in(const void* base, size_t elem, int64_t part_stride) {
    InPair<IN> r;
    const int32_t* src = static_cast<const int32_t*>(base) + elem;
#pragma unroll
    for (int j = 0; j < (IN >= 2 ? IN : 1); ++j)
        r.p[j] = *reinterpret_cast<const int2*>(src + j * part_stride);
    return r;
}

template <int IN>
__device__ __forceinline__ int2 in_to_q17(const InPair<IN>& in) {
    if constexpr (IN == kInQ17) {
        return in.p[0];
    } else if constexpr (IN == kInF32) {
        return make_int2(f32_to_q17(__int_as_float(in.p[0].x)), f32_to_q17(__int_as_float(in.p[0].y)));
    } else {
        float x[IN], y[IN];
#pragma unroll
        for (int j = 0; j < IN; ++j) {
            x[j] = __int_as_float(in.p[j].x);
            y[j] = __int_as_float(in.p[j].y);
        }
        return make_int2(f32_to_q17(reduce_parts<IN>(x)), f32_to_q17(reduce_parts<IN>(y)));
    }
}

// Quantize this wave's (k rotated, v) row and write it at token `pos` of
// `page`.  Lane l holds channels 2l, 2l+1; G32 group g = lanes 16g..16g+15.
// Returns the lane's code bytes and its group's shifts.
struct RowCodes {
    uint32_t k0, k1, v0, v1;   // code bytes
    uint32_t sk, sv;           // G32 shifts of the lane's group
};

__device__ __forceinline__ RowCodes row_codes(int32_t k0, int32_t k1, int32_t v0, int32_t v1) {
    const uint32_t mk = row16_max(max(magnitude(k0), magnitude(k1)));
    const uint32_t mv = row16_max(max(magnitude(v0), magnitude(v1)));
    RowCodes rc;
    rc.sk = g32_shift(mk);
    rc.sv = g32_shift(mv);
    rc.k0 = g32_code_byte(k0, rc.sk);
    rc.k1 = g32_code_byte(k1, rc.sk);
    rc.v0 = g32_code_byte(v0, rc.sv);
    rc.v1 = g32_code_byte(v1, rc.sv);
    return rc;
}

// The row's stores through a buffer resource over the page: 32-bit lane
// offsets, the row's offset in an SGPR.
__device__ __forceinline__ void store_row(__amdgpu_buffer_rsrc_t page, int seq_cap, int pos, int lane,
                                          const RowCodes& rc) {
    __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(rc.k0 | (rc.k1 << 8)), page, lane * 2,
                                          pos * kCodeBytes, 0);
    __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(rc.v0 | (rc.v1 << 8)), page, lane * 2,
                                          (seq_cap + pos) * kCodeBytes, 0);
    if ((lane & 15) == 0) {
        const v2f sc = {shift_scale(rc.sk), shift_scale(rc.sv)};
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, sc), page, (lane >> 4) * 8,
                                              seq_cap * (2 * kCodeBytes) + pos * kScaleBytes, 0);
    }
}

__device__ __forceinline__ RowCodes append_row_codes(int8_t* page, int seq_cap, int pos, int lane, int32_t k0,
                                                     int32_t k1, int32_t v0, int32_t v1) {
    const RowCodes rc = row_codes(k0, k1, v0, v1);
    const int64_t row = static_cast<int64_t>(pos) * kCodeBytes;
    reinterpret_cast<uint16_t*>(page + row)[lane] = static_cast<uint16_t>(rc.k0 | (rc.k1 << 8));
    reinterpret_cast<uint16_t*>(page + static_cast<int64_t>(seq_cap) * kCodeBytes + row)[lane] =
        static_cast<uint16_t>(rc.v0 | (rc.v1 << 8));
    if ((lane & 15) == 0) {
        float2* sc = reinterpret_cast<float2*>(page + static_cast<int64_t>(seq_cap) * (2 * kCodeBytes) +
                                               static_cast<int64_t>(pos) * kScaleBytes);
        sc[lane >> 4] = make_float2(shift_scale(rc.sk), shift_scale(rc.sv));
    }
    return rc;
}

// The same, returning the dequantized values code * 2^(s-17) of the lane's channels.
__device__ __forceinline__ void append_row_dequant(int8_t* page, int seq_cap, int pos, int lane, int32_t k0,
                                                   int32_t k1, int32_t v0, int32_t v1, float& kh0, float& kh1,
                                                   float& vh0, float& vh1) {
    const RowCodes rc = append_row_codes(page, seq_cap, pos, lane, k0, k1, v0, v1);
    const float fk = shift_scale(rc.sk), fv = shift_scale(rc.sv);
    kh0 = static_cast<float>(static_cast<int8_t>(rc.k0)) * fk;
    kh1 = static_cast<float>(static_cast<int8_t>(rc.k1)) * fk;
    vh0 = static_cast<float>(static_cast<int8_t>(rc.v0)) * fv;
    vh1 = static_cast<float>(static_cast<int8_t>(rc.v1)) * fv;
}

__device__ __forceinline__ void append_row(int8_t* page, int seq_cap, int pos, int lane, int32_t k0, int32_t k1,
                                           int32_t v0, int32_t v1) {
    float a, b, c, d;
    append_row_dequant(page, seq_cap, pos, lane, k0, k1, v0, v1, a, b, c, d);
}

}  // namespace dev
}  // namespace swiftkv
