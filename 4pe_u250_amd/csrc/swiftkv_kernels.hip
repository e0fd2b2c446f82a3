// swiftkv_kernels.hip -- CDNA4 (gfx950) kernels of the SwiftKV decode-attention
// stage.  Three kernels per decode step:
//
//   append   one wavefront per (sequence, head).  Lane l owns RoPE pair l
//            (channels 2l, 2l+1): FP32 -> Q15.17, integer rotation, G32
//            max by a 16-lane butterfly (one G32 group = 16 lanes), INT8
//            codes, and the appended row (128-B coalesced code rows and the
//            scale pair).  Also writes the rotated query as FP32.
//   attend   split-context scan (flash-decoding).  A 256-thread workgroup
//            scans split_tokens tokens of one (sequence, head); each wave
//            takes 64-token blocks.  Lane = (chunk c = lane&7, row r =
//            lane>>3): one dwordx4 per lane reads a 16-channel chunk, so one
//            wave instruction reads 8 full 128-B code rows.  INT8 codes are
//            dequantized in VGPRs, partial dots are reduced over the 8 chunk
//            lanes with DPP, and the running (max, sum, acc) lives in VGPRs.
//            Waves merge through LDS; one partial (m, l, acc[128]) per split.
//   combine  log-sum-exp merge of the splits per (sequence, head), the FP32
//            output, and optionally the A14/E8M0 epilogue.
//
// No MFMA: q_len = 1 multi-head attention is a memory-bound GEMV.
#include "swiftkv_device.hpp"

namespace swiftkv {
namespace {

using namespace dev;

// Grid (8, batch): 4 waves per workgroup, wave = head.
template <bool Q17>
__global__ __launch_bounds__(256) void append_step_kernel(StepArgs a) {
    const int b = blockIdx.y;
    const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int pos = a.positions[b];
    const size_t elem = static_cast<size_t>(b) * kModelDim + h * kHeadDim + 2 * lane;
    const int2 cs = a.lut[static_cast<size_t>(pos) * kRopePairs + lane];
    const int2 qi = load_pair<Q17>(a.q, elem);
    const int2 ki = load_pair<Q17>(a.k, elem);
    const int2 vi = load_pair<Q17>(a.v, elem);
    int32_t q0, q1, k0, k1;
    rope_pair(qi.x, qi.y, cs, q0, q1);
    rope_pair(ki.x, ki.y, cs, k0, k1);
    reinterpret_cast<float2*>(a.qhat)[elem >> 1] =
        make_float2(static_cast<float>(q0) * 0x1p-17f, static_cast<float>(q1) * 0x1p-17f);
    append_row(page_ptr(a.kv, a.slot0 + b, a.layer, h), a.kv.seq_cap, pos, lane, k0, k1, vi.x, vi.y);
}

// Grid (n, 8): token t = blockIdx.x, wave = head.
template <bool Q17>
__global__ __launch_bounds__(256) void append_bulk_kernel(BulkArgs a) {
    const int t = blockIdx.x;
    const int h = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int pos = a.pos0 + t;
    const size_t elem = static_cast<size_t>(t) * kModelDim + h * kHeadDim + 2 * lane;
    const int2 cs = a.lut[static_cast<size_t>(pos) * kRopePairs + lane];
    const int2 ki = load_pair<Q17>(a.k, elem);
    const int2 vi = load_pair<Q17>(a.v, elem);
    int32_t k0, k1;
    rope_pair(ki.x, ki.y, cs, k0, k1);
    append_row(page_ptr(a.kv, a.slot, a.layer, h), a.kv.seq_cap, pos, lane, k0, k1, vi.x, vi.y);
}

__global__ __launch_bounds__(256) void convert_kernel(const float* __restrict__ in, int32_t* __restrict__ out,
                                                      size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = f32_to_q17(in[i]);
}

// ---------------------------------------------------------------- attend

// 16 int8 codes of one dwordx4 times 16 query values.
__device__ __forceinline__ float dot16(const float* q, int4 w) {
    const int32_t d[4] = {w.x, w.y, w.z, w.w};
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int byte = 0; byte < 4; ++byte) {
            const float code = static_cast<float>(static_cast<int8_t>(d[j] >> (8 * byte)));
            acc = __builtin_fmaf(q[4 * j + byte], code, acc);
        }
    }
    return acc;
}

__device__ __forceinline__ void axpy16(float* acc, float w, int4 v) {
    const int32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int byte = 0; byte < 4; ++byte) {
            const float code = static_cast<float>(static_cast<int8_t>(d[j] >> (8 * byte)));
            acc[4 * j + byte] = __builtin_fmaf(w, code, acc[4 * j + byte]);
        }
    }
}

// Grid (splits, 32 heads, batch), 256 threads.
__global__ __launch_bounds__(kAttendWaves * 64) void attend_kernel(StepArgs a) {
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int len = a.positions[b] + 1;
    const int t_begin = split * a.split_tokens;
    if (t_begin >= len) return;
    const int t_end = min(t_begin + a.split_tokens, len);

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = lane & 7, r = lane >> 3;
    const int8_t* page = page_ptr(a.kv, a.slot0 + b, a.layer, h);
    const int64_t cap = a.kv.seq_cap;
    const int8_t* kp = page + c * 16;
    const int8_t* vp = page + cap * kCodeBytes + c * 16;
    const float* sp = reinterpret_cast<const float*>(page + cap * (2 * kCodeBytes)) + (c >> 1) * 2;

    // Query chunk, pre-scaled by 1/sqrt(128) * log2(e): scores live in the
    // log2 domain so the softmax uses v_exp_f32 directly.
    const float kScoreScale = (1.0f / 11.313708498984761f) * 1.4426950408889634f;
    float qf[16];
    {
        const float4* qs = reinterpret_cast<const float4*>(a.qhat + static_cast<size_t>(b) * kModelDim +
                                                           h * kHeadDim + c * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 x = qs[j];
            qf[4 * j + 0] = x.x * kScoreScale;
            qf[4 * j + 1] = x.y * kScoreScale;
            qf[4 * j + 2] = x.z * kScoreScale;
            qf[4 * j + 3] = x.w * kScoreScale;
        }
    }

    float m_run = -INFINITY, l_run = 0.0f;
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;

    for (int t0 = t_begin + wave * kBlockTokens; t0 < t_end; t0 += kAttendWaves * kBlockTokens) {
        int4 kw[8], vw[8];
        float2 sw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t t = t0 + 8 * i + r;
            kw[i] = *reinterpret_cast<const int4*>(kp + t * kCodeBytes);
            sw[i] = *reinterpret_cast<const float2*>(sp + t * 8);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t t = t0 + 8 * i + r;
            vw[i] = *reinterpret_cast<const int4*>(vp + t * kCodeBytes);
        }
        float s[8];
        float blk = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float d = octet_sum(dot16(qf, kw[i]) * sw[i].x);
            s[i] = (t0 + 8 * i + r < t_end) ? d : -INFINITY;
            blk = fmaxf(blk, s[i]);
        }
        blk = across_octets_max(blk);
        const float m_new = fmaxf(m_run, blk);
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const bool valid = t0 + 8 * i + r < t_end;
            const float p = valid ? fast_exp2(s[i] - m_new) : 0.0f;
            l_run += p;
            axpy16(acc, valid ? p * sw[i].y : 0.0f, vw[i]);
        }
    }

    // Reduce over the 8 rows (token phases) of the wave.
    l_run = across_octets_sum(l_run);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = across_octets_sum(acc[j]);

    __shared__ float s_acc[kAttendWaves][kHeadDim];
    __shared__ float s_m[kAttendWaves], s_l[kAttendWaves];
    if (r == 0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) s_acc[wave][c * 16 + j] = acc[j];
        if (c == 0) {
            s_m[wave] = m_run;
            s_l[wave] = l_run;
        }
    }
    __syncthreads();
    if (threadIdx.x < kHeadDim) {
        const int d = threadIdx.x;
        float mx = s_m[0];
#pragma unroll
        for (int w = 1; w < kAttendWaves; ++w) mx = fmaxf(mx, s_m[w]);
        float o = 0.0f, l = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttendWaves; ++w) {
            const float sc = fast_exp2(s_m[w] - mx);   // waves with no tokens: 2^-inf = 0
            o += sc * s_acc[w][d];
            l += sc * s_l[w];
        }
        float* part = a.partials +
                      ((static_cast<size_t>(b) * kHeads + h) * a.max_splits + split) * kPartialStride;
        part[4 + d] = o;
        if (d == 0) {
            part[0] = mx;
            part[1] = l;
        }
    }
}

// ---------------------------------------------------------------- combine

// Grid (32 heads, batch), 128 threads: thread d = output channel d.
__global__ __launch_bounds__(kHeadDim) void combine_kernel(StepArgs a) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int len = a.positions[b] + 1;
    const int n = (len + a.split_tokens - 1) / a.split_tokens;
    const float* part = a.partials + (static_cast<size_t>(b) * kHeads + h) * a.max_splits * kPartialStride;
    float mx = -INFINITY;
    for (int j = 0; j < n; ++j) mx = fmaxf(mx, part[j * kPartialStride]);
    float num = 0.0f, den = 0.0f;
    for (int j = 0; j < n; ++j) {
        const float w = fast_exp2(part[j * kPartialStride] - mx);
        den += w * part[j * kPartialStride + 1];
        num += w * part[j * kPartialStride + 4 + d];
    }
    const float o = num / den;
    a.out[static_cast<size_t>(b) * kModelDim + h * kHeadDim + d] = o;

    if (a.act_q == nullptr) return;
    // A14/G32 + E8M0 (swiftkv_attention.cpp:1715-1771, 2656-2682): per 32
    // outputs, e = frexp exponent of max|o|, q = trunc(clamp(o*2^(13-e) +-
    // 0.5, +-8191)), code = e + 127 (0 for an all-zero group).
    float mx_abs = fabsf(o);
#pragma unroll
    for (int s = 1; s < 32; s <<= 1) mx_abs = fmaxf(mx_abs, __shfl_xor(mx_abs, s));
    int e = 0;
    int16_t q14 = 0;
    uint8_t code = 0;
    if (mx_abs != 0.0f) {
        (void)frexpf(mx_abs, &e);
        const float inv = ldexpf(1.0f, 13 - e);
        const float sc = __fmul_rn(o, inv);
        float rr = sc >= 0.0f ? __fadd_rn(sc, 0.5f) : __fsub_rn(sc, 0.5f);
        rr = fminf(fmaxf(rr, -8191.0f), 8191.0f);
        q14 = static_cast<int16_t>(static_cast<int>(rr));
        code = static_cast<uint8_t>(e + 127);
    }
    __shared__ int16_t s_q[kHeadDim];
    s_q[d] = q14;
    __syncthreads();
    const size_t grp0 = static_cast<size_t>(b) * (kHeads * kGroupsPerHead) + h * kGroupsPerHead;
    if ((d & 31) == 0) a.act_scale[grp0 + (d >> 5)] = code;
    // 4 groups x 14 dwords of packed 14-bit lanes (lane i at bits [14i, 14i+13]).
    if (d < kGroupsPerHead * 14) {
        const int g = d / 14, w = d % 14;
        uint32_t word = 0;
        const int bit0 = 32 * w;
        for (int i = bit0 / 14; i <= (bit0 + 31) / 14 && i < 32; ++i) {
            const uint32_t val = static_cast<uint32_t>(static_cast<uint16_t>(s_q[g * 32 + i])) & 0x3fffu;
            const int sh = 14 * i - bit0;
            word |= sh >= 0 ? (val << sh) : (val >> -sh);
        }
        reinterpret_cast<uint32_t*>(a.act_q + (grp0 + g) * 56)[w] = word;
    }
}

}  // namespace

// ---------------------------------------------------------------- launchers

hipError_t launch_append_step(const StepArgs& a, bool q17, hipStream_t s) {
    const dim3 grid(kHeads / 4, a.batch);
    if (q17) append_step_kernel<true><<<grid, 256, 0, s>>>(a);
    else append_step_kernel<false><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_attend(const StepArgs& a, int grid_splits, hipStream_t s) {
    attend_kernel<<<dim3(grid_splits, kHeads, a.batch), kAttendWaves * 64, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_combine(const StepArgs& a, hipStream_t s) {
    combine_kernel<<<dim3(kHeads, a.batch), kHeadDim, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_append_bulk(const BulkArgs& a, bool q17, hipStream_t s) {
    const dim3 grid(a.n, kHeads / 4);
    if (q17) append_bulk_kernel<true><<<grid, 256, 0, s>>>(a);
    else append_bulk_kernel<false><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_convert(const float* in, int32_t* out, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    convert_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(in, out, n);
    return hipGetLastError();
}

}  // namespace swiftkv
