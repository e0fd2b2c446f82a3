// swiftkv_kernels.hip -- CDNA4 (gfx950) kernels of the SwiftKV decode-attention
// stage.
//
// step kernel (one launch per decode step and layer), grid (splits, 32 heads,
// batch rows) of 4-wave workgroups (8 waves when the launch has at most one
// workgroup per CU and 512-token-multiple splits); workgroup (j, h, z) owns tokens
// [j*C, min((j+1)*C, position+1)) of head h of the sequence that row z names
// (rows come longest first, so a ragged batch does not end on long heads):
//   1. every lane loads its channel pair of the new row's q/k/v (Q15.17,
//      FP32, or the upstream linear stage's split-K FP32 partials, reduced in
//      the reference's order), then the first cache block, before any math;
//      it converts and rotates its q pair (integer RoPE from the Q1.17 table)
//      and gathers the 16 query channels of its chunk from its neighbours;
//   2. the workgroup whose range holds `position` also converts, rotates and
//      G32-quantizes the new K/V row, appends it to the cache, and forwards it
//      into its own merge as one more partial -- the new token is written once
//      and never read back (the reference does the same, hpp:37-41);
//   3. the waves scan the cached tokens in 64-token blocks.  Lane = (chunk
//      c = lane&7, row r = lane>>3): one nontemporal dwordx4 per lane reads a
//      16-channel chunk, so one wave instruction covers 8 full 128-B code
//      rows.  Codes are dequantized in VGPRs, partial dots reduced over the 8
//      chunk lanes with DPP, the running (max, sum, acc) stays in VGPRs;
//   4. waves (plus the forwarded row) merge through LDS;
//   5. a head held by one split is finished in place (FP32 output and the
//      optional A14/E8M0 words); otherwise each split publishes its partial
//      (m, l, acc[128]) and the last split of the head to arrive merges them
//      (log-sum-exp) and finishes the head -- no second kernel.
//
// No MFMA: q_len = 1 multi-head attention is a memory-bound GEMV.
#include "swiftkv_device.hpp"

// Split workspace of the allocation-free step entry (swiftkv_attention_f32_noalloc):
// every GPU the library runs on holds its own copy until the process ends.
// Host code never passes this name to a kernel (on the host it is only a
// stand-in for the symbol): bind_noalloc_scratch resolves the device address
// once per device and the entry passes that address.
static __device__ __align__(256) unsigned char scratch[swiftkv::kNoAllocScratchBytes];

namespace swiftkv {
namespace {

using namespace dev;

static_assert(kMaxSplits <= kHeadDim, "one merge thread per split statistic");

// Scores are kept in the log2 domain: the query is pre-scaled by
// 1/sqrt(128) * log2(e) so the softmax uses v_exp_f32 (2^x) directly.
constexpr float kScoreScale = (1.0f / 11.313708498984761f) * 1.4426950408889634f;

// The cache is streamed exactly once per step, so every cache load is
// nontemporal: it keeps the stream from displacing reusable lines in L2/MALL
// (streaming reads reach ~88% of HBM peak this way versus ~78% with
// default-policy loads).

// 16 int8 codes of one dwordx4 times 16 query values.
__device__ __forceinline__ float dot16(const float* q, v4i w) {
    const int32_t d[4] = {w[0], w[1], w[2], w[3]};
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

__device__ __forceinline__ void axpy16(float* acc, float w, v4i v) {
    const int32_t d[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int byte = 0; byte < 4; ++byte) {
            const float code = static_cast<float>(static_cast<int8_t>(d[j] >> (8 * byte)));
            acc[4 * j + byte] = __builtin_fmaf(w, code, acc[4 * j + byte]);
        }
    }
}

// ---------------------------------------------------------------- pieces

// A page is read through one buffer resource held in SGPRs: the per-lane
// offset is fixed for the whole scan and the token offset is a wave-uniform
// SGPR, so the 24 loads of a block need no per-load 64-bit address VGPRs.
// Reads past the page return zero instead of faulting.
struct PageReader {
    __amdgpu_buffer_rsrc_t rsrc;
    int32_t k_lane;       // lane's byte offset in the K plane (row r, chunk c)
    int32_t v_lane;       // the same in the V plane
    int32_t s_lane;       // lane's (K, V) scale pair of group c/2 in the scale plane
};

constexpr int kNontemporal = 2;                // cache policy: nt

__device__ __forceinline__ PageReader make_reader(const int8_t* page, int64_t cap, int c, int r) {
    PageReader pr;
    pr.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(page), static_cast<short>(0),
                                                static_cast<int32_t>(cap * kTokenBytes), kBufferWord3);
    pr.k_lane = r * kCodeBytes + c * 16;
    pr.v_lane = static_cast<int32_t>(cap * kCodeBytes) + r * kCodeBytes + c * 16;
    pr.s_lane = static_cast<int32_t>(cap * 2 * kCodeBytes) + r * kScaleBytes + (c >> 1) * 8;
    return pr;
}

// The 24 loads of one 64-token block: 8 x 16 B of K codes, 8 x 8 B of scale
// pairs, 8 x 16 B of V codes per lane.
struct BlockLoads {
    v4i k[8], v[8];
    v2f s[8];
};

__device__ __forceinline__ void issue_block(const PageReader& pr, int t0, BlockLoads& bl) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int32_t tok = t0 + 8 * i;
        bl.k[i] = __builtin_amdgcn_raw_buffer_load_b128(pr.rsrc, pr.k_lane, tok * kCodeBytes, kNontemporal);
        bl.s[i] = __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(pr.rsrc, pr.s_lane,
                                                                                tok * kScaleBytes, kNontemporal));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int32_t tok = t0 + 8 * i;
        bl.v[i] = __builtin_amdgcn_raw_buffer_load_b128(pr.rsrc, pr.v_lane, tok * kCodeBytes, kNontemporal);
    }
    // Keep all 24 loads in flight before any math: without this fence the
    // scheduler sinks V loads next to their uses (to save VGPRs) and
    // serializes them at full memory latency.
    __builtin_amdgcn_sched_barrier(0);
}

// Online-softmax update with one block [t0, t0+64); MASKED blocks drop
// tokens >= t_stop.
template <bool MASKED>
__device__ __forceinline__ void consume_block(const BlockLoads& bl, const float* qf, int t0, int t_stop, int r,
                                              float& m_run, float& l_run, float* acc) {
    float s[8];
    float blk = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        s[i] = octet_sum(dot16(qf, bl.k[i]) * bl.s[i][0]);
        if (MASKED && t0 + 8 * i + r >= t_stop) s[i] = -INFINITY;
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
        float p = fast_exp2(s[i] - m_new);            // masked: 2^-inf = 0
        float w = p * bl.s[i][1];
        if (MASKED && t0 + 8 * i + r >= t_stop) w = 0.0f;   // never multiply a stale scale
        l_run += p;
        axpy16(acc, w, bl.v[i]);
    }
}

// One wave's online-softmax scan over the 64-token blocks t0, t0+stride, ...
// below t_stop, lane layout (c, r); the caller has already issued the loads
// of the first block into `bl` (so its prologue overlaps them).  On return
// every lane holds the wave's (m, l) and, for its chunk c, acc[16] summed
// over the 8 rows.
__device__ __forceinline__ void scan_range(const PageReader& pr, BlockLoads& bl, const float* qf, int t0,
                                           int t_stop, int stride, int r, float& m_run, float& l_run,
                                           float* acc) {
    m_run = -INFINITY;
    l_run = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
    // Full blocks, then at most one partial tail block.  (Both variants in one
    // loop body would double the live VGPRs.)
    bool first = true;
    for (; t0 + kBlockTokens <= t_stop; t0 += stride, first = false) {
        if (!first) issue_block(pr, t0, bl);
        consume_block<false>(bl, qf, t0, t_stop, r, m_run, l_run, acc);
    }
    if (t0 < t_stop) {
        if (!first) issue_block(pr, t0, bl);
        consume_block<true>(bl, qf, t0, t_stop, r, m_run, l_run, acc);
    }
    l_run = across_octets_sum(l_run);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = across_octets_sum(acc[j]);
}

// Per-(sequence, head) output: FP32 row and, when requested, A14/G32 + E8M0
// (swiftkv_attention.cpp:1715-1771, 2656-2682): per 32 outputs, e = frexp
// exponent of max|o| clamped at -127, q = trunc(clamp(o*2^(13-e) +- 0.5,
// +-8191)), code = e + 127 (0 for an all-zero group).  Called by every thread of the block;
// threads d < 128 supply output channel d.
__device__ __forceinline__ void finalize_head(const StepArgs& a, int b, int h, float o) {
    const int d = threadIdx.x;
    const bool active = d < kHeadDim;
    if (active) a.out[static_cast<size_t>(b) * kModelDim + h * kHeadDim + d] = o;
    if (a.act_q == nullptr) return;
    float mx_abs = active ? fabsf(o) : 0.0f;
#pragma unroll
    for (int s = 1; s < 32; s <<= 1) mx_abs = fmaxf(mx_abs, __shfl_xor(mx_abs, s));
    int16_t q14 = 0;
    uint8_t code = 0;
    if (mx_abs != 0.0f) {
        // The reference clamps the group exponent at -127 (swiftkv_attention.cpp:1722-1724).
        // o * 2^(13-e) is formed with ldexpf: it equals the product with the
        // power of two wherever that power is a finite float, and stays finite
        // for a group max below 2^-115, where 2^(13-e) would overflow to inf.
        int e = 0;
        (void)frexpf(mx_abs, &e);
        e = max(e, -127);
        const float sc = ldexpf(o, 13 - e);
        float rr = sc >= 0.0f ? __fadd_rn(sc, 0.5f) : __fsub_rn(sc, 0.5f);
        rr = fminf(fmaxf(rr, -8191.0f), 8191.0f);
        q14 = static_cast<int16_t>(static_cast<int>(rr));
        code = static_cast<uint8_t>(e + 127);
    }
    __shared__ int16_t s_q14[kHeadDim];
    if (active) s_q14[d] = q14;
    __syncthreads();
    const size_t grp0 = static_cast<size_t>(b) * (kHeads * kGroupsPerHead) + h * kGroupsPerHead;
    if (active && (d & 31) == 0) a.act_scale[grp0 + (d >> 5)] = code;
    // 4 groups x 14 dwords of packed 14-bit lanes (lane i at bits [14i, 14i+13]).
    if (d < kGroupsPerHead * 14) {
        const int g = d / 14, w = d % 14;
        uint32_t word = 0;
        const int bit0 = 32 * w;
        for (int i = bit0 / 14; i <= (bit0 + 31) / 14 && i < 32; ++i) {
            const uint32_t val = static_cast<uint32_t>(static_cast<uint16_t>(s_q14[g * 32 + i])) & 0x3fffu;
            const int sh = 14 * i - bit0;
            word |= sh >= 0 ? (val << sh) : (val >> -sh);
        }
        reinterpret_cast<uint32_t*>(a.act_q + (grp0 + g) * 56)[w] = word;
    }
}

// Split partials are exchanged through device memory inside one launch.
// Writers publish with agent-scope atomic stores (write-through to the
// device coherence point, no dirty L2 lines) and wait for their completion;
// the last split of a head, identified by a device-scope counter, reads them
// back with agent-scope atomic loads.  No L2 writeback or invalidation is
// needed on either side.
__device__ __forceinline__ void publish(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float fetch(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Log-sum-exp merge of n split partials; threads d < 128 get output channel d.
// Every load of the merge goes out at once -- the split statistics (thread j
// loads split j) and thread d's accumulator column of the first kMergeInline
// splits -- so up to kMergeInline splits cost one memory round trip and one
// barrier.  Further splits (only when a caller forces small splits) are
// fetched in a second pass.  Every thread reduces the statistics in the same
// order, so all agree on the maximum and the denominator.
constexpr int kMergeInline = 8;

__device__ __forceinline__ float merge_partials(const float* part, int n) {
    const int d = threadIdx.x;
    __shared__ float s_m[kMaxSplits], s_l[kMaxSplits];
    float col[kMergeInline];
    if (d < n) {
        s_m[d] = fetch(part + d * kPartialStride);
        s_l[d] = fetch(part + d * kPartialStride + 1);
    }
#pragma unroll
    for (int j = 0; j < kMergeInline; ++j)
        col[j] = (d < kHeadDim && j < n) ? fetch(part + j * kPartialStride + 4 + d) : 0.0f;
    __syncthreads();
    float mx = s_m[0];
    for (int j = 1; j < n; ++j) mx = fmaxf(mx, s_m[j]);
    float den = 0.0f, num = 0.0f;
#pragma unroll
    for (int j = 0; j < kMergeInline; ++j) {
        if (j < n) {
            const float w = fast_exp2(s_m[j] - mx);
            den += w * s_l[j];
            num += w * col[j];
        }
    }
    for (int j = kMergeInline; j < n; ++j) {
        const float w = fast_exp2(s_m[j] - mx);
        den += w * s_l[j];
        if (d < kHeadDim) num += w * fetch(part + j * kPartialStride + 4 + d);
    }
    return num / den;
}

// ---------------------------------------------------------------- step

// Grid (splits, 32 heads, batch), 256 threads; grid row z serves rows[z].
template <int IN, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void step_kernel(StepArgs a) {
    const uint32_t row = a.rows[blockIdx.z];
    const int split = blockIdx.x, h = blockIdx.y, b = static_cast<int>(row & 0xffu);
    const int pos = static_cast<int>(row >> 8);
    const int len = pos + 1;
    const int C = a.split_tokens;
    const int t_begin = split * C;
    if (t_begin >= len) return;
    const int t_end = min(t_begin + C, len);
    const int nsplit = (len + C - 1) / C;
    const bool owner = pos < t_end;               // this split holds the new token

    // wave index made provably uniform so token offsets stay in SGPRs (the
    // buffer loads' soffset operand) instead of forcing waterfall loops
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int c = lane & 7, r = lane >> 3;
    int8_t* page = page_ptr(a.kv, a.slot0 + b, a.layer, h);
    const int64_t cap = a.kv.seq_cap;

    __shared__ float s_acc[WAVES + 1][kHeadDim];
    __shared__ float s_m[WAVES + 1], s_l[WAVES + 1];

    // Loads go out before any math, in the order they are needed: this
    // lane's channel pair (2*lane, 2*lane+1) of the new row's q, k, v and its
    // RoPE pair, then the first cache block.  The conversions below wait only
    // for the row loads (vector loads retire in issue order), so they overlap
    // the block's flight.  All of them are unconditional and in bounds: a
    // load under a branch makes the compiler wait for the prefetched block at
    // the join.
    const size_t row_elem = static_cast<size_t>(b) * kModelDim + h * kHeadDim + 2 * lane;
    const int2 row_cs = a.lut[static_cast<size_t>(pos) * kRopePairs + lane];
    const InPair<IN> row_q = load_in<IN>(a.q, row_elem, a.part_stride);
    const InPair<IN> row_k = load_in<IN>(a.k, row_elem, a.part_stride);
    const InPair<IN> row_v = load_in<IN>(a.v, row_elem, a.part_stride);
    const PageReader pr = make_reader(page, cap, c, r);
    const int t_first = t_begin + wave * kBlockTokens;
    const int t_stop = owner ? pos : t_end;       // the new token is forwarded, not scanned
    // A wave with no tokens loads the split's first block (always in the page)
    // and discards it: every path then has the same loads in flight.
    BlockLoads bl;
    issue_block(pr, t_first < t_stop ? t_first : t_begin, bl);

    // Query: each lane converts and rotates its own pair, pre-scales it, and
    // gathers the 16 channels of its chunk c (pairs 8c..8c+7, held by lanes
    // 8c..8c+7).  The new row's k is rotated and v converted here too, which
    // frees the raw row registers before the scan.
    const int2 qi = in_to_q17<IN>(row_q);
    int32_t q0, q1;
    rope_pair(qi.x, qi.y, row_cs, q0, q1);
    const float qs0 = (static_cast<float>(q0) * 0x1p-17f) * kScoreScale;
    const float qs1 = (static_cast<float>(q1) * 0x1p-17f) * kScoreScale;
    float qf[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        qf[2 * j] = __shfl(qs0, 8 * c + j);
        qf[2 * j + 1] = __shfl(qs1, 8 * c + j);
    }
    const int2 ki = in_to_q17<IN>(row_k), vi = in_to_q17<IN>(row_v);
    int32_t k0, k1;
    rope_pair(ki.x, ki.y, row_cs, k0, k1);

    float m_run, l_run, acc[16];
    scan_range(pr, bl, qf, t_first, t_stop, WAVES * kBlockTokens, r, m_run, l_run, acc);

    // The new row: quantize, append; forward (k^ . q', v^) into the merge as
    // one more partial.
    if (owner && wave == 0) {
        float kh0, kh1, vh0, vh1;
        append_row_dequant(page, a.kv.seq_cap, pos, lane, k0, k1, vi.x, vi.y, kh0, kh1, vh0, vh1);
        float sp = qs0 * kh0 + qs1 * kh1;
#pragma unroll
        for (int s = 1; s < 64; s <<= 1) sp += __shfl_xor(sp, s);
        s_acc[WAVES][2 * lane] = vh0;
        s_acc[WAVES][2 * lane + 1] = vh1;
        if (lane == 0) {
            s_m[WAVES] = sp;
            s_l[WAVES] = 1.0f;
        }
    }
    if (r == 0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) s_acc[wave][c * 16 + j] = acc[j];
        if (c == 0) {
            s_m[wave] = m_run;
            s_l[wave] = l_run;
        }
    }
    __syncthreads();

    const int nparts = owner ? WAVES + 1 : WAVES;
    const int d = threadIdx.x;
    float o = 0.0f, l = 0.0f, mx = -INFINITY;
    if (d < kHeadDim) {
        mx = s_m[0];
        for (int w = 1; w < nparts; ++w) mx = fmaxf(mx, s_m[w]);
        for (int w = 0; w < nparts; ++w) {
            const float sc = fast_exp2(s_m[w] - mx);     // parts with no tokens: 2^-inf = 0
            o += sc * s_acc[w][d];
            l += sc * s_l[w];
        }
    }
    if (nsplit == 1) {
        finalize_head(a, b, h, o / l);
        return;
    }

    // Several splits: publish this split's partial, count arrivals, and let
    // the last split of the head merge all partials and finish the head.
    const size_t head_row = static_cast<size_t>(b) * kHeads + h;
    float* parts = a.partials + head_row * a.max_splits * kPartialStride;
    if (d < kHeadDim) {
        float* part = parts + static_cast<size_t>(split) * kPartialStride;
        publish(part + 4 + d, o);
        if (d == 0) {
            publish(part, mx);
            publish(part + 1, l);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);   // this thread's stores are complete before the barrier
    __syncthreads();
    __shared__ int s_last;
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(a.counters + head_row * kCounterStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 static_cast<unsigned>(nsplit - 1);
    __syncthreads();
    if (!s_last) return;
    finalize_head(a, b, h, merge_partials(parts, nsplit));
    if (threadIdx.x == 0)   // ready for the next launch
        __hip_atomic_store(a.counters + head_row * kCounterStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- utilities

constexpr int kAppendTokens = 2;   // prefill rows per wave (their loads in flight together)

// Grid (ceil(n / kAppendTokens), 8): wave = head (4 per workgroup), each
// wave kAppendTokens consecutive tokens.  All of the wave's loads (k, v and
// the RoPE pair of every token) go out before any row is quantized, so a
// wave keeps kAppendTokens rows in flight; tokens past n load the last token
// and store nothing.
template <bool Q17>
__global__ __launch_bounds__(256) void append_bulk_kernel(BulkArgs a) {
    // wave-uniform through readfirstlane, so the page's buffer resource stays in SGPRs
    const int h = blockIdx.y * 4 + __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * kAppendTokens;
    int2 cs[kAppendTokens], ki[kAppendTokens], vi[kAppendTokens];
#pragma unroll
    for (int j = 0; j < kAppendTokens; ++j) {
        const int t = min(t0 + j, a.n - 1);
        const size_t elem = static_cast<size_t>(t) * kModelDim + h * kHeadDim + 2 * lane;
        cs[j] = a.lut[static_cast<size_t>(a.pos0 + t) * kRopePairs + lane];
        ki[j] = load_pair<Q17>(a.k, elem);
        vi[j] = load_pair<Q17>(a.v, elem);
    }
    const __amdgpu_buffer_rsrc_t page = __builtin_amdgcn_make_buffer_rsrc(
        page_ptr(a.kv, a.slot, a.layer, h), static_cast<short>(0), static_cast<int32_t>(a.kv.page_bytes), kBufferWord3);
#pragma unroll
    for (int j = 0; j < kAppendTokens; ++j) {
        if (t0 + j >= a.n) break;
        int32_t k0, k1;
        rope_pair(ki[j].x, ki[j].y, cs[j], k0, k1);
        store_row(page, a.kv.seq_cap, a.pos0 + t0 + j, lane, row_codes(k0, k1, vi[j].x, vi[j].y));
    }
}

// out[i] = Q15.17 of in[i] (NP = 1) or of the NP reduced split-K partials.
template <int NP>
__global__ __launch_bounds__(256) void convert_kernel(const float* __restrict__ in, int64_t part_stride,
                                                      int32_t* __restrict__ out, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        if constexpr (NP == 1) {
            out[i] = f32_to_q17(in[i]);
        } else {
            float p[NP];
#pragma unroll
            for (int j = 0; j < NP; ++j) p[j] = in[i + j * part_stride];
            out[i] = f32_to_q17(reduce_parts<NP>(p));
        }
    }
}

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* __restrict__ p, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

}  // namespace

// ---------------------------------------------------------------- launchers

hipError_t bind_noalloc_scratch(hipStream_t s, void** device_ptr) {
    static_assert(kNoAllocScratchBytes % 4 == 0 && kNoAllocCounterBytes % 256 == 0, "workspace layout");
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    const size_t words = kNoAllocScratchBytes / 4;
    zero_words_kernel<<<1024, 256, 0, s>>>(static_cast<uint32_t*>(p), words);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
    *device_ptr = p;
    return hipSuccess;
}

template <int WAVES>
hipError_t launch_step_waves(const StepArgs& a, dim3 grid, InputFormat in, hipStream_t s) {
    const dim3 block(WAVES * 64);
    switch (in) {
    case kInF32: step_kernel<kInF32, WAVES><<<grid, block, 0, s>>>(a); break;
    case kInQ17: step_kernel<kInQ17, WAVES><<<grid, block, 0, s>>>(a); break;
    case kInParts2: step_kernel<kInParts2, WAVES><<<grid, block, 0, s>>>(a); break;
    case kInParts4: step_kernel<kInParts4, WAVES><<<grid, block, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

int step_workgroups_per_cu() {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, step_kernel<kInF32, kAttendWaves>, kAttendWaves * 64, 0) !=
        hipSuccess)
        return 0;
    return n;
}

hipError_t launch_step(const StepArgs& a, int grid_splits, int waves, InputFormat in, hipStream_t s) {
    const dim3 grid(grid_splits, kHeads, a.batch);
    if (waves == kAttendWaves) return launch_step_waves<kAttendWaves>(a, grid, in, s);
    if (waves == kWideWaves && a.split_tokens % (kWideWaves * kBlockTokens) == 0)
        return launch_step_waves<kWideWaves>(a, grid, in, s);
    return hipErrorInvalidValue;
}

hipError_t launch_append_bulk(const BulkArgs& a, bool q17, hipStream_t s) {
    const dim3 grid((a.n + kAppendTokens - 1) / kAppendTokens, kHeads / 4);
    if (q17) append_bulk_kernel<true><<<grid, 256, 0, s>>>(a);
    else append_bulk_kernel<false><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_convert(const float* in, int32_t parts, int64_t part_stride, int32_t* out, size_t n,
                          hipStream_t s) {
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    const unsigned g = static_cast<unsigned>(blocks);
    switch (parts) {
    case 1: convert_kernel<1><<<g, 256, 0, s>>>(in, part_stride, out, n); break;
    case 2: convert_kernel<2><<<g, 256, 0, s>>>(in, part_stride, out, n); break;
    case 4: convert_kernel<4><<<g, 256, 0, s>>>(in, part_stride, out, n); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace swiftkv
