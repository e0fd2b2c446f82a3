// swiftkv_kernels.hip -- CDNA4 (gfx950) kernels of the SwiftKV decode-attention
// stage.
//
// step kernel (one launch per decode step and layer), grid (splits, 32 heads,
// batch rows) of workgroups in one of three shapes, chosen by the host per
// launch: 8 waves on 32-token blocks for launches of up to one residency round
// of 4-wave workgroups, 8 waves on 64-token blocks for larger launches whose
// every range holds at least 2048 tokens, 4 waves on 64-token blocks for the
// rest; workgroup (j, h, z) owns tokens
// [j*C, min((j+1)*C, position+1)) of head h of the sequence that row z names
// (rows come longest first, so a ragged batch does not end on long heads):
//   1. every lane loads its channel pair of the new row's q (and, in the one
//      wave that appends the row, of k and v) -- Q15.17, FP32, or the
//      upstream linear stage's split-K FP32 partials, reduced in the
//      reference's order -- then the first cache block, before any math; it
//      converts and rotates its q pair (integer RoPE from the Q1.17 table),
//      splits it into signed-byte limbs and gathers the limbs of its chunk's
//      16 query channels from its neighbours;
//   2. the workgroup whose range holds `position` also converts, rotates and
//      G32-quantizes the new K/V row, appends it to the cache, and forwards it
//      into its own merge as one more partial -- the new token is written once
//      and never read back (the reference does the same, hpp:37-41);
//   3. the waves scan the cached tokens in blocks taken round-robin.
//      Lane = (chunk c = lane&7, row r = lane>>3): one nontemporal
//      dwordx4 per lane reads a 16-channel chunk, so one wave instruction
//      covers 8 full 128-B code rows.  K rows are dotted with the query limbs
//      by v_dot4 on the int8 codes, V codes are dequantized in VGPRs, partial
//      dots reduced over the 8 chunk lanes with DPP, the running (max, sum,
//      acc) stays in VGPRs;
//   4. waves (plus the forwarded row) merge through LDS;
//   5. a head held by one split is finished in place (FP32 output and the
//      optional A14/E8M0 words); otherwise each split publishes its partial
//      (m, l, acc[128]) as tagged words and the last split of the head to
//      count its arrival merges them (log-sum-exp, in split order) and
//      finishes the head -- no second kernel.
//
// No MFMA: q_len = 1 multi-head attention is a memory-bound GEMV.
#include "swiftkv_device.hpp"

// Split workspace of the allocation-free step entry (swiftkv_attention_f32_noalloc):
// every GPU the library runs on holds its own copy until the process ends.
// Host code never passes this name to a kernel (on the host it is only a
// stand-in for the symbol): bind_noalloc_scratch resolves the device address
// once per device and the entry passes that address.
static __device__ __align__(256) unsigned char scratch[swiftkv::kNoAllocScratchBytes];

#include "swiftkv_stamps.hpp"

namespace swiftkv {
namespace {

using namespace dev;

static_assert(kMaxSplits <= 4 * 64, "one merge thread per split statistic (workgroups have >= 4 waves)");

// Scores are kept in the log2 domain: the query is pre-scaled by
// 1/sqrt(128) * log2(e) so the softmax uses v_exp_f32 (2^x) directly.
constexpr float kScoreScale = (1.0f / 11.313708498984761f) * 1.4426950408889634f;

// The cache is streamed exactly once per step, so every cache load is
// nontemporal: it keeps the stream from displacing reusable lines in L2/MALL
// (streaming reads reach ~88% of HBM peak this way versus ~78% with
// default-policy loads).

// The rotated query of a lane's 16-channel chunk as three signed-byte limbs:
// m_c = q'_c / 2^E rounded, m_c = l0 + 2^8 l1 + 2^16 l2, with the chunk's
// shift E = max(0, msb(max_c |q'_c|) - 21), so |m_c| <= 2^22 and l2 stays
// within +-64.  The K dot product is then four signed-byte v_dot4 per limb
// against the int8 codes, exact in integers; only its conversion to float
// rounds.  For |q| below 16 (Q15.17 words below 2^21) E = 0 and the products
// are the exact ones; above, m keeps 22 significant bits.  `scale` =
// 2^(E-17) * kScoreScale turns the integer dot into the log2-domain score.
struct QueryChunk {
    int32_t w[3][4];   // limb k of channels 4j .. 4j+3, one byte each, in dword j
    float scale;
};

// Lane l holds the rotated pair (q0, q1) = channels (2l, 2l+1), so chunk c
// (channels 16c .. 16c+15) lives in lanes 8c .. 8c+7 and is consumed by the
// lanes with lane & 7 == c.  Each lane splits its own pair, with the shift of
// its chunk (a DPP maximum over its octet); two neighbouring lanes join their
// 16-bit limb halves, and each consumer reads its four dwords per limb.
__device__ __forceinline__ QueryChunk chunk_limbs(int32_t q0, int32_t q1, int c) {
    uint32_t mx = max(magnitude(q0), magnitude(q1));
    mx = max(mx, dpp_u<kDppQuadXor1>(mx));
    mx = max(mx, dpp_u<kDppQuadXor2>(mx));
    mx = max(mx, dpp_u<kDppHalfMirror>(mx));
    const int msb = mx ? 31 - static_cast<int>(__clz(mx)) : 0;
    const int e = max(0, msb - 21);
    uint32_t half[3] = {0u, 0u, 0u};
    const int32_t pair[2] = {q0, q1};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int32_t v = pair[i];
        const int32_t m = e ? (v >> e) + ((v >> (e - 1)) & 1) : v;   // half up; |m| <= 2^22
        const int32_t l0 = static_cast<int8_t>(static_cast<uint8_t>(m));
        const int32_t r = (m - l0) >> 8;
        const int32_t l1 = static_cast<int8_t>(static_cast<uint8_t>(r));
        const int32_t l2 = (r - l1) >> 8;
        half[0] |= static_cast<uint32_t>(static_cast<uint8_t>(l0)) << (8 * i);
        half[1] |= static_cast<uint32_t>(static_cast<uint8_t>(l1)) << (8 * i);
        half[2] |= static_cast<uint32_t>(static_cast<uint8_t>(l2)) << (8 * i);
    }
    QueryChunk Q;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        // even lanes 2p: channels 4p .. 4p+3 of their octet's chunk (valid at even lanes)
        const uint32_t dword = half[k] | (dpp_u<kDppQuadXor1>(half[k]) << 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) Q.w[k][j] = static_cast<int32_t>(__shfl(dword, 8 * c + 2 * j));
    }
    Q.scale = ldexpf(kScoreScale, __shfl(e, 8 * c) - 17);
    return Q;
}

// 16 int8 codes of one dwordx4 times the chunk's query, as float (before
// the chunk and token scales): per limb the exact sum of 16 byte products
// (|sum| <= 16 * 128 * 128), limbs 0 and 1 combined exactly in 32 bits.
__device__ __forceinline__ float kdot16(const QueryChunk& Q, v4i w) {
    int32_t s[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        int32_t acc = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_sdot4(Q.w[k][j], w[j], acc, false);
        s[k] = acc;
    }
    const int32_t low = s[0] + s[1] * 256;   // |low| < 2^27
    return __builtin_fmaf(65536.0f, static_cast<float>(s[2]), static_cast<float>(low));
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
    int32_t past_end;     // added to a lane offset, puts any load of the page past its range
};

constexpr int kNontemporal = 2;                // cache policy: nt

__device__ __forceinline__ PageReader make_reader(const int8_t* page, int64_t cap, int c, int r) {
    PageReader pr;
    pr.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(page), static_cast<short>(0),
                                                static_cast<int32_t>(cap * kTokenBytes), kBufferWord3);
    pr.k_lane = r * kCodeBytes + c * 16;
    pr.v_lane = static_cast<int32_t>(cap * kCodeBytes) + r * kCodeBytes + c * 16;
    pr.s_lane = static_cast<int32_t>(cap * 2 * kCodeBytes) + r * kScaleBytes + (c >> 1) * 8;
    pr.past_end = static_cast<int32_t>(cap * kTokenBytes);   // <= 32768 * 288: lane offset + token offset stay < 2^31
    return pr;
}

// The loads of one block of 8 * NI tokens (NI rows per lane): NI x 16 B of K
// codes, NI x 8 B of scale pairs, NI x 16 B of V codes per lane -- 24 loads
// for a 64-token block.
template <int NI>
struct BlockLoads {
    v4i k[NI], v[NI];
    v2f s[NI];
};

template <int NI>
__device__ __forceinline__ void issue_block(const PageReader& pr, int t0, BlockLoads<NI>& bl) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int32_t tok = t0 + 8 * i;
        bl.k[i] = __builtin_amdgcn_raw_buffer_load_b128(pr.rsrc, pr.k_lane, tok * kCodeBytes, kNontemporal);
        bl.s[i] = __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(pr.rsrc, pr.s_lane,
                                                                                tok * kScaleBytes, kNontemporal));
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int32_t tok = t0 + 8 * i;
        bl.v[i] = __builtin_amdgcn_raw_buffer_load_b128(pr.rsrc, pr.v_lane, tok * kCodeBytes, kNontemporal);
    }
    // Keep all 24 loads in flight before any math: without this fence the
    // scheduler sinks V loads next to their uses (to save VGPRs) and
    // serializes them at full memory latency.
    __builtin_amdgcn_sched_barrier(0);
}

// The same loads for a block that may extend past t_stop: the rows at or past
// it get a lane offset beyond the page's buffer range, so the hardware's
// range check returns zeros for them without fetching (their scores and
// weights are masked anyway).  Used for the last block of a range, and for
// the first block of every wave: a wave with no tokens then issues its loads
// with every row masked and moves no data.
template <int NI>
__device__ __forceinline__ void issue_block_masked(const PageReader& pr, int t0, int t_stop, int r,
                                                   BlockLoads<NI>& bl) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int32_t tok = t0 + 8 * i;
        const int32_t past = tok + r >= t_stop ? pr.past_end : 0;
        bl.k[i] = __builtin_amdgcn_raw_buffer_load_b128(pr.rsrc, pr.k_lane + past, tok * kCodeBytes, kNontemporal);
        bl.s[i] = __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(pr.rsrc, pr.s_lane + past,
                                                                                tok * kScaleBytes, kNontemporal));
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int32_t tok = t0 + 8 * i;
        const int32_t past = tok + r >= t_stop ? pr.past_end : 0;
        bl.v[i] = __builtin_amdgcn_raw_buffer_load_b128(pr.rsrc, pr.v_lane + past, tok * kCodeBytes, kNontemporal);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Online-softmax update with one block [t0, t0 + 8 * NI); MASKED blocks drop
// tokens >= t_stop.
template <bool MASKED, int NI>
__device__ __forceinline__ void consume_block(const BlockLoads<NI>& bl, const QueryChunk& Q, int t0, int t_stop, int r,
                                              float& m_run, float& l_run, float* acc) {
    float s[NI];
    float blk = -INFINITY;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        s[i] = octet_sum(kdot16(Q, bl.k[i]) * (Q.scale * bl.s[i][0]));
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
    for (int i = 0; i < NI; ++i) {
        float p = fast_exp2(s[i] - m_new);            // masked: 2^-inf = 0
        float w = p * bl.s[i][1];
        if (MASKED && t0 + 8 * i + r >= t_stop) w = 0.0f;   // never multiply a stale scale
        l_run += p;
        axpy16(acc, w, bl.v[i]);
    }
}

// One wave's online-softmax scan over the blocks of 8 * NI tokens t0, t0+stride, ...
// below t_stop, lane layout (c, r); the caller has already issued the loads
// of the first block into `bl` (so its prologue overlaps them).  On return
// every lane holds the wave's (m, l) and, for its chunk c, acc[16] summed
// over the 8 rows.
template <int NI>
__device__ __forceinline__ void scan_range(const PageReader& pr, BlockLoads<NI>& bl, const QueryChunk& Q, int t0,
                                           int t_stop, int stride, int r, float& m_run, float& l_run,
                                           float* acc) {
    m_run = -INFINITY;
    l_run = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
    // Full blocks, then at most one partial tail block.  (Both variants in one
    // loop body would double the live VGPRs.)
    bool first = true;
    for (; t0 + 8 * NI <= t_stop; t0 += stride, first = false) {
        if (!first) issue_block(pr, t0, bl);
        consume_block<false, NI>(bl, Q, t0, t_stop, r, m_run, l_run, acc);
    }
    if (t0 < t_stop) {
        if (!first) issue_block_masked(pr, t0, t_stop, r, bl);
        consume_block<true, NI>(bl, Q, t0, t_stop, r, m_run, l_run, acc);
    }
    l_run = across_octets_sum(l_run);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = across_octets_sum(acc[j]);
}

// Max over the 16 lanes of an aligned DPP row, as float (every lane gets it).
__device__ __forceinline__ float row16_maxf(float x) {
    x = fmaxf(x, dpp_f<kDppQuadXor1>(x));
    x = fmaxf(x, dpp_f<kDppQuadXor2>(x));
    x = fmaxf(x, dpp_f<kDppHalfMirror>(x));
    return fmaxf(x, dpp_f<kDppRowRor8>(x));
}

__device__ __forceinline__ float readlane_f(float x, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Per-(sequence, head) output: FP32 row and, when requested, A14/G32 + E8M0
// (swiftkv_attention.cpp:1715-1771, 2656-2682): per 32 outputs, e = frexp
// exponent of max|o| clamped at -127, q = trunc(clamp(o*2^(13-e) +- 0.5,
// +-8191)), code = e + 127 (0 for an all-zero group).  Called by waves 0-1
// only, thread d supplying output channel d: each G32 group is one half-wave,
// so the group maximum (DPP within 16-lane rows, then the two rows of the
// half) and the packing of the 14-bit lanes (lane-to-lane reads) stay inside
// the wave, with no LDS and no barrier.
// The argument-block fields the end of a step uses: its outputs and the split
// exchange.  The step kernel loads them into SGPRs while its first loads are
// in flight; loaded where they are used, each was a scalar round trip ahead
// of the merge or the output stores.
struct StepTail {
    float* out;
    uint8_t* act_q;
    uint8_t* act_scale;
    uint64_t* partials;
    uint32_t* fault;
    int32_t slot_stride;
    uint32_t merge_tag_skew;
    uint32_t merge_polls;
    int32_t slot0;
};

__device__ __forceinline__ void finalize_head(const StepTail& a, int b, int h, float o) {
    const int d = threadIdx.x;
    a.out[static_cast<size_t>(b) * kModelDim + h * kHeadDim + d] = o;
    if (a.act_q == nullptr) return;
    const int lane = d & 63;
    const float row_max = row16_maxf(fabsf(o));
    const float lo = fmaxf(readlane_f(row_max, 0), readlane_f(row_max, 16));
    const float hi = fmaxf(readlane_f(row_max, 32), readlane_f(row_max, 48));
    const float mx_abs = lane < 32 ? lo : hi;
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
    // Lane gl < 14 of a group builds 32-bit word gl of its 448-bit A14 word
    // (lane i of the group at bits [14i, 14i+13]): the lanes floor(32gl/14)
    // to floor((32gl+31)/14), at most four, reach it.
    const int gl = lane & 31, base = lane & 32;
    const int i0 = (32 * gl) / 14;
    const uint32_t q = static_cast<uint32_t>(static_cast<uint16_t>(q14)) & 0x3fffu;
    uint32_t src[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) src[k] = __shfl(q, base + min(i0 + k, 31));
    const size_t grp = static_cast<size_t>(b) * (kHeads * kGroupsPerHead) + h * kGroupsPerHead + (d >> 5);
    if (gl < 14) {
        const int bit0 = 32 * gl;
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = i0 + k;
            if (i < 32 && 14 * i <= bit0 + 31) {
                const int sh = 14 * i - bit0;
                word |= sh >= 0 ? (src[k] << sh) : (src[k] >> -sh);
            }
        }
        reinterpret_cast<uint32_t*>(a.act_q + grp * kA14WordBytes)[gl] = word;
    }
    if (gl == 0) a.act_scale[grp] = code;
}

// Split partials are exchanged through device memory inside one launch as
// 64-bit words: the launch's 32-bit tag above the value's bits, written and
// read with agent-scope atomic accesses (write-through to the device
// coherence point, no L2 writeback or invalidate on either side).  A 64-bit
// atomic access is single-copy atomic, so a word that carries this launch's
// tag holds the value this launch's split wrote: the merger needs no ordering
// between the words, the arrival count and the stores of other workgroups --
// splits publish without waiting for their stores, and the merger re-reads a
// word until its tag is current.  The tag is the (row, head)'s generation
// plus one; the merger advances the generation for the next launch.
__device__ __forceinline__ void publish_tagged(uint64_t* p, uint32_t tag, float v) {
    __hip_atomic_store(p, (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t fetch_word(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls (rounds of re-reads) a merger makes in all before it gives up
// (StepArgs::merge_polls; the host passes kMergePolls).  Every split it waits
// for has counted its arrival, so it is resident, and nothing its waves 0-1
// do before their stores waits for another workgroup: its words will land.
// The bound only keeps a fault in this protocol from hanging the GPU.  A
// merger that gives up takes NaN for the words it still lacks (so the fault
// shows in the output) and records its (slot, head) in the context's fault
// word, which the host reports.

__device__ __forceinline__ bool current(uint64_t w, uint32_t tag) { return static_cast<uint32_t>(w >> 32) == tag; }

// The value of the word at p (first read w), re-read until it carries `tag`
// while the thread's poll budget lasts -- one budget for every word the
// thread waits for, so a merge that cannot complete gives up after `budget`
// polls in all -- and NaN, with gave_up set, once it has run out.
__device__ __forceinline__ float tagged_value(const uint64_t* p, uint64_t w, uint32_t tag, uint32_t& budget,
                                              bool& gave_up) {
    while (!current(w, tag)) {
        if (budget == 0) {
            gave_up = true;
            return __builtin_nanf("");
        }
        --budget;
        __builtin_amdgcn_s_sleep(1);
        w = fetch_word(p);
    }
    return __uint_as_float(static_cast<uint32_t>(w));
}

// Records a merge that gave up: the fault word is host memory, written through
// at system scope so the host sees it once the launch has ended (or earlier).
__device__ __forceinline__ void report_merge_fault(uint32_t* fault, uint32_t code) {
    __hip_atomic_store(fault, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Log-sum-exp merge of a head's n split partials; threads d < 128 get output
// channel d.  Up to kMergeInline splits the merge is inline: every thread
// reads all of its words at once -- each split's m and l (the same words in
// every lane) and its own channel of each split's acc -- with no barrier, and
// a split's own words stand in registers.  More splits (only when a caller
// forces small splits) take a looped merge with the statistics staged
// through LDS.  The terms are summed in split order whichever split merges,
// so the result does not depend on the arrival order.
constexpr int kMergeInline = 8;

struct InlineWords {
    uint64_t m[kMergeInline], l[kMergeInline], o[kMergeInline];
};

// First read of the other splits' words; the split's own words carry `tag`
// (they are never read).  Threads past 127 read channel 127.
__device__ __forceinline__ void fetch_inline(const uint64_t* slots, int n, int own, uint32_t tag, float own_m,
                                             float own_l, float own_o, InlineWords& w) {
    const int d = min(static_cast<int>(threadIdx.x), kHeadDim - 1);
    const uint64_t own_tag = static_cast<uint64_t>(tag) << 32;
#pragma unroll
    for (int j = 0; j < kMergeInline; ++j) {
        w.m[j] = own_tag | __float_as_uint(own_m);
        w.l[j] = own_tag | __float_as_uint(own_l);
        w.o[j] = own_tag | __float_as_uint(own_o);
        if (j < n && j != own) {
            const uint64_t* sl = slots + j * kSlotWords;
            w.m[j] = fetch_word(sl);
            w.l[j] = fetch_word(sl + 1);
            w.o[j] = fetch_word(sl + 2 + d);
        }
    }
}

__device__ __forceinline__ bool inline_stale(const InlineWords& w, uint32_t tag) {
    bool stale = false;
#pragma unroll
    for (int j = 0; j < kMergeInline; ++j) stale |= !current(w.m[j], tag) || !current(w.l[j], tag) || !current(w.o[j], tag);
    return stale;
}

// Inline merge of words first read by fetch_inline: words whose store had not
// landed yet are read again, all of them in one round trip per round, for at
// most `polls` rounds.
__device__ __forceinline__ float merge_inline(const uint64_t* slots, int n, uint32_t tag, uint32_t polls,
                                              InlineWords& w, bool& gave_up) {
    const int d = min(static_cast<int>(threadIdx.x), kHeadDim - 1);
    for (uint32_t spin = 0;; ++spin) {
        if (!inline_stale(w, tag)) break;
        if (spin == polls) {
            const uint64_t nan_word = (static_cast<uint64_t>(tag) << 32) | 0x7fc00000u;   // NaN shows in the output
#pragma unroll
            for (int j = 0; j < kMergeInline; ++j) w.o[j] = nan_word;
            gave_up = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int j = 0; j < kMergeInline; ++j) {
            const uint64_t* sl = slots + j * kSlotWords;
            if (!current(w.m[j], tag)) w.m[j] = fetch_word(sl);
            if (!current(w.l[j], tag)) w.l[j] = fetch_word(sl + 1);
            if (!current(w.o[j], tag)) w.o[j] = fetch_word(sl + 2 + d);
        }
    }
    float m[kMergeInline], l[kMergeInline], o[kMergeInline];
#pragma unroll
    for (int j = 0; j < kMergeInline; ++j) {
        m[j] = __uint_as_float(static_cast<uint32_t>(w.m[j]));
        l[j] = __uint_as_float(static_cast<uint32_t>(w.l[j]));
        o[j] = __uint_as_float(static_cast<uint32_t>(w.o[j]));
    }
    float mx = m[0];
#pragma unroll
    for (int j = 1; j < kMergeInline; ++j)
        if (j < n) mx = fmaxf(mx, m[j]);
    float den = 0.0f, num = 0.0f;
#pragma unroll
    for (int j = 0; j < kMergeInline; ++j) {
        if (j < n) {
            const float wt = fast_exp2(m[j] - mx);
            den += wt * l[j];
            num += wt * o[j];
        }
    }
    return num / den;
}

// Looped merge of n > kMergeInline partials by the split `own` (its (m, l, o)
// in registers), called by every wave: it stages the statistics through LDS
// behind a barrier.  Lanes past 127 read channel 127 and their result is
// unused.  One poll budget serves every word the thread waits for.
__device__ __forceinline__ float merge_looped(const uint64_t* slots, int n, int own, uint32_t tag, uint32_t polls,
                                              float own_m, float own_l, float own_o, bool& gave_up) {
    const int d = min(static_cast<int>(threadIdx.x), kHeadDim - 1);
    __shared__ float s_m[kMaxSplits], s_l[kMaxSplits];
    const int t = threadIdx.x;
    uint32_t budget = polls;
    if (t < n) {
        const uint64_t* sl = slots + t * kSlotWords;
        s_m[t] = t == own ? own_m : tagged_value(sl, fetch_word(sl), tag, budget, gave_up);
        s_l[t] = t == own ? own_l : tagged_value(sl + 1, fetch_word(sl + 1), tag, budget, gave_up);
    }
    __syncthreads();
    float mx = s_m[0];
    for (int j = 1; j < n; ++j) mx = fmaxf(mx, s_m[j]);
    float den = 0.0f, num = 0.0f;
    for (int j = 0; j < n; ++j) {
        const uint64_t* sl = slots + j * kSlotWords + 2 + d;
        const float wt = fast_exp2(s_m[j] - mx);
        den += wt * s_l[j];
        num += wt * (j == own ? own_o : tagged_value(sl, fetch_word(sl), tag, budget, gave_up));
    }
    return num / den;
}

// ---------------------------------------------------------------- step

// Grid (splits, 32 heads, batch) of WAVES-wave workgroups scanning blocks of
// 8 * NI tokens (NI rows per lane); grid row z serves rows[z].
//
// The arguments every first load depends on come first and travel in SGPRs:
// the library is compiled with kernarg preloading (-amdgpu-kernarg-preload-
// count), so the dispatcher writes them into each wave's user SGPRs and no
// wave waits on a scalar load of the argument block before its first vector
// loads (a wave that had to load them chained three scalar round trips ahead
// of its first cache block).  Firmware without the feature runs the code
// object's own prologue, which loads the same SGPRs.  StepPreload (host and
// kernel) packs them; the rest of the arguments stay in StepArgs.  `aux` is
// the arrival words' address, except for the split-K partial formats, whose
// q/k/v loads need the stride between partials first: for them it carries
// part_stride as a pointer-sized integer and the arrival words come from
// StepArgs (their load is not waited for until the end).  It stays a
// pointer parameter so that the compiler knows the arrival words are global
// memory: a generic pointer made from an integer is read with a flat load,
// which counts against both wait counters and made the query conversion wait
// for the whole first block.
template <int IN, int WAVES, int NI>
__global__ __launch_bounds__(WAVES * 64) void step_kernel(const int8_t* layer_pages, uint32_t geometry,
                                                          uint32_t dispatch, const void* q_in, const void* k_in,
                                                          const void* v_in, const int2* lut, const void* aux,
                                                          StepArgs a) {
    constexpr bool kParts = IN >= kInParts2;
    const int64_t part_stride = kParts ? static_cast<int64_t>(reinterpret_cast<uintptr_t>(aux)) : 0;
    uint64_t* const arrivals = kParts ? a.arrivals : static_cast<uint64_t*>(const_cast<void*>(aux));
    constexpr int kBlk = 8 * NI;
    SKV_STAMP_DECL;
    SKV_STAMP(0);
    // A launch whose sequences all stand at one position names it in
    // `dispatch` and its rows are the identity (set_rows keeps equal positions
    // in sequence order); only other launches read rows[].
    const uint32_t uniform_pos = dispatch & StepPreload::kRowsListed;
    const uint32_t row = uniform_pos != StepPreload::kRowsListed ? pack_row(blockIdx.z, uniform_pos)
                                                                 : a.rows[blockIdx.z];
    const int split = blockIdx.x, h = blockIdx.y, b = static_cast<int>(row & 0xffu);
    const int pos = static_cast<int>(row >> 8);
    const int len = pos + 1;
    const int C = static_cast<int>(dispatch >> 16) * kSplitQuantum;
    const int t_begin = split * C;
    if (t_begin >= len) {
        SKV_STAMP_FLUSH();
        return;
    }
    const int t_end = min(t_begin + C, len);
    const int nsplit = (len + C - 1) / C;
    const bool owner = pos < t_end;               // this split holds the new token

    // wave index made provably uniform so token offsets stay in SGPRs (the
    // buffer loads' soffset operand) instead of forcing waterfall loops
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int c = lane & 7, r = lane >> 3;
    const int64_t cap = geometry & 0xffffu;
    const int64_t page_bytes = cap * kTokenBytes;
    int8_t* page = const_cast<int8_t*>(layer_pages) +
                   (static_cast<int64_t>(b) * (geometry >> 16) * kHeads + h) * page_bytes;

    __shared__ float s_acc[WAVES + 1][kHeadDim];
    __shared__ float s_m[WAVES + 1], s_l[WAVES + 1];

    // Loads go out before any math, in the order they are needed: this
    // lane's channel pair (2*lane, 2*lane+1) of the new row's RoPE pair and
    // q -- and of its k and v in the one wave that appends the row -- then
    // the first cache block.  The conversions below wait only for the row
    // loads (vector loads retire in issue order), so they overlap the block's
    // flight.  The block loads are unconditional and in bounds: a block load
    // under a branch makes the compiler wait for it at the join.  The k/v
    // loads are under a wave-uniform branch ahead of the block, so every wait
    // for a later load keeps its count on both paths.  (Loading q once per
    // workgroup and handing it to the other waves through LDS measured slower
    // at batch 1: 12.5-12.9 against 11.7-11.9 us/layer.)
    const size_t row_elem = static_cast<size_t>(b) * kModelDim + h * kHeadDim + 2 * lane;
    const bool appends = owner && wave == 0;       // this wave writes and forwards the new row
    const int2 row_cs = lut[static_cast<size_t>(pos) * kRopePairs + lane];
    const InPair<IN> row_q = load_in<IN>(q_in, row_elem, part_stride);
    InPair<IN> row_k{}, row_v{};
    if (appends) {
        row_k = load_in<IN>(k_in, row_elem, part_stride);
        row_v = load_in<IN>(v_in, row_elem, part_stride);
    }
    const PageReader pr = make_reader(page, cap, c, r);
    const int t_first = t_begin + wave * kBlk;
    const int t_stop = owner ? pos : t_end;       // the new token is forwarded, not scanned
    // A wave with no tokens issues the split's first block with every row
    // masked (no data moves): every path then has the same loads in flight.
    BlockLoads<NI> bl;
    issue_block_masked(pr, t_first < t_stop ? t_first : t_begin, t_first < t_stop ? t_stop : 0, r, bl);
    // The (row, head)'s arrival word, for the tag of a split partial.  Read
    // on every path (unused by a head held by one split): a load under a
    // branch would make the compiler wait for the block at the join.
    const size_t head_row = static_cast<size_t>(b) * kHeads + h;
    uint64_t* arrival = arrivals + head_row * kArrivalStride;
    const uint64_t arrival_word = fetch_word(arrival);
    const StepTail tail{a.out,         a.act_q,          a.act_scale,  a.partials, a.fault,
                        a.slot_stride, a.merge_tag_skew, a.merge_polls, a.slot0};
    __builtin_amdgcn_sched_barrier(0);   // issue their loads here, not at the first wait

    // Query: each lane converts and rotates its own pair and splits it into
    // byte limbs; each lane then gathers the limbs of its chunk c.  The new
    // row's k is rotated and v converted here too, which frees the raw row
    // registers before the scan.
    SKV_STAMP_WAIT();
    SKV_STAMP(1);
    SKV_WAVE_FIRST_LOADS();
    const int2 qi = in_to_q17<IN>(row_q);
    int32_t q0, q1;
    rope_pair(qi.x, qi.y, row_cs, q0, q1);
    const float qs0 = (static_cast<float>(q0) * 0x1p-17f) * kScoreScale;
    const float qs1 = (static_cast<float>(q1) * 0x1p-17f) * kScoreScale;
    const QueryChunk Q = chunk_limbs(q0, q1, c);
    const int2 ki = in_to_q17<IN>(row_k), vi = in_to_q17<IN>(row_v);
    int32_t k0, k1;
    rope_pair(ki.x, ki.y, row_cs, k0, k1);
    // The tail's fields are in SGPRs from here on (the wait for them, if any,
    // falls in the wait for the first block).
    asm volatile("" ::"s"(tail.out), "s"(tail.act_q), "s"(tail.act_scale), "s"(tail.partials), "s"(tail.fault),
                 "s"(tail.slot_stride), "s"(tail.merge_tag_skew), "s"(tail.merge_polls), "s"(tail.slot0));

    float m_run, l_run, acc[16];
    scan_range<NI>(pr, bl, Q, t_first, t_stop, WAVES * kBlk, r, m_run, l_run, acc);
    SKV_WAVE_SCAN_DONE();

    // The new row: quantize, append; forward (k^ . q', v^) into the merge as
    // one more partial.
    if (appends) {
        float kh0, kh1, vh0, vh1;
        append_row_dequant(page, static_cast<int>(cap), pos, lane, k0, k1, vi.x, vi.y, kh0, kh1, vh0, vh1);
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
    SKV_STAMP(2);

    const int d = threadIdx.x;
    float o = 0.0f, l = 0.0f, mx = -INFINITY;
    if (d < kHeadDim) {
        const int nparts = owner ? WAVES + 1 : WAVES;
        mx = s_m[0];
        for (int w = 1; w < nparts; ++w) mx = fmaxf(mx, s_m[w]);
        for (int w = 0; w < nparts; ++w) {
            const float sc = fast_exp2(s_m[w] - mx);     // parts with no tokens: 2^-inf = 0
            o += sc * s_acc[w][d];
            l += sc * s_l[w];
        }
    }
    if (nsplit == 1) {
        if (d < kHeadDim) finalize_head(tail, b, h, o / l);
        SKV_STAMP(5);
        SKV_STAMP_FLUSH();
        return;
    }

    // Several splits: count this split's arrival, publish its partial as
    // tagged words without waiting for them to land, and let the split that
    // arrives last merge the head's partials and finish the head.  (Reading
    // the other splits' words in the same round trip as the count, so that a
    // split finding them all current could merge at once, measured 0.9-1.0 us
    // slower at batch 1: every split then reads every other split's words at
    // device scope, about 2.7 MB in one burst as the stream ends, and the
    // splits of a head finish together, so the last one still finds some
    // words stale.)
    // Both halves of the word stay in their registers until here: with the
    // low half dead early, the compiler reused its register in the prologue,
    // and a write to a register that a load is still filling waits for every
    // load in flight, the first cache block included.
    asm volatile("" ::"v"(arrival_word));
    const uint32_t tag = static_cast<uint32_t>(arrival_word >> 32) + 1u;
    uint64_t* slots = tail.partials + head_row * static_cast<size_t>(tail.slot_stride) * kSlotWords;
    const bool inline_merge = nsplit <= kMergeInline;
    // The count goes out from thread 128, in a wave that publishes nothing,
    // so waiting for its result never waits for the stores of waves 0-1.
    constexpr unsigned kCountThread = kHeadDim;
    static_assert(kCountThread < kAttendWaves * 64, "the counting thread exists in every workgroup");
    uint64_t before = 0;
    if (threadIdx.x == kCountThread)
        before = __hip_atomic_fetch_add(arrival, uint64_t(1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d < kHeadDim) {
        uint64_t* mine = slots + static_cast<size_t>(split) * kSlotWords;
        publish_tagged(mine + 2 + d, tag, o);
        if (d == 0) {
            publish_tagged(mine, tag, mx);
            publish_tagged(mine + 1, tag, l);
        }
    }
    __shared__ int s_last;
    if (threadIdx.x == kCountThread) s_last = static_cast<uint32_t>(before) == static_cast<uint32_t>(nsplit - 1);
    __syncthreads();
    // Only waves 0-1 (the output channels) merge and finish, except that the
    // looped merge of more than kMergeInline splits needs every wave at its barrier.
    SKV_STAMP(3);
    SKV_STAMP_FLAG(2);
    if (!s_last || (inline_merge && d >= kHeadDim)) {
        SKV_STAMP_FLUSH();
        return;
    }
    // The merger waits for words tagged `want` (a testing aid can make it wait
    // for a tag no word carries, so that the wait gives up).
    const uint32_t want = tag + tail.merge_tag_skew;
    bool gave_up = false;
    float merged;
    if (inline_merge) {
        InlineWords w;
        fetch_inline(slots, nsplit, split, want, mx, l, o, w);
        merged = merge_inline(slots, nsplit, want, tail.merge_polls, w, gave_up);
    } else {
        merged = merge_looped(slots, nsplit, split, want, tail.merge_polls, mx, l, o, gave_up);
    }
    SKV_STAMP(4);
    if (gave_up) report_merge_fault(tail.fault, static_cast<uint32_t>(tail.slot0 + b) * kHeads + h + 1u);
    if (d >= kHeadDim) return;
    finalize_head(tail, b, h, merged);
    SKV_STAMP(5);
    SKV_STAMP_FLAG(1);
    SKV_STAMP_FLUSH();
    // Every split has counted its arrival and its words have been read: reset
    // the count and advance the generation for the next launch.  Tags run
    // over 1 .. 2^32-1; when they wrap, the head's slots are cleared first
    // (tag 0 is never current), so no word left from 2^32-1 launches ago can
    // pass for a current one.
    if (tag == 0xffffffffu) {
        for (int i = d; i < tail.slot_stride * kSlotWords; i += kHeadDim)
            __hip_atomic_store(slots + i, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (d == 0)
        __hip_atomic_store(arrival, static_cast<uint64_t>(tag == 0xffffffffu ? 0u : tag) << 32, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- utilities

// Prefill rows: one instruction covers two token rows (lane l takes channels
// 4(l & 31) .. 4(l & 31) + 3 of row l >> 5), and a wave takes kAppendPairs
// such pairs with all of their loads in flight together.  One pair per wave
// and default-policy k/v loads measured fastest: more pairs per wave cost
// occupancy, and nontemporal loads lose the MALL hits of k/v that a
// projection has just written.
constexpr int kAppendPairs = 1;
constexpr int kAppendTokens = 2 * kAppendPairs;
constexpr bool kAppendNontemporal = false;

// Q15.17 of four FP32 values by the saturating conversion alone, which maps
// NaN to 0; the caller sends a wave holding a NaN through f32_to_q17.
__device__ __forceinline__ int32_t q17_no_nan(float x) {
    int32_t v;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(v) : "v"(__builtin_rintf(x * 131072.0f)));
    return v;
}
__device__ __forceinline__ int4 quad_q17_no_nan(float4 f) {
    return make_int4(q17_no_nan(f.x), q17_no_nan(f.y), q17_no_nan(f.z), q17_no_nan(f.w));
}
__device__ __forceinline__ int4 quad_q17(float4 f) {
    return make_int4(f32_to_q17(f.x), f32_to_q17(f.y), f32_to_q17(f.z), f32_to_q17(f.w));
}

// The rotation's sat32((a*c - b*s) >> 17) in double precision.  The table's
// (cos, sin) are signed 19-bit values (generated or loaded, both saturate to
// 19 bits) and |a|, |b| <= 2^31, so each product has at most 49 significant
// bits and the fused sum at most 50: every step below is exact, floor is the
// arithmetic shift, and the double-to-int conversion saturates.
__device__ __forceinline__ int32_t floor_sat32(double x) {
    int32_t v;
    asm("v_cvt_i32_f64 %0, %1" : "=v"(v) : "v"(__builtin_floor(x)));
    return v;
}
__device__ __forceinline__ void rope_pair_f64(int32_t a, int32_t b, int2 cs, int32_t& x0, int32_t& x1) {
    const double c = static_cast<double>(cs.x) * 0x1p-17, s = static_cast<double>(cs.y) * 0x1p-17;
    const double da = a, db = b;
    x0 = floor_sat32(__builtin_fma(da, c, -(db * s)));
    x1 = floor_sat32(__builtin_fma(da, s, db * c));
}

// Max over the 8 lanes of an aligned octet (one G32 group of a row when a
// lane holds four channels); every lane gets it.
__device__ __forceinline__ uint32_t octet_max_u(uint32_t x) {
    x = max(x, dpp_u<kDppQuadXor1>(x));
    x = max(x, dpp_u<kDppQuadXor2>(x));
    return max(x, dpp_u<kDppHalfMirror>(x));
}

// The largest magnitude of a quad, at least 1 (the shift rule gives 0 for a
// maximum of 0 and of 1 alike): max(max r, 0) against 0 - min(min r, 0),
// which is 2^31 for INT32_MIN.
__device__ __forceinline__ uint32_t quad_magnitude1(int4 r) {
    const int32_t hi = max(max(max(max(r.x, r.y), r.z), r.w), 0);
    const int32_t lo = min(min(min(min(r.x, r.y), r.z), r.w), 0);
    return max(max(static_cast<uint32_t>(hi), 0u - static_cast<uint32_t>(lo)), 1u);
}

// G32 shift of a maximum m >= 1: msb(m) - 6, floored at 0.
__device__ __forceinline__ uint32_t g32_shift1(uint32_t m) {
    return static_cast<uint32_t>(max(25 - __builtin_clz(m), 0));
}

__device__ __forceinline__ uint32_t pack_code_bytes(int32_t c0, int32_t c1, int32_t c2, int32_t c3) {
    const uint32_t lo = __builtin_amdgcn_perm(static_cast<uint32_t>(c1), static_cast<uint32_t>(c0), 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(static_cast<uint32_t>(c3), static_cast<uint32_t>(c2), 0x0c0c0400u);
    return lo | (hi << 16);
}

// Codes of a quad under any shift (g32_code_byte).
__device__ __forceinline__ uint32_t quad_codes(int4 r, uint32_t s) {
    return g32_code_byte(r.x, s) | (g32_code_byte(r.y, s) << 8) | (g32_code_byte(r.z, s) << 16) |
           (g32_code_byte(r.w, s) << 24);
}

// Codes of a quad whose shift s is in [1, 23]: sign * min(127, (|r| + 2^(s-1))
// >> s) is clamp((r + 2^(s-1) - [r < 0]) >> s, -127, 127) with an arithmetic
// shift (for r < 0 the floor of (r + 2^(s-1) - 1) / 2^s is minus the rounded
// magnitude), and r + 2^(s-1) < 2^31 because |r| < 2^(s+7) <= 2^30.
__device__ __forceinline__ int32_t code_mid(int32_t r, uint32_t s, int32_t rnd) {
    return min(max((r + rnd + (r >> 31)) >> s, -127), 127);
}
__device__ __forceinline__ uint32_t quad_codes_mid(int4 r, uint32_t s) {
    const int32_t rnd = static_cast<int32_t>(1u << (s - 1u));
    return pack_code_bytes(code_mid(r.x, s, rnd), code_mid(r.y, s, rnd), code_mid(r.z, s, rnd),
                           code_mid(r.w, s, rnd));
}

template <bool NT>
__device__ __forceinline__ v4i load_quad_bits(const void* base, size_t elem) {
    const v4i* p = reinterpret_cast<const v4i*>(static_cast<const int32_t*>(base) + elem);
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

// Grid (ceil(n / kAppendTokens), 8): wave = head (4 per workgroup), with
// kAppendPairs row pairs per wave.  All of a wave's k, v and RoPE loads go
// out first; rows past n load the last token and store nothing.  The append
// rule is the step's (row_codes): per G32 group the shift of the magnitude
// maximum, then the round-half-away codes.  Wave-uniform branches keep the
// common case short: a wave with a NaN among its FP32 inputs converts them
// again by the NaN rule, and a row pair with a group shift of 0 or above 23
// forms its codes by the general rule.
template <bool Q17>
__global__ __launch_bounds__(256) void append_bulk_kernel(BulkArgs a) {
    // wave-uniform through readfirstlane, so the page's buffer resource stays in SGPRs
    const int h = blockIdx.y * 4 + __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int half = lane >> 5, cl = lane & 31;   // row of a pair; channels 4cl .. 4cl+3 (pairs 2cl, 2cl+1)
    const int t0 = blockIdx.x * kAppendTokens;    // < n: the grid has ceil(n / kAppendTokens) rows
    int4 cs[kAppendPairs];
    v4i kq[kAppendPairs], vq[kAppendPairs];       // FP32 or Q15.17 bits
#pragma unroll
    for (int j = 0; j < kAppendPairs; ++j) {
        const int t = min(t0 + 2 * j + half, a.n - 1);
        const size_t elem = static_cast<size_t>(t) * kModelDim + h * kHeadDim + 4 * cl;
        cs[j] = *reinterpret_cast<const int4*>(a.lut + static_cast<size_t>(a.pos0 + t) * kRopePairs + 2 * cl);
        kq[j] = load_quad_bits<kAppendNontemporal>(a.k, elem);
        vq[j] = load_quad_bits<kAppendNontemporal>(a.v, elem);
    }
    int4 ki[kAppendPairs], vi[kAppendPairs];
    if constexpr (Q17) {
#pragma unroll
        for (int j = 0; j < kAppendPairs; ++j) {
            ki[j] = make_int4(kq[j].x, kq[j].y, kq[j].z, kq[j].w);
            vi[j] = make_int4(vq[j].x, vq[j].y, vq[j].z, vq[j].w);
        }
    } else {
        // isunordered(x, y): either is NaN, one compare per pair of values,
        // whose lane masks combine on the scalar unit
        uint64_t nan = 0;
#pragma unroll
        for (int j = 0; j < kAppendPairs; ++j) {
            const v4f k4 = __builtin_bit_cast(v4f, kq[j]), v4 = __builtin_bit_cast(v4f, vq[j]);
            const float4 kf = make_float4(k4.x, k4.y, k4.z, k4.w), vf = make_float4(v4.x, v4.y, v4.z, v4.w);
            ki[j] = quad_q17_no_nan(kf);
            vi[j] = quad_q17_no_nan(vf);
            nan |= __builtin_amdgcn_ballot_w64(__builtin_isunordered(kf.x, kf.y)) |
                   __builtin_amdgcn_ballot_w64(__builtin_isunordered(kf.z, kf.w)) |
                   __builtin_amdgcn_ballot_w64(__builtin_isunordered(vf.x, vf.y)) |
                   __builtin_amdgcn_ballot_w64(__builtin_isunordered(vf.z, vf.w));
        }
        if (nan != 0) {
#pragma unroll
            for (int j = 0; j < kAppendPairs; ++j) {
                const v4f k4 = __builtin_bit_cast(v4f, kq[j]), v4 = __builtin_bit_cast(v4f, vq[j]);
                ki[j] = quad_q17(make_float4(k4.x, k4.y, k4.z, k4.w));
                vi[j] = quad_q17(make_float4(v4.x, v4.y, v4.z, v4.w));
            }
        }
    }
    const __amdgpu_buffer_rsrc_t page = __builtin_amdgcn_make_buffer_rsrc(
        page_ptr(a.kv, a.slot, a.layer, h), static_cast<short>(0), static_cast<int32_t>(a.kv.page_bytes), kBufferWord3);
    const int cap = a.kv.seq_cap;
#pragma unroll
    for (int j = 0; j < kAppendPairs; ++j) {
        if (t0 + 2 * j >= a.n) break;              // wave-uniform: neither row of the pair exists
        int4 k;
        rope_pair_f64(ki[j].x, ki[j].y, make_int2(cs[j].x, cs[j].y), k.x, k.y);
        rope_pair_f64(ki[j].z, ki[j].w, make_int2(cs[j].z, cs[j].w), k.z, k.w);
        const uint32_t sk = g32_shift1(octet_max_u(quad_magnitude1(k)));
        const uint32_t sv = g32_shift1(octet_max_u(quad_magnitude1(vi[j])));
        uint32_t kw, vw;
        if (__builtin_amdgcn_ballot_w64(sk - 1u >= 23u || sv - 1u >= 23u) == 0) {
            kw = quad_codes_mid(k, sk);
            vw = quad_codes_mid(vi[j], sv);
        } else {
            kw = quad_codes(k, sk);
            vw = quad_codes(vi[j], sv);
        }
        if (t0 + 2 * j + half < a.n) {             // the pair's second row may be past n
            const int row = a.pos0 + t0 + 2 * j;   // first row of the pair (SGPR); this lane's is row + half
            __builtin_amdgcn_raw_buffer_store_b32(kw, page, half * kCodeBytes + 4 * cl, row * kCodeBytes, 0);
            __builtin_amdgcn_raw_buffer_store_b32(vw, page, half * kCodeBytes + 4 * cl, (cap + row) * kCodeBytes, 0);
            if ((cl & 7) == 0) {
                const v2f sc = {shift_scale(sk), shift_scale(sv)};
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, sc), page,
                                                      half * kScaleBytes + (cl >> 3) * 8,
                                                      cap * (2 * kCodeBytes) + row * kScaleBytes, 0);
            }
        }
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

__global__ __launch_bounds__(256) void fill_u64_kernel(uint64_t* __restrict__ p, size_t n, uint64_t value) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = value;
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

hipError_t launch_fill_u64(uint64_t* p, size_t n, uint64_t value, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
    fill_u64_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(p, n, value);
    return hipGetLastError();
}

template <int WAVES, int BLOCK>
hipError_t launch_step_shape(const StepArgs& a, const StepPreload& p, dim3 grid, InputFormat in, hipStream_t s) {
    constexpr int NI = BLOCK / 8;
    const dim3 block(WAVES * 64);
    const void* arrivals = a.arrivals;
    const void* part_stride = reinterpret_cast<const void*>(static_cast<uintptr_t>(a.part_stride));
#define SKV_STEP_ARGS(AUX) p.layer_pages, p.geometry, p.dispatch, a.q, a.k, a.v, a.lut, AUX, a
    switch (in) {
    case kInF32: step_kernel<kInF32, WAVES, NI><<<grid, block, 0, s>>>(SKV_STEP_ARGS(arrivals)); break;
    case kInQ17: step_kernel<kInQ17, WAVES, NI><<<grid, block, 0, s>>>(SKV_STEP_ARGS(arrivals)); break;
    case kInParts2: step_kernel<kInParts2, WAVES, NI><<<grid, block, 0, s>>>(SKV_STEP_ARGS(part_stride)); break;
    case kInParts4: step_kernel<kInParts4, WAVES, NI><<<grid, block, 0, s>>>(SKV_STEP_ARGS(part_stride)); break;
    default: return hipErrorInvalidValue;
    }
#undef SKV_STEP_ARGS
    return hipGetLastError();
}

// The preloaded arguments of a launch (StepPreload); launch_step has checked
// that its geometry and split fit the packing.
StepPreload step_preload(const StepArgs& a) {
    StepPreload p;
    p.layer_pages = page_ptr(a.kv, a.slot0, a.layer, 0);
    p.geometry = static_cast<uint32_t>(a.kv.seq_cap) | (static_cast<uint32_t>(a.kv.layers) << 16);
    uint32_t common = StepPreload::kRowsListed;
    if (a.batch > 0) {
        common = a.rows[0] >> 8;
        for (int z = 0; z < a.batch; ++z)
            if (a.rows[z] != pack_row(z, static_cast<int>(common))) common = StepPreload::kRowsListed;
    }
    p.dispatch = common | (static_cast<uint32_t>(a.split_tokens / kSplitQuantum) << 16);
    return p;
}

int step_workgroups_per_cu() {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, step_kernel<kInF32, kAttendWaves, kBlockTokens / 8>,
                                                     kAttendWaves * 64, 0) != hipSuccess)
        return 0;
    return n;
}

hipError_t launch_step(const StepArgs& a, int grid_splits, StepShape shape, InputFormat in, hipStream_t s) {
    const dim3 grid(grid_splits, kHeads, a.batch);
    if (a.split_tokens <= 0 || a.split_tokens % kSplitQuantum != 0 || a.split_tokens > kMaxSeq ||
        a.kv.seq_cap > kMaxSeq || a.kv.layers > 0xffff)
        return hipErrorInvalidValue;   // outside what StepPreload packs
    const StepPreload p = step_preload(a);
#define SKV_LAUNCH_SHAPE(W, B) \
    if (shape == StepShape{W, B}) return launch_step_shape<W, B>(a, p, grid, in, s);
    SWIFTKV_STEP_SHAPES(SKV_LAUNCH_SHAPE)
#undef SKV_LAUNCH_SHAPE
    return hipErrorInvalidValue;
}

bool step_shape_compiled(StepShape shape) {
#define SKV_IS_SHAPE(W, B) \
    if (shape == StepShape{W, B}) return true;
    SWIFTKV_STEP_SHAPES(SKV_IS_SHAPE)
#undef SKV_IS_SHAPE
    return false;
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
