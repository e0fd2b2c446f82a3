// swiftkv_common.hpp -- geometry, cache layout and kernel argument blocks
// shared by the host C-ABI (swiftkv_capi.cpp) and the HIP kernels
// (swiftkv_kernels.hip, swiftkv_exact.hip, swiftkv_synth.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace swiftkv {

// Geometry fixed by the reference (kernel_HLS/swiftkv_attention.hpp:5-13).
constexpr int kHeads = 32;
constexpr int kHeadDim = 128;
constexpr int kModelDim = kHeads * kHeadDim;
constexpr int kGroup = 32;                       // G32 quantization group
constexpr int kGroupsPerHead = kHeadDim / kGroup;
constexpr int kRopePairs = kHeadDim / 2;         // adjacent pairs (2j, 2j+1)

// Page of one (sequence, layer, head): K codes [S][128] int8, V codes
// [S][128] int8, scales [S][8] float interleaved (K_g, V_g) per group g.
constexpr int kCodeBytes = kHeadDim;             // 128 B per token per plane
constexpr int kScaleBytes = 8 * 4;               // 32 B per token
constexpr int kTokenBytes = 2 * kCodeBytes + kScaleBytes;  // 288 B
constexpr int kSeqAlign = 64;                    // capacity granularity (tokens)
constexpr int kA14WordBytes = 56;                // ap_uint<448>: 32 x 14-bit lanes

// Split-context work: a workgroup of kAttendWaves wavefronts scans a range of
// split_tokens tokens; each wave takes 64-token blocks round-robin.
constexpr int kAttendWaves = 4;
constexpr int kBlockTokens = 64;
// Launches of up to one residency round of 4-wave workgroups use 8 waves on
// 32-token blocks (123 VGPRs): each wave holds half a block, so less math is
// left when the last data arrives, and a CU keeps 8 or 16 waves' loads in
// flight (16 waves on 32-token blocks, the same bytes per wave, measured
// slower: the CU then asks for twice the data it can have in flight, and
// issues its waves' loads oldest wave first, so its youngest waves start
// their scans last).  Larger launches whose every workgroup holds at least
// kLongRangeTokens run 8 waves on 64-token blocks, one workgroup per CU.
constexpr int kWideWaves = 8;
constexpr int kWideBlockTokens = 32;
constexpr int kLongWaves = 8;
constexpr int kLongBlockTokens = 64;
constexpr int kLongRangeTokens = 2048;

// A step launch's shape: waves per workgroup and tokens per block.
struct StepShape {
    int waves;
    int block_tokens;
    constexpr bool operator==(const StepShape& o) const { return waves == o.waves && block_tokens == o.block_tokens; }
};
constexpr StepShape kNarrowShape{kAttendWaves, kBlockTokens};
constexpr StepShape kWideShape{kWideWaves, kWideBlockTokens};
constexpr StepShape kLongShape{kLongWaves, kLongBlockTokens};
// Every shape the step kernel is compiled for, as X(waves, block_tokens).
#define SWIFTKV_STEP_SHAPES(X) X(4, 64) X(8, 32) X(8, 64)
constexpr int kSplitQuantum = kAttendWaves * kBlockTokens;   // 256
constexpr int kMaxSeq = 32768;                   // longest cache accepted (tokens per sequence)
constexpr int kMaxSplits = kMaxSeq / kSplitQuantum;   // 128 partials per (sequence, head)

// A split's partial (m, l, acc[128]) travels as kSlotWords 64-bit words, each
// the launch's 32-bit tag above the value's bits.
constexpr int kSlotWords = 2 + kHeadDim;
// Slots per (row, head) in the allocation-free layout (the heuristic never
// splits a head more than 8 ways).
constexpr int kFixedSlots = 8;

// Polls a split merger makes in all (each a round of re-reads of the words
// still missing, about a microsecond) before it gives up on a partial that
// never arrives: seconds, far beyond any wait the protocol can need.
constexpr uint32_t kMergePolls = 1u << 22;

// Per (row, head) arrival word {generation:32 | arrivals:32}, one per 128-byte
// cache line: the splits of all heads finish together, and words sharing a
// line serialize their atomics.
constexpr int kArrivalStride = 16;               // uint64 words

// Sequences per launch: positions travel by value in the kernel arguments.
constexpr int kMaxBatchPerLaunch = 256;

// How the step's q/k/v arrive.  kInParts2/kInParts4: FP32 split-K partial sums
// of the upstream Q/K/V linear stage, reduced in the reference's fixed order
// before the Q15.17 conversion -- fl(p0 + p1), or fl(fl(p0 + p1) + fl(p2 +
// p3)) (int4_linear_controller.cpp:1039-1054, 1655-1667, 1100-1118).  The
// enumerator values of the partial formats are their part counts.
enum InputFormat : int { kInF32 = 0, kInQ17 = 1, kInParts2 = 2, kInParts4 = 4 };

static_assert(kTokenBytes == 288, "algorithmic bytes per token-head");
static_assert(kGroupsPerHead == 4, "four G32 groups per head");

struct CacheView {
    int8_t* base;         // arena: pages ordered [slot][layer][head]
    int64_t page_bytes;   // seq_cap * 288
    int32_t seq_cap;      // tokens per page (multiple of 64)
    int32_t layers;
};

__host__ __device__ inline int8_t* page_ptr(const CacheView& v, int slot, int layer, int head) {
    return v.base + ((static_cast<int64_t>(slot) * v.layers + layer) * kHeads + head) * v.page_bytes;
}

// One decode step over a chunk of <= kMaxBatchPerLaunch sequences.
struct StepArgs {
    const void* q;            // [batch][4096] FP32 or Q15.17; partial formats: part p at + p * part_stride
    const void* k;
    const void* v;
    int64_t part_stride;      // elements between split-K partials (partial formats only)
    CacheView kv;
    const int2* lut;          // [lut_positions][64] (cos, sin) Q1.17
    int32_t lut_positions;
    int32_t layer;
    int32_t batch;            // sequences in this launch
    int32_t slot0;            // cache slot of sequence 0 of this launch
    int32_t split_tokens;     // multiple of kSplitQuantum
    int32_t slot_stride;      // split slots per (row, head) in `partials`, >= the launch's splits
    uint64_t* partials;       // [rows][32][slot_stride][kSlotWords] tagged words
    // [rows][32] arrival words, kArrivalStride apart: the generation of the
    // (row, head) in the upper half, this launch's arrivals (zero between
    // launches) in the lower half.  Each split workspace holds its own, ahead
    // of its partials, so the tags of one workspace never meet the words of
    // another.
    uint64_t* arrivals;
    float* out;               // [batch][4096]
    uint8_t* act_q;           // [batch][128][56] or null
    uint8_t* act_scale;       // [batch][128] or null
    // Split merges: the polls a merger makes in all before it gives up
    // (kMergePolls), a testing aid's skew of the tag it waits for (0 in
    // service), and the context's fault word, where a merger that gave up
    // leaves its slot * 32 + head + 1.
    uint32_t merge_polls;
    uint32_t merge_tag_skew;
    uint32_t* fault;
    // Dispatch row z serves sequence rows[z] & 0xff at position rows[z] >> 8
    // (one scalar load gives both).  The host orders rows by descending
    // position, longest first, so ragged batches do not end on a tail of long
    // heads.
    uint32_t rows[kMaxBatchPerLaunch];
};
static_assert(kMaxBatchPerLaunch <= 256, "rows[] holds sequence indices in 8 bits");
static_assert(kMaxSeq <= (1 << 24), "rows[] holds positions in 24 bits");

__host__ __device__ inline uint32_t pack_row(int seq, int pos) {
    return (static_cast<uint32_t>(pos) << 8) | static_cast<uint32_t>(seq);
}

// The packed leading arguments of the step kernel, derived from a StepArgs
// by the launcher.  With q, k, v, the RoPE table and the arrival words (or,
// for the split-K partial formats, the part stride) they fill the 14 user
// SGPRs left beside the argument-block pointer, preloaded by the dispatcher:
// everything the kernel's first loads depend on.
//   layer_pages: the page of (sequence 0 of the launch, layer, head 0);
//                page (b, h) = layer_pages + (b * layers * 32 + h) * seq_cap * 288
//   geometry:    seq_cap (bits 0-15) | layers (bits 16-31)
//   dispatch:    the launch's common position, or kRowsListed when its
//                positions differ (rows[] then names each row's) (bits
//                0-15) | split_tokens / kSplitQuantum (bits 16-31)
struct StepPreload {
    static constexpr uint32_t kRowsListed = 0xffffu;
    const int8_t* layer_pages;
    uint32_t geometry;
    uint32_t dispatch;
};
static_assert(kMaxSeq <= 0x8000 && kMaxSeq / kSplitQuantum <= 0xffff, "StepPreload packs positions and splits in 16 bits");

// Bulk append of n tokens of one sequence (prefill).
struct BulkArgs {
    const void* k;            // [n][4096]
    const void* v;
    CacheView kv;
    const int2* lut;
    int32_t lut_positions;
    int32_t layer;
    int32_t slot;
    int32_t pos0;
    int32_t n;
};

// Workspace of the allocation-free step entry: one file-scope device array
// per GPU (swiftkv_kernels.hip), the split-arrival counters first, then the
// split partials, for kFixedSlots splits per head of kNoAllocSplitRows
// sequences per launch (the launch plan splits heads only in launches of
// fewer than 32 sequences at 256 CUs; a caller's forced split of more runs
// as launches of kNoAllocSplitRows).  Bound once per device by
// bind_noalloc_scratch.
constexpr int kNoAllocSplitRows = 32;
constexpr size_t kNoAllocCounterBytes = sizeof(uint64_t) * kNoAllocSplitRows * kHeads * kArrivalStride;
constexpr size_t kNoAllocPartialBytes =
    sizeof(uint64_t) * kNoAllocSplitRows * kHeads * kFixedSlots * kSlotWords;
constexpr size_t kNoAllocScratchBytes = kNoAllocCounterBytes + kNoAllocPartialBytes;

// Launchers (swiftkv_kernels.hip).
// shape: one of SWIFTKV_STEP_SHAPES (hipErrorInvalidValue otherwise).
hipError_t launch_step(const StepArgs& a, int grid_splits, StepShape shape, InputFormat in, hipStream_t s);
bool step_shape_compiled(StepShape shape);
// Workgroups of the 4-wave step kernel one CU holds at once (0 on error).
int step_workgroups_per_cu();
hipError_t launch_append_bulk(const BulkArgs& a, bool q17, hipStream_t s);
// p[0 .. n) = value, on stream s.
hipError_t launch_fill_u64(uint64_t* p, size_t n, uint64_t value, hipStream_t s);
// Device address of the allocation-free workspace on the current device,
// zero-filled by a kernel on `s` (waits for it).  Call once per device.
hipError_t bind_noalloc_scratch(hipStream_t s, void** device_ptr);
// Integer-compatibility step (one workgroup per (sequence, head)); a.out is
// int32 Q15.17; exp_lut holds the 33 Q30 exp2 entries.
hipError_t launch_exact(const StepArgs& a, const uint32_t* exp_lut, bool q17, hipStream_t s);
// out[i] = Q15.17 of in[i] (parts = 1) or of the reduced split-K partials
// in[i + p * part_stride] (parts = 2 or 4).
hipError_t launch_convert(const float* in, int32_t parts, int64_t part_stride, int32_t* out, size_t n,
                          hipStream_t s);
// Synthetic inputs (swiftkv_synth.hip).
hipError_t launch_fill_f32(float* out, size_t n, uint64_t first, uint64_t seed, uint64_t stream, int dist,
                           int outliers, hipStream_t s);
hipError_t launch_fill_cache(const CacheView& kv, const int2* lut, uint64_t seed, int layer0, int nlayers,
                             int slot0, int nslots, int ntok, int dist, int k_outliers, hipStream_t s);

}  // namespace swiftkv
