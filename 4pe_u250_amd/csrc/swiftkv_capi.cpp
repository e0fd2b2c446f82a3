// swiftkv_capi.cpp -- host side of the SwiftKV C ABI (include/swiftkv.h).
//
// Owns the HIP stream, the device-resident RoPE table and KV arena, the
// split-context workspace and the argument validation that the reference's
// XRT host performs before each launch (host/decode_host.cpp:1340-1349).
// Kernels live in swiftkv_kernels.hip (the step, bulk append, conversion),
// swiftkv_exact.hip (the integer-compatibility step) and swiftkv_synth.hip
// (synthetic inputs); this file only validates, sizes and enqueues.  No exception crosses the C boundary: every entry point converts
// failures to a negative status and a thread-local message.
#include "../../include/swiftkv.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "swiftkv_common.hpp"

namespace {

using namespace swiftkv;

constexpr int kTimerSlots = 64;
constexpr int kProfilePairs = 8192;
constexpr size_t kRopeEntryBytes = sizeof(int2);
constexpr int kMaxSplitTokens = SWIFTKV_MAX_SEQ;

static_assert(SWIFTKV_HEADS == kHeads && SWIFTKV_HEAD_DIM == kHeadDim, "geometry");
static_assert(SWIFTKV_ROPE_LUT_BYTES_PER_POSITION == 512, "RoPE LUT image: 8 x 64-byte words per position");
static_assert(SWIFTKV_RECORD_BYTES == 5 * 64, "record is [meta, K0, K1, V0, V1]");
static_assert(SWIFTKV_NOALLOC_WORKSPACE_BYTES == kNoAllocScratchBytes, "allocation-free workspace size");
static_assert(SWIFTKV_A14_WORD_BYTES == kA14WordBytes, "A14 word: 32 x 14 bits");

// A fixed buffer, so that reporting an error never allocates.
thread_local char g_last_error[512];

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_last_error[0] = '\0';
    return SWIFTKV_OK;
}

#define SKV_HIP(expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return fail(SWIFTKV_EHIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                        __LINE__);                                                             \
    } while (0)

struct ProfilePair {
    hipEvent_t begin;
    hipEvent_t end;
    int kind;
};

// Device address of the allocation-free entry's workspace, per device,
// resolved and zeroed once (by the first context created on the device).
std::mutex g_scratch_mutex;
std::vector<void*> g_scratch;

hipError_t scratch_for_device(int device, int count, hipStream_t s, void** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch.size() < static_cast<size_t>(count)) g_scratch.resize(static_cast<size_t>(count), nullptr);
    if (!g_scratch[device]) {
        void* p = nullptr;
        const hipError_t e = bind_noalloc_scratch(s, &p);
        if (e != hipSuccess) return e;
        g_scratch[device] = p;
    }
    *out = g_scratch[device];
    return hipSuccess;
}

}  // namespace

struct swiftkv_context {
    int device = 0;
    int cus = 256;              // compute units of the device
    int step_per_cu = 3;        // 4-wave step workgroups one CU holds at once
    hipStream_t stream = nullptr;
    int32_t split_tokens = 0;   // 0: heuristic
    StepShape forced_shape{0, 0};   // testing aid: waves 0 = the launch plan's shape
    // split-context workspace: [partial_rows][32] arrival words (kArrivalStride
    // apart), then [partial_rows][32][partial_slots][kSlotWords] tagged words,
    // zero-filled when allocated (generation 0; tag 0 is never current)
    uint64_t* partials = nullptr;
    int32_t partial_rows = 0;
    int32_t partial_slots = 0;
    // Graphs record the workspace pointer in their kernel nodes.  Each graph
    // names the buffer it recorded (if any), with a count of live graphs per
    // buffer here; a buffer the workspace outgrows is freed at once unless a
    // live graph recorded it, and is then kept in `retired` until the last
    // such graph is destroyed.
    std::unordered_map<void*, int64_t> graph_refs;
    std::vector<void*> retired;
    bool capture_uses_workspace = false;   // a split launch of the capture in progress used `partials`
    // [kMaxBatchPerLaunch][32] arrival words (kArrivalStride apart), zero, for
    // launches that split no head: the step reads its arrival word on every
    // path but only a split head's merge writes one
    uint64_t* arrivals = nullptr;
    uint8_t* scratch = nullptr;     // this device's allocation-free workspace (arrival words, then partials)
    // Fault word of the split merges: pinned host memory that a step kernel
    // writes (system scope) when a merge gives up on a partial, read without
    // a device round trip by swiftkv_synchronize, the step entries and graph
    // launches, which report it once and clear it.
    uint32_t* fault_host = nullptr;
    uint32_t* fault_dev = nullptr;
    bool merge_fault_test = false;  // testing aid: merges wait for a tag no word carries
    // timing
    hipEvent_t timers[kTimerSlots] = {};
    bool profiling = false;
    std::vector<ProfilePair> profile_pool;
    size_t profile_used = 0;
    bool capturing = false;     // the stream is being recorded into a graph
    // host-memory I/O mode: step inputs/outputs are host pointers staged here
    bool host_io = false;
    uint8_t* io_stage = nullptr;
    size_t io_bytes = 0;
    // Objects created from the context (caches, tables, graphs, device
    // buffers) may outlive swiftkv_context_destroy: the context is only
    // marked released then, and freed when the last of them is destroyed.
    int64_t children = 0;
    bool released = false;
    std::unordered_set<void*> buffers;   // swiftkv_device_alloc allocations not yet freed
};

struct swiftkv_graph {
    swiftkv_context* ctx = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    void* workspace = nullptr;   // the split workspace buffer its launches recorded, if any
};

struct swiftkv_rope_lut {
    swiftkv_context* ctx = nullptr;
    int32_t positions = 0;
    int2* table = nullptr;              // device [positions][64] (cos, sin)
    std::vector<int2> host;             // host copy for export
};

struct swiftkv_kv_cache {
    swiftkv_context* ctx = nullptr;
    int32_t layers = 0;
    int32_t max_batch = 0;
    int32_t seq_cap = 0;
    int64_t page_bytes = 0;
    size_t bytes = 0;
    int8_t* base = nullptr;
};

namespace {

int set_device(const swiftkv_context* ctx) {
    if (ctx->released) return fail(SWIFTKV_ESTATE, "the context has been destroyed");
    SKV_HIP(hipSetDevice(ctx->device));
    return SWIFTKV_OK;
}

void free_context(swiftkv_context* ctx);

// One object created from `ctx` has been destroyed.
void release_child(swiftkv_context* ctx) {
    if (--ctx->children == 0 && ctx->released) free_context(ctx);
}

// Entry points that synchronize, copy, allocate or memset cannot be recorded.
int not_capturing(const swiftkv_context* ctx, const char* what) {
    if (ctx && ctx->capturing) return fail(SWIFTKV_ESTATE, "%s is not allowed during graph capture", what);
    return SWIFTKV_OK;
}

// A split merge that gave up waiting for another split's partial (its head's
// output holds NaN) left slot * 32 + head + 1 in the context's fault word:
// report it once, as a HIP-side failure, and clear the word.
int take_fault(swiftkv_context* ctx) {
    if (!ctx->fault_host) return SWIFTKV_OK;
    const uint32_t f = __atomic_exchange_n(ctx->fault_host, 0u, __ATOMIC_ACQ_REL);
    if (f == 0) return SWIFTKV_OK;
    const uint32_t slot = (f - 1) / kHeads, head = (f - 1) % kHeads;
    return fail(SWIFTKV_EHIP, "a split merge of an earlier step gave up waiting for another split's partial "
                "(cache slot %u, head %u, perhaps among others): that head's output holds NaN", slot, head);
}

// A graph that recorded workspace buffer `p` has been destroyed: when no live
// graph records it any more and the workspace has outgrown it, free it.
int release_graph_workspace(swiftkv_context* ctx, void* p) {
    auto it = ctx->graph_refs.find(p);
    if (it == ctx->graph_refs.end() || --it->second > 0) return SWIFTKV_OK;
    ctx->graph_refs.erase(it);
    auto r = std::find(ctx->retired.begin(), ctx->retired.end(), p);
    if (r == ctx->retired.end()) return SWIFTKV_OK;   // still the current workspace
    ctx->retired.erase(r);
    const hipError_t sync = hipStreamSynchronize(ctx->stream);
    const hipError_t fr = hipFree(p);
    if (sync != hipSuccess || fr != hipSuccess)
        return fail(SWIFTKV_EHIP, "releasing a split workspace: %s",
                    hipGetErrorString(sync != hipSuccess ? sync : fr));
    return SWIFTKV_OK;
}

// Growth of the host-memory I/O stage.  The old buffer may still be read by
// queued kernels, so the stream is drained before it is released (graphs
// never use the stage: host-memory I/O cannot be captured).
template <typename T>
int ensure(swiftkv_context* ctx, T*& ptr, size_t& have, size_t need) {
    if (need <= have) return SWIFTKV_OK;
    if (ptr) {
        SKV_HIP(hipStreamSynchronize(ctx->stream));
        SKV_HIP(hipFree(ptr));
        ptr = nullptr;
        have = 0;
    }
    void* p = nullptr;
    if (hipMalloc(&p, need * sizeof(T)) != hipSuccess)
        return fail(SWIFTKV_ENOMEM, "hipMalloc of %zu bytes failed", need * sizeof(T));
    ptr = static_cast<T*>(p);
    have = need;
    return SWIFTKV_OK;
}

// Words of a split workspace for `rows` sequences: the arrival words, then
// the partials of `slots` splits per (row, head).
size_t arrival_words(int32_t rows) { return static_cast<size_t>(rows) * kHeads * kArrivalStride; }
size_t workspace_words(int32_t rows, int32_t slots) {
    return arrival_words(rows) + static_cast<size_t>(rows) * kHeads * slots * kSlotWords;
}

// The split workspace for a launch of `rows` sequences split `slots` ways.
// The layout (rows, slots) stays fixed for the life of a buffer, so a word
// left by an earlier launch sits where the same (row, head, split) wrote it,
// with an older generation's tag; a new buffer is zero-filled.  Each buffer
// carries its own arrival words: a buffer kept for a graph counts its own
// generations, so the tag wrap that clears one buffer's slots can never let
// another buffer's old words pass for current ones.
int ensure_partials(swiftkv_context* ctx, int32_t rows, int32_t slots) {
    if (rows <= ctx->partial_rows && slots <= ctx->partial_slots) return SWIFTKV_OK;
    if (ctx->capturing)
        return fail(SWIFTKV_ESTATE, "split workspace too small during graph capture (%d x %d slots < %d x %d): run "
                    "the call once before capturing", ctx->partial_rows, ctx->partial_slots, rows, slots);
    const int32_t new_rows = std::max(rows, ctx->partial_rows);
    const int32_t new_slots = std::max({slots, ctx->partial_slots, kFixedSlots});
    if (ctx->partials) {
        if (ctx->graph_refs.count(ctx->partials)) {
            ctx->retired.push_back(ctx->partials);
        } else {
            SKV_HIP(hipStreamSynchronize(ctx->stream));
            SKV_HIP(hipFree(ctx->partials));
        }
        ctx->partials = nullptr;
        ctx->partial_rows = ctx->partial_slots = 0;
    }
    const size_t bytes = sizeof(uint64_t) * workspace_words(new_rows, new_slots);
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return fail(SWIFTKV_ENOMEM, "hipMalloc of %zu bytes failed", bytes);
    const hipError_t e = hipMemsetAsync(p, 0, bytes, ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return fail(SWIFTKV_EHIP, "split workspace zero-fill: %s", hipGetErrorString(e));
    }
    ctx->partials = static_cast<uint64_t*>(p);
    ctx->partial_rows = new_rows;
    ctx->partial_slots = new_slots;
    return SWIFTKV_OK;
}

// Closed form of scripts/generate_rope_lut.py:67-91: RNE(2^17 cos|sin(pos *
// theta^(-j/64))), saturated to signed 19 bits.
int32_t q17_19bit(double x) {
    double r = std::nearbyint(x * 131072.0);
    r = std::min(262143.0, std::max(-262144.0, r));
    return static_cast<int32_t>(r);
}

uint32_t get_bits(const uint8_t* base, int bit, int width) {
    uint32_t v = 0;
    for (int b = 0; b < width; ++b) {
        const int src = bit + b;
        v |= static_cast<uint32_t>((base[src >> 3] >> (src & 7)) & 1u) << b;
    }
    return v;
}

void put_bits(uint8_t* base, int bit, int width, uint32_t value) {
    for (int b = 0; b < width; ++b) {
        const int dst = bit + b;
        if ((value >> b) & 1u) base[dst >> 3] |= static_cast<uint8_t>(1u << (dst & 7));
    }
}

int32_t sext19(uint32_t raw) {
    return (raw & 0x40000u) ? static_cast<int32_t>(raw | 0xfff80000u) : static_cast<int32_t>(raw);
}

int upload_lut(swiftkv_context* ctx, std::vector<int2>&& host, int32_t positions, swiftkv_rope_lut** out) {
    swiftkv_rope_lut* lut = new (std::nothrow) swiftkv_rope_lut();
    if (!lut) return fail(SWIFTKV_ENOMEM, "out of host memory");
    lut->ctx = ctx;
    lut->positions = positions;
    lut->host = std::move(host);
    const size_t bytes = lut->host.size() * kRopeEntryBytes;
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        delete lut;
        return fail(SWIFTKV_ENOMEM, "hipMalloc of RoPE table (%zu bytes) failed", bytes);
    }
    lut->table = static_cast<int2*>(p);
    hipError_t e = hipMemcpy(lut->table, lut->host.data(), bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(lut->table);
        delete lut;
        return fail(SWIFTKV_EHIP, "RoPE table upload: %s", hipGetErrorString(e));
    }
    ++ctx->children;
    *out = lut;
    return ok();
}

// Tokens per split.  A launch runs best when it fills one residency round:
// one 8-wave workgroup per CU (step_shape picks 8 waves for such launches),
// or step_per_cu 4-wave workgroups per CU.  So
//   batch x 32 heads <= CUs:  splits = CUs / heads (at most 8);
//   otherwise:                splits = step_per_cu x CUs / heads (at least 1),
// rounded to whole 256-token quanta.  Measured on 256 CUs, 32 layers,
// us/layer with this rule's split against forced ones:
//   batch 1, context 4096: 512 tokens (8 splits) 10.44-10.47; 768 10.72,
//   1024 11.8-12.1;  context 2048: 256 (8 splits) 7.94-7.98; 512 8.45-8.72;
//   batch 2: 1024 (4 splits) 15.79-15.89; 512 16.5-16.7, 1280 16.3-16.4;
//   batch 3 and 4: 2048 (2 splits) 21.4 and 26.6; 1024 23.9 and 27.8;
//   batch 8: none 47.4; 2048 49.6-49.9.  Earlier builds: batch 16, 32 and
//   64 unsplit (98.4, 189.8, 361 against 101.2, 192.1, 377 with 4, 2, 2).
// No split is longer than kMaxSplitTokensHeuristic: on long contexts a
// split's exchange is small against its scan and finer work balances better
// (batch 16 decoding from position 32256: 698 us/step with 8192-token splits
// against 703-705 with none).  At most kMaxSplitsPerHead splits: at batch 1
// the merge's latency grows with the split count faster than the shorter
// scans save (16 splits: 15.7 us against 14.5 with 8, at 4 waves per
// workgroup).
constexpr int64_t kMaxSplitsPerHead = 8;
constexpr int64_t kMaxSplitTokensHeuristic = 8192;

// What the launch plan depends on: the device's compute units, the 4-wave
// step workgroups one CU holds, and the forced split (0: the heuristic).
struct SplitPolicy {
    int32_t cus;
    int32_t step_per_cu;
    int32_t split_tokens;
    StepShape forced_shape;   // waves 0: the heuristic's
};
SplitPolicy policy_of(const swiftkv_context* ctx) {
    return {ctx->cus, ctx->step_per_cu, ctx->split_tokens, ctx->forced_shape};
}

int32_t choose_split(const SplitPolicy& pol, const int32_t* positions, int32_t batch) {
    if (pol.split_tokens > 0) return pol.split_tokens;
    int32_t max_len = 1;
    for (int32_t b = 0; b < batch; ++b) max_len = std::max(max_len, positions[b] + 1);
    const int64_t heads = static_cast<int64_t>(batch) * kHeads;
    const int64_t slots = heads <= pol.cus ? pol.cus : static_cast<int64_t>(pol.cus) * pol.step_per_cu;
    const int64_t by_length = (max_len + kMaxSplitTokensHeuristic - 1) / kMaxSplitTokensHeuristic;
    const int64_t splits_per_head =
        std::min<int64_t>(kMaxSplitsPerHead, std::max<int64_t>({int64_t(1), slots / heads, by_length}));
    const int64_t tokens = (max_len + splits_per_head - 1) / splits_per_head;
    const int64_t quanta = std::max<int64_t>(1, (tokens + kSplitQuantum - 1) / kSplitQuantum);
    return static_cast<int32_t>(std::min<int64_t>(quanta * kSplitQuantum, kMaxSeq));
}

// Launch shape.  Up to one residency round of 4-wave workgroups (step_per_cu
// per CU), a launch runs 8 waves per workgroup on 32-token blocks.  A larger
// launch runs 8 waves on 64-token blocks, one workgroup per CU, when every
// workgroup's range holds at least kLongRangeTokens (its shortest row's
// length or the split, whichever is less); otherwise 4 waves on 64-token
// blocks, three workgroups per CU overlapping each other's prologues.
// 32 layers, us/layer, one process, interleaved rounds, against the 4-wave
// shape (measured before the leading kernel arguments were preloaded, which
// took about 0.4 us off every small launch in every shape): batch 1 to 8 at
// context 4096 10.75 / 16.16 / 26.85 / 47.65 against
// 12.05 / 17.42 / 28.14 / 49.0 (and 11.25 / 16.45 / 27.55 / 48.5 with 16
// waves on 32-token blocks); batch 1 at context 2048 8.47 against 8.76;
// batch 12 (two splits) 72.6 against 73.55; batch 16 92.4 against 93.0;
// with 8 waves on 64-token blocks batch 32 / 48 / 64 180.7 / 268.65 / 357.2
// against 181.75 / 270.6 / 359.8, and batch 16 at context 32768 695.6
// against 699.7 per layer; the ragged batch 64 (rows of 256 to 4096 tokens)
// 216.35 with 4 waves against 216.8 with 8.
StepShape step_shape(const SplitPolicy& pol, int32_t grid_splits, int32_t batch, int32_t split_tokens,
                     int32_t min_len) {
    if (pol.forced_shape.waves != 0) return pol.forced_shape;
    const int64_t workgroups = static_cast<int64_t>(grid_splits) * kHeads * batch;
    if (workgroups <= static_cast<int64_t>(pol.cus) * pol.step_per_cu) return kWideShape;
    return std::min(split_tokens, min_len) >= kLongRangeTokens ? kLongShape : kNarrowShape;
}

// Dispatch rows of one launch: (position, sequence) longest first, equal
// positions in sequence order (so a uniform batch keeps its natural order).
// The keys are unique, so an in-place sort of them (no allocation) is stable.
void set_rows(StepArgs& a, const int32_t* positions) {
    uint32_t key[kMaxBatchPerLaunch];
    for (int32_t b = 0; b < a.batch; ++b)
        key[b] = (static_cast<uint32_t>(kMaxSeq - 1 - positions[b]) << 8) | static_cast<uint32_t>(b);
    std::sort(key, key + a.batch);
    for (int32_t z = 0; z < a.batch; ++z) {
        const int32_t b = static_cast<int32_t>(key[z] & 0xffu);
        a.rows[z] = pack_row(b, positions[b]);
    }
}

// How a step's q/k/v arrive: the format and, for split-K partials, the
// element distance between consecutive partials of one tensor.
struct StepInput {
    InputFormat format;
    int64_t part_stride;
    int parts() const { return format == kInParts2 || format == kInParts4 ? static_cast<int>(format) : 1; }
    // Elements one tensor spans for `batch` rows.
    size_t extent(int32_t batch) const {
        return static_cast<size_t>(parts() - 1) * static_cast<size_t>(part_stride) +
               static_cast<size_t>(batch) * kModelDim;
    }
};
constexpr StepInput kF32Input{kInF32, 0}, kQ17Input{kInQ17, 0};

// Largest distance between split-K partials (2^40 elements, 4 TiB): keeps
// every extent computed from it far from overflow.
constexpr int64_t kMaxPartStride = int64_t(1) << 40;

// Positions the integer-compatibility entry accepts: the reference's own
// bound.  Its position is ap_uint<12> and SWIFTKV_MAX_SEQ_LEN = 4096
// (swiftkv_attention.hpp:26-30); Z, a Q13.17 sum of at most position + 1
// coefficients of at most 1.0 wrapped to 30 bits, cannot wrap only while the
// sequence stays below 2^13 tokens, which the reference asserts at compile
// time (swiftkv_attention.cpp:112-119).  Past the bound the recurrence would
// wrap where the reference has no defined result.
constexpr int32_t kExactPositions = SWIFTKV_REFERENCE_MAX_SEQ;

// exact: the integer-compatibility entry, which also refuses positions at or
// past kExactPositions.
int validate_step(swiftkv_context* ctx, const void* q, const void* k, const void* v,
                  const swiftkv_kv_cache* kv, const swiftkv_rope_lut* lut, const uint8_t* act_q,
                  const uint8_t* act_scale, int32_t layer, const int32_t* positions, int32_t batch,
                  const float* out, bool exact = false) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (!q || !k || !v || !out) return fail(SWIFTKV_EINVAL, "null q/k/v/out pointer");
    if (!kv || kv->ctx != ctx) return fail(SWIFTKV_EINVAL, "kv_cache is null or belongs to another context");
    if (!lut || lut->ctx != ctx) return fail(SWIFTKV_EINVAL, "rope_lut is null or belongs to another context");
    if ((act_q == nullptr) != (act_scale == nullptr))
        return fail(SWIFTKV_EINVAL, "activation_q and activation_scale must both be set or both be null");
    if (!positions) return fail(SWIFTKV_EINVAL, "null positions");
    if (batch < 1 || batch > kv->max_batch)
        return fail(SWIFTKV_ERANGE, "batch %d outside [1, %d]", batch, kv->max_batch);
    if (layer < 0 || layer >= kv->layers)
        return fail(SWIFTKV_ERANGE, "layer_index %d outside [0, %d)", layer, kv->layers);
    const int32_t limit = std::min(kv->seq_cap, lut->positions);
    for (int32_t b = 0; b < batch; ++b)
        if (positions[b] < 0 || positions[b] >= limit)
            return fail(SWIFTKV_ERANGE, "positions[%d] = %d outside [0, %d) (cache %d, RoPE table %d)", b,
                        positions[b], limit, kv->seq_cap, lut->positions);
    if (exact)
        for (int32_t b = 0; b < batch; ++b)
            if (positions[b] >= kExactPositions)
                return fail(SWIFTKV_ERANGE, "positions[%d] = %d: the integer-compatibility entry keeps the "
                            "reference's bound position < %d (its Q13.17 normalizer may wrap beyond it)", b,
                            positions[b], kExactPositions);
    return SWIFTKV_OK;
}

ProfilePair* profile_begin(swiftkv_context* ctx, int kind) {
    if (!ctx->profiling || ctx->capturing || ctx->profile_used >= ctx->profile_pool.size()) return nullptr;
    ProfilePair* p = &ctx->profile_pool[ctx->profile_used++];
    p->kind = kind;
    if (hipEventRecord(p->begin, ctx->stream) != hipSuccess) return nullptr;
    return p;
}

void profile_end(swiftkv_context* ctx, ProfilePair* p) {
    if (p) (void)hipEventRecord(p->end, ctx->stream);
}

// The arguments of one step call, for the launches it makes.
struct StepCall {
    const void* q;
    const void* k;
    const void* v;
    StepInput in;
    swiftkv_kv_cache* kv;
    const swiftkv_rope_lut* lut;
    uint8_t* act_q;
    uint8_t* act_scale;
    int32_t layer;
    const int32_t* positions;
    float* out;
};

// One step launch over the call's sequences [b0, b0 + nb) with the given
// split and shape.  noalloc: the split workspace is this device's fixed
// array (split launches of at most kNoAllocSplitRows sequences).
int launch_rows(swiftkv_context* ctx, const StepCall& c, int32_t b0, int32_t nb, int32_t split_tokens,
                StepShape shape, bool noalloc) {
    constexpr size_t elem_bytes = 4;
    StepArgs a;
    std::memset(&a, 0, sizeof(a));
    const size_t row0 = static_cast<size_t>(b0) * kModelDim;
    a.q = static_cast<const char*>(c.q) + row0 * elem_bytes;
    a.k = static_cast<const char*>(c.k) + row0 * elem_bytes;
    a.v = static_cast<const char*>(c.v) + row0 * elem_bytes;
    a.part_stride = c.in.part_stride;
    a.kv = CacheView{c.kv->base, c.kv->page_bytes, c.kv->seq_cap, c.kv->layers};
    a.lut = c.lut->table;
    a.lut_positions = c.lut->positions;
    a.layer = c.layer;
    a.batch = nb;
    a.slot0 = b0;
    int32_t max_pos = 0;
    for (int32_t b = 0; b < nb; ++b) max_pos = std::max(max_pos, c.positions[b0 + b]);
    set_rows(a, c.positions + b0);
    a.split_tokens = split_tokens;
    const int32_t grid_splits = (max_pos + 1 + split_tokens - 1) / split_tokens;
    int rc;
    if (grid_splits > 1 && noalloc) {
        a.arrivals = reinterpret_cast<uint64_t*>(ctx->scratch);
        a.partials = reinterpret_cast<uint64_t*>(ctx->scratch + kNoAllocCounterBytes);
        a.slot_stride = kFixedSlots;
    } else if (grid_splits > 1) {
        if ((rc = ensure_partials(ctx, nb, grid_splits))) return rc;
        if (ctx->capturing) ctx->capture_uses_workspace = true;
        a.arrivals = ctx->partials;
        a.partials = ctx->partials + arrival_words(ctx->partial_rows);
        a.slot_stride = ctx->partial_slots;
    } else {
        a.arrivals = ctx->arrivals;   // read, never written, by a launch that splits no head
        a.partials = nullptr;
        a.slot_stride = 0;
    }
    a.out = c.out + row0;
    a.act_q = c.act_q ? c.act_q + static_cast<size_t>(b0) * kHeads * kGroupsPerHead * SWIFTKV_A14_WORD_BYTES
                      : nullptr;
    a.act_scale = c.act_scale ? c.act_scale + static_cast<size_t>(b0) * kHeads * kGroupsPerHead : nullptr;
    a.merge_polls = ctx->merge_fault_test ? 1u : kMergePolls;
    a.merge_tag_skew = ctx->merge_fault_test ? 1u : 0u;
    a.fault = ctx->fault_dev;
    ProfilePair* p = profile_begin(ctx, SWIFTKV_KERNEL_STEP);
    SKV_HIP(launch_step(a, grid_splits, shape, c.in.format, ctx->stream));
    profile_end(ctx, p);
    return SWIFTKV_OK;
}

// The call runs one launch per kMaxBatchPerLaunch sequences, each planned
// (split and shape) on its own sequences.  noalloc: the split workspace is
// this device's fixed file-scope array instead of the context's growable
// buffer.  It holds kFixedSlots splits per head of kNoAllocSplitRows
// sequences: a plan that splits heads more ways is refused (SWIFTKV_ERANGE)
// before anything is enqueued, and a split launch of more sequences runs as
// launches of kNoAllocSplitRows sequences with the same plan, so every head
// sees the same split and shape, and gives the same bits, as in the
// allocating entry.
int run_step(swiftkv_context* ctx, const void* q, const void* k, const void* v, StepInput in,
             swiftkv_kv_cache* kv, const swiftkv_rope_lut* lut, uint8_t* act_q, uint8_t* act_scale,
             int32_t layer, const int32_t* positions, int32_t batch, float* out, bool noalloc = false) {
    int rc = validate_step(ctx, q, k, v, kv, lut, act_q, act_scale, layer, positions, batch, out);
    if (rc) return rc;
    if ((rc = set_device(ctx))) return rc;
    if (noalloc) {   // check every launch first, so a refused call enqueues nothing
        for (int32_t b0 = 0; b0 < batch; b0 += kMaxBatchPerLaunch) {
            const int32_t nb = std::min<int32_t>(kMaxBatchPerLaunch, batch - b0);
            int32_t max_pos = 0;
            for (int32_t b = 0; b < nb; ++b) max_pos = std::max(max_pos, positions[b0 + b]);
            const int32_t split = choose_split(policy_of(ctx), positions + b0, nb);
            const int32_t splits = (max_pos + split) / split;
            if (splits > kFixedSlots)
                return fail(SWIFTKV_ERANGE, "the step splits a head %d ways (%d-token splits of up to %d tokens); the "
                            "allocation-free entry's workspace holds %d splits per head: use longer splits", splits,
                            split, max_pos + 1, kFixedSlots);
        }
    }
    const StepCall call{q, k, v, in, kv, lut, act_q, act_scale, layer, positions, out};
    for (int32_t b0 = 0; b0 < batch; b0 += kMaxBatchPerLaunch) {
        const int32_t nb = std::min<int32_t>(kMaxBatchPerLaunch, batch - b0);
        int32_t max_pos = 0, min_pos = kMaxSeq;
        for (int32_t b = 0; b < nb; ++b) {
            max_pos = std::max(max_pos, positions[b0 + b]);
            min_pos = std::min(min_pos, positions[b0 + b]);
        }
        const int32_t split = choose_split(policy_of(ctx), positions + b0, nb);
        const int32_t grid_splits = (max_pos + split) / split;
        const StepShape shape = step_shape(policy_of(ctx), grid_splits, nb, split, min_pos + 1);
        const int32_t rows = noalloc && grid_splits > 1 ? kNoAllocSplitRows : nb;
        for (int32_t s0 = 0; s0 < nb; s0 += rows)
            if ((rc = launch_rows(ctx, call, b0 + s0, std::min(rows, nb - s0), split, shape, noalloc))) return rc;
    }
    return ok();
}

// Q30 exp2 table RNE(2^(30 + i/32)), i = 0..32 (swiftkv_attention.cpp:185-195).
const uint32_t* exp2_table() {
    static const std::vector<uint32_t> table = [] {
        std::vector<uint32_t> t(33);
        for (int i = 0; i < 33; ++i)
            t[i] = static_cast<uint32_t>(std::nearbyint(std::ldexp(std::pow(2.0, i / 32.0), 30)));
        return t;
    }();
    return table.data();
}

int run_exact(swiftkv_context* ctx, const void* q, const void* k, const void* v, StepInput in,
              swiftkv_kv_cache* kv, const swiftkv_rope_lut* lut, uint8_t* act_q, uint8_t* act_scale,
              int32_t layer, const int32_t* positions, int32_t batch, int32_t* out) {
    int rc = validate_step(ctx, q, k, v, kv, lut, act_q, act_scale, layer, positions, batch,
                           reinterpret_cast<const float*>(out), true);
    if (rc) return rc;
    if ((rc = set_device(ctx))) return rc;
    for (int32_t b0 = 0; b0 < batch; b0 += kMaxBatchPerLaunch) {
        const int32_t nb = std::min<int32_t>(kMaxBatchPerLaunch, batch - b0);
        StepArgs a;
        std::memset(&a, 0, sizeof(a));
        const size_t row0 = static_cast<size_t>(b0) * kModelDim;
        a.q = static_cast<const char*>(q) + row0 * 4;
        a.k = static_cast<const char*>(k) + row0 * 4;
        a.v = static_cast<const char*>(v) + row0 * 4;
        a.kv = CacheView{kv->base, kv->page_bytes, kv->seq_cap, kv->layers};
        a.lut = lut->table;
        a.lut_positions = lut->positions;
        a.layer = layer;
        a.batch = nb;
        a.slot0 = b0;
        set_rows(a, positions + b0);
        a.out = reinterpret_cast<float*>(out + row0);
        a.act_q = act_q ? act_q + static_cast<size_t>(b0) * kHeads * kGroupsPerHead * SWIFTKV_A14_WORD_BYTES
                        : nullptr;
        a.act_scale = act_scale ? act_scale + static_cast<size_t>(b0) * kHeads * kGroupsPerHead : nullptr;
        ProfilePair* p = profile_begin(ctx, SWIFTKV_KERNEL_EXACT);
        SKV_HIP(launch_exact(a, exp2_table(), in.format == kInQ17, ctx->stream));
        profile_end(ctx, p);
    }
    return ok();
}

// Entry dispatch.  In host-memory I/O mode the step's q/k/v, output and
// activation pointers are host memory: inputs are copied into a context-owned
// device stage on the context stream, the step runs on the staged copies, the
// outputs are copied back and the call waits for them, so the host buffers
// are valid on return (the reference host does the same around each PE call:
// DMA in, run, DMA out, decode_host.cpp:1358-1485).
int dispatch_step(swiftkv_context* ctx, bool exact, const void* q, const void* k, const void* v, StepInput in,
                  swiftkv_kv_cache* kv, const swiftkv_rope_lut* lut, uint8_t* act_q, uint8_t* act_scale,
                  int32_t layer, const int32_t* positions, int32_t batch, void* out) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (int rc = take_fault(ctx)) return rc;
    if (!ctx->host_io) {
        return exact ? run_exact(ctx, q, k, v, in, kv, lut, act_q, act_scale, layer, positions, batch,
                                 static_cast<int32_t*>(out))
                     : run_step(ctx, q, k, v, in, kv, lut, act_q, act_scale, layer, positions, batch,
                                static_cast<float*>(out));
    }
    int rc = validate_step(ctx, q, k, v, kv, lut, act_q, act_scale, layer, positions, batch,
                           static_cast<const float*>(out), exact);
    if (rc) return rc;
    if ((rc = set_device(ctx))) return rc;
    auto align = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    const size_t in_bytes = in.extent(batch) * 4;   // one input tensor, all its partials
    const size_t row_bytes = static_cast<size_t>(batch) * kModelDim * 4;
    const size_t aq_bytes = static_cast<size_t>(batch) * kHeads * kGroupsPerHead * SWIFTKV_A14_WORD_BYTES;
    const size_t as_bytes = static_cast<size_t>(batch) * kHeads * kGroupsPerHead;
    const size_t off_k = align(in_bytes), off_v = 2 * align(in_bytes), off_out = 3 * align(in_bytes);
    const size_t off_aq = off_out + align(row_bytes);
    const size_t off_as = off_aq + align(aq_bytes), total = off_as + align(as_bytes);
    if ((rc = ensure(ctx, ctx->io_stage, ctx->io_bytes, total))) return rc;
    uint8_t* st = ctx->io_stage;
    SKV_HIP(hipMemcpyAsync(st, q, in_bytes, hipMemcpyHostToDevice, ctx->stream));
    SKV_HIP(hipMemcpyAsync(st + off_k, k, in_bytes, hipMemcpyHostToDevice, ctx->stream));
    SKV_HIP(hipMemcpyAsync(st + off_v, v, in_bytes, hipMemcpyHostToDevice, ctx->stream));
    uint8_t* d_aq = act_q ? st + off_aq : nullptr;
    uint8_t* d_as = act_scale ? st + off_as : nullptr;
    rc = exact ? run_exact(ctx, st, st + off_k, st + off_v, in, kv, lut, d_aq, d_as, layer, positions, batch,
                           reinterpret_cast<int32_t*>(st + off_out))
               : run_step(ctx, st, st + off_k, st + off_v, in, kv, lut, d_aq, d_as, layer, positions, batch,
                          reinterpret_cast<float*>(st + off_out));
    if (rc) return rc;
    SKV_HIP(hipMemcpyAsync(out, st + off_out, row_bytes, hipMemcpyDeviceToHost, ctx->stream));
    if (act_q) {
        SKV_HIP(hipMemcpyAsync(act_q, d_aq, aq_bytes, hipMemcpyDeviceToHost, ctx->stream));
        SKV_HIP(hipMemcpyAsync(act_scale, d_as, as_bytes, hipMemcpyDeviceToHost, ctx->stream));
    }
    SKV_HIP(hipStreamSynchronize(ctx->stream));
    if ((rc = take_fault(ctx))) return rc;
    return ok();
}

int check_cache_range(const swiftkv_context* ctx, const swiftkv_kv_cache* kv, int32_t seq, int32_t layer,
                      int32_t head, int32_t tok0, int32_t n) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (!kv || kv->ctx != ctx) return fail(SWIFTKV_EINVAL, "kv_cache is null or belongs to another context");
    if (seq < 0 || seq >= kv->max_batch) return fail(SWIFTKV_ERANGE, "sequence %d outside [0, %d)", seq, kv->max_batch);
    if (layer < 0 || layer >= kv->layers) return fail(SWIFTKV_ERANGE, "layer %d outside [0, %d)", layer, kv->layers);
    if (head < 0 || head >= kHeads) return fail(SWIFTKV_ERANGE, "head %d outside [0, %d)", head, kHeads);
    if (n < 0 || tok0 < 0 || static_cast<int64_t>(tok0) + n > kv->seq_cap)
        return fail(SWIFTKV_ERANGE, "tokens [%d, %d) outside the cache capacity %d", tok0, tok0 + n, kv->seq_cap);
    return SWIFTKV_OK;
}

// Shift of a stored G32 scale 2^(s-17): the biased exponent minus 110.
bool scale_to_shift(float scale, uint8_t* s) {
    uint32_t bits;
    std::memcpy(&bits, &scale, 4);
    const uint32_t e = bits >> 23;   // sign bit must be zero
    if ((bits & 0x7fffffu) != 0 || e < 110u || e > 110u + 31u) return false;
    *s = static_cast<uint8_t>(e - 110u);
    return true;
}

float shift_to_scale(uint32_t s) {
    const uint32_t bits = (s + 110u) << 23;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Releases everything the context owns (after its last object is gone).
void free_context(swiftkv_context* ctx) {
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->partials) (void)hipFree(ctx->partials);
    for (void* p : ctx->retired) (void)hipFree(p);
    if (ctx->arrivals) (void)hipFree(ctx->arrivals);
    if (ctx->io_stage) (void)hipFree(ctx->io_stage);
    if (ctx->fault_host) (void)hipHostFree(ctx->fault_host);
    for (auto& t : ctx->timers)
        if (t) (void)hipEventDestroy(t);
    for (auto& p : ctx->profile_pool) {
        (void)hipEventDestroy(p.begin);
        (void)hipEventDestroy(p.end);
    }
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

}  // namespace

extern "C" {

const char* swiftkv_last_error(void) { return g_last_error; }

const char* swiftkv_version(void) { return "swiftkv-mi355x 0.1 (gfx950)"; }

int swiftkv_context_create(int device, swiftkv_context** out) {
    if (!out) return fail(SWIFTKV_EINVAL, "null output pointer");
    *out = nullptr;
    int count = 0;
    SKV_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return fail(SWIFTKV_ERANGE, "device %d outside [0, %d)", device, count);
    SKV_HIP(hipSetDevice(device));
    swiftkv_context* ctx = new (std::nothrow) swiftkv_context();
    if (!ctx) return fail(SWIFTKV_ENOMEM, "out of host memory");
    ctx->device = device;
    hipError_t e = hipDeviceGetAttribute(&ctx->cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e == hipSuccess) ctx->step_per_cu = std::max(1, step_workgroups_per_cu());
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    for (int i = 0; e == hipSuccess && i < kTimerSlots; ++i) e = hipEventCreate(&ctx->timers[i]);
    const size_t arrival_bytes = sizeof(uint64_t) * kMaxBatchPerLaunch * kHeads * kArrivalStride;
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&ctx->arrivals), arrival_bytes);
    if (e == hipSuccess) e = hipMemset(ctx->arrivals, 0, arrival_bytes);
    void* scratch = nullptr;
    if (e == hipSuccess) e = scratch_for_device(device, count, ctx->stream, &scratch);
    ctx->scratch = static_cast<uint8_t*>(scratch);
    void* fault = nullptr;
    if (e == hipSuccess) e = hipHostMalloc(&fault, sizeof(uint32_t), hipHostMallocMapped | hipHostMallocCoherent);
    if (e == hipSuccess) {
        ctx->fault_host = static_cast<uint32_t*>(fault);
        *ctx->fault_host = 0u;
        void* dev = nullptr;
        e = hipHostGetDevicePointer(&dev, fault, 0);
        ctx->fault_dev = static_cast<uint32_t*>(dev);
    }
    if (e != hipSuccess) {
        swiftkv_context_destroy(ctx);
        return fail(SWIFTKV_EHIP, "stream/event creation: %s", hipGetErrorString(e));
    }
    *out = ctx;
    return ok();
}

int swiftkv_context_destroy(swiftkv_context* ctx) {
    if (!ctx) return ok();
    if (ctx->released) return fail(SWIFTKV_ESTATE, "the context has already been destroyed");
    if (ctx->capturing) {   // abandon the recording so the stream can be released
        hipGraph_t g = nullptr;
        (void)hipSetDevice(ctx->device);
        if (hipStreamEndCapture(ctx->stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        ctx->capturing = false;
    }
    ctx->released = true;
    if (ctx->children == 0) free_context(ctx);
    return ok();
}

int swiftkv_synchronize(swiftkv_context* ctx) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    int rc = not_capturing(ctx, "swiftkv_synchronize");
    if (rc) return rc;
    rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(hipStreamSynchronize(ctx->stream));
    if ((rc = take_fault(ctx))) return rc;
    return ok();
}

int swiftkv_debug_force_merge_timeout(swiftkv_context* ctx, int32_t enable) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    ctx->merge_fault_test = enable != 0;
    return ok();
}

int swiftkv_set_split_tokens(swiftkv_context* ctx, int32_t split_tokens) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (split_tokens != 0 &&
        (split_tokens < kSplitQuantum || split_tokens > kMaxSplitTokens || split_tokens % kSplitQuantum != 0))
        return fail(SWIFTKV_EINVAL, "split_tokens %d must be 0 or a multiple of %d in [%d, %d]", split_tokens,
                    kSplitQuantum, kSplitQuantum, kMaxSplitTokens);
    ctx->split_tokens = split_tokens;
    return ok();
}

int swiftkv_debug_set_step_shape(swiftkv_context* ctx, int32_t waves, int32_t block_tokens) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    const StepShape shape{waves, block_tokens};
    if (waves != 0 && !step_shape_compiled(shape))
        return fail(SWIFTKV_EINVAL, "no step kernel is compiled for %d waves on %d-token blocks", waves,
                    block_tokens);
    ctx->forced_shape = waves != 0 ? shape : StepShape{0, 0};
    return ok();
}

int swiftkv_debug_step_plan(int32_t cus, int32_t workgroups_per_cu, int32_t split_tokens, const int32_t* positions,
                            int32_t batch, int32_t* out_split_tokens, int32_t* out_grid_splits, int32_t* out_waves,
                            int32_t* out_block_tokens, int32_t* out_rows) {
    if (!positions || !out_split_tokens || !out_grid_splits || !out_waves)
        return fail(SWIFTKV_EINVAL, "null argument");
    if (cus < 1 || workgroups_per_cu < 1)
        return fail(SWIFTKV_EINVAL, "cus %d and workgroups_per_cu %d must be positive", cus, workgroups_per_cu);
    if (batch < 1 || batch > kMaxBatchPerLaunch)
        return fail(SWIFTKV_ERANGE, "batch %d outside [1, %d] (one launch)", batch, kMaxBatchPerLaunch);
    if (split_tokens != 0 &&
        (split_tokens < kSplitQuantum || split_tokens > kMaxSplitTokens || split_tokens % kSplitQuantum != 0))
        return fail(SWIFTKV_EINVAL, "split_tokens %d must be 0 or a multiple of %d in [%d, %d]", split_tokens,
                    kSplitQuantum, kSplitQuantum, kMaxSplitTokens);
    int32_t max_pos = 0, min_pos = kMaxSeq;
    for (int32_t b = 0; b < batch; ++b) {
        if (positions[b] < 0 || positions[b] >= kMaxSeq)
            return fail(SWIFTKV_ERANGE, "position %d outside [0, %d)", positions[b], kMaxSeq);
        max_pos = std::max(max_pos, positions[b]);
        min_pos = std::min(min_pos, positions[b]);
    }
    const SplitPolicy pol{cus, workgroups_per_cu, split_tokens, StepShape{0, 0}};
    StepArgs a{};
    a.batch = batch;
    set_rows(a, positions);
    *out_split_tokens = choose_split(pol, positions, batch);
    *out_grid_splits = (max_pos + *out_split_tokens) / *out_split_tokens;
    const StepShape shape = step_shape(pol, *out_grid_splits, batch, *out_split_tokens, min_pos + 1);
    *out_waves = shape.waves;
    if (out_block_tokens) *out_block_tokens = shape.block_tokens;
    if (out_rows)
        for (int32_t z = 0; z < batch; ++z) out_rows[z] = static_cast<int32_t>(a.rows[z] & 0xffu);
    return ok();
}

int swiftkv_debug_set_split_generation(swiftkv_context* ctx, uint32_t generation, int32_t noalloc) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    int rc = not_capturing(ctx, "swiftkv_debug_set_split_generation");
    if (rc) return rc;
    if (generation == 0xffffffffu)
        return fail(SWIFTKV_EINVAL, "generation 0xffffffff is reserved (a launch's tag is its generation + 1, and "
                    "tags run over 1 .. 0xffffffff)");
    if ((rc = set_device(ctx))) return rc;
    uint64_t* base = nullptr;
    int32_t rows = 0, slots = 0;
    if (noalloc) {
        base = reinterpret_cast<uint64_t*>(ctx->scratch);
        rows = kNoAllocSplitRows;
        slots = kFixedSlots;
    } else {
        base = ctx->partials;
        rows = ctx->partial_rows;
        slots = ctx->partial_slots;
    }
    if (!base) return ok();   // no split workspace yet: the first one starts at generation 0
    const size_t arrivals = arrival_words(rows);
    SKV_HIP(launch_fill_u64(base, arrivals, static_cast<uint64_t>(generation) << 32, ctx->stream));
    SKV_HIP(launch_fill_u64(base + arrivals, workspace_words(rows, slots) - arrivals, 0, ctx->stream));
    return ok();
}

int swiftkv_set_host_io(swiftkv_context* ctx, int32_t enable) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    int rc = not_capturing(ctx, "swiftkv_set_host_io");
    if (rc) return rc;
    ctx->host_io = enable != 0;
    return ok();
}

// ---------------------------------------------------------------- RoPE table

int swiftkv_rope_lut_load(swiftkv_context* ctx, const void* image, size_t image_bytes, swiftkv_rope_lut** out) {
    if (!ctx || !image || !out) return fail(SWIFTKV_EINVAL, "null argument");
    *out = nullptr;
    if (int rc0 = not_capturing(ctx, "swiftkv_rope_lut_load")) return rc0;
    if (image_bytes == 0 || image_bytes % SWIFTKV_ROPE_LUT_BYTES_PER_POSITION != 0)
        return fail(SWIFTKV_EINVAL, "RoPE image of %zu bytes is not a whole number of %d-byte positions",
                    image_bytes, SWIFTKV_ROPE_LUT_BYTES_PER_POSITION);
    const size_t npos = image_bytes / SWIFTKV_ROPE_LUT_BYTES_PER_POSITION;
    if (npos > static_cast<size_t>(SWIFTKV_MAX_SEQ))
        return fail(SWIFTKV_ERANGE, "RoPE image holds %zu positions, more than %d", npos, SWIFTKV_MAX_SEQ);
    int rc = set_device(ctx);
    if (rc) return rc;
    const uint8_t* bytes = static_cast<const uint8_t*>(image);
    std::vector<int2> host(npos * kRopePairs);
    for (size_t p = 0; p < npos; ++p)
        for (int j = 0; j < kRopePairs; ++j) {
            const uint8_t* slot = bytes + (p * 4 + static_cast<size_t>(j / 16)) * 128;
            const int lane = j % 16;
            host[p * kRopePairs + j] =
                make_int2(sext19(get_bits(slot, 38 * lane, 19)), sext19(get_bits(slot, 38 * lane + 19, 19)));
        }
    return upload_lut(ctx, std::move(host), static_cast<int32_t>(npos), out);
}

int swiftkv_rope_lut_generate(swiftkv_context* ctx, int32_t positions, double theta, swiftkv_rope_lut** out) {
    if (!ctx || !out) return fail(SWIFTKV_EINVAL, "null argument");
    *out = nullptr;
    if (int rc0 = not_capturing(ctx, "swiftkv_rope_lut_generate")) return rc0;
    if (positions < 1 || positions > SWIFTKV_MAX_SEQ)
        return fail(SWIFTKV_ERANGE, "positions %d outside [1, %d]", positions, SWIFTKV_MAX_SEQ);
    if (!(theta > 1.0) || !std::isfinite(theta)) return fail(SWIFTKV_EINVAL, "theta must be finite and > 1");
    int rc = set_device(ctx);
    if (rc) return rc;
    std::vector<int2> host(static_cast<size_t>(positions) * kRopePairs);
    for (int32_t p = 0; p < positions; ++p)
        for (int j = 0; j < kRopePairs; ++j) {
            const double freq = 1.0 / std::pow(theta, static_cast<double>(j) / kRopePairs);
            const double ang = static_cast<double>(p) * freq;
            host[static_cast<size_t>(p) * kRopePairs + j] = make_int2(q17_19bit(std::cos(ang)), q17_19bit(std::sin(ang)));
        }
    return upload_lut(ctx, std::move(host), positions, out);
}

int swiftkv_rope_lut_destroy(swiftkv_rope_lut* lut) {
    if (!lut) return ok();
    swiftkv_context* ctx = lut->ctx;
    if (int rc = not_capturing(ctx, "swiftkv_rope_lut_destroy")) return rc;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (lut->table) (void)hipFree(lut->table);
    delete lut;
    release_child(ctx);
    return ok();
}

int32_t swiftkv_rope_lut_positions(const swiftkv_rope_lut* lut) { return lut ? lut->positions : 0; }

int swiftkv_rope_lut_export(const swiftkv_rope_lut* lut, int32_t pos0, int32_t n, void* image) {
    if (!lut || !image) return fail(SWIFTKV_EINVAL, "null argument");
    if (pos0 < 0 || n < 0 || static_cast<int64_t>(pos0) + n > lut->positions)
        return fail(SWIFTKV_ERANGE, "positions [%d, %d) outside the table (%d)", pos0, pos0 + n, lut->positions);
    uint8_t* bytes = static_cast<uint8_t*>(image);
    std::memset(bytes, 0, static_cast<size_t>(n) * SWIFTKV_ROPE_LUT_BYTES_PER_POSITION);
    for (int32_t p = 0; p < n; ++p)
        for (int j = 0; j < kRopePairs; ++j) {
            const int2 cs = lut->host[static_cast<size_t>(pos0 + p) * kRopePairs + j];
            uint8_t* slot = bytes + (static_cast<size_t>(p) * 4 + static_cast<size_t>(j / 16)) * 128;
            const int lane = j % 16;
            put_bits(slot, 38 * lane, 19, static_cast<uint32_t>(cs.x) & 0x7ffffu);
            put_bits(slot, 38 * lane + 19, 19, static_cast<uint32_t>(cs.y) & 0x7ffffu);
        }
    return ok();
}

// ---------------------------------------------------------------- KV cache

int swiftkv_kv_cache_create(swiftkv_context* ctx, int32_t layers, int32_t max_batch, int32_t max_seq_len,
                            swiftkv_kv_cache** out) {
    if (!ctx || !out) return fail(SWIFTKV_EINVAL, "null argument");
    *out = nullptr;
    if (int rc0 = not_capturing(ctx, "swiftkv_kv_cache_create")) return rc0;
    if (layers < 1 || layers > 64) return fail(SWIFTKV_EINVAL, "layers %d outside [1, 64]", layers);
    if (max_batch < 1 || max_batch > 4096) return fail(SWIFTKV_EINVAL, "max_batch %d outside [1, 4096]", max_batch);
    if (max_seq_len < 1 || max_seq_len > SWIFTKV_MAX_SEQ)
        return fail(SWIFTKV_EINVAL, "max_seq_len %d outside [1, %d]", max_seq_len, SWIFTKV_MAX_SEQ);
    int rc = set_device(ctx);
    if (rc) return rc;
    swiftkv_kv_cache* kv = new (std::nothrow) swiftkv_kv_cache();
    if (!kv) return fail(SWIFTKV_ENOMEM, "out of host memory");
    kv->ctx = ctx;
    kv->layers = layers;
    kv->max_batch = max_batch;
    kv->seq_cap = (max_seq_len + kSeqAlign - 1) / kSeqAlign * kSeqAlign;
    kv->page_bytes = static_cast<int64_t>(kv->seq_cap) * kTokenBytes;
    kv->bytes = static_cast<size_t>(kv->page_bytes) * kHeads * layers * max_batch;
    void* p = nullptr;
    if (hipMalloc(&p, kv->bytes) != hipSuccess) {
        delete kv;
        return fail(SWIFTKV_ENOMEM, "hipMalloc of KV cache (%zu bytes) failed", static_cast<size_t>(kv->bytes));
    }
    kv->base = static_cast<int8_t*>(p);
    hipError_t e = hipMemsetAsync(kv->base, 0, kv->bytes, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(kv->base);
        delete kv;
        return fail(SWIFTKV_EHIP, "KV cache zero-fill: %s", hipGetErrorString(e));
    }
    ++ctx->children;
    *out = kv;
    return ok();
}

int swiftkv_kv_cache_destroy(swiftkv_kv_cache* kv) {
    if (!kv) return ok();
    swiftkv_context* ctx = kv->ctx;
    if (int rc = not_capturing(ctx, "swiftkv_kv_cache_destroy")) return rc;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (kv->base) (void)hipFree(kv->base);
    delete kv;
    release_child(ctx);
    return ok();
}

int swiftkv_kv_cache_zero(swiftkv_context* ctx, swiftkv_kv_cache* kv) {
    if (!ctx || !kv || kv->ctx != ctx) return fail(SWIFTKV_EINVAL, "null or foreign argument");
    int rc = not_capturing(ctx, "swiftkv_kv_cache_zero");
    if (rc) return rc;
    rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(hipMemsetAsync(kv->base, 0, kv->bytes, ctx->stream));
    return ok();
}

size_t swiftkv_kv_cache_bytes(const swiftkv_kv_cache* kv) { return kv ? kv->bytes : 0; }

int swiftkv_kv_cache_read(swiftkv_context* ctx, const swiftkv_kv_cache* kv, int32_t seq, int32_t layer,
                          int32_t head, int32_t tok0, int32_t n, int8_t* k_codes, int8_t* v_codes,
                          float* k_scales, float* v_scales) {
    int rc = check_cache_range(ctx, kv, seq, layer, head, tok0, n);
    if (rc) return rc;
    if ((rc = not_capturing(ctx, "swiftkv_kv_cache_read"))) return rc;
    if ((rc = set_device(ctx))) return rc;
    if (n == 0) return ok();
    const int8_t* page = page_ptr(CacheView{kv->base, kv->page_bytes, kv->seq_cap, kv->layers}, seq, layer, head);
    const size_t cap = static_cast<size_t>(kv->seq_cap);
    SKV_HIP(hipStreamSynchronize(ctx->stream));
    if (k_codes)
        SKV_HIP(hipMemcpy(k_codes, page + static_cast<size_t>(tok0) * kCodeBytes,
                          static_cast<size_t>(n) * kCodeBytes, hipMemcpyDeviceToHost));
    if (v_codes)
        SKV_HIP(hipMemcpy(v_codes, page + (cap + tok0) * kCodeBytes, static_cast<size_t>(n) * kCodeBytes,
                          hipMemcpyDeviceToHost));
    if (k_scales || v_scales) {
        std::vector<float> sc(static_cast<size_t>(n) * 8);
        SKV_HIP(hipMemcpy(sc.data(), page + cap * 2 * kCodeBytes + static_cast<size_t>(tok0) * kScaleBytes,
                          sc.size() * sizeof(float), hipMemcpyDeviceToHost));
        for (int32_t t = 0; t < n; ++t)
            for (int g = 0; g < kGroupsPerHead; ++g) {
                if (k_scales) k_scales[static_cast<size_t>(t) * 4 + g] = sc[static_cast<size_t>(t) * 8 + 2 * g];
                if (v_scales) v_scales[static_cast<size_t>(t) * 4 + g] = sc[static_cast<size_t>(t) * 8 + 2 * g + 1];
            }
    }
    return ok();
}

int swiftkv_kv_cache_export_records(swiftkv_context* ctx, const swiftkv_kv_cache* kv, int32_t seq, int32_t layer,
                                    int32_t head, int32_t tok0, int32_t n, void* records) {
    if (!records && n > 0) return fail(SWIFTKV_EINVAL, "null records");
    std::vector<int8_t> kc(static_cast<size_t>(n) * kCodeBytes), vc(kc.size());
    std::vector<float> ks(static_cast<size_t>(n) * 4), vs(ks.size());
    int rc = swiftkv_kv_cache_read(ctx, kv, seq, layer, head, tok0, n, kc.data(), vc.data(), ks.data(), vs.data());
    if (rc) return rc;
    uint8_t* out = static_cast<uint8_t*>(records);
    for (int32_t t = 0; t < n; ++t) {
        uint8_t* rec = out + static_cast<size_t>(t) * SWIFTKV_RECORD_BYTES;
        std::memset(rec, 0, SWIFTKV_RECORD_BYTES);
        for (int g = 0; g < kGroupsPerHead; ++g) {
            uint8_t sk = 0, sv = 0;
            if (!scale_to_shift(ks[static_cast<size_t>(t) * 4 + g], &sk) ||
                !scale_to_shift(vs[static_cast<size_t>(t) * 4 + g], &sv))
                return fail(SWIFTKV_ESTATE, "token %d group %d holds a scale that is not 2^(s-17), s in [0, 31]",
                            tok0 + t, g);
            put_bits(rec, 5 * g, 5, sk);
            put_bits(rec, 20 + 5 * g, 5, sv);
        }
        std::memcpy(rec + 64, kc.data() + static_cast<size_t>(t) * kCodeBytes, kCodeBytes);
        std::memcpy(rec + 192, vc.data() + static_cast<size_t>(t) * kCodeBytes, kCodeBytes);
    }
    return ok();
}

int swiftkv_kv_cache_import_records(swiftkv_context* ctx, swiftkv_kv_cache* kv, int32_t seq, int32_t layer,
                                    int32_t head, int32_t tok0, int32_t n, const void* records) {
    int rc = check_cache_range(ctx, kv, seq, layer, head, tok0, n);
    if (rc) return rc;
    if (!records && n > 0) return fail(SWIFTKV_EINVAL, "null records");
    if ((rc = not_capturing(ctx, "swiftkv_kv_cache_import_records"))) return rc;
    if ((rc = set_device(ctx))) return rc;
    if (n == 0) return ok();
    const uint8_t* in = static_cast<const uint8_t*>(records);
    std::vector<int8_t> kc(static_cast<size_t>(n) * kCodeBytes), vc(kc.size());
    std::vector<float> sc(static_cast<size_t>(n) * 8);
    for (int32_t t = 0; t < n; ++t) {
        const uint8_t* rec = in + static_cast<size_t>(t) * SWIFTKV_RECORD_BYTES;
        for (int g = 0; g < kGroupsPerHead; ++g) {
            sc[static_cast<size_t>(t) * 8 + 2 * g] = shift_to_scale(get_bits(rec, 5 * g, 5));
            sc[static_cast<size_t>(t) * 8 + 2 * g + 1] = shift_to_scale(get_bits(rec, 20 + 5 * g, 5));
        }
        std::memcpy(kc.data() + static_cast<size_t>(t) * kCodeBytes, rec + 64, kCodeBytes);
        std::memcpy(vc.data() + static_cast<size_t>(t) * kCodeBytes, rec + 192, kCodeBytes);
    }
    int8_t* page = page_ptr(CacheView{kv->base, kv->page_bytes, kv->seq_cap, kv->layers}, seq, layer, head);
    const size_t cap = static_cast<size_t>(kv->seq_cap);
    SKV_HIP(hipStreamSynchronize(ctx->stream));
    SKV_HIP(hipMemcpy(page + static_cast<size_t>(tok0) * kCodeBytes, kc.data(), kc.size(), hipMemcpyHostToDevice));
    SKV_HIP(hipMemcpy(page + (cap + tok0) * kCodeBytes, vc.data(), vc.size(), hipMemcpyHostToDevice));
    SKV_HIP(hipMemcpy(page + cap * 2 * kCodeBytes + static_cast<size_t>(tok0) * kScaleBytes, sc.data(),
                      sc.size() * sizeof(float), hipMemcpyHostToDevice));
    return ok();
}

// ---------------------------------------------------------------- the step

int swiftkv_attention_f32(swiftkv_context* ctx, const float* q, const float* k, const float* v,
                          swiftkv_kv_cache* kv_cache, const swiftkv_rope_lut* rope_lut, uint8_t* activation_q,
                          uint8_t* activation_scale, int32_t layer_index, const int32_t* positions,
                          int32_t batch, float* out) {
    return dispatch_step(ctx, false, q, k, v, kF32Input, kv_cache, rope_lut, activation_q, activation_scale,
                         layer_index, positions, batch, out);
}

int swiftkv_attention_q17(swiftkv_context* ctx, const int32_t* q, const int32_t* k, const int32_t* v,
                          swiftkv_kv_cache* kv_cache, const swiftkv_rope_lut* rope_lut, uint8_t* activation_q,
                          uint8_t* activation_scale, int32_t layer_index, const int32_t* positions,
                          int32_t batch, float* out) {
    return dispatch_step(ctx, false, q, k, v, kQ17Input, kv_cache, rope_lut, activation_q, activation_scale,
                         layer_index, positions, batch, out);
}

int swiftkv_attention_f32_noalloc(swiftkv_context* ctx, const float* q, const float* k, const float* v,
                                  swiftkv_kv_cache* kv_cache, const swiftkv_rope_lut* rope_lut,
                                  uint8_t* activation_q, uint8_t* activation_scale, int32_t layer_index,
                                  const int32_t* positions, int32_t batch, float* out) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (int rc = take_fault(ctx)) return rc;
    if (ctx->host_io)
        return fail(SWIFTKV_ESTATE, "host-memory I/O mode stages through an allocated buffer: switch it off for "
                    "the allocation-free entry");
    return run_step(ctx, q, k, v, kF32Input, kv_cache, rope_lut, activation_q, activation_scale, layer_index,
                    positions, batch, out, true);
}

int swiftkv_attention_partials(swiftkv_context* ctx, const float* q, const float* k, const float* v,
                               int32_t parts, int64_t part_stride, swiftkv_kv_cache* kv_cache,
                               const swiftkv_rope_lut* rope_lut, uint8_t* activation_q, uint8_t* activation_scale,
                               int32_t layer_index, const int32_t* positions, int32_t batch, float* out) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (parts != 1 && parts != 2 && parts != 4) return fail(SWIFTKV_EINVAL, "parts = %d: must be 1, 2 or 4", parts);
    const int64_t rows_elems = static_cast<int64_t>(batch) * kModelDim;
    if (parts > 1 && part_stride > kMaxPartStride)
        return fail(SWIFTKV_EINVAL, "part_stride %lld exceeds %lld elements", static_cast<long long>(part_stride),
                    static_cast<long long>(kMaxPartStride));
    if (parts > 1 && part_stride < rows_elems)
        return fail(SWIFTKV_EINVAL, "part_stride %lld is below batch * 4096 = %lld: partials would overlap",
                    static_cast<long long>(part_stride), static_cast<long long>(rows_elems));
    const StepInput in{parts == 1 ? kInF32 : static_cast<InputFormat>(parts), parts == 1 ? 0 : part_stride};
    return dispatch_step(ctx, false, q, k, v, in, kv_cache, rope_lut, activation_q, activation_scale, layer_index,
                         positions, batch, out);
}

int swiftkv_attention_exact(swiftkv_context* ctx, const void* q, const void* k, const void* v, int32_t q17,
                            swiftkv_kv_cache* kv_cache, const swiftkv_rope_lut* rope_lut, uint8_t* activation_q,
                            uint8_t* activation_scale, int32_t layer_index, const int32_t* positions,
                            int32_t batch, int32_t* out_q17) {
    return dispatch_step(ctx, true, q, k, v, q17 ? kQ17Input : kF32Input, kv_cache, rope_lut, activation_q,
                         activation_scale, layer_index, positions, batch, out_q17);
}

int swiftkv_append_tokens(swiftkv_context* ctx, const void* k, const void* v, int32_t q17,
                          swiftkv_kv_cache* kv_cache, const swiftkv_rope_lut* rope_lut, int32_t layer_index,
                          int32_t seq, int32_t pos0, int32_t n) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (!k || !v) return fail(SWIFTKV_EINVAL, "null k/v pointer");
    if (!ctx->host_io && ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u))
        return fail(SWIFTKV_EINVAL, "k and v must be 16-byte aligned (the kernel reads four channels per lane)");
    if (!rope_lut || rope_lut->ctx != ctx) return fail(SWIFTKV_EINVAL, "rope_lut is null or belongs to another context");
    int rc = check_cache_range(ctx, kv_cache, seq, layer_index, 0, pos0, n);
    if (rc) return rc;
    if (static_cast<int64_t>(pos0) + n > rope_lut->positions)
        return fail(SWIFTKV_ERANGE, "positions [%d, %d) exceed the RoPE table (%d)", pos0, pos0 + n,
                    rope_lut->positions);
    if (n == 0) return ok();
    if ((rc = set_device(ctx))) return rc;
    const size_t rows_bytes = static_cast<size_t>(n) * kModelDim * 4;
    if (ctx->host_io) {   // stage the host rows (see dispatch_step)
        const size_t half = (rows_bytes + 255) & ~static_cast<size_t>(255);
        if ((rc = ensure(ctx, ctx->io_stage, ctx->io_bytes, 2 * half))) return rc;
        SKV_HIP(hipMemcpyAsync(ctx->io_stage, k, rows_bytes, hipMemcpyHostToDevice, ctx->stream));
        SKV_HIP(hipMemcpyAsync(ctx->io_stage + half, v, rows_bytes, hipMemcpyHostToDevice, ctx->stream));
        k = ctx->io_stage;
        v = ctx->io_stage + half;
    }
    BulkArgs a;
    a.k = k;
    a.v = v;
    a.kv = CacheView{kv_cache->base, kv_cache->page_bytes, kv_cache->seq_cap, kv_cache->layers};
    a.lut = rope_lut->table;
    a.lut_positions = rope_lut->positions;
    a.layer = layer_index;
    a.slot = seq;
    a.pos0 = pos0;
    a.n = n;
    ProfilePair* p = profile_begin(ctx, SWIFTKV_KERNEL_APPEND);
    SKV_HIP(launch_append_bulk(a, q17 != 0, ctx->stream));
    profile_end(ctx, p);
    if (ctx->host_io) SKV_HIP(hipStreamSynchronize(ctx->stream));   // the stage is reused by the next call
    return ok();
}

// ---------------------------------------------------------------- synthetic data

int swiftkv_fill_synthetic_f32(swiftkv_context* ctx, float* out, size_t n, uint64_t first, uint64_t seed,
                               uint64_t stream, int32_t distribution, int32_t outliers) {
    if (!ctx || (n && !out)) return fail(SWIFTKV_EINVAL, "null argument");
    if (first & 1u) return fail(SWIFTKV_EINVAL, "first element %llu must be even", (unsigned long long)first);
    if (distribution != SWIFTKV_DIST_NORMAL && distribution != SWIFTKV_DIST_STUDENT_T3)
        return fail(SWIFTKV_EINVAL, "unknown distribution %d", distribution);
    int rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(launch_fill_f32(out, n, first, seed, stream, distribution, outliers != 0, ctx->stream));
    return ok();
}

int swiftkv_kv_cache_fill_synthetic(swiftkv_context* ctx, swiftkv_kv_cache* kv, const swiftkv_rope_lut* rope_lut,
                                    int32_t layer0, int32_t nlayers, int32_t seq0, int32_t nseq, int32_t ntok,
                                    uint64_t seed, int32_t distribution, int32_t k_outliers) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (!kv || kv->ctx != ctx) return fail(SWIFTKV_EINVAL, "kv_cache is null or belongs to another context");
    if (!rope_lut || rope_lut->ctx != ctx) return fail(SWIFTKV_EINVAL, "rope_lut is null or belongs to another context");
    if (distribution != SWIFTKV_DIST_NORMAL && distribution != SWIFTKV_DIST_STUDENT_T3)
        return fail(SWIFTKV_EINVAL, "unknown distribution %d", distribution);
    if (layer0 < 0 || nlayers < 1 || static_cast<int64_t>(layer0) + nlayers > kv->layers)
        return fail(SWIFTKV_ERANGE, "layers [%d, %d) outside [0, %d)", layer0, layer0 + nlayers, kv->layers);
    if (seq0 < 0 || nseq < 1 || static_cast<int64_t>(seq0) + nseq > kv->max_batch)
        return fail(SWIFTKV_ERANGE, "sequences [%d, %d) outside [0, %d)", seq0, seq0 + nseq, kv->max_batch);
    if (ntok < 0 || ntok > kv->seq_cap || ntok > rope_lut->positions)
        return fail(SWIFTKV_ERANGE, "ntok %d exceeds the cache (%d) or the RoPE table (%d)", ntok, kv->seq_cap,
                    rope_lut->positions);
    if (ntok == 0) return ok();
    int rc = set_device(ctx);
    if (rc) return rc;
    const CacheView view{kv->base, kv->page_bytes, kv->seq_cap, kv->layers};
    // grid.z = sequences x layers per launch, kept below the 65535 limit
    const int32_t per_launch = std::max<int32_t>(1, 65535 / nlayers);
    for (int32_t s0 = 0; s0 < nseq; s0 += per_launch) {
        const int32_t ns = std::min(per_launch, nseq - s0);
        SKV_HIP(launch_fill_cache(view, rope_lut->table, seed, layer0, nlayers, seq0 + s0, ns, ntok, distribution,
                                  k_outliers != 0, ctx->stream));
    }
    return ok();
}

// ---------------------------------------------------------------- memory

int swiftkv_device_alloc(swiftkv_context* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return fail(SWIFTKV_EINVAL, "null argument");
    *out = nullptr;
    int rc = not_capturing(ctx, "swiftkv_device_alloc");
    if (rc) return rc;
    rc = set_device(ctx);
    if (rc) return rc;
    if (hipMalloc(out, bytes ? bytes : 1) != hipSuccess) return fail(SWIFTKV_ENOMEM, "hipMalloc of %zu bytes failed", bytes);
    ctx->buffers.insert(*out);
    ++ctx->children;
    return ok();
}

// Also accepted after swiftkv_context_destroy, like the other destroy calls.
int swiftkv_device_free(swiftkv_context* ctx, void* ptr) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (!ptr) return ok();
    int rc = not_capturing(ctx, "swiftkv_device_free");
    if (rc) return rc;
    if (ctx->buffers.erase(ptr) == 0)
        return fail(SWIFTKV_EINVAL, "%p was not allocated by swiftkv_device_alloc on this context, or was freed", ptr);
    SKV_HIP(hipSetDevice(ctx->device));
    const hipError_t sync = hipStreamSynchronize(ctx->stream);
    const hipError_t fr = hipFree(ptr);
    release_child(ctx);
    if (sync != hipSuccess || fr != hipSuccess)
        return fail(SWIFTKV_EHIP, "hipFree: %s", hipGetErrorString(sync != hipSuccess ? sync : fr));
    return ok();
}

int swiftkv_memcpy_h2d(swiftkv_context* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(SWIFTKV_EINVAL, "null argument");
    int rc = not_capturing(ctx, "swiftkv_memcpy_h2d");
    if (rc) return rc;
    rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(hipStreamSynchronize(ctx->stream));
    if (bytes) SKV_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return ok();
}

int swiftkv_memcpy_d2h(swiftkv_context* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(SWIFTKV_EINVAL, "null argument");
    int rc = not_capturing(ctx, "swiftkv_memcpy_d2h");
    if (rc) return rc;
    rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(hipStreamSynchronize(ctx->stream));
    if (bytes) SKV_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return ok();
}

int swiftkv_memset_d(swiftkv_context* ctx, void* dst, int value, size_t bytes) {
    if (!ctx || (bytes && !dst)) return fail(SWIFTKV_EINVAL, "null argument");
    int rc = not_capturing(ctx, "swiftkv_memset_d");
    if (rc) return rc;
    rc = set_device(ctx);
    if (rc) return rc;
    if (bytes) SKV_HIP(hipMemsetAsync(dst, value, bytes, ctx->stream));
    return ok();
}

int swiftkv_convert_f32_q17(swiftkv_context* ctx, const float* in, int32_t* out, size_t n) {
    if (!ctx || (n && (!in || !out))) return fail(SWIFTKV_EINVAL, "null argument");
    int rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(launch_convert(in, 1, 0, out, n, ctx->stream));
    return ok();
}

int swiftkv_convert_partials_q17(swiftkv_context* ctx, const float* in, int32_t parts, int64_t part_stride,
                                 int32_t* out, size_t n) {
    if (!ctx || (n && (!in || !out))) return fail(SWIFTKV_EINVAL, "null argument");
    if (parts != 1 && parts != 2 && parts != 4) return fail(SWIFTKV_EINVAL, "parts = %d: must be 1, 2 or 4", parts);
    if (parts > 1 && part_stride > kMaxPartStride)
        return fail(SWIFTKV_EINVAL, "part_stride %lld exceeds %lld elements", static_cast<long long>(part_stride),
                    static_cast<long long>(kMaxPartStride));
    if (parts > 1 && (part_stride < 0 || static_cast<uint64_t>(part_stride) < n))
        return fail(SWIFTKV_EINVAL, "part_stride %lld is below n = %zu: partials would overlap",
                    static_cast<long long>(part_stride), n);
    int rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(launch_convert(in, parts, parts > 1 ? part_stride : 0, out, n, ctx->stream));
    return ok();
}

// ---------------------------------------------------------------- A14 words (host)

int swiftkv_a14_unpack(const uint8_t* words, size_t groups, int16_t* lanes) {
    if (groups && (!words || !lanes)) return fail(SWIFTKV_EINVAL, "null argument");
    for (size_t g = 0; g < groups; ++g) {
        const uint8_t* w = words + g * SWIFTKV_A14_WORD_BYTES;
        for (int i = 0; i < kGroup; ++i) {
            const int bit = 14 * i;
            // 14 bits starting at `bit` span at most three bytes of the word
            uint32_t raw = 0;
            for (int b = 0; b < 3 && (bit >> 3) + b < SWIFTKV_A14_WORD_BYTES; ++b)
                raw |= static_cast<uint32_t>(w[(bit >> 3) + b]) << (8 * b);
            const uint32_t v = (raw >> (bit & 7)) & 0x3fffu;
            lanes[g * kGroup + i] = static_cast<int16_t>((v & 0x2000u) ? static_cast<int32_t>(v) - 0x4000 : v);
        }
    }
    return ok();
}

int swiftkv_a14_decode(const uint8_t* words, const uint8_t* e8m0, size_t groups, float* values) {
    if (groups && (!words || !e8m0 || !values)) return fail(SWIFTKV_EINVAL, "null argument");
    int16_t lanes[kGroup];
    for (size_t g = 0; g < groups; ++g) {
        (void)swiftkv_a14_unpack(words + g * SWIFTKV_A14_WORD_BYTES, 1, lanes);
        const int e = static_cast<int>(e8m0[g]) - 127 - 13;
        for (int i = 0; i < kGroup; ++i) values[g * kGroup + i] = std::ldexp(static_cast<float>(lanes[i]), e);
    }
    return ok();
}

// ---------------------------------------------------------------- graphs

int swiftkv_capture_begin(swiftkv_context* ctx) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (ctx->capturing) return fail(SWIFTKV_ESTATE, "a capture is already in progress");
    if (ctx->host_io) return fail(SWIFTKV_ESTATE, "host-memory I/O mode cannot be captured: switch it off first");
    int rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    ctx->capture_uses_workspace = false;
    return ok();
}

int swiftkv_capture_end(swiftkv_context* ctx, swiftkv_graph** out) {
    if (!ctx || !out) return fail(SWIFTKV_EINVAL, "null argument");
    *out = nullptr;
    if (!ctx->capturing) return fail(SWIFTKV_ESTATE, "no capture in progress");
    ctx->capturing = false;
    int rc = set_device(ctx);
    if (rc) return rc;
    hipGraph_t graph = nullptr;
    SKV_HIP(hipStreamEndCapture(ctx->stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return fail(SWIFTKV_EHIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    swiftkv_graph* g = new (std::nothrow) swiftkv_graph();
    if (!g) {
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(graph);
        return fail(SWIFTKV_ENOMEM, "out of host memory");
    }
    g->ctx = ctx;
    g->graph = graph;
    g->exec = exec;
    // A capture cannot grow the workspace, so every split launch it recorded
    // used the current buffer.
    if (ctx->capture_uses_workspace) {
        g->workspace = ctx->partials;
        ++ctx->graph_refs[g->workspace];
    }
    ++ctx->children;
    *out = g;
    return ok();
}

int swiftkv_graph_launch(swiftkv_context* ctx, const swiftkv_graph* graph) {
    if (!ctx || !graph) return fail(SWIFTKV_EINVAL, "null argument");
    if (graph->ctx != ctx) return fail(SWIFTKV_EINVAL, "graph belongs to another context");
    int rc = not_capturing(ctx, "swiftkv_graph_launch");
    if (rc) return rc;
    if ((rc = take_fault(ctx))) return rc;
    if ((rc = set_device(ctx))) return rc;
    SKV_HIP(hipGraphLaunch(graph->exec, ctx->stream));
    return ok();
}

int swiftkv_graph_destroy(swiftkv_graph* graph) {
    if (!graph) return ok();
    swiftkv_context* ctx = graph->ctx;
    if (int rc = not_capturing(ctx, "swiftkv_graph_destroy")) return rc;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    const int rc = graph->workspace ? release_graph_workspace(ctx, graph->workspace) : SWIFTKV_OK;
    delete graph;
    release_child(ctx);
    return rc ? rc : ok();
}

// ---------------------------------------------------------------- timing

int swiftkv_timer_record(swiftkv_context* ctx, int32_t slot) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    if (slot < 0 || slot >= kTimerSlots) return fail(SWIFTKV_ERANGE, "timer slot %d outside [0, %d)", slot, kTimerSlots);
    int rc = not_capturing(ctx, "swiftkv_timer_record");
    if (rc) return rc;
    rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(hipEventRecord(ctx->timers[slot], ctx->stream));
    return ok();
}

int swiftkv_timer_elapsed(swiftkv_context* ctx, int32_t slot_begin, int32_t slot_end, float* ms) {
    if (!ctx || !ms) return fail(SWIFTKV_EINVAL, "null argument");
    if (slot_begin < 0 || slot_begin >= kTimerSlots || slot_end < 0 || slot_end >= kTimerSlots)
        return fail(SWIFTKV_ERANGE, "timer slot outside [0, %d)", kTimerSlots);
    int rc = not_capturing(ctx, "swiftkv_timer_elapsed");
    if (rc) return rc;
    rc = set_device(ctx);
    if (rc) return rc;
    SKV_HIP(hipEventSynchronize(ctx->timers[slot_end]));
    SKV_HIP(hipEventElapsedTime(ms, ctx->timers[slot_begin], ctx->timers[slot_end]));
    return ok();
}

int swiftkv_profile_enable(swiftkv_context* ctx, int32_t on) {
    if (!ctx) return fail(SWIFTKV_EINVAL, "null context");
    int rc = set_device(ctx);
    if (rc) return rc;
    if (on && ctx->profile_pool.empty()) {
        ctx->profile_pool.resize(kProfilePairs);
        for (auto& p : ctx->profile_pool) {
            SKV_HIP(hipEventCreate(&p.begin));
            SKV_HIP(hipEventCreate(&p.end));
        }
    }
    ctx->profiling = on != 0;
    ctx->profile_used = 0;
    return ok();
}

int swiftkv_profile_collect(swiftkv_context* ctx, int64_t counts[SWIFTKV_KERNEL_KINDS],
                            double ms[SWIFTKV_KERNEL_KINDS]) {
    if (!ctx || !counts || !ms) return fail(SWIFTKV_EINVAL, "null argument");
    int rc = not_capturing(ctx, "swiftkv_profile_collect");
    if (rc) return rc;
    rc = set_device(ctx);
    if (rc) return rc;
    for (int i = 0; i < SWIFTKV_KERNEL_KINDS; ++i) {
        counts[i] = 0;
        ms[i] = 0.0;
    }
    SKV_HIP(hipStreamSynchronize(ctx->stream));
    for (size_t i = 0; i < ctx->profile_used; ++i) {
        const ProfilePair& p = ctx->profile_pool[i];
        float t = 0.0f;
        SKV_HIP(hipEventElapsedTime(&t, p.begin, p.end));
        counts[p.kind] += 1;
        ms[p.kind] += t;
    }
    ctx->profile_used = 0;
    return ok();
}

}  // extern "C"
