/*
 * swiftkv.h -- C ABI of the MI355X SwiftKV decode-attention stage.
 *
 * Drop-in for the reference's local-PE attention entry
 *   void int4_swiftkv_attention_pe{0..3}(q, k, v, kv_cache, rope_lut_ddr,
 *        activation_q, activation_scale, layer_index, position)
 * (kernel_HLS/swiftkv_attention.hpp:167-209, swiftkv_attention.cpp:2821-2883).
 * One call performs, for every (sequence, head) of a batch:
 *   1. FP32 -> Q15.17 conversion of q/k/v, exactly as the upstream linear
 *      finalize does (int4_linear_controller.cpp:38-83) -- skipped by the
 *      _q17 entry, which takes Q15.17 words as the reference does;
 *   2. adjacent-pair integer RoPE of q and k from the position-indexed Q1.17
 *      table (swiftkv_attention.cpp:20-95);
 *   3. INT8/G32 quantization of the new K/V row and its append to the cache
 *      at `position` (swiftkv_attention.cpp:348-582, 752-786) -- bit-exact;
 *   4. attention of the rotated query over cached tokens [0, position]
 *      (swiftkv_attention.cpp:934-1880), evaluated with the reference's FP32
 *      softmax formula (llama2_decoder_sw_emulator.cpp:1164-1194) over the
 *      dequantized INT8 cache;
 *   5. optionally the A14/G32 + E8M0 output quantization for the O projection
 *      (swiftkv_attention.cpp:1715-1771, 2656-2682).
 *
 * All 32 heads of a layer run on one GPU (the reference shards 8 heads per
 * FPGA PE).  Conventions:
 *   - every function returns 0 (SWIFTKV_OK) or a negative SWIFTKV_E* code;
 *     no C++ exception crosses the boundary; swiftkv_last_error() describes
 *     the most recent failure of the calling thread;
 *   - tensors passed to the step functions are DEVICE pointers (allocate with
 *     swiftkv_device_alloc or any HIP allocator), or host pointers in a
 *     context switched to host-memory I/O (swiftkv_set_host_io);
 *     position/length arrays are HOST pointers;
 *   - work is issued asynchronously on the context's HIP stream; call
 *     swiftkv_synchronize() before reading results on the host;
 *   - a failure found on the device is reported by the next call that looks
 *     for it: a split merge that gave up waiting for another split's partial
 *     (its head's output then holds NaN) makes swiftkv_synchronize, or the
 *     next step entry or graph launch (which then enqueue nothing), return
 *     SWIFTKV_EHIP with a message naming the cache slot and head, once (the
 *     reference host turns a stalled run into an error the same way,
 *     decode_host.cpp:1433-1467);
 *   - calls on one context are not thread-safe; distinct contexts are.
 */
#ifndef SWIFTKV_H
#define SWIFTKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Geometry fixed by the reference (swiftkv_attention.hpp:5-13, config.json). */
#define SWIFTKV_HEADS 32
#define SWIFTKV_HEAD_DIM 128
#define SWIFTKV_MODEL_DIM (SWIFTKV_HEADS * SWIFTKV_HEAD_DIM)
#define SWIFTKV_GROUP 32
#define SWIFTKV_GROUPS_PER_HEAD (SWIFTKV_HEAD_DIM / SWIFTKV_GROUP)
/* Reference limits: position is ap_uint<12>, SWIFTKV_MAX_SEQ_LEN = 4096
 * (hpp:26-30).  The FP32 step entries accept longer caches (up to 32768
 * tokens) with the RoPE table extended by the same closed form; the
 * integer-compatibility entry keeps the reference's bound. */
#define SWIFTKV_REFERENCE_MAX_SEQ 4096
#define SWIFTKV_MAX_SEQ 32768
/* Byte sizes of the reference formats. */
#define SWIFTKV_ROPE_LUT_BYTES_PER_POSITION 512 /* 4 LUT words x 2 x 64 B */
#define SWIFTKV_RECORD_BYTES 320                /* [meta, K0, K1, V0, V1] x 64 B */
#define SWIFTKV_A14_WORD_BYTES 56               /* ap_uint<448>: 32 x int14 */

/* Status codes. */
#define SWIFTKV_OK 0
#define SWIFTKV_EINVAL (-1)  /* null pointer, bad size or geometry */
#define SWIFTKV_ERANGE (-2)  /* position / layer / sequence out of range */
#define SWIFTKV_EHIP (-3)    /* HIP runtime error (no device, launch failure) */
#define SWIFTKV_ENOMEM (-4)  /* device or host allocation failed */
#define SWIFTKV_ESTATE (-5)  /* object not ready (e.g. RoPE table not loaded) */

typedef struct swiftkv_context swiftkv_context;
typedef struct swiftkv_kv_cache swiftkv_kv_cache;
typedef struct swiftkv_rope_lut swiftkv_rope_lut;
typedef struct swiftkv_graph swiftkv_graph;

/* Thread-local description of the last failure ("" after success). */
const char* swiftkv_last_error(void);
/* Library version string. */
const char* swiftkv_version(void);

/* --------------------------------------------------------------------------
 * Context: device, HIP stream, split-context workspace.
 * Replaces the per-PE compute-unit handle the XRT host launches
 * (host/decode_host.cpp:1256-1294, 1378-1404).
 * ------------------------------------------------------------------------ */
int swiftkv_context_create(int device, swiftkv_context** out);
/* Objects created from a context (KV caches, RoPE tables, graphs, device
 * buffers) may be destroyed before or after it, in any order: the context
 * then refuses new work (SWIFTKV_ESTATE) but stays valid for those destroy
 * calls, and its resources are released with the last of them. */
int swiftkv_context_destroy(swiftkv_context* ctx);
/* Waits for the context's work; SWIFTKV_EHIP if a split merge of that work
 * gave up (see above). */
int swiftkv_synchronize(swiftkv_context* ctx);
/* Tokens per split-context work item; 0 selects the built-in heuristic.
 * Must be 0 or a multiple of 256 in [256, 32768]. */
int swiftkv_set_split_tokens(swiftkv_context* ctx, int32_t split_tokens);
/* Testing aid with no counterpart in the reference: every later step launch
 * of the context runs the step kernel of `waves` waves per workgroup on
 * `block_tokens`-token blocks instead of the shape the launch plan picks;
 * waves = 0 returns to the plan's choice.  The compiled shapes (waves,
 * block_tokens) are (4, 64), (8, 32) and (8, 64); any other is refused
 * (SWIFTKV_EINVAL).  All compute the same function: tests force each one on
 * every kind of launch. */
int swiftkv_debug_set_step_shape(swiftkv_context* ctx, int32_t waves, int32_t block_tokens);
/* Testing aid with no counterpart in the reference, host-only (no device or
 * context needed): the launch plan the step entries use for one launch of
 * batch <= 256 sequences at positions[batch], on a device of `cus` compute
 * units each holding `workgroups_per_cu` 4-wave step workgroups (a context
 * takes both from the device), with split_tokens as swiftkv_set_split_tokens
 * sets it (0: the built-in heuristic).  Writes the tokens per split, the
 * splits of the longest sequence (the grid's split dimension), the shape --
 * waves per workgroup and tokens per block: 8 on 32 up to cus x
 * workgroups_per_cu workgroups; beyond that 8 on 64 when every workgroup's
 * range holds at least 2048 tokens, else 4 on 64 -- (out_block_tokens may be
 * null) and, when out_rows is not null, the sequence served by each grid row
 * (longest first, equal positions in sequence order). */
int swiftkv_debug_step_plan(int32_t cus, int32_t workgroups_per_cu, int32_t split_tokens, const int32_t* positions,
                            int32_t batch, int32_t* out_split_tokens, int32_t* out_grid_splits, int32_t* out_waves,
                            int32_t* out_block_tokens, int32_t* out_rows);
/* Testing aid with no counterpart in the reference.  A head split across
 * workgroups is merged inside the launch through 64-bit words tagged with the
 * (sequence row, head)'s generation + 1, which every launch that merges the
 * head advances; tags run over 1 .. 0xffffffff and wrap to 1, clearing the
 * head's words first.  This sets every generation of the context's split
 * workspace (noalloc = 0) or of this device's allocation-free workspace
 * (noalloc != 0) to `generation` and zeroes its partial words, on the context
 * stream, so a test can run launches across the wrap without 2^32 of them.
 * A context with no split workspace yet is left as it is (its first one
 * starts at generation 0).  Buffers the context keeps only for graphs that
 * recorded them (see the graph section) are not reached.  `generation`
 * 0xffffffff is refused (SWIFTKV_EINVAL), and so is a call during graph
 * capture (SWIFTKV_ESTATE). */
int swiftkv_debug_set_split_generation(swiftkv_context* ctx, uint32_t generation, int32_t noalloc);
/* Testing aid with no counterpart in the reference.  While enabled, every split
 * merge of the context's step launches waits for a tag that no partial carries,
 * so it gives up after one poll: the merged heads' outputs hold NaN and the
 * failure is reported as above.  Every kernel still exits normally and the
 * split workspace stays consistent, so steps after it is disabled are exact
 * again.  Host-only; affects launches enqueued while it is on. */
int swiftkv_debug_force_merge_timeout(swiftkv_context* ctx, int32_t enable);

/* --------------------------------------------------------------------------
 * RoPE table (kernel_HLS/swiftkv_attention.hpp:55-81; rope_lut.bin format of
 * scripts/generate_rope_lut.py:20-41, 104-150): per position, 64 (cos, sin)
 * pairs as signed 19-bit Q1.17, packed 16 pairs per 608-bit LUT word, each
 * LUT word padded into two 64-byte DDR words (512 bytes per position).
 * ------------------------------------------------------------------------ */
/* Load `positions` positions from the reference file image (host bytes,
 * positions * 512 bytes, e.g. the 2 MiB rope_lut.bin). */
int swiftkv_rope_lut_load(swiftkv_context* ctx, const void* image, size_t image_bytes,
                          swiftkv_rope_lut** out);
/* Closed form RNE(2^17 cos|sin(pos * theta^(-j/64))) for pos < positions
 * (reproduces rope_lut.bin bit for bit at theta = 10000, 4096 positions). */
int swiftkv_rope_lut_generate(swiftkv_context* ctx, int32_t positions, double theta,
                              swiftkv_rope_lut** out);
int swiftkv_rope_lut_destroy(swiftkv_rope_lut* lut);
int32_t swiftkv_rope_lut_positions(const swiftkv_rope_lut* lut);
/* Write positions [pos0, pos0+n) back in the reference file format (host). */
int swiftkv_rope_lut_export(const swiftkv_rope_lut* lut, int32_t pos0, int32_t n, void* image);

/* --------------------------------------------------------------------------
 * KV cache: GPU-resident INT8 codes with per-(token, head) G32 FP32 scales
 * 2^(shift-17).  Replaces the reference's per-PE DDR region
 * [layer][local_head][token][meta,K0,K1,V0,V1] (hpp:98-110; sized and zeroed
 * by host/decode_host.cpp:98-119, 1256-1259, 1291-1294).
 * Layout (one page per sequence x layer x head, capacity S tokens):
 *   K codes  [S][128] int8   | V codes [S][128] int8 |
 *   scales   [S][8] float  = (K_g0, V_g0, K_g1, V_g1, K_g2, V_g2, K_g3, V_g3)
 * The cache is zero-filled on creation.
 * ------------------------------------------------------------------------ */
int swiftkv_kv_cache_create(swiftkv_context* ctx, int32_t layers, int32_t max_batch,
                            int32_t max_seq_len, swiftkv_kv_cache** out);
int swiftkv_kv_cache_destroy(swiftkv_kv_cache* kv);
int swiftkv_kv_cache_zero(swiftkv_context* ctx, swiftkv_kv_cache* kv);
/* Bytes held on the device (codes + scales). */
size_t swiftkv_kv_cache_bytes(const swiftkv_kv_cache* kv);
/* Copy tokens [tok0, tok0+n) of (seq, layer, head) to host buffers:
 * k_codes/v_codes [n][128] int8, k_scales/v_scales [n][4] float (any may be
 * NULL).  Synchronizes the context stream. */
int swiftkv_kv_cache_read(swiftkv_context* ctx, const swiftkv_kv_cache* kv, int32_t seq,
                          int32_t layer, int32_t head, int32_t tok0, int32_t n,
                          int8_t* k_codes, int8_t* v_codes, float* k_scales, float* v_scales);
/* Reference record format [meta, K0, K1, V0, V1] (320 bytes per token-head,
 * hpp:94-110, swiftkv_attention.cpp:534-581): export to / import from host
 * memory, records [n][320] for tokens [tok0, tok0+n) of (seq, layer, head). */
int swiftkv_kv_cache_export_records(swiftkv_context* ctx, const swiftkv_kv_cache* kv,
                                    int32_t seq, int32_t layer, int32_t head, int32_t tok0,
                                    int32_t n, void* records);
int swiftkv_kv_cache_import_records(swiftkv_context* ctx, swiftkv_kv_cache* kv, int32_t seq,
                                    int32_t layer, int32_t head, int32_t tok0, int32_t n,
                                    const void* records);

/* --------------------------------------------------------------------------
 * The decode-attention step (the drop-in for int4_swiftkv_attention_peN).
 *   q, k, v        device [batch][4096]: FP32 (…_f32) or Q15.17 int32 (…_q17)
 *   kv_cache       persistent cache; sequence b of the batch uses cache slot b
 *   rope_lut       table covering every position used
 *   activation_q   optional device [batch][128][56] bytes: A14 words, group
 *                  index = head*4 + g, lane 0 in bits [13:0] (may be NULL)
 *   activation_scale optional device [batch][128] E8M0 codes (may be NULL;
 *                  must be NULL iff activation_q is NULL)
 *   layer_index    0 <= layer < kv_cache layers
 *   positions      host [batch]: cached-token count of each sequence; the
 *                  step writes token `positions[b]` and attends [0, positions[b]]
 *   out            device [batch][4096] FP32 attention output (required)
 * ------------------------------------------------------------------------ */
int swiftkv_attention_f32(swiftkv_context* ctx, const float* q, const float* k, const float* v,
                          swiftkv_kv_cache* kv_cache, const swiftkv_rope_lut* rope_lut,
                          uint8_t* activation_q, uint8_t* activation_scale, int32_t layer_index,
                          const int32_t* positions, int32_t batch, float* out);
int swiftkv_attention_q17(swiftkv_context* ctx, const int32_t* q, const int32_t* k,
                          const int32_t* v, swiftkv_kv_cache* kv_cache,
                          const swiftkv_rope_lut* rope_lut, uint8_t* activation_q,
                          uint8_t* activation_scale, int32_t layer_index,
                          const int32_t* positions, int32_t batch, float* out);

/* Allocation-free variant of swiftkv_attention_f32.  It has no counterpart in
 * the reference; it is for callers that cannot allocate device memory: code
 * recorded into a HIP graph, tight serving loops, harnesses that forbid it.
 * Same arguments, kernels and results as swiftkv_attention_f32, but the split
 * workspace (per-head arrival words and the split partials) is a fixed
 * file-scope device array that every GPU the library runs on holds until the
 * process ends (SWIFTKV_NOALLOC_WORKSPACE_BYTES, 8.25 MiB: 128 KiB of
 * arrival words and 8.1 MiB of partials, for up to 8 splits per head of 32
 * sequences per launch), bound once per device when the first context on it
 * is created.  The call allocates nothing, host or device.
 *   - A call that would split a head more than 8 ways (only a forced split,
 *     swiftkv_set_split_tokens, does) returns SWIFTKV_ERANGE before any work
 *     is enqueued; the built-in heuristic never does.
 *   - A launch whose plan splits the heads of more than 32 sequences (only a
 *     forced split does; the heuristic splits heads only for fewer) runs as
 *     launches of 32 sequences with that plan, so the outputs are still
 *     those of swiftkv_attention_f32, bit for bit.
 *   - Every call on one GPU shares that GPU's array: calls that overlap in
 *     time on one GPU (two contexts, or two streams) race and must not be
 *     issued.  Calls in order on one context are safe; the kernels leave the
 *     arrival counts at zero.
 *   - Host-memory I/O mode is refused (SWIFTKV_ESTATE): it stages through an
 *     allocated buffer. */
#define SWIFTKV_NOALLOC_WORKSPACE_BYTES 8650752u
int swiftkv_attention_f32_noalloc(swiftkv_context* ctx, const float* q, const float* k, const float* v,
                                  swiftkv_kv_cache* kv_cache, const swiftkv_rope_lut* rope_lut,
                                  uint8_t* activation_q, uint8_t* activation_scale, int32_t layer_index,
                                  const int32_t* positions, int32_t batch, float* out);

/* The step fed directly by a split-K Q/K/V projection: q, k, v are each
 * `parts` FP32 partial sums, part p of a tensor at  base + p * part_stride
 * (elements, >= batch * 4096), each part [batch][4096].  The step reduces
 * them in the reference's fixed order -- fl(p0 + p1) for two parts,
 * fl(fl(p0 + p1) + fl(p2 + p3)) for four -- and converts the sum to Q15.17,
 * as the Q/K/V linear stage's pair reduction and finalize do before the
 * attention stage sees its inputs (int4_linear_controller.cpp:1039-1054,
 * 1655-1667, 1089-1118; finalize converts for the Q/K/V modes only, :129-132).
 * The reduction happens in the step's own input loads, so no separate
 * reduce/convert pass or intermediate buffer is needed.
 *   parts        1 (same as swiftkv_attention_f32), 2 or 4; other values
 *                SWIFTKV_EINVAL
 *   part_stride  ignored for parts = 1; otherwise batch * 4096 <= part_stride
 *                <= 2^40, else SWIFTKV_EINVAL
 * Other arguments as for swiftkv_attention_f32. */
int swiftkv_attention_partials(swiftkv_context* ctx, const float* q, const float* k, const float* v,
                               int32_t parts, int64_t part_stride, swiftkv_kv_cache* kv_cache,
                               const swiftkv_rope_lut* rope_lut, uint8_t* activation_q,
                               uint8_t* activation_scale, int32_t layer_index,
                               const int32_t* positions, int32_t batch, float* out);

/* Integer-compatibility step: the same append, then the reference's own
 * Q15.17 arithmetic instead of the FP32 formula -- 44-bit wrapped G32 dot
 * products, score * RNE(2^17/sqrt(128)) >> 24, the single-pass (max, Z, Y)
 * recurrence with the 33-entry Q30 exp2 table, the Q13.17 normalizer with
 * its 30-bit wrap, the 18-bit reciprocal and Y * 1/Z
 * (swiftkv_attention.cpp:934-1880; llama2_decoder_sw_emulator.cpp:633-711),
 * and the integer-path A14/E8M0 epilogue (swiftkv_attention.cpp:1694-1771).
 * activation_q / activation_scale equal what int4_swiftkv_attention_peN
 * writes, bit for bit.  The recurrence is sequential in the token index, so
 * this entry is a compatibility and verification path (one to four
 * workgroups per (sequence, head)), not the fast path.
 *   q, k, v   device [batch][4096], FP32 when q17 == 0, Q15.17 int32 otherwise
 *   out_q17   device [batch][4096] int32: the normalized Q15.17 state
 *   positions each below SWIFTKV_REFERENCE_MAX_SEQ (4096), the reference's
 *             own bound (position is ap_uint<12>; its Q13.17 normalizer is
 *             proven not to wrap only below 2^13 tokens,
 *             swiftkv_attention.cpp:112-119): a call with any position at or
 *             past it returns SWIFTKV_ERANGE and enqueues nothing
 * Other arguments as for swiftkv_attention_f32. */
int swiftkv_attention_exact(swiftkv_context* ctx, const void* q, const void* k, const void* v,
                            int32_t q17, swiftkv_kv_cache* kv_cache, const swiftkv_rope_lut* rope_lut,
                            uint8_t* activation_q, uint8_t* activation_scale, int32_t layer_index,
                            const int32_t* positions, int32_t batch, int32_t* out_q17);

/* Host-memory I/O mode (default off).  When on, the q/k/v, out and
 * activation pointers of swiftkv_attention_f32/_q17/_partials/_exact and the k/v of
 * swiftkv_append_tokens are host memory: the call stages them through a
 * context-owned device buffer on the context stream and returns after its
 * outputs are back in host memory (the reference host's DMA-in / run /
 * DMA-out around each PE call, decode_host.cpp:1358-1485).  Pinned host
 * memory copies fastest.  Not allowed during graph capture, and a capture
 * cannot begin while it is on (SWIFTKV_ESTATE). */
int swiftkv_set_host_io(swiftkv_context* ctx, int32_t enable);

/* Bulk append (prompt prefill): apply the append rule -- conversion, RoPE of
 * k at its own position, G32 quantization -- to n tokens [pos0, pos0+n) of
 * one sequence without attending.  k, v: device [n][4096], FP32 when
 * q17 == 0, Q15.17 int32 otherwise, each 16-byte aligned (SWIFTKV_EINVAL
 * otherwise; swiftkv_device_alloc returns such memory).  The reference has
 * no prefill entry; it feeds prompt tokens through the decode step one at a
 * time (host/decode_host.cpp:1340-1556). */
int swiftkv_append_tokens(swiftkv_context* ctx, const void* k, const void* v, int32_t q17,
                          swiftkv_kv_cache* kv_cache, const swiftkv_rope_lut* rope_lut,
                          int32_t layer_index, int32_t seq, int32_t pos0, int32_t n);

/* --------------------------------------------------------------------------
 * Synthetic inputs for benchmarks and capacity tests (no reference
 * counterpart; the reference's testbenches read weight files or fixed
 * generators).  A synthetic stream (seed, stream) is an FP32 tensor whose
 * element i comes from a counter-based generator (splitmix64 + Box-Muller):
 * N(0,1), or unit-variance Student-t(3); with `outliers` set, elements whose
 * channel i % 4096 is one of ~1% seed-selected channels are scaled by 20.
 * ------------------------------------------------------------------------ */
#define SWIFTKV_DIST_NORMAL 0
#define SWIFTKV_DIST_STUDENT_T3 1
/* Elements [first, first+n) of stream (seed, stream) into device memory;
 * `first` must be even. */
int swiftkv_fill_synthetic_f32(swiftkv_context* ctx, float* out, size_t n, uint64_t first, uint64_t seed,
                               uint64_t stream, int32_t distribution, int32_t outliers);
/* Tokens [0, ntok) of sequences [seq0, seq0+nseq) x layers [layer0,
 * layer0+nlayers) through the append rule, K row t of (slot s, layer l) =
 * elements [4096t, 4096t+4096) of stream 2*(64s + l) (with k_outliers),
 * V row of stream 2*(64s + l) + 1. */
int swiftkv_kv_cache_fill_synthetic(swiftkv_context* ctx, swiftkv_kv_cache* kv,
                                    const swiftkv_rope_lut* rope_lut, int32_t layer0, int32_t nlayers,
                                    int32_t seq0, int32_t nseq, int32_t ntok, uint64_t seed,
                                    int32_t distribution, int32_t k_outliers);

/* --------------------------------------------------------------------------
 * Device-memory helpers for FFI callers without a GPU framework (ctypes).
 * swiftkv_device_free takes only pointers from swiftkv_device_alloc on the
 * same context (anything else, or a second free: SWIFTKV_EINVAL); it waits
 * for the context stream before freeing.
 * ------------------------------------------------------------------------ */
int swiftkv_device_alloc(swiftkv_context* ctx, size_t bytes, void** out);
int swiftkv_device_free(swiftkv_context* ctx, void* ptr);
int swiftkv_memcpy_h2d(swiftkv_context* ctx, void* dst, const void* src, size_t bytes);
int swiftkv_memcpy_d2h(swiftkv_context* ctx, void* dst, const void* src, size_t bytes);
int swiftkv_memset_d(swiftkv_context* ctx, void* dst, int value, size_t bytes);

/* Elementwise FP32 -> Q15.17 on the device (the conversion of step 1),
 * n elements, device pointers.  Exposed for exhaustive conversion tests. */
int swiftkv_convert_f32_q17(swiftkv_context* ctx, const float* in, int32_t* out, size_t n);

/* The Q/K/V linear stage's finalize on the device: out[i] = Q15.17 of the
 * `parts` FP32 partials in[i + p * part_stride] reduced in the reference's
 * order (see swiftkv_attention_partials; int4_linear_controller.cpp:1089-1118).
 * parts 1, 2 or 4; n <= part_stride <= 2^40 for parts > 1; device pointers.  Feeds
 * swiftkv_attention_exact (q17 = 1) with the inputs the reference's attention
 * stage receives. */
int swiftkv_convert_partials_q17(swiftkv_context* ctx, const float* in, int32_t parts,
                                 int64_t part_stride, int32_t* out, size_t n);

/* A14 activation words on the host (no device work).  A word is 56 bytes,
 * the reference's ap_uint<448>: 32 signed 14-bit lanes, lane i at bits
 * [14i, 14i+13] (swiftkv_attention.cpp:1761-1768).  _unpack writes the lanes
 * as int16 [groups][32]; _decode writes what the O projection multiplies,
 * lane * 2^(code - 140) as float [groups][32], with code the group's E8M0
 * byte (the consumer takes code - 127 - 13 as the group exponent,
 * int4_linear_controller.cpp:643-645).  Returns SWIFTKV_EINVAL on a null
 * pointer with groups > 0. */
int swiftkv_a14_unpack(const uint8_t* words, size_t groups, int16_t* lanes);
int swiftkv_a14_decode(const uint8_t* words, const uint8_t* e8m0, size_t groups, float* values);

/* --------------------------------------------------------------------------
 * HIP graphs: record a sequence of asynchronous calls (steps, appends,
 * synthetic fills) once and replay it with one launch, e.g. the 32 per-layer
 * calls of a decode step.  The recording keeps every argument, including the
 * positions, so a replay repeats exactly the recorded work.  Run each
 * recorded call once outside capture first: the split workspace must already
 * be large enough.  Eager calls after a capture may still grow the workspace:
 * the buffer a graph recorded stays allocated until the last graph that
 * recorded it is destroyed, so replays remain valid (a buffer no graph
 * recorded is freed when the workspace outgrows it).  While capturing,
 * calls that synchronize, copy, allocate or memset return SWIFTKV_ESTATE.
 * ------------------------------------------------------------------------ */
int swiftkv_capture_begin(swiftkv_context* ctx);
int swiftkv_capture_end(swiftkv_context* ctx, swiftkv_graph** out);
int swiftkv_graph_launch(swiftkv_context* ctx, const swiftkv_graph* graph);
int swiftkv_graph_destroy(swiftkv_graph* graph);

/* --------------------------------------------------------------------------
 * Timing (hipEvents on the context stream).  Stands in for the host's
 * per-stage timers (host/decode_host.cpp:1539-1553).
 * ------------------------------------------------------------------------ */
/* Record timestamp slot `slot` (0..63) on the context stream. */
int swiftkv_timer_record(swiftkv_context* ctx, int32_t slot);
/* Milliseconds between two recorded slots (waits for the later one). */
int swiftkv_timer_elapsed(swiftkv_context* ctx, int32_t slot_begin, int32_t slot_end, float* ms);
/* Per-kernel timing: when enabled, every launch of each kernel is bracketed
 * by events; swiftkv_profile_collect() synchronizes and returns, per kernel
 * kind, the launch count and the summed duration in ms, then clears the
 * record. */
#define SWIFTKV_KERNEL_APPEND 0  /* bulk append (prefill) */
#define SWIFTKV_KERNEL_STEP 1    /* the step kernel: append, split scan, merge, output */
#define SWIFTKV_KERNEL_EXACT 2   /* the integer-compatibility step */
#define SWIFTKV_KERNEL_KINDS 3
int swiftkv_profile_enable(swiftkv_context* ctx, int32_t on);
int swiftkv_profile_collect(swiftkv_context* ctx, int64_t counts[SWIFTKV_KERNEL_KINDS],
                            double ms[SWIFTKV_KERNEL_KINDS]);

#ifdef __cplusplus
}
#endif
#endif /* SWIFTKV_H */
