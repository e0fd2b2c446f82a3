// swiftkv_host.cpp -- native host driver of the SwiftKV decode-attention stage.
//
// The reference drives its attention PEs from a C++ host program
// (host/decode_host.cpp): it allocates and zeroes the KV banks, loads the
// 2 MiB rope_lut.bin image with a size check, and issues one attention call
// per layer and token, timing each stage.  This program does the same for the
// MI355X stage, through the C ABI only (include/swiftkv.h): it owns a device
// context, the RoPE table (the reference image, or the same values in closed
// form), the KV cache and the per-layer q/k/v buffers, runs decode steps over
// every layer of a batch, and reports microseconds per layer, algorithmic
// HBM bytes per second and tokens per second.
//
// The stage has no weights of its own, so its inputs are synthetic: cached
// rows go through the append rule from the library's seeded generators, and
// q/k/v per layer come from the same generators (FP32, converted to Q15.17
// on the device for --q17, or as split-K FP32 partial sums for --parts).
//
//   swiftkv_host --batch 64 --context 4096 --steps 10
//   swiftkv_host --batch 1 --graph
//   swiftkv_host --decode --batch 16 --context 32257 --steps 512 --layers 1 --t3
//   swiftkv_host --exact --batch 4 --context 1024 --rope-lut rope_lut.bin
//   swiftkv_host --batch 64 --parts 4
//   swiftkv_host --batch 1 --noalloc --graph
//   swiftkv_host --batch 3 --layers 2 --context 700 --steps 2 --dump /tmp/run
#include "swiftkv.h"

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <limits>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

constexpr int kModelDim = SWIFTKV_MODEL_DIM;
constexpr int kGroupsPerSequence = SWIFTKV_HEADS * SWIFTKV_HEAD_DIM / 32;   // A14/E8M0 groups
constexpr std::size_t kTokenHeadBytes = 2 * SWIFTKV_HEAD_DIM + 8 * sizeof(float);
constexpr std::size_t kRopeBytesPerPosition = SWIFTKV_ROPE_LUT_BYTES_PER_POSITION;
constexpr std::size_t kReferenceRopeBytes =
    static_cast<std::size_t>(SWIFTKV_REFERENCE_MAX_SEQ) * kRopeBytesPerPosition;

static_assert(kModelDim == 4096, "Llama-2-7B model width");
static_assert(kTokenHeadBytes == 288, "cache bytes per token-head: codes and G32 scales");
static_assert(kReferenceRopeBytes == 2097152, "the reference rope_lut.bin is 2 MiB");

using Clock = std::chrono::steady_clock;

double elapsed_ms(Clock::time_point begin, Clock::time_point end) {
    return std::chrono::duration<double, std::milli>(end - begin).count();
}

// Any failing C-ABI call ends the run with the library's own message.
void check(int status, const char* what) {
    if (status != SWIFTKV_OK) {
        std::ostringstream msg;
        msg << what << " failed (status " << status << "): " << swiftkv_last_error();
        throw std::runtime_error(msg.str());
    }
}

// Reads a whole file whose size must be a positive multiple of `unit` bytes
// and at least `min_bytes`.
std::vector<std::uint8_t> read_file_checked(const std::string& path, std::size_t unit, std::size_t min_bytes) {
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) throw std::runtime_error("cannot open " + path);
    const std::streamoff end = in.tellg();
    if (end <= 0) throw std::runtime_error("cannot size " + path + " (empty or unreadable)");
    const auto bytes = static_cast<std::size_t>(end);
    if (bytes % unit != 0 || bytes < min_bytes) {
        std::ostringstream msg;
        msg << path << " holds " << bytes << " bytes: need a multiple of " << unit << " and at least " << min_bytes;
        throw std::runtime_error(msg.str());
    }
    std::vector<std::uint8_t> data(bytes);
    in.seekg(0);
    constexpr std::size_t kChunk = 16u << 20;
    for (std::size_t done = 0; done < bytes;) {
        const std::size_t n = std::min(kChunk, bytes - done);
        in.read(reinterpret_cast<char*>(data.data() + done), static_cast<std::streamsize>(n));
        if (static_cast<std::size_t>(in.gcount()) != n) throw std::runtime_error("short read in " + path);
        done += n;
    }
    return data;
}

// Writes `bytes` bytes to `path`, replacing the file.
void write_file(const std::string& path, const void* data, std::size_t bytes) {
    std::ofstream out(path, std::ios::binary | std::ios::trunc);
    if (!out) throw std::runtime_error("cannot create " + path);
    out.write(static_cast<const char*>(data), static_cast<std::streamsize>(bytes));
    if (!out) throw std::runtime_error("short write to " + path);
}

// Algorithmic HBM bytes of one (sequence, layer) step at `position`: every
// cached token-head read once, the new row written, FP32 q/k/v in (each as
// `parts` partial rows) and the output out.
std::uint64_t step_bytes(int position, int parts) {
    return static_cast<std::uint64_t>(SWIFTKV_HEADS) *
           (static_cast<std::uint64_t>(position) * kTokenHeadBytes + kTokenHeadBytes +
            (3ull * static_cast<std::uint64_t>(parts) + 1ull) * SWIFTKV_HEAD_DIM * 4);
}

struct Config {
    int device = 0;
    int layers = 32;
    int batch = 1;
    int context = 4096;       // tokens attended at the first timed step (position context-1)
    int steps = 10;
    int warmup = 3;
    int split = 0;            // tokens per split, 0 = the library's heuristic
    std::string rope_lut;     // reference image; empty = closed form
    double theta = 10000.0;
    std::uint64_t seed = 2026;
    bool q17 = false;         // Q15.17 inputs (swiftkv_attention_q17)
    bool exact = false;       // integer-compatibility entry
    int parts = 1;            // split-K FP32 partials per input (swiftkv_attention_partials) when 2 or 4
    bool noalloc = false;     // the allocation-free entry (swiftkv_attention_f32_noalloc)
    bool decode = false;      // step s runs at position context-1+s, appending as it goes
    bool graph = false;       // record one step as a HIP graph and replay it
    bool host_io = false;     // host-memory q/k/v and outputs
    bool t3 = false;          // Student-t(3) data instead of N(0,1)
    bool outliers = false;    // 1% of K channels x20
    std::string dump;         // directory for the last call's outputs and the appended rows
};

void print_usage(const char* program) {
    std::cout
        << "Usage: " << program << " [options]\n"
        << "  --device N       GPU index (0)\n"
        << "  --layers N       layers per step (32)\n"
        << "  --batch N        sequences (1)\n"
        << "  --context N      tokens attended at the first timed step, i.e. position N-1 (4096)\n"
        << "  --steps N        timed steps (10)\n"
        << "  --warmup N       untimed steps first (3; none with --decode)\n"
        << "  --split N        tokens per split, a multiple of 256 (0 = heuristic)\n"
        << "  --rope-lut PATH  the reference rope_lut.bin image (default: closed form)\n"
        << "  --theta X        RoPE base for the closed form (10000)\n"
        << "  --seed N         synthetic-data seed (2026)\n"
        << "  --q17            Q15.17 inputs (default FP32)\n"
        << "  --exact          the integer-compatibility entry (bit-exact A14 words)\n"
        << "  --parts N        inputs as N = 2 or 4 split-K FP32 partial sums (swiftkv_attention_partials;\n"
        << "                   with --exact they are finalized once by swiftkv_convert_partials_q17)\n"
        << "  --noalloc        the allocation-free entry (swiftkv_attention_f32_noalloc: FP32 device inputs,\n"
        << "                   split workspace in the library's fixed per-GPU array)\n"
        << "  --decode         advance the position every step (a real decode run)\n"
        << "  --graph          record one step as a HIP graph and time its replays\n"
        << "  --host-io        inputs and outputs in host memory (PCIe included)\n"
        << "  --t3             Student-t(3) data, unit variance\n"
        << "  --outliers       1% of K channels scaled x20\n"
        << "  --dump DIR       write the last layer's outputs of the last step (output.bin, activation_q.bin,\n"
        << "                   activation_scale.bin), the rows appended by that step for every sequence,\n"
        << "                   layer and head as reference records (appended.bin) and meta.json into DIR\n"
        << "  --help           this text\n";
}

long long parse_integer(const std::string& flag, const char* text, long long lo, long long hi) {
    if (text == nullptr) throw std::runtime_error(flag + " needs a value");
    char* end = nullptr;
    errno = 0;
    const long long v = std::strtoll(text, &end, 10);
    if (errno != 0 || end == text || *end != '\0' || v < lo || v > hi) {
        std::ostringstream msg;
        msg << flag << " " << text << ": expected an integer in [" << lo << ", " << hi << "]";
        throw std::runtime_error(msg.str());
    }
    return v;
}

Config parse_args(int argc, char** argv, bool* help) {
    Config c;
    *help = false;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto value = [&]() -> const char* { return i + 1 < argc ? argv[++i] : nullptr; };
        if (a == "--help" || a == "-h") {
            *help = true;
        } else if (a == "--device") {
            c.device = static_cast<int>(parse_integer(a, value(), 0, 63));
        } else if (a == "--layers") {
            c.layers = static_cast<int>(parse_integer(a, value(), 1, 64));
        } else if (a == "--batch") {
            c.batch = static_cast<int>(parse_integer(a, value(), 1, 4096));
        } else if (a == "--context") {
            c.context = static_cast<int>(parse_integer(a, value(), 1, SWIFTKV_MAX_SEQ));
        } else if (a == "--steps") {
            c.steps = static_cast<int>(parse_integer(a, value(), 1, 1 << 20));
        } else if (a == "--warmup") {
            c.warmup = static_cast<int>(parse_integer(a, value(), 0, 1000));
        } else if (a == "--split") {
            c.split = static_cast<int>(parse_integer(a, value(), 0, SWIFTKV_MAX_SEQ));
        } else if (a == "--rope-lut") {
            const char* v = value();
            if (v == nullptr) throw std::runtime_error("--rope-lut needs a path");
            c.rope_lut = v;
        } else if (a == "--theta") {
            const char* v = value();
            char* end = nullptr;
            c.theta = v ? std::strtod(v, &end) : 0.0;
            if (v == nullptr || end == v || *end != '\0' || !(c.theta > 1.0) || !std::isfinite(c.theta))
                throw std::runtime_error("--theta needs a finite number > 1");
        } else if (a == "--seed") {
            c.seed = static_cast<std::uint64_t>(parse_integer(a, value(), 0, std::numeric_limits<long long>::max()));
        } else if (a == "--q17") {
            c.q17 = true;
        } else if (a == "--exact") {
            c.exact = true;
        } else if (a == "--parts") {
            c.parts = static_cast<int>(parse_integer(a, value(), 1, 4));
            if (c.parts == 3) throw std::runtime_error("--parts must be 1, 2 or 4");
        } else if (a == "--noalloc") {
            c.noalloc = true;
        } else if (a == "--decode") {
            c.decode = true;
        } else if (a == "--graph") {
            c.graph = true;
        } else if (a == "--host-io") {
            c.host_io = true;
        } else if (a == "--t3") {
            c.t3 = true;
        } else if (a == "--outliers") {
            c.outliers = true;
        } else if (a == "--dump") {
            const char* v = value();
            if (v == nullptr || *v == '\0') throw std::runtime_error("--dump needs a directory");
            c.dump = v;
        } else {
            throw std::runtime_error("unknown option " + a + " (try --help)");
        }
    }
    if (c.decode && c.graph)
        throw std::runtime_error("--graph replays the recorded positions; it cannot advance them (--decode)");
    if (c.host_io && c.graph) throw std::runtime_error("--host-io calls synchronize; they cannot be recorded (--graph)");
    if (c.parts > 1 && c.q17) throw std::runtime_error("--parts gives FP32 partial sums; it excludes --q17");
    if (c.noalloc && (c.q17 || c.exact || c.parts > 1 || c.host_io))
        throw std::runtime_error("--noalloc takes FP32 device inputs; it excludes --q17, --exact, --parts and --host-io");
    const long long last = static_cast<long long>(c.context) - 1 + (c.decode ? c.steps - 1 : 0);
    if (last >= SWIFTKV_MAX_SEQ) {
        std::ostringstream msg;
        msg << "the run reaches position " << last << ", beyond the cache limit " << SWIFTKV_MAX_SEQ - 1;
        throw std::runtime_error(msg.str());
    }
    if (c.exact && last >= SWIFTKV_REFERENCE_MAX_SEQ) {
        std::ostringstream msg;
        msg << "the run reaches position " << last << "; --exact keeps the reference's bound (positions below "
            << SWIFTKV_REFERENCE_MAX_SEQ << ")";
        throw std::runtime_error(msg.str());
    }
    return c;
}

// Owners of the C-ABI handles (released in reverse order of creation).
struct ContextHandle {
    swiftkv_context* p = nullptr;
    ~ContextHandle() { swiftkv_context_destroy(p); }
};
struct LutHandle {
    swiftkv_rope_lut* p = nullptr;
    ~LutHandle() { swiftkv_rope_lut_destroy(p); }
};
struct CacheHandle {
    swiftkv_kv_cache* p = nullptr;
    ~CacheHandle() { swiftkv_kv_cache_destroy(p); }
};
struct GraphHandle {
    swiftkv_graph* p = nullptr;
    ~GraphHandle() { swiftkv_graph_destroy(p); }
};
struct DeviceBuffer {
    swiftkv_context* ctx = nullptr;
    void* p = nullptr;
    DeviceBuffer(swiftkv_context* c, std::size_t bytes) : ctx(c) { check(swiftkv_device_alloc(c, bytes, &p), "device alloc"); }
    ~DeviceBuffer() { swiftkv_device_free(ctx, p); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
};

int run(const Config& cfg) {
    const int p0 = cfg.context - 1;                                  // first timed position
    const int capacity = p0 + 1 + (cfg.decode ? cfg.steps - 1 : 0);  // last written position + 1
    const std::size_t row_elems = static_cast<std::size_t>(cfg.batch) * kModelDim;
    const std::size_t layer_elems = row_elems;
    const std::size_t all_elems = layer_elems * static_cast<std::size_t>(cfg.layers);
    const int dist = cfg.t3 ? SWIFTKV_DIST_STUDENT_T3 : SWIFTKV_DIST_NORMAL;

    ContextHandle ctx;
    check(swiftkv_context_create(cfg.device, &ctx.p), "swiftkv_context_create");
    check(swiftkv_set_split_tokens(ctx.p, cfg.split), "swiftkv_set_split_tokens");

    const auto t_setup = Clock::now();
    LutHandle lut;
    if (!cfg.rope_lut.empty()) {
        const std::vector<std::uint8_t> image =
            read_file_checked(cfg.rope_lut, kRopeBytesPerPosition, static_cast<std::size_t>(capacity) * kRopeBytesPerPosition);
        check(swiftkv_rope_lut_load(ctx.p, image.data(), image.size(), &lut.p), "swiftkv_rope_lut_load");
    } else {
        check(swiftkv_rope_lut_generate(ctx.p, std::max(capacity, SWIFTKV_REFERENCE_MAX_SEQ), cfg.theta, &lut.p),
              "swiftkv_rope_lut_generate");
    }

    CacheHandle kv;
    check(swiftkv_kv_cache_create(ctx.p, cfg.layers, cfg.batch, capacity, &kv.p), "swiftkv_kv_cache_create");
    if (p0 > 0)
        check(swiftkv_kv_cache_fill_synthetic(ctx.p, kv.p, lut.p, 0, cfg.layers, 0, cfg.batch, p0, cfg.seed, dist,
                                              cfg.outliers ? 1 : 0),
              "swiftkv_kv_cache_fill_synthetic");

    // q/k/v of every layer, generated once on the device: [layer][batch][4096]
    // FP32, or with --parts [part][layer][batch][4096] partial sums (part
    // stride all_elems).  --q17, and --exact with partials, convert them to
    // Q15.17 once here, as the upstream finalize would.
    const std::size_t in_elems = all_elems * static_cast<std::size_t>(cfg.parts);
    DeviceBuffer qkv_f32[3] = {{ctx.p, in_elems * 4}, {ctx.p, in_elems * 4}, {ctx.p, in_elems * 4}};
    for (int i = 0; i < 3; ++i)
        check(swiftkv_fill_synthetic_f32(ctx.p, static_cast<float*>(qkv_f32[i].p), in_elems, 0, cfg.seed + 1,
                                         1000 + i, dist, (cfg.outliers && i == 1) ? 1 : 0),
              "swiftkv_fill_synthetic_f32");
    const bool finalized = cfg.q17 || (cfg.exact && cfg.parts > 1);
    std::unique_ptr<DeviceBuffer> qkv_q17[3];
    if (finalized) {
        for (int i = 0; i < 3; ++i) {
            qkv_q17[i] = std::make_unique<DeviceBuffer>(ctx.p, all_elems * 4);
            const float* src = static_cast<const float*>(qkv_f32[i].p);
            std::int32_t* dst = static_cast<std::int32_t*>(qkv_q17[i]->p);
            if (cfg.parts > 1)
                check(swiftkv_convert_partials_q17(ctx.p, src, cfg.parts, static_cast<std::int64_t>(all_elems), dst,
                                                   all_elems),
                      "swiftkv_convert_partials_q17");
            else
                check(swiftkv_convert_f32_q17(ctx.p, src, dst, all_elems), "swiftkv_convert_f32_q17");
        }
    }
    const int step_parts = finalized ? 1 : cfg.parts;   // partial rows each step call reads per input
    const std::size_t feed_elems = finalized ? all_elems : in_elems;
    auto input = [&](int i) -> void* { return finalized ? qkv_q17[i]->p : qkv_f32[i].p; };

    // Outputs: FP32 rows (or the Q15.17 state for --exact) and the A14/E8M0 words.
    DeviceBuffer out(ctx.p, row_elems * 4);
    DeviceBuffer act_q(ctx.p, static_cast<std::size_t>(cfg.batch) * kGroupsPerSequence * SWIFTKV_A14_WORD_BYTES);
    DeviceBuffer act_scale(ctx.p, static_cast<std::size_t>(cfg.batch) * kGroupsPerSequence);

    // Host-memory I/O: the same inputs copied to host memory once.
    std::vector<std::vector<std::uint8_t>> host_in;
    std::vector<std::uint8_t> host_out, host_aq, host_as;
    if (cfg.host_io) {
        check(swiftkv_synchronize(ctx.p), "swiftkv_synchronize");
        for (int i = 0; i < 3; ++i) {
            host_in.emplace_back(feed_elems * 4);
            check(swiftkv_memcpy_d2h(ctx.p, host_in.back().data(), input(i), feed_elems * 4), "swiftkv_memcpy_d2h");
        }
        host_out.resize(row_elems * 4);
        host_aq.resize(static_cast<std::size_t>(cfg.batch) * kGroupsPerSequence * SWIFTKV_A14_WORD_BYTES);
        host_as.resize(static_cast<std::size_t>(cfg.batch) * kGroupsPerSequence);
        check(swiftkv_set_host_io(ctx.p, 1), "swiftkv_set_host_io");
    }

    std::vector<std::int32_t> positions(static_cast<std::size_t>(cfg.batch));
    auto one_step = [&](int position) {
        std::fill(positions.begin(), positions.end(), position);
        for (int layer = 0; layer < cfg.layers; ++layer) {
            const std::size_t off = static_cast<std::size_t>(layer) * layer_elems * 4;
            const void* q;
            const void* k;
            const void* v;
            void* o;
            std::uint8_t* aq;
            std::uint8_t* as;
            if (cfg.host_io) {
                q = host_in[0].data() + off;
                k = host_in[1].data() + off;
                v = host_in[2].data() + off;
                o = host_out.data();
                aq = host_aq.data();
                as = host_as.data();
            } else {
                q = static_cast<const std::uint8_t*>(input(0)) + off;
                k = static_cast<const std::uint8_t*>(input(1)) + off;
                v = static_cast<const std::uint8_t*>(input(2)) + off;
                o = out.p;
                aq = static_cast<std::uint8_t*>(act_q.p);
                as = static_cast<std::uint8_t*>(act_scale.p);
            }
            if (cfg.exact) {
                check(swiftkv_attention_exact(ctx.p, q, k, v, finalized ? 1 : 0, kv.p, lut.p, aq, as, layer,
                                              positions.data(), cfg.batch, static_cast<std::int32_t*>(o)),
                      "swiftkv_attention_exact");
            } else if (step_parts > 1) {
                check(swiftkv_attention_partials(ctx.p, static_cast<const float*>(q), static_cast<const float*>(k),
                                                 static_cast<const float*>(v), step_parts,
                                                 static_cast<std::int64_t>(all_elems), kv.p, lut.p, aq, as, layer,
                                                 positions.data(), cfg.batch, static_cast<float*>(o)),
                      "swiftkv_attention_partials");
            } else if (cfg.noalloc) {
                check(swiftkv_attention_f32_noalloc(ctx.p, static_cast<const float*>(q), static_cast<const float*>(k),
                                                    static_cast<const float*>(v), kv.p, lut.p, aq, as, layer,
                                                    positions.data(), cfg.batch, static_cast<float*>(o)),
                      "swiftkv_attention_f32_noalloc");
            } else if (cfg.q17) {
                check(swiftkv_attention_q17(ctx.p, static_cast<const std::int32_t*>(q),
                                            static_cast<const std::int32_t*>(k), static_cast<const std::int32_t*>(v),
                                            kv.p, lut.p, aq, as, layer, positions.data(), cfg.batch,
                                            static_cast<float*>(o)),
                      "swiftkv_attention_q17");
            } else {
                check(swiftkv_attention_f32(ctx.p, static_cast<const float*>(q), static_cast<const float*>(k),
                                            static_cast<const float*>(v), kv.p, lut.p, aq, as, layer,
                                            positions.data(), cfg.batch, static_cast<float*>(o)),
                      "swiftkv_attention_f32");
            }
        }
    };

    // Untimed steps; a graph needs at least one eager step first (it sizes the
    // split workspace, which cannot grow while a graph is being recorded).
    const int warmup = cfg.decode ? 0 : std::max(cfg.warmup, cfg.graph ? 1 : 0);
    for (int w = 0; w < warmup; ++w) one_step(p0);
    if (!cfg.host_io) check(swiftkv_synchronize(ctx.p), "swiftkv_synchronize");
    const double setup_ms = elapsed_ms(t_setup, Clock::now());

    GraphHandle graph;
    if (cfg.graph) {
        check(swiftkv_capture_begin(ctx.p), "swiftkv_capture_begin");
        one_step(p0);
        check(swiftkv_capture_end(ctx.p, &graph.p), "swiftkv_capture_end");
        check(swiftkv_graph_launch(ctx.p, graph.p), "swiftkv_graph_launch");   // one untimed replay
    }

    const auto t0 = Clock::now();
    check(swiftkv_timer_record(ctx.p, 0), "swiftkv_timer_record");
    for (int s = 0; s < cfg.steps; ++s) {
        if (cfg.graph)
            check(swiftkv_graph_launch(ctx.p, graph.p), "swiftkv_graph_launch");
        else
            one_step(cfg.decode ? p0 + s : p0);
    }
    check(swiftkv_timer_record(ctx.p, 1), "swiftkv_timer_record");
    float device_ms = 0.0f;
    check(swiftkv_timer_elapsed(ctx.p, 0, 1, &device_ms), "swiftkv_timer_elapsed");
    const double wall_ms = elapsed_ms(t0, Clock::now());
    if (cfg.host_io) check(swiftkv_set_host_io(ctx.p, 0), "swiftkv_set_host_io");

    // The last layer's output must be finite (and, for the integer path, the
    // Q15.17 state non-trivial).
    std::vector<std::uint8_t> last(row_elems * 4);
    if (cfg.host_io)
        last = host_out;
    else
        check(swiftkv_memcpy_d2h(ctx.p, last.data(), out.p, last.size()), "swiftkv_memcpy_d2h");
    double max_abs = 0.0;
    for (std::size_t i = 0; i < row_elems; ++i) {
        double x;
        if (cfg.exact) {
            std::int32_t raw;
            std::memcpy(&raw, last.data() + 4 * i, 4);
            x = std::ldexp(static_cast<double>(raw), -17);
        } else {
            float f;
            std::memcpy(&f, last.data() + 4 * i, 4);
            x = f;
        }
        if (!std::isfinite(x)) throw std::runtime_error("non-finite attention output");
        max_abs = std::max(max_abs, std::fabs(x));
    }
    if (max_abs == 0.0) throw std::runtime_error("attention output is all zero");

    if (!cfg.dump.empty()) {
        // The outputs of the last call (the last layer of the last step) and
        // the row that step appended for every (sequence, layer, head), in the
        // reference's 320-byte record format, for an offline comparison with
        // an independent model of the stage.
        const int p_last = cfg.decode ? p0 + cfg.steps - 1 : p0;
        std::vector<std::uint8_t> aq_bytes(static_cast<std::size_t>(cfg.batch) * kGroupsPerSequence *
                                           SWIFTKV_A14_WORD_BYTES),
            as_bytes(static_cast<std::size_t>(cfg.batch) * kGroupsPerSequence);
        if (cfg.host_io) {
            aq_bytes = host_aq;
            as_bytes = host_as;
        } else {
            check(swiftkv_memcpy_d2h(ctx.p, aq_bytes.data(), act_q.p, aq_bytes.size()), "swiftkv_memcpy_d2h");
            check(swiftkv_memcpy_d2h(ctx.p, as_bytes.data(), act_scale.p, as_bytes.size()), "swiftkv_memcpy_d2h");
        }
        std::vector<std::uint8_t> records(static_cast<std::size_t>(cfg.batch) * cfg.layers * SWIFTKV_HEADS *
                                          SWIFTKV_RECORD_BYTES);
        for (int b = 0; b < cfg.batch; ++b)
            for (int layer = 0; layer < cfg.layers; ++layer)
                for (int h = 0; h < SWIFTKV_HEADS; ++h) {
                    const std::size_t idx = (static_cast<std::size_t>(b) * cfg.layers + layer) * SWIFTKV_HEADS + h;
                    check(swiftkv_kv_cache_export_records(ctx.p, kv.p, b, layer, h, p_last, 1,
                                                          records.data() + idx * SWIFTKV_RECORD_BYTES),
                          "swiftkv_kv_cache_export_records");
                }
        write_file(cfg.dump + "/output.bin", last.data(), last.size());
        write_file(cfg.dump + "/activation_q.bin", aq_bytes.data(), aq_bytes.size());
        write_file(cfg.dump + "/activation_scale.bin", as_bytes.data(), as_bytes.size());
        write_file(cfg.dump + "/appended.bin", records.data(), records.size());
        std::ostringstream meta;
        meta << "{\"batch\": " << cfg.batch << ", \"layers\": " << cfg.layers << ", \"layer\": " << cfg.layers - 1
             << ", \"first_position\": " << p0 << ", \"position\": " << p_last << ", \"steps\": " << cfg.steps
             << ", \"decode\": " << (cfg.decode ? "true" : "false") << ", \"seed\": " << cfg.seed
             << ", \"input_seed\": " << cfg.seed + 1 << ", \"input_streams\": [1000, 1001, 1002]"
             << ", \"distribution\": " << dist << ", \"outliers\": " << (cfg.outliers ? "true" : "false")
             << ", \"parts\": " << cfg.parts << ", \"q17\": " << (cfg.q17 ? "true" : "false")
             << ", \"exact\": " << (cfg.exact ? "true" : "false")
             << ", \"noalloc\": " << (cfg.noalloc ? "true" : "false")
             << ", \"input_layout\": \"[part][layer][batch][4096] FP32\""
             << ", \"output\": \"" << (cfg.exact ? "int32 Q15.17" : "float32") << " [batch][4096]\""
             << ", \"appended\": \"records [batch][layer][head][320] of token position\"}\n";
        const std::string text = meta.str();
        write_file(cfg.dump + "/meta.json", text.data(), text.size());
    }

    // With host I/O the calls are synchronous, so the wall clock is the time.
    const double ms = cfg.host_io ? wall_ms : static_cast<double>(device_ms);
    std::uint64_t bytes = 0;
    for (int s = 0; s < cfg.steps; ++s)
        bytes += static_cast<std::uint64_t>(cfg.batch) * cfg.layers * step_bytes(cfg.decode ? p0 + s : p0, step_parts);
    const double us_per_layer = 1000.0 * ms / cfg.steps / cfg.layers;
    const double gbps = static_cast<double>(bytes) / (ms * 1e-3) / 1e9;
    const double tokens_per_s = static_cast<double>(cfg.batch) * cfg.steps / (ms * 1e-3);

    std::cout << std::fixed << std::setprecision(2)
              << "swiftkv_host: " << swiftkv_version() << "\n"
              << "  batch " << cfg.batch << ", " << cfg.layers << " layers, position " << p0
              << (cfg.decode ? " advancing" : "") << ", " << cfg.steps << " steps"
              << (cfg.exact ? ", integer-compatibility entry" : (cfg.q17 ? ", Q15.17 inputs" : ", FP32 inputs"))
              << (cfg.noalloc ? ", allocation-free entry" : "")
              << (cfg.parts > 1 ? ", " + std::to_string(cfg.parts) + " split-K partials per input" : std::string())
              << (cfg.graph ? ", graph replay" : "") << (cfg.host_io ? ", host-memory I/O" : "") << "\n"
              << "  setup " << setup_ms << " ms; timed " << ms << " ms (" << (cfg.host_io ? "wall" : "device")
              << " clock; wall " << wall_ms << " ms)\n"
              << "  " << us_per_layer << " us/layer, " << gbps << " GB/s (" << 100.0 * gbps / 8000.0
              << "% of 8 TB/s), " << tokens_per_s << " tokens/s\n"
              << "result: {\"us_per_layer\": " << us_per_layer << ", \"gbps\": " << gbps
              << ", \"tokens_per_s\": " << tokens_per_s << ", \"max_abs_output\": " << std::setprecision(6)
              << max_abs << "}" << std::endl;
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        bool help = false;
        const Config cfg = parse_args(argc, argv, &help);
        if (help) {
            print_usage(argv[0]);
            return 0;
        }
        return run(cfg);
    } catch (const std::exception& e) {
        std::cerr << "swiftkv_host: " << e.what() << std::endl;
        return 1;
    }
}
