// swiftkv_synth.hip -- synthetic inputs generated on the device.
//
// A "synthetic stream" (seed, stream) is an endless FP32 tensor whose element i
// is drawn from a counter-based generator: splitmix64 keyed by (seed, stream,
// i/2), Box-Muller for N(0,1), and N / sqrt(chi2_3 / 3) / sqrt(3) for the
// unit-variance Student-t(3).  With `outliers` set, element i is multiplied by
// 20 when its channel i % 4096 is one of the ~1% channels selected by the seed.
//
// Two consumers: swiftkv_fill_synthetic_f32 writes elements [first, first+n) of a stream
// (q/k/v step inputs, or a copy of a cache's source rows for checking), and
// swiftkv_kv_cache_fill_synthetic feeds rows of the streams
//   K: stream 2*(slot*64 + layer),  V: stream 2*(slot*64 + layer) + 1,
//   row t = elements [t*4096, (t+1)*4096)
// through the append rule (FP32 -> Q15.17, RoPE of k at position t, G32
// quantization) into a cache, so a multi-GB cache is filled without host
// staging and holds exactly what the append kernels would have written.
#include "swiftkv_device.hpp"

namespace swiftkv {
namespace {

using namespace dev;

__device__ __forceinline__ uint64_t smix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Stream {
    uint64_t key;        // smix(seed ^ smix(stream))
    uint64_t outlier_key;
    int32_t dist;        // 0 normal, 1 Student-t(3)
    int32_t outliers;
};

__device__ __forceinline__ float2 normal2(uint64_t key, uint64_t j) {
    const uint64_t z = smix(key + j);
    const float u1 = static_cast<float>((z >> 40) + 1u) * 0x1p-24f;            // (0, 1]
    const float u2 = static_cast<float>((z >> 16) & 0xFFFFFFu) * 0x1p-24f;     // [0, 1)
    const float r = sqrtf(-2.0f * logf(u1));
    float s, c;
    sincospif(2.0f * u2, &s, &c);
    return make_float2(r * c, r * s);
}

// Elements 2j and 2j+1 of a stream.
__device__ __forceinline__ float2 stream_pair(const Stream& st, uint64_t j) {
    float2 x;
    if (st.dist == 1) {
        const float2 n = normal2(st.key, 4 * j);
        const float2 a = normal2(st.key, 4 * j + 1);
        const float2 b = normal2(st.key, 4 * j + 2);
        const float2 c = normal2(st.key, 4 * j + 3);
        const float chi0 = a.x * a.x + a.y * a.y + b.x * b.x;
        const float chi1 = b.y * b.y + c.x * c.x + c.y * c.y;
        const float k = 0.57735026918962576f;   // 1/sqrt(3): unit variance
        x = make_float2(n.x * rsqrtf(chi0 * (1.0f / 3.0f)) * k, n.y * rsqrtf(chi1 * (1.0f / 3.0f)) * k);
    } else {
        x = normal2(st.key, j);
    }
    if (st.outliers) {
        const uint32_t ch = static_cast<uint32_t>((2 * j) % kModelDim);
        if (smix(st.outlier_key + ch) % 100u == 0u) x.x *= 20.0f;
        if (smix(st.outlier_key + ch + 1) % 100u == 0u) x.y *= 20.0f;
    }
    return x;
}

__device__ __forceinline__ Stream make_stream(uint64_t seed, uint64_t stream, int dist, int outliers) {
    Stream st;
    st.key = smix(seed ^ smix(stream));
    st.outlier_key = smix(seed ^ 0x0123456789ABCDEFull);
    st.dist = dist;
    st.outliers = outliers;
    return st;
}

// Elements [2*pair0, 2*pair0 + n) of a stream (n may be odd).
__global__ __launch_bounds__(256) void fill_f32_kernel(float* __restrict__ out, size_t npairs, uint64_t pair0,
                                                       uint64_t seed, uint64_t stream, int dist, int outliers,
                                                       int odd_tail) {
    const Stream st = make_stream(seed, stream, dist, outliers);
    const size_t step = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t j = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < npairs; j += step) {
        const float2 x = stream_pair(st, pair0 + j);
        if (odd_tail && j + 1 == npairs) {
            out[2 * j] = x.x;
        } else {
            reinterpret_cast<float2*>(out)[j] = x;
        }
    }
}

struct FillArgs {
    CacheView kv;
    const int2* lut;
    uint64_t seed;
    int32_t layer0, nlayers, slot0, ntok;
    int32_t dist, k_outliers;
};

// Grid (ceil(ntok/16), 8, nslots * nlayers); wave = head, 16 tokens per wave.
__global__ __launch_bounds__(256) void fill_cache_kernel(FillArgs a) {
    const int h = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int slot = a.slot0 + static_cast<int>(blockIdx.z) / a.nlayers;
    const int layer = a.layer0 + static_cast<int>(blockIdx.z) % a.nlayers;
    const uint64_t sid = 2ull * (static_cast<uint64_t>(slot) * 64u + static_cast<uint64_t>(layer));
    const Stream sk = make_stream(a.seed, sid, a.dist, a.k_outliers);
    const Stream sv = make_stream(a.seed, sid + 1, a.dist, 0);
    int8_t* page = page_ptr(a.kv, slot, layer, h);
    const int t_end = min(a.ntok, static_cast<int>(blockIdx.x + 1) * 16);
    for (int t = blockIdx.x * 16; t < t_end; ++t) {
        const uint64_t j = (static_cast<uint64_t>(t) * kModelDim + h * kHeadDim + 2 * lane) >> 1;
        const float2 kf = stream_pair(sk, j);
        const float2 vf = stream_pair(sv, j);
        int32_t k0, k1;
        rope_pair(f32_to_q17(kf.x), f32_to_q17(kf.y), a.lut[static_cast<size_t>(t) * kRopePairs + lane], k0, k1);
        append_row(page, a.kv.seq_cap, t, lane, k0, k1, f32_to_q17(vf.x), f32_to_q17(vf.y));
    }
}

}  // namespace

hipError_t launch_fill_f32(float* out, size_t n, uint64_t first, uint64_t seed, uint64_t stream, int dist,
                           int outliers, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const size_t npairs = (n + 1) / 2;
    size_t blocks = (npairs + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    fill_f32_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(out, npairs, first / 2, seed, stream, dist,
                                                                   outliers, static_cast<int>(n & 1));
    return hipGetLastError();
}

hipError_t launch_fill_cache(const CacheView& kv, const int2* lut, uint64_t seed, int layer0, int nlayers,
                             int slot0, int nslots, int ntok, int dist, int k_outliers, hipStream_t s) {
    FillArgs a{kv, lut, seed, layer0, nlayers, slot0, ntok, dist, k_outliers};
    const dim3 grid((ntok + 15) / 16, kHeads / 4, nslots * nlayers);
    fill_cache_kernel<<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace swiftkv
