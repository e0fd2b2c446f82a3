// ref_shim.cpp -- C exports around the reference emulator's attention stage.
//
// TEST INFRASTRUCTURE ONLY (oracle/_ref).  Built by oracle/Makefile from the
// reference sources where they lie (software_sim/llama2_decoder_sw_emulator.cpp
// is included, not copied); the output library travels with the tree so the
// CPU baseline can time the reference's own code on the GPU host.  Nothing in
// the product links it.
//
// Exported functions wrap, without changing, the emulator's static functions:
//   float_to_q17            (emulator:481-505)
//   apply_rope_q17          (emulator:526-541, uses the global RoPE table)
//   swiftkv_shift_for_group (emulator:543-554)
//   swiftkv_quantize_raw    (emulator:556-564)
//   swiftkv_exp_negative_q17(emulator:575-595)
//   swiftkv_attention_4pe   (emulator:602-714), layer 0 of a one-layer cache
#define main swiftkv_reference_emulator_main
#include "llama2_decoder_sw_emulator.cpp"
#undef main

namespace {
struct RefCache {
    int seq_len;
    KVCachePE pe[NUM_PES];
};
}  // namespace

extern "C" {

int32_t ref_float_to_q17(float x) { return float_to_q17(x); }

void ref_float_to_q17_array(const float* in, int32_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = float_to_q17(in[i]);
}

uint32_t ref_exp_negative_q17(int32_t x) { return swiftkv_exp_negative_q17(x); }

uint8_t ref_shift_for_group(const int32_t* values32) { return swiftkv_shift_for_group(values32); }

int8_t ref_quantize_raw(int32_t raw, uint8_t shift) { return swiftkv_quantize_raw(raw, shift); }

// Install a RoPE table [npos][64] (cos, sin as signed Q1.17).
void ref_set_rope(const int32_t* cosv, const int32_t* sinv, int npos) {
    g_rope.cosine.assign(cosv, cosv + static_cast<size_t>(npos) * 64);
    g_rope.sine.assign(sinv, sinv + static_cast<size_t>(npos) * 64);
    g_rope.loaded = true;
}

// Rotate a full 4096-channel vector (32 heads) at `pos`.
void ref_apply_rope(int32_t* vec4096, int pos) { apply_rope_q17(vec4096, pos); }

void* ref_cache_create(int seq_len) {
    RefCache* c = new RefCache();
    c->seq_len = seq_len;
    const size_t tokens = static_cast<size_t>(LOCAL_HEADS) * seq_len;
    for (auto& pe : c->pe) {
        pe.k_cache.assign(tokens * HEAD_DIM, 0);
        pe.v_cache.assign(tokens * HEAD_DIM, 0);
        pe.k_shift.assign(tokens * 4, 0);
        pe.v_shift.assign(tokens * 4, 0);
    }
    return c;
}

void ref_cache_destroy(void* h) { delete static_cast<RefCache*>(h); }

// Write (dir=0) or read (dir=1) one cached row of global head `head`.
void ref_cache_row(void* h, int dir, int head, int token, int8_t* kc, uint8_t* ks, int8_t* vc, uint8_t* vs) {
    RefCache* c = static_cast<RefCache*>(h);
    KVCachePE& pe = c->pe[head / LOCAL_HEADS];
    const size_t rec = static_cast<size_t>(head % LOCAL_HEADS) * c->seq_len + token;
    int8_t* pk = pe.k_cache.data() + rec * HEAD_DIM;
    int8_t* pv = pe.v_cache.data() + rec * HEAD_DIM;
    uint8_t* sk = pe.k_shift.data() + rec * 4;
    uint8_t* sv = pe.v_shift.data() + rec * 4;
    if (dir == 0) {
        std::memcpy(pk, kc, HEAD_DIM); std::memcpy(pv, vc, HEAD_DIM);
        std::memcpy(sk, ks, 4); std::memcpy(sv, vs, 4);
    } else {
        std::memcpy(kc, pk, HEAD_DIM); std::memcpy(vc, pv, HEAD_DIM);
        std::memcpy(ks, sk, 4); std::memcpy(vs, sv, 4);
    }
}

// Write n consecutive rows [tok0, tok0+n) of global head `head`: codes
// [n][128], shifts [n][4] (one call instead of one per row for long caches).
void ref_cache_rows(void* h, int head, int tok0, int n, const int8_t* kc, const uint8_t* ks, const int8_t* vc,
                    const uint8_t* vs) {
    RefCache* c = static_cast<RefCache*>(h);
    KVCachePE& pe = c->pe[head / LOCAL_HEADS];
    const size_t rec = static_cast<size_t>(head % LOCAL_HEADS) * c->seq_len + tok0;
    std::memcpy(pe.k_cache.data() + rec * HEAD_DIM, kc, static_cast<size_t>(n) * HEAD_DIM);
    std::memcpy(pe.v_cache.data() + rec * HEAD_DIM, vc, static_cast<size_t>(n) * HEAD_DIM);
    std::memcpy(pe.k_shift.data() + rec * 4, ks, static_cast<size_t>(n) * 4);
    std::memcpy(pe.v_shift.data() + rec * 4, vs, static_cast<size_t>(n) * 4);
}

// One attention stage of one sequence at `pos` on layer 0: q/k rotated,
// v raw (all Q15.17, 4096 channels).  Appends, scans, A14-quantizes.
void ref_attention(void* h, const int32_t* q, const int32_t* k, const int32_t* v, int pos,
                   int16_t* act_q4096, float* act_scale128) {
    RefCache* c = static_cast<RefCache*>(h);
    g_cache_seq_len = c->seq_len;
    QuantizedActivation out;
    swiftkv_attention_4pe(q, k, v, c->pe, 0, pos, out);
    std::memcpy(act_q4096, out.q.data(), sizeof(int16_t) * DIM);
    std::memcpy(act_scale128, out.scale.data(), sizeof(float) * (DIM / GROUP_SIZE));
}

int ref_omp_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

}  // extern "C"
