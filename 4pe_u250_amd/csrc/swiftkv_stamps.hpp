// swiftkv_stamps.hpp -- phase stamps of the step kernel, the tracing facility
// behind 4pe_u250_amd/phase_stamps.py.  Included by swiftkv_kernels.hip only.
//
// The instrumented build (libswiftkv_stamps.so, compiled with
// SWIFTKV_PHASE_STAMPS) records, per workgroup of the step kernel, thread 0's
// s_memrealtime (100 MHz) at entry, when wave 0's first loads have all arrived
// (an added wait for them), after the workgroup's LDS merge, when the arrival
// count is known, after the merge and after the epilogue; lane 0 of every wave
// records when its first loads arrived and when its scan ended; slot 7 holds
// the workgroup's XCD (low half) and HW_ID register (high half: CU, shader
// array and engine).  The product library compiles every hook below away.
#pragma once

#include <hip/hip_runtime.h>

#ifdef SWIFTKV_PHASE_STAMPS
constexpr int kStampWorkgroups = 8192;
constexpr int kStampSlots = 8;   // entry, first loads, LDS merge, arrival, merge, epilogue, flags, XCD + HW_ID
__device__ unsigned long long g_phase_stamps[kStampWorkgroups * kStampSlots];
__device__ unsigned long long g_wave_stamps[kStampWorkgroups * 16 * 2];
#define SKV_STAMP_DECL unsigned long long skv_st[kStampSlots] = {0, 0, 0, 0, 0, 0, 0, 0}
#define SKV_STAMP(i) do { if (threadIdx.x == 0) skv_st[i] = __builtin_amdgcn_s_memrealtime(); } while (0)
#define SKV_STAMP_FLAG(f) do { skv_st[6] |= (f); } while (0)
#define SKV_STAMP_WAIT() __builtin_amdgcn_s_waitcnt(0)
#define SKV_WAVE_STAMP(k, t) do {                                                                   \
        const size_t wg_ = (static_cast<size_t>(blockIdx.z) * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x; \
        if ((threadIdx.x & 63) == 0 && wg_ < kStampWorkgroups)                                      \
            g_wave_stamps[(wg_ * 16 + (threadIdx.x >> 6)) * 2 + (k)] = (t);                         \
    } while (0)
// A wave's first loads have arrived (after SKV_STAMP_WAIT); its scan is done.
#define SKV_WAVE_FIRST_LOADS() const unsigned long long skv_first = __builtin_amdgcn_s_memrealtime()
#define SKV_WAVE_SCAN_DONE() do {                                                                   \
        SKV_WAVE_STAMP(0, skv_first);                                                               \
        SKV_WAVE_STAMP(1, __builtin_amdgcn_s_memrealtime());                                        \
    } while (0)
#define SKV_STAMP_FLUSH() do {                                                                      \
        const size_t wg_ = (static_cast<size_t>(blockIdx.z) * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x; \
        if (threadIdx.x == 0 && wg_ < kStampWorkgroups) {                                           \
            unsigned xcc_, hw_;                                                                     \
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc_));                    \
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw_));                      \
            skv_st[7] = xcc_ | (static_cast<unsigned long long>(hw_) << 32);                        \
            for (int i_ = 0; i_ < kStampSlots; ++i_) g_phase_stamps[wg_ * kStampSlots + i_] = skv_st[i_]; \
        }                                                                                           \
    } while (0)

// Copies the stamps of the last step launch (workgroups [0, 8192)): phase
// [8192][8] then wave [8192][16][2] 64-bit words (instrumented build only,
// not part of the C ABI).
extern "C" int swiftkv_debug_phase_stamps(unsigned long long* phase, unsigned long long* wave) {
    if (hipMemcpyFromSymbol(phase, HIP_SYMBOL(g_phase_stamps), sizeof(g_phase_stamps), 0, hipMemcpyDeviceToHost) !=
        hipSuccess)
        return -3;
    return hipMemcpyFromSymbol(wave, HIP_SYMBOL(g_wave_stamps), sizeof(g_wave_stamps), 0, hipMemcpyDeviceToHost) ==
                   hipSuccess
               ? 0
               : -3;
}
#else
#define SKV_STAMP_DECL do {} while (0)
#define SKV_STAMP(i) do {} while (0)
#define SKV_STAMP_FLAG(f) do {} while (0)
#define SKV_STAMP_WAIT() do {} while (0)
#define SKV_WAVE_FIRST_LOADS() do {} while (0)
#define SKV_WAVE_SCAN_DONE() do {} while (0)
#define SKV_STAMP_FLUSH() do {} while (0)
#endif
