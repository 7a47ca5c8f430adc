// ibh_common.h -- shared device/host helpers for libibhip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ibhip.h"

// ── host-side error plumbing (ibh_runtime.hip) ─────────────────────────────
extern "C" void ibh_set_error(const char* fmt, ...);
hipStream_t ibh_resolve_stream(void* s);

#define IBH_CHECK_LAUNCH(what)                                                  \
    do {                                                                        \
        hipError_t e_ = hipGetLastError();                                      \
        if (e_ != hipSuccess) {                                                 \
            ibh_set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
            return IBH_ERROR_INTERNAL;                                          \
        }                                                                       \
    } while (0)

#define IBH_HIP(call, what)                                                     \
    do {                                                                        \
        hipError_t e_ = (call);                                                 \
        if (e_ != hipSuccess) {                                                 \
            ibh_set_error("%s: %s", what, hipGetErrorString(e_));               \
            return IBH_ERROR_INTERNAL;                                          \
        }                                                                       \
    } while (0)

// ── device helpers ─────────────────────────────────────────────────────────
namespace ibh {

constexpr int kWave = 64;

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);   // exact widening
}

template <int KIND>
__device__ __forceinline__ float load_scale(const void* s, int i) {
    if constexpr (KIND == IBH_SCALE_F16) return f16_to_f32(((const uint16_t*)s)[i]);
    else return ((const float*)s)[i];
}

// Butterfly sum over the 64 lanes of a wavefront (every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// 16-byte streaming load (weights are read exactly once per call).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Byte b of a dword as float (lowers to v_cvt_f32_ubyteN).
template <int B>
__device__ __forceinline__ float ubyte(uint32_t v) {
    return (float)((v >> (8 * B)) & 0xffu);
}

}  // namespace ibh
