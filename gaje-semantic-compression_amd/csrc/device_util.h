// Device-side helpers shared by the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace gaje {

constexpr int WAVE = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// AND that instcombine cannot see through, so that byte-wise conversions of
// the masked nibbles stay v_cvt_f32_ubyte{0..3} instead of bitfield extracts.
__device__ __forceinline__ uint32_t opaque_and(uint32_t a, uint32_t m) {
    uint32_t r;
    asm volatile("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(m));
    return r;
}

__device__ __forceinline__ float ubyte0(uint32_t v) { return (float)(v & 0xFFu); }
__device__ __forceinline__ float ubyte1(uint32_t v) { return (float)((v >> 8) & 0xFFu); }
__device__ __forceinline__ float ubyte2(uint32_t v) { return (float)((v >> 16) & 0xFFu); }
__device__ __forceinline__ float ubyte3(uint32_t v) { return (float)(v >> 24); }

__device__ __forceinline__ float half_lo(uint32_t v) {
    union { uint16_t u; _Float16 h; } c;
    c.u = (uint16_t)(v & 0xFFFFu);
    return (float)c.h;
}
__device__ __forceinline__ float half_hi(uint32_t v) {
    union { uint16_t u; _Float16 h; } c;
    c.u = (uint16_t)(v >> 16);
    return (float)c.h;
}
__device__ __forceinline__ float half_bits(uint16_t v) {
    union { uint16_t u; _Float16 h; } c;
    c.u = v;
    return (float)c.h;
}

template <bool NT>
__device__ __forceinline__ uint32_t ld_u32(const void *p) {
    if constexpr (NT) return __builtin_nontemporal_load((const uint32_t *)p);
    else return *(const uint32_t *)p;
}

typedef float vf4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ float4 ld_f4(const float *p) {
    vf4 v;
    if constexpr (NT) v = __builtin_nontemporal_load((const vf4 *)p);
    else v = *(const vf4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}

// Orderable encoding of a float: a > b  <=>  key(a) > key(b) (NaN excluded).
__device__ __forceinline__ uint32_t order_key(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float order_key_inv(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(u);
}

// The reference's |t| < 1e-6 -> 0 flush of the 4-bit dots (genomic.rs:198-203,331-335).
__device__ __forceinline__ float flush_small(float t) { return fabsf(t) < 1e-6f ? 0.0f : t; }

__device__ __forceinline__ void nan_flag(DevState *st, int layer, int stage) {
    if (st && stage >= 0) atomicMin(&st->nan_code, (uint32_t)(layer * 8 + stage));
}

// swiglu_balanced for one element (activation.rs:40-49).
__device__ __forceinline__ float swiglu1(float g, float u) {
    float gs = g;
    if (gs < -64.0f) gs = -64.0f;
    if (gs > 64.0f) gs = 64.0f;
    float sig;
    if (gs >= 0.0f) {
        sig = 1.0f / (1.0f + expf(-gs));
    } else {
        float ex = expf(gs);
        sig = ex / (1.0f + ex);
    }
    return (g * sig) * u;
}

}  // namespace gaje
