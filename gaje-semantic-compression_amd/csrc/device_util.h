// Device-side helpers shared by the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "expf_ref.h"
#include "kernels.h"

namespace gaje {

constexpr int WAVE = 64;

// Workgroup barrier that orders LDS only: unlike __syncthreads it does not wait
// for the wave's outstanding global loads (s_waitcnt lgkmcnt(0); s_barrier),
// so weight loads issued earlier stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// lds_barrier that also returns whether pred held in any thread of the block;
// slots: one int per wave in LDS, used by no other barrier_or in flight.
template <int NWAVES>
__device__ __forceinline__ bool barrier_or(int pred, int *slots) {
    const bool any = __any(pred);
    if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = any;
    lds_barrier();
    bool r = false;
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) r |= slots[w] != 0;
    return r;
}

// LDS byte address of a pointer into the workgroup's shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

// One wave instruction: each active lane copies the 16 bytes at g into LDS at
// lds + 16 * lane (lds is wave-uniform).  M0 is set inside the statement; the
// kernels that use it hold nothing else in M0 (checked in their assembly).
// The default is a streaming (non-temporal) read; TEMPORAL keeps the line in
// the caches for data that other workgroups read again.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <bool TEMPORAL = false>
__device__ __forceinline__ void lds_dma16(const void *g, uint32_t lds) {
    if constexpr (TEMPORAL)
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                     :
                     : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
                     : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                     :
                     : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
                     : "memory", "m0");
}
// The same copy addressed as a wave-uniform base (SGPR pair) plus a 32-bit
// per-lane byte offset: one VGPR per address instead of two.  base must be
// wave-uniform; it is moved to SGPRs with readfirstlane (a uniform value the
// compiler computed on the VALU is still in VGPRs).
__device__ __forceinline__ void lds_dma16_so(const void *base, uint32_t voff, uint32_t lds) {
    // (readfirstlane returns int: each half goes through uint32_t, or the low
    // half would sign-extend into the high one)
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint64_t bs = ((uint64_t)hi << 32) | lo;
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(bs), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}
// lds_dma16_so as a streaming (non-temporal) read.
__device__ __forceinline__ void lds_dma16_so_nt(const void *base, uint32_t voff, uint32_t lds) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint64_t bs = ((uint64_t)hi << 32) | lo;
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(voff), "s"(bs), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt for at most n outstanding vector memory operations (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

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
typedef uint32_t vu2 __attribute__((ext_vector_type(2)));
typedef uint32_t vu4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ vu2 ld_u2(const uint8_t *p) {
    if constexpr (NT) return __builtin_nontemporal_load((const vu2 *)p);
    else return *(const vu2 *)p;
}
template <bool NT>
__device__ __forceinline__ vu4 ld_u4(const uint8_t *p) {
    if constexpr (NT) return __builtin_nontemporal_load((const vu4 *)p);
    else return *(const vu4 *)p;
}

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
// Key of a logit for the first-maximum searches: -0 is taken as +0 first, so
// that the two zeros tie as they do under the reference's strict '>'
// (llm/forward.rs:262-271) and the lower index wins.
__device__ __forceinline__ uint32_t max_key(float f) { return order_key(f == 0.0f ? 0.0f : f); }
__device__ __forceinline__ float order_key_inv(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(u);
}

// The AVX2 reduction ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) of the eight chains
// held by lanes 8r..8r+7 (chain l in lane 8r + l), valid in lane 8r: three DPP
// row_shl adds (lane i reads lane i + n of its 16-lane row; the lanes whose
// sums are used read inside their own 8-lane group, and addition commutes).
__device__ __forceinline__ float red8_dpp(float a) {
    const float u = a + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), 0x104, 0xF, 0xF, false));
    const float v = u + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, u), 0x102, 0xF, 0xF, false));
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x101, 0xF, 0xF, false));
}

// x of lane i + 8 (of its 16-lane row): the second row of a pair whose
// reductions sit in lanes 16k and 16k + 8.
__device__ __forceinline__ float dpp_shl8(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x108, 0xF, 0xF, false));
}

// The reference's |t| < 1e-6 -> 0 flush of the 4-bit dots (genomic.rs:198-203,331-335).
__device__ __forceinline__ float flush_small(float t) { return fabsf(t) < 1e-6f ? 0.0f : t; }

// GenomicLinear::get_row_core (linear/forward.rs:195-285) element k of `row`
// for the embedding formats: F32 copy, Q4_0 / Q8_0 dequantize_weight from the
// packed rows, LUT-4bit table lookup (high nibble first), 2-bit centroid
// lookup; rows past rows_valid read as zeros.
__device__ __forceinline__ float embed_value(const EmbedParams &p, int64_t row, int64_t k) {
    const int64_t nb = p.K / 32;
    float v = 0.0f;
    if (row < p.rows_valid) {
        if (p.fmt == FMT_F32) {
            v = ((const float *)p.w)[row * p.K + k];
        } else if (k < nb * 32) {
            const int64_t b = k / 32;
            const int i = (int)(k % 32);
            if (p.fmt == FMT_Q8_0) {
                // packed rows (launch_pack_q8_0: tiles of 8 rows, per group of
                // four blocks the rows' 128 code bytes, then their 8 scale bytes):
                // dequantize_weight, q * scale (blocks.rs:43-49)
                const int64_t G = (nb + 3) / 4;
                const uint8_t *tile = p.w + (row >> 3) * G * 1088;
                const int k = (int)(row & 7), bb = (int)(b & 3), l = i & 7, c = i >> 3;
                const float q = (float)(int32_t)(int8_t)tile[(b / 4) * 1024 + 128 * k + 16 * l + 4 * bb + c];
                const uint8_t *sp = tile + G * 1024 + (b / 4) * 64 + 8 * k + 2 * bb;
                const uint16_t sh = (uint16_t)sp[0] | ((uint16_t)sp[1] << 8);
                v = __fmul_rn(q, half_bits(sh));
            } else if (p.fmt == FMT_Q4_0) {
                // packed rows (launch_pack_q4_0): element i of block b is
                // chain i % 8, chunk i / 8 of group b / 4
                const int64_t G = (nb + 3) / 4;
                const uint8_t *grp = p.w + (row * G + b / 4) * 80;
                const int bb = (int)(b & 3), l = i & 7, c = i >> 3;
                const uint32_t word = *(const uint32_t *)(grp + 8 * l + 4 * (bb >> 1));
                const float q = (float)((word >> (8 * c + 4 * (bb & 1))) & 0x0Fu);
                const uint32_t sm = *(const uint32_t *)(grp + 64 + 4 * bb);
                v = __fadd_rn(__fmul_rn(q, half_lo(sm)), half_hi(sm));
            } else if (p.fmt == FMT_G2) {
                // get_row_core on Genomic2Bit (linear/forward.rs:210-237): the
                // block's own four centroids where the table holds them, else
                // its first four; codes 00/01/11/10 -> c0/c1/c2/c3, MSB first
                // (dequantize_embedding_core, compute/quantize/dequantize.rs:6-42)
                int64_t off = 0;
                if (p.lut_block_stride) {
                    const int64_t own = (row * nb + b) * 4;
                    off = p.lut_rows_own == 0 ? b * 4 : own + 4 <= p.lut_len ? own : 0;
                }
                const float *c = p.lut + off;
                const uint8_t byte = p.w[(row * nb + b) * 8 + i / 4];
                const int bits = (byte >> ((3 - (i & 3)) * 2)) & 3;
                v = bits == 0 ? c[0] : bits == 1 ? c[1] : bits == 3 ? c[2] : c[3];
            } else {
                const float *t = p.lut + (row < p.lut_rows_own ? row * nb * 16 : 0) + b * p.lut_block_stride;
                const uint8_t byte = p.w[(row * nb + b) * 16 + i / 2];
                v = t[(i % 2 == 0) ? (byte >> 4) : (byte & 0x0F)];
            }
        }
    }
    return v;
}

__device__ __forceinline__ void nan_flag(DevState *st, int layer, int stage) {
    if (st && stage >= 0) atomicMin(&st->nan_code, (uint32_t)(layer * 8 + stage));
}

// swiglu_balanced for one element (activation.rs:40-49), with the reference's
// exponential (expf_ref; tab is its table, kExp2Tab or an LDS copy) and every
// operation rounded as written there.
__device__ __forceinline__ float swiglu1(float g, float u, const uint64_t *tab = kExp2Tab) {
    float gs = g;
    if (gs < -64.0f) gs = -64.0f;
    if (gs > 64.0f) gs = 64.0f;
    float sig;
    if (gs >= 0.0f) {
        const float den = 1.0f + expf_ref_t(-gs, tab);
        sig = 1.0f / den;
    } else {
        const float ex = expf_ref_t(gs, tab);
        const float den = 1.0f + ex;
        sig = ex / den;
    }
    const float silu = g * sig;
    return silu * u;
}

// sum + e[0] + e[1] + ... + e[n - 1] in order in this lane (the reference's
// serial accumulation loops), n % 64 == 0 and n >= 64; e is an LDS array that
// is read 32 floats past its end (the values are not used).  The loop is
// written out because the compiler's schedule waits for every LDS read before
// each block of adds: here the reads run one block of 32 values ahead, with one
// wait per block, and v100..v163 hold the two blocks.  Uniform n.
__device__ __forceinline__ float chain_lds(float sum, const float *e, int n) {
    uint32_t p = (uint32_t)(uintptr_t)e;
    int c = __builtin_amdgcn_readfirstlane(n >> 6);  // uniform: lives in an SGPR
    asm volatile(
        "ds_read_b128 v[100:103], %[p] offset:0\n"
        "ds_read_b128 v[104:107], %[p] offset:16\n"
        "ds_read_b128 v[108:111], %[p] offset:32\n"
        "ds_read_b128 v[112:115], %[p] offset:48\n"
        "ds_read_b128 v[116:119], %[p] offset:64\n"
        "ds_read_b128 v[120:123], %[p] offset:80\n"
        "ds_read_b128 v[124:127], %[p] offset:96\n"
        "ds_read_b128 v[128:131], %[p] offset:112\n"
        "1:\n"
        "ds_read_b128 v[132:135], %[p] offset:128\n"
        "ds_read_b128 v[136:139], %[p] offset:144\n"
        "ds_read_b128 v[140:143], %[p] offset:160\n"
        "ds_read_b128 v[144:147], %[p] offset:176\n"
        "ds_read_b128 v[148:151], %[p] offset:192\n"
        "ds_read_b128 v[152:155], %[p] offset:208\n"
        "ds_read_b128 v[156:159], %[p] offset:224\n"
        "ds_read_b128 v[160:163], %[p] offset:240\n"
        "s_waitcnt lgkmcnt(8)\n"
        "v_add_f32 %[s], %[s], v100\n"
        "v_add_f32 %[s], %[s], v101\n"
        "v_add_f32 %[s], %[s], v102\n"
        "v_add_f32 %[s], %[s], v103\n"
        "v_add_f32 %[s], %[s], v104\n"
        "v_add_f32 %[s], %[s], v105\n"
        "v_add_f32 %[s], %[s], v106\n"
        "v_add_f32 %[s], %[s], v107\n"
        "v_add_f32 %[s], %[s], v108\n"
        "v_add_f32 %[s], %[s], v109\n"
        "v_add_f32 %[s], %[s], v110\n"
        "v_add_f32 %[s], %[s], v111\n"
        "v_add_f32 %[s], %[s], v112\n"
        "v_add_f32 %[s], %[s], v113\n"
        "v_add_f32 %[s], %[s], v114\n"
        "v_add_f32 %[s], %[s], v115\n"
        "v_add_f32 %[s], %[s], v116\n"
        "v_add_f32 %[s], %[s], v117\n"
        "v_add_f32 %[s], %[s], v118\n"
        "v_add_f32 %[s], %[s], v119\n"
        "v_add_f32 %[s], %[s], v120\n"
        "v_add_f32 %[s], %[s], v121\n"
        "v_add_f32 %[s], %[s], v122\n"
        "v_add_f32 %[s], %[s], v123\n"
        "v_add_f32 %[s], %[s], v124\n"
        "v_add_f32 %[s], %[s], v125\n"
        "v_add_f32 %[s], %[s], v126\n"
        "v_add_f32 %[s], %[s], v127\n"
        "v_add_f32 %[s], %[s], v128\n"
        "v_add_f32 %[s], %[s], v129\n"
        "v_add_f32 %[s], %[s], v130\n"
        "v_add_f32 %[s], %[s], v131\n"
        "ds_read_b128 v[100:103], %[p] offset:256\n"
        "ds_read_b128 v[104:107], %[p] offset:272\n"
        "ds_read_b128 v[108:111], %[p] offset:288\n"
        "ds_read_b128 v[112:115], %[p] offset:304\n"
        "ds_read_b128 v[116:119], %[p] offset:320\n"
        "ds_read_b128 v[120:123], %[p] offset:336\n"
        "ds_read_b128 v[124:127], %[p] offset:352\n"
        "ds_read_b128 v[128:131], %[p] offset:368\n"
        "s_waitcnt lgkmcnt(8)\n"
        "v_add_f32 %[s], %[s], v132\n"
        "v_add_f32 %[s], %[s], v133\n"
        "v_add_f32 %[s], %[s], v134\n"
        "v_add_f32 %[s], %[s], v135\n"
        "v_add_f32 %[s], %[s], v136\n"
        "v_add_f32 %[s], %[s], v137\n"
        "v_add_f32 %[s], %[s], v138\n"
        "v_add_f32 %[s], %[s], v139\n"
        "v_add_f32 %[s], %[s], v140\n"
        "v_add_f32 %[s], %[s], v141\n"
        "v_add_f32 %[s], %[s], v142\n"
        "v_add_f32 %[s], %[s], v143\n"
        "v_add_f32 %[s], %[s], v144\n"
        "v_add_f32 %[s], %[s], v145\n"
        "v_add_f32 %[s], %[s], v146\n"
        "v_add_f32 %[s], %[s], v147\n"
        "v_add_f32 %[s], %[s], v148\n"
        "v_add_f32 %[s], %[s], v149\n"
        "v_add_f32 %[s], %[s], v150\n"
        "v_add_f32 %[s], %[s], v151\n"
        "v_add_f32 %[s], %[s], v152\n"
        "v_add_f32 %[s], %[s], v153\n"
        "v_add_f32 %[s], %[s], v154\n"
        "v_add_f32 %[s], %[s], v155\n"
        "v_add_f32 %[s], %[s], v156\n"
        "v_add_f32 %[s], %[s], v157\n"
        "v_add_f32 %[s], %[s], v158\n"
        "v_add_f32 %[s], %[s], v159\n"
        "v_add_f32 %[s], %[s], v160\n"
        "v_add_f32 %[s], %[s], v161\n"
        "v_add_f32 %[s], %[s], v162\n"
        "v_add_f32 %[s], %[s], v163\n"
        "v_add_u32 %[p], 256, %[p]\n"
        "s_sub_i32 %[c], %[c], 1\n"
        "s_cmp_gt_i32 %[c], 0\n"
        "s_cbranch_scc1 1b\n"
        "s_waitcnt lgkmcnt(0)\n"
        : [s] "+v"(sum), [p] "+v"(p), [c] "+s"(c)
        :
        : "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111", "v112", "v113", "v114", "v115",
          "v116", "v117", "v118", "v119", "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127", "v128", "v129", "v130", "v131",
          "v132", "v133", "v134", "v135", "v136", "v137", "v138", "v139", "v140", "v141", "v142", "v143", "v144", "v145", "v146", "v147",
          "v148", "v149", "v150", "v151", "v152", "v153", "v154", "v155", "v156", "v157", "v158", "v159", "v160", "v161", "v162", "v163", "scc", "memory");
    return sum;
}

// fma(e[i], e[i], acc) for i = 0..n-1 in order in this lane (the sum-of-squares
// chain of rms_norm), with the same loop, limits and read-ahead as chain_lds.
__device__ __forceinline__ float chain_lds_sq(float acc, const float *e, int n) {
    uint32_t p = (uint32_t)(uintptr_t)e;
    int c = __builtin_amdgcn_readfirstlane(n >> 6);  // uniform: lives in an SGPR
    asm volatile(
        "ds_read_b128 v[100:103], %[p] offset:0\n"
        "ds_read_b128 v[104:107], %[p] offset:16\n"
        "ds_read_b128 v[108:111], %[p] offset:32\n"
        "ds_read_b128 v[112:115], %[p] offset:48\n"
        "ds_read_b128 v[116:119], %[p] offset:64\n"
        "ds_read_b128 v[120:123], %[p] offset:80\n"
        "ds_read_b128 v[124:127], %[p] offset:96\n"
        "ds_read_b128 v[128:131], %[p] offset:112\n"
        "1:\n"
        "ds_read_b128 v[132:135], %[p] offset:128\n"
        "ds_read_b128 v[136:139], %[p] offset:144\n"
        "ds_read_b128 v[140:143], %[p] offset:160\n"
        "ds_read_b128 v[144:147], %[p] offset:176\n"
        "ds_read_b128 v[148:151], %[p] offset:192\n"
        "ds_read_b128 v[152:155], %[p] offset:208\n"
        "ds_read_b128 v[156:159], %[p] offset:224\n"
        "ds_read_b128 v[160:163], %[p] offset:240\n"
        "s_waitcnt lgkmcnt(8)\n"
        "v_fmac_f32 %[s], v100, v100\n"
        "v_fmac_f32 %[s], v101, v101\n"
        "v_fmac_f32 %[s], v102, v102\n"
        "v_fmac_f32 %[s], v103, v103\n"
        "v_fmac_f32 %[s], v104, v104\n"
        "v_fmac_f32 %[s], v105, v105\n"
        "v_fmac_f32 %[s], v106, v106\n"
        "v_fmac_f32 %[s], v107, v107\n"
        "v_fmac_f32 %[s], v108, v108\n"
        "v_fmac_f32 %[s], v109, v109\n"
        "v_fmac_f32 %[s], v110, v110\n"
        "v_fmac_f32 %[s], v111, v111\n"
        "v_fmac_f32 %[s], v112, v112\n"
        "v_fmac_f32 %[s], v113, v113\n"
        "v_fmac_f32 %[s], v114, v114\n"
        "v_fmac_f32 %[s], v115, v115\n"
        "v_fmac_f32 %[s], v116, v116\n"
        "v_fmac_f32 %[s], v117, v117\n"
        "v_fmac_f32 %[s], v118, v118\n"
        "v_fmac_f32 %[s], v119, v119\n"
        "v_fmac_f32 %[s], v120, v120\n"
        "v_fmac_f32 %[s], v121, v121\n"
        "v_fmac_f32 %[s], v122, v122\n"
        "v_fmac_f32 %[s], v123, v123\n"
        "v_fmac_f32 %[s], v124, v124\n"
        "v_fmac_f32 %[s], v125, v125\n"
        "v_fmac_f32 %[s], v126, v126\n"
        "v_fmac_f32 %[s], v127, v127\n"
        "v_fmac_f32 %[s], v128, v128\n"
        "v_fmac_f32 %[s], v129, v129\n"
        "v_fmac_f32 %[s], v130, v130\n"
        "v_fmac_f32 %[s], v131, v131\n"
        "ds_read_b128 v[100:103], %[p] offset:256\n"
        "ds_read_b128 v[104:107], %[p] offset:272\n"
        "ds_read_b128 v[108:111], %[p] offset:288\n"
        "ds_read_b128 v[112:115], %[p] offset:304\n"
        "ds_read_b128 v[116:119], %[p] offset:320\n"
        "ds_read_b128 v[120:123], %[p] offset:336\n"
        "ds_read_b128 v[124:127], %[p] offset:352\n"
        "ds_read_b128 v[128:131], %[p] offset:368\n"
        "s_waitcnt lgkmcnt(8)\n"
        "v_fmac_f32 %[s], v132, v132\n"
        "v_fmac_f32 %[s], v133, v133\n"
        "v_fmac_f32 %[s], v134, v134\n"
        "v_fmac_f32 %[s], v135, v135\n"
        "v_fmac_f32 %[s], v136, v136\n"
        "v_fmac_f32 %[s], v137, v137\n"
        "v_fmac_f32 %[s], v138, v138\n"
        "v_fmac_f32 %[s], v139, v139\n"
        "v_fmac_f32 %[s], v140, v140\n"
        "v_fmac_f32 %[s], v141, v141\n"
        "v_fmac_f32 %[s], v142, v142\n"
        "v_fmac_f32 %[s], v143, v143\n"
        "v_fmac_f32 %[s], v144, v144\n"
        "v_fmac_f32 %[s], v145, v145\n"
        "v_fmac_f32 %[s], v146, v146\n"
        "v_fmac_f32 %[s], v147, v147\n"
        "v_fmac_f32 %[s], v148, v148\n"
        "v_fmac_f32 %[s], v149, v149\n"
        "v_fmac_f32 %[s], v150, v150\n"
        "v_fmac_f32 %[s], v151, v151\n"
        "v_fmac_f32 %[s], v152, v152\n"
        "v_fmac_f32 %[s], v153, v153\n"
        "v_fmac_f32 %[s], v154, v154\n"
        "v_fmac_f32 %[s], v155, v155\n"
        "v_fmac_f32 %[s], v156, v156\n"
        "v_fmac_f32 %[s], v157, v157\n"
        "v_fmac_f32 %[s], v158, v158\n"
        "v_fmac_f32 %[s], v159, v159\n"
        "v_fmac_f32 %[s], v160, v160\n"
        "v_fmac_f32 %[s], v161, v161\n"
        "v_fmac_f32 %[s], v162, v162\n"
        "v_fmac_f32 %[s], v163, v163\n"
        "v_add_u32 %[p], 256, %[p]\n"
        "s_sub_i32 %[c], %[c], 1\n"
        "s_cmp_gt_i32 %[c], 0\n"
        "s_cbranch_scc1 1b\n"
        "s_waitcnt lgkmcnt(0)\n"
        : [s] "+v"(acc), [p] "+v"(p), [c] "+s"(c)
        :
        : "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111", "v112", "v113", "v114", "v115",
          "v116", "v117", "v118", "v119", "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127", "v128", "v129", "v130", "v131",
          "v132", "v133", "v134", "v135", "v136", "v137", "v138", "v139", "v140", "v141", "v142", "v143", "v144", "v145", "v146", "v147",
          "v148", "v149", "v150", "v151", "v152", "v153", "v154", "v155", "v156", "v157", "v158", "v159", "v160", "v161", "v162", "v163", "scc", "memory");
    return acc;
}

// rms_norm's 1/rms of xs[0..n) (norm.rs:52-88): sum of squares in eight FMA
// chains over 8-float chunks, reduced ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)),
// scalar tail, inv = 1/sqrt(ss/n + eps), stored by thread 0 in *inv_slot.
// Threads 0..7 of the block compute it; the caller synchronises.
__device__ inline void rms_inv_plain(const float *xs, int64_t n, float eps, float *inv_slot) {
    const int tid = threadIdx.x;
    if (tid >= 8) return;
    float acc = 0.0f;
    const int64_t chunks = n / 8;
    int64_t i = 0;
    for (; i + 8 <= chunks; i += 8) {  // eight LDS reads in flight, then the chain
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = xs[8 * (i + u) + tid];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = fmaf(v[u], v[u], acc);
    }
    for (; i < chunks; ++i) {
        const float v = xs[8 * i + tid];
        acc = fmaf(v, v, acc);
    }
    const float u = acc + __shfl(acc, (tid + 4) & 7, 8);  // lane l<4: a_l + a_{l+4}
    const float v = u + __shfl(u, (tid + 1) & 7, 8);      // lane 0: u0+u1, lane 2: u2+u3
    const float tot = v + __shfl(v, (tid + 2) & 7, 8);    // lane 0: (u0+u1) + (u2+u3)
    if (tid == 0) {
        float ss = tot;
        for (int64_t k = chunks * 8; k < n; ++k) {
            const float sq = xs[k] * xs[k];
            ss = ss + sq;
        }
        const float mean = ss / (float)n;
        *inv_slot = 1.0f / sqrtf(mean + eps);
    }
}

// rms_norm of xs[0..n) in place: out = (x * inv) * w, each product rounded.
// Called by every thread of the block (it contains a barrier).
__device__ inline void rmsnorm_inplace(float *xs, int64_t n, const float *w, float eps, float *inv_slot) {
    rms_inv_plain(xs, n, eps, inv_slot);
    __syncthreads();
    const float inv = *inv_slot;
    for (int64_t k = threadIdx.x; k < n; k += blockDim.x) {
        const float t = xs[k] * inv;
        xs[k] = t * w[k];
    }
}

// lateral_inhibition_kwta (compute/kernels/lut.rs:45-61) over the n floats at
// xs (LDS, 16-byte aligned, n % 4 == 0) by one wave: thr = the k-th largest
// value, found as kwta_kernel finds it (order_key, 8-bit passes from the top
// byte, each pass's 256-bin histogram of the keys that match the prefix chosen
// so far, the bin that holds the rank-th largest key taken from a scan in
// descending bin order), then x < thr -> -1e9 in place.  Rows of up to
// 64 * 4 * KW_WQ values keep their keys in registers (read once, with 16-byte
// reads) and count them without branches; once the chosen bin holds a single
// key, that key is the threshold and the remaining passes are skipped.
// Longer rows re-read the keys from LDS each pass.  hist: 4 x 320 words (a
// histogram per pass, and dummy words).  Returns thr (-inf, masking nothing,
// when n <= k or k <= 0).  LDS operations of one wave complete in issue order;
// the explicit waits only keep the compiler from moving them across phases.
constexpr int KW_WQ = 6;  // quads of keys per lane held in registers (n <= 1536)

// Inclusive prefix sum over the 64 lanes of a wave with DPP: row_shr 1, 2, 4, 8
// within each row of 16 lanes (lanes with no source add 0), then row_bcast:15
// (lane 15 of a row into the next row) and row_bcast:31 (lane 31 into rows 2
// and 3).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, true);  // row_shr:1
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, true);  // row_shr:2
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, true);  // row_shr:4
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, true);  // row_shr:8
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xA, 0xF, false); // row_bcast:15
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xC, 0xF, false); // row_bcast:31
    return x;
}

// wave_kwta for rows past the register budget: the keys re-read from LDS each
// pass.
__device__ __forceinline__ float wave_kwta_long(float *xs, int n, int64_t k, uint32_t *hist, int lane) {
    constexpr int HS = 256 + WAVE;
    uint32_t prefix = 0u, mask = 0u, rank = (uint32_t)k;
#pragma unroll
    for (int z = 0; z < 4; ++z) *(uint4 *)(hist + HS * z + 4 * lane) = make_uint4(0u, 0u, 0u, 0u);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        uint32_t *h = hist + HS * pass;
        for (int i = lane; i < n; i += WAVE) {
            const uint32_t kk = order_key(xs[i]);
            if ((kk & mask) == prefix) atomicAdd(&h[(kk >> shift) & 255u], 1u);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const uint4 hv = *(const uint4 *)(h + 252 - 4 * lane);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const uint32_t v0 = hv.w, v1 = hv.z, v2 = hv.y, v3 = hv.x;
        const uint32_t t = v0 + v1 + v2 + v3;
        const uint32_t incl = wave_incl_scan(t);
        const uint32_t e0 = incl - t, c0 = e0 + v0, c1 = c0 + v1, c2 = c1 + v2;
        const int src = __ffsll((long long)__ballot(e0 < rank && incl >= rank)) - 1;
        const int jl = c0 >= rank ? 0 : c1 >= rank ? 1 : c2 >= rank ? 2 : 3;
        const uint32_t bl = c0 >= rank ? e0 : c1 >= rank ? c0 : c2 >= rank ? c1 : c2;
        prefix |= (uint32_t)(255 - (4 * src + __builtin_amdgcn_readlane(jl, src))) << shift;
        mask |= 255u << shift;
        rank -= (uint32_t)__builtin_amdgcn_readlane((int)bl, src);
    }
    const float thr = order_key_inv(prefix);
    for (int i = lane; i < n; i += WAVE)
        if (xs[i] < thr) xs[i] = -1e9f;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    return thr;
}

__device__ __forceinline__ float wave_kwta(float *xs, int n, int64_t k, uint32_t *hist, int lane) {
    if ((int64_t)n <= k || k <= 0) return -INFINITY;
    constexpr int HS = 256 + WAVE;  // a pass's bins, then one dummy word per lane
    const int n4 = n >> 2;
    if (n4 > WAVE * KW_WQ) return wave_kwta_long(xs, n, k, hist, lane);
    const int jn = (n4 + WAVE - 1) / WAVE;  // quads per lane (uniform)
    uint32_t key[KW_WQ][4];
    bool ok[KW_WQ];
#pragma unroll
    for (int j = 0; j < KW_WQ; ++j) {
        const int q = lane + WAVE * j;
        ok[j] = q < n4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j < jn) v = *(const float4 *)(xs + 4 * (ok[j] ? q : 0));
        key[j][0] = order_key(v.x);
        key[j][1] = order_key(v.y);
        key[j][2] = order_key(v.z);
        key[j][3] = order_key(v.w);
    }
#pragma unroll
    for (int z = 0; z < 4; ++z) *(uint4 *)(hist + HS * z + 4 * lane) = make_uint4(0u, 0u, 0u, 0u);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    uint32_t prefix = 0u, mask = 0u, rank = (uint32_t)k;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        uint32_t *h = hist + HS * pass;
        // every key adds once, without branches: a key outside the prefix (or
        // past n) into its lane's dummy word
#pragma unroll
        for (int j = 0; j < KW_WQ; ++j) {
            if (j < jn) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const bool m = ok[j] && (key[j][c] & mask) == prefix;
                    atomicAdd(&h[m ? ((key[j][c] >> shift) & 255u) : 256u + lane], 1u);
                }
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // lane L holds bins 255 - 4L .. 252 - 4L, in that (descending) order
        const uint4 hv = *(const uint4 *)(h + 252 - 4 * lane);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const uint32_t v0 = hv.w, v1 = hv.z, v2 = hv.y, v3 = hv.x;
        const uint32_t t = v0 + v1 + v2 + v3;
        const uint32_t incl = wave_incl_scan(t);
        const uint32_t e0 = incl - t, c0 = e0 + v0, c1 = c0 + v1, c2 = c1 + v2;
        // the lane whose bins' range of ranks (e0, incl] holds rank (exactly
        // one: the counts sum to at least rank), and in it the bin
        const int src = __ffsll((long long)__ballot(e0 < rank && incl >= rank)) - 1;
        const int jl = c0 >= rank ? 0 : c1 >= rank ? 1 : c2 >= rank ? 2 : 3;
        const uint32_t bl = c0 >= rank ? e0 : c1 >= rank ? c0 : c2 >= rank ? c1 : c2;
        const uint32_t vl = c0 >= rank ? v0 : c1 >= rank ? v1 : c2 >= rank ? v2 : v3;
        const int jj = __builtin_amdgcn_readlane(jl, src);
        const uint32_t bb = (uint32_t)__builtin_amdgcn_readlane((int)bl, src);
        const uint32_t cnt = (uint32_t)__builtin_amdgcn_readlane((int)vl, src);
        prefix |= (uint32_t)(255 - (4 * src + jj)) << shift;
        mask |= 255u << shift;
        rank -= bb;
        if (cnt == 1u && pass < 3) {
            // one key has this prefix: it is the k-th largest
            uint32_t lo = 0u;
            bool any = false;
#pragma unroll
            for (int j = 0; j < KW_WQ; ++j) {
                if (j < jn) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const bool m = ok[j] && (key[j][c] & mask) == prefix;
                        lo |= m ? key[j][c] : 0u;
                        any |= m;
                    }
                }
            }
            prefix = (uint32_t)__builtin_amdgcn_readlane((int)lo, __ffsll((long long)__ballot(any)) - 1);
            break;
        }
    }
    const float thr = order_key_inv(prefix);
    // order_key is a bijection on the bit patterns: its inverse gives x back
#pragma unroll
    for (int j = 0; j < KW_WQ; ++j) {
        if (j < jn && ok[j]) {
            float m4[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float x = order_key_inv(key[j][c]);
                m4[c] = x < thr ? -1e9f : x;
            }
            *(float4 *)(xs + 4 * (lane + WAVE * j)) = make_float4(m4[0], m4[1], m4[2], m4[3]);
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    return thr;
}

}  // namespace gaje
