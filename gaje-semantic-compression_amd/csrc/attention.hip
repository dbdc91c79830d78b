// GQA decode attention over the device KV cache (gfx950), bit-exact.
//
// Restates GenomicAttention::forward_attention_core (src/nn/attention.rs:87-127)
// with its rounding sequence for one query head h (kv head h / (n_head/n_head_kv)):
//   s_t   = dot_product(q_h, k_t) * (1/sqrt(hd))   eight FMA chains + the
//           dot.rs horizontal sum, then one rounded multiply;
//   max   = largest s_t ('>' over t; the order does not change a maximum);
//   e_t   = expf(s_t - max)                        glibc's expf (expf_ref.h);
//   sum   = e_0 + e_1 + ... in t order              one serial chain;
//   inv   = 1 / (sum + 1e-12);  w_t = e_t * inv;
//   out_i = sum over t of (w_t * v_t[i]) in t order, product and sum each rounded.
// The current token's k/v were appended by the fused QKV kernel, so the range
// 0..pos is the causal window.
//
// Cache layout: K is [kv head][position][dim] (a score reads one contiguous
// row); V is [kv head][dim][position] (an output dimension's chain reads one
// contiguous row).
//
// Scores, exponentials and products are computed in parallel over positions;
// the two serial chains (the softmax sum, and each output dimension's
// accumulation) run one lane per chain as the reference's loops do, reading
// LDS.  A chain is bound by its own length, so the parallel work is spread over
// several workgroups per head (one per slice of output dimensions) to keep the
// loads that feed the chains short.
#include "common.h"
#include "device_util.h"

namespace gaje {

namespace {

constexpr int THREADS = 256;

// dot_product(a, b) of dot.rs:43-67 for one thread: chains l = 0..7 over the
// 8-float chunks, ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)), then the scalar tail.
__device__ __forceinline__ float dot_ref(const float *a, const float *b, int n) {
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
    const int chunks = n / 8;
    for (int i = 0; i < chunks; ++i) {
        const float4 a0 = *(const float4 *)(a + 8 * i), a1 = *(const float4 *)(a + 8 * i + 4);
        const float4 b0 = *(const float4 *)(b + 8 * i), b1 = *(const float4 *)(b + 8 * i + 4);
        acc[0] = fmaf(a0.x, b0.x, acc[0]);
        acc[1] = fmaf(a0.y, b0.y, acc[1]);
        acc[2] = fmaf(a0.z, b0.z, acc[2]);
        acc[3] = fmaf(a0.w, b0.w, acc[3]);
        acc[4] = fmaf(a1.x, b1.x, acc[4]);
        acc[5] = fmaf(a1.y, b1.y, acc[5]);
        acc[6] = fmaf(a1.z, b1.z, acc[6]);
        acc[7] = fmaf(a1.w, b1.w, acc[7]);
    }
    const float u0 = acc[0] + acc[4], u1 = acc[1] + acc[5], u2 = acc[2] + acc[6], u3 = acc[3] + acc[7];
    float sum = (u0 + u1) + (u2 + u3);
    for (int i = chunks * 8; i < n; ++i) {
        const float prod = a[i] * b[i];
        sum = sum + prod;
    }
    return sum;
}

// The same dot product with the key row already in registers (HD % 8 == 0).
template <int HD>
__device__ __forceinline__ float dot_regs(const float *q, const float4 (&k)[HD / 4]) {
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
#pragma unroll
    for (int c = 0; c < HD / 8; ++c) {
        const float4 a0 = *(const float4 *)(q + 8 * c), a1 = *(const float4 *)(q + 8 * c + 4);
        const float4 b0 = k[2 * c], b1 = k[2 * c + 1];
        acc[0] = fmaf(a0.x, b0.x, acc[0]);
        acc[1] = fmaf(a0.y, b0.y, acc[1]);
        acc[2] = fmaf(a0.z, b0.z, acc[2]);
        acc[3] = fmaf(a0.w, b0.w, acc[3]);
        acc[4] = fmaf(a1.x, b1.x, acc[4]);
        acc[5] = fmaf(a1.y, b1.y, acc[5]);
        acc[6] = fmaf(a1.z, b1.z, acc[6]);
        acc[7] = fmaf(a1.w, b1.w, acc[7]);
    }
    const float u0 = acc[0] + acc[4], u1 = acc[1] + acc[5], u2 = acc[2] + acc[6], u3 = acc[3] + acc[7];
    return (u0 + u1) + (u2 + u3);
}

// Largest score over the block (every thread passes its own running max).
__device__ __forceinline__ float block_max(float mx, float *red) {
    const int tid = threadIdx.x;
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < THREADS / WAVE; ++w) m = fmaxf(m, red[w]);
    return m;
}

// e[0] + e[1] + ... + e[n-1] in order, one chain (called by one thread): the
// softmax denominator and every output dimension's accumulation.  LDS reads
// run one 32-float batch ahead of the adds.
__device__ __forceinline__ void add8(float &sum, const float4 (&v)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        sum = sum + v[u].x;
        sum = sum + v[u].y;
        sum = sum + v[u].z;
        sum = sum + v[u].w;
    }
}
__device__ __forceinline__ void read8(float4 (&v)[8], const float *e) {
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = *(const float4 *)(e + 4 * u);
}

__device__ __forceinline__ float serial_sum(const float *e, int n) {
    float sum = 0.0f;
    int t = 0;
    if (n >= 32) {
        float4 a[8], b[8];
        read8(a, e);
        while (true) {
            const bool more_b = t + 64 <= n;
            if (more_b) read8(b, e + t + 32);
            add8(sum, a);
            t += 32;
            if (!more_b) break;
            const bool more_a = t + 64 <= n;
            if (more_a) read8(a, e + t + 32);
            add8(sum, b);
            t += 32;
            if (!more_a) break;
        }
    }
    for (; t + 4 <= n; t += 4) {
        const float4 v = *(const float4 *)(e + t);
        sum = sum + v.x;
        sum = sum + v.y;
        sum = sum + v.z;
        sum = sum + v.w;
    }
    for (; t < n; ++t) sum = sum + e[t];
    return sum;
}

// Streaming kernel: head dimension HD known at compile time (64 or 128),
// capacity % 4 == 0.  Workgroup (h, slice) owns output dimensions
// [slice*ds, slice*ds + ds) of query head h: it computes all of the head's
// scores (parallel, one round of key loads per thread for contexts up to
// PPR * 256), and copies only its ds rows of V into LDS with LDS-direct loads
// issued first, so they land while the scores are computed and both serial
// chains read LDS only.
typedef __attribute__((address_space(3))) void lds_void;

template <int HD>
__global__ __launch_bounds__(THREADS) void attn_decode_fast(AttnParams p, int ds) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float red[THREADS / WAVE];
    __shared__ float inv_slot;
    DevState *st = p.st;
    if (st && st->halted) return;  // before any LDS-direct copy is in flight

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x;
    const int d0 = blockIdx.y * ds;
    const int g = h / (p.n_head / p.n_head_kv);
    const int ctx = st ? st->pos + 1 : (int)p.ctx;
    const float scale = 1.0f / sqrtf((float)HD);
    const int vstride = (int)p.kv_cap + 4;  // LDS row stride of the V slice (bank spread)

    float *qh = smem;           // HD floats
    float *sc = smem + HD;      // kv_cap scores, then exponentials
    float *vs = sc + p.kv_cap;  // ds rows of vstride: V, then the products
    const float *Kh = p.k_cache + (size_t)g * p.kv_head_stride;
    const float *Vh = p.v_cache + (size_t)g * p.kv_head_stride + (size_t)d0 * p.kv_cap;

    // ---- V slice -> LDS: one wave instruction copies 256 positions of a row
    // (lane i its quad i); quads at or past ctx are not copied, and a copied
    // quad ends before the row's capacity (kv_cap % 4 == 0) ----
    const int nchunk = (ctx + 255) >> 8;
    for (int c = wave; c < ds * nchunk; c += THREADS / WAVE) {
        const int j = c / nchunk, ch = c - j * nchunk;
        const int t = ch * 256 + lane * 4;
        if (t < ctx)
            __builtin_amdgcn_global_load_lds((const void *)(Vh + (size_t)j * p.kv_cap + t),
                                             (lds_void *)(vs + j * vstride + ch * 256), 16, 0, 0);
    }

    if (tid < HD) qh[tid] = p.q[(size_t)h * HD + tid];
    __syncthreads();

    // ---- scores: PPR positions per thread per round, key rows loaded first ----
    constexpr int PPR = HD <= 64 ? 3 : 1;
    float mx = -INFINITY;
    for (int t0 = tid; t0 < ctx; t0 += PPR * THREADS) {
        float4 k[PPR][HD / 4];
#pragma unroll
        for (int j = 0; j < PPR; ++j) {
            const int t = t0 + j * THREADS < ctx ? t0 + j * THREADS : t0;
            const float4 *kr = (const float4 *)(Kh + (size_t)t * HD);
#pragma unroll
            for (int u = 0; u < HD / 4; ++u) k[j][u] = kr[u];
        }
#pragma unroll
        for (int j = 0; j < PPR; ++j) {
            const int t = t0 + j * THREADS;
            if (t < ctx) {
                const float s = dot_regs<HD>(qh, k[j]) * scale;
                sc[t] = s;
                mx = fmaxf(mx, s);  // NaN never wins, as with the reference's '>'
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's LDS-direct copies have landed
    const float max_s = block_max(mx, red);  // (its barrier publishes them to the block)

    for (int t = tid; t < ctx; t += THREADS) sc[t] = expf_ref(sc[t] - max_s);
    __syncthreads();
    if (tid == 0) inv_slot = 1.0f / (serial_sum(sc, ctx) + 1e-12f);
    __syncthreads();
    const float inv = inv_slot;

    // products w_t * v_t[i] in place, w_t = e_t * inv rounded first
    for (int t = tid; t < ctx; t += THREADS) {
        const float w = sc[t] * inv;
        for (int j = 0; j < ds; ++j) {
            float &v = vs[j * vstride + t];
            v = w * v;
        }
    }
    __syncthreads();

    // ---- out_i = sum_t products, one chain per output dimension ----
    if (tid < ds) p.out[(size_t)h * HD + d0 + tid] = serial_sum(vs + tid * vstride, ctx);
}

// Output dimensions per workgroup of the streaming kernel for this capacity,
// or 0 if even one V row does not fit.
int fast_slice(int head_dim, int64_t cap) {
    for (int ds = 16; ds >= 1; ds >>= 1) {
        if (head_dim % ds) continue;
        const size_t lds = (size_t)(head_dim + cap + (size_t)ds * (cap + 4)) * 4;
        if (lds + 1024 <= max_lds_per_block()) return ds;
    }
    return 0;
}

// Any head_dim <= 256 with head_dim % 4 == 0 (and any capacity).
__global__ __launch_bounds__(THREADS) void attn_decode_generic(AttnParams p) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float red[THREADS / WAVE];
    __shared__ float inv_slot;
    DevState *st = p.st;
    if (st && st->halted) return;

    const int tid = threadIdx.x;
    const int h = blockIdx.x;
    const int hd = p.head_dim;
    const int g = h / (p.n_head / p.n_head_kv);
    const int ctx = st ? st->pos + 1 : (int)p.ctx;
    const float scale = 1.0f / sqrtf((float)hd);

    float *qh = smem;                            // hd floats (hd % 4 == 0)
    float *sc = smem + ((hd + 3) & ~3);          // ctx scores, then weights
    for (int i = tid; i < hd; i += THREADS) qh[i] = p.q[(size_t)h * hd + i];
    __syncthreads();

    const float *Kh = p.k_cache + (size_t)g * p.kv_head_stride;
    const float *Vh = p.v_cache + (size_t)g * p.kv_head_stride;

    float mx = -INFINITY;
    for (int t = tid; t < ctx; t += THREADS) {
        const float d = dot_ref(qh, Kh + (size_t)t * hd, hd);
        const float s = d * scale;
        sc[t] = s;
        mx = fmaxf(mx, s);
    }
    const float max_s = block_max(mx, red);

    for (int t = tid; t < ctx; t += THREADS) sc[t] = expf_ref(sc[t] - max_s);
    __syncthreads();
    if (tid == 0) inv_slot = 1.0f / (serial_sum(sc, ctx) + 1e-12f);
    __syncthreads();
    const float inv = inv_slot;
    for (int t = tid; t < ctx; t += THREADS) sc[t] = sc[t] * inv;
    __syncthreads();

    for (int i = tid; i < hd; i += THREADS) {
        float acc = 0.0f;
        const float *v = Vh + (size_t)i * p.kv_cap;
        for (int t = 0; t < ctx; ++t) {
            const float prod = sc[t] * v[t];
            acc = acc + prod;
        }
        p.out[(size_t)h * hd + i] = acc;
    }
}

}  // namespace

size_t attention_lds_bytes(int head_dim, int64_t max_ctx) {
    return (size_t)(((head_dim + 3) & ~3) + ((max_ctx + 3) & ~(int64_t)3)) * 4;
}

int launch_attention(const AttnParams &p, hipStream_t s) {
    if (!p.q || !p.k_cache || !p.v_cache || !p.out)
        return set_error(GAJE_ERR_INVALID_ARG, "attention: null buffer");
    if (p.kv_cap <= 0 || p.kv_head_stride != p.kv_cap * p.head_dim)
        return set_error(GAJE_ERR_INVALID_ARG, "attention: bad cache geometry");
    if (!p.st && (p.ctx <= 0 || p.ctx > p.kv_cap))
        return set_error(GAJE_ERR_INVALID_ARG, "attention: context %lld outside 1..%lld", (long long)p.ctx,
                         (long long)p.kv_cap);
    if (p.n_head_kv <= 0 || p.n_head % p.n_head_kv != 0)
        return set_error(GAJE_ERR_UNSUPPORTED, "attention: n_head %d / n_head_kv %d not supported", p.n_head,
                         p.n_head_kv);
    if (p.head_dim <= 0 || p.head_dim > THREADS || p.head_dim % 4 != 0)
        return set_error(GAJE_ERR_UNSUPPORTED, "attention: head_dim %d not supported (need <= 256, %% 4 == 0)",
                         p.head_dim);
    const size_t lds = attention_lds_bytes(p.head_dim, p.kv_cap);
    if (lds + 1024 > max_lds_per_block())
        return set_error(GAJE_ERR_UNSUPPORTED, "attention: context capacity %lld exceeds the LDS score buffer",
                         (long long)p.kv_cap);
    const int ds = (p.kv_cap % 4 == 0 && (p.head_dim == 64 || p.head_dim == 128)) ? fast_slice(p.head_dim, p.kv_cap) : 0;
    if (ds > 0) {
        const size_t flds = (size_t)(p.head_dim + p.kv_cap + (size_t)ds * (p.kv_cap + 4)) * 4;
        auto fn = p.head_dim == 64 ? attn_decode_fast<64> : attn_decode_fast<128>;
        hipLaunchKernelGGL(fn, dim3(p.n_head, p.head_dim / ds), dim3(THREADS), flds, s, p, ds);
    } else {
        hipLaunchKernelGGL(attn_decode_generic, dim3(p.n_head), dim3(THREADS), lds, s, p);
    }
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
