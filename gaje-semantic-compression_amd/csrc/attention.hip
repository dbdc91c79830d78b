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
// 0..pos is the causal window.  One workgroup per query head: scores are
// computed in parallel over positions, the two serial chains (the sum and each
// output dimension's accumulation) run one lane per chain, as the reference's
// loops do; the scores live in LDS.
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

__global__ __launch_bounds__(THREADS) void attn_decode_kernel(AttnParams p) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float red[THREADS / WAVE];
    __shared__ float inv_slot;
    DevState *st = p.st;
    if (st && st->halted) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

    // scores and their maximum
    float mx = -INFINITY;
    for (int t = tid; t < ctx; t += THREADS) {
        const float d = dot_ref(qh, Kh + (size_t)t * hd, hd);
        const float s = d * scale;
        sc[t] = s;
        mx = fmaxf(mx, s);  // NaN never wins, as with the reference's '>'
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float max_s = red[0];
    for (int w = 1; w < THREADS / WAVE; ++w) max_s = fmaxf(max_s, red[w]);

    for (int t = tid; t < ctx; t += THREADS) sc[t] = expf_ref(sc[t] - max_s);
    __syncthreads();

    // sum_e in position order: a single chain
    if (tid == 0) {
        float sum = 0.0f;
        int t = 0;
        for (; t + 4 <= ctx; t += 4) {
            const float4 e = *(const float4 *)(sc + t);
            sum = sum + e.x;
            sum = sum + e.y;
            sum = sum + e.z;
            sum = sum + e.w;
        }
        for (; t < ctx; ++t) sum = sum + sc[t];
        inv_slot = 1.0f / (sum + 1e-12f);
    }
    __syncthreads();
    const float inv = inv_slot;
    for (int t = tid; t < ctx; t += THREADS) sc[t] = sc[t] * inv;
    __syncthreads();

    // out_i = sum_t w_t * v_t[i], one chain per output dimension
    for (int i = tid; i < hd; i += THREADS) {
        float acc = 0.0f;
        const float *v = Vh + i;
        int t = 0;
        for (; t + 4 <= ctx; t += 4) {
            const float4 w = *(const float4 *)(sc + t);
            const float v0 = v[(size_t)t * hd], v1 = v[(size_t)(t + 1) * hd], v2 = v[(size_t)(t + 2) * hd],
                        v3 = v[(size_t)(t + 3) * hd];
            const float p0 = w.x * v0, p1 = w.y * v1, p2 = w.z * v2, p3 = w.w * v3;
            acc = acc + p0;
            acc = acc + p1;
            acc = acc + p2;
            acc = acc + p3;
        }
        for (; t < ctx; ++t) {
            const float prod = sc[t] * v[(size_t)t * hd];
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
    if (!p.st && (p.ctx <= 0 || p.ctx > p.max_ctx))
        return set_error(GAJE_ERR_INVALID_ARG, "attention: context %lld outside 1..%lld", (long long)p.ctx,
                         (long long)p.max_ctx);
    if (p.n_head_kv <= 0 || p.n_head % p.n_head_kv != 0)
        return set_error(GAJE_ERR_UNSUPPORTED, "attention: n_head %d / n_head_kv %d not supported", p.n_head,
                         p.n_head_kv);
    if (p.head_dim <= 0 || p.head_dim > THREADS || p.head_dim % 4 != 0)
        return set_error(GAJE_ERR_UNSUPPORTED, "attention: head_dim %d not supported (need <= 256, %% 4 == 0)",
                         p.head_dim);
    const size_t lds = attention_lds_bytes(p.head_dim, p.max_ctx);
    if (lds + 1024 > 64 * 1024)
        return set_error(GAJE_ERR_UNSUPPORTED, "attention: context capacity %lld exceeds the LDS score buffer",
                         (long long)p.max_ctx);
    hipLaunchKernelGGL(attn_decode_kernel, dim3(p.n_head), dim3(THREADS), lds, s, p);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
