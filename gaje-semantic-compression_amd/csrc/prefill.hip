// Prompt prefill pieces between the MFMA matrix products: RoPE with the
// KV-cache append for a batch of positions, and causal GQA attention of a
// batch of queries over the cache.
//
// The reference feeds a prompt one token at a time through forward_core
// (llm/forward.rs:229-232), so token t attends to positions 0..t; here a
// chunk of P tokens at positions pos0..pos0+P-1 is processed at once with the
// same causal extent per query.
#include <hip/hip_runtime.h>

#include "common.h"
#include "device_util.h"
#include "kernels.h"

namespace gaje {
namespace {

// RoPE of GenomicAttention::forward_attention_core (attention.rs:56-84) on the
// q and k rows of each token, from the host-built table of the decode path,
// each product rounded as in the decode epilogue; k and v appended to the
// cache at the token's position.  One workgroup per token.
__global__ __launch_bounds__(256) void rope_kv_kernel(PrefillRopeParams p) {
    const int64_t t = blockIdx.x;
    int64_t pos = p.pos0 + t;
    if (p.seq_pos) {
        pos = p.seq_pos[t];
        if (pos < 0) return;
        p.k_cache += t * p.seq_kv_stride;
        p.v_cache += t * p.seq_kv_stride;
    }
    const float *row = p.qkv + t * p.ldq;
    const int hd = p.head_dim, half = hd >> 1;
    const int64_t q_rows = (int64_t)p.n_head * hd, kv_rows = (int64_t)p.n_kv * hd;
    const int64_t pairs = (int64_t)(p.n_head + p.n_kv) * half;
    for (int64_t pr = threadIdx.x; pr < pairs; pr += blockDim.x) {
        const int64_t head = pr / half;
        const int i = (int)(pr - head * half);
        const int d0 = p.rope_split ? i : 2 * i;
        const int d1 = p.rope_split ? i + half : 2 * i + 1;
        const float y0 = row[head * hd + d0], y1 = row[head * hd + d1];
        const float cs = p.rope_cos[pos * half + i], sn = p.rope_sin[pos * half + i];
        const float t0 = y0 * cs, t1 = y1 * sn, t2 = y0 * sn, t3 = y1 * cs;
        const float o0 = t0 - t1, o1 = t2 + t3;
        if (head < p.n_head) {
            p.q_out[t * q_rows + head * hd + d0] = o0;
            p.q_out[t * q_rows + head * hd + d1] = o1;
        } else {
            float *kc = p.k_cache + (head - p.n_head) * hd * p.cap + pos;
            kc[(int64_t)d0 * p.cap] = o0;
            kc[(int64_t)d1 * p.cap] = o1;
        }
    }
    for (int64_t j = threadIdx.x; j < kv_rows; j += blockDim.x) {
        const int64_t vh = j / hd, d = j - vh * hd;
        p.v_cache[(vh * hd + d) * p.cap + pos] = row[q_rows + kv_rows + j];
    }
}

// One workgroup per (query token, KV head), serving the GQA group's query
// heads h = g*G .. g*G+G-1 (kv head h / (n_head / n_head_kv), attention.rs:91)
// so each key and value row is read once per group: scores against positions
// 0..pos0+t scaled by 1/sqrt(head_dim); softmax exp(s - max) with the
// reference's exponential and 1/(sum + 1e-12); out = sum_j (e_j * inv) v_j
// (attention.rs:87-127).  The summation orders are not the reference's serial
// ones (fp32 accuracy, not bit-exact).  Scores live in LDS ([G][ctx]); in the
// P.V product each of the 8 waves owns HD/8 output dimensions of every group
// head, its lanes striding over positions (coalesced V rows).
template <int HD, int G>
__global__ __launch_bounds__(512) void prefill_attn_kernel(PrefillAttnParams p) {
    extern __shared__ __align__(16) float sc[];
    __shared__ float qs[G][HD];
    __shared__ float red[8];
    __shared__ float stat[G][2];
    const int64_t t = blockIdx.x;
    const int g = blockIdx.y;
    const int64_t ctx = p.pos0 + t + 1;
    const int64_t stride = (ctx + 3) & ~3;  // score row stride
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t q_rows = (int64_t)p.n_head * HD;
    for (int i = tid; i < G * HD; i += 512) qs[i / HD][i % HD] = p.q[t * q_rows + ((int64_t)g * G) * HD + i];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    const float *kb = p.k_cache + (int64_t)g * HD * p.cap;
    float mx[G];
#pragma unroll
    for (int h = 0; h < G; ++h) mx[h] = -INFINITY;
    for (int64_t j = tid; j < ctx; j += 512) {
        float s[G];
#pragma unroll
        for (int h = 0; h < G; ++h) s[h] = 0.0f;
#pragma unroll 4
        for (int d = 0; d < HD; ++d) {
            const float kv = kb[(int64_t)d * p.cap + j];
#pragma unroll
            for (int h = 0; h < G; ++h) s[h] = fmaf(qs[h][d], kv, s[h]);
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float v = s[h] * scale;
            sc[h * stride + j] = v;
            mx[h] = fmaxf(mx[h], v);
        }
    }
    // per head: max, then exp and sum
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float v = wave_max(mx[h]);
        __syncthreads();
        if (lane == 0) red[wave] = v;
        __syncthreads();
        if (tid == 0) {
            float r = red[0];
            for (int w = 1; w < 8; ++w) r = fmaxf(r, red[w]);
            stat[h][0] = r;
        }
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float m = stat[h][0];
        float sum = 0.0f;
        for (int64_t j = tid; j < ctx; j += 512) {
            const float e = expf_ref(sc[h * stride + j] - m);
            sc[h * stride + j] = e;
            sum += e;
        }
        sum = wave_sum(sum);
        __syncthreads();
        if (lane == 0) red[wave] = sum;
        __syncthreads();
        if (tid == 0) {
            float r = red[0];
            for (int w = 1; w < 8; ++w) r += red[w];
            stat[h][1] = 1.0f / (r + 1e-12f);
        }
    }
    __syncthreads();
    constexpr int NA = HD / 8;
    const float *vb = p.v_cache + ((int64_t)g * HD + wave * NA) * p.cap;
    float acc[G][NA];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int a = 0; a < NA; ++a) acc[h][a] = 0.0f;
    float inv[G];
#pragma unroll
    for (int h = 0; h < G; ++h) inv[h] = stat[h][1];
    for (int64_t j = lane; j < ctx; j += 64) {
        float w[G];
#pragma unroll
        for (int h = 0; h < G; ++h) w[h] = sc[h * stride + j] * inv[h];
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const float v = vb[(int64_t)a * p.cap + j];
#pragma unroll
            for (int h = 0; h < G; ++h) acc[h][a] = fmaf(w[h], v, acc[h][a]);
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float *o = p.out + t * q_rows + ((int64_t)g * G + h) * HD + wave * NA;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const float v = wave_sum(acc[h][a]);
            if (lane == 0) o[a] = v;
        }
    }
}

template <int HD>
int launch_attn_hd(const PrefillAttnParams &p, hipStream_t s) {
    const int G = p.n_head / p.n_kv;
    const size_t lds = (size_t)G * ((p.pos0 + p.P + 3) & ~3) * 4;
    if (lds + 8192 > max_lds_per_block()) return set_error(GAJE_ERR_UNSUPPORTED, "prefill attention: context too long");
    const dim3 grid((unsigned)p.P, (unsigned)p.n_kv);
    switch (G) {
        case 1: hipLaunchKernelGGL((prefill_attn_kernel<HD, 1>), grid, dim3(512), lds, s, p); break;
        case 2: hipLaunchKernelGGL((prefill_attn_kernel<HD, 2>), grid, dim3(512), lds, s, p); break;
        case 3: hipLaunchKernelGGL((prefill_attn_kernel<HD, 3>), grid, dim3(512), lds, s, p); break;
        case 4: hipLaunchKernelGGL((prefill_attn_kernel<HD, 4>), grid, dim3(512), lds, s, p); break;
        case 5: hipLaunchKernelGGL((prefill_attn_kernel<HD, 5>), grid, dim3(512), lds, s, p); break;
        case 6: hipLaunchKernelGGL((prefill_attn_kernel<HD, 6>), grid, dim3(512), lds, s, p); break;
        case 7: hipLaunchKernelGGL((prefill_attn_kernel<HD, 7>), grid, dim3(512), lds, s, p); break;
        case 8: hipLaunchKernelGGL((prefill_attn_kernel<HD, 8>), grid, dim3(512), lds, s, p); break;
        default: return set_error(GAJE_ERR_UNSUPPORTED, "prefill attention: %d query heads per KV head (at most 8)", G);
    }
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace

int launch_rope_kv(const PrefillRopeParams &p, hipStream_t s) {
    if (p.P <= 0 || !p.qkv || !p.q_out || !p.k_cache || !p.v_cache || p.head_dim <= 0 || p.head_dim % 2 ||
        (!p.seq_pos && (p.pos0 < 0 || p.pos0 + p.P > p.cap)))
        return set_error(GAJE_ERR_INVALID_ARG, "rope/kv: bad arguments");
    hipLaunchKernelGGL(rope_kv_kernel, dim3((unsigned)p.P), dim3(256), 0, s, p);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_prefill_attention(const PrefillAttnParams &p, hipStream_t s) {
    if (p.P <= 0 || !p.q || !p.k_cache || !p.v_cache || !p.out || p.n_kv <= 0 || p.n_head % p.n_kv ||
        p.pos0 < 0 || p.pos0 + p.P > p.cap || p.P > 65535)
        return set_error(GAJE_ERR_INVALID_ARG, "prefill attention: bad arguments");
    if (p.head_dim == 64) return launch_attn_hd<64>(p, s);
    if (p.head_dim == 128) return launch_attn_hd<128>(p, s);
    return set_error(GAJE_ERR_UNSUPPORTED, "prefill attention: head_dim %d (64 or 128 only)", p.head_dim);
}

}  // namespace gaje
