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

// Causal GQA attention of a chunk on the fp32 matrix cores (flash-style, one
// wave per 16 query tokens of one query head).  Per key tile of 16 positions:
//   S = Q K^T (v_mfma_f32_16x16x4_f32 over the head dimension), scaled by
//   1/sqrt(head_dim), masked past each query's position; the running row max
//   m and sum l are updated (e = expf(s - m), earlier terms rescaled by
//   expf(m_old - m)); O += P V (P reshaped through LDS into the A layout, the
//   V tile staged in LDS).  out = O / (l + 1e-12).  Products and sums are
//   fp32 with another association than the reference's serial loops
//   (attention.rs:87-127): fp32 accuracy, not its bits.
// Lane layout of the instruction (lane i, checked on the device): A[i%16][i/16],
// B[i/16][i%16], D[4*(i/16)+r][i%16] in component r.
typedef float f4v __attribute__((ext_vector_type(4)));

// Reductions over the 16 lanes of a DPP row (the lanes holding one 4-row group
// of a tile): xor 1, xor 2, the half-row mirror and the row mirror.  Each step
// combines symmetric pairs, so all 16 lanes end with the same value.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    return fmaxf(v, dpp_f<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v = v + dpp_f<0xB1>(v);
    v = v + dpp_f<0x4E>(v);
    v = v + dpp_f<0x141>(v);
    return v + dpp_f<0x140>(v);
}

// Workgroup (query block, query head, key chunk c) walks keys [c*kch,
// (c+1)*kch) and writes its rows' running max m, sum l and unnormalised O to
// the workspace; prefill_attn_merge_kernel combines the chunks.
// HD / 64 waves per workgroup: wave w owns head dimensions [64w, 64w + 64),
// both for its partial S = Q K^T (the partials are exchanged through LDS and
// summed as wave 0's + wave 1's in both waves, so both hold the same S and
// run the same softmax) and for its 64 columns of O.
template <int HD>
__global__ __launch_bounds__(HD) void prefill_attn_mfma_kernel(PrefillAttnParams p, int64_t kch) {
    constexpr int NW = HD / 64;   // waves
    constexpr int NS = 16;        // k-steps of a wave's partial S (64 dimensions)
    constexpr int NT = 4;         // 16-column tiles of a wave's O
    constexpr int NV = 4;         // float4s of a wave's V tile per lane
    constexpr int VS = 17;        // LDS stride (floats) of a V-tile row (one row per dimension)
    __shared__ float ps[NW][16 * 16];
    __shared__ float vt[NW][64 * VS];
    __shared__ f4v sx[NW > 1 ? NW : 1][64];
    __shared__ uint64_t tab[32];  // the exponential's table
    const int tid = threadIdx.x, w = tid >> 6, i = tid & 63, c16 = i & 15, q4 = i >> 4;
    if (tid < 32) tab[tid] = kExp2Tab[tid];
    const int nqb = (int)((p.P + 15) / 16);
    const int qb = nqb - 1 - (int)blockIdx.x;  // longest blocks first
    const int h = blockIdx.y;
    const int g = h / (p.n_head / p.n_kv);
    const int64_t t0 = (int64_t)qb * 16;
    const int64_t q_rows = (int64_t)p.n_head * HD;
    const float scale = 1.0f / sqrtf((float)HD);
    const float *Kh = p.k_cache + ((int64_t)g * HD + 64 * w) * p.cap;
    const float *Vh = p.v_cache + ((int64_t)g * HD + 64 * w) * p.cap;
    const int64_t last_key = p.pos0 + p.P - 1;  // keys past it are not written yet

    // A operand of S: Q[t0 + i%16][h*HD + 64w + 4s + i/16] (zero past the chunk)
    float qa[NS];
    {
        const int64_t t = t0 + c16;
        const float *qr = p.q + (t < p.P ? t : 0) * q_rows + (int64_t)h * HD + 64 * w;
#pragma unroll
        for (int st = 0; st < NS; ++st) qa[st] = t < p.P ? qr[4 * st + q4] : 0.0f;
    }
    f4v o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = f4v{0.f, 0.f, 0.f, 0.f};
    float m[4], l[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.0f;
    }
    const int64_t tmax = (t0 + 15 < p.P ? t0 + 15 : p.P - 1);
    const int64_t kbeg = (int64_t)blockIdx.z * kch;
    if (kbeg > p.pos0 + tmax) return;  // uniform: no key of this chunk is seen by the block
    const int64_t kend = (p.pos0 + tmax < kbeg + kch - 1 ? p.pos0 + tmax : kbeg + kch - 1);  // last key walked
    // a tile's operands: K as the B values of the partial S (K[64w + 4s + i/16]
    // [key k0 + i%16]), V as quads (dimension 64w + e/4, keys k0 + 4(e%4) ..);
    // keys past last_key read as 0.  The next tile's are in flight while this
    // one is computed.
    float kb[NS];
    float4 vq[NV];
    auto load_tile = [&](int64_t k0) {
        const int64_t kk = k0 + c16;
        const float *kp = Kh + (kk <= last_key ? kk : 0);
#pragma unroll
        for (int st = 0; st < NS; ++st) kb[st] = kk <= last_key ? kp[(int64_t)(4 * st + q4) * p.cap] : 0.0f;
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int e = i + 64 * u;
            const int64_t key = k0 + (e & 3) * 4;
            const float *vr = Vh + (int64_t)(e >> 2) * p.cap;
            if (key + 3 <= last_key) {
                vq[u] = *(const float4 *)(vr + key);
            } else {
                vq[u].x = key <= last_key ? vr[key] : 0.0f;
                vq[u].y = key + 1 <= last_key ? vr[key + 1] : 0.0f;
                vq[u].z = key + 2 <= last_key ? vr[key + 2] : 0.0f;
                vq[u].w = 0.0f;
            }
        }
    };
    load_tile(kbeg);
    for (int64_t k0 = kbeg; k0 <= kend; k0 += 16) {
        const int64_t kk = k0 + c16;
        f4v sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < NS; ++st) sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[st], kb[st], sacc, 0, 0, 0);
        lds_barrier();  // the previous tile's reads of vt, ps and sx are done (LDS only: the prefetch stays in flight)
        if constexpr (NW > 1) sx[w][i] = sacc;
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int e = i + 64 * u;
            float *dst = vt[w] + (e >> 2) * VS + (e & 3) * 4;
            dst[0] = vq[u].x;
            dst[1] = vq[u].y;
            dst[2] = vq[u].z;
            dst[3] = vq[u].w;
        }
        if (k0 + 16 <= kend) load_tile(k0 + 16);  // uniform
        if constexpr (NW > 1) {
            lds_barrier();
            sacc = sx[0][i] + sx[1][i];  // the same sum in both waves
        }
        // ---- online softmax over the tile's rows 4*(i/16) + r ----
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row_pos = p.pos0 + t0 + 4 * q4 + r;  // this row's query position
            const bool ok = kk <= row_pos && kk <= last_key;
            const float sv = ok ? sacc[r] * scale : -INFINITY;
            const float mn = fmaxf(m[r], row16_max(sv));
            const float alpha = mn == -INFINITY ? 1.0f : expf_ref_t(m[r] - mn, tab);
            const float pv = sv == -INFINITY ? 0.0f : expf_ref_t(sv - mn, tab);
            l[r] = l[r] * alpha + row16_sum(pv);
            m[r] = mn;
#pragma unroll
            for (int t = 0; t < NT; ++t) o[t][r] *= alpha;
            pr[r] = pv;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) ps[w][(4 * q4 + r) * 16 + c16] = pr[r];
        lds_barrier();
        // ---- O += P V: A = P[i%16][4s + i/16], B = V[key 4s + i/16][dim 16t + i%16] ----
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const float a = ps[w][c16 * 16 + 4 * st + q4];
#pragma unroll
            for (int t = 0; t < NT; ++t)
                o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vt[w][(16 * t + c16) * VS + 4 * st + q4], o[t], 0, 0, 0);
        }
    }
    // ---- partials of the block's rows inside the chunk: ws[c][t][h] = {m, l, O[HD]} ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t t = t0 + 4 * q4 + r;
        if (t >= p.P) continue;
        float *rec = p.ws + (((int64_t)blockIdx.z * p.P + t) * p.n_head + h) * (HD + 2);
        if (w == 0 && c16 == 0) {
            rec[0] = m[r];
            rec[1] = l[r];
        }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) rec[2 + 64 * w + 16 * tt + c16] = o[tt][r];
    }
}

// out[t][h] = (sum_c O_c e^(m_c - m)) / (sum_c l_c e^(m_c - m) + 1e-12), m = max_c m_c,
// over the chunks that hold keys at or before the row's position.  One
// workgroup per (token, head), one thread per dimension.
__global__ __launch_bounds__(128) void prefill_attn_merge_kernel(PrefillAttnParams p, int64_t kch) {
    const int64_t t = blockIdx.x;
    const int h = blockIdx.y, d = threadIdx.x, HD = p.head_dim;
    const int nc = (int)((p.pos0 + t) / kch) + 1;
    const int64_t rs = (int64_t)p.n_head * (HD + 2);
    const float *rec = p.ws + (t * p.n_head + h) * (HD + 2);
    const int64_t cstride = p.P * rs;
    float mx = -INFINITY;
    for (int c = 0; c < nc; ++c) mx = fmaxf(mx, rec[c * cstride]);
    float l = 0.0f, o = 0.0f;
    for (int c = 0; c < nc; ++c) {
        const float *rc = rec + c * cstride;
        const float e = expf_ref(rc[0] - mx);
        l = l + rc[1] * e;
        if (d < HD) o = o + rc[2 + d] * e;
    }
    if (d < HD) p.out[t * (int64_t)p.n_head * HD + (int64_t)h * HD + d] = o * (1.0f / (l + 1e-12f));
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

int64_t prefill_attn_ws_floats(int64_t P, int64_t n_head, int64_t head_dim) {
    return (int64_t)PREFILL_ATTN_CHUNKS * P * n_head * (head_dim + 2);
}

int launch_prefill_attention(const PrefillAttnParams &p, hipStream_t s) {
    if (p.P <= 0 || !p.q || !p.k_cache || !p.v_cache || !p.out || p.n_kv <= 0 || p.n_head % p.n_kv ||
        p.pos0 < 0 || p.pos0 + p.P > p.cap || p.P > 65535)
        return set_error(GAJE_ERR_INVALID_ARG, "prefill attention: bad arguments");
    if (p.cap % 4) return set_error(GAJE_ERR_UNSUPPORTED, "prefill attention: KV capacity %% 4 != 0");
    if (p.head_dim == 64 || p.head_dim == 128) {
        if (!p.ws) return set_error(GAJE_ERR_INVALID_ARG, "prefill attention: no workspace");
        // key chunks of at least 128 keys, at most PREFILL_ATTN_CHUNKS of them
        const int64_t keys = p.pos0 + p.P;
        int64_t kch = (keys + PREFILL_ATTN_CHUNKS - 1) / PREFILL_ATTN_CHUNKS;
        kch = kch < 128 ? 128 : (kch + 15) / 16 * 16;
        const int64_t nch = (keys + kch - 1) / kch;
        const dim3 grid((unsigned)((p.P + 15) / 16), (unsigned)p.n_head, (unsigned)nch);
        if (p.head_dim == 64) hipLaunchKernelGGL(prefill_attn_mfma_kernel<64>, grid, dim3(64), 0, s, p, kch);
        else hipLaunchKernelGGL(prefill_attn_mfma_kernel<128>, grid, dim3(128), 0, s, p, kch);
        GAJE_HIP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(prefill_attn_merge_kernel, dim3((unsigned)p.P, (unsigned)p.n_head), dim3(128), 0, s, p, kch);
        GAJE_HIP_CHECK(hipGetLastError());
        return GAJE_OK;
    }
    return set_error(GAJE_ERR_UNSUPPORTED, "prefill attention: head_dim %d (64 or 128 only)", p.head_dim);
}

}  // namespace gaje
