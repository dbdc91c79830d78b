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
// cache at the token's position.  One workgroup per token.  In prefill the row
// may first be reduced from the qkv product's split-K partials (its deferred
// reduce, in gemm_reduce_kernel's order), and the keys and values are also
// written as the attention's f16 pairs (prefill_kv16_kernel's layouts).
__global__ __launch_bounds__(256) void rope_kv_kernel(PrefillRopeParams p) {
    extern __shared__ __align__(16) float rowbuf[];  // the reduced row (with part)
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
    if (p.part) {
        // float4s, two per thread per round, every partial of a round in flight
        // before any sum (the first nine; more are added after, in order)
        const int64_t n4 = (q_rows + 2 * kv_rows) >> 2, pstride = p.P * p.ldq;
        for (int64_t i0 = threadIdx.x; i0 < n4; i0 += 2 * blockDim.x) {
            float4 sv[2], q[2][8];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int64_t i = min(i0 + (int64_t)u * blockDim.x, n4 - 1);
                const float *pp = p.part + t * p.ldq + 4 * i;
                sv[u] = *(const float4 *)pp;
#pragma unroll
                for (int j = 0; j < 8; ++j) q[u][j] = *(const float4 *)(pp + (int64_t)min(1 + j, p.nsplit - 1) * pstride);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int64_t i = i0 + (int64_t)u * blockDim.x;
                if (i >= n4) continue;
                float4 v = sv[u];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (1 + j < p.nsplit) {
                        v.x += q[u][j].x;
                        v.y += q[u][j].y;
                        v.z += q[u][j].z;
                        v.w += q[u][j].w;
                    }
                for (int z = 9; z < p.nsplit; ++z) {
                    const float4 r = *(const float4 *)(p.part + t * p.ldq + 4 * i + (int64_t)z * pstride);
                    v.x += r.x;
                    v.y += r.y;
                    v.z += r.z;
                    v.w += r.w;
                }
                float a[4] = {flush_small(v.x), flush_small(v.y), flush_small(v.z), flush_small(v.w)};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (4 * i + j < p.bias_len) a[j] = a[j] + p.bias[4 * i + j];
                *(float4 *)(rowbuf + 4 * i) = make_float4(a[0], a[1], a[2], a[3]);
            }
        }
        __syncthreads();
        row = rowbuf;
    }
    // the attention's f16 pairs: K16[g][pos][d / 32][hi 32 | lo 32],
    // V16[g][d][pos / 32][hi 32 | lo 32] at slot 8 kg + 4 u + r of key 16 u + 4 kg + r
    const int64_t nt = p.kv16_ntiles;
    uint16_t *k16 = p.kv16, *v16 = p.kv16 ? p.kv16 + (int64_t)p.n_kv * nt * 32 * 2 * hd : nullptr;
    auto put_pair = [](uint16_t *dst, float x) {
        const _Float16 hi = (_Float16)x;
        dst[0] = __builtin_bit_cast(uint16_t, hi);
        dst[32] = __builtin_bit_cast(uint16_t, (_Float16)(x - (float)hi));
    };
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
            const int64_t g = head - p.n_head;
            float *kc = p.k_cache + g * hd * p.cap + pos;
            kc[(int64_t)d0 * p.cap] = o0;
            kc[(int64_t)d1 * p.cap] = o1;
            if (k16) {
                uint16_t *kr = k16 + (g * nt * 32 + pos) * 2 * hd;
                put_pair(kr + (d0 >> 5) * 64 + (d0 & 31), o0);
                put_pair(kr + (d1 >> 5) * 64 + (d1 & 31), o1);
            }
        }
    }
    const int w = (int)(pos & 31);
    const int slot = 8 * ((w & 15) >> 2) + 4 * (w >> 4) + (w & 3);
    for (int64_t j = threadIdx.x; j < kv_rows; j += blockDim.x) {
        const int64_t vh = j / hd, d = j - vh * hd;
        const float v = row[q_rows + kv_rows + j];
        p.v_cache[(vh * hd + d) * p.cap + pos] = v;
        if (v16) put_pair(v16 + ((vh * hd + d) * nt + (pos >> 5)) * 64 + slot, v);
    }
}

// The prefill's RoPE and KV append by tiles of 32 tokens x one head (grid:
// token tiles x (n_head + 2 n_kv) heads, q heads then k heads then v heads),
// so that the cache's position-major rows and the attention's f16 pairs are
// written along positions: the tile's values (from the qkv rows, or reduced
// from the qkv product's split-K partials as gemm_reduce_kernel would: the
// partials in split order, flush_small, bias) are staged in LDS; q and k
// heads are rotated as rope_kv_kernel does (attention.rs:56-84, the decode
// epilogue's rounding); q rows go to q_out, k and v to the cache at positions
// pos0 + t and to kv16 (the layouts of prefill_kv16_kernel).
__global__ __launch_bounds__(1024) void prefill_rope_kernel(PrefillRopeParams p) {
    __shared__ float tile[32][129];  // [token][dimension], head_dim <= 128
    const int tid = threadIdx.x, hd = p.head_dim, half = hd >> 1, hd4 = hd >> 2;
    const int head = blockIdx.y;
    const int64_t t0 = (int64_t)blockIdx.x * 32;
    const int nt = (int)min((int64_t)32, p.P - t0);
    const int64_t col0 = (int64_t)head * hd;
    const int64_t q_rows = (int64_t)p.n_head * hd;
    const bool is_q = head < p.n_head, is_v = head >= p.n_head + p.n_kv;
    // this thread's rotation angles (pairs tid, tid + 1024 of the tile: 32 x half
    // <= 2048), read with the tile's loads rather than after them
    float rc[2] = {0.0f, 0.0f}, rsn[2] = {0.0f, 0.0f};
    if (!is_v) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int kk = tid + 1024 * u, r = kk & 31, i = kk >> 5;
            if (kk < 32 * half && r < nt) {
                const int64_t pos = p.pos0 + t0 + r;
                rc[u] = p.rope_cos[pos * half + i];
                rsn[u] = p.rope_sin[pos * half + i];
            }
        }
    }
    // ---- the tile: 32 x hd values, one float4 per thread (hd <= 128), all nine
    // partial loads of a thread issued before any sum ----
    const int k = tid;
    if (k < 32 * hd4) {
        const int r = k / hd4, c4 = k - r * hd4;
        const int64_t t = t0 + min(r, nt - 1);
        float4 v;
        if (p.part) {
            const int64_t pstride = p.P * p.ldq;
            const float *pp = p.part + t * p.ldq + col0 + 4 * c4;
            float4 q[8];
            v = *(const float4 *)pp;
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = *(const float4 *)(pp + (int64_t)min(1 + j, p.nsplit - 1) * pstride);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (1 + j < p.nsplit) {
                    v.x += q[j].x;
                    v.y += q[j].y;
                    v.z += q[j].z;
                    v.w += q[j].w;
                }
            for (int z = 9; z < p.nsplit; ++z) {
                const float4 w = *(const float4 *)(pp + (int64_t)z * pstride);
                v.x += w.x;
                v.y += w.y;
                v.z += w.z;
                v.w += w.w;
            }
            float a[4] = {flush_small(v.x), flush_small(v.y), flush_small(v.z), flush_small(v.w)};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t n = col0 + 4 * c4 + j;
                if (n < p.bias_len) a[j] = a[j] + p.bias[n];
            }
            v = make_float4(a[0], a[1], a[2], a[3]);
        } else {
            v = *(const float4 *)(p.qkv + t * p.ldq + col0 + 4 * c4);
        }
        tile[r][4 * c4] = v.x;
        tile[r][4 * c4 + 1] = v.y;
        tile[r][4 * c4 + 2] = v.z;
        tile[r][4 * c4 + 3] = v.w;
    }
    __syncthreads();
    // ---- rotation of q and k heads, in place: pair (r, i), tokens fastest ----
    if (!is_v) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int k = tid + 1024 * u;
            if (k >= 32 * half) break;
            const int r = k & 31, i = k >> 5;
            if (r >= nt) continue;
            const int d0 = p.rope_split ? i : 2 * i;
            const int d1 = p.rope_split ? i + half : 2 * i + 1;
            const float y0 = tile[r][d0], y1 = tile[r][d1];
            const float cs = rc[u], sn = rsn[u];
            const float a0 = y0 * cs, a1 = y1 * sn, a2 = y0 * sn, a3 = y1 * cs;
            tile[r][d0] = a0 - a1;
            tile[r][d1] = a2 + a3;
        }
        __syncthreads();
    }
    if (is_q) {  // q rows, dimensions fastest
        for (int k = tid; k < 32 * hd; k += 1024) {
            const int r = k / hd, d = k - r * hd;
            if (r < nt) p.q_out[(t0 + r) * q_rows + col0 + d] = tile[r][d];
        }
        return;
    }
    const int64_t g = is_v ? head - p.n_head - p.n_kv : head - p.n_head;
    float *cache = (is_v ? p.v_cache : p.k_cache) + g * hd * p.cap + p.pos0 + t0;
    // the cache's rows [d][pos]: tokens fastest
    for (int k = tid; k < 32 * hd; k += 1024) {
        const int r = k & 31, d = k >> 5;
        if (r < nt) cache[(int64_t)d * p.cap + r] = tile[r][d];
    }
    if (!p.kv16) return;
    const int64_t ntl = p.kv16_ntiles;
    auto put_pair = [](uint16_t *dst, float x) {
        const _Float16 hi = (_Float16)x;
        dst[0] = __builtin_bit_cast(uint16_t, hi);
        dst[32] = __builtin_bit_cast(uint16_t, (_Float16)(x - (float)hi));
    };
    if (!is_v) {  // K16[g][pos][d / 32][hi 32 | lo 32]: dimensions fastest
        uint16_t *k16 = p.kv16 + (g * ntl * 32 + p.pos0 + t0) * 2 * hd;
        for (int k = tid; k < 32 * hd; k += 1024) {
            const int r = k / hd, d = k - r * hd;
            if (r < nt) put_pair(k16 + (int64_t)r * 2 * hd + (d >> 5) * 64 + (d & 31), tile[r][d]);
        }
    } else {  // V16[g][d][pos / 32][slot]: tokens fastest
        uint16_t *v16 = p.kv16 + (int64_t)p.n_kv * ntl * 32 * 2 * hd + g * hd * ntl * 64;
        for (int k = tid; k < 32 * hd; k += 1024) {
            const int r = k & 31, d = k >> 5;
            if (r >= nt) continue;
            const int64_t pos = p.pos0 + t0 + r;
            const int w = (int)(pos & 31);
            const int slot = 8 * ((w & 15) >> 2) + 4 * (w >> 4) + (w & 3);
            put_pair(v16 + ((int64_t)d * ntl + (pos >> 5)) * 64 + slot, tile[r][d]);
        }
    }
}

// Causal GQA attention of a chunk on the f16 matrix cores, each fp32 operand
// split into an f16 pair (hi = f16(x), lo = f16(x - hi)) and each product
// taken as hi.hi + hi.lo + lo.hi (v_mfma_f32_16x16x32_f16, fp32
// accumulation; the dropped lo.lo term is below 2^-22 relative).  One wave
// per 16 queries of one query head and one chunk of keys, walked 32 keys at a
// time, all transposed so that every lane keeps one query:
//   S^T = K Q^T   (keys x queries; lane (fr, kg) holds keys 4 kg + r and
//                  16 + 4 kg + r of query fr),
//   scaled by log2(e)/sqrt(head_dim) and masked past the query's position;
//   the running max m (over the four lanes of the query) and the lane's
//   partial sum l are updated (e = exp2(s - m) on the hardware exp2, ~1 ulp,
//   earlier terms rescaled by exp2(m_old - m));
//   O^T += V^T P^T (dims x queries; P^T straight from the lanes of S^T, whose
//                  key order the converted V tiles follow).
// out = O / (l + 1e-12) in the merge.  Products and sums are fp32 with another
// association than the reference's serial loops (attention.rs:87-127): fp32
// accuracy, not its bits.  Operands must stay below 65504 in magnitude (the
// f16 range of the hi part).
// Lane layout of v_mfma_f32_16x16x32_f16 (lane i): A[i % 16][8 (i / 16) + e],
// B[8 (i / 16) + e][i % 16], D[4 (i / 16) + r][i % 16] in component r.
typedef _Float16 ah8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// The f16 pairs of the cache's keys and values [0, keys) (zero up to a
// multiple of 32), in the layouts of the fragments above:
//   K16[g][pos][s][hi 32 | lo 32]: dimensions 32 s .. 32 s + 31 of key pos;
//   V16[g][d][tile][hi 32 | lo 32]: keys of the 32-key tile, slot 8 kg + 4 u + r
//   holding key 32 tile + 16 u + 4 kg + r (the key order of P^T's lanes).
// One workgroup per (tile, kv head, 32 dimensions); four elements of each
// operand per thread.
__global__ __launch_bounds__(256) void prefill_kv16_kernel(PrefillAttnParams p, int ntiles) {
    __shared__ float kt[32][33];  // this tile's keys, [dimension][key]
    const int tile = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, HD = p.head_dim;
    const int d0 = 32 * (int)blockIdx.z;
    const int64_t k0 = (int64_t)tile * 32, keys = p.pos0 + p.P;
    const float *K = p.k_cache + ((int64_t)g * HD + d0) * p.cap, *V = p.v_cache + ((int64_t)g * HD + d0) * p.cap;
    uint16_t *k16 = p.kv16 + (int64_t)g * ntiles * 32 * 2 * HD;
    uint16_t *v16 = p.kv16 + (int64_t)p.n_kv * ntiles * 32 * 2 * HD + ((int64_t)g * HD + d0) * ntiles * 64;
    float kv[4], vv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = tid + 256 * q, d = e >> 5, j = e & 31;
        const int kg = j >> 3, u = (j >> 2) & 1, r = j & 3;
        const int64_t pos = k0 + 16 * u + 4 * kg + r;
        kv[q] = k0 + j < keys ? K[(int64_t)d * p.cap + k0 + j] : 0.0f;
        vv[q] = pos < keys ? V[(int64_t)d * p.cap + pos] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = tid + 256 * q, d = e >> 5, j = e & 31;
        kt[d][j] = kv[q];
        _Float16 hi, lo;
        split_f16(vv[q], hi, lo);
        uint16_t *dst = v16 + ((int64_t)d * ntiles + tile) * 64;
        dst[j] = __builtin_bit_cast(uint16_t, hi);
        dst[32 + j] = __builtin_bit_cast(uint16_t, lo);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = tid + 256 * q, j = e >> 5, d = e & 31;
        _Float16 hi, lo;
        split_f16(kt[d][j], hi, lo);
        uint16_t *dst = k16 + (k0 + j) * 2 * HD + d0 * 2 + d;
        dst[0] = __builtin_bit_cast(uint16_t, hi);
        dst[32] = __builtin_bit_cast(uint16_t, lo);
    }
}

// Workgroup (query block, query head, key chunk c) walks keys [c*kch,
// (c+1)*kch) and writes its rows' running max m, sum l and unnormalised O to
// the workspace; prefill_attn_merge_kernel combines the chunks.
template <int HD>
__global__ __launch_bounds__(64) void prefill_attn_f16_kernel(PrefillAttnParams p, int64_t kch, int ntiles) {
    constexpr int NS = HD / 32;  // k-steps of S^T over the head dimension
    constexpr int NT = HD / 16;  // 16-dimension tiles of O^T
    const int i = threadIdx.x, fr = i & 15, kg = i >> 4;
    const int nqb = (int)((p.P + 15) / 16);
    const int qb = nqb - 1 - (int)blockIdx.x;  // longest blocks first
    const int h = blockIdx.y;
    const int g = h / (p.n_head / p.n_kv);
    const int64_t t0 = (int64_t)qb * 16;
    const int64_t q_rows = (int64_t)p.n_head * HD;
    const float scale_l2 = 1.4426950408889634f / sqrtf((float)HD);  // log2(e) / sqrt(head_dim)
    const int64_t tmax = (t0 + 15 < p.P ? t0 + 15 : p.P - 1);
    const int64_t kbeg = (int64_t)blockIdx.z * kch;
    if (kbeg > p.pos0 + tmax) return;  // uniform: no key of this chunk is seen by the block
    const int64_t kend = (p.pos0 + tmax < kbeg + kch - 1 ? p.pos0 + tmax : kbeg + kch - 1);  // last key walked
    const int64_t t = t0 + fr, qpos = p.pos0 + t;  // this lane's query and its position

    // B operand of S^T: Q[t][h HD + 32 s + 8 kg + e] (zero past the chunk)
    ah8 qh[NS], ql[NS];
    {
        const float *qr = p.q + (t < p.P ? t : 0) * q_rows + (int64_t)h * HD + 8 * kg;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float4 a = *(const float4 *)(qr + 32 * s), b = *(const float4 *)(qr + 32 * s + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                _Float16 hi, lo;
                split_f16(t < p.P ? v[e] : 0.0f, hi, lo);
                qh[s][e] = hi;
                ql[s][e] = lo;
            }
        }
    }
    const uint16_t *k16 = p.kv16 + (int64_t)g * ntiles * 32 * 2 * HD + 8 * kg;
    const uint16_t *v16 = p.kv16 + (int64_t)p.n_kv * ntiles * 32 * 2 * HD + (int64_t)g * HD * ntiles * 64 + 8 * kg;
    f4v o[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) o[tt] = f4v{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;
    // the key fragments of a tile (loaded one tile ahead, during the previous
    // tile's softmax and P V) and its value fragments (loaded before its softmax)
    ah8 kf[2][NS][2], vf[NT][2];
    auto load_k = [&](int64_t k0) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint16_t *kr = k16 + (k0 + 16 * u + fr) * 2 * HD;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                kf[u][s][0] = *(const ah8 *)(kr + 64 * s);
                kf[u][s][1] = *(const ah8 *)(kr + 64 * s + 32);
            }
        }
    };
    load_k(kbeg);
    for (int64_t k0 = kbeg; k0 <= kend; k0 += 32) {
        // ---- S^T over keys k0 + 16 u + fr ----
        f4v sacc[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            sacc[u] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                sacc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[u][s][0], qh[s], sacc[u], 0, 0, 0);
                sacc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[u][s][0], ql[s], sacc[u], 0, 0, 0);
                sacc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[u][s][1], qh[s], sacc[u], 0, 0, 0);
            }
        }
        {
            const uint16_t *vt = v16 + (k0 >> 5) * 64;
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
                const uint16_t *vr = vt + (int64_t)(16 * tt + fr) * ntiles * 64;
                vf[tt][0] = *(const ah8 *)vr;
                vf[tt][1] = *(const ah8 *)(vr + 32);
            }
        }
        if (k0 + 32 <= kend) load_k(k0 + 32);  // uniform
        // ---- online softmax of query fr over keys k0 + 16 u + 4 kg + r ----
        // scores in log2 units (s / sqrt(head_dim) * log2(e)), so that the
        // exponentials are exp2; masked keys are -inf, whose exp2 is 0
        float sv[2][4], mx = -INFINITY;
        const int rel = (int)(qpos - k0);  // keys k0 + j with j <= rel are seen
        if (p.pos0 + t0 - k0 >= 31) {      // uniform: no key of the tile is masked for the block
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sv[u][r] = sacc[u][r] * scale_l2;
                    mx = fmaxf(mx, sv[u][r]);
                }
        } else {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sv[u][r] = 16 * u + 4 * kg + r <= rel ? sacc[u][r] * scale_l2 : -INFINITY;
                    mx = fmaxf(mx, sv[u][r]);
                }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
        const float mb = mn == -INFINITY ? 0.0f : mn;
        ah8 ph, pl;
        float psum = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pv = __builtin_amdgcn_exp2f(sv[u][r] - mb);
                psum = psum + pv;
                _Float16 hi, lo;
                split_f16(pv, hi, lo);
                ph[4 * u + r] = hi;
                pl[4 * u + r] = lo;
            }
        l = l * alpha + psum;
        m = mn;
        // ---- O^T += V^T P^T over dimensions 16 tt + fr ----
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            o[tt] = o[tt] * alpha;
            o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[tt][0], ph, o[tt], 0, 0, 0);
            o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[tt][0], pl, o[tt], 0, 0, 0);
            o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[tt][1], ph, o[tt], 0, 0, 0);
        }
    }
    // the query's sum over its four lanes; partials ws[c][t][h] = {m, l, -, -, O[HD]}
    l = l + __shfl_xor(l, 16);
    l = l + __shfl_xor(l, 32);
    if (t < p.P) {
        float *rec = p.ws + (((int64_t)blockIdx.z * p.P + t) * p.n_head + h) * (HD + PREFILL_ATTN_REC_PAD);
        if (kg == 0) {
            rec[0] = m;
            rec[1] = l;
        }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
            *(f4v *)(rec + PREFILL_ATTN_REC_PAD + 16 * tt + 4 * kg) = o[tt];
    }
}

// The same attention with the key and value fragments shared by a GQA group:
// workgroup (query block, kv head g, key chunk c) runs one wave per query head
// of the group (R = n_head / n_kv waves), and each 32-key tile's K and V
// fragments are staged once into LDS by all the waves (read one tile ahead
// into registers, double-buffered, one barrier per tile) instead of being read
// from memory by every wave.  Each wave's products, softmax and record are
// prefill_attn_f16_kernel's, operand for operand.  LDS rows are padded (a key
// row by 16 bytes, a value row by 16 bytes) so that the fragment reads of
// consecutive rows fall in distinct banks.
constexpr int GQA_PER = 8;  // staged float4s per thread and tile, at most
template <int HD> struct GqaShape {
    static constexpr int KROW = 2 * HD + 8;                // halves per key row
    static constexpr int VROW = 64 + 8;                    // halves per value row
    static constexpr int TILE = 32 * KROW + HD * VROW;     // halves per tile
    static constexpr int F4 = 16 * HD;                     // float4s per tile (keys, then values)
};
size_t prefill_gqa_lds_bytes(int head_dim) {
    return (size_t)2 * (head_dim == 64 ? GqaShape<64>::TILE : GqaShape<128>::TILE) * 2;
}
bool prefill_gqa_fits(int head_dim, int R) {
    return R >= 1 && R <= 8 && 16 * head_dim <= GQA_PER * 64 * R;
}

template <int HD>
__global__ __launch_bounds__(512) void prefill_attn_gqa_kernel(PrefillAttnParams p, int64_t kch, int ntiles) {
    using Q = GqaShape<HD>;
    constexpr int NS = HD / 32, NT = HD / 16;
    extern __shared__ __align__(16) uint16_t gq_lds[];  // [2][TILE]
    const int R = p.n_head / p.n_kv, NTH = 64 * R;
    const int tid = threadIdx.x, wave = tid >> 6, i = tid & 63, fr = i & 15, kg = i >> 4;
    const int nqb = (int)((p.P + 15) / 16);
    const int qb = nqb - 1 - (int)blockIdx.x;  // longest blocks first
    const int g = blockIdx.y, h = g * R + wave;
    const int64_t t0 = (int64_t)qb * 16;
    const int64_t q_rows = (int64_t)p.n_head * HD;
    const float scale_l2 = 1.4426950408889634f / sqrtf((float)HD);
    const int64_t tmax = (t0 + 15 < p.P ? t0 + 15 : p.P - 1);
    const int64_t kbeg = (int64_t)blockIdx.z * kch;
    if (kbeg > p.pos0 + tmax) return;  // uniform over the workgroup
    const int64_t kend = (p.pos0 + tmax < kbeg + kch - 1 ? p.pos0 + tmax : kbeg + kch - 1);
    const int64_t t = t0 + fr, qpos = p.pos0 + t;

    ah8 qh[NS], ql[NS];
    {
        const float *qr = p.q + (t < p.P ? t : 0) * q_rows + (int64_t)h * HD + 8 * kg;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float4 a = *(const float4 *)(qr + 32 * s), b = *(const float4 *)(qr + 32 * s + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                _Float16 hi, lo;
                split_f16(t < p.P ? v[e] : 0.0f, hi, lo);
                qh[s][e] = hi;
                ql[s][e] = lo;
            }
        }
    }
    // the group's converted keys [pos][2 HD] and values [d][tile][64]
    const uint16_t *k16 = p.kv16 + (int64_t)g * ntiles * 32 * 2 * HD;
    const uint16_t *v16 = p.kv16 + (int64_t)p.n_kv * ntiles * 32 * 2 * HD + (int64_t)g * HD * ntiles * 64;
    // staging: float4 e of a tile is key row e / (HD / 4), chunk e % (HD / 4)
    // (e < 8 HD), else value row (e - 8 HD) / 8, chunk (e - 8 HD) % 8; every
    // row of the tile lies inside the converted range (whole 32-key tiles)
    float4 rg[GQA_PER];
    auto stage_load = [&](int64_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < GQA_PER; ++j) {
            const int e = tid + j * NTH;
            const uint16_t *src;
            if (e < 8 * HD) {
                const int row = e / (HD / 4), c = e % (HD / 4);
                src = k16 + (k0 + row) * 2 * HD + 8 * c;
            } else {
                const int e2 = (e < Q::F4 ? e : Q::F4 - 1) - 8 * HD, d = e2 >> 3, c = e2 & 7;
                src = v16 + ((int64_t)d * ntiles + (k0 >> 5)) * 64 + 8 * c;
            }
            float4 x = float4{0.f, 0.f, 0.f, 0.f};
            if (e < Q::F4) x = *(const float4 *)src;
            rg[j] = x;
        }
    };
    auto stage_store = [&](int buf) __attribute__((always_inline)) {
        uint16_t *dst0 = gq_lds + buf * Q::TILE;
#pragma unroll
        for (int j = 0; j < GQA_PER; ++j) {
            const int e = tid + j * NTH;
            if (e >= Q::F4) break;  // the later j lie beyond it too
            uint16_t *dst;
            if (e < 8 * HD) {
                const int row = e / (HD / 4), c = e % (HD / 4);
                dst = dst0 + row * Q::KROW + 8 * c;
            } else {
                const int e2 = e - 8 * HD, d = e2 >> 3, c = e2 & 7;
                dst = dst0 + 32 * Q::KROW + d * Q::VROW + 8 * c;
            }
            *(float4 *)dst = rg[j];
        }
    };
    stage_load(kbeg);
    stage_store(0);
    __syncthreads();

    f4v o[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) o[tt] = f4v{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;
    int buf = 0;
    for (int64_t k0 = kbeg; k0 <= kend; k0 += 32) {
        const bool more = k0 + 32 <= kend;  // uniform
        if (more) stage_load(k0 + 32);      // in flight during this tile
        const uint16_t *kt = gq_lds + buf * Q::TILE + 8 * kg;
        const uint16_t *vt = gq_lds + buf * Q::TILE + 32 * Q::KROW + 8 * kg;
        // ---- S^T over keys k0 + 16 u + fr (one key half's fragments live at a time) ----
        f4v sacc[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            ah8 kf[NS][2];
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const uint16_t *kr = kt + (16 * u + fr) * Q::KROW + 64 * s;
                kf[s][0] = *(const ah8 *)kr;
                kf[s][1] = *(const ah8 *)(kr + 32);
            }
            sacc[u] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                sacc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[s][0], qh[s], sacc[u], 0, 0, 0);
                sacc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[s][0], ql[s], sacc[u], 0, 0, 0);
                sacc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[s][1], qh[s], sacc[u], 0, 0, 0);
            }
        }
        // ---- online softmax of query fr over keys k0 + 16 u + 4 kg + r (log2 units) ----
        float sv[2][4], mx = -INFINITY;
        const int rel = (int)(qpos - k0);
        if (p.pos0 + t0 - k0 >= 31) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sv[u][r] = sacc[u][r] * scale_l2;
                    mx = fmaxf(mx, sv[u][r]);
                }
        } else {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sv[u][r] = 16 * u + 4 * kg + r <= rel ? sacc[u][r] * scale_l2 : -INFINITY;
                    mx = fmaxf(mx, sv[u][r]);
                }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
        const float mb = mn == -INFINITY ? 0.0f : mn;
        ah8 ph, pl;
        float psum = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pv = __builtin_amdgcn_exp2f(sv[u][r] - mb);
                psum = psum + pv;
                _Float16 hi, lo;
                split_f16(pv, hi, lo);
                ph[4 * u + r] = hi;
                pl[4 * u + r] = lo;
            }
        l = l * alpha + psum;
        m = mn;
        // ---- O^T += V^T P^T over dimensions 16 tt + fr ----
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            const uint16_t *vr = vt + (16 * tt + fr) * Q::VROW;
            const ah8 vf0 = *(const ah8 *)vr, vf1 = *(const ah8 *)(vr + 32);
            o[tt] = o[tt] * alpha;
            o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf0, ph, o[tt], 0, 0, 0);
            o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf0, pl, o[tt], 0, 0, 0);
            o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf1, ph, o[tt], 0, 0, 0);
        }
        // the next tile into the other buffer (every wave finished reading it
        // before the previous barrier), then one barrier
        if (more) stage_store(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    l = l + __shfl_xor(l, 16);
    l = l + __shfl_xor(l, 32);
    if (t < p.P) {
        float *rec = p.ws + (((int64_t)blockIdx.z * p.P + t) * p.n_head + h) * (HD + PREFILL_ATTN_REC_PAD);
        if (kg == 0) {
            rec[0] = m;
            rec[1] = l;
        }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
            *(f4v *)(rec + PREFILL_ATTN_REC_PAD + 16 * tt + 4 * kg) = o[tt];
    }
}

// out[t][h] = (sum_c O_c 2^(m_c - m)) / (sum_c l_c 2^(m_c - m) + 1e-12), m = max_c m_c
// (the chunks' maxima are in log2 units),
// over the chunks that hold keys at or before the row's position.  One
// workgroup per (token, head), one thread per dimension.
__global__ __launch_bounds__(128) void prefill_attn_merge_kernel(PrefillAttnParams p, int64_t kch) {
    const int64_t t = blockIdx.x;
    const int h = blockIdx.y, d = threadIdx.x, HD = p.head_dim;
    const int nc = (int)((p.pos0 + t) / kch) + 1;  // <= PREFILL_ATTN_CHUNKS
    const int64_t rs = (int64_t)p.n_head * (HD + PREFILL_ATTN_REC_PAD);
    const float *rec = p.ws + (t * p.n_head + h) * (HD + PREFILL_ATTN_REC_PAD);
    const int64_t cstride = p.P * rs;
    // every chunk's record read at once (one round trip)
    float mc[PREFILL_ATTN_CHUNKS], lc[PREFILL_ATTN_CHUNKS], oc[PREFILL_ATTN_CHUNKS];
#pragma unroll
    for (int c = 0; c < PREFILL_ATTN_CHUNKS; ++c) {
        const float *rc = rec + (c < nc ? c : 0) * cstride;
        mc[c] = rc[0];
        lc[c] = rc[1];
        oc[c] = d < HD ? rc[PREFILL_ATTN_REC_PAD + d] : 0.0f;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < PREFILL_ATTN_CHUNKS; ++c)
        if (c < nc) mx = fmaxf(mx, mc[c]);
    float l = 0.0f, o = 0.0f;
#pragma unroll
    for (int c = 0; c < PREFILL_ATTN_CHUNKS; ++c)
        if (c < nc) {
            const float e = exp2f(mc[c] - mx);
            l = l + lc[c] * e;
            o = o + oc[c] * e;
        }
    if (d < HD) p.out[t * (int64_t)p.n_head * HD + (int64_t)h * HD + d] = o * (1.0f / (l + 1e-12f));
}

}  // namespace

int launch_rope_kv(const PrefillRopeParams &p, hipStream_t s) {
    if (p.P <= 0 || !p.qkv || !p.q_out || !p.k_cache || !p.v_cache || p.head_dim <= 0 || p.head_dim % 2 ||
        (!p.seq_pos && (p.pos0 < 0 || p.pos0 + p.P > p.cap)))
        return set_error(GAJE_ERR_INVALID_ARG, "rope/kv: bad arguments");
    const int64_t row = (int64_t)(p.n_head + 2 * p.n_kv) * p.head_dim;
    if ((p.part || p.kv16) && (p.seq_pos || p.head_dim % 32))
        return set_error(GAJE_ERR_INVALID_ARG, "rope/kv: bad prefill arguments");
    if (p.part && (p.nsplit < 1 || p.ldq < row || p.ldq % 4 || row * 4 > 65536 || p.bias_len < 0 || (p.bias_len > 0 && !p.bias) ||
                   ((uintptr_t)p.part & 15)))
        return set_error(GAJE_ERR_INVALID_ARG, "rope/kv: bad split-K prologue");
    if (p.kv16 && (int64_t)p.kv16_ntiles * 32 < p.pos0 + p.P)
        return set_error(GAJE_ERR_INVALID_ARG, "rope/kv: f16 key tiles too few");
    if (!p.seq_pos && p.head_dim <= 128 && p.head_dim % 4 == 0 && p.ldq % 4 == 0 && !((uintptr_t)p.qkv & 15)) {
        hipLaunchKernelGGL(prefill_rope_kernel, dim3((unsigned)((p.P + 31) / 32), (unsigned)(p.n_head + 2 * p.n_kv)),
                           dim3(1024), 0, s, p);
        GAJE_HIP_CHECK(hipGetLastError());
        return GAJE_OK;
    }
    hipLaunchKernelGGL(rope_kv_kernel, dim3((unsigned)p.P), dim3(256), p.part ? (size_t)row * 4 : 0, s, p);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int64_t prefill_attn_ws_floats(int64_t P, int64_t n_head, int64_t head_dim) {
    return (int64_t)PREFILL_ATTN_CHUNKS * P * n_head * (head_dim + PREFILL_ATTN_REC_PAD);
}

int64_t prefill_kv16_halves(int64_t keys, int64_t n_kv, int64_t head_dim) {
    return 4 * n_kv * ((keys + 31) / 32 * 32) * head_dim;
}

// key chunks of at least 128 keys (whole 32-key tiles), at most PREFILL_ATTN_CHUNKS of them
// (64-key chunks measured slower at 512 tokens: 29.0 against 25.9 us per layer
// for the per-head kernel, 19.6 against 14.7 us for the GQA-shared one)
int64_t prefill_attn_kch(int64_t keys) {
    int64_t kch = (keys + PREFILL_ATTN_CHUNKS - 1) / PREFILL_ATTN_CHUNKS;
    return kch < 128 ? 128 : (kch + 31) / 32 * 32;
}

int launch_prefill_attention(const PrefillAttnParams &p, hipStream_t s) {
    if (p.P <= 0 || !p.q || !p.k_cache || !p.v_cache || (!p.out && !p.merged_later) || p.n_kv <= 0 ||
        p.n_head % p.n_kv || p.pos0 < 0 || p.pos0 + p.P > p.cap || p.P > 65535)
        return set_error(GAJE_ERR_INVALID_ARG, "prefill attention: bad arguments");
    if (p.head_dim != 64 && p.head_dim != 128)
        return set_error(GAJE_ERR_UNSUPPORTED, "prefill attention: head_dim %d (64 or 128 only)", p.head_dim);
    const int64_t keys = p.pos0 + p.P;
    if (!p.ws || !p.kv16 || p.kv16_keys < keys)
        return set_error(GAJE_ERR_INVALID_ARG, "prefill attention: workspace too small");
    // the converted keys and values, [0, keys) padded to whole 32-key tiles:
    // the tiles before the chunk here (when launch_rope_kv wrote the chunk's
    // positions), or all of them
    const int ntiles = (int)((keys + 31) / 32);
    const int conv = p.kv16_rope ? (int)((p.pos0 + 31) / 32) : ntiles;
    if (conv > 0) {
        hipLaunchKernelGGL(prefill_kv16_kernel, dim3((unsigned)conv, (unsigned)p.n_kv, (unsigned)(p.head_dim / 32)),
                           dim3(256), 0, s, p, ntiles);
        GAJE_HIP_CHECK(hipGetLastError());
    }
    const int64_t kch = prefill_attn_kch(keys);
    const int64_t nch = (keys + kch - 1) / kch;
    const int R = p.n_head / p.n_kv;
    if (prefill_gqa_fits(p.head_dim, R) && prefill_gqa_lds_bytes(p.head_dim) + 1024 <= max_lds_per_block()) {
        const dim3 grid((unsigned)((p.P + 15) / 16), (unsigned)p.n_kv, (unsigned)nch);
        const size_t lds = prefill_gqa_lds_bytes(p.head_dim);
        if (p.head_dim == 64) hipLaunchKernelGGL(prefill_attn_gqa_kernel<64>, grid, dim3(64 * R), lds, s, p, kch, ntiles);
        else hipLaunchKernelGGL(prefill_attn_gqa_kernel<128>, grid, dim3(64 * R), lds, s, p, kch, ntiles);
    } else {
        const dim3 grid((unsigned)((p.P + 15) / 16), (unsigned)p.n_head, (unsigned)nch);
        if (p.head_dim == 64) hipLaunchKernelGGL(prefill_attn_f16_kernel<64>, grid, dim3(64), 0, s, p, kch, ntiles);
        else hipLaunchKernelGGL(prefill_attn_f16_kernel<128>, grid, dim3(64), 0, s, p, kch, ntiles);
    }
    GAJE_HIP_CHECK(hipGetLastError());
    if (!p.merged_later) {
        hipLaunchKernelGGL(prefill_attn_merge_kernel, dim3((unsigned)p.P, (unsigned)p.n_head), dim3(128), 0, s, p, kch);
        GAJE_HIP_CHECK(hipGetLastError());
    }
    return GAJE_OK;
}

}  // namespace gaje
