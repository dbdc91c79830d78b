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
// Cache layout: K and V are both [kv head][dim][position].  A thread scoring
// four consecutive positions reads one 16-byte quad of each key dimension's
// row, so a wave's key loads are contiguous 1 KiB runs; an output dimension's
// chain reads one contiguous V row.
//
// Scores, exponentials and products are computed in parallel over positions;
// the two serial chains (the softmax sum, and each output dimension's
// accumulation) run one lane per chain as the reference's loops do, reading
// LDS.  A chain is bound by its own length, so the parallel work is spread over
// several workgroups per head (one per slice of output dimensions) to keep the
// loads that feed the chains short.
#include "common.h"
#include "device_util.h"

#include <cstddef>
#include <type_traits>

namespace gaje {

static_assert(offsetof(DevState, pos) == 0 && offsetof(DevState, halted) == 12,
              "the attention kernel reads pos and halted with one 16-byte load");

namespace {

constexpr int THREADS = 256;

// dot_product(a, b) of dot.rs:43-67 for one thread, b read with a stride:
// chains l = 0..7 over the 8-float chunks, ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)),
// then the scalar tail.
__device__ __forceinline__ float dot_ref(const float *a, const float *b, int64_t bstride, int n) {
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
    const int chunks = n / 8;
    for (int i = 0; i < chunks; ++i) {
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(a[8 * i + l], b[(8 * i + l) * bstride], acc[l]);
    }
    const float u0 = acc[0] + acc[4], u1 = acc[1] + acc[5], u2 = acc[2] + acc[6], u3 = acc[3] + acc[7];
    float sum = (u0 + u1) + (u2 + u3);
    for (int i = chunks * 8; i < n; ++i) {
        const float prod = a[i] * b[i * bstride];
        sum = sum + prod;
    }
    return sum;
}

// dot_product(q, k_t) chains for the four positions t4..t4+3 of one thread
// (dot.rs:43-67): acc[u][l] is chain l of position t4+u over dimensions
// 8c+l.  Key dimension d of the four positions is one quad of row d (byte
// offset off + d * rowb).  A ring of RING 8-dimension chunks of quads is in
// flight ahead of the FMAs.  q comes from uniform (scalar) loads for HD = 64;
// a 128-float q does not fit the scalar registers and is read from LDS (qs),
// and the chunks walk a loop of RING-chunk rounds so that the compiler cannot
// hoist all 128 key loads of the round (they would spill).
template <int HD>
__device__ __forceinline__ void key_round(float (&acc)[4][8], const char *kb, uint32_t rowb, uint32_t off,
                                          const float *qg, const float *qs) {
    constexpr int NCH = HD / 8, RING = 4;
    float4 kr[RING][8];
#pragma unroll
    for (int c = 0; c < RING; ++c)
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            kr[c][l] = *(const float4 *)(kb + off);
            off += rowb;
        }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[u][l] = 0.0f;
    auto chunk = [&](int c, float4 (&k8)[8]) {
        const float *q8 = HD > 64 ? qs + 8 * c : qg + 8 * c;
        const float4 qa = *(const float4 *)q8, qb = *(const float4 *)(q8 + 4);
        const float qc[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const float4 k = k8[l];
            acc[0][l] = fmaf(qc[l], k.x, acc[0][l]);
            acc[1][l] = fmaf(qc[l], k.y, acc[1][l]);
            acc[2][l] = fmaf(qc[l], k.z, acc[2][l]);
            acc[3][l] = fmaf(qc[l], k.w, acc[3][l]);
        }
        if (c + RING < NCH) {
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                k8[l] = *(const float4 *)(kb + off);
                off += rowb;
            }
        }
    };
    if constexpr (HD > 64) {
#pragma unroll 1
        for (int c0 = 0; c0 < NCH; c0 += RING)
#pragma unroll
            for (int i = 0; i < RING; ++i) chunk(c0 + i, kr[i]);
    } else {
#pragma unroll
        for (int c = 0; c < NCH; ++c) chunk(c, kr[c % RING]);
    }
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
// softmax denominator and every output dimension's accumulation.
__device__ __forceinline__ float serial_sum(const float *e, int n) {
    float sum = 0.0f;
    int t = 0;
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

// The chains run over chain_len(ctx) values: the values past ctx are +0.  A
// chain starts at +0 and a rounded sum is -0 only when both addends are, so it
// is never -0 and adding +0 leaves it unchanged: the padded chain equals the
// unpadded one.

// Padded chain length for ctx positions, and the LDS row length that holds it
// plus the chain's read-ahead (chain_lds reads 32 floats past the end).
__host__ __device__ constexpr int chain_len(int64_t ctx) { return (int)((ctx + 63) / 64 * 64); }
__host__ __device__ constexpr int chain_row(int64_t cap) { return chain_len(cap) + 64; }

// Streaming kernel: head dimension HD known at compile time (64 or 128),
// capacity % 4 == 0.  Workgroup (h, slice) owns output dimensions
// [slice*DS, slice*DS + DS) of query head h: it computes all of the head's
// scores (one quad of positions per thread and round), and copies only its DS
// rows of V into LDS with LDS-direct loads, so they land while the scores are
// computed and both serial chains read LDS only.
typedef __attribute__((address_space(3))) void lds_void;

template <int HD, int DS>
__global__ __launch_bounds__(THREADS) void attn_decode_fast(AttnParams p) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float red[THREADS / WAVE];
    __shared__ float inv_slot;
    __shared__ uint64_t tab[32];  // the exponential's table, read from LDS

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x;
    const uint64_t tabv = tid < 32 ? kExp2Tab[tid] : 0;
    int ctx = (int)p.ctx;
    if (p.seq_pos) {  // batched decode: this block's sequence
        const int z = blockIdx.z;
        const int pos = p.seq_pos[z];
        if (pos < 0) return;
        ctx = pos + 1;
        p.q += z * p.seq_q_stride;
        p.out += z * p.seq_q_stride;
        p.k_cache += z * p.seq_kv_stride;
        p.v_cache += z * p.seq_kv_stride;
    } else if (p.st) {
        typedef int vi4 __attribute__((ext_vector_type(4)));
        const vi4 s4 = *(const volatile vi4 *)p.st;  // pos, token, step, halted: one load
        if (s4.w) return;                            // before any LDS-direct copy is in flight
        ctx = s4.x + 1;
    }

    const int d0 = blockIdx.y * DS;
    const int g = h / (p.n_head / p.n_head_kv);
    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t cap = p.kv_cap;
    const int n = chain_len(ctx);
    const int vstride = chain_row(cap) + 4;  // LDS row stride of the V slice (bank spread)

    float *sc = smem;                   // chain_row(cap) scores, then exponentials
    float *vs = sc + chain_row(cap);    // DS rows of vstride: V, then the products
    const float *qg = p.q + (size_t)h * HD;
    // q: uniform (scalar) loads for HD = 64; a 128-float q does not fit the
    // scalar registers (the compiler spills them), so it is read from LDS
    __shared__ float qs[HD > 64 ? HD : 1];
    if constexpr (HD > 64) {
        if (tid < HD / 4) *(float4 *)(qs + 4 * tid) = *(const float4 *)(qg + 4 * tid);
        __syncthreads();
    }
    const float *Kh = p.k_cache + (size_t)g * p.kv_head_stride;
    const float *Vh = p.v_cache + (size_t)g * p.kv_head_stride + (size_t)d0 * cap;

    // ---- scores: thread j takes positions 4j..4j+3 of each round; key
    // dimension d of those positions is one quad of row d (a 32-bit byte
    // offset walks the rows).  RING 8-dimension chunks of the quads are in
    // flight ahead of the FMAs.  A quad that runs past ctx stays inside the row
    // (kv_cap % 4 == 0); its extra lanes are dropped.  q is read with uniform
    // loads ----
    const uint32_t rowb = (uint32_t)cap * 4;
    float mx = -INFINITY;
    for (int t4 = 4 * tid; t4 < ctx; t4 += 4 * THREADS) {
        float acc[4][8];
        key_round<HD>(acc, (const char *)Kh, rowb, (uint32_t)t4 * 4, qg, qs);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float u0 = acc[u][0] + acc[u][4], u1 = acc[u][1] + acc[u][5];
            const float u2 = acc[u][2] + acc[u][6], u3 = acc[u][3] + acc[u][7];
            const float s = ((u0 + u1) + (u2 + u3)) * scale;
            if (t4 + u < ctx) {
                sc[t4 + u] = s;
                mx = fmaxf(mx, s);  // NaN never wins, as with the reference's '>'
            }
        }
    }
    // ---- V slice -> LDS, issued by the last wave once its scores are done
    // (the first 768 positions leave it none), so the other waves' key loads
    // never wait behind the copies (loads complete in order).  One wave
    // instruction copies 256 positions of a row (lane i its quad i); quads at or
    // past ctx are not copied, and a copied quad ends before the row's capacity
    // (kv_cap % 4 == 0) ----
    if (wave == THREADS / WAVE - 1) {
        const int nchunk = (ctx + 255) >> 8;
        for (int j = 0; j < DS; ++j)
            for (int ch = 0; ch < nchunk; ++ch) {
                const int t = ch * 256 + lane * 4;
                if (t < ctx)
                    __builtin_amdgcn_global_load_lds((const void *)(Vh + (size_t)j * cap + t),
                                                     (lds_void *)(vs + j * vstride + ch * 256), 16, 0, 0);
            }
    }
    if (tid < 32) tab[tid] = tabv;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's LDS-direct copies have landed
    const float max_s = block_max(mx, red);  // (its barrier publishes them to the block)

    // exponentials, +0 up to the padded chain length
    for (int t = tid; t < n; t += THREADS) sc[t] = t < ctx ? expf_ref_t(sc[t] - max_s, tab) : 0.0f;
    __syncthreads();
    if (tid == 0) inv_slot = 1.0f / (chain_lds(0.0f, sc, n) + 1e-12f);
    __syncthreads();
    const float inv = inv_slot;

    // products w_t * v_t[i] in place, w_t = e_t * inv rounded first; +0 past ctx
    for (int t = 4 * tid; t < n; t += 4 * THREADS) {
        const float4 e = *(const float4 *)(sc + t);
        const float w[4] = {e.x * inv, e.y * inv, e.z * inv, e.w * inv};
#pragma unroll
        for (int j = 0; j < DS; ++j) {
            float4 &v4 = *(float4 *)(vs + j * vstride + t);
            const float4 v = v4;
            v4 = make_float4(t < ctx ? w[0] * v.x : 0.0f, t + 1 < ctx ? w[1] * v.y : 0.0f,
                             t + 2 < ctx ? w[2] * v.z : 0.0f, t + 3 < ctx ? w[3] * v.w : 0.0f);
        }
    }
    __syncthreads();

    // ---- out_i = sum_t products, one chain per output dimension ----
    if (tid < DS) p.out[(size_t)h * HD + d0 + tid] = chain_lds(0.0f, vs + tid * vstride, n);
}

// Batched decode (several sequences per launch): one workgroup per (query
// head, sequence) computes the head's scores once; after the softmax each
// output dimension's chain runs in its own thread (threads 0..HD-1), reading
// its V row straight from memory (the row is contiguous and the loads run
// ahead of the adds).  Same rounding sequence as attn_decode_fast.
template <int HD>
__global__ __launch_bounds__(THREADS) void attn_decode_batch(AttnParams p) {
    extern __shared__ __align__(16) float smem[];  // chain_row(cap): scores, exponentials, weights
    __shared__ float red[THREADS / WAVE];
    __shared__ float inv_slot;
    __shared__ uint64_t tab[32];
    const int tid = threadIdx.x;
    const int h = blockIdx.x, z = blockIdx.z;
    const int pos = p.seq_pos[z];
    if (pos < 0) return;
    const int ctx = pos + 1;
    if (tid < 32) tab[tid] = kExp2Tab[tid];
    const int g = h / (p.n_head / p.n_head_kv);
    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t cap = p.kv_cap;
    const int n = chain_len(ctx);
    float *sc = smem;
    const float *qg = p.q + z * p.seq_q_stride + (size_t)h * HD;
    const float *Kh = p.k_cache + z * p.seq_kv_stride + (size_t)g * p.kv_head_stride;
    const float *Vh = p.v_cache + z * p.seq_kv_stride + (size_t)g * p.kv_head_stride;
    // q: uniform (scalar) loads for HD = 64; a 128-float q does not fit the
    // scalar registers (the compiler spills them), so it is read from LDS
    __shared__ float qs[HD > 64 ? HD : 1];
    if constexpr (HD > 64) {
        if (tid < HD / 4) *(float4 *)(qs + 4 * tid) = *(const float4 *)(qg + 4 * tid);
        __syncthreads();
    }

    // scores: thread j takes positions 4j..4j+3 of each round (as attn_decode_fast)
    const uint32_t rowb = (uint32_t)cap * 4;
    float mx = -INFINITY;
    for (int t4 = 4 * tid; t4 < ctx; t4 += 4 * THREADS) {
        float acc[4][8];
        key_round<HD>(acc, (const char *)Kh, rowb, (uint32_t)t4 * 4, qg, qs);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float u0 = acc[u][0] + acc[u][4], u1 = acc[u][1] + acc[u][5];
            const float u2 = acc[u][2] + acc[u][6], u3 = acc[u][3] + acc[u][7];
            const float s = ((u0 + u1) + (u2 + u3)) * scale;
            if (t4 + u < ctx) {
                sc[t4 + u] = s;
                mx = fmaxf(mx, s);
            }
        }
    }
    const float max_s = block_max(mx, red);
    for (int t = tid; t < n; t += THREADS) sc[t] = t < ctx ? expf_ref_t(sc[t] - max_s, tab) : 0.0f;
    __syncthreads();
    if (tid == 0) inv_slot = 1.0f / (chain_lds(0.0f, sc, n) + 1e-12f);
    __syncthreads();
    const float inv = inv_slot;
    for (int t = tid; t < ctx; t += THREADS) sc[t] = sc[t] * inv;
    __syncthreads();

    // out_i = ((w_0 v_0[i]) + (w_1 v_1[i])) + ..., products and sums rounded in t order.
    // AH quads (4 AH positions) of the V row are in flight ahead of the chain, so
    // a load issued one block ahead has the block's arithmetic to land.  Full
    // blocks run without selects; the block holding ctx adds +0 past it (the
    // chain starts at +0, so it is never -0 and +0 leaves it unchanged), and its
    // w reads stay inside the scores' row: t < chain_len(ctx) (a multiple of 4 AH), where
    // w_t = +0.
    if (tid < HD) {
        const float *v = Vh + (size_t)tid * cap;
        float acc = 0.0f;
        constexpr int AH = 16;
        static_assert(64 % (4 * AH) == 0, "blocks must tile chain_len");
        float4 vq[AH];
#pragma unroll
        for (int a = 0; a < AH; ++a) vq[a] = *(const float4 *)(v + (4 * a < ctx ? 4 * a : 0));
        auto block = [&](int t0, auto full) {
#pragma unroll
            for (int a = 0; a < AH; ++a) {
                const int t = t0 + 4 * a;
                const float4 vv = vq[a];
                const int tn = t + 4 * AH;
                vq[a] = *(const float4 *)(v + (tn < ctx ? tn : 0));
                const float4 w = *(const float4 *)(sc + t);
                const float pr[4] = {w.x * vv.x, w.y * vv.y, w.z * vv.z, w.w * vv.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) acc = acc + ((decltype(full)::value || t + j < ctx) ? pr[j] : 0.0f);
            }
        };
        int t0 = 0;
        for (; t0 + 4 * AH <= ctx; t0 += 4 * AH) block(t0, std::true_type{});
        if (t0 < ctx) block(t0, std::false_type{});
        const int64_t i = (int64_t)h * HD + tid, rows = (int64_t)p.n_head * HD;
        p.out[z * p.seq_q_stride + (p.out_chain_major ? (i & 7) * (rows / 8) + (i >> 3) : i)] = acc;
    }
}

// Output dimensions per workgroup of the streaming kernel for this capacity,
// or 0 if even one V row does not fit.
size_t fast_lds_bytes(int64_t cap, int ds) { return (size_t)(chain_row(cap) + (size_t)ds * (chain_row(cap) + 4)) * 4; }
int fast_slice(int head_dim, int64_t cap) {
    for (int ds = 8; ds >= 1; ds >>= 1) {
        if (head_dim % ds) continue;
        if (fast_lds_bytes(cap, ds) + 1024 <= max_lds_per_block()) return ds;
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
    int ctx = st ? st->pos + 1 : (int)p.ctx;
    if (p.seq_pos) {  // batched decode: this block's sequence
        const int z = blockIdx.z;
        if (p.seq_pos[z] < 0) return;
        ctx = p.seq_pos[z] + 1;
        p.q += z * p.seq_q_stride;
        p.out += z * p.seq_q_stride;
        p.k_cache += z * p.seq_kv_stride;
        p.v_cache += z * p.seq_kv_stride;
    }
    const float scale = 1.0f / sqrtf((float)hd);

    float *qh = smem;                            // hd floats (hd % 4 == 0)
    float *sc = smem + ((hd + 3) & ~3);          // ctx scores, then weights
    for (int i = tid; i < hd; i += THREADS) qh[i] = p.q[(size_t)h * hd + i];
    __syncthreads();

    const float *Kh = p.k_cache + (size_t)g * p.kv_head_stride;
    const float *Vh = p.v_cache + (size_t)g * p.kv_head_stride;

    float mx = -INFINITY;
    for (int t = tid; t < ctx; t += THREADS) {
        const float d = dot_ref(qh, Kh + t, p.kv_cap, hd);
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
        const int64_t o = (int64_t)h * hd + i, rows = (int64_t)p.n_head * hd;
        p.out[p.out_chain_major ? (o & 7) * (rows / 8) + (o >> 3) : o] = acc;
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
    if (!p.st && !p.seq_pos && (p.ctx <= 0 || p.ctx > p.kv_cap))
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
    if (p.seq_pos && (p.n_seq <= 0 || p.n_seq > 65535)) return set_error(GAJE_ERR_INVALID_ARG, "attention: bad batch");
    const unsigned nz = p.seq_pos ? (unsigned)p.n_seq : 1u;
    if (p.out_chain_major && (!p.seq_pos || ((int64_t)p.n_head * p.head_dim) % 8))
        return set_error(GAJE_ERR_INVALID_ARG, "attention: chain-major output needs a batch and n_head*head_dim %% 8 == 0");
    const bool batch_kernel = p.seq_pos && p.kv_cap % 4 == 0 && (p.head_dim == 64 || p.head_dim == 128) &&
                              (size_t)chain_row(p.kv_cap) * 4 + 1024 <= max_lds_per_block();
    if (batch_kernel) {
        const size_t blds = (size_t)chain_row(p.kv_cap) * 4;
        if (p.head_dim == 64) hipLaunchKernelGGL(attn_decode_batch<64>, dim3(p.n_head, 1, nz), dim3(THREADS), blds, s, p);
        else hipLaunchKernelGGL(attn_decode_batch<128>, dim3(p.n_head, 1, nz), dim3(THREADS), blds, s, p);
        GAJE_HIP_CHECK(hipGetLastError());
        return GAJE_OK;
    }
    // the batched generic path (any head_dim) or batch 1
    const int ds = (!p.seq_pos && p.kv_cap % 4 == 0 && (p.head_dim == 64 || p.head_dim == 128)) ? fast_slice(p.head_dim, p.kv_cap) : 0;
    if (ds > 0) {
        const size_t flds = fast_lds_bytes(p.kv_cap, ds);
        void (*fn)(AttnParams);
        if (p.head_dim == 64)
            fn = ds == 8 ? attn_decode_fast<64, 8> : ds == 4 ? attn_decode_fast<64, 4> : ds == 2 ? attn_decode_fast<64, 2> : attn_decode_fast<64, 1>;
        else
            fn = ds == 8 ? attn_decode_fast<128, 8> : ds == 4 ? attn_decode_fast<128, 4> : ds == 2 ? attn_decode_fast<128, 2> : attn_decode_fast<128, 1>;
        hipLaunchKernelGGL(fn, dim3(p.n_head, p.head_dim / ds, nz), dim3(THREADS), flds, s, p);
    } else {
        hipLaunchKernelGGL(attn_decode_generic, dim3(p.n_head, 1, nz), dim3(THREADS), lds, s, p);
    }
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
