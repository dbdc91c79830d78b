// GQA decode attention over the device KV cache (gfx950, wave64).
//
// Semantics of GenomicAttention::forward_attention_core (src/nn/attention.rs:87-127):
// for every query head h, kv head h / (n_head / n_head_kv); scores
// q_h . k_t / sqrt(hd) over every cached position t (the current token was
// appended by the fused QKV kernel, so attention is causal by construction);
// softmax with max subtraction and 1 / (sum + 1e-12); weighted sum of v_t.
//
// Split-K (flash decoding): grid (n_kv, splits).  Workgroup (g, s) owns a
// contiguous range of 64-position tiles and all query heads of KV group g, so
// each K/V row is read from HBM once per group.  Per tile a wave computes 64
// scores (lane = position), rescales its running (max, sum, output) and
// accumulates p_t * v_t with lane = dimension.  Partials go to a small buffer;
// the last workgroup of a group (agent-scope counter) merges them, so no second
// kernel is needed.  The split count is fixed, the tile range per split is
// derived from the device-side position, so one captured graph serves every
// context length.
#include "common.h"
#include "device_util.h"

namespace gaje {

namespace {

constexpr int THREADS = 256;

__global__ __launch_bounds__(THREADS) void attn_decode_kernel(AttnParams p) {
    extern __shared__ __align__(16) float qsm[];
    __shared__ int is_last;
    DevState *st = p.st;
    if (st->halted) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = blockIdx.x, s = blockIdx.y, S = p.splits;
    const int hd = p.head_dim, G = p.n_head / p.n_head_kv;
    const int ctx = st->pos + 1;
    const int tiles = (ctx + 63) / 64;
    const int tps = (tiles + S - 1) / S;
    const int t_begin = min(ctx, s * tps * 64), t_end = min(ctx, (s + 1) * tps * 64);
    const float scale = 1.0f / sqrtf((float)hd);

    for (int i = tid; i < G * hd; i += THREADS) qsm[i] = p.q[(size_t)g * G * hd + i];
    __syncthreads();

    const float *Kh = p.k_cache + (size_t)g * p.kv_head_stride;
    const float *Vh = p.v_cache + (size_t)g * p.kv_head_stride;
    const bool d0 = lane < hd, d1 = lane + 64 < hd;

    for (int hl = wave; hl < G; hl += 4) {
        const int h = g * G + hl;
        const float *qh = qsm + hl * hd;
        float m = -INFINITY, l = 0.0f, o0 = 0.0f, o1 = 0.0f;
        for (int t0 = t_begin; t0 < t_end; t0 += 64) {
            const int t = t0 + lane;
            const bool valid = t < t_end;
            float sc = -INFINITY;
            if (valid) {
                const float *kr = Kh + (size_t)t * hd;
                float d = 0.0f;
                for (int e = 0; e < hd; e += 4) {
                    const float4 kv = *(const float4 *)(kr + e);
                    const float4 qv = *(const float4 *)(qh + e);
                    d = fmaf(qv.x, kv.x, d);
                    d = fmaf(qv.y, kv.y, d);
                    d = fmaf(qv.z, kv.z, d);
                    d = fmaf(qv.w, kv.w, d);
                }
                sc = d * scale;
            }
            const float mn = fmaxf(m, wave_max(sc));
            const float pe = valid ? expf(sc - mn) : 0.0f;
            const float corr = expf(m - mn);
            l = l * corr + wave_sum(pe);
            o0 *= corr;
            o1 *= corr;
            const int cnt = min(64, t_end - t0);
            const float *vt = Vh + (size_t)t0 * hd;
            for (int tt = 0; tt < cnt; ++tt) {
                const float pt = __shfl(pe, tt, 64);
                if (d0) o0 = fmaf(pt, vt[lane], o0);
                if (d1) o1 = fmaf(pt, vt[lane + 64], o1);
                vt += hd;
            }
            m = mn;
        }
        float *pp = p.partial + ((size_t)h * S + s) * (hd + 2);
        if (lane == 0) {
            pp[0] = m;
            pp[1] = l;
        }
        if (d0) pp[2 + lane] = o0;
        if (d1) pp[2 + lane + 64] = o1;
    }

    // ---- last workgroup of the group merges the partials ----
    __threadfence();
    __syncthreads();
    if (tid == 0) is_last = atomicAdd(&st->attn_counter[g], 1u) == (unsigned)(S - 1);
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int hl = wave; hl < G; hl += 4) {
        const int h = g * G + hl;
        const float *base = p.partial + (size_t)h * S * (hd + 2);
        float M = -INFINITY;
        for (int j = 0; j < S; ++j) M = fmaxf(M, base[(size_t)j * (hd + 2)]);
        float L = 0.0f, O0 = 0.0f, O1 = 0.0f;
        for (int j = 0; j < S; ++j) {
            const float *pp = base + (size_t)j * (hd + 2);
            const float mj = pp[0];
            const float w = mj == -INFINITY ? 0.0f : expf(mj - M);
            L = fmaf(pp[1], w, L);
            if (d0) O0 = fmaf(pp[2 + lane], w, O0);
            if (d1) O1 = fmaf(pp[2 + lane + 64], w, O1);
        }
        const float inv = 1.0f / (L + 1e-12f);
        if (d0) p.out[(size_t)h * hd + lane] = O0 * inv;
        if (d1) p.out[(size_t)h * hd + lane + 64] = O1 * inv;
    }
    if (tid == 0) st->attn_counter[g] = 0;
}

}  // namespace

int launch_attention(const AttnParams &p, hipStream_t s) {
    if (!p.st || !p.q || !p.k_cache || !p.v_cache || !p.partial || !p.out)
        return set_error(GAJE_ERR_INVALID_ARG, "attention: null buffer");
    if (p.n_head_kv <= 0 || p.n_head % p.n_head_kv != 0 || p.n_head_kv > 64)
        return set_error(GAJE_ERR_UNSUPPORTED, "attention: n_head %d / n_head_kv %d not supported", p.n_head,
                         p.n_head_kv);
    if (p.head_dim <= 0 || p.head_dim > 128 || p.head_dim % 4 != 0)
        return set_error(GAJE_ERR_UNSUPPORTED, "attention: head_dim %d not supported (need <= 128, %% 4 == 0)",
                         p.head_dim);
    if (p.splits <= 0) return set_error(GAJE_ERR_INVALID_ARG, "attention: splits must be positive");
    const int G = p.n_head / p.n_head_kv;
    const size_t lds = (size_t)G * p.head_dim * 4;
    if (lds > 64 * 1024) return set_error(GAJE_ERR_UNSUPPORTED, "attention: query group too large");
    hipLaunchKernelGGL(attn_decode_kernel, dim3(p.n_head_kv, p.splits), dim3(THREADS), lds, s, p);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
