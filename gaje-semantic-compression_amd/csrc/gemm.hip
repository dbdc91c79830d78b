// Q4_0 x FP32 matrix products on the MFMA units (prompt prefill, expert FFNs).
//
// Y[m][n] = sum_k X[m][k] W[n][k] with W the Q4_0 rows of GenomicLinear
// (d = fma(q, scale, min), blocks.rs:18-30 / genomic.rs:298-316) and X fp32.
// The reference has no matrix product: it runs compute_single_row
// (linear/forward.rs:11-117) once per activation row.  The result here is the
// same dot product to fp32 accuracy, not the same bits.
//
// Precision.  One f16 MFMA operand carries 11 significant bits, which puts a
// matvec 0.1 away from the reference under the floored relative metric; so
// both operands are split into an f16 pair, v = hi + lo with
// hi = f16(v') and lo = f16(v' - hi), v' = v * 2^e (e a power-of-two scale
// per activation row and per weight row that puts the row's largest magnitude
// in [2^14, 2^15), away from f16 overflow and from subnormal lo parts).  Three
// products hi*hi + hi*lo + lo*hi, accumulated in fp32 by the MFMA, carry
// about 22 bits per term; the dropped lo*lo term is 2^-22 relative.  The
// epilogue multiplies by 2^-(e_x + e_w) (exact).
//
// Tiling (gfx950, wave64).  A workgroup owns MT activation rows x 128 weight
// rows; its waves are (MT/64) x 2, each holding a 64 x 64 tile as 4 x 4
// accumulators of v_mfma_f32_16x16x32_f16 (K = 32 = one Q4_0 block per
// step).  Per block the workgroup stages both activation planes and the
// dequantised weight planes into LDS (double-buffered, one barrier per block);
// weights are dequantised once per workgroup and shared by all its waves.
// Rows of a tile in LDS are 80 bytes apart (32 halves + 8 pad), so the
// 16-byte fragment reads of 16 consecutive rows fall in distinct banks.
// Split-K over blocks fills the device when there are few output tiles; the
// partial products are summed in a fixed order by gemm_reduce_kernel.
#include <hip/hip_runtime.h>
#include <type_traits>

#include "common.h"
#include "device_util.h"
#include "kernels.h"

namespace gaje {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

enum SplitPrologue { SPLIT_PLAIN = 0, SPLIT_NORM = 1, SPLIT_SWIGLU = 2 };

// swiglu_balanced (activation.rs:40-49: the gate clamped to [-64, 64], the
// sigmoid from exp(-|g|), silu(g) * u) for the MFMA paths, which are held to
// fp32 accuracy rather than the reference's bits: the exponential on the
// hardware exp2 and the quotient on the hardware reciprocal (each ~1 ulp),
// without branches.
__device__ __forceinline__ float swiglu_fast(float g, float u) {
    const float gs = fminf(fmaxf(g, -64.0f), 64.0f);
    const float ex = __builtin_amdgcn_exp2f(-fabsf(gs) * 1.4426950408889634f);
    const float r = __builtin_amdgcn_rcpf(1.0f + ex);
    const float sig = gs >= 0.0f ? r : ex * r;
    return (g * sig) * u;
}

constexpr int GM_NT = 128;   // weight rows per workgroup
constexpr int GM_ROW = 40;   // halves per LDS tile row (32 + 8 pad)

// e such that maxabs * 2^e lies in [2^14, 2^15); 0 when maxabs is 0 or not finite.
__device__ __forceinline__ int split_exponent(float maxabs) {
    if (!(maxabs > 0.0f) || !(maxabs <= 3.402823466e38f)) return 0;
    int e;
    (void)frexpf(maxabs, &e);  // maxabs = f * 2^e, f in [0.5, 1)
    return 15 - e;
}

// Per weight row: the exponent of its largest |d| = max(|min|, |fma(15, scale, min)|)
// over its blocks (d is affine in the code, so the extremes are codes 0 and 15).
// One wave per row.
struct RowExpBatch {
    const uint8_t *w[MOE_MAX_EXPERTS];
};

// blockIdx.y selects the matrix of a batch (w = b.w[y], ew advanced by y*N).
__global__ __launch_bounds__(256) void q4_row_exp_kernel(const uint8_t *w, int64_t N, int nb, int *ew,
                                                         RowExpBatch b) {
    if (gridDim.y > 1) {
        w = b.w[blockIdx.y];
        ew += (int64_t)blockIdx.y * N;
    }
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const int lane = threadIdx.x & 63;
    const int G = (nb + 3) >> 2;
    const uint8_t *rp = w + (size_t)row * G * 80;
    float mx = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const uint32_t sm = *(const uint32_t *)(rp + (size_t)(b >> 2) * 80 + 64 + 4 * (b & 3));
        const float s = half_lo(sm), m = half_hi(sm);
        mx = fmaxf(mx, fmaxf(fabsf(m), fabsf(fmaf(15.0f, s, m))));
    }
    mx = wave_max(mx);
    if (lane == 0) ew[row] = split_exponent(mx);
}

// One activation row per workgroup: a prologue (none, rms_norm (norm.rs:52-88),
// or swiglu_balanced of a gate/up pair (activation.rs:35-51) with the optional
// use_genomic_norm scaling of block/forward.rs:115-123; or the deferred
// split-K reduce of the producing product), the NaN guards of
// RustGenomicBlock::forward_core that the prologue's values decide, then the
// row's exponent and its f16 hi/lo planes.  The MFMA paths this feeds are held
// to fp32 accuracy, not the reference's bits, so the row's sums are taken as
// trees (the lanes' partials, then the waves') rather than in the chain order.
// Latency-bound: every input load of a thread is issued at once, the row's
// values stay in registers (NTH threads x IT float4s), and the pass has three
// barriers.
template <int PRO, int NTH, int IT>
__global__ __launch_bounds__(NTH) void split_rows_kernel(SplitParams p) {
    constexpr int NWV = NTH / 64;
    extern __shared__ __align__(16) float xs[];
    __shared__ float red[2][NWV];
    __shared__ int badw[NWV];
    const int64_t m = blockIdx.x;
    const int tid = threadIdx.x, wv = tid >> 6;
    const int64_t K = p.K, K4 = K >> 2;
    const int64_t src_row = p.rows ? (int64_t)p.rows[m] : m;
    const float *xr = p.x + src_row * p.ldx;
    int bad = 0;  // bit 0: st_a, 1: st_b, 2: st_ya, 3: st_yb
    float4 v[IT];
    // ---- every load first ----
    float4 g4[IT], u4[IT], b4[IT], r4[IT], pv[IT];
    // attention-merge prologue: the row's float4 i lies in head 4 i / hd; the
    // records of its key chunks c < nc (clamped reads)
    constexpr int NCH = PREFILL_ATTN_CHUNKS;
    float am[PRO == SPLIT_PLAIN ? IT : 1][NCH], al[PRO == SPLIT_PLAIN ? IT : 1][NCH];
    float4 ao[PRO == SPLIT_PLAIN ? IT : 1][NCH];
    const int anc = p.attn_ws ? (int)((p.attn_pos0 + m) / p.attn_kch) + 1 : 0;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int64_t i = tid + (int64_t)NTH * it;
        if (i < K4) {
            if constexpr (PRO == SPLIT_PLAIN) {
                if (p.attn_ws) {
                    const int64_t h = 4 * i / p.attn_hd, d = 4 * i - h * p.attn_hd;
                    const int64_t rs = (int64_t)p.attn_hd + PREFILL_ATTN_REC_PAD;
#pragma unroll
                    for (int c = 0; c < NCH; ++c) {
                        const float *rc = p.attn_ws + (((int64_t)min(c, anc - 1) * p.M + m) * p.attn_heads + h) * rs;
                        am[it][c] = rc[0];
                        al[it][c] = rc[1];
                        ao[it][c] = *(const float4 *)(rc + PREFILL_ATTN_REC_PAD + d);
                    }
                    continue;
                }
            }
            if constexpr (PRO == SPLIT_SWIGLU) {
                g4[it] = *(const float4 *)(xr + 4 * i);
                u4[it] = *(const float4 *)(p.up + src_row * p.ldx + 4 * i);
            } else if (p.part) {
                pv[it] = *(const float4 *)(p.part + m * p.K + 4 * i);
                if (4 * i + 4 <= p.bias_len) {
                    b4[it] = *(const float4 *)(p.bias + 4 * i);
                } else {
                    float bb[4] = {0.f, 0.f, 0.f, 0.f};
                    for (int j = 0; j < 4; ++j)
                        if (4 * i + j < p.bias_len) bb[j] = p.bias[4 * i + j];
                    b4[it] = make_float4(bb[0], bb[1], bb[2], bb[3]);
                }
                r4[it] = p.resid ? *(const float4 *)(p.resid + m * p.ldx + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                g4[it] = *(const float4 *)(xr + 4 * i);
            }
            if constexpr (PRO == SPLIT_NORM) u4[it] = *(const float4 *)(p.norm_w + 4 * i);
        }
    }
    // ---- the prologue's row ----
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int64_t i = tid + (int64_t)NTH * it;
        v[it] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i >= K4) continue;
        if constexpr (PRO == SPLIT_SWIGLU) {
            const float4 g = g4[it], u = u4[it];
            bad |= isnan(u.x) | isnan(u.y) | isnan(u.z) | isnan(u.w);
            float4 o;
            o.x = swiglu_fast(g.x, u.x);
            o.y = swiglu_fast(g.y, u.y);
            o.z = swiglu_fast(g.z, u.z);
            o.w = swiglu_fast(g.w, u.w);
            bad |= (isnan(o.x) | isnan(o.y) | isnan(o.z) | isnan(o.w)) << 1;
            v[it] = o;
        } else if (p.part) {
            // the deferred split-K reduce, in gemm_reduce_kernel's order: the
            // partials in split order (eight in flight, clamped reads), flush,
            // bias, residual
            const float *pp = p.part + m * p.K + 4 * i;
            const int64_t pstride = p.M * p.K;
            float4 s = pv[it];
            for (int z0 = 1; z0 < p.nsplit; z0 += 8) {
                float4 q[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) q[j] = *(const float4 *)(pp + min(z0 + j, p.nsplit - 1) * pstride);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const bool ok = z0 + j < p.nsplit;
                    s.x = ok ? s.x + q[j].x : s.x;
                    s.y = ok ? s.y + q[j].y : s.y;
                    s.z = ok ? s.z + q[j].z : s.z;
                    s.w = ok ? s.w + q[j].w : s.w;
                }
            }
            float a[4] = {flush_small(s.x), flush_small(s.y), flush_small(s.z), flush_small(s.w)};
            const float bb[4] = {b4[it].x, b4[it].y, b4[it].z, b4[it].w}, rr[4] = {r4[it].x, r4[it].y, r4[it].z, r4[it].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (4 * i + j < p.bias_len) a[j] = a[j] + bb[j];
                bad |= isnan(a[j]) << 2;
                if (p.resid) a[j] = rr[j] + a[j];
                bad |= isnan(a[j]) << 3;
            }
            v[it] = make_float4(a[0], a[1], a[2], a[3]);
            *(float4 *)(const_cast<float *>(p.x) + m * p.ldx + 4 * i) = v[it];  // x is the product's output here
            bad |= isnan(a[0]) | isnan(a[1]) | isnan(a[2]) | isnan(a[3]);
        } else if (PRO == SPLIT_PLAIN && p.attn_ws) {
            // out = (sum_c O_c 2^(m_c - m)) / (sum_c l_c 2^(m_c - m) + 1e-12), m =
            // max_c m_c, as prefill_attn_merge_kernel (the maxima in log2 units)
            if constexpr (PRO == SPLIT_PLAIN) {
                float mx = -INFINITY;
#pragma unroll
                for (int c = 0; c < NCH; ++c)
                    if (c < anc) mx = fmaxf(mx, am[it][c]);
                float l = 0.0f;
                float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int c = 0; c < NCH; ++c)
                    if (c < anc) {
                        const float e = exp2f(am[it][c] - mx);
                        l = l + al[it][c] * e;
                        o.x = o.x + ao[it][c].x * e;
                        o.y = o.y + ao[it][c].y * e;
                        o.z = o.z + ao[it][c].z * e;
                        o.w = o.w + ao[it][c].w * e;
                    }
                const float r = 1.0f / (l + 1e-12f);
                v[it] = make_float4(o.x * r, o.y * r, o.z * r, o.w * r);
                bad |= isnan(v[it].x) | isnan(v[it].y) | isnan(v[it].z) | isnan(v[it].w);
            }
        } else {
            v[it] = g4[it];
            bad |= isnan(v[it].x) | isnan(v[it].y) | isnan(v[it].z) | isnan(v[it].w);
        }
    }
    // a block reduction of one float (op 0: sum, 1: max) over all threads; slot k alternates
    auto block_reduce = [&](float x, int op, int k) -> float {
        x = op ? wave_max(x) : wave_sum(x);
        if ((tid & 63) == 0) red[k][wv] = x;
        __syncthreads();
        float r = red[k][0];
#pragma unroll
        for (int w = 1; w < NWV; ++w) r = op ? fmaxf(r, red[k][w]) : r + red[k][w];
        return r;
    };
    if constexpr (PRO == SPLIT_NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int it = 0; it < IT; ++it) ss += v[it].x * v[it].x + v[it].y * v[it].y + v[it].z * v[it].z + v[it].w * v[it].w;
        const float inv = 1.0f / sqrtf(block_reduce(ss, 0, 0) / (float)K + p.eps);
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int64_t i = tid + (int64_t)NTH * it;
            if (i >= K4) continue;
            const float4 g = u4[it];
            v[it].x = (v[it].x * inv) * g.x;
            v[it].y = (v[it].y * inv) * g.y;
            v[it].z = (v[it].z * inv) * g.z;
            v[it].w = (v[it].w * inv) * g.w;
            bad |= (isnan(v[it].x) | isnan(v[it].y) | isnan(v[it].z) | isnan(v[it].w)) << 1;
        }
    }
    if constexpr (PRO == SPLIT_SWIGLU) {
        if (p.gnorm) {  // the reference's rayon sum has no fixed order: a tree here
            float ss = 0.0f;
#pragma unroll
            for (int it = 0; it < IT; ++it) ss += v[it].x * v[it].x + v[it].y * v[it].y + v[it].z * v[it].z + v[it].w * v[it].w;
            const float rms = sqrtf(block_reduce(ss, 0, 0) / (float)K + p.eps);
            if (rms > p.h_scale) {
                const float sc = p.h_scale / rms;
#pragma unroll
                for (int it = 0; it < IT; ++it) {
                    v[it].x = v[it].x * sc;
                    v[it].y = v[it].y * sc;
                    v[it].z = v[it].z * sc;
                    v[it].w = v[it].w * sc;
                }
            }
        }
    }
    float mx = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int64_t i = tid + (int64_t)NTH * it;
        if (i >= K4) continue;
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[it].x), fabsf(v[it].y)), fmaxf(fabsf(v[it].z), fabsf(v[it].w))));
        *(float4 *)(xs + 4 * i) = v[it];
        if (p.x_out) *(float4 *)(p.x_out + m * p.ldo + 4 * i) = v[it];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) bad |= __shfl_xor(bad, off);
    if ((tid & 63) == 0) badw[wv] = bad;
    const int e = split_exponent(block_reduce(mx, 1, 1));  // (its barrier also publishes xs and badw)
    if (tid == 0) {
        p.ex[m] = e;
        int b = 0;
#pragma unroll
        for (int w = 0; w < NWV; ++w) b |= badw[w];
        if (p.part) {
            if (b & 4) nan_flag(p.st, p.y_layer, p.st_ya);
            if (b & 8) nan_flag(p.st, p.y_layer, p.st_yb);
        }
        if (b & 1) nan_flag(p.st, p.layer, p.st_a);
        if ((b & 2) && PRO != SPLIT_PLAIN) nan_flag(p.st, p.layer, p.st_b);
    }
    if (p.sh) {
        // block-scaled layout: one plane, block b at halves 64 b.. holding its
        // 32 hi halves then its 32 lo halves; position 8 kg + t of each holds
        // element 32 b + 2 kg + 8 (t & 3) + (t >> 2).  Chunk u (8 halves) is
        // (block u >> 2, kg = u & 3); the block sum 2^-5 sum x' (|x'| < 2^15)
        // is the four chunks' partials over consecutive lanes.
        const int64_t nb = K >> 5;
        for (int64_t u0 = 0; u0 < (K >> 3); u0 += NTH) {
            const int64_t u = u0 + tid;
            float s8 = 0.0f;
            if (u < (K >> 3)) {
                const int64_t e0 = 32 * (u >> 2) + 2 * (u & 3);
                h8 hi, lo;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const float a = ldexpf(xs[e0 + 8 * (t & 3) + (t >> 2)], e);
                    hi[t] = (_Float16)a;
                    lo[t] = (_Float16)(a - (float)hi[t]);
                    s8 += a;
                }
                _Float16 *row = (_Float16 *)p.xh + m * p.ldh + 64 * (u >> 2) + 8 * (u & 3);
                *(h8 *)row = hi;
                *(h8 *)(row + 32) = lo;
            }
            s8 += __shfl_xor(s8, 1);
            s8 += __shfl_xor(s8, 2);
            if (u < (K >> 3) && (u & 3) == 0) {
                const float sv = ldexpf(s8, -5);
                const _Float16 hv = (_Float16)sv;
                ((_Float16 *)p.sh)[m * p.ldsum + (u >> 2)] = hv;
                ((_Float16 *)p.sl)[m * p.ldsum + (u >> 2)] = (_Float16)(sv - (float)hv);
            }
        }
        for (int64_t b = nb + tid; b < p.ldsum; b += NTH) {  // zero past the last block
            ((_Float16 *)p.sh)[m * p.ldsum + b] = (_Float16)0.0f;
            ((_Float16 *)p.sl)[m * p.ldsum + b] = (_Float16)0.0f;
        }
        return;
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int64_t i = tid + (int64_t)NTH * it;
        if (i >= K4) continue;
        const float a[4] = {ldexpf(v[it].x, e), ldexpf(v[it].y, e), ldexpf(v[it].z, e), ldexpf(v[it].w, e)};
        h4 hi, lo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hi[j] = (_Float16)a[j];
            lo[j] = (_Float16)(a[j] - (float)hi[j]);
        }
        *(h4 *)((_Float16 *)p.xh + m * p.ldh + 4 * i) = hi;
        *(h4 *)((_Float16 *)p.xl + m * p.ldh + 4 * i) = lo;
    }
}

__device__ __forceinline__ uint32_t word_of(const vu4 (&wq)[4], int j) { return wq[j >> 2][j & 3]; }

// GA (global activations): each wave reads its activation fragments straight
// from the planes (one block ahead, in registers) and LDS holds the weight
// tiles only, so two workgroups share a compute unit.
template <int MT, bool GA>
__global__ __launch_bounds__(MT * 2, GA ? 2 : 1) void gemm_q4_mfma_kernel(GemmQ4Params p) {
    constexpr int NTH = MT * 2;
    constexpr int TPR = NTH / GM_NT;  // staging threads per weight row: 2 or 4
    constexpr int CPT = 4 / TPR;      // 8-element chunks of a block per staging thread
    constexpr int APL = GA ? 0 : MT * GM_ROW;  // halves per activation plane in LDS
    constexpr int BPL = GM_NT * GM_ROW;
    extern __shared__ __align__(16) _Float16 lds[];
    _Float16 *As = lds;                // [buf][plane][MT][GM_ROW] (not GA)
    _Float16 *Bs = lds + 4 * APL;      // [buf][plane][GM_NT][GM_ROW]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t n0 = (int64_t)blockIdx.x * GM_NT;
    // rows [m0, m_end) of the planes and of y, and the weights they multiply
    int64_t m0 = (int64_t)blockIdx.y * MT, m_end = p.M;
    const uint8_t *W = p.w;
    const int *EW = p.ew;
    if (p.g_counts) {  // grouped: tile `mt` of expert e (uniform)
        const int e = (int)blockIdx.y / p.g_mtiles, mt = (int)blockIdx.y - e * p.g_mtiles;
        const int64_t cnt = p.g_counts[e];
        if ((int64_t)mt * MT >= cnt) return;
        m0 = p.g_offsets[e] + (int64_t)mt * MT;
        m_end = p.g_offsets[e] + cnt;
        W = p.gw[e];
        EW = p.gew[e];
    }
    const int z = blockIdx.z;
    const int b0 = z * p.kb_per;
    const int b1 = min(p.nb, b0 + p.kb_per);
    const int G = (p.nb + 3) >> 2;

    // activation staging: row ar, 16 halves at column 16*ah of each plane
    const int ar = tid >> 1, ah = tid & 1;
    int64_t am = m0 + ar;
    if (am >= m_end) am = m_end - 1;
    const _Float16 *xhp = (const _Float16 *)p.xh + am * p.ldh + 16 * ah;
    const _Float16 *xlp = (const _Float16 *)p.xl + am * p.ldh + 16 * ah;
    // weight staging: row br, chunks c = bq*CPT .. of each block
    const int br = tid / TPR, bq = tid % TPR;
    int64_t bn = n0 + br;
    if (bn >= p.N) bn = p.N - 1;
    const uint8_t *wrow = W + (size_t)bn * G * 80;
    const float wsc = ldexpf(1.0f, EW[bn]);

    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

    // two activation blocks (GA: their fragments) and two weight groups (GA:
    // one) in flight
    vu4 xa[2][4];
    vu4 wq[2][4], ws[2];
    auto load_x = [&](int b, vu4 (&r)[4]) {
        const int bb = b < b1 ? b : b1 - 1;  // clamped, so every load is in bounds
        r[0] = *(const vu4 *)(xhp + 32 * bb);
        r[1] = *(const vu4 *)(xhp + 32 * bb + 8);
        r[2] = *(const vu4 *)(xlp + 32 * bb);
        r[3] = *(const vu4 *)(xlp + 32 * bb + 8);
    };
    auto load_w = [&](int g, vu4 (&q)[4], vu4 &s) {
        const int gg = g < G ? g : G - 1;
        const uint8_t *gp = wrow + (size_t)gg * 80;
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = *(const vu4 *)(gp + 16 * i);
        s = *(const vu4 *)(gp + 64);
    };

    const int g0 = b0 >> 2;  // b0 is a multiple of 4
    const int g1 = (b1 + 3) >> 2;
    const int fr = lane & 15, fk = 8 * (lane >> 4);
    // GA: fragment rows of this wave (clamped into the tile's rows, as 32-bit
    // half offsets from the planes)
    uint32_t fo[4];
    h8 fa[2][2][4];  // [block & 1][plane][i]: the next two blocks
    if constexpr (GA) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int64_t r = m0 + wm * 64 + 16 * i + fr;
            if (r >= m_end) r = m_end - 1;
            fo[i] = (uint32_t)(r * p.ldh + fk);
        }
    }
    const _Float16 *xhb = (const _Float16 *)p.xh, *xlb = (const _Float16 *)p.xl;
    auto load_frag = [&](int b, h8 (&hi)[4], h8 (&lo)[4]) {
        const uint32_t bo = 32u * (uint32_t)(b < b1 ? b : b1 - 1);  // clamped, so every load is in bounds
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            hi[i] = *(const h8 *)(xhb + fo[i] + bo);
            lo[i] = *(const h8 *)(xlb + fo[i] + bo);
        }
    };
    load_w(g0, wq[0], ws[0]);
    if constexpr (GA) {
        load_frag(b0, fa[0][0], fa[0][1]);
        load_frag(b0 + 1, fa[1][0], fa[1][1]);
    } else {
        load_x(b0, xa[0]);
        load_x(b0 + 1, xa[1]);
    }
    if constexpr (!GA) load_w(g0 + 1, wq[1], ws[1]);

    int buf = 0;
    for (int g = g0; g < g1; ++g) {
        const int wi = GA ? 0 : (g - g0) & 1;  // GA: one weight group in flight (registers)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // Every group runs all four blocks, branch-free (a branch here makes
            // the compiler wait for every load in flight).  Blocks past nb only
            // occur in the last group: their packed codes, scales and mins are
            // zero, and their activations are masked to zero here.
            const int b = 4 * g + u;
            const int xi = u & 1;
            const uint32_t live = b < b1 ? 0xFFFFFFFFu : 0u;
            // stage block b into LDS buffer buf
            {
                if constexpr (!GA) {
                    _Float16 *ad = As + buf * 2 * APL + ar * GM_ROW + 16 * ah;
                    *(vu4 *)ad = xa[xi][0] & live;
                    *(vu4 *)(ad + 8) = xa[xi][1] & live;
                    *(vu4 *)(ad + APL) = xa[xi][2] & live;
                    *(vu4 *)(ad + APL + 8) = xa[xi][3] & live;
                }
                const uint32_t smw = ws[wi][u];
                const float s = half_lo(smw), mn = half_hi(smw);
                const int hb = u >> 1;
                const int sh = 4 * (u & 1);
#pragma unroll
                for (int cc = 0; cc < CPT; ++cc) {
                    const int c = bq * CPT + cc;
                    h8 hi, lo;
#pragma unroll
                    for (int l = 0; l < 8; ++l) {
                        const uint32_t code = (word_of(wq[wi], 2 * l + hb) >> (8 * c + sh)) & 0xFu;
                        const float d = fmaf((float)code, s, mn) * wsc;
                        hi[l] = (_Float16)d;
                        lo[l] = (_Float16)(d - (float)hi[l]);
                    }
                    _Float16 *bd = Bs + buf * 2 * BPL + br * GM_ROW + 8 * c;
                    *(h8 *)bd = hi;
                    *(h8 *)(bd + BPL) = lo;
                }
            }
            // refill: activations two blocks ahead; the next-but-one weight group
            if constexpr (!GA) load_x(b + 2, xa[xi]);
            if (u == 3) load_w(GA ? g + 1 : g + 2, wq[wi], ws[wi]);
            lds_barrier();
            // 4 x 4 tiles x 3 products from buffer buf; every accumulator takes
            // hi*hi, hi*lo, lo*hi in that order
            const _Float16 *Bb = Bs + buf * 2 * BPL + (wn * 64 + fr) * GM_ROW + fk;
            if constexpr (GA) {
                // weights column tile by column tile, so two fragments are live.
                // No activation mask: a split ends on a group boundary, and the
                // blocks past nb in the row's last group have zero codes, scales
                // and mins, so their products with the (clamped, finite)
                // activations are zero.
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const h8 bh = *(const h8 *)(Bb + 16 * j * GM_ROW);
                    const h8 bl = *(const h8 *)(Bb + 16 * j * GM_ROW + BPL);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[xi][0][i], bh, acc[i][j], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[xi][0][i], bl, acc[i][j], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[xi][1][i], bh, acc[i][j], 0, 0, 0);
                }
                load_frag(b + 2, fa[xi][0], fa[xi][1]);  // two blocks ahead
            } else {
                const _Float16 *Ab = As + buf * 2 * APL + (wm * 64 + fr) * GM_ROW + fk;
                h8 ahi[4], alo[4], bhi[4], blo[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    ahi[i] = *(const h8 *)(Ab + 16 * i * GM_ROW);
                    alo[i] = *(const h8 *)(Ab + 16 * i * GM_ROW + APL);
                    bhi[i] = *(const h8 *)(Bb + 16 * i * GM_ROW);
                    blo[i] = *(const h8 *)(Bb + 16 * i * GM_ROW + BPL);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[i], bhi[j], acc[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[i], blo[j], acc[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[i], bhi[j], acc[i][j], 0, 0, 0);
            }
            buf ^= 1;
        }
    }

    // epilogue: lane holds rows 4*(lane>>4)+r, column lane&15 of each 16x16 tile
    int bad_a = 0, bad_b = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + wn * 64 + 16 * j + fr;
        if (n >= p.N) continue;
        const int en = EW[n];
        const float bias = (!p.part && n < p.bias_len) ? p.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm * 64 + 16 * i + 4 * (lane >> 4) + r;
                if (m >= m_end) continue;
                float v = ldexpf(acc[i][j][r], -(p.ex[m] + en));
                if (p.part) {
                    p.part[((int64_t)z * p.M + m) * p.N + n] = v;
                } else {
                    v = flush_small(v);
                    if (n < p.bias_len) v = v + bias;
                    bad_a |= isnan(v);
                    if (p.resid) v = p.resid[m * p.ldr + n] + v;
                    bad_b |= isnan(v);
                    p.y[m * p.ldy + n] = v;
                }
            }
        }
    }
    if (p.st) {
        if (__any(bad_a) && lane == 0) nan_flag(p.st, p.layer, p.st_a);
        if (__any(bad_b) && lane == 0) nan_flag(p.st, p.layer, p.st_b);
    }
}

// Sums the split-K partials in split order, then the row epilogue of
// compute_single_row: flush, + bias; + residual (block/forward.rs:70-72,131-133).
__global__ void gemm_reduce_kernel(GemmQ4Params p, int S) {
    const int64_t total = p.M * p.N;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = t / p.N, n = t - m * p.N;
        float v = p.part[t];
        for (int z0 = 1; z0 < S; z0 += 8) {  // eight partials in flight (clamped reads), added in split order
            float q[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = p.part[(int64_t)min(z0 + j, S - 1) * total + t];
#pragma unroll
            for (int j = 0; j < 8; ++j) v = z0 + j < S ? v + q[j] : v;
        }
        v = flush_small(v);
        if (n < p.bias_len) v = v + p.bias[n];
        if (isnan(v)) nan_flag(p.st, p.layer, p.st_a);
        if (p.resid) v = p.resid[m * p.ldr + n] + v;
        if (isnan(v)) nan_flag(p.st, p.layer, p.st_b);
        p.y[m * p.ldy + n] = v;
    }
}

template <int MT, bool GA>
size_t gemm_lds() { return (size_t)((GA ? 0 : 4 * MT * GM_ROW) + 4 * GM_NT * GM_ROW) * sizeof(_Float16); }

// ---------------------------------------------------------------------------
// Block-scaled product (the dense products of prefill and
// gaje_hip_q4_0_gemm_mfma).
//
// The Q4_0 dot product regrouped by block b (blocks.rs:18-30, d = fma(q, s, mn)):
//   sum_k x_k (q_k s_b + mn_b) = sum_b s_b P_b + sum_b mn_b X_b,
//   P_b = sum_{k in b} x_k q_k,   X_b = sum_{k in b} x_k.
// The codes q (0..15) are exact f16 operands, so P_b takes two MFMA products
// (x_hi q + x_lo q, fp32 accumulation) where an f16 pair for the dequantised
// weight takes three; s_b scales each block's 16 x 16 partial in fp32 on the
// VALU, beside the matrix core.  The min term is one more product over the
// block index: the block sums X'' = 2^-5 X' (an f16 pair) times the f16 mins.
// Row result: 2^-ex (32 sum_b mn_b X''_b + sum_b s_b P'_b), x' = 2^ex x.
//
// Operand layout.  Packed Q4_0 word 4 kg + hh of a group holds, in byte c,
// element 8 c + 2 kg of blocks 2 hh (low nibble) and 2 hh + 1 (high nibble);
// word 4 kg + 2 + hh holds element 8 c + 2 kg + 1.  The split pass writes
// each activation block permuted to match: position 8 kg + t holds element
// 2 kg + 8 (t & 3) + (t >> 2), so the 8 halves of MFMA lane group kg are the
// 8 codes of that word pair.  A code byte becomes f16 1024 + q by v_perm
// against 0x64 bytes, then q by a packed f16 subtraction.  This expansion runs
// once per weight matrix (q4_frag_kernel): the products read the codes as f16
// fragments, [16-row tile][block][64 lanes][8 halves] (1 KiB per tile and
// block, in the MFMA's lane order), and the scales as fp32 [tile][block][16],
// both zero past the last row and block: four times the packed bytes, traded
// for no expansion work in the product's loop.
//
// Tiling (gfx950, wave64).  A workgroup is W waves of 32 activation rows and
// 9 tiles of 16 weight rows (144); every wave holds 2 x 9 accumulators of
// v_mfma_f32_16x16x32_f16 (one Q4_0 block per step).  Eight waves (two per
// SIMD) for a 256-row tile, so that one wave's LDS waits and expansions
// overlap the other's MFMAs.  (Measured by wall clock on 256 workgroups: one
// wave per SIMD issuing 16x16x32 f16 MFMAs reaches ~1.7-1.9 PFLOP/s with up to
// two independent fp32 fmas per MFMA, and VALU issue binds from about three.
// The block scales cost two fmas per MFMA here, so the VALU work beside them
// must stay small.)
// - Activations: the split pass stores each block's hi and lo halves together
//   (128 bytes per row); each wave streams its own rows into a private LDS
//   ring of three blocks with global_load_lds, two blocks ahead, XOR-swizzled
//   by 16-byte chunk so that fragment reads are conflict-free.
// - Weights: each pair of blocks' code fragments and scales is copied into LDS
//   by all waves together, two pairs ahead (three buffers, one barrier per
//   pair).
// - No other vector memory access is made in the main loop, so the explicit
//   vmcnt waits are exact.
// - The grid is ordered so that the workgroups of one activation tile and
//   split share an XCD, and so its L2.
// Split-K over groups fills the device when there are few output tiles; the
// partials are summed in a fixed order by gemm_reduce_kernel.
constexpr int BS_J = 9;                         // 16-row weight tiles per workgroup
constexpr int BS_NT = 16 * BS_J;                // 144 weight rows
constexpr int BS_WR = BS_WR_ROWS;               // activation rows per wave
constexpr int BS_ABLK = BS_WR * 128;            // one block of a wave's rows (hi | lo)
constexpr int BS_ADMA = BS_ABLK / 1024;         // its copy instructions
constexpr int BS_BF = BS_J * 1024;              // one block's code fragments

// W waves of 32 rows, BPI blocks per interval between barriers; a weight
// buffer holds an interval's BPI x 9 fragments, then its BPI x 144 scales
// (one 1 KiB copy per block).  R activation ring slots per wave (R - 1 blocks
// copied ahead), NB weight buffers (NB - 1 intervals copied ahead).
template <int W, int BPI, int R = 3, int NB = 3>
struct BsShape {
    static constexpr int BCOPY = (BS_J + 1) * BPI;             // weight copy instructions per interval
    static constexpr int BDMA = (BCOPY + W - 1) / W;           // of them per wave
    static constexpr int PB = BPI * (BS_BF + 1024);            // bytes per weight buffer
    static constexpr size_t LDS = (size_t)W * R * BS_ABLK + NB * PB;
    static constexpr int WG_PER_CU = BPI == 1 ? 2 : 1;
};
template <int W, int BPI, int R = 3, int NB = 3>
constexpr size_t bs_lds() { return BsShape<W, BPI, R, NB>::LDS; }

struct BsGrid {
    int32_t ntiles, splits, kb_per, units, total;  // units: 16-row weight units ceil(N / 16)
};

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// f16 1024 + byte (bytes 2 s, 2 s + 1 of t), minus 1024: the two codes as f16.
template <int S>
__device__ __forceinline__ uint32_t code_pair(uint32_t t) {
    constexpr uint32_t sel = S == 0 ? 0x04010400u : 0x04030402u;
    const uint32_t v = __builtin_amdgcn_perm(0x64646464u, t, sel);
    const h2 r = __builtin_bit_cast(h2, v) + (h2){(_Float16)-1024.0f, (_Float16)-1024.0f};
    return __builtin_bit_cast(uint32_t, r);
}

template <int W, int BPI, int R = 3, int NB = 3>
__global__ __launch_bounds__(64 * W, (BsShape<W, BPI, R, NB>::WG_PER_CU)) void gemm_q4_bs_kernel(GemmBsParams p, BsGrid gd) {
    using S = BsShape<W, BPI, R, NB>;
    constexpr int BDMA = S::BDMA, BCOPY = S::BCOPY, PB = S::PB;
    static_assert((BPI == 1 || (R == 3 && NB == 3)) && R >= 2 && NB >= 3, "shapes");
    static_assert(4 * BS_ADMA + 3 * BDMA < 64 && (R - 1) * (BS_ADMA + BDMA) + BDMA < 64 &&
                      (NB - 2) * (BS_ADMA + BDMA) + BS_ADMA < 64 && S::LDS * S::WG_PER_CU <= 163840,
                  "limits");
    extern __shared__ __align__(16) uint8_t bs_mem[];
    // w through readfirstlane: the copies' bases must be provably wave-uniform (SGPRs)
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 15, kg = lane >> 4;

    // consecutive workgroups alternate over the 8 XCDs; XCD x takes the x-th
    // contiguous run of (row tile, split, weight tile) indices
    const int Q = (int)(gridDim.x >> 3);
    const int idx = (int)(blockIdx.x & 7) * Q + (int)(blockIdx.x >> 3);
    if (idx >= gd.total) return;
    const int t = idx % gd.ntiles, mz = idx / gd.ntiles;
    const int z = mz % gd.splits, mt = mz / gd.splits;
    const int ubase = gd.units / gd.ntiles, urem = gd.units % gd.ntiles;
    const int nj = ubase + (t < urem ? 1 : 0);  // 16-row weight units of this tile (<= BS_J)
    const int64_t n0 = 16 * (int64_t)(t * ubase + min(t, urem));
    int64_t m0 = (int64_t)mt * (BS_WR * W) + BS_WR * w;  // this wave's first activation row
    int64_t mend = p.M;                                   // rows at or past it are not stored
    if (p.g_counts) {  // grouped: row tile mtl of group e, with that group's operands (uniform)
        const int e = mt / p.g_mtiles, mtl = mt - e * p.g_mtiles;
        const int64_t cnt = p.g_counts[e];
        if ((int64_t)mtl * (BS_WR * W) >= cnt) return;  // before any copy or barrier
        m0 = p.g_offsets[e] + (int64_t)mtl * (BS_WR * W) + BS_WR * w;
        mend = p.g_offsets[e] + cnt;
        p.wf += e * p.g_wf_stride;
        p.wsc += e * p.g_wsc_stride;
        p.mins += e * p.g_mins_stride;
    }
    const int b0 = z * gd.kb_per, b1 = min(p.nb, b0 + gd.kb_per);
    const int nblk = b1 - b0, npr = (nblk + BPI - 1) / BPI;  // blocks, intervals of this split
    const int64_t t16 = n0 >> 4;                        // the tile's first 16-row fragment tile

    uint8_t *ring = bs_mem + w * (R * BS_ABLK);
    uint8_t *bfr = bs_mem + W * R * BS_ABLK;  // [NB][PB]: fragments, then scales (block e at 144 e floats)

    // activation copies: per block a wave copies its 32 rows x 128 bytes (the
    // block's hi | lo halves, one cache line per row).  Instruction q takes rows
    // 8q..8q+7: lane -> row R = 8q + (lane >> 3), LDS chunk lane & 7, holding
    // global chunk (lane & 7) ^ ((R >> 1) & 7), so that the fragment reads of
    // 16 consecutive rows fall in distinct banks.  (R >> 1) & 7 is
    // (lane >> 4) ^ 4 (q & 1): one lane offset for even q, one for odd.  The
    // plane holds plane_rows >= the tile's rows, so no row is clamped, and its
    // byte offsets fit 32 bits (both checked by the launcher).
    const uint32_t arow = (uint32_t)((lane >> 3) * 2 * p.ldh);
    const uint32_t aoffs[2] = {arow + 16 * ((lane & 7) ^ (lane >> 4)), arow + 16 * ((lane & 7) ^ (lane >> 4) ^ 4)};
    auto dma_a = [&](int kk, int slot) {
        const int64_t b = b0 + min(kk, nblk - 1);
        const uint32_t dst = lds_addr(ring + slot * BS_ABLK);
        const uint8_t *base = (const uint8_t *)p.xh + m0 * 2 * p.ldh + 128 * b;
#pragma unroll
        for (int q = 0; q < BS_ADMA; ++q) lds_dma16_so(base + q * 16 * p.ldh, aoffs[q & 1], dst + q * 1024);
    };

    // weight copies of interval pp into buffer pb: copy ci < 9 BPI takes the
    // 1 KiB fragment of (block e = ci / 9, tile j = ci % 9), as it lies in
    // global memory; the BPI copies after them take the interval's BPI x 9 x
    // 16 scales, lane l of copy s reading chunk c = min(64 s + l, 36 BPI - 1)
    // of four (block c / 36, tile (c % 36) / 4, quarter c % 4).  Tiles past
    // nj - 1 repeat the last one.  Wave w issues copies w, w + W, ..; in place
    // of one past the last it issues copy w again (same bytes, same place), so
    // that every wave issues BDMA copies and no lane branches: the compiler
    // would otherwise sink the fmas of a block below its later MFMAs.  Offsets
    // fit 32 bits (checked by the launcher).
    int cidx[BDMA];
    uint32_t coff[BDMA], cdst[BDMA];
#pragma unroll
    for (int r = 0; r < BDMA; ++r) {
        const int ci = w + W * r < BCOPY ? w + W * r : w;
        cidx[r] = ci;
        if (ci < BPI * BS_J) {
            const int e = ci / BS_J, j = min(ci % BS_J, nj - 1);
            coff[r] = (uint32_t)(((t16 + j) * p.nbp4 + e) * 1024 + lane * 16);
            cdst[r] = (uint32_t)((e * BS_J + ci % BS_J) * 1024);
        } else {
            const int c = min(64 * (ci - BPI * BS_J) + lane, 36 * BPI - 1);
            const int e = c / 36, j = min((c % 36) / 4, nj - 1);
            coff[r] = (uint32_t)((((t16 + j) * p.nbp4 + e) * 16 + 4 * (c % 4)) * 4);
            cdst[r] = (uint32_t)(BPI * BS_BF + (ci - BPI * BS_J) * 1024);
        }
    }
    auto dma_b = [&](int pp, int pb) {
        const int64_t b = b0 + BPI * (int64_t)min(pp, npr - 1);
        const uint8_t *fbase = (const uint8_t *)p.wf + b * 1024;
        const uint8_t *sbase = (const uint8_t *)p.wsc + b * 64;
        const uint32_t base = lds_addr(bfr + pb * PB);
#pragma unroll
        for (int r = 0; r < BDMA; ++r) {
            // cidx is wave-uniform: the source is chosen without a lane branch
            const uint8_t *src = cidx[r] < BPI * BS_J ? fbase : sbase;
            lds_dma16_so(src, coff[r], base + cdst[r]);
        }
    };

    f4 acc[2][BS_J];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < BS_J; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

    // One block: activation fragments of ring slot `slot`, code fragments and
    // scales of block e of pair buffer pb.  Software-pipelined by weight tile: the fragment of
    // tile j + 1 is read while tile j computes, and the MFMAs of tile j issue
    // one by one between the fmas of tile j - 1 (sched_group_barrier); a
    // scheduling barrier per tile keeps the compiler from hoisting every
    // product (and its registers) ahead of the fmas.
    // Fragment (i, plane P) of lane (fr, kg): row 16 i + fr, chunk (4 P + kg) ^ ((fr >> 1) & 7).
    const uint32_t aoff0 = fr * 128 + 16 * (kg ^ ((fr >> 1) & 7)), aoff1 = aoff0 ^ 64;
    auto compute = [&](int slot, int pb, int e) {
        const uint8_t *ab = ring + slot * BS_ABLK;
        h8 a[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            a[i][0] = *(const h8 *)(ab + i * 2048 + aoff0);
            a[i][1] = *(const h8 *)(ab + i * 2048 + aoff1);
        }
        const uint8_t *bq = bfr + pb * PB + e * BS_BF + lane * 16;
        // (volatile, through an LDS pointer: the compiler would otherwise move
        // each scale read to just before its first use, exposing its latency)
        typedef const __attribute__((address_space(3))) volatile float lds_vf;
        lds_vf *sp = (lds_vf *)((const float *)(bfr + pb * PB + BPI * BS_BF) + e * BS_NT + fr);
        f4 pr[2][2];
        // scales of tiles j - 1 (fmas this step), j and j + 1 (read this step)
        float s_prev = 0.0f, s_cur = sp[0];
        h8 bcur = *(const h8 *)bq;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j <= BS_J; ++j) {
            h8 bnext = bcur;
            float s_next = 0.0f;
            if (j + 1 < BS_J) {
                bnext = *(const h8 *)(bq + (j + 1) * 1024);
                s_next = sp[16 * (j + 1)];
            }
            if (j < BS_J) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    pr[j & 1][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][0], bcur, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    pr[j & 1][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][1], bcur, pr[j & 1][i], 0, 0, 0);
            }
            if (j > 0) {
                const int jp = j - 1;
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][jp][r] = fmaf(s_prev, pr[jp & 1][i][r], acc[i][jp][r]);
            }
            if (j > 0 && j < BS_J) {
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // the next fragment and scale
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two fmas
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            bcur = bnext;
            s_prev = s_cur;
            s_cur = s_next;
        }
    };

    // prologue: the weights of intervals 0 .. NB - 2, activation blocks 0 .. R - 1 in flight
#pragma unroll
    for (int i = 0; i < NB - 1; ++i) dma_b(i, i);
#pragma unroll
    for (int i = 0; i < R; ++i) dma_a(i, i);

    // the min term over this split's blocks: MFMAs over the block index, the
    // block-sum planes against the dense f16 mins (blocks outside [b0, b1)
    // masked), one tile at a time into a temporary, so that the accumulators
    // are only ever VALU operands
    {
        const _Float16 *sh = (const _Float16 *)p.sh, *sl = (const _Float16 *)p.sl;
        int64_t srow[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            int64_t r = m0 + 16 * i + fr;
            if (r >= p.M) r = p.M - 1;
            srow[i] = r * p.ldsum;
        }
        const uint16_t *mrow[BS_J];
#pragma unroll
        for (int j = 0; j < BS_J; ++j) {
            int c = 16 * j + fr;
            if (c >= 16 * nj) c = 16 * nj - 1;
            int64_t n = n0 + c;
            if (n >= p.N) n = p.N - 1;
            mrow[j] = p.mins + n * p.ldm;
        }
        for (int c = b0 >> 5; c <= (b1 - 1) >> 5; ++c) {
            const int bl = 32 * c + 8 * kg;  // this lane's first block
            h8 xs[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                xs[i][0] = *(const h8 *)(sh + srow[i] + bl);
                xs[i][1] = *(const h8 *)(sl + srow[i] + bl);
            }
            vu4 mq[BS_J];
#pragma unroll
            for (int j = 0; j < BS_J; ++j) mq[j] = *(const vu4 *)(mrow[j] + bl);
            // all of the chunk's loads in flight together (one round trip): the
            // scheduler would otherwise move each tile's loads to its MFMAs
            __builtin_amdgcn_sched_barrier(0);
            uint32_t keep[4];  // the halves of blocks bl + 2 q, bl + 2 q + 1 inside [b0, b1)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                keep[q] = (bl + 2 * q >= b0 && bl + 2 * q < b1 ? 0x0000FFFFu : 0u) |
                          (bl + 2 * q + 1 >= b0 && bl + 2 * q + 1 < b1 ? 0xFFFF0000u : 0u);
#pragma unroll
            for (int j = 0; j < BS_J; ++j) {
                const vu4 mn = {mq[j][0] & keep[0], mq[j][1] & keep[1], mq[j][2] & keep[2], mq[j][3] & keep[3]};
                const h8 mh = __builtin_bit_cast(h8, mn);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    f4 tm = __builtin_amdgcn_mfma_f32_16x16x32_f16(xs[i][0], mh, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    tm = __builtin_amdgcn_mfma_f32_16x16x32_f16(xs[i][1], mh, tm, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(32.0f, tm[r], acc[i][j][r]);
                }
            }
        }
    }

    wait_vmcnt<0>();
    lds_barrier();   // pairs 0 and 1 of every wave's weight copies

    // One interval between barriers per BPI blocks (interval p: blocks BPI p ..):
    // issue the weights of interval p + NB - 1 into buffer (p + NB - 1) % NB
    // (it held interval p - 1, computed before this interval's barrier), then
    // compute interval p from buffer p % NB.
    // - The activation copy of block k + R takes the ring slot of block k once
    //   block k is computed (R - 1 blocks of work ahead of its use); each wave
    //   waits for its own copies only, so no barrier is needed for them.
    // - The weights of interval p + 1 (issued NB - 2 intervals earlier) are
    //   waited for at the end of interval p, before the barrier that publishes them.
    // Copies a wave has issued after the one it waits for (in issue order):
    //   BPI = 2 (R = NB = 3):
    //            A(2p):   B(p+1), A(2p+1), A(2p+2), B(p+2)          = 2 ADMA + 2 BDMA
    //            A(2p+1): A(2p+2), B(p+2), A(2p+3)                  = 2 ADMA + BDMA
    //            B(p+1):  A(2p+1), A(2p+2), B(p+2), A(2p+3), A(2p+4) = 4 ADMA + BDMA
    //   BPI = 1: A(p), issued in interval p - R: then B and A in each of
    //            intervals p - R + 1 .. p - 1, then B(p + NB - 1)     = (R - 1)(ADMA + BDMA) + BDMA
    //            B(p+1), issued in interval p + 2 - NB: then A in that interval,
    //            B and A in each of intervals p + 3 - NB .. p         = (NB - 2)(ADMA + BDMA) + ADMA
    //            (R = NB = 3: 2 ADMA + 3 BDMA and 2 ADMA + BDMA)
    // (each wait on the ring is followed by a compiler memory barrier, so that
    // no ring read is scheduled above it).
    int slot = 0, pb = 0;
    for (int pp = 0; pp < npr; ++pp) {
        const int k = BPI * pp;
        dma_b(pp + NB - 1, pb == 0 ? NB - 1 : pb - 1);
        if constexpr (BPI == 2) {
            wait_vmcnt<2 * BS_ADMA + 2 * BDMA>();
            __asm__ volatile("" ::: "memory");
            compute(slot, pb, 0);
            dma_a(k + 3, slot);
            slot = slot == R - 1 ? 0 : slot + 1;
            wait_vmcnt<2 * BS_ADMA + BDMA>();
            __asm__ volatile("" ::: "memory");
            compute(slot, pb, 1);
            dma_a(k + 4, slot);
            slot = slot == R - 1 ? 0 : slot + 1;
            wait_vmcnt<4 * BS_ADMA + BDMA>();
        } else {
            wait_vmcnt<(R - 1) * (BS_ADMA + BDMA) + BDMA>();
            __asm__ volatile("" ::: "memory");
            compute(slot, pb, 0);
            dma_a(k + R, slot);
            slot = slot == R - 1 ? 0 : slot + 1;
            wait_vmcnt<(NB - 2) * (BS_ADMA + BDMA) + BS_ADMA>();
        }
        lds_barrier();
        pb = pb == NB - 1 ? 0 : pb + 1;
    }
    wait_vmcnt<0>();  // no copy into LDS outlives the workgroup

    // epilogue: lane holds rows 4 (lane >> 4) + r of column lane & 15 of each
    // tile.  Every global read is issued before its stores (row exponents and
    // biases once, residuals per weight tile, at clamped addresses), so the
    // stores, predicated on the row and column, do not wait one round trip each.
    int exr[2][4];
    bool mok[2][4];
    int64_t mrow[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t m = m0 + 16 * i + 4 * kg + r;
            mok[i][r] = m < mend;
            mrow[i][r] = mok[i][r] ? m : p.M - 1;
            exr[i][r] = p.ex[mrow[i][r]];
        }
    int bad_a = 0, bad_b = 0;
#pragma unroll
    for (int j = 0; j < BS_J; ++j) {
        const int64_t n = n0 + 16 * j + fr;
        const bool nok = j < nj && n < p.N;
        const int64_t nc = nok ? n : n0;
        if (p.part) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (nok && mok[i][r])
                        p.part[((int64_t)z * p.M + mrow[i][r]) * p.N + nc] = ldexpf(acc[i][j][r], -exr[i][r]);
            continue;
        }
        const float bias = nc < p.bias_len ? p.bias[nc] : 0.0f;
        float res[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) res[i][r] = p.resid ? p.resid[mrow[i][r] * p.ldr + nc] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = flush_small(ldexpf(acc[i][j][r], -exr[i][r]));
                if (nc < p.bias_len) v = v + bias;
                const bool ok = nok && mok[i][r];
                bad_a |= ok && isnan(v);
                if (p.resid) v = res[i][r] + v;
                bad_b |= ok && isnan(v);
                if (ok) p.y[mrow[i][r] * p.ldy + nc] = v;
            }
    }
    if (p.st) {
        if (__any(bad_a) && lane == 0) nan_flag(p.st, p.layer, p.st_a);
        if (__any(bad_b) && lane == 0) nan_flag(p.st, p.layer, p.st_b);
    }
}

// mins[n][b] = the f16 min of block b of row n (the high half of word b % 4
// of the group's scale words, at byte 64 of its 80), 0 for b >= nb.
__global__ __launch_bounds__(256) void q4_mins_kernel(const uint8_t *w, int64_t N, int nb, uint16_t *mins, int64_t ldm) {
    const int64_t G = (nb + 3) / 4, total = N * ldm;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int64_t n = e / ldm;
        const int b = (int)(e - n * ldm);
        uint16_t v = 0;
        if (b < nb) v = (uint16_t)(*(const uint32_t *)(w + (n * G + (b >> 2)) * 80 + 64 + 4 * (b & 3)) >> 16);
        mins[e] = v;
    }
}

// The product's weight operands from packed Q4_0 rows: per 16-row tile and
// block, the MFMA fragment of its codes as f16 (lane (fr, kg) holds the codes
// of row 16 tile + fr, block b, elements 2 kg + 8 (t & 3) + (t >> 2), t =
// 0..7, the activation plane's order), and the 16 rows' scales as fp32; zero
// past row N and block nb.  One wave per (tile, block).
__global__ __launch_bounds__(256) void q4_frag_kernel(const uint8_t *w, int64_t N, int nb, int64_t nbp4, uint16_t *wf,
                                                      float *wsc) {
    const int lane = threadIdx.x & 63, fr = lane & 15, kg = lane >> 4;
    const int64_t T = (N + 15) / 16, G = (nb + 3) / 4;
    const int64_t chunk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (chunk >= T * nbp4) return;
    const int64_t tile = chunk / nbp4;
    const int b = (int)(chunk - tile * nbp4);
    const int64_t n = 16 * tile + fr;
    vu4 f = {0u, 0u, 0u, 0u};
    float scale = 0.0f;
    if (n < N && b < nb) {
        const uint8_t *grp = w + (n * G + (b >> 2)) * 80;
        const vu4 q = *(const vu4 *)(grp + 16 * kg);
        const int u = b & 3;
        uint32_t wa = u & 2 ? q[1] : q[0], wb = u & 2 ? q[3] : q[2];
        if (u & 1) {
            wa >>= 4;
            wb >>= 4;
        }
        wa &= 0x0F0F0F0Fu;
        wb &= 0x0F0F0F0Fu;
        f = (vu4){code_pair<0>(wa), code_pair<1>(wa), code_pair<0>(wb), code_pair<1>(wb)};
        scale = half_lo(*(const uint32_t *)(grp + 64 + 4 * u));
    }
    *(vu4 *)(wf + chunk * 512 + lane * 8) = f;
    if (kg == 0) wsc[chunk * 16 + fr] = scale;
}

}  // namespace

int64_t q4_frag_nbp4(int64_t K) { return (K / 32 + 3) / 4 * 4; }
int64_t q4_frag_halves(int64_t N, int64_t K) { return (N + 15) / 16 * q4_frag_nbp4(K) * 512; }
int64_t q4_frag_scale_floats(int64_t N, int64_t K) { return (N + 15) / 16 * q4_frag_nbp4(K) * 16; }

int launch_q4_frags(const uint8_t *packed, int64_t N, int64_t K, uint16_t *wf, float *wsc, hipStream_t s) {
    if (!packed || !wf || !wsc || N <= 0 || K <= 0 || K % 32)
        return set_error(GAJE_ERR_INVALID_ARG, "q4 fragments: bad arguments");
    const int64_t chunks = (N + 15) / 16 * q4_frag_nbp4(K);
    if ((chunks + 3) / 4 > 0x7fffffff) return set_error(GAJE_ERR_UNSUPPORTED, "q4 fragments: too many");
    hipLaunchKernelGGL(q4_frag_kernel, dim3((unsigned)((chunks + 3) / 4)), dim3(256), 0, s, packed, N, (int)(K / 32),
                       q4_frag_nbp4(K), wf, wsc);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_q4_row_exponents(const uint8_t *packed, int64_t N, int64_t K, int *ew, hipStream_t s) {
    if (!packed || !ew || N <= 0 || K <= 0 || K % 32) return set_error(GAJE_ERR_INVALID_ARG, "row exponents: bad arguments");
    hipLaunchKernelGGL(q4_row_exp_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, s, packed, N, (int)(K / 32), ew,
                       RowExpBatch{});
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_q4_row_exponents_batch(const uint8_t *const *packed, int n, int64_t N, int64_t K, int *ew, hipStream_t s) {
    if (!packed || !ew || n <= 0 || n > MOE_MAX_EXPERTS || N <= 0 || K <= 0 || K % 32)
        return set_error(GAJE_ERR_INVALID_ARG, "row exponents: bad arguments");
    if (n == 1) return launch_q4_row_exponents(packed[0], N, K, ew, s);
    RowExpBatch b{};
    for (int i = 0; i < n; ++i) {
        if (!packed[i]) return set_error(GAJE_ERR_INVALID_ARG, "row exponents: matrix %d is null", i);
        b.w[i] = packed[i];
    }
    hipLaunchKernelGGL(q4_row_exp_kernel, dim3((unsigned)((N + 3) / 4), (unsigned)n), dim3(256), 0, s, packed[0], N,
                       (int)(K / 32), ew, b);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_split_rows(const SplitParams &p, hipStream_t s) {
    if (p.M < 0 || p.K <= 0 || p.K % 32 || (p.M > 0 && (!p.x || !p.xh || (!p.xl && !p.sh) || !p.ex)) || p.ldx < p.K ||
        p.ldh < (p.sh ? 2 : 1) * p.K)
        return set_error(GAJE_ERR_INVALID_ARG, "split rows: bad arguments");
    if (p.sh && (!p.sl || p.ldsum < gemm_bs_sum_cols(p.K) || p.ldh % 8))
        return set_error(GAJE_ERR_INVALID_ARG, "split rows: bad block-sum planes");
    if (p.M == 0) return GAJE_OK;
    const size_t lds = (size_t)p.K * 4;
    if (lds + 1024 > max_lds_per_block() || p.K > 40960)
        return set_error(GAJE_ERR_UNSUPPORTED, "split rows: K = %lld does not fit LDS", (long long)p.K);
    if (p.up && p.norm_w) return set_error(GAJE_ERR_INVALID_ARG, "split rows: norm and swiglu prologues are exclusive");
    if (p.part && (p.up || p.rows || p.nsplit < 1 || p.ldx != p.K || (p.resid && p.resid != p.x) || p.bias_len < 0 ||
                   (p.bias_len > 0 && !p.bias) || ((uintptr_t)p.part & 15)))
        return set_error(GAJE_ERR_INVALID_ARG, "split rows: bad split-K prologue");
    if (p.attn_ws && (p.up || p.norm_w || p.part || p.rows || p.attn_hd <= 0 || p.attn_hd % 4 || p.attn_heads <= 0 ||
                      (int64_t)p.attn_heads * p.attn_hd != p.K || p.attn_kch <= 0 || p.attn_pos0 < 0 ||
                      (p.attn_pos0 + p.M + p.attn_kch - 1) / p.attn_kch > PREFILL_ATTN_CHUNKS))
        return set_error(GAJE_ERR_INVALID_ARG, "split rows: bad attention-merge prologue");
    // threads x float4s per thread covering the row: 256 x 2, 256 x 4, 1024 x 4, 1024 x 10
    const int64_t K4 = p.K / 4;
    const dim3 grid((unsigned)p.M);
    auto go = [&](auto pro) {
        constexpr int PRO = decltype(pro)::value;
        if (K4 <= 512) split_rows_kernel<PRO, 256, 2><<<grid, dim3(256), lds, s>>>(p);
        else if (K4 <= 1024) split_rows_kernel<PRO, 256, 4><<<grid, dim3(256), lds, s>>>(p);
        else if (K4 <= 4096) split_rows_kernel<PRO, 1024, 4><<<grid, dim3(1024), lds, s>>>(p);
        else split_rows_kernel<PRO, 1024, 10><<<grid, dim3(1024), lds, s>>>(p);
    };
    if (p.up) go(std::integral_constant<int, SPLIT_SWIGLU>{});
    else if (p.norm_w) go(std::integral_constant<int, SPLIT_NORM>{});
    else go(std::integral_constant<int, SPLIT_PLAIN>{});
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

// The 128-row product reads its activation fragments from global memory.
constexpr bool GEMM_GA = true;

GemmPlan plan_gemm_q4(int64_t M, int64_t N, int64_t K) {
    GemmPlan pl{};
    pl.mt = M > 128 ? 256 : 128;
    const int64_t tiles = ((M + pl.mt - 1) / pl.mt) * ((N + GM_NT - 1) / GM_NT);
    const int64_t nb = K / 32;
    // resident workgroups: the 256-row tile's LDS allows one per compute unit
    const int64_t cu = (pl.mt == 128 && GEMM_GA ? 2 : 1) * device_cu_count();
    int64_t S = 1;
    if (tiles < cu) S = (cu + tiles - 1) / tiles;
    int64_t kb = (nb + S - 1) / S;
    if (kb < 8) kb = 8;          // at least two weight groups per split
    kb = (kb + 3) / 4 * 4;       // splits start on group boundaries
    pl.kb_per = (int)kb;
    pl.splits = (int)((nb + kb - 1) / kb);
    pl.part_floats = pl.splits > 1 ? pl.splits * M * N : 0;
    return pl;
}

GemmPlan plan_gemm_q4_grouped(int64_t R, int64_t E, int64_t N, int64_t K) {
    GemmPlan pl{};
    // 128-row tiles although the experts hold R/E rows on average (64 at the
    // benchmark's 256 tokens x top-2 over 8 experts): each workgroup
    // dequantises its 128 weight rows once, and 64-row tiles, which dequantise
    // them once per 64 rows, measured slower (343 against 259 us per layer)
    pl.mt = 128;
    // tiles that hold rows: at most R/128 full ones plus one partial per group
    const int64_t tiles = ((R + 127) / 128 + E) * ((N + GM_NT - 1) / GM_NT);
    const int64_t nb = K / 32;
    const int64_t cu = (GEMM_GA ? 2 : 1) * device_cu_count();  // resident 128-row workgroups
    int64_t S = 1;
    if (tiles < cu) S = (cu + tiles - 1) / tiles;
    int64_t kb = (nb + S - 1) / S;
    if (kb < 8) kb = 8;
    kb = (kb + 3) / 4 * 4;
    pl.kb_per = (int)kb;
    pl.splits = (int)((nb + kb - 1) / kb);
    pl.part_floats = pl.splits > 1 ? pl.splits * R * N : 0;
    return pl;
}

int64_t gemm_bs_sum_cols(int64_t K) { return (K / 32 + 31) / 32 * 32; }

int launch_q4_mins(const uint8_t *packed, int64_t N, int64_t K, uint16_t *mins, int64_t ldm, hipStream_t s) {
    if (!packed || !mins || N <= 0 || K <= 0 || K % 32 || ldm < gemm_bs_sum_cols(K) || N * ldm >= ((int64_t)1 << 40))
        return set_error(GAJE_ERR_INVALID_ARG, "q4 block mins: bad arguments");
    const int64_t total = N * ldm;
    int64_t g = (total + 255) / 256;
    if (g > 65536) g = 65536;
    hipLaunchKernelGGL(q4_mins_kernel, dim3((unsigned)g), dim3(256), 0, s, packed, N, (int)(K / 32), mins, ldm);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}
int64_t gemm_bs_plane_rows(int64_t M) { return (M + 255) / 256 * 256; }

GemmBsPlan plan_gemm_q4_bs(int64_t M, int64_t N, int64_t K) {
    GemmBsPlan pl{};
    // 256-row tiles of eight waves, one workgroup per compute unit; below 129
    // rows 128- or 64-row tiles, two workgroups per compute unit
    pl.waves = M <= 64 ? 2 : (M <= 128 ? 4 : 8);
    const int64_t mt = BS_WR * pl.waves;
    pl.mtiles = (int)((M + mt - 1) / mt);
    const int64_t units = (N + 15) / 16;
    pl.ntiles = (int)((units + BS_J - 1) / BS_J);
    const int64_t tiles = (int64_t)pl.mtiles * pl.ntiles;
    const int64_t nb = K / 32;
    const int64_t cu = (pl.waves == 8 ? 1 : 2) * device_cu_count();  // resident workgroups
    const int64_t S = tiles < cu ? cu / tiles : 1;
    int64_t kb = (nb + S - 1) / S;
    kb = (kb + 3) / 4 * 4;  // splits start on group boundaries
    if (kb < 4) kb = 4;
    pl.kb_per = (int)kb;
    pl.splits = (int)((nb + kb - 1) / kb);
    pl.part_floats = pl.splits > 1 ? (int64_t)pl.splits * M * N : 0;
    return pl;
}

GemmBsPlan plan_gemm_q4_bs_grouped(int64_t R, int64_t E, int64_t T, int64_t N, int64_t K) {
    GemmBsPlan pl{};
    // the tile height follows the mean group: up to 1.5x the mean fits one
    // tile, so most groups read their weight operands once (the MoE's 256
    // tokens x top-2 over 8 experts: 52-80 rows each, one 128-row tile;
    // measured 164 us per layer against 217 with 64-row tiles, which split
    // half of the experts in two, and 234 with 256-row tiles); a group holds
    // at most T rows, so every group has T / tile row tiles in the grid, and
    // the empty ones return at once
    const int64_t mean = (R + E - 1) / E;
    pl.waves = mean <= 32 ? 2 : (mean <= 96 ? 4 : 8);
    const int64_t mt = BS_WR * pl.waves;
    pl.mtiles = (int)(E * ((T + mt - 1) / mt));
    const int64_t units = (N + 15) / 16;
    pl.ntiles = (int)((units + BS_J - 1) / BS_J);
    const int64_t active = ((R + mt - 1) / mt + E - 1) * pl.ntiles;  // tiles holding rows, at most
    const int64_t nb = K / 32;
    const int64_t cu = (pl.waves == 8 ? 1 : 2) * device_cu_count();
    const int64_t S = active < cu ? cu / active : 1;
    int64_t kb = (nb + S - 1) / S;
    kb = (kb + 3) / 4 * 4;
    if (kb < 4) kb = 4;
    pl.kb_per = (int)kb;
    pl.splits = (int)((nb + kb - 1) / kb);
    pl.part_floats = pl.splits > 1 ? (int64_t)pl.splits * R * N : 0;
    return pl;
}

int launch_gemm_q4_bs(const GemmBsParams &p, const GemmBsPlan &pl, hipStream_t s) {
    if (p.M < 0 || p.N <= 0 || p.nb <= 0 || !p.wf || !p.wsc || p.nbp4 != q4_frag_nbp4(32 * (int64_t)p.nb) ||
        (p.M > 0 && (!p.xh || !p.sh || !p.sl || !p.ex || !p.y || p.ldh < 64 * (int64_t)p.nb ||
                     p.ldsum < gemm_bs_sum_cols(32 * (int64_t)p.nb))))
        return set_error(GAJE_ERR_INVALID_ARG, "q4 block-scaled gemm: bad arguments");
    if (p.M > 0 && (!p.mins || p.ldm < gemm_bs_sum_cols(32 * (int64_t)p.nb)))
        return set_error(GAJE_ERR_INVALID_ARG, "q4 block-scaled gemm: no block mins");
    if ((((uintptr_t)p.xh | (uintptr_t)p.sh | (uintptr_t)p.sl | (uintptr_t)p.mins) & 15) || p.ldh % 8 || p.ldsum % 8 ||
        p.ldm % 8)
        return set_error(GAJE_ERR_INVALID_ARG, "q4 block-scaled gemm: planes must be 16-byte aligned");
    if (p.M == 0) return GAJE_OK;
    const int64_t mt = BS_WR * (int64_t)pl.waves;
    const bool grouped = p.g_counts != nullptr;
    if (grouped && (!p.g_offsets || p.g_groups <= 0 || p.g_groups > MOE_MAX_EXPERTS || p.g_mtiles <= 0 ||
                    pl.mtiles != (int64_t)p.g_groups * p.g_mtiles || p.g_wf_stride % 512 || p.g_wsc_stride % 16 ||
                    p.g_mins_stride % 8 || p.g_wf_stride < q4_frag_halves(p.N, 32 * (int64_t)p.nb) ||
                    p.g_wsc_stride < q4_frag_scale_floats(p.N, 32 * (int64_t)p.nb) || p.g_mins_stride < p.N * p.ldm))
        return set_error(GAJE_ERR_INVALID_ARG, "q4 block-scaled gemm: bad groups");
    // rows read: a grouped tile starts inside the M rows and reads one tile on
    const int64_t rows_read = grouped ? p.M + (int64_t)p.g_mtiles * mt : (int64_t)pl.mtiles * mt;
    if (p.plane_rows < rows_read)
        return set_error(GAJE_ERR_INVALID_ARG, "q4 block-scaled gemm: the activation plane holds %lld rows, the tiles read %lld",
                         (long long)p.plane_rows, (long long)rows_read);
    if (2 * p.plane_rows * p.ldh >= ((int64_t)1 << 32) ||
        2 * q4_frag_halves(p.N, 32 * (int64_t)p.nb) >= ((int64_t)1 << 32))
        return set_error(GAJE_ERR_UNSUPPORTED, "q4 block-scaled gemm: operands beyond 4 GiB");
    if (((uintptr_t)p.wf | (uintptr_t)p.wsc) & 15)
        return set_error(GAJE_ERR_INVALID_ARG, "q4 block-scaled gemm: weight fragments must be 16-byte aligned");
    if ((pl.waves != 2 && pl.waves != 4 && pl.waves != 8) || (!grouped && pl.mtiles != (p.M + mt - 1) / mt) || pl.ntiles <= 0 ||
        pl.ntiles * (int64_t)BS_J < (p.N + 15) / 16 || pl.kb_per % 4 || pl.kb_per <= 0 ||
        (int64_t)pl.splits * pl.kb_per < p.nb || (int64_t)(pl.splits - 1) * pl.kb_per >= p.nb ||
        (pl.splits > 1 && !p.part))
        return set_error(GAJE_ERR_INVALID_ARG, "q4 block-scaled gemm: bad plan");
    GemmBsParams q = p;
    if (pl.splits == 1) q.part = nullptr;
    BsGrid gd{};
    gd.ntiles = pl.ntiles;
    gd.splits = pl.splits;
    gd.kb_per = pl.kb_per;
    gd.units = (int32_t)((p.N + 15) / 16);
    const int64_t total = (int64_t)pl.mtiles * pl.splits * pl.ntiles;
    if (total > (1 << 30)) return set_error(GAJE_ERR_UNSUPPORTED, "q4 block-scaled gemm: too many tiles");
    gd.total = (int32_t)total;
    const dim3 grid((unsigned)((total + 7) / 8 * 8));
    if (bs_lds<8, 2>() > max_lds_per_block()) return set_error(GAJE_ERR_UNSUPPORTED, "q4 block-scaled gemm: LDS");
    switch (pl.waves) {
    case 2:
        gemm_q4_bs_kernel<2, 1><<<grid, dim3(128), bs_lds<2, 1>(), s>>>(q, gd);
        break;
    case 4:
        // grouped (expert) tiles: a two-slot activation ring measured ~2% faster
        // (a deeper weight ring, four buffers, measured the same as three)
        if (grouped)
            gemm_q4_bs_kernel<4, 1, 2, 3><<<grid, dim3(256), bs_lds<4, 1, 2, 3>(), s>>>(q, gd);
        else
            gemm_q4_bs_kernel<4, 1><<<grid, dim3(256), bs_lds<4, 1>(), s>>>(q, gd);
        break;
    default:
        gemm_q4_bs_kernel<8, 2><<<grid, dim3(512), bs_lds<8, 2>(), s>>>(q, gd);
        break;
    }
    GAJE_HIP_CHECK(hipGetLastError());
    if (pl.splits > 1 && !p.defer_reduce) {
        GemmQ4Params r{};
        r.bias = p.bias;
        r.bias_len = p.bias_len;
        r.resid = p.resid;
        r.ldr = p.ldr;
        r.y = p.y;
        r.ldy = p.ldy;
        r.part = p.part;
        r.M = p.M;
        r.N = p.N;
        r.st = p.st;
        r.layer = p.layer;
        r.st_a = p.st_a;
        r.st_b = p.st_b;
        const int64_t elems = p.M * p.N;
        int64_t g = (elems + 255) / 256;
        if (g > 4096) g = 4096;
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)g), dim3(256), 0, s, r, pl.splits);
        GAJE_HIP_CHECK(hipGetLastError());
    }
    return GAJE_OK;
}

int launch_gemm_q4(const GemmQ4Params &p0, const GemmPlan &pl, hipStream_t s) {
    GemmQ4Params p = p0;
    const bool grouped = p.g_counts != nullptr;
    if (p.M < 0 || p.N <= 0 || p.nb <= 0 || (!grouped && (!p.w || !p.ew)) ||
        (grouped && (!p.g_offsets || p.g_groups <= 0 || p.g_groups > MOE_MAX_EXPERTS || p.g_mtiles <= 0 || pl.mt != 128)) ||
        (p.M > 0 && (!p.xh || !p.xl || !p.ex || !p.y)))
        return set_error(GAJE_ERR_INVALID_ARG, "q4 gemm: bad arguments");
    if (grouped)
        for (int e = 0; e < p.g_groups; ++e)
            if (!p.gw[e] || !p.gew[e]) return set_error(GAJE_ERR_INVALID_ARG, "q4 gemm: group %d has no weights", e);
    if (p.M == 0) return GAJE_OK;
    if (pl.kb_per % 4 || pl.kb_per <= 0 || (int64_t)pl.splits * pl.kb_per < p.nb || (pl.splits > 1 && !p.part))
        return set_error(GAJE_ERR_INVALID_ARG, "q4 gemm: bad plan");
    p.kb_per = pl.kb_per;
    if (pl.splits == 1) p.part = nullptr;
    const unsigned gy = grouped ? (unsigned)(p.g_groups * p.g_mtiles) : (unsigned)((p.M + pl.mt - 1) / pl.mt);
    const dim3 grid((unsigned)((p.N + GM_NT - 1) / GM_NT), gy, (unsigned)pl.splits);
    if (pl.mt == 256) {
        const size_t lds = gemm_lds<256, false>();
        if (lds + 1024 > max_lds_per_block()) return set_error(GAJE_ERR_UNSUPPORTED, "q4 gemm: LDS");
        hipLaunchKernelGGL((gemm_q4_mfma_kernel<256, false>), grid, dim3(512), lds, s, p);
    } else {
        const size_t lds = gemm_lds<128, GEMM_GA>();
        hipLaunchKernelGGL((gemm_q4_mfma_kernel<128, GEMM_GA>), grid, dim3(256), lds, s, p);
    }
    GAJE_HIP_CHECK(hipGetLastError());
    if (pl.splits > 1) {
        const int64_t total = p.M * p.N;
        int64_t g = (total + 255) / 256;
        if (g > 4096) g = 4096;
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)g), dim3(256), 0, s, p, pl.splits);
        GAJE_HIP_CHECK(hipGetLastError());
    }
    return GAJE_OK;
}

}  // namespace gaje
