// Bit-exact fused matvec for batch-1 decode on gfx950 (wave64).
//
// Every output row is computed with the reference's own rounding sequence:
//   Q4_0   genomic_dot_product_q4_0_avx2 (genomic.rs:263-336): eight FMA chains
//          (AVX lane l takes element 8c+l of every block's chunk c), each element
//          dequantised with fma(q, scale, min), chains walked block by block in
//          order, reduced ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)), |t|<1e-6 -> 0;
//   f32    dot_product (dot.rs:43-67): eight FMA chains over 8-float chunks,
//          reduced ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)), then the scalar tail;
//   LUT    genomic_dot_product_4bit (genomic.rs:148-204): four mul-then-add
//          chains (element e goes to chain e % 4), summed left to right, flush;
// followed by compute_single_row's anchors and bias (linear/forward.rs:103-115).
// The fused prologue restates rms_norm's eight-chain sum of squares
// (norm.rs:52-88); the epilogues restate the block's residual adds, SwiGLU and
// the QKV split with RoPE (block/forward.rs:57-136, attention.rs:62-86).
// Device code is compiled without FP contraction, so every a*b+c the reference
// rounds twice is rounded twice here, and every fma is an explicit fmaf.
//
// Work mapping.  A chain is serial by construction, so parallelism comes from
// rows and chains: LPR lanes cooperate on one row (one or more chains each) and
// walk the row's blocks in order; 2*LPR lanes hold a row pair (the RoPE / SwiGLU
// partners or two consecutive rows), so the pair's epilogue runs in one lane.
// The activation vector sits in LDS; weights stream straight from HBM in their
// file packing.
#include "common.h"
#include "device_util.h"

namespace gaje {

namespace {

constexpr int THREADS = 256;
constexpr int MAX_GRID = 8192;

__device__ __forceinline__ void pair_rows(const GemvParams &p, int64_t pr, int64_t &r0, int64_t &r1) {
    if (p.mode == MODE_QKV) {
        const int half = p.head_dim >> 1;
        const int64_t head = pr / half;
        const int64_t i = pr - head * half;
        if (p.rope_split) {
            r0 = head * p.head_dim + i;
            r1 = r0 + half;
        } else {
            r0 = head * p.head_dim + 2 * i;
            r1 = r0 + 1;
        }
    } else if (p.mode == MODE_SWIGLU) {
        r0 = pr;
        r1 = pr + p.ffn;
    } else {
        r0 = 2 * pr;
        r1 = (2 * pr + 1 < p.N) ? 2 * pr + 1 : -1;
    }
}

__device__ __forceinline__ float shfl(float v, int src) { return __shfl(v, src, WAVE); }

// ---------------------------------------------------------------- Q4_0 ----
// LPR = 8: lane s owns chain s.  LPR = 4: lane p owns chains 2p and 2p+1.
template <int LPR, bool NT>
__device__ __forceinline__ float row_q4_0(const GemvParams &p, const float *xs, int64_t row, int s, int base) {
    constexpr int CH = 8 / LPR;  // chains per lane
    float acc[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) acc[i] = 0.0f;
    const uint8_t *rowp = p.w + (size_t)row * p.nb * 20;
    for (int j = 0; j < p.nb; ++j) {
        const uint8_t *blk = rowp + (size_t)j * 20;
        const uint32_t sm = ld_u32<NT>(blk);
        const uint32_t qc[4] = {ld_u32<NT>(blk + 4), ld_u32<NT>(blk + 8), ld_u32<NT>(blk + 12), ld_u32<NT>(blk + 16)};
        const float scale = half_lo(sm), mn = half_hi(sm);
        const float *xb = xs + (size_t)j * 32;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const int chain = (LPR == 8) ? s : 2 * s + i;  // element 8c + chain of the block
                const uint32_t nib = __builtin_amdgcn_ubfe(qc[c], 8 * (chain >> 1) + 4 * (chain & 1), 4);
                const float d = fmaf((float)nib, scale, mn);
                acc[i] = fmaf(d, xb[8 * c + chain], acc[i]);
            }
        }
    }
    float total;
    if constexpr (LPR == 8) {
        const float a = acc[0];
        const float u = a + shfl(a, base + ((s + 4) & 7));  // lane l<4: a_l + a_{l+4}
        const float v = u + shfl(u, base + ((s + 2) & 7));  // lane 0: u0+u2, lane 1: u1+u3
        total = v + shfl(v, base + ((s + 1) & 7));          // lane 0: (u0+u2) + (u1+u3)
    } else {
        // lane p holds chains (2p, 2p+1)
        const float u0 = acc[0] + shfl(acc[0], base + ((s + 2) & 3));  // lane 0: a0+a4, lane 1: a2+a6
        const float u1 = acc[1] + shfl(acc[1], base + ((s + 2) & 3));  // lane 0: a1+a5, lane 1: a3+a7
        const float v0 = u0 + shfl(u0, base + ((s + 1) & 3));          // lane 0: (a0+a4)+(a2+a6)
        const float v1 = u1 + shfl(u1, base + ((s + 1) & 3));          // lane 0: (a1+a5)+(a3+a7)
        total = v0 + v1;
    }
    return flush_small(total);
}

// ----------------------------------------------------------------- f32 ----
// LPR = 2: lane h owns chains 4h..4h+3 (one float4 of each 8-float chunk).
template <bool NT>
__device__ __forceinline__ float row_f32(const GemvParams &p, const float *xs, int64_t row, int s, int base) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    const float *wr = (const float *)p.w + (size_t)row * p.K;
    const int64_t chunks = p.K / 8;
    for (int64_t t = 0; t < chunks; ++t) {
        const float4 w = ld_f4<NT>(wr + 8 * t + 4 * s);
        const float4 x = *(const float4 *)(xs + 8 * t + 4 * s);
        a0 = fmaf(x.x, w.x, a0);
        a1 = fmaf(x.y, w.y, a1);
        a2 = fmaf(x.z, w.z, a2);
        a3 = fmaf(x.w, w.w, a3);
    }
    // lane 0 holds chains 0..3, lane 1 chains 4..7: ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7))
    const float u0 = a0 + shfl(a0, base + 1), u1 = a1 + shfl(a1, base + 1);
    const float u2 = a2 + shfl(a2, base + 1), u3 = a3 + shfl(a3, base + 1);
    float sum = (u0 + u1) + (u2 + u3);
    for (int64_t i = chunks * 8; i < p.K; ++i) {  // scalar tail, mul then add
        const float prod = xs[i] * wr[i];
        sum = sum + prod;
    }
    return sum;
}

// ----------------------------------------------------------------- LUT ----
// LPR = 4: lane m owns chain m (elements e of a block with e % 4 == m).  The
// block's 16-entry table goes through this row group's LDS slot.
template <bool NT>
__device__ __forceinline__ float row_lut4(const GemvParams &p, const float *xs, int64_t row, int s, int base,
                                          float *tbl) {
    float acc = 0.0f;
    const uint8_t *rowp = p.w + (size_t)row * p.nb * 16;
    const float *lrow = p.lut + (row < p.lut_rows_own ? (size_t)row * p.nb * 16 : 0);
    for (int j = 0; j < p.nb; ++j) {
        const uint8_t *blk = rowp + (size_t)j * 16;
        const uint32_t c[4] = {ld_u32<NT>(blk), ld_u32<NT>(blk + 4), ld_u32<NT>(blk + 8), ld_u32<NT>(blk + 12)};
        const float4 tv = ld_f4<NT>(lrow + (size_t)j * p.lut_block_stride + 4 * s);
        *(float4 *)(tbl + 4 * s) = tv;
        __builtin_amdgcn_wave_barrier();
        const float *xb = xs + (size_t)j * 32;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int e = 4 * t + s;  // element; even e = high nibble of byte e/2
            const int byte = e >> 1;
            const uint32_t idx = __builtin_amdgcn_ubfe(c[byte >> 2], 8 * (byte & 3) + ((e & 1) ? 0 : 4), 4);
            const float prod = tbl[idx] * xb[e];
            acc = acc + prod;
        }
        __builtin_amdgcn_wave_barrier();
    }
    const float s1 = shfl(acc, base + 1), s2 = shfl(acc, base + 2), s3 = shfl(acc, base + 3);
    const float total = ((acc + s1) + s2) + s3;  // s0 + s1 + s2 + s3, left to right
    return flush_small(total);
}

__device__ __forceinline__ float finish_row(const GemvParams &p, const float *xs, int64_t r, float v) {
    if (p.a_ptr) {
        for (int64_t k = p.a_ptr[r]; k < p.a_ptr[r + 1]; ++k) {
            const float prod = xs[p.a_col[k]] * half_bits(p.a_val[k]);
            v = v + prod;
        }
    }
    if (r < p.bias_len) v = v + p.bias[r];
    return v;
}

template <int FMT, int LPR, bool NT>
__global__ __launch_bounds__(THREADS) void gemv_kernel(GemvParams p, int64_t npairs) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float inv_slot;
    DevState *st = p.st;
    if (st && st->halted) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K = p.K;
    float *xs = smem;

    // ---- prologue: activation vector into LDS (normalised if requested) ----
    int bad_in = 0;
    for (int64_t k = tid; k < K; k += THREADS) {
        const float v = p.x[k];
        xs[k] = v;
        bad_in |= isnan(v);
    }
    if (__syncthreads_or(bad_in) && p.st_in >= 0 && tid == 0) nan_flag(st, p.layer, p.st_in);
    if (p.norm_w) {
        rmsnorm_inplace(xs, K, p.norm_w, p.eps, &inv_slot);
        int bad = 0;
        for (int64_t k = tid; k < K; k += THREADS) bad |= isnan(xs[k]);
        if (__syncthreads_or(bad) && p.st_norm >= 0 && tid == 0) nan_flag(st, p.layer, p.st_norm);
    }
    if (p.gnorm) {
        // use_genomic_norm (block/forward.rs:115-123) sums with a rayon
        // reduction whose order is not fixed upstream; a sequential sum here.
        if (tid == 0) {
            float ss = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float sq = xs[k] * xs[k];
                ss = ss + sq;
            }
            inv_slot = sqrtf(ss / (float)K + p.eps);
        }
        __syncthreads();
        const float rms = inv_slot;
        if (rms > p.h_scale) {
            const float sc = p.h_scale / rms;
            for (int64_t k = tid; k < K; k += THREADS) xs[k] = xs[k] * sc;
        }
    }
    __syncthreads();
    if (p.x_out && blockIdx.x == 0)
        for (int64_t k = tid; k < K; k += THREADS) p.x_out[k] = xs[k];

    // ---- row pairs ----
    constexpr int PAIR_LANES = 2 * LPR;
    constexpr int PAIRS_PER_WAVE = WAVE / PAIR_LANES;
    const int pslot = lane / PAIR_LANES;
    const int half = (lane % PAIR_LANES) / LPR;
    const int s = lane % LPR;
    const int row_base = lane - s;  // first lane of this row's group
    const int pair_base = pslot * PAIR_LANES;
    const int pairs_per_block = PAIRS_PER_WAVE * (THREADS / WAVE);
    float *tbl = smem + ((K + 3) & ~(int64_t)3) + (size_t)(tid / LPR) * 16;  // LUT slot of this row group

    float best_v = -INFINITY;
    int64_t best_i = 0;

    for (int64_t pr0 = (int64_t)blockIdx.x * pairs_per_block; pr0 < npairs; pr0 += (int64_t)gridDim.x * pairs_per_block) {
        const int64_t pr = pr0 + wave * PAIRS_PER_WAVE + pslot;
        const bool pair_ok = pr < npairs;
        int64_t r0 = 0, r1 = -1;
        if (pair_ok) pair_rows(p, pr, r0, r1);
        const int64_t row = half ? r1 : r0;
        const bool has_work = (FMT == FMT_F32) ? p.K > 0 : p.nb > 0;
        const bool row_ok = pair_ok && row >= 0 && row < p.rows_valid && has_work;
        float v = 0.0f;
        // all lanes of a row group share row_ok, so each row function's
        // shuffles only read lanes that execute it
        if (row_ok) {
            if constexpr (FMT == FMT_Q4_0) v = row_q4_0<LPR, NT>(p, xs, row, s, row_base);
            else if constexpr (FMT == FMT_F32) v = row_f32<NT>(p, xs, row, s, row_base);
            else v = row_lut4<NT>(p, xs, row, s, row_base, tbl);
        }
        const float v1 = shfl(v, pair_base + LPR);  // r1's result (lane 0 of its group)
        if (!pair_ok || lane != pair_base) continue;

        // ---- epilogue (one lane per row pair) ----
        const float y0 = finish_row(p, xs, r0, v);
        const float y1 = r1 >= 0 ? finish_row(p, xs, r1, v1) : 0.0f;
        switch (p.mode) {
            case MODE_STORE:
                p.y[r0] = y0;
                if (r1 >= 0) p.y[r1] = y1;
                break;
            case MODE_RESIDUAL: {
                if (isnan(y0) || (r1 >= 0 && isnan(y1))) nan_flag(st, p.layer, p.st_a);
                const float h0 = p.y[r0] + y0;
                p.y[r0] = h0;
                bool bad = isnan(h0);
                if (r1 >= 0) {
                    const float h1 = p.y[r1] + y1;
                    p.y[r1] = h1;
                    bad |= isnan(h1);
                }
                if (bad) nan_flag(st, p.layer, p.st_b);
                break;
            }
            case MODE_QKV: {
                // attention.rs:62-82 with the host-built cos/sin table:
                // (v0*cos - v1*sin, v0*sin + v1*cos), every product rounded.
                const int hh = p.head_dim >> 1;
                const int pos = st->pos;
                const int i = (int)(pr % hh);
                const float cs = p.rope_cos[(size_t)pos * hh + i], sn = p.rope_sin[(size_t)pos * hh + i];
                const float t0 = y0 * cs, t1 = y1 * sn, t2 = y0 * sn, t3 = y1 * cs;
                const float o0 = t0 - t1, o1 = t2 + t3;
                if (r0 < p.q_rows) {
                    p.q_out[r0] = o0;
                    p.q_out[r1] = o1;
                } else if (r0 < p.q_rows + p.kv_rows) {
                    const int64_t kh = (r0 - p.q_rows) / p.head_dim;
                    const int64_t b = p.q_rows + kh * p.head_dim;
                    float *kc = p.k_cache + kh * p.kv_head_stride + (size_t)pos * p.head_dim;
                    kc[r0 - b] = o0;
                    kc[r1 - b] = o1;
                } else {
                    const int64_t vh = (r0 - p.q_rows - p.kv_rows) / p.head_dim;
                    const int64_t b = p.q_rows + p.kv_rows + vh * p.head_dim;
                    float *vc = p.v_cache + vh * p.kv_head_stride + (size_t)pos * p.head_dim;
                    vc[r0 - b] = y0;
                    vc[r1 - b] = y1;
                }
                break;
            }
            case MODE_SWIGLU: {
                if (isnan(y1)) nan_flag(st, p.layer, p.st_a);
                const float o = swiglu1(y0, y1);
                if (isnan(o)) nan_flag(st, p.layer, p.st_b);
                p.y[pr] = o;
                break;
            }
            case MODE_ARGMAX: {
                p.y[r0] = y0;
                if (y0 > best_v) { best_v = y0; best_i = r0; }
                if (r1 >= 0) {
                    p.y[r1] = y1;
                    if (y1 > best_v) { best_v = y1; best_i = r1; }
                }
                break;
            }
        }
    }
    if (p.mode == MODE_ARGMAX && st) {
        unsigned long long key =
            best_v > -INFINITY
                ? ((unsigned long long)order_key(best_v) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)best_i)
                : 0ull;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(key, o, WAVE);
            key = other > key ? other : key;
        }
        if (lane == 0 && key) atomicMax(&st->argmax_key, key);
    }
}

using KernelFn = void (*)(GemvParams, int64_t);

}  // namespace

size_t gemv_lds_bytes(int64_t K, int fmt) {
    size_t b = (size_t)((K + 3) & ~(int64_t)3) * 4;
    if (fmt == FMT_LUT4) b += (size_t)(THREADS / 4) * 16 * 4;  // one 16-entry table per row group
    return b;
}

int launch_gemv(const GemvParams &p, hipStream_t s) {
    if (p.N < 0 || p.K <= 0 || !p.x || !p.y)
        return set_error(GAJE_ERR_INVALID_ARG, "gemv: invalid shape or null buffer");
    if (p.nb != (int32_t)(p.K / 32)) return set_error(GAJE_ERR_INVALID_ARG, "gemv: nb must be K/32");
    if (p.fmt == FMT_F32 && p.K % 4 != 0)
        return set_error(GAJE_ERR_UNSUPPORTED, "gemv: f32 rows need in_features %% 4 == 0 (got %lld)",
                         (long long)p.K);
    if (p.rows_valid > 0 && !p.w) return set_error(GAJE_ERR_INVALID_ARG, "gemv: null weights");
    if (p.fmt == FMT_LUT4 && p.nb > 0 && p.rows_valid > 0 && !p.lut)
        return set_error(GAJE_ERR_INVALID_ARG, "gemv: null LUT");
    const size_t lds = gemv_lds_bytes(p.K, p.fmt);
    if (lds + 1024 > 64 * 1024)  // dynamic + the kernel's static LDS within 64 KiB
        return set_error(GAJE_ERR_UNSUPPORTED, "gemv: in_features %lld exceeds the LDS budget", (long long)p.K);
    int64_t npairs;
    switch (p.mode) {
        case MODE_QKV:
            if (!p.st || p.head_dim <= 0 || p.head_dim % 2 || p.q_rows % p.head_dim || p.kv_rows % p.head_dim ||
                p.N < p.q_rows + 2 * p.kv_rows || !p.q_out || !p.k_cache || !p.v_cache || !p.rope_cos || !p.rope_sin)
                return set_error(GAJE_ERR_INVALID_ARG, "gemv: bad fused-QKV arguments");
            npairs = (p.q_rows + 2 * p.kv_rows) / 2;
            break;
        case MODE_SWIGLU:
            if (p.ffn <= 0 || 2 * p.ffn > p.N) return set_error(GAJE_ERR_INVALID_ARG, "gemv: bad SwiGLU arguments");
            npairs = p.ffn;
            break;
        case MODE_ARGMAX:
            if (!p.st) return set_error(GAJE_ERR_INVALID_ARG, "gemv: argmax needs the device state");
            npairs = (p.N + 1) / 2;
            break;
        case MODE_STORE:
        case MODE_RESIDUAL:
            npairs = (p.N + 1) / 2;
            break;
        default:
            return set_error(GAJE_ERR_INVALID_ARG, "gemv: unknown mode %d", p.mode);
    }
    if (npairs == 0) return GAJE_OK;
    KernelFn fn;
    int lpr;
    if (p.fmt == FMT_Q4_0) {
        // one chain per lane when rows are few (more lanes in flight), two otherwise
        const bool few_rows = npairs < 2048;
        lpr = few_rows ? 8 : 4;
        fn = few_rows ? gemv_kernel<FMT_Q4_0, 8, false> : gemv_kernel<FMT_Q4_0, 4, false>;
    } else if (p.fmt == FMT_LUT4) {
        lpr = 4;
        fn = gemv_kernel<FMT_LUT4, 4, false>;
    } else {
        lpr = 2;
        fn = p.nontemporal ? gemv_kernel<FMT_F32, 2, true> : gemv_kernel<FMT_F32, 2, false>;
    }
    const int64_t pairs_per_block = (WAVE / (2 * lpr)) * (THREADS / WAVE);
    int64_t grid = (npairs + pairs_per_block - 1) / pairs_per_block;
    if (grid > MAX_GRID) grid = MAX_GRID;
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(THREADS), lds, s, p, npairs);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
