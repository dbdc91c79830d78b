// Fused matvec for batch-1 decode on gfx950 (wave64).
//
// One kernel template serves every GEMV of the decode step:
//   prologue  x -> LDS, optional rms_norm (norm.rs:17-131) with the block's NaN
//             guards, optional use_genomic_norm scaling (block/forward.rs:115-123);
//   body      the row dot of compute_single_row (linear/forward.rs:11-117) for
//             Q4_0 blocks (genomic.rs:263-336), LUT-4bit blocks (genomic.rs:148-204)
//             or f32 rows (dot.rs:23-94);
//   epilogue  flush |t| < 1e-6 (4-bit formats), sparse anchors, bias, then one of:
//             store, residual add (block/forward.rs:78-82,132-136), fused QKV with
//             RoPE and KV append (attention.rs:62-86), fused SwiGLU
//             (block/forward.rs:87-109), or logits + greedy argmax.
//
// Work mapping.  Rows are processed in pairs (the RoPE and SwiGLU partners of
// the fused epilogues, or two consecutive rows).  A wave covers 16 blocks of 32
// weights per chunk: lane = 4 * block + quarter, each lane owning 8 weights
// (one dword of Q4_0 codes).  The lane's 8 activations stay in registers for
// the whole kernel (CW chunks), so the inner loop is loads + v_cvt_f32_ubyte +
// FMA only.  For long rows (nb > 64 blocks) the four waves of a workgroup split
// K and combine through LDS (KW = 4); otherwise each wave owns whole row pairs.
#include "common.h"
#include "device_util.h"

namespace gaje {

namespace {

constexpr int THREADS = 256;
constexpr int LUT_SLOT_FLOATS = 2 * 16 * 16;  // per wave: 2 rows x 16 blocks x 16 entries
constexpr int MAX_GRID = 4096;

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

template <int FMT, bool NT>
__device__ __forceinline__ float quarter_dot(const GemvParams &p, int64_t row, int b, int j, const float (&xv)[8],
                                             float sx, float *tbl) {
    if constexpr (FMT == FMT_Q4_0) {
        const uint8_t *blk = p.w + ((size_t)row * p.nb + b) * 20;
        const uint32_t sm = ld_u32<NT>(blk);
        const uint32_t q = ld_u32<NT>(blk + 4 + 4 * j);
        const uint32_t lo = opaque_and(q, 0x0F0F0F0Fu), hi = opaque_and(q >> 4, 0x0F0F0F0Fu);
        float d = ubyte0(lo) * xv[0];
        d = fmaf(ubyte0(hi), xv[1], d);
        d = fmaf(ubyte1(lo), xv[2], d);
        d = fmaf(ubyte1(hi), xv[3], d);
        d = fmaf(ubyte2(lo), xv[4], d);
        d = fmaf(ubyte2(hi), xv[5], d);
        d = fmaf(ubyte3(lo), xv[6], d);
        d = fmaf(ubyte3(hi), xv[7], d);
        // sum_i (q_i*scale + min) x_i = scale * sum_i q_i x_i + min * sum_i x_i
        return fmaf(half_lo(sm), d, half_hi(sm) * sx);
    } else if constexpr (FMT == FMT_LUT4) {
        const float *t = p.lut + (row < p.lut_rows_own ? (size_t)row * p.nb * 16 : 0) + (size_t)b * p.lut_block_stride;
        const float4 tv = ld_f4<NT>(t + 4 * j);
        *(float4 *)(tbl + 4 * j) = tv;  // the block's 16-entry table, 4 lanes x 4 entries
        __builtin_amdgcn_wave_barrier();
        const uint32_t q = ld_u32<NT>(p.w + ((size_t)row * p.nb + b) * 16 + 4 * j);
        float d = 0.0f;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t by = (q >> (8 * m)) & 0xFFu;
            d = fmaf(tbl[by >> 4], xv[2 * m], d);      // high nibble = even element
            d = fmaf(tbl[by & 15u], xv[2 * m + 1], d);
        }
        __builtin_amdgcn_wave_barrier();
        return d;
    } else {
        const float *wr = (const float *)p.w + (size_t)row * p.K + (size_t)b * 32 + 8 * j;
        const float4 a = ld_f4<NT>(wr), c = ld_f4<NT>(wr + 4);
        float d = a.x * xv[0];
        d = fmaf(a.y, xv[1], d);
        d = fmaf(a.z, xv[2], d);
        d = fmaf(a.w, xv[3], d);
        d = fmaf(c.x, xv[4], d);
        d = fmaf(c.y, xv[5], d);
        d = fmaf(c.z, xv[6], d);
        d = fmaf(c.w, xv[7], d);
        return d;
    }
}

__device__ __forceinline__ float finish_row(const GemvParams &p, const float *xs, int64_t r, float acc, bool flush) {
    float v = flush ? flush_small(acc) : acc;
    if (p.a_ptr) {
        for (int64_t k = p.a_ptr[r]; k < p.a_ptr[r + 1]; ++k) v += xs[p.a_col[k]] * half_bits(p.a_val[k]);
    }
    if (r < p.bias_len) v += p.bias[r];
    return v;
}

__device__ __forceinline__ float block_sum(float v, float *scratch4) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) scratch4[wave] = v;
    __syncthreads();
    return (scratch4[0] + scratch4[1]) + (scratch4[2] + scratch4[3]);
}

template <int FMT, bool NT, int KW, int CW>
__global__ __launch_bounds__(THREADS) void gemv_kernel(GemvParams p, int64_t npairs) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float red[2][4][2];
    __shared__ float scratch4[4];
    DevState *st = p.st;
    if (st && st->halted) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K = p.K;
    float *xs = smem;

    // ---- prologue: activation vector into LDS (normalised if requested) ----
    float ss = 0.0f;
    int bad_in = 0;
    for (int64_t k = tid; k < K; k += THREADS) {
        const float v = p.x[k];
        xs[k] = v;
        ss = fmaf(v, v, ss);
        bad_in |= isnan(v);
    }
    if (p.st_in >= 0 && __syncthreads_or(bad_in) && tid == 0) nan_flag(st, p.layer, p.st_in);
    if (p.norm_w) {
        const float tot = block_sum(ss, scratch4);
        const float inv = 1.0f / sqrtf(tot / (float)K + p.eps);
        int bad = 0;
        for (int64_t k = tid; k < K; k += THREADS) {
            const float v = (xs[k] * inv) * p.norm_w[k];
            xs[k] = v;
            bad |= isnan(v);
        }
        if (p.st_norm >= 0 && __syncthreads_or(bad) && tid == 0) nan_flag(st, p.layer, p.st_norm);
    }
    if (p.gnorm) {
        float s2 = 0.0f;
        for (int64_t k = tid; k < K; k += THREADS) s2 = fmaf(xs[k], xs[k], s2);
        const float tot = block_sum(s2, scratch4);
        const float rms = sqrtf(tot / (float)K + p.eps);
        if (rms > p.h_scale) {
            const float sc = p.h_scale / rms;
            for (int64_t k = tid; k < K; k += THREADS) xs[k] *= sc;
        }
    }
    __syncthreads();
    if (p.x_out && blockIdx.x == 0)
        for (int64_t k = tid; k < K; k += THREADS) p.x_out[k] = xs[k];

    // ---- per-lane activations in registers ----
    const int j = lane & 3, bl = lane >> 2;
    const int kg = (KW == 1) ? 0 : wave;
    const int per = (p.nb + KW - 1) / KW;
    const int kb0 = kg * per;
    const int kb1 = min(p.nb, kb0 + per);
    float xv[CW][8];
    float sx[CW];
    bool bvalid[CW];
    int bidx[CW];
#pragma unroll
    for (int c = 0; c < CW; ++c) {
        const int b = kb0 + c * 16 + bl;
        bvalid[c] = b < kb1;
        bidx[c] = bvalid[c] ? b : (kb1 > 0 ? kb1 - 1 : 0);
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            xv[c][e] = bvalid[c] ? xs[(size_t)b * 32 + 8 * j + e] : 0.0f;
            s += xv[c][e];
        }
        sx[c] = s;
    }
    float *tbl = smem + ((K + 3) & ~(int64_t)3) + wave * LUT_SLOT_FLOATS;

    const bool flush = FMT != FMT_F32;
    const int slots = 4 / KW;
    const int slot = (KW == 1) ? wave : 0;
    const bool have_blocks = p.nb > 0 && kb0 < kb1;
    float best_v = -INFINITY;
    int64_t best_i = 0;
    int par = 0;

    for (int64_t pr = (int64_t)blockIdx.x * slots + slot; pr < npairs; pr += (int64_t)gridDim.x * slots) {
        int64_t r0, r1;
        pair_rows(p, pr, r0, r1);
        float a0 = 0.0f, a1 = 0.0f;
        if (have_blocks) {
            const bool v0 = r0 < p.rows_valid, v1 = r1 >= 0 && r1 < p.rows_valid;
#pragma unroll
            for (int c = 0; c < CW; ++c) {
                if (v0) {
                    const float d = quarter_dot<FMT, NT>(p, r0, bidx[c], j, xv[c], sx[c], tbl + bl * 16);
                    a0 += bvalid[c] ? d : 0.0f;
                }
                if (v1) {
                    const float d = quarter_dot<FMT, NT>(p, r1, bidx[c], j, xv[c], sx[c], tbl + 256 + bl * 16);
                    a1 += bvalid[c] ? d : 0.0f;
                }
            }
        }
        a0 = wave_sum(a0);
        a1 = wave_sum(a1);
        if constexpr (KW > 1) {
            if (lane == 0) {
                red[par][wave][0] = a0;
                red[par][wave][1] = a1;
            }
            __syncthreads();
            a0 = (red[par][0][0] + red[par][1][0]) + (red[par][2][0] + red[par][3][0]);
            a1 = (red[par][0][1] + red[par][1][1]) + (red[par][2][1] + red[par][3][1]);
            par ^= 1;
        }
        if (lane != 0 || (KW > 1 && wave != 0)) continue;

        // ---- epilogue (one lane per row pair) ----
        const float y0 = finish_row(p, xs, r0, a0, flush);
        const float y1 = r1 >= 0 ? finish_row(p, xs, r1, a1, flush) : 0.0f;
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
                const int half = p.head_dim >> 1;
                const int pos = st->pos;
                const int i = (int)(pr % half);
                const float cs = p.rope_cos[(size_t)pos * half + i], sn = p.rope_sin[(size_t)pos * half + i];
                if (r0 < p.q_rows) {
                    p.q_out[r0] = y0 * cs - y1 * sn;
                    p.q_out[r1] = y0 * sn + y1 * cs;
                } else if (r0 < p.q_rows + p.kv_rows) {
                    const int64_t kh = (r0 - p.q_rows) / p.head_dim;
                    const int64_t base = p.q_rows + kh * p.head_dim;
                    float *kc = p.k_cache + kh * p.kv_head_stride + (size_t)pos * p.head_dim;
                    kc[r0 - base] = y0 * cs - y1 * sn;
                    kc[r1 - base] = y0 * sn + y1 * cs;
                } else {
                    const int64_t vh = (r0 - p.q_rows - p.kv_rows) / p.head_dim;
                    const int64_t base = p.q_rows + p.kv_rows + vh * p.head_dim;
                    float *vc = p.v_cache + vh * p.kv_head_stride + (size_t)pos * p.head_dim;
                    vc[r0 - base] = y0;
                    vc[r1 - base] = y1;
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
    if (p.mode == MODE_ARGMAX && st && best_v > -INFINITY) {
        const unsigned long long key =
            ((unsigned long long)order_key(best_v) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)best_i);
        atomicMax(&st->argmax_key, key);
    }
}

using KernelFn = void (*)(GemvParams, int64_t);

// KW = 1 serves rows of up to 64 blocks (CW <= 4); KW = 4 up to 512 (CW <= 8).
template <int FMT, bool NT>
KernelFn pick_kw(int kw, int cw) {
    if (kw == 1) {
        switch (cw) {
            case 1: return gemv_kernel<FMT, NT, 1, 1>;
            case 2: return gemv_kernel<FMT, NT, 1, 2>;
            case 3: return gemv_kernel<FMT, NT, 1, 3>;
            case 4: return gemv_kernel<FMT, NT, 1, 4>;
        }
    } else {
        switch (cw) {
            case 1: return gemv_kernel<FMT, NT, 4, 1>;
            case 2: return gemv_kernel<FMT, NT, 4, 2>;
            case 3: return gemv_kernel<FMT, NT, 4, 3>;
            case 4: return gemv_kernel<FMT, NT, 4, 4>;
            case 5: return gemv_kernel<FMT, NT, 4, 5>;
            case 6: return gemv_kernel<FMT, NT, 4, 6>;
            case 7: return gemv_kernel<FMT, NT, 4, 7>;
            case 8: return gemv_kernel<FMT, NT, 4, 8>;
        }
    }
    return nullptr;
}

}  // namespace

size_t gemv_lds_bytes(int64_t K, int fmt) {
    size_t b = (size_t)((K + 3) & ~(int64_t)3) * 4;
    if (fmt == FMT_LUT4) b += 4 * LUT_SLOT_FLOATS * 4;
    return b;
}

int launch_gemv(const GemvParams &p, hipStream_t s) {
    if (p.N < 0 || p.K <= 0 || !p.x || !p.y)
        return set_error(GAJE_ERR_INVALID_ARG, "gemv: invalid shape or null buffer");
    if (p.nb != (int32_t)(p.K / 32)) return set_error(GAJE_ERR_INVALID_ARG, "gemv: nb must be K/32");
    if (p.fmt == FMT_F32 && p.K % 32 != 0)
        return set_error(GAJE_ERR_UNSUPPORTED, "gemv: f32 rows need in_features %% 32 == 0 (got %lld)",
                         (long long)p.K);
    if (p.nb > 0 && !p.w) return set_error(GAJE_ERR_INVALID_ARG, "gemv: null weights");
    if (p.fmt == FMT_LUT4 && p.nb > 0 && !p.lut) return set_error(GAJE_ERR_INVALID_ARG, "gemv: null LUT");
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
    int kw, cw;
    if (p.nb <= 64) {
        kw = 1;
        cw = p.nb == 0 ? 1 : (p.nb + 15) / 16;
    } else {
        kw = 4;
        cw = ((p.nb + 3) / 4 + 15) / 16;
    }
    KernelFn fn = nullptr;
    if (p.fmt == FMT_Q4_0) fn = pick_kw<FMT_Q4_0, false>(kw, cw);
    else if (p.fmt == FMT_LUT4) fn = pick_kw<FMT_LUT4, false>(kw, cw);
    else if (p.fmt == FMT_F32) fn = p.nontemporal ? pick_kw<FMT_F32, true>(kw, cw) : pick_kw<FMT_F32, false>(kw, cw);
    if (!fn) return set_error(GAJE_ERR_UNSUPPORTED, "gemv: in_features %lld too large", (long long)p.K);
    const int slots = 4 / kw;
    int64_t grid = (npairs + slots - 1) / slots;
    if (grid > MAX_GRID) grid = MAX_GRID;
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(THREADS), lds, s, p, npairs);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
