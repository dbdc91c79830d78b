// Batched decode: one token for each of up to 16 independent sequences per
// step, as if as many GenomicLLM instances (llm/forward.rs:7-64) stepped
// together over shared weights.  Every product and reduction follows the
// batch-1 decode kernels' order, so each sequence's values are bit-identical
// to its own forward_core: the weight rows are read and dequantised once per
// step and consumed by every sequence's chains.
#include <hip/hip_runtime.h>

#include "common.h"
#include "device_util.h"
#include "kernels.h"

namespace gaje {
namespace {

constexpr int BQ_CHUNK = 512;              // activation elements per staged chunk (4 packed groups)
constexpr int BQ_CROW = BQ_CHUNK / 8 + 4;  // LDS floats per (vector, chain) row of a chunk

__device__ __forceinline__ void seq_flag(uint32_t *codes, int s, int layer, int stage) {
    if (codes && stage >= 0) atomicMin(&codes[s], (uint32_t)(layer * 8 + stage));
}

// dequantised values of one packed group for chain l (genomic.rs:298-316): d = fma(q, scale, min)
__device__ __forceinline__ void group_dequant(float (&d)[16], vu2 n, vu4 s) {
    const uint32_t c[4] = {opaque_and(n.x, 0x0F0F0F0Fu), opaque_and(n.x >> 4, 0x0F0F0F0Fu),
                           opaque_and(n.y, 0x0F0F0F0Fu), opaque_and(n.y >> 4, 0x0F0F0F0Fu)};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const float scale = half_lo(s[b]), mn = half_hi(s[b]);
        d[4 * b + 0] = fmaf(ubyte0(c[b]), scale, mn);
        d[4 * b + 1] = fmaf(ubyte1(c[b]), scale, mn);
        d[4 * b + 2] = fmaf(ubyte2(c[b]), scale, mn);
        d[4 * b + 3] = fmaf(ubyte3(c[b]), scale, mn);
    }
}

// Packed Q4_0 rows x NV activation vectors (genomic_dot_product_q4_0_avx2,
// genomic.rs:263-336, per vector).  Lane = (row slot lane>>3, chain l =
// lane&7); a slot holds R rows (rows slot + 8j of the workgroup's 8R), so
// each activation value read from LDS feeds R rows' chains; wave w owns
// vectors vz + w*VPW.. (their accumulators; vz = blockIdx.y * NV, the
// workgroup's share of the batch); the waves share the rows and the staged
// chunk of all NV vectors.  Activations arrive chain-major
// ([vector][chain l][K/8]: element k at chain k%8, column k/8), so a chunk is
// 8 contiguous runs per vector, copied to LDS through registers
// (double-buffered, loads always issued, clamped at the end).  Groups past the
// row's end read as zero codes/scales against zero activations, and
// fma(0, 0, acc) = acc (acc is never -0), so every chunk runs branch-free.
template <int NV, int VPW, int R>
__global__ __launch_bounds__(NV / VPW * 64) void gemv_batch_q4_kernel(BatchGemvParams p) {
    constexpr int NTH = NV / VPW * 64;
    constexpr int RUN = BQ_CHUNK / 8;                 // floats of one chain per chunk
    constexpr int BUF = NV * 8 * BQ_CROW;
    constexpr int UPT = NV * 8 * (RUN / 4) / NTH;     // float4s staged per thread per chunk
    extern __shared__ __align__(16) float xs[];       // [2][NV][8][BQ_CROW]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l = lane & 7;
    const int nb = p.nb, G = (nb + 3) >> 2;
    const int64_t K8 = (int64_t)nb * 4;               // column count of a chain row
    const int nch = (int)((K8 + RUN - 1) / RUN);
    int64_t row[R];
    const uint8_t *wr[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        row[j] = (int64_t)blockIdx.x * 8 * R + 8 * j + (lane >> 3);
        wr[j] = p.w + (size_t)(row[j] < p.N ? row[j] : p.N - 1) * G * 80;
    }
    const int v0 = wave * VPW;
    const int vz = blockIdx.y * NV;  // first vector of this workgroup's share of the batch

    vf4 st[UPT];
    auto load_chunk = [&](int c) {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            const int u = tid + i * NTH, vl = u / (RUN / 4), q = u % (RUN / 4);  // vl = v * 8 + l
            const int64_t col = (int64_t)c * RUN + 4 * q;
            const bool in = col < K8;
            const float *src = p.x + (size_t)(vz + (vl >> 3)) * p.ldx + (size_t)(vl & 7) * K8 + (in ? col : 0);
            const vf4 a = *(const vf4 *)src;
            st[i] = in ? a : (vf4){0.f, 0.f, 0.f, 0.f};
        }
    };
    auto store_chunk = [&](int buf) {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            const int u = tid + i * NTH, vl = u / (RUN / 4), q = u % (RUN / 4);
            *(vf4 *)(xs + buf * BUF + vl * BQ_CROW + 4 * q) = st[i];
        }
    };
    vu2 wn[2][R][4];
    vu4 ws[2][R][4];
    auto load_w = [&](int c, int slot) {
#pragma unroll
        for (int j = 0; j < R; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int g = 4 * c + i;
                const bool in = g < G;
                const uint8_t *gp = wr[j] + (size_t)(in ? g : G - 1) * 80;
                const vu2 n = *(const vu2 *)(gp + 8 * l);
                const vu4 s = *(const vu4 *)(gp + 64);
                const uint32_t keep = in ? 0xFFFFFFFFu : 0u;
                wn[slot][j][i] = n & keep;
                ws[slot][j][i] = s & keep;
            }
    };

    float acc[R][VPW];
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
        for (int v = 0; v < VPW; ++v) acc[j][v] = 0.0f;

    load_chunk(0);
    load_w(0, 0);
    store_chunk(0);
    lds_barrier();
    // one chunk from buffer `cur` (a constant at each call: the rings are
    // indexed statically); the next chunk's loads are in flight meanwhile.
    // The activations are issued before the weights: loads complete in order,
    // so staging them waits for them alone, and the barriers order LDS only,
    // leaving the next chunk's weights in flight across them.
    auto chunk = [&](int c, int cur) {
        const int cn = c + 1 < nch ? c + 1 : c;
        load_chunk(cn);
        load_w(cn, cur ^ 1);
        const float *xb = xs + cur * BUF + (v0 * 8 + l) * BQ_CROW;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float d[R][16];
#pragma unroll
            for (int j = 0; j < R; ++j) group_dequant(d[j], wn[cur][j][i], ws[cur][j][i]);
#pragma unroll
            for (int v = 0; v < VPW; ++v) {
                const float *xv = xb + v * 8 * BQ_CROW + 16 * i;
                const float4 x0 = *(const float4 *)xv, x1 = *(const float4 *)(xv + 4);
                const float4 x2 = *(const float4 *)(xv + 8), x3 = *(const float4 *)(xv + 12);
                const float xx[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                                      x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
#pragma unroll
                for (int j = 0; j < R; ++j) {
                    float a = acc[j][v];
#pragma unroll
                    for (int e = 0; e < 16; ++e) a = fmaf(d[j][e], xx[e], a);
                    acc[j][v] = a;
                }
            }
        }
        store_chunk(cur ^ 1);
        lds_barrier();
    };
    for (int c = 0; c < nch; c += 2) {
        chunk(c, 0);
        if (c + 1 < nch) chunk(c + 1, 1);
    }

    // per (row, vector): ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) in lane l = 0, then the row epilogue
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
        for (int v = 0; v < VPW; ++v) {
            const float a = acc[j][v];
            const float t = red8_dpp(a);  // valid in lane 8r
            const int s = vz + v0 + v;
            const int64_t r = row[j];
            if (l != 0 || r >= p.N || s >= p.nv) continue;
            float y = flush_small(t);
            if (p.a_ptr) {  // sparse anchors, then the bias (forward.rs:103-115)
                for (int64_t k = p.a_ptr[r]; k < p.a_ptr[r + 1]; ++k) {
                    const uint32_t col = p.a_col[k];
                    const float prod = p.x[(size_t)s * p.ldx + (col & 7) * K8 + (col >> 3)] * half_bits(p.a_val[k]);
                    y = y + prod;
                }
            }
            if (r < p.bias_len) y = y + p.bias[r];
            float *dst = p.y + (size_t)s * p.ldy + r;
            if (p.mode == MODE_RESIDUAL) {
                if (isnan(y)) seq_flag(p.nan_codes, s, p.layer, p.st_a);
                const float h = *dst + y;
                *dst = h;
                if (isnan(h)) seq_flag(p.nan_codes, s, p.layer, p.st_b);
            } else {
                *dst = y;
            }
        }
}

// F32 rows in the tiled layout x NV vectors (dot_product, dot.rs:23-94, per
// vector): lanes 2r, 2r+1 of a wave own row r of the wave's 32-row tile,
// chains 0..3 and 4..7; each chunk of the tile is one coalesced KiB.  All NV
// vectors sit in LDS in plain layout.
template <int NV>
__global__ __launch_bounds__(256) void gemv_batch_f32_kernel(BatchGemvParams p) {
    extern __shared__ __align__(16) float xs[];  // [NV][K]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K = p.K, K4 = K / 4;
    for (int64_t i = tid; i < NV * K4; i += 256) {
        const int64_t v = i / K4, q = i - v * K4;
        *(float4 *)(xs + v * K + 4 * q) = *(const float4 *)(p.x + (size_t)v * p.ldx + 4 * q);
    }
    __syncthreads();
    const int s = lane & 1;
    const int64_t row = (int64_t)blockIdx.x * 128 + wave * 32 + (lane >> 1);
    const bool row_ok = row < p.N;
    const int64_t lrow = row_ok ? row : p.N - 1;
    const float *wl = (const float *)p.w + (size_t)(lrow >> 5) * (size_t)K * 32 + (lrow & 31) * 8 + 4 * s;
    const int64_t chunks = K / 8;
    float acc[NV][4];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v][0] = acc[v][1] = acc[v][2] = acc[v][3] = 0.0f;
    constexpr int AHEAD = 8;
    float4 ring[AHEAD];
#pragma unroll
    for (int u = 0; u < AHEAD; ++u) ring[u] = ld_f4<true>(wl + 256 * (u < chunks ? u : chunks - 1));
    for (int64_t c0 = 0; c0 < chunks; c0 += AHEAD) {
#pragma unroll
        for (int u = 0; u < AHEAD; ++u) {
            const int64_t c = c0 + u;
            if (c >= chunks) break;
            const float4 w = ring[u];
            const int64_t cn = c + AHEAD < chunks ? c + AHEAD : chunks - 1;
            ring[u] = ld_f4<true>(wl + 256 * cn);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const float4 x = *(const float4 *)(xs + v * K + 8 * c + 4 * s);
                acc[v][0] = fmaf(x.x, w.x, acc[v][0]);
                acc[v][1] = fmaf(x.y, w.y, acc[v][1]);
                acc[v][2] = fmaf(x.z, w.z, acc[v][2]);
                acc[v][3] = fmaf(x.w, w.w, acc[v][3]);
            }
        }
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        // lane 2r: chains 0..3, lane 2r+1: 4..7 -> ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7))
        const float u0 = acc[v][0] + __shfl_xor(acc[v][0], 1, WAVE);
        const float u1 = acc[v][1] + __shfl_xor(acc[v][1], 1, WAVE);
        const float u2 = acc[v][2] + __shfl_xor(acc[v][2], 1, WAVE);
        const float u3 = acc[v][3] + __shfl_xor(acc[v][3], 1, WAVE);
        if (s != 0 || !row_ok || v >= p.nv) continue;
        float y = (u0 + u1) + (u2 + u3);
        if (row < p.bias_len) y = y + p.bias[row];
        p.y[(size_t)v * p.ldy + row] = y;
    }
}

// The same products for a batch of 16, register-blocked over rows: lanes 2r,
// 2r+1 of a wave own rows r + 32j (j < RB; one 32-row tile each) of the
// wave's 32*RB rows, chains 0..3 and 4..7 as above, and a workgroup takes VG
// of the vectors, so each activation quad read from LDS feeds RB rows.
// VG = 16 (all vectors, when their activations fit LDS): every weight row is
// read once.  VG = 4: the batch splits over the grid, workgroups b, b+8,
// b+16, b+24 taking one row block's four vector groups; consecutive
// workgroups go to the eight XCDs in turn, so the four land on one XCD and its
// L2 serves the block's rows three times of four (measured: 372 us for the
// 151936 x 1536 lm_head of batch 16, its L2-to-CU traffic four times the
// weights; VG = 16 reads them once).
constexpr int F32B_AHEAD = 4;
template <int RB, int NT> constexpr int64_t f32b_rows() { return NT / 2 * RB; }  // rows per workgroup

template <int RB, int VG, int NT>
__global__ __launch_bounds__(NT) void gemv_batch_f32_rb_kernel(BatchGemvParams p, int64_t nblk) {
    constexpr int AHEAD = F32B_AHEAD, NVG = 16 / VG;
    constexpr int64_t F32B_ROWS = f32b_rows<RB, NT>();
    extern __shared__ __align__(16) float xs[];  // [VG][K]
    const int b = blockIdx.x;
    const int64_t blk = NVG == 1 ? (int64_t)b : (((int64_t)(b >> 5) << 3) | (b & 7));
    if (blk >= nblk) return;  // whole workgroup: the grid is rounded up to 32 (NVG = 4)
    const int vz = NVG == 1 ? 0 : ((b >> 3) & 3) * VG;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K = p.K, K4 = K / 4;
    for (int64_t i = tid; i < VG * K4; i += NT) {
        const int64_t v = i / K4, q = i - v * K4;
        *(float4 *)(xs + v * K + 4 * q) = *(const float4 *)(p.x + (size_t)(vz + v) * p.ldx + 4 * q);
    }
    __syncthreads();
    const int s = lane & 1;
    const int64_t r0 = blk * F32B_ROWS + wave * (32 * RB) + (lane >> 1);
    const float *wl[RB];
#pragma unroll
    for (int j = 0; j < RB; ++j) {
        const int64_t row = r0 + 32 * j;
        const int64_t lrow = row < p.N ? row : p.N - 1;
        wl[j] = (const float *)p.w + (size_t)(lrow >> 5) * (size_t)K * 32 + (lrow & 31) * 8 + 4 * s;
    }
    const int64_t chunks = K / 8;
    float acc[RB][VG][4];
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
        for (int v = 0; v < VG; ++v) acc[j][v][0] = acc[j][v][1] = acc[j][v][2] = acc[j][v][3] = 0.0f;
    float4 ring[AHEAD][RB];
#pragma unroll
    for (int u = 0; u < AHEAD; ++u)
#pragma unroll
        for (int j = 0; j < RB; ++j) ring[u][j] = ld_f4<true>(wl[j] + 256 * (u < chunks ? u : chunks - 1));
    for (int64_t c0 = 0; c0 < chunks; c0 += AHEAD) {
#pragma unroll
        for (int u = 0; u < AHEAD; ++u) {
            const int64_t c = c0 + u;
            if (c >= chunks) break;
            float4 w[RB];
#pragma unroll
            for (int j = 0; j < RB; ++j) w[j] = ring[u][j];
            const int64_t cn = c + AHEAD < chunks ? c + AHEAD : chunks - 1;
#pragma unroll
            for (int j = 0; j < RB; ++j) ring[u][j] = ld_f4<true>(wl[j] + 256 * cn);
#pragma unroll
            for (int v = 0; v < VG; ++v) {
                const float4 x = *(const float4 *)(xs + v * K + 8 * c + 4 * s);
#pragma unroll
                for (int j = 0; j < RB; ++j) {
                    acc[j][v][0] = fmaf(x.x, w[j].x, acc[j][v][0]);
                    acc[j][v][1] = fmaf(x.y, w[j].y, acc[j][v][1]);
                    acc[j][v][2] = fmaf(x.z, w[j].z, acc[j][v][2]);
                    acc[j][v][3] = fmaf(x.w, w[j].w, acc[j][v][3]);
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < RB; ++j) {
        const int64_t row = r0 + 32 * j;
#pragma unroll
        for (int v = 0; v < VG; ++v) {
            // lane 2r: chains 0..3, lane 2r+1: 4..7 -> ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7))
            const float u0 = acc[j][v][0] + __shfl_xor(acc[j][v][0], 1, WAVE);
            const float u1 = acc[j][v][1] + __shfl_xor(acc[j][v][1], 1, WAVE);
            const float u2 = acc[j][v][2] + __shfl_xor(acc[j][v][2], 1, WAVE);
            const float u3 = acc[j][v][3] + __shfl_xor(acc[j][v][3], 1, WAVE);
            const int sv = vz + v;
            if (s != 0 || row >= p.N || sv >= p.nv) continue;
            float y = (u0 + u1) + (u2 + u3);
            if (row < p.bias_len) y = y + p.bias[row];
            p.y[(size_t)sv * p.ldy + row] = y;
        }
    }
}

// rms_norm per sequence row (norm.rs:52-88): threads 0..7 run the chains,
// out = (x * inv) * w.  Guards: st_a on the input, st_b on the output.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(BatchRowParams p) {
    extern __shared__ __align__(16) float xs[];
    __shared__ float inv_slot;
    const int s = blockIdx.x;
    const int tid = threadIdx.x;
    const float *x = p.x + (size_t)s * p.ldx;
    int bad = 0;
    for (int64_t k = tid; k < p.K; k += 256) {
        const float v = x[k];
        bad |= isnan(v);
        xs[k] = v;
    }
    if (__syncthreads_or(bad) && tid == 0) seq_flag(p.nan_codes, s, p.layer, p.st_a);
    float inv = 1.0f;
    if (p.w) {
        rms_inv_plain(xs, p.K, p.eps, &inv_slot);
        __syncthreads();
        inv = inv_slot;
    }
    bad = 0;
    const int64_t K8 = p.K / 8;
    for (int64_t k = tid; k < p.K; k += 256) {
        float o = xs[k];  // no weight: the plain rows (an empty norm tensor is skipped, block/forward.rs:18-28)
        if (p.w) {
            const float t = o * inv;
            o = t * p.w[k];
        }
        bad |= isnan(o);
        p.y[(size_t)s * p.ldy + (p.chain_major ? (k & 7) * K8 + (k >> 3) : k)] = o;
    }
    if (__syncthreads_or(bad) && tid == 0) seq_flag(p.nan_codes, s, p.layer, p.st_b);
}

// The same norm for K % 32 == 0 and K <= 16 * 256: each thread loads its
// float4s of x and of the weights in one batch, the eight sum-of-squares
// chains (thread l: elements 8i + l, fma(v, v, acc) in i order) read a
// chain-major LDS copy whose rows are zero past K/8 (fma(0, 0, acc) = acc, acc
// >= +0), and the outputs are formed from the registers.  The reduction
// ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)) and the rounding of every step are
// those of rmsnorm_rows_kernel.
constexpr int RN_XB4 = 4;
__host__ __device__ constexpr int rn_chain_row(int64_t K) { return (int)((K / 8 + 63) / 64 * 64 + 36); }

__global__ __launch_bounds__(256) void rmsnorm_rows_cm_kernel(BatchRowParams p) {
    extern __shared__ __align__(16) float xs[];  // [8][rn_chain_row(K)]
    __shared__ float inv_slot;
    const int s = blockIdx.x, tid = threadIdx.x;
    const int64_t K = p.K, K4 = K / 4, K8 = K / 8;
    const int row = rn_chain_row(K), n = (int)((K8 + 63) / 64 * 64), tail = row - (int)K8;
    const float *x = p.x + (size_t)s * p.ldx;
    float4 xr[RN_XB4], wr[RN_XB4];
#pragma unroll
    for (int u = 0; u < RN_XB4; ++u) {
        const int64_t m = u * 256 + tid;
        xr[u] = m < K4 ? *(const float4 *)(x + 4 * m) : make_float4(0.f, 0.f, 0.f, 0.f);
        wr[u] = (p.w && m < K4) ? *(const float4 *)(p.w + 4 * m) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // the rows' zero tails [K8, row) (the chains read up to n + 32)
    for (int t = tid; t < 8 * tail; t += 256) xs[(t / tail) * row + K8 + t % tail] = 0.0f;
    int bad = 0;
#pragma unroll
    for (int u = 0; u < RN_XB4; ++u) {
        const int64_t m = u * 256 + tid;
        if (m >= K4) continue;
        const float v[4] = {xr[u].x, xr[u].y, xr[u].z, xr[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t k = 4 * m + j;
            xs[(k & 7) * row + (k >> 3)] = v[j];
            bad |= isnan(v[j]);
        }
    }
    if (__syncthreads_or(bad) && tid == 0) seq_flag(p.nan_codes, s, p.layer, p.st_a);
    float inv = 1.0f;
    if (p.w) {
        if (tid < 8) {
            const float acc = chain_lds_sq(0.0f, xs + tid * row, n);
            const float a = acc + __shfl(acc, (tid + 4) & 7, 8);  // lane l<4: a_l + a_{l+4}
            const float b = a + __shfl(a, (tid + 1) & 7, 8);      // lane 0: u0+u1, lane 2: u2+u3
            const float tot = b + __shfl(b, (tid + 2) & 7, 8);    // lane 0: (u0+u1) + (u2+u3)
            if (tid == 0) {
                const float mean = tot / (float)K;
                inv_slot = 1.0f / sqrtf(mean + p.eps);
            }
        }
        __syncthreads();
        inv = inv_slot;
    }
    bad = 0;
    float *y = p.y + (size_t)s * p.ldy;
#pragma unroll
    for (int u = 0; u < RN_XB4; ++u) {
        const int64_t m = u * 256 + tid;
        if (m >= K4) continue;
        const float v[4] = {xr[u].x, xr[u].y, xr[u].z, xr[u].w}, w[4] = {wr[u].x, wr[u].y, wr[u].z, wr[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t k = 4 * m + j;
            float o = v[j];  // no weight: the plain rows
            if (p.w) {
                const float t = o * inv;
                o = t * w[j];
            }
            bad |= isnan(o);
            y[p.chain_major ? (k & 7) * K8 + (k >> 3) : k] = o;
        }
    }
    if (__syncthreads_or(bad) && tid == 0) seq_flag(p.nan_codes, s, p.layer, p.st_b);
}

// swiglu_balanced per element (block/forward.rs:87-113) without the genomic
// norm: a grid over (sequence, 256-element slices).
__global__ __launch_bounds__(256) void swiglu_elems_kernel(BatchRowParams p) {
    const int s = blockIdx.y;
    const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const float *g = p.x + (size_t)s * p.ldx, *u = g + p.K;
    int bad_u = 0, bad_o = 0;
    if (k < p.K) {
        const float uv = u[k];
        bad_u = isnan(uv);
        const float o = swiglu1(g[k], uv);
        bad_o = isnan(o);
        p.y[(size_t)s * p.ldy + (p.chain_major ? (k & 7) * (p.K / 8) + (k >> 3) : k)] = o;
    }
    if (__any(bad_u) && (threadIdx.x & 63) == 0) seq_flag(p.nan_codes, s, p.layer, p.st_a);
    if (__any(bad_o) && (threadIdx.x & 63) == 0) seq_flag(p.nan_codes, s, p.layer, p.st_b);
}

// swiglu_balanced per element of each sequence's gate/up row pair
// (block/forward.rs:87-113), with use_genomic_norm (:115-123) when set.
__global__ __launch_bounds__(256) void swiglu_rows_kernel(BatchRowParams p) {
    extern __shared__ __align__(16) float xs[];
    __shared__ float rms_slot;
    const int s = blockIdx.x;
    const int tid = threadIdx.x;
    const float *g = p.x + (size_t)s * p.ldx, *u = g + p.K;
    int bad_u = 0, bad_o = 0;
    for (int64_t k = tid; k < p.K; k += 256) {
        const float uv = u[k];
        bad_u |= isnan(uv);
        const float o = swiglu1(g[k], uv);
        bad_o |= isnan(o);
        xs[k] = o;
    }
    const bool any_u = __syncthreads_or(bad_u);
    const bool any_o = __syncthreads_or(bad_o);
    if (tid == 0) {
        if (any_u) seq_flag(p.nan_codes, s, p.layer, p.st_a);
        if (any_o) seq_flag(p.nan_codes, s, p.layer, p.st_b);
    }
    float sc = 1.0f;
    if (p.gnorm) {
        if (tid == 0) {
            float ss = 0.0f;
            for (int64_t k = 0; k < p.K; ++k) {
                const float sq = xs[k] * xs[k];
                ss = ss + sq;
            }
            rms_slot = sqrtf(ss / (float)p.K + p.eps);
        }
        __syncthreads();
        const float rms = rms_slot;
        if (rms > p.h_scale) sc = p.h_scale / rms;
    }
    for (int64_t k = tid; k < p.K; k += 256)
        p.y[(size_t)s * p.ldy + (p.chain_major ? (k & 7) * (p.K / 8) + (k >> 3) : k)] = p.gnorm ? xs[k] * sc : xs[k];
}

// Greedy argmax per sequence (llm/forward.rs:262-271: strict '>', so the first
// maximum; NaN never wins; all-NaN gives 0).
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float *x, int64_t n, int64_t ld, uint32_t *out) {
    __shared__ unsigned long long best[16];
    const int s = blockIdx.x;
    const int tid = threadIdx.x;
    unsigned long long key = 0ull;
    for (int64_t i = tid; i < n; i += 1024) {
        const float v = x[(size_t)s * ld + i];
        if (isnan(v)) continue;
        const unsigned long long k = ((unsigned long long)max_key(v) << 32) | (0xFFFFFFFFu - (uint32_t)i);
        key = k > key ? k : key;
    }
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long other = __shfl_xor(key, o, WAVE);
        key = other > key ? other : key;
    }
    if ((tid & 63) == 0) best[tid >> 6] = key;
    __syncthreads();
    if (tid == 0) {
        unsigned long long k = best[0];
        for (int w = 1; w < 16; ++w) k = best[w] > k ? best[w] : k;
        out[s] = k ? 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull) : 0u;
    }
}

// Start of a step: sequence s takes token ids[s * n + i] (forced tokens) or
// keeps tok[s] (its previous greedy output); it runs at its cached length
// unless it is past nseq, halted, or fed the inactive id.
__global__ void batch_begin_kernel(BatchState b, const uint32_t *ids, int64_t n, int64_t i) {
    const int s = threadIdx.x;
    if (s >= b.lanes) return;
    uint32_t t = b.tok[s];
    if (ids && s < b.nseq) t = ids[(size_t)s * n + i];
    b.tok[s] = t;
    const bool run = s < b.nseq && !b.halted[s] && t != BATCH_INACTIVE;
    b.cur_pos[s] = run ? b.pos[s] : -1;
    b.nan_codes[s] = NAN_NONE;
    b.embed_ids[s] = run ? t : 0u;
}

// End of a step: a sequence whose guards held advances and (greedy) feeds its
// argmax back; one whose guard fired halts with the stage code.
__global__ void batch_end_kernel(BatchState b, uint32_t *out, int64_t n, int64_t i, int greedy) {
    const int s = threadIdx.x;
    if (s >= b.nseq || b.cur_pos[s] < 0) return;
    if (b.nan_codes[s] != NAN_NONE) {
        b.halted[s] = 1;
        b.err[s] = b.nan_codes[s];
        return;
    }
    b.pos[s] += 1;
    const uint32_t nx = b.next[s];
    if (greedy) b.tok[s] = nx;
    if (out) out[(size_t)s * n + i] = nx;
}

template <int NV, int VPW>
int launch_q4(const BatchGemvParams &p, hipStream_t s) {
    // two rows per lane halve the LDS reads per FMA (long matrices); one row
    // per lane when that leaves too few workgroups, and then the batch is
    // split over the grid's second dimension, four vectors per workgroup (two
    // waves of two): with fewer rows than lanes to fill the chip, more and
    // smaller workgroups keep more SIMDs busy (Qwen2.5-1.5B shapes, batch 16:
    // 5.45 -> 4.96 ms per step)
    if (p.N >= 16 * 1024) {
        const size_t lds = (size_t)2 * NV * 8 * BQ_CROW * 4;
        hipLaunchKernelGGL((gemv_batch_q4_kernel<NV, VPW, 2>), dim3((unsigned)((p.N + 15) / 16)), dim3(NV / VPW * 64), lds, s, p);
    } else {
        constexpr int SNV = 4, SVPW = 2;
        static_assert(NV % SNV == 0, "the batch splits into groups of four vectors");
        const size_t lds = (size_t)2 * SNV * 8 * BQ_CROW * 4;
        hipLaunchKernelGGL((gemv_batch_q4_kernel<SNV, SVPW, 1>), dim3((unsigned)((p.N + 7) / 8), NV / SNV),
                           dim3(SNV / SVPW * 64), lds, s, p);
    }
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

template <int NV>
int launch_f32(const BatchGemvParams &p, hipStream_t s) {
    const size_t lds = (size_t)NV * p.K * 4;
    if (lds + 1024 > max_lds_per_block())
        return set_error(GAJE_ERR_UNSUPPORTED, "batched f32 matvec: %d x %lld activations exceed LDS", NV, (long long)p.K);
    hipLaunchKernelGGL((gemv_batch_f32_kernel<NV>), dim3((unsigned)((p.N + 127) / 128)), dim3(256), lds, s, p);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace

int batch_lanes(int64_t n) { return n <= 4 ? 4 : n <= 8 ? 8 : 16; }

int launch_gemv_batch(const BatchGemvParams &p, hipStream_t s) {
    if (!p.w || !p.x || !p.y || p.N <= 0 || p.nv <= 0 || p.nv > 16 || p.ldx < p.K || p.ldy < p.N)
        return set_error(GAJE_ERR_INVALID_ARG, "batched matvec: bad arguments");
    const int nv = batch_lanes(p.nv);
    if (p.fmt == FMT_Q4_0) {
        if (p.nb <= 0 || (int64_t)p.nb * 32 != p.K) return set_error(GAJE_ERR_INVALID_ARG, "batched matvec: bad K");
        if (nv == 4) return launch_q4<4, 4>(p, s);
        if (nv == 8) return launch_q4<8, 4>(p, s);
        return launch_q4<16, 4>(p, s);
    }
    if (p.fmt == FMT_F32) {
        if (!p.f32_tiled || p.K % 8) return set_error(GAJE_ERR_UNSUPPORTED, "batched matvec: f32 rows must be tiled");
        if (p.mode != MODE_STORE) return set_error(GAJE_ERR_UNSUPPORTED, "batched matvec: f32 rows store only");
        if (nv == 4) return launch_f32<4>(p, s);
        if (nv == 8) return launch_f32<8>(p, s);
        if ((size_t)16 * p.K * 4 + 1024 <= max_lds_per_block()) {
            // all 16 vectors in one workgroup of 8 waves (two per SIMD: the
            // workgroup's LDS allows one per compute unit), one row per lane
            constexpr int RB = 1, NT = 512;
            const int64_t nblk = (p.N + f32b_rows<RB, NT>() - 1) / f32b_rows<RB, NT>();
            hipLaunchKernelGGL((gemv_batch_f32_rb_kernel<RB, 16, NT>), dim3((unsigned)nblk), dim3(NT),
                               (size_t)16 * p.K * 4, s, p, nblk);
            GAJE_HIP_CHECK(hipGetLastError());
            return GAJE_OK;
        }
        if ((size_t)4 * p.K * 4 + 1024 <= max_lds_per_block()) {
            constexpr int RB = 4, NT = 256;
            const int64_t nblk = (p.N + f32b_rows<RB, NT>() - 1) / f32b_rows<RB, NT>();
            const int64_t grid = (nblk + 7) / 8 * 32;  // 4 vector groups per block
            hipLaunchKernelGGL((gemv_batch_f32_rb_kernel<RB, 4, NT>), dim3((unsigned)grid), dim3(NT), (size_t)4 * p.K * 4,
                               s, p, nblk);
            GAJE_HIP_CHECK(hipGetLastError());
            return GAJE_OK;
        }
        return launch_f32<16>(p, s);
    }
    return set_error(GAJE_ERR_UNSUPPORTED, "batched matvec: weight format %d", p.fmt);
}

int launch_rmsnorm_rows(const BatchRowParams &p, hipStream_t s) {
    if (!p.x || !p.y || p.K <= 0 || p.nv <= 0 || (p.chain_major && p.K % 8))
        return set_error(GAJE_ERR_INVALID_ARG, "rmsnorm rows: bad arguments");
    if (p.K % 32 == 0 && p.K <= RN_XB4 * 4 * 256 && p.ldx % 4 == 0 && !(((uintptr_t)p.x | (uintptr_t)p.w) & 15)) {
        hipLaunchKernelGGL(rmsnorm_rows_cm_kernel, dim3((unsigned)p.nv), dim3(256), (size_t)8 * rn_chain_row(p.K) * 4, s, p);
        GAJE_HIP_CHECK(hipGetLastError());
        return GAJE_OK;
    }
    if ((size_t)p.K * 4 + 1024 > max_lds_per_block()) return set_error(GAJE_ERR_UNSUPPORTED, "rmsnorm rows: K too large");
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((unsigned)p.nv), dim3(256), (size_t)p.K * 4, s, p);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_swiglu_rows(const BatchRowParams &p, hipStream_t s) {
    if (!p.x || !p.y || p.K <= 0 || p.nv <= 0) return set_error(GAJE_ERR_INVALID_ARG, "swiglu rows: bad arguments");
    if (!p.gnorm) {
        hipLaunchKernelGGL(swiglu_elems_kernel, dim3((unsigned)((p.K + 255) / 256), (unsigned)p.nv), dim3(256), 0, s, p);
        GAJE_HIP_CHECK(hipGetLastError());
        return GAJE_OK;
    }
    if ((size_t)p.K * 4 + 1024 > max_lds_per_block()) return set_error(GAJE_ERR_UNSUPPORTED, "swiglu rows: K too large");
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3((unsigned)p.nv), dim3(256), (size_t)p.K * 4, s, p);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_batch_begin(const BatchState &b, const uint32_t *ids, int64_t n, int64_t i, hipStream_t s) {
    hipLaunchKernelGGL(batch_begin_kernel, dim3(1), dim3(64), 0, s, b, ids, n, i);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_batch_end(const BatchState &b, uint32_t *out, int64_t n, int64_t i, int greedy, hipStream_t s) {
    hipLaunchKernelGGL(batch_end_kernel, dim3(1), dim3(64), 0, s, b, out, n, i, greedy);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_argmax_rows(const float *x, int64_t n, int64_t ld, int64_t rows, uint32_t *out, hipStream_t s) {
    if (!x || !out || n <= 0 || rows <= 0 || n > 0xFFFFFFFFll) return set_error(GAJE_ERR_INVALID_ARG, "argmax rows: bad arguments");
    hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)rows), dim3(1024), 0, s, x, n, ld, out);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
