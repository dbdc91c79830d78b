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
// Cache layout: K and V are both [kv head][dim][position].  A lane scoring
// four consecutive positions reads one 16-byte quad of each of its key
// dimensions' rows, so a wave's key loads are contiguous runs; an output
// dimension's chain reads one contiguous V row.
//
// Scores, exponentials and products are computed in parallel over positions;
// the two serial chains (the softmax sum, and each output dimension's
// accumulation) keep the reference's order, one add at a time.  A chain is
// bound by its own length, so the parallel work is spread over several
// workgroups per head (one per slice of output dimensions) to keep the loads
// that feed the chains short.
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

typedef __attribute__((address_space(3))) void lds_void;

// v_mov_b32_dpp of a float (CTRL: quad_perm 0x00-0xFF, row_shl:n 0x100+n,
// wave_ror:1 0x13C).  Lanes whose source lane lies outside the row get an
// unspecified value; every use below reads only lanes with a valid source.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// "Baton" chains: G = 64 / L serial sums run in one wave, the sum of chain g
// being v_g[0] + v_g[1] + ... + v_g[32 P - 1] in order, rounded after every add.
// At phase p (0 <= p < P) lane (g L + p) mod 64 holds chain g's running sum and
// adds the 32 values v_g[32 p .. 32 p + 31] from its own registers; the first
// of those adds takes the sum from the lane before (DPP wave_ror:1: lane i
// reads lane i - 1), which hands each chain on to the next lane.  Every lane
// executes every add (the sums held by the other lanes are discarded), so a
// phase is 32 dependent adds with no LDS read in the chain.  Values are read
// from LDS (chain g's row at base + g * stride, 16-byte aligned) one tile of L
// phases ahead, lane j of region r = lane / L holding phase t L + j of chain
// (r - t) mod G in tile t.  P is even and L a multiple of 4.  Returns each
// lane's sum; chain g's result is in lane (g L + P - 1) mod 64.
constexpr int BATON_KT = 32;  // values per lane and phase

// acc = wave_ror1(acc) + x; the two wait states cover the VALU write of acc
// that the DPP read follows.
__device__ __forceinline__ float ror_add(float acc, float x) {
    asm volatile("s_nop 1\n\tv_add_f32_dpp %0, %0, %1 wave_ror:1 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(x));
    return acc;
}

struct NoWait {
    __device__ void operator()(int) const {}
};

// ready(t) is called before tile t's values are read.
template <int L, class Ready = NoWait>
__device__ __forceinline__ float baton_chains(const float *base, int stride, int P, int lane, Ready ready = {}) {
    constexpr int G = 64 / L, KT = BATON_KT;
    const int r = lane / L, j = lane % L;
    float va[KT], vb[KT];
    auto load = [&](float (&v)[KT], int t) {
        ready(t);
        const int ph = min(t * L + j, P - 1);  // lanes past the last phase re-read it (unused)
        const int g = ((r - t) % G + G) % G;
        const float4 *src = (const float4 *)(base + g * stride + ph * KT);
#pragma unroll
        for (int i = 0; i < KT / 4; ++i) {
            const float4 x = src[i];
            v[4 * i] = x.x;
            v[4 * i + 1] = x.y;
            v[4 * i + 2] = x.z;
            v[4 * i + 3] = x.w;
        }
    };
    auto run = [&](const float (&v)[KT], int t, float acc) {
        const int nph = min(L, P - t * L);
        for (int q = 0; q < nph; q += 2) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                acc = ror_add(acc, v[0]);
#pragma unroll
                for (int i = 1; i < KT; ++i) acc = acc + v[i];
            }
        }
        return acc;
    };
    float acc = 0.0f;  // +0 in every lane: the first hand-off passes +0 to each chain's first lane
    const int T = (P + L - 1) / L;
    load(va, 0);
    for (int t = 0; t < T; t += 2) {
        if (t + 1 < T) load(vb, t + 1);
        acc = run(va, t, acc);
        if (t + 1 >= T) break;
        if (t + 2 < T) load(va, t + 2);
        acc = run(vb, t + 1, acc);
    }
    return acc;
}

// Wide decode attention: head dimension HD (64 or 128) known at compile time,
// kv_cap % 4 == 0, one workgroup of WIDE threads per (query head, slice of DS
// output dimensions).
//
// Scores.  A quad of four consecutive positions is scored by LQ = HD / 16
// lanes: lane m of the quad runs dot.rs's chains l = m and m + 4 (HD = 64) or
// l = m (HD = 128) over the key dimensions 8c + l, so each lane keeps 16 key
// loads (quads of rows of the [dim][position] cache) in flight, and the QW
// quads of a wave sit in consecutive lanes so that each row's reads coalesce.
// The horizontal sum ((a0 + a4) + (a1 + a5)) + ((a2 + a6) + (a3 + a7)) is
// formed with lane shuffles: a_l + a_{l+4} in one lane (HD = 64) or across
// lanes m ^ 4 (HD = 128), then the pair sums across lanes m ^ 1 and m ^ 2;
// addition is commutative, so every lane of the quad holds the same four
// totals, and lane m (m < 4) keeps position t4 + m.  The waves whose quads lie
// below 256 positions issue their first-round key loads before the decode
// state is read (up to the capacity), so that the state's latency hides behind
// them; the others read the position first and load only quads below the
// context.  Scores at or past the context are dropped.  Each wave takes q with
// one load and lane shuffles, so no barrier precedes the dot products.
//
// Softmax and output.  The exponentials are formed in parallel; the softmax
// sum (one chain) and the DS output dimensions' sums (DS chains) each run in
// one wave as baton chains.  Four waves copy the slice's V rows into LDS with
// LDS-direct loads while the softmax sum runs; the other waves then replace
// them, tile by tile, by the products w_t * v_t[i] (w_t = e_t * inv rounded
// first, +0 past the context) while wave 0 runs the output chains.
constexpr int WIDE = 1024;

template <int HD>
struct WideShape {
    static constexpr int LQ = HD / 16;        // lanes per quad of positions
    static constexpr int QW = WAVE / LQ;      // quads per wave
    static constexpr int CPL = 8 / LQ;        // dot chains per lane
    static constexpr int NCH = HD / 8;        // 8-dimension chunks
    static constexpr int NK = NCH * CPL;      // key quads (loads) per lane
    static constexpr int PR = WIDE / LQ * 4;  // positions per round
    static_assert(NK == 16, "16 key loads per lane");
};

// Key quads of one lane: k[c * CPL + h] is row 8c + m + 4h at byte offset off.
template <int HD>
__device__ __forceinline__ void wide_keys(float4 (&k)[16], const char *kb, uint32_t rowb, uint32_t off, int m) {
    using S = WideShape<HD>;
#pragma unroll
    for (int c = 0; c < S::NCH; ++c)
#pragma unroll
        for (int h = 0; h < S::CPL; ++h) k[c * S::CPL + h] = *(const float4 *)(kb + (uint32_t)(8 * c + m + 4 * h) * rowb + off);
}

// dot_product(q, k_t) * scale for position t4 + (m & 3) (valid in lanes m < 4).
// Lane m of a quad is lane m * QW + (quad % QW) of its wave.
template <int HD>
__device__ __forceinline__ float wide_score(const float4 (&k)[16], const float (&qv)[16], int m, float scale) {
    using S = WideShape<HD>;
    float acc[S::CPL][4];
#pragma unroll
    for (int h = 0; h < S::CPL; ++h)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[h][u] = 0.0f;
#pragma unroll
    for (int c = 0; c < S::NCH; ++c)
#pragma unroll
        for (int h = 0; h < S::CPL; ++h) {
            const int e = c * S::CPL + h;
            acc[h][0] = fmaf(qv[e], k[e].x, acc[h][0]);
            acc[h][1] = fmaf(qv[e], k[e].y, acc[h][1]);
            acc[h][2] = fmaf(qv[e], k[e].z, acc[h][2]);
            acc[h][3] = fmaf(qv[e], k[e].w, acc[h][3]);
        }
    float tot[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        float pair;  // a_l + a_{l+4}
        if constexpr (S::CPL == 2) pair = acc[0][u] + acc[1][u];
        else pair = acc[0][u] + __shfl_xor(acc[0][u], 4 * S::QW, WAVE);
        const float s2 = pair + __shfl_xor(pair, S::QW, WAVE);  // (u0 + u1), (u2 + u3)
        tot[u] = (s2 + __shfl_xor(s2, 2 * S::QW, WAVE)) * scale;
    }
    const int u = m & 3;
    return u == 0 ? tot[0] : u == 1 ? tot[1] : u == 2 ? tot[2] : tot[3];
}

// Bounded spin on an LDS counter: returns true once *c >= target, false if
// the bound (2^22 polls, tens of milliseconds) runs out.  The producers and
// consumers of the kernels below wait on each other only along chains that
// always end, so the bound is never reached; it keeps a mistake from turning
// into a hang, and the caller reports a wait that ran out (ST_WAIT in the
// sequence's guard code) so the host returns an error instead of the outputs.
__device__ __forceinline__ void wait_ran_out(const AttnParams &p, int z) {
    const uint32_t code = (uint32_t)(p.layer * 8 + ST_WAIT);
    if (p.seq_nan) atomicMin(&p.seq_nan[z], code);
    else if (p.st) atomicMin(&p.st->nan_code, code);
}

__device__ __forceinline__ bool lds_wait_ge(int *c, int target) {
    bool ok = false;
    for (int spin = 0; spin < (1 << 22); ++spin) {
        if (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) {
            ok = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    return ok;
}

template <int HD, int DS>
__global__ __launch_bounds__(WIDE) void attn_decode_wide(AttnParams p) {
    using S = WideShape<HD>;
    extern __shared__ __align__(16) float smem[];
    __shared__ float red[WIDE / WAVE];
    __shared__ float inv_slot;
    __shared__ uint64_t tab[32];              // the exponential's table, read from LDS
    __shared__ int pdone[32];                 // producer waves done with each product tile

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x;
    const int d0 = blockIdx.y * DS;
    const int g = h / (p.n_head / p.n_head_kv);
    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t cap = p.kv_cap;
    const float *Kh = p.k_cache + (size_t)g * p.kv_head_stride;
    const float *Vh = p.v_cache + (size_t)g * p.kv_head_stride + (size_t)d0 * cap;
    const uint32_t rowb = (uint32_t)cap * 4;
    // lane m of quad `quad`: the QW quads of a wave are its lanes 0..QW-1, so that
    // QW lanes read consecutive quads of one key row (coalesced 16-byte reads)
    const int m = lane / S::QW, quad = wave * S::QW + lane % S::QW;

    // ---- issue: the decode state, q, the first round of key quads ----
    typedef int vi4 __attribute__((ext_vector_type(4)));
    vi4 s4 = {0, 0, 0, 0};
    // pos, token, step, halted: one vector load, waited for only where it is
    // used (nothing writes the state during this kernel).  A volatile load would
    // be waited for at once, and a scalar load shares its wait count with the
    // kernel arguments, so the address is moved into VGPRs.
    if (p.st) {
        uint64_t sp = (uint64_t)(uintptr_t)p.st;
        asm volatile("" : "+v"(sp));
        s4 = *(const __attribute__((address_space(1))) vi4 *)sp;
    }
    // q: every wave loads the head's q (lane i element i, and 64 + i for HD =
    // 128) and hands each lane its 16 values with lane shuffles, so no barrier
    // stands between the key loads and the dot products
    const float qa = p.q[(size_t)h * HD + lane];
    const float qb = HD > 64 ? p.q[(size_t)h * HD + 64 + lane] : 0.0f;
    const uint64_t tabv = tid < 32 ? kExp2Tab[tid] : 0;
    // Round 0.  The waves whose quads start below SPEC positions load them before
    // the context is known (up to the capacity; a quad past it re-reads the last
    // quad below it), so that the state's latency hides behind their loads; the
    // other waves wait for the state and load only quads below the context.
    // (Measured: 256 keeps a 128..384-token decode from loading keys it does
    // not use, 1130 -> 1149 tok/s, and leaves a 512..768 one unchanged.)
    constexpr int SPEC = 256;
    const int wpos = wave * S::QW * 4;
    float4 k[16];
    if (p.st && wpos < SPEC) {
        const int lim0 = (int)min(cap, (int64_t)S::PR);
        wide_keys<HD>(k, (const char *)Kh, rowb, (uint32_t)min(4 * quad, lim0 - 4) * 4, m);
    } else {
        // the position through the scalar cache: a vector load would queue behind
        // the other waves' key loads
        int pos = 0;
        if (p.st) asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(pos) : "s"(p.st) : "memory");
        const int c1 = p.st ? (int)min((int64_t)max(pos + 1, 1), cap) : (int)p.ctx;
        if (wpos < c1) {
            const int lim0 = min((c1 + 3) & ~3, S::PR);
            wide_keys<HD>(k, (const char *)Kh, rowb, (uint32_t)min(4 * quad, lim0 - 4) * 4, m);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) k[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    float qv[16];  // qv[c * CPL + h] = q[8c + m + 4h]
#pragma unroll
    for (int c = 0; c < S::NCH; ++c)
#pragma unroll
        for (int hh = 0; hh < S::CPL; ++hh) {
            const int j0 = 8 * c + 4 * hh;  // + m
            qv[c * S::CPL + hh] = __shfl(j0 < 64 ? qa : qb, (j0 & 63) + m, WAVE);
        }
    if (tid < 32) tab[tid] = tabv;  // (published by the barrier after the scores)
    int ctx = (int)p.ctx;
    if (p.st) {  // (the state is uniform: readfirstlane keeps the loop bounds scalar)
        if (__builtin_amdgcn_readfirstlane(s4.w)) return;  // halted: nothing of this step runs
        ctx = __builtin_amdgcn_readfirstlane(s4.x) + 1;
    }
    const int n = chain_len(ctx);
    const int vstride = chain_row(cap) + 4;  // LDS row stride of the V slice (bank spread)
    float *sc = smem;                        // chain_row(cap) scores, then exponentials
    float *vs = sc + chain_row(cap);         // DS rows of vstride: V, then the products

    // ---- scores ----
    float mx = -INFINITY;
    for (int t0 = 0;;) {
        const float s = wide_score<HD>(k, qv, m, scale);
        const int t = t0 + 4 * quad + (m & 3);
        if (m < 4 && t < ctx) {
            sc[t] = s;
            mx = fmaxf(mx, s);  // NaN never wins, as with the reference's '>'
        }
        t0 += S::PR;
        if (t0 >= ctx) break;
        wide_keys<HD>(k, (const char *)Kh, rowb, (uint32_t)min(t0 + 4 * quad, ((ctx + 3) & ~3) - 4) * 4, m);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float max_s = red[0];
#pragma unroll
    for (int w = 1; w < WIDE / WAVE; ++w) max_s = fmaxf(max_s, red[w]);

    // exponentials, +0 up to the padded chain length
    for (int t = tid; t < n; t += WIDE) sc[t] = t < ctx ? expf_ref_t(sc[t] - max_s, tab) : 0.0f;
    if (tid < 32) pdone[tid] = 0;
    __syncthreads();
    const int P = n / BATON_KT;
    if (wave == 0) {
        const float acc = baton_chains<64>(sc, 0, P, lane);
        const float sum = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), (P - 1) & 63));
        if (lane == 0) inv_slot = 1.0f / (sum + 1e-12f);
    }
    // ---- V slice -> LDS (waves 12..15, lane i copies quad i of a 256-position
    // chunk; quads at or past ctx are not copied, a copied quad ends before the
    // row's capacity).  Issued while wave 0 runs the softmax sum, once the key
    // loads are done (so that they do not queue behind them) ----
    constexpr int VW = 4;
    if (wave >= WIDE / WAVE - VW) {
        const int nchunk = (ctx + 255) >> 8;
        for (int task = wave - (WIDE / WAVE - VW); task < DS * nchunk; task += VW) {
            const int j = task / nchunk, ch = task - j * nchunk;
            const int t = ch * 256 + lane * 4;
            if (t < ctx)
                __builtin_amdgcn_global_load_lds((const void *)(Vh + (size_t)j * cap + t),
                                                 (lds_void *)(vs + j * vstride + ch * 256), 16, 0, 0);
        }
    }

    __builtin_amdgcn_s_waitcnt(0);  // the V copies of this thread have landed
    __syncthreads();
    const float inv = inv_slot;

    // ---- products w_t * v_t[i] in place (w_t = e_t * inv rounded first; +0
    // past ctx), formed by waves 1..15 tile by tile in the order the output
    // chains read them (a tile: positions [t TP, t TP + TP) of every row), each
    // wave counting the tiles it has written in pdone; wave 0 runs the DS output
    // chains and waits for a tile's count before reading it.  The producers wait
    // for nothing, so every wait ends. ----
    constexpr int L = 64 / DS, TP = L * BATON_KT, NPROD = WIDE / WAVE - 1;
    static_assert((TP & 3) == 0, "tiles of whole quads");
    const int nq = n >> 2, T = (n + TP - 1) / TP;  // T <= 32: n <= 64 TP (the capacity check bounds n)
    if (wave != 0) {
        for (int t = 0; t < T; ++t) {
            const int qa = t * (TP / 4), nt = min(nq - qa, TP / 4);
            for (int task = tid - WAVE; task < DS * nt; task += WIDE - WAVE) {
                const int j = task % DS, t4 = 4 * (qa + task / DS);
                const float4 e = *(const float4 *)(sc + t4);
                float4 &v4 = *(float4 *)(vs + j * vstride + t4);
                const float4 v = v4;
                v4 = make_float4(t4 < ctx ? (e.x * inv) * v.x : 0.0f, t4 + 1 < ctx ? (e.y * inv) * v.y : 0.0f,
                                 t4 + 2 < ctx ? (e.z * inv) * v.z : 0.0f, t4 + 3 < ctx ? (e.w * inv) * v.w : 0.0f);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // this wave's writes of the tile come first
            if (lane == 0) __hip_atomic_fetch_add(&pdone[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    } else {
        // ---- out_i = sum_t products, DS chains in wave 0 ----
        bool waited_out = false;
        auto ready = [&](int t) {
            if (!lds_wait_ge(&pdone[t], NPROD)) waited_out = true;
        };
        const float acc = baton_chains<L>(vs, vstride, P, lane, ready);
        const int rel = (lane - (P - 1)) & 63;
        if (rel % L == 0) p.out[(size_t)h * HD + d0 + rel / L] = acc;
        if (waited_out && lane == 0) wait_ran_out(p, 0);
    }
}


// Batched decode, wide form: one workgroup of WIDE threads per (query head,
// sequence).  Scores, exponentials and the softmax sum as attn_decode_wide
// (the context is known from seq_pos, so no load is speculative).  The output
// then streams V through a ring of BW_NB LDS tiles of BW_TP(HD) positions x HD
// rows: waves 4..15 (producers) load the V rows with coalesced reads BW_D
// tiles ahead (the first BW_D during the softmax sum), form the products w_t * v_t[i] (w_t = e_t * inv rounded first,
// +0 past the context) into buffer t % BW_NB and count the tile in ready[];
// waves 0..3 run HD / 4 output chains each as baton chains over the tiles and
// count each tile in freed[] once its values are in registers.  A producer
// waits for buffer t % BW_NB to be freed by tile t - BW_NB, and a chain wave
// for tile t to be ready; since the chains never wait for a tile past the one
// after the tile they run, and BW_NB >= 2, every wait ends.
constexpr int BW_NB = 3;      // tile buffers
constexpr int BW_NCW = 4;     // chain waves
constexpr int BW_D = 6;       // V tiles in flight per producer thread (registers)
template <int HD> struct BwShape {
    static constexpr int G = HD / BW_NCW;          // chains per chain wave
    static constexpr int L = WAVE / G;             // lanes per chain
    static constexpr int TP = L * BATON_KT;        // positions per tile
    static constexpr int TPS = TP + 4;             // LDS row stride (bank spread)
    static constexpr int TILE = HD * TPS;          // floats per buffer
    static constexpr int NPW = WIDE / WAVE - BW_NCW;  // producer waves
    static constexpr int TASKS = HD * TP / 4;      // float4 products per tile
    static constexpr int PT = (TASKS + NPW * WAVE - 1) / (NPW * WAVE);  // per producer thread
};
size_t batch_wide_lds_bytes(int head_dim, int64_t cap) {
    const int64_t tile = head_dim == 64 ? BwShape<64>::TILE : BwShape<128>::TILE;
    return (size_t)(chain_row(cap) + BW_NB * tile) * 4;
}

template <int HD>
__global__ __launch_bounds__(WIDE) void attn_batch_wide(AttnParams p) {
    using S = WideShape<HD>;
    using B = BwShape<HD>;
    extern __shared__ __align__(16) float smem[];
    __shared__ float red[WIDE / WAVE];
    __shared__ float inv_slot;
    __shared__ uint64_t tab[32];
    __shared__ int ready[BW_NB], freed[BW_NB], inv_flag;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // XCD-aware order: workgroup i runs on XCD i % 8, and the R = n_head / n_kv
    // query heads of one (kv head, sequence) group take ids of one residue, so
    // they share an L2 and its K/V rows are fetched from memory once
    const int R = p.n_head / p.n_head_kv, id = blockIdx.x, slot = id >> 3;
    const int group = (slot / R) * 8 + (id & 7);
    if (group >= p.n_head_kv * p.n_seq) return;  // padding of the grid (uniform)
    const int g = group % p.n_head_kv, z = group / p.n_head_kv, h = g * R + slot % R;
    const int pos = p.seq_pos[z];
    if (pos < 0) return;  // (uniform)
    const int ctx = pos + 1;
    const float *q = p.q + z * p.seq_q_stride + (size_t)h * HD;
    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t cap = p.kv_cap;
    const float *Kh = p.k_cache + z * p.seq_kv_stride + (size_t)g * p.kv_head_stride;
    const float *Vh = p.v_cache + z * p.seq_kv_stride + (size_t)g * p.kv_head_stride;
    const uint32_t rowb = (uint32_t)cap * 4;
    const int m = lane / S::QW, quad = wave * S::QW + lane % S::QW;
    const int n = chain_len(ctx);
    float *sc = smem;                  // chain_row(cap) scores, then exponentials
    float *tiles = sc + chain_row(cap);  // [BW_NB][HD][TPS] products

    const float qa = q[lane];
    const float qb = HD > 64 ? q[64 + lane] : 0.0f;
    if (tid < 32) tab[tid] = kExp2Tab[tid];
    if (tid < BW_NB) ready[tid] = freed[tid] = 0;
    if (tid == 0) inv_flag = 0;
    float4 k[16];
    const int ctx4 = (ctx + 3) & ~3;
    if (wave * S::QW * 4 < ctx)
        wide_keys<HD>(k, (const char *)Kh, rowb, (uint32_t)min(4 * quad, min(ctx4, S::PR) - 4) * 4, m);
    else
#pragma unroll
        for (int i = 0; i < 16; ++i) k[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float qv[16];
#pragma unroll
    for (int c = 0; c < S::NCH; ++c)
#pragma unroll
        for (int hh = 0; hh < S::CPL; ++hh) {
            const int j0 = 8 * c + 4 * hh;
            qv[c * S::CPL + hh] = __shfl(j0 < 64 ? qa : qb, (j0 & 63) + m, WAVE);
        }

    // ---- scores ----
    float mx = -INFINITY;
    for (int t0 = 0;;) {
        const float sv = wide_score<HD>(k, qv, m, scale);
        const int t = t0 + 4 * quad + (m & 3);
        if (m < 4 && t < ctx) {
            sc[t] = sv;
            mx = fmaxf(mx, sv);
        }
        t0 += S::PR;
        if (t0 >= ctx) break;
        wide_keys<HD>(k, (const char *)Kh, rowb, (uint32_t)min(t0 + 4 * quad, ctx4 - 4) * 4, m);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float max_s = red[0];
#pragma unroll
    for (int w = 1; w < WIDE / WAVE; ++w) max_s = fmaxf(max_s, red[w]);
    for (int t = tid; t < n; t += WIDE) sc[t] = t < ctx ? expf_ref_t(sc[t] - max_s, tab) : 0.0f;

    const int T = (n + B::TP - 1) / B::TP;
    const int P = n / BATON_KT;
    __syncthreads();  // the exponentials (and the counters' zeros) are in LDS

    if (wave >= BW_NCW) {
        // ---- producers: the first BW_D tiles' V loads go out while wave 0 runs
        // the softmax sum; the products wait for inv (inv_flag) ----
        const int pt = tid - BW_NCW * WAVE;  // producer thread index (waves 4..15)
        float4 vr[BW_D][B::PT];
        auto loadV = [&](float4 (&v)[B::PT], int t) {
#pragma unroll
            for (int i = 0; i < B::PT; ++i) {
                const int task = pt + i * B::NPW * WAVE;
                const int row = task / (B::TP / 4), q4 = task % (B::TP / 4);
                const int t4 = t * B::TP + 4 * q4;
                v[i] = task < B::TASKS && t4 < ctx ? *(const float4 *)(Vh + (size_t)row * cap + t4)
                                                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        };
#pragma unroll
        for (int d = 0; d < BW_D; ++d)
            if (d < T) loadV(vr[d], d);
        bool waited_out = !lds_wait_ge(&inv_flag, 1);
        const float inv = inv_slot;
        auto produce = [&](const float4 (&v)[B::PT], int t) {
            const int b = t % BW_NB;
            if (t >= BW_NB && !lds_wait_ge(&freed[b], BW_NCW * (t / BW_NB))) waited_out = true;
            float *dst = tiles + b * B::TILE;
#pragma unroll
            for (int i = 0; i < B::PT; ++i) {
                const int task = pt + i * B::NPW * WAVE;
                if (task >= B::TASKS) continue;
                const int row = task / (B::TP / 4), q4 = task % (B::TP / 4);
                const int t4 = t * B::TP + 4 * q4;
                const float4 e = *(const float4 *)(sc + min(t4, n - 4));
                const float4 x = v[i];
                *(float4 *)(dst + row * B::TPS + 4 * q4) =
                    make_float4(t4 < ctx ? (e.x * inv) * x.x : 0.0f, t4 + 1 < ctx ? (e.y * inv) * x.y : 0.0f,
                                t4 + 2 < ctx ? (e.z * inv) * x.z : 0.0f, t4 + 3 < ctx ? (e.w * inv) * x.w : 0.0f);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_fetch_add(&ready[b], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        };
        for (int t0 = 0; t0 < T; t0 += BW_D) {
#pragma unroll
            for (int d = 0; d < BW_D; ++d) {
                const int t = t0 + d;
                if (t < T) {
                    produce(vr[d], t);
                    if (t + BW_D < T) loadV(vr[d], t + BW_D);
                }
            }
        }
        if (waited_out && lane == 0) wait_ran_out(p, z);
        return;
    }

    if (wave == 0) {  // the softmax sum; inv is published through inv_flag
        const float acc = baton_chains<64>(sc, 0, P, lane);
        const float sum = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), (P - 1) & 63));
        if (lane == 0) {
            inv_slot = 1.0f / (sum + 1e-12f);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __hip_atomic_store(&inv_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }

    // ---- chain waves: chains wave * G .. wave * G + G - 1 (output dimensions) ----
    {
        constexpr int L = B::L, G = B::G, KT = BATON_KT;
        const int r = lane / L, j = lane % L;
        float xa[KT], xb[KT];
        bool waited_out = false;
        auto load = [&](float (&x)[KT], int t) {
            if (!lds_wait_ge(&ready[t % BW_NB], B::NPW * (t / BW_NB + 1))) waited_out = true;
            const int jj = min(j, P - 1 - t * L);  // lanes past the last phase re-read it (unused)
            const int gg = ((r - t) % G + G) % G;
            const float4 *src = (const float4 *)(tiles + (t % BW_NB) * B::TILE + (wave * G + gg) * B::TPS + jj * KT);
#pragma unroll
            for (int i = 0; i < KT / 4; ++i) {
                const float4 v = src[i];
                x[4 * i] = v.x;
                x[4 * i + 1] = v.y;
                x[4 * i + 2] = v.z;
                x[4 * i + 3] = v.w;
            }
        };
        auto run = [&](const float (&x)[KT], int t, float acc) {
            const int nph = min(L, P - t * L);
            for (int qq = 0; qq < nph; qq += 2) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    acc = ror_add(acc, x[0]);
#pragma unroll
                    for (int i = 1; i < KT; ++i) acc = acc + x[i];
                }
            }
            // this tile's values are in registers (the adds used them): its buffer is free
            if (lane == 0) __hip_atomic_fetch_add(&freed[t % BW_NB], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            return acc;
        };
        const int Tc = (P + L - 1) / L;  // == T
        float acc = 0.0f;
        load(xa, 0);
        for (int t = 0; t < Tc; t += 2) {
            if (t + 1 < Tc) load(xb, t + 1);
            acc = run(xa, t, acc);
            if (t + 1 >= Tc) break;
            if (t + 2 < Tc) load(xa, t + 2);
            acc = run(xb, t + 1, acc);
        }
        const int rel = (lane - (P - 1)) & 63;
        if (rel % L == 0) {
            const int64_t i = (int64_t)h * HD + wave * G + rel / L, rows = (int64_t)p.n_head * HD;
            p.out[z * p.seq_q_stride + (p.out_chain_major ? (i & 7) * (rows / 8) + (i >> 3) : i)] = acc;
        }
        if (waited_out && lane == 0) wait_ran_out(p, z);
    }
}

// Batched decode (several sequences per launch): one workgroup per (query
// head, sequence) computes the head's scores once; after the softmax each
// output dimension's chain runs in its own thread (threads 0..HD-1), reading
// its V row straight from memory (the row is contiguous and the loads run
// ahead of the adds).  Same rounding sequence as attn_decode_wide.
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

    // scores: thread j takes positions 4j..4j+3 of each round
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
// The wide kernel's slice: the largest DS whose rows fit LDS, with at most 32
// product tiles of 64 / DS * BATON_KT positions (its per-tile counters).
int fast_slice(int head_dim, int64_t cap) {
    for (int ds = 8; ds >= 1; ds >>= 1) {
        if (head_dim % ds) continue;
        if (fast_lds_bytes(cap, ds) + 1024 <= max_lds_per_block() && chain_len(cap) <= 32 * (64 / ds) * BATON_KT)
            return ds;
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
    if (batch_kernel && batch_wide_lds_bytes(p.head_dim, p.kv_cap) + 1024 <= max_lds_per_block()) {
        const size_t blds = batch_wide_lds_bytes(p.head_dim, p.kv_cap);
        const int64_t groups = (int64_t)p.n_head_kv * nz, R = p.n_head / p.n_head_kv;
        const dim3 grid((unsigned)((groups + 7) / 8 * 8 * R));  // ids: (8 groups) x R per block of rows
        if (p.head_dim == 64) hipLaunchKernelGGL(attn_batch_wide<64>, grid, dim3(WIDE), blds, s, p);
        else hipLaunchKernelGGL(attn_batch_wide<128>, grid, dim3(WIDE), blds, s, p);
        GAJE_HIP_CHECK(hipGetLastError());
        return GAJE_OK;
    }
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
            fn = ds == 8 ? attn_decode_wide<64, 8> : ds == 4 ? attn_decode_wide<64, 4> : ds == 2 ? attn_decode_wide<64, 2> : attn_decode_wide<64, 1>;
        else
            fn = ds == 8 ? attn_decode_wide<128, 8> : ds == 4 ? attn_decode_wide<128, 4> : ds == 2 ? attn_decode_wide<128, 2> : attn_decode_wide<128, 1>;
        hipLaunchKernelGGL(fn, dim3(p.n_head, p.head_dim / ds, nz), dim3(WIDE), flds, s, p);
    } else {
        hipLaunchKernelGGL(attn_decode_generic, dim3(p.n_head, 1, nz), dim3(THREADS), lds, s, p);
    }
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
