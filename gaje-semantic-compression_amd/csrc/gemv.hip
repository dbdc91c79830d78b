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
// The time of a launch is the length of one lane's instruction stream, so the
// Q4_0 rows use a packed layout (below) that gives each chain lane its codes in
// one 8-byte load per four blocks, and the activations sit in LDS in chain-major
// order so a lane reads a block's four inputs with one 16-byte LDS read.  A
// lane's first weight loads are issued before the prologue and then run 8-16
// groups ahead of the arithmetic; the epilogue's operands (bias, residual,
// RoPE factors) are loaded while the row is computed.
#include "common.h"
#include "device_util.h"

namespace gaje {

namespace {

constexpr int THREADS = 256;
constexpr int MAX_GRID = 8192;

// Stands in for the weights of a tensor with no complete row, so that the
// weight ring's first loads never need a branch (they are not used).
__device__ __align__(256) uint8_t kZeroRows[65536];
constexpr int Q4_PREFETCH = 8;  // packed groups (4 blocks each) in flight per lane, short rows

__device__ __forceinline__ void pair_rows(const GemvParams &p, int mode, int64_t pr, int64_t &r0, int64_t &r1) {
    if (mode == MODE_QKV) {
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
    } else if (mode == MODE_SWIGLU) {
        r0 = pr;
        r1 = pr + p.ffn;
    } else {
        r0 = 2 * pr;
        r1 = (2 * pr + 1 < p.N) ? 2 * pr + 1 : -1;
    }
}

__device__ __forceinline__ float shfl(float v, int src) { return __shfl(v, src, WAVE); }

// Activation vector in LDS.  Q4_0 rows read it chain-major: element k sits at
// (k % 8) * stride + k / 8, so chain l's inputs are one contiguous LDS row.
struct XView {
    float *x;
    int stride;  // 0: plain layout
    __device__ __forceinline__ float &at(int64_t k) const {
        return stride ? x[(k & 7) * stride + (k >> 3)] : x[k];
    }
};

// Stores elements 4m..4m+3 of the activation vector.  Chain-major: they sit
// in chain rows 4(m&1)..4(m&1)+3 at column m/2, one 32-bit base and three
// row-stride steps; plain: one float4.
template <bool CHAIN_MAJOR>
__device__ __forceinline__ void store_quad(const XView &xv, int m, const float (&v)[4]) {
    if constexpr (CHAIN_MAJOR) {
        float *xp = xv.x + (m & 1) * 4 * xv.stride + (m >> 1);
        xp[0] = v[0];
        xp[xv.stride] = v[1];
        xp[2 * xv.stride] = v[2];
        xp[3 * xv.stride] = v[3];
    } else {
        *(float4 *)(xv.x + 4 * m) = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// ------------------------------------------------------------- Q4_0 ----
// Packed device layout of a Q4_0 row: groups of four Q4_0Blocks (128 weights,
// 80 bytes, the file's own size), written once when the weights are uploaded:
//   bytes [8l, 8l+8)  chain l (l = 0..7): dword h covers blocks 4g+2h (low
//                     nibbles) and 4g+2h+1 (high nibbles); byte c holds the code
//                     of element 8c+l of its block
//   bytes [64, 80)    the four blocks' (scale | min << 16) words
// Blocks past nb in a row's last group are zero and are never read.
// Dequantises the four codes of one block for chain l: fma(q, scale, min).
__device__ __forceinline__ void q4_dequant(float (&d)[4], uint32_t codes, uint32_t sm) {
    const float scale = half_lo(sm), mn = half_hi(sm);
    d[0] = fmaf(ubyte0(codes), scale, mn);
    d[1] = fmaf(ubyte1(codes), scale, mn);
    d[2] = fmaf(ubyte2(codes), scale, mn);
    d[3] = fmaf(ubyte3(codes), scale, mn);
}

__device__ __forceinline__ float q4_chain(float acc, const float (&d)[4], const float4 x) {
    acc = fmaf(d[0], x.x, acc);
    acc = fmaf(d[1], x.y, acc);
    acc = fmaf(d[2], x.z, acc);
    acc = fmaf(d[3], x.w, acc);
    return acc;
}

// x of one packed group for chain l: its four blocks' four inputs.
struct X4 {
    float4 b0, b1, b2, b3;
};
__device__ __forceinline__ X4 read_x4(const float *xg) {
    return X4{*(const float4 *)(xg), *(const float4 *)(xg + 4), *(const float4 *)(xg + 8), *(const float4 *)(xg + 12)};
}

// One full packed group (blocks 4g .. 4g+3): the sixteen dequantised values
// are formed before the chain consumes them, so the conversions overlap the
// LDS reads instead of alternating with the dependent FMAs.
//
// The codes are never converted to float on their own.  A 4-bit code q masked
// into bits 0..3 of a 16-bit half is the f16 subnormal q * 2^-24, and masked
// into bits 4..7 it is q * 2^-20; v_fma_mix_f32 reads such a half exactly, so
// fma(q * 2^-k, scale * 2^k, min) with the f32 scale * 2^k (exact: a power-of-
// two shift of an f16) has the exact product q * scale and rounds once, the
// same value as fma(q, scale, min) for every scale and min.  A chain dword h
// holds block 2h's codes in the low nibbles (element c in byte c) and block
// 2h+1's in the high ones, so one AND gives two of block 2h's codes at 2^-24
// (elements 0 and 2 in the halves) and one two of block 2h+1's at 2^-20; the
// dword shifted right by 8 gives elements 1 and 3 the same way.  Per group
// that is 2 shifts, 8 ANDs and 4 scale products instead of 16 byte-to-float
// conversions (half-rate instructions) and 6 masks.
__device__ __forceinline__ float f16_lo(uint32_t v) {
    union { uint16_t u; _Float16 h; } c;
    c.u = (uint16_t)v;
    return (float)c.h;
}
__device__ __forceinline__ float f16_hi(uint32_t v) {
    union { uint16_t u; _Float16 h; } c;
    c.u = (uint16_t)(v >> 16);
    return (float)c.h;
}

// The four values of block 2h (dq = 0) or 2h+1 (dq = 1) of chain dword n,
// with sm its scale | min << 16 word.
template <int DQ>
__device__ __forceinline__ void q4_dequant_dw(float (&d)[4], uint32_t n, uint32_t sm) {
    constexpr uint32_t M = DQ ? 0x00F000F0u : 0x000F000Fu;
    // S = scale * 2^20 or 2^24 in one v_fma_mix_f32 reading the f16 scale from
    // the low half (exact: a power-of-two shift of an f16; + -0 keeps the
    // product's sign, zeros included), in place of a conversion and a multiply
    float S;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]"
        : "=v"(S)
        : "v"(sm), "v"(DQ ? 1048576.0f : 16777216.0f), "v"(-0.0f));
    const float mn = half_hi(sm);
    const uint32_t e02 = opaque_and(n, M), e13 = opaque_and(n >> 8, M);
    d[0] = fmaf(f16_lo(e02), S, mn);
    d[1] = fmaf(f16_lo(e13), S, mn);
    d[2] = fmaf(f16_hi(e02), S, mn);
    d[3] = fmaf(f16_hi(e13), S, mn);
}

__device__ __forceinline__ float q4_group(float acc, const vu2 n, const vu4 s, const X4 &x) {
    float d0[4], d1[4], d2[4], d3[4];
    q4_dequant_dw<0>(d0, n.x, s.x);
    q4_dequant_dw<1>(d1, n.x, s.y);
    q4_dequant_dw<0>(d2, n.y, s.z);
    q4_dequant_dw<1>(d3, n.y, s.w);
    acc = q4_chain(acc, d0, x.b0);
    acc = q4_chain(acc, d1, x.b1);
    acc = q4_chain(acc, d2, x.b2);
    acc = q4_chain(acc, d3, x.b3);
    return acc;
}

// Register ring of D packed groups of one row (this lane's chain bytes and
// the group's scale/min words).
template <int D>
struct Q4Ring {
    vu2 n[D];
    vu4 s[D];
};

// The row's last groups from ring slots 0..T-1, branch-free: `left` blocks
// remain.  A slot past the row holds finite or non-finite bytes of the
// following rows or of the tensor's padding, so the scale/min word of every
// block that does not exist is replaced by zero (its four values dequantise to
// +0), and the chain-major activation rows are zero past their last block
// (q4_zero_x_pad).  The step fma(+0, +0, acc) returns acc unchanged (acc starts
// at +0 and is never -0), so the chain's rounding sequence is the row's own and
// the selects stay off the dependent chain.  xc holds slot 0's inputs.
template <int T, int D>
__device__ __forceinline__ float q4_tail(float acc, const Q4Ring<D> &r, const float *xg, X4 xc, int left) {
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const X4 xn = read_x4(xg + 16 * (i + 1));
        const int b = left - 4 * i;  // blocks of this group that exist (<= 0: none)
        vu4 s = r.s[i];
        s.x = b > 0 ? s.x : 0u;
        s.y = b > 1 ? s.y : 0u;
        s.z = b > 2 ? s.z : 0u;
        s.w = b > 3 ? s.w : 0u;
        acc = q4_group(acc, r.n[i], s, xc);
        xc = xn;
    }
    return acc;
}

// Issues the loads of the row's first D groups.  A row shorter than D groups
// reads into the next row or the tensor's tail padding (Q4_TAIL_PAD); those
// values are never used.
template <bool NT, int D>
__device__ __forceinline__ void q4_prefetch(const uint8_t *w, const GemvParams &p, int64_t row, int l, Q4Ring<D> &r) {
    const int G = (p.nb + 3) >> 2;
    const uint8_t *rp = w + (size_t)row * G * 80;
#pragma unroll
    for (int i = 0; i < D; ++i) {
        r.n[i] = ld_u2<NT>(rp + i * 80 + 8 * l);
        r.s[i] = ld_u4<NT>(rp + i * 80 + 64);
    }
}

// Walks the row's groups in order (chain l of the row); each ring slot is
// refilled D groups ahead right after it is consumed (past the row's end the
// refills read the next row or the padding and are not used).  The LDS reads
// of a group's inputs are issued one group ahead of its arithmetic.  Returns
// the flushed dot product in lane `base`.
template <bool NT, int D>
__device__ __forceinline__ float q4_consume(const GemvParams &p, const XView &xv, int64_t row, int l, int base,
                                            Q4Ring<D> &r) {
    const int nb = p.nb;
    const int G = (nb + 3) >> 2;  // groups, the last one possibly partial
    const int Gf = nb >> 2;       // full groups
    const uint8_t *gp = p.w + (size_t)row * G * 80 + D * 80 + 8 * l;  // next group to load (chain bytes)
    const float *xg = xv.x + l * xv.stride;
    float acc = 0.0f;
    X4 xc = read_x4(xg);
    int g = 0;
    for (; g + D <= Gf; g += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const X4 xn = read_x4(xg + 16 * (i + 1));
            acc = q4_group(acc, r.n[i], r.s[i], xc);
            r.n[i] = ld_u2<NT>(gp + i * 80);
            r.s[i] = ld_u4<NT>(gp + i * 80 + 64 - 8 * l);
            xc = xn;
        }
        gp += D * 80;
        xg += 16 * D;
    }
    // the last <= D groups are already in the ring, in order: one branch-free
    // pass over T slots (T = D - 1, D or D/2)
    const int rem = G - g;
    if (rem == D - 1) acc = q4_tail<D - 1, D>(acc, r, xg, xc, nb - 4 * g);
    else if (rem > D / 2) acc = q4_tail<D, D>(acc, r, xg, xc, nb - 4 * g);
    else if (rem > 0) acc = q4_tail<D / 2, D>(acc, r, xg, xc, nb - 4 * g);
    // lanes base..base+7 hold chains 0..7; the sum is valid in lane base
    return flush_small(red8_dpp(acc));
}

// Ring depth of the Q4_0 row walk for rows of nb blocks: a short row's groups
// are all in flight at once; long rows keep 16 groups (64 blocks) ahead.
__host__ __device__ constexpr int q4_depth(int nb) { return (nb + 3) / 4 > Q4_PREFETCH ? 2 * Q4_PREFETCH : Q4_PREFETCH; }

// Floats of a chain-major activation row that the row walk may read: every
// group's 16 inputs, plus the slots a tail pass reads past the last group.
__host__ __device__ constexpr int q4_xrow(int nb) { return 16 * ((nb + 3) / 4 + q4_depth(nb) / 2); }

// Zeroes chain-major positions [4 nb, q4_xrow(nb)) of the eight activation rows
// (inputs of blocks that do not exist, read by the tail pass).
__device__ __forceinline__ void q4_zero_x_pad(const XView &xv, int nb) {
    const int from = 4 * nb, per_row = (q4_xrow(nb) - from) >> 2;  // float4s per row (from % 4 == 0)
    for (int t = threadIdx.x; t < 8 * per_row; t += blockDim.x) {
        const int l = t / per_row, c = t - l * per_row;
        *(float4 *)(xv.x + l * xv.stride + from + 4 * c) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// ---------------------------------------------------------------- Q8_0 ----
// Packed Q8_0 rows (genomic_dot_product_q8_0_avx2, genomic.rs:377-448, has
// the Q4_0 kernel's chain structure: lane l owns element 8c+l of every block),
// in tiles of 8 rows, so that the 8 rows a wave walks together are read with
// contiguous, aligned loads.  A tile of G groups (four Q8_0Blocks, 128
// weights, each) holds, for group g:
//   codes   [1024 g, 1024 g + 1024): row k's 128 bytes at 128 k, chain l's 16
//           at 16 l within them: dword b = block 4g+b, byte c = element 8c+l
//           (signed)
//   scales  [1024 G + 64 g, + 64): row k's four f16 scales at 8 k
// 1088 bytes per group and tile: the file's 136 per group and row.  Rows past
// N in the last tile and blocks past nb are zero.
constexpr int Q8_CODES = 1024;                     // bytes of one group's codes in a tile
constexpr int Q8_SCALES = 64;                      // bytes of one group's scales in a tile
constexpr int Q8_TILE_GROUP = Q8_CODES + Q8_SCALES;

template <int D>
struct Q8Ring {
    vu4 n[D];
    vu2 s[D];
};

// A row's group-0 codes (chain 0) and scales; group indices past the row's
// last group read the last group (loaded, never used), so every read stays in
// the row's tile.  G is the tensor's groups per row.
struct Q8Row {
    const uint8_t *c, *s;
    int last;
};
__device__ __forceinline__ Q8Row q8_row(const uint8_t *w, int64_t row, int G) {
    const uint8_t *t = w + (size_t)(row >> 3) * G * Q8_TILE_GROUP;
    return Q8Row{t + (row & 7) * 128, t + (size_t)G * Q8_CODES + (row & 7) * 8, G - 1};
}
template <bool NT>
__device__ __forceinline__ void q8_load(const Q8Row &q, int g, int l, vu4 &n, vu2 &sc) {
    const int gi = g < q.last ? g : q.last;
    n = ld_u4<NT>(q.c + (size_t)gi * Q8_CODES + 16 * l);
    sc = ld_u2<NT>(q.s + (size_t)gi * Q8_SCALES);
}

// dq = f32(q) * scale (genomic.rs:425-428): an exact product
__device__ __forceinline__ void q8_dequant(float (&d)[4], uint32_t codes, float scale) {
#pragma unroll
    for (int c = 0; c < 4; ++c) d[c] = (float)(int32_t)(int8_t)(codes >> (8 * c)) * scale;
}

__device__ __forceinline__ float q8_group(float acc, const vu4 n, const vu2 s, const X4 &x) {
    float d0[4], d1[4], d2[4], d3[4];
    q8_dequant(d0, n.x, half_lo(s.x));
    q8_dequant(d1, n.y, half_hi(s.x));
    q8_dequant(d2, n.z, half_lo(s.y));
    q8_dequant(d3, n.w, half_hi(s.y));
    acc = q4_chain(acc, d0, x.b0);
    acc = q4_chain(acc, d1, x.b1);
    acc = q4_chain(acc, d2, x.b2);
    acc = q4_chain(acc, d3, x.b3);
    return acc;
}

// Group i's scales with those of blocks past the row's end (b = blocks left
// from the group's first block) set to +0: their values dequantise to +-0
// against zero activations.
__device__ __forceinline__ vu2 q8_mask_scales(vu2 s, int b) {
    s.x = (b > 0 ? s.x & 0xFFFFu : 0u) | (b > 1 ? s.x & 0xFFFF0000u : 0u);
    s.y = (b > 2 ? s.y & 0xFFFFu : 0u) | (b > 3 ? s.y & 0xFFFF0000u : 0u);
    return s;
}

// The row's last groups, as q4_tail.
template <int T, int D>
__device__ __forceinline__ float q8_tail(float acc, const Q8Ring<D> &r, const float *xg, X4 xc, int left) {
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const X4 xn = read_x4(xg + 16 * (i + 1));
        acc = q8_group(acc, r.n[i], q8_mask_scales(r.s[i], left - 4 * i), xc);
        xc = xn;
    }
    return acc;
}

// The ring's D slots <- groups 0..D-1 of the row.  Gw: the groups per row of
// the tensor at w (1 for the zero stand-in of a tensor with no stored row).
template <bool NT, int D>
__device__ __forceinline__ void q8_prefetch(const uint8_t *w, int Gw, int64_t row, int l, Q8Ring<D> &r) {
    const Q8Row q = q8_row(w, row, Gw);
#pragma unroll
    for (int i = 0; i < D; ++i) q8_load<NT>(q, i, l, r.n[i], r.s[i]);
}

// q4_consume for packed Q8_0 rows: the same walk, ring and reduction.
template <bool NT, int D>
__device__ __forceinline__ float q8_consume(const GemvParams &p, const XView &xv, int64_t row, int l, int base,
                                            Q8Ring<D> &r) {
    const int nb = p.nb;
    const int G = (nb + 3) >> 2;
    const int Gf = nb >> 2;
    const Q8Row q = q8_row(p.w, row, G);
    const float *xg = xv.x + l * xv.stride;
    float acc = 0.0f;
    X4 xc = read_x4(xg);
    int g = 0;
    for (; g + D <= Gf; g += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const X4 xn = read_x4(xg + 16 * (i + 1));
            acc = q8_group(acc, r.n[i], r.s[i], xc);
            q8_load<NT>(q, g + D + i, l, r.n[i], r.s[i]);
            xc = xn;
        }
        xg += 16 * D;
    }
    const int rem = G - g;
    if (rem == D - 1) acc = q8_tail<D - 1, D>(acc, r, xg, xc, nb - 4 * g);
    else if (rem > D / 2) acc = q8_tail<D, D>(acc, r, xg, xc, nb - 4 * g);
    else if (rem > 0) acc = q8_tail<D / 2, D>(acc, r, xg, xc, nb - 4 * g);
    return flush_small(red8_dpp(acc));  // valid in lane base
}

// Q8_0Block rows (file layout, 34 bytes per block) -> the tiled layout; one
// thread per (tile, group, row of the tile).
__global__ void pack_q8_0_kernel(const uint8_t *src, uint8_t *dst, int64_t N, int nb) {
    const int G = (nb + 3) >> 2;
    const int64_t tiles = (N + 7) >> 3, total = tiles * G * 8;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int k = (int)(t & 7);
        const int64_t tg = t >> 3, tile = tg / G;
        const int g = (int)(tg - tile * G);
        const int64_t row = tile * 8 + k;
        uint8_t *tb = dst + (size_t)tile * G * Q8_TILE_GROUP;
        uint32_t *codes = (uint32_t *)(tb + (size_t)g * Q8_CODES + 128 * k);
        uint32_t *scales = (uint32_t *)(tb + (size_t)G * Q8_CODES + (size_t)g * Q8_SCALES + 8 * k);
        const uint8_t *rs = src + (size_t)(row < N ? row : 0) * nb * 34;
        for (int l = 0; l < 8; ++l)
            for (int b = 0; b < 4; ++b) {
                const int j = 4 * g + b;
                uint32_t word = 0;
                if (row < N && j < nb)
                    for (int c = 0; c < 4; ++c) word |= (uint32_t)rs[(size_t)j * 34 + 2 + 8 * c + l] << (8 * c);
                codes[4 * l + b] = word;
            }
        for (int h = 0; h < 2; ++h) {
            uint32_t w2 = 0;
            for (int half = 0; half < 2; ++half) {
                const int j = 4 * g + 2 * h + half;
                if (row < N && j < nb)
                    w2 |= ((uint32_t)rs[(size_t)j * 34] | ((uint32_t)rs[(size_t)j * 34 + 1] << 8)) << (16 * half);
            }
            scales[h] = w2;
        }
    }
    uint32_t *pad = (uint32_t *)(dst + (size_t)tiles * G * Q8_TILE_GROUP);
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < Q8_TAIL_PAD / 4; t += (int64_t)gridDim.x * blockDim.x)
        pad[t] = 0;
}

// Packs Q4_0Block rows (file layout) into the layout above; one thread per
// (row, group).
__global__ void pack_q4_0_kernel(const uint8_t *src, uint8_t *dst, int64_t N, int nb) {
    const int G = (nb + 3) >> 2;
    const int64_t total = N * G;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = t / G;
        const int g = (int)(t - row * G);
        const uint8_t *rs = src + (size_t)row * nb * 20;
        uint32_t *out = (uint32_t *)(dst + ((size_t)row * G + g) * 80);
        for (int l = 0; l < 8; ++l) {
            for (int h = 0; h < 2; ++h) {
                uint32_t word = 0;
                for (int half = 0; half < 2; ++half) {
                    const int b = 4 * g + 2 * h + half;
                    if (b >= nb) continue;
                    const uint8_t *qs = rs + (size_t)b * 20 + 4;
                    for (int c = 0; c < 4; ++c) {
                        const int e = 8 * c + l;  // even element = low nibble of byte e/2
                        const uint32_t code = (qs[e >> 1] >> ((e & 1) * 4)) & 0x0Fu;
                        word |= code << (8 * c + 4 * half);
                    }
                }
                out[2 * l + h] = word;
            }
        }
        for (int b = 0; b < 4; ++b) {
            const int j = 4 * g + b;
            uint32_t sm = 0;
            if (j < nb) {
                const uint8_t *blk = rs + (size_t)j * 20;
                sm = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8) | ((uint32_t)blk[2] << 16) | ((uint32_t)blk[3] << 24);
            }
            out[16 + b] = sm;
        }
    }
    uint32_t *pad = (uint32_t *)(dst + (size_t)total * 80);  // the tail padding reads as zeros
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < Q4_TAIL_PAD / 4; t += (int64_t)gridDim.x * blockDim.x)
        pad[t] = 0;
}

// Row-major f32 rows -> tiled layout; one thread per 8-float chunk slot.
__global__ void pack_f32_tiled_kernel(const float *src, float *dst, int64_t N, int64_t K) {
    const int64_t C = K / 8;
    const int64_t total = (N + 31) / 32 * 32 * C;  // chunk slots
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = t & 31, tc = t >> 5;  // row in tile, (tile, chunk)
        const int64_t tile = tc / C, c = tc - tile * C;
        const int64_t row = tile * 32 + r;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
        if (row < N) {
            a = *(const float4 *)(src + row * K + 8 * c);
            b = *(const float4 *)(src + row * K + 8 * c + 4);
        }
        *(float4 *)(dst + 8 * t) = a;
        *(float4 *)(dst + 8 * t + 4) = b;
    }
}

// ----------------------------------------------------------------- f32 ----
// LPR = 2: lane h owns chains 4h..4h+3 (one float4 of each 8-float chunk).
// F32_AHEAD chunks of the row are in flight per lane.  Row-major rows step 8
// floats from chunk to chunk; tiled rows (a wave's 32 rows are one tile) step
// one KiB, and each of the wave's chunk loads is one contiguous KiB.
constexpr int F32_AHEAD = 16;
struct F32Ring {
    float4 w[F32_AHEAD];
};

// This lane's first weight quad of `row` and the float stride between its chunks.
__device__ __forceinline__ const float *f32_lane_ptr(const uint8_t *w, const GemvParams &p, int64_t row, int s,
                                                     int64_t &cstride) {
    if (p.f32_tiled) {
        cstride = 256;
        return (const float *)w + (size_t)(row >> 5) * (size_t)p.K * 32 + (row & 31) * 8 + 4 * s;
    }
    cstride = 8;
    return (const float *)w + (size_t)row * p.K + 4 * s;
}

template <bool NT>
__device__ __forceinline__ void f32_prefetch(const uint8_t *w, const GemvParams &p, int64_t row, int s, F32Ring &r) {
    const int64_t chunks = p.K / 8;
    int64_t cs;
    const float *wl = f32_lane_ptr(w, p, row, s, cs);
#pragma unroll
    for (int u = 0; u < F32_AHEAD; ++u) r.w[u] = ld_f4<NT>(wl + cs * (u < chunks ? u : (chunks > 0 ? chunks - 1 : 0)));
}

template <bool NT>
__device__ __forceinline__ float f32_consume(const GemvParams &p, const float *xs, int64_t row, int s, int base,
                                             F32Ring &r) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    const float *wr = (const float *)p.w + (size_t)row * p.K;  // row-major only (scalar tail)
    int64_t cs;
    const float *wl = f32_lane_ptr(p.w, p, row, s, cs);
    const float *xl = xs + 4 * s;
    const int64_t chunks = p.K / 8;
    int64_t t = 0;
    for (; t + F32_AHEAD <= chunks; t += F32_AHEAD) {
#pragma unroll
        for (int u = 0; u < F32_AHEAD; ++u) {
            const float4 w = r.w[u];
            const int64_t tn = t + u + F32_AHEAD < chunks ? t + u + F32_AHEAD : chunks - 1;
            r.w[u] = ld_f4<NT>(wl + cs * tn);
            const float4 x = *(const float4 *)(xl + 8 * (t + u));
            a0 = fmaf(x.x, w.x, a0);
            a1 = fmaf(x.y, w.y, a1);
            a2 = fmaf(x.z, w.z, a2);
            a3 = fmaf(x.w, w.w, a3);
        }
    }
#pragma unroll
    for (int u = 0; u < F32_AHEAD; ++u) {
        if (t + u < chunks) {
            const float4 w = r.w[u];
            const float4 x = *(const float4 *)(xl + 8 * (t + u));
            a0 = fmaf(x.x, w.x, a0);
            a1 = fmaf(x.y, w.y, a1);
            a2 = fmaf(x.z, w.z, a2);
            a3 = fmaf(x.w, w.w, a3);
        }
    }
    // lane 0 holds chains 0..3, lane 1 chains 4..7: ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7))
    const float u0 = a0 + shfl(a0, base + 1), u1 = a1 + shfl(a1, base + 1);
    const float u2 = a2 + shfl(a2, base + 1), u3 = a3 + shfl(a3, base + 1);
    float sum = (u0 + u1) + (u2 + u3);
    for (int64_t i = chunks * 8; i < p.K; ++i) {  // scalar tail (row-major rows), mul then add
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

// ------------------------------------------------------------- 2-bit ----
// Genomic2Bit rows (genomic_dot_product, genomic.rs:17-144, in the x86 AVX2
// branch the reference runs): 8 bytes of MSB-first 2-bit codes per block of
// 32, four centroids per block; code 00/01/10/11 selects c0/c1/c3/c2 (times
// the modulation factors).  Per block the reference accumulates the 32
// products in two 8-lane FMA accumulators over two 4-byte steps (weights
// 16t..16t+7 to the first, 16t+8..16t+15 to the second), sums them lane by
// lane and reduces ((a0+a4)+(a1+a5))+((a2+a6)+(a3+a7)); the row sum adds the
// block values in block order and flushes |sum| < 1e-5.  Here lane s of the
// row's LPR computes whole blocks s, s+LPR, ...; the row sum then takes the
// LPR block values of each round from the lanes in order.

// Lanes per row: rows of more than 8 blocks spread over 32 lanes (one round of
// whole blocks per lane for K <= 1024), so few-row matvecs keep short lane
// streams.
inline int g2_lanes(int nb) { return nb > 8 ? 32 : 8; }

// Code bits at `pos` (low bit) of `word` -> the selected centroid: two
// sign-extended bit fields used as select masks (v_bfi).
__device__ __forceinline__ float g2_pick(uint32_t word, int pos, uint32_t c00, uint32_t c01, uint32_t c10,
                                         uint32_t c11) {
    const uint32_t b0 = (uint32_t)__builtin_amdgcn_sbfe((int)word, pos, 1);
    const uint32_t b1 = (uint32_t)__builtin_amdgcn_sbfe((int)word, pos + 1, 1);
    const uint32_t lo = (b0 & c01) | (~b0 & c00), hi = (b0 & c11) | (~b0 & c10);
    return __uint_as_float((b1 & hi) | (~b1 & lo));
}

template <bool NT, int LPR>
__device__ __forceinline__ float row_g2(const GemvParams &p, const float *xs, int64_t row, int s, int base) {
    const int nb = p.nb;
    const uint8_t *rowp = p.w + (size_t)row * nb * 8;
    const float *crow = p.lut + (row < p.lut_rows_own ? (size_t)row * nb * 4 : 0);
    float sum = 0.0f;
    for (int j0 = 0; j0 < nb; j0 += LPR) {
        const int j = j0 + s;
        float bv = 0.0f;
        if (j < nb) {
            const vu2 cw = ld_u2<NT>(rowp + (size_t)j * 8);
            float4 c = ld_f4<NT>(crow + (size_t)j * p.lut_block_stride);
            if (p.g2_modulated) {  // uniform
                c.x = c.x * p.g2_mod[0];
                c.y = c.y * p.g2_mod[1];
                c.z = c.z * p.g2_mod[2];
                c.w = c.w * p.g2_mod[3];
            }
            // codes 00, 01, 10, 11 -> c0, c1, c3, c2
            const uint32_t k00 = __float_as_uint(c.x), k01 = __float_as_uint(c.y), k10 = __float_as_uint(c.w),
                           k11 = __float_as_uint(c.z);
            const float *xb = xs + (size_t)j * 32;
            float acc0[8], acc1[8];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint32_t word = t ? cw.y : cw.x;  // bytes 4t..4t+3, byte q at bits 8q
                const float4 x0 = *(const float4 *)(xb + 16 * t), x1 = *(const float4 *)(xb + 16 * t + 4);
                const float4 x2 = *(const float4 *)(xb + 16 * t + 8), x3 = *(const float4 *)(xb + 16 * t + 12);
                const float xv[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                                      x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int pos = 8 * (e >> 2) + 6 - 2 * (e & 3);  // weight e of the step, MSB first
                    const float w = g2_pick(word, pos, k00, k01, k10, k11);
                    if (e < 8) acc0[e] = fmaf(w, xv[e], t ? acc0[e] : 0.0f);
                    else acc1[e - 8] = fmaf(w, xv[e], t ? acc1[e - 8] : 0.0f);
                }
            }
            float a[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = acc0[e] + acc1[e];
            bv = ((a[0] + a[4]) + (a[1] + a[5])) + ((a[2] + a[6]) + (a[3] + a[7]));
        }
        const int nv = nb - j0 < LPR ? nb - j0 : LPR;  // uniform
        for (int t = 0; t < nv; ++t) sum = sum + shfl(bv, base + t);
    }
    return fabsf(sum) < 1e-5f ? 0.0f : sum;
}

// compute_single_row's tail: anchors, then the bias (already loaded) if the
// row has one.
__device__ __forceinline__ float finish_row(const GemvParams &p, const XView &xv, int64_t r, float v, float bias) {
    if (p.a_ptr) {
        for (int64_t k = p.a_ptr[r]; k < p.a_ptr[r + 1]; ++k) {
            const float prod = xv.at(p.a_col[k]) * half_bits(p.a_val[k]);
            v = v + prod;
        }
    }
    if (r < p.bias_len) v = v + bias;
    return v;
}

// rms_norm's reduction of the eight sum-of-squares chains held by lanes 0..7:
// ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)), read out of the lanes (no LDS round
// trip), the same value in every lane.
__device__ __forceinline__ float rms_tot8(float a) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), i));
    return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
}

// rms_norm's 1/rms over the chain-major LDS copy (norm.rs:52-88): lane l < 8
// walks chain l (elements 8i + l), which is its own LDS row, reduces the eight
// chains, and lane 0 stores 1/sqrt(ss/n + eps) in *inv_slot.  K % 32 == 0 here,
// so there is no tail.  The rows are zero past their K/8 values
// (q4_zero_x_pad) for at least the rounding to 64 plus the chain's read-ahead,
// and fma(0, 0, acc) leaves the chain unchanged (acc >= +0), so it runs over
// the rounded length.  The caller synchronises before reading the slot.
__device__ inline void rms_inv_chain_major(const XView &xv, int64_t K, float eps, float *inv_slot) {
    const int tid = threadIdx.x;
    if (tid >= 8) return;
    const int n8 = (int)(K / 8);
    const float acc = chain_lds_sq(0.0f, xv.x + tid * xv.stride, (n8 + 63) & ~63);
    const float tot = rms_tot8(acc);  // ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7))
    if (tid == 0) {
        const float mean = tot / (float)K;
        *inv_slot = 1.0f / sqrtf(mean + eps);
    }
}

// The fused QKV epilogue of a RoPE pair (attention.rs:62-82 with the
// host-built cos/sin table): q and k get (v0*cos - v1*sin, v0*sin + v1*cos),
// every product rounded; q goes to q_out, k and v to the cache at position pos.
__device__ __forceinline__ void qkv_store(const GemvParams &p, int64_t r0, int64_t r1, float y0, float y1, float cs,
                                          float sn, int pos) {
    const float t0 = y0 * cs, t1 = y1 * sn, t2 = y0 * sn, t3 = y1 * cs;
    const float o0 = t0 - t1, o1 = t2 + t3;
    if (r0 < p.q_rows) {
        p.q_out[r0] = o0;
        p.q_out[r1] = o1;
    } else if (r0 < p.q_rows + p.kv_rows) {
        // K cache: [kv head][dim][position]
        const int64_t kh = (r0 - p.q_rows) / p.head_dim;
        const int64_t b = p.q_rows + kh * p.head_dim;
        float *kc = p.k_cache + kh * p.kv_head_stride + pos;
        kc[(r0 - b) * p.kv_cap] = o0;
        kc[(r1 - b) * p.kv_cap] = o1;
    } else {
        // V cache: [kv head][dim][position]
        const int64_t vh = (r0 - p.q_rows - p.kv_rows) / p.head_dim;
        const int64_t b = p.q_rows + p.kv_rows + vh * p.head_dim;
        float *vc = p.v_cache + vh * p.kv_head_stride + pos;
        vc[(r0 - b) * p.kv_cap] = y0;
        vc[(r1 - b) * p.kv_cap] = y1;
    }
}

// Row pair -> its rows (r1 = -1 if none) and this lane's row.
struct PairRows {
    int64_t r0, r1, row;
    bool pair_ok, row_ok;
};

template <int FMT>
__device__ __forceinline__ PairRows locate(const GemvParams &p, int mode, int64_t pr, int64_t npairs, int half) {
    PairRows q;
    q.pair_ok = pr < npairs;
    q.r0 = 0;
    q.r1 = -1;
    if (q.pair_ok) pair_rows(p, mode, pr, q.r0, q.r1);
    q.row = half ? q.r1 : q.r0;
    const bool has_work = (FMT == FMT_F32) ? p.K > 0 : p.nb > 0;
    q.row_ok = q.pair_ok && q.row >= 0 && q.row < p.rows_valid && has_work;
    return q;
}

// MODE >= 0 specialises the kernel to one epilogue (a smaller kernel, whose
// instructions are fetched cold at every launch); -1 reads p.mode.
template <int FMT, int LPR, bool NT, int D, int MODE = -1>
__global__ __launch_bounds__(THREADS) void gemv_kernel(GemvParams p, int64_t npairs, int xstride, int nw_off) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float inv_slot;
    __shared__ uint64_t etab[32];  // SwiGLU: the exponential's table, read from LDS
    __shared__ int or_in[THREADS / WAVE], or_norm[THREADS / WAVE];  // barrier_or slots
    DevState *st = p.st;
    const int mode = MODE >= 0 ? MODE : p.mode;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K = p.K;
    constexpr bool CHAIN_X = FMT == FMT_Q4_0 || FMT == FMT_Q8_0;  // chain-major activations
    const XView xv{smem, CHAIN_X ? xstride : 0};

    constexpr int PAIR_LANES = 2 * LPR;
    constexpr int PAIRS_PER_WAVE = WAVE / PAIR_LANES;
    const int pslot = lane / PAIR_LANES;
    const int half = (lane % PAIR_LANES) / LPR;
    const int s = lane % LPR;
    const int row_base = lane - s;  // first lane of this row's group
    const int pair_base = pslot * PAIR_LANES;
    const int pairs_per_block = PAIRS_PER_WAVE * (THREADS / WAVE);
    float *tbl = smem + ((K + 3) & ~(int64_t)3) + (size_t)(tid / LPR) * 16;  // LUT slot of this row group

    int64_t pr0 = (int64_t)blockIdx.x * pairs_per_block;
    PairRows q = locate<FMT>(p, mode, pr0 + wave * PAIRS_PER_WAVE + pslot, npairs, half);
    Q4Ring<D> q4r;
    Q8Ring<FMT == FMT_Q8_0 ? D : 1> q8r;
    F32Ring f32r;
    const int halted = st ? st->halted : 0;
    const bool swiglu = mode == MODE_SWIGLU;
    const uint64_t tabv = swiglu && tid < 32 ? kExp2Tab[tid] : 0;

    // ---- prologue: activation vector (and the norm weights) into LDS, one
    // batch of loads in flight per thread; normalised if requested ----
    float *nw = smem + nw_off;  // plain copy of norm_w when the vector spans several batches
    int bad_in = 0;
    // float4s of the activation vector per thread and batch: Q4_0 rows with
    // the short ring have K <= 1024, which one float4 per thread covers
    constexpr int XB4 = (CHAIN_X && D == Q4_PREFETCH) ? 1 : 6;
    float4 xr[XB4], wr[XB4];
    if constexpr (FMT == FMT_LUT4) {
        constexpr int XB = 8;
        for (int64_t k0 = 0; k0 < K; k0 += XB * THREADS) {
            float xr[XB], wr[XB];
#pragma unroll
            for (int u = 0; u < XB; ++u) {
                const int64_t k = k0 + u * THREADS + tid;
                xr[u] = k < K ? p.x[k] : 0.0f;
                wr[u] = (p.norm_w && k < K) ? p.norm_w[k] : 0.0f;
            }
            if (k0 == 0 && halted) return;  // uniform; checked once the first loads are in flight
#pragma unroll
            for (int u = 0; u < XB; ++u) {
                const int64_t k = k0 + u * THREADS + tid;
                if (k < K) {
                    xv.at(k) = xr[u];
                    if (p.norm_w) nw[k] = wr[u];
                    bad_in |= isnan(xr[u]);
                }
            }
        }
    } else {
        // K % 4 == 0 and 16-byte aligned x / norm_w (checked at launch).  When
        // the vector fits one batch its values stay in registers for the norm.
        // The first batch of activation loads is issued first, then the first
        // row pair's weight ring, with no branch in between: the loads complete
        // in order, so the first use of the activations waits for them alone and
        // the weights stream in while the prologue runs.  Rows without work
        // prefetch row 0 (never used).
        const int64_t K4 = K >> 2;
        const bool one_batch = K4 <= XB4 * THREADS;
        const float4 *x4 = (const float4 *)p.x;
        const float4 *w4 = (const float4 *)p.norm_w;
#pragma unroll
        for (int u = 0; u < XB4; ++u) {
            const int64_t m = u * THREADS + tid;
            xr[u] = x4[m < K4 ? m : K4 - 1];
        }
        if (w4) {
#pragma unroll
            for (int u = 0; u < XB4; ++u) {
                const int64_t m = u * THREADS + tid;
                wr[u] = w4[m < K4 ? m : K4 - 1];
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the ring
        {
            const uint8_t *wbase = p.rows_valid > 0 ? p.w : kZeroRows;
            const int64_t prow = q.row_ok ? q.row : 0;
            if constexpr (FMT == FMT_Q4_0) q4_prefetch<NT, D>(wbase, p, prow, s, q4r);
            else if constexpr (FMT == FMT_Q8_0) q8_prefetch<NT, D>(wbase, p.rows_valid > 0 ? (p.nb + 3) >> 2 : 1, prow, s, q8r);
            else if constexpr (FMT == FMT_F32) f32_prefetch<NT>(wbase, p, prow, s, f32r);
        }
        if (halted) return;  // uniform; checked once the first loads are in flight
        auto store_batch = [&](int64_t m0) {
#pragma unroll
            for (int u = 0; u < XB4; ++u) {
                const int64_t m = m0 + u * THREADS + tid;
                if (m < K4) {
                    const float4 v = xr[u];
                    const float q[4] = {v.x, v.y, v.z, v.w};
                    store_quad<CHAIN_X>(xv, (int)m, q);
                    if (p.norm_w && !one_batch) *(float4 *)(nw + 4 * m) = wr[u];
                    bad_in |= isnan(v.x) | isnan(v.y) | isnan(v.z) | isnan(v.w);
                }
            }
        };
        store_batch(0);  // (peeled: no join between the loads above and this use)
        for (int64_t m0 = XB4 * THREADS; m0 < K4; m0 += XB4 * THREADS) {
#pragma unroll
            for (int u = 0; u < XB4; ++u) {
                const int64_t m = m0 + u * THREADS + tid;
                const int64_t mc = m < K4 ? m : K4 - 1;
                xr[u] = x4[mc];
                if (w4) wr[u] = w4[mc];
            }
            store_batch(m0);
        }
        if constexpr (CHAIN_X) q4_zero_x_pad(xv, p.nb);
        if (swiglu && tid < 32) etab[tid] = tabv;
        // barriers from here on order LDS only: the weight ring stays in flight
        if (barrier_or<THREADS / WAVE>(bad_in, or_in) && p.st_in >= 0 && tid == 0) nan_flag(st, p.layer, p.st_in);
        if (p.norm_w) {
            if constexpr (CHAIN_X) rms_inv_chain_major(xv, K, p.eps, &inv_slot);
            else rms_inv_plain(smem, K, p.eps, &inv_slot);
            lds_barrier();
            const float inv = inv_slot;
            int bad = 0;
            if (one_batch) {
#pragma unroll
                for (int u = 0; u < XB4; ++u) {
                    const int64_t m = u * THREADS + tid;
                    if (m < K4) {
                        float t[4] = {xr[u].x * inv, xr[u].y * inv, xr[u].z * inv, xr[u].w * inv};
                        const float w4[4] = {wr[u].x, wr[u].y, wr[u].z, wr[u].w};
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            t[c] = t[c] * w4[c];  // (x * inv) * w, each product rounded
                            bad |= isnan(t[c]);
                        }
                        store_quad<CHAIN_X>(xv, (int)m, t);
                    }
                }
            } else {
                for (int64_t k = tid; k < K; k += THREADS) {
                    float &x = xv.at(k);
                    const float t = x * inv;
                    x = t * nw[k];
                    bad |= isnan(x);
                }
            }
            if (barrier_or<THREADS / WAVE>(bad, or_norm) && p.st_norm >= 0 && tid == 0) nan_flag(st, p.layer, p.st_norm);
        }
    }
    if constexpr (FMT == FMT_LUT4) {
        if (swiglu && tid < 32) etab[tid] = tabv;
        if (__syncthreads_or(bad_in) && p.st_in >= 0 && tid == 0) nan_flag(st, p.layer, p.st_in);
        if (p.norm_w) {
            rmsnorm_inplace(smem, K, nw, p.eps, &inv_slot);
            int bad = 0;
            for (int64_t k = tid; k < K; k += THREADS) bad |= isnan(xv.at(k));
            if (__syncthreads_or(bad) && p.st_norm >= 0 && tid == 0) nan_flag(st, p.layer, p.st_norm);
        }
    }
    if (p.gnorm) {
        // use_genomic_norm (block/forward.rs:115-123) sums with a rayon
        // reduction whose order is not fixed upstream; a sequential sum here.
        if (tid == 0) {
            float ss = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float xk = xv.at(k);
                const float sq = xk * xk;
                ss = ss + sq;
            }
            inv_slot = sqrtf(ss / (float)K + p.eps);
        }
        lds_barrier();
        const float rms = inv_slot;
        if (rms > p.h_scale) {
            const float sc = p.h_scale / rms;
            for (int64_t k = tid; k < K; k += THREADS) xv.at(k) = xv.at(k) * sc;
        }
        lds_barrier();
    }
    if (p.x_out && blockIdx.x == 0)
        for (int64_t k = tid; k < K; k += THREADS) p.x_out[k] = xv.at(k);

    // ---- row pairs ----
    float best_v = -INFINITY;
    int64_t best_i = 0;
    const int hh = p.head_dim >> 1;

    for (bool first = true; pr0 < npairs; pr0 += (int64_t)gridDim.x * pairs_per_block, first = false) {
        const int64_t pr = pr0 + wave * PAIRS_PER_WAVE + pslot;
        if (!first) {
            q = locate<FMT>(p, mode, pr, npairs, half);
            if (q.row_ok) {
                if constexpr (FMT == FMT_Q4_0) q4_prefetch<NT, D>(p.w, p, q.row, s, q4r);
                else if constexpr (FMT == FMT_Q8_0) q8_prefetch<NT, D>(p.w, (p.nb + 3) >> 2, q.row, s, q8r);
                else if constexpr (FMT == FMT_F32) f32_prefetch<NT>(p.w, p, q.row, s, f32r);
            }
        }
        const int64_t r0 = q.r0, r1 = q.r1;
        const bool leader = q.pair_ok && lane == pair_base;
        // epilogue operands, loaded while the rows are computed
        float b0 = 0.0f, b1 = 0.0f, old0 = 0.0f, old1 = 0.0f, cs = 0.0f, sn = 0.0f;
        int pos = 0;
        if (leader) {
            if (r0 < p.bias_len) b0 = p.bias[r0];
            if (r1 >= 0 && r1 < p.bias_len) b1 = p.bias[r1];
            if (mode == MODE_RESIDUAL) {
                old0 = p.y[r0];
                if (r1 >= 0) old1 = p.y[r1];
            } else if (mode == MODE_QKV) {
                pos = st->pos;
                const int i = (int)(pr % hh);
                cs = p.rope_cos[(size_t)pos * hh + i];
                sn = p.rope_sin[(size_t)pos * hh + i];
            }
        }
        float v = 0.0f;
        // all lanes of a row group share row_ok, so each row function's
        // shuffles only read lanes that execute it
        if (q.row_ok) {
            if constexpr (FMT == FMT_Q4_0) v = q4_consume<NT, D>(p, xv, q.row, s, row_base, q4r);
            else if constexpr (FMT == FMT_Q8_0) v = q8_consume<NT, D>(p, xv, q.row, s, row_base, q8r);
            else if constexpr (FMT == FMT_F32) v = f32_consume<NT>(p, smem, q.row, s, row_base, f32r);
            else if constexpr (FMT == FMT_G2) v = row_g2<NT, LPR>(p, smem, q.row, s, row_base);
            else v = row_lut4<NT>(p, smem, q.row, s, row_base, tbl);
        }
        const float v1 = shfl(v, pair_base + LPR);  // r1's result (lane 0 of its group)
        if (!leader) continue;

        // ---- epilogue (one lane per row pair) ----
        const float y0 = finish_row(p, xv, r0, v, b0);
        const float y1 = r1 >= 0 ? finish_row(p, xv, r1, v1, b1) : 0.0f;
        switch (mode) {
            case MODE_STORE:
                p.y[r0] = y0;
                if (r1 >= 0) p.y[r1] = y1;
                break;
            case MODE_RESIDUAL: {
                if (isnan(y0) || (r1 >= 0 && isnan(y1))) nan_flag(st, p.layer, p.st_a);
                const float h0 = old0 + y0;
                p.y[r0] = h0;
                bool bad = isnan(h0);
                if (r1 >= 0) {
                    const float h1 = old1 + y1;
                    p.y[r1] = h1;
                    bad |= isnan(h1);
                }
                if (bad) nan_flag(st, p.layer, p.st_b);
                break;
            }
            case MODE_QKV:
                qkv_store(p, r0, r1, y0, y1, cs, sn, pos);
                break;
            case MODE_SWIGLU: {
                if (isnan(y1)) nan_flag(st, p.layer, p.st_a);
                const float o = swiglu1(y0, y1, etab);
                if (isnan(o)) nan_flag(st, p.layer, p.st_b);
                p.y[pr] = o;
                if (p.y_cm) p.y_cm[(pr & 7) * p.cm_stride + (pr >> 3)] = o;
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
    if (mode == MODE_ARGMAX && st) {
        unsigned long long key =
            best_v > -INFINITY
                ? ((unsigned long long)max_key(best_v) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)best_i)
                : 0ull;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(key, o, WAVE);
            key = other > key ? other : key;
        }
        if (lane == 0 && key) atomicMax(&st->argmax_key, key);
    }
}

// ------------------------------------------ Q8_0, streamed long matrices ----
// The Q8_0 lm_head (N = vocabulary, K = n_embd <= 1024): a resident grid, 8
// lanes per row (lane l runs chain l of q8_consume), row group rg walking rows
// rg, rg + R, rg + 2R, ... (R row groups in the grid, so a wave covers 8
// adjacent rows, one contiguous run of packed groups).  Two register rings
// alternate: the next row's groups are loaded before the current row is
// computed, so every wave keeps a row's weights in flight under its
// arithmetic.  Values, chain order and reduction are those of q8_consume, so
// the result is the same bit for bit.
constexpr int Q8S_D = 8;  // ring slots: rows of at most 8 packed groups (K <= 1024)
__device__ float kSinkOut[WAVE];  // stores of rows past N (never read)

// All Q8S_D slots are loaded and walked with no branch (the wait counts then
// stay exact, so the other ring's loads remain in flight): slots past the
// row's G groups reload its last group and enter with +0 scales against zero
// activations.
template <bool NT>
__device__ __forceinline__ void q8s_load(const Q8Row &q, int l, Q8Ring<Q8S_D> &r) {
#pragma unroll
    for (int i = 0; i < Q8S_D; ++i) q8_load<NT>(q, i, l, r.n[i], r.s[i]);
}

// Chain l's sum over one row: the groups in order, the scales of blocks past
// nb set to +0 (as q8_tail).  A slot past the row adds fma(+-0, +0, acc),
// which leaves acc unchanged except that -0 may become +0; the row total is
// flushed to +0 when it is that small, so the result is unchanged.
__device__ __forceinline__ float q8s_row(const float *xg, int nb, const Q8Ring<Q8S_D> &r) {
    float acc = 0.0f;
    X4 xc = read_x4(xg);
#pragma unroll
    for (int i = 0; i < Q8S_D; ++i) {
        const X4 xn = read_x4(xg + 16 * (i + 1));
        acc = q8_group(acc, r.n[i], q8_mask_scales(r.s[i], nb - 4 * i), xc);
        xc = xn;
    }
    return acc;
}

template <bool NT, int MODE>
__global__ __launch_bounds__(THREADS) void gemv_q8_stream_kernel(GemvParams p, int xstride) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float inv_slot;
    __shared__ int or_in[THREADS / WAVE], or_norm[THREADS / WAVE];
    DevState *st = p.st;
    const int tid = threadIdx.x, lane = tid & 63;
    const int l = lane & 7, base = lane - l;
    const int64_t K4 = p.K >> 2, N = p.N;
    const int nb = p.nb, G = (nb + 3) >> 2;
    const XView xv{smem, xstride};
    const int64_t R = (int64_t)gridDim.x * (THREADS / 8);
    int64_t row = (int64_t)blockIdx.x * (THREADS / 8) + (tid >> 3);
    const uint8_t *wb = p.rows_valid > 0 ? p.w : kZeroRows;
    const int Gw = p.rows_valid > 0 ? G : 1;
    // rows past the stored ones (and past N) read row 0: loaded, never used
    auto rowp = [&](int64_t r) { return q8_row(wb, r < p.rows_valid ? r : 0, Gw); };

    // ---- prologue: the activation quad of this thread, the first row's
    // weights, then the chain-major copy (normalised if requested) ----
    const bool mine = tid < K4;
    const float4 *x4 = (const float4 *)p.x;
    const float4 *w4 = (const float4 *)p.norm_w;
    const float4 xr = x4[mine ? tid : K4 - 1];
    const float4 wr = w4 ? w4[mine ? tid : K4 - 1] : make_float4(0.f, 0.f, 0.f, 0.f);
    __builtin_amdgcn_sched_barrier(0);
    Q8Ring<Q8S_D> ra, rb;
    q8s_load<NT>(rowp(row), l, ra);
    if (st && st->halted) return;  // uniform
    int bad_in = 0;
    if (mine) {
        const float q[4] = {xr.x, xr.y, xr.z, xr.w};
        store_quad<true>(xv, tid, q);
        bad_in = isnan(xr.x) || isnan(xr.y) || isnan(xr.z) || isnan(xr.w);
    }
    q4_zero_x_pad(xv, nb);
    if (barrier_or<THREADS / WAVE>(bad_in, or_in) && p.st_in >= 0 && tid == 0) nan_flag(st, p.layer, p.st_in);
    if (p.norm_w) {
        rms_inv_chain_major(xv, p.K, p.eps, &inv_slot);
        lds_barrier();
        const float inv = inv_slot;
        int bad = 0;
        if (mine) {
            float t[4] = {xr.x * inv, xr.y * inv, xr.z * inv, xr.w * inv};
            const float w[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                t[c] = t[c] * w[c];  // (x * inv) * w, each product rounded
                bad |= isnan(t[c]);
            }
            store_quad<true>(xv, tid, t);
        }
        if (barrier_or<THREADS / WAVE>(bad, or_norm) && p.st_norm >= 0 && tid == 0) nan_flag(st, p.layer, p.st_norm);
    }
    if (p.x_out && blockIdx.x == 0)
        for (int64_t k = tid; k < p.K; k += THREADS) p.x_out[k] = xv.at(k);

    // ---- rows, two per iteration: ring A holds `row`, ring B row + R; each
    // ring is reloaded as soon as it has been walked.  The loop body has no
    // branch: a second row at or past N walks a clamped row and stores into a
    // sink, and the bias is read from a zero row where there is none, so the
    // compiler's wait counts stay exact and a ring's loads stay in flight
    // while the other ring is walked. ----
    const float *xg = xv.x + l * xv.stride;
    float best_v = -INFINITY;
    int64_t best_i = 0;
    auto bias_at = [&](int64_t r) {
        return *(r < p.bias_len ? p.bias + r : (const float *)kZeroRows);
    };
    auto finish = [&](int64_t r, float acc, float bias) {
        const float u = acc + shfl(acc, base + ((l + 4) & 7));
        const float v = u + shfl(u, base + ((l + 2) & 7));
        float y = shfl(flush_small(v + shfl(v, base + ((l + 1) & 7))), base);  // lane 0's order
        y = r < p.rows_valid ? y : 0.0f;
        y = r < p.bias_len ? y + bias : y;  // finish_row without anchors
        *(r < N ? p.y + r : kSinkOut + lane) = y;  // the row group's lanes store the same value
        if constexpr (MODE == MODE_ARGMAX) {
            const bool better = r < N && y > best_v;
            best_v = better ? y : best_v;
            best_i = better ? r : best_i;
        }
    };
    auto clamp = [&](int64_t r) { return r < N ? r : row; };
    q8s_load<NT>(rowp(clamp(row + R)), l, rb);
    __builtin_amdgcn_sched_barrier(0);
    while (row < N) {
        const int64_t r1 = row + R;
        const float b0 = bias_at(row), b1 = bias_at(r1);
        const float a0 = q8s_row(xg, nb, ra);
        q8s_load<NT>(rowp(clamp(row + 2 * R)), l, ra);
        __builtin_amdgcn_sched_barrier(0);
        const float a1 = q8s_row(xg, nb, rb);
        q8s_load<NT>(rowp(clamp(row + 3 * R)), l, rb);
        __builtin_amdgcn_sched_barrier(0);
        finish(row, a0, b0);
        finish(r1, a1, b1);
        row += 2 * R;
    }
    if constexpr (MODE == MODE_ARGMAX) {
        unsigned long long key =
            best_v > -INFINITY
                ? ((unsigned long long)max_key(best_v) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)best_i)
                : 0ull;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(key, o, WAVE);
            key = other > key ? other : key;
        }
        if (lane == 0 && key) atomicMax(&st->argmax_key, key);
    }
}

// ------------------------------------------ Q4_0 rows through LDS-direct ----
// Rows of at most 8 packed groups (K <= 1024) streamed through LDS.  A wave
// walks 8-row tiles (tile t = rows 8t..8t+7, whose packed bytes are one
// contiguous run; a SwiGLU tile adds the up rows ffn+8t..): it copies each
// tile into its own LDS stages with global_load_lds_dwordx4 (each lane 16
// bytes, one KiB per instruction, no VGPRs), up to Q4L stages ahead, and lane
// (row r, chain l) then reads its chain's codes (8 bytes) and the group's
// scale/min words (16 bytes, the same for the row's 8 lanes) from LDS.  Against
// loading them into VGPRs this issues a fifth of the load instructions and
// fetches the scale/min words once instead of eight times.  The values, the
// chain order and the reduction are q4_consume's: a row's last group is zero
// past its nb blocks in the packed layout (scale = min = 0, codes 0), and the
// activation rows are zero there too, so fma(+0, +0, acc) leaves the chain as
// it is.
//
// Every load of the kernel is such a copy (the activations, the norm weights
// and the exponential's table too), issued as inline assembly so that the
// compiler's wait-count model, which would otherwise wait for all of them
// before each LDS read, leaves them alone; the kernel waits for its own copies
// with explicit s_waitcnt vmcnt counts.  Loads return in order, so "at most n
// outstanding" means every copy but the last n has landed.  A wave only reads
// the stages it filled itself, so no barrier orders them; the shared prologue
// data is copied by wave 0 before its tiles and published with a barrier.

// A 32-bit load through the scalar data cache (uniform address), waited for.
__device__ __forceinline__ int32_t s_load_i32(const void *p) {
    int32_t v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
}

// wait_vmcnt<k * per> for a wave-uniform k in [0, KMAX].
template <int per, int KMAX>
__device__ __forceinline__ void wait_vmcnt_stages(int k) {
    if constexpr (KMAX > 0) {
        if (k >= KMAX) {
            wait_vmcnt<KMAX * per>();
            return;
        }
        wait_vmcnt_stages<per, KMAX - 1>(k);
    } else {
        wait_vmcnt<0>();
    }
}

// wait_vmcnt<a * NA + b * NB> for wave-uniform a, b in [0, KMAX].
template <int NA, int NB, int KMAX, int A = KMAX, int B = KMAX>
__device__ __forceinline__ void wait_vmcnt_ab(int a, int b) {
    static_assert(KMAX * (NA + NB) < 64, "vmcnt is six bits");
    if (a == A && b == B) {
        wait_vmcnt<A * NA + B * NB>();
        return;
    }
    if constexpr (B > 0) wait_vmcnt_ab<NA, NB, KMAX, A, B - 1>(a, b);
    else if constexpr (A > 0) wait_vmcnt_ab<NA, NB, KMAX, A - 1, KMAX>(a, b);
    else wait_vmcnt<0>();
}

// Copies the N KiB from byte `off` of the weights into LDS at `dst` (wave
// uniform).  Lanes whose bytes lie at or past `end` (the tile's last byte, or
// the tensor's allocation end if that comes first) read the tile's first 16
// bytes again: those LDS bytes are never read as rows of this tile, and
// re-reading bytes the tile fetches anyway keeps the next tile's rows (another
// workgroup's, often on another L2) out of this one's memory traffic.
template <int N>
__device__ __forceinline__ void q4l_copy(const uint8_t *w, int64_t off, int64_t end, uint32_t dst, int lane) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        int64_t a = off + i * 1024 + lane * 16;
        a = a + 16 <= end ? a : off;
        lds_dma16(w + a, dst + i * 1024);
    }
}

// q4l_copy for a tile that lies wholly before the allocation's end: the
// tile's address is wave-uniform (SGPRs) and each lane adds a loop-invariant
// offset, v16 = 16 lane for the whole KiBs and vlast for the last one (its
// bytes, or the tile's first 16 again past the tile's TB bytes), so a copy
// costs no vector instruction.
template <int N>
__device__ __forceinline__ void q4l_copy_full(const uint8_t *w, int64_t off, uint32_t dst, uint32_t v16,
                                              uint32_t vlast) {
#pragma unroll
    for (int i = 0; i < N - 1; ++i) lds_dma16_so_nt(w + off + i * 1024, v16, dst + i * 1024);
    lds_dma16_so_nt(w + off, vlast, dst + (N - 1) * 1024);
}

// Copies n bytes (n % 16 == 0) from g to LDS at dst with one wave.
__device__ __forceinline__ void lds_copy_bytes(const void *g, int64_t n, uint32_t dst, int lane) {
    for (int64_t o = 0; o < n; o += 1024)
        if (o + lane * 16 < n) lds_dma16((const uint8_t *)g + o + lane * 16, dst + (uint32_t)o);
}

// Chain l of the rows at rp0 and rp1 (LDS), interleaved: groups 0..G-1 in
// order, then the reduction and the flush (q4_consume's sequence).  xr holds
// chain l's activations (16 per group), in registers for the whole kernel.
// Lane `base` holds the rows.
template <int G>
__device__ __forceinline__ void q4l_rows2(const uint8_t *rp0, const uint8_t *rp1, const float4 (&xr)[4 * G], int l,
                                          int base, float &y0, float &y1) {
    // the two rows' chain steps alternate, so that each step has the other
    // row's step between it and its predecessor (a dependent fma waits for
    // its input).  Reading the next group's LDS words a group ahead would
    // take more registers than the kernel has left (x's registers spill).
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const vu2 m0 = *(const vu2 *)(rp0 + g * 80 + 8 * l), m1 = *(const vu2 *)(rp1 + g * 80 + 8 * l);
        const vu4 t0 = *(const vu4 *)(rp0 + g * 80 + 64), t1 = *(const vu4 *)(rp1 + g * 80 + 64);
        float d0[4][4], d1[4][4];
        q4_dequant_dw<0>(d0[0], m0.x, t0.x);
        q4_dequant_dw<1>(d0[1], m0.x, t0.y);
        q4_dequant_dw<0>(d0[2], m0.y, t0.z);
        q4_dequant_dw<1>(d0[3], m0.y, t0.w);
        q4_dequant_dw<0>(d1[0], m1.x, t1.x);
        q4_dequant_dw<1>(d1[1], m1.x, t1.y);
        q4_dequant_dw<0>(d1[2], m1.y, t1.z);
        q4_dequant_dw<1>(d1[3], m1.y, t1.w);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float4 x = xr[4 * g + b];
            a0 = fmaf(d0[b][0], x.x, a0);
            a1 = fmaf(d1[b][0], x.x, a1);
            a0 = fmaf(d0[b][1], x.y, a0);
            a1 = fmaf(d1[b][1], x.y, a1);
            a0 = fmaf(d0[b][2], x.z, a0);
            a1 = fmaf(d1[b][2], x.z, a1);
            a0 = fmaf(d0[b][3], x.w, a0);
            a1 = fmaf(d1[b][3], x.w, a1);
        }
    }
    y0 = flush_small(red8_dpp(a0));
    y1 = flush_small(red8_dpp(a1));
}

// Tolerance mode (gaje_hip_q4_0_gemv_tol): the same rows regrouped by block,
// sum_k (q_k s + mn) x_k = s (sum_k q_k x_k) + mn (sum_k x_k), as the
// block-scaled MFMA product regroups them.  Chain l's four codes of a block
// enter as the f16 subnormals q 2^-24 or q 2^-20 (q4_dequant_dw's masks) and
// its inputs are held pre-scaled by 2^24 or 2^20 (exact powers of two; the
// launcher's workgroups fall back to the exact walk when some |x| >= 2^100),
// so each block costs four v_fma_mix_f32 for the code products, one for
// s * P with the f16 scale read in place and one for mn * X with the f16 min
// and the chain's block sum X of the unscaled inputs: 1.5 VALU instructions
// per weight plus the masks, against 2.875 for the exact walk.  The result
// differs from the reference's chained fmas by rounding only (the tests hold
// it to 1e-4 of the row's sum of |w x|); the |t| < 1e-6 flush is kept.
template <int G>
__device__ __forceinline__ void q4l_rows2_tol(const uint8_t *rp0, const uint8_t *rp1, const float4 (&xr)[4 * G],
                                              const float (&xsum)[4 * G], int l, float &y0, float &y1) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const vu2 m0 = *(const vu2 *)(rp0 + g * 80 + 8 * l), m1 = *(const vu2 *)(rp1 + g * 80 + 8 * l);
        const vu4 t0 = *(const vu4 *)(rp0 + g * 80 + 64), t1 = *(const vu4 *)(rp1 + g * 80 + 64);
        const uint32_t n0[2] = {m0.x, m0.y}, n1[2] = {m1.x, m1.y};
        const uint32_t s0[4] = {t0.x, t0.y, t0.z, t0.w}, s1[4] = {t1.x, t1.y, t1.z, t1.w};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t M = (b & 1) ? 0x00F000F0u : 0x000F000Fu;
            const uint32_t e02a = opaque_and(n0[b >> 1], M), e13a = opaque_and(n0[b >> 1] >> 8, M);
            const uint32_t e02b = opaque_and(n1[b >> 1], M), e13b = opaque_and(n1[b >> 1] >> 8, M);
            const float4 x = xr[4 * g + b];
            float pa = fmaf(f16_lo(e02a), x.x, -0.0f), pb = fmaf(f16_lo(e02b), x.x, -0.0f);
            pa = fmaf(f16_lo(e13a), x.y, pa);
            pb = fmaf(f16_lo(e13b), x.y, pb);
            pa = fmaf(f16_hi(e02a), x.z, pa);
            pb = fmaf(f16_hi(e02b), x.z, pb);
            pa = fmaf(f16_hi(e13a), x.w, pa);
            pb = fmaf(f16_hi(e13b), x.w, pb);
            a0 = fmaf(half_lo(s0[b]), pa, a0);
            a1 = fmaf(half_lo(s1[b]), pb, a1);
            a0 = fmaf(half_hi(s0[b]), xsum[4 * g + b], a0);
            a1 = fmaf(half_hi(s1[b]), xsum[4 * g + b], a1);
        }
    }
    y0 = flush_small(red8_dpp(a0));
    y1 = flush_small(red8_dpp(a1));
}

// One chain: q4l_rows2 for the row at rp alone.
template <int G>
__device__ __forceinline__ float q4l_row1(const uint8_t *rp, const float4 (&xr)[4 * G], int l, int base) {
    float a = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const vu2 n = *(const vu2 *)(rp + g * 80 + 8 * l);
        const vu4 sm = *(const vu4 *)(rp + g * 80 + 64);
        a = q4_group(a, n, sm, X4{xr[4 * g], xr[4 * g + 1], xr[4 * g + 2], xr[4 * g + 3]});
    }
    return flush_small(red8_dpp(a));
}

// Modes: MODE_STORE (y[r] = row r; a tile is 8 ROWS rows, lane (r, l) walks
// rows r (and r + 8)) and MODE_SWIGLU (y[p] = swiglu(row p, row p + ffn) with
// the NaN guards of block/forward.rs:97-113; a tile is 8 gate rows and their
// up rows, lane (r, l) walks gate row r and its up row).  No bias, anchors or
// genomic norm (the launcher routes those elsewhere).  G = packed groups per
// row.
template <int MODE, int WAVES, int STAGES, int G, int ROWS, bool TOL = false>
__global__ __launch_bounds__(WAVES * WAVE) void gemv_q4_lds_kernel(GemvParams p, int xstride, int64_t limit, int raw_bytes) {
    static_assert(ROWS == 2 || (ROWS == 1 && MODE == MODE_STORE), "one or two rows per lane");
    static_assert(!TOL || (MODE == MODE_STORE && ROWS == 2), "the regrouped walk: STORE streams");
    constexpr int ROW_BYTES = G * 80;
    constexpr int TROWS = MODE == MODE_SWIGLU ? 4 * ROWS : 8 * ROWS;  // output rows per tile
    constexpr int HALF = (TROWS * ROW_BYTES + 1023) / 1024;           // copies per TROWS rows
    constexpr int PER = MODE == MODE_SWIGLU ? 2 * HALF : HALF;        // copies per stage
    extern __shared__ __align__(16) float smem[];
    __shared__ float inv_slot;
    __shared__ int or_in[WAVES], or_norm[WAVES];
    DevState *st = p.st;
    // the wave index through readfirstlane: the compiler then keeps every
    // tile and stage address in scalar registers
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = lane & 7, r = lane >> 3, base = lane - l;
    const int64_t K4 = p.K >> 2;
    const XView xv{smem, xstride};
    uint8_t *raw = (uint8_t *)(smem + 8 * xstride);  // x, then norm_w, then the exponential table
    uint8_t *stages = raw + raw_bytes + (size_t)wave * STAGES * PER * 1024;
    constexpr int TBI = TROWS * ROW_BYTES;  // bytes of TROWS rows
    const uint32_t v16 = (uint32_t)lane * 16;
    const uint32_t vlast = (HALF - 1) * 1024 + v16 + 16 <= (uint32_t)TBI ? (HALF - 1) * 1024 + v16 : 0u;
    const int64_t rows = MODE == MODE_SWIGLU ? p.ffn : p.N;
    const int64_t ntiles = (rows + TROWS - 1) / TROWS;
    const int64_t gw = (int64_t)blockIdx.x * WAVES + wave, nw = (int64_t)gridDim.x * WAVES;
    // tile t: rows 8 ROWS t.. (store), or gate rows 8t.. then up rows ffn + 8t..
    auto issue = [&](int64_t t, int stage) {
        const uint32_t dst = lds_addr(stages + stage * PER * 1024);
        constexpr int64_t TB = (int64_t)TROWS * ROW_BYTES;
        if constexpr (MODE == MODE_SWIGLU) {
            const int64_t g0 = t * TB, u0 = (t * TROWS + p.ffn) * ROW_BYTES;
            if (u0 + HALF * 1024 <= limit) {
                q4l_copy_full<HALF>(p.w, g0, dst, v16, vlast);
                q4l_copy_full<HALF>(p.w, u0, dst + HALF * 1024, v16, vlast);
            } else {
                q4l_copy<HALF>(p.w, g0, g0 + TB < limit ? g0 + TB : limit, dst, lane);
                q4l_copy<HALF>(p.w, u0, u0 + TB < limit ? u0 + TB : limit, dst + HALF * 1024, lane);
            }
        } else {
            const int64_t o0 = t * TB;
            if (o0 + PER * 1024 <= limit) q4l_copy_full<PER>(p.w, o0, dst, v16, vlast);
            else q4l_copy<PER>(p.w, o0, o0 + TB < limit ? o0 + TB : limit, dst, lane);
        }
    };

    // ---- prologue: wave 0 copies the activations (and the norm weights and
    // the exponential's table), then every wave its first tiles ----
    const int64_t xb = p.K * 4;  // raw layout: x [0, xb), norm_w [xb, 2 xb), exp table after
    const int64_t tb = p.norm_w ? 2 * xb : xb;
    if (wave == 0) {
        lds_copy_bytes(p.x, xb, lds_addr(raw), lane);
        if (p.norm_w) lds_copy_bytes(p.norm_w, xb, lds_addr(raw + xb), lane);
        if (MODE == MODE_SWIGLU) lds_copy_bytes(kExp2Tab, 256, lds_addr(raw + tb), lane);
    }
    int first = 0;  // tiles this wave has in flight
    for (int i = 0; i < STAGES; ++i)
        if (gw + i * nw < ntiles) {
            issue(gw + i * nw, i);
            ++first;
        }
    if (st && s_load_i32(&st->halted)) {
        wait_vmcnt<0>();  // no copy may land after the workgroup's LDS is released
        return;  // uniform
    }
    if (wave == 0) wait_vmcnt_stages<PER, STAGES>(first);  // the shared data has landed
    lds_barrier();
    const float *xraw = (const float *)raw, *wraw = (const float *)(raw + xb);
    const uint64_t *etab = (const uint64_t *)(raw + tb);
    constexpr int NT = WAVES * WAVE;
    int bad_in = 0;
    for (int64_t m = tid; m < K4; m += NT) {
        const float4 v = *(const float4 *)(xraw + 4 * m);
        const float q[4] = {v.x, v.y, v.z, v.w};
        store_quad<true>(xv, (int)m, q);
        bad_in |= isnan(v.x) || isnan(v.y) || isnan(v.z) || isnan(v.w);
    }
    q4_zero_x_pad(xv, p.nb);
    if (barrier_or<WAVES>(bad_in, or_in) && p.st_in >= 0 && tid == 0) nan_flag(st, p.layer, p.st_in);
    if (p.norm_w) {
        rms_inv_chain_major(xv, p.K, p.eps, &inv_slot);
        lds_barrier();
        const float inv = inv_slot;
        int bad = 0;
        for (int64_t m = tid; m < K4; m += NT) {
            const float4 xq = *(const float4 *)(xraw + 4 * m), wq = *(const float4 *)(wraw + 4 * m);
            float t[4] = {xq.x * inv, xq.y * inv, xq.z * inv, xq.w * inv};
            const float w[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                t[c] = t[c] * w[c];  // (x * inv) * w, each product rounded
                bad |= isnan(t[c]);
            }
            store_quad<true>(xv, (int)m, t);
        }
        if (barrier_or<WAVES>(bad, or_norm) && p.st_norm >= 0 && tid == 0) nan_flag(st, p.layer, p.st_norm);
    }

    // ---- tiles: wait for the oldest stage, walk its rows, store them, refill
    // the stage with the tile STAGES ahead.  Issued after this stage's copies
    // are the stores of the last min(it, STAGES - 1) tiles (NST each: rows past
    // the end store into a sink, so the count is fixed) and the copies of the
    // next min(left, STAGES - 1) tiles; the wait lets exactly those remain
    // (a NaN flag's atomic only makes it wait longer). ----
    constexpr int NST = MODE == MODE_SWIGLU ? 2 : ROWS;  // SwiGLU: y and the chain-major copy (or the sink)
    float4 xr4[4 * G];  // chain l's activations, read once
    {
        const float *xg = xv.x + l * xv.stride;
#pragma unroll
        for (int i = 0; i < 4 * G; ++i) xr4[i] = *(const float4 *)(xg + 4 * i);
    }
    // TOL: the chain's block sums of x, then x scaled by 2^24 (low-nibble
    // blocks) or 2^20 (high-nibble blocks) unless some |x| >= 2^100 in the
    // wave's chains (which cover all of x): then this wave walks exactly
    float xsum[TOL ? 4 * G : 1];
    bool exact = !TOL;
    if constexpr (TOL) {
        int big = 0;
#pragma unroll
        for (int i = 0; i < 4 * G; ++i) {
            const float4 v = xr4[i];
            xsum[i] = (v.x + v.y) + (v.z + v.w);
            big |= !(fabsf(v.x) < 0x1p100f) | !(fabsf(v.y) < 0x1p100f) | !(fabsf(v.z) < 0x1p100f) |
                   !(fabsf(v.w) < 0x1p100f);
        }
        exact = __any(big);
        if (!exact) {
#pragma unroll
            for (int i = 0; i < 4 * G; ++i) {
                const float sc = (i & 1) ? 0x1p20f : 0x1p24f;  // block i % 4: low (even) or high (odd) nibbles
                xr4[i] = make_float4(xr4[i].x * sc, xr4[i].y * sc, xr4[i].z * sc, xr4[i].w * sc);
            }
        }
    }
    int stage = 0, it = 0;
    int64_t left = gw < ntiles ? (ntiles - 1 - gw) / nw : 0;  // this wave's tiles after t
    for (int64_t t = gw; t < ntiles; t += nw, --left, ++it) {
        wait_vmcnt_ab<NST, PER, STAGES - 1>(it < STAGES - 1 ? it : STAGES - 1,
                                            (int)(left < STAGES - 1 ? left : STAGES - 1));
        const uint8_t *st0 = stages + stage * PER * 1024;
        float y0, y1 = 0.0f;
        if constexpr (MODE == MODE_SWIGLU) {
            q4l_rows2<G>(st0 + r * ROW_BYTES, st0 + HALF * 1024 + r * ROW_BYTES, xr4, l, base, y0, y1);
        } else if constexpr (ROWS == 2) {
            if (!exact) {
                if constexpr (TOL) q4l_rows2_tol<G>(st0 + r * ROW_BYTES, st0 + (r + 8) * ROW_BYTES, xr4, xsum, l, y0, y1);
            } else {
                q4l_rows2<G>(st0 + r * ROW_BYTES, st0 + (r + 8) * ROW_BYTES, xr4, l, base, y0, y1);
            }
        } else {
            y0 = q4l_row1<G>(st0 + r * ROW_BYTES, xr4, l, base);
        }
        if (lane == base) {
            if constexpr (MODE == MODE_STORE) {
                const int64_t row = t * TROWS + r;
                *(row < rows ? p.y + row : kSinkOut + lane) = y0;
                if constexpr (ROWS == 2) *(row + 8 < rows ? p.y + row + 8 : kSinkOut + lane) = y1;
            } else {
                const int64_t row = t * TROWS + r;
                const bool ok = row < rows;
                if (ok && isnan(y1)) nan_flag(st, p.layer, p.st_a);
                const float o = swiglu1(y0, y1, etab);
                if (ok && isnan(o)) nan_flag(st, p.layer, p.st_b);
                *(ok ? p.y + row : kSinkOut + lane) = o;
                *(ok && p.y_cm ? p.y_cm + (row & 7) * p.cm_stride + (row >> 3) : kSinkOut + lane) = o;
            }
        }
        if (t + STAGES * nw < ntiles) {
            // the stage's LDS reads have returned: it can be refilled
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            issue(t + STAGES * nw, stage);
        }
        stage = stage + 1 == STAGES ? 0 : stage + 1;
    }
    wait_vmcnt<0>();
}

constexpr int Q8L_WAVES = 4, Q8L_STAGES = 2;  // the Q8_0 LDS kernel's shape
// ------------------------------------- Q8_0 rows through LDS-direct copies ----
// The Q8_0 lm_head (and other long Q8_0 STORE matrices) with the staging of
// gemv_q4_lds_kernel: persistent workgroups of WAVES waves, each wave walking
// super-tiles of two consecutive 8-row tiles (16 rows: one contiguous run of
// 2 G Q8_TILE_GROUP bytes), copied into its own LDS stages with LDS-direct
// loads, STAGES ahead.  Lane (r, l) walks chain l of row r of both tiles,
// their steps alternated.  Values, chain order, reduction and epilogue are
// q8_consume's and gemv_q8_stream_kernel's, so each row's result is the same
// bits; rows at or past N (zero in the packed tiles) store into a sink, and
// the first-maximum key of the walked rows goes to the decode state.
// Requires rows_valid == N, no bias, anchors or genomic norm (the launcher
// routes those to the register-ring kernel).  Stores issued after a stage's
// copies that the wait counts leave out (x_out, a NaN flag) only make the
// waits stricter.
template <int G>
__device__ __forceinline__ void q8l_rows2(const uint8_t *ta, const uint8_t *tb, int r, int l,
                                          const float4 (&xr)[4 * G], float &y0, float &y1) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const vu4 na = *(const vu4 *)(ta + g * Q8_CODES + r * 128 + 16 * l);
        const vu4 nbv = *(const vu4 *)(tb + g * Q8_CODES + r * 128 + 16 * l);
        const vu2 sa = *(const vu2 *)(ta + G * Q8_CODES + g * Q8_SCALES + r * 8);
        const vu2 sb = *(const vu2 *)(tb + G * Q8_CODES + g * Q8_SCALES + r * 8);
        float da[4][4], db[4][4];
        q8_dequant(da[0], na.x, half_lo(sa.x));
        q8_dequant(da[1], na.y, half_hi(sa.x));
        q8_dequant(da[2], na.z, half_lo(sa.y));
        q8_dequant(da[3], na.w, half_hi(sa.y));
        q8_dequant(db[0], nbv.x, half_lo(sb.x));
        q8_dequant(db[1], nbv.y, half_hi(sb.x));
        q8_dequant(db[2], nbv.z, half_lo(sb.y));
        q8_dequant(db[3], nbv.w, half_hi(sb.y));
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float4 x = xr[4 * g + b];
            a0 = fmaf(da[b][0], x.x, a0);
            a1 = fmaf(db[b][0], x.x, a1);
            a0 = fmaf(da[b][1], x.y, a0);
            a1 = fmaf(db[b][1], x.y, a1);
            a0 = fmaf(da[b][2], x.z, a0);
            a1 = fmaf(db[b][2], x.z, a1);
            a0 = fmaf(da[b][3], x.w, a0);
            a1 = fmaf(db[b][3], x.w, a1);
        }
    }
    y0 = flush_small(red8_dpp(a0));
    y1 = flush_small(red8_dpp(a1));
}

template <int MODE, int WAVES, int STAGES, int G>
__global__ __launch_bounds__(WAVES * WAVE) void gemv_q8_lds_kernel(GemvParams p, int xstride, int64_t limit) {
    constexpr int TB = G * Q8_TILE_GROUP;  // bytes of one 8-row tile
    constexpr int SB = 2 * TB;             // of a super-tile
    constexpr int PER = (SB + 1023) / 1024;
    constexpr int NST = 2;                 // stores per super-tile (the two rows of lane base)
    extern __shared__ __align__(16) float smem[];
    __shared__ float inv_slot;
    __shared__ int or_in[WAVES], or_norm[WAVES];
    DevState *st = p.st;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = lane & 7, r = lane >> 3, base = lane - l;
    const int64_t K4 = p.K >> 2, N = p.N;
    const XView xv{smem, xstride};
    uint8_t *raw = (uint8_t *)(smem + 8 * xstride);  // x, then norm_w
    const int64_t xb = p.K * 4;
    const int raw_bytes = (int)((p.norm_w ? 2 * xb : xb) + 15) & ~15;
    uint8_t *stages = raw + raw_bytes + (size_t)wave * STAGES * PER * 1024;
    const uint32_t v16 = (uint32_t)lane * 16;
    const uint32_t vlast = (PER - 1) * 1024 + v16 + 16 <= (uint32_t)SB ? (PER - 1) * 1024 + v16 : 0u;
    const int64_t nsup = (N + 15) / 16;  // super-tiles
    const int64_t gw = (int64_t)blockIdx.x * WAVES + wave, nw = (int64_t)gridDim.x * WAVES;
    auto issue = [&](int64_t t, int stage) {
        const uint32_t dst = lds_addr(stages + stage * PER * 1024);
        const int64_t o0 = t * SB;
        if (o0 + PER * 1024 <= limit) q4l_copy_full<PER>(p.w, o0, dst, v16, vlast);
        else q4l_copy<PER>(p.w, o0, o0 + SB < limit ? o0 + SB : limit, dst, lane);
    };

    // ---- prologue (gemv_q4_lds_kernel's): wave 0 copies x and the norm
    // weights, every wave its first super-tiles ----
    if (wave == 0) {
        lds_copy_bytes(p.x, xb, lds_addr(raw), lane);
        if (p.norm_w) lds_copy_bytes(p.norm_w, xb, lds_addr(raw + xb), lane);
    }
    int first = 0;
    for (int i = 0; i < STAGES; ++i)
        if (gw + i * nw < nsup) {
            issue(gw + i * nw, i);
            ++first;
        }
    if (st && s_load_i32(&st->halted)) {
        wait_vmcnt<0>();  // no copy may land after the workgroup's LDS is released
        return;           // uniform
    }
    if (wave == 0) wait_vmcnt_stages<PER, STAGES>(first);  // the shared data has landed
    lds_barrier();
    const float *xraw = (const float *)raw, *wraw = (const float *)(raw + xb);
    constexpr int NT = WAVES * WAVE;
    int bad_in = 0;
    for (int64_t m = tid; m < K4; m += NT) {
        const float4 v = *(const float4 *)(xraw + 4 * m);
        const float q[4] = {v.x, v.y, v.z, v.w};
        store_quad<true>(xv, (int)m, q);
        bad_in |= isnan(v.x) || isnan(v.y) || isnan(v.z) || isnan(v.w);
    }
    q4_zero_x_pad(xv, p.nb);
    if (barrier_or<WAVES>(bad_in, or_in) && p.st_in >= 0 && tid == 0) nan_flag(st, p.layer, p.st_in);
    if (p.norm_w) {
        rms_inv_chain_major(xv, p.K, p.eps, &inv_slot);
        lds_barrier();
        const float inv = inv_slot;
        int bad = 0;
        for (int64_t m = tid; m < K4; m += NT) {
            const float4 xq = *(const float4 *)(xraw + 4 * m), wq = *(const float4 *)(wraw + 4 * m);
            float t[4] = {xq.x * inv, xq.y * inv, xq.z * inv, xq.w * inv};
            const float w[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                t[c] = t[c] * w[c];  // (x * inv) * w, each product rounded
                bad |= isnan(t[c]);
            }
            store_quad<true>(xv, (int)m, t);
        }
        if (barrier_or<WAVES>(bad, or_norm) && p.st_norm >= 0 && tid == 0) nan_flag(st, p.layer, p.st_norm);
    }
    if (p.x_out && blockIdx.x == 0)
        for (int64_t k = tid; k < p.K; k += NT) p.x_out[k] = xv.at(k);

    // ---- super-tiles (as gemv_q4_lds_kernel's tiles) ----
    float4 xr4[4 * G];  // chain l's activations, read once
    {
        const float *xg = xv.x + l * xv.stride;
#pragma unroll
        for (int i = 0; i < 4 * G; ++i) xr4[i] = *(const float4 *)(xg + 4 * i);
    }
    float best_v = -INFINITY;
    int64_t best_i = 0;
    int stage = 0, it = 0;
    int64_t left = gw < nsup ? (nsup - 1 - gw) / nw : 0;
    for (int64_t t = gw; t < nsup; t += nw, --left, ++it) {
        wait_vmcnt_ab<NST, PER, STAGES - 1>(it < STAGES - 1 ? it : STAGES - 1,
                                            (int)(left < STAGES - 1 ? left : STAGES - 1));
        const uint8_t *s0 = stages + stage * PER * 1024;
        float y0, y1;
        q8l_rows2<G>(s0, s0 + TB, r, l, xr4, y0, y1);
        if (lane == base) {
            const int64_t ra = t * 16 + r, rb = ra + 8;
            *(ra < N ? p.y + ra : kSinkOut + lane) = y0;
            *(rb < N ? p.y + rb : kSinkOut + lane) = y1;
            if constexpr (MODE == MODE_ARGMAX) {  // rows in increasing order: strict '>' keeps the first
                const bool b0 = ra < N && y0 > best_v;
                best_v = b0 ? y0 : best_v;
                best_i = b0 ? ra : best_i;
                const bool b1 = rb < N && y1 > best_v;
                best_v = b1 ? y1 : best_v;
                best_i = b1 ? rb : best_i;
            }
        }
        if (t + STAGES * nw < nsup) {
            // the stage's LDS reads have returned: it can be refilled
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            issue(t + STAGES * nw, stage);
        }
        stage = stage + 1 == STAGES ? 0 : stage + 1;
    }
    wait_vmcnt<0>();
    if constexpr (MODE == MODE_ARGMAX) {
        unsigned long long key =
            best_v > -INFINITY
                ? ((unsigned long long)max_key(best_v) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)best_i)
                : 0ull;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(key, o, WAVE);
            key = other > key ? other : key;
        }
        if (lane == 0 && key) atomicMax(&st->argmax_key, key);
    }
}

template <int MODE, int WAVES, int STAGES>
void *q8l_kernel(int G) {
    switch (G) {
        case 1: return (void *)gemv_q8_lds_kernel<MODE, WAVES, STAGES, 1>;
        case 2: return (void *)gemv_q8_lds_kernel<MODE, WAVES, STAGES, 2>;
        case 3: return (void *)gemv_q8_lds_kernel<MODE, WAVES, STAGES, 3>;
        case 4: return (void *)gemv_q8_lds_kernel<MODE, WAVES, STAGES, 4>;
        case 5: return (void *)gemv_q8_lds_kernel<MODE, WAVES, STAGES, 5>;
        case 6: return (void *)gemv_q8_lds_kernel<MODE, WAVES, STAGES, 6>;
        case 7: return (void *)gemv_q8_lds_kernel<MODE, WAVES, STAGES, 7>;
        default: return (void *)gemv_q8_lds_kernel<MODE, WAVES, STAGES, 8>;
    }
}

// LUT-4bit rows stored whole (MODE_STORE, optional bias, no anchors or
// prologue), LDS-staged: one wave per workgroup takes 16 rows (lane 4 r + c:
// row r, chain c) and copies, all at once with LDS-direct loads, x, the 16
// rows' codes (16 B per block, contiguous) and their 16-entry tables (one per
// row and block, or the one shared table); then each lane walks its chain
// (elements e of a block with e % 4 == c, blocks in order: genomic.rs:148-204)
// with its table lookups and x reads from LDS.  Against row_lut4, which waits
// for each block's table before its lookups, every byte of the tile is in
// flight from the start.
constexpr int LUTL_ROWS = 16;
// Tables in LDS: row q's nb tables at q nb 64 bytes, as the tile lies in
// memory (one copy per KiB).  For even nb every row's tables then begin on the
// same LDS bank, so a block's lookups from the 16 rows conflict; padding the
// rows apart (one copy per row and KiB) measured slower (9.2 against 7.3 us
// per C0-LUT launch).
__host__ __device__ constexpr int64_t lut4_trow_bytes(int64_t nb) { return nb * 64; }
size_t lut4_lds_bytes(int64_t K, int64_t nb, bool shared_table) {
    const size_t xb = (size_t)K * 4, cb = (size_t)LUTL_ROWS * nb * 16;
    const size_t tb = shared_table ? 64 : (size_t)LUTL_ROWS * lut4_trow_bytes(nb);
    return (xb + 1023) / 1024 * 1024 + (cb + 1023) / 1024 * 1024 + (tb + 1023) / 1024 * 1024;
}

template <bool SHARED>
__global__ __launch_bounds__(WAVE) void gemv_lut4_lds_kernel(GemvParams p) {
    extern __shared__ __align__(16) float smem[];
    const int lane = threadIdx.x, r = lane >> 2, c = lane & 3, base = lane & ~3;
    const int nb = p.nb;
    const int64_t K = p.K;
    const int64_t r0 = (int64_t)blockIdx.x * LUTL_ROWS;
    float *xs = smem;
    const int64_t xb = K * 4, cb = (int64_t)LUTL_ROWS * nb * 16;
    const int64_t trs = lut4_trow_bytes(nb);
    uint8_t *codes = (uint8_t *)smem + (xb + 1023) / 1024 * 1024;
    float *tabs = (float *)(codes + (cb + 1023) / 1024 * 1024);
    // ---- every copy at once: x, the codes, the tables ----
    lds_copy_bytes(p.x, xb, lds_addr(xs), lane);
    {
        // codes of rows r0 .. r0 + 15 (contiguous); lanes past the tensor re-read its start
        const uint8_t *cw = p.w + r0 * nb * 16;
        const int64_t cend = (p.N - r0) * nb * 16;
        for (int64_t o = 0; o < cb; o += 1024) {
            const int64_t a = o + lane * 16;
            lds_dma16(cw + (a + 16 <= cend ? a : 0), lds_addr(codes) + (uint32_t)o);
        }
    }
    if constexpr (SHARED) {
        if (lane < 4) lds_dma16<true>(p.lut + 4 * lane, lds_addr(tabs));
    } else {
        // row q's table set (nb 64 bytes) starts at q nb 64 bytes if q < lut_rows_own,
        // else at 0; rows past the tensor copy row r0's
        const uint32_t rs = (uint32_t)nb * 64;
        const uint8_t *lb = (const uint8_t *)p.lut;
        const int64_t tb = (int64_t)LUTL_ROWS * rs;
        if (r0 + LUTL_ROWS <= p.lut_rows_own && r0 + LUTL_ROWS <= p.N) {
            for (int64_t o = 0; o < tb; o += 1024) lds_dma16(lb + r0 * rs + o + lane * 16, lds_addr(tabs) + (uint32_t)o);
        } else {
            for (int64_t o = 0; o < tb; o += 1024) {
                const uint32_t a = (uint32_t)o + lane * 16;
                int64_t q = r0 + a / rs;
                q = q < p.N ? q : r0;
                const int64_t src = (q < p.lut_rows_own ? q * rs : 0) + a % rs;
                lds_dma16(lb + src, lds_addr(tabs) + (uint32_t)o);
            }
        }
    }
    if (p.st && s_load_i32(&p.st->halted)) {
        wait_vmcnt<0>();
        return;
    }
    wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    // ---- the chain: acc = acc + tbl[code] * x[e], mul then add, blocks in order ----
    float acc = 0.0f;
    const uint8_t *crow = codes + (size_t)r * nb * 16;
    const float *trow = SHARED ? tabs : (const float *)((const uint8_t *)tabs + r * trs);
    for (int j = 0; j < nb; ++j) {
        const vu4 cw = *(const vu4 *)(crow + (size_t)j * 16);
        const float *t = SHARED ? trow : trow + (size_t)j * 16;
        const float *xj = xs + (size_t)j * 32 + c;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            // element e = 4 u + c; even e is the high nibble of byte e / 2
            const uint32_t word = (u >> 1) == 0 ? cw.x : (u >> 1) == 1 ? cw.y : (u >> 1) == 2 ? cw.z : cw.w;
            // byte e / 2 = 2 u + c / 2 of the block: bits 8 ((2u + c/2) & 3) of word u / 2
            const uint32_t idx = __builtin_amdgcn_ubfe(word, 8 * ((2 * u + (c >> 1)) & 3) + ((c & 1) ? 0 : 4), 4);
            const float prod = t[idx] * xj[4 * u];
            acc = acc + prod;
        }
    }
    const float s1 = shfl(acc, base + 1), s2 = shfl(acc, base + 2), s3 = shfl(acc, base + 3);
    float total = flush_small(((acc + s1) + s2) + s3);  // s0 + s1 + s2 + s3, left to right
    const int64_t row = r0 + r;
    if (c == 0 && row < p.N) {
        if (row < p.bias_len) total = total + p.bias[row];
        p.y[row] = total;
    }
}

template <int MODE, int WAVES, int STAGES, int ROWS, bool TOL = false>
void *q4l_kernel(int G) {
    switch (G) {
        case 1: return (void *)gemv_q4_lds_kernel<MODE, WAVES, STAGES, 1, ROWS, TOL>;
        case 2: return (void *)gemv_q4_lds_kernel<MODE, WAVES, STAGES, 2, ROWS, TOL>;
        case 3: return (void *)gemv_q4_lds_kernel<MODE, WAVES, STAGES, 3, ROWS, TOL>;
        case 4: return (void *)gemv_q4_lds_kernel<MODE, WAVES, STAGES, 4, ROWS, TOL>;
        case 5: return (void *)gemv_q4_lds_kernel<MODE, WAVES, STAGES, 5, ROWS, TOL>;
        case 6: return (void *)gemv_q4_lds_kernel<MODE, WAVES, STAGES, 6, ROWS, TOL>;
        case 7: return (void *)gemv_q4_lds_kernel<MODE, WAVES, STAGES, 7, ROWS, TOL>;
        default: return (void *)gemv_q4_lds_kernel<MODE, WAVES, STAGES, 8, ROWS, TOL>;
    }
}

// LDS stage bytes of the LDS-staged Q4_0 kernel for rows of G groups.
int q4l_stage_bytes(int mode, int G, int rows) {
    const int trows = mode == MODE_SWIGLU ? 4 * rows : 8 * rows;
    const int half = (trows * G * 80 + 1023) / 1024;
    return 1024 * (mode == MODE_SWIGLU ? 2 * half : half);
}

// ------------------------------------------------- Q4_0, split waves ----
// A matvec with too few rows to fill the chip is bound by the length of one
// lane's instruction stream, and per element that stream is a byte-to-float
// conversion, the dequantising fma and the chain's fma.  Here a workgroup
// takes 4 row pairs (8 rows) and splits the work: wave 0 walks their 64
// chains (lanes 16i..16i+7: pair i's first row, 16i+8..16i+15 its second;
// chain = lane % 8), reading the dequantised values from LDS, while waves 1..3
// load and dequantise the weights one stage (SPLIT_SQ packed groups) ahead
// into a double-buffered LDS ring, one barrier per stage.  Wave 0 also runs
// the prologue (the activations, their RMSNorm) and the epilogue.  The values
// and the chain order are those of q4_consume, so the result is the same bit
// for bit.
constexpr int SPLIT_PAIRS = 4;                    // row pairs per workgroup
constexpr int64_t SPLIT_MAX_ROWS = 4096;          // beyond this the row-per-lane kernel fills the chip
constexpr int SPLIT_PQ = 2;                       // groups per producer wave and stage
constexpr int SPLIT_SQ = 3 * SPLIT_PQ;            // groups per stage
constexpr int SPLIT_DSTRIDE = 16 * SPLIT_SQ + 4;  // ring floats per chain lane (stride / 4 odd: no bank conflicts)
constexpr int64_t SPLIT_NORM_MAX_K4 = 8 * 64;     // RMSNorm from wave 0's registers: one batch of 8 float4 per lane

// Floats of a chain-major activation row in the split kernel: every group's 16
// inputs and, for the RMSNorm's sum-of-squares chain, the rounding to 64 plus
// its read-ahead of 32, all zero past the 4 nb values; a multiple of 8 (the
// row stride, 4 more, is then an odd number of float4s).
__host__ __device__ constexpr int split_xrow(int nb) {
    const int g16 = 16 * ((nb + 3) / 4), sq = (4 * nb + 63) / 64 * 64 + 32;
    const int m = g16 > sq ? g16 : sq;
    return (m + 7) / 8 * 8;
}

__device__ __forceinline__ float q4_chain4(float acc, const float4 d, const float4 x) {
    acc = fmaf(d.x, x.x, acc);
    acc = fmaf(d.y, x.y, acc);
    acc = fmaf(d.z, x.z, acc);
    acc = fmaf(d.w, x.w, acc);
    return acc;
}

template <int MODE, bool NORM>
__global__ __launch_bounds__(THREADS) void gemv_q4_split_kernel(GemvParams p, int64_t npairs, int xstride) {
    extern __shared__ __align__(16) float smem[];
    DevState *st = p.st;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K = p.K, K4 = K >> 2;
    const int nb = p.nb, G = (nb + 3) >> 2, nstage = (G + SPLIT_SQ - 1) / SPLIT_SQ;
    const XView xv{smem, xstride};
    float *ring = smem + 8 * xstride;  // [2][64 chain lanes][SPLIT_DSTRIDE]
    const int l = lane & 7;
    const int64_t pr = (int64_t)blockIdx.x * SPLIT_PAIRS + (lane >> 4);
    PairRows q;  // (locate, with the pairing of this kernel's mode only)
    q.pair_ok = pr < npairs;
    q.r0 = 0;
    q.r1 = -1;
    if (q.pair_ok) {
        if constexpr (MODE == MODE_QKV) {
            pair_rows(p, MODE_QKV, pr, q.r0, q.r1);
        } else {
            q.r0 = 2 * pr;
            q.r1 = 2 * pr + 1 < p.N ? 2 * pr + 1 : -1;
        }
    }
    q.row = ((lane >> 3) & 1) ? q.r1 : q.r0;
    q.row_ok = q.pair_ok && q.row >= 0 && q.row < p.rows_valid;
    const int halted = st ? st->halted : 0;

    if (wave > 0) {
        // ---- producers: wave 1 + pw dequantises groups pw*PQ .. pw*PQ + PQ-1
        // of every stage for the 64 chain lanes; loads run two stages ahead.
        // Stages are produced in pairs with no branch around the loads (past
        // the row they re-read its last group), so each wait is for the stage
        // being dequantised alone; an odd stage count ends with one unused
        // stage, matched by one extra barrier in wave 0 ----
        const int pw = wave - 1;
        const uint8_t *wrow = (p.rows_valid > 0 ? p.w : kZeroRows) + (size_t)(q.row_ok ? q.row : 0) * G * 80;
        vu2 an[SPLIT_PQ], bn[SPLIT_PQ];
        vu4 as[SPLIT_PQ], bs[SPLIT_PQ];
        auto load = [&](int stg, vu2(&n)[SPLIT_PQ], vu4(&sw)[SPLIT_PQ]) {
#pragma unroll
            for (int j = 0; j < SPLIT_PQ; ++j) {
                int g = stg * SPLIT_SQ + pw * SPLIT_PQ + j;
                g = g < G ? g : G - 1;  // groups past the row are never read by the chain
                n[j] = ld_u2<false>(wrow + (size_t)g * 80 + 8 * l);
                sw[j] = ld_u4<false>(wrow + (size_t)g * 80 + 64);
            }
        };
        auto produce = [&](int buf, const vu2(&n)[SPLIT_PQ], const vu4(&sw)[SPLIT_PQ]) {
            float *dst = ring + (buf * 64 + lane) * SPLIT_DSTRIDE + 16 * pw * SPLIT_PQ;
#pragma unroll
            for (int j = 0; j < SPLIT_PQ; ++j) {
                float d[4][4];
                q4_dequant(d[0], opaque_and(n[j].x, 0x0F0F0F0Fu), sw[j].x);
                q4_dequant(d[1], opaque_and(n[j].x >> 4, 0x0F0F0F0Fu), sw[j].y);
                q4_dequant(d[2], opaque_and(n[j].y, 0x0F0F0F0Fu), sw[j].z);
                q4_dequant(d[3], opaque_and(n[j].y >> 4, 0x0F0F0F0Fu), sw[j].w);
#pragma unroll
                for (int b = 0; b < 4; ++b) *(float4 *)(dst + 16 * j + 4 * b) = make_float4(d[b][0], d[b][1], d[b][2], d[b][3]);
            }
        };
        load(0, an, as);
        load(1, bn, bs);
        if (halted) return;  // uniform
        for (int s = 0; s < nstage; s += 2) {
            produce(0, an, as);
            load(s + 2, an, as);
            lds_barrier();
            produce(1, bn, bs);
            load(s + 3, bn, bs);
            lds_barrier();
        }
        return;  // wave 0 passes no further barrier
    }

    // ---- wave 0 ----
    if (halted) return;
    // activations -> chain-major LDS (batches of 8 float4 per lane); with a
    // norm the vector is one batch and stays in registers for the normalising
    const bool leader = q.pair_ok && (lane & 15) == 0;
    float b0 = 0.0f, b1 = 0.0f, old0 = 0.0f, old1 = 0.0f, cs = 0.0f, sn = 0.0f;
    int pos = 0;
    const float4 *x4 = (const float4 *)p.x;
    const float4 *w4 = (const float4 *)p.norm_w;  // non-null exactly when NORM
    int bad_in = 0;
    float4 v[8], w[NORM ? 8 : 1];
    for (int64_t m0 = 0; m0 < K4; m0 += 8 * 64) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t m = m0 + u * 64 + lane;
            v[u] = x4[m < K4 ? m : K4 - 1];
        }
        if constexpr (NORM) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t m = m0 + u * 64 + lane;
                w[u] = w4[m < K4 ? m : K4 - 1];
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t m = m0 + u * 64 + lane;
            if (m < K4) {
                const float qd[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
                store_quad<true>(xv, (int)m, qd);
                bad_in |= isnan(v[u].x) | isnan(v[u].y) | isnan(v[u].z) | isnan(v[u].w);
            }
        }
    }
    // the epilogue operands, loaded while the chains run (once the
    // activations are in: a load issued before them would hold up their use)
    if (leader) {
        if (q.r0 < p.bias_len) b0 = p.bias[q.r0];
        if (q.r1 >= 0 && q.r1 < p.bias_len) b1 = p.bias[q.r1];
        if constexpr (MODE == MODE_RESIDUAL) {
            old0 = p.y[q.r0];
            if (q.r1 >= 0) old1 = p.y[q.r1];
        } else if constexpr (MODE == MODE_QKV) {
            pos = st->pos;
            const int hh = p.head_dim >> 1;
            const int i = (int)(pr % hh);
            cs = p.rope_cos[(size_t)pos * hh + i];
            sn = p.rope_sin[(size_t)pos * hh + i];
        }
    }
    {  // zero past the 4 nb values of each chain row: the partial last group's
       // inputs and, with a norm, the sum-of-squares chain's range (split_xrow)
        const int from = 4 * nb, to = NORM ? xstride - 4 : 16 * G;  // from and to are multiples of 4
        for (int c = from + 4 * (lane & 7); c < to; c += 32)
            *(float4 *)(xv.x + (lane >> 3) * xstride + c) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (__any(bad_in) && p.st_in >= 0 && lane == 0) nan_flag(st, p.layer, p.st_in);
    if constexpr (NORM) {
        // rms_norm (norm.rs:52-88): the eight chains of the chain-major rows,
        // then (x * inv) * w from the registers, each product rounded
        float ss = 0.0f;
        if (lane < 8) ss = chain_lds_sq(0.0f, xv.x + lane * xstride, (4 * nb + 63) & ~63);
        const float u1 = ss + __shfl(ss, (lane + 4) & 7, 8);
        const float u2 = u1 + __shfl(u1, (lane + 1) & 7, 8);
        const float tot = u2 + __shfl(u2, (lane + 2) & 7, 8);
        const float inv = __shfl(1.0f / sqrtf(tot / (float)K + p.eps), 0, WAVE);
        int bad = 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t m = u * 64 + lane;
            if (m < K4) {
                float t[4] = {v[u].x * inv, v[u].y * inv, v[u].z * inv, v[u].w * inv};
                const float wn[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    t[c] = t[c] * wn[c];
                    bad |= isnan(t[c]);
                }
                store_quad<true>(xv, (int)m, t);
            }
        }
        if (__any(bad) && p.st_norm >= 0 && lane == 0) nan_flag(st, p.layer, p.st_norm);
    }
    // the 64 chains, one stage per barrier
    float acc = 0.0f;
    const float *xg = xv.x + l * xstride;
    const int nbar = (nstage + 1) & ~1;  // the producers' barriers (stages in pairs)
    for (int s = 0; s < nbar; ++s) {
        lds_barrier();
        if (s >= nstage) break;  // (the producers' unused last stage)
        const float *dl = ring + ((s & 1) * 64 + lane) * SPLIT_DSTRIDE;
#pragma unroll
        for (int j = 0; j < SPLIT_SQ; ++j) {
            const int g = s * SPLIT_SQ + j;
            if (g < G) {
                const X4 x = read_x4(xg + 16 * g);
                const X4 d = read_x4(dl + 16 * j);
                acc = q4_chain4(acc, d.b0, x.b0);
                acc = q4_chain4(acc, d.b1, x.b1);
                acc = q4_chain4(acc, d.b2, x.b2);
                acc = q4_chain4(acc, d.b3, x.b3);
            }
        }
    }
    // lanes 8r..8r+7 hold a row's chains 0..7: the reduction of q4_consume
    const float total = q.row_ok ? flush_small(red8_dpp(acc)) : 0.0f;  // valid in lane 8r
    const float v1 = dpp_shl8(total);  // the pair's second row
    if (!leader) return;
    const int64_t r0 = q.r0, r1 = q.r1;
    const float y0 = finish_row(p, xv, r0, total, b0);
    const float y1 = r1 >= 0 ? finish_row(p, xv, r1, v1, b1) : 0.0f;
    if constexpr (MODE == MODE_STORE) {
        p.y[r0] = y0;
        if (r1 >= 0) p.y[r1] = y1;
    } else if constexpr (MODE == MODE_RESIDUAL) {
        if (isnan(y0) || (r1 >= 0 && isnan(y1))) nan_flag(st, p.layer, p.st_a);
        const float h0 = old0 + y0;
        p.y[r0] = h0;
        bool bad = isnan(h0);
        if (r1 >= 0) {
            const float h1 = old1 + y1;
            p.y[r1] = h1;
            bad |= isnan(h1);
        }
        if (bad) nan_flag(st, p.layer, p.st_b);
    } else {
        qkv_store(p, r0, r1, y0, y1, cs, sn, pos);
    }
}

// ----------------------------------- Q4_0, one chain wave fed from LDS ----
// The split kernel's division of labour on a narrower tile, for matvecs of up
// to a few thousand rows.  Wave 0 of a workgroup walks the 32 chains of 4 rows
// (2 row pairs; lane 8ρ + l is chain l of row ρ, lanes 32..63 idle in the
// walk) and does nothing per weight but its fma: the dequantised values come
// from an LDS ring that waves 1..3 fill one stage (CH_SQ packed groups) ahead,
// one producer lane per (chain, group) of the stage.  Measured on the 896-row
// matvecs of a 0.5B decode, an 8-row walk is bound by the LDS port (the eight
// rows of a chain read the same activations, and each read costs its full
// width), at about 13 cycles per step against the 4.6 of one wave's fma issue;
// with 4 rows the bytes per step fit under the fma rate.
//
// Everything the workgroup reads is copied into LDS when it starts, with
// global_load_lds_dwordx4 (inline assembly, waited with explicit vmcnt counts):
// each producer copies its 4 rows x 2 groups (640 bytes, one instruction) of
// every stage before dequantising the first, and wave 0 copies the activations
// (and the norm weights).  The chains read the activations in their natural
// layout (element 128g + 32b + 8c + l for chain l's value c of block b of
// group g: ds_read2 pairs), so nothing is rearranged before the first step.
// The values, the chain order, the reduction and the epilogues are the split
// kernel's, so the result is the same bit for bit.
constexpr int CH_PAIRS = 2;                     // row pairs per workgroup
constexpr int CH_LANES = 16 * CH_PAIRS;         // chain lanes (4 rows x 8 chains)
constexpr int CH_SQ = 3 * WAVE / CH_LANES;      // groups per stage: one per producer lane
constexpr int CH_DSTRIDE = 16 * CH_SQ + 4;      // ring floats per chain lane (stride / 4 odd)
constexpr int CH_UNIT = 2 * CH_PAIRS * 2 * 80;  // bytes one producer copies per stage
constexpr int CH_MAX_STAGES = 60;               // one copy per stage within the six-bit vmcnt
constexpr int CH_AHEAD = 2;                     // groups of ring reads in flight ahead of the fmas
constexpr int CH_XREG_MAX = 8;                  // rows of up to this many groups keep x in registers
static_assert(CH_SQ == 6 && CH_UNIT <= 1024, "one copy instruction per producer and stage");

// The rows of chain lane cl (0..CH_LANES-1) of this workgroup.
template <int MODE>
__device__ __forceinline__ PairRows chain_rows(const GemvParams &p, int64_t npairs, int cl) {
    PairRows q;
    const int64_t pr = (int64_t)blockIdx.x * CH_PAIRS + (cl >> 4);
    q.pair_ok = pr < npairs;
    q.r0 = 0;
    q.r1 = -1;
    if (q.pair_ok) {
        if constexpr (MODE == MODE_QKV) {
            pair_rows(p, MODE_QKV, pr, q.r0, q.r1);
        } else {
            q.r0 = 2 * pr;
            q.r1 = 2 * pr + 1 < p.N ? 2 * pr + 1 : -1;
        }
    }
    q.row = ((cl >> 3) & 1) ? q.r1 : q.r0;
    q.row_ok = q.pair_ok && q.row >= 0 && q.row < p.rows_valid;
    return q;
}

// Chain-major row stride (floats) of gemv_q4_chain_kernel: 16 per packed
// group, plus 4 so that stride / 4 is odd (the eight rows' 16-byte reads fall
// in distinct banks).
__host__ __device__ constexpr int chain_xstride(int64_t K) { return (int)(16 * ((K / 32 + 3) / 4) + 4); }

// LDS bytes of gemv_q4_chain_kernel: the ring, the activations as copied (zero
// to the last group's end), with a norm its weights, the chain-major copy and
// the stages' copies.
__host__ __device__ constexpr int64_t chain_lds_bytes(int64_t K, bool norm) {
    const int64_t G = (K / 32 + 3) / 4, xf = 128 * G, nstage = (G + CH_SQ - 1) / CH_SQ;
    return (2 * CH_LANES * CH_DSTRIDE + xf + (norm ? K : 0) + 8 * (int64_t)chain_xstride(K)) * 4 +
           nstage * 3 * CH_UNIT + 4 * 320 * 4;
}

template <int MODE, bool NORM, int GX>
__global__ __launch_bounds__(THREADS) void gemv_q4_chain_kernel(GemvParams p, int64_t npairs, int xstride) {
    extern __shared__ __align__(16) float smem[];
    DevState *st = p.st;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K = p.K, K4 = K >> 2;
    const int nb = p.nb, G = GX > 0 ? GX : (nb + 3) >> 2, nstage = (G + CH_SQ - 1) / CH_SQ;  // (G == GX: launcher)
    const int64_t XF = 128 * (int64_t)G;
    float *ring = smem;                              // [2][CH_LANES][CH_DSTRIDE]
    float *xs = ring + 2 * CH_LANES * CH_DSTRIDE;    // activations as copied, zero from K to XF
    float *wn = xs + XF;                             // NORM: the norm weights (K)
    float *xcm = wn + (NORM ? K : 0);                // the chain-major copy: 8 rows of xstride
    uint8_t *tile = (uint8_t *)(xcm + 8 * xstride);  // [stage][producer][CH_UNIT]
    uint32_t *khist = (uint32_t *)(tile + (size_t)nstage * 3 * CH_UNIT);  // the fused K-WTA's histogram

    if (wave > 0) {
        // ---- producers: copy every stage's bytes, then dequantise stage by
        // stage as the copies land.  Copy lane i (i < 40) moves bytes 16i..16i+15
        // of the unit: (row ρ, group j) at 160 ρ + 80 j ----
        const int pw = wave - 1;
        const uint8_t *src;
        int jj;
        {
            const int b = lane * 16 < CH_UNIT ? lane * 16 : 0, u = b / 80;
            jj = u & 1;
            const PairRows q = chain_rows<MODE>(p, npairs, 8 * (u >> 1));
            src = (p.rows_valid > 0 ? p.w : kZeroRows) + (size_t)(q.row_ok ? q.row : 0) * G * 80 + b % 80;
        }
        for (int sg = 0; sg < nstage; ++sg) {
            int g = sg * CH_SQ + 2 * pw + jj;
            g = g < G ? g : G - 1;  // past the row: its last group again, never read by a chain
            if (lane < CH_UNIT / 16)
                lds_dma16(src + (size_t)g * 80, lds_addr(tile + (size_t)(sg * 3 + pw) * CH_UNIT));
        }
        if (st && s_load_i32(&st->halted)) {
            wait_vmcnt<0>();  // no copy may land after the workgroup's LDS is released
            return;           // uniform
        }
        const int cl = lane & (CH_LANES - 1), l = cl & 7, jl = lane >> 5;
        for (int sg = 0; sg < nstage; ++sg) {
            wait_vmcnt_stages<1, CH_MAX_STAGES>(nstage - 1 - sg);
            const uint8_t *u = tile + (size_t)(sg * 3 + pw) * CH_UNIT + (cl >> 3) * 160 + jl * 80;
            const vu2 n = *(const vu2 *)(u + 8 * l);
            const vu4 sw = *(const vu4 *)(u + 64);
            float d[4][4];
            q4_dequant_dw<0>(d[0], n.x, sw.x);
            q4_dequant_dw<1>(d[1], n.x, sw.y);
            q4_dequant_dw<0>(d[2], n.y, sw.z);
            q4_dequant_dw<1>(d[3], n.y, sw.w);
            float *dst = ring + ((sg & 1) * CH_LANES + cl) * CH_DSTRIDE + 16 * (2 * pw + jl);
#pragma unroll
            for (int b = 0; b < 4; ++b) *(float4 *)(dst + 4 * b) = make_float4(d[b][0], d[b][1], d[b][2], d[b][3]);
            lds_barrier();
        }
        // the activations landed before wave 0's first barrier: NaN inputs are
        // flagged here, off the chains' path (longer rows: from the chain-major
        // copy, quad m = row m % 8, c = 4 (m / 8))
        int bad = 0;
        for (int64_t m = (int64_t)(wave - 1) * WAVE + lane; m < K4; m += 3 * WAVE) {
            const float4 v = GX > 0 ? *(const float4 *)(xs + 4 * m)
                                    : *(const float4 *)(xcm + (m & 7) * xstride + 4 * (m >> 3));
            bad |= isnan(v.x) | isnan(v.y) | isnan(v.z) | isnan(v.w);
        }
        if (__any(bad) && p.st_in >= 0 && lane == 0) nan_flag(st, p.layer, p.st_in);
        return;  // wave 0 passes no further barrier
    }

    // ---- wave 0: the activations (and the norm weights), then the
    // epilogue operands (they land with them) ----
    const PairRows q = chain_rows<MODE>(p, npairs, lane & (CH_LANES - 1));
    const bool leader = lane < CH_LANES && q.pair_ok && (lane & 15) == 0;
    float b0 = 0.0f, b1 = 0.0f, old0 = 0.0f, old1 = 0.0f, cs = 0.0f, sn = 0.0f, kthr = -INFINITY;
    int pos = 0;
    // longer rows whose producer also wrote the chain-major copy (x_cm, the
    // launcher checks its stride): that copy is this kernel's xcm as it stands
    const bool have_cm = GX == 0 && !NORM && p.x_cm != nullptr;
    if (have_cm) {
        lds_copy_bytes(p.x_cm, (int64_t)8 * xstride * 4, lds_addr(xcm), lane);
    } else {
        for (int64_t m = K4 + lane; m < XF / 4; m += WAVE) *(float4 *)(xs + 4 * m) = make_float4(0.f, 0.f, 0.f, 0.f);
        lds_copy_bytes(p.x, K * 4, lds_addr(xs), lane);
        if constexpr (NORM) lds_copy_bytes(p.norm_w, K * 4, lds_addr(wn), lane);
    }
    if (leader) {  // (after the copies: their addresses need no kernel argument)
        if (q.r0 < p.bias_len) b0 = p.bias[q.r0];
        if (q.r1 >= 0 && q.r1 < p.bias_len) b1 = p.bias[q.r1];
        if constexpr (MODE == MODE_RESIDUAL) {
            old0 = p.y[q.r0];
            if (q.r1 >= 0) old1 = p.y[q.r1];
            if (p.kwta_k > 0) kthr = *p.kwta_thr;
        } else if constexpr (MODE == MODE_QKV) {
            pos = st->pos;
            const int hh = p.head_dim >> 1;
            const int i = (int)(((int64_t)blockIdx.x * CH_PAIRS + (lane >> 4)) % hh);
            cs = p.rope_cos[(size_t)pos * hh + i];
            sn = p.rope_sin[(size_t)pos * hh + i];
        }
    }
    if (st && s_load_i32(&st->halted)) {
        wait_vmcnt<0>();
        return;
    }
    wait_vmcnt<0>();  // this wave's copies have landed (it alone reads them before the barriers)
    if constexpr (MODE == MODE_QKV) {
        // the previous block's K-WTA on this workgroup's copy of x (every
        // workgroup finds the same threshold; workgroup 0 keeps it for the
        // residual of the attention output)
        if (p.kwta_k > 0) {
            const float thr = wave_kwta(xs, (int)K, p.kwta_k, khist, lane);
            if (blockIdx.x == 0 && lane == 0) *p.kwta_thr = thr;
        }
    }
    const int l = lane & 7;
    float4 xq[GX > 0 ? 4 * GX : 1];  // GX > 0: chain l's values c = 4i..4i+3 at xq[i]
    const float *xr = xcm + l * xstride;  // GX == 0: chain l's row of the chain-major copy
    if constexpr (GX > 0) {
        // rows of at most 8 groups: each chain lane reads its 16 GX values
        // straight from the copy (element 8c + l, zero from K), no chain-major
        // copy.  With a norm: rms_norm (norm.rs:52-88), eight fma chains over
        // elements 8c + l (lanes 0..7, from registers; fma(0, 0, acc) leaves a
        // chain as it is past K / 8), ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)),
        // then (x * inv) * w for every element, each product rounded, into
        // the normalised copy (xcm's space, natural layout), which the lanes
        // then read as above
        const float *src = xs;
        if constexpr (NORM) {
            float ss = 0.0f;
            if (lane < 8) {
                // reads two 16-value chunks ahead of the fmas (pinned)
                constexpr int NC = GX;  // chunks of 16 values
                float v[3][16];
                auto load = [&](int k, float (&d)[16]) {
#pragma unroll
                    for (int c = 0; c < 16; ++c) d[c] = xs[8 * (16 * k + c) + lane];
                };
                load(0, v[0]);
                if (NC > 1) load(1, v[1]);
#pragma unroll
                for (int k = 0; k < NC; ++k) {
                    if (k + 2 < NC) load(k + 2, v[(k + 2) % 3]);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int c = 0; c < 16; ++c) ss = fmaf(v[k % 3][c], v[k % 3][c], ss);
                }
            }
            const float tot = rms_tot8(ss);
            const float inv = 1.0f / sqrtf(tot / (float)K + p.eps);
            constexpr int NQ = (32 * GX + WAVE - 1) / WAVE;  // quads of XF per lane
            float4 a[NQ], w[NQ];
#pragma unroll
            for (int u = 0; u < NQ; ++u) {
                const int m = u * WAVE + lane < 32 * GX ? u * WAVE + lane : 0;
                a[u] = *(const float4 *)(xs + 4 * m);
                w[u] = *(const float4 *)(wn + 4 * (m < K4 ? m : 0));
            }
            int bad = 0;
#pragma unroll
            for (int u = 0; u < NQ; ++u) {
                const int m = u * WAVE + lane;
                if (m < 32 * GX) {
                    const float4 o = make_float4((a[u].x * inv) * w[u].x, (a[u].y * inv) * w[u].y,
                                                 (a[u].z * inv) * w[u].z, (a[u].w * inv) * w[u].w);
                    if (m < K4) bad |= isnan(o.x) | isnan(o.y) | isnan(o.z) | isnan(o.w);
                    *(float4 *)(xcm + 4 * m) = m < K4 ? o : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
            if (__any(bad) && p.st_norm >= 0 && lane == 0) nan_flag(st, p.layer, p.st_norm);
            src = xcm;
        }
        if (lane < CH_LANES) {
#pragma unroll
            for (int i = 0; i < 4 * GX; ++i)
                xq[i] = make_float4(src[32 * i + l], src[32 * i + 8 + l], src[32 * i + 16 + l], src[32 * i + 24 + l]);
        }
    } else {
        // longer rows: the chain-major copy, row l holding elements 8c + l at c
        // (zero from K / 8): 32 elements (8 quads) per lane and round, chain l
        // of elements 32q.. being (x[32q + l], x[32q + 8 + l], x[32q + 16 + l],
        // x[32q + 24 + l]) at c = 4q of row l
        for (int64_t qd = have_cm ? XF / 32 : lane; qd < XF / 32; qd += WAVE) {
            float4 f[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) f[k] = *(const float4 *)(xs + 32 * qd + 4 * k);
#pragma unroll
            for (int ll = 0; ll < 8; ++ll) {
                const int h = ll >> 2;
                auto pick = [&](const float4 &v) { return (ll & 3) == 0 ? v.x : (ll & 3) == 1 ? v.y : (ll & 3) == 2 ? v.z : v.w; };
                *(float4 *)(xcm + ll * xstride + 4 * qd) = make_float4(pick(f[h]), pick(f[2 + h]), pick(f[4 + h]), pick(f[6 + h]));
            }
        }
        if constexpr (NORM) {
            // rms_norm as above, over the chain-major rows, in place
            float ss = 0.0f;
            if (lane < 8) {
                const float4 *r4 = (const float4 *)(xcm + lane * xstride);
#pragma unroll 8
                for (int64_t c = 0; c < XF / 32; ++c) {
                    const float4 v = r4[c];
                    ss = fmaf(v.x, v.x, ss);
                    ss = fmaf(v.y, v.y, ss);
                    ss = fmaf(v.z, v.z, ss);
                    ss = fmaf(v.w, v.w, ss);
                }
            }
            const float u1 = ss + __shfl(ss, (lane + 4) & 7, 8);
            const float u2 = u1 + __shfl(u1, (lane + 1) & 7, 8);
            const float tot = u2 + __shfl(u2, (lane + 2) & 7, 8);
            const float inv = __shfl(1.0f / sqrtf(tot / (float)K + p.eps), 0, WAVE);
            int bad = 0;
            for (int64_t m = lane; m < K4; m += WAVE) {  // quad m: row m % 8, c = 4 (m / 8) < K / 8
                const int ll = (int)(m & 7);
                const int64_t c = 4 * (m >> 3);
                float4 &v = *(float4 *)(xcm + ll * xstride + c);
                const float4 a = v;
                const float *w = wn + 8 * c + ll;
                v = make_float4((a.x * inv) * w[0], (a.y * inv) * w[8], (a.z * inv) * w[16], (a.w * inv) * w[24]);
                bad |= isnan(v.x) | isnan(v.y) | isnan(v.z) | isnan(v.w);
            }
            if (__any(bad) && p.st_norm >= 0 && lane == 0) nan_flag(st, p.layer, p.st_norm);
        }
    }

    // ---- the 32 chains, one stage per barrier.  Each group's ring values
    // (and, from LDS, activations) are read CH_AHEAD groups ahead of its fmas,
    // the order pinned with scheduling barriers (the compiler otherwise moves
    // each read to just before its use and waits out its latency).  With
    // GX > 0 (rows of GX <= 8 packed groups) chain l's activations sit in
    // registers for the whole walk: a wave pays about 9 cycles of issue per
    // 512-byte LDS read against 4.6 per fma, so halving the reads per group
    // is most of the walk's speed ----
    float acc = 0.0f;
    auto walk_stage = [&](int sg) {
        const float *dl = ring + ((sg & 1) * CH_LANES + lane) * CH_DSTRIDE;
        const int g0 = sg * CH_SQ;
        auto getx = [&](int j) -> X4 {
            if constexpr (GX > 0) {
                const int g = g0 + j < GX ? g0 + j : GX - 1;
                return X4{xq[4 * g], xq[4 * g + 1], xq[4 * g + 2], xq[4 * g + 3]};
            } else {
                return read_x4(xr + 16 * (g0 + j < G ? g0 + j : G - 1));
            }
        };
        X4 d[CH_AHEAD], x[CH_AHEAD];
#pragma unroll
        for (int k = 0; k < CH_AHEAD; ++k) {
            d[k] = read_x4(dl + 16 * k);
            x[k] = getx(k);
        }
#pragma unroll
        for (int j = 0; j < CH_SQ; ++j) {
            X4 dn = d[CH_AHEAD - 1], xn = x[CH_AHEAD - 1];
            if (j + CH_AHEAD < CH_SQ) {
                dn = read_x4(dl + 16 * (j + CH_AHEAD));
                xn = getx(j + CH_AHEAD);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (j == 0 || g0 + j < G) {  // (group g0 exists: sg < nstage)
                acc = q4_chain4(acc, d[0].b0, x[0].b0);
                acc = q4_chain4(acc, d[0].b1, x[0].b1);
                acc = q4_chain4(acc, d[0].b2, x[0].b2);
                acc = q4_chain4(acc, d[0].b3, x[0].b3);
            }
#pragma unroll
            for (int k = 0; k + 1 < CH_AHEAD; ++k) {
                d[k] = d[k + 1];
                x[k] = x[k + 1];
            }
            d[CH_AHEAD - 1] = dn;
            x[CH_AHEAD - 1] = xn;
        }
    };
    if constexpr (GX > 0) {
        constexpr int NST = (GX + CH_SQ - 1) / CH_SQ;
#pragma unroll
        for (int sg = 0; sg < NST; ++sg) {
            lds_barrier();
            if (lane < CH_LANES) walk_stage(sg);
        }
    } else {
        for (int sg = 0; sg < nstage; ++sg) {
            lds_barrier();
            if (lane < CH_LANES) walk_stage(sg);
        }
    }
    // lanes 8ρ..8ρ+7 hold a row's chains 0..7: the reduction of q4_consume
    const float total = q.row_ok ? flush_small(red8_dpp(acc)) : 0.0f;  // valid in lane 8r
    const float v1 = dpp_shl8(total);  // the pair's second row
    if (!leader) return;
    auto finish = [&](int64_t r, float v, float bias) {  // finish_row over this kernel's copy of x
        if (p.a_ptr) {
            for (int64_t k = p.a_ptr[r]; k < p.a_ptr[r + 1]; ++k) {
                const int64_t e = p.a_col[k];
                const float xe = GX > 0 ? (NORM ? xcm[e] : xs[e]) : xcm[(e & 7) * xstride + (e >> 3)];
                const float prod = xe * half_bits(p.a_val[k]);
                v = v + prod;
            }
        }
        if (r < p.bias_len) v = v + bias;
        return v;
    };
    const int64_t r0 = q.r0, r1 = q.r1;
    const float y0 = finish(r0, total, b0);
    const float y1 = r1 >= 0 ? finish(r1, v1, b1) : 0.0f;
    if constexpr (MODE == MODE_STORE) {
        p.y[r0] = y0;
        if (r1 >= 0) p.y[r1] = y1;
    } else if constexpr (MODE == MODE_RESIDUAL) {
        if (isnan(y0) || (r1 >= 0 && isnan(y1))) nan_flag(st, p.layer, p.st_a);
        if (p.kwta_k > 0) {  // the previous block's K-WTA on the residual (the MODE_QKV launch's threshold)
            old0 = old0 < kthr ? -1e9f : old0;
            old1 = old1 < kthr ? -1e9f : old1;
        }
        const float h0 = old0 + y0;
        p.y[r0] = h0;
        bool bad = isnan(h0);
        if (r1 >= 0) {
            const float h1 = old1 + y1;
            p.y[r1] = h1;
            bad |= isnan(h1);
        }
        if (bad) nan_flag(st, p.layer, p.st_b);
    } else {
        qkv_store(p, r0, r1, y0, y1, cs, sn, pos);
    }
}

// gemv_q4_chain_kernel for a mode, norm and row length (G packed groups).
template <int MODE, bool NORM, int GX = CH_XREG_MAX>
void (*chain_kernel_g(int G))(GemvParams, int64_t, int) {
    if constexpr (GX == 0) {
        return gemv_q4_chain_kernel<MODE, NORM, 0>;
    } else {
        if (G == GX) return gemv_q4_chain_kernel<MODE, NORM, GX>;
        return chain_kernel_g<MODE, NORM, GX - 1>(G);
    }
}
void (*chain_kernel(int mode, bool norm, int G))(GemvParams, int64_t, int) {
    if (mode == MODE_QKV) return norm ? chain_kernel_g<MODE_QKV, true>(G) : chain_kernel_g<MODE_QKV, false>(G);
    if (mode == MODE_RESIDUAL) return norm ? chain_kernel_g<MODE_RESIDUAL, true>(G) : chain_kernel_g<MODE_RESIDUAL, false>(G);
    return norm ? chain_kernel_g<MODE_STORE, true>(G) : chain_kernel_g<MODE_STORE, false>(G);
}

using KernelFn = void (*)(GemvParams, int64_t, int, int);

// LDS row stride (floats) of the chain-major activation copy: the floats the
// row walk reads (q4_xrow), padded so that stride / 4 is odd (the eight chain
// rows' 16-byte reads then fall in distinct banks).
int q4_xstride(int64_t K) { return q4_xrow((int)(K / 32)) + 4; }

}  // namespace

int gemv_chain_stride(int64_t K) { return chain_xstride(K); }
int64_t q4_0_packed_bytes(int64_t N, int64_t K) { return N * ((K / 32 + 3) / 4) * 80 + Q4_TAIL_PAD; }
int64_t q8_0_packed_bytes(int64_t N, int64_t K) { return (N + 7) / 8 * ((K / 32 + 3) / 4) * Q8_TILE_GROUP + Q8_TAIL_PAD; }

int launch_pack_q8_0(const uint8_t *src, uint8_t *dst, int64_t N, int64_t K, hipStream_t s) {
    if (N < 0 || K <= 0 || K % 32 != 0 || (N > 0 && (!src || !dst)))
        return set_error(GAJE_ERR_INVALID_ARG, "pack_q8_0: bad arguments");
    const int64_t G = (K / 32 + 3) / 4;
    int64_t grid = ((N + 7) / 8 * G * 8 + 255) / 256;
    if (grid < 1) grid = 1;
    if (grid > 65535) grid = 65535;
    hipLaunchKernelGGL(pack_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0, s, src, dst, N, (int)(K / 32));
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

namespace {

// genomic_dot_product_q4_0 on the file's own Q4_0Blocks (20 bytes: f16 scale,
// f16 min, 16 code bytes, element e in byte e / 2, the low nibble for even e:
// blocks.rs:18-30), with no packing: lanes 8r..8r+7 of a wave hold row r's
// eight chains (chain l = element 8c + l of each block's chunk c,
// genomic.rs:263-336), d = fma(f32(q), scale, min) and acc = fma(d, x, acc)
// block by block, then the AVX2 reduction ((a0+a4)+(a2+a6)) +
// ((a1+a5)+(a3+a7)), the flush and the bias.  A lane reads its block's five
// dwords (the scale/min word and the four code dwords that hold its nibbles)
// and its four inputs, QB_AHEAD blocks ahead of the arithmetic.
constexpr int QB_AHEAD = 4;
__global__ __launch_bounds__(256) void gemv_q4_blocks_kernel(const uint8_t *blocks, const float *x, const float *bias,
                                                            int64_t bias_len, float *y, int64_t n, int nb) {
    const int lane = threadIdx.x & 63, l = lane & 7;
    const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    const bool ok = row < n;
    const uint32_t *rb = (const uint32_t *)(blocks + (size_t)(ok ? row : 0) * nb * 20);
    const int sh = 8 * (l >> 1) + 4 * (l & 1);  // the nibble of element 8c + l in code dword c
    float acc = 0.0f;
    uint32_t w[QB_AHEAD][5];
    float xv[QB_AHEAD][4];
    auto load = [&](int j, int s) {
        const uint32_t *b = rb + 5 * (j < nb ? j : nb - 1);
#pragma unroll
        for (int i = 0; i < 5; ++i) w[s][i] = b[i];
        const float *xb = x + 32 * (int64_t)(j < nb ? j : nb - 1) + l;
#pragma unroll
        for (int c = 0; c < 4; ++c) xv[s][c] = xb[8 * c];
    };
#pragma unroll
    for (int s = 0; s < QB_AHEAD; ++s) load(s, s);
    for (int j0 = 0; j0 < nb; j0 += QB_AHEAD) {
#pragma unroll
        for (int s = 0; s < QB_AHEAD; ++s) {
            const int j = j0 + s;
            if (j < nb) {
                const float scale = half_bits((uint16_t)(w[s][0] & 0xFFFFu));
                const float mn = half_bits((uint16_t)(w[s][0] >> 16));
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float q = (float)((w[s][1 + c] >> sh) & 15u);
                    const float d = fmaf(q, scale, mn);
                    acc = fmaf(d, xv[s][c], acc);
                }
            }
            load(j + QB_AHEAD, s);  // past the row: its last block again, never used
        }
    }
    float t = flush_small(red8_dpp(acc));  // valid in lane 8r
    if (ok && l == 0) {
        if (row < bias_len) t = t + bias[row];
        y[row] = t;
    }
}

}  // namespace

int launch_q4_0_gemv_blocks(const uint8_t *blocks, const float *x, const float *bias, int64_t bias_len, float *y,
                            int64_t n, int64_t k, hipStream_t s) {
    if (n < 0 || k <= 0 || k % 32 != 0)
        return set_error(GAJE_ERR_INVALID_ARG, "q4_0 gemv: in_features must be a positive multiple of 32 (got %lld)",
                         (long long)k);
    if (n == 0) return GAJE_OK;
    if (!blocks || !x || !y || (bias_len > 0 && !bias)) return set_error(GAJE_ERR_INVALID_ARG, "q4_0 gemv: null buffer");
    if (((uintptr_t)blocks & 3) || ((uintptr_t)x & 3))
        return set_error(GAJE_ERR_INVALID_ARG, "q4_0 gemv: blocks and x must be 4-byte aligned");
    const int64_t grid = (n * 8 + 255) / 256;
    hipLaunchKernelGGL(gemv_q4_blocks_kernel, dim3((unsigned)grid), dim3(256), 0, s, blocks, x, bias, bias_len, y, n,
                       (int)(k / 32));
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_pack_q4_0(const uint8_t *src, uint8_t *dst, int64_t N, int64_t K, hipStream_t s) {
    if (N < 0 || K <= 0 || K % 32 != 0) return set_error(GAJE_ERR_INVALID_ARG, "pack: K must be a positive multiple of 32");
    if (N == 0) return GAJE_OK;
    if (!src || !dst) return set_error(GAJE_ERR_INVALID_ARG, "pack: null buffer");
    const int nb = (int)(K / 32);
    const int64_t total = N * ((nb + 3) / 4);
    int64_t grid = (total + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(pack_q4_0_kernel, dim3((unsigned)grid), dim3(256), 0, s, src, dst, N, nb);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int64_t f32_tiled_bytes(int64_t N, int64_t K) { return (N + 31) / 32 * 32 * K * 4; }

int launch_pack_f32_tiled(const float *src, float *dst, int64_t N, int64_t K, hipStream_t s) {
    if (N < 0 || K <= 0 || K % 8 != 0) return set_error(GAJE_ERR_INVALID_ARG, "f32 tiling: K must be a positive multiple of 8");
    if (N == 0) return GAJE_OK;
    if (!src || !dst || (((uintptr_t)src | (uintptr_t)dst) & 15)) return set_error(GAJE_ERR_INVALID_ARG, "f32 tiling: null or unaligned buffer");
    const int64_t total = (N + 31) / 32 * 32 * (K / 8);
    int64_t grid = (total + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(pack_f32_tiled_kernel, dim3((unsigned)grid), dim3(256), 0, s, src, dst, N, K);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

// LDS floats before the norm-weight copy: the activation vector (chain-major
// for Q4_0, plain otherwise) and, for LUT rows, one 16-entry table per row group.
static int64_t gemv_x_floats(int64_t K, int fmt) {
    if (fmt == FMT_Q4_0 || fmt == FMT_Q8_0) return (int64_t)8 * q4_xstride(K);
    int64_t f = (K + 3) & ~(int64_t)3;
    if (fmt == FMT_LUT4) f += (int64_t)(THREADS / 4) * 16;
    return f;
}

// LDS floats of the split-wave Q4_0 kernel: the chain-major activation rows
// (split_xrow + 4 floats each; the sum-of-squares chain's read-ahead ends in
// the row) and the two ring buffers.
static int64_t split_lds_floats(int64_t K) { return 8 * ((int64_t)split_xrow((int)(K / 32)) + 4) + 2 * 64 * SPLIT_DSTRIDE; }

size_t gemv_lds_bytes(int64_t K, int fmt, bool norm) {
    // Q4_0: + what the reads ahead may touch past the last chain row: the row
    // walk's next group (16 floats) and the sum-of-squares chain's read-ahead
    // (up to 28 floats with the short ring); never used
    const int64_t slack = (fmt == FMT_Q4_0 || fmt == FMT_Q8_0) ? 32 : 0;
    return (size_t)(gemv_x_floats(K, fmt) + (norm ? ((K + 3) & ~(int64_t)3) : 0) + slack) * 4;
}

// The chain kernel's conditions: latency-bound Q4_0 matvecs (few rows) in the
// modes it serves, with its stages and LDS within bounds.
static bool chain_ok(const GemvParams &p, int64_t npairs) {
    if (!(p.fmt == FMT_Q4_0 && (p.mode == MODE_STORE || p.mode == MODE_RESIDUAL || p.mode == MODE_QKV) && !p.gnorm &&
          !p.x_out && p.nb > 0 && (npairs + CH_PAIRS - 1) / CH_PAIRS <= 2 * (int64_t)device_cu_count()))
        return false;
    const int64_t G = (p.nb + 3) / 4;
    const size_t clds = (size_t)chain_lds_bytes(p.K, p.norm_w != nullptr);
    return (G + CH_SQ - 1) / CH_SQ <= CH_MAX_STAGES && G * 80 <= (int64_t)sizeof(kZeroRows) &&
           clds + 1024 <= max_lds_per_block();
}

bool gemv_chain_serves(const GemvParams &p) {
    if (p.N <= 0 || p.K <= 0 || p.nb != (int32_t)(p.K / 32)) return false;
    int64_t npairs;
    if (p.mode == MODE_QKV) npairs = (p.q_rows + 2 * p.kv_rows) / 2;
    else if (p.mode == MODE_STORE || p.mode == MODE_RESIDUAL) npairs = (p.N + 1) / 2;
    else return false;
    return npairs > 0 && chain_ok(p, npairs);
}

int launch_gemv(const GemvParams &p, hipStream_t s) {
    if (p.N < 0 || p.K <= 0 || !p.x || !p.y)
        return set_error(GAJE_ERR_INVALID_ARG, "gemv: invalid shape or null buffer");
    if (p.nb != (int32_t)(p.K / 32)) return set_error(GAJE_ERR_INVALID_ARG, "gemv: nb must be K/32");
    if (p.fmt == FMT_F32 && p.K % 4 != 0)
        return set_error(GAJE_ERR_UNSUPPORTED, "gemv: f32 rows need in_features %% 4 == 0 (got %lld)",
                         (long long)p.K);
    if (p.fmt == FMT_F32 && p.f32_tiled && p.K % 8 != 0)
        return set_error(GAJE_ERR_INVALID_ARG, "gemv: tiled f32 rows need in_features %% 8 == 0");
    if ((p.fmt == FMT_Q4_0 || p.fmt == FMT_Q8_0) && p.K % 32 != 0)
        return set_error(GAJE_ERR_UNSUPPORTED, "gemv: Q4_0/Q8_0 rows need in_features %% 32 == 0 (got %lld)",
                         (long long)p.K);
    if (p.fmt < FMT_F32 || p.fmt > FMT_G2) return set_error(GAJE_ERR_INVALID_ARG, "gemv: unknown format %d", p.fmt);
    if (p.fmt == FMT_G2 && (p.K % 32 != 0 || (p.rows_valid > 0 && !p.lut)))
        return set_error(GAJE_ERR_UNSUPPORTED, "gemv: 2-bit rows need in_features %% 32 == 0 and centroids");
    if (p.fmt != FMT_LUT4 && (((uintptr_t)p.x | (uintptr_t)p.norm_w) & 15))
        return set_error(GAJE_ERR_INVALID_ARG, "gemv: x and norm_w must be 16-byte aligned");
    if (p.rows_valid > 0 && !p.w) return set_error(GAJE_ERR_INVALID_ARG, "gemv: null weights");
    if (p.fmt == FMT_LUT4 && p.nb > 0 && p.rows_valid > 0 && !p.lut)
        return set_error(GAJE_ERR_INVALID_ARG, "gemv: null LUT");
    const size_t lds = gemv_lds_bytes(p.K, p.fmt, p.norm_w != nullptr);
    if (lds + 1024 > max_lds_per_block())  // dynamic + the kernel's static LDS
        return set_error(GAJE_ERR_UNSUPPORTED, "gemv: in_features %lld exceeds the LDS budget", (long long)p.K);
    int64_t npairs;
    switch (p.mode) {
        case MODE_QKV:
            if (!p.st || p.head_dim <= 0 || p.head_dim % 2 || p.q_rows % p.head_dim || p.kv_rows % p.head_dim ||
                p.N < p.q_rows + 2 * p.kv_rows || !p.q_out || !p.k_cache || !p.v_cache || !p.rope_cos ||
                !p.rope_sin || p.kv_cap <= 0 || p.kv_head_stride != p.kv_cap * p.head_dim)
                return set_error(GAJE_ERR_INVALID_ARG, "gemv: bad fused-QKV arguments");
            npairs = (p.q_rows + 2 * p.kv_rows) / 2;
            break;
        case MODE_SWIGLU:
            if (p.ffn <= 0 || 2 * p.ffn > p.N) return set_error(GAJE_ERR_INVALID_ARG, "gemv: bad SwiGLU arguments");
            if (p.y_cm && p.cm_stride < (p.ffn + 7) / 8)
                return set_error(GAJE_ERR_INVALID_ARG, "gemv: chain-major output stride too short");
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
    const bool chain = chain_ok(p, npairs);
    if (p.kwta_k > 0 && (!chain || (p.mode != MODE_QKV && p.mode != MODE_RESIDUAL) || !p.kwta_thr || p.x_cm ||
                         (p.mode == MODE_QKV && p.K > INT32_MAX)))
        return set_error(GAJE_ERR_UNSUPPORTED, "gemv: the fused K-WTA runs only on the chain kernel (QKV / residual)");
    // latency-bound Q4_0 matvecs (few rows): split waves
    if (chain) {
        const int64_t G = (p.nb + 3) / 4;
        const size_t clds = (size_t)chain_lds_bytes(p.K, p.norm_w != nullptr);
        const int64_t grid = (npairs + CH_PAIRS - 1) / CH_PAIRS;
        void (*fn)(GemvParams, int64_t, int) = chain_kernel(p.mode, p.norm_w != nullptr, (int)G);
        GemvParams pc = p;  // x_cm only in the layout this kernel copies whole
        if (pc.x_cm && (pc.cm_stride != chain_xstride(p.K) || ((uintptr_t)pc.x_cm & 15))) pc.x_cm = nullptr;
        hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(THREADS), clds, s, pc, npairs, chain_xstride(p.K));
        GAJE_HIP_CHECK(hipGetLastError());
        return GAJE_OK;
    }
    if (p.fmt == FMT_Q4_0 && (p.mode == MODE_STORE || p.mode == MODE_RESIDUAL || p.mode == MODE_QKV) && !p.gnorm &&
        !p.x_out && 2 * npairs <= SPLIT_MAX_ROWS && p.nb > 0 && (!p.norm_w || p.K / 4 <= SPLIT_NORM_MAX_K4)) {
        const size_t slds = (size_t)split_lds_floats(p.K) * 4;
        if (slds + 1024 <= max_lds_per_block()) {
            const int64_t grid = (npairs + SPLIT_PAIRS - 1) / SPLIT_PAIRS;
            const int xs = split_xrow(p.nb) + 4;
            void (*fn)(GemvParams, int64_t, int);
            if (p.mode == MODE_QKV) fn = p.norm_w ? gemv_q4_split_kernel<MODE_QKV, true> : gemv_q4_split_kernel<MODE_QKV, false>;
            else if (p.mode == MODE_RESIDUAL) fn = p.norm_w ? gemv_q4_split_kernel<MODE_RESIDUAL, true> : gemv_q4_split_kernel<MODE_RESIDUAL, false>;
            else fn = p.norm_w ? gemv_q4_split_kernel<MODE_STORE, true> : gemv_q4_split_kernel<MODE_STORE, false>;
            hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(THREADS), slds, s, p, npairs, xs);
            GAJE_HIP_CHECK(hipGetLastError());
            return GAJE_OK;
        }
    }
    // Q4_0 rows of at most 8 packed groups, every row stored: the LDS-staged
    // kernel (SwiGLU pairs only as streams: for a few thousand pairs the
    // row-per-lane kernel, whose four waves share the RMSNorm prologue and
    // whose lanes each walk one chain, measured faster: 6.7 against 7.5 us at
    // 4864 pairs of K = 896)
    if (p.fmt == FMT_Q4_0 && (p.mode == MODE_STORE || p.mode == MODE_SWIGLU) && !p.gnorm && !p.a_ptr && !p.x_out &&
        p.bias_len == 0 && p.nb > 0 && (p.nb + 3) / 4 <= 8 && p.rows_valid == p.N &&
        (p.mode == MODE_STORE || (p.ffn + 3) / 4 > 8 * (int64_t)device_cu_count())) {
        const int64_t rows = p.mode == MODE_SWIGLU ? p.ffn : p.N;
        const int xs = q4_xstride(p.K);
        const int G = (p.nb + 3) / 4;
        const int raw = (int)(p.K * 4 * (p.norm_w ? 2 : 1) + (p.mode == MODE_SWIGLU ? 256 : 0));
        const size_t fixed = (size_t)8 * xs * 4 + raw + 1024;
        const bool swiglu = p.mode == MODE_SWIGLU;
        void *fn = nullptr;
        int waves = 0, nst = 0;
        size_t stage = 0;
        int64_t grid = 0;
        const int64_t trows1 = swiglu ? 4 : 8;  // output rows per tile with one row per lane
        if ((rows + trows1 - 1) / trows1 <= 8 * (int64_t)device_cu_count()) {
            // few tiles (rows, not SwiGLU pairs): one 8-row tile (one row per lane) per
            // wave, all at once; single-wave workgroups, or four waves sharing one
            // RMSNorm prologue
            stage = (size_t)q4l_stage_bytes(p.mode, G, 1);
            waves = p.norm_w ? 4 : 1;
            nst = 1;
            grid = ((rows + trows1 - 1) / trows1 + waves - 1) / waves;
            fn = p.norm_w ? q4l_kernel<MODE_STORE, 4, 1, 1>(G) : q4l_kernel<MODE_STORE, 1, 1, 1>(G);
        } else {
            // streams: persistent workgroups, 16-row tiles (two rows per lane); two waves
            // per SIMD with two stages each where the LDS holds them, else one with three
            stage = (size_t)q4l_stage_bytes(p.mode, G, 2);
            const bool two = fixed + 8 * 2 * stage <= max_lds_per_block();
            waves = two ? 8 : 4;
            nst = two ? 2 : 3;
            const int64_t ntiles = (rows + 2 * trows1 - 1) / (2 * trows1);
            grid = std::min<int64_t>((ntiles + waves - 1) / waves, device_cu_count());
            if (swiglu) fn = two ? q4l_kernel<MODE_SWIGLU, 8, 2, 2>(G) : q4l_kernel<MODE_SWIGLU, 4, 3, 2>(G);
            else if (p.tol) fn = two ? q4l_kernel<MODE_STORE, 8, 2, 2, true>(G) : q4l_kernel<MODE_STORE, 4, 3, 2, true>(G);
            else fn = two ? q4l_kernel<MODE_STORE, 8, 2, 2>(G) : q4l_kernel<MODE_STORE, 4, 3, 2>(G);
        }
        const size_t lds = fixed - 1024 + (size_t)waves * nst * stage;
        if (lds + 1024 <= max_lds_per_block()) {
            const int64_t limit = q4_0_packed_bytes(p.N, p.K);
            hipLaunchKernelGGL((void (*)(GemvParams, int, int64_t, int))fn, dim3((unsigned)grid), dim3(waves * WAVE),
                               lds, s, p, xs, limit, raw);
            GAJE_HIP_CHECK(hipGetLastError());
            return GAJE_OK;
        }
    }
    // Q8_0 rows of at most 8 packed groups: long matrices (the lm_head) through
    // the LDS-staged kernel, the others on the register-ring stream
    if (p.fmt == FMT_Q8_0 && (p.mode == MODE_ARGMAX || p.mode == MODE_STORE) && !p.gnorm && !p.a_ptr && p.nb > 0 &&
        (p.nb + 3) / 4 <= 8 && p.bias_len == 0 && p.rows_valid == p.N &&
        (p.N + 15) / 16 >= 4 * (int64_t)device_cu_count()) {
        const int G = (p.nb + 3) / 4;
        const int xs = q4_xstride(p.K);
        const int raw = (int)(((p.norm_w ? 2 : 1) * p.K * 4 + 15) & ~15);
        const size_t per = (size_t)(2 * G * Q8_TILE_GROUP + 1023) / 1024 * 1024;
        constexpr int W = Q8L_WAVES, S = Q8L_STAGES;
        const size_t lds = (size_t)8 * xs * 4 + raw + (size_t)W * S * per;
        if (lds + 1024 <= max_lds_per_block()) {
            const int64_t nsup = (p.N + 15) / 16;
            const int64_t grid = std::min<int64_t>((nsup + W - 1) / W, device_cu_count());
            void (*fn)(GemvParams, int, int64_t) =
                (void (*)(GemvParams, int, int64_t))(p.mode == MODE_ARGMAX ? q8l_kernel<MODE_ARGMAX, W, S>(G)
                                                                           : q8l_kernel<MODE_STORE, W, S>(G));
            hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(W * WAVE), lds, s, p, xs, q8_0_packed_bytes(p.N, p.K));
            GAJE_HIP_CHECK(hipGetLastError());
            return GAJE_OK;
        }
    }
    if (p.fmt == FMT_Q8_0 && (p.mode == MODE_ARGMAX || p.mode == MODE_STORE) && !p.gnorm && !p.a_ptr && p.nb > 0 &&
        (p.nb + 3) / 4 <= Q8S_D) {
        void (*sf)(GemvParams, int);
        if (p.mode == MODE_ARGMAX) sf = p.nontemporal ? gemv_q8_stream_kernel<true, MODE_ARGMAX> : gemv_q8_stream_kernel<false, MODE_ARGMAX>;
        else sf = p.nontemporal ? gemv_q8_stream_kernel<true, MODE_STORE> : gemv_q8_stream_kernel<false, MODE_STORE>;
        // one workgroup per compute unit streams best (measured on a 151936 x
        // 896 matrix: 43.9 us against 46.0 with two and 53.0 with three)
        int64_t grid = (p.N + THREADS / 8 - 1) / (THREADS / 8);
        if (grid > device_cu_count()) grid = device_cu_count();
        hipLaunchKernelGGL(sf, dim3((unsigned)grid), dim3(THREADS), lds, s, p, q4_xstride(p.K));
        GAJE_HIP_CHECK(hipGetLastError());
        return GAJE_OK;
    }
    // LUT rows stored whole: the LDS-staged kernel (tables per row and block,
    // or the one shared table)
    if (p.fmt == FMT_LUT4 && p.mode == MODE_STORE && !p.gnorm && !p.a_ptr && !p.x_out && !p.norm_w && p.nb > 0 &&
        p.rows_valid == p.N && p.st_in < 0 && (p.lut_block_stride == 0 || p.lut_block_stride == 16) &&
        ((uintptr_t)p.x & 15) == 0 && ((uintptr_t)p.lut & 15) == 0 && ((uintptr_t)p.w & 15) == 0) {
        const bool shared = p.lut_block_stride == 0;
        const size_t llds = lut4_lds_bytes(p.K, p.nb, shared);
        if (llds + 1024 <= max_lds_per_block()) {
            const int64_t grid = (p.N + LUTL_ROWS - 1) / LUTL_ROWS;
            hipLaunchKernelGGL(shared ? gemv_lut4_lds_kernel<true> : gemv_lut4_lds_kernel<false>, dim3((unsigned)grid),
                               dim3(WAVE), llds, s, p);
            GAJE_HIP_CHECK(hipGetLastError());
            return GAJE_OK;
        }
    }
    KernelFn fn;
    int lpr;
    if (p.fmt == FMT_Q4_0) {
        const bool long_rows = q4_depth(p.nb) == 2 * Q4_PREFETCH;
        lpr = 8;
        if (long_rows)
            fn = p.nontemporal ? gemv_kernel<FMT_Q4_0, 8, true, 2 * Q4_PREFETCH>
                               : gemv_kernel<FMT_Q4_0, 8, false, 2 * Q4_PREFETCH>;
        else if (p.mode == MODE_SWIGLU && !p.nontemporal)
            fn = gemv_kernel<FMT_Q4_0, 8, false, Q4_PREFETCH, MODE_SWIGLU>;
        else
            fn = p.nontemporal ? gemv_kernel<FMT_Q4_0, 8, true, Q4_PREFETCH> : gemv_kernel<FMT_Q4_0, 8, false, Q4_PREFETCH>;
    } else if (p.fmt == FMT_Q8_0) {
        const bool long_rows = q4_depth(p.nb) == 2 * Q4_PREFETCH;
        lpr = 8;
        if (long_rows)
            fn = p.nontemporal ? gemv_kernel<FMT_Q8_0, 8, true, 2 * Q4_PREFETCH>
                               : gemv_kernel<FMT_Q8_0, 8, false, 2 * Q4_PREFETCH>;
        else if (p.mode == MODE_ARGMAX && p.nontemporal)
            fn = gemv_kernel<FMT_Q8_0, 8, true, Q4_PREFETCH, MODE_ARGMAX>;
        else
            fn = p.nontemporal ? gemv_kernel<FMT_Q8_0, 8, true, Q4_PREFETCH> : gemv_kernel<FMT_Q8_0, 8, false, Q4_PREFETCH>;
    } else if (p.fmt == FMT_LUT4) {
        lpr = 4;
        fn = gemv_kernel<FMT_LUT4, 4, false, 1>;
    } else if (p.fmt == FMT_G2) {
        lpr = g2_lanes(p.nb);
        if (lpr == 8) fn = p.nontemporal ? gemv_kernel<FMT_G2, 8, true, 1> : gemv_kernel<FMT_G2, 8, false, 1>;
        else fn = p.nontemporal ? gemv_kernel<FMT_G2, 32, true, 1> : gemv_kernel<FMT_G2, 32, false, 1>;
    } else {
        lpr = 2;
        if (p.mode == MODE_ARGMAX && p.nontemporal) fn = gemv_kernel<FMT_F32, 2, true, 1, MODE_ARGMAX>;
        else fn = p.nontemporal ? gemv_kernel<FMT_F32, 2, true, 1> : gemv_kernel<FMT_F32, 2, false, 1>;
    }
    const int64_t pairs_per_block = (WAVE / (2 * lpr)) * (THREADS / WAVE);
    int64_t grid = (npairs + pairs_per_block - 1) / pairs_per_block;
    if (grid > MAX_GRID) grid = MAX_GRID;
    // tiled f32 rows stream at the best rate with one workgroup per compute
    // unit walking its share of the tiles (measured on a 151936 x 896 matrix)
    if (p.fmt == FMT_F32 && p.f32_tiled && grid > device_cu_count()) grid = device_cu_count();
    // long Q8_0 matrices (the lm_head): one wave of resident workgroups walks
    // the row pairs, so the activation prologue runs once per workgroup and
    // each lane's next row streams in while it finishes the current one
    if (p.fmt == FMT_Q8_0) {
        int per_cu = 0;
        GAJE_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, THREADS, lds));
        const int64_t resident = (int64_t)(per_cu > 0 ? per_cu : 1) * device_cu_count();
        if (grid > resident) grid = resident;
    }
    const int xstride = (p.fmt == FMT_Q4_0 || p.fmt == FMT_Q8_0) ? q4_xstride(p.K) : 0;
    const int nw_off = (int)gemv_x_floats(p.K, p.fmt);
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(THREADS), lds, s, p, npairs, xstride, nw_off);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
