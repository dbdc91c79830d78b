// Mixture-of-experts SwiGLU FFN layer over Q4_0 experts (top-2 routing).
//
// The reference has no MoE; this layer composes its primitives:
//   router logit l_e = dot_product(x, router_e)      dot.rs:23-94 (bit-exact order)
//   e_e = expf(l_e - max_e l),  p_e = e_e / (e_0 + e_1 + ... )   (serial sum in e order)
//   top-2 by p (ties to the lower expert id), weights renormalised:
//     w_a = p_a / (p_a + p_b),  w_b = p_b / (p_a + p_b)
//   expert FFN_e(x) = down_e(swiglu_balanced(gate_e(x), up_e(x)))   linear/forward.rs,
//                                                      activation.rs:35-51
//   y = (w_a * FFN_a(x)) + (w_b * FFN_b(x))
// Routing is computed bit-exactly, so the expert choice matches the oracle;
// the expert products run on the MFMA units (fp32 accuracy, not bit-exact).
// Dispatch is a deterministic prefix scan: expert e's rows are its tokens in
// token order, experts concatenated in id order.
#include <hip/hip_runtime.h>

#include "common.h"
#include "device_util.h"
#include "kernels.h"

namespace gaje {
namespace {

// One workgroup per token, one wave per expert: the token's activations are
// staged in LDS by the whole workgroup, then lanes 0..7 of each expert's wave
// run the eight FMA chains of dot_product over the 8-float chunks (router
// weights read in batches of 8 chunks ahead of the FMAs), then
// ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)) and the scalar tail.  Thread 0 then
// forms the softmax, the top-2 and the renormalised weights.
__global__ __launch_bounds__(64 * MOE_MAX_EXPERTS) void moe_route_kernel(MoeParams p) {
    extern __shared__ __align__(16) float xs[];
    __shared__ float logit[MOE_MAX_EXPERTS];
    const int64_t t = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, e = tid >> 6;
    const float *xg = p.x + t * p.ldx;
    for (int64_t k = tid; k < p.h; k += 64 * MOE_MAX_EXPERTS) xs[k] = xg[k];
    __syncthreads();
    const float *x = xs;
    if (e < p.n_expert && lane < 8) {
        const float *w = p.router + (size_t)e * p.h;
        float a = 0.0f;
        const int64_t chunks = p.h / 8;
        int64_t c = 0;
        for (; c + 8 <= chunks; c += 8) {
            float wv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) wv[u] = w[8 * (c + u) + lane];
#pragma unroll
            for (int u = 0; u < 8; ++u) a = fmaf(x[8 * (c + u) + lane], wv[u], a);
        }
        for (; c < chunks; ++c) a = fmaf(x[8 * c + lane], w[8 * c + lane], a);
        const float a4 = __shfl(a, (lane + 4) & 7, 8);
        const float u = a + a4;                          // lane l<4: a_l + a_{l+4}
        const float u1 = __shfl(u, (lane + 1) & 7, 8);   // lane 0: u1, lane 2: u3
        const float v = u + u1;                          // lane 0: u0+u1, lane 2: u2+u3
        const float v2 = __shfl(v, (lane + 2) & 7, 8);
        if (lane == 0) {
            float sum = v + v2;
            for (int64_t k = chunks * 8; k < p.h; ++k) {
                const float prod = x[k] * w[k];
                sum = sum + prod;
            }
            logit[e] = sum;
        }
    }
    __syncthreads();
    if (tid != 0) return;
    const int E = p.n_expert;
    float mx = logit[0];
    for (int i = 1; i < E; ++i) mx = logit[i] > mx ? logit[i] : mx;
    float ex[MOE_MAX_EXPERTS];
    float s = 0.0f;
    for (int i = 0; i < E; ++i) {
        ex[i] = expf_ref(logit[i] - mx);
        s = s + ex[i];
    }
    int a = 0;
    for (int i = 1; i < E; ++i)
        if (ex[i] / s > ex[a] / s) a = i;
    int b = a == 0 ? 1 : 0;
    for (int i = 0; i < E; ++i)
        if (i != a && ex[i] / s > ex[b] / s) b = i;
    const float pa = ex[a] / s, pb = ex[b] / s;
    const float den = pa + pb;
    p.top_idx[2 * t] = a;
    p.top_idx[2 * t + 1] = b;
    p.top_w[2 * t] = pa / den;
    p.top_w[2 * t + 1] = pb / den;
}

// The router with everything staged in LDS (16-byte aligned x rows and router,
// h % 4 == 0): one workgroup of 256 threads per token copies the router and
// the token's activations into LDS with LDS-direct loads (all in flight at
// once, spread over the four waves), then lane SL e + l (l < 8, SL = 256 /
// EMAX lanes per expert slot) runs chain l of dot_product over the chunks for
// expert e, reading both operands from LDS; two or four experts per wave, so
// the chains are spread over the four SIMDs.  The reduction, the scalar tail
// and the softmax / top-2 compute moe_route_kernel's values: wave 0 forms one
// exponential and one quotient per lane (the exponential's table in LDS) and
// hands them round with lane shuffles.  (Four tokens per workgroup used a
// quarter of the CUs and waited longer on their copies: 10 against 7 us for
// 256 tokens x 8 experts x 1536.)
template <int EMAX>  // 8 or 16 experts at most
__global__ __launch_bounds__(256) void moe_route_lds_kernel(MoeParams p) {
    constexpr int SL = 256 / EMAX;
    extern __shared__ __align__(16) float sm[];
    __shared__ float logit[EMAX];
    __shared__ uint64_t tab[32];  // the exponential's table
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < 32) tab[tid] = kExp2Tab[tid];
    const int E = p.n_expert;
    const int64_t h = p.h, t = blockIdx.x;
    // router rows h + 8 floats apart, so that the experts' reads of one chunk
    // element fall in different banks
    const int64_t rs = h + 8;
    float *rw = sm;            // [E][rs]
    float *xs = sm + E * rs;   // [h]
    {
        const int64_t xb = h * 4, nx = (xb + 1023) / 1024;  // bytes and KiB copies of a row
        for (int64_t q = wave; q < (E + 1) * nx; q += 4) {
            const int64_t r = q / nx, c = q % nx;
            if (1024 * c + 16 * lane < xb) {
                if (r < E)
                    lds_dma16<true>((const uint8_t *)(p.router + r * h) + 1024 * c + 16 * lane,
                                    lds_addr(rw + r * rs) + (uint32_t)(1024 * c));
                else
                    lds_dma16((const uint8_t *)(p.x + t * p.ldx) + 1024 * c + 16 * lane, lds_addr(xs) + (uint32_t)(1024 * c));
            }
        }
        wait_vmcnt<0>();
    }
    __syncthreads();
    const int e = tid / SL, l = tid % SL;
    const bool on = l < 8 && e < E;
    const float *w = rw + (on ? e : 0) * rs;
    float a = 0.0f;
    const int64_t chunks = h / 8;
    if (on) {
        int64_t c = 0;
        for (; c + 8 <= chunks; c += 8) {
            float xv[8], wv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                xv[u] = xs[8 * (c + u) + l];
                wv[u] = w[8 * (c + u) + l];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) a = fmaf(xv[u], wv[u], a);
        }
        for (; c < chunks; ++c) a = fmaf(xs[8 * c + l], w[8 * c + l], a);
    }
    // lanes SL e .. SL e + 7 are an aligned group of 8
    const float a4 = __shfl(a, (lane + 4) & 7, 8);
    const float u = a + a4;                          // lane l<4: a_l + a_{l+4}
    const float u1 = __shfl(u, (lane + 1) & 7, 8);   // lane 0: u1, lane 2: u3
    const float v = u + u1;                          // lane 0: u0+u1, lane 2: u2+u3
    const float v2 = __shfl(v, (lane + 2) & 7, 8);
    if (on && l == 0) {
        float sum = v + v2;
        for (int64_t k = chunks * 8; k < h; ++k) {
            const float prod = xs[k] * w[k];
            sum = sum + prod;
        }
        logit[e] = sum;
    }
    __syncthreads();
    if (wave != 0) return;
    // softmax over the token's logits: e_j = expf(l_j - max) in lane j, the sum
    // in expert order (every lane forms the same one), p_j = e_j / sum; lane 0
    // then takes the top-2 and the weights
    float lg[EMAX];
#pragma unroll
    for (int i = 0; i < EMAX; ++i) lg[i] = i < E ? logit[i] : -INFINITY;
    float mx = lg[0];
#pragma unroll
    for (int i = 1; i < EMAX; ++i)
        if (i < E) mx = lg[i] > mx ? lg[i] : mx;
    const float ej = expf_ref_t(logit[lane < E ? lane : 0] - mx, tab);
    float ex[EMAX];
#pragma unroll
    for (int i = 0; i < EMAX; ++i) ex[i] = __shfl(ej, i, WAVE);
    float ssum = 0.0f;
#pragma unroll
    for (int i = 0; i < EMAX; ++i)
        if (i < E) ssum = ssum + ex[i];
    const float pj = ej / ssum;
    float pr[EMAX];
#pragma unroll
    for (int i = 0; i < EMAX; ++i) pr[i] = __shfl(pj, i, WAVE);
    if (lane != 0) return;
    int ia = 0;
    float pa = pr[0];
#pragma unroll
    for (int i = 1; i < EMAX; ++i)
        if (i < E && pr[i] > pa) ia = i, pa = pr[i];
    int ib = ia == 0 ? 1 : 0;
    float pb = pr[ib];
#pragma unroll
    for (int i = 0; i < EMAX; ++i)
        if (i < E && i != ia && pr[i] > pb) ib = i, pb = pr[i];
    const float den = pa + pb;
    p.top_idx[2 * t] = ia;
    p.top_idx[2 * t + 1] = ib;
    p.top_w[2 * t] = pa / den;
    p.top_w[2 * t + 1] = pb / den;
}

// Dispatch plan (one workgroup): for each expert, its tokens in token order;
// rows[] holds the token of every dispatched row (experts concatenated in id
// order), slot[t][k] the row of token t's k-th expert, counts/offsets per
// expert.  Chunks of 1024 tokens; within a chunk an expert's rank of a token
// is the ballot of its wave's flags below the lane plus the counts of the
// earlier waves.  A first pass counts, a second assigns the rows.
__global__ __launch_bounds__(1024) void moe_plan_kernel(MoeParams p) {
    constexpr int NW = 1024 / 64;
    __shared__ int wcnt[NW][MOE_MAX_EXPERTS];
    __shared__ int run[MOE_MAX_EXPERTS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = p.n_expert;
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    if (tid < MOE_MAX_EXPERTS) run[tid] = 0;
    __syncthreads();
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1) {  // offsets from the counts: experts in id order
            if (tid == 0) {
                int o = 0;
                for (int e = 0; e < E; ++e) {
                    const int c = run[e];
                    p.counts[e] = c;
                    p.offsets[e] = o;
                    run[e] = o;
                    o += c;
                }
            }
            __syncthreads();
        }
        for (int64_t t0 = 0; t0 < p.T; t0 += 1024) {
            const int64_t t = t0 + tid;
            const int ea = t < p.T ? p.top_idx[2 * t] : -1, eb = t < p.T ? p.top_idx[2 * t + 1] : -1;
            int pre_a = 0, pre_b = 0;
            for (int e = 0; e < E; ++e) {
                const uint64_t m = __ballot(ea == e || eb == e);
                if (lane == 0) wcnt[wave][e] = __popcll(m);
                const int pre = __popcll(m & below);
                if (ea == e) pre_a = pre;
                if (eb == e) pre_b = pre;
            }
            __syncthreads();
            if (pass == 1 && t < p.T) {
                int wa = 0, wb = 0;
                for (int w = 0; w < wave; ++w) {
                    wa += wcnt[w][ea];
                    wb += wcnt[w][eb];
                }
                const int ra = run[ea] + wa + pre_a, rb = run[eb] + wb + pre_b;
                p.rows[ra] = (int32_t)t;
                p.rows[rb] = (int32_t)t;
                p.slot[2 * t] = ra;
                p.slot[2 * t + 1] = rb;
            }
            __syncthreads();
            if (tid < E) {
                int c = 0;
                for (int w = 0; w < NW; ++w) c += wcnt[w][tid];
                run[tid] += c;
            }
            __syncthreads();
        }
    }
}

// y[t] = (w_a * Y[slot_a]) + (w_b * Y[slot_b]), each product rounded.
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeParams p, const float *Y) {
    const int64_t t = blockIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= p.h) return;
    const int ra = p.slot[2 * t], rb = p.slot[2 * t + 1];
    const float wa = p.top_w[2 * t], wb = p.top_w[2 * t + 1];
    const float ya = wa * Y[(size_t)ra * p.h + j];
    const float yb = wb * Y[(size_t)rb * p.h + j];
    p.y[t * p.ldy + j] = ya + yb;
}

// The combine with the down product's split-K reduce folded in: expert row r's
// output is formed from the S partials part[z][r][.] (R rows each) as
// gemm_reduce_kernel forms it (summed in split order, then flush_small; the
// expert products carry no bias or residual), then weighted as above.
__global__ __launch_bounds__(256) void moe_combine_split_kernel(MoeParams p, const float *part, int S, int64_t R) {
    const int64_t t = blockIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= p.h) return;
    const int ra = p.slot[2 * t], rb = p.slot[2 * t + 1];
    const float wa = p.top_w[2 * t], wb = p.top_w[2 * t + 1];
    const int64_t plane = R * p.h;
    const float *pa = part + (int64_t)ra * p.h + j, *pb = part + (int64_t)rb * p.h + j;
    float va = pa[0], vb = pb[0];
    for (int z = 1; z < S; ++z) {
        va = va + pa[z * plane];
        vb = vb + pb[z * plane];
    }
    const float ya = wa * flush_small(va);
    const float yb = wb * flush_small(vb);
    p.y[t * p.ldy + j] = ya + yb;
}

}  // namespace

int launch_moe_route(const MoeParams &p, hipStream_t s) {
    if (p.T <= 0 || p.T > 65535 || p.n_expert < 2 || p.n_expert > MOE_MAX_EXPERTS || !p.x || !p.router || p.h <= 0)
        return set_error(GAJE_ERR_INVALID_ARG, "moe route: bad arguments");
    if ((size_t)p.h * 4 + 1024 > max_lds_per_block()) return set_error(GAJE_ERR_UNSUPPORTED, "moe route: hidden too large");
    const size_t slds = ((size_t)p.n_expert * (p.h + 8) + (size_t)p.h) * 4;
    const bool staged = p.h % 4 == 0 && p.ldx % 4 == 0 && (((uintptr_t)p.x | (uintptr_t)p.router) & 15) == 0 &&
                        slds + 1024 <= max_lds_per_block();
    if (staged) {
        if (p.n_expert <= 8) hipLaunchKernelGGL(moe_route_lds_kernel<8>, dim3((unsigned)p.T), dim3(256), slds, s, p);
        else hipLaunchKernelGGL(moe_route_lds_kernel<16>, dim3((unsigned)p.T), dim3(256), slds, s, p);
    } else {
        hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)p.T), dim3(64 * MOE_MAX_EXPERTS), (size_t)p.h * 4, s, p);
    }
    GAJE_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(1024), 0, s, p);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_moe_combine(const MoeParams &p, const float *Y, hipStream_t s) {
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((p.h + 255) / 256), (unsigned)p.T), dim3(256), 0, s, p, Y);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

int launch_moe_combine_split(const MoeParams &p, const float *part, int nsplit, int64_t R, hipStream_t s) {
    if (!part || nsplit < 1 || R < 2 * p.T) return set_error(GAJE_ERR_INVALID_ARG, "moe combine: bad partials");
    hipLaunchKernelGGL(moe_combine_split_kernel, dim3((unsigned)((p.h + 255) / 256), (unsigned)p.T), dim3(256), 0, s, p,
                       part, nsplit, R);
    GAJE_HIP_CHECK(hipGetLastError());
    return GAJE_OK;
}

}  // namespace gaje
