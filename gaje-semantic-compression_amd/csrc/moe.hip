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

// One workgroup per token, one wave per expert: lanes 0..7 run the eight FMA
// chains of dot_product over the 8-float chunks, then
// ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)) and the scalar tail.  Thread 0 then
// forms the softmax, the top-2 and the renormalised weights.
__global__ __launch_bounds__(64 * MOE_MAX_EXPERTS) void moe_route_kernel(MoeParams p) {
    __shared__ float logit[MOE_MAX_EXPERTS];
    const int64_t t = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, e = tid >> 6;
    const float *x = p.x + t * p.ldx;
    if (e < p.n_expert && lane < 8) {
        const float *w = p.router + (size_t)e * p.h;
        float a = 0.0f;
        const int64_t chunks = p.h / 8;
        for (int64_t c = 0; c < chunks; ++c) a = fmaf(x[8 * c + lane], w[8 * c + lane], a);
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

// Dispatch plan (one workgroup): for each expert, its tokens in token order
// (an exclusive scan of the routing flags); rows[] holds the token of every
// dispatched row (experts concatenated in id order), slot[t][k] the row of
// token t's k-th expert, counts/offsets per expert.
__global__ __launch_bounds__(1024) void moe_plan_kernel(MoeParams p) {
    __shared__ int scan[1024];
    __shared__ int base_s;
    const int tid = threadIdx.x;
    if (tid == 0) base_s = 0;
    __syncthreads();
    for (int e = 0; e < p.n_expert; ++e) {
        const int start = base_s;
        for (int64_t t0 = 0; t0 < p.T; t0 += 1024) {
            const int64_t t = t0 + tid;
            int k = -1;
            if (t < p.T) k = p.top_idx[2 * t] == e ? 0 : p.top_idx[2 * t + 1] == e ? 1 : -1;
            const int f = k >= 0;
            scan[tid] = f;
            __syncthreads();
            for (int o = 1; o < 1024; o <<= 1) {  // inclusive Hillis-Steele scan
                const int v = tid >= o ? scan[tid - o] : 0;
                __syncthreads();
                scan[tid] += v;
                __syncthreads();
            }
            const int run = base_s;
            if (f) {
                const int r = run + scan[tid] - 1;
                p.rows[r] = (int32_t)t;
                p.slot[2 * t + k] = r;
            }
            __syncthreads();
            if (tid == 1023) base_s = run + scan[1023];
            __syncthreads();
        }
        if (tid == 0) {
            p.counts[e] = base_s - start;
            p.offsets[e] = start;
        }
        __syncthreads();
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

}  // namespace

int launch_moe_route(const MoeParams &p, hipStream_t s) {
    if (p.T <= 0 || p.T > 65535 || p.n_expert < 2 || p.n_expert > MOE_MAX_EXPERTS || !p.x || !p.router || p.h <= 0)
        return set_error(GAJE_ERR_INVALID_ARG, "moe route: bad arguments");
    hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)p.T), dim3(64 * MOE_MAX_EXPERTS), 0, s, p);
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

}  // namespace gaje
