// C ABI: error reporting, runtime helpers and the operator entry points.
// Model entry points live in model.cpp, the synthetic writer in synth.cpp.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "common.h"
#include "kernels.h"

namespace gaje {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error.clear(); }

size_t max_lds_per_block() {
    // The device's own limit (160 KiB per workgroup on gfx950).
    static std::atomic<size_t> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
    size_t v = cache[dev].load(std::memory_order_relaxed);
    if (!v) {
        int a = 0;
        if (hipDeviceGetAttribute(&a, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || a <= 0)
            a = 64 * 1024;
        v = std::min<size_t>((size_t)a, 160 * 1024);
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (!v) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

}  // namespace gaje

using namespace gaje;

namespace {

hipStream_t as_stream(void *s) { return (hipStream_t)s; }

GemvParams plain_gemv(int fmt, const void *w, const float *x, const float *bias, int64_t bias_len, float *y, int64_t n,
                      int64_t k) {
    GemvParams p;
    memset(&p, 0, sizeof p);
    p.w = (const uint8_t *)w;
    p.fmt = fmt;
    p.nb = (int32_t)(k / 32);
    p.rows_valid = n;
    p.N = n;
    p.K = k;
    p.x = x;
    p.h_scale = 1.0f;
    p.bias = bias;
    p.bias_len = bias ? bias_len : 0;
    p.mode = MODE_STORE;
    p.y = y;
    p.st_in = p.st_norm = p.st_a = p.st_b = ST_NONE;
    return p;
}

int check_dims(int64_t n, int64_t k) {
    if (n < 0 || k <= 0) return set_error(GAJE_ERR_INVALID_ARG, "invalid shape n=%lld k=%lld", (long long)n, (long long)k);
    if (k > (int64_t)1 << 30 || n > (int64_t)1 << 40) return set_error(GAJE_ERR_INVALID_ARG, "shape too large");
    return GAJE_OK;
}

}  // namespace

extern "C" const char *gaje_hip_last_error(void) { return g_last_error.c_str(); }

// ------------------------------------------------------------------ runtime --

extern "C" int gaje_hip_device_count(int *count) {
    if (!count) return set_error(GAJE_ERR_INVALID_ARG, "null argument");
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) {
        *count = 0;
        return GAJE_OK;
    }
    GAJE_HIP_CHECK(e);
    return GAJE_OK;
}

extern "C" int gaje_hip_set_device(int device) {
    GAJE_HIP_CHECK(hipSetDevice(device));
    return GAJE_OK;
}

extern "C" int gaje_hip_device_name(int device, char *buf, size_t buflen) {
    if (!buf || buflen == 0) return set_error(GAJE_ERR_INVALID_ARG, "null buffer");
    hipDeviceProp_t prop;
    GAJE_HIP_CHECK(hipGetDeviceProperties(&prop, device));
    snprintf(buf, buflen, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    return GAJE_OK;
}

extern "C" int gaje_hip_malloc(void **ptr, size_t bytes) {
    if (!ptr) return set_error(GAJE_ERR_INVALID_ARG, "null argument");
    *ptr = nullptr;
    if (bytes == 0) return GAJE_OK;
    GAJE_HIP_CHECK(hipMalloc(ptr, bytes));
    return GAJE_OK;
}

extern "C" int gaje_hip_free(void *ptr) {
    if (ptr) GAJE_HIP_CHECK(hipFree(ptr));
    return GAJE_OK;
}

extern "C" int gaje_hip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    if (bytes) GAJE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return GAJE_OK;
}

extern "C" int gaje_hip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    if (bytes) GAJE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return GAJE_OK;
}

extern "C" int gaje_hip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    if (bytes) GAJE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return GAJE_OK;
}

extern "C" int gaje_hip_memset(void *dst, int value, size_t bytes) {
    if (bytes) GAJE_HIP_CHECK(hipMemset(dst, value, bytes));
    return GAJE_OK;
}

extern "C" int gaje_hip_device_synchronize(void) {
    GAJE_HIP_CHECK(hipDeviceSynchronize());
    return GAJE_OK;
}

extern "C" int gaje_hip_stream_create(void **stream) {
    if (!stream) return set_error(GAJE_ERR_INVALID_ARG, "null argument");
    hipStream_t s;
    GAJE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = (void *)s;
    return GAJE_OK;
}

extern "C" int gaje_hip_stream_destroy(void *stream) {
    if (stream) GAJE_HIP_CHECK(hipStreamDestroy(as_stream(stream)));
    return GAJE_OK;
}

extern "C" int gaje_hip_stream_synchronize(void *stream) {
    GAJE_HIP_CHECK(hipStreamSynchronize(as_stream(stream)));
    return GAJE_OK;
}

extern "C" int gaje_hip_event_create(void **event) {
    if (!event) return set_error(GAJE_ERR_INVALID_ARG, "null argument");
    hipEvent_t e;
    GAJE_HIP_CHECK(hipEventCreate(&e));
    *event = (void *)e;
    return GAJE_OK;
}

extern "C" int gaje_hip_event_destroy(void *event) {
    if (event) GAJE_HIP_CHECK(hipEventDestroy((hipEvent_t)event));
    return GAJE_OK;
}

extern "C" int gaje_hip_event_record(void *event, void *stream) {
    GAJE_HIP_CHECK(hipEventRecord((hipEvent_t)event, as_stream(stream)));
    return GAJE_OK;
}

extern "C" int gaje_hip_event_synchronize(void *event) {
    GAJE_HIP_CHECK(hipEventSynchronize((hipEvent_t)event));
    return GAJE_OK;
}

extern "C" int gaje_hip_event_elapsed_ms(void *start, void *stop, float *ms) {
    if (!ms) return set_error(GAJE_ERR_INVALID_ARG, "null argument");
    GAJE_HIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return GAJE_OK;
}

// ------------------------------------------------------------- operators --

extern "C" int64_t gaje_hip_q4_0_packed_bytes(int64_t n, int64_t k) {
    if (n < 0 || k <= 0 || k % 32 != 0) return -1;
    return q4_0_packed_bytes(n, k);
}

extern "C" int gaje_hip_q4_0_pack(const void *blocks, void *packed, int64_t n, int64_t k, void *stream) {
    GAJE_TRY(check_dims(n, k));
    return launch_pack_q4_0((const uint8_t *)blocks, (uint8_t *)packed, n, k, as_stream(stream));
}

extern "C" int gaje_hip_q4_0_gemv(const void *packed, const float *x, const float *bias, int64_t bias_len, float *y,
                                  int64_t n, int64_t k, void *stream) {
    GAJE_TRY(check_dims(n, k));
    return launch_gemv(plain_gemv(FMT_Q4_0, packed, x, bias, bias_len, y, n, k), as_stream(stream));
}

extern "C" int gaje_hip_q4_0_gemv_tol(const void *packed, const float *x, const float *bias, int64_t bias_len,
                                      float *y, int64_t n, int64_t k, void *stream) {
    clear_error();
    GAJE_TRY(check_dims(n, k));
    GemvParams p = plain_gemv(FMT_Q4_0, packed, x, bias, bias_len, y, n, k);
    p.tol = 1;
    return launch_gemv(p, as_stream(stream));
}

extern "C" int gaje_hip_q4_0_gemv_blocks(const void *blocks, const float *x, const float *bias, int64_t bias_len,
                                         float *y, int64_t n, int64_t k, void *stream) {
    clear_error();
    GAJE_TRY(check_dims(n, k));
    return launch_q4_0_gemv_blocks((const uint8_t *)blocks, x, bias, bias_len, y, n, k, as_stream(stream));
}

extern "C" int gaje_hip_q4_0_gemm(const void *packed, const float *X, const float *bias, int64_t bias_len, float *Y,
                                  int64_t m, int64_t n, int64_t k, void *stream) {
    GAJE_TRY(check_dims(n, k));
    if (m < 0 || (m > 0 && (!X || !Y))) return set_error(GAJE_ERR_INVALID_ARG, "bad gemm arguments");
    for (int64_t r = 0; r < m; ++r)
        GAJE_TRY(launch_gemv(plain_gemv(FMT_Q4_0, packed, X + r * k, bias, bias_len, Y + r * n, n, k), as_stream(stream)));
    return GAJE_OK;
}

namespace {

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Workspace of gaje_hip_q4_0_gemm_mfma: activation row exponents, the f16
// activation plane (hi | lo per block, rows padded to gemm_bs_plane_rows),
// the two block-sum planes, split-K partials.
struct GemmWorkspace {
    int *ex;
    uint16_t *xh, *sh, *sl, *mins, *wf;
    float *wsc;
    int64_t plane_rows, ldsum;
    float *part;
    size_t bytes;
};

GemmWorkspace gemm_workspace(char *base, int64_t m, int64_t n, int64_t k, const GemmBsPlan &pl) {
    GemmWorkspace w{};
    size_t off = 0;
    w.ex = (int *)(base + off);
    off = align256(off + (size_t)m * 4);
    w.plane_rows = gemm_bs_plane_rows(m);
    w.xh = (uint16_t *)(base + off);
    off = align256(off + (size_t)(w.plane_rows * 2 * k) * 2);
    w.ldsum = gemm_bs_sum_cols(k);
    w.sh = (uint16_t *)(base + off);
    off = align256(off + (size_t)(m * w.ldsum) * 2);
    w.sl = (uint16_t *)(base + off);
    off = align256(off + (size_t)(m * w.ldsum) * 2);
    w.part = (float *)(base + off);
    off = align256(off + (size_t)pl.part_floats * 4);
    w.mins = (uint16_t *)(base + off);  // [n][ldsum]: the weight rows' block mins
    off = align256(off + (size_t)(n * w.ldsum) * 2);
    w.wf = (uint16_t *)(base + off);    // the weight rows' code fragments and scales
    off = align256(off + (size_t)q4_frag_halves(n, k) * 2);
    w.wsc = (float *)(base + off);
    off = align256(off + (size_t)q4_frag_scale_floats(n, k) * 4);
    w.bytes = off;
    return w;
}

}  // namespace

extern "C" int64_t gaje_hip_q4_0_gemm_mfma_workspace(int64_t m, int64_t n, int64_t k) {
    if (m < 0 || n <= 0 || k <= 0 || k % 32 != 0) return -1;
    if (m == 0) return 0;
    return (int64_t)gemm_workspace(nullptr, m, n, k, plan_gemm_q4_bs(m, n, k)).bytes;
}

extern "C" int gaje_hip_q4_0_gemm_mfma(const void *packed, const float *X, const float *bias, int64_t bias_len,
                                       float *Y, int64_t m, int64_t n, int64_t k, void *workspace,
                                       int64_t workspace_bytes, void *stream) {
    GAJE_TRY(check_dims(n, k));
    if (k % 32 || m < 0 || (m > 0 && (!X || !Y || !packed || !workspace)) || bias_len < 0 || (bias_len > 0 && !bias))
        return set_error(GAJE_ERR_INVALID_ARG, "bad gemm arguments");
    if (m == 0 || n == 0) return GAJE_OK;
    if (((uintptr_t)workspace & 15) != 0) return set_error(GAJE_ERR_INVALID_ARG, "gemm workspace must be 16-byte aligned");
    const GemmBsPlan pl = plan_gemm_q4_bs(m, n, k);
    const GemmWorkspace w = gemm_workspace((char *)workspace, m, n, k, pl);
    if ((int64_t)w.bytes > workspace_bytes)
        return set_error(GAJE_ERR_INVALID_ARG, "gemm workspace of %lld bytes is smaller than the %zu needed",
                         (long long)workspace_bytes, w.bytes);
    hipStream_t s = as_stream(stream);
    SplitParams sp{};
    sp.x = X;
    sp.ldx = k;
    sp.xh = w.xh;
    sp.ldh = 2 * k;
    sp.ex = w.ex;
    sp.M = m;
    sp.K = k;
    sp.sh = w.sh;
    sp.sl = w.sl;
    sp.ldsum = w.ldsum;
    GAJE_TRY(launch_split_rows(sp, s));
    GAJE_TRY(launch_q4_mins((const uint8_t *)packed, n, k, w.mins, w.ldsum, s));
    GAJE_TRY(launch_q4_frags((const uint8_t *)packed, n, k, w.wf, w.wsc, s));
    GemmBsParams p{};
    p.wf = w.wf;
    p.wsc = w.wsc;
    p.nbp4 = q4_frag_nbp4(k);
    p.mins = w.mins;
    p.ldm = w.ldsum;
    p.xh = w.xh;
    p.plane_rows = w.plane_rows;
    p.sh = w.sh;
    p.sl = w.sl;
    p.ex = w.ex;
    p.ldh = 2 * k;
    p.ldsum = w.ldsum;
    p.bias = bias;
    p.bias_len = bias_len;
    p.y = Y;
    p.ldy = n;
    p.part = w.part;
    p.M = m;
    p.N = n;
    p.nb = (int32_t)(k / 32);
    return launch_gemm_q4_bs(p, pl, s);
}

namespace {

// Scratch of gaje_hip_q4_0_gemm_mfma_noalloc: a file-scope device array (each
// GPU holds its own copy for the life of the process), whose address is taken
// once per device with that device current and kept; host code uses only
// that address, never the array's name.
static __device__ __align__(256) uint8_t scratch[GAJE_NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
std::atomic<void *> g_scratch_ptr[NOALLOC_MAX_DEVICES];

int scratch_ptr(void **out) {
    int dev = 0;
    GAJE_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return set_error(GAJE_ERR_UNSUPPORTED, "device %d beyond the %d this build's scratch table holds", dev,
                         NOALLOC_MAX_DEVICES);
    void *p = g_scratch_ptr[dev].load();
    if (!p) {
        GAJE_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch_ptr[dev].store(p);
    }
    *out = p;
    return GAJE_OK;
}

}  // namespace

extern "C" int gaje_hip_q4_0_gemm_mfma_noalloc(const void *packed, const float *X, const float *bias, int64_t bias_len,
                                               float *Y, int64_t m, int64_t n, int64_t k, void *stream) {
    clear_error();
    GAJE_TRY(check_dims(n, k));
    if (k % 32 || m < 0) return set_error(GAJE_ERR_INVALID_ARG, "bad gemm arguments");
    if (m == 0 || n == 0) return GAJE_OK;  // an empty product, as gaje_hip_q4_0_gemm_mfma returns it
    const int64_t need = gaje_hip_q4_0_gemm_mfma_workspace(m, n, k);
    if (need < 0) return set_error(GAJE_ERR_INVALID_ARG, "bad gemm arguments");
    if (need > GAJE_NOALLOC_SCRATCH_BYTES)
        return set_error(GAJE_ERR_UNSUPPORTED,
                         "gemm of %lld x %lld x %lld needs %lld bytes of scratch, beyond the %lld this entry point holds",
                         (long long)m, (long long)n, (long long)k, (long long)need,
                         (long long)GAJE_NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    GAJE_TRY(scratch_ptr(&ws));
    return gaje_hip_q4_0_gemm_mfma(packed, X, bias, bias_len, Y, m, n, k, ws, GAJE_NOALLOC_SCRATCH_BYTES, stream);
}

namespace {

// Workspace of gaje_hip_moe_ffn.
struct MoeWorkspace {
    int *ew_gu, *ew_dn;              // [E][2 ffn], [E][h] weight row exponents
    int32_t *top_idx, *rows, *slot, *counts, *offsets;
    float *top_w;
    uint16_t *xh, *xl;               // [2T][max(h, ffn)] planes
    int *ex;                         // [2T]
    float *GU, *Y, *part;            // [2T][2 ffn], [2T][h], split-K partials
    int64_t part_floats;
    size_t bytes;
};

MoeWorkspace moe_workspace(char *base, int64_t T, int64_t h, int64_t ffn, int64_t E) {
    MoeWorkspace w{};
    const int64_t R = 2 * T, kmax = std::max(h, ffn);
    int64_t part = 0;
    part = std::max(plan_gemm_q4_grouped(R, E, 2 * ffn, h).part_floats, plan_gemm_q4_grouped(R, E, h, ffn).part_floats);
    w.part_floats = part;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char *p = base + off;
        off = align256(off + bytes);
        return p;
    };
    w.ew_gu = (int *)take((size_t)(E * 2 * ffn) * 4);
    w.ew_dn = (int *)take((size_t)(E * h) * 4);
    w.top_idx = (int32_t *)take((size_t)R * 4);
    w.top_w = (float *)take((size_t)R * 4);
    w.rows = (int32_t *)take((size_t)R * 4);
    w.slot = (int32_t *)take((size_t)R * 4);
    w.counts = (int32_t *)take((size_t)E * 4);
    w.offsets = (int32_t *)take((size_t)E * 4);
    w.xh = (uint16_t *)take((size_t)(R * kmax) * 2);
    w.xl = (uint16_t *)take((size_t)(R * kmax) * 2);
    w.ex = (int *)take((size_t)R * 4);
    w.GU = (float *)take((size_t)(R * 2 * ffn) * 4);
    w.Y = (float *)take((size_t)(R * h) * 4);
    w.part = (float *)take((size_t)part * 4);
    w.bytes = off;
    return w;
}

int check_moe(int64_t T, int64_t h, int64_t ffn, int64_t E) {
    if (T <= 0 || T > 65535 || h <= 0 || h % 32 || ffn <= 0 || ffn % 32 || E < 2 || E > MOE_MAX_EXPERTS)
        return set_error(GAJE_ERR_INVALID_ARG, "moe: T %lld (1..65535), h %lld and ffn %lld (multiples of 32), %lld experts (2..%d)",
                         (long long)T, (long long)h, (long long)ffn, (long long)E, MOE_MAX_EXPERTS);
    return GAJE_OK;
}

}  // namespace

extern "C" int64_t gaje_hip_moe_ffn_workspace(int64_t T, int64_t h, int64_t ffn, int64_t n_expert) {
    if (check_moe(T, h, ffn, n_expert) != GAJE_OK) return -1;
    return (int64_t)moe_workspace(nullptr, T, h, ffn, n_expert).bytes;
}

extern "C" int gaje_hip_moe_ffn(const float *x, int64_t T, int64_t h, const float *router, int64_t n_expert,
                                const void *const *gate_up, const void *const *down, int64_t ffn, float *y,
                                int32_t *top_idx, float *top_w, void *workspace, int64_t workspace_bytes,
                                void *stream) {
    GAJE_TRY(check_moe(T, h, ffn, n_expert));
    if (!x || !router || !gate_up || !down || !y || !workspace) return set_error(GAJE_ERR_INVALID_ARG, "moe: null argument");
    for (int64_t e = 0; e < n_expert; ++e)
        if (!gate_up[e] || !down[e]) return set_error(GAJE_ERR_INVALID_ARG, "moe: expert %lld has no weights", (long long)e);
    const MoeWorkspace w = moe_workspace((char *)workspace, T, h, ffn, n_expert);
    if ((int64_t)w.bytes > workspace_bytes)
        return set_error(GAJE_ERR_INVALID_ARG, "moe workspace of %lld bytes is smaller than the %zu needed",
                         (long long)workspace_bytes, w.bytes);
    hipStream_t s = as_stream(stream);
    const int64_t R = 2 * T;
    GAJE_TRY(launch_q4_row_exponents_batch((const uint8_t *const *)gate_up, (int)n_expert, 2 * ffn, h, w.ew_gu, s));
    GAJE_TRY(launch_q4_row_exponents_batch((const uint8_t *const *)down, (int)n_expert, h, ffn, w.ew_dn, s));
    MoeParams mp{};
    mp.x = x;
    mp.ldx = h;
    mp.T = T;
    mp.h = h;
    mp.router = router;
    mp.n_expert = (int32_t)n_expert;
    mp.top_idx = w.top_idx;
    mp.top_w = w.top_w;
    mp.rows = w.rows;
    mp.slot = w.slot;
    mp.counts = w.counts;
    mp.offsets = w.offsets;
    mp.y = y;
    mp.ldy = h;
    GAJE_TRY(launch_moe_route(mp, s));

    // gate_up of every expert over its gathered tokens
    SplitParams sp{};
    sp.x = x;
    sp.ldx = h;
    sp.xh = w.xh;
    sp.xl = w.xl;
    sp.ldh = h;
    sp.ex = w.ex;
    sp.M = R;
    sp.K = h;
    sp.rows = w.rows;
    GAJE_TRY(launch_split_rows(sp, s));
    // one grouped launch per product: every expert's rows (counts and offsets
    // stay on the device; an expert holds at most T rows)
    auto gemm = [&](const void *const *wt, const int *ew, int64_t N, int64_t K, float *Y) {
        GemmQ4Params p{};
        p.xh = w.xh;
        p.xl = w.xl;
        p.ex = w.ex;
        p.ldh = K;
        p.y = Y;
        p.ldy = N;
        p.part = w.part;
        p.M = R;
        p.N = N;
        p.nb = (int32_t)(K / 32);
        p.g_counts = w.counts;
        p.g_offsets = w.offsets;
        p.g_groups = (int32_t)n_expert;
        p.g_mtiles = (int32_t)((T + 127) / 128);
        for (int64_t e = 0; e < n_expert; ++e) {
            p.gw[e] = (const uint8_t *)wt[e];
            p.gew[e] = ew + e * N;
        }
        return launch_gemm_q4(p, plan_gemm_q4_grouped(R, n_expert, N, K), s);
    };
    GAJE_TRY(gemm(gate_up, w.ew_gu, 2 * ffn, h, w.GU));
    // swiglu of every dispatched row, then down
    sp = SplitParams{};
    sp.x = w.GU;
    sp.up = w.GU + ffn;
    sp.ldx = 2 * ffn;
    sp.h_scale = 1.0f;
    sp.xh = w.xh;
    sp.xl = w.xl;
    sp.ldh = ffn;
    sp.ex = w.ex;
    sp.M = R;
    sp.K = ffn;
    sp.st_a = sp.st_b = -1;
    GAJE_TRY(launch_split_rows(sp, s));
    GAJE_TRY(gemm(down, w.ew_dn, h, ffn, w.Y));
    GAJE_TRY(launch_moe_combine(mp, w.Y, s));
    if (top_idx) GAJE_HIP_CHECK(hipMemcpyAsync(top_idx, w.top_idx, (size_t)R * 4, hipMemcpyDeviceToDevice, s));
    if (top_w) GAJE_HIP_CHECK(hipMemcpyAsync(top_w, w.top_w, (size_t)R * 4, hipMemcpyDeviceToDevice, s));
    return GAJE_OK;
}

namespace {

// The prepared experts of gaje_hip_moe_prepare: for each of the two products
// (gate_up: N = 2 ffn, K = h; down: N = h, K = ffn) every expert's code
// fragments, fragment scales and dense block mins (the block-scaled product's
// weight operands), one expert after the other at fixed strides.
struct MoePrepared {
    int64_t wf_stride[2], wsc_stride[2], mins_stride[2], ldm[2];
    uint16_t *wf[2];
    float *wsc[2];
    uint16_t *mins[2];
    size_t bytes;
};

MoePrepared moe_prepared(char *base, int64_t h, int64_t ffn, int64_t E) {
    MoePrepared w{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char *p = base + off;
        off = align256(off + bytes);
        return p;
    };
    const int64_t NN[2] = {2 * ffn, h}, KK[2] = {h, ffn};
    for (int i = 0; i < 2; ++i) {
        w.ldm[i] = gemm_bs_sum_cols(KK[i]);
        w.wf_stride[i] = (q4_frag_halves(NN[i], KK[i]) + 511) / 512 * 512;
        w.wsc_stride[i] = (q4_frag_scale_floats(NN[i], KK[i]) + 63) / 64 * 64;
        w.mins_stride[i] = (NN[i] * w.ldm[i] + 127) / 128 * 128;
        w.wf[i] = (uint16_t *)take((size_t)(E * w.wf_stride[i]) * 2);
        w.wsc[i] = (float *)take((size_t)(E * w.wsc_stride[i]) * 4);
        w.mins[i] = (uint16_t *)take((size_t)(E * w.mins_stride[i]) * 2);
    }
    w.bytes = off;
    return w;
}

// Workspace of gaje_hip_moe_ffn_prepared: the routing, the block-scaled
// activation planes of the dispatched rows, the two products' results and
// their split-K partials.
struct MoeBsWorkspace {
    int32_t *top_idx, *rows, *slot, *counts, *offsets;
    float *top_w;
    uint16_t *xh, *sh, *sl;          // [plane_rows][2 kmax], [2T][ldsum] x 2
    int64_t plane_rows, ldsum;
    int *ex;                         // [2T]
    float *GU, *Y, *part;            // [2T][2 ffn], [2T][h], split-K partials
    GemmBsPlan pgu, pdn;
    size_t bytes;
};

MoeBsWorkspace moe_bs_workspace(char *base, int64_t T, int64_t h, int64_t ffn, int64_t E) {
    MoeBsWorkspace w{};
    const int64_t R = 2 * T, kmax = std::max(h, ffn);
    w.pgu = plan_gemm_q4_bs_grouped(R, E, T, 2 * ffn, h);
    w.pdn = plan_gemm_q4_bs_grouped(R, E, T, h, ffn);
    const int64_t mt = BS_WR_ROWS * std::max(w.pgu.waves, w.pdn.waves);
    const int64_t gm = std::max(w.pgu.mtiles, w.pdn.mtiles) / E;  // row tiles per group
    w.plane_rows = gemm_bs_plane_rows(R + gm * mt);
    w.ldsum = gemm_bs_sum_cols(kmax);
    const int64_t part = std::max(w.pgu.part_floats, w.pdn.part_floats);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char *p = base + off;
        off = align256(off + bytes);
        return p;
    };
    w.top_idx = (int32_t *)take((size_t)R * 4);
    w.top_w = (float *)take((size_t)R * 4);
    w.rows = (int32_t *)take((size_t)R * 4);
    w.slot = (int32_t *)take((size_t)R * 4);
    w.counts = (int32_t *)take((size_t)E * 4);
    w.offsets = (int32_t *)take((size_t)E * 4);
    w.xh = (uint16_t *)take((size_t)(w.plane_rows * 2 * kmax) * 2);
    w.sh = (uint16_t *)take((size_t)(R * w.ldsum) * 2);
    w.sl = (uint16_t *)take((size_t)(R * w.ldsum) * 2);
    w.ex = (int *)take((size_t)R * 4);
    w.GU = (float *)take((size_t)(R * 2 * ffn) * 4);
    w.Y = (float *)take((size_t)(R * h) * 4);
    w.part = (float *)take((size_t)part * 4);
    w.bytes = off;
    return w;
}

}  // namespace

extern "C" int64_t gaje_hip_moe_prepared_bytes(int64_t h, int64_t ffn, int64_t n_expert) {
    clear_error();
    if (check_moe(1, h, ffn, n_expert) != GAJE_OK) return -1;
    return (int64_t)moe_prepared(nullptr, h, ffn, n_expert).bytes;
}

extern "C" int gaje_hip_moe_prepare(const void *const *gate_up, const void *const *down, int64_t h, int64_t ffn,
                                    int64_t n_expert, void *prepared, int64_t prepared_bytes, void *stream) {
    clear_error();
    GAJE_TRY(check_moe(1, h, ffn, n_expert));
    if (!gate_up || !down || !prepared) return set_error(GAJE_ERR_INVALID_ARG, "moe prepare: null argument");
    for (int64_t e = 0; e < n_expert; ++e)
        if (!gate_up[e] || !down[e]) return set_error(GAJE_ERR_INVALID_ARG, "moe prepare: expert %lld has no weights", (long long)e);
    const MoePrepared w = moe_prepared((char *)prepared, h, ffn, n_expert);
    if ((int64_t)w.bytes > prepared_bytes)
        return set_error(GAJE_ERR_INVALID_ARG, "moe prepare: %lld bytes given, %zu needed", (long long)prepared_bytes, w.bytes);
    if ((uintptr_t)prepared & 255) return set_error(GAJE_ERR_INVALID_ARG, "moe prepare: the buffer must be 256-byte aligned");
    hipStream_t s = as_stream(stream);
    const int64_t NN[2] = {2 * ffn, h}, KK[2] = {h, ffn};
    for (int i = 0; i < 2; ++i)
        for (int64_t e = 0; e < n_expert; ++e) {
            const uint8_t *pk = (const uint8_t *)(i == 0 ? gate_up[e] : down[e]);
            GAJE_TRY(launch_q4_frags(pk, NN[i], KK[i], w.wf[i] + e * w.wf_stride[i], w.wsc[i] + e * w.wsc_stride[i], s));
            GAJE_TRY(launch_q4_mins(pk, NN[i], KK[i], w.mins[i] + e * w.mins_stride[i], w.ldm[i], s));
        }
    return GAJE_OK;
}

extern "C" int64_t gaje_hip_moe_ffn_prepared_workspace(int64_t T, int64_t h, int64_t ffn, int64_t n_expert) {
    clear_error();
    if (check_moe(T, h, ffn, n_expert) != GAJE_OK) return -1;
    return (int64_t)moe_bs_workspace(nullptr, T, h, ffn, n_expert).bytes;
}

extern "C" int gaje_hip_moe_ffn_prepared(const float *x, int64_t T, int64_t h, const float *router, int64_t n_expert,
                                         const void *prepared, int64_t ffn, float *y, int32_t *top_idx, float *top_w,
                                         void *workspace, int64_t workspace_bytes, void *stream) {
    clear_error();
    GAJE_TRY(check_moe(T, h, ffn, n_expert));
    if (!x || !router || !prepared || !y || !workspace) return set_error(GAJE_ERR_INVALID_ARG, "moe: null argument");
    if ((uintptr_t)prepared & 255) return set_error(GAJE_ERR_INVALID_ARG, "moe: the prepared experts must be 256-byte aligned");
    const MoePrepared pw = moe_prepared((char *)prepared, h, ffn, n_expert);
    const MoeBsWorkspace w = moe_bs_workspace((char *)workspace, T, h, ffn, n_expert);
    if ((int64_t)w.bytes > workspace_bytes)
        return set_error(GAJE_ERR_INVALID_ARG, "moe workspace of %lld bytes is smaller than the %zu needed",
                         (long long)workspace_bytes, w.bytes);
    hipStream_t s = as_stream(stream);
    const int64_t R = 2 * T;
    MoeParams mp{};
    mp.x = x;
    mp.ldx = h;
    mp.T = T;
    mp.h = h;
    mp.router = router;
    mp.n_expert = (int32_t)n_expert;
    mp.top_idx = w.top_idx;
    mp.top_w = w.top_w;
    mp.rows = w.rows;
    mp.slot = w.slot;
    mp.counts = w.counts;
    mp.offsets = w.offsets;
    mp.y = y;
    mp.ldy = h;
    GAJE_TRY(launch_moe_route(mp, s));

    // the dispatched rows (gathered in expert order) in the block-scaled layout
    SplitParams sp{};
    sp.x = x;
    sp.ldx = h;
    sp.xh = w.xh;
    sp.ldh = 2 * h;
    sp.sh = w.sh;
    sp.sl = w.sl;
    sp.ldsum = w.ldsum;
    sp.ex = w.ex;
    sp.M = R;
    sp.K = h;
    sp.rows = w.rows;
    GAJE_TRY(launch_split_rows(sp, s));
    // one grouped launch per product over every expert's rows (counts and
    // offsets stay on the device; an expert holds at most T rows)
    auto gemm = [&](int i, const GemmBsPlan &pl, int64_t N, int64_t K, float *Y) {
        GemmBsParams p{};
        p.wf = pw.wf[i];
        p.wsc = pw.wsc[i];
        p.nbp4 = q4_frag_nbp4(K);
        p.mins = pw.mins[i];
        p.ldm = pw.ldm[i];
        p.xh = w.xh;
        p.plane_rows = w.plane_rows;
        p.sh = w.sh;
        p.sl = w.sl;
        p.ex = w.ex;
        p.ldh = 2 * K;
        p.ldsum = w.ldsum;
        p.y = Y;
        p.ldy = N;
        p.part = w.part;
        p.M = R;
        p.N = N;
        p.nb = (int32_t)(K / 32);
        p.g_counts = w.counts;
        p.g_offsets = w.offsets;
        p.g_groups = (int32_t)n_expert;
        p.g_mtiles = (int32_t)(pl.mtiles / n_expert);
        p.g_wf_stride = pw.wf_stride[i];
        p.g_wsc_stride = pw.wsc_stride[i];
        p.g_mins_stride = pw.mins_stride[i];
        p.defer_reduce = i == 1 && pl.splits > 1;  // down: the combine sums its partials
        return launch_gemm_q4_bs(p, pl, s);
    };
    GAJE_TRY(gemm(0, w.pgu, 2 * ffn, h, w.GU));
    // swiglu of every dispatched row into the planes, then down
    sp = SplitParams{};
    sp.x = w.GU;
    sp.up = w.GU + ffn;
    sp.ldx = 2 * ffn;
    sp.h_scale = 1.0f;
    sp.xh = w.xh;
    sp.ldh = 2 * ffn;
    sp.sh = w.sh;
    sp.sl = w.sl;
    sp.ldsum = w.ldsum;
    sp.ex = w.ex;
    sp.M = R;
    sp.K = ffn;
    sp.st_a = sp.st_b = -1;
    GAJE_TRY(launch_split_rows(sp, s));
    GAJE_TRY(gemm(1, w.pdn, h, ffn, w.Y));
    if (w.pdn.splits > 1)
        GAJE_TRY(launch_moe_combine_split(mp, w.part, w.pdn.splits, R, s));
    else
        GAJE_TRY(launch_moe_combine(mp, w.Y, s));
    if (top_idx) GAJE_HIP_CHECK(hipMemcpyAsync(top_idx, w.top_idx, (size_t)R * 4, hipMemcpyDeviceToDevice, s));
    if (top_w) GAJE_HIP_CHECK(hipMemcpyAsync(top_w, w.top_w, (size_t)R * 4, hipMemcpyDeviceToDevice, s));
    return GAJE_OK;
}

extern "C" int gaje_hip_lut4_gemv(const uint8_t *codes, const float *lut, int64_t lut_len, const float *x,
                                  const float *bias, int64_t bias_len, float *y, int64_t n, int64_t k, void *stream) {
    GAJE_TRY(check_dims(n, k));
    GemvParams p = plain_gemv(FMT_LUT4, codes, x, bias, bias_len, y, n, k);
    const int64_t per_row = (k / 32) * 16;
    p.lut = lut;
    if (lut_len == 16) {
        p.lut_block_stride = 0;
        p.lut_rows_own = 0;
    } else if (per_row > 0 && lut_len >= per_row) {
        p.lut_block_stride = 16;
        p.lut_rows_own = lut_len == per_row ? 0 : lut_len / per_row;
    } else {
        return set_error(GAJE_ERR_INVALID_ARG, "lut_len %lld is neither 16 nor >= k/32*16", (long long)lut_len);
    }
    return launch_gemv(p, as_stream(stream));
}

extern "C" int gaje_hip_2bit_gemv(const uint8_t *codes, const float *centroids, int64_t c_len, const float *modulation,
                                  const float *x, const float *bias, int64_t bias_len, float *y, int64_t n, int64_t k,
                                  void *stream) {
    GAJE_TRY(check_dims(n, k));
    if (k % 32) return set_error(GAJE_ERR_UNSUPPORTED, "2-bit rows need k %% 32 == 0 (got %lld)", (long long)k);
    GemvParams p = plain_gemv(FMT_G2, codes, x, bias, bias_len, y, n, k);
    const int64_t per_row = (k / 32) * 4;
    p.lut = centroids;
    if (c_len == 0) {
        p.rows_valid = 0;  // compute_single_row: no centroids, the dot is 0 (linear/forward.rs:47)
    } else if (c_len == 4) {
        p.lut_block_stride = 0;
        p.lut_rows_own = 0;
    } else if (c_len >= per_row) {
        p.lut_block_stride = 4;
        p.lut_rows_own = c_len == per_row ? 0 : c_len / per_row;
    } else {
        return set_error(GAJE_ERR_INVALID_ARG, "c_len %lld is neither 0, 4 nor >= k/32*4", (long long)c_len);
    }
    if (c_len && !centroids) return set_error(GAJE_ERR_INVALID_ARG, "2-bit gemv: null centroids");
    if (modulation) {
        p.g2_modulated = 1;
        for (int i = 0; i < 4; ++i) p.g2_mod[i] = modulation[i];
    }
    return launch_gemv(p, as_stream(stream));
}

extern "C" int gaje_hip_f32_gemv(const float *w, const float *x, const float *bias, int64_t bias_len, float *y,
                                 int64_t n, int64_t k, void *stream) {
    GAJE_TRY(check_dims(n, k));
    GemvParams p = plain_gemv(FMT_F32, w, x, bias, bias_len, y, n, k);
    p.nontemporal = 1;
    return launch_gemv(p, as_stream(stream));
}

extern "C" int gaje_hip_q4_0_dequant(const void *blocks, float *out, int64_t nblocks, void *stream) {
    return launch_dequant_q4_0((const uint8_t *)blocks, out, nblocks, as_stream(stream));
}

extern "C" int gaje_hip_q8_0_dequant(const void *blocks, float *out, int64_t nblocks, void *stream) {
    return launch_dequant_q8_0((const uint8_t *)blocks, out, nblocks, as_stream(stream));
}

extern "C" int64_t gaje_hip_q8_0_packed_bytes(int64_t n, int64_t k) {
    if (n < 0 || k <= 0 || k % 32 != 0) return -1;
    return q8_0_packed_bytes(n, k);
}

extern "C" int gaje_hip_q8_0_pack(const void *blocks, void *packed, int64_t n, int64_t k, void *stream) {
    GAJE_TRY(check_dims(n, k));
    return launch_pack_q8_0((const uint8_t *)blocks, (uint8_t *)packed, n, k, as_stream(stream));
}

extern "C" int gaje_hip_q8_0_gemv(const void *packed, const float *x, const float *bias, int64_t bias_len, float *y,
                                  int64_t n, int64_t k, void *stream) {
    GAJE_TRY(check_dims(n, k));
    return launch_gemv(plain_gemv(FMT_Q8_0, packed, x, bias, bias_len, y, n, k), as_stream(stream));
}

extern "C" int gaje_hip_rmsnorm(const float *x, const float *w, float eps, float *y, int64_t n, void *stream) {
    return launch_rmsnorm(x, w, eps, y, n, as_stream(stream));
}

extern "C" int gaje_hip_swiglu(const float *gate, const float *up, float *out, int64_t n, void *stream) {
    return launch_swiglu(gate, up, out, n, as_stream(stream));
}

extern "C" int gaje_hip_expf(const float *x, float *y, int64_t n, void *stream) {
    return launch_expf(x, y, n, as_stream(stream));
}

extern "C" int gaje_hip_attention(const float *q, const float *k_cache, const float *v_cache, int64_t seq_len,
                                  int64_t capacity, int n_head, int n_head_kv, int head_dim, float *out,
                                  void *stream) {
    AttnParams p{};
    memset(&p, 0, sizeof p);
    p.q = q;
    p.k_cache = k_cache;
    p.v_cache = v_cache;
    p.kv_head_stride = capacity * head_dim;
    p.n_head = n_head;
    p.n_head_kv = n_head_kv;
    p.head_dim = head_dim;
    p.kv_cap = capacity;
    p.out = out;
    p.st = nullptr;
    p.ctx = seq_len;
    return launch_attention(p, as_stream(stream));
}

extern "C" int gaje_hip_kwta(float *scores, int64_t n, int64_t k, void *stream) {
    return launch_kwta(scores, n, k, nullptr, as_stream(stream));
}

extern "C" int gaje_hip_argmax(const float *x, int64_t n, uint32_t *idx, void *stream) {
    return launch_argmax(x, n, idx, as_stream(stream));
}

namespace {

// Average device time per launch of `per_pass` launches issued by launch_all on
// stream s, repeated until `iters` launches ran: captured once in a HIP graph
// and replayed, timed with HIP events on s.  With GAJE_HIP_PROFILE set the
// launches are issued one by one instead, so that a kernel tracer sees each.
template <class F>
int time_launches(F &&launch_all, int per_pass, int iters, hipStream_t s, float *avg_ms) {
    int rc = launch_all();  // warm-up, eager (validates the arguments)
    const int reps = (iters + per_pass - 1) / per_pass;
    // untimed passes right before the timed ones, ~640 launches: the core clock
    // climbs for ~20 ms after the GPU has idled (here: while the graph is
    // captured and instantiated), and a launch-bound or VALU-bound kernel's
    // rate follows it
    const int warm = (640 + per_pass - 1) / per_pass;
    float ms = 0.0f;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    if (rc == GAJE_OK && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
        rc = set_error(GAJE_ERR_HIP, "event create failed");
    if (rc == GAJE_OK && getenv("GAJE_HIP_PROFILE")) {
        for (int r = 0; r < warm && rc == GAJE_OK; ++r) rc = launch_all();
        (void)hipEventRecord(e0, s);
        for (int r = 0; r < reps && rc == GAJE_OK; ++r) rc = launch_all();
        (void)hipEventRecord(e1, s);
    } else if (rc == GAJE_OK) {
        if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) {
            rc = set_error(GAJE_ERR_HIP, "graph capture failed");
        } else {
            rc = launch_all();
            if (hipStreamEndCapture(s, &g) != hipSuccess && rc == GAJE_OK)
                rc = set_error(GAJE_ERR_HIP, "graph capture failed");
        }
        if (rc == GAJE_OK && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess)
            rc = set_error(GAJE_ERR_HIP, "graph instantiate failed");
        if (rc == GAJE_OK) {
            for (int r = 0; r < warm; ++r) (void)hipGraphLaunch(ge, s);  // (the first uploads the graph)
            (void)hipEventRecord(e0, s);
            for (int r = 0; r < reps; ++r) (void)hipGraphLaunch(ge, s);
            (void)hipEventRecord(e1, s);
        }
    }
    if (rc == GAJE_OK) {
        if (hipEventSynchronize(e1) != hipSuccess) rc = set_error(GAJE_ERR_HIP, "benchmark replay failed");
        else (void)hipEventElapsedTime(&ms, e0, e1);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (ge) (void)hipGraphExecDestroy(ge);
    if (g) (void)hipGraphDestroy(g);
    (void)hipStreamSynchronize(s);
    GAJE_TRY(rc);
    *avg_ms = ms / (float)(reps * per_pass);
    return GAJE_OK;
}

}  // namespace

extern "C" int gaje_hip_bench_gemv(int format, const void *w_base, size_t copy_stride, const float *lut_base,
                                   size_t lut_stride, int copies, const float *x, float *y, int64_t n, int64_t k,
                                   int iters, float *avg_ms) {
    clear_error();
    GAJE_TRY(check_dims(n, k));
    if (!avg_ms || copies <= 0 || iters <= 0 || !w_base || (format == FMT_LUT4 && !lut_base))
        return set_error(GAJE_ERR_INVALID_ARG, "bad benchmark arguments");
    // format 3: the Q4_0 matvec in tolerance mode (gaje_hip_q4_0_gemv_tol)
    const bool tol = format == 3;
    if (tol) format = FMT_Q4_0;
    if (format != FMT_F32 && format != FMT_Q4_0 && format != FMT_LUT4)
        return set_error(GAJE_ERR_INVALID_ARG, "unknown format %d", format);
    hipStream_t s;
    GAJE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    // one pass launches `per_pass` matvecs cycling through the copies (at least
    // 128, so that a replayed graph is not dominated by its own launch cost)
    const int per_pass = copies < 128 ? ((128 + copies - 1) / copies) * copies : copies;
    auto launch_all = [&]() -> int {
        for (int i = 0; i < per_pass; ++i) {
            const int c = i % copies;
            GemvParams p = plain_gemv(format, (const uint8_t *)w_base + (size_t)c * copy_stride, x, nullptr, 0, y, n, k);
            if (format == FMT_LUT4) {
                p.lut = (const float *)((const uint8_t *)lut_base + (size_t)c * lut_stride);
                p.lut_block_stride = 16;
                p.lut_rows_own = n;
            }
            if (format == FMT_F32) p.nontemporal = 1;
            p.tol = tol ? 1 : 0;
            GAJE_TRY(launch_gemv(p, s));
        }
        return GAJE_OK;
    };
    const int rc = time_launches(launch_all, per_pass, iters, s, avg_ms);
    (void)hipStreamDestroy(s);
    return rc;
}

extern "C" int gaje_hip_bench_floor(const void *buf, int64_t bytes, int grid, int block, int iters, float *avg_ms) {
    clear_error();
    if (!avg_ms || iters <= 0 || grid <= 0 || block <= 0 || bytes < 0)
        return set_error(GAJE_ERR_INVALID_ARG, "bad benchmark arguments");
    hipStream_t s;
    GAJE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    auto launch_all = [&]() -> int {
        for (int i = 0; i < 128; ++i) GAJE_TRY(launch_floor_probe(buf, bytes, (unsigned)grid, (unsigned)block, s));
        return GAJE_OK;
    };
    const int rc = time_launches(launch_all, 128, iters, s, avg_ms);
    (void)hipStreamDestroy(s);
    return rc;
}
