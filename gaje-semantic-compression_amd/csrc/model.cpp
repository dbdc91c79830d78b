// Device-resident GAJE model: load a .gaje.flat into HBM and run the decode
// step as one captured HIP graph.
//
// Reference structure mirrored here:
//   load_genomic_auto / GajeFlatFileReader::load_genomic  src/io/flat_reader.rs:124-252
//   GenomicLinear::new format dispatch and LUT expansion  src/nn/linear/init.rs:12-160
//   GenomicLLM::forward_core / forward_with_hidden_core   src/nn/llm/forward.rs:7-113
//   RustGenomicBlock::forward_core                        src/nn/block/forward.rs:10-157
//   generate_native_core                                  src/nn/llm/forward.rs:215-330
//   set_k_wta_ratio                                       src/nn/llm/python.rs:53-59
//
// HBM layout per model: every weight tensor in its file packing (20-byte Q4_0
// blocks, 16-byte LUT code blocks + f32 tables, f32 rows), fused QKV and
// gate_up row orders as the exporter writes them; KV cache [L][n_kv][cap][hd]
// f32 (positions of one head contiguous for the attention kernel); a RoPE
// cos/sin table [cap][hd/2] built on the host with the C library's powf/sinf/cosf,
// the same functions the reference calls per head and token (attention.rs:66-68).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "flat.h"
#include "kernels.h"

namespace gaje {
namespace {

constexpr int64_t DEFAULT_CTX = 1024;

struct HostLinear {
    std::string name;
    int fmt = -1;
    int64_t N = 0, K = 0;
    std::vector<uint8_t> w;        // weight bytes (native packing)
    std::vector<float> lut;        // LUT-4bit tables as stored (not expanded)
    std::vector<float> bias;
    std::vector<int64_t> a_ptr;    // anchors CSR (empty = none)
    std::vector<uint32_t> a_col;
    std::vector<uint16_t> a_val;
};

struct DevLinear {
    int fmt = -1;
    int f32_tiled = 0;  // FMT_F32 rows in the GEMV's tiled layout
    int64_t N = 0, K = 0, rows_valid = 0, lut_rows_own = 0, lut_len = 0;
    int lut_block_stride = 0;
    uint8_t *w = nullptr;
    float *lut = nullptr;
    float *bias = nullptr;
    int64_t bias_len = 0;
    int64_t *a_ptr = nullptr;
    uint32_t *a_col = nullptr;
    uint16_t *a_val = nullptr;
    int64_t bytes = 0;
    uint16_t *mins = nullptr;  // FMT_Q4_0: the block mins [N][ldm] the MFMA prefill's products read
    int64_t ldm = 0;
    uint16_t *wf = nullptr;    // and their code fragments and scales (launch_q4_frags)
    float *wsc = nullptr;
};

struct Layer {
    float *attn_norm = nullptr;  // null: the reference skips the norm when the tensor is empty
    float *ffn_norm = nullptr;
    DevLinear qkv, o, gate_up, down;
};

const char *nan_message(int stage) {
    switch (stage) {
        case ST_INPUT: return "Input x is NaN";
        case ST_ATTN_NORM: return "NaN after attn rms_norm";
        case ST_UP: return "NaN in up";
        case ST_FFN_OUT: return "NaN in ffn_out";
        case ST_PROJ_FFN: return "NaN in projected_ffn";
        case ST_FINAL: return "NaN after projected_ffn addition";
        case ST_WAIT: return "attention: an in-kernel wait ran out of its bound (internal error; the step's outputs are invalid)";
        default: return "NaN";
    }
}

// GenomicLinear::new anchor parsing (init.rs:61-107) into CSR with the column
// already reduced modulo in_features (compute_single_row, forward.rs:103-112).
void parse_anchors(const uint8_t *buf, uint64_t len, HostLinear &L) {
    if (len < 8 || memcmp(buf, "GAJE", 4) != 0) return;
    uint32_t count;
    memcpy(&count, buf + 4, 4);
    const uint64_t idx_s = 8, val_s = idx_s + (uint64_t)count * 4, ptr_s = val_s + (uint64_t)count * 2;
    if (val_s + (uint64_t)count * 2 > len) return;  // the reference would panic on the slice
    std::vector<uint32_t> idx(count);
    std::vector<uint16_t> val(count);
    memcpy(idx.data(), buf + idx_s, (size_t)count * 4);
    memcpy(val.data(), buf + val_s, (size_t)count * 2);
    std::vector<int64_t> ptr(L.N + 1, 0);
    if (len >= ptr_s + (uint64_t)(L.N + 1) * 8) {
        for (int64_t i = 0; i <= L.N; ++i) {
            uint64_t v;
            memcpy(&v, buf + ptr_s + i * 8, 8);
            ptr[i] = (int64_t)v;
        }
    } else {
        int64_t cur = 0;
        for (uint32_t a = 0; a < count; ++a) {
            int64_t r = (int64_t)(idx[a] / (uint64_t)L.K);
            while (cur < r && cur < L.N) ptr[++cur] = a;
        }
        while (cur < L.N) ptr[++cur] = count;
    }
    // Rows whose range fails the reference's a_s < a_e <= count test add nothing.
    L.a_ptr.assign(L.N + 1, 0);
    for (int64_t i = 0; i < L.N; ++i) {
        int64_t a_s = ptr[i], a_e = ptr[i + 1];
        bool ok = a_s < a_e && a_e <= (int64_t)count;
        for (int64_t k = ok ? a_s : 0; ok && k < a_e; ++k) {
            L.a_col.push_back((uint32_t)(idx[k] % (uint64_t)L.K));
            L.a_val.push_back(val[k]);
        }
        L.a_ptr[i + 1] = (int64_t)L.a_col.size();
    }
    if (L.a_col.empty()) L.a_ptr.clear();
}

// GajeFlatFileReader::get_linear + GenomicLinear::new dispatch.
int read_linear(const FlatFile &f, const std::string &name, HostLinear &L) {
    const TensorEntry *e = f.find(name);
    if (!e) return set_error(GAJE_ERR_NOT_FOUND, "Flat tensor entry '%s' not found", name.c_str());
    L = HostLinear();
    L.name = name;
    L.N = (int64_t)e->out_features;
    L.K = (int64_t)e->in_features;
    const uint8_t *dna, *c, *anc, *bias;
    GAJE_TRY(f.slice(e->dna_off, e->dna_len, &dna));
    GAJE_TRY(f.slice(e->c_off, e->c_len, &c));
    GAJE_TRY(f.slice(e->anc_off, e->anc_len, &anc));
    GAJE_TRY(f.slice(e->bias_off, e->bias_len, &bias));
    const uint8_t bit_depth = (uint8_t)e->bit_depth;  // `entry.bit_depth as u8`
    const uint64_t n_cent = e->c_len / 4;
    if (bit_depth == 4) L.fmt = n_cent == 0 ? FMT_Q4_0 : FMT_LUT4;
    else if (bit_depth == 32) L.fmt = FMT_F32;
    else if (bit_depth == 8) L.fmt = FMT_Q8_0;  // init.rs:40-45
    else L.fmt = FMT_G2;                        // every other bit_depth: Genomic2Bit (init.rs:53)
    if (L.fmt == FMT_G2) {
        // the row dot reads 4 centroids per block from a row's table or, for
        // rows without one, from the table's start (linear/forward.rs:40-45),
        // and get_row indexes 4 of them: shorter tables are read past upstream
        const uint64_t nbk = (uint64_t)(L.K / 32);
        if ((n_cent > 0 && n_cent < 4) || (n_cent > 4 && n_cent < nbk * 4))
            return set_error(GAJE_ERR_UNSUPPORTED, "tensor '%s': 2-bit centroid table of %llu floats (need 4 or >= %llu)",
                             name.c_str(), (unsigned long long)n_cent, (unsigned long long)(nbk * 4));
    }
    if (e->dna_len) L.w.assign(dna, dna + e->dna_len);
    if (L.fmt == FMT_LUT4 || L.fmt == FMT_G2) {
        L.lut.resize(n_cent);
        memcpy(L.lut.data(), c, n_cent * 4);
    }
    const uint64_t nb = e->bias_len / 4;
    L.bias.resize(nb);
    if (nb) memcpy(L.bias.data(), bias, nb * 4);
    if (e->anc_len) parse_anchors(anc, e->anc_len, L);
    return GAJE_OK;
}

int read_norm(const FlatFile &f, const std::string &name, std::vector<float> &out) {
    const TensorEntry *e = f.find(name);
    if (!e) return set_error(GAJE_ERR_NOT_FOUND, "Flat tensor entry '%s' not found", name.c_str());
    const uint8_t *p;
    GAJE_TRY(f.slice(e->dna_off, e->dna_len, &p));
    out.resize(e->dna_len / 4);
    if (!out.empty()) memcpy(out.data(), p, out.size() * 4);
    return GAJE_OK;
}

int64_t rows_valid_of(const HostLinear &L) {
    const int64_t nb = L.K / 32;
    if (L.fmt == FMT_F32) return L.K ? std::min<int64_t>(L.N, (int64_t)(L.w.size() / 4) / L.K) : 0;
    if (nb == 0) return 0;
    if (L.fmt == FMT_Q4_0) return std::min<int64_t>(L.N, (int64_t)(L.w.size() / 20) / nb);
    if (L.fmt == FMT_Q8_0) return std::min<int64_t>(L.N, (int64_t)(L.w.size() / 34) / nb);
    if (L.fmt == FMT_G2) return L.lut.size() < 4 ? 0 : std::min<int64_t>(L.N, (int64_t)L.w.size() / (nb * 8));
    if (L.lut.size() < 16) return 0;  // no table: compute_single_row yields 0
    return std::min<int64_t>(L.N, (int64_t)L.w.size() / (nb * 16));
}

// Row-concatenate split tensors into the fused order the kernels expect
// ([q;k;v] as at export_gaje_flat.py:378-406, [gate;up] as at :413-417).
int fuse_linears(std::vector<HostLinear> parts, const std::string &name, HostLinear &out) {
    out = HostLinear();
    out.name = name;
    out.fmt = parts[0].fmt;
    out.K = parts[0].K;
    const int64_t nb = out.K / 32;
    bool any_bias = false, any_anchor = false;
    for (auto &p : parts) {
        if (p.fmt != out.fmt || p.K != out.K)
            return set_error(GAJE_ERR_UNSUPPORTED, "%s: split tensors differ in format or in_features", name.c_str());
        if (rows_valid_of(p) != p.N)
            return set_error(GAJE_ERR_UNSUPPORTED, "%s: truncated split tensor", name.c_str());
        out.N += p.N;
        any_bias |= !p.bias.empty();
        any_anchor |= !p.a_ptr.empty();
    }
    for (auto &p : parts) {
        size_t row_bytes = out.fmt == FMT_Q4_0   ? nb * 20
                           : out.fmt == FMT_Q8_0 ? nb * 34
                           : out.fmt == FMT_LUT4 ? nb * 16
                           : out.fmt == FMT_G2   ? nb * 8
                                                 : out.K * 4;
        out.w.insert(out.w.end(), p.w.begin(), p.w.begin() + row_bytes * p.N);
        if (out.fmt == FMT_G2) {  // per-row centroid tables, as the row dot reads them
            const size_t per_row = nb * 4;
            for (int64_t r = 0; r < p.N; ++r) {
                if (p.lut.size() == 4) {  // init.rs:125-131
                    for (int64_t b = 0; b < nb; ++b) out.lut.insert(out.lut.end(), p.lut.begin(), p.lut.end());
                    continue;
                }
                const float *src = p.lut.size() >= (size_t)(r + 1) * per_row && p.lut.size() != per_row
                                       ? p.lut.data() + r * per_row
                                       : p.lut.data();  // the column table, or the table's start
                out.lut.insert(out.lut.end(), src, src + per_row);
            }
        }
        if (out.fmt == FMT_LUT4) {  // expand to per-row tables (init.rs:109-124)
            const size_t per_row = nb * 16;
            for (int64_t r = 0; r < p.N; ++r) {
                const float *src;
                if (p.lut.size() == 16) {
                    for (int64_t b = 0; b < nb; ++b) out.lut.insert(out.lut.end(), p.lut.begin(), p.lut.begin() + 16);
                    continue;
                } else if (p.lut.size() == per_row) {
                    src = p.lut.data();
                } else if (p.lut.size() >= (size_t)(r + 1) * per_row) {
                    src = p.lut.data() + r * per_row;
                } else if (p.lut.size() >= per_row) {
                    src = p.lut.data();
                } else {
                    return set_error(GAJE_ERR_INVALID_DATA, "%s: centroid table too short", p.name.c_str());
                }
                out.lut.insert(out.lut.end(), src, src + per_row);
            }
        }
        if (any_bias) {
            for (int64_t r = 0; r < p.N; ++r) out.bias.push_back(r < (int64_t)p.bias.size() ? p.bias[r] : 0.0f);
        }
        if (any_anchor) {
            if (out.a_ptr.empty()) out.a_ptr.push_back(0);
            for (int64_t r = 0; r < p.N; ++r) {
                if (!p.a_ptr.empty())
                    for (int64_t k = p.a_ptr[r]; k < p.a_ptr[r + 1]; ++k) {
                        out.a_col.push_back(p.a_col[k]);
                        out.a_val.push_back(p.a_val[k]);
                    }
                out.a_ptr.push_back((int64_t)out.a_col.size());
            }
        }
    }
    return GAJE_OK;
}

}  // namespace
}  // namespace gaje

using namespace gaje;

struct gaje_hip_model {
    int device = 0;
    hipStream_t stream = nullptr;
    ModelConfig cfg;
    int64_t n_embd = 0, n_head = 0, n_kv = 0, hd = 0, ffn = 0, vocab_embd = 0, vocab_out = 0, n_layers = 0;
    int64_t q_rows = 0, kv_rows = 0;
    int32_t arch_family = 0;
    int rope_split = 1;
    float rope_base = 10000.0f, eps = 0.0f;
    bool use_genomic_norm = false;
    int body_fmt = FMT_Q4_0;

    DevLinear embd, lm_head;
    float *output_norm = nullptr;
    std::vector<Layer> layers;

    // activations and scratch
    float *h = nullptr, *q = nullptr, *attn_out = nullptr, *act = nullptr, *logits = nullptr, *hnorm = nullptr;
    // the SwiGLU output also in the chain-major layout (8 rows of act_cm_stride
    // floats, zero past ffn / 8), which the down matvec copies as it stands
    float *act_cm = nullptr;
    int32_t act_cm_stride = 0;
    DevState *st = nullptr;
    uint32_t *out_tokens = nullptr;
    int64_t out_cap = 0;
    // greedy generate loop on the device: its state, the seen-set bitmap and
    // the generated tokens (grown on demand)
    GenState *gen = nullptr;
    uint32_t *gen_seen = nullptr, *gen_tokens = nullptr;
    int64_t gen_cap = 0;
    // KV cache and RoPE table
    float *k_cache = nullptr, *v_cache = nullptr, *rope_cos = nullptr, *rope_sin = nullptr;
    int64_t cap = 0;

    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    int64_t graph_block_k = 0;      // block K-WTA k baked into the captured graph (0 = none)

    float kwta_ratio = 0.5f;        // GenomicLLM k_wta_ratio after load_genomic (flat_reader.rs:234)
    float block_kwta_ratio = 0.0f;  // RustGenomicBlock k_wta_ratio (block/init.rs:42)
    int64_t pos = 0;                // cached positions (k_cache_len of block 0)
    int64_t weight_bytes = 0;
    bool profile = false;
    float last_blocks_ms = 0.0f, last_head_ms = 0.0f;

    // prompt prefill on the MFMA units: per-chunk activations, grown on demand
    struct Prefill {
        int64_t rows = 0;        // chunk rows the buffers hold
        int64_t part_floats = 0; // split-K partials they hold
        float *H = nullptr, *QKV = nullptr, *Q = nullptr, *ATT = nullptr, *GU = nullptr, *part = nullptr, *aws = nullptr;
        uint16_t *xh = nullptr;                 // activation plane [gemm_bs_plane_rows(rows)][2 kmax]
        uint16_t *sh = nullptr, *sl = nullptr;  // block-sum planes [rows][gemm_bs_sum_cols(kmax)]
        int *ex = nullptr;
        uint32_t *ids = nullptr;
        uint16_t *kv16 = nullptr;  // attention's f16 keys and values, prefill_kv16_halves(kv16_keys, ..)
        int64_t kv16_keys = 0;
    } pf;

    std::vector<void *> allocs;
    std::vector<gaje_hip_batch *> batches;  // open batches over these weights

    ~gaje_hip_model() {
        if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
        if (graph) (void)hipGraphDestroy(graph);
        for (void *p : allocs) (void)hipFree(p);
        if (stream) (void)hipStreamDestroy(stream);
    }

    template <class T>
    int alloc(T **p, size_t count) {
        *p = nullptr;
        if (count == 0) return GAJE_OK;
        void *v = nullptr;
        GAJE_HIP_CHECK(hipMalloc(&v, count * sizeof(T)));
        allocs.push_back(v);
        *p = (T *)v;
        return GAJE_OK;
    }
    template <class T>
    int upload(T **p, const T *src, size_t count) {
        GAJE_TRY(alloc(p, count));
        if (count) GAJE_HIP_CHECK(hipMemcpy(*p, src, count * sizeof(T), hipMemcpyHostToDevice));
        weight_bytes += (int64_t)(count * sizeof(T));
        return GAJE_OK;
    }
    void release(void *p) {
        for (auto it = allocs.begin(); it != allocs.end(); ++it)
            if (*it == p) {
                (void)hipFree(p);
                allocs.erase(it);
                return;
            }
    }
};

namespace {

// tile_f32: store FMT_F32 rows in the GEMV's tiled layout (not for the
// embedding, whose rows are looked up one at a time).
int upload_linear(gaje_hip_model *m, const HostLinear &L, DevLinear &D, bool tile_f32 = true) {
    D = DevLinear();
    D.fmt = L.fmt;
    D.N = L.N;
    D.K = L.K;
    D.rows_valid = rows_valid_of(L);
    const int64_t nb = L.K / 32;
    if (L.fmt == FMT_Q4_0) {
        // stage the file's Q4_0Block rows and pack them into the GEMV layout
        const size_t raw = (size_t)D.rows_valid * nb * 20;
        const int64_t packed = q4_0_packed_bytes(D.rows_valid, L.K);
        uint8_t *tmp = nullptr;
        GAJE_TRY(m->upload(&tmp, L.w.data(), raw));
        m->weight_bytes -= (int64_t)raw;
        int rc = m->alloc(&D.w, (size_t)packed);
        if (rc == GAJE_OK && packed > 0) rc = launch_pack_q4_0(tmp, D.w, D.rows_valid, L.K, m->stream);
        if (rc == GAJE_OK) rc = hipStreamSynchronize(m->stream) == hipSuccess ? GAJE_OK
                                                                               : set_error(GAJE_ERR_HIP, "Q4_0 pack failed");
        m->release(tmp);
        GAJE_TRY(rc);
        m->weight_bytes += packed;
    } else if (L.fmt == FMT_Q8_0) {
        // stage the file's Q8_0Block rows and pack them into 144-byte groups
        const size_t raw = (size_t)D.rows_valid * nb * 34;
        const int64_t packed = q8_0_packed_bytes(D.rows_valid, L.K);
        uint8_t *tmp = nullptr;
        GAJE_TRY(m->upload(&tmp, L.w.data(), raw));
        m->weight_bytes -= (int64_t)raw;
        int rc = m->alloc(&D.w, (size_t)packed);
        if (rc == GAJE_OK && packed > 0) rc = launch_pack_q8_0(tmp, D.w, D.rows_valid, L.K, m->stream);
        if (rc == GAJE_OK) rc = hipStreamSynchronize(m->stream) == hipSuccess ? GAJE_OK
                                                                               : set_error(GAJE_ERR_HIP, "Q8_0 pack failed");
        m->release(tmp);
        GAJE_TRY(rc);
        m->weight_bytes += packed;
    } else if (L.fmt == FMT_F32 && tile_f32 && L.K % 8 == 0 && D.rows_valid > 0) {
        // stage the row-major rows and tile them (32-row tiles, KiB chunks)
        const size_t raw = (size_t)D.rows_valid * L.K * 4;
        const int64_t tiled = f32_tiled_bytes(D.rows_valid, L.K);
        uint8_t *tmp = nullptr;
        GAJE_TRY(m->upload(&tmp, L.w.data(), raw));
        m->weight_bytes -= (int64_t)raw;
        int rc = m->alloc(&D.w, (size_t)tiled);
        if (rc == GAJE_OK) rc = launch_pack_f32_tiled((const float *)tmp, (float *)D.w, D.rows_valid, L.K, m->stream);
        if (rc == GAJE_OK) rc = hipStreamSynchronize(m->stream) == hipSuccess ? GAJE_OK
                                                                               : set_error(GAJE_ERR_HIP, "f32 tiling failed");
        m->release(tmp);
        GAJE_TRY(rc);
        m->weight_bytes += tiled;
        D.f32_tiled = 1;
    } else {
        GAJE_TRY(m->upload(&D.w, L.w.data(), L.w.size()));
    }
    if (L.fmt == FMT_G2 && L.lut.size() >= 4) {
        const size_t n = L.lut.size(), per_row = (size_t)nb * 4;
        if (n == 4) {
            D.lut_block_stride = 0;  // one table for every block (init.rs:125-131)
            D.lut_rows_own = 0;
        } else {
            D.lut_block_stride = 4;  // n >= per_row (read_linear)
            D.lut_rows_own = n == per_row ? 0 : (int64_t)(n / per_row);
        }
        D.lut_len = (int64_t)n;
        GAJE_TRY(m->upload(&D.lut, L.lut.data(), n));
    }
    if (L.fmt == FMT_LUT4 && !L.lut.empty()) {
        const size_t n = L.lut.size(), per_row = (size_t)nb * 16;
        if (n == 16) {
            D.lut_block_stride = 0;
            D.lut_rows_own = 0;
        } else if (per_row > 0 && n >= per_row) {
            D.lut_block_stride = 16;
            D.lut_rows_own = n == per_row ? 0 : (int64_t)(n / per_row);
        } else {
            return set_error(GAJE_ERR_INVALID_DATA, "tensor '%s': centroid table of %zu floats is shorter than a row",
                             L.name.c_str(), n);
        }
        GAJE_TRY(m->upload(&D.lut, L.lut.data(), n));
    }
    D.bias_len = (int64_t)L.bias.size();
    GAJE_TRY(m->upload(&D.bias, L.bias.data(), L.bias.size()));
    if (!L.a_ptr.empty()) {
        GAJE_TRY(m->upload(&D.a_ptr, L.a_ptr.data(), L.a_ptr.size()));
        GAJE_TRY(m->upload(&D.a_col, L.a_col.data(), L.a_col.size()));
        GAJE_TRY(m->upload(&D.a_val, L.a_val.data(), L.a_val.size()));
    }
    return GAJE_OK;
}

GemvParams gemv_base(const gaje_hip_model *m, const DevLinear &D, const float *x) {
    GemvParams p;
    memset(&p, 0, sizeof p);
    p.w = D.w;
    p.fmt = D.fmt;
    p.f32_tiled = D.f32_tiled;
    p.lut = D.lut;
    p.lut_rows_own = D.lut_rows_own;
    p.lut_block_stride = D.lut_block_stride;
    p.nb = (int32_t)(D.K / 32);
    p.rows_valid = D.rows_valid;
    p.N = D.N;
    p.K = D.K;
    p.x = x;
    p.eps = m->eps;
    p.h_scale = 1.0f;
    p.bias = D.bias;
    p.bias_len = D.bias_len;
    p.a_ptr = D.a_ptr;
    p.a_col = D.a_col;
    p.a_val = D.a_val;
    p.st = m->st;
    p.st_in = p.st_norm = p.st_a = p.st_b = ST_NONE;
    return p;
}

int build_rope(gaje_hip_model *m, int64_t cap, float **cos_out, float **sin_out) {
    const int64_t half = m->hd / 2;
    std::vector<float> c((size_t)(cap * half)), s((size_t)(cap * half));
    for (int64_t i = 0; i < half; ++i) {
        const float expo = (2.0f * (float)i) / (float)m->hd;
        const float freq = 1.0f / powf(m->rope_base, expo);
        for (int64_t pos = 0; pos < cap; ++pos) {
            const float theta = (float)pos * freq;
            c[pos * half + i] = cosf(theta);
            s[pos * half + i] = sinf(theta);
        }
    }
    GAJE_TRY(m->alloc(cos_out, c.size()));
    GAJE_TRY(m->alloc(sin_out, s.size()));
    GAJE_HIP_CHECK(hipMemcpy(*cos_out, c.data(), c.size() * 4, hipMemcpyHostToDevice));
    GAJE_HIP_CHECK(hipMemcpy(*sin_out, s.data(), s.size() * 4, hipMemcpyHostToDevice));
    return GAJE_OK;
}

void drop_graph(gaje_hip_model *m) {
    if (m->graph_exec) (void)hipGraphExecDestroy(m->graph_exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->graph_exec = nullptr;
    m->graph = nullptr;
}

// Grow the KV cache and RoPE table to hold `positions` tokens.
int reserve_ctx(gaje_hip_model *m, int64_t positions) {
    if (positions <= m->cap) return GAJE_OK;
    if (positions > MAX_CTX)
        return set_error(GAJE_ERR_UNSUPPORTED, "context of %lld positions exceeds this build's limit of %lld",
                         (long long)positions, (long long)MAX_CTX);
    int64_t cap = std::max<int64_t>(positions, m->cap ? 2 * m->cap : DEFAULT_CTX);
    cap = std::min<int64_t>((cap + 63) / 64 * 64, MAX_CTX);
    const int64_t L = std::max<int64_t>(m->n_layers, 1);
    const size_t per_head_new = (size_t)cap * m->hd, per_head_old = (size_t)m->cap * m->hd;
    float *kc, *vc, *rc, *rs;
    GAJE_TRY(m->alloc(&kc, (size_t)L * m->n_kv * per_head_new));
    GAJE_TRY(m->alloc(&vc, (size_t)L * m->n_kv * per_head_new));
    if (m->k_cache && m->pos > 0) {
        for (int64_t l = 0; l < m->n_layers; ++l)
            for (int64_t g = 0; g < m->n_kv; ++g) {
                const size_t src = ((size_t)l * m->n_kv + g) * per_head_old, dst = ((size_t)l * m->n_kv + g) * per_head_new;
                // K and V rows are [dim][position]: a prefix of every dimension's row
                GAJE_HIP_CHECK(hipMemcpy2DAsync(kc + dst, (size_t)cap * 4, m->k_cache + src, (size_t)m->cap * 4,
                                                (size_t)m->pos * 4, (size_t)m->hd, hipMemcpyDeviceToDevice, m->stream));
                GAJE_HIP_CHECK(hipMemcpy2DAsync(vc + dst, (size_t)cap * 4, m->v_cache + src, (size_t)m->cap * 4,
                                                (size_t)m->pos * 4, (size_t)m->hd, hipMemcpyDeviceToDevice, m->stream));
            }
        GAJE_HIP_CHECK(hipStreamSynchronize(m->stream));
    }
    GAJE_TRY(build_rope(m, cap, &rc, &rs));
    if (m->k_cache) m->release(m->k_cache);
    if (m->v_cache) m->release(m->v_cache);
    if (m->rope_cos) m->release(m->rope_cos);
    if (m->rope_sin) m->release(m->rope_sin);
    m->k_cache = kc;
    m->v_cache = vc;
    m->rope_cos = rc;
    m->rope_sin = rs;
    m->cap = cap;
    drop_graph(m);
    return GAJE_OK;
}

// k of the blocks' lateral_inhibition_kwta (block/forward.rs:144-148,
// k = max(1, n_embd * ratio)), or 0 when the ratio leaves it off.
int64_t block_kwta_k(const gaje_hip_model *m) {
    if (!(m->block_kwta_ratio > 0.0f && m->block_kwta_ratio < 1.0f)) return 0;
    const int64_t k = (int64_t)((float)m->n_embd * m->block_kwta_ratio);
    return k < 1 ? 1 : k;
}

// Output norm -> lm_head logits with the running argmax -> next token, advance
// (llm/forward.rs:38-46) for the hidden state in m->h.
int enqueue_head(gaje_hip_model *m) {
    GemvParams p = gemv_base(m, m->lm_head, m->h);
    p.norm_w = m->output_norm;
    p.mode = MODE_ARGMAX;
    p.y = m->logits;
    p.x_out = m->hnorm;
    p.nontemporal = 1;
    p.layer = (int32_t)m->n_layers;
    GAJE_TRY(launch_gemv(p, m->stream));
    return launch_finalize(m->st, m->out_tokens, m->stream);
}

// Enqueue one decode step (embedding -> blocks -> output norm -> lm_head ->
// argmax/advance) on the model stream.
int enqueue_token(gaje_hip_model *m, hipEvent_t ev_blocks_done) {
    EmbedParams ep;
    memset(&ep, 0, sizeof ep);
    ep.w = m->embd.w;
    ep.fmt = m->embd.fmt;
    ep.lut = m->embd.lut;
    ep.lut_rows_own = m->embd.lut_rows_own;
    ep.lut_block_stride = m->embd.lut_block_stride;
    ep.lut_len = m->embd.lut_len;
    ep.vocab = m->vocab_embd;
    ep.rows_valid = m->embd.rows_valid;
    ep.K = m->n_embd;
    ep.h = m->h;
    ep.st = m->st;
    GAJE_TRY(launch_embed(ep, m->stream));

    const size_t layer_kv = (size_t)m->n_kv * m->cap * m->hd;
    auto qkv_params = [&](int64_t l) {
        Layer &Ly = m->layers[l];
        GemvParams p = gemv_base(m, Ly.qkv, m->h);
        p.norm_w = Ly.attn_norm;
        p.layer = (int32_t)l;
        p.st_in = ST_INPUT;
        p.st_norm = Ly.attn_norm ? ST_ATTN_NORM : ST_NONE;
        p.mode = MODE_QKV;
        p.y = m->q;
        p.q_out = m->q;
        p.head_dim = (int32_t)m->hd;
        p.rope_split = m->rope_split;
        p.q_rows = m->q_rows;
        p.kv_rows = m->kv_rows;
        p.rope_cos = m->rope_cos;
        p.rope_sin = m->rope_sin;
        p.k_cache = m->k_cache + l * layer_kv;
        p.v_cache = m->v_cache + l * layer_kv;
        p.kv_head_stride = m->cap * m->hd;
        p.kv_cap = m->cap;
        return p;
    };
    auto o_params = [&](int64_t l) {
        GemvParams p = gemv_base(m, m->layers[l].o, m->attn_out);
        p.layer = (int32_t)l;
        p.mode = MODE_RESIDUAL;
        p.y = m->h;
        return p;
    };
    // The blocks' K-WTA (block/forward.rs:144-148) after block l < L - 1 runs
    // inside block l + 1's QKV launch (threshold and mask of its copy of h) and
    // attention-output launch (the same mask on the residual h it adds to),
    // when both run on the chain kernel; after the last block, and otherwise,
    // as its own launch.
    const int64_t bk = block_kwta_k(m);
    bool fuse = bk > 0;
    for (int64_t l = 1; fuse && l < m->n_layers; ++l)
        fuse = gemv_chain_serves(qkv_params(l)) && gemv_chain_serves(o_params(l));
    for (int64_t l = 0; l < m->n_layers; ++l) {
        Layer &Ly = m->layers[l];
        const bool fused_in = fuse && l > 0;
        GemvParams p = qkv_params(l);
        if (fused_in) {
            p.kwta_k = bk;
            p.kwta_thr = &m->st->kwta_thr;
        }
        GAJE_TRY(launch_gemv(p, m->stream));

        AttnParams ap{};
        ap.q = m->q;
        ap.k_cache = m->k_cache + l * layer_kv;
        ap.v_cache = m->v_cache + l * layer_kv;
        ap.kv_head_stride = m->cap * m->hd;
        ap.n_head = (int32_t)m->n_head;
        ap.n_head_kv = (int32_t)m->n_kv;
        ap.head_dim = (int32_t)m->hd;
        ap.kv_cap = m->cap;
        ap.out = m->attn_out;
        ap.st = m->st;
        ap.layer = (int32_t)l;
        GAJE_TRY(launch_attention(ap, m->stream));

        p = o_params(l);
        if (fused_in) {
            p.kwta_k = bk;
            p.kwta_thr = &m->st->kwta_thr;
        }
        GAJE_TRY(launch_gemv(p, m->stream));

        p = gemv_base(m, Ly.gate_up, m->h);
        p.norm_w = Ly.ffn_norm;
        p.layer = (int32_t)l;
        p.mode = MODE_SWIGLU;
        p.ffn = m->ffn;
        p.y = m->act;
        p.y_cm = m->act_cm;
        p.cm_stride = m->act_cm_stride;
        p.st_a = ST_UP;
        p.st_b = ST_FFN_OUT;
        GAJE_TRY(launch_gemv(p, m->stream));

        p = gemv_base(m, Ly.down, m->act);
        p.x_cm = m->act_cm;
        p.cm_stride = m->act_cm_stride;
        p.layer = (int32_t)l;
        p.gnorm = m->use_genomic_norm;
        p.mode = MODE_RESIDUAL;
        p.y = m->h;
        p.st_a = ST_PROJ_FFN;
        p.st_b = ST_FINAL;
        GAJE_TRY(launch_gemv(p, m->stream));

        if (bk > 0 && (!fuse || l + 1 == m->n_layers)) GAJE_TRY(launch_kwta(m->h, m->n_embd, bk, m->st, m->stream));
    }
    if (ev_blocks_done) GAJE_HIP_CHECK(hipEventRecord(ev_blocks_done, m->stream));
    return enqueue_head(m);
}

// The graph bakes the block K-WTA k into a kernel argument, so it is keyed by
// that k: a ratio change that changes k recaptures it.
int ensure_graph(gaje_hip_model *m) {
    const int64_t bk = block_kwta_k(m);
    if (m->graph_exec && m->graph_block_k == bk) return GAJE_OK;
    drop_graph(m);
    GAJE_HIP_CHECK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_token(m, nullptr);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc != GAJE_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return set_error(GAJE_ERR_HIP, "graph capture failed: %s", hipGetErrorString(e));
    m->graph = g;
    GAJE_HIP_CHECK(hipGraphInstantiate(&m->graph_exec, g, nullptr, nullptr, 0));
    m->graph_block_k = bk;
    return GAJE_OK;
}

int run_token(gaje_hip_model *m) {
    if (m->profile) {
        hipEvent_t e0, e1, e2;
        GAJE_HIP_CHECK(hipEventCreate(&e0));
        GAJE_HIP_CHECK(hipEventCreate(&e1));
        GAJE_HIP_CHECK(hipEventCreate(&e2));
        GAJE_HIP_CHECK(hipEventRecord(e0, m->stream));
        int rc = enqueue_token(m, e1);
        GAJE_HIP_CHECK(hipEventRecord(e2, m->stream));
        GAJE_HIP_CHECK(hipEventSynchronize(e2));
        (void)hipEventElapsedTime(&m->last_blocks_ms, e0, e1);
        (void)hipEventElapsedTime(&m->last_head_ms, e1, e2);
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        (void)hipEventDestroy(e2);
        return rc;
    }
    GAJE_TRY(ensure_graph(m));
    GAJE_HIP_CHECK(hipGraphLaunch(m->graph_exec, m->stream));
    return GAJE_OK;
}

int read_state(gaje_hip_model *m, DevState &s) {
    GAJE_HIP_CHECK(hipMemcpyAsync(&s, m->st, sizeof s, hipMemcpyDeviceToHost, m->stream));
    GAJE_HIP_CHECK(hipStreamSynchronize(m->stream));
    return GAJE_OK;
}

int nan_error(const DevState &s) {
    const int stage = (int)(s.nan_code % 8);
    return set_error(stage == ST_WAIT ? GAJE_ERR_HIP : GAJE_ERR_NAN, "%s", nan_message(stage));
}

int64_t kwta_k(int64_t n, float ratio) {
    int64_t k = (int64_t)((float)n * ratio);
    return k < 1 ? 1 : k;
}

// forward_core for one token; leaves the logits on the device (K-WTA applied
// when `apply_kwta`), the state read back into `s`.
int forward_device(gaje_hip_model *m, uint32_t token, bool clear, bool apply_kwta, DevState &s) {
    if (clear) m->pos = 0;
    GAJE_TRY(reserve_ctx(m, m->pos + 1));
    GAJE_TRY(launch_state_set(m->st, (int32_t)m->pos, token, -1, -1, 1, m->stream));
    GAJE_TRY(run_token(m));
    if (apply_kwta && m->kwta_ratio > 0.0f && m->kwta_ratio < 1.0f)
        GAJE_TRY(launch_kwta(m->logits, m->vocab_out, kwta_k(m->vocab_out, m->kwta_ratio), m->st, m->stream));
    GAJE_TRY(read_state(m, s));
    if (s.halted || s.nan_code != NAN_NONE) return nan_error(s);
    m->pos += 1;
    return GAJE_OK;
}

int check_model(gaje_hip_model *m) {
    if (!m) return set_error(GAJE_ERR_INVALID_ARG, "null model handle");
    GAJE_HIP_CHECK(hipSetDevice(m->device));
    return GAJE_OK;
}

uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace

extern "C" int gaje_hip_open(const char *path, int device, gaje_hip_model **out) {
    clear_error();
    if (!path || !out) return set_error(GAJE_ERR_INVALID_ARG, "gaje_hip_open: null argument");
    *out = nullptr;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0)
        return set_error(GAJE_ERR_NO_DEVICE, "no HIP device available");
    if (device < 0 || device >= ndev) return set_error(GAJE_ERR_INVALID_ARG, "device %d out of range", device);
    GAJE_HIP_CHECK(hipSetDevice(device));

    FlatFile f;
    GAJE_TRY(f.open(path));
    std::unique_ptr<gaje_hip_model> m(new gaje_hip_model());
    m->device = device;
    GAJE_TRY(f.model_config(m->cfg));
    const ModelConfig &c = m->cfg;
    if (c.n_head == 0) return set_error(GAJE_ERR_MODEL, "n_head is 0");
    m->n_embd = (int64_t)c.n_embd;
    m->n_head = (int64_t)c.n_head;
    m->n_kv = (int64_t)c.n_head_kv;
    m->n_layers = (int64_t)c.n_blocks;
    m->hd = m->n_embd / m->n_head;  // load_genomic: n_embd / n_head (flat_reader.rs:142)
    m->eps = c.eps;
    m->rope_base = c.rope_base;
    m->rope_split = c.rope_style == "split" ? 1 : 0;
    m->use_genomic_norm = c.use_genomic_norm;
    m->arch_family = (int32_t)f.header().arch_family;
    m->q_rows = m->n_head * m->hd;
    m->kv_rows = m->n_kv * m->hd;
    if (m->n_layers > 0 && (m->n_kv == 0 || m->n_head % m->n_kv != 0))
        return set_error(GAJE_ERR_MODEL, "n_head %lld is not a multiple of n_head_kv %lld", (long long)m->n_head,
                         (long long)m->n_kv);
    if (m->n_layers > 0 && (m->hd <= 0 || m->hd > 128 || m->hd % 4 != 0))
        return set_error(GAJE_ERR_UNSUPPORTED, "head_dim %lld not supported (need <= 128, multiple of 4)",
                         (long long)m->hd);
    if (m->n_kv > 64) return set_error(GAJE_ERR_UNSUPPORTED, "more than 64 KV heads");
    m->profile = getenv("GAJE_HIP_PROFILE") != nullptr;

    GAJE_HIP_CHECK(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));

    HostLinear L;
    GAJE_TRY(read_linear(f, "token_embd", L));
    if (L.K != m->n_embd)
        return set_error(GAJE_ERR_MODEL, "token_embd in_features %lld != n_embd %lld", (long long)L.K,
                         (long long)m->n_embd);
    m->vocab_embd = L.N;
    if (m->vocab_embd == 0) return set_error(GAJE_ERR_MODEL, "token_embd has no rows");
    GAJE_TRY(upload_linear(m.get(), L, m->embd, false));
    std::vector<float> norm;
    GAJE_TRY(read_norm(f, "output_norm", norm));
    if ((int64_t)norm.size() != m->n_embd) return set_error(GAJE_ERR_MODEL, "output_norm length != n_embd");
    GAJE_TRY(m->upload(&m->output_norm, norm.data(), norm.size()));
    GAJE_TRY(read_linear(f, "lm_head", L));
    if (L.N == 0) return set_error(GAJE_ERR_MODEL, "LM Head out_features is 0!");
    if (L.K != m->n_embd) return set_error(GAJE_ERR_MODEL, "lm_head in_features != n_embd");
    m->vocab_out = L.N;
    GAJE_TRY(upload_linear(m.get(), L, m->lm_head));

    m->layers.resize((size_t)m->n_layers);
    for (int64_t i = 0; i < m->n_layers; ++i) {
        const std::string p = "blk." + std::to_string(i) + ".";
        Layer &Ly = m->layers[i];
        GAJE_TRY(read_norm(f, p + "attn_norm", norm));
        if (!norm.empty()) {
            if ((int64_t)norm.size() != m->n_embd) return set_error(GAJE_ERR_MODEL, "%sattn_norm length != n_embd", p.c_str());
            GAJE_TRY(m->upload(&Ly.attn_norm, norm.data(), norm.size()));
        }
        GAJE_TRY(read_norm(f, p + "ffn_norm", norm));
        if ((int64_t)norm.size() != m->n_embd) return set_error(GAJE_ERR_MODEL, "%sffn_norm length != n_embd", p.c_str());
        GAJE_TRY(m->upload(&Ly.ffn_norm, norm.data(), norm.size()));

        HostLinear qkv, gu, o, down;
        if (f.find(p + "attn_qkv")) {
            GAJE_TRY(read_linear(f, p + "attn_qkv", qkv));
        } else {
            std::vector<HostLinear> parts(3);
            GAJE_TRY(read_linear(f, p + "attn_q", parts[0]));
            GAJE_TRY(read_linear(f, p + "attn_k", parts[1]));
            GAJE_TRY(read_linear(f, p + "attn_v", parts[2]));
            GAJE_TRY(fuse_linears(std::move(parts), p + "attn_qkv", qkv));
        }
        GAJE_TRY(read_linear(f, p + "attn_output", o));
        if (f.find(p + "ffn_gate_up")) {
            GAJE_TRY(read_linear(f, p + "ffn_gate_up", gu));
        } else {
            std::vector<HostLinear> parts(2);
            GAJE_TRY(read_linear(f, p + "ffn_gate", parts[0]));
            GAJE_TRY(read_linear(f, p + "ffn_up", parts[1]));
            GAJE_TRY(fuse_linears(std::move(parts), p + "ffn_gate_up", gu));
        }
        GAJE_TRY(read_linear(f, p + "ffn_down", down));
        if (qkv.K != m->n_embd || qkv.N < m->q_rows + 2 * m->kv_rows)
            return set_error(GAJE_ERR_MODEL, "%sattn_qkv shape %lldx%lld does not match the architecture", p.c_str(),
                             (long long)qkv.N, (long long)qkv.K);
        if (o.K != m->q_rows || o.N != m->n_embd)
            return set_error(GAJE_ERR_MODEL, "%sattn_output shape does not match the architecture", p.c_str());
        if (gu.K != m->n_embd || gu.N < 2)
            return set_error(GAJE_ERR_MODEL, "%sffn_gate_up shape does not match the architecture", p.c_str());
        const int64_t ffn = gu.N / 2;  // block/forward.rs:89
        if (i == 0) m->ffn = ffn;
        if (ffn != m->ffn) return set_error(GAJE_ERR_UNSUPPORTED, "blocks with different FFN widths");
        if (down.K != ffn || down.N != m->n_embd)
            return set_error(GAJE_ERR_MODEL, "%sffn_down shape does not match the architecture", p.c_str());
        if (i == 0) m->body_fmt = qkv.fmt;
        GAJE_TRY(upload_linear(m.get(), qkv, Ly.qkv));
        GAJE_TRY(upload_linear(m.get(), o, Ly.o));
        GAJE_TRY(upload_linear(m.get(), gu, Ly.gate_up));
        GAJE_TRY(upload_linear(m.get(), down, Ly.down));
    }

    // activations, scratch, state
    const int64_t qn = std::max<int64_t>(m->q_rows, 1);
    GAJE_TRY(m->alloc(&m->h, (size_t)m->n_embd));
    GAJE_TRY(m->alloc(&m->hnorm, (size_t)m->n_embd));
    GAJE_TRY(m->alloc(&m->q, (size_t)qn));
    GAJE_TRY(m->alloc(&m->attn_out, (size_t)qn));
    GAJE_TRY(m->alloc(&m->act, (size_t)std::max<int64_t>(m->ffn, 1)));
    if (m->ffn > 0) {
        m->act_cm_stride = gemv_chain_stride(m->ffn);
        GAJE_TRY(m->alloc(&m->act_cm, (size_t)8 * m->act_cm_stride));
        GAJE_HIP_CHECK(hipMemset(m->act_cm, 0, (size_t)8 * m->act_cm_stride * sizeof(float)));
    }
    GAJE_TRY(m->alloc(&m->logits, (size_t)m->vocab_out));
    GAJE_TRY(m->alloc(&m->st, 1));
    GAJE_HIP_CHECK(hipMemset(m->st, 0, sizeof(DevState)));
    m->out_cap = 4096;
    GAJE_TRY(m->alloc(&m->out_tokens, (size_t)m->out_cap));
    if (m->n_layers > 0) GAJE_TRY(reserve_ctx(m.get(), DEFAULT_CTX));
    GAJE_TRY(launch_state_set(m->st, 0, 0, (int32_t)m->out_cap, 0, 1, m->stream));
    GAJE_HIP_CHECK(hipStreamSynchronize(m->stream));
    *out = m.release();
    return GAJE_OK;
}

void batch_detach(gaje_hip_batch *b);

extern "C" void gaje_hip_close(gaje_hip_model *m) {
    if (!m) return;
    (void)hipSetDevice(m->device);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    // a batch outliving its model keeps only its handle (its close then frees it)
    for (gaje_hip_batch *b : m->batches) batch_detach(b);
    delete m;
}

extern "C" int gaje_hip_model_info_get(const gaje_hip_model *m, gaje_hip_model_info *info) {
    if (!m || !info) return set_error(GAJE_ERR_INVALID_ARG, "null argument");
    memset(info, 0, sizeof *info);
    info->n_embd = m->n_embd;
    info->n_head = m->n_head;
    info->n_head_kv = m->n_kv;
    info->n_blocks = m->n_layers;
    info->head_dim = m->hd;
    info->ffn = m->ffn;
    info->vocab_size = m->vocab_embd;
    info->eps = m->eps;
    info->rope_base = m->rope_base;
    info->rope_split = m->rope_split;
    info->arch_family = m->arch_family;
    info->body_format = m->body_fmt;
    info->use_genomic_norm = m->use_genomic_norm;
    info->max_ctx = m->cap;
    info->weight_bytes = m->weight_bytes;
    info->n_logits = m->vocab_out;
    return GAJE_OK;
}

extern "C" int gaje_hip_forward(gaje_hip_model *m, uint32_t token, int clear_cache, float *logits_host) {
    clear_error();
    GAJE_TRY(check_model(m));
    DevState s;
    GAJE_TRY(forward_device(m, token, clear_cache != 0, true, s));
    if (logits_host)
        GAJE_HIP_CHECK(hipMemcpy(logits_host, m->logits, (size_t)m->vocab_out * 4, hipMemcpyDeviceToHost));
    return GAJE_OK;
}

extern "C" int gaje_hip_forward_hidden(gaje_hip_model *m, uint32_t token, int clear_cache, float *logits_host,
                                       float *h_norm_host) {
    clear_error();
    GAJE_TRY(check_model(m));
    DevState s;
    GAJE_TRY(forward_device(m, token, clear_cache != 0, false, s));
    if (logits_host)
        GAJE_HIP_CHECK(hipMemcpy(logits_host, m->logits, (size_t)m->vocab_out * 4, hipMemcpyDeviceToHost));
    if (h_norm_host)
        GAJE_HIP_CHECK(hipMemcpy(h_norm_host, m->hnorm, (size_t)m->n_embd * 4, hipMemcpyDeviceToHost));
    return GAJE_OK;
}

extern "C" int gaje_hip_clear_cache(gaje_hip_model *m) {
    GAJE_TRY(check_model(m));
    m->pos = 0;
    return GAJE_OK;
}

extern "C" int gaje_hip_cache_len(const gaje_hip_model *m, int64_t *len) {
    if (!m || !len) return set_error(GAJE_ERR_INVALID_ARG, "null argument");
    *len = m->pos;
    return GAJE_OK;
}

extern "C" int gaje_hip_set_kwta(gaje_hip_model *m, float ratio) {
    GAJE_TRY(check_model(m));
    m->kwta_ratio = ratio;
    m->block_kwta_ratio = ratio;  // set_k_wta_ratio also sets every block (python.rs:55-57)
    return GAJE_OK;
}

extern "C" int gaje_hip_get_kwta(const gaje_hip_model *m, float *ratio) {
    if (!m || !ratio) return set_error(GAJE_ERR_INVALID_ARG, "null argument");
    *ratio = m->kwta_ratio;
    return GAJE_OK;
}

extern "C" int gaje_hip_reserve(gaje_hip_model *m, int64_t positions) {
    GAJE_TRY(check_model(m));
    if (positions < 0) return set_error(GAJE_ERR_INVALID_ARG, "negative reservation");
    return m->n_layers > 0 ? reserve_ctx(m, positions) : GAJE_OK;
}

extern "C" int gaje_hip_prefill(gaje_hip_model *m, const uint32_t *ids, int64_t n, float *last_logits_host) {
    clear_error();
    GAJE_TRY(check_model(m));
    if (n < 0 || (n > 0 && !ids)) return set_error(GAJE_ERR_INVALID_ARG, "bad prefill arguments");
    if (n == 0) return GAJE_OK;
    GAJE_TRY(reserve_ctx(m, m->pos + n));
    if (!m->profile) GAJE_TRY(ensure_graph(m));
    GAJE_TRY(launch_state_set(m->st, (int32_t)m->pos, ids[0], -1, -1, 1, m->stream));
    for (int64_t i = 0; i < n; ++i) {
        // after the first token only the input id changes; a halted state stays halted
        if (i > 0) GAJE_TRY(launch_state_set(m->st, -1, ids[i], -1, -1, 0, m->stream));
        GAJE_TRY(run_token(m));
    }
    if (last_logits_host && m->kwta_ratio > 0.0f && m->kwta_ratio < 1.0f)
        GAJE_TRY(launch_kwta(m->logits, m->vocab_out, kwta_k(m->vocab_out, m->kwta_ratio), m->st, m->stream));
    DevState s;
    GAJE_TRY(read_state(m, s));
    const int64_t done = (int64_t)s.pos - m->pos;
    m->pos = s.pos;
    if (s.halted || s.nan_code != NAN_NONE) {
        (void)done;
        return nan_error(s);
    }
    if (last_logits_host)
        GAJE_HIP_CHECK(hipMemcpy(last_logits_host, m->logits, (size_t)m->vocab_out * 4, hipMemcpyDeviceToHost));
    return GAJE_OK;
}

namespace {

// Tokens per MFMA prefill pass (the activation buffers hold one chunk).
constexpr int64_t PREFILL_CHUNK = 1024;

int prefill_mfma_supported(const gaje_hip_model *m) {
    if (m->n_layers == 0) return GAJE_OK;
    if (m->hd != 64 && m->hd != 128)
        return set_error(GAJE_ERR_UNSUPPORTED, "MFMA prefill: head_dim %lld (64 or 128 only)", (long long)m->hd);
    for (const Layer &Ly : m->layers)
        for (const DevLinear *D : {&Ly.qkv, &Ly.o, &Ly.gate_up, &Ly.down})
            if (D->fmt != FMT_Q4_0 || D->a_ptr || D->rows_valid != D->N)
                return set_error(GAJE_ERR_UNSUPPORTED,
                                 "MFMA prefill needs complete Q4_0 body tensors without anchors (use gaje_hip_prefill)");
    return GAJE_OK;
}

int64_t prefill_kmax(const gaje_hip_model *m) { return std::max({m->n_embd, m->q_rows, m->ffn}); }

// Grow the prefill buffers to `rows` tokens (and the split-K partials their
// products need).
int prefill_reserve(gaje_hip_model *m, int64_t rows) {
    auto &f = m->pf;
    const Layer &L0 = m->layers[0];
    int64_t part = 0;
    for (const DevLinear *D : {&L0.qkv, &L0.o, &L0.gate_up, &L0.down})
        part = std::max(part, plan_gemm_q4_bs(rows, D->N, D->K).part_floats);
    if (rows <= f.rows && part <= f.part_floats) return GAJE_OK;
    rows = std::max(rows, f.rows);
    part = std::max(part, f.part_floats);
    GAJE_HIP_CHECK(hipStreamSynchronize(m->stream));
    for (void *p : {(void *)f.H, (void *)f.QKV, (void *)f.Q, (void *)f.ATT, (void *)f.GU, (void *)f.part, (void *)f.xh,
                    (void *)f.sh, (void *)f.sl, (void *)f.ex, (void *)f.ids, (void *)f.aws})
        if (p) m->release(p);
    uint16_t *kv16 = f.kv16;
    const int64_t kv16_keys = f.kv16_keys;
    f = gaje_hip_model::Prefill();
    f.kv16 = kv16;
    f.kv16_keys = kv16_keys;
    const int64_t kmax = prefill_kmax(m);
    GAJE_TRY(m->alloc(&f.H, (size_t)(rows * m->n_embd)));
    GAJE_TRY(m->alloc(&f.QKV, (size_t)(rows * L0.qkv.N)));
    GAJE_TRY(m->alloc(&f.Q, (size_t)(rows * m->q_rows)));
    GAJE_TRY(m->alloc(&f.ATT, (size_t)(rows * m->q_rows)));
    GAJE_TRY(m->alloc(&f.GU, (size_t)(rows * L0.gate_up.N)));
    GAJE_TRY(m->alloc(&f.xh, (size_t)(gemm_bs_plane_rows(rows) * 2 * kmax)));
    GAJE_TRY(m->alloc(&f.sh, (size_t)(rows * gemm_bs_sum_cols(kmax))));
    GAJE_TRY(m->alloc(&f.sl, (size_t)(rows * gemm_bs_sum_cols(kmax))));
    GAJE_TRY(m->alloc(&f.ex, (size_t)rows));
    GAJE_TRY(m->alloc(&f.ids, (size_t)rows));
    GAJE_TRY(m->alloc(&f.part, (size_t)part));
    GAJE_TRY(m->alloc(&f.aws, (size_t)prefill_attn_ws_floats(rows, m->n_head, m->hd)));
    f.rows = rows;
    f.part_floats = part;
    return GAJE_OK;
}

SplitParams prefill_split(const gaje_hip_model *m, const float *x, int64_t ldx, int64_t P, int64_t K) {
    SplitParams sp{};
    sp.x = x;
    sp.ldx = ldx;
    sp.eps = m->eps;
    sp.h_scale = 1.0f;
    sp.xh = m->pf.xh;
    sp.ldh = 2 * K;
    sp.ex = m->pf.ex;
    sp.M = P;
    sp.K = K;
    sp.sh = m->pf.sh;
    sp.sl = m->pf.sl;
    sp.ldsum = gemm_bs_sum_cols(K);
    sp.st = m->st;
    sp.st_a = sp.st_b = ST_NONE;
    return sp;
}

// Y[P][D.N] = rows of the current activation planes x D (+ bias) (+ resid).
// A deferred split-K reduce: the product's partials wait in pf.part for the
// next split pass, which forms the rows itself (SplitParams' prologue).
struct PendingReduce {
    int32_t nsplit = 0;  // 0: none
    const float *bias = nullptr;
    int64_t bias_len = 0;
    bool resid = false;
    int32_t st_a = ST_NONE, st_b = ST_NONE, layer = 0;
};

void take_pending(const gaje_hip_model *m, PendingReduce &pr, SplitParams &sp) {
    if (!pr.nsplit) return;
    sp.part = m->pf.part;
    sp.nsplit = pr.nsplit;
    sp.bias = pr.bias;
    sp.bias_len = pr.bias_len;
    sp.resid = pr.resid ? sp.x : nullptr;
    sp.st_ya = pr.st_a;
    sp.st_yb = pr.st_b;
    sp.y_layer = pr.layer;
    pr = PendingReduce();
}

// With `pending`, a split-K product leaves its reduce to the next split pass.
int prefill_gemm(gaje_hip_model *m, const DevLinear &D, int64_t P, float *y, const float *resid, int32_t layer,
                 int32_t st_a, int32_t st_b, PendingReduce *pending = nullptr) {
    const auto &f = m->pf;
    const GemmBsPlan pl = plan_gemm_q4_bs(P, D.N, D.K);
    if (pl.part_floats > f.part_floats) return set_error(GAJE_ERR_INVALID_ARG, "prefill: split-K buffer too small");
    GemmBsParams p{};
    p.wf = D.wf;
    p.wsc = D.wsc;
    p.nbp4 = q4_frag_nbp4(D.K);
    p.mins = D.mins;
    p.ldm = D.ldm;
    p.xh = f.xh;
    p.plane_rows = gemm_bs_plane_rows(f.rows);
    p.sh = f.sh;
    p.sl = f.sl;
    p.ex = f.ex;
    p.ldh = 2 * D.K;
    p.ldsum = gemm_bs_sum_cols(D.K);
    p.bias = D.bias;
    p.bias_len = D.bias_len;
    p.resid = resid;
    p.ldr = D.N;
    p.y = y;
    p.ldy = D.N;
    p.part = f.part;
    p.M = P;
    p.N = D.N;
    p.nb = (int32_t)(D.K / 32);
    p.st = m->st;
    p.layer = layer;
    p.st_a = st_a;
    p.st_b = st_b;
    if (pending && pl.splits > 1 && (!resid || resid == y)) {
        p.defer_reduce = 1;
        pending->nsplit = pl.splits;
        pending->bias = D.bias;
        pending->bias_len = D.bias_len;
        pending->resid = resid != nullptr;
        pending->st_a = st_a;
        pending->st_b = st_b;
        pending->layer = layer;
    }
    return launch_gemm_q4_bs(p, pl, m->stream);
}

// One block (RustGenomicBlock::forward_core, block/forward.rs:10-157) for the
// P tokens of the current chunk at positions pos..pos+P-1, in place on pf.H.
// `pending`: the previous block's down product may leave its split-K reduce
// to this block's first split pass, and this block's may leave its own to the
// next block's (never the last block's: its rows go to the head).
int prefill_layer(gaje_hip_model *m, int64_t l, int64_t pos, int64_t P, PendingReduce &pending) {
    Layer &Ly = m->layers[l];
    auto &f = m->pf;
    hipStream_t s = m->stream;
    const int32_t li = (int32_t)l;
    const size_t layer_kv = (size_t)m->n_kv * m->cap * m->hd;

    SplitParams sp = prefill_split(m, f.H, m->n_embd, P, m->n_embd);
    take_pending(m, pending, sp);
    sp.norm_w = Ly.attn_norm;
    sp.layer = li;
    sp.st_a = ST_INPUT;
    sp.st_b = Ly.attn_norm ? ST_ATTN_NORM : ST_NONE;
    GAJE_TRY(launch_split_rows(sp, s));
    PendingReduce qkv_pending;
    GAJE_TRY(prefill_gemm(m, Ly.qkv, P, f.QKV, nullptr, li, ST_NONE, ST_NONE, &qkv_pending));

    PrefillRopeParams rp{};
    rp.qkv = f.QKV;
    rp.ldq = Ly.qkv.N;
    rp.q_out = f.Q;
    rp.k_cache = m->k_cache + l * layer_kv;
    rp.v_cache = m->v_cache + l * layer_kv;
    rp.cap = m->cap;
    rp.pos0 = pos;
    rp.P = P;
    rp.n_head = (int32_t)m->n_head;
    rp.n_kv = (int32_t)m->n_kv;
    rp.head_dim = (int32_t)m->hd;
    rp.rope_split = m->rope_split;
    rp.rope_cos = m->rope_cos;
    rp.rope_sin = m->rope_sin;
    if (qkv_pending.nsplit) {  // the qkv product's reduce, in the RoPE pass
        rp.part = f.part;
        rp.nsplit = qkv_pending.nsplit;
        rp.bias = qkv_pending.bias;
        rp.bias_len = qkv_pending.bias_len;
    }
    rp.kv16 = f.kv16;
    rp.kv16_ntiles = (int32_t)((pos + P + 31) / 32);
    GAJE_TRY(launch_rope_kv(rp, s));

    PrefillAttnParams ap{};
    ap.q = f.Q;
    ap.k_cache = rp.k_cache;
    ap.v_cache = rp.v_cache;
    ap.cap = m->cap;
    ap.pos0 = pos;
    ap.P = P;
    ap.n_head = (int32_t)m->n_head;
    ap.n_kv = (int32_t)m->n_kv;
    ap.head_dim = (int32_t)m->hd;
    ap.out = f.ATT;
    ap.ws = f.aws;
    ap.kv16 = f.kv16;
    ap.kv16_keys = f.kv16_keys;
    ap.kv16_rope = 1;
    ap.merged_later = 1;  // the merge is the next split pass's prologue
    GAJE_TRY(launch_prefill_attention(ap, s));

    sp = prefill_split(m, f.ATT, m->q_rows, P, m->q_rows);
    sp.attn_ws = f.aws;
    sp.attn_kch = prefill_attn_kch(pos + P);
    sp.attn_pos0 = pos;
    sp.attn_hd = (int32_t)m->hd;
    sp.attn_heads = (int32_t)m->n_head;
    GAJE_TRY(launch_split_rows(sp, s));
    GAJE_TRY(prefill_gemm(m, Ly.o, P, f.H, f.H, li, ST_NONE, ST_NONE, &pending));

    sp = prefill_split(m, f.H, m->n_embd, P, m->n_embd);
    take_pending(m, pending, sp);
    sp.norm_w = Ly.ffn_norm;
    GAJE_TRY(launch_split_rows(sp, s));
    GAJE_TRY(prefill_gemm(m, Ly.gate_up, P, f.GU, nullptr, li, ST_NONE, ST_NONE));

    sp = prefill_split(m, f.GU, Ly.gate_up.N, P, m->ffn);
    sp.up = f.GU + m->ffn;
    sp.gnorm = m->use_genomic_norm;
    sp.layer = li;
    sp.st_a = ST_UP;
    sp.st_b = ST_FFN_OUT;
    GAJE_TRY(launch_split_rows(sp, s));
    const bool kwta = m->block_kwta_ratio > 0.0f && m->block_kwta_ratio < 1.0f;
    GAJE_TRY(prefill_gemm(m, Ly.down, P, f.H, f.H, li, ST_PROJ_FFN, ST_FINAL,
                          l + 1 < m->n_layers && !kwta ? &pending : nullptr));

    if (kwta) {
        const int64_t k = kwta_k(m->n_embd, m->block_kwta_ratio);
        for (int64_t t = 0; t < P; ++t) GAJE_TRY(launch_kwta(f.H + t * m->n_embd, m->n_embd, k, m->st, s));
    }
    return GAJE_OK;
}

}  // namespace

extern "C" int gaje_hip_prefill_mfma(gaje_hip_model *m, const uint32_t *ids, int64_t n, float *last_logits_host) {
    clear_error();
    GAJE_TRY(check_model(m));
    if (n < 0 || (n > 0 && !ids)) return set_error(GAJE_ERR_INVALID_ARG, "bad prefill arguments");
    if (n == 0) return GAJE_OK;
    GAJE_TRY(prefill_mfma_supported(m));
    const int64_t pos0 = m->pos;
    GAJE_TRY(reserve_ctx(m, pos0 + n));
    hipStream_t s = m->stream;
    if (m->n_layers > 0 && !m->layers[0].qkv.mins) {
        // the products' dense block mins and code fragments, built once per body tensor
        for (Layer &Ly : m->layers)
            for (DevLinear *D : {&Ly.qkv, &Ly.o, &Ly.gate_up, &Ly.down}) {
                D->ldm = gemm_bs_sum_cols(D->K);
                GAJE_TRY(m->alloc(&D->mins, (size_t)(D->N * D->ldm)));
                GAJE_TRY(launch_q4_mins(D->w, D->N, D->K, D->mins, D->ldm, s));
                GAJE_TRY(m->alloc(&D->wf, (size_t)q4_frag_halves(D->N, D->K)));
                GAJE_TRY(m->alloc(&D->wsc, (size_t)q4_frag_scale_floats(D->N, D->K)));
                GAJE_TRY(launch_q4_frags(D->w, D->N, D->K, D->wf, D->wsc, s));
            }
    }
    if (m->n_layers > 0 && m->pf.kv16_keys < pos0 + n) {
        // the attention's converted keys and values, for every position this prompt reaches
        GAJE_HIP_CHECK(hipStreamSynchronize(s));
        if (m->pf.kv16) m->release(m->pf.kv16);
        m->pf.kv16 = nullptr;
        m->pf.kv16_keys = 0;
        const int64_t keys = (pos0 + n + 255) / 256 * 256;
        GAJE_TRY(m->alloc(&m->pf.kv16, (size_t)prefill_kv16_halves(keys, m->n_kv, m->hd)));
        // zero once: the attention reads whole 32-key tiles, and its value
        // tiles past the last key must hold finite numbers
        GAJE_HIP_CHECK(hipMemsetAsync(m->pf.kv16, 0, (size_t)prefill_kv16_halves(keys, m->n_kv, m->hd) * 2, s));
        m->pf.kv16_keys = keys;
    }
    GAJE_TRY(launch_state_set(m->st, (int32_t)pos0, ids[n - 1], -1, -1, 1, s));
    int64_t last_rows = 0;
    for (int64_t c0 = 0; c0 < n; c0 += PREFILL_CHUNK) {
        const int64_t P = std::min(PREFILL_CHUNK, n - c0);
        if (m->n_layers > 0) GAJE_TRY(prefill_reserve(m, P));
        else if (m->pf.rows < P) {
            if (m->pf.H) m->release(m->pf.H);
            if (m->pf.ids) m->release(m->pf.ids);
            GAJE_TRY(m->alloc(&m->pf.H, (size_t)(P * m->n_embd)));
            GAJE_TRY(m->alloc(&m->pf.ids, (size_t)P));
            m->pf.rows = P;
        }
        auto &f = m->pf;
        GAJE_HIP_CHECK(hipMemcpyAsync(f.ids, ids + c0, (size_t)P * 4, hipMemcpyHostToDevice, s));
        EmbedParams ep;
        memset(&ep, 0, sizeof ep);
        ep.w = m->embd.w;
        ep.fmt = m->embd.fmt;
        ep.lut = m->embd.lut;
        ep.lut_rows_own = m->embd.lut_rows_own;
        ep.lut_block_stride = m->embd.lut_block_stride;
        ep.lut_len = m->embd.lut_len;
        ep.vocab = m->vocab_embd;
        ep.rows_valid = m->embd.rows_valid;
        ep.K = m->n_embd;
        ep.h = f.H;
        GAJE_TRY(launch_embed_rows(ep, f.ids, P, s));
        PendingReduce pending;
        for (int64_t l = 0; l < m->n_layers; ++l) GAJE_TRY(prefill_layer(m, l, pos0 + c0, P, pending));
        last_rows = P;
        // the ids copy reads host memory the caller owns only for this call
        GAJE_HIP_CHECK(hipStreamSynchronize(s));
    }
    DevState st;
    GAJE_TRY(read_state(m, st));
    if (st.nan_code != NAN_NONE) return nan_error(st);  // nothing is committed: the cache length stays pos0

    // the last token's logits, argmax and position advance, as the decode step ends
    GAJE_HIP_CHECK(hipMemcpyAsync(m->h, m->pf.H + (last_rows - 1) * m->n_embd, (size_t)m->n_embd * 4,
                                  hipMemcpyDeviceToDevice, s));
    GAJE_TRY(launch_state_set(m->st, (int32_t)(pos0 + n - 1), ids[n - 1], -1, -1, 1, s));
    GAJE_TRY(enqueue_head(m));
    if (last_logits_host && m->kwta_ratio > 0.0f && m->kwta_ratio < 1.0f)
        GAJE_TRY(launch_kwta(m->logits, m->vocab_out, kwta_k(m->vocab_out, m->kwta_ratio), m->st, s));
    GAJE_TRY(read_state(m, st));
    if (st.halted || st.nan_code != NAN_NONE) return nan_error(st);
    m->pos = st.pos;
    if (last_logits_host)
        GAJE_HIP_CHECK(hipMemcpy(last_logits_host, m->logits, (size_t)m->vocab_out * 4, hipMemcpyDeviceToHost));
    return GAJE_OK;
}

// ------------------------------------------------------------ batched decode --

struct gaje_hip_batch {
    gaje_hip_model *m = nullptr;
    int64_t nseq = 0, lanes = 0, cap = 0;
    float *k_cache = nullptr, *v_cache = nullptr;  // [layer][seq][n_kv][head_dim][cap]
    float *rope_cos = nullptr, *rope_sin = nullptr;
    float *H = nullptr, *XN = nullptr, *QKV = nullptr, *Q = nullptr, *ATT = nullptr, *GU = nullptr, *ACT = nullptr,
          *LOG = nullptr;
    uint32_t *ids = nullptr, *out = nullptr;  // fed tokens / greedy outputs [seq][n]
    int64_t ids_cap = 0, out_cap = 0;
    BatchState st{};
    std::vector<int32_t> pos;  // host mirror of st.pos
    std::vector<void *> allocs;

    ~gaje_hip_batch() {
        for (void *p : allocs) (void)hipFree(p);
    }
    template <class T>
    int alloc(T **p, size_t count) {
        *p = nullptr;
        if (count == 0) return GAJE_OK;
        void *v = nullptr;
        GAJE_HIP_CHECK(hipMalloc(&v, count * sizeof(T)));
        allocs.push_back(v);
        *p = (T *)v;
        return GAJE_OK;
    }
    void release(void *p) {
        for (auto it = allocs.begin(); it != allocs.end(); ++it)
            if (*it == p) {
                (void)hipFree(p);
                allocs.erase(it);
                return;
            }
    }
};

namespace {

int batch_supported(const gaje_hip_model *m) {
    for (const Layer &Ly : m->layers)
        for (const DevLinear *D : {&Ly.qkv, &Ly.o, &Ly.gate_up, &Ly.down})
            if (D->fmt != FMT_Q4_0 || D->rows_valid != D->N)
                return set_error(GAJE_ERR_UNSUPPORTED, "batched decode needs complete Q4_0 body tensors");
    const DevLinear &H = m->lm_head;
    if (H.fmt != FMT_F32 || !H.f32_tiled || H.rows_valid != H.N || H.a_ptr)
        return set_error(GAJE_ERR_UNSUPPORTED, "batched decode needs an f32 lm_head (K %% 8 == 0) without anchors");
    return GAJE_OK;
}

BatchGemvParams batch_gemv(const gaje_hip_batch *b, const DevLinear &D, const float *x, int64_t ldx, float *y,
                           int64_t ldy) {
    BatchGemvParams p{};
    p.w = D.w;
    p.fmt = D.fmt;
    p.f32_tiled = D.f32_tiled;
    p.nb = (int32_t)(D.K / 32);
    p.N = D.N;
    p.K = D.K;
    p.x = x;
    p.ldx = ldx;
    p.nv = (int32_t)b->lanes;
    p.bias = D.bias;
    p.bias_len = D.bias_len;
    p.a_ptr = D.a_ptr;
    p.a_col = D.a_col;
    p.a_val = D.a_val;
    p.mode = MODE_STORE;
    p.y = y;
    p.ldy = ldy;
    p.nan_codes = b->st.nan_codes;
    p.st_a = p.st_b = ST_NONE;
    return p;
}

BatchRowParams batch_rows(const gaje_hip_batch *b, const float *x, int64_t ldx, float *y, int64_t ldy, int64_t K) {
    BatchRowParams r{};
    r.x = x;
    r.ldx = ldx;
    r.y = y;
    r.ldy = ldy;
    r.K = K;
    r.nv = (int32_t)b->lanes;
    r.eps = b->m->eps;
    r.h_scale = 1.0f;
    r.nan_codes = b->st.nan_codes;
    r.st_a = r.st_b = ST_NONE;
    return r;
}

// One step of every running sequence (the batched counterpart of enqueue_token).
int batch_enqueue_step(gaje_hip_batch *b, const uint32_t *ids, int64_t n, int64_t i, uint32_t *out, bool greedy) {
    gaje_hip_model *m = b->m;
    hipStream_t s = m->stream;
    const int64_t L = b->lanes, E = m->n_embd;
    GAJE_TRY(launch_batch_begin(b->st, ids, n, i, s));
    EmbedParams ep;
    memset(&ep, 0, sizeof ep);
    ep.w = m->embd.w;
    ep.fmt = m->embd.fmt;
    ep.lut = m->embd.lut;
    ep.lut_rows_own = m->embd.lut_rows_own;
    ep.lut_block_stride = m->embd.lut_block_stride;
    ep.lut_len = m->embd.lut_len;
    ep.vocab = m->vocab_embd;
    ep.rows_valid = m->embd.rows_valid;
    ep.K = E;
    ep.h = b->H;
    GAJE_TRY(launch_embed_rows(ep, b->st.embed_ids, L, s));
    const int64_t seq_kv = m->n_kv * m->hd * b->cap;
    const int64_t qkvN = m->layers.empty() ? 0 : m->layers[0].qkv.N, guN = m->layers.empty() ? 0 : m->layers[0].gate_up.N;
    for (int64_t l = 0; l < m->n_layers; ++l) {
        Layer &Ly = m->layers[l];
        const int32_t li = (int32_t)l;
        float *kc = b->k_cache + l * b->nseq * seq_kv, *vc = b->v_cache + l * b->nseq * seq_kv;
        BatchRowParams r = batch_rows(b, b->H, E, b->XN, E, E);
        r.w = Ly.attn_norm;  // null: the rows as they are
        r.chain_major = 1;
        r.layer = li;
        r.st_a = ST_INPUT;
        r.st_b = Ly.attn_norm ? ST_ATTN_NORM : ST_NONE;
        GAJE_TRY(launch_rmsnorm_rows(r, s));
        GAJE_TRY(launch_gemv_batch(batch_gemv(b, Ly.qkv, b->XN, E, b->QKV, qkvN), s));
        PrefillRopeParams rp{};
        rp.qkv = b->QKV;
        rp.ldq = qkvN;
        rp.q_out = b->Q;
        rp.k_cache = kc;
        rp.v_cache = vc;
        rp.cap = b->cap;
        rp.P = L;
        rp.n_head = (int32_t)m->n_head;
        rp.n_kv = (int32_t)m->n_kv;
        rp.head_dim = (int32_t)m->hd;
        rp.rope_split = m->rope_split;
        rp.rope_cos = b->rope_cos;
        rp.rope_sin = b->rope_sin;
        rp.seq_pos = b->st.cur_pos;
        rp.seq_kv_stride = seq_kv;
        GAJE_TRY(launch_rope_kv(rp, s));
        AttnParams ap{};
        ap.q = b->Q;
        ap.k_cache = kc;
        ap.v_cache = vc;
        ap.kv_head_stride = b->cap * m->hd;
        ap.n_head = (int32_t)m->n_head;
        ap.n_head_kv = (int32_t)m->n_kv;
        ap.head_dim = (int32_t)m->hd;
        ap.kv_cap = b->cap;
        ap.out = b->ATT;
        ap.seq_pos = b->st.cur_pos;
        ap.seq_kv_stride = seq_kv;
        ap.seq_q_stride = m->q_rows;
        ap.n_seq = (int32_t)b->nseq;
        ap.out_chain_major = 1;
        ap.seq_nan = b->st.nan_codes;
        ap.layer = (int32_t)li;
        GAJE_TRY(launch_attention(ap, s));
        BatchGemvParams g = batch_gemv(b, Ly.o, b->ATT, m->q_rows, b->H, E);
        g.mode = MODE_RESIDUAL;
        GAJE_TRY(launch_gemv_batch(g, s));
        r = batch_rows(b, b->H, E, b->XN, E, E);
        r.w = Ly.ffn_norm;
        r.chain_major = 1;
        GAJE_TRY(launch_rmsnorm_rows(r, s));
        GAJE_TRY(launch_gemv_batch(batch_gemv(b, Ly.gate_up, b->XN, E, b->GU, guN), s));
        r = batch_rows(b, b->GU, guN, b->ACT, m->ffn, m->ffn);
        r.gnorm = m->use_genomic_norm;
        r.chain_major = 1;
        r.layer = li;
        r.st_a = ST_UP;
        r.st_b = ST_FFN_OUT;
        GAJE_TRY(launch_swiglu_rows(r, s));
        g = batch_gemv(b, Ly.down, b->ACT, m->ffn, b->H, E);
        g.mode = MODE_RESIDUAL;
        g.layer = li;
        g.st_a = ST_PROJ_FFN;
        g.st_b = ST_FINAL;
        GAJE_TRY(launch_gemv_batch(g, s));
        if (m->block_kwta_ratio > 0.0f && m->block_kwta_ratio < 1.0f) {
            const int64_t k = kwta_k(E, m->block_kwta_ratio);
            for (int64_t q = 0; q < b->nseq; ++q) GAJE_TRY(launch_kwta(b->H + q * E, E, k, nullptr, s));
        }
    }
    BatchRowParams r = batch_rows(b, b->H, E, b->XN, E, E);
    r.w = m->output_norm;
    GAJE_TRY(launch_rmsnorm_rows(r, s));
    GAJE_TRY(launch_gemv_batch(batch_gemv(b, m->lm_head, b->XN, E, b->LOG, m->vocab_out), s));
    GAJE_TRY(launch_argmax_rows(b->LOG, m->vocab_out, m->vocab_out, b->nseq, b->st.next, s));
    return launch_batch_end(b->st, out, n, i, greedy ? 1 : 0, s);
}

// Reads the device state back; a sequence halted by a guard reports the
// reference's message (the first such sequence's).
int batch_sync(gaje_hip_batch *b, int32_t *status) {
    std::vector<int32_t> halted((size_t)b->lanes);
    std::vector<uint32_t> err((size_t)b->lanes);
    hipStream_t s = b->m->stream;
    GAJE_HIP_CHECK(hipMemcpyAsync(b->pos.data(), b->st.pos, (size_t)b->lanes * 4, hipMemcpyDeviceToHost, s));
    GAJE_HIP_CHECK(hipMemcpyAsync(halted.data(), b->st.halted, (size_t)b->lanes * 4, hipMemcpyDeviceToHost, s));
    GAJE_HIP_CHECK(hipMemcpyAsync(err.data(), b->st.err, (size_t)b->lanes * 4, hipMemcpyDeviceToHost, s));
    GAJE_HIP_CHECK(hipStreamSynchronize(s));
    int first = -1;
    for (int64_t q = 0; q < b->nseq; ++q) {
        if (status) status[q] = halted[q] ? (int32_t)(err[q] % 8) + 1 : 0;
        if (halted[q] && first < 0) first = (int)q;
    }
    if (first >= 0)
        return set_error((int)(err[first] % 8) == ST_WAIT ? GAJE_ERR_HIP : GAJE_ERR_NAN, "%s",
                         nan_message((int)(err[first] % 8)));
    return GAJE_OK;
}

int batch_check(gaje_hip_batch *b, int64_t steps) {
    if (!b) return set_error(GAJE_ERR_INVALID_ARG, "null batch handle");
    if (!b->m) return set_error(GAJE_ERR_INVALID_ARG, "the batch's model was closed");
    GAJE_HIP_CHECK(hipSetDevice(b->m->device));
    for (int64_t q = 0; q < b->nseq; ++q)
        if (b->pos[q] + steps > b->cap)
            return set_error(GAJE_ERR_INVALID_ARG, "sequence %lld: %lld cached + %lld steps exceed the capacity %lld",
                             (long long)q, (long long)b->pos[q], (long long)steps, (long long)b->cap);
    return GAJE_OK;
}

}  // namespace

extern "C" int gaje_hip_batch_open(gaje_hip_model *m, int64_t n_seq, int64_t capacity, gaje_hip_batch **out) {
    clear_error();
    GAJE_TRY(check_model(m));
    if (!out) return set_error(GAJE_ERR_INVALID_ARG, "null output");
    *out = nullptr;
    if (n_seq < 1 || n_seq > 16) return set_error(GAJE_ERR_INVALID_ARG, "batch of %lld sequences (1..16)", (long long)n_seq);
    if (capacity < 1 || capacity > MAX_CTX)
        return set_error(GAJE_ERR_INVALID_ARG, "capacity %lld outside 1..%lld", (long long)capacity, (long long)MAX_CTX);
    GAJE_TRY(batch_supported(m));
    std::unique_ptr<gaje_hip_batch> b(new gaje_hip_batch());
    b->m = m;
    b->nseq = n_seq;
    b->lanes = batch_lanes(n_seq);
    b->cap = (capacity + 63) / 64 * 64;
    b->cap = std::min<int64_t>(b->cap, MAX_CTX);
    const int64_t L = b->lanes, E = m->n_embd;
    const size_t kv = (size_t)std::max<int64_t>(m->n_layers, 1) * n_seq * m->n_kv * m->hd * b->cap;
    GAJE_TRY(b->alloc(&b->k_cache, kv));
    GAJE_TRY(b->alloc(&b->v_cache, kv));
    {
        // the decode path's RoPE table (build_rope) at this capacity
        const int64_t half = m->hd / 2;
        std::vector<float> c((size_t)(b->cap * half)), sn((size_t)(b->cap * half));
        for (int64_t i = 0; i < half; ++i) {
            const float expo = (2.0f * (float)i) / (float)m->hd;
            const float freq = 1.0f / powf(m->rope_base, expo);
            for (int64_t p = 0; p < b->cap; ++p) {
                const float theta = (float)p * freq;
                c[p * half + i] = cosf(theta);
                sn[p * half + i] = sinf(theta);
            }
        }
        GAJE_TRY(b->alloc(&b->rope_cos, c.size()));
        GAJE_TRY(b->alloc(&b->rope_sin, sn.size()));
        GAJE_HIP_CHECK(hipMemcpy(b->rope_cos, c.data(), c.size() * 4, hipMemcpyHostToDevice));
        GAJE_HIP_CHECK(hipMemcpy(b->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    }
    const int64_t qkvN = m->layers.empty() ? 1 : m->layers[0].qkv.N, guN = m->layers.empty() ? 2 : m->layers[0].gate_up.N;
    const int64_t qn = std::max<int64_t>(m->q_rows, 1), ffn = std::max<int64_t>(m->ffn, 1);
    GAJE_TRY(b->alloc(&b->H, (size_t)(L * E)));
    GAJE_TRY(b->alloc(&b->XN, (size_t)(L * E)));
    GAJE_TRY(b->alloc(&b->QKV, (size_t)(L * qkvN)));
    GAJE_TRY(b->alloc(&b->Q, (size_t)(L * qn)));
    GAJE_TRY(b->alloc(&b->ATT, (size_t)(L * qn)));
    GAJE_TRY(b->alloc(&b->GU, (size_t)(L * guN)));
    GAJE_TRY(b->alloc(&b->ACT, (size_t)(L * ffn)));
    GAJE_TRY(b->alloc(&b->LOG, (size_t)(L * m->vocab_out)));
    // rows of idle lanes are computed and discarded; zeroed, they stay finite
    GAJE_HIP_CHECK(hipMemset(b->H, 0, (size_t)(L * E) * 4));
    GAJE_HIP_CHECK(hipMemset(b->XN, 0, (size_t)(L * E) * 4));
    GAJE_HIP_CHECK(hipMemset(b->QKV, 0, (size_t)(L * qkvN) * 4));
    GAJE_HIP_CHECK(hipMemset(b->Q, 0, (size_t)(L * qn) * 4));
    GAJE_HIP_CHECK(hipMemset(b->ATT, 0, (size_t)(L * qn) * 4));
    GAJE_HIP_CHECK(hipMemset(b->GU, 0, (size_t)(L * guN) * 4));
    GAJE_HIP_CHECK(hipMemset(b->ACT, 0, (size_t)(L * ffn) * 4));
    BatchState &st = b->st;
    st.nseq = (int32_t)n_seq;
    st.lanes = (int32_t)L;
    GAJE_TRY(b->alloc(&st.pos, (size_t)L));
    GAJE_TRY(b->alloc(&st.cur_pos, (size_t)L));
    GAJE_TRY(b->alloc(&st.halted, (size_t)L));
    GAJE_TRY(b->alloc(&st.err, (size_t)L));
    GAJE_TRY(b->alloc(&st.tok, (size_t)L));
    GAJE_TRY(b->alloc(&st.embed_ids, (size_t)L));
    GAJE_TRY(b->alloc(&st.next, (size_t)L));
    GAJE_TRY(b->alloc(&st.nan_codes, (size_t)L));
    for (void *p : {(void *)st.pos, (void *)st.cur_pos, (void *)st.halted, (void *)st.err, (void *)st.tok,
                    (void *)st.embed_ids, (void *)st.next})
        GAJE_HIP_CHECK(hipMemset(p, 0, (size_t)L * 4));
    b->pos.assign((size_t)L, 0);
    m->batches.push_back(b.get());
    *out = b.release();
    return GAJE_OK;
}

void batch_detach(gaje_hip_batch *b) {
    for (void *p : b->allocs) (void)hipFree(p);
    b->allocs.clear();
    b->m = nullptr;
}

extern "C" void gaje_hip_batch_close(gaje_hip_batch *b) {
    if (!b) return;
    if (b->m) {
        (void)hipSetDevice(b->m->device);
        (void)hipStreamSynchronize(b->m->stream);
        auto &v = b->m->batches;
        v.erase(std::remove(v.begin(), v.end(), b), v.end());
    }
    delete b;
}

extern "C" int gaje_hip_batch_reset(gaje_hip_batch *b, int64_t seq) {
    clear_error();
    GAJE_TRY(batch_check(b, 0));
    if (seq < -1 || seq >= b->nseq) return set_error(GAJE_ERR_INVALID_ARG, "sequence %lld out of range", (long long)seq);
    for (int64_t q = 0; q < b->nseq; ++q)
        if (seq < 0 || q == seq) {
            const int32_t zero = 0;
            GAJE_HIP_CHECK(hipMemcpyAsync(b->st.pos + q, &zero, 4, hipMemcpyHostToDevice, b->m->stream));
            GAJE_HIP_CHECK(hipMemcpyAsync(b->st.halted + q, &zero, 4, hipMemcpyHostToDevice, b->m->stream));
            GAJE_HIP_CHECK(hipStreamSynchronize(b->m->stream));
            b->pos[q] = 0;
        }
    return GAJE_OK;
}

extern "C" int gaje_hip_batch_cache_len(const gaje_hip_batch *b, int64_t seq, int64_t *len) {
    if (!b || !b->m || !len || seq < 0 || seq >= b->nseq) return set_error(GAJE_ERR_INVALID_ARG, "bad arguments");
    *len = b->pos[seq];
    return GAJE_OK;
}

extern "C" int gaje_hip_batch_feed(gaje_hip_batch *b, const uint32_t *ids, int64_t n, float *last_logits_host,
                                   int32_t *status) {
    clear_error();
    GAJE_TRY(batch_check(b, n));
    if (n < 0 || (n > 0 && !ids)) return set_error(GAJE_ERR_INVALID_ARG, "bad feed arguments");
    if (n == 0) return GAJE_OK;
    gaje_hip_model *m = b->m;
    hipStream_t s = m->stream;
    const size_t need = (size_t)(b->nseq * n);
    if ((int64_t)need > b->ids_cap) {
        if (b->ids) b->release(b->ids);
        GAJE_TRY(b->alloc(&b->ids, need));
        b->ids_cap = (int64_t)need;
    }
    GAJE_HIP_CHECK(hipMemcpyAsync(b->ids, ids, need * 4, hipMemcpyHostToDevice, s));
    for (int64_t i = 0; i < n; ++i) GAJE_TRY(batch_enqueue_step(b, b->ids, n, i, nullptr, false));
    if (last_logits_host && m->kwta_ratio > 0.0f && m->kwta_ratio < 1.0f)
        for (int64_t q = 0; q < b->nseq; ++q)
            GAJE_TRY(launch_kwta(b->LOG + q * m->vocab_out, m->vocab_out, kwta_k(m->vocab_out, m->kwta_ratio), nullptr, s));
    const int rc = batch_sync(b, status);
    if (last_logits_host)
        GAJE_HIP_CHECK(hipMemcpy(last_logits_host, b->LOG, (size_t)(b->nseq * m->vocab_out) * 4, hipMemcpyDeviceToHost));
    return rc;
}

extern "C" int gaje_hip_batch_decode_greedy(gaje_hip_batch *b, const uint32_t *first, int64_t n, uint32_t *out_tokens,
                                            int32_t *status) {
    clear_error();
    GAJE_TRY(batch_check(b, n));
    if (n < 0 || (n > 0 && (!first || !out_tokens))) return set_error(GAJE_ERR_INVALID_ARG, "bad decode arguments");
    if (n == 0) return GAJE_OK;
    gaje_hip_model *m = b->m;
    hipStream_t s = m->stream;
    const size_t need = (size_t)(b->nseq * n);
    if ((int64_t)need > b->out_cap) {
        if (b->out) b->release(b->out);
        GAJE_TRY(b->alloc(&b->out, need));
        b->out_cap = (int64_t)need;
    }
    GAJE_HIP_CHECK(hipMemcpyAsync(b->st.tok, first, (size_t)b->nseq * 4, hipMemcpyHostToDevice, s));
    GAJE_TRY(launch_fill_u32(b->out, 0u, (int64_t)need, s));
    for (int64_t i = 0; i < n; ++i) GAJE_TRY(batch_enqueue_step(b, nullptr, n, i, b->out, true));
    const int rc = batch_sync(b, status);
    GAJE_HIP_CHECK(hipMemcpy(out_tokens, b->out, need * 4, hipMemcpyDeviceToHost));
    return rc;
}

extern "C" int gaje_hip_greedy_next(gaje_hip_model *m, uint32_t token, uint32_t *next) {
    clear_error();
    GAJE_TRY(check_model(m));
    if (!next) return set_error(GAJE_ERR_INVALID_ARG, "null output");
    DevState s;
    GAJE_TRY(forward_device(m, token, false, false, s));
    *next = s.token;
    return GAJE_OK;
}

extern "C" int gaje_hip_decode_greedy(gaje_hip_model *m, uint32_t first_token, int64_t n, uint32_t *out_tokens) {
    clear_error();
    GAJE_TRY(check_model(m));
    if (n < 0 || (n > 0 && !out_tokens)) return set_error(GAJE_ERR_INVALID_ARG, "bad decode arguments");
    if (n == 0) return GAJE_OK;
    GAJE_TRY(reserve_ctx(m, m->pos + n));
    if (n > m->out_cap) {
        m->release(m->out_tokens);
        m->out_cap = n;
        GAJE_TRY(m->alloc(&m->out_tokens, (size_t)n));
        drop_graph(m);
    }
    if (!m->profile) GAJE_TRY(ensure_graph(m));
    GAJE_TRY(launch_state_set(m->st, (int32_t)m->pos, first_token, (int32_t)m->out_cap, 0, 1, m->stream));
    for (int64_t i = 0; i < n; ++i) GAJE_TRY(run_token(m));
    DevState s;
    GAJE_HIP_CHECK(hipMemcpyAsync(out_tokens, m->out_tokens, (size_t)n * 4, hipMemcpyDeviceToHost, m->stream));
    GAJE_TRY(read_state(m, s));
    m->pos = s.pos;
    if (s.halted || s.nan_code != NAN_NONE) return nan_error(s);
    return GAJE_OK;
}

namespace {

// generate_native_core's greedy loop (temperature <= 1e-5) with the choice,
// the penalty, EOS and the loop detector on the device: after each token step
// gen_select (penalty > 1, over the K-WTA-filtered logits) and gen_control run
// on the stream, and the host only reads the loop's state every GEN_CHUNK
// tokens to stop enqueuing.  The prompt has been fed; the state's token is
// the argmax of its last logits.
constexpr int64_t GEN_CHUNK = 32;

int generate_device(gaje_hip_model *m, int64_t max_new, float repetition_penalty, const uint32_t *eos_ids,
                    int64_t n_eos, uint32_t *out_tokens, int64_t *n_out) {
    if (!m->gen) {
        GAJE_TRY(m->alloc(&m->gen, 1));
        GAJE_TRY(m->alloc(&m->gen_seen, (size_t)((m->vocab_out + 31) / 32)));
    }
    if (max_new > m->gen_cap) {
        if (m->gen_tokens) m->release(m->gen_tokens);
        m->gen_tokens = nullptr;
        m->gen_cap = 0;
        GAJE_TRY(m->alloc(&m->gen_tokens, (size_t)max_new));
        m->gen_cap = max_new;
    }
    GAJE_TRY(reserve_ctx(m, m->pos + max_new));
    if (!m->profile) GAJE_TRY(ensure_graph(m));
    GenState g;
    memset(&g, 0, sizeof g);
    g.n_eos = (int32_t)n_eos;
    g.penalty = repetition_penalty;
    for (int64_t i = 0; i < n_eos; ++i) g.eos[i] = eos_ids[i];
    GAJE_HIP_CHECK(hipMemcpyAsync(m->gen, &g, sizeof g, hipMemcpyHostToDevice, m->stream));
    GAJE_TRY(launch_fill_u32(m->gen_seen, 0u, (m->vocab_out + 31) / 32, m->stream));
    const bool select = repetition_penalty > 1.0f;
    const bool kwta = m->kwta_ratio > 0.0f && m->kwta_ratio < 1.0f;
    DevState s;
    GenState gs;
    for (int64_t i = 0; i < max_new;) {
        const int64_t end = std::min(max_new, i + GEN_CHUNK);
        for (; i < end; ++i) {
            if (i > 0) GAJE_TRY(run_token(m));  // forward_core of the previous token
            if (select) {
                // forward_core's K-WTA, then the penalised choice (K-WTA keeps the
                // maximum, so without a penalty the token step's argmax stands)
                if (kwta) GAJE_TRY(launch_kwta(m->logits, m->vocab_out, kwta_k(m->vocab_out, m->kwta_ratio), m->st, m->stream));
                GAJE_TRY(launch_gen_select(m->logits, m->vocab_out, m->gen_seen, m->st, m->gen, m->stream));
            }
            GAJE_TRY(launch_gen_control(m->st, m->gen, m->gen_seen, m->vocab_out, m->gen_tokens, select, m->stream));
        }
        // a loop that ends by count forwards its last token too (llm/forward.rs:320)
        if (i == max_new) GAJE_TRY(run_token(m));
        GAJE_HIP_CHECK(hipMemcpyAsync(&gs, m->gen, sizeof gs, hipMemcpyDeviceToHost, m->stream));
        GAJE_TRY(read_state(m, s));
        if (s.halted) break;
    }
    m->pos = s.pos;
    if (gs.n_gen > 0)
        GAJE_HIP_CHECK(hipMemcpy(out_tokens, m->gen_tokens, (size_t)gs.n_gen * 4, hipMemcpyDeviceToHost));
    if (n_out) *n_out = gs.n_gen;
    if (s.halted && gs.stop == GEN_RUNNING) return nan_error(s);
    return GAJE_OK;
}

}  // namespace

extern "C" int gaje_hip_generate(gaje_hip_model *m, const uint32_t *prompt, int64_t n_prompt, int64_t max_new,
                                 float temperature, float repetition_penalty, const uint32_t *eos_ids, int64_t n_eos,
                                 uint64_t seed, uint32_t *out_tokens, int64_t *n_out) {
    clear_error();
    GAJE_TRY(check_model(m));
    if (n_out) *n_out = 0;
    if (n_prompt <= 0 || !prompt) return set_error(GAJE_ERR_MODEL, "Prompt tokens cannot be empty");
    if (max_new < 0 || (max_new > 0 && !out_tokens) || (n_eos > 0 && !eos_ids))
        return set_error(GAJE_ERR_INVALID_ARG, "bad generate arguments");
    m->pos = 0;  // clear_cache_core
    GAJE_TRY(gaje_hip_prefill(m, prompt, n_prompt, nullptr));
    if (max_new == 0) return GAJE_OK;
    if (temperature <= 1e-5f && n_eos <= GEN_MAX_EOS)
        return generate_device(m, max_new, repetition_penalty, eos_ids, n_eos, out_tokens, n_out);
    // multinomial sampling (or more EOS ids than the device list holds): the
    // loop on the host, over the logits of each step
    const bool kwta = m->kwta_ratio > 0.0f && m->kwta_ratio < 1.0f;
    if (kwta) GAJE_TRY(launch_kwta(m->logits, m->vocab_out, kwta_k(m->vocab_out, m->kwta_ratio), m->st, m->stream));
    std::vector<float> logits((size_t)m->vocab_out);
    std::vector<uint32_t> gen;
    uint64_t rng = seed;
    auto is_eos = [&](uint32_t t) {
        for (int64_t i = 0; i < n_eos; ++i)
            if (eos_ids[i] == t) return true;
        return false;
    };
    for (int64_t step = 0; step < max_new; ++step) {
        GAJE_HIP_CHECK(hipMemcpyAsync(logits.data(), m->logits, logits.size() * 4, hipMemcpyDeviceToHost, m->stream));
        GAJE_HIP_CHECK(hipStreamSynchronize(m->stream));
        if (repetition_penalty > 1.0f) {
            std::vector<uint32_t> seen;
            for (uint32_t t : gen)
                if (!is_eos(t) && std::find(seen.begin(), seen.end(), t) == seen.end()) seen.push_back(t);
            for (uint32_t t : seen)
                if (t < logits.size()) {
                    if (logits[t] < 0.0f) logits[t] *= repetition_penalty;
                    else logits[t] /= repetition_penalty;
                }
        }
        uint32_t next = 0;
        if (temperature <= 1e-5f) {
            float best = -INFINITY;
            for (size_t i = 0; i < logits.size(); ++i)
                if (logits[i] > best) {
                    best = logits[i];
                    next = (uint32_t)i;
                }
        } else {
            float mx = -INFINITY;
            for (float v : logits)
                if (v > mx) mx = v;
            std::vector<float> probs(logits.size());
            float sum = 0.0f;
            for (size_t i = 0; i < logits.size(); ++i) {
                probs[i] = expf((logits[i] - mx) / temperature);
                sum += probs[i];
            }
            rng += 0x9E3779B97F4A7C15ull;
            const float u = (float)(mix64(rng) >> 40) * 0x1.0p-24f;
            const float r = u * sum;
            float cum = 0.0f;
            for (size_t i = 0; i < probs.size(); ++i) {
                cum += probs[i];
                if (r <= cum) {
                    next = (uint32_t)i;
                    break;
                }
            }
        }
        gen.push_back(next);
        out_tokens[gen.size() - 1] = next;
        if (n_out) *n_out = (int64_t)gen.size();
        if (is_eos(next)) break;
        bool repeated = false;
        for (size_t w = 2; w <= 48 && !repeated; ++w) {
            if (gen.size() >= w * 3) {
                const size_t n = gen.size();
                bool same = true;
                for (size_t i = 0; i < w && same; ++i)
                    same = gen[n - w + i] == gen[n - 2 * w + i] && gen[n - w + i] == gen[n - 3 * w + i];
                repeated = same;
            }
        }
        if (repeated) break;
        DevState s;
        GAJE_TRY(forward_device(m, next, false, true, s));
    }
    return GAJE_OK;
}

extern "C" int gaje_hip_truncate_cache(gaje_hip_model *m, int64_t len) {
    GAJE_TRY(check_model(m));
    if (len < 0 || len > m->pos)
        return set_error(GAJE_ERR_INVALID_ARG, "cannot truncate a cache of %lld positions to %lld", (long long)m->pos,
                         (long long)len);
    m->pos = len;
    return GAJE_OK;
}

extern "C" int gaje_hip_time_stage(gaje_hip_model *m, int stage, int64_t layer, int iters, float *avg_ms,
                                   int64_t *bytes) {
    clear_error();
    GAJE_TRY(check_model(m));
    if (!avg_ms || iters <= 0) return set_error(GAJE_ERR_INVALID_ARG, "bad timing arguments");
    if (stage >= GAJE_STAGE_QKV && stage <= GAJE_STAGE_DOWN && (layer < 0 || layer >= m->n_layers))
        return set_error(GAJE_ERR_INVALID_ARG, "layer %lld out of range", (long long)layer);
    GAJE_TRY(reserve_ctx(m, m->pos + 1));
    if (stage == GAJE_STAGE_TOKEN && !m->profile) GAJE_TRY(ensure_graph(m));
    GAJE_TRY(launch_state_set(m->st, (int32_t)m->pos, 0, -1, -1, 1, m->stream));
    const int64_t nb_q = m->n_embd / 32;
    const size_t layer_kv = (size_t)m->n_kv * m->cap * m->hd;
    auto wbytes = [](const DevLinear &D) -> int64_t {
        const int64_t nb = D.K / 32;
        int64_t b = D.fmt == FMT_Q4_0   ? D.N * nb * 20
                    : D.fmt == FMT_Q8_0 ? D.N * nb * 34
                    : D.fmt == FMT_LUT4 ? D.N * nb * 16
                    : D.fmt == FMT_G2   ? D.N * nb * 8
                                        : D.N * D.K * 4;
        if (D.fmt == FMT_LUT4 && D.lut) b += (D.lut_block_stride ? (D.lut_rows_own ? D.N : 1) * nb * 16 * 4 : 64);
        if (D.fmt == FMT_G2 && D.lut) b += (D.lut_block_stride ? (D.lut_rows_own ? D.N : 1) * nb * 4 * 4 : 16);
        return b;
    };
    int64_t algo = 0;
    auto one = [&]() -> int {
        switch (stage) {
            case GAJE_STAGE_QKV:
            case GAJE_STAGE_O:
            case GAJE_STAGE_GATE_UP:
            case GAJE_STAGE_DOWN: {
                Layer &Ly = m->layers[layer];
                GemvParams p;
                if (stage == GAJE_STAGE_QKV) {
                    p = gemv_base(m, Ly.qkv, m->h);
                    p.norm_w = Ly.attn_norm;
                    p.mode = MODE_QKV;
                    p.y = m->q;
                    p.q_out = m->q;
                    p.head_dim = (int32_t)m->hd;
                    p.rope_split = m->rope_split;
                    p.q_rows = m->q_rows;
                    p.kv_rows = m->kv_rows;
                    p.rope_cos = m->rope_cos;
                    p.rope_sin = m->rope_sin;
                    p.k_cache = m->k_cache + layer * layer_kv;
                    p.v_cache = m->v_cache + layer * layer_kv;
                    p.kv_head_stride = m->cap * m->hd;
                    p.kv_cap = m->cap;
                    algo = wbytes(Ly.qkv) + (m->n_embd * 2 + m->q_rows + 2 * m->kv_rows) * 4;
                } else if (stage == GAJE_STAGE_O) {
                    p = gemv_base(m, Ly.o, m->attn_out);
                    p.mode = MODE_RESIDUAL;
                    p.y = m->h;
                    algo = wbytes(Ly.o) + (m->q_rows + 2 * m->n_embd) * 4;
                } else if (stage == GAJE_STAGE_GATE_UP) {
                    p = gemv_base(m, Ly.gate_up, m->h);
                    p.norm_w = Ly.ffn_norm;
                    p.mode = MODE_SWIGLU;
                    p.ffn = m->ffn;
                    p.y = m->act;
                    p.y_cm = m->act_cm;
                    p.cm_stride = m->act_cm_stride;
                    algo = wbytes(Ly.gate_up) + (2 * m->n_embd + m->ffn) * 4;
                } else {
                    p = gemv_base(m, Ly.down, m->act);
                    p.x_cm = m->act_cm;
                    p.cm_stride = m->act_cm_stride;
                    p.mode = MODE_RESIDUAL;
                    p.y = m->h;
                    algo = wbytes(Ly.down) + (m->ffn + 2 * m->n_embd) * 4;
                }
                p.layer = (int32_t)layer;
                return launch_gemv(p, m->stream);
            }
            case GAJE_STAGE_ATTENTION: {
                AttnParams ap{};
                ap.q = m->q;
                ap.k_cache = m->k_cache + layer * layer_kv;
                ap.v_cache = m->v_cache + layer * layer_kv;
                ap.kv_head_stride = m->cap * m->hd;
                ap.n_head = (int32_t)m->n_head;
                ap.n_head_kv = (int32_t)m->n_kv;
                ap.head_dim = (int32_t)m->hd;
                ap.kv_cap = m->cap;
                ap.out = m->attn_out;
                ap.st = m->st;
                ap.layer = (int32_t)layer;
                algo = (int64_t)(m->pos + 1) * 2 * m->kv_rows * 4 + 2 * m->q_rows * 4;
                return launch_attention(ap, m->stream);
            }
            case GAJE_STAGE_LM_HEAD: {
                GemvParams p = gemv_base(m, m->lm_head, m->h);
                p.norm_w = m->output_norm;
                p.mode = MODE_ARGMAX;
                p.y = m->logits;
                p.x_out = m->hnorm;
                p.nontemporal = 1;
                p.layer = (int32_t)m->n_layers;
                algo = wbytes(m->lm_head) + (2 * m->n_embd + m->vocab_out) * 4;
                return launch_gemv(p, m->stream);
            }
            case GAJE_STAGE_TOKEN: {
                int64_t a = wbytes(m->lm_head) + m->n_embd * 4;
                for (auto &Ly : m->layers) a += wbytes(Ly.qkv) + wbytes(Ly.o) + wbytes(Ly.gate_up) + wbytes(Ly.down);
                a += m->n_layers * (int64_t)(m->pos + 1) * 2 * m->kv_rows * 4;
                algo = a;
                // profiling builds launch the token's kernels one by one: the
                // kernel tracer faults on graph replays
                if (m->profile) GAJE_TRY(enqueue_token(m, nullptr));
                else GAJE_HIP_CHECK(hipGraphLaunch(m->graph_exec, m->stream));
                // keep the position fixed so every replay is the same token
                return launch_state_set(m->st, (int32_t)m->pos, 0, -1, -1, 1, m->stream);
            }
            default:
                return set_error(GAJE_ERR_INVALID_ARG, "unknown stage %d", stage);
        }
    };
    (void)nb_q;
    GAJE_TRY(one());  // warm-up launch (also validates the arguments)
    hipEvent_t e0, e1;
    GAJE_HIP_CHECK(hipEventCreate(&e0));
    GAJE_HIP_CHECK(hipEventCreate(&e1));
    GAJE_HIP_CHECK(hipEventRecord(e0, m->stream));
    int rc = GAJE_OK;
    for (int i = 0; i < iters && rc == GAJE_OK; ++i) rc = one();
    GAJE_HIP_CHECK(hipEventRecord(e1, m->stream));
    GAJE_HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    GAJE_TRY(rc);
    *avg_ms = ms / (float)iters;
    if (bytes) *bytes = algo;
    GAJE_TRY(launch_state_set(m->st, (int32_t)m->pos, 0, -1, -1, 1, m->stream));
    GAJE_HIP_CHECK(hipStreamSynchronize(m->stream));
    return GAJE_OK;
}

extern "C" int gaje_hip_last_timing(const gaje_hip_model *m, float *blocks_ms, float *head_ms) {
    if (!m) return set_error(GAJE_ERR_INVALID_ARG, "null model");
    if (blocks_ms) *blocks_ms = m->last_blocks_ms;
    if (head_ms) *head_ms = m->last_head_ms;
    return GAJE_OK;
}
