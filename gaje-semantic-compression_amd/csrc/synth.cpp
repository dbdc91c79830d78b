// Random-init .gaje.flat writer for the benchmark shapes.
//
// Container layout follows the reference exporter
// (scripts/export_gaje_flat.py:184-483): 4096-byte header packed as
// "<4sIIIQQQQIIIIIIII", metadata JSON, directory JSON, zero padding to the
// 4096-aligned weights_offset, then every sub-blob 64-byte aligned relative to
// weights_offset (add_blob_data, :207-212), tensors in exporter order.
//
// Values come from a counter-based PRNG so any element can be regenerated
// independently (and restated in numpy by the tests):
//   key(seed, name) = mix64(seed ^ fnv1a64(name))
//   r(key, i)       = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)   (splitmix64)
//   u01(r)          = (r >> 11) * 2^-53
//   normal(key, i)  = sqrt(-2 ln(1 - u01(r(key, 2i)))) * cos(2 pi u01(r(key, 2i+1)))
// Q4_0 / LUT body recipe (4-bit codes uniform, per-block scale s ~ U(0.01,0.05),
// table z_j * s with z_j = Phi^-1((j + 0.5) / 16)):
//   code(row, col)  = r(key(name#codes), row*k + col) >> 60
//   s(row, b)       = 0.01 + 0.04 * u01(r(key(name#scale), row*nb + b))
//   Q4_0 block      : scale = f16(f32(s * (z15 - z0) / 15)), min = f16(f32(s * z0)),
//                     qs[m] = code[2m] | code[2m+1] << 4      (low nibble = even)
//   LUT-4bit block  : byte m = code[2m] << 4 | code[2m+1]      (high nibble = even),
//                     lut[row][b][j] = f32(z_j * s)
// 2-bit body recipe (Genomic2Bit, bit_depth 2; 2-bit codes uniform, four
// centroids per (row, block) at the quartile midpoints y_j = Phi^-1((j + 0.5) / 4)):
//   code(row, col)  = r(key(name#codes), row*k + col) >> 62
//   block byte m    = code[4m] << 6 | code[4m+1] << 4 | code[4m+2] << 2 | code[4m+3]
//   centroids[row][b][j] = f32(y_j * s(row, b))   (ascending: codes 00, 01, 11, 10)
// Sparse f16 anchors (the "GAJE" buffer of GenomicLinear::new, init.rs:61-107),
// optional for body tensors: row r > 0 holds r(key(name#anchors), r) >> 62
// anchors (0..3), row 0 1 + (r(key, 0) >> 63), anchor j at column r(key(name#anchors), n + 4r + j) % k, value
// f16(0.05 * normal(key(name#anchors), 4r + j)), in row then column order.
// The buffer is "GAJE", count, the u32 flat indices, the f16 values, then:
//   form 1  n+1 u64 row pointers (the CSR path of init.rs:82-90); indices
//           r*k + col + k*n*(j & 1), so odd anchors sit past the tensor and
//           only index % in_features (forward.rs:106) places them; row 1's
//           range is inverted (pointer[2] = pointer[1] - 1, skipped, :104),
//           and row 2 then starts one anchor early
//   form 2  the two pointers {0, count} of genomize_4bit_core
//           (genomize.rs:373-376): too short for n > 1, so the rows come from
//           the flat indices (:91-103)
//   form 3  no pointers (the same fallback)
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "common.h"
#include "flat.h"
#include "quantize.h"

namespace gaje {
namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t fnv1a64(const std::string &s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

inline uint64_t stream_key(uint64_t seed, const std::string &name) { return mix64(seed ^ fnv1a64(name)); }
inline uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull); }
inline double u01(uint64_t r) { return (double)(r >> 11) * 0x1.0p-53; }

inline double normal_at(uint64_t key, uint64_t i) {
    double u1 = 1.0 - u01(draw(key, 2 * i));
    double u2 = u01(draw(key, 2 * i + 1));
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2);
}

// Phi^-1 by bisection on Phi(z) = erfc(-z / sqrt 2) / 2, to double precision.
double probit(double p) {
    double lo = -40.0, hi = 40.0;
    for (int i = 0; i < 200; ++i) {
        double mid = 0.5 * (lo + hi);
        if (mid == lo || mid == hi) break;
        if (0.5 * std::erfc(-mid / std::sqrt(2.0)) < p) lo = mid;
        else hi = mid;
    }
    return 0.5 * (lo + hi);
}

const double *quantile_table() {
    static double z[16];
    static bool init = false;
    if (!init) {
        for (int j = 0; j < 16; ++j) z[j] = probit((j + 0.5) / 16.0);
        init = true;
    }
    return z;
}

template <class F>
void parallel_rows(int64_t n, F f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 4;
    if (nt > 16) nt = 16;
    if (n < 64) nt = 1;
    std::vector<std::thread> th;
    int64_t per = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        int64_t a = t * per, b = std::min<int64_t>(n, a + per);
        if (a >= b) break;
        th.emplace_back([=] { f(a, b); });
    }
    for (auto &x : th) x.join();
}

void gen_q4_0(uint64_t seed, const std::string &name, int64_t n, int64_t k, uint8_t *out) {
    const int64_t nb = k / 32;
    const double *z = quantile_table();
    const uint64_t kc = stream_key(seed, name + "#codes"), ks = stream_key(seed, name + "#scale");
    const double span = (z[15] - z[0]) / 15.0;
    parallel_rows(n, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r)
            for (int64_t b = 0; b < nb; ++b) {
                uint8_t *blk = out + (r * nb + b) * 20;
                double s = 0.01 + 0.04 * u01(draw(ks, (uint64_t)(r * nb + b)));
                uint16_t hs = f32_to_f16((float)(s * span)), hm = f32_to_f16((float)(s * z[0]));
                memcpy(blk, &hs, 2);
                memcpy(blk + 2, &hm, 2);
                for (int m = 0; m < 16; ++m) {
                    uint64_t i = (uint64_t)(r * k + b * 32 + 2 * m);
                    uint8_t c0 = (uint8_t)(draw(kc, i) >> 60), c1 = (uint8_t)(draw(kc, i + 1) >> 60);
                    blk[4 + m] = (uint8_t)(c0 | (c1 << 4));
                }
            }
    });
}

void gen_2bit(uint64_t seed, const std::string &name, int64_t n, int64_t k, uint8_t *codes, float *cent) {
    const int64_t nb = k / 32;
    double y[4];
    for (int j = 0; j < 4; ++j) y[j] = probit((j + 0.5) / 4.0);
    const uint64_t kc = stream_key(seed, name + "#codes"), ks = stream_key(seed, name + "#scale");
    parallel_rows(n, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r)
            for (int64_t b = 0; b < nb; ++b) {
                double s = 0.01 + 0.04 * u01(draw(ks, (uint64_t)(r * nb + b)));
                float *t = cent + (r * nb + b) * 4;
                for (int j = 0; j < 4; ++j) t[j] = (float)(y[j] * s);
                uint8_t *blk = codes + (r * nb + b) * 8;
                for (int m = 0; m < 8; ++m) {
                    uint64_t i = (uint64_t)(r * k + b * 32 + 4 * m);
                    uint8_t byte = 0;
                    for (int q = 0; q < 4; ++q) byte = (uint8_t)((byte << 2) | (draw(kc, i + q) >> 62));
                    blk[m] = byte;
                }
            }
    });
}

void gen_lut4(uint64_t seed, const std::string &name, int64_t n, int64_t k, uint8_t *codes, float *lut) {
    const int64_t nb = k / 32;
    const double *z = quantile_table();
    const uint64_t kc = stream_key(seed, name + "#codes"), ks = stream_key(seed, name + "#scale");
    parallel_rows(n, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r)
            for (int64_t b = 0; b < nb; ++b) {
                double s = 0.01 + 0.04 * u01(draw(ks, (uint64_t)(r * nb + b)));
                float *t = lut + (r * nb + b) * 16;
                for (int j = 0; j < 16; ++j) t[j] = (float)(z[j] * s);
                uint8_t *blk = codes + (r * nb + b) * 16;
                for (int m = 0; m < 16; ++m) {
                    uint64_t i = (uint64_t)(r * k + b * 32 + 2 * m);
                    uint8_t c0 = (uint8_t)(draw(kc, i) >> 60), c1 = (uint8_t)(draw(kc, i + 1) >> 60);
                    blk[m] = (uint8_t)((c0 << 4) | c1);
                }
            }
    });
}

void gen_normal(uint64_t seed, const std::string &name, int64_t count, double mean, double sd, float *out) {
    const uint64_t key = stream_key(seed, name);
    parallel_rows(count, [&](int64_t a, int64_t b) {
        for (int64_t i = a; i < b; ++i) out[i] = (float)(mean + sd * normal_at(key, (uint64_t)i));
    });
}

// The anchor buffer of an n x k body tensor in the given form (1..3).
std::vector<uint8_t> gen_anchors(uint64_t seed, const std::string &name, int64_t n, int64_t k, int form) {
    const uint64_t key = stream_key(seed, name + "#anchors");
    std::vector<uint32_t> idx;
    std::vector<uint16_t> val;
    std::vector<uint64_t> ptr(1, 0);
    for (int64_t r = 0; r < n; ++r) {
        const int cnt = r == 0 ? 1 + (int)(draw(key, 0) >> 63) : (int)(draw(key, (uint64_t)r) >> 62);
        std::vector<int64_t> cols;
        for (int j = 0; j < cnt; ++j) cols.push_back((int64_t)(draw(key, (uint64_t)(n + 4 * r + j)) % (uint64_t)k));
        std::sort(cols.begin(), cols.end());
        for (int j = 0; j < cnt; ++j) {
            int64_t flat = r * k + cols[j];
            if (form == 1 && (j & 1)) flat += k * n;
            idx.push_back((uint32_t)flat);
            val.push_back(f32_to_f16((float)(0.05 * normal_at(key, (uint64_t)(4 * r + j)))));
        }
        ptr.push_back(idx.size());
    }
    if (form == 1 && n > 2 && ptr[1] >= 1) ptr[2] = ptr[1] - 1;
    if (form == 2) ptr = {0, (uint64_t)idx.size()};
    if (form == 3) ptr.clear();
    const uint32_t count = (uint32_t)idx.size();
    std::vector<uint8_t> buf(8 + (size_t)count * 6 + ptr.size() * 8);
    memcpy(buf.data(), "GAJE", 4);
    memcpy(buf.data() + 4, &count, 4);
    memcpy(buf.data() + 8, idx.data(), (size_t)count * 4);
    memcpy(buf.data() + 8 + (size_t)count * 4, val.data(), (size_t)count * 2);
    memcpy(buf.data() + 8 + (size_t)count * 6, ptr.data(), ptr.size() * 8);
    return buf;
}

// One directory entry plus the generator of its bytes.
struct Blob {
    std::string name;
    uint64_t bit_depth, out_f, in_f;
    uint64_t dna_len, c_len, bias_len;  // bytes
    uint64_t dna_off = 0, c_off = 0, anc_off = 0, bias_off = 0;
    std::vector<uint8_t> anchors;       // the GAJE anchor buffer, empty for none
    // generators: 0 normal f32, 1 q4_0, 2 lut4, 3 norm weights, 4 normal f32 quantised to Q8_0,
    // 5 2-bit codes and centroids
    int kind;
    std::string stream;  // PRNG stream name of the dna values
    bool has_bias = false;
    std::string bias_stream;
};

uint64_t align64(uint64_t x) { return (x + 63) & ~uint64_t(63); }

std::string fmt_float(float f) {
    char buf[64];
    snprintf(buf, sizeof buf, "%.9g", (double)f);
    std::string s(buf);
    if (s.find_first_of(".eEn") == std::string::npos) s += ".0";
    return s;
}

}  // namespace
}  // namespace gaje

using namespace gaje;

extern "C" int gaje_synth_q4_0(uint64_t seed, const char *name, int64_t n, int64_t k, uint8_t *out) {
    if (!name || !out || n < 0 || k < 0) return set_error(GAJE_ERR_INVALID_ARG, "gaje_synth_q4_0: bad arguments");
    gen_q4_0(seed, name, n, k, out);
    return GAJE_OK;
}

extern "C" int gaje_synth_lut4(uint64_t seed, const char *name, int64_t n, int64_t k, uint8_t *codes, float *lut) {
    if (!name || !codes || !lut || n < 0 || k < 0)
        return set_error(GAJE_ERR_INVALID_ARG, "gaje_synth_lut4: bad arguments");
    gen_lut4(seed, name, n, k, codes, lut);
    return GAJE_OK;
}

extern "C" int gaje_synth_2bit(uint64_t seed, const char *name, int64_t n, int64_t k, uint8_t *codes, float *centroids) {
    if (!name || !codes || !centroids || n < 0 || k < 0)
        return set_error(GAJE_ERR_INVALID_ARG, "gaje_synth_2bit: bad arguments");
    gen_2bit(seed, name, n, k, codes, centroids);
    return GAJE_OK;
}

extern "C" int gaje_synth_normal(uint64_t seed, const char *name, int64_t count, float mean, float sd, float *out) {
    if (!name || !out || count < 0) return set_error(GAJE_ERR_INVALID_ARG, "gaje_synth_normal: bad arguments");
    gen_normal(seed, name, count, mean, sd, out);
    return GAJE_OK;
}

extern "C" int gaje_synth_write_flat(const char *path, const gaje_synth_config *cfg) {
    if (!path || !cfg) return set_error(GAJE_ERR_INVALID_ARG, "gaje_synth_write_flat: null argument");
    const gaje_synth_config &c = *cfg;
    if (c.n_embd <= 0 || c.n_head <= 0 || c.n_head_kv <= 0 || c.n_blocks < 0 || c.ffn <= 0 ||
        c.vocab_size <= 0 || c.n_embd % c.n_head != 0 ||
        (c.body_format != 1 && c.body_format != 2 && c.body_format != 4))
        return set_error(GAJE_ERR_INVALID_ARG, "gaje_synth_write_flat: invalid shape");
    const int64_t h = c.n_embd, hd = h / c.n_head, qd = c.n_head * hd, kvd = c.n_head_kv * hd;
    const int fmt = c.body_format;

    std::vector<Blob> blobs;
    auto dense = [&](const std::string &name, int64_t out_f, int64_t in_f, const std::string &stream) {
        Blob b{name, 32, (uint64_t)out_f, (uint64_t)in_f, (uint64_t)(out_f * in_f * 4), 0, 0};
        b.kind = 0;
        b.stream = stream;
        return b;
    };
    auto norm = [&](const std::string &name) {
        Blob b{name, 32, (uint64_t)h, 1, (uint64_t)(h * 4), 0, 0};
        b.kind = 3;
        b.stream = name;
        return b;
    };
    // bytes of a 2-bit tensor's centroid table: the leading part of the per
    // (row, block) tables that the chosen form keeps
    auto g2_table_bytes = [&](int64_t out_f, int64_t nb) -> uint64_t {
        switch (c.g2_tables) {
            case 1: return (uint64_t)(nb * 4 * 4);
            case 2: return 16;
            case 3: return (uint64_t)(((out_f / 2) * nb * 4 + 6) * 4);
            default: return (uint64_t)(out_f * nb * 4 * 4);
        }
    };
    auto body = [&](const std::string &name, int64_t out_f, int64_t in_f) {
        int64_t nb = in_f / 32;
        Blob b{name, 4, (uint64_t)out_f, (uint64_t)in_f, 0, 0, 0};
        b.kind = fmt;
        b.stream = name;
        if (fmt == 1) {
            b.dna_len = (uint64_t)(out_f * nb * 20);
        } else if (fmt == 4) {  // Genomic2Bit: bit_depth 2, 8 code bytes and 4 centroids per block
            b.bit_depth = 2;
            b.kind = 5;
            b.dna_len = (uint64_t)(out_f * nb * 8);
            b.c_len = g2_table_bytes(out_f, nb);
        } else {
            b.dna_len = (uint64_t)(out_f * nb * 16);
            b.c_len = (uint64_t)(out_f * nb * 16 * 4);
        }
        if (c.anchors) b.anchors = gen_anchors(c.seed, name, out_f, in_f, c.anchors);
        return b;
    };

    // --quant-embed (export_gaje_flat.py:25-32): token_embd and lm_head as Q8_0 (bit_depth 8)
    auto embed = [&](const std::string &name, const std::string &stream) {
        Blob b = dense(name, c.vocab_size, h, stream);
        if (c.quant_embed == 1) {
            b.bit_depth = 8;
            b.kind = 4;
            b.dna_len = (uint64_t)(c.vocab_size * (h / 32) * 34);
        } else if (c.quant_embed == 2) {
            b.bit_depth = 2;
            b.kind = 5;
            b.dna_len = (uint64_t)(c.vocab_size * (h / 32) * 8);
            b.c_len = g2_table_bytes(c.vocab_size, h / 32);
        }
        return b;
    };
    if (c.quant_embed < 0 || c.quant_embed > 2 || c.g2_tables < 0 || c.g2_tables > 3 || c.anchors < 0 ||
        c.anchors > 3)
        return set_error(GAJE_ERR_INVALID_ARG, "gaje_synth_write_flat: quant_embed 0-2, g2_tables 0-3, anchors 0-3");
    if (c.quant_embed && h % 32)
        return set_error(GAJE_ERR_INVALID_ARG, "gaje_synth_write_flat: quantised embeddings need n_embd %% 32 == 0");
    blobs.push_back(embed("token_embd", "token_embd"));
    blobs.push_back(norm("output_norm"));
    blobs.push_back(embed("lm_head", c.tied_embeddings ? "token_embd" : "lm_head"));
    for (int64_t i = 0; i < c.n_blocks; ++i) {
        std::string p = "blk." + std::to_string(i) + ".";
        blobs.push_back(norm(p + "attn_norm"));
        blobs.push_back(norm(p + "ffn_norm"));
        if (c.fused) {
            Blob q = body(p + "attn_qkv", qd + 2 * kvd, h);
            if (c.qkv_bias) {
                q.has_bias = true;
                q.bias_len = (uint64_t)((qd + 2 * kvd) * 4);
                q.bias_stream = p + "attn_qkv.bias";
            }
            blobs.push_back(q);
        } else {
            const char *nm[3] = {"attn_q", "attn_k", "attn_v"};
            int64_t rows[3] = {qd, kvd, kvd};
            for (int t = 0; t < 3; ++t) {
                Blob q = body(p + nm[t], rows[t], h);
                if (c.qkv_bias) {
                    q.has_bias = true;
                    q.bias_len = (uint64_t)(rows[t] * 4);
                    q.bias_stream = p + nm[t] + ".bias";
                }
                blobs.push_back(q);
            }
        }
        blobs.push_back(body(p + "attn_output", h, qd));
        if (c.fused) {
            blobs.push_back(body(p + "ffn_gate_up", 2 * c.ffn, h));
        } else {
            blobs.push_back(body(p + "ffn_gate", c.ffn, h));
            blobs.push_back(body(p + "ffn_up", c.ffn, h));
        }
        blobs.push_back(body(p + "ffn_down", h, c.ffn));
    }

    // Offsets exactly as add_blob_data assigns them: dna, centroids, anchors,
    // then (if present) bias, each padded to 64 bytes.
    uint64_t cur = 0;
    for (Blob &b : blobs) {
        b.dna_off = cur;
        cur = align64(cur + b.dna_len);
        if (b.kind == 3) {  // norms are appended directly (no centroid/anchor slots)
            b.c_off = b.anc_off = 0;
            continue;
        }
        b.c_off = cur;
        cur = align64(cur + b.c_len);
        b.anc_off = cur;
        cur = align64(cur + b.anchors.size());
        if (b.has_bias) {
            b.bias_off = cur;
            cur = align64(cur + b.bias_len);
        }
    }
    const uint64_t weights_len = cur;

    std::string meta = "{\"config\": {\"name\": \"gaje-synthetic\", \"version\": \"0.9.8\", \"tokenizer_id\": \"none\", "
                       "\"rope_base\": " + fmt_float(c.rope_base) + ", \"ffn_act\": \"swiglu\", \"use_genomic_norm\": " +
                       (c.use_genomic_norm ? "true" : "false") + ", \"rope_style\": \"" +
                       (c.rope_interleaved ? "interleaved" : "split") + "\"}, "
                       "\"n_embd\": " + std::to_string(h) + ", \"n_head\": " + std::to_string(c.n_head) +
                       ", \"n_head_kv\": " + std::to_string(c.n_head_kv) + ", \"n_blocks\": " +
                       std::to_string(c.n_blocks) + ", \"vocab_size\": " + std::to_string(c.vocab_size) +
                       ", \"eps\": " + fmt_float(c.eps) + ", \"tokenizer\": \"\"}";
    std::string dir = "[";
    for (size_t i = 0; i < blobs.size(); ++i) {
        const Blob &b = blobs[i];
        char buf[1024];
        snprintf(buf, sizeof buf,
                 "%s{\"name\": \"%s\", \"bit_depth\": %llu, \"out_features\": %llu, \"in_features\": %llu, "
                 "\"dna_off\": %llu, \"dna_len\": %llu, \"c_off\": %llu, \"c_len\": %llu, \"anc_off\": %llu, "
                 "\"anc_len\": %llu, \"bias_off\": %llu, \"bias_len\": %llu}",
                 i ? ", " : "", b.name.c_str(), (unsigned long long)b.bit_depth, (unsigned long long)b.out_f,
                 (unsigned long long)b.in_f, (unsigned long long)b.dna_off, (unsigned long long)b.dna_len,
                 (unsigned long long)b.c_off, (unsigned long long)b.c_len, (unsigned long long)b.anc_off,
                 (unsigned long long)b.anchors.size(),
                 (unsigned long long)(b.has_bias ? b.bias_off : 0), (unsigned long long)(b.has_bias ? b.bias_len : 0));
        dir += buf;
    }
    dir += "]";

    uint64_t weights_offset = 4096 + meta.size() + dir.size();
    weights_offset = (weights_offset + 4095) / 4096 * 4096;

    FlatHeaderV2 hdr;
    memset(&hdr, 0, sizeof hdr);
    memcpy(hdr.magic, "GAJE", 4);
    hdr.version = 0x000908;
    hdr.flags = c.fused ? 0x3 : 0x0;
    hdr.num_tensors = (uint32_t)blobs.size();
    hdr.meta_len = meta.size();
    hdr.dir_len = dir.size();
    hdr.weights_offset = weights_offset;
    hdr.weights_len = weights_len;
    hdr.group_size = 32;
    hdr.quant_format = fmt == 1 ? 1 : 0;
    hdr.arch_family = (uint32_t)c.arch_family;
    hdr.arch_n_embd = (uint32_t)h;
    hdr.arch_n_head = (uint32_t)c.n_head;
    hdr.arch_n_head_kv = (uint32_t)c.n_head_kv;
    hdr.arch_n_blocks = (uint32_t)c.n_blocks;
    hdr.arch_qk_permute = 0;

    FILE *f = fopen(path, "wb");
    if (!f) return set_error(GAJE_ERR_IO, "%s: %s", path, strerror(errno));
    std::vector<uint8_t> pad(4096, 0);
    bool ok = fwrite(&hdr, sizeof hdr, 1, f) == 1 && fwrite(meta.data(), 1, meta.size(), f) == meta.size() &&
              fwrite(dir.data(), 1, dir.size(), f) == dir.size();
    uint64_t pos = 4096 + meta.size() + dir.size();
    if (ok && weights_offset > pos) ok = fwrite(pad.data(), 1, weights_offset - pos, f) == weights_offset - pos;
    uint64_t written = 0;  // bytes of blob written so far
    auto put = [&](const void *data, uint64_t off, uint64_t len) {
        if (!ok) return;
        while (written < off) {
            uint64_t n = std::min<uint64_t>(off - written, pad.size());
            ok = ok && fwrite(pad.data(), 1, n, f) == n;
            written += n;
        }
        if (len) ok = ok && fwrite(data, 1, len, f) == len;
        written += len;
    };
    for (const Blob &b : blobs) {
        std::vector<uint8_t> dna(b.dna_len);
        std::vector<float> lut;
        switch (b.kind) {
            case 0:
                gen_normal(c.seed, b.stream, (int64_t)(b.dna_len / 4), 0.0, 0.02, (float *)dna.data());
                break;
            case 3:
                gen_normal(c.seed, b.stream, (int64_t)(b.dna_len / 4), 1.0, 0.1, (float *)dna.data());
                break;
            case 1:
                gen_q4_0(c.seed, b.stream, (int64_t)b.out_f, (int64_t)b.in_f, dna.data());
                break;
            case 2:
                lut.resize(b.c_len / 4);
                gen_lut4(c.seed, b.stream, (int64_t)b.out_f, (int64_t)b.in_f, dna.data(), lut.data());
                break;
            case 5:  // the full per (row, block) tables; the blob keeps the first c_len bytes
                lut.resize((size_t)(b.out_f * (b.in_f / 32) * 4));
                gen_2bit(c.seed, b.stream, (int64_t)b.out_f, (int64_t)b.in_f, dna.data(), lut.data());
                break;
            case 4: {
                std::vector<float> w((size_t)(b.out_f * b.in_f));
                gen_normal(c.seed, b.stream, (int64_t)w.size(), 0.0, 0.02, w.data());
                quantize_q8_0(w.data(), (int64_t)w.size(), dna.data());
                break;
            }
        }
        put(dna.data(), b.dna_off, b.dna_len);
        if (b.c_len) put(lut.data(), b.c_off, b.c_len);
        if (!b.anchors.empty()) put(b.anchors.data(), b.anc_off, b.anchors.size());
        if (b.has_bias) {
            std::vector<float> bias(b.bias_len / 4);
            gen_normal(c.seed, b.bias_stream, (int64_t)bias.size(), 0.0, 0.02, bias.data());
            put(bias.data(), b.bias_off, b.bias_len);
        }
    }
    put(nullptr, weights_len, 0);
    if (fclose(f) != 0) ok = false;
    if (!ok) return set_error(GAJE_ERR_IO, "%s: write failed", path);
    return GAJE_OK;
}
