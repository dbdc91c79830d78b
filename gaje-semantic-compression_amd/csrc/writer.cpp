// Native .gaje.flat writer from f32 weights: the container and tensor
// routines of scripts/export_gaje_flat.py with the quantisers the exporter
// calls through GenomicLayer (python/gaje/nn/stabilized.py:242-323):
//   - a 4096-byte header packed "<4sIIIQQQQIIIIIIII" (:433-465), the metadata
//     JSON, the directory JSON, zeros to the 4096-aligned weights_offset;
//   - add_blob_data (:207-212): each sub-blob appended, then zeros to a 64-byte
//     boundary; a tensor adds its dna, centroid and anchor blobs in that order
//     and its bias blob only when it has a bias (:214-260); norms add one blob
//     with centroid and anchor offsets 0 (:321-336);
//   - directory entries in the order the tensors were added, printed as
//     json.dumps prints a list of dicts.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include <cerrno>

#include "common.h"
#include "flat.h"
#include "quantize.h"

struct gaje_flat_writer {
    struct Entry {
        std::string name;
        uint64_t bit_depth, out_f, in_f, dna_off, dna_len, c_off, c_len, anc_off, anc_len, bias_off, bias_len;
    };
    std::vector<Entry> dir;
    std::vector<uint8_t> blob;

    uint64_t add_blob(const void *data, size_t len) {
        const uint64_t off = blob.size();
        if (len) blob.insert(blob.end(), (const uint8_t *)data, (const uint8_t *)data + len);
        blob.resize((blob.size() + 63) / 64 * 64, 0);
        return off;
    }
    // process_and_add_layer: dna, centroids, anchors, then the bias if any
    void add_layer(const char *name, uint64_t bit_depth, int64_t out_f, int64_t in_f, const void *dna, size_t dna_len,
                   const void *c, size_t c_len, const void *anc, size_t anc_len, const float *bias, int64_t bias_len) {
        Entry e{name, bit_depth, (uint64_t)out_f, (uint64_t)in_f, 0, dna_len, 0, c_len, 0, anc_len, 0, 0};
        e.dna_off = add_blob(dna, dna_len);
        e.c_off = add_blob(c, c_len);
        e.anc_off = add_blob(anc, anc_len);
        if (bias && bias_len > 0) {
            e.bias_off = add_blob(bias, (size_t)bias_len * 4);
            e.bias_len = (uint64_t)bias_len * 4;
        }
        dir.push_back(e);
    }
};

using namespace gaje;

namespace {

bool bad_name(const char *name) {
    if (!name || !*name) return true;
    for (const char *p = name; *p; ++p)
        if (*p == '"' || *p == '\\' || (unsigned char)*p < 0x20) return true;
    return false;
}

int check_layer(gaje_flat_writer *w, const char *name, const float *weights, int64_t out_f, int64_t in_f,
                const float *bias, int64_t bias_len) {
    if (!w || bad_name(name) || !weights || out_f <= 0 || in_f <= 0 || bias_len < 0 || (bias_len > 0 && !bias))
        return set_error(GAJE_ERR_INVALID_ARG, "flat writer: bad tensor arguments");
    return GAJE_OK;
}

}  // namespace

extern "C" int gaje_flat_writer_create(gaje_flat_writer **out) {
    clear_error();
    if (!out) return set_error(GAJE_ERR_INVALID_ARG, "flat writer: null handle");
    *out = new gaje_flat_writer();
    return GAJE_OK;
}

extern "C" void gaje_flat_writer_free(gaje_flat_writer *w) { delete w; }

extern "C" int gaje_flat_writer_add_norm(gaje_flat_writer *w, const char *name, const float *weights, int64_t n) {
    clear_error();
    GAJE_TRY(check_layer(w, name, weights, n, 1, nullptr, 0));
    gaje_flat_writer::Entry e{name, 32, (uint64_t)n, 1, 0, (uint64_t)n * 4, 0, 0, 0, 0, 0, 0};
    e.dna_off = w->add_blob(weights, (size_t)n * 4);
    w->dir.push_back(e);
    return GAJE_OK;
}

extern "C" int gaje_flat_writer_add_f32(gaje_flat_writer *w, const char *name, const float *weights, int64_t out_f,
                                        int64_t in_f, const float *bias, int64_t bias_len) {
    clear_error();
    GAJE_TRY(check_layer(w, name, weights, out_f, in_f, bias, bias_len));
    w->add_layer(name, 32, out_f, in_f, weights, (size_t)(out_f * in_f) * 4, nullptr, 0, nullptr, 0, bias, bias_len);
    return GAJE_OK;
}

extern "C" int gaje_flat_writer_add_q4_0(gaje_flat_writer *w, const char *name, const float *weights, int64_t out_f,
                                         int64_t in_f, const float *bias, int64_t bias_len) {
    clear_error();
    GAJE_TRY(check_layer(w, name, weights, out_f, in_f, bias, bias_len));
    if ((out_f * in_f) % 32) return set_error(GAJE_ERR_INVALID_ARG, "Weights length must be divisible by 32");
    std::vector<uint8_t> dna((size_t)(out_f * in_f / 32) * 20);
    quantize_q4_0(weights, out_f * in_f, dna.data());
    w->add_layer(name, 4, out_f, in_f, dna.data(), dna.size(), nullptr, 0, nullptr, 0, bias, bias_len);
    return GAJE_OK;
}

extern "C" int gaje_flat_writer_add_q8_0(gaje_flat_writer *w, const char *name, const float *weights, int64_t out_f,
                                         int64_t in_f, const float *bias, int64_t bias_len) {
    clear_error();
    GAJE_TRY(check_layer(w, name, weights, out_f, in_f, bias, bias_len));
    if ((out_f * in_f) % 32) return set_error(GAJE_ERR_INVALID_ARG, "Weights length must be divisible by 32");
    std::vector<uint8_t> dna((size_t)(out_f * in_f / 32) * 34);
    quantize_q8_0(weights, out_f * in_f, dna.data());
    w->add_layer(name, 8, out_f, in_f, dna.data(), dna.size(), nullptr, 0, nullptr, 0, bias, bias_len);
    return GAJE_OK;
}

extern "C" int gaje_flat_writer_add_lut4(gaje_flat_writer *w, const char *name, const float *weights, int64_t out_f,
                                         int64_t in_f, float anchor_threshold, const float *bias, int64_t bias_len) {
    clear_error();
    GAJE_TRY(check_layer(w, name, weights, out_f, in_f, bias, bias_len));
    std::vector<uint8_t> codes, anchors;
    std::vector<float> cent;
    if (!genomize_4bit(weights, out_f * in_f, 32, anchor_threshold, codes, cent, anchors))
        return set_error(GAJE_ERR_INVALID_ARG, "genomize: a density anchor threshold over data holding NaN");
    w->add_layer(name, 4, out_f, in_f, codes.data(), codes.size(), cent.data(), cent.size() * 4, anchors.data(),
                 anchors.size(), bias, bias_len);
    return GAJE_OK;
}

extern "C" int gaje_flat_writer_write(gaje_flat_writer *w, const char *path, const char *metadata_json,
                                      const gaje_flat_writer_header *h) {
    clear_error();
    if (!w || !path || !metadata_json || !h) return set_error(GAJE_ERR_INVALID_ARG, "flat writer: null argument");
    std::string dir = "[";
    for (size_t i = 0; i < w->dir.size(); ++i) {
        const auto &e = w->dir[i];
        char buf[512];
        snprintf(buf, sizeof buf,
                 "{\"name\": \"%s\", \"bit_depth\": %llu, \"out_features\": %llu, \"in_features\": %llu, "
                 "\"dna_off\": %llu, \"dna_len\": %llu, \"c_off\": %llu, \"c_len\": %llu, \"anc_off\": %llu, "
                 "\"anc_len\": %llu, \"bias_off\": %llu, \"bias_len\": %llu}",
                 e.name.c_str(), (unsigned long long)e.bit_depth, (unsigned long long)e.out_f,
                 (unsigned long long)e.in_f, (unsigned long long)e.dna_off, (unsigned long long)e.dna_len,
                 (unsigned long long)e.c_off, (unsigned long long)e.c_len, (unsigned long long)e.anc_off,
                 (unsigned long long)e.anc_len, (unsigned long long)e.bias_off, (unsigned long long)e.bias_len);
        if (i) dir += ", ";
        dir += buf;
    }
    dir += "]";
    const size_t meta_len = strlen(metadata_json);
    uint64_t weights_offset = 4096 + meta_len + dir.size();
    weights_offset = (weights_offset + 4095) / 4096 * 4096;

    FlatHeaderV2 hdr;
    memset(&hdr, 0, sizeof hdr);
    memcpy(hdr.magic, "GAJE", 4);
    hdr.version = 0x000908;
    hdr.flags = h->flags;
    hdr.num_tensors = (uint32_t)w->dir.size();
    hdr.meta_len = meta_len;
    hdr.dir_len = dir.size();
    hdr.weights_offset = weights_offset;
    hdr.weights_len = w->blob.size();
    hdr.group_size = h->group_size;
    hdr.quant_format = h->quant_format;
    hdr.arch_family = h->arch_family;
    hdr.arch_n_embd = h->n_embd;
    hdr.arch_n_head = h->n_head;
    hdr.arch_n_head_kv = h->n_head_kv;
    hdr.arch_n_blocks = h->n_blocks;
    hdr.arch_qk_permute = h->qk_permute;

    FILE *f = fopen(path, "wb");
    if (!f) return set_error(GAJE_ERR_IO, "%s: %s", path, strerror(errno));
    const std::vector<uint8_t> pad((size_t)(weights_offset - (4096 + meta_len + dir.size())), 0);
    bool ok = fwrite(&hdr, sizeof hdr, 1, f) == 1 && fwrite(metadata_json, 1, meta_len, f) == meta_len &&
              fwrite(dir.data(), 1, dir.size(), f) == dir.size() && fwrite(pad.data(), 1, pad.size(), f) == pad.size() &&
              fwrite(w->blob.data(), 1, w->blob.size(), f) == w->blob.size();
    if (fclose(f) != 0) ok = false;
    if (!ok) return set_error(GAJE_ERR_IO, "%s: write failed", path);
    return GAJE_OK;
}

extern "C" int gaje_quantize_q4_0(const float *weights, int64_t n, uint8_t *blocks_out) {
    clear_error();
    if (!weights || !blocks_out || n < 0 || n % 32) return set_error(GAJE_ERR_INVALID_ARG, "Weights length must be divisible by 32");
    quantize_q4_0(weights, n, blocks_out);
    return GAJE_OK;
}

extern "C" int gaje_quantize_q8_0(const float *weights, int64_t n, uint8_t *blocks_out) {
    clear_error();
    if (!weights || !blocks_out || n < 0 || n % 32) return set_error(GAJE_ERR_INVALID_ARG, "Weights length must be divisible by 32");
    quantize_q8_0(weights, n, blocks_out);
    return GAJE_OK;
}

extern "C" int gaje_genomize_4bit(const float *weights, int64_t n, int64_t block_size, float anchor_threshold,
                                  uint8_t *codes_out, float *centroids_out, uint8_t *anchors_out, int64_t *anchors_len) {
    clear_error();
    if (!weights || n < 0 || block_size <= 0 || block_size % 2 || !anchors_len)
        return set_error(GAJE_ERR_INVALID_ARG, "genomize: bad arguments");
    std::vector<uint8_t> codes, anchors;
    std::vector<float> cent;
    if (!genomize_4bit(weights, n, block_size, anchor_threshold, codes, cent, anchors))
        return set_error(GAJE_ERR_INVALID_ARG, "genomize: a density anchor threshold over data holding NaN");
    const int64_t cap = *anchors_len;
    *anchors_len = (int64_t)anchors.size();
    if (codes_out && !codes.empty()) memcpy(codes_out, codes.data(), codes.size());
    if (centroids_out && !cent.empty()) memcpy(centroids_out, cent.data(), cent.size() * 4);
    if (anchors_out) {
        if (cap < (int64_t)anchors.size()) return set_error(GAJE_ERR_INVALID_ARG, "genomize: anchor buffer too small");
        memcpy(anchors_out, anchors.data(), anchors.size());
    }
    return GAJE_OK;
}
