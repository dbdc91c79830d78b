// .gaje.flat v2 reader (see flat.h for the reference citations).
#include "flat.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>

#include "common.h"
#include "json.h"

namespace gaje {

QuantFormat quantization_type(const FlatHeaderV2 &h) {
    switch (h.quant_format) {
        case 0: return QuantFormat::LegacyCentroids;
        case 1: return QuantFormat::Q4_0;
        case 2: return QuantFormat::Q8_0;
        default: return QuantFormat::Unknown;
    }
}

uint32_t effective_group_size(const FlatHeaderV2 &h) { return h.group_size == 0 ? 16 : h.group_size; }

bool architecture_descriptor(const FlatHeaderV2 &h, ArchDescriptor &d) {
    if (h.arch_family == 0) return false;
    d = ArchDescriptor();
    d.family = (int)h.arch_family;
    d.n_embd = h.arch_n_embd;
    d.n_head = h.arch_n_head;
    d.n_head_kv = h.arch_n_head_kv;
    d.n_blocks = h.arch_n_blocks;
    d.head_dim = h.arch_n_head > 0 ? h.arch_n_embd / h.arch_n_head : 0;
    d.qk_permute = h.arch_qk_permute != 0;
    d.rope_style = "split";
    switch (h.arch_family) {
        case 1: d.rope_base = 10000.0f; d.ffn_act = "swiglu"; break;    // Llama
        case 2: d.rope_base = 100000.0f; d.ffn_act = "swiglu"; break;   // SmolLM
        case 3:                                                        // Qwen2
        case 4: d.rope_base = 1000000.0f; d.ffn_act = "swiglu"; break;  // Qwen2.5
        case 5: d.rope_base = 10000.0f; d.ffn_act = "geglu"; break;     // Gemma
        default: d.rope_base = 10000.0f; d.ffn_act = "silu"; break;     // Unknown
    }
    return true;
}

namespace {

int bad(const char *what, const char *key) {
    return set_error(GAJE_ERR_INVALID_DATA, "%s `%s`", what, key);
}

// serde: a usize field must be a non-negative integer literal.
int get_usize(const JsonValue &o, const char *key, bool required, uint64_t &out, bool *present) {
    if (o.count(key) > 1) return bad("duplicate field", key);
    const JsonValue *v = o.get(key);
    if (present) *present = false;
    if (!v) return required ? bad("missing field", key) : GAJE_OK;
    if (v->type != JsonValue::Number || !v->is_integer || v->negative)
        return bad("invalid type (expected usize) for", key);
    out = v->uinteger;
    if (present) *present = true;
    return GAJE_OK;
}

int get_f32(const JsonValue &o, const char *key, bool required, float &out) {
    if (o.count(key) > 1) return bad("duplicate field", key);
    const JsonValue *v = o.get(key);
    if (!v) return required ? bad("missing field", key) : GAJE_OK;
    if (v->type != JsonValue::Number) return bad("invalid type (expected f32) for", key);
    out = (float)v->number;
    return GAJE_OK;
}

int get_bool(const JsonValue &o, const char *key, bool &out) {
    if (o.count(key) > 1) return bad("duplicate field", key);
    const JsonValue *v = o.get(key);
    if (!v) return GAJE_OK;
    if (v->type != JsonValue::Bool) return bad("invalid type (expected bool) for", key);
    out = v->boolean;
    return GAJE_OK;
}

int get_string(const JsonValue &o, const char *key, bool required, std::string &out) {
    if (o.count(key) > 1) return bad("duplicate field", key);
    const JsonValue *v = o.get(key);
    if (!v) return required ? bad("missing field", key) : GAJE_OK;
    if (v->type != JsonValue::String) return bad("invalid type (expected string) for", key);
    out = v->str;
    return GAJE_OK;
}

}  // namespace

int parse_model_config(const char *json, size_t len, ModelConfig &c) {
    JsonValue root;
    std::string err;
    if (!json_parse(json, len, root, err))
        return set_error(GAJE_ERR_INVALID_DATA, "metadata JSON: %s", err.c_str());
    if (root.type != JsonValue::Object)
        return set_error(GAJE_ERR_INVALID_DATA, "metadata JSON: expected struct ModelConfig");
    c = ModelConfig();
    if (root.count("config") > 1) return bad("duplicate field", "config");
    const JsonValue *cfg = root.get("config");
    if (!cfg) return bad("missing field", "config");
    if (cfg->type != JsonValue::Object) return bad("invalid type (expected struct ArchConfig) for", "config");
    std::string ignored;
    float fignored = 0.0f;
    bool bignored = false;
    GAJE_TRY(get_string(*cfg, "name", false, c.name));
    GAJE_TRY(get_string(*cfg, "version", false, ignored));
    GAJE_TRY(get_string(*cfg, "tokenizer_id", false, ignored));
    GAJE_TRY(get_f32(*cfg, "rope_base", false, c.rope_base));
    GAJE_TRY(get_string(*cfg, "ffn_act", false, c.ffn_act));
    GAJE_TRY(get_bool(*cfg, "use_genomic_norm", c.use_genomic_norm));
    GAJE_TRY(get_string(*cfg, "rope_style", false, c.rope_style));
    GAJE_TRY(get_f32(*cfg, "anchor_threshold", false, fignored));
    GAJE_TRY(get_f32(*cfg, "ffn_anchor_threshold", false, fignored));
    GAJE_TRY(get_f32(*cfg, "rna_threshold", false, c.rna_threshold));
    GAJE_TRY(get_bool(*cfg, "unpermute_weights", c.unpermute_weights));
    GAJE_TRY(get_bool(*cfg, "apply_smollm_rope_patch", bignored));
    GAJE_TRY(get_bool(*cfg, "tie_word_embeddings", bignored));
    GAJE_TRY(get_string(*cfg, "dni", false, ignored));
    GAJE_TRY(get_string(*cfg, "state", false, ignored));
    GAJE_TRY(get_usize(root, "n_embd", true, c.n_embd, nullptr));
    GAJE_TRY(get_usize(root, "n_head", true, c.n_head, nullptr));
    GAJE_TRY(get_usize(root, "n_head_kv", true, c.n_head_kv, nullptr));
    GAJE_TRY(get_usize(root, "n_blocks", true, c.n_blocks, nullptr));
    if (root.count("vocab_size") > 1) return bad("duplicate field", "vocab_size");
    const JsonValue *vs = root.get("vocab_size");
    if (vs && vs->type != JsonValue::Null)
        GAJE_TRY(get_usize(root, "vocab_size", false, c.vocab_size, &c.has_vocab_size));
    GAJE_TRY(get_f32(root, "eps", true, c.eps));
    return GAJE_OK;
}

FlatFile::~FlatFile() {
    if (base_) munmap((void *)base_, size_);
}

int FlatFile::open(const char *path) {
    int fd = ::open(path, O_RDONLY);
    if (fd < 0) return set_error(GAJE_ERR_IO, "%s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        int e = errno;
        ::close(fd);
        return set_error(GAJE_ERR_IO, "%s: %s", path, strerror(e));
    }
    size_ = (size_t)st.st_size;
    if (size_ > 0) {
        void *p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            int e = errno;
            ::close(fd);
            size_ = 0;
            return set_error(GAJE_ERR_IO, "mmap %s: %s", path, strerror(e));
        }
        base_ = (const uint8_t *)p;
    }
    ::close(fd);
    // load_genomic_auto sends a file without the magic to the redb loader,
    // which this build does not carry (flat_reader.rs:240-251).
    if (size_ < 4 || memcmp(base_, "GAJE", 4) != 0)
        return set_error(GAJE_ERR_INVALID_MAGIC, "Invalid magic bytes (expected 'GAJE')");
    if (size_ < sizeof(FlatHeaderV2))
        return set_error(GAJE_ERR_TOO_SHORT, "Header buffer is less than 4096 bytes");
    memcpy(&header_, base_, sizeof(header_));

    const uint64_t meta_start = 4096, meta_len = header_.meta_len, dir_len = header_.dir_len;
    if (meta_len > size_ - meta_start || dir_len > size_ - meta_start - meta_len)
        return set_error(GAJE_ERR_INVALID_DATA, "metadata/directory range exceeds the file");
    const uint8_t *meta = base_ + meta_start;
    if (!utf8_valid(meta, meta_len))
        return set_error(GAJE_ERR_INVALID_DATA, "metadata is not valid UTF-8");
    metadata_.assign((const char *)meta, meta_len);

    const uint8_t *dir = meta + meta_len;
    JsonValue root;
    std::string err;
    if (!utf8_valid(dir, dir_len)) return set_error(GAJE_ERR_INVALID_DATA, "directory is not valid UTF-8");
    if (!json_parse((const char *)dir, dir_len, root, err))
        return set_error(GAJE_ERR_INVALID_DATA, "tensor directory JSON: %s", err.c_str());
    if (root.type != JsonValue::Array)
        return set_error(GAJE_ERR_INVALID_DATA, "tensor directory JSON: expected a sequence");
    tensors_.clear();
    for (const JsonValue &e : root.items) {
        if (e.type != JsonValue::Object)
            return set_error(GAJE_ERR_INVALID_DATA, "tensor directory JSON: expected struct FlatTensorEntry");
        TensorEntry t;
        GAJE_TRY(get_string(e, "name", true, t.name));
        GAJE_TRY(get_usize(e, "bit_depth", true, t.bit_depth, nullptr));
        GAJE_TRY(get_usize(e, "out_features", true, t.out_features, nullptr));
        GAJE_TRY(get_usize(e, "in_features", true, t.in_features, nullptr));
        GAJE_TRY(get_usize(e, "dna_off", true, t.dna_off, nullptr));
        GAJE_TRY(get_usize(e, "dna_len", true, t.dna_len, nullptr));
        GAJE_TRY(get_usize(e, "c_off", true, t.c_off, nullptr));
        GAJE_TRY(get_usize(e, "c_len", true, t.c_len, nullptr));
        GAJE_TRY(get_usize(e, "anc_off", true, t.anc_off, nullptr));
        GAJE_TRY(get_usize(e, "anc_len", true, t.anc_len, nullptr));
        GAJE_TRY(get_usize(e, "bias_off", true, t.bias_off, nullptr));
        GAJE_TRY(get_usize(e, "bias_len", true, t.bias_len, nullptr));
        tensors_[t.name] = t;  // HashMap::insert: a later duplicate wins
    }
    return GAJE_OK;
}

const TensorEntry *FlatFile::find(const std::string &name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

int FlatFile::slice(uint64_t off, uint64_t len, const uint8_t **out) const {
    *out = nullptr;
    if (len == 0) return GAJE_OK;
    uint64_t start = header_.weights_offset + off;
    if (start < header_.weights_offset || start > size_ || len > size_ - start)
        return set_error(GAJE_ERR_INVALID_DATA, "tensor range [%llu, +%llu) exceeds the file",
                         (unsigned long long)start, (unsigned long long)len);
    *out = base_ + start;
    return GAJE_OK;
}

int FlatFile::model_config(ModelConfig &c) const {
    GAJE_TRY(parse_model_config(metadata_.data(), metadata_.size(), c));
    ArchDescriptor d;
    if (architecture_descriptor(header_, d)) {
        c.n_embd = d.n_embd;
        c.n_head = d.n_head;
        c.n_head_kv = d.n_head_kv;
        c.n_blocks = d.n_blocks;
        c.rope_base = d.rope_base;
        c.rope_style = d.rope_style;
        c.ffn_act = d.ffn_act;
        c.unpermute_weights = d.qk_permute;
    }
    return GAJE_OK;
}

}  // namespace gaje

// ------------------------------------------------------------- C ABI ----

namespace {

void fill_header(const gaje::FlatHeaderV2 &h, gaje_flat_header *o) {
    memset(o, 0, sizeof *o);
    o->version = h.version;
    o->flags = h.flags;
    o->num_tensors = h.num_tensors;
    o->group_size = h.group_size;
    o->quant_format = h.quant_format;
    o->arch_family = h.arch_family;
    o->arch_n_embd = h.arch_n_embd;
    o->arch_n_head = h.arch_n_head;
    o->arch_n_head_kv = h.arch_n_head_kv;
    o->arch_n_blocks = h.arch_n_blocks;
    o->arch_qk_permute = h.arch_qk_permute;
    o->quant_type = (int32_t)gaje::quantization_type(h);
    o->effective_group_size = gaje::effective_group_size(h);
    o->meta_len = h.meta_len;
    o->dir_len = h.dir_len;
    o->weights_offset = h.weights_offset;
    o->weights_len = h.weights_len;
}

}  // namespace

extern "C" int gaje_flat_header_from_bytes(const uint8_t *bytes, size_t len, gaje_flat_header *out) {
    gaje::clear_error();
    if (!out || (len > 0 && !bytes)) return gaje::set_error(GAJE_ERR_INVALID_ARG, "null argument");
    if (len < sizeof(gaje::FlatHeaderV2))
        return gaje::set_error(GAJE_ERR_TOO_SHORT, "Header buffer is less than 4096 bytes");
    gaje::FlatHeaderV2 h;
    memcpy(&h, bytes, sizeof h);
    if (memcmp(h.magic, "GAJE", 4) != 0)
        return gaje::set_error(GAJE_ERR_INVALID_MAGIC, "Invalid magic bytes (expected 'GAJE')");
    fill_header(h, out);
    return GAJE_OK;
}

extern "C" int gaje_flat_inspect(const char *path, gaje_flat_info *out) {
    gaje::clear_error();
    if (!path || !out) return gaje::set_error(GAJE_ERR_INVALID_ARG, "null argument");
    gaje::FlatFile f;
    GAJE_TRY(f.open(path));
    gaje::ModelConfig c;
    GAJE_TRY(f.model_config(c));
    memset(out, 0, sizeof *out);
    fill_header(f.header(), &out->header);
    out->n_embd = (int64_t)c.n_embd;
    out->n_head = (int64_t)c.n_head;
    out->n_head_kv = (int64_t)c.n_head_kv;
    out->n_blocks = (int64_t)c.n_blocks;
    out->vocab_size = c.has_vocab_size ? (int64_t)c.vocab_size : -1;
    out->eps = c.eps;
    out->rope_base = c.rope_base;
    out->rope_split = c.rope_style == "split" ? 1 : 0;
    out->use_genomic_norm = c.use_genomic_norm ? 1 : 0;
    out->has_descriptor = f.header().arch_family != 0 ? 1 : 0;
    out->n_tensors = (int32_t)f.entry_count();
    return GAJE_OK;
}

extern "C" int gaje_flat_tensor_entry(const char *path, const char *name, gaje_flat_tensor *out) {
    gaje::clear_error();
    if (!path || !name || !out) return gaje::set_error(GAJE_ERR_INVALID_ARG, "null argument");
    gaje::FlatFile f;
    GAJE_TRY(f.open(path));
    const gaje::TensorEntry *e = f.find(name);
    if (!e) return gaje::set_error(GAJE_ERR_NOT_FOUND, "Flat tensor entry '%s' not found", name);
    out->bit_depth = e->bit_depth;
    out->out_features = e->out_features;
    out->in_features = e->in_features;
    out->dna_off = e->dna_off;
    out->dna_len = e->dna_len;
    out->c_off = e->c_off;
    out->c_len = e->c_len;
    out->anc_off = e->anc_off;
    out->anc_len = e->anc_len;
    out->bias_off = e->bias_off;
    out->bias_len = e->bias_len;
    return GAJE_OK;
}
