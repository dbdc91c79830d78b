// .gaje.flat v2 container: header, metadata JSON, tensor directory, blob.
//
// Layout and semantics follow the reference reader:
//   FlatHeaderV2                    src/io/header/flat.rs:14-80
//   architecture_descriptor()       src/io/header/flat.rs:82-148, src/io/arch.rs:8-32
//   ModelConfig / ArchConfig        src/io/config.rs:17-48,92-145
//   FlatTensorEntry / open / slices src/io/flat_reader.rs:9-90
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>

namespace gaje {

#pragma pack(push, 1)
struct FlatHeaderV2 {
    char magic[4];
    uint32_t version;
    uint32_t flags;
    uint32_t num_tensors;
    uint64_t meta_len;
    uint64_t dir_len;
    uint64_t weights_offset;
    uint64_t weights_len;
    uint32_t group_size;
    uint32_t quant_format;
    uint32_t arch_family;
    uint32_t arch_n_embd;
    uint32_t arch_n_head;
    uint32_t arch_n_head_kv;
    uint32_t arch_n_blocks;
    uint32_t arch_qk_permute;
    uint8_t reserved[4016];
};
#pragma pack(pop)

static_assert(sizeof(FlatHeaderV2) == 4096, "FlatHeaderV2::SIZE");
static_assert(offsetof(FlatHeaderV2, version) == 4, "version at 4");
static_assert(offsetof(FlatHeaderV2, meta_len) == 16, "meta_len at 16");
static_assert(offsetof(FlatHeaderV2, weights_offset) == 32, "weights_offset at 32");
static_assert(offsetof(FlatHeaderV2, group_size) == 48, "group_size at 48");
static_assert(offsetof(FlatHeaderV2, quant_format) == 52, "quant_format at 52");
static_assert(offsetof(FlatHeaderV2, arch_family) == 56, "arch_family at 56");
static_assert(offsetof(FlatHeaderV2, arch_qk_permute) == 76, "arch_qk_permute at 76");
static_assert(offsetof(FlatHeaderV2, reserved) == 80, "reserved at 80");

enum class QuantFormat { LegacyCentroids = 0, Q4_0 = 1, Q8_0 = 2, Unknown = 3 };

QuantFormat quantization_type(const FlatHeaderV2 &h);
uint32_t effective_group_size(const FlatHeaderV2 &h);

// ArchitectureDescriptor (src/io/arch.rs:20-32); present when arch_family != 0.
struct ArchDescriptor {
    int family = 0;
    uint64_t n_embd = 0, n_head = 0, n_head_kv = 0, n_blocks = 0, head_dim = 0;
    float rope_base = 10000.0f;
    std::string rope_style = "split", ffn_act = "swiglu";
    bool qk_permute = false;
};
bool architecture_descriptor(const FlatHeaderV2 &h, ArchDescriptor &out);

// ModelConfig with its ArchConfig (serde defaults of config.rs:92-121).
struct ModelConfig {
    std::string name = "GAJE-Model", rope_style = "split", ffn_act = "swiglu";
    float rope_base = 10000.0f;
    bool use_genomic_norm = false;
    float rna_threshold = 0.5f;
    bool unpermute_weights = false;
    uint64_t n_embd = 0, n_head = 0, n_head_kv = 0, n_blocks = 0;
    bool has_vocab_size = false;
    uint64_t vocab_size = 0;
    float eps = 0.0f;
};
// Parses metadata JSON with serde's rules; GAJE_OK or GAJE_ERR_INVALID_DATA.
int parse_model_config(const char *json, size_t len, ModelConfig &out);

struct TensorEntry {
    std::string name;
    uint64_t bit_depth = 0, out_features = 0, in_features = 0;
    uint64_t dna_off = 0, dna_len = 0, c_off = 0, c_len = 0;
    uint64_t anc_off = 0, anc_len = 0, bias_off = 0, bias_len = 0;
};

// GajeFlatFileReader: a read-only mapping of one .gaje.flat file.
class FlatFile {
public:
    FlatFile() = default;
    ~FlatFile();
    FlatFile(const FlatFile &) = delete;
    FlatFile &operator=(const FlatFile &) = delete;

    int open(const char *path);  // GAJE_OK or a GAJE_ERR_* code (message recorded)

    const FlatHeaderV2 &header() const { return header_; }
    const std::string &metadata() const { return metadata_; }
    const TensorEntry *find(const std::string &name) const;
    // Bytes [weights_offset + off, + len) of the file, bounds-checked.
    int slice(uint64_t off, uint64_t len, const uint8_t **out) const;
    // load_genomic's config: JSON, then the header descriptor overrides
    // n_embd/n_head/n_head_kv/n_blocks/rope_base/rope_style/ffn_act/unpermute
    // (src/io/flat_reader.rs:125-139).
    int model_config(ModelConfig &out) const;
    size_t size() const { return size_; }
    size_t entry_count() const { return tensors_.size(); }

private:
    const uint8_t *base_ = nullptr;
    size_t size_ = 0;
    FlatHeaderV2 header_{};
    std::string metadata_;
    std::unordered_map<std::string, TensorEntry> tensors_;
};

}  // namespace gaje
