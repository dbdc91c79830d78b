// Launch interface between the host model code and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace gaje {

// Weight formats a GEMV can stream.
enum WeightFormat : int32_t {
    FMT_F32 = 0,   // GenomicF32 rows (lm_head / token_embd)
    FMT_Q4_0 = 1,  // 20-byte Q4_0Block rows
    FMT_LUT4 = 2,  // Genomic4Bit: 16-byte code blocks + 16-entry f32 tables
    FMT_Q8_0 = 3,  // 34-byte Q8_0Block rows
    FMT_G2 = 4,    // Genomic2Bit: 8-byte blocks of MSB-first 2-bit codes + 4 f32 centroids per block
};

constexpr uint32_t NAN_NONE = 0xFFFFFFFFu;

// Per-model device state read by the captured token graph.  Everything that
// changes between tokens lives here so the graph itself never changes.
struct DevState {
    int32_t pos;               // cached positions before the current token
    uint32_t token;            // current input token id
    int32_t step;              // index of the next greedy output token
    int32_t halted;            // a NaN guard fired: later graph replays do nothing
    uint32_t nan_code;         // min(layer * 8 + stage) over failed guards
    int32_t out_cap;           // capacity of the greedy output buffer
    unsigned long long argmax_key;  // packed (orderable logit, ~index) maximum
    float kwta_thr;            // the block K-WTA threshold of the current layer's input
};

// State of the greedy generate loop kept on the device (generate_native_core,
// llm/forward.rs:236-327): the generated tokens, their seen-set as a bitmap,
// the penalty and the EOS ids.  Its kernels run after each token step.
constexpr int GEN_MAX_EOS = 64;
struct GenState {
    int32_t n_gen;             // tokens generated so far (written to the token buffer)
    int32_t stop;              // 0 running, 1 EOS, 2 repetition-loop detector
    int32_t n_eos;
    float penalty;             // repetition_penalty, applied when > 1
    unsigned long long key;    // penalised argmax (orderable logit, ~index)
    uint32_t eos[GEN_MAX_EOS];
};
enum GenStop : int32_t { GEN_RUNNING = 0, GEN_EOS = 1, GEN_LOOP = 2 };

// NaN guard stages of RustGenomicBlock::forward_core (block/forward.rs).
enum NanStage : int32_t {
    ST_INPUT = 0,       // "Input x is NaN"                    :11-13
    ST_ATTN_NORM = 1,   // "NaN after attn rms_norm"           :22-24
    ST_UP = 2,          // "NaN in up"                         :97-99
    ST_FFN_OUT = 3,     // "NaN in ffn_out"                    :111-113
    ST_PROJ_FFN = 4,    // "NaN in projected_ffn"              :128-130
    ST_FINAL = 5,       // "NaN after projected_ffn addition"  :138-140
    ST_WAIT = 6,        // a bounded in-kernel wait ran out (an internal error:
                        // that step's attention outputs are invalid)
    ST_NONE = -1,
};

enum GemvMode : int32_t {
    MODE_STORE = 0,     // y[r] = row result
    MODE_RESIDUAL = 1,  // y[r] += row result (y is the residual stream)
    MODE_QKV = 2,       // fused QKV: RoPE on q/k rows, k/v appended to the cache
    MODE_SWIGLU = 3,    // fused gate_up: y[p] = swiglu(row p, row p + ffn)
    MODE_ARGMAX = 4,    // lm_head: y[r] = logit, running argmax into DevState
};

struct GemvParams {
    // weights: FMT_Q4_0 rows in the packed layout of launch_pack_q4_0; FMT_F32
    // rows row-major, or in the tiled layout of launch_pack_f32_tiled
    const uint8_t *w;
    int32_t fmt;
    int32_t f32_tiled;       // FMT_F32 weights in the tiled layout (K % 8 == 0)
    int32_t nontemporal;     // stream the weights past the caches (read-once tensors)
    int32_t tol;             // Q4_0 STORE streams: the regrouped walk, held to 1e-4 of each row's mass
    const float *lut;        // FMT_LUT4 tables / FMT_G2 centroids (T = 16 or 4 floats per block)
    int64_t lut_rows_own;    // rows r < lut_rows_own use the tables from r*nb*T, others from 0
    int32_t lut_block_stride;// T = one table per block, 0 = one shared table
    int32_t g2_modulated;    // FMT_G2: centroid k times g2_mod[k] (genomic.rs:60-63)
    float g2_mod[4];
    int32_t nb;              // K / 32
    int64_t rows_valid;      // rows with a complete weight row (others read as 0)
    int64_t N, K;
    // input and prologue
    const float *x;
    const float *norm_w;     // rms_norm weight (prologue) or null
    float eps;
    int32_t gnorm;           // use_genomic_norm scaling of the input (block/forward.rs:115-123)
    float h_scale;
    float *x_out;            // if set, workgroup 0 writes the prologue output here
    // per-row additive terms
    const float *bias;
    int64_t bias_len;
    const int64_t *a_ptr;    // sparse anchors (CSR over rows) or null
    const uint32_t *a_col;
    const uint16_t *a_val;
    // epilogue
    int32_t mode;
    float *y;
    int32_t head_dim;
    int32_t rope_split;
    int64_t q_rows, kv_rows;
    const float *rope_cos, *rope_sin;  // [max_ctx][head_dim/2]
    float *q_out;
    float *k_cache;                    // this layer: [n_kv][head_dim][kv_cap]
    float *v_cache;                    // this layer: [n_kv][head_dim][kv_cap]
    int64_t kv_head_stride;            // kv_cap * head_dim
    int64_t kv_cap;                    // positions per cache row
    int64_t ffn;
    // chain-major copies (element e at (e % 8) * cm_stride + e / 8, rows of
    // cm_stride = gemv_chain_stride(K) floats, zero past K / 8): y_cm, when
    // set, receives a SwiGLU output as well as y; x_cm, when set, holds x in
    // that layout for the kernels that read it so (the others read x)
    float *y_cm;
    const float *x_cm;
    int32_t cm_stride;
    // the previous block's lateral_inhibition_kwta, fused (kwta_k > 0; the
    // chain kernel only): MODE_QKV selects the threshold of x (its k-th largest
    // value), applies x < thr -> -1e9 to its copy and has workgroup 0 store thr
    // at kwta_thr; MODE_RESIDUAL applies the same mask to the residual it reads
    int64_t kwta_k;
    float *kwta_thr;
    // guards (stage < 0 disables a check)
    DevState *st;
    int32_t layer;
    int32_t st_in, st_norm, st_a, st_b;
};

// Validates shapes against what the kernels assume and launches; returns a
// GAJE_* status.
int launch_gemv(const GemvParams &p, hipStream_t s);
// Whether launch_gemv runs p on the chain kernel, the one kernel that takes
// the fused K-WTA fields (launch_gemv rejects kwta_k > 0 elsewhere).
bool gemv_chain_serves(const GemvParams &p);
// Row stride (floats) of the chain-major activation layout for in_features K.
int gemv_chain_stride(int64_t K);
// Q4_0Block rows (file layout, K % 32 == 0) -> the GEMV's packed row layout.
// A packed tensor is followed by Q4_TAIL_PAD bytes that the GEMV's prefetch
// may read (and never uses); q4_0_packed_bytes includes them.
constexpr int64_t Q4_TAIL_PAD = 2048;
int launch_pack_q4_0(const uint8_t *src, uint8_t *dst, int64_t N, int64_t K, hipStream_t s);
// genomic_dot_product_q4_0 straight from Q4_0Block rows (no packing).
int launch_q4_0_gemv_blocks(const uint8_t *blocks, const float *x, const float *bias, int64_t bias_len, float *y,
                            int64_t n, int64_t k, hipStream_t s);
int64_t q4_0_packed_bytes(int64_t N, int64_t K);
// Q8_0Block rows (K % 32 == 0) -> tiles of 8 rows: per group of four blocks,
// the 8 rows' codes (128 bytes each, chain l's at [16l, 16l+16)) and then
// their four f16 scales (8 bytes each); Q8_TAIL_PAD zero bytes follow.
constexpr int64_t Q8_TAIL_PAD = 4096;
int launch_pack_q8_0(const uint8_t *src, uint8_t *dst, int64_t N, int64_t K, hipStream_t s);
int64_t q8_0_packed_bytes(int64_t N, int64_t K);
// Row-major f32 rows (K % 8 == 0) -> the tiled layout: tiles of 32 rows, and in
// a tile the 8-float chunk c of rows 0..31 is one contiguous KiB, so a wave
// holding the tile's rows reads each chunk with one coalesced load.  Rows past
// N in the last tile are zero.
int launch_pack_f32_tiled(const float *src, float *dst, int64_t N, int64_t K, hipStream_t s);
int64_t f32_tiled_bytes(int64_t N, int64_t K);
// Dynamic LDS a workgroup may use on the current device.
size_t max_lds_per_block();
// Compute units of the current device.
int device_cu_count();
// Dynamic LDS the GEMV needs for in_features K (so callers can check limits).
size_t gemv_lds_bytes(int64_t K, int fmt, bool norm);

struct AttnParams {
    const float *q;          // roped queries [n_head * head_dim]
    const float *k_cache;    // this layer: [n_kv][head_dim][kv_cap]
    const float *v_cache;    // this layer: [n_kv][head_dim][kv_cap]
    int64_t kv_head_stride;  // kv_cap * head_dim
    int32_t n_head, n_head_kv, head_dim;
    int64_t kv_cap;          // KV capacity (sizes the LDS score buffer)
    float *out;              // [n_head * head_dim]
    DevState *st;            // positions 0..st->pos are attended; if null, 0..ctx-1
    int64_t ctx;
    // batched decode (seq_pos non-null): blockIdx.z = sequence z attends to
    // positions 0..seq_pos[z] of its own cache (k/v_cache + z * seq_kv_stride);
    // its q and out rows are z * seq_q_stride floats on; seq_pos[z] < 0 skips
    // it; out_chain_major writes each out row chain-major over n_head*head_dim
    const int32_t *seq_pos;
    int64_t seq_kv_stride, seq_q_stride;
    int32_t n_seq;
    int32_t out_chain_major;
    // where a kernel whose LDS producers and consumers wait on each other
    // reports a wait that ran out of its spin bound (layer * 8 + ST_WAIT):
    // st->nan_code for one sequence, seq_nan[z] for batched sequence z
    uint32_t *seq_nan;
    int32_t layer;
};
int launch_attention(const AttnParams &p, hipStream_t s);
size_t attention_lds_bytes(int head_dim, int64_t max_ctx);
// Largest KV capacity whose scores fit the attention kernel's LDS buffer.
constexpr int64_t MAX_CTX = 12288;

struct EmbedParams {
    const uint8_t *w;        // FMT_Q4_0 / FMT_Q8_0: packed rows
    int32_t fmt;
    const float *lut;
    int64_t lut_rows_own;
    int32_t lut_block_stride;
    int64_t lut_len;         // floats in lut (FMT_G2: blocks past it read the first table)
    int64_t vocab, rows_valid, K;
    float *h;
    DevState *st;
};
int launch_embed(const EmbedParams &p, hipStream_t s);
// Embedding rows of ids[0..n) into p.h [n][K] (p.st unused).
int launch_embed_rows(const EmbedParams &p, const uint32_t *ids, int64_t n, hipStream_t s);

// Activation rows -> the f16 hi/lo planes of the MFMA matrix product (optional
// rms_norm first).  Row m of the planes holds x' = x * 2^ex[m] split as
// hi = f16(x'), lo = f16(x' - hi).
struct SplitParams {
    const float *x;          // [M][ldx] fp32 rows (with `up`: the gate rows)
    int64_t ldx;
    const float *norm_w;     // rms_norm weight [K] or null
    float eps;
    const float *up;         // swiglu prologue: up rows [M][ldx], or null
    int32_t gnorm;           // with `up`: use_genomic_norm scaling (h_scale)
    float h_scale;
    float *x_out;            // the prologue's output rows [M][ldo], or null
    int64_t ldo;
    DevState *st;            // NaN guards (stage < 0 or st null: none): st_a on the
    int32_t layer;           // input (or the up rows), st_b on the norm / swiglu output
    int32_t st_a, st_b;
    uint16_t *xh, *xl;       // f16 planes [M][ldh]
    int64_t ldh;
    int *ex;                 // [M] row exponents
    int64_t M, K;
    const int32_t *rows;     // plane row m takes input row rows[m] (a gather), or null
    // With sh set, xh alone takes the block-scaled product's layout (per
    // block its hi then its lo halves, each block permuted, see gemm.hip;
    // ldh >= 2K, xl unused) and sh/sl [M][ldsum] receive the block sums
    // 2^-5 * sum_{k in b} x'[k] as an f16 pair (zero past K/32).
    uint16_t *sh, *sl;
    int64_t ldsum;
    // Split-K prologue (without up or rows): the input rows are first formed
    // from the partials of a block-scaled product whose reduce was deferred,
    // as gemm_reduce_kernel would: x = resid + (flush_small(sum_z part[z]) +
    // bias), written to x (in place over resid when they alias) before the split.
    const float *part;       // [nsplit][M][K], or null
    int32_t nsplit;
    const float *bias;
    int64_t bias_len;
    const float *resid;      // [M][ldx] or null
    int32_t st_ya, st_yb;    // the product's NaN guards (after the bias, after resid)
    int32_t y_layer;         // the product's layer, for those guards
    // Attention-merge prologue (without up, rows, part or norm): row t is the
    // causal attention output of query t, merged from the key chunks' partials
    // (PrefillAttnParams::ws, chunks of attn_kch keys; K = n_head * head_dim).
    const float *attn_ws;
    int64_t attn_kch, attn_pos0;
    int32_t attn_hd, attn_heads;
};
int launch_split_rows(const SplitParams &p, hipStream_t s);
// Per packed Q4_0 row: the exponent that scales its largest |d| into [2^14, 2^15).
int launch_q4_row_exponents(const uint8_t *packed, int64_t N, int64_t K, int *ew, hipStream_t s);
// The same for n matrices of one shape in one launch: ew[i*N .. ] for packed[i].
int launch_q4_row_exponents_batch(const uint8_t *const *packed, int n, int64_t N, int64_t K, int *ew, hipStream_t s);

// Y = X W^T over packed Q4_0 rows on the MFMA units (f16 hi/lo operand pairs,
// fp32 accumulation): per row, the dot flushed like the reference's, + bias,
// + residual.
// Experts of one MoE layer (and of a grouped matrix product).
constexpr int MOE_MAX_EXPERTS = 16;

struct GemmQ4Params {
    const uint8_t *w;        // packed rows (launch_pack_q4_0)
    const int *ew;           // [N] weight row exponents
    const uint16_t *xh, *xl; // activation planes (launch_split_rows)
    const int *ex;
    int64_t ldh;
    const float *bias;
    int64_t bias_len;
    const float *resid;      // Y = resid + row result, or null (may alias y)
    int64_t ldr;
    float *y;
    int64_t ldy;
    float *part;             // split-K partials [splits][M][N] (plan.part_floats)
    int64_t M, N;
    int32_t nb;              // K / 32
    int32_t kb_per;          // set by launch_gemm_q4 from the plan
    DevState *st;            // NaN guards (or null): st_a on the row result,
    int32_t layer;           // st_b after the residual add
    int32_t st_a, st_b;
    // grouped products (one launch for every expert): with g_counts set,
    // blockIdx.y = e * g_mtiles + tile, expert e owns rows [g_offsets[e],
    // g_offsets[e] + g_counts[e]) of the planes and of y (M = all rows) and
    // multiplies them by gw[e] (row exponents gew[e])
    const int32_t *g_counts, *g_offsets;
    int32_t g_groups, g_mtiles;
    const uint8_t *gw[MOE_MAX_EXPERTS];
    const int *gew[MOE_MAX_EXPERTS];
};
struct GemmPlan {
    int mt;                  // activation rows per workgroup (128 or 256)
    int splits;              // K splits
    int kb_per;              // blocks per split (multiple of 4)
    int64_t part_floats;     // partial buffer the splits need (0 if one split)
};
GemmPlan plan_gemm_q4(int64_t M, int64_t N, int64_t K);

// Block-scaled Q4_0 product (the dense products of prefill and
// gaje_hip_q4_0_gemm_mfma): Y = X W^T as sum_b scale_b P_b + sum_b min_b X_b
// per block b, P_b on the MFMA units with the 4-bit codes as exact f16
// operands.  Its activation planes come from launch_split_rows with sh set.
struct GemmBsParams {
    const uint16_t *wf;      // the rows' code fragments (launch_q4_frags)
    const float *wsc;        // and their scales
    int64_t nbp4;            // q4_frag_nbp4(K)
    const uint16_t *mins;    // the rows' block mins as f16, [N][ldm] (launch_q4_mins)
    int64_t ldm;             // >= gemm_bs_sum_cols(K)
    const uint16_t *xh;      // activation plane [plane_rows][ldh] (hi | lo per block, ldh >= 2K)
    int64_t plane_rows;      // rows allocated: >= gemm_bs_plane_rows(M) (rows past M are read, not used)
    const uint16_t *sh, *sl; // block-sum planes [M][ldsum]
    const int *ex;           // [M] activation row exponents
    int64_t ldh, ldsum;
    const float *bias;
    int64_t bias_len;
    const float *resid;      // Y = resid + row result, or null (may alias y)
    int64_t ldr;
    float *y;
    int64_t ldy;
    float *part;             // split-K partials [splits][M][N] (plan.part_floats)
    int64_t M, N;
    int32_t nb;              // K / 32
    DevState *st;            // NaN guards as in GemmQ4Params
    int32_t layer;
    int32_t st_a, st_b;
    int32_t defer_reduce;    // splits > 1: leave the partials for a split pass's prologue
    // grouped products (the MoE experts, one launch for every expert): with
    // g_counts set, the row tiles are g_groups x g_mtiles; tile mt of group e
    // covers rows g_offsets[e] + mt * tile.. of the planes and of y, up to
    // g_offsets[e] + g_counts[e] (M = all rows), and multiplies them by group
    // e's operands at wf + e * g_wf_stride halves, wsc + e * g_wsc_stride
    // floats and mins + e * g_mins_stride halves
    const int32_t *g_counts, *g_offsets;
    int32_t g_groups, g_mtiles;
    int64_t g_wf_stride, g_wsc_stride, g_mins_stride;
};
struct GemmBsPlan {
    int waves;               // 32-row wave tiles per workgroup (2, 4 or 8)
    int mtiles, ntiles;      // activation-row tiles, weight-row tiles (<= 144 rows)
    int splits, kb_per;      // K splits of kb_per blocks (a multiple of 4)
    int64_t part_floats;     // partial buffer the splits need (0 if one split)
};
constexpr int BS_WR_ROWS = 32;  // activation rows per wave tile of the block-scaled product
GemmBsPlan plan_gemm_q4_bs(int64_t M, int64_t N, int64_t K);
// Grouped plan: R rows over E groups of at most T rows each (mtiles = E x the
// tiles of T rows; the tile height follows the mean group size).
GemmBsPlan plan_gemm_q4_bs_grouped(int64_t R, int64_t E, int64_t T, int64_t N, int64_t K);
int launch_gemm_q4_bs(const GemmBsParams &p, const GemmBsPlan &plan, hipStream_t s);
// Columns of the block-sum planes for a K: K/32 rounded up to a multiple of 32.
int64_t gemm_bs_sum_cols(int64_t K);
// The block mins of packed Q4_0 rows as a dense f16 matrix [N][ldm] (zero past
// K / 32 blocks), ldm >= gemm_bs_sum_cols(K): the min term's operand.
int launch_q4_mins(const uint8_t *packed, int64_t N, int64_t K, uint16_t *mins, int64_t ldm, hipStream_t s);
// The block-scaled product's weight operands from packed Q4_0 rows: per
// 16-row tile and block, the MFMA fragment of the codes as f16 (1 KiB) and the
// 16 scales as fp32, zero past row N and block K / 32 (blocks padded to a
// multiple of 4): q4_frag_halves(N, K) halves and q4_frag_scale_floats(N, K) floats.
int64_t q4_frag_nbp4(int64_t K);
int64_t q4_frag_halves(int64_t N, int64_t K);
int64_t q4_frag_scale_floats(int64_t N, int64_t K);
int launch_q4_frags(const uint8_t *packed, int64_t N, int64_t K, uint16_t *wf, float *wsc, hipStream_t s);
// Rows the activation plane must hold for M activation rows (a multiple of 256).
int64_t gemm_bs_plane_rows(int64_t M);

// Grouped plan: 128-row tiles, splits sized for R rows spread over E groups.
GemmPlan plan_gemm_q4_grouped(int64_t R, int64_t E, int64_t N, int64_t K);
int launch_gemm_q4(const GemmQ4Params &p, const GemmPlan &plan, hipStream_t s);

// Prompt prefill: RoPE + KV append for P tokens at positions pos0.. of one layer.
struct PrefillRopeParams {
    const float *qkv;        // [P][ldq] rows q | k | v (bias added)
    int64_t ldq;
    float *q_out;            // [P][n_head * head_dim] roped queries
    float *k_cache, *v_cache;// this layer: [n_kv][head_dim][cap]
    int64_t cap, pos0, P;
    int32_t n_head, n_kv, head_dim, rope_split;
    const float *rope_cos, *rope_sin;  // [cap][head_dim / 2]
    // batched decode: row t is sequence t at position seq_pos[t] (< 0: skipped)
    // of its own cache (k/v_cache + t * seq_kv_stride); pos0 unused
    const int32_t *seq_pos;
    int64_t seq_kv_stride;
    // prefill: the qkv rows from a split-K product's partials, [nsplit][P][ldq]
    // (its deferred reduce: flush_small(sum) + bias), or null
    const float *part;
    int32_t nsplit;
    const float *bias;
    int64_t bias_len;
    // prefill: also the keys' and values' f16 pairs for the attention
    // (PrefillAttnParams::kv16, kv16_ntiles 32-key tiles), or null
    uint16_t *kv16;
    int32_t kv16_ntiles;
};
int launch_rope_kv(const PrefillRopeParams &p, hipStream_t s);
// Causal GQA attention of P queries (positions pos0..) over the cache.
struct PrefillAttnParams {
    const float *q;          // [P][n_head * head_dim] roped
    const float *k_cache, *v_cache;  // this layer: [n_kv][head_dim][cap]
    int64_t cap, pos0, P;
    int32_t n_head, n_kv, head_dim;
    float *out;              // [P][n_head * head_dim]
    float *ws;               // key-chunk partials: prefill_attn_ws_floats(P, n_head, head_dim) floats
    uint16_t *kv16;          // f16 pairs of the keys and values: prefill_kv16_halves(kv16_keys, ..) halves
    int64_t kv16_keys;       // positions kv16 holds (>= pos0 + P)
    int32_t merged_later;    // the chunks' partials are left for a split pass (SplitParams::attn_ws)
    int32_t kv16_rope;       // launch_rope_kv wrote the chunk's positions of kv16
};
// Keys are split into at most PREFILL_ATTN_CHUNKS chunks per query block,
// each computed by its own workgroup and merged afterwards.
constexpr int PREFILL_ATTN_CHUNKS = 8;
int64_t prefill_attn_ws_floats(int64_t P, int64_t n_head, int64_t head_dim);
// Key chunk length of the attention's partials for `keys` keys (the merge's kch).
int64_t prefill_attn_kch(int64_t keys);
// A record of the partials: {m, l, -, -, O[head_dim]} (O 16-byte aligned).
constexpr int PREFILL_ATTN_REC_PAD = 4;
int64_t prefill_kv16_halves(int64_t keys, int64_t n_kv, int64_t head_dim);
int launch_prefill_attention(const PrefillAttnParams &p, hipStream_t s);

// Batched decode: NV (<= 16) activation vectors per matvec, each product in
// the batch-1 order (bit-identical per vector).
struct BatchGemvParams {
    const uint8_t *w;        // FMT_Q4_0 packed rows, or FMT_F32 tiled rows
    int32_t fmt;
    int32_t f32_tiled;
    int32_t nb;              // K / 32 (Q4_0)
    int64_t N, K;
    const float *x;          // [nv][ldx]; FMT_Q4_0: each row chain-major (element k at (k%8)*K/8 + k/8)
    int64_t ldx;
    int32_t nv;              // vectors (sequences)
    const float *bias;
    int64_t bias_len;
    const int64_t *a_ptr;    // sparse anchors (Q4_0 only) or null
    const uint32_t *a_col;
    const uint16_t *a_val;
    int32_t mode;            // MODE_STORE or MODE_RESIDUAL (y += row result)
    float *y;                // [nv][ldy]
    int64_t ldy;
    uint32_t *nan_codes;     // [nv] min(layer * 8 + stage) of failed guards, or null
    int32_t layer, st_a, st_b;
};
int launch_gemv_batch(const BatchGemvParams &p, hipStream_t s);
// Activation lanes a batch of n sequences is padded to (4, 8 or 16).
int batch_lanes(int64_t n);
// Per-sequence row passes of the batched step.
struct BatchRowParams {
    const float *x;          // [nv][ldx] (swiglu: gate | up rows of K each)
    int64_t ldx;
    float *y;                // [nv][ldy]
    int64_t ldy;
    const float *w;          // rms_norm weight [K]
    int64_t K;
    int32_t nv;
    float eps, h_scale;
    int32_t gnorm;
    int32_t chain_major;     // write y rows chain-major (input of a batched Q4_0 matvec)
    uint32_t *nan_codes;
    int32_t layer, st_a, st_b;
};
int launch_rmsnorm_rows(const BatchRowParams &p, hipStream_t s);
int launch_swiglu_rows(const BatchRowParams &p, hipStream_t s);
int launch_argmax_rows(const float *x, int64_t n, int64_t ld, int64_t rows, uint32_t *out, hipStream_t s);
// Device-side per-sequence state of a batched decode (arrays of `lanes`).
constexpr uint32_t BATCH_INACTIVE = 0xFFFFFFFFu;
struct BatchState {
    int32_t nseq, lanes;
    int32_t *pos;            // cached length per sequence
    int32_t *cur_pos;        // this step's position, -1 = not stepping
    int32_t *halted;         // a guard fired: the sequence stops
    uint32_t *err;           // the stage code that halted it
    uint32_t *tok;           // this step's token (greedy: the previous argmax)
    uint32_t *embed_ids;     // embedding row ids of this step (0 for idle lanes)
    uint32_t *next;          // argmax of this step's logits
    uint32_t *nan_codes;     // guards of this step
};
int launch_batch_begin(const BatchState &b, const uint32_t *ids, int64_t n, int64_t i, hipStream_t s);
int launch_batch_end(const BatchState &b, uint32_t *out, int64_t n, int64_t i, int greedy, hipStream_t s);

// Mixture-of-experts FFN (top-2 routing over Q4_0 SwiGLU experts).
struct MoeParams {
    const float *x;          // [T][ldx] token activations
    int64_t ldx, T, h;
    const float *router;     // [n_expert][h] f32 router rows
    int32_t n_expert;
    int32_t *top_idx;        // [T][2] chosen experts (top-1, top-2)
    float *top_w;            // [T][2] renormalised weights
    int32_t *rows;           // [2T] token of each dispatched row (experts in id order)
    int32_t *slot;           // [T][2] dispatched row of each (token, choice)
    int32_t *counts, *offsets;  // [n_expert]
    float *y;                // [T][ldy] output
    int64_t ldy;
};
int launch_moe_route(const MoeParams &p, hipStream_t s);
int launch_moe_combine(const MoeParams &p, const float *Y, hipStream_t s);
// The combine over the S = nsplit split-K partials [S][R][h] of the down
// product (its reduce deferred): sums them as gemm_reduce_kernel would.
int launch_moe_combine_split(const MoeParams &p, const float *part, int nsplit, int64_t R, hipStream_t s);

int launch_finalize(DevState *st, uint32_t *out_tokens, hipStream_t s);
int launch_kwta(float *x, int64_t n, int64_t k, DevState *st, hipStream_t s);
// Greedy generate step on the device: gen_select replaces st->token with the
// argmax of the penalised logits (penalty > 1) into gs->key; gen_control takes
// that choice (select) or st->token, appends it to the generated tokens and
// stops the loop (halting the state) on EOS or a repetition loop.  seen:
// ceil(n / 32) words.
int launch_gen_select(const float *logits, int64_t n, const uint32_t *seen, DevState *st, GenState *gs, hipStream_t s);
int launch_gen_control(DevState *st, GenState *gs, uint32_t *seen, int64_t n_seen, uint32_t *tokens, int select,
                       hipStream_t s);
int launch_argmax(const float *x, int64_t n, uint32_t *idx, hipStream_t s);
int launch_dequant_q4_0(const uint8_t *blocks, float *out, int64_t nblocks, hipStream_t s);
int launch_dequant_q8_0(const uint8_t *blocks, float *out, int64_t nblocks, hipStream_t s);
int launch_rmsnorm(const float *x, const float *w, float eps, float *y, int64_t n, hipStream_t s);
int launch_swiglu(const float *g, const float *u, float *out, int64_t n, hipStream_t s);
int launch_expf(const float *x, float *y, int64_t n, hipStream_t s);
int launch_fill_u32(uint32_t *p, uint32_t v, int64_t n, hipStream_t s);
// bytes == 0: an empty kernel of grid x block; else a plain read of `bytes`
// (>= 256) of buf, whose first 256 bytes it may overwrite.
int launch_floor_probe(const void *buf, int64_t bytes, unsigned grid, unsigned block, hipStream_t s);
// Host-driven state update ordered on the stream.  Negative pos / out_cap /
// step keep the current value; reset_guards clears halted, nan_code and the
// argmax.
int launch_state_set(DevState *st, int32_t pos, uint32_t token, int32_t out_cap, int32_t step, int reset_guards,
                     hipStream_t s);

}  // namespace gaje
