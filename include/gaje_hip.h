/*
 * gaje_hip.h — C ABI of the MI355X (gfx950) GAJE quantised decode path.
 *
 * Each entry point names the reference interface it replaces (paths are in
 * the erickaguilar/gaje-semantic-compression tree).  A Rust `extern "C"` shim
 * in the upstream crate binds these from GenomicLinear::forward_core /
 * GenomicLLM::forward_core; the ctypes mirror in gaje_hip/ binds them for
 * Python callers.
 *
 * Conventions
 *   - Status: 0 = success, negative = one of the GAJE_ERR_* codes below; the
 *     message of the last failure on the calling thread is gaje_hip_last_error()
 *     and carries the reference's own text where one exists.
 *   - Ownership: host buffers are caller-owned.  Device buffers passed to the
 *     operator API are caller-owned device pointers.  A model handle owns its
 *     HBM weights, KV cache, stream and captured graphs.
 *   - Threading: a model handle is not re-entrant (the reference's &mut self);
 *     distinct handles are independent, each with its own stream.
 *   - `stream` arguments are hipStream_t values cast to void*; NULL = the
 *     default stream.
 */
#ifndef GAJE_HIP_H
#define GAJE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status -- */
enum {
    GAJE_OK = 0,
    GAJE_ERR_INVALID_ARG = -1,   /* bad argument (null pointer, size out of range)        */
    GAJE_ERR_IO = -2,            /* std::io::Error from open/mmap (flat_reader.rs:33-35)  */
    GAJE_ERR_TOO_SHORT = -3,     /* HeaderError::TooShort (header/types.rs:16)            */
    GAJE_ERR_INVALID_MAGIC = -4, /* HeaderError::InvalidMagic (header/types.rs:17)        */
    GAJE_ERR_INVALID_DATA = -5,  /* io::ErrorKind::InvalidData: utf-8/JSON (flat_reader.rs:47-55,125-126) */
    GAJE_ERR_NOT_FOUND = -6,     /* io::ErrorKind::NotFound: missing tensor (flat_reader.rs:93-98) */
    GAJE_ERR_NAN = -7,           /* Err("NaN ...") guards of RustGenomicBlock::forward_core */
    GAJE_ERR_MODEL = -8,         /* other Err(String): "LM Head out_features is 0!", "Prompt tokens cannot be empty" */
    GAJE_ERR_UNSUPPORTED = -9,   /* a tensor format or shape this build does not run */
    GAJE_ERR_HIP = -10,          /* HIP runtime failure */
    GAJE_ERR_NO_DEVICE = -11     /* no usable gfx950 device */
};

/* Message of the last failure on this thread (thread-local copy). */
const char *gaje_hip_last_error(void);

/* --------------------------------------------------------------- runtime -- */
/* Thin device-memory / stream / event helpers so that a foreign caller (the
 * Rust shim, ctypes) can drive the operator API without its own HIP binding. */
int gaje_hip_device_count(int *count);
int gaje_hip_set_device(int device);
int gaje_hip_device_name(int device, char *buf, size_t buflen);
int gaje_hip_malloc(void **ptr, size_t bytes);
int gaje_hip_free(void *ptr);
int gaje_hip_memcpy_h2d(void *dst, const void *src, size_t bytes);
int gaje_hip_memcpy_d2h(void *dst, const void *src, size_t bytes);
int gaje_hip_memcpy_d2d(void *dst, const void *src, size_t bytes);
int gaje_hip_memset(void *dst, int value, size_t bytes);
int gaje_hip_device_synchronize(void);
int gaje_hip_stream_create(void **stream);
int gaje_hip_stream_destroy(void *stream);
int gaje_hip_stream_synchronize(void *stream);
int gaje_hip_event_create(void **event);
int gaje_hip_event_destroy(void *event);
int gaje_hip_event_record(void *event, void *stream);
int gaje_hip_event_synchronize(void *event);
int gaje_hip_event_elapsed_ms(void *start, void *stop, float *ms);

/* ------------------------------------------------------ operator API ------ */
/* All pointers are device pointers; y/out are overwritten.  k = in_features,
 * n = out_features; row i of a Q4_0 tensor is blocks [i*(k/32), (i+1)*(k/32)).
 * bias may be NULL; rows i < bias_len add bias[i] (compute_single_row's
 * `self.bias.get(i)`, linear/forward.rs:113-115). */

/* Q4_0 weights are packed once on the device before the matvec reads them,
 * as the reference builds its GenomicQ4_0 weights once from the mmap'd file
 * (GenomicLinear::new, linear/init.rs:12-40).  The packed layout permutes the
 * nibbles and scale/min words inside each group of four Q4_0Blocks (80 bytes)
 * so that every accumulation chain reads its codes with one load; it holds the
 * same bits.  gaje_hip_q4_0_packed_bytes gives its size for an n x k tensor
 * (n * ceil(k/128) * 80; equal to the file's n * k/32 * 20 when k % 128 == 0)
 * or -1 if k is not a positive multiple of 32. */
int64_t gaje_hip_q4_0_packed_bytes(int64_t n, int64_t k);
int gaje_hip_q4_0_pack(const void *blocks, void *packed, int64_t n, int64_t k, void *stream);

/* One Q4_0 matvec over packed rows: GenomicLinear::forward_core on the
 * GenomicQ4_0 variant (linear/forward.rs:84-92,119-132) with the per-row
 * genomic_dot_product_q4_0 (compute/kernels/genomic.rs:210-336), including its
 * |t| < 1e-6 -> 0 flush before the bias add. */
int gaje_hip_q4_0_gemv(const void *packed, const float *x, const float *bias, int64_t bias_len,
                       float *y, int64_t n, int64_t k, void *stream);

/* The same matvec in tolerance mode, for callers that accept the 1e-4 bound
 * of the GEMV rather than the reference's bits: each row regrouped by block
 * as scale * sum(q x) + min * sum(x) (genomic_dot_product_q4_0's value,
 * compute/kernels/genomic.rs:210-336, in another summation order, then the
 * same |t| < 1e-6 flush and bias add), held to 1e-4 of the row's sum of
 * |w x|.  No reference function has this form: it replaces
 * genomic_dot_product_q4_0 where that bound is the contract.  Long matrices
 * (the streaming kernel's shapes, no bias) run the regrouped walk; other
 * shapes and inputs with some |x| >= 2^100 run the exact one. */
int gaje_hip_q4_0_gemv_tol(const void *packed, const float *x, const float *bias, int64_t bias_len, float *y,
                           int64_t n, int64_t k, void *stream);

/* The same matvec straight from the file's Q4_0Block rows (20 bytes per
 * block, n * k/32 blocks, 4-byte aligned), with no packing: the operator as
 * genomic_dot_product_q4_0(&[Q4_0Block], &[f32]) takes it
 * (compute/kernels/genomic.rs:210-336), bit for bit like gaje_hip_q4_0_gemv.
 * The packed entry above is the faster one for weights that are read again. */
int gaje_hip_q4_0_gemv_blocks(const void *blocks, const float *x, const float *bias, int64_t bias_len, float *y,
                              int64_t n, int64_t k, void *stream);

/* The same Q4_0 matvec for m activation rows at once (Y[m][n] = X[m][k] W^T):
 * m independent GenomicLinear::forward_core calls sharing one weight read.
 * No reference function batches rows; semantics are per row as above. */
int gaje_hip_q4_0_gemm(const void *packed, const float *X, const float *bias, int64_t bias_len,
                       float *Y, int64_t m, int64_t n, int64_t k, void *stream);

/* The same product on the MFMA units, for prompt prefill and other calls
 * with many activation rows (Y[m][n] = X[m][k] W^T, + bias).  Not bit-exact:
 * the dot product is regrouped by Q4_0 block (scale times the block's
 * code product, plus min times the block's activation sum), the activations
 * carried as f16 hi/lo pairs and the 4-bit codes exactly, with fp32
 * accumulation, so each output is the reference's dot product
 * (genomic.rs:263-336, then the |t| < 1e-6 flush and the bias add of
 * linear/forward.rs:84-92,113-115) to about fp32 accuracy in a different
 * summation order.  `workspace` is 16-byte aligned device memory of at least
 * gaje_hip_q4_0_gemm_mfma_workspace(m, n, k) bytes (-1 for an invalid shape);
 * it also holds the weight rows' codes as f16 MFMA fragments (about two bytes
 * per weight), rebuilt from `packed` on each call; calls that share a
 * workspace must not overlap. */
int64_t gaje_hip_q4_0_gemm_mfma_workspace(int64_t m, int64_t n, int64_t k);
int gaje_hip_q4_0_gemm_mfma(const void *packed, const float *X, const float *bias, int64_t bias_len,
                            float *Y, int64_t m, int64_t n, int64_t k, void *workspace,
                            int64_t workspace_bytes, void *stream);

/* gaje_hip_q4_0_gemm_mfma without a workspace argument and without allocating:
 * no counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  The workspace is a file-scope device array of
 * GAJE_NOALLOC_SCRATCH_BYTES that each GPU holds for the life of the process;
 * a product whose gaje_hip_q4_0_gemm_mfma_workspace(m, n, k) exceeds it fails
 * with GAJE_ERR_UNSUPPORTED.  Every call on one GPU shares that array: calls
 * that overlap on one GPU (several streams or host threads) race.  Results are
 * those of gaje_hip_q4_0_gemm_mfma bit for bit. */
#define GAJE_NOALLOC_SCRATCH_BYTES (64ll << 20)
int gaje_hip_q4_0_gemm_mfma_noalloc(const void *packed, const float *X, const float *bias, int64_t bias_len,
                                    float *Y, int64_t m, int64_t n, int64_t k, void *stream);

/* Mixture-of-experts SwiGLU FFN layer with top-2 routing over Q4_0 experts.
 * No reference counterpart (the reference has no MoE); a composition of its
 * primitives: router logits l_e = dot_product(x_t, router_e) (dot.rs:23-94,
 * bit-exact), p = softmax(l) with expf(l_e - max) and a serial sum in expert
 * order, the two largest p (ties to the lower expert id) with weights
 * renormalised to w/(p_a + p_b), expert FFN_e(x) = down_e(swiglu_balanced(
 * gate_e(x), up_e(x))) (linear/forward.rs:84-92, activation.rs:35-51), and
 * y_t = (w_a FFN_a(x_t)) + (w_b FFN_b(x_t)).  Routing is exact; the expert
 * products run on the MFMA units (fp32 accuracy, as gaje_hip_q4_0_gemm_mfma).
 * x, y: [T][h] device f32; router: [n_expert][h] device f32; gate_up[e] and
 * down[e] (host arrays of device pointers): packed Q4_0 rows (gaje_hip_q4_0_pack)
 * of [2 ffn][h] (gate rows then up rows) and [h][ffn]; top_idx, top_w
 * (optional, device [T][2]) receive the routing.  h and ffn multiples of 32,
 * 2..16 experts, T <= 65535. */
int64_t gaje_hip_moe_ffn_workspace(int64_t T, int64_t h, int64_t ffn, int64_t n_expert);
int gaje_hip_moe_ffn(const float *x, int64_t T, int64_t h, const float *router, int64_t n_expert,
                     const void *const *gate_up, const void *const *down, int64_t ffn, float *y,
                     int32_t *top_idx, float *top_w, void *workspace, int64_t workspace_bytes, void *stream);

/* The same layer over prepared experts: gaje_hip_moe_prepare builds, once per
 * set of experts, the block-scaled product's weight operands (per expert and
 * product: the codes as f16 MFMA fragments, the fragment scales and the dense
 * block mins; about 3.3x the packed bytes) into a caller-owned, 256-byte
 * aligned device buffer of gaje_hip_moe_prepared_bytes; gaje_hip_moe_ffn_
 * prepared then runs the layer with one grouped block-scaled product per
 * projection (a row tile per ~64 dispatched rows, no dequantisation per
 * tile).  Routing, composition, accuracy and arguments as gaje_hip_moe_ffn;
 * no reference counterpart.  The prepared buffer depends only on the experts'
 * packed rows: prepare again after changing them. */
int64_t gaje_hip_moe_prepared_bytes(int64_t h, int64_t ffn, int64_t n_expert);
int gaje_hip_moe_prepare(const void *const *gate_up, const void *const *down, int64_t h, int64_t ffn,
                         int64_t n_expert, void *prepared, int64_t prepared_bytes, void *stream);
int64_t gaje_hip_moe_ffn_prepared_workspace(int64_t T, int64_t h, int64_t ffn, int64_t n_expert);
int gaje_hip_moe_ffn_prepared(const float *x, int64_t T, int64_t h, const float *router, int64_t n_expert,
                              const void *prepared, int64_t ffn, float *y, int32_t *top_idx, float *top_w,
                              void *workspace, int64_t workspace_bytes, void *stream);

/* Q8_0 rows (Q8_0Block {f16 scale; i8 qs[32]}, blocks.rs:36-49; the
 * --quant-embed format of token_embd / lm_head): packing into tiles of 8 rows
 * (per group of four blocks: the 8 rows' codes, 1 KiB, then their scales, 64
 * bytes; ceil(n/8) * ceil(k/128) * 1088 + 4 KiB of zero padding), the matvec
 * of GenomicLinear::forward_core on GenomicQ8_0 (linear/forward.rs:93-101) with
 * genomic_dot_product_q8_0_avx2's order (genomic.rs:377-448) and flush, and
 * dequantize_weight over file-layout blocks, all bit-exact. */
int64_t gaje_hip_q8_0_packed_bytes(int64_t n, int64_t k);
int gaje_hip_q8_0_pack(const void *blocks, void *packed, int64_t n, int64_t k, void *stream);
int gaje_hip_q8_0_gemv(const void *packed, const float *x, const float *bias, int64_t bias_len,
                       float *y, int64_t n, int64_t k, void *stream);
int gaje_hip_q8_0_dequant(const void *blocks, float *out, int64_t nblocks, void *stream);

/* LUT-4bit matvec (layout Genomic4Bit, high nibble = even element):
 * genomic_dot_product_4bit (genomic.rs:148-204) over the row slicing of
 * linear/forward.rs:59-83.  lut_len floats as stored in the file: 16 (one
 * table), k/32*16 (one per block column) or >= n*k/32*16 (per row and block),
 * i.e. the expansion of linear/init.rs:109-124. */
int gaje_hip_lut4_gemv(const uint8_t *codes, const float *lut, int64_t lut_len, const float *x,
                       const float *bias, int64_t bias_len, float *y, int64_t n, int64_t k,
                       void *stream);

/* 2-bit matvec (Genomic2Bit rows: per block of 32, 8 bytes of MSB-first 2-bit
 * codes): genomic_dot_product (genomic.rs:17-144, the AVX2 branch's order) over
 * the row slicing of linear/forward.rs:33-57, |sum| < 1e-5 flushed.  c_len
 * floats of centroids: 4 (one table), k/32*4 (one per block column) or more
 * (rows r < c_len/(k/32*4) own their tables, later rows read the table's
 * start), 0 (every row dot is 0).  modulation: 4 host floats multiplying
 * centroids 0..3 (forward_core's modulation_factors), or NULL for 1. */
int gaje_hip_2bit_gemv(const uint8_t *codes, const float *centroids, int64_t c_len, const float *modulation,
                       const float *x, const float *bias, int64_t bias_len, float *y, int64_t n, int64_t k,
                       void *stream);

/* FP32 matvec (lm_head, GenomicF32 rows): dot_product per row
 * (compute/kernels/dot.rs:23-94 via linear/forward.rs:20-32). */
int gaje_hip_f32_gemv(const float *w, const float *x, const float *bias, int64_t bias_len,
                      float *y, int64_t n, int64_t k, void *stream);

/* Bit-exact Q4_0Block::dequantize_weight (io/header/blocks.rs:18-30) of
 * nblocks whole blocks into out[nblocks*32]. */
int gaje_hip_q4_0_dequant(const void *blocks, float *out, int64_t nblocks, void *stream);

/* rms_norm (compute/kernels/norm.rs:17-131): y = (x * inv_rms) * w. */
int gaje_hip_rmsnorm(const float *x, const float *w, float eps, float *y, int64_t n, void *stream);

/* swiglu_balanced (compute/kernels/activation.rs:35-51). */
int gaje_hip_swiglu(const float *gate, const float *up, float *out, int64_t n, void *stream);

/* f32::exp as the reference calls it (attention.rs:106, activation.rs:42-44):
 * the host C library's expf, reproduced bit for bit on the device. */
int gaje_hip_expf(const float *x, float *y, int64_t n, void *stream);

/* The GQA softmax attention of GenomicAttention::forward_attention_core
 * (nn/attention.rs:87-127) over seq_len cached positions, bit-exact.  q is
 * [n_head][head_dim] (already rotated); k_cache and v_cache are both
 * [n_head_kv][head_dim][capacity] (positions 0..seq_len-1 used); out is
 * [n_head][head_dim]. */
int gaje_hip_attention(const float *q, const float *k_cache, const float *v_cache, int64_t seq_len,
                       int64_t capacity, int n_head, int n_head_kv, int head_dim, float *out, void *stream);

/* lateral_inhibition_kwta (compute/kernels/lut.rs:45-61), in place. */
int gaje_hip_kwta(float *scores, int64_t n, int64_t k, void *stream);

/* Greedy argmax with the reference's strict '>' (first maximum, NaN never
 * wins, all -inf/NaN -> 0): llm/forward.rs:262-271.  *idx is a device u32. */
int gaje_hip_argmax(const float *x, int64_t n, uint32_t *idx, void *stream);

/* --------------------------------------------------------- model API ------ */
typedef struct gaje_hip_model gaje_hip_model;

typedef struct {
    int64_t n_embd, n_head, n_head_kv, n_blocks, head_dim, ffn, vocab_size;
    float eps, rope_base;
    int32_t rope_split;          /* 1 = "split" rope_style, 0 = interleaved */
    int32_t arch_family;         /* header arch_family (0 = none)           */
    int32_t body_format;         /* 1 = Q4_0 blocks, 2 = LUT-4bit, 4 = 2-bit */
    int32_t use_genomic_norm;
    int64_t max_ctx;             /* KV capacity currently allocated          */
    int64_t weight_bytes;        /* bytes of weights resident in HBM         */
    int64_t n_logits;            /* lm_head out_features (length of logits)  */
} gaje_hip_model_info;

/* load_genomic_auto for a .gaje.flat file (io/flat_reader.rs:240-252 ->
 * GajeFlatFileReader::open/load_genomic :33-236): mmap, header, metadata and
 * directory, ArchitectureDescriptor-over-JSON precedence, one upload per tensor
 * into HBM (Q4_0 tensors packed as for gaje_hip_q4_0_pack, the rest as stored).
 * k_wta_ratio starts at 0.5 (:234). */
int gaje_hip_open(const char *flat_path, int device, gaje_hip_model **out);
void gaje_hip_close(gaje_hip_model *m);
int gaje_hip_model_info_get(const gaje_hip_model *m, gaje_hip_model_info *info);

/* GenomicLLM::forward_core (nn/llm/forward.rs:7-64): one token through every
 * block, output norm, lm_head and (0 < ratio < 1) K-WTA; logits_host[vocab]. */
int gaje_hip_forward(gaje_hip_model *m, uint32_t token, int clear_cache, float *logits_host);

/* GenomicLLM::forward_with_hidden_core (nn/llm/forward.rs:76-113): logits
 * without K-WTA plus the normalised hidden state h_norm_host[n_embd]. */
int gaje_hip_forward_hidden(gaje_hip_model *m, uint32_t token, int clear_cache, float *logits_host,
                            float *h_norm_host);

/* GenomicLLM::clear_cache_core (nn/llm/forward.rs:174-178). */
int gaje_hip_clear_cache(gaje_hip_model *m);

/* Number of cached positions (GenomicAttention::k_cache_len, attention.rs:134). */
int gaje_hip_cache_len(const gaje_hip_model *m, int64_t *len);

/* set_k_wta_ratio (nn/llm/python.rs:53-59): sets the LLM ratio and every
 * block's ratio. */
int gaje_hip_set_kwta(gaje_hip_model *m, float ratio);
int gaje_hip_get_kwta(const gaje_hip_model *m, float *ratio);

/* Reserve KV capacity for at least `positions` cached tokens (the reference's
 * cache is an unbounded Vec; this only pre-sizes the device buffers). */
int gaje_hip_reserve(gaje_hip_model *m, int64_t positions);

/* Token-by-token prefill (nn/llm/forward.rs:229-232): ids[0..n) through
 * forward_core in order; last_logits_host (may be NULL) gets the last
 * token's K-WTA-filtered logits. */
int gaje_hip_prefill(gaje_hip_model *m, const uint32_t *ids, int64_t n, float *last_logits_host);

/* Prompt prefill on the MFMA units: the same result as gaje_hip_prefill
 * (ids[0..n) appended to the cache, last_logits_host (may be NULL) = the last
 * token's K-WTA-filtered logits, the next greedy token kept on device) with
 * the n tokens processed in chunks of up to 1024 as matrix products.  Not
 * bit-exact: the body products carry fp32 accuracy in another summation order
 * (see gaje_hip_q4_0_gemm_mfma), attention sums in another order.  The
 * reference has no batched prefill (it loops forward_core, llm/forward.rs:229-232).
 * Needs Q4_0 body tensors without anchors and head_dim 64 or 128, else
 * GAJE_ERR_UNSUPPORTED.  On a NaN guard the cache length is left unchanged. */
int gaje_hip_prefill_mfma(gaje_hip_model *m, const uint32_t *ids, int64_t n, float *last_logits_host);

/* Batched decode: n_seq (1..16) independent sequences over one model's
 * weights, each with its own KV cache of `capacity` positions, as n_seq
 * GenomicLLM instances (llm/forward.rs:7-64) stepping together.  Every
 * sequence's logits are bit-identical to its own forward_core: the matvecs
 * read each weight row once per step and run every sequence's accumulation
 * chains in the reference order.  Needs Q4_0 body tensors and an f32 lm_head
 * (GAJE_ERR_UNSUPPORTED otherwise).  No reference function batches
 * sequences. */
typedef struct gaje_hip_batch gaje_hip_batch;
#define GAJE_BATCH_INACTIVE 0xFFFFFFFFu /* a fed id that skips its sequence for that step */
int gaje_hip_batch_open(gaje_hip_model *m, int64_t n_seq, int64_t capacity, gaje_hip_batch **out);
void gaje_hip_batch_close(gaje_hip_batch *b);
/* clear_cache_core of one sequence (seq = -1: all); also clears a NaN halt */
int gaje_hip_batch_reset(gaje_hip_batch *b, int64_t seq);
int gaje_hip_batch_cache_len(const gaje_hip_batch *b, int64_t seq, int64_t *len);
/* n steps with given ids (ids[s * n + i] for sequence s, step i; prompt
 * prefill): last_logits_host (NULL or [n_seq][n_logits]) gets the last step's
 * K-WTA-filtered logits; status (NULL or [n_seq]) gets 0, or 1 + the NaN
 * stage of a sequence a guard halted (the call then fails with its message). */
int gaje_hip_batch_feed(gaje_hip_batch *b, const uint32_t *ids, int64_t n, float *last_logits_host,
                        int32_t *status);
/* n greedy steps on device from first[s]: out_tokens[s * n + i] = argmax of
 * step i's logits (llm/forward.rs:262-271), fed back as step i+1's token. */
int gaje_hip_batch_decode_greedy(gaje_hip_batch *b, const uint32_t *first, int64_t n, uint32_t *out_tokens,
                                 int32_t *status);

/* One greedy step on device: forward(token) then argmax of the logits
 * (nn/llm/forward.rs:262-271); no logits cross PCIe. */
int gaje_hip_greedy_next(gaje_hip_model *m, uint32_t token, uint32_t *next);

/* Fixed-length greedy loop of benchmarks/performance/gaje_flat_benchmark.py:94-96:
 * out[0] = argmax(forward(first)), out[i] = argmax(forward(out[i-1])), all on
 * device (graph replays, no host round trip per token). */
int gaje_hip_decode_greedy(gaje_hip_model *m, uint32_t first_token, int64_t n, uint32_t *out_tokens);

/* generate_native_core (nn/llm/forward.rs:215-330): clear, prefill, then up to
 * max_new tokens with repetition penalty, greedy (temperature <= 1e-5) or
 * multinomial sampling (seeded here; upstream uses thread_rng), EOS stop and
 * the repetition-loop detector.  *n_out receives the number generated. */
int gaje_hip_generate(gaje_hip_model *m, const uint32_t *prompt, int64_t n_prompt, int64_t max_new,
                      float temperature, float repetition_penalty, const uint32_t *eos_ids,
                      int64_t n_eos, uint64_t seed, uint32_t *out_tokens, int64_t *n_out);

/* Per-stage device times of the last forward, if GAJE_HIP_PROFILE is set
 * (the reference's GAJE_PROFILE_VERBOSE timers, nn/llm/forward.rs:50-55). */
int gaje_hip_last_timing(const gaje_hip_model *m, float *blocks_ms, float *head_ms);

/* Benchmark helpers (no reference counterpart; the reference's benchmarks
 * time whole forward calls from Python, benchmarks/performance/bench_decode.py). */

/* Keep only the first `len` cached positions (len <= current length): lets a
 * benchmark replay the same decode from a fixed prompt state. */
int gaje_hip_truncate_cache(gaje_hip_model *m, int64_t len);

enum {
    GAJE_STAGE_QKV = 1,        /* rms_norm + fused QKV GEMV + RoPE + KV append */
    GAJE_STAGE_ATTENTION = 2,  /* split-K GQA decode attention                 */
    GAJE_STAGE_O = 3,          /* attn_output GEMV + residual                  */
    GAJE_STAGE_GATE_UP = 4,    /* rms_norm + ffn_gate_up GEMV + SwiGLU          */
    GAJE_STAGE_DOWN = 5,       /* ffn_down GEMV + residual                     */
    GAJE_STAGE_LM_HEAD = 6,    /* output rms_norm + f32 lm_head GEMV + argmax  */
    GAJE_STAGE_TOKEN = 7       /* one whole captured decode step               */
};
/* Average device time of `iters` back-to-back launches of one stage's kernel
 * with the model's own arguments (layer selects the block), measured with HIP
 * events on the model stream; *bytes gets the stage's algorithmic HBM bytes
 * (weights + activations in/out + KV read).  Overwrites the activations and
 * the cache slot of the next position, which the next forward rewrites. */
int gaje_hip_time_stage(gaje_hip_model *m, int stage, int64_t layer, int iters, float *avg_ms,
                        int64_t *bytes);

/* Average device time per launch of the operator matvec for `format`
 * (1 = Q4_0, 3 = Q4_0 in tolerance mode, 2 = LUT-4bit with per-row tables,
 * 0 = f32) over `copies` weight
 * copies laid out `copy_stride` bytes apart (copy i of the LUT tables at
 * lut_base + i * lut_stride), cycling through the copies so that the set can
 * exceed the caches.  The launches are captured once in a HIP graph and
 * replayed until `iters` launches ran, after about 640 untimed launches (the
 * core clock's climb under load); timed with HIP events on a private
 * stream.  With GAJE_HIP_PROFILE set in the environment the launches are
 * issued one by one instead (no graph), so that a kernel tracer records each;
 * the model's token step is likewise launched kernel by kernel then. */
int gaje_hip_bench_gemv(int format, const void *w_base, size_t copy_stride, const float *lut_base,
                        size_t lut_stride, int copies, const float *x, float *y, int64_t n, int64_t k,
                        int iters, float *avg_ms);

/* Average device time per launch of a floor probe, timed as
 * gaje_hip_bench_gemv times its launches: bytes == 0 launches an empty kernel
 * of grid x block threads (the launch boundary alone); bytes >= 256 a plain
 * read of the first `bytes` of the device buffer buf (16-byte loads, block <=
 * 256), whose first 256 bytes it may overwrite.  No reference counterpart:
 * the floors that a matvec launch of the same grid cannot go below. */
int gaje_hip_bench_floor(const void *buf, int64_t bytes, int grid, int block, int iters, float *avg_ms);

/* ------------------------------------------------- .gaje.flat reader --- */
/* Host-only entry points over the reader that gaje_hip_open uses, so a
 * file can be inspected (and the reader tested) without a GPU. */
typedef struct {
    uint32_t version, flags, num_tensors;
    uint32_t group_size, quant_format;
    uint32_t arch_family, arch_n_embd, arch_n_head, arch_n_head_kv, arch_n_blocks, arch_qk_permute;
    int32_t quant_type;             /* quantization_type(): 0 legacy centroids, 1 Q4_0, 2 Q8_0, 3 unknown */
    uint32_t effective_group_size;  /* effective_group_size(): group_size, or 16 when 0 */
    uint32_t pad_;
    uint64_t meta_len, dir_len, weights_offset, weights_len;
} gaje_flat_header;

/* FlatHeaderV2::from_bytes (io/header/flat.rs:46-59) with quantization_type
 * and effective_group_size (:63-79): GAJE_ERR_TOO_SHORT if len < 4096, then
 * GAJE_ERR_INVALID_MAGIC unless the bytes start with "GAJE". */
int gaje_flat_header_from_bytes(const uint8_t *bytes, size_t len, gaje_flat_header *out);

typedef struct {
    gaje_flat_header header;
    int64_t n_embd, n_head, n_head_kv, n_blocks;
    int64_t vocab_size;          /* metadata config.vocab_size, -1 if absent */
    float eps, rope_base;
    int32_t rope_split;          /* rope_style == "split" */
    int32_t use_genomic_norm;
    int32_t has_descriptor;      /* arch_family != 0: the header overrides the JSON */
    int32_t n_tensors;           /* entries in the tensor directory */
} gaje_flat_info;

/* GajeFlatFileReader::open (io/flat_reader.rs:33-69) and load_genomic's
 * config resolution, JSON then header descriptor (:124-139).  Errors as
 * gaje_hip_open reports them for a bad file. */
int gaje_flat_inspect(const char *path, gaje_flat_info *out);

typedef struct {
    uint64_t bit_depth, out_features, in_features;
    uint64_t dna_off, dna_len, c_off, c_len, anc_off, anc_len, bias_off, bias_len;
} gaje_flat_tensor;

/* The FlatTensorEntry named `name` (io/flat_reader.rs:9-22);
 * GAJE_ERR_NOT_FOUND if the directory has none. */
int gaje_flat_tensor_entry(const char *path, const char *name, gaje_flat_tensor *out);

/* ------------------------------------------- .gaje.flat writer (f32 in) --- */
/* The exporter's container and tensor routines (scripts/export_gaje_flat.py:
 * 184-483) over f32 weights, with the quantisers its GenomicLayer calls
 * (python/gaje/nn/stabilized.py:242-323).  Tensors are added in file order;
 * each becomes a directory entry and 64-byte-aligned dna / centroid / anchor
 * (/ bias) sub-blobs.  A writer handle is not re-entrant. */
typedef struct gaje_flat_writer gaje_flat_writer;
typedef struct {
    uint32_t flags;          /* 0x3 = fused qkv + gate_up (informational)        */
    uint32_t group_size;     /* 32                                               */
    uint32_t quant_format;   /* 0 legacy/LUT, 1 Q4_0, 2 Q8_0 (not read by loaders) */
    uint32_t arch_family, n_embd, n_head, n_head_kv, n_blocks, qk_permute;
} gaje_flat_writer_header;
int gaje_flat_writer_create(gaje_flat_writer **out);
void gaje_flat_writer_free(gaje_flat_writer *w);
/* A norm weight: bit_depth 32, in_features 1, centroid/anchor offsets 0. */
int gaje_flat_writer_add_norm(gaje_flat_writer *w, const char *name, const float *weights, int64_t n);
/* [out][in] row-major f32 weights as bit_depth 32 (token_embd / lm_head). */
int gaje_flat_writer_add_f32(gaje_flat_writer *w, const char *name, const float *weights, int64_t out_features,
                             int64_t in_features, const float *bias, int64_t bias_len);
/* quantize_q4_0_native (compute/quantize/python.rs:151-232) -> bit_depth 4, no centroids. */
int gaje_flat_writer_add_q4_0(gaje_flat_writer *w, const char *name, const float *weights, int64_t out_features,
                              int64_t in_features, const float *bias, int64_t bias_len);
/* quantize_q8_0_native (compute/quantize/python.rs:235-300) -> bit_depth 8 (--quant-embed). */
int gaje_flat_writer_add_q8_0(gaje_flat_writer *w, const char *name, const float *weights, int64_t out_features,
                              int64_t in_features, const float *bias, int64_t bias_len);
/* genomize_4bit_core (compute/quantize/genomize.rs:286-382) with block 32 ->
 * bit_depth 4 with per-(row, block) centroids and its anchor buffer. */
int gaje_flat_writer_add_lut4(gaje_flat_writer *w, const char *name, const float *weights, int64_t out_features,
                              int64_t in_features, float anchor_threshold, const float *bias, int64_t bias_len);
/* Header, metadata JSON (json.dumps of the exporter's metadata dict), directory and blobs. */
int gaje_flat_writer_write(gaje_flat_writer *w, const char *path, const char *metadata_json,
                           const gaje_flat_writer_header *header);

/* The quantisers alone.  n % 32 == 0; blocks_out holds n/32 * 20 (Q4_0) or
 * n/32 * 34 (Q8_0) bytes.  gaje_genomize_4bit: codes_out n/block_size *
 * block_size/2 bytes, centroids_out n/block_size * 16 floats, anchors_out (may
 * be NULL to query) *anchors_len bytes in, the buffer's size out. */
int gaje_quantize_q4_0(const float *weights, int64_t n, uint8_t *blocks_out);
int gaje_quantize_q8_0(const float *weights, int64_t n, uint8_t *blocks_out);
int gaje_genomize_4bit(const float *weights, int64_t n, int64_t block_size, float anchor_threshold,
                       uint8_t *codes_out, float *centroids_out, uint8_t *anchors_out, int64_t *anchors_len);

/* ----------------------------------------------- synthetic .flat writer --- */
/* Random-init model writer for the benchmark shapes (no checkpoints exist in
 * this environment).  Writes the .gaje.flat v2 layout of
 * scripts/export_gaje_flat.py:184-483 with a counter-based PRNG. */
typedef struct {
    int64_t n_embd, n_head, n_head_kv, n_blocks, ffn, vocab_size;
    float eps, rope_base;          /* rope_base goes to the metadata JSON        */
    int32_t arch_family;           /* header descriptor; 0 = JSON-only config    */
    int32_t qkv_bias;              /* 1 = write an N(0,0.02) bias for attn_qkv   */
    int32_t tied_embeddings;       /* 1 = lm_head rows equal token_embd rows     */
    int32_t body_format;           /* 1 = Q4_0 blocks, 2 = LUT-4bit per row/block, 4 = 2-bit per row/block */
    int32_t fused;                 /* 1 = attn_qkv / ffn_gate_up, 0 = split      */
    int32_t rope_interleaved;      /* metadata rope_style "interleaved" (else "split") */
    int32_t use_genomic_norm;      /* metadata config.use_genomic_norm           */
    int32_t quant_embed;           /* 1 = token_embd / lm_head as Q8_0 (bit_depth 8, --quant-embed), 2 = as 2-bit */
    int32_t g2_tables;             /* 2-bit centroid tables: 0 per (row, block), 1 per block column,
                                      2 one shared table, 3 the first half of the rows' tables + 6 floats */
    int32_t anchors;               /* sparse f16 anchors on every body tensor (GenomicLinear::new's
                                      "GAJE" buffer, init.rs:61-107): 0 none, 1 with n+1 row pointers
                                      (some column indices past in_features, one inverted row range),
                                      2 with genomize_4bit_core's two pointers, 3 with none */
    uint64_t seed;
} gaje_synth_config;

int gaje_synth_write_flat(const char *path, const gaje_synth_config *cfg);
/* Standalone tensors with the same recipe (row-major, k = in_features). */
int gaje_synth_q4_0(uint64_t seed, const char *name, int64_t n, int64_t k, uint8_t *blocks_out);
int gaje_synth_lut4(uint64_t seed, const char *name, int64_t n, int64_t k, uint8_t *codes_out,
                    float *lut_out);
int gaje_synth_2bit(uint64_t seed, const char *name, int64_t n, int64_t k, uint8_t *codes_out,
                    float *centroids_out);
int gaje_synth_normal(uint64_t seed, const char *name, int64_t count, float mean, float stddev,
                      float *out);

#ifdef __cplusplus
}
#endif
#endif /* GAJE_HIP_H */
