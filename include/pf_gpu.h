/*
 * pf_gpu.h -- C ABI of libpocketforge_amd.so, the MI355X (gfx950) drop-in
 * for PocketForge's MTP speculative-decoding hot path.
 *
 * Plain pointers and sizes only; no C++ or torch types cross this boundary.
 * Every call returns PF_OK (0) or a negative pf_status; pf_last_error()
 * gives the message (pf_last_error(NULL) for a failed pf_init).  Pointers named *_dev are device (HBM) pointers; all
 * other pointers are host pointers.  Work is issued on the context's own
 * HIP stream (default priority); calls that return host data synchronize
 * that stream.  A context is not re-entrant: one host thread per context,
 * as the reference's engine assumes (one Engine per process,
 * src/forge_server.cpp:11).
 *
 * Reference interfaces replaced (reference file:line):
 *   matmul kernels   include/forge/matmul_neon.hpp:20-92
 *   3-tier KV cache  include/forge/kv_cache.hpp:33-56
 *   MTP heads        include/forge/mtp.hpp:31-53
 *   engine           include/forge/engine.hpp:15-74
 *   types            include/forge/types.hpp:36-41, 220-268
 */
#ifndef PF_GPU_H
#define PF_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t pf_status;
#define PF_OK 0
#define PF_ERR_ARG -1          /* invalid argument or shape */
#define PF_ERR_HIP -2          /* HIP runtime error (message has the code) */
#define PF_ERR_RANGE -3        /* block scales outside the exact-sum range */
#define PF_ERR_UNSUPPORTED -4  /* shape outside what the kernels support */
#define PF_ERR_STATE -5        /* call out of order (e.g. model incomplete) */
#define PF_ERR_CAPACITY -6     /* position/token capacity exceeded */
#define PF_ERR_FORMAT -7       /* malformed or unsupported file contents */
#define PF_ERR_DEVICE -8       /* a bounded device-side wait timed out (results of that call are invalid) */

typedef struct pf_ctx pf_ctx;
typedef struct pf_model pf_model;
typedef struct pf_engine pf_engine;
typedef struct pf_kv pf_kv;
typedef struct pf_matrix pf_matrix;

/* Weight formats: 32-element blocks with an fp16 scale d.
 * Interchange layout (host): codes [rows][cols/32][16 (Q4) | 8 (Q2, Q1.5)
 * | 32 (Q8)] with the reference's element order (Q4: byte j = elements 2j
 * (low nibble) and 2j+1, code = nibble - 8; Q2: byte j = elements
 * 4j..4j+3 at bits 0,2,4,6, code = c - 2; Q1.5: same packing, code = c - 1
 * for c in {0,1,2}; Q8: byte j = element j, code = the signed byte, as
 * Q8_0 of include/forge/types.hpp:17-20), scales [rows][cols/32] as IEEE
 * binary16 bits. */
#define PF_FMT_Q4 0
#define PF_FMT_Q2 1
#define PF_FMT_Q15 2
#define PF_FMT_Q8 3

/* Matrix ids within a layer follow the .squeeze matrix ids of
 * src/quant_tool.cpp (0-6 = Q K V O gate up down). */
#define PF_MAT_Q 0
#define PF_MAT_K 1
#define PF_MAT_V 2
#define PF_MAT_O 3
#define PF_MAT_GATE 4
#define PF_MAT_UP 5
#define PF_MAT_DOWN 6

/* ------------------------------------------------------------ context */
pf_status pf_init(int device, pf_ctx** out);
void pf_destroy(pf_ctx* ctx);
const char* pf_last_error(const pf_ctx* ctx);
/* Device name and compute units, for reports. */
pf_status pf_device_info(pf_ctx* ctx, char* name, size_t name_len, int* compute_units);
pf_status pf_synchronize(pf_ctx* ctx);
/* Device bytes currently held by all objects of this context. */
size_t pf_device_bytes(const pf_ctx* ctx);
/* Device memory for the *_dev arguments (plumbing for callers without
 * their own allocator).  pf_memcpy kind: 0 host->device, 1 device->host,
 * 2 device->device; it synchronizes the context's stream. */
pf_status pf_malloc(pf_ctx* ctx, size_t bytes, void** out_dev);
pf_status pf_free(pf_ctx* ctx, void* dev, size_t bytes);
pf_status pf_memcpy(pf_ctx* ctx, void* dst, const void* src, size_t bytes, int32_t kind);

/* ------------------------------------- weights (host side, no GPU use) */
/* N(0, std^2) weights from Philox4x32-10 + Box-Muller (seed, stream), then
 * the reference's block code rules (src/quant_format.cpp:77-154, with a
 * multiplicative fp16 scale and Q1.5 threshold 0.35*amax). */
pf_status pf_gen_matrix(uint64_t seed, uint32_t stream, float stddev, uint32_t rows, uint32_t cols,
                        int32_t fmt, uint8_t* codes, uint16_t* scales);
/* Quantizes given float weights with the same code rules. */
pf_status pf_quantize_matrix(const float* w, uint32_t rows, uint32_t cols, int32_t fmt,
                             uint8_t* codes, uint16_t* scales);

/* ---------------------------- matmul_neon.hpp (device pointers, stream) */
/* quantize_activation_row (include/forge/matmul_neon.hpp:20-25) on M rows. */
pf_status pf_quantize_activation_rows(pf_ctx* ctx, const float* src_dev, int8_t* dst_dev,
                                      float* scales_dev, uint32_t M, uint32_t K);
/* matmul_int8 (include/forge/matmul_neon.hpp:55-62): C = A * B^T, int32. */
pf_status pf_matmul_int8(pf_ctx* ctx, const int8_t* A_dev, const int8_t* B_dev, int32_t* C_dev,
                         uint32_t M, uint32_t N, uint32_t K);
/* matmul_quantized (include/forge/matmul_neon.hpp:68-77): per-row fp32
 * weight scales; act_scales_dev may be NULL (computed per row). */
pf_status pf_matmul_quantized(pf_ctx* ctx, const float* A_dev, const int8_t* B_dev, float* C_dev,
                              uint32_t M, uint32_t N, uint32_t K, const float* w_scales_dev,
                              const float* act_scales_dev);

/* Block-quantized matrices resident in HBM. */
pf_status pf_matrix_upload(pf_ctx* ctx, int32_t fmt, uint32_t rows, uint32_t cols, const uint8_t* codes,
                           const uint16_t* scales, int32_t rowmajor, pf_matrix** out);
void pf_matrix_free(pf_matrix* m);
/* y[M][rows] = quantize_activation_row(x[m]) x W (tiled matrices), the
 * fused matmul_quantized path with per-block scales.  M <= 8 runs the GEMV,
 * 8 < M <= 512 the int8 MFMA GEMM; both give the same exact sums. */
pf_status pf_gemv_q(pf_ctx* ctx, const pf_matrix* W, const float* x_dev, float* y_dev, uint32_t M);
/* pf_gemv_q without allocating: the same kernels and results, with the
 * M > 8 path's int8 activation rows and scales in a fixed device array of
 * the library (1 MiB of activation codes plus 2 KB of scales per GPU, held
 * until the process ends) instead of memory the context allocates.  It has
 * no counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops).
 * Requires ceil(M / 32) * 32 * W's cols <= 1 MiB, else PF_ERR_CAPACITY.
 * All calls on one GPU share the array: calls that overlap on one GPU
 * (other streams or contexts) race. */
pf_status pf_gemv_q_noalloc(pf_ctx* ctx, const pf_matrix* W, const float* x_dev, float* y_dev, uint32_t M);
/* y[M][rows] = fp32 x[m] . dequantized W rows (row-major Q4 matrices). */
pf_status pf_gemv_f32(pf_ctx* ctx, const pf_matrix* W, const float* x_dev, float* y_dev, uint32_t M);

/* dot_product, softmax, rmsnorm (include/forge/matmul_neon.hpp:79-92) on
 * device buffers, in the canonical orders (CANON(4) sums); *out_dev is one
 * float.  MTPHeads::argmax (include/forge/mtp.hpp:49): first index of the
 * maximum of n floats, written to *out_dev. */
pf_status pf_dot_product(pf_ctx* ctx, const float* a_dev, const float* b_dev, uint32_t n, float* out_dev);
pf_status pf_softmax(pf_ctx* ctx, float* vals_dev, uint32_t n);
pf_status pf_rmsnorm(pf_ctx* ctx, float* out_dev, const float* x_dev, const float* w_dev, uint32_t n);
pf_status pf_argmax(pf_ctx* ctx, const float* x_dev, uint32_t n, int32_t* out_dev);

/* --------------------------------------------- mtp.hpp (standalone heads) */
/* MTPHeads (include/forge/mtp.hpp:31-53) outside an engine: n_heads chained
 * heads of n_embd x n_embd Q4 gate/up/down (n_embd a multiple of 256, up to
 * 2048), unembedded with an fp32 tied table [n_vocab][n_embd] given by the
 * caller (pf_mtp_set_table, host pointer, copied to HBM; NULL removes it).
 * Without a table, forward writes the reference's placeholder logits
 * (src/mtp.cpp:117-121).  hidden/logits are host pointers. */
typedef struct pf_mtp pf_mtp;
pf_status pf_mtp_create(pf_ctx* ctx, uint32_t n_heads, uint32_t n_embd, uint32_t n_vocab, pf_mtp** out);
void pf_mtp_destroy(pf_mtp* m);
pf_status pf_mtp_set_head(pf_mtp* m, uint32_t head, int32_t which, const uint8_t* codes, const uint16_t* scales);
pf_status pf_mtp_set_table(pf_mtp* m, const float* table);
pf_status pf_mtp_heads_forward(pf_mtp* m, const float* hidden, float* logits);
size_t pf_mtp_memory(const pf_mtp* m);

/* ----------------------------------------------- kv_cache.hpp (3-tier) */
typedef struct {
    uint32_t n_layers, n_kv_heads, head_dim;
    uint32_t sink_size, window_size, pool_block, max_context;
} pf_kv_config;   /* KVCacheConfig, include/forge/kv_cache.hpp:23-31 */

pf_status pf_kv_create(pf_ctx* ctx, const pf_kv_config* cfg, pf_kv** out);
void pf_kv_destroy(pf_kv* kv);
/* KVCache::store (include/forge/kv_cache.hpp:37-38); key/value are host
 * pointers of head_dim floats. */
pf_status pf_kv_store(pf_kv* kv, uint32_t layer, uint32_t head, uint32_t pos, const float* key,
                      const float* value);
/* KVCache::attention_scores (kv_cache.hpp:41-45): writes *count scores. */
pf_status pf_kv_attention_scores(pf_kv* kv, uint32_t layer, uint32_t head, const float* query,
                                 float* scores_out, uint32_t* count);
/* KVCache::attention_weighted_sum (kv_cache.hpp:47-52), 64-entry chunks. */
pf_status pf_kv_attention_weighted_sum(pf_kv* kv, uint32_t layer, uint32_t head, const float* scores,
                                       float* output, uint32_t count);
uint32_t pf_kv_size(const pf_kv* kv);
pf_status pf_kv_clear(pf_kv* kv);
size_t pf_kv_memory_usage(const pf_kv* kv);

/* --------------------------------------------------------------- model */
typedef struct {
    uint32_t n_layers, n_embd, n_heads, head_dim, n_ff, n_vocab, n_mtp;
} pf_model_desc;  /* ModelConfig subset, include/forge/types.hpp:220-254 (MHA) */

/* n_vocab <= 16384 (the on-chip sampler's limit): larger vocabularies,
 * such as ModelConfig's default 130560, return PF_ERR_UNSUPPORTED. */
pf_status pf_model_create(pf_ctx* ctx, const pf_model_desc* desc, pf_model** out);
void pf_model_destroy(pf_model* m);
/* Layer matrix `id` (PF_MAT_*), interchange layout.  Q/K/V must share a
 * format, as must gate/up. */
pf_status pf_model_set_matrix(pf_model* m, uint32_t layer, int32_t id, int32_t fmt, const uint8_t* codes,
                              const uint16_t* scales);
/* Tied embedding / unembedding table [n_vocab][n_embd], Q4. */
pf_status pf_model_set_embedding(pf_model* m, const uint8_t* codes, const uint16_t* scales);
/* The same in format fmt: PF_FMT_Q4 or PF_FMT_Q8 (the .squeeze default,
 * src/quant_tool.cpp:193-194). */
pf_status pf_model_set_embedding_fmt(pf_model* m, int32_t fmt, const uint8_t* codes, const uint16_t* scales);
/* MTP head k matrix which (0 gate, 1 up, 2 down), n_embd x n_embd Q4. */
pf_status pf_model_set_mtp(pf_model* m, uint32_t head, int32_t which, const uint8_t* codes,
                           const uint16_t* scales);
/* RMSNorm weights: which 7 = attention, 8 = FFN (default 1.0). */
pf_status pf_model_set_norm(pf_model* m, uint32_t layer, int32_t which, const float* w);

/* ------------------------------------------------------ .squeeze files */
/* WeightLoader (include/forge/quant_format.hpp:92-140, src/quant_format.cpp:
 * 227-444) on the host: the file is mapped, matrices are zstd-decompressed
 * (the system's libzstd.so.1) with their block scales parsed, and
 * pf_squeeze_load_model uploads a whole model in the device layout. */
typedef struct pf_squeeze pf_squeeze;
typedef struct {
    uint32_t version, n_blocks;
    uint32_t n_layers, n_embd, n_heads, n_kv_heads, n_ff, n_vocab, max_seq_len, mtp_heads;
} pf_squeeze_info;   /* SqueezeHeader, include/forge/quant_format.hpp:30-46 */

/* WeightLoader::open: mapped, magic and index checked. */
pf_status pf_squeeze_open(const char* path, pf_squeeze** out);
void pf_squeeze_close(pf_squeeze* s);
/* Message of the last failed call on s (or of the last failed open). */
const char* pf_squeeze_last_error(const pf_squeeze* s);
/* WeightLoader::config. */
pf_status pf_squeeze_get_info(const pf_squeeze* s, pf_squeeze_info* out);
/* Shape and quant type (0 Q8, 1 Q4, 2 Q2, 3 Q1.5) of matrix `matrix` of
 * layer `layer` (WeightBlock, include/forge/types.hpp:205-214). */
pf_status pf_squeeze_block_shape(const pf_squeeze* s, uint32_t layer, uint32_t matrix, uint32_t* rows,
                                 uint32_t* cols, uint32_t* quant_type);
/* WeightLoader::load_block_with_scales with the block scales parsed:
 * codes [rows * cols] (signed), block_scales [ceil(rows * cols / 32)], the
 * multiplier of each 32-element block of the flattened matrix (1 / the
 * stored inverse scale; 1 for Q1.5). */
pf_status pf_squeeze_load_block(pf_squeeze* s, uint32_t layer, uint32_t matrix, int8_t* codes,
                                float* block_scales);
/* Engine::load_model + load_layer_weights (src/engine.cpp:48-201, 606-640):
 * layer matrices 0-6 (Q4 / Q2 / Q1.5, repacked with the fp16 scale
 * 1 / inverse scale), norms 7-8, the Q4 tied embedding (layer 0, matrix 10),
 * all resident.  MTP heads are not stored in the format: set them with
 * pf_model_set_mtp. */
pf_status pf_squeeze_load_model(pf_ctx* ctx, pf_squeeze* s, pf_model** out);

/* -------------------------------------------------------------- engine */
typedef struct {
    float temperature;
    float top_p;
    uint32_t top_k;
    int32_t greedy;
} pf_sampling;  /* SamplingConfig, include/forge/types.hpp:36-41 */

typedef struct {
    uint32_t n_tokens;        /* tokens written (prompt included) */
    int32_t mtp_accepted;
    int32_t mtp_rejected;
    int32_t oom_protected;
    uint32_t rounds;          /* MTP rounds */
    uint32_t passes;          /* forward passes issued (prefill excluded) */
    uint32_t continued;       /* rounds whose one-row first verify segment was continued by a second one */
    double prefill_seconds;
    double decode_seconds;
} pf_gen_result;  /* GenerationResult, include/forge/types.hpp:260-268 */

typedef struct {
    uint32_t sink_size, window_size, pool_block, max_context;
} pf_cache_desc;

pf_status pf_engine_create(pf_model* m, const pf_cache_desc* cache, pf_engine** out);
void pf_engine_destroy(pf_engine* e);
/* Clears the cache and the position counter. */
pf_status pf_engine_reset(pf_engine* e);
uint32_t pf_engine_position(const pf_engine* e);
/* (new) State snapshot of one KV plane, for parity checks from a state and
 * checkpoints; the reference keeps this state inside KVCache
 * (src/kv_cache.cpp:59-127) with no export.  Writes the plane of (sequence
 * seq, layer, head) at the sequence's position: counts[0] sink rows,
 * counts[1] pooled rows, counts[2] window rows oldest first (KVCache's
 * attention order, src/kv_cache.cpp:137-155), then counts[3] evicted window
 * rows, in eviction order, that the next pooled row will fold (the
 * reference's running double sum, src/kv_cache.cpp:77-109).  k, v
 * [cap][head_dim] int8 codes, ks, vs [cap] row scales. */
pf_status pf_engine_kv_export(pf_engine* e, uint32_t seq, uint32_t layer, uint32_t head, int8_t* k, float* ks,
                              int8_t* v, float* vs, uint32_t cap, uint32_t* counts);
/* Engine::forward_with_hidden (engine.hpp:38-41) for n <= 8 consecutive
 * tokens in one pass; row j equals the j-th of n sequential forwards.
 * logits [n][n_vocab] and hidden [n][n_embd] may be NULL. */
pf_status pf_forward(pf_engine* e, const int32_t* tokens, uint32_t n, float* logits, float* hidden);
/* MTPHeads::forward (mtp.hpp:40-43) with the tied table: logits
 * [n_mtp][n_vocab] from a pre-norm hidden state. */
pf_status pf_mtp_forward(pf_engine* e, const float* hidden, float* logits);
/* Engine::step_mtp (src/engine.cpp:402-448) with the heads present, on the
 * device: MTPHeads::forward from `hidden` (pre-norm, [n_embd]), one sample per
 * head (cfg, seed, draws from *draw_index, advanced like pf_sample's), one
 * pass over [current_token, d0 .. d{n-2}] at the engine's next positions,
 * and the greedy check of row k against draft k up to the first mismatch.
 * The engine's position advances by the rows the reference forwards
 * (accepted + 1 on a rejection, n_mtp otherwise).  *accepted_out is the
 * count; on a rejection *acc_out = 0, *rej_out = n_mtp - accepted and
 * logits_out [n_vocab] (may be NULL) receives the rejecting row's logits
 * with *has_logits = 1; when every draft is accepted *acc_out = accepted,
 * *rej_out = 0 and *has_logits = 0.  PF_ERR_STATE without heads. */
pf_status pf_step_mtp(pf_engine* e, int32_t current_token, const float* hidden, const pf_sampling* cfg,
                      uint64_t seed, uint64_t* draw_index, int32_t* accepted_out, int32_t* acc_out,
                      int32_t* rej_out, float* logits_out, int32_t* has_logits);
/* Engine::sample (engine.hpp:54-60) on a host logits row; *draw_index is
 * the stochastic draw counter (incremented when a uniform is used). */
pf_status pf_sample(pf_engine* e, const float* logits, const pf_sampling* cfg, uint64_t seed,
                    uint64_t* draw_index, int32_t* token);
/* Engine::generate (engine.hpp:27-32) with the sampling configuration
 * passed explicitly.  tokens_out receives prompt + generated tokens. */
pf_status pf_generate(pf_engine* e, const int32_t* prompt, uint32_t n_prompt, uint32_t max_new_tokens,
                      const pf_sampling* cfg, uint64_t seed, int32_t* tokens_out, uint32_t tokens_cap,
                      pf_gen_result* result);
/* Engine::set_mtp_enabled (engine.hpp:23): with 0, generate runs the
 * single-token loop only (src/engine.cpp:304, 367-386). */
pf_status pf_engine_set_mtp_enabled(pf_engine* e, int32_t enabled);
/* (new) How pf_generate verifies a round's drafts; tokens are the same
 * either way.  The reference forwards the verify rows one at a time and
 * stops at the first mismatch (src/engine.cpp:332-365).  By default (0) a
 * round that follows a round with no accepted draft verifies its first
 * draft with a one-row pass and, if that draft is accepted, the rest in a
 * second pass; other rounds verify every draft in one (n_mtp + 1)-row pass.
 * With 1, every round uses the one (n_mtp + 1)-row pass. */
pf_status pf_engine_set_verify_full(pf_engine* e, int32_t full);
/* Engine::set_max_memory (engine.hpp:25): generate stops with
 * oom_protected when the context's device bytes exceed this (0 = off). */
pf_status pf_engine_set_max_memory(pf_engine* e, size_t bytes);
/* Engine::set_layer_skip_threshold (engine.hpp:24, src/engine.cpp:266-269)
 * plus the controller's anchor interval (ModelConfig::skip_interval,
 * types.hpp): LayerSkipController (src/layer_skip.cpp:22-67) on the FFN
 * input of every layer of every pass.  On while threshold > 0 (default off;
 * the reference's ModelConfig default is 0.01); switching it on starts from
 * zeroed caches.  While it is on, every MTP round verifies all drafts in
 * one (n_mtp + 1)-row pass. */
pf_status pf_engine_set_layer_skip(pf_engine* e, float threshold, uint32_t interval);
/* FFN blocks skipped since creation or pf_engine_reset (the reference's
 * GenerationResult::layers_skipped reads a counter that is never
 * incremented, src/engine.cpp:393). */
pf_status pf_engine_layer_skip_count(pf_engine* e, uint64_t* count);

/* HIP events around every decode segment of pf_generate (on: 1), which
 * pf_engine_round_time reports; off by default, since recording them costs
 * about 10 us of wall time per round.  No counterpart in the reference:
 * instrumentation for benchmarks and profilers. */
pf_status pf_engine_set_round_timing(pf_engine* e, int32_t on);
/* Average device time (us, HIP events on the engine's stream) of the MTP
 * rounds of the last pf_generate run with round timing on: base pass +
 * draft + verify + accept (0 with it off; rounds counts the rounds either
 * way). */
pf_status pf_engine_round_time(const pf_engine* e, double* round_us, uint32_t* rounds);
/* Average device time in microseconds of the verify passes (every verify
 * segment) and base passes of the last pf_generate run without captured
 * graphs (profiling modes 1 and 2), measured with HIP events around each
 * pass on the engine's stream.  Mode 2 adds no events inside a pass, so
 * its pass times are the undisturbed ones. */
pf_status pf_engine_pass_times(const pf_engine* e, double* verify_us, double* base_us,
                               uint32_t* verify_n, uint32_t* base_n);

/* Profiling mode.  0: off (captured graphs).  1: pf_generate issues its
 * kernels one by one (no captured graphs) and every int8 GEMV and attention
 * dispatch of the verify passes carries HIP start/stop events.  2: kernels
 * one by one with events around each pass only.  Other values:
 * PF_ERR_ARG. */
pf_status pf_engine_profile(pf_engine* e, int32_t enable);
/* Launch count, average duration (us) and average algorithmic bytes
 * (packed weights + int8 activations + fp32 outputs) of the GEMV launches
 * recorded by the last pf_generate in profiling mode. */
pf_status pf_engine_gemv_stats(pf_engine* e, uint32_t* launches, double* avg_us, double* avg_bytes);
/* The same launches grouped by algorithmic bytes, one group per matrix shape
 * (ascending bytes): up to `cap` groups are written, *n receives the number
 * of groups.  Profiling aid; no reference counterpart. */
pf_status pf_engine_gemv_by_size(const pf_engine* e, uint32_t cap, double* bytes, uint32_t* launches,
                                 double* avg_us, uint32_t* n);
/* Launch count and average duration (us) of the attention kernel of the
 * verify passes recorded by the last pf_generate / pf_batch_generate in
 * profiling mode (one launch per layer and pass). */
pf_status pf_engine_attn_stats(const pf_engine* e, uint32_t* launches, double* avg_us);

/* ------------------------------------------------- multi-sequence engine
 * No counterpart in the reference, which decodes one sequence per Engine
 * (include/forge/engine.hpp:20-74).  An engine of n_seq independent
 * sequences (n_seq * (n_mtp + 1) <= 512) over one model: each sequence owns
 * its 3-tier KV cache, position, decode state, seed and draw counter, and
 * produces exactly the tokens of a single-sequence engine given the same
 * prompt and seed (Engine::generate, src/engine.cpp:276-396, per
 * sequence).  Passes are batched across sequences: a round runs one base
 * pass of n_seq rows and one verify pass of n_seq * (n_mtp + 1) rows.
 * pf_engine_destroy, pf_engine_reset, pf_engine_profile and the timing
 * queries apply; pf_forward and pf_generate need n_seq == 1. */
pf_status pf_batch_create(pf_model* m, const pf_cache_desc* cache, uint32_t n_seq, pf_engine** out);
uint32_t pf_batch_sequences(const pf_engine* e);
/* Next position of sequence `seq` (tokens it has forwarded). */
uint32_t pf_batch_position(const pf_engine* e, uint32_t seq);
/* Forwards n prompt tokens of one sequence at its next positions. */
pf_status pf_batch_prefill(pf_engine* e, uint32_t seq, const int32_t* tokens, uint32_t n);
/* One batched pass: sequence seqs[i] (distinct) forwards tokens
 * [i * rows_per_seq, (i + 1) * rows_per_seq) at its next positions; row r
 * of logits [n * rows_per_seq][n_vocab] and hidden [..][n_embd] (either
 * may be NULL) equals the matching row of pf_forward on that sequence.
 * With outputs, n * rows_per_seq <= max(8, n_seq * (n_mtp + 1)). */
pf_status pf_batch_forward(pf_engine* e, const uint32_t* seqs, uint32_t n, uint32_t rows_per_seq,
                           const int32_t* tokens, float* logits, float* hidden);
/* Engine::generate for every sequence: prompts concatenated (prompt_lens
 * [n_seq]), seeds [n_seq], tokens_out [n_seq][tokens_cap] (prompt
 * included), results [n_seq]. */
pf_status pf_batch_generate(pf_engine* e, const int32_t* prompts, const uint32_t* prompt_lens,
                            uint32_t max_new_tokens, const pf_sampling* cfg, const uint64_t* seeds,
                            int32_t* tokens_out, uint32_t tokens_cap, pf_gen_result* results);
/* (new) Continuous batching: requests join and leave between rounds.  The
 * reference serves each request with its own Engine::generate call
 * (src/forge_server.cpp:280, 398); here every admitted sequence's tokens
 * and counters equal that call's for its prompt and seed (src/engine.cpp:
 * 276-396), whatever else runs beside it.  pf_batch_open starts a session
 * (every slot free; cfg for every request, tokens_cap per slot; it replaces
 * the token buffers of an earlier pf_batch_generate); pf_batch_admit
 * prefills a prompt (n_prompt >= 1) into a free slot from an empty cache,
 * with its own budget and seed; pf_batch_step runs one round (base pass,
 * drafts, one verify pass, acceptance and corrective, batched over the
 * generating slots) and lists in finished[] (n_seq entries, may be NULL)
 * the slots that reached their budget; pf_batch_take copies a slot's
 * tokens (prompt included) and counters and frees it (a slot still
 * generating leaves the batch).  Layer skip must be off. */
pf_status pf_batch_open(pf_engine* e, const pf_sampling* cfg, uint32_t tokens_cap);
pf_status pf_batch_admit(pf_engine* e, uint32_t seq, const int32_t* prompt, uint32_t n_prompt,
                         uint32_t max_new_tokens, uint64_t seed);
pf_status pf_batch_step(pf_engine* e, uint32_t* finished, uint32_t* n_finished);
pf_status pf_batch_take(pf_engine* e, uint32_t seq, int32_t* tokens_out, uint32_t tokens_cap,
                        pf_gen_result* result);

#ifdef __cplusplus
}
#endif
#endif
