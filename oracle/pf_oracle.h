/*
 * pf_oracle.h -- CPU restatement of PocketForge's MTP speculative-decoding hot
 * path, used ONLY as a checker: by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg.  Nothing in the product (pocketforge_amd/)
 * links, loads or calls it.
 *
 * Every function cites the reference file:line it restates.  Where the
 * reference sums floats in a sequential order that a GPU cannot reproduce
 * efficiently, this file fixes a canonical order (documented per function)
 * and the HIP kernels reproduce that order bit for bit.  Integer work
 * (activation codes, int8 dots, weight codes, KV row codes) is bit-exact
 * with the reference.
 */
#ifndef PF_ORACLE_H
#define PF_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- basics */
void     orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float    orc_uniform(uint64_t seed, uint64_t idx);
float    orc_expf(float x);
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* ------------------------------------- src/matmul_neon.cpp (reference order) */
void  orc_quantize_activation_row(const float* src, int8_t* dst, float* scale_out, uint32_t n);
void  orc_dequant_q4_to_int8(const uint8_t* q4, int8_t* out, float scale, uint32_t n);
void  orc_dequant_q2_to_int8(const uint8_t* q2, int8_t* out, float scale, uint32_t n);
void  orc_dequant_ternary_to_int8(const uint8_t* t, int8_t* out, uint32_t n);
void  orc_matmul_int8(const int8_t* A, const int8_t* B, int32_t* C,
                      uint32_t M, uint32_t N, uint32_t K);
void  orc_matmul_quantized(const float* A, const int8_t* B, float* C,
                           uint32_t M, uint32_t N, uint32_t K,
                           const float* w_scales, const float* act_scales);
float orc_dot_product(const float* a, const float* b, uint32_t n);
void  orc_softmax_ref(float* v, uint32_t n);                 /* libm exp, sequential sum */
void  orc_rmsnorm_ref(float* out, const float* x, const float* w, uint32_t n);

/* ---------------------------------------------- canonical reductions */
float orc_canon_sum(const float* x, uint32_t n, uint32_t waves);
float orc_canon_sumsq(const float* x, uint32_t n, uint32_t waves);
void  orc_softmax(float* v, uint32_t n);                     /* canonical, own exp */
float orc_dot_canon(const float* a, const float* b, uint32_t n);  /* CANON(4) of products */
void  orc_rmsnorm(float* out, const float* x, const float* w, uint32_t n);
void  orc_engine_rmsnorm(float* out, const float* x, const float* w, uint32_t n);

/* ------------------------------------------------- block-quant matrices */
enum { ORC_Q4 = 0, ORC_Q2 = 1, ORC_Q15 = 2, ORC_Q8 = 3 };

typedef struct {
    int32_t         fmt;     /* ORC_Q4 / ORC_Q2 / ORC_Q15 / ORC_Q8 */
    uint32_t        rows;    /* N: output features */
    uint32_t        cols;    /* K: input features, multiple of 32 */
    const uint8_t*  codes;   /* [rows][cols/32][16 (Q4) | 8 (Q2, Q1.5)] */
    const uint16_t* scales;  /* [rows][cols/32] fp16 block scale d */
} orc_qmat;

uint32_t orc_block_bytes(int32_t fmt);
void  orc_quantize_matrix(const float* w, uint32_t rows, uint32_t cols, int32_t fmt,
                          uint8_t* codes, uint16_t* scales);
int   orc_block_code(const orc_qmat* W, uint32_t row, uint32_t col);
void  orc_gemv_i8(const orc_qmat* W, const int8_t* a, float a_scale, float* y);
void  orc_gemv_f32(const orc_qmat* W, const float* h, float* y);
void  orc_dequant_row(const orc_qmat* W, uint32_t row, float* out);
void  orc_gemv_f32_dense(const float* E, uint32_t rows, uint32_t cols, const float* h, float* y);
/* MTPHeads::forward with n_heads chained heads ([n_heads][3] gate/up/down)
 * and an fp32 tied table [V][d] (NULL: placeholder logits). */
void  orc_mtp_heads_forward(const orc_qmat* heads, uint32_t n_heads, uint32_t d, uint32_t V,
                            const float* table, const float* hidden, float* logits);

/* --------------------------------------------- src/kv_cache.cpp (3-tier) */
typedef struct orc_kv orc_kv;
orc_kv*  orc_kv_create(uint32_t n_layers, uint32_t n_kv_heads, uint32_t head_dim,
                       uint32_t sink_size, uint32_t window_size, uint32_t pool_block,
                       uint32_t max_context);
void     orc_kv_destroy(orc_kv* kv);
void     orc_kv_store(orc_kv* kv, uint32_t layer, uint32_t head, uint32_t pos,
                      const float* key, const float* value);
uint32_t orc_kv_attention_scores(orc_kv* kv, uint32_t layer, uint32_t head,
                                 const float* q, float* scores_out);
void     orc_kv_attention_weighted_sum_ref(orc_kv* kv, uint32_t layer, uint32_t head,
                                           const float* scores, float* out, uint32_t count);
void     orc_kv_attention_weighted_sum(orc_kv* kv, uint32_t layer, uint32_t head,
                                       const float* scores, float* out, uint32_t count);
uint32_t orc_kv_size(const orc_kv* kv);
/* One head of the engine's attention over the cache's visible entries plus
 * the fp32 self entry (k_self, v_self): canonical chunked order, and the
 * reference's own order. */
void     orc_attn_head(orc_kv* kv, uint32_t layer, uint32_t head, const float* q, const float* k_self,
                       const float* v_self, float* out);
void     orc_attn_head_ref(orc_kv* kv, uint32_t layer, uint32_t head, const float* q, const float* k_self,
                           const float* v_self, float* out);
void     orc_kv_clear(orc_kv* kv);
uint32_t orc_kv_pool_count(const orc_kv* kv, uint32_t layer, uint32_t head);
/* Copies the visible rows of (layer, head) in attention order:
 * k/v [count][head_dim] int8 and their row scales.  Returns count. */
uint32_t orc_kv_export(const orc_kv* kv, uint32_t layer, uint32_t head,
                       int8_t* k, float* ks, int8_t* v, float* vs);
/* Sets (layer, head) to a state: sink, pooled and window rows (oldest
 * first, the oldest at position win_pos0), then n_pend evicted rows not yet
 * folded into a pooled row (eviction order). */
void     orc_kv_import(orc_kv* kv, uint32_t layer, uint32_t head, uint32_t n_sink, uint32_t n_pool,
                       uint32_t n_win, uint32_t win_pos0, uint32_t n_pend, const int8_t* k, const float* ks,
                       const int8_t* v, const float* vs);

/* ------------------------------------------------ model + engine */
typedef struct {
    uint32_t n_layers, n_embd, n_heads, head_dim, n_ff, n_vocab, n_mtp;
    uint32_t sink_size, window_size, pool_block, max_context;
    const orc_qmat* layers;        /* [n_layers][7]: Q K V O gate up down */
    const orc_qmat* emb;           /* tied [n_vocab][n_embd] (Q4) */
    const orc_qmat* mtp;           /* [n_mtp][3]: gate up down, each n_embd x n_embd */
    const float*    attn_norm;     /* [n_layers][n_embd] */
    const float*    ffn_norm;      /* [n_layers][n_embd] */
} orc_model_desc;

typedef struct {
    float    temperature;
    float    top_p;
    uint32_t top_k;
    int32_t  greedy;
} orc_sampling;

typedef struct orc_engine orc_engine;
orc_engine* orc_engine_create(const orc_model_desc* d);
void     orc_engine_destroy(orc_engine* e);
void     orc_engine_reset(orc_engine* e);
uint32_t orc_engine_pos(const orc_engine* e);
orc_kv*  orc_engine_kv(orc_engine* e);
void     orc_engine_set_state(orc_engine* e, uint32_t pos, const float* hidden);
void     orc_rope_table(uint32_t head_dim, uint32_t pos, float* cos_out, float* sin_out);
void     orc_rope_rotate(float* x, uint32_t head_dim, const float* cos_t, const float* sin_t);
void     orc_forward(orc_engine* e, int32_t token, float* logits, float* hidden);
/* LayerSkipController (src/layer_skip.cpp) in the forward pass: threshold
 * (0 = off, the default here; the reference's ModelConfig default is 0.01)
 * and anchor interval (default 4). */
void     orc_engine_set_layer_skip(orc_engine* e, float threshold, uint32_t interval);
uint32_t orc_engine_skip_count(const orc_engine* e);
float    orc_skip_delta(const float* a, const float* b, uint32_t n);
/* One should_skip_ffn decision on caller-held caches [L][D]: returns 1 to
 * skip layer l's FFN; updates cache l when the FFN runs. */
int      orc_skip_decide(float* caches, uint32_t L, uint32_t D, float threshold, uint32_t interval, uint32_t l,
                         const float* normed);
void     orc_mtp_forward(orc_engine* e, const float* hidden, float* logits);
int32_t  orc_argmax(const float* x, uint32_t n);
int32_t  orc_sample(const float* logits, uint32_t n_vocab, const orc_sampling* cfg,
                    uint64_t seed, uint64_t* draw_idx);
/* An abstract model for the decode control flow: forward one token
 * (logits may be NULL), whether a hidden state exists, and the MTP heads on
 * `hidden` (NULL: the last forward's hidden state) writing [n_mtp][V]. */
typedef struct {
    void*    ctx;
    uint32_t n_vocab, n_mtp;
    void     (*forward)(void* ctx, int32_t token, float* logits);
    int32_t  (*hidden_valid)(void* ctx);
    void     (*mtp)(void* ctx, const float* hidden, float* logits);
} orc_gen_ops;
int32_t  orc_generate_ops(const orc_gen_ops* ops, const int32_t* prompt, uint32_t n_prompt,
                          uint32_t max_new, const orc_sampling* cfg, uint64_t seed,
                          int32_t* tokens_out, uint32_t tokens_cap, uint32_t* n_tokens,
                          int32_t* mtp_accepted, int32_t* mtp_rejected);
int32_t  orc_step_mtp_ops(const orc_gen_ops* ops, int32_t current_token, const float* hidden, int32_t has_table,
                          const orc_sampling* cfg, uint64_t seed, uint64_t* draw, float* logits_out,
                          uint32_t* n_logits, int32_t* acc_out, int32_t* rej_out);
int32_t  orc_step_mtp(orc_engine* e, int32_t current_token, const float* hidden, int32_t has_table,
                      const orc_sampling* cfg, uint64_t seed, uint64_t* draw, float* logits_out,
                      uint32_t* n_logits, int32_t* acc_out, int32_t* rej_out);
/* Engine::generate's decode loop (src/engine.cpp:294-389) from the engine's
 * state with current token `cur`: tokens_out receives the generated tokens
 * only. */
int32_t  orc_generate_continue(orc_engine* e, int32_t cur, uint32_t max_new, const orc_sampling* cfg,
                               uint64_t seed, int32_t* tokens_out, uint32_t tokens_cap, uint32_t* n_tokens,
                               int32_t* mtp_accepted, int32_t* mtp_rejected);
int32_t  orc_generate(orc_engine* e, const int32_t* prompt, uint32_t n_prompt,
                      uint32_t max_new, const orc_sampling* cfg, uint64_t seed,
                      int32_t* tokens_out, uint32_t tokens_cap, uint32_t* n_tokens,
                      int32_t* mtp_accepted, int32_t* mtp_rejected);
int      orc_num_threads(void);
void     orc_set_num_threads(int n);
double   orc_last_decode_seconds(void);

#ifdef __cplusplus
}
#endif
#endif
