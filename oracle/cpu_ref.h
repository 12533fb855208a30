/*
 * cpu_ref — CPU restatement of the codon-infer ESM-2 bidirectional forward
 * and of its autoregressive (KV-cache) forward and generation loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle the HIP path is
 * checked against and the timed CPU baseline in bench.py.  Nothing in the
 * product (codon-infer_amd/) links, loads or calls it.
 *
 * Every function follows a reference routine in src/lib.rs of
 * OsbaldoG/codon-infer; each definition in cpu_ref.c cites file:line.
 */
#ifndef CODON_CPU_REF_H
#define CODON_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { CR_FP32 = 0, CR_Q8_0 = 1, CR_Q4_0 = 2 };

#define CR_Q8_BLOCK_BYTES 36 /* {f32 d; i8 qs[32]}  lib.rs:640-645 */
#define CR_Q4_BLOCK_BYTES 20 /* {f32 d; u8 qs[16]}  lib.rs:1043-1050 */

typedef struct cr_config {
    int32_t dim, hidden_dim, n_layers, n_heads, vocab_size;
} cr_config;

/* Weight tensors in the reference's in-memory layout (EsmWeights /
 * EsmWeightsQ8 / EsmWeightsQ4, lib.rs:299-307, 675-687, 1113-1125): every
 * tensor is tensor-major over layers; matrices are [out][in]; quantized
 * matrices are packed arrays of 36-byte (Q8_0) or 20-byte (Q4_0) blocks.
 * For Q8_0 models the token embedding is Q8_0, for Q4_0 models it is FP32. */
typedef struct cr_weights {
    int32_t dtype;
    const void *token_embedding_table;
    const float *ln_1_weight, *ln_1_bias;
    const void *wq; const float *bq;
    const void *wk; const float *bk;
    const void *wv; const float *bv;
    const void *wo; const float *bo;
    const float *ln_2_weight, *ln_2_bias;
    const void *fc1_weight; const float *fc1_bias;
    const void *fc2_weight; const float *fc2_bias;
    const float *ln_f_weight, *ln_f_bias;
    const float *classifier_weights; int64_t classifier_len;
} cr_weights;

/* Outputs of one forward_bidirectional_* call (BidirectionalRunState fields,
 * lib.rs:2488-2508).  NULL pointers are skipped. */
typedef struct cr_outputs {
    float *logits;       /* [S][V]                                        */
    float *hidden;       /* [S][d]   state.x after the final LayerNorm     */
    float *final_att;    /* [S][S]   head-mean of the last layer's P       */
    float *contacts;     /* [n][n]   n = S-2; non-NULL turns contacts on   */
    float *attn;         /* [L][H][S][S] every softmax row (export)        */
    float *layer_hidden; /* [L][S][d] x after each layer (on_layer hook)   */
    const float *contact_w; /* [L*H] regression weights, l-major          */
    float contact_b;
} cr_outputs;

/* formats */
void cr_quantize_q8(const float *src, int64_t n, uint8_t *dst);
void cr_dequantize_q8(const uint8_t *blocks, int64_t nblocks, float *dst);
void cr_quantize_q4(const float *src, int64_t n, uint8_t *dst);
void cr_dequantize_q4(const uint8_t *blocks, int64_t nblocks, float *dst);

/* tokenizer: returns the token count (text length + 2) or -1 if cap too small */
int32_t cr_tokenize(const char *text, int32_t *out, int32_t cap);

/* elementwise primitives */
void cr_layer_norm(float *out, const float *x, const float *w, const float *b, int32_t dim);
float cr_erf(float x);
void cr_gelu(float *out, const float *x, int64_t n);
void cr_softmax(float *x, int32_t n);
void cr_rope_tables(int32_t max_len, int32_t head_dim, float *cos_t, float *sin_t);
void cr_apply_rope(float *q, float *k, const float *cos_t, const float *sin_t,
                   int32_t pos, int32_t dim, int32_t n_heads);
void cr_log_softmax_canonical(const float *logits, float *out33);
void cr_dms_score(const float *logits33, int32_t wt_tok, float *deltas20, float *entropy);
void cr_accumulate_head_apc(const float *head_att, float *contact_logits,
                            int32_t seq_len, int32_t n_res, float w_lh);

/* out[p][i] = sum_k W[i][k] * x[p][k] + bias[i]  (matmul_tiled_*_parallel) */
void cr_matmul_tiled(int32_t wdtype, float *out, const float *x, const void *w,
                     const float *bias, int32_t in_dim, int32_t out_dim,
                     int32_t seq_len, int32_t num_threads);

/* one sequence, one forward.  Returns 0 or a negative error code. */
/* Attention micro-kernel choice: at head_dim 64 on an AVX-512F host the
 * reference uses its 512-bit dot/axpy (lib.rs:3398-3434), else the 256-bit
 * ones.  cr_set_attention_isa(1) forces the 256-bit path (0: as the host). */
void cr_set_attention_isa(int32_t avx_only);
int32_t cr_attention_uses_avx512(int32_t head_dim);

int32_t cr_forward(const cr_config *cfg, const cr_weights *w, const int32_t *tokens,
                   int32_t seq_len, int32_t num_threads, const cr_outputs *out);

/* ---- autoregressive path ---------------------------------------------- */

/* out[i] = sum_k W[i][k] * x[k] + bias[i]  (matmul_{,q8_,q4_}parallel) */
void cr_matmul_vec(int32_t wdtype, float *out, const float *x, const void *w, const float *bias,
                   int32_t in_dim, int32_t out_dim, int32_t num_threads);

/* RunState (lib.rs:2459-2486) */
typedef struct cr_run_state {
    int32_t max_len;
    float *key_cache, *value_cache; /* [L][max_len][d] */
    float *rope_cos, *rope_sin;     /* [max_len][hd/2] */
    float *logits;                  /* [V] */
} cr_run_state;
cr_run_state *cr_run_state_new(const cr_config *cfg, int32_t max_len);
void cr_run_state_free(cr_run_state *s);

/* forward_parallel / forward_q8 / forward_q4 (lib.rs:3558, 3741, 4016):
 * token at pos, K/V written to the cache at pos, logits in s->logits.
 * 0, -2 (token out of range) or -3 (pos out of range). */
int32_t cr_forward_step(const cr_config *cfg, const cr_weights *w, int32_t token, int32_t pos,
                        cr_run_state *s, int32_t num_threads);

/* SimpleRng and sample (lib.rs:3506-3530) */
uint64_t cr_rng_seed(uint64_t seed);
uint32_t cr_rng_next_u32(uint64_t *state);
float cr_rng_next_f32(uint64_t *state);
int32_t cr_sample(float *logits, int32_t vocab, float temperature, uint64_t *rng_state);

/* generate_sequence* (lib.rs:6551-6827) from prompt token ids; returns the
 * number of generated tokens or < 0 */
int32_t cr_generate(const cr_config *cfg, const cr_weights *w, const int32_t *prompt, int32_t n_prompt,
                    float temperature, int32_t max_new, uint64_t seed, int32_t max_seq_len,
                    int32_t num_threads, int32_t *out, int32_t out_cap);

/* metrics (lib.rs:2271-2377) */
float cr_cosine_similarity(const float *a, const float *b, int64_t n);
float cr_rmse(const float *a, const float *b, int64_t n);
float cr_top1_match_rate(const float *a, const float *b, int64_t n, int32_t vocab);
float cr_kl_divergence(const float *a, const float *b, int64_t n, int32_t vocab);

#ifdef __cplusplus
}
#endif
#endif
