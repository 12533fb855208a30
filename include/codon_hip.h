/*
 * codon_hip.h — C ABI of the MI355X (gfx950) ESM-2 bidirectional encoder.
 *
 * A drop-in for the GPU side of codon-infer's forward_bidirectional* family.
 * Plain C types only: pointers, sizes, int status codes.  Every entry point
 * returns 0 (CIH_OK) or a negative cih_status; on failure
 * cih_last_error() (thread-local) describes the problem.  Nothing aborts or
 * throws across the ABI.
 *
 * Reference interfaces each entry replaces are cited as file:line into
 * OsbaldoG/codon-infer.
 */
#ifndef CODON_HIP_H
#define CODON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CIH_ABI_VERSION 1

/* ---- status codes --------------------------------------------------- */
enum cih_status {
    CIH_OK = 0,
    CIH_ERR_ARG = -1,        /* null pointer / invalid argument            */
    CIH_ERR_SHAPE = -2,      /* unsupported or inconsistent shape          */
    CIH_ERR_CAPACITY = -3,   /* batch/length above cih_model_reserve's     */
    CIH_ERR_CONTACTS = -4,   /* contacts requested with n_res > 1024       */
    CIH_ERR_HIP = -5,        /* HIP runtime error (no device, OOM, ...)    */
    CIH_ERR_IO = -6,         /* file open/read failure                     */
    CIH_ERR_FORMAT = -7,     /* bad magic/version/dtype/size in a file     */
    CIH_ERR_TOKEN = -8       /* token id outside [0, vocab)                */
};

/* ---- weight formats: the CODQ dtype ids (lib.rs:873-876) -------------- */
enum cih_dtype { CIH_DTYPE_FP32 = 0, CIH_DTYPE_Q8_0 = 1, CIH_DTYPE_Q4_0 = 2 };

#define CIH_Q8_0_BLOCK_BYTES 36 /* BlockQ8_0 {f32 d; i8 qs[32]}, lib.rs:640-645  */
#define CIH_Q4_0_BLOCK_BYTES 20 /* BlockQ4_0 {f32 d; u8 qs[16]}, lib.rs:1043-1050 */

/* EsmConfig (lib.rs:76-84).  head_dim = dim / n_heads must be one of
 * 16, 24, 32, 64; dim and hidden_dim must be multiples of 32. */
typedef struct cih_config {
    int32_t dim;
    int32_t hidden_dim;
    int32_t n_layers;
    int32_t n_heads;
    int32_t vocab_size;
    int32_t max_seq_len;
} cih_config;

/* Host tensors in EsmWeights / EsmWeightsQ8 / EsmWeightsQ4 field order
 * (lib.rs:299-307, 675-687, 1113-1125).  Layer tensors are stacked
 * tensor-major; matrices are [out][in].  Quantized matrices point at packed
 * 36-byte (Q8_0) / 20-byte (Q4_0) blocks.  token_embedding_table is Q8_0
 * blocks for Q8_0 models and FP32 otherwise.  classifier_weights is
 * [lm_ln_w, lm_ln_b, dense_w, dense_b, dec_w, dec_b] (lib.rs:5389-5396); a
 * shorter classifier selects the tied-embedding decoder (lib.rs:5427-5439).
 * The library copies everything to the device; the caller keeps ownership. */
typedef struct cih_host_weights {
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
    const float *classifier_weights;
    int64_t classifier_len;
} cih_host_weights;

typedef struct cih_model cih_model;

/* ---- forward flags ---------------------------------------------------- */
#define CIH_OUT_LOGITS       (1u << 0) /* logits       [B][S_max][V]               */
#define CIH_OUT_HIDDEN       (1u << 1) /* hidden       [B][S_max][d] (after LN_f)   */
#define CIH_OUT_FINAL_ATT    (1u << 2) /* final_att    [B][S_max][S_max]            */
#define CIH_OUT_CONTACTS     (1u << 3) /* contacts     [B][S_max-2][S_max-2]        */
#define CIH_OUT_ATTN         (1u << 4) /* attn         [B][L][H][S_max][S_max]      */
#define CIH_OUT_LAYER_HIDDEN (1u << 5) /* layer_hidden [B][L][S_max][d]             */
#define CIH_IO_DEVICE        (1u << 16) /* tokens + outputs are device pointers     */

/* Caller-owned output buffers, all row-major with the padded strides above.
 * Only rows/cols inside each sequence's true length are written; padding is
 * left untouched.  NULL entries are allowed when their flag is off. */
typedef struct cih_outputs {
    float *logits;
    float *hidden;
    float *final_att;
    float *contacts;
    float *attn;
    float *layer_hidden;
} cih_outputs;

/* ---- lifecycle ---------------------------------------------------------- */

/* Replaces EsmWeights/EsmWeightsQ8/EsmWeightsQ4 construction +
 * BidirectionalRunState ownership (lib.rs:310, 744, 1156, 2510).
 * contact_w: [n_layers*n_heads] regression weights (l-major) and contact_b
 * its bias, as returned by EsmConfig::contact_head_weights (lib.rs:154-177);
 * contact_w may be NULL when contacts are never requested.
 * Uses the current HIP device; creates one HIP stream per model.
 * Device memory: the weights in their own format, plus, for Q8_0 / Q4_0
 * models, the layer quants once more as f16 integers (2 bytes per weight:
 * the operand of the large-batch GEMM); CIH_GEMM_F16=0 leaves that copy out. */
int cih_model_create(const cih_config *cfg, int32_t dtype, const cih_host_weights *w,
                     const float *contact_w, float contact_b, cih_model **out);

/* Replaces load_model_weights (main.rs:137-244) + EsmConfig::detect_from_file
 * (lib.rs:277-296): reads a CODQ (FP32/Q8_0/Q4_0) or headerless
 * grouped_canonical_v1 / sequential_hf FP32 file.  quantize_to: -1 keeps the
 * file's dtype; CIH_DTYPE_Q8_0 / CIH_DTYPE_Q4_0 quantize an FP32 file in
 * memory (lib.rs:559-607).  Contact weights as in cih_model_create.
 * The file body goes to the GPU as is (parallel reads into pinned staging
 * buffers, asynchronous copies); the repack and any quantization run there.
 * CIH_LOAD_THREADS / CIH_LOAD_CHUNK_MB size the staging (default 2 x 8 MiB). */
int cih_model_create_from_file(const char *path, int32_t quantize_to, const float *contact_w,
                               float contact_b, cih_model **out);

/* Sizes the per-model device workspace (BidirectionalRunState::new max_len,
 * lib.rs:2510).  Output kinds not named in flags cannot be requested later
 * without another reserve.  cih_forward never allocates. */
int cih_model_reserve(cih_model *m, int32_t max_batch, int32_t max_seq_len, uint32_t flags);

int cih_model_config(const cih_model *m, cih_config *cfg, int32_t *dtype);
int cih_model_destroy(cih_model *m);

/* ---- the forward -------------------------------------------------------- */

/* Replaces forward_bidirectional / _parallel / _parallel_ext (lib.rs:5078,
 * 5087, 5097), forward_bidirectional_q8 (5442) and forward_bidirectional_q4 /
 * _q4_ext (5790, 5800) for a batch of B independent sequences.
 * tokens: [B][S_max] int32 ids (padding ignored), lens: [B] host array with
 * 1 <= lens[b] <= S_max.  B=1, lens[0]=S equals one reference call on
 * tokens[0..S].  Synchronous: outputs are complete on return.
 * Token ids outside [0, vocab) return CIH_ERR_TOKEN: checked on the host, or
 * with CIH_IO_DEVICE on the device during the forward (the outputs are then
 * undefined).
 * Range: the default kernels hand activations to the GEMMs and to attention
 * as two f16 limbs, which hold |x| < 65520 only.  A forward whose residual
 * stream turns non-finite, or whose final or LM-head LayerNorm writes a value
 * of 65520 or more in magnitude (the input of the LM head's limb GEMMs), is
 * run once more with the full-range kernels (three bf16 limbs, FP32-MFMA
 * attention and FP32-MFMA LM head, the whole FP32 exponent range), and those
 * results are returned.  Covered: an overflow inside a layer (it reaches the
 * residual stream) and at the LM head's inputs. */
int cih_forward(cih_model *m, const int32_t *tokens, const int32_t *lens, int32_t B,
                int32_t S_max, uint32_t flags, const cih_outputs *out);

/* ---- autoregressive decoding --------------------------------------------- */

typedef struct cih_decoder cih_decoder;

/* Replaces RunState::new (lib.rs:2464-2486) for n_slots independent
 * sequences: a K and a V cache of [n_layers][n_slots][max_len][dim] floats
 * on the device, RoPE tables for max_len positions, and row buffers for up
 * to max_rows rows per cih_decode call.  max_len <= 15000. */
int cih_decoder_create(cih_model *m, int32_t n_slots, int32_t max_len, int32_t max_rows,
                       cih_decoder **out);
int cih_decoder_destroy(cih_decoder *d);
/* Forgets a slot's cache contents (slot < 0: every slot). */
int cih_decoder_reset(cih_decoder *d, int32_t slot);

/* Replaces forward / forward_parallel / forward_q8 / forward_q4
 * (lib.rs:3554, 3558, 3741, 4016) for n rows at once: row i feeds
 * tokens[i] at position pos[i] of slot slots[i] (its K and V are written to
 * the cache there, then it attends to the slot's positions 0..pos[i]).
 * The rows of one slot must be consecutive positions starting at most at the
 * slot's first unwritten position (a prompt can prefill in one call;
 * rewriting earlier positions is allowed, as in the reference).  logits:
 * host [n][vocab] (may be NULL).  Synchronous. */
int cih_decode(cih_decoder *d, const int32_t *slots, const int32_t *tokens, const int32_t *pos,
               int32_t n, float *logits);

/* Replaces generate_sequence / _parallel / _q8 / _q4 (lib.rs:6538-6827) for
 * n independent streams.  Stream i uses slot slots[i] and the prompt ids
 * prompts[offsets[i] .. offsets[i+1]) (Tokenizer::encode of the prompt
 * without its trailing <eos>, as the reference feeds it), its own SimpleRng
 * seed seeds[i], a shared temperature (<= 0: greedy) and max_new_tokens
 * (< 0: none).  max_seq_len (<= 0: the decoder's max_len) caps positions as
 * config.max_seq_len does.  Each stream's prompt is prefilled in its own
 * calls; then all live streams decode together, one token each per step, each
 * stopping at <eos> (2) or its limit.  out_tokens: [n][out_cap] generated
 * ids; n_generated[i] their counts; prefill_ms / generation_ms (may be NULL)
 * the wall times of the two phases.  A stream's tokens do not depend on the
 * other streams while at most 8 streams decode together. */
int cih_generate(cih_decoder *d, int32_t n, const int32_t *slots, const int32_t *prompts,
                 const int32_t *offsets, float temperature, int32_t max_new_tokens,
                 const uint64_t *seeds, int32_t max_seq_len, int32_t *out_tokens, int32_t out_cap,
                 int32_t *n_generated, double *prefill_ms, double *generation_ms);

/* ---- in-silico deep mutational scan -------------------------------------- */

enum cih_dms_mode { CIH_DMS_MASKED_MARGINAL = 0, CIH_DMS_WILDTYPE_MARGINAL = 1 };

/* Replaces run_pipeline_dms_with_mode (pipeline.rs:76-280) for one protein.
 * residues: the n token ids between BOS and EOS (Tokenizer::encode of the
 * sequence without its first and last entries).  window / stride as the
 * reference (0 = the whole protein, capped at the model's max_seq_len).
 * Masked marginal: one forward per position with that position set to
 * <mask> (32), run as batches of `chunk` masked copies (0 or > reserved
 * max_batch = max_batch); wild-type marginal: one unmasked forward per
 * window.  Scoring (canonical log-softmax, entropy, deltas) runs on the GPU;
 * outputs are host arrays: deltas [n][20] in CANONICAL_AAS order
 * (A C D E F G H I K L M N P Q R S T V W Y, benchmark.rs:702-707; exactly 0
 * in the wild-type column) and entropy [n].  Needs a workspace reserved for
 * max_seq_len >= window + 2; allocates nothing. */
int cih_dms(cih_model *m, const int32_t *residues, int32_t n, int32_t window, int32_t stride, int32_t mode,
            int32_t chunk, float *deltas, float *entropy);

/* ---- kernel-level entry points (host pointers; each call stages through
 * freshly allocated device memory — for tests, not for the hot loop) ------ */

/* matmul_tiled_{fp32,q8,q4}_parallel (lib.rs:4803, 4870, 4937):
 * out[p][i] = sum_k W[i][k] x[p][k] + bias[i] for p < seq_len.
 * w: [out_dim][in_dim] FP32 or packed blocks of that matrix. */
int cih_matmul_tiled(int32_t dtype, float *out, const float *x, const void *w,
                     const float *bias, int32_t in_dim, int32_t out_dim, int32_t seq_len);

/* No counterpart in the reference: a variant of cih_matmul_tiled for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  out, x, w and bias are
 * DEVICE pointers (w 4-byte aligned, x 16-byte aligned; w in the same
 * reference layout as above); the call is enqueued on `stream` (a
 * hipStream_t; NULL = the null stream) and returns without waiting.  It
 * calls no allocator: the repacked weight matrix and the partial sums of a
 * k-split live in one fixed device array per GPU (48 MiB, held from the time
 * the library's code is loaded on that GPU until the process ends), so a
 * matrix whose repacked form exceeds 32 MiB returns CIH_ERR_CAPACITY (650M
 * FC1 in Q8_0 is 7.4 MB; a 3B FC1 in Q8_0 29.5 MB).  Every call on one GPU
 * uses the same array: calls that overlap on one GPU (other streams, other
 * threads) race; calls in order on one stream do not.  Results equal
 * cih_matmul_tiled's bit for bit. */
int cih_matmul_tiled_noalloc(int32_t dtype, float *out, const float *x, const void *w, const float *bias,
                             int32_t in_dim, int32_t out_dim, int32_t seq_len, void *stream);

/* Dequantizes nblocks blocks on the GPU with the decode routine the GEMMs
 * use (BlockQ8_0/BlockQ4_0::dequantize_to, lib.rs:663-667, 1074-1082). */
int cih_dequantize_device(int32_t dtype, const void *blocks, int64_t nblocks, float *out);

/* quantize_slice_to_q8 / quantize_slice_to_q4 (lib.rs:670-673, 1085-1088)
 * on the GPU, with the kernel that cih_model_create_from_file(quantize_to)
 * runs on FP32 weights; bit-identical to cih_quantize_q8 / cih_quantize_q4.
 * n must be a multiple of 32; dst holds n/32 blocks. */
int cih_quantize_device(int32_t dtype, const float *src, int64_t n, void *dst);

/* ---- host helpers (no GPU) ---------------------------------------------- */

/* quantize_slice_to_q8 / quantize_slice_to_q4 (lib.rs:670-673, 1085-1088);
 * n must be a multiple of 32; dst holds n/32 blocks. */
int cih_quantize_q8(const float *src, int64_t n, void *dst);
int cih_quantize_q4(const float *src, int64_t n, void *dst);
int cih_dequantize_q8(const void *blocks, int64_t nblocks, float *dst);
int cih_dequantize_q4(const void *blocks, int64_t nblocks, float *dst);

/* Tokenizer::encode (lib.rs:6511-6521).  Returns the token count (>= 2) or a
 * negative status if cap is too small. */
int cih_tokenize(const char *text, int32_t *out, int32_t cap);

/* log_softmax_canonical (lib.rs:4426-4441) over one row of 33 logits. */
int cih_log_softmax_canonical(const float *logits, float *out33);

/* ---- per-kernel timing (HIP events on the model's stream) ---------------- */
enum cih_kernel_class {
    CIH_KC_GEMM_QUANT = 0, /* Q8_0 / Q4_0 weight GEMMs                    */
    CIH_KC_GEMM_FP32 = 1,  /* FP32-weight GEMMs (FP32 models, LM head)    */
    CIH_KC_ATTENTION = 2,  /* attention                                   */
    CIH_KC_OTHER = 3,      /* embedding, LayerNorm, contacts, scatter     */
    CIH_KC_COUNT = 4
};

typedef struct cih_kernel_stats {
    int64_t launches;
    double total_ms;   /* summed launch durations (hipEventElapsedTime)   */
    double flops;      /* algorithmic FLOPs of those launches             */
    double bytes;      /* algorithmic HBM bytes (weights + activations)   */
} cih_kernel_stats;

/* enable != 0 resets the totals and starts recording (one event pair per
 * launch, summed after each cih_forward); enable == 0 stops recording and
 * keeps the totals for cih_profile_read. */
int cih_profile_enable(cih_model *m, int32_t enable);
int cih_profile_read(const cih_model *m, int32_t kernel_class, cih_kernel_stats *out);

const char *cih_last_error(void);
int cih_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif
