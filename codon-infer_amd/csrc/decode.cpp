// Autoregressive decoding on the device-resident model: RunState with its
// KV cache (src/lib.rs:2459-2486), forward / forward_q8 / forward_q4 for a
// batch of rows (3554-4233), SimpleRng + sample (3506-3530) and the
// generate_sequence* loop (6538-6827).
//
// A decoder owns n_slots independent KV caches.  One decode call runs any
// number of rows, each (slot, token, position): the weights are read once
// for all rows (the GEMV for up to 8 rows, the MFMA GEMM above), so
// independent sequences decode together and a prompt prefills in one call.
#include <chrono>
#include <cmath>
#include <cstring>
#include <map>
#include <tuple>

#include "model.h"

struct cih_decoder {
    cih_model *m = nullptr;
    int slots = 0, max_len = 0, max_rows = 0;
    int64_t slot_stride = 0;  // floats between slots in one layer's cache
    float *kc = nullptr, *vc = nullptr;  // [L][slots][max_len][d]
    float *rope_c = nullptr, *rope_s = nullptr;
    float *x = nullptr, *xb = nullptr, *qkv = nullptr, *ao = nullptr, *h = nullptr, *logits = nullptr;
    int *d_tokens = nullptr, *d_rows = nullptr, *d_cu = nullptr, *d_lens = nullptr;
    int *h_meta = nullptr;  // pinned: tokens[max_rows] | rows[max_rows][2] | status word read back
    float *h_logits = nullptr;  // pinned: [max_rows][V] logits read back (then copied to pageable buffers)
    int *d_flag = nullptr;  // device status word of a step (FLAG_* bits)
    cih::PartialBuf part;
    std::vector<int> filled;  // positions written per slot (0..filled-1 valid)
    bool unique = false;      // staged rows: every slot at most once
    // (rows, fused, kernel switches) -> captured step
    std::map<std::tuple<int, bool, std::string>, hipGraphExec_t> graphs;
    std::vector<void *> allocs;
};

using namespace cih;

namespace {

void destroy(cih_decoder *dc) {
    if (!dc) return;
    if (dc->m && dc->m->stream) hipStreamSynchronize(dc->m->stream);
    for (auto &g : dc->graphs) hipGraphExecDestroy(g.second);
    free_list(dc->allocs);
    if (dc->h_meta) hipHostFree(dc->h_meta);
    if (dc->h_logits) hipHostFree(dc->h_logits);
    delete dc;
}

// A step of at most GEMV_MAX_M rows of a quantized model runs its layer
// projections on the f16-MFMA GEMV, with the activations handed over as f16
// limbs and the split-K partial sums added by the next kernel (the fused
// attention: QKV's; the residual LayerNorm: Wo's and FC2's; FC2: FC1's).
bool step_gemv16(const cih_decoder *dc, int n) {
    const cih_model *m = dc->m;
    if (n > GEMV_MAX_M || full_range_mode() || m->layers.empty() || m->cfg.dim % 32 || m->cfg.hidden_dim % 32)
        return false;
    const Layer &ly = m->layers[0];
    return gemv16_applies(ly.wqkv, AF_H2, n, EPI_NONE) && gemv16_applies(ly.wo, AF_H2, n, EPI_NONE) &&
           gemv16_applies(ly.w1, AF_H2, n, EPI_NONE) && gemv16_applies(ly.w2, AF_H2, n, EPI_NONE);
}

// Steps whose activations travel as f16 limbs (|x| < 65504) report a residual
// that is no longer finite, and run again in full range.
bool step_limbs(const cih_decoder *dc, int n) { return n > GEMV_MAX_M ? !full_range_mode() : step_gemv16(dc, n); }

// The rows' forward from the staged device tokens / rows: embedding
// (constant 0.88 scale, <mask> -> 0), the layers with cached causal
// attention, final LN and LM head -> dc->logits.  Kernel launches only, so
// that a step can be captured into a graph.
int enqueue_rows(cih_decoder *dc, int n, bool fused) {
    cih_model *m = dc->m;
    const int d = m->cfg.dim, F = m->cfg.hidden_dim, V = m->cfg.vocab_size, H = m->cfg.n_heads, L = m->cfg.n_layers;
    hipStream_t st = m->stream;
    // forward_* embedding (lib.rs:3567-3575, 3753-3765): every row is a
    // one-token sequence, for which the token-dropout scale is 0.88 exactly
    {
        ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * n * d);
        HIPCHK(launch_embed(dc->d_tokens, SeqMeta{dc->d_cu, dc->d_lens, n, 1}, m->emb.fmt, m->emb.q, m->emb.sc, d,
                            V, dc->x, st));
    }
    const int64_t layer = (int64_t)dc->slots * dc->slot_stride;
    // algorithmic attention work of the rows: keys 0..pos of their slot
    double keys = 0;
    for (int i = 0; i < n; i++) keys += dc->h_meta[dc->max_rows + 2 * i + 1] + 1;
    const bool g16 = step_gemv16(dc, n);
    const size_t part_half = dc->part.floats / 2 / 64 * 64;
    float *const part_a = dc->part.part, *const part_b = dc->part.part + part_half;
    int pend_splits = 0;  // FC2 splits waiting in part_a
    const float *pend_bias = nullptr;
    // attention and Wo in one kernel (head sizes 32 / 64, quantized Wo) for
    // one or two rows: each (row, head, 256 columns) workgroup reads its Wo
    // columns itself, which the GEMV reads once for all rows (650M Q4_0:
    // one stream 854 -> 888 tokens/s, 8 streams 6012 -> 4557); CIH_FEW_WO=0: apart
    const char *few_wo_env = getenv("CIH_FEW_WO");
    const bool fuse_wo = n <= 2 && (m->hd == 32 || m->hd == 64) && L > 0 &&
                         (m->layers[0].wo.fmt == WF_Q8 || m->layers[0].wo.fmt == WF_Q4) &&
                         (size_t)H * n * d <= part_half && !(few_wo_env && !strcmp(few_wo_env, "0"));
    // one row: the residual LayerNorms are formed inside the QKV and FC1
    // GEMVs (every workgroup normalises the row itself; the new residual goes
    // to xb, then back to x), two launches fewer per layer; CIH_DECODE_LN=0: apart
    const char *ln_env = getenv("CIH_DECODE_LN");
    const bool ln_fused = g16 && n == 1 && d <= GEMV16_LN_MAX_K && !(ln_env && !strcmp(ln_env, "0"));
    for (int l = 0; l < L && g16; l++) {
        const Layer &ly = m->layers[l];
        const unsigned short *xbh = reinterpret_cast<const unsigned short *>(dc->xb);
        if (!ln_fused) {
            ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * n * d);
            HIPCHK(launch_residual_layernorm(dc->x, pend_splits ? part_a : nullptr, pend_splits, pend_bias, ly.ln1w,
                                             ly.ln1b, dc->xb, AF_H2, n, d, st));
        }
        int sq = 0, so = 0, s1 = 0;
        if (ln_fused) {
            ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * ly.wqkv.N * d,
                         wbytes(ly.wqkv) + 4.0 * (pend_splits + 2) * d + 4.0 * ly.wqkv.N);
            HIPCHK(launch_gemv16_ln_partials(ly.wqkv, dc->x, dc->xb, pend_splits ? part_a : nullptr, pend_splits,
                                             pend_bias, ly.ln1w, ly.ln1b, part_b, part_half, &sq, st));
        } else {
            ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * n * ly.wqkv.N * d, wbytes(ly.wqkv) + 4.0 * n * d + 4.0 * n * ly.wqkv.N);
            HIPCHK(launch_gemv16_partials(ly.wqkv, xbh, n, part_b, part_half, &sq, st));
        }
        float *kc = dc->kc + l * layer, *vc = dc->vc + l * layer;
        {
            ProfScope ps(m, CIH_KC_ATTENTION, 4.0 * keys * d, 8.0 * keys * d + 24.0 * n * d);
            if (fused && fuse_wo) {
                // attention and each head's share of Wo in one kernel: the heads are Wo's splits
                HIPCHK(launch_decode_attention_fused_wo(dc->qkv, part_b, sq, ly.bqkv, d, H, dc->d_rows, n,
                                                        dc->max_len, dc->rope_c, dc->rope_s, kc, vc, dc->slot_stride,
                                                        ly.wo, part_a, part_half, st));
                so = H;
            } else if (fused) {
                HIPCHK(launch_decode_attention_fused(dc->qkv, part_b, sq, ly.bqkv, d, H, dc->d_rows, n, dc->max_len,
                                                     dc->rope_c, dc->rope_s, kc, vc, dc->slot_stride, dc->ao, st,
                                                     AF_H2));
            } else {
                HIPCHK(launch_gemv16_fold(part_b, sq, n, 3 * d, ly.bqkv, dc->qkv, 3 * d, EPI_NONE, st));
                HIPCHK(launch_rope_kv(dc->qkv, d, m->hd, dc->d_rows, n, dc->rope_c, dc->rope_s, kc, vc,
                                      dc->slot_stride, st));
                HIPCHK(launch_decode_attention(dc->qkv, d, H, dc->d_rows, n, dc->max_len, kc, vc, dc->slot_stride,
                                               dc->ao, st, AF_H2));
            }
        }
        if (!(fused && fuse_wo)) {
            ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * n * d * d, wbytes(ly.wo) + 8.0 * n * d);
            HIPCHK(launch_gemv16_partials(ly.wo, reinterpret_cast<const unsigned short *>(dc->ao), n, part_a,
                                          part_half, &so, st));
        }
        if (ln_fused) {
            ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * F * d, wbytes(ly.w1) + 4.0 * (so + 2) * d + 4.0 * F);
            HIPCHK(launch_gemv16_ln_partials(ly.w1, dc->xb, dc->x, part_a, so, ly.bo, ly.ln2w, ly.ln2b, part_b,
                                             part_half, &s1, st));
        } else {
            {
                ProfScope ps(m, CIH_KC_OTHER, 0, 4.0 * so * n * d + 12.0 * n * d);
                HIPCHK(launch_residual_layernorm(dc->x, part_a, so, ly.bo, ly.ln2w, ly.ln2b, dc->xb, AF_H2, n, d, st));
            }
            ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * n * F * d, wbytes(ly.w1) + 4.0 * n * (d + F));
            HIPCHK(launch_gemv16_partials(ly.w1, xbh, n, part_b, part_half, &s1, st));
        }
        {
            ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * n * F * d, wbytes(ly.w2) + 4.0 * s1 * n * F + 4.0 * n * d);
            HIPCHK(launch_gemv16_gelu_partials(ly.w2, part_b, s1, ly.b1, n, part_a, part_half, &pend_splits, st));
            pend_bias = ly.b2;
        }
    }
    for (int l = 0; l < L && !g16; l++) {
        const Layer &ly = m->layers[l];
        {
            ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * n * d);
            HIPCHK(launch_layernorm(dc->x, ly.ln1w, ly.ln1b, dc->xb, AF_F32, n, d, st));
        }
        // one row per sequence through the GEMV: the attention kernel adds
        // the QKV partial sums itself (no separate reduction)
        const bool qkv_parts = fused && use_gemv(n, AF_F32, EPI_NONE);
        int splits = 0;
        if (qkv_parts) {
            ProfScope ps(m, ly.wqkv.fmt == WF_F32 ? CIH_KC_GEMM_FP32 : CIH_KC_GEMM_QUANT, 2.0 * n * ly.wqkv.N * d,
                         wbytes(ly.wqkv) + 4.0 * n * d + 4.0 * n * ly.wqkv.N);
            HIPCHK(launch_gemv_partials(ly.wqkv, dc->xb, d, n, dc->part, &splits, st));
        } else {
            HIPCHK(model_gemm(m, dc->part, ly.wqkv, dc->xb, d, AF_F32, ly.bqkv, dc->qkv, 3 * d, n, EPI_NONE));
        }
        float *kc = dc->kc + l * layer, *vc = dc->vc + l * layer;
        {
            // K and V read once per key, Q read, rows written
            ProfScope ps(m, CIH_KC_ATTENTION, 4.0 * keys * d, 8.0 * keys * d + 24.0 * n * d);
            if (fused) {
                HIPCHK(launch_decode_attention_fused(dc->qkv, qkv_parts ? dc->part.part : nullptr, splits, ly.bqkv, d,
                                                     H, dc->d_rows, n, dc->max_len, dc->rope_c, dc->rope_s, kc, vc,
                                                     dc->slot_stride, dc->ao, st));
            } else {
                HIPCHK(launch_rope_kv(dc->qkv, d, m->hd, dc->d_rows, n, dc->rope_c, dc->rope_s, kc, vc,
                                      dc->slot_stride, st));
                HIPCHK(launch_decode_attention(dc->qkv, d, H, dc->d_rows, n, dc->max_len, kc, vc, dc->slot_stride,
                                               dc->ao, st));
            }
        }
        HIPCHK(model_gemm(m, dc->part, ly.wo, dc->ao, d, AF_F32, ly.bo, dc->x, d, n, EPI_RESIDUAL));
        {
            ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * n * d);
            HIPCHK(launch_layernorm(dc->x, ly.ln2w, ly.ln2b, dc->xb, AF_F32, n, d, st));
        }
        HIPCHK(model_gemm(m, dc->part, ly.w1, dc->xb, d, AF_F32, ly.b1, dc->h, F, n, EPI_GELU));
        HIPCHK(model_gemm(m, dc->part, ly.w2, dc->h, F, AF_F32, ly.b2, dc->x, d, n, EPI_RESIDUAL));
    }
    {
        // more rows than the GEMV takes go through GEMMs on f16 limbs: the
        // final LayerNorm reports a residual that overflowed them
        ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * n * d);
        int *flag = step_limbs(dc, n) ? dc->d_flag : nullptr;
        if (pend_splits)
            HIPCHK(launch_residual_layernorm(dc->x, part_a, pend_splits, pend_bias, m->lnfw, m->lnfb, dc->ao, AF_F32, n,
                                             d, st, flag));
        else
            HIPCHK(launch_layernorm(dc->x, m->lnfw, m->lnfb, dc->ao, AF_F32, n, d, st, flag));
    }
    // project_lm_head_* (lib.rs:3952-4015): dense + GELU, LN, decoder; or the
    // tied embedding without bias
    if (m->has_head) {
        HIPCHK(model_gemm(m, dc->part, m->dense, dc->ao, d, AF_F32, m->dense_b, dc->h, d, n, EPI_GELU));
        {
            ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * n * d);
            // its output feeds the decoder's GEMM, which splits it into f16
            // limbs for more rows than the GEMV takes
            HIPCHK(launch_layernorm(dc->h, m->lm_lnw, m->lm_lnb, dc->xb, AF_F32, n, d, st,
                                    step_limbs(dc, n) ? dc->d_flag : nullptr));
        }
        HIPCHK(model_gemm(m, dc->part, m->dec, dc->xb, d, AF_F32, m->dec_b, dc->logits, V, n, EPI_NONE));
    } else {
        HIPCHK(model_gemm(m, dc->part, m->emb, dc->ao, d, AF_F32, nullptr, dc->logits, V, n, EPI_NONE));
    }
    return 0;
}

// Decode steps (at most GEMV_MAX_M rows) replay a captured graph of the
// whole step, one per (rows, fused); the graph reads tokens and positions
// from the decoder's device buffers, which are refreshed before each replay.
// Profiling runs and CIH_DECODE_GRAPH=0 launch kernel by kernel.
bool use_graph(const cih_decoder *dc, int n) {
    const char *e = getenv("CIH_DECODE_GRAPH");
    return n <= GEMV_MAX_M && !dc->m->prof.on && !(e && !std::strcmp(e, "0"));
}

int run_rows(cih_decoder *dc, int n) {
    hipStream_t st = dc->m->stream;
    const bool fused = dc->unique;
    HIPCHK(hipMemcpyAsync(dc->d_tokens, dc->h_meta, (size_t)n * 4, hipMemcpyHostToDevice, st));
    HIPCHK(hipMemcpyAsync(dc->d_rows, dc->h_meta + dc->max_rows, (size_t)n * 8, hipMemcpyHostToDevice, st));
    // Rows whose activations travel as f16 limbs: a non-finite residual (an
    // overflowed limb) runs the rows again in full-range mode, kernel by
    // kernel, rewriting the same cache positions.
    const bool limbs = step_limbs(dc, n);
    int *h_flag = dc->h_meta + 3 * dc->max_rows;
    auto check = [&]() -> int {
        HIPCHK(hipMemcpyAsync(h_flag, dc->d_flag, sizeof(int), hipMemcpyDeviceToHost, st));
        HIPCHK(hipStreamSynchronize(st));
        if (*h_flag & FLAG_NONFINITE) return in_full_range([&] { return enqueue_rows(dc, n, fused); });
        return 0;
    };
    if (limbs) HIPCHK(hipMemsetAsync(dc->d_flag, 0, sizeof(int), st));
    if (!use_graph(dc, n)) {
        if (int rc = enqueue_rows(dc, n, fused)) return rc;
        return limbs ? check() : 0;
    }
    auto key = std::make_tuple(n, fused, kernel_switches());
    auto it = dc->graphs.find(key);
    if (it == dc->graphs.end()) {
        hipGraph_t g = nullptr;
        HIPCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        const int rc = enqueue_rows(dc, n, fused);
        const hipError_t e = hipStreamEndCapture(st, &g);
        if (rc || e != hipSuccess) {
            if (g) hipGraphDestroy(g);
            return rc ? rc : set_error(CIH_ERR_HIP, "decode step capture failed: %s", hipGetErrorString(e));
        }
        hipGraphExec_t ex = nullptr;
        const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (ei != hipSuccess) return set_error(CIH_ERR_HIP, "decode step graph: %s", hipGetErrorString(ei));
        it = dc->graphs.emplace(key, ex).first;
    }
    HIPCHK(hipGraphLaunch(it->second, st));
    return limbs ? check() : 0;
}

// Validates rows and stages them; rows of one slot must continue its
// cache: consecutive positions starting at most at the slot's filled count.
int stage_rows(cih_decoder *dc, const int32_t *slots, const int32_t *tokens, const int32_t *pos, int n) {
    const int V = dc->m->cfg.vocab_size;
    if (n < 1 || n > dc->max_rows) return set_error(CIH_ERR_CAPACITY, "%d rows outside [1, %d]", n, dc->max_rows);
    std::map<int, int> next;  // slot -> next position this call may write
    for (int i = 0; i < n; i++) {
        const int s = slots[i], p = pos[i], t = tokens[i];
        if (s < 0 || s >= dc->slots) return set_error(CIH_ERR_ARG, "row %d: slot %d outside [0, %d)", i, s, dc->slots);
        if (t < 0 || t >= V) return set_error(CIH_ERR_TOKEN, "row %d: token %d outside [0, %d)", i, t, V);
        if (p < 0 || p >= dc->max_len)
            return set_error(CIH_ERR_CAPACITY, "row %d: position %d outside [0, %d)", i, p, dc->max_len);
        auto it = next.find(s);
        const int allowed = it == next.end() ? dc->filled[s] : it->second;
        if (it == next.end() ? p > allowed : p != allowed)
            return set_error(CIH_ERR_ARG, "row %d: slot %d position %d does not continue its cache (next %d)", i, s, p,
                             allowed);
        next[s] = p + 1;
        dc->h_meta[i] = t;
        dc->h_meta[dc->max_rows + 2 * i] = s;
        dc->h_meta[dc->max_rows + 2 * i + 1] = p;
    }
    for (auto &kv : next) dc->filled[kv.first] = std::max(dc->filled[kv.first], kv.second);
    dc->unique = (int)next.size() == n;
    return 0;
}

// SimpleRng (lib.rs:3506-3511): xorshift64 (13, 7, 17); seed 0 is replaced.
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed == 0 ? 0x123456789abcdefULL : seed) {}
    uint32_t next_u32() {
        uint64_t x = s;
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        s = x;
        return (uint32_t)x;
    }
    float next_f32() { return (float)next_u32() / (float)UINT32_MAX; }
};

// sample (lib.rs:3513-3530): ids 4..=23 and <eos> only; argmax for T <= 0,
// else softmax(logits / T) and the first id whose running sum reaches r.
int sample(float *lg, int V, float temperature, Rng &rng) {
    for (int i = 0; i < V; i++)
        if (!((i >= 4 && i <= 23) || i == 2)) lg[i] = -INFINITY;
    if (temperature <= 0.0f) {
        float mv = lg[0];
        int mi = 0;
        for (int i = 1; i < V; i++)
            if (lg[i] > mv) { mv = lg[i]; mi = i; }
        return mi;
    }
    const float inv_temp = 1.0f / temperature;
    for (int i = 0; i < V; i++)
        if (lg[i] != -INFINITY) lg[i] *= inv_temp;
    float mx = -INFINITY;
    for (int i = 0; i < V; i++) mx = std::fmax(mx, lg[i]);
    float sum = 0.0f;
    for (int i = 0; i < V; i++) { lg[i] = std::exp(lg[i] - mx); sum += lg[i]; }
    const float inv = 1.0f / sum;
    for (int i = 0; i < V; i++) lg[i] *= inv;
    const float r = rng.next_f32();
    float cum = 0.0f;
    for (int i = 0; i < V; i++) {
        if (std::isnan(lg[i]) || lg[i] == 0.0f) continue;
        cum += lg[i];
        if (r <= cum) return i;
    }
    return 4;
}

double ms_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

}  // namespace

extern "C" {

int cih_decoder_create(cih_model *m, int32_t n_slots, int32_t max_len, int32_t max_rows, cih_decoder **out) {
    if (!m || !out) return set_error(CIH_ERR_ARG, "null argument");
    *out = nullptr;
    if (n_slots < 1 || max_len < 1 || max_rows < 1) return set_error(CIH_ERR_ARG, "n_slots, max_len, max_rows must be >= 1");
    if (max_len > 15000) return set_error(CIH_ERR_SHAPE, "max_len %d above the attention kernel's 15000", max_len);
    const size_t d = m->cfg.dim, F = m->cfg.hidden_dim, V = m->cfg.vocab_size, L = m->cfg.n_layers;
    const size_t R = max_rows;
    cih_decoder *dc = new cih_decoder();
    dc->m = m;
    dc->slots = n_slots;
    dc->max_len = max_len;
    dc->max_rows = max_rows;
    dc->slot_stride = (int64_t)max_len * d;
    dc->filled.assign(n_slots, 0);
    auto &al = dc->allocs;
    const size_t cache = L * n_slots * (size_t)max_len * d;
    bool good = dalloc(dc->kc, cache, al) == hipSuccess && dalloc(dc->vc, cache, al) == hipSuccess &&
                dalloc(dc->rope_c, (size_t)max_len * (m->hd / 2), al) == hipSuccess &&
                dalloc(dc->rope_s, (size_t)max_len * (m->hd / 2), al) == hipSuccess &&
                dalloc(dc->x, R * d, al) == hipSuccess && dalloc(dc->xb, R * d, al) == hipSuccess &&
                dalloc(dc->qkv, R * 3 * d, al) == hipSuccess && dalloc(dc->ao, R * d, al) == hipSuccess &&
                dalloc(dc->h, R * std::max(F, d), al) == hipSuccess && dalloc(dc->logits, R * V, al) == hipSuccess &&
                dalloc(dc->d_tokens, R, al) == hipSuccess && dalloc(dc->d_rows, 2 * R, al) == hipSuccess &&
                dalloc(dc->d_cu, R, al) == hipSuccess && dalloc(dc->d_lens, R, al) == hipSuccess &&
                dalloc(dc->d_flag, 1, al) == hipSuccess;
    dc->part.floats = model_part_floats(m);
    good = good && dalloc(dc->part.part, dc->part.floats, al) == hipSuccess &&
           hipHostMalloc((void **)&dc->h_meta, (3 * R + 1) * sizeof(int)) == hipSuccess &&
           hipHostMalloc((void **)&dc->h_logits, R * V * sizeof(float)) == hipSuccess;
    if (!good) {
        destroy(dc);
        return set_error(CIH_ERR_HIP, "decoder allocation failed (%zu MiB of KV cache)", 2 * cache * 4 >> 20);
    }
    std::vector<float> c, s;
    rope_tables_host(max_len, m->hd, c, s);
    std::vector<int> cu(R), lens(R, 1);
    for (size_t i = 0; i < R; i++) cu[i] = (int)i;
    hipError_t e = hipMemcpy(dc->rope_c, c.data(), c.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dc->rope_s, s.data(), s.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dc->d_cu, cu.data(), R * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dc->d_lens, lens.data(), R * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        destroy(dc);
        return set_error(CIH_ERR_HIP, "decoder set-up failed: %s", hipGetErrorString(e));
    }
    *out = dc;
    return CIH_OK;
}

int cih_decoder_destroy(cih_decoder *dc) {
    destroy(dc);
    return CIH_OK;
}

int cih_decoder_reset(cih_decoder *dc, int32_t slot) {
    if (!dc) return set_error(CIH_ERR_ARG, "null decoder");
    if (slot < 0) std::fill(dc->filled.begin(), dc->filled.end(), 0);
    else if (slot < dc->slots) dc->filled[slot] = 0;
    else return set_error(CIH_ERR_ARG, "slot %d outside [0, %d)", slot, dc->slots);
    return CIH_OK;
}

int cih_decode(cih_decoder *dc, const int32_t *slots, const int32_t *tokens, const int32_t *pos, int32_t n,
               float *logits) {
    if (!dc || !slots || !tokens || !pos) return set_error(CIH_ERR_ARG, "null argument");
    if (int rc = stage_rows(dc, slots, tokens, pos, n)) return rc;
    if (int rc = run_rows(dc, n)) return rc;
    const size_t lb = (size_t)n * dc->m->cfg.vocab_size * 4;
    if (logits) HIPCHK(hipMemcpyAsync(dc->h_logits, dc->logits, lb, hipMemcpyDeviceToHost, dc->m->stream));
    HIPCHK(hipStreamSynchronize(dc->m->stream));
    if (logits) std::memcpy(logits, dc->h_logits, lb);
    profile_collect(dc->m);
    return CIH_OK;
}

int cih_generate(cih_decoder *dc, int32_t n, const int32_t *slots, const int32_t *prompts, const int32_t *offsets,
                 float temperature, int32_t max_new_tokens, const uint64_t *seeds, int32_t max_seq_len,
                 int32_t *out_tokens, int32_t out_cap, int32_t *n_generated, double *prefill_ms,
                 double *generation_ms) {
    if (!dc || !slots || !prompts || !offsets || !seeds || !out_tokens || !n_generated)
        return set_error(CIH_ERR_ARG, "null argument");
    if (n < 1) return set_error(CIH_ERR_ARG, "n must be >= 1");
    const int V = dc->m->cfg.vocab_size;
    const int msl = max_seq_len > 0 ? std::min(max_seq_len, dc->max_len) : dc->max_len;
    std::vector<int> pos(n, 0), limit(n), count(n, 0);
    std::vector<char> seen(dc->slots, 0);
    for (int i = 0; i < n; i++) {
        if (slots[i] < 0 || slots[i] >= dc->slots) return set_error(CIH_ERR_ARG, "slot %d out of range", slots[i]);
        if (seen[slots[i]]++) return set_error(CIH_ERR_ARG, "slot %d used by two streams", slots[i]);
        if (offsets[i + 1] < offsets[i]) return set_error(CIH_ERR_ARG, "offsets must not decrease");
        for (int k = offsets[i]; k < offsets[i + 1]; k++)
            if (prompts[k] < 0 || prompts[k] >= V) return set_error(CIH_ERR_TOKEN, "prompt token %d out of range", prompts[k]);
        pos[i] = std::min(offsets[i + 1] - offsets[i], msl);
        limit[i] = max_new_tokens >= 0 ? std::min(pos[i] + max_new_tokens, msl) : msl;
        if (limit[i] - pos[i] > out_cap)
            return set_error(CIH_ERR_CAPACITY, "stream %d may generate %d tokens, out_cap is %d", i, limit[i] - pos[i],
                             out_cap);
    }
    std::vector<float> lg((size_t)n * V);
    // prefill: each stream's prompt through the model, one call per stream
    // (chunks of max_rows positions), so a stream's cache does not depend on
    // which other streams run with it
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < n; i++) {
        dc->filled[slots[i]] = 0;
        for (int p0 = 0; p0 < pos[i]; p0 += dc->max_rows) {
            const int k = std::min(dc->max_rows, pos[i] - p0);
            std::vector<int32_t> sl(k, slots[i]), tk(prompts + offsets[i] + p0, prompts + offsets[i] + p0 + k), ps(k);
            for (int j = 0; j < k; j++) ps[j] = p0 + j;
            if (int rc = stage_rows(dc, sl.data(), tk.data(), ps.data(), k)) return rc;
            if (int rc = run_rows(dc, k)) return rc;
            if (p0 + k == pos[i]) {
                HIPCHK(hipMemcpyAsync(dc->h_logits, dc->logits + (size_t)(k - 1) * V, V * 4, hipMemcpyDeviceToHost,
                                      dc->m->stream));
                HIPCHK(hipStreamSynchronize(dc->m->stream));
                std::memcpy(&lg[(size_t)i * V], dc->h_logits, V * 4);
            }
        }
    }
    HIPCHK(hipStreamSynchronize(dc->m->stream));
    profile_collect(dc->m);
    const double t_prefill = ms_since(t0);
    // generation: every live stream samples from its last logits and feeds the
    // token back at its next position; all live streams share one call
    const auto t1 = std::chrono::steady_clock::now();
    std::vector<Rng> rng;
    for (int i = 0; i < n; i++) rng.emplace_back(seeds[i]);
    std::vector<char> live(n, 1);
    std::vector<int> idx;
    std::vector<int32_t> sl, tk, ps;
    std::vector<float> tmp(V);
    for (;;) {
        idx.clear(); sl.clear(); tk.clear(); ps.clear();
        for (int i = 0; i < n; i++) {
            if (!live[i]) continue;
            if (pos[i] >= limit[i]) { live[i] = 0; continue; }
            std::memcpy(tmp.data(), &lg[(size_t)i * V], V * 4);
            const int t = sample(tmp.data(), V, temperature, rng[i]);
            if (t == 2) { live[i] = 0; continue; }
            out_tokens[(size_t)i * out_cap + count[i]++] = t;
            idx.push_back(i); sl.push_back(slots[i]); tk.push_back(t); ps.push_back(pos[i]++);
        }
        if (idx.empty()) break;
        for (size_t j0 = 0; j0 < idx.size(); j0 += dc->max_rows) {
            const int k = (int)std::min<size_t>(dc->max_rows, idx.size() - j0);
            if (int rc = stage_rows(dc, &sl[j0], &tk[j0], &ps[j0], k)) return rc;
            if (int rc = run_rows(dc, k)) return rc;
            HIPCHK(hipMemcpyAsync(dc->h_logits, dc->logits, (size_t)k * V * 4, hipMemcpyDeviceToHost, dc->m->stream));
            HIPCHK(hipStreamSynchronize(dc->m->stream));
            for (int j = 0; j < k; j++) std::memcpy(&lg[(size_t)idx[j0 + j] * V], dc->h_logits + (size_t)j * V, V * 4);
            profile_collect(dc->m);
        }
    }
    for (int i = 0; i < n; i++) n_generated[i] = count[i];
    if (prefill_ms) *prefill_ms = t_prefill;
    if (generation_ms) *generation_ms = ms_since(t1);
    return CIH_OK;
}

}  // extern "C"
