// C ABI of the gfx950 ESM-2 encoder: model residency, workspace, and the
// batched bidirectional forward that replaces codon-infer's
// forward_bidirectional* family (src/lib.rs:5078-6147).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "host.h"
#include "kernels.h"

using namespace cih;

namespace cih {
static thread_local std::string g_err;

int set_error(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
}  // namespace cih

#include "model.h"

namespace cih {
static thread_local bool g_full_range = false;
bool full_range_mode() { return g_full_range; }
void set_full_range_mode(bool on) { g_full_range = on; }

std::string kernel_switches() {
    static const char *const names[] = {"CIH_ATT",     "CIH_ATT_QB", "CIH_ATT_SPLIT", "CIH_SPLITK",
                                        "CIH_QGEMM",   "CIH_ACT",    "CIH_LIMBS",     "CIH_GEMV",
                                        "CIH_GEMV_NB", "CIH_GEMM_LDS", "CIH_GEMM_TILE", "CIH_GEMM_TILE_N",
                                        "CIH_GEMM_TILE_N_GELU", "CIH_ATT_IMG", "CIH_GEMV16", "CIH_GEMV16_KW",
                                        "CIH_FEW_WO", "CIH_DECODE_LN", "CIH_ATT_XCD", "CIH_GEMM_SCHED",
                                        "CIH_GEMM_PLAN", "CIH_GEMM_PERSIST", "CIH_GEMM_KW"};
    std::string s = g_full_range ? "R|" : "|";
    for (const char *n : names) {
        const char *v = getenv(n);
        s += v ? v : "";
        s += '|';
    }
    return s;
}
}  // namespace cih

namespace cih {

void free_list(std::vector<void *> &l) {
    for (void *p : l) hipFree(p);
    l.clear();
}

int check_config(const cih_config *c) {
    if (!c) return set_error(CIH_ERR_ARG, "null config");
    if (c->dim <= 0 || c->n_heads <= 0 || c->n_layers <= 0 || c->hidden_dim <= 0 || c->vocab_size <= 0)
        return set_error(CIH_ERR_SHAPE, "non-positive config dimension");
    if (c->dim % c->n_heads) return set_error(CIH_ERR_SHAPE, "dim %d not divisible by n_heads %d", c->dim, c->n_heads);
    const int hd = c->dim / c->n_heads;
    if (hd != 16 && hd != 24 && hd != 32 && hd != 64)
        return set_error(CIH_ERR_SHAPE, "head_dim %d not in {16, 24, 32, 64}", hd);
    if (c->dim % 32 || c->hidden_dim % 32)
        return set_error(CIH_ERR_SHAPE, "dim and hidden_dim must be multiples of 32 (got %d, %d)", c->dim,
                         c->hidden_dim);
    if (c->dim > 2560) return set_error(CIH_ERR_SHAPE, "dim %d above the LayerNorm kernel's 2560", c->dim);
    if (c->vocab_size <= 32) return set_error(CIH_ERR_SHAPE, "vocab_size must be > 32 (<mask> is id 32)");
    return 0;
}

}  // namespace cih

namespace {

void clear_graphs(Workspace &ws) {
    for (auto &g : ws.graphs) hipGraphExecDestroy(g.second);
    ws.graphs.clear();
}

// Forwards replay captured graphs unless profiling (event pairs per launch)
// or CIH_FORWARD_GRAPH=0.
bool use_forward_graph(const cih_model *m) {
    const char *e = getenv("CIH_FORWARD_GRAPH");
    return !m->prof.on && !(e && !std::strcmp(e, "0"));
}

void free_workspace(Workspace &ws) {
    clear_graphs(ws);
    free_list(ws.dev);
    for (void *p : ws.host) hipHostFree(p);
    ws.host.clear();
    ws = Workspace();
}


}  // namespace

namespace cih {

double wbytes(const DevMatrix &W) {
    const double e = (double)W.N * W.K;
    return W.fmt == WF_F32 ? 4.0 * e : (W.fmt == WF_Q8 ? 1.125 * e : 0.625 * e);
}

// A few tokens go to the weight-streaming GEMV (CIH_GEMV=0 turns it off).
bool use_gemv(int M, int a_fmt, int epi) {
    const char *e = getenv("CIH_GEMV");
    return !(e && !std::strcmp(e, "0")) && M <= GEMV_MAX_M && a_fmt == AF_F32 && epi != EPI_GELU_X3 &&
           epi != EPI_GELU_H2;
}

}  // namespace cih

namespace {

}  // namespace

namespace cih {

hipError_t model_gemm(cih_model *m, const PartialBuf &pb, const DevMatrix &W, const void *X, int ldx, int a_fmt,
                      const float *bias, void *Y, int ldy, int M, int epi, int *defer) {
    if (defer) *defer = 0;
    const double flops = 2.0 * M * W.N * W.K;
    const double in_b = a_fmt == AF_X3 ? 6.0 : 4.0, out_b = epi == EPI_GELU_X3 ? 6.0 : 4.0;  // H2: 4 B/element
    const double bytes = wbytes(W) + in_b * M * W.K + out_b * M * W.N * (epi == EPI_RESIDUAL ? 2 : 1);
    ProfScope ps(m, W.fmt == WF_F32 ? CIH_KC_GEMM_FP32 : CIH_KC_GEMM_QUANT, flops, bytes);
    if (use_gemv(M, a_fmt, epi))
        return launch_gemv(W, (const float *)X, ldx, M, bias, (float *)Y, ldy, epi, pb, m->stream);
    if (gemv16_applies(W, a_fmt, M, epi))
        return launch_gemv16(W, (const unsigned short *)X, M, bias, Y, ldy, epi, &pb, m->stream);
    return launch_gemm(W, X, ldx, a_fmt, bias, Y, ldy, M, epi, &pb, m->stream, defer);
}

void profile_collect(cih_model *m) {
    if (m->prof.on) {
        for (size_t i = 0; i < m->prof.used; i++) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, m->prof.ev[2 * i], m->prof.ev[2 * i + 1]) != hipSuccess) continue;
            cih_kernel_stats &s = m->prof.st[m->prof.cls[i]];
            s.launches++;
            s.total_ms += ms;
            s.flops += m->prof.flops[i];
            s.bytes += m->prof.bytes[i];
        }
    }
    m->prof.used = 0;
}

size_t model_part_floats(const cih_model *m, size_t tokens) {
    size_t pf = 0;
    std::vector<const DevMatrix *> mats = {&m->emb};
    if (m->has_head) mats.insert(mats.end(), {&m->dense, &m->dec});
    if (!m->layers.empty()) {
        const Layer &ly = m->layers[0];
        mats.insert(mats.end(), {&ly.wqkv, &ly.wo, &ly.w1, &ly.w2});
    }
    for (const DevMatrix *w : mats) pf = std::max(pf, gemv_part_floats(w->N, w->K));
    // the LDS GEMM's split-K form (residual projections, N = dim): up to 4
    // splits of tokens x dim while that is below 256 tiles of 128 x 128
    const size_t split = std::min(tokens * m->cfg.dim, (size_t)256 * 128 * 128) * 4;
    return std::max({pf, SPLITK_PART_FLOATS, split});
}

// RoPE tables (BidirectionalRunState::new / RunState::new, lib.rs:2513-2522,
// 2466-2474): the same f32 powf / cos / sin calls, evaluated on the host.
void rope_tables_host(size_t max_len, int hd, std::vector<float> &c, std::vector<float> &s) {
    const size_t half = hd / 2;
    c.assign(max_len * half, 0.0f);
    s.assign(max_len * half, 0.0f);
    for (size_t pos = 0; pos < max_len; pos++)
        for (size_t j = 0; j < half; j++) {
            const float freq = 1.0f / std::pow(10000.0f, (float)(j * 2) / (float)hd);
            const float val = (float)pos * freq;
            c[pos * half + j] = std::cos(val);
            s[pos * half + j] = std::sin(val);
        }
}

}  // namespace cih

namespace {

hipError_t gemm(cih_model *m, const DevMatrix &W, const void *X, int ldx, int a_fmt, const float *bias, void *Y, int ldy,
                int M, int epi, int *defer = nullptr) {
    return model_gemm(m, m->ws.part, W, X, ldx, a_fmt, bias, Y, ldy, M, epi, defer);
}

}  // namespace

// =============================================================================

extern "C" {

const char *cih_last_error(void) { return g_err.c_str(); }
int cih_abi_version(void) { return CIH_ABI_VERSION; }

int cih_model_config(const cih_model *m, cih_config *cfg, int32_t *dtype) {
    if (!m) return set_error(CIH_ERR_ARG, "null model");
    if (cfg) *cfg = m->cfg;
    if (dtype) *dtype = m->dtype;
    return CIH_OK;
}

int cih_model_destroy(cih_model *m) {
    if (!m) return CIH_OK;
    if (m->stream) hipStreamSynchronize(m->stream);
    free_workspace(m->ws);
    free_list(m->allocs);
    for (auto e : m->prof.ev) hipEventDestroy(e);
    if (m->stream) hipStreamDestroy(m->stream);
    delete m;
    return CIH_OK;
}

int cih_model_reserve(cih_model *m, int32_t max_batch, int32_t max_seq_len, uint32_t flags) {
    if (!m) return set_error(CIH_ERR_ARG, "null model");
    if (max_batch < 1 || max_seq_len < 1) return set_error(CIH_ERR_ARG, "max_batch and max_seq_len must be >= 1");
    if ((flags & CIH_OUT_CONTACTS) && !m->has_contacts)
        return set_error(CIH_ERR_ARG, "contacts requested but the model has no contact weights");
    HIPCHK(hipStreamSynchronize(m->stream));
    free_workspace(m->ws);
    Workspace &ws = m->ws;
    ws.maxB = max_batch;
    ws.maxS = max_seq_len;
    ws.flags = flags;
    const size_t B = max_batch, S = max_seq_len, T = B * S;
    const size_t d = m->cfg.dim, F = m->cfg.hidden_dim, V = m->cfg.vocab_size, H = m->cfg.n_heads,
                 L = m->cfg.n_layers, half = m->hd / 2;
    const size_t n = S >= 2 ? S - 2 : 0;
    auto &dl = ws.dev;
    auto ok = [&](hipError_t e) {
        if (e != hipSuccess) set_error(CIH_ERR_HIP, "workspace allocation failed: %s", hipGetErrorString(e));
        return e == hipSuccess;
    };
    bool good = ok(dalloc(ws.tokens, T, dl)) && ok(dalloc(ws.cu, B, dl)) && ok(dalloc(ws.lens, B, dl)) &&
                // xb, ao and hbuf also hold the three-limb bf16 form (6 B/element)
                ok(dalloc(ws.x, T * d, dl)) && ok(dalloc(ws.xb, T * d * 3 / 2, dl)) &&
                ok(dalloc(ws.qkv, T * 3 * d, dl)) && ok(dalloc(ws.ao, T * d * 3 / 2, dl)) &&
                ok(dalloc(ws.hbuf, T * std::max(F * 3 / 2, d), dl)) &&
                ok(dalloc(ws.logits, T * V, dl)) && ok(dalloc(ws.rope_c, S * half, dl)) &&
                ok(dalloc(ws.rope_s, S * half, dl));
    if (good) {
        ws.part.floats = model_part_floats(m, T);
        const size_t nd = std::max(B, S);
        ws.attp_floats = attention_part_floats((int)m->hd);
        good = ok(dalloc(ws.part.part, ws.part.floats, dl)) && ok(dalloc(ws.dms_meta, nd * 2, dl)) &&
               ok(dalloc(ws.dms_out, nd * 21, dl)) && ok(dalloc(ws.attp, ws.attp_floats, dl));
    }
    const bool need_P = flags & (CIH_OUT_CONTACTS | CIH_OUT_FINAL_ATT | CIH_OUT_ATTN);
    if (good && need_P) good = ok(dalloc(ws.P, B * H * S * S, dl));
    if (good && attention_img_supported((int)m->hd)) {
        // tile images for every (tile row, head): at most B ceil(S / 32) tile rows;
        // zeroed once, so dims past hd stay zero (nothing writes them)
        const size_t img = B * ((S + 31) / 32) * H * kv_image_bytes((int)m->hd);
        good = ok(dalloc(ws.kv_img, img, dl)) && ok(dalloc(ws.kv_tb, B, dl)) && ok(dalloc(ws.kv_pk, T, dl)) &&
               ok(dalloc(ws.kv_pos, T, dl)) && ok(dalloc(ws.kv_ti, B * ((S + 31) / 32) * 4, dl)) &&
               ok(hipMemset(ws.kv_img, 0, img));
    }
    if (good && (flags & CIH_OUT_CONTACTS))
        good = ok(dalloc(ws.M, B * n * n, dl)) && ok(dalloc(ws.r, L * H * B * n, dl)) &&
               ok(dalloc(ws.coef, L * H * B, dl)) && ok(dalloc(ws.rowsum, B * H * S, dl)) &&
               ok(dalloc(ws.colpart, B * H * ((n + 31) / 32) * n, dl));
    if (good && !(flags & CIH_IO_DEVICE)) {
        if (flags & CIH_OUT_LOGITS) good = good && ok(dalloc(ws.o_logits, T * V, dl));
        if (flags & CIH_OUT_HIDDEN) good = good && ok(dalloc(ws.o_hidden, T * d, dl));
        if (flags & CIH_OUT_FINAL_ATT) good = good && ok(dalloc(ws.o_final, B * S * S, dl));
        if (flags & CIH_OUT_CONTACTS) good = good && ok(dalloc(ws.o_contacts, B * n * n, dl));
        if (flags & CIH_OUT_ATTN) good = good && ok(dalloc(ws.o_attn, B * L * H * S * S, dl));
        if (flags & CIH_OUT_LAYER_HIDDEN) good = good && ok(dalloc(ws.o_layer, B * L * S * d, dl));
        // pinned staging: the largest single output, at most 64 MiB (whole
        // rows at a time; a row is at most max(V, d, S) floats)
        size_t need = 0;
        if (flags & CIH_OUT_LOGITS) need = std::max(need, T * V);
        if (flags & CIH_OUT_HIDDEN) need = std::max(need, T * d);
        if (flags & CIH_OUT_FINAL_ATT) need = std::max(need, B * S * S);
        if (flags & CIH_OUT_CONTACTS) need = std::max(need, B * n * n);
        if (flags & CIH_OUT_ATTN) need = std::max(need, B * L * H * S * S);
        if (flags & CIH_OUT_LAYER_HIDDEN) need = std::max(need, B * L * S * d);
        void *hp = nullptr;
        if (good && need) {
            need = std::max(std::min(need, (size_t)16 << 20), std::max(std::max(V, d), S));
            if (!ok(hipHostMalloc(&hp, need * sizeof(float)))) good = false;
            else {
                ws.host.push_back(hp);
                ws.h_stage = (float *)hp;
                ws.h_stage_floats = need;
            }
        }
    }
    if (good) {
        void *hp = nullptr;
        if (!ok(hipHostMalloc(&hp, (2 * B + 1) * sizeof(int)))) good = false;
        else { ws.host.push_back(hp); ws.h_meta = (int *)hp; }
        good = good && ok(dalloc(ws.flag, 1, dl));
    }
    if (!good) {
        free_workspace(ws);
        return CIH_ERR_HIP;
    }
    std::vector<float> c, s;
    rope_tables_host(S, m->hd, c, s);
    HIPCHK(hipMemcpy(ws.rope_c, c.data(), c.size() * 4, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(ws.rope_s, s.data(), s.size() * 4, hipMemcpyHostToDevice));
    return CIH_OK;
}

}  // extern "C"

namespace {

// The forward behind cih_forward.  keep_logits: compute the LM head into the
// workspace's packed logits ws.logits [T][V] (rows cu[b] + pos) even when no
// logits output is requested (the DMS driver scores them on the device).
int forward_impl(cih_model *m, const int32_t *tokens, const int32_t *lens, int32_t B, int32_t S_max, uint32_t flags,
                 const cih_outputs *out, bool keep_logits) {
    if (!m || !tokens || !lens || !out) return set_error(CIH_ERR_ARG, "null argument");
    Workspace &ws = m->ws;
    if (ws.maxB == 0) return set_error(CIH_ERR_CAPACITY, "cih_model_reserve has not been called");
    if (B < 1 || S_max < 1) return set_error(CIH_ERR_ARG, "B and S_max must be >= 1");
    if (B > ws.maxB || S_max > ws.maxS)
        return set_error(CIH_ERR_CAPACITY, "batch %d x %d exceeds the reserved %d x %d", B, S_max, ws.maxB, ws.maxS);
    const uint32_t kinds = flags & 0xFFFFu;
    if (kinds & ~ws.flags & 0x3Fu) return set_error(CIH_ERR_CAPACITY, "output kinds 0x%x were not reserved", kinds);
    const bool dev_io = flags & CIH_IO_DEVICE;
    if (!dev_io && (ws.flags & CIH_IO_DEVICE) && (kinds & 0x3Fu))
        return set_error(CIH_ERR_CAPACITY, "workspace reserved for device I/O only");
    const bool want_logits = kinds & CIH_OUT_LOGITS, want_hidden = kinds & CIH_OUT_HIDDEN,
               want_final = kinds & CIH_OUT_FINAL_ATT, want_contacts = kinds & CIH_OUT_CONTACTS,
               want_attn = kinds & CIH_OUT_ATTN, want_layer = kinds & CIH_OUT_LAYER_HIDDEN;
    if ((want_logits && !out->logits) || (want_hidden && !out->hidden) || (want_final && !out->final_att) ||
        (want_contacts && !out->contacts) || (want_attn && !out->attn) || (want_layer && !out->layer_hidden))
        return set_error(CIH_ERR_ARG, "null output buffer for a requested output");

    const int d = m->cfg.dim, F = m->cfg.hidden_dim, V = m->cfg.vocab_size, H = m->cfg.n_heads, L = m->cfg.n_layers;
    int *cu = ws.h_meta, *hl = ws.h_meta + ws.maxB;
    int T = 0;
    for (int b = 0; b < B; b++) {
        if (lens[b] < 1 || lens[b] > S_max)
            return set_error(CIH_ERR_ARG, "lens[%d] = %d outside [1, %d]", b, lens[b], S_max);
        // accumulate_head_apc's row_sums is [f32; 1024] (lib.rs:5046)
        if (want_contacts && lens[b] - 2 > 1024)
            return set_error(CIH_ERR_CONTACTS, "contacts need n_res <= 1024 (sequence %d has %d)", b, lens[b] - 2);
        cu[b] = T;
        hl[b] = lens[b];
        T += lens[b];
    }
    if (!dev_io) {
        for (int b = 0; b < B; b++)
            for (int s = 0; s < lens[b]; s++) {
                const int t = tokens[(size_t)b * S_max + s];
                if (t < 0 || t >= V) return set_error(CIH_ERR_TOKEN, "token %d at [%d][%d] outside [0, %d)", t, b, s, V);
            }
    }
    hipStream_t st = m->stream;
    const int n_max = S_max >= 2 ? S_max - 2 : 0;
    const size_t SS = (size_t)S_max * S_max;

    HIPCHK(hipMemcpyAsync(ws.tokens, tokens, (size_t)B * S_max * 4, dev_io ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st));
    HIPCHK(hipMemcpyAsync(ws.cu, cu, B * 4, hipMemcpyHostToDevice, st));
    HIPCHK(hipMemcpyAsync(ws.lens, hl, B * 4, hipMemcpyHostToDevice, st));
    const SeqMeta sm{ws.cu, ws.lens, B, S_max};

    // output targets on the device (caller's buffers or staging)
    float *t_logits = dev_io ? out->logits : ws.o_logits, *t_hidden = dev_io ? out->hidden : ws.o_hidden,
          *t_final = dev_io ? out->final_att : ws.o_final, *t_contacts = dev_io ? out->contacts : ws.o_contacts,
          *t_attn = dev_io ? out->attn : ws.o_attn, *t_layer = dev_io ? out->layer_hidden : ws.o_layer;

    // Activations reach the quantized GEMMs already split into f16 limbs
    // (AF_H2, written by LayerNorm / attention / FC1's epilogue: same bytes as
    // FP32, no conversion in the GEMM).  CIH_ACT=f32 hands over FP32 (split in
    // the GEMM), CIH_ACT=x3 the three-limb bf16 form; CIH_LIMBS=bf16x3 and
    // CIH_QGEMM=fp32 imply FP32 hand-off.  Batches of at most GEMV_MAX_M
    // tokens take the f16-MFMA GEMV (k_gemv16), which reads limbs too; with
    // any of those switches, CIH_GEMV16=0 or in full range the FP32 GEMV.
    int af = AF_F32;
    {
        const char *qpath = getenv("CIH_QGEMM"), *apath = getenv("CIH_ACT"), *lpath = getenv("CIH_LIMBS");
        const bool fp32_gemm = qpath && !std::strcmp(qpath, "fp32");
        const bool bf16 = lpath && !std::strcmp(lpath, "bf16x3");
        if (m->dtype != DT_FP32 && !fp32_gemm && T > GEMV_MAX_M) {
            if ((apath && !std::strcmp(apath, "x3")) || full_range_mode()) af = AF_X3;
            else if (!(apath && !std::strcmp(apath, "f32")) && !bf16) af = AF_H2;
        } else if (m->dtype == DT_FP32 && !fp32_gemm && !bf16 && !apath && !full_range_mode() && T > GEMV_MAX_M &&
                   L > 0 && m->layers[0].wqkv.p16) {
            // FP32 weights through their f16 pair copies: the activations as
            // f16 limbs too (the same split the GEMM makes of FP32 ones, so the
            // same bits), which the LDS-staged GEMM reads; CIH_ACT=f32: FP32
            af = AF_H2;
        } else if (m->dtype != DT_FP32 && !fp32_gemm && !apath && !bf16 && !full_range_mode() && L > 0 &&
                   gemv16_applies(m->layers[0].wqkv, AF_H2, T, EPI_NONE) &&
                   gemv16_applies(m->layers[0].wo, AF_H2, T, EPI_NONE) &&
                   gemv16_applies(m->layers[0].w1, AF_H2, T, EPI_NONE) &&
                   gemv16_applies(m->layers[0].w2, AF_H2, T, EPI_NONE) && d % 32 == 0 && F % 32 == 0) {
            af = AF_H2;  // few tokens: the f16-MFMA GEMV (k_gemv16) reads limbs
        }
    }
    const int epi_fc1 = af == AF_X3 ? EPI_GELU_X3 : (af == AF_H2 ? EPI_GELU_H2 : EPI_GELU);
    // Few tokens (af == AF_H2 at T <= GEMV_MAX_M: the f16-MFMA GEMV): each
    // projection leaves split-K partial sums in one half of the partial
    // buffer, and the kernel after it adds them (attention: the QKV splits;
    // the residual LayerNorm: Wo's, and FC2's of the layer before; FC2: FC1's,
    // with bias and GELU), so a layer is LN, QKV, attention, Wo, LN, FC1, FC2
    // with no separate reductions.  FC2's splits stay pending until the next
    // LayerNorm (or a per-layer hidden-state export).
    const bool few = af == AF_H2 && T <= GEMV_MAX_M;
    const size_t part_half = ws.part.floats / 2 / 64 * 64;
    const char *few_wo_env = getenv("CIH_FEW_WO");
    float *const part_a = ws.part.part, *const part_b = ws.part.part + part_half;
    int pend_splits = 0;  // FC2 splits waiting in part_a
    const float *pend_bias = nullptr;
    // split residual projections of the other paths defer their splits to the
    // LayerNorm after them (which writes FP32 or f16 limbs)
    const bool defer_ok = (af == AF_F32 || af == AF_H2) && d % 32 == 0 && d <= 8192;
    // K/V tile images: the QKV projection's epilogue rotates K, splits K and V
    // into f16 limbs and lays them out as attention's LDS tiles, once per
    // key; attention copies them (CIH_ATT_IMG=0: K/V as FP32 rows, staged by
    // attention itself).  Needs the LDS GEMM for the projection and the
    // f16-limb attention.
    // Other projections (GEMV, register-staged GEMMs, FP32 weights) write FP32
    // rows; from 2048 tokens on a prep kernel builds the same images from them,
    // below that attention stages K/V itself (one launch less).  All paths
    // give the same bits, so results do not depend on the batch they are in.
    // CIH_ATT_IMG=prep: images by the prep kernel at any size.
    bool use_img = false, epi_img = false;
    int tile_rows = 0;
    {
        const char *ie = getenv("CIH_ATT_IMG"), *ae = getenv("CIH_ATT");
        const bool prep_only = ie && !std::strcmp(ie, "prep");
        use_img = ws.kv_img && L > 0 && !(ie && !std::strcmp(ie, "0")) && !(ae && !std::strcmp(ae, "fp32")) &&
                  !full_range_mode() && attention_img_supported((int)m->hd);
        // the QKV epilogue has forms for head sizes 16, 32 and 64; head size 24 takes the prep kernel
        epi_img = use_img && !prep_only && af == AF_H2 && (m->hd == 16 || m->hd == 32 || m->hd == 64) &&
                  gemm_lds_applies(m->layers[0].wqkv, af, T, EPI_NONE);
        // without the epilogue, images cost a prep kernel per layer: it pays
        // from 2048 tokens on (35M B=8 ragged, head size 24: prep 8.3 us,
        // attention 38.6 -> 28.8 us per layer)
        if (!epi_img && !prep_only && T < 2048) use_img = false;
        // batches small enough for attention's split over waves stage K/V
        // there (from FP32 rows; images would take the kernel without it)
        if (!epi_img && attention_wave_split(B, S_max, H)) use_img = false;
        for (int b = 0; b < B; b++) tile_rows += (lens[b] + 31) / 32;
    }
    const int epi_qkv = m->hd == 16 ? EPI_QKV16 : (m->hd == 32 ? EPI_QKV32 : EPI_QKV64);
    QkvOut qo;
    qo.pk = ws.kv_pk;
    qo.pos = ws.kv_pos;
    qo.rc = ws.rope_c;
    qo.rs = ws.rope_s;
    qo.img = ws.kv_img;
    qo.d = d;
    qo.H = H;

    m->prof.used = 0;
    // the contact accumulator and the status word are cleared outside the
    // (possibly captured) kernel sequence
    if (want_contacts) HIPCHK(hipMemsetAsync(ws.M, 0, (size_t)B * n_max * n_max * 4, st));
    HIPCHK(hipMemsetAsync(ws.flag, 0, sizeof(int), st));

    // Everything from the embedding to the output scatters is kernel
    // launches only; a shape seen before replays a captured graph of it.
    auto enqueue = [&]() -> int {
    {
        ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * T * d);
        HIPCHK(launch_embed(ws.tokens, sm, m->emb.fmt, m->emb.q, m->emb.sc, d, V, ws.x, st, ws.flag));
    }
    if (use_img) {
        ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * T);
        HIPCHK(launch_kv_setup(sm, (int)m->hd, H, ws.kv_tb, ws.kv_pk, ws.kv_pos, ws.kv_ti, ws.kv_img, st));
    }

    for (int l = 0; l < L; l++) {
        const Layer &ly = m->layers[l];
        // probabilities: straight into the attention-map output when exported
        float *P = nullptr;
        int64_t pb = 0, ph = SS;
        const bool need_P = want_attn || want_contacts || (want_final && l == L - 1);
        if (want_attn) {
            P = t_attn + (size_t)l * H * SS;
            pb = (int64_t)L * H * SS;
        } else if (need_P) {
            P = ws.P;
            pb = (int64_t)H * SS;
        }
        if (few) {
            {
                ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * T * d);
                HIPCHK(launch_residual_layernorm(ws.x, pend_splits ? part_a : nullptr, pend_splits, pend_bias,
                                                 ly.ln1w, ly.ln1b, ws.xb, AF_H2, T, d, st));
            }
            int sq = 0;
            {
                ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * T * ly.wqkv.N * ly.wqkv.K,
                             wbytes(ly.wqkv) + 4.0 * T * d + 4.0 * T * 3 * d);
                HIPCHK(launch_gemv16_partials(ly.wqkv, (const unsigned short *)ws.xb, T, part_b, part_half, &sq, st));
            }
            // head sizes of whole 32-wide blocks: attention and Wo in one kernel
            // (each head's share of Wo, the heads as splits); CIH_FEW_WO=0: apart
            const bool fuse_wo = !need_P && m->hd % 32 == 0 && m->hd <= FEW_MAX_HD &&
                                 (ly.wo.fmt == WF_Q8 || ly.wo.fmt == WF_Q4) && (size_t)H * T * d <= part_half &&
                                 !(few_wo_env && !std::strcmp(few_wo_env, "0"));
            if (fuse_wo) {
                double fl = 0;
                for (int b = 0; b < B; b++) fl += 4.0 * (double)lens[b] * lens[b] * d;
                ProfScope ps(m, CIH_KC_ATTENTION, fl + 2.0 * T * ly.wo.N * ly.wo.K, 16.0 * T * d + wbytes(ly.wo));
                HIPCHK(launch_attention_few_wo(part_b, sq, T, ly.bqkv, ly.wo, d, H, sm, ws.rope_c, ws.rope_s, part_a,
                                               part_half, st));
            } else if (!need_P && m->hd % 8 == 0 && m->hd <= FEW_MAX_HD) {
                double fl = 0;
                for (int b = 0; b < B; b++) fl += 4.0 * (double)lens[b] * lens[b] * d;
                ProfScope ps(m, CIH_KC_ATTENTION, fl, 16.0 * T * d);
                HIPCHK(launch_attention_few(part_b, sq, T, ly.bqkv, d, H, sm, ws.rope_c, ws.rope_s, ws.ao, AF_H2, st));
            } else {
                {
                    ProfScope ps(m, CIH_KC_OTHER, 0, 4.0 * sq * T * 3 * d);
                    HIPCHK(launch_gemv16_fold(part_b, sq, T, 3 * d, ly.bqkv, ws.qkv, 3 * d, EPI_NONE, st));
                }
                double fl = 0;
                for (int b = 0; b < B; b++) fl += 4.0 * (double)lens[b] * lens[b] * d;
                ProfScope ps(m, CIH_KC_ATTENTION, fl, 16.0 * T * d);
                float *rsum = want_contacts && m->nz[l] > 0 ? ws.rowsum : nullptr;
                HIPCHK(launch_attention(ws.qkv, d, H, sm, ws.rope_c, ws.rope_s, ws.ao, af, P, pb, ph, rsum, ws.attp,
                                        ws.attp_floats, st));
            }
            if (want_contacts && m->nz[l] > 0) {
                ProfScope ps(m, CIH_KC_OTHER, 0, 0);
                HIPCHK(launch_apc_layer(P, pb, ph, H, l, m->d_contact_w, m->d_heads + (size_t)l * H, m->nz[l], sm,
                                        ws.rowsum, ws.colpart, ws.M, ws.r, st));
            }
            if (want_final && l == L - 1) {
                ProfScope ps(m, CIH_KC_OTHER, 0, 0);
                HIPCHK(launch_head_mean(P, pb, ph, H, sm, t_final, st));
            }
            int so = fuse_wo ? H : 0, s1 = 0, s2 = 0;
            if (!fuse_wo) {
                ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * T * ly.wo.N * ly.wo.K, wbytes(ly.wo) + 8.0 * T * d);
                HIPCHK(launch_gemv16_partials(ly.wo, (const unsigned short *)ws.ao, T, part_a, part_half, &so, st));
            }
            {
                ProfScope ps(m, CIH_KC_OTHER, 0, 4.0 * so * T * d + 12.0 * T * d);
                HIPCHK(launch_residual_layernorm(ws.x, part_a, so, ly.bo, ly.ln2w, ly.ln2b, ws.xb, AF_H2, T, d, st));
            }
            {
                ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * T * ly.w1.N * ly.w1.K, wbytes(ly.w1) + 4.0 * T * (d + F));
                HIPCHK(launch_gemv16_partials(ly.w1, (const unsigned short *)ws.xb, T, part_b, part_half, &s1, st));
            }
            {
                // FC2 forms GELU(FC1 + b1) from FC1's splits while staging its operand
                ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * T * ly.w2.N * ly.w2.K,
                             wbytes(ly.w2) + 4.0 * s1 * T * F + 4.0 * T * d);
                HIPCHK(launch_gemv16_gelu_partials(ly.w2, part_b, s1, ly.b1, T, part_a, part_half, &s2, st));
            }
            pend_splits = s2;
            pend_bias = ly.b2;
            if (want_layer) {
                {
                    ProfScope ps(m, CIH_KC_OTHER, 0, 4.0 * s2 * T * d + 8.0 * T * d);
                    HIPCHK(launch_gemv16_fold(part_a, s2, T, d, ly.b2, ws.x, d, EPI_RESIDUAL, st));
                }
                pend_splits = 0;
                HIPCHK(launch_scatter_rows(ws.x, d, sm, t_layer + (size_t)l * S_max * d, (int64_t)L * S_max * d, st));
            }
            continue;
        }
        {
            ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * T * d);
            if (pend_splits)
                HIPCHK(launch_residual_layernorm(ws.x, part_a, pend_splits, pend_bias, ly.ln1w, ly.ln1b, ws.xb, af, T,
                                                 d, st));
            else
                HIPCHK(launch_layernorm(ws.x, ly.ln1w, ly.ln1b, ws.xb, af, T, d, st));
        }
        if (epi_img) {
            const double bytes = wbytes(ly.wqkv) + 4.0 * T * d + 4.0 * T * 3 * d;
            ProfScope ps(m, CIH_KC_GEMM_QUANT, 2.0 * T * ly.wqkv.N * ly.wqkv.K, bytes);
            HIPCHK(launch_gemm_lds(ly.wqkv, ws.xb, ly.bqkv, ws.qkv, 3 * d, T, epi_qkv, st, &qo));
        } else {
            HIPCHK(gemm(m, ly.wqkv, ws.xb, d, af, ly.bqkv, ws.qkv, 3 * d, T, EPI_NONE));
            if (use_img) {
                ProfScope ps(m, CIH_KC_OTHER, 0, 16.0 * T * d);
                HIPCHK(launch_kv_prep(ws.qkv, d, H, ws.kv_ti, tile_rows, ws.rope_c, ws.rope_s, ws.kv_img, st));
            }
        }
        {
            double fl = 0;
            for (int b = 0; b < B; b++) fl += 4.0 * (double)lens[b] * lens[b] * d;
            ProfScope ps(m, CIH_KC_ATTENTION, fl, 16.0 * T * d);
            float *rsum = want_contacts && m->nz[l] > 0 ? ws.rowsum : nullptr;
            if (use_img)
                HIPCHK(launch_attention_img(ws.qkv, d, H, sm, ws.kv_tb, ws.kv_img, ws.rope_c, ws.rope_s, ws.ao, af, P,
                                            pb, ph, rsum, ws.attp, ws.attp_floats, st));
            else
                HIPCHK(launch_attention(ws.qkv, d, H, sm, ws.rope_c, ws.rope_s, ws.ao, af, P, pb, ph, rsum, ws.attp,
                                        ws.attp_floats, st));
        }
        if (want_contacts && m->nz[l] > 0) {
            ProfScope ps(m, CIH_KC_OTHER, 0, 0);
            HIPCHK(launch_apc_layer(P, pb, ph, H, l, m->d_contact_w, m->d_heads + (size_t)l * H, m->nz[l], sm,
                                    ws.rowsum, ws.colpart, ws.M, ws.r, st));
        }
        if (want_final && l == L - 1) {
            ProfScope ps(m, CIH_KC_OTHER, 0, 0);
            HIPCHK(launch_head_mean(P, pb, ph, H, sm, t_final, st));
        }
        // A residual projection that splits K leaves its partial sums for the
        // LayerNorm after it (k_rln adds them, the bias and the residual):
        // Wo's for LN2, FC2's for the next layer's LN1 or the final LN.
        int so = 0, s2 = 0;
        HIPCHK(gemm(m, ly.wo, ws.ao, d, af, ly.bo, ws.x, d, T, EPI_RESIDUAL, defer_ok ? &so : nullptr));
        {
            ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * T * d + 4.0 * so * T * d);
            if (so)
                HIPCHK(launch_residual_layernorm(ws.x, part_a, so, ly.bo, ly.ln2w, ly.ln2b, ws.xb, af, T, d, st));
            else
                HIPCHK(launch_layernorm(ws.x, ly.ln2w, ly.ln2b, ws.xb, af, T, d, st));
        }
        HIPCHK(gemm(m, ly.w1, ws.xb, d, af, ly.b1, ws.hbuf, F, T, epi_fc1));
        HIPCHK(gemm(m, ly.w2, ws.hbuf, F, af, ly.b2, ws.x, d, T, EPI_RESIDUAL,
                    defer_ok && !want_layer ? &s2 : nullptr));
        pend_splits = s2;
        pend_bias = ly.b2;
        if (want_layer) HIPCHK(launch_scatter_rows(ws.x, d, sm, t_layer + (size_t)l * S_max * d, (int64_t)L * S_max * d, st));
    }
    if (want_contacts) {
        ProfScope ps(m, CIH_KC_OTHER, 0, 0);
        HIPCHK(launch_apc_finalize(ws.M, ws.r, ws.coef, m->d_contact_w, L * H, sm, m->contact_b, t_contacts, n_max, st));
    }
    // final LayerNorm: state.x = LN_f(x) (lib.rs:5379-5387).  It also
    // reports a residual row that is no longer finite (the f16 limbs hold
    // |x| < 65520 only, and an overflow there makes the residual non-finite)
    // and an output the LM head's limbs cannot hold.  Without a hidden-state
    // export it hands the LM head's dense layer (FP32 weights through their
    // pair copy) f16 limbs: the split that GEMM makes of FP32 rows, so the
    // same bits, and from 64 rows on the LDS-staged kernel reads them.
    const bool lm_h2 = (want_logits || keep_logits) && m->has_head && !want_hidden && af == AF_H2 &&
                       T > GEMV_MAX_M && m->dense.fmt == WF_F32 && m->dense.p16 && m->dense.psc && d % 32 == 0;
    {
        ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * T * d);
        const int lf = lm_h2 ? AF_H2 : AF_F32;
        if (pend_splits)
            HIPCHK(launch_residual_layernorm(ws.x, part_a, pend_splits, pend_bias, m->lnfw, m->lnfb, ws.ao, lf, T, d,
                                             st, ws.flag));
        else
            HIPCHK(launch_layernorm(ws.x, m->lnfw, m->lnfb, ws.ao, lf, T, d, st, ws.flag));
    }
    if (want_hidden) HIPCHK(launch_scatter_rows(ws.ao, d, sm, t_hidden, (int64_t)S_max * d, st));
    if (want_logits || keep_logits) {
        if (m->has_head) {
            HIPCHK(gemm(m, m->dense, ws.ao, d, lm_h2 ? AF_H2 : AF_F32, m->dense_b, ws.hbuf, d, T, EPI_GELU));
            {
                ProfScope ps(m, CIH_KC_OTHER, 0, 8.0 * T * d);
                // its output feeds the decoder's GEMM, which splits it into f16 limbs
                HIPCHK(launch_layernorm(ws.hbuf, m->lm_lnw, m->lm_lnb, ws.xb, AF_F32, T, d, st, ws.flag));
            }
            HIPCHK(gemm(m, m->dec, ws.xb, d, AF_F32, m->dec_b, ws.logits, V, T, EPI_NONE));
        } else {
            HIPCHK(gemm(m, m->emb, ws.ao, d, AF_F32, nullptr, ws.logits, V, T, EPI_NONE));
        }
        if (want_logits) HIPCHK(launch_scatter_rows(ws.logits, V, sm, t_logits, (int64_t)S_max * V, st));
    }
    return 0;
    };
    if (!use_forward_graph(m)) {
        if (int rc = enqueue()) return rc;
    } else {
        // the shape fixes every grid and pointer of the sequence: batch,
        // padded length, token count, 32-key tiles, outputs and their
        // destinations
        const FwdGraphKey key{B, S_max, T, tile_rows, flags | (keep_logits ? 1u << 31 : 0u),
                              {t_logits, t_hidden, t_final, t_contacts, t_attn, t_layer}, kernel_switches()};
        hipGraphExec_t ex = nullptr;
        for (auto &g : ws.graphs)
            if (g.first == key) ex = g.second;
        if (!ex) {
            if (ws.graphs.size() >= 16) clear_graphs(ws);
            hipGraph_t g = nullptr;
            HIPCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            const int rc = enqueue();
            const hipError_t e = hipStreamEndCapture(st, &g);
            if (rc || e != hipSuccess) {
                if (g) hipGraphDestroy(g);
                return rc ? rc : set_error(CIH_ERR_HIP, "forward capture failed: %s", hipGetErrorString(e));
            }
            const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
            hipGraphDestroy(g);
            if (ei != hipSuccess) return set_error(CIH_ERR_HIP, "forward graph: %s", hipGetErrorString(ei));
            ws.graphs.emplace_back(key, ex);
        }
        HIPCHK(hipGraphLaunch(ex, st));
    }
    int *h_flag = ws.h_meta + 2 * ws.maxB;
    HIPCHK(hipMemcpyAsync(h_flag, ws.flag, sizeof(int), hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    if (*h_flag & FLAG_BAD_TOKEN) {
        m->prof.used = 0;
        return set_error(CIH_ERR_TOKEN, "a token id outside [0, %d) in the device token buffer", V);
    }
    // Non-finite residual: run the forward again in full-range mode (three
    // bf16 limbs, FP32-MFMA attention), whose results then stand, finite or
    // not, as the reference's would.
    if ((*h_flag & FLAG_NONFINITE) && !full_range_mode())
        return in_full_range([&] { return forward_impl(m, tokens, lens, B, S_max, flags, out, keep_logits); });

    if (!dev_io) {
        // Rows [0, nrows) of width floats from the device staging at src to
        // the caller's dst (same layout), the first keep(r) floats of row r
        // only (the rest is padding, left untouched): blocks of whole rows
        // are copied into pinned memory, which runs at link speed (a copy
        // into pageable memory is bounced row by row), and the kept parts of
        // each row are copied from there on the host.
        auto stage_rows = [&](float *dst, const float *src, size_t nrows, size_t width, auto keep) -> int {
            const size_t per = std::max<size_t>(1, ws.h_stage_floats / width);
            for (size_t r0 = 0; r0 < nrows; r0 += per) {
                const size_t nr = std::min(per, nrows - r0);
                HIPCHK(hipMemcpy(ws.h_stage, src + r0 * width, nr * width * 4, hipMemcpyDeviceToHost));
                for (size_t r = 0; r < nr; r++) {
                    const size_t k = keep(r0 + r);
                    if (k) std::memcpy(dst + (r0 + r) * width, ws.h_stage + r * width, k * 4);
                }
            }
            return 0;
        };
        int rc = 0;
        for (int b = 0; b < B && !rc; b++) {
            const size_t nb = lens[b];
            auto all_of = [](size_t w) { return [w](size_t) { return w; }; };
            if (want_logits)
                rc = stage_rows(out->logits + (int64_t)b * S_max * V, t_logits + (int64_t)b * S_max * V, nb, V,
                                all_of(V));
            if (!rc && want_hidden)
                rc = stage_rows(out->hidden + (int64_t)b * S_max * d, t_hidden + (int64_t)b * S_max * d, nb, d,
                                all_of(d));
            if (!rc && want_final)
                rc = stage_rows(out->final_att + b * SS, t_final + b * SS, nb, S_max, all_of(nb));
            if (!rc && want_contacts && nb > 2) {
                const size_t nr = nb - 2, nn = (size_t)n_max * n_max;
                rc = stage_rows(out->contacts + b * nn, t_contacts + b * nn, nr, n_max, all_of(nr));
            }
            // a sequence's per-layer rows and maps are contiguous: [L][S_max][d], [L][H][S_max][S_max]
            if (!rc && want_layer) {
                const int64_t o = (int64_t)b * L * S_max * d;
                rc = stage_rows(out->layer_hidden + o, t_layer + o, (size_t)L * S_max, d,
                                [&](size_t r) { return r % S_max < nb ? (size_t)d : 0; });
            }
            if (!rc && want_attn) {
                const int64_t o = (int64_t)b * L * H * SS;
                rc = stage_rows(out->attn + o, t_attn + o, (size_t)L * H * S_max, S_max,
                                [&](size_t r) { return r % S_max < nb ? nb : 0; });
            }
        }
        if (rc) return rc;
    }
    profile_collect(m);
    return CIH_OK;
}

// Scores `count` positions whose logits are rows meta[2i] of ws.logits and
// copies deltas / entropy to dst_d[idx[i]][20], dst_e[idx[i]].
int dms_score_rows(cih_model *m, const std::vector<int> &meta, const std::vector<int> &idx, float *dst_d,
                   float *dst_e) {
    Workspace &ws = m->ws;
    const int count = (int)idx.size();
    if (count == 0) return CIH_OK;
    std::vector<float> h((size_t)count * 21);
    HIPCHK(hipMemcpyAsync(ws.dms_meta, meta.data(), (size_t)count * 2 * sizeof(int), hipMemcpyHostToDevice, m->stream));
    HIPCHK(launch_dms_score(ws.logits, m->cfg.vocab_size, ws.dms_meta, count, ws.dms_out, m->stream));
    HIPCHK(hipMemcpyAsync(h.data(), ws.dms_out, h.size() * sizeof(float), hipMemcpyDeviceToHost, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    for (int i = 0; i < count; i++) {
        std::memcpy(dst_d + (size_t)idx[i] * 20, &h[(size_t)i * 21], 20 * sizeof(float));
        dst_e[idx[i]] = h[(size_t)i * 21 + 20];
    }
    return CIH_OK;
}

}  // namespace

extern "C" {

int cih_forward(cih_model *m, const int32_t *tokens, const int32_t *lens, int32_t B, int32_t S_max, uint32_t flags,
                const cih_outputs *out) {
    return forward_impl(m, tokens, lens, B, S_max, flags, out, false);
}

int cih_dms(cih_model *m, const int32_t *residues, int32_t n, int32_t window, int32_t stride, int32_t mode,
            int32_t chunk, float *deltas, float *entropy) {
    if (!m || !residues || !deltas || !entropy) return set_error(CIH_ERR_ARG, "null argument");
    if (n < 1) return set_error(CIH_ERR_ARG, "the sequence is empty");
    if (mode != CIH_DMS_MASKED_MARGINAL && mode != CIH_DMS_WILDTYPE_MARGINAL) return set_error(CIH_ERR_ARG, "bad mode");
    Workspace &ws = m->ws;
    if (ws.maxB == 0) return set_error(CIH_ERR_CAPACITY, "cih_model_reserve has not been called");
    const int V = m->cfg.vocab_size;
    for (int i = 0; i < n; i++)
        if (residues[i] < 0 || residues[i] >= V)
            return set_error(CIH_ERR_TOKEN, "residue token %d at %d outside [0, %d)", residues[i], i, V);
    // window of the scan (pipeline.rs:87-91)
    const int max_len = m->cfg.max_seq_len;
    const int aw = (n <= window || window == 0) ? std::min(n, max_len) : std::min(window, max_len);
    if (aw + 2 > ws.maxS)
        return set_error(CIH_ERR_CAPACITY, "the scan's windows need max_seq_len >= %d (reserved %d)", aw + 2, ws.maxS);
    const int S = aw + 2;
    const cih_outputs none{};
    std::vector<int32_t> toks, lens;
    std::vector<int> meta, idx;
    if (mode == CIH_DMS_MASKED_MARGINAL) {
        // one masked copy per position, window centred on it (pipeline.rs:111-122)
        const int cb = (chunk <= 0 || chunk > ws.maxB) ? ws.maxB : chunk, half = aw / 2;
        for (int p0 = 0; p0 < n; p0 += cb) {
            const int B = std::min(cb, n - p0);
            toks.assign((size_t)B * S, 0);
            lens.assign(B, 0);
            meta.clear();
            idx.clear();
            int row0 = 0;
            for (int b = 0; b < B; b++) {
                const int p = p0 + b;
                const int w0 = p < half ? 0 : (p + half > n ? std::max(n - aw, 0) : p - half);
                const int w1 = std::min(w0 + aw, n);
                int32_t *t = &toks[(size_t)b * S];
                t[0] = 0;
                for (int i = w0; i < w1; i++) t[1 + i - w0] = residues[i];
                t[1 + w1 - w0] = 2;
                lens[b] = w1 - w0 + 2;
                const int tp = p - w0 + 1;
                meta.push_back(row0 + tp);
                meta.push_back(t[tp]);
                idx.push_back(p);
                t[tp] = 32;  // <mask>
                row0 += lens[b];
            }
            if (int rc = forward_impl(m, toks.data(), lens.data(), B, S, 0, &none, true)) return rc;
            if (int rc = dms_score_rows(m, meta, idx, deltas, entropy)) return rc;
        }
        return CIH_OK;
    }
    // wild-type marginal: one unmasked forward per window (pipeline.rs:196-265)
    const int step = (stride > 0 && stride <= aw) ? stride : std::max(aw / 2, 1);
    int covered = 0, w0 = 0;
    while (covered < n) {
        const int w1 = std::min(w0 + aw, n);
        toks.assign(S, 0);
        toks[0] = 0;
        for (int i = w0; i < w1; i++) toks[1 + i - w0] = residues[i];
        toks[1 + w1 - w0] = 2;
        lens.assign(1, w1 - w0 + 2);
        meta.clear();
        idx.clear();
        for (int p = covered; p < w1; p++) {
            meta.push_back(p - w0 + 1);
            meta.push_back(residues[p]);
            idx.push_back(p);
        }
        if (int rc = forward_impl(m, toks.data(), lens.data(), 1, S, 0, &none, true)) return rc;
        if (int rc = dms_score_rows(m, meta, idx, deltas, entropy)) return rc;
        covered = w1;
        if (w1 >= n) break;
        w0 = std::min(w0 + step, std::max(n - aw, 0));
    }
    return CIH_OK;
}

int cih_profile_enable(cih_model *m, int32_t enable) {
    if (!m) return set_error(CIH_ERR_ARG, "null model");
    // enabling starts a new measurement; disabling keeps the totals readable
    if (enable && !m->prof.on)
        for (auto &s : m->prof.st) s = cih_kernel_stats{};
    m->prof.on = enable != 0;
    return CIH_OK;
}

int cih_profile_read(const cih_model *m, int32_t kc, cih_kernel_stats *out) {
    if (!m || !out || kc < 0 || kc >= CIH_KC_COUNT) return set_error(CIH_ERR_ARG, "bad argument");
    *out = m->prof.st[kc];
    return CIH_OK;
}

// ---- kernel-level entry points ------------------------------------------------

int cih_matmul_tiled(int32_t dtype, float *out, const float *x, const void *w, const float *bias, int32_t in_dim,
                     int32_t out_dim, int32_t seq_len) {
    if (!out || !x || !w || !bias) return set_error(CIH_ERR_ARG, "null argument");
    if (in_dim <= 0 || out_dim <= 0 || seq_len < 0 || in_dim % 32)
        return set_error(CIH_ERR_SHAPE, "bad GEMM shape %d x %d x %d", seq_len, out_dim, in_dim);
    if (dtype != DT_FP32 && dtype != DT_Q8 && dtype != DT_Q4) return set_error(CIH_ERR_ARG, "bad dtype");
    if (seq_len == 0) return CIH_OK;
    cih_model tmp;  // owns the temporary allocations
    int rc = upload_matrix(&tmp, dtype, dtype, in_dim, {{w, out_dim}}, tmp.emb);
    float *dx = nullptr, *db = nullptr, *dy = nullptr;
    if (!rc) rc = upload(&tmp, dx, x, (size_t)seq_len * in_dim);
    if (!rc) rc = upload(&tmp, db, bias, (size_t)out_dim);
    if (!rc && dalloc(dy, (size_t)seq_len * out_dim, tmp.allocs) != hipSuccess)
        rc = set_error(CIH_ERR_HIP, "allocation failed");
    PartialBuf gs;
    // a few rows of quantized weights: limbs (in the partial-sum buffer) and the f16-MFMA GEMV
    const bool g16 = dtype != DT_FP32 && gemv16_applies(tmp.emb, AF_H2, seq_len, EPI_NONE);
    const bool gv = use_gemv(seq_len, AF_F32, EPI_NONE);
    gs.floats = std::max({gemv_part_floats(out_dim, in_dim), SPLITK_PART_FLOATS, (size_t)seq_len * in_dim});
    if (!rc && dalloc(gs.part, gs.floats, tmp.allocs) != hipSuccess) rc = set_error(CIH_ERR_HIP, "allocation failed");
    if (!rc) {
        unsigned short *xh = reinterpret_cast<unsigned short *>(gs.part);
        hipError_t e = g16   ? launch_to_h2(dx, seq_len, in_dim, xh, nullptr)
                       : gv  ? launch_gemv(tmp.emb, dx, in_dim, seq_len, db, dy, out_dim, EPI_NONE, gs, nullptr)
                             : launch_gemm(tmp.emb, dx, in_dim, AF_F32, db, dy, out_dim, seq_len, EPI_NONE, &gs, nullptr);
        if (g16 && e == hipSuccess) {
            PartialBuf rest{gs.part + (size_t)seq_len * in_dim, gs.floats - (size_t)seq_len * in_dim};
            e = launch_gemv16(tmp.emb, xh, seq_len, db, dy, out_dim, EPI_NONE, &rest, nullptr);
        }
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e == hipSuccess) e = hipMemcpy(out, dy, (size_t)seq_len * out_dim * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = set_error(CIH_ERR_HIP, "GEMM failed: %s", hipGetErrorString(e));
    }
    free_list(tmp.allocs);
    return rc;
}

int cih_dequantize_device(int32_t dtype, const void *blocks, int64_t nblocks, float *out) {
    if (!blocks || !out || nblocks < 0) return set_error(CIH_ERR_ARG, "bad argument");
    if (dtype != DT_Q8 && dtype != DT_Q4) return set_error(CIH_ERR_ARG, "dtype must be Q8_0 or Q4_0");
    if (nblocks == 0) return CIH_OK;
    if (nblocks > INT32_MAX / 32) return set_error(CIH_ERR_SHAPE, "too many blocks");
    // one row of nblocks blocks: K = 32 * nblocks, N = 1
    cih_model tmp;
    int rc = upload_matrix(&tmp, dtype, dtype, (int)(nblocks * 32), {{blocks, 1}}, tmp.emb);
    float *dy = nullptr;
    if (!rc && dalloc(dy, (size_t)nblocks * 32, tmp.allocs) != hipSuccess) rc = set_error(CIH_ERR_HIP, "alloc failed");
    if (!rc) {
        hipError_t e = launch_dequant(tmp.emb, dy, nullptr);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e == hipSuccess) e = hipMemcpy(out, dy, (size_t)nblocks * 32 * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = set_error(CIH_ERR_HIP, "dequantize failed: %s", hipGetErrorString(e));
    }
    free_list(tmp.allocs);
    return rc;
}

int cih_quantize_device(int32_t dtype, const float *src, int64_t n, void *dst) {
    if (!src || !dst || n < 0 || n % 32) return set_error(CIH_ERR_ARG, "n must be a non-negative multiple of 32");
    if (dtype != DT_Q8 && dtype != DT_Q4) return set_error(CIH_ERR_ARG, "dtype must be Q8_0 or Q4_0");
    if (n == 0) return CIH_OK;
    if (n > INT32_MAX / 32 * 32) return set_error(CIH_ERR_SHAPE, "too many values");
    // one row of n values quantized by the loader's kernel: qs [n/32][1][qb], sc [n/32]
    cih_model tmp;
    int rc = upload_matrix(&tmp, DT_FP32, dtype, (int)n, {{src, 1}}, tmp.emb);
    const int64_t nb = n / 32, qb = block_bytes(dtype) - 4;
    std::vector<uint8_t> qs(nb * qb);
    std::vector<float> sc(nb);
    if (!rc) {
        hipError_t e = hipMemcpy(qs.data(), tmp.emb.q, qs.size(), hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(sc.data(), tmp.emb.sc, nb * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = set_error(CIH_ERR_HIP, "quantize failed: %s", hipGetErrorString(e));
    }
    free_list(tmp.allocs);
    if (rc) return rc;
    uint8_t *o = (uint8_t *)dst;
    for (int64_t b = 0; b < nb; b++) {
        std::memcpy(o + b * (qb + 4), &sc[b], 4);
        std::memcpy(o + b * (qb + 4) + 4, &qs[b * qb], qb);
    }
    return CIH_OK;
}

// ---- host helpers ----------------------------------------------------------------

int cih_quantize_q8(const float *src, int64_t n, void *dst) {
    if (!src || !dst || n < 0 || n % 32) return set_error(CIH_ERR_ARG, "n must be a non-negative multiple of 32");
    quantize_matrix(DT_Q8, src, n, (uint8_t *)dst);
    return CIH_OK;
}

int cih_quantize_q4(const float *src, int64_t n, void *dst) {
    if (!src || !dst || n < 0 || n % 32) return set_error(CIH_ERR_ARG, "n must be a non-negative multiple of 32");
    quantize_matrix(DT_Q4, src, n, (uint8_t *)dst);
    return CIH_OK;
}

int cih_dequantize_q8(const void *blocks, int64_t nblocks, float *dst) {
    if (!blocks || !dst || nblocks < 0) return set_error(CIH_ERR_ARG, "bad argument");
    for (int64_t b = 0; b < nblocks; b++) dequantize_q8_block((const uint8_t *)blocks + b * 36, dst + b * 32);
    return CIH_OK;
}

int cih_dequantize_q4(const void *blocks, int64_t nblocks, float *dst) {
    if (!blocks || !dst || nblocks < 0) return set_error(CIH_ERR_ARG, "bad argument");
    for (int64_t b = 0; b < nblocks; b++) dequantize_q4_block((const uint8_t *)blocks + b * 20, dst + b * 32);
    return CIH_OK;
}

int cih_tokenize(const char *text, int32_t *out, int32_t cap) {
    if (!text || !out) return set_error(CIH_ERR_ARG, "null argument");
    const int n = tokenize(text, out, cap);
    return n < 0 ? set_error(CIH_ERR_ARG, "output capacity %d too small", cap) : n;
}

int cih_log_softmax_canonical(const float *logits, float *out33) {
    if (!logits || !out33) return set_error(CIH_ERR_ARG, "null argument");
    log_softmax_canonical(logits, out33);
    return CIH_OK;
}

}  // extern "C"
