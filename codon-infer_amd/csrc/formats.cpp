// Host-side formats: Q8_0 / Q4_0 block quantizers, the tokenizer, the
// canonical log-softmax and the weight-file reader (CODQ header, FP32
// grouped_canonical_v1 / sequential_hf layouts).  Pure host code.
#include "host.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>

namespace cih {

// ---- Q8_0: BlockQ8_0::quantize (codon-infer src/lib.rs:648-660) ----------
// d = absmax / 127; id = d == 0 ? 0 : 1/d; q = clamp(round(x*id), -127, 127),
// round half away from zero; NaN quantizes to 0 (Rust's `NaN as i8`).
void quantize_q8_block(const float *x, uint8_t *blk) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = std::fabs(x[i]) > amax ? std::fabs(x[i]) : amax;
    const float d = amax / 127.0f;
    const float id = d == 0.0f ? 0.0f : 1.0f / d;
    std::memcpy(blk, &d, 4);
    for (int i = 0; i < 32; i++) {
        float r = std::round(x[i] * id);
        int8_t q = 0;
        if (!std::isnan(r)) q = (int8_t)(r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r));
        blk[4 + i] = (uint8_t)q;
    }
}

// ---- Q4_0: BlockQ4_0::quantize (lib.rs:1054-1071, docs/Q4_0_SPEC.md:42-81)
// max = first element of largest |x| (keeps its sign); d = max / -8;
// q = clamp(round(x*id) + 8, 0, 15); byte j = q_j | q_{j+16} << 4.
static inline long long sat_i32(float f) {
    if (std::isnan(f)) return 0;
    if (f >= 2147483647.0f) return 2147483647LL;
    if (f <= -2147483648.0f) return -2147483648LL;
    return (long long)f;
}

void quantize_q4_block(const float *x, uint8_t *blk) {
    float mx = 0.0f;
    for (int i = 0; i < 32; i++)
        if (std::fabs(x[i]) > std::fabs(mx)) mx = x[i];
    const float d = mx == 0.0f ? 0.0f : mx / -8.0f;
    const float id = d == 0.0f ? 0.0f : 1.0f / d;
    std::memcpy(blk, &d, 4);
    for (int j = 0; j < 16; j++) {
        long long lo = sat_i32(std::round(x[j] * id)) + 8, hi = sat_i32(std::round(x[j + 16] * id)) + 8;
        lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
        hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
        blk[4 + j] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
    }
}

void dequantize_q8_block(const uint8_t *blk, float *out) {
    float d;
    std::memcpy(&d, blk, 4);
    for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)blk[4 + i] * d;
}

void dequantize_q4_block(const uint8_t *blk, float *out) {
    float d;
    std::memcpy(&d, blk, 4);
    for (int j = 0; j < 16; j++) {
        out[j] = (float)((int)(blk[4 + j] & 0xF) - 8) * d;
        out[j + 16] = (float)((int)(blk[4 + j] >> 4) - 8) * d;
    }
}

void quantize_matrix(int dtype, const float *src, int64_t n, uint8_t *dst) {
    const int bb = block_bytes(dtype);
    parallel_for(n / 32, [&](int64_t b0, int64_t b1) {
        for (int64_t b = b0; b < b1; b++) {
            if (dtype == DT_Q8) quantize_q8_block(src + b * 32, dst + b * bb);
            else quantize_q4_block(src + b * 32, dst + b * bb);
        }
    });
}

// ---- Tokenizer::encode (lib.rs:6511-6521) ---------------------------------
static int aa_id(unsigned c) {
    static const char *aas = "LAGVSERTIDPKQNFYMHWC";
    for (int i = 0; i < 20; i++)
        if ((unsigned)aas[i] == c) return 4 + i;
    switch (c) {
    case 'X': return 24; case 'B': return 25; case 'U': return 26; case 'Z': return 27;
    case 'O': return 28; case '.': return 29; case '-': return 30; case '*': return 32;
    default: return 3;
    }
}

int tokenize(const char *text, int32_t *out, int32_t cap) {
    // <cls>, then one id per Unicode scalar value ("<mask_1>"/"<mask>" -> 32), <eos>
    int n = 0;
    if (cap < 2) return -1;
    out[n++] = 0;
    const unsigned char *s = (const unsigned char *)text;
    while (*s) {
        int id;
        if (!std::strncmp((const char *)s, "<mask_1>", 8)) { id = 32; s += 8; }
        else if (!std::strncmp((const char *)s, "<mask>", 6)) { id = 32; s += 6; }
        else {
            const unsigned c = *s;
            const int len = c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : c >= 0xC0 ? 2 : 1;
            id = len == 1 ? aa_id(c) : 3;
            for (int i = 0; i < len && *s; i++) s++;
        }
        if (n + 1 >= cap) return -1;
        out[n++] = id;
    }
    out[n++] = 2;
    return n;
}

// ---- log_softmax_canonical (lib.rs:4426-4441): ids 4..=23 only -------------
void log_softmax_canonical(const float *logits, float *out) {
    for (int i = 0; i < 33; i++) out[i] = -INFINITY;
    float m = -INFINITY;
    for (int i = 4; i <= 23; i++) m = logits[i] > m ? logits[i] : m;
    float s = 0.0f;
    for (int i = 4; i <= 23; i++) s += std::exp(logits[i] - m);
    const float lse = m + std::log(s);
    for (int i = 4; i <= 23; i++) out[i] = logits[i] - lse;
}

// ---- weight files ----------------------------------------------------------
// EsmConfig presets (lib.rs:86-145) and CODQ arch ids (lib.rs:878-882).
static const struct { int arch; cih_config cfg; } kPresets[] = {
    {0, {320, 1280, 6, 20, 33, 1024}},   {1, {480, 1920, 12, 20, 33, 1024}},
    {2, {640, 2560, 30, 20, 33, 1024}},  {3, {1280, 5120, 33, 20, 33, 1024}},
    {4, {2560, 10240, 36, 40, 33, 1024}},
};

static int64_t lm_head_floats(const cih_config &c) {
    return 3LL * c.dim + (int64_t)c.dim * c.dim + (int64_t)c.vocab_size * c.dim + c.vocab_size;
}

// grouped_canonical_floats (lib.rs:195-204)
static int64_t grouped_floats(const cih_config &c) {
    const int64_t d = c.dim, F = c.hidden_dim;
    return (int64_t)c.vocab_size * d + (int64_t)c.n_layers * (4 * d * d + 9 * d + 2 * d * F + F) + 2 * d +
           lm_head_floats(c);
}

// sequential_hf_floats (lib.rs:212-218): + inv_freq + contact head
static int64_t sequential_floats(const cih_config &c) {
    return grouped_floats(c) + (c.dim / c.n_heads) / 2 + (int64_t)c.n_layers * c.n_heads + 1;
}

namespace {
struct Reader {
    FILE *f = nullptr;
    ~Reader() { if (f) std::fclose(f); }
    bool floats(std::vector<float> &v, int64_t n) {
        v.resize(n);
        return n == 0 || std::fread(v.data(), 4, n, f) == (size_t)n;
    }
    bool bytes(std::vector<uint8_t> &v, int64_t n) {
        v.resize(n);
        return n == 0 || std::fread(v.data(), 1, n, f) == (size_t)n;
    }
};
}  // namespace

// EsmWeights::from_file FP32 layouts (lib.rs:310-547) after an optional
// 64-byte CODQ header.  Both grouped_canonical_v1 and sequential_hf are
// accepted by exact byte count.
static int read_fp32_body(Reader &r, int64_t remaining, const cih_config &c, HostModel &hm) {
    const int64_t d = c.dim, F = c.hidden_dim, L = c.n_layers, V = c.vocab_size;
    if (remaining % 4) return set_error(CIH_ERR_FORMAT, "unaligned trailing bytes: %lld", (long long)remaining);
    const int64_t nf = remaining / 4;
    hm.dtype = DT_FP32;
    auto &t = hm.f;
    if (nf == grouped_floats(c)) {
        bool ok = r.floats(t.emb, V * d) && r.floats(t.ln1w, L * d) && r.floats(t.ln1b, L * d) &&
                  r.floats(t.wq, L * d * d) && r.floats(t.bq, L * d) && r.floats(t.wk, L * d * d) &&
                  r.floats(t.bk, L * d) && r.floats(t.wv, L * d * d) && r.floats(t.bv, L * d) &&
                  r.floats(t.wo, L * d * d) && r.floats(t.bo, L * d) && r.floats(t.ln2w, L * d) &&
                  r.floats(t.ln2b, L * d) && r.floats(t.fc1, L * F * d) && r.floats(t.fc1b, L * F) &&
                  r.floats(t.fc2, L * d * F) && r.floats(t.fc2b, L * d) && r.floats(t.lnfw, d) &&
                  r.floats(t.lnfb, d) && r.floats(t.cls, lm_head_floats(c));
        return ok ? 0 : set_error(CIH_ERR_IO, "short read in grouped_canonical_v1 body");
    }
    if (nf == sequential_floats(c)) {
        // per layer: wq bq wk bk wv bv wo bo ln1w ln1b fc1 fc1b fc2 fc2b ln2w ln2b (lib.rs:396-499)
        std::vector<float> tmp;
        if (!r.floats(t.emb, V * d) || !r.floats(tmp, (d / c.n_heads) / 2)) return set_error(CIH_ERR_IO, "short read");
        t.ln1w.resize(L * d); t.ln1b.resize(L * d); t.wq.resize(L * d * d); t.bq.resize(L * d);
        t.wk.resize(L * d * d); t.bk.resize(L * d); t.wv.resize(L * d * d); t.bv.resize(L * d);
        t.wo.resize(L * d * d); t.bo.resize(L * d); t.ln2w.resize(L * d); t.ln2b.resize(L * d);
        t.fc1.resize(L * F * d); t.fc1b.resize(L * F); t.fc2.resize(L * d * F); t.fc2b.resize(L * d);
        auto rd = [&](std::vector<float> &dst, int64_t off, int64_t n) {
            return n == 0 || std::fread(dst.data() + off, 4, n, r.f) == (size_t)n;
        };
        for (int64_t l = 0; l < L; l++) {
            bool ok = rd(t.wq, l * d * d, d * d) && rd(t.bq, l * d, d) && rd(t.wk, l * d * d, d * d) &&
                      rd(t.bk, l * d, d) && rd(t.wv, l * d * d, d * d) && rd(t.bv, l * d, d) &&
                      rd(t.wo, l * d * d, d * d) && rd(t.bo, l * d, d) && rd(t.ln1w, l * d, d) &&
                      rd(t.ln1b, l * d, d) && rd(t.fc1, l * F * d, F * d) && rd(t.fc1b, l * F, F) &&
                      rd(t.fc2, l * d * F, d * F) && rd(t.fc2b, l * d, d) && rd(t.ln2w, l * d, d) &&
                      rd(t.ln2b, l * d, d);
            if (!ok) return set_error(CIH_ERR_IO, "short read in sequential_hf layer %lld", (long long)l);
        }
        std::vector<float> lm_bias, dw, db, lw, lb, decw;
        bool ok = r.floats(t.lnfw, d) && r.floats(t.lnfb, d) && r.floats(tmp, L * c.n_heads + 1) &&
                  r.floats(lm_bias, V) && r.floats(dw, d * d) && r.floats(db, d) && r.floats(lw, d) &&
                  r.floats(lb, d) && r.floats(decw, V * d);
        if (!ok) return set_error(CIH_ERR_IO, "short read in sequential_hf head");
        t.cls.clear();
        for (auto *v : {&lw, &lb, &dw, &db, &decw, &lm_bias}) t.cls.insert(t.cls.end(), v->begin(), v->end());
        return 0;
    }
    return set_error(CIH_ERR_FORMAT,
                     "invalid FP32 weights size: %lld floats, expected %lld (grouped_canonical_v1) or %lld "
                     "(sequential_hf)",
                     (long long)nf, (long long)grouped_floats(c), (long long)sequential_floats(c));
}

// EsmWeightsQ8::from_file / EsmWeightsQ4::from_file (lib.rs:744-830,
// 1156-1242): blocks and floats in field order; the classifier is whatever
// floats remain.
static int read_quant_body(Reader &r, int64_t remaining, const cih_config &c, int dtype, HostModel &hm) {
    const int64_t d = c.dim, F = c.hidden_dim, L = c.n_layers, V = c.vocab_size;
    const int64_t bb = block_bytes(dtype);
    hm.dtype = dtype;
    auto &t = hm.f;
    auto &q = hm.q;
    int64_t used = 0;
    auto qb = [&](std::vector<uint8_t> &v, int64_t elems) {
        used += elems / 32 * bb;
        return r.bytes(v, elems / 32 * bb);
    };
    auto fl = [&](std::vector<float> &v, int64_t n) {
        used += n * 4;
        return r.floats(v, n);
    };
    bool ok = (dtype == DT_Q8 ? qb(q.emb, V * d) : fl(t.emb, V * d)) && fl(t.ln1w, L * d) && fl(t.ln1b, L * d) &&
              qb(q.wq, L * d * d) && fl(t.bq, L * d) && qb(q.wk, L * d * d) && fl(t.bk, L * d) &&
              qb(q.wv, L * d * d) && fl(t.bv, L * d) && qb(q.wo, L * d * d) && fl(t.bo, L * d) &&
              fl(t.ln2w, L * d) && fl(t.ln2b, L * d) && qb(q.fc1, L * F * d) && fl(t.fc1b, L * F) &&
              qb(q.fc2, L * d * F) && fl(t.fc2b, L * d) && fl(t.lnfw, d) && fl(t.lnfb, d);
    if (!ok || used > remaining) return set_error(CIH_ERR_IO, "short read in quantized weights body");
    const int64_t rest = remaining - used;
    if (rest % 4) return set_error(CIH_ERR_FORMAT, "unaligned trailing bytes: %lld", (long long)rest);
    if (!r.floats(t.cls, rest / 4)) return set_error(CIH_ERR_IO, "short read in classifier");
    return 0;
}

int load_file(const char *path, HostModel &hm) {
    Reader r;
    r.f = std::fopen(path, "rb");
    if (!r.f) return set_error(CIH_ERR_IO, "cannot open %s", path);
    std::fseek(r.f, 0, SEEK_END);
    const int64_t flen = std::ftell(r.f);
    std::fseek(r.f, 0, SEEK_SET);
    unsigned char hdr[64] = {0};
    const bool has_hdr = flen >= 64 && std::fread(hdr, 1, 64, r.f) == 64 && !std::memcmp(hdr, "CODQ", 4);
    if (has_hdr) {
        // CodqHeader (lib.rs:887-898): magic, version, dtype, arch, n_layers, dim, hidden, vocab, 32 reserved
        uint32_t h[8];
        std::memcpy(h, hdr, 32);
        if (h[1] != 1) return set_error(CIH_ERR_FORMAT, "unsupported CODQ version %u", h[1]);
        if (h[3] > 4) return set_error(CIH_ERR_FORMAT, "unknown CODQ arch id %u", h[3]);
        const cih_config &c = kPresets[h[3]].cfg;
        if ((int)h[4] != c.n_layers || (int)h[5] != c.dim || (int)h[6] != c.hidden_dim || (int)h[7] != c.vocab_size)
            return set_error(CIH_ERR_FORMAT, "incoherent CODQ dimensions for arch %u", h[3]);
        hm.cfg = c;
        if (h[2] == DT_FP32) return read_fp32_body(r, flen - 64, c, hm);
        if (h[2] == DT_Q8 || h[2] == DT_Q4) return read_quant_body(r, flen - 64, c, (int)h[2], hm);
        return set_error(CIH_ERR_FORMAT, "unsupported CODQ dtype %u", h[2]);
    }
    std::fseek(r.f, 0, SEEK_SET);
    for (const auto &p : kPresets) {
        if (flen == grouped_floats(p.cfg) * 4 || flen == sequential_floats(p.cfg) * 4) {
            hm.cfg = p.cfg;
            return read_fp32_body(r, flen, p.cfg, hm);
        }
    }
    return set_error(CIH_ERR_FORMAT, "unrecognized weights file %s (%lld bytes): no CODQ header and not an exact "
                                     "FP32 ESM-2 size", path, (long long)flen);
}

void quantize_host_model(HostModel &hm, int dtype) {
    const cih_config &c = hm.cfg;
    const int64_t d = c.dim, F = c.hidden_dim, L = c.n_layers, V = c.vocab_size;
    const int64_t bb = block_bytes(dtype);
    auto qz = [&](std::vector<float> &src, std::vector<uint8_t> &dst) {
        dst.resize(src.size() / 32 * bb);
        quantize_matrix(dtype, src.data(), (int64_t)src.size(), dst.data());
        std::vector<float>().swap(src);
    };
    (void)d; (void)F; (void)L; (void)V;
    qz(hm.f.wq, hm.q.wq); qz(hm.f.wk, hm.q.wk); qz(hm.f.wv, hm.q.wv); qz(hm.f.wo, hm.q.wo);
    qz(hm.f.fc1, hm.q.fc1); qz(hm.f.fc2, hm.q.fc2);
    if (dtype == DT_Q8) qz(hm.f.emb, hm.q.emb);  // the Q8 model quantizes the embedding (lib.rs:561)
    hm.dtype = dtype;
}

}  // namespace cih
