// Host-side formats: Q8_0 / Q4_0 block quantizers, the tokenizer and the
// canonical log-softmax.  Pure host code.
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

}  // namespace cih
