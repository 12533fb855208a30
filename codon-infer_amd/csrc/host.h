// Internal host-side declarations shared by formats.cpp and api.cpp.
#pragma once
#include <stdint.h>

#include <algorithm>
#include <functional>
#include <thread>
#include <vector>

#include "../../include/codon_hip.h"

namespace cih {

enum { DT_FP32 = CIH_DTYPE_FP32, DT_Q8 = CIH_DTYPE_Q8_0, DT_Q4 = CIH_DTYPE_Q4_0 };

inline int block_bytes(int dtype) {
    return dtype == DT_Q8 ? CIH_Q8_0_BLOCK_BYTES : (dtype == DT_Q4 ? CIH_Q4_0_BLOCK_BYTES : 0);
}

// Records a message for cih_last_error() and returns code.
int set_error(int code, const char *fmt, ...);

// Splits [0, n) into contiguous chunks over up to 16 host threads.
template <class F>
void parallel_for(int64_t n, F fn) {
    const int64_t min_chunk = 1 << 14;
    int nt = (int)std::min<int64_t>(16, std::max<int64_t>(1, n / min_chunk));
    nt = std::min<int>(nt, (int)std::max(1u, std::thread::hardware_concurrency()));
    if (nt <= 1) { fn(0, n); return; }
    std::vector<std::thread> th;
    const int64_t chunk = (n + nt - 1) / nt;
    for (int t = 0; t < nt; t++) {
        const int64_t a = t * chunk, b = std::min(n, a + chunk);
        if (a < b) th.emplace_back([=, &fn] { fn(a, b); });
    }
    for (auto &t : th) t.join();
}

void quantize_q8_block(const float *x, uint8_t *blk);
void quantize_q4_block(const float *x, uint8_t *blk);
void dequantize_q8_block(const uint8_t *blk, float *out);
void dequantize_q4_block(const uint8_t *blk, float *out);
void quantize_matrix(int dtype, const float *src, int64_t n, uint8_t *dst);
int tokenize(const char *text, int32_t *out, int32_t cap);
void log_softmax_canonical(const float *logits, float *out33);

}  // namespace cih
