// One attention head's share of the output projection Wo for a few rows
// (the head's output o, FP32, already in LDS): Wo's k-blocks of the head
// times o, on v_mfma_f32_16x16x32_f16 as k_gemv16 multiplies (A row =
// token + 8 limb, lane l holds A[l % 16][8 (l / 16) ..]; B = the quants of
// 16 columns as f16 integers; each block's sum times its scale).  For heads
// of whole 32-wide blocks (hd = 32 nkb, nkb <= HW_KB), 512 threads, P passes
// of 8 waves x 16 columns.
#pragma once

#include "kernels.h"
#include "x3.h"

namespace cih {

constexpr int HW_KB = FEW_MAX_HD / 32;  // k-blocks of a head, at most

template <int WF, int P> struct HeadWo {
    typedef unsigned u2_t __attribute__((ext_vector_type(2)));
    u2_t wq[P][HW_KB];
    float dsc[P][HW_KB];

    // weights and scales of columns [c0, c1) of k-blocks kb0 .. kb0 + nkb - 1,
    // pass p covering c0 + 128 p + [0, 128); columns past c1 re-read column
    // c1 - 1 (never stored)
    __device__ __forceinline__ void load(const unsigned char *__restrict__ Wq, const float *__restrict__ Wsc, int N,
                                         int kb0, int nkb, int c0, int c1) {
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            const int col = min(c0 + 128 * ps + 16 * w + c16, c1 - 1);
#pragma unroll
            for (int k = 0; k < HW_KB; k++) {
                if (k >= nkb) continue;
                const size_t blk = (size_t)(kb0 + k) * N + col;
                if constexpr (WF == WF_Q8) wq[ps][k] = *reinterpret_cast<const u2_t *>(Wq + blk * 32 + 8 * g);
                else wq[ps][k] = *reinterpret_cast<const u2_t *>(Wq + blk * 16 + 8 * (g & 1));
                dsc[ps][k] = Wsc[blk];
            }
        }
    }

    // rows t < n of o (o + t ldo, FP32 in LDS) times the loaded columns:
    // dst[t N + col] for col in [c0, c1)
    __device__ __forceinline__ void run(const float *o, int ldo, int n, int nkb, int N, int c0, int c1,
                                        float *__restrict__ dst) const {
        typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
        typedef unsigned u4_t __attribute__((ext_vector_type(4)));
        typedef float f4_t __attribute__((ext_vector_type(4)));
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
        // the operand: row c16 = token (c16 & 7) limb (c16 >> 3), dims 32 k + 8 g + e
        h8_t xa[HW_KB];
        const int tok = min(c16 & 7, n - 1), limb = c16 >> 3;
        const float *orow = o + (size_t)tok * ldo;
#pragma unroll
        for (int k = 0; k < HW_KB; k++) {
            if (k >= nkb) continue;
            unsigned pk[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float v0 = orow[32 * k + 8 * g + 2 * e], v1 = orow[32 * k + 8 * g + 2 * e + 1];
                limb_source(v0);
                limb_source(v1);
                const unsigned short h0 = f16_bits(v0), h1 = f16_bits(v1);
                const unsigned short b0 = limb ? f16_bits(v0 - f16_val(h0)) : h0;
                const unsigned short b1 = limb ? f16_bits(v1 - f16_val(h1)) : h1;
                pk[e] = (unsigned)b0 | ((unsigned)b1 << 16);
            }
            xa[k] = __builtin_bit_cast(h8_t, u4_t{pk[0], pk[1], pk[2], pk[3]});
        }
        const int shift = (g >> 1) * 4;
        const f4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ps = 0; ps < P; ps++) {
            const int col = c0 + 128 * ps + 16 * w + c16;
            f4_t acc = zero;
#pragma unroll
            for (int k = 0; k < HW_KB; k++) {
                if (k >= nkb) continue;
                const f4_t t =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[k], quants_f16<WF>(wq[ps][k], shift), zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(dsc[ps][k], t[i], acc[i]);
            }
            // lanes g < 2 hold the hi rows of tokens 4 g + i; lane + 32 the lo rows
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] += __shfl_down(acc[i], 32);
            if (g >= 2 || col >= c1) continue;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 4 * g + i;
                if (t < n) dst[(size_t)t * N + col] = acc[i];
            }
        }
    }
};

}  // namespace cih
