// Internal launch interface of the gfx950 kernels (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "x3.h"

namespace cih {

// Weight formats of the device-resident matrices.  All use a k-block-major
// layout so that one 32-wide k-block of BN consecutive output rows is a
// single contiguous span (coalesced loads for both the MFMA GEMM and GEMV):
//   F32: w  [K/32][N][32] float
//   Q8 : qs [K/32][N][32] int8,   sc [K/32][N] float
//   Q4 : qs [K/32][N][16] uint8,  sc [K/32][N] float   (reference nibble order)
enum WFmt { WF_F32 = 0, WF_Q8 = 1, WF_Q4 = 2 };

// GEMM epilogue applied to v = acc + bias[n]; EPI_GELU_X3 writes gelu(v)
// in the three-limb bf16 format of x3.h (for the next quantized GEMM).
enum Epi { EPI_NONE = 0, EPI_GELU = 1, EPI_RESIDUAL = 2, EPI_GELU_X3 = 3 };

struct DevMatrix {
    int fmt = WF_F32;
    int N = 0, K = 0;          // out_dim, in_dim
    const void *q = nullptr;   // F32 values or packed quants
    const float *sc = nullptr; // per-block scales (quantized formats)
};

// Y[M][N] (row stride ldy) = epi(X[M][K] * W^T + bias).  X is FP32 with row
// stride ldx (a_fmt AF_F32) or three-limb bf16 (AF_X3, quantized W only).
hipError_t launch_gemm(const DevMatrix &W, const void *X, int ldx, int a_fmt, const float *bias, void *Y,
                       int ldy, int M, int epi, hipStream_t st);

// Q8_0/Q4_0 GEMM on bf16 MFMA: exact integer weights, activations split
// into three bf16 limbs (FP32-equivalent products), block scale in FP32.
hipError_t launch_gemm_x3(const DevMatrix &W, const void *X, int ldx, int a_fmt, const float *bias, void *Y,
                          int ldy, int M, int epi, hipStream_t st);

// Dequantizes nblocks of a device matrix in k-block-major layout back to the
// reference's row-major [N][K] FP32 (test path).
hipError_t launch_dequant(const DevMatrix &W, float *out, hipStream_t st);

struct SeqMeta {
    const int *cu;    // [B] first packed row of each sequence
    const int *lens;  // [B] tokens per sequence
    int B, S_max;
};

// Embedding + token-dropout rescale, packed rows.
hipError_t launch_embed(const int *tokens, SeqMeta sm, int emb_fmt, const void *emb_q,
                        const float *emb_sc, int d, int V, float *x, hipStream_t st);

// out = LayerNorm(x) over rows of width d (eps 1e-5); out_fmt AF_F32 or AF_X3
hipError_t launch_layernorm(const float *x, const float *w, const float *b, void *out, int out_fmt, int rows,
                            int d, hipStream_t st);

// Bidirectional rotary attention over packed Q|K|V rows.  When P != nullptr
// every softmax row is stored at P[b*pb + h*ph + q*S_max + k].
// out: [T][d] FP32 (out_fmt AF_F32) or three-limb bf16 (AF_X3).
hipError_t launch_attention(const float *qkv, int d, int H, SeqMeta sm, const float *rope_cos,
                            const float *rope_sin, void *out, int out_fmt, float *P, int64_t pb, int64_t ph,
                            hipStream_t st);

// final_att[b][p][t] = sum_h P_h[p][t] * (1/H), h ascending
hipError_t launch_head_mean(const float *P, int64_t pb, int64_t ph, int H, SeqMeta sm, float *final_att,
                            hipStream_t st);

// Contacts (APC).  For layer l, heads with w != 0:
//   M[b][i][j]   += sum_h w_lh * P_lh[i+1][j+1]
//   r[l][h][b][i] = sum_j P_lh[i+1][j+1] + P_lh[j+1][i+1]   (residues only)
hipError_t launch_apc_layer(const float *P, int64_t pb, int64_t ph, int H, int l, const float *w_dev,
                            const int *heads_dev, int n_heads_nz, SeqMeta sm, float *M, float *r,
                            hipStream_t st);
// contacts[b][i][j] = sigmoid(M_ij + M_ji - sum_lh (w_lh / T_lh) r_i r_j + bias)
// coef: [L*H][B] scratch for w_lh / T_lh.
hipError_t launch_apc_finalize(const float *M, const float *r, float *coef, const float *w_dev, int LH, SeqMeta sm,
                               float bias, float *contacts, int n_stride, hipStream_t st);

// Copies packed rows [T][width] into padded [B][S_max][width] (valid rows only).
hipError_t launch_scatter_rows(const float *src, int width, SeqMeta sm, float *dst, int64_t dst_b_stride,
                               hipStream_t st);

}  // namespace cih
