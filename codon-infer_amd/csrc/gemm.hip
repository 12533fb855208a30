// Dequantizing GEMMs for gfx950: Y = epi(X * W^T + b) on FP32 MFMA.
//
// Replaces matmul_tiled_{fp32,q8,q4}_parallel (codon-infer src/lib.rs:4766-4961).
// The reference unpacks each weight row to FP32 as (float)q * d
// (lib.rs:4687, 4724-4741) and runs an FP32 FMA dot product per token; this
// kernel forms the same FP32 weights in registers (one f32 multiply of the
// exact integer by the block scale) and feeds them, with FP32 activations, to
// v_mfma_f32_32x32x2_f32.  Products are exact-precision FP32; only the
// summation order differs from the CPU path.
//
// Tiling: 256 threads = 4 waves (2x2), workgroup tile BM x BN, BK = 32 (one
// quantization block).  Each wave owns (BM/2) x (BN/2) outputs as 32x32 MFMA
// tiles.  Within a k-block, lane (i = lane%32, half = lane/32) feeds k-slot
// `half` with k = half*16 + s at step s; for Q4_0 that makes half 0 read the
// low nibbles and half 1 the high nibbles of the same 16 bytes, which is the
// reference's packing (element j low, element j+16 high, lib.rs:1064-1068).
// A and the raw quantized B tile are double-buffered in LDS; the next k-block
// is fetched into registers while the current one is multiplied.
#include <stdlib.h>

#include <algorithm>
#include <string.h>

#include "kernels.h"

namespace cih {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int A_LD = 36;    // floats per LDS row of the A tile (32 + 4 pad: conflict-free b128 reads)
constexpr int F32_LD = 36;  // same for FP32 weight rows
constexpr int Q8_LD = 48;   // bytes per LDS column of Q8 quants (32 + 16 pad)
constexpr int Q4_LD = 16;   // bytes per LDS column of Q4 quants

template <int WF, int BN>
struct BTileBytes {
    static constexpr int value = WF == WF_F32 ? BN * F32_LD * 4 : (WF == WF_Q8 ? BN * Q8_LD : BN * Q4_LD);
};

// Tile order: bijective remap so that the workgroups the dispatcher sends to
// one XCD (round-robin over 8) are consecutive in tile order, then grouped
// rows (GROUP_M row tiles swept across N) so concurrently resident tiles
// share A rows and B columns in that XCD's L2.
__device__ __forceinline__ void tile_of(int bid, int total, int nM, int nN, int &mt, int &nt) {
    constexpr int XCD = 8, GROUP_M = 8;
    int xcd = bid % XCD, local = bid / XCD;
    int per = total / XCD, rem = total % XCD;
    int id = (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
    int in_group = GROUP_M * nN;
    int g = id / in_group;
    int first = g * GROUP_M;
    int gsize = min(nM - first, GROUP_M);
    int r = id % in_group;
    mt = first + r % gsize;
    nt = r / gsize;
}

// SPLIT: workgroup (tile, y) sums k-blocks [y * kps, (y + 1) * kps) only and,
// with part, leaves the raw sums in part[y][M][N] for k_splitk_reduce.
template <int WF, int EPI, int BM, int BN, bool SPLIT>
__global__ __launch_bounds__(256, 2) void k_gemm(const float *__restrict__ X, int ldx, const void *__restrict__ Wq,
                                                 const float *__restrict__ Wsc, const float *__restrict__ bias,
                                                 float *__restrict__ Y, int ldy, int M, int N, int K, int kps,
                                                 float *__restrict__ part) {
    constexpr int MT = BM / 64;  // 32-row MFMA tiles per wave
    constexpr int NT = BN / 64;  // 32-col MFMA tiles per wave
    constexpr int A_LOADS = BM / 32;  // float4 per thread for the A tile
    constexpr int BBYTES = BTileBytes<WF, BN>::value;
    __shared__ __attribute__((aligned(16))) float As[2][BM * A_LD];
    __shared__ __attribute__((aligned(16))) unsigned char Bs[2][BBYTES];
    __shared__ float Ss[2][BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 31, hh = lane >> 5;
    const int nM = (M + BM - 1) / BM, nN = (N + BN - 1) / BN;
    int mt, nt;
    tile_of(blockIdx.x, nM * nN, nM, nN, mt, nt);
    const int m0 = mt * BM, n0 = nt * BN;
    const int KB = K / 32;

    // ---- global -> register prefetch state
    float4 ra[A_LOADS];
    constexpr int B_LOADS = WF == WF_F32 ? (BN * 8 + 255) / 256 : (WF == WF_Q8 ? (BN * 2 + 255) / 256 : (BN + 255) / 256);
    uint4 rb[B_LOADS];
    float rs = 0.0f;

    auto gload = [&](int kb) {
#pragma unroll
        for (int i = 0; i < A_LOADS; i++) {
            int row = (tid >> 3) + 32 * i, c4 = tid & 7;
            int gr = m0 + row;
            ra[i] = gr < M ? *reinterpret_cast<const float4 *>(X + (size_t)gr * ldx + kb * 32 + c4 * 4)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if constexpr (WF == WF_F32) {
            const float *w = reinterpret_cast<const float *>(Wq) + (size_t)kb * N * 32;
#pragma unroll
            for (int i = 0; i < B_LOADS; i++) {
                int idx = tid + 256 * i, col = idx >> 3, c4 = idx & 7;
                int gc = n0 + col;
                rb[i] = (col < BN && gc < N) ? *reinterpret_cast<const uint4 *>(w + (size_t)gc * 32 + c4 * 4)
                                             : make_uint4(0, 0, 0, 0);
            }
        } else if constexpr (WF == WF_Q8) {
            const unsigned char *w = reinterpret_cast<const unsigned char *>(Wq) + (size_t)kb * N * 32;
#pragma unroll
            for (int i = 0; i < B_LOADS; i++) {
                int idx = tid + 256 * i, col = idx >> 1, half = idx & 1;
                int gc = n0 + col;
                rb[i] = (col < BN && gc < N) ? *reinterpret_cast<const uint4 *>(w + (size_t)gc * 32 + half * 16)
                                             : make_uint4(0, 0, 0, 0);
            }
        } else {
            const unsigned char *w = reinterpret_cast<const unsigned char *>(Wq) + (size_t)kb * N * 16;
#pragma unroll
            for (int i = 0; i < B_LOADS; i++) {
                int col = tid + 256 * i;
                int gc = n0 + col;
                rb[i] = (col < BN && gc < N) ? *reinterpret_cast<const uint4 *>(w + (size_t)gc * 16)
                                             : make_uint4(0, 0, 0, 0);
            }
        }
        if constexpr (WF != WF_F32) {
            int gc = n0 + tid;
            rs = (tid < BN && gc < N) ? Wsc[(size_t)kb * N + gc] : 0.0f;
        }
    };

    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LOADS; i++) {
            int row = (tid >> 3) + 32 * i, c4 = tid & 7;
            *reinterpret_cast<float4 *>(&As[buf][row * A_LD + c4 * 4]) = ra[i];
        }
        if constexpr (WF == WF_F32) {
#pragma unroll
            for (int i = 0; i < B_LOADS; i++) {
                int idx = tid + 256 * i, col = idx >> 3, c4 = idx & 7;
                if (col < BN) *reinterpret_cast<uint4 *>(&Bs[buf][(col * F32_LD + c4 * 4) * 4]) = rb[i];
            }
        } else if constexpr (WF == WF_Q8) {
#pragma unroll
            for (int i = 0; i < B_LOADS; i++) {
                int idx = tid + 256 * i, col = idx >> 1, half = idx & 1;
                if (col < BN) *reinterpret_cast<uint4 *>(&Bs[buf][col * Q8_LD + half * 16]) = rb[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < B_LOADS; i++) {
                int col = tid + 256 * i;
                if (col < BN) *reinterpret_cast<uint4 *>(&Bs[buf][col * Q4_LD]) = rb[i];
            }
        }
        if constexpr (WF != WF_F32) {
            if (tid < BN) Ss[buf][tid] = rs;
        }
    };

    f32x16 acc[MT][NT];
#pragma unroll
    for (int r = 0; r < MT; r++)
#pragma unroll
        for (int c = 0; c < NT; c++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[r][c][q] = 0.0f;

    const int kb0 = SPLIT ? (int)blockIdx.y * kps : 0, kend = SPLIT ? min(KB, kb0 + kps) : KB;
    gload(kb0);
    sstore(0);
    __syncthreads();

    for (int kb = kb0; kb < kend; kb++) {
        const int cur = (kb - kb0) & 1;
        if (kb + 1 < kend) gload(kb + 1);

        float a[MT][16];
#pragma unroll
        for (int r = 0; r < MT; r++) {
            const float *src = &As[cur][(wm * (BM / 2) + r * 32 + li) * A_LD + hh * 16];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float4 t = *reinterpret_cast<const float4 *>(src + 4 * v);
                a[r][4 * v + 0] = t.x; a[r][4 * v + 1] = t.y; a[r][4 * v + 2] = t.z; a[r][4 * v + 3] = t.w;
            }
        }
        float b[NT][16];
#pragma unroll
        for (int c = 0; c < NT; c++) {
            const int col = wn * (BN / 2) + c * 32 + li;
            if constexpr (WF == WF_F32) {
                const float *src = reinterpret_cast<const float *>(&Bs[cur][0]) + col * F32_LD + hh * 16;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    float4 t = *reinterpret_cast<const float4 *>(src + 4 * v);
                    b[c][4 * v + 0] = t.x; b[c][4 * v + 1] = t.y; b[c][4 * v + 2] = t.z; b[c][4 * v + 3] = t.w;
                }
            } else if constexpr (WF == WF_Q8) {
                const uint4 raw = *reinterpret_cast<const uint4 *>(&Bs[cur][col * Q8_LD + hh * 16]);
                const float d = Ss[cur][col];
                const unsigned w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int v = 0; v < 4; v++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        b[c][4 * v + e] = (float)(signed char)((w4[v] >> (8 * e)) & 0xFF) * d;
            } else {
                const uint4 raw = *reinterpret_cast<const uint4 *>(&Bs[cur][col * Q4_LD]);
                const float d = Ss[cur][col];
                const unsigned w4[4] = {raw.x, raw.y, raw.z, raw.w};
                const int sh = hh * 4;
#pragma unroll
                for (int v = 0; v < 4; v++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        b[c][4 * v + e] = (float)((int)((w4[v] >> (8 * e + sh)) & 0xF) - 8) * d;
            }
        }
#pragma unroll
        for (int s = 0; s < 16; s++)
#pragma unroll
            for (int r = 0; r < MT; r++)
#pragma unroll
                for (int c = 0; c < NT; c++)
                    acc[r][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[r][s], b[c][s], acc[r][c], 0, 0, 0);

        if (kb + 1 < kend) sstore(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue: lane holds column li of each 32x32 tile, rows 8*(q/4) + 4*hh + q%4
    if (SPLIT && part) {  // raw partial sums; bias and epilogue in k_splitk_reduce
#pragma unroll
        for (int c = 0; c < NT; c++) {
            const int col = n0 + wn * (BN / 2) + c * 32 + li;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < MT; r++)
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    const int row = m0 + wm * (BM / 2) + r * 32 + 8 * (q >> 2) + 4 * hh + (q & 3);
                    if (row < M) part[((size_t)blockIdx.y * M + row) * N + col] = acc[r][c][q];
                }
        }
        return;
    }
    // Every output value is formed before the first store (bias and residual
    // reads share one wait, and no store follows a pending load, which would
    // make the compiler wait for each earlier store at every bounds branch);
    // tiles inside the matrix store without bounds branches.
    float bv[NT];
#pragma unroll
    for (int c = 0; c < NT; c++) bv[c] = bias ? bias[min(n0 + wn * (BN / 2) + c * 32 + li, N - 1)] : 0.0f;
    float res[NT][MT][16];
    if constexpr (EPI == EPI_RESIDUAL) {
#pragma unroll
        for (int c = 0; c < NT; c++) {
            const int col = min(n0 + wn * (BN / 2) + c * 32 + li, N - 1);
#pragma unroll
            for (int r = 0; r < MT; r++)
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    const int row = min(m0 + wm * (BM / 2) + r * 32 + 8 * (q >> 2) + 4 * hh + (q & 3), M - 1);
                    res[c][r][q] = Y[(size_t)row * ldy + col];
                }
        }
    }
#pragma unroll
    for (int c = 0; c < NT; c++)
#pragma unroll
        for (int r = 0; r < MT; r++)
#pragma unroll
            for (int q = 0; q < 16; q++) {
                float v = acc[r][c][q] + bv[c];
                if constexpr (EPI == EPI_GELU) v = gelu_as(v);
                if constexpr (EPI == EPI_RESIDUAL) v = res[c][r][q] + v;
                acc[r][c][q] = v;
            }
    auto store = [&](bool guard) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < NT; c++) {
            const int col = n0 + wn * (BN / 2) + c * 32 + li;
            if (guard && col >= N) continue;
#pragma unroll
            for (int r = 0; r < MT; r++)
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    const int row = m0 + wm * (BM / 2) + r * 32 + 8 * (q >> 2) + 4 * hh + (q & 3);
                    if (guard && row >= M) continue;
                    Y[(size_t)row * ldy + col] = acc[r][c][q];
                }
        }
    };
    if (m0 + BM <= M && n0 + BN <= N)
        store(false);
    else
        store(true);
}

// Split K when the tiles alone leave the GPU mostly idle (small token
// counts: 256 tokens of the 8M model give 6-20 workgroups): up to ~1024
// workgroups, at least 4 k-blocks per split, partials within pb; the ordered
// reduction then adds bias and the epilogue.  CIH_SPLITK=0 turns it off.
template <int WF, int EPI, int BM, int BN>
static hipError_t launch_t(const DevMatrix &W, const float *X, int ldx, const float *bias, float *Y, int ldy, int M,
                           const PartialBuf *pb, hipStream_t st) {
    const int nM = (M + BM - 1) / BM, nN = (W.N + BN - 1) / BN, KB = W.K / 32;
    const long wgs = (long)nM * nN;
    int S = 1, kps = KB;
    const char *e = getenv("CIH_SPLITK");
    if (pb && pb->part && !(e && !strcmp(e, "0")) && wgs < 512 && KB >= 8) {
        S = (int)std::min<long>(1024 / wgs, KB / 4);
        while (S > 1 && (size_t)S * M * W.N > pb->floats) S--;
        if (S > 1) {
            kps = (KB + S - 1) / S;
            S = (KB + kps - 1) / kps;
        }
    }
    if (S > 1) {
        hipLaunchKernelGGL((k_gemm<WF, EPI, BM, BN, true>), dim3(nM * nN, S), dim3(256), 0, st, X, ldx, W.q, W.sc,
                           bias, Y, ldy, M, W.N, W.K, kps, pb->part);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        return launch_splitk_reduce(pb->part, S, M, W.N, bias, Y, ldy, EPI, st);
    }
    hipLaunchKernelGGL((k_gemm<WF, EPI, BM, BN, false>), dim3(nM * nN), dim3(256), 0, st, X, ldx, W.q, W.sc, bias, Y,
                       ldy, M, W.N, W.K, KB, nullptr);
    return hipGetLastError();
}

template <int WF, int EPI>
static hipError_t launch_shape(const DevMatrix &W, const float *X, int ldx, const float *bias, float *Y, int ldy,
                               int M, const PartialBuf *pb, hipStream_t st) {
    const bool small_m = M <= 64, small_n = W.N <= 64;
    if (small_m && small_n) return launch_t<WF, EPI, 64, 64>(W, X, ldx, bias, Y, ldy, M, pb, st);
    if (small_m) return launch_t<WF, EPI, 64, 128>(W, X, ldx, bias, Y, ldy, M, pb, st);
    if (small_n) return launch_t<WF, EPI, 128, 64>(W, X, ldx, bias, Y, ldy, M, pb, st);
    return launch_t<WF, EPI, 128, 128>(W, X, ldx, bias, Y, ldy, M, pb, st);
}

template <int WF>
static hipError_t launch_epi(const DevMatrix &W, const float *X, int ldx, const float *bias, float *Y, int ldy, int M,
                             int epi, const PartialBuf *pb, hipStream_t st) {
    switch (epi) {
    case EPI_GELU: return launch_shape<WF, EPI_GELU>(W, X, ldx, bias, Y, ldy, M, pb, st);
    case EPI_RESIDUAL: return launch_shape<WF, EPI_RESIDUAL>(W, X, ldx, bias, Y, ldy, M, pb, st);
    default: return launch_shape<WF, EPI_NONE>(W, X, ldx, bias, Y, ldy, M, pb, st);
    }
}

hipError_t launch_gemm(const DevMatrix &W, const void *Xv, int ldx, int a_fmt, const float *bias, void *Yv, int ldy,
                       int M, int epi, const PartialBuf *pb, hipStream_t st, int *defer) {
    if (defer) *defer = 0;
    if (M <= 0) return hipSuccess;
    if (W.K % 32 != 0) return hipErrorInvalidValue;
    // Quantized weights go to the 16-bit-limb MFMA kernel (FP32 or pre-split
    // activations) unless CIH_QGEMM=fp32 selects the FP32-MFMA kernel, which
    // gives the same results to FP32 rounding and is kept for A/B runs.
    const char *path = getenv("CIH_QGEMM");
    const bool fp32_path = path && !strcmp(path, "fp32");
    if (W.fmt != WF_F32) {
        if (a_fmt != AF_F32 || !fp32_path) return launch_gemm_x3(W, Xv, ldx, a_fmt, bias, Yv, ldy, M, epi, pb, st, defer);
    }
    // FP32 weights with a pair copy: the same f16-limb GEMM on [hi | lo]
    // (CIH_QGEMM=fp32, CIH_LIMBS=bf16x3 and full range keep FP32 MFMA)
    const char *lv = getenv("CIH_LIMBS");
    if (W.fmt == WF_F32 && W.p16 && W.psc && !fp32_path && !(lv && !strcmp(lv, "bf16x3")) && !full_range_mode() &&
        (a_fmt == AF_F32 || a_fmt == AF_H2)) {
        DevMatrix P;
        P.fmt = WF_F16P;
        P.N = W.N;
        P.K = W.K;
        P.q = W.p16;
        P.sc = W.psc;
        return launch_gemm_x3(P, Xv, ldx, a_fmt, bias, Yv, ldy, M, epi, pb, st, defer);
    }
    if (a_fmt != AF_F32 || epi == EPI_GELU_X3 || epi == EPI_GELU_H2 || ldx % 4 != 0) return hipErrorInvalidValue;
    const float *X = reinterpret_cast<const float *>(Xv);
    float *Y = reinterpret_cast<float *>(Yv);
    if (W.fmt == WF_Q8) return launch_epi<WF_Q8>(W, X, ldx, bias, Y, ldy, M, epi, pb, st);
    if (W.fmt == WF_Q4) return launch_epi<WF_Q4>(W, X, ldx, bias, Y, ldy, M, epi, pb, st);
    return launch_epi<WF_F32>(W, X, ldx, bias, Y, ldy, M, epi, pb, st);
}

// Test path: k-block-major device matrix -> row-major [N][K] FP32, with the
// exact decode expression the GEMM uses.
__global__ void k_dequant(int fmt, const void *__restrict__ q, const float *__restrict__ sc, int N, int K,
                          float *__restrict__ out) {
    const int KB = K / 32;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // (kb, n, e)
    const size_t total = (size_t)KB * N * 32;
    if (idx >= total) return;
    const int e = idx % 32;
    const int n = (idx / 32) % N;
    const int kb = idx / ((size_t)32 * N);
    float v;
    if (fmt == WF_Q8) {
        const signed char qv = reinterpret_cast<const signed char *>(q)[((size_t)kb * N + n) * 32 + e];
        v = (float)qv * sc[(size_t)kb * N + n];
    } else if (fmt == WF_Q4) {
        const unsigned char byte = reinterpret_cast<const unsigned char *>(q)[((size_t)kb * N + n) * 16 + (e & 15)];
        const int nib = e < 16 ? (byte & 0xF) : (byte >> 4);
        v = (float)(nib - 8) * sc[(size_t)kb * N + n];
    } else {
        v = reinterpret_cast<const float *>(q)[((size_t)kb * N + n) * 32 + e];
    }
    out[(size_t)n * K + kb * 32 + e] = v;
}

hipError_t launch_dequant(const DevMatrix &W, float *out, hipStream_t st) {
    const size_t total = (size_t)(W.K / 32) * W.N * 32;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, W.fmt, W.q, W.sc, W.N, W.K,
                       out);
    return hipGetLastError();
}

}  // namespace cih
