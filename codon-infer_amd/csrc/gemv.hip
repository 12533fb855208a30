// Weight-streaming GEMV for a few tokens (M <= GEMV_MAX_M): Y = epi(X W^T + b).
//
// Arithmetic of the reference's row dequant + FMA dot product
// (src/lib.rs:4669-4756 forms each weight as (q as f32) * d, 4443-4531
// accumulates FP32 FMAs): here each weight is formed bit-exactly as
// round(q * d) (fma(u, d, -128 d) on the biased byte u = q + 128, or
// fma(n, d, -8 d) on a Q4 nibble) and multiplied into FP32 accumulators.
//
// At M <= 8 the GEMM moves 1.125 B (Q8) per weight and does <= 8 FMAs with
// it, so it is bound by HBM, not arithmetic.  Decomposition:
//   - a lane owns one output column and all M tokens (M accumulators);
//   - a workgroup (4 waves) owns 64 consecutive columns and 4 NB k-blocks;
//     wave w takes k-blocks w, w + 4, ..., so the waves of a workgroup read
//     adjacent 2 KiB spans of the k-block-major weight layout, and all NB
//     blocks of a wave are requested before the first is used;
//   - activations are wave-uniform, read through the scalar cache;
//   - the 4 waves are combined in LDS in wave order.  With one k-split the
//     workgroup applies bias and epilogue itself; with several (gridDim.y),
//     each writes its partial sums and a second kernel adds them in split
//     order.  Either way the result does not depend on scheduling.
#include <algorithm>
#include <cstdlib>

#include "kernels.h"

namespace cih {

namespace {

// raw weights of one (k-block, column)
template <int WF> struct Raw;
template <> struct Raw<WF_Q8> { uint4 a, b; float d; };
template <> struct Raw<WF_Q4> { uint4 a; float d; };
template <> struct Raw<WF_F32> { float4 v[8]; };

template <int WF>
__device__ __forceinline__ Raw<WF> load_raw(const void *__restrict__ Wq, const float *__restrict__ Wsc, int N, int kb,
                                            int n) {
    Raw<WF> r;
    const size_t blk = (size_t)kb * N + n;
    if constexpr (WF == WF_Q8) {
        const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const unsigned char *>(Wq) + blk * 32);
        r.a = p[0];
        r.b = p[1];
        r.d = Wsc[blk];
    } else if constexpr (WF == WF_Q4) {
        r.a = *reinterpret_cast<const uint4 *>(static_cast<const unsigned char *>(Wq) + blk * 16);
        r.d = Wsc[blk];
    } else {
        const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(Wq) + blk * 32);
#pragma unroll
        for (int v = 0; v < 8; v++) r.v[v] = p[v];
    }
    return r;
}

// w[e] = weight e of the block, bit-identical to the reference's dequant;
// all zero when !live (a clamped block past the wave's range)
template <int WF>
__device__ __forceinline__ void dequant(const Raw<WF> &r, bool live, float w[32]) {
    if constexpr (WF == WF_Q8) {
        const unsigned u[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        const float d = live ? r.d : 0.0f;
        const float dn = -128.0f * d;
#pragma unroll
        for (int e = 0; e < 32; e++) {
            const unsigned v = u[e >> 2] ^ 0x80808080u;  // byte q + 128
            w[e] = fmaf((float)((v >> (8 * (e & 3))) & 0xFFu), d, dn);
        }
    } else if constexpr (WF == WF_Q4) {
        const unsigned u[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const float d = live ? r.d : 0.0f;
        const float dn = -8.0f * d;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const unsigned lo = u[e >> 2] & 0x0F0F0F0Fu, hi = (u[e >> 2] >> 4) & 0x0F0F0F0Fu;
            w[e] = fmaf((float)((lo >> (8 * (e & 3))) & 0xFFu), d, dn);
            w[e + 16] = fmaf((float)((hi >> (8 * (e & 3))) & 0xFFu), d, dn);
        }
    } else {
        const float z = live ? 1.0f : 0.0f;
#pragma unroll
        for (int v = 0; v < 8; v++) {
            w[4 * v] = r.v[v].x * z;
            w[4 * v + 1] = r.v[v].y * z;
            w[4 * v + 2] = r.v[v].z * z;
            w[4 * v + 3] = r.v[v].w * z;
        }
    }
}

__device__ __forceinline__ void store_out(int epi, float v, const float *__restrict__ bias, int n,
                                          float *__restrict__ dst) {
    v += bias ? bias[n] : 0.0f;
    if (epi == EPI_GELU) v = gelu_as(v);
    else if (epi == EPI_RESIDUAL) v += *dst;
    *dst = v;
}

}  // namespace

template <int WF, int MM, int NB>
__global__ __launch_bounds__(256) void k_gemv(const float *__restrict__ X, int ldx, const void *__restrict__ Wq,
                                              const float *__restrict__ Wsc, int N, int KB,
                                              const float *__restrict__ bias, float *__restrict__ Y, int ldy, int epi,
                                              float *__restrict__ part, int to_part) {
    __shared__ float red[4][MM][64];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: X reads become scalar
    const int n = blockIdx.x * 64 + lane;
    const int nc = n < N ? n : N - 1;  // lanes past N load a valid column; their sums are dropped
    const int kb0 = blockIdx.y * 4 * NB;

    // The wave's NB k-blocks (kb0 + wv + 4 j) are requested before any is used; one past
    // K (last split only) is clamped to the last k-block and enters with zero weights
    // (unconditional use keeps every load ahead of the arithmetic).
    Raw<WF> raw[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) raw[j] = load_raw<WF>(Wq, Wsc, N, min(kb0 + wv + 4 * j, KB - 1), nc);
    float acc[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) acc[m] = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int kb = min(kb0 + wv + 4 * j, KB - 1);
        float w[32];
        dequant<WF>(raw[j], kb0 + wv + 4 * j < KB, w);
#pragma unroll
        for (int m = 0; m < MM; m++) {
            const float4 *xr = reinterpret_cast<const float4 *>(X + (size_t)m * ldx + kb * 32);
#pragma unroll
            for (int v = 0; v < 8; v++) {
                const float4 x4 = xr[v];
                acc[m] = fmaf(w[4 * v], x4.x, acc[m]);
                acc[m] = fmaf(w[4 * v + 1], x4.y, acc[m]);
                acc[m] = fmaf(w[4 * v + 2], x4.z, acc[m]);
                acc[m] = fmaf(w[4 * v + 3], x4.w, acc[m]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MM; m++) red[wv][m][lane] = acc[m];
    __syncthreads();

    for (int t = threadIdx.x; t < MM * 64; t += 256) {
        const int m = t >> 6, c = t & 63, nn = blockIdx.x * 64 + c;
        if (nn >= N) continue;
        const float s = ((red[0][m][c] + red[1][m][c]) + red[2][m][c]) + red[3][m][c];
        if (gridDim.y == 1 && !to_part) store_out(epi, s, bias, nn, Y + (size_t)m * ldy + nn);
        else part[((size_t)blockIdx.y * MM + m) * N + nn] = s;
    }
}

// Y[m][n] = epi(sum over splits of part[split][m][n] + bias[n]).  Eight
// lanes per output: lane j adds splits j, j + 8, ... (its loads issued
// together), then a fixed xor tree joins the eight lanes.  The order depends
// on the split count only, not on M, so a row's result does not depend on
// the other rows.
__global__ __launch_bounds__(256) void k_gemv_reduce(const float *__restrict__ part, int splits, int M, int N,
                                                     const float *__restrict__ bias, float *__restrict__ Y, int ldy,
                                                     int epi) {
    const int MN = M * N;
    const int gid = blockIdx.x * 256 + threadIdx.x;
    const int e = gid >> 3, j = gid & 7;
    const int ec = e < MN ? e : MN - 1;  // lanes past the end join the shuffles with a valid address
    float s = 0.0f;
    for (int y = j; y < splits; y += 8) s += part[(size_t)y * MN + ec];
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (j == 0 && e < MN) {
        const int m = e / N, n = e - m * N;
        store_out(epi, s, bias, n, Y + (size_t)m * ldy + n);
    }
}

GemvGrid gemv_grid(int N, int K) {
    GemvGrid g;
    const int KB = K / 32;
    g.cols = (N + 63) / 64;
    // blocks per wave: the fewest (1, 2 or 4) that keep the grid within 1024
    // workgroups (four per CU); CIH_GEMV_NB overrides
    g.nb = 1;
    while (g.nb < 4 && (size_t)g.cols * ((KB + 4 * g.nb - 1) / (4 * g.nb)) > 1024) g.nb *= 2;
    if (const char *e = getenv("CIH_GEMV_NB")) {
        const int v = atoi(e);
        if (v == 1 || v == 2 || v == 4) g.nb = v;
    }
    g.splits = (KB + 4 * g.nb - 1) / (4 * g.nb);
    return g;
}

size_t gemv_part_floats(int N, int K) {
    const GemvGrid g = gemv_grid(N, K);
    return g.splits > 1 ? (size_t)g.splits * GEMV_MAX_M * N : 0;
}

template <int WF, int MM>
static void launch_mm(const DevMatrix &W, const float *X, int ldx, const float *bias, float *Y, int ldy, int epi,
                      float *part, int to_part, const GemvGrid &g, hipStream_t st) {
    const dim3 grid(g.cols, g.splits);
    const int KB = W.K / 32;
    if (g.nb == 1)
        hipLaunchKernelGGL((k_gemv<WF, MM, 1>), grid, dim3(256), 0, st, X, ldx, W.q, W.sc, W.N, KB, bias, Y, ldy, epi,
                           part, to_part);
    else if (g.nb == 2)
        hipLaunchKernelGGL((k_gemv<WF, MM, 2>), grid, dim3(256), 0, st, X, ldx, W.q, W.sc, W.N, KB, bias, Y, ldy, epi,
                           part, to_part);
    else
        hipLaunchKernelGGL((k_gemv<WF, MM, 4>), grid, dim3(256), 0, st, X, ldx, W.q, W.sc, W.N, KB, bias, Y, ldy, epi,
                           part, to_part);
}

template <int WF>
static void launch_fmt(const DevMatrix &W, const float *X, int ldx, int M, const float *bias, float *Y, int ldy,
                       int epi, float *part, int to_part, const GemvGrid &g, hipStream_t st) {
    switch (M) {
    case 1: return launch_mm<WF, 1>(W, X, ldx, bias, Y, ldy, epi, part, to_part, g, st);
    case 2: return launch_mm<WF, 2>(W, X, ldx, bias, Y, ldy, epi, part, to_part, g, st);
    case 3: return launch_mm<WF, 3>(W, X, ldx, bias, Y, ldy, epi, part, to_part, g, st);
    case 4: return launch_mm<WF, 4>(W, X, ldx, bias, Y, ldy, epi, part, to_part, g, st);
    case 5: return launch_mm<WF, 5>(W, X, ldx, bias, Y, ldy, epi, part, to_part, g, st);
    case 6: return launch_mm<WF, 6>(W, X, ldx, bias, Y, ldy, epi, part, to_part, g, st);
    case 7: return launch_mm<WF, 7>(W, X, ldx, bias, Y, ldy, epi, part, to_part, g, st);
    default: return launch_mm<WF, 8>(W, X, ldx, bias, Y, ldy, epi, part, to_part, g, st);
    }
}

static void launch_any(const DevMatrix &W, const float *X, int ldx, int M, const float *bias, float *Y, int ldy,
                       int epi, float *part, int to_part, const GemvGrid &g, hipStream_t st) {
    if (W.fmt == WF_Q8) launch_fmt<WF_Q8>(W, X, ldx, M, bias, Y, ldy, epi, part, to_part, g, st);
    else if (W.fmt == WF_Q4) launch_fmt<WF_Q4>(W, X, ldx, M, bias, Y, ldy, epi, part, to_part, g, st);
    else launch_fmt<WF_F32>(W, X, ldx, M, bias, Y, ldy, epi, part, to_part, g, st);
}

hipError_t launch_gemv_partials(const DevMatrix &W, const float *X, int ldx, int M, const PartialBuf &s, int *splits,
                                hipStream_t st) {
    if (M <= 0 || M > GEMV_MAX_M || W.K % 32 || ldx < W.K || ldx % 4) return hipErrorInvalidValue;
    const GemvGrid g = gemv_grid(W.N, W.K);
    if (!s.part || s.floats < (size_t)g.splits * M * W.N) return hipErrorInvalidValue;
    launch_any(W, X, ldx, M, nullptr, nullptr, 0, EPI_NONE, s.part, 1, g, st);
    *splits = g.splits;
    return hipGetLastError();
}

hipError_t launch_gemv(const DevMatrix &W, const float *X, int ldx, int M, const float *bias, float *Y, int ldy,
                       int epi, const PartialBuf &s, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (M > GEMV_MAX_M || W.K % 32 || ldx < W.K || ldx % 4 || ldy < W.N ||
        (epi != EPI_NONE && epi != EPI_GELU && epi != EPI_RESIDUAL))
        return hipErrorInvalidValue;
    const GemvGrid g = gemv_grid(W.N, W.K);
    if (g.splits > 1 && (!s.part || s.floats < (size_t)g.splits * M * W.N)) return hipErrorInvalidValue;
    launch_any(W, X, ldx, M, bias, Y, ldy, epi, s.part, 0, g, st);
    if (g.splits > 1)
        hipLaunchKernelGGL(k_gemv_reduce, dim3((M * W.N * 8 + 255) / 256), dim3(256), 0, st, s.part, g.splits, M,
                           W.N, bias, Y, ldy, epi);
    return hipGetLastError();
}

}  // namespace cih
