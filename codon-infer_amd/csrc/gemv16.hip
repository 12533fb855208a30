// Few-token GEMM on f16 MFMA (M <= GEMV_MAX_M tokens): Y = epi(X W^T + b) with
// X in two f16 limbs (H2 form of x3.h) and W in Q8_0 / Q4_0.
//
// Same arithmetic as the batched quantized GEMM (the reference's row dequant +
// FMA dot product, src/lib.rs:4669-4756 and 4443-4531, regrouped per 32-wide
// block): the quants are exact in f16, each activation is hi + lo, the MFMA
// forms sum_k q x per block in FP32 and the block scale is applied in FP32,
// acc += d * tmp.
//
// One v_mfma_f32_16x16x32_f16 covers a whole k-block of 16 columns for all
// tokens and both limbs: A row r is token r % 8, limb r / 8 (rows of tokens
// past M repeat the last token and are dropped), B column c is weight column
// n0 + c.  Lane l holds A[l % 16][8 g .. 8 g + 7] and B[8 g .. 8 g + 7][l % 16]
// with g = l / 16 (so it needs 8 consecutive quants of one column: 8 bytes of
// a Q8_0 block, or 8 nibbles of one half of a Q4_0 block) and receives
// D[4 g + i][l % 16], i = 0..3; lanes g and g + 2 hold the hi and lo rows of
// the same tokens, added with one cross-lane move.
//
// A workgroup of 4 waves owns 64 columns (16 per wave) and a range of k-blocks,
// processed in rounds of KW: the weights of a round are requested first, the
// round's activations (KW x 1 KiB, the same for the 4 waves) are staged in LDS
// once, then KW MFMAs per wave.  At a few tokens every launch is latency-bound
// and a compute unit streams only so many bytes at once, so K is split across
// workgroups (grid.y = S splits of KW blocks: 8-20 KiB of weights per
// workgroup): the splits leave [S][M][N] partial sums, which the consumer adds
// in split order (k_gemv16_fold, or the few-token LayerNorm and attention
// kernels), so the result does not depend on scheduling.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "kernels.h"
#include "x3.h"

namespace cih {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

}  // namespace

// X: [M][KB][hi 32 | lo 32] f16 (H2).  Grid (ceil(N / 64), S), 256 threads;
// workgroup y covers k-blocks [y * rounds * KW, (y + 1) * rounds * KW).  part:
// partial sums [S][M][N]; without part (S == 1) the epilogue is applied here.
//
// AG: the activations are GELU(sum of the aS splits of apart + abias) instead
// (apart: [aS][M][K] partial sums of the projection before, FC1's), formed
// and split into limbs while staging: that projection needs no fold kernel.
//
// LN (one row, K <= GEMV16_LN_MAX_K): the activations are LayerNorm(x + abias
// + sum of the aS splits of apart) with weights ln.w, ln.b: every workgroup
// forms the whole row (k_rln's sums in k_rln's order, row_stats64), so the
// residual LayerNorm needs no launch of its own; workgroup (0, 0) stores the
// new residual x + ... to ln.xo (a buffer other than ln.x, which the other
// workgroups are still reading).  apart == nullptr: LayerNorm(x).
template <int WF, int KW, int EPI, bool AG, bool LN = false>
__global__ __launch_bounds__(256) void k_gemv16(const unsigned short *__restrict__ X, int M, int KB,
                                                const void *__restrict__ Wq, const float *__restrict__ Wsc, int N,
                                                const float *__restrict__ bias, void *__restrict__ Yv, int ldy,
                                                float *__restrict__ part, int rounds, const float *__restrict__ apart,
                                                int aS, const float *__restrict__ abias, const LnIn ln) {
    static_assert(!(AG && LN), "one activation form");
    __shared__ u32x4 xs[KW][64];  // per k-block of the round: the A operand of each lane
    __shared__ f32x4 lnv[LN ? GEMV16_LN_MAX_K / 4 : 1];  // LN: the row, then its LayerNorm
    __shared__ float lnst[2];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    if constexpr (LN) {
        const int d = KB * 32, n4 = d >> 2;
        constexpr int UPT = (GEMV16_LN_MAX_K / 4 + 255) / 256;  // quads per thread
        const int nu = (n4 - tid + 255) / 256;                 // this thread's quads: tid + 256 i, i < nu
        f32x4 v[UPT], g4[UPT], b4[UPT];
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int c = min(tid + 256 * i, n4 - 1);
            v[i] = reinterpret_cast<const f32x4 *>(ln.x)[c];
            g4[i] = reinterpret_cast<const f32x4 *>(ln.w)[c];
            b4[i] = reinterpret_cast<const f32x4 *>(ln.b)[c];
        }
        if (apart) {
            // fold_splits4 for all of the thread's quads at once: the same
            // additions in the same order, every load of a chunk in flight
            fold4_t acc[UPT];
#pragma unroll
            for (int i = 0; i < UPT; i++) acc[i] = fold4_t{0.0f, 0.0f, 0.0f, 0.0f};
            for (int s0 = 0; s0 < aS; s0 += FOLD_CHUNK) {
                fold4_t t[UPT][FOLD_CHUNK];
#pragma unroll
                for (int i = 0; i < UPT; i++)
#pragma unroll
                    for (int u = 0; u < FOLD_CHUNK; u++)
                        t[i][u] = s0 + u < aS && i < nu
                                      ? *reinterpret_cast<const fold4_t *>(apart + (size_t)(s0 + u) * KB * 32 +
                                                                           4 * (tid + 256 * i))
                                      : fold4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int i = 0; i < UPT; i++)
#pragma unroll
                    for (int u = 0; u < FOLD_CHUNK; u++) acc[i] += t[i][u];
            }
#pragma unroll
            for (int i = 0; i < UPT; i++) {
                const f32x4 bb = reinterpret_cast<const f32x4 *>(abias)[min(tid + 256 * i, n4 - 1)];
                v[i] = v[i] + (acc[i] + bb);
            }
        }
        const bool writer = blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
        for (int i = 0; i < UPT; i++)
            if (i < nu) {
                lnv[tid + 256 * i] = v[i];
                if (writer) reinterpret_cast<f32x4 *>(ln.xo)[tid + 256 * i] = v[i];
            }
        __syncthreads();
        if (w == 0) {
            float mean, var;
            row_stats64(lnv, n4, d, lane, mean, var);
            if (lane == 0) {
                lnst[0] = mean;
                lnst[1] = 1.0f / sqrtf(var + 1e-5f);
            }
        }
        __syncthreads();
        const float mean = lnst[0], inv = lnst[1];
#pragma unroll
        for (int i = 0; i < UPT; i++)
            if (i < nu) {
                f32x4 y;
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = g4[i][e] * (v[i][e] - mean) * inv + b4[i][e];
                lnv[tid + 256 * i] = y;
            }
        __syncthreads();
    }
    const int g = lane >> 4, c = lane & 15;
    const bool live = blockIdx.x * 64 + 16 * w < N;  // wave-uniform (N % 16 == 0)
    const int n = live ? blockIdx.x * 64 + 16 * w + c : N - 1;
    const unsigned char *wb = static_cast<const unsigned char *>(Wq);
    const int shift = (g >> 1) * 4;  // Q4_0: lanes g = 2, 3 take the high nibbles

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int XE = (KW * 64 + 255) / 256;  // staged operand entries per thread
    for (int r = 0; r < rounds; r++) {
        const int kb0 = (blockIdx.y * rounds + r) * KW;
        // the round's activations first (they are needed first, and loads
        // complete in order), then its weights (blocks past K read the last
        // block and enter with a zero scale)
        u32x4 xe[XE];
        constexpr int UE = (KW * 32 + 255) / 256;  // AG: (k-block, token, 8 k) units per thread
        fold4_t ga[UE][2], gb[UE][2];
        if constexpr (AG) {
            const int K = KB * 32;
#pragma unroll
            for (int q = 0; q < UE; q++) {
                const int u = min(tid + 256 * q, KW * 32 - 1), j = u >> 5, tok = min(u & 7, M - 1);
                const int k0 = min(kb0 + j, KB - 1) * 32 + 8 * ((u >> 3) & 3);
                const float *pp = apart + (size_t)tok * K + k0;
                ga[q][0] = fold_splits4(pp, aS, (size_t)M * K);
                ga[q][1] = fold_splits4(pp + 4, aS, (size_t)M * K);
                gb[q][0] = *reinterpret_cast<const fold4_t *>(abias + k0);
                gb[q][1] = *reinterpret_cast<const fold4_t *>(abias + k0 + 4);
            }
        } else if constexpr (LN) {
            // the row's LayerNorm as limbs (h2_store4's split): lane l of k-block
            // j holds k = 32 kb + 8 (l >> 4) .. + 7, hi limbs for l % 16 < 8
#pragma unroll
            for (int q = 0; q < XE; q++) {
                const int e = min(tid + 256 * q, KW * 64 - 1), j = e >> 6, l = e & 63;
                const int kb = min(kb0 + j, KB - 1), c4 = kb * 8 + 2 * (l >> 4);
                const bool lo = (l & 15) >= 8;
                unsigned h[4];
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    float y0 = lnv[c4 + (p >> 1)][2 * (p & 1)], y1 = lnv[c4 + (p >> 1)][2 * (p & 1) + 1];
                    limb_source(y0);
                    limb_source(y1);
                    unsigned short a0 = f16_bits(y0), a1 = f16_bits(y1);
                    if (lo) {
                        a0 = f16_bits(y0 - f16_val(a0));
                        a1 = f16_bits(y1 - f16_val(a1));
                    }
                    h[p] = (unsigned)a0 | ((unsigned)a1 << 16);
                }
                xe[q] = u32x4{h[0], h[1], h[2], h[3]};
            }
        } else {
#pragma unroll
            for (int q = 0; q < XE; q++) {
                const int e = min(tid + 256 * q, KW * 64 - 1), j = e >> 6, l = e & 63, lc = l & 15;
                const int tok = min(lc & 7, M - 1), kb = min(kb0 + j, KB - 1);
                xe[q] = *reinterpret_cast<const u32x4 *>(X + ((size_t)tok * KB + kb) * 64 + (lc >> 3) * 32 + 8 * (l >> 4));
            }
        }
        u32x2 wq[KW];
        float d[KW];
#pragma unroll
        for (int j = 0; j < KW; j++) {
            const int kb = min(kb0 + j, KB - 1);
            const size_t blk = (size_t)kb * N + n;
            if constexpr (WF == WF_Q8) wq[j] = *reinterpret_cast<const u32x2 *>(wb + blk * 32 + 8 * g);
            else wq[j] = *reinterpret_cast<const u32x2 *>(wb + blk * 16 + 8 * (g & 1));
            d[j] = Wsc[blk];
        }
        if (r > 0) __syncthreads();  // the previous round's operands are read
        if constexpr (AG) {
            // h = GELU(v + bias) as the FC1 epilogue forms it, limbs hi = f16(h),
            // lo = f16(h - hi): lane 16 g + t takes token t's hi limbs of k-group g,
            // lane 16 g + 8 + t its lo limbs
#pragma unroll
            for (int q = 0; q < UE; q++) {
                const int u = tid + 256 * q;
                if (KW * 32 % 256 != 0 && u >= KW * 32) break;
                const int j = u >> 5, t = u & 7, gq = (u >> 3) & 3;
                unsigned hi[4], lo[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float h0 = gelu_as(ga[q][e >> 1][2 * (e & 1)] + gb[q][e >> 1][2 * (e & 1)]);
                    float h1 = gelu_as(ga[q][e >> 1][2 * (e & 1) + 1] + gb[q][e >> 1][2 * (e & 1) + 1]);
                    limb_source(h0);
                    limb_source(h1);
                    const unsigned short a0 = f16_bits(h0), a1 = f16_bits(h1);
                    hi[e] = (unsigned)a0 | ((unsigned)a1 << 16);
                    lo[e] = (unsigned)f16_bits(h0 - f16_val(a0)) | ((unsigned)f16_bits(h1 - f16_val(a1)) << 16);
                }
                xs[j][16 * gq + t] = u32x4{hi[0], hi[1], hi[2], hi[3]};
                xs[j][16 * gq + 8 + t] = u32x4{lo[0], lo[1], lo[2], lo[3]};
            }
        } else {
#pragma unroll
            for (int q = 0; q < XE; q++) {
                const int e = tid + 256 * q;
                if (KW * 64 % 256 == 0 || e < KW * 64) xs[e >> 6][e & 63] = xe[q];
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < KW; j++) {
            const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, xs[j][lane]),
                                                                   quants_f16<WF>(wq[j], shift), zero, 0, 0, 0);
            const float dj = kb0 + j < KB ? d[j] : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(dj, t[i], acc[i]);
        }
    }
    // lanes g < 2: hi rows of tokens 4 g + i; lane + 32: the lo rows of the same tokens
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] += __shfl_down(acc[i], 32);
    if (!live || g >= 2) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = 4 * g + i;
        if (t >= M) break;
        if (part) {
            part[((size_t)blockIdx.y * M + t) * N + n] = acc[i];
            continue;
        }
        float v = acc[i] + (bias ? bias[n] : 0.0f);
        if constexpr (EPI == EPI_GELU_H2) {
            h2_store(static_cast<unsigned short *>(Yv), t, n, N, gelu_as(v));
        } else {
            float *dst = static_cast<float *>(Yv) + (size_t)t * ldy + n;
            if constexpr (EPI == EPI_GELU) v = gelu_as(v);
            if constexpr (EPI == EPI_RESIDUAL) v = *dst + v;
            *dst = v;
        }
    }
}

// Y = epi(sum over splits of part[s] + bias), splits in order
template <int EPI>
__global__ __launch_bounds__(256) void k_gemv16_fold(const float *__restrict__ part, int S, int M, int N,
                                                     const float *__restrict__ bias, void *__restrict__ Yv, int ldy) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= M * N) return;
    const int t = i / N, n = i - t * N;
    float v = fold_splits(part + i, S, (size_t)M * N) + (bias ? bias[n] : 0.0f);
    if constexpr (EPI == EPI_GELU_H2) {
        h2_store(static_cast<unsigned short *>(Yv), t, n, N, gelu_as(v));
    } else {
        float *dst = static_cast<float *>(Yv) + (size_t)t * ldy + n;
        if constexpr (EPI == EPI_GELU) v = gelu_as(v);
        if constexpr (EPI == EPI_RESIDUAL) v = *dst + v;
        *dst = v;
    }
}

// FP32 rows -> H2 limbs (the same split as the LayerNorm's limb output), for
// callers that hold FP32 activations
__global__ __launch_bounds__(256) void k_to_h2(const float *__restrict__ x, int n4, int K,
                                               unsigned short *__restrict__ out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const int e = 4 * i, row = e / K;
    h2_store4(out, row, e - row * K, K, reinterpret_cast<const float4 *>(x)[i]);
}

hipError_t launch_to_h2(const float *x, int M, int K, unsigned short *out, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (K % 32 || reinterpret_cast<uintptr_t>(x) % 16) return hipErrorInvalidValue;
    const int n4 = M * K / 4;
    hipLaunchKernelGGL(k_to_h2, dim3((n4 + 255) / 256), dim3(256), 0, st, x, n4, K, out);
    return hipGetLastError();
}

bool gemv16_applies(const DevMatrix &W, int a_fmt, int M, int epi) {
    if (const char *e = getenv("CIH_GEMV16"); e && !std::strcmp(e, "0")) return false;
    return a_fmt == AF_H2 && M >= 1 && M <= GEMV_MAX_M && (W.fmt == WF_Q8 || W.fmt == WF_Q4) && W.N % 16 == 0 &&
           W.K % 32 == 0 && W.K > 0 &&
           (epi == EPI_NONE || epi == EPI_RESIDUAL || epi == EPI_GELU || epi == EPI_GELU_H2);
}

// k-blocks per round: 4 when K <= 1280 and N <= 1280 (few columns: more
// workgroups), else 8 while the splits stay within one fold chunk, else 20.
// CIH_GEMV16_KW=4/8/10/20 forces one.
Gemv16Grid gemv16_grid(int N, int K) {
    const int KB = K / 32;
    int kw = (KB <= 40 && N <= 1280) ? 4 : (KB <= 8 * FOLD_CHUNK ? 8 : 20);
    if (const char *e = getenv("CIH_GEMV16_KW")) {
        const int v = atoi(e);
        if (v == 4 || v == 8 || v == 10 || v == 20) kw = v;
    }
    Gemv16Grid g;
    g.kw = kw;
    g.splits = (KB + kw - 1) / kw;
    return g;
}

// activations of the AG form (GELU of a projection's splits + bias)
struct GeluIn {
    const float *part = nullptr;
    int S = 0;
    const float *bias = nullptr;
};

template <int WF, int KW>
static void launch_kw(const DevMatrix &W, const unsigned short *X, int M, const float *bias, void *Y, int ldy, int epi,
                      float *part, int S, const GeluIn &gi, const LnIn *ln, hipStream_t st) {
    const int KB = W.K / 32;
    const int rounds = (KB + S * KW - 1) / (S * KW);
    const dim3 grid((W.N + 63) / 64, S), block(256);
    const LnIn noln{nullptr, nullptr, nullptr, nullptr};
#define CIH_G16(E)                                                                                                  \
    hipLaunchKernelGGL((k_gemv16<WF, KW, E, false>), grid, block, 0, st, X, M, KB, W.q, W.sc, W.N, bias, Y, ldy,  \
                       part, rounds, nullptr, 0, nullptr, noln)
    if (ln) {  // gi: the residual's splits
        hipLaunchKernelGGL((k_gemv16<WF, KW, EPI_NONE, false, true>), grid, block, 0, st, nullptr, 1, KB, W.q, W.sc,
                           W.N, nullptr, nullptr, 0, part, rounds, gi.part, gi.S, gi.bias, *ln);
        return;
    }
    if (gi.part) {
        hipLaunchKernelGGL((k_gemv16<WF, KW, EPI_NONE, true>), grid, block, 0, st, nullptr, M, KB, W.q, W.sc, W.N,
                           nullptr, nullptr, 0, part, rounds, gi.part, gi.S, gi.bias, noln);
        return;
    }
    if (part) CIH_G16(EPI_NONE);
    else if (epi == EPI_RESIDUAL) CIH_G16(EPI_RESIDUAL);
    else if (epi == EPI_GELU) CIH_G16(EPI_GELU);
    else if (epi == EPI_GELU_H2) CIH_G16(EPI_GELU_H2);
    else CIH_G16(EPI_NONE);
#undef CIH_G16
}

static void launch_any(const DevMatrix &W, const unsigned short *X, int M, const float *bias, void *Y, int ldy,
                       int epi, float *part, int S, int kw, hipStream_t st, const GeluIn &gi = GeluIn(),
                       const LnIn *ln = nullptr) {
#define CIH_KW(WF)                                                                                                  \
    switch (kw) {                                                                                                  \
    case 4: launch_kw<WF, 4>(W, X, M, bias, Y, ldy, epi, part, S, gi, ln, st); break;                              \
    case 10: launch_kw<WF, 10>(W, X, M, bias, Y, ldy, epi, part, S, gi, ln, st); break;                            \
    case 20: launch_kw<WF, 20>(W, X, M, bias, Y, ldy, epi, part, S, gi, ln, st); break;                            \
    default: launch_kw<WF, 8>(W, X, M, bias, Y, ldy, epi, part, S, gi, ln, st);                                    \
    }
    if (W.fmt == WF_Q8) {
        CIH_KW(WF_Q8)
    } else {
        CIH_KW(WF_Q4)
    }
#undef CIH_KW
}

hipError_t launch_gemv16_partials(const DevMatrix &W, const unsigned short *X, int M, float *part, size_t part_floats,
                                  int *splits, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (!gemv16_applies(W, AF_H2, M, EPI_NONE) || !X || !part) return hipErrorInvalidValue;
    const Gemv16Grid g = gemv16_grid(W.N, W.K);
    if ((size_t)g.splits * M * W.N > part_floats) return hipErrorInvalidValue;
    launch_any(W, X, M, nullptr, nullptr, 0, EPI_NONE, part, g.splits, g.kw, st);
    *splits = g.splits;
    return hipGetLastError();
}

hipError_t launch_gemv16_gelu_partials(const DevMatrix &W, const float *apart, int aS, const float *abias, int M,
                                       float *part, size_t part_floats, int *splits, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (!gemv16_applies(W, AF_H2, M, EPI_NONE) || !apart || aS < 1 || !abias || !part) return hipErrorInvalidValue;
    const Gemv16Grid g = gemv16_grid(W.N, W.K);
    if ((size_t)g.splits * M * W.N > part_floats) return hipErrorInvalidValue;
    GeluIn gi;
    gi.part = apart;
    gi.S = aS;
    gi.bias = abias;
    launch_any(W, nullptr, M, nullptr, nullptr, 0, EPI_NONE, part, g.splits, g.kw, st, gi);
    *splits = g.splits;
    return hipGetLastError();
}

hipError_t launch_gemv16_ln_partials(const DevMatrix &W, const float *x, float *xo, const float *rpart, int rS,
                                     const float *rbias, const float *lnw, const float *lnb, float *part,
                                     size_t part_floats, int *splits, hipStream_t st) {
    if (!gemv16_applies(W, AF_H2, 1, EPI_NONE) || W.K > GEMV16_LN_MAX_K || !x || !xo || x == xo || !lnw || !lnb ||
        !part || (rpart && (rS < 1 || !rbias)))
        return hipErrorInvalidValue;
    const Gemv16Grid g = gemv16_grid(W.N, W.K);
    if ((size_t)g.splits * W.N > part_floats) return hipErrorInvalidValue;
    GeluIn ri;
    ri.part = rpart;
    ri.S = rpart ? rS : 0;
    ri.bias = rbias;
    const LnIn ln{x, xo, lnw, lnb};
    launch_any(W, nullptr, 1, nullptr, nullptr, 0, EPI_NONE, part, g.splits, g.kw, st, ri, &ln);
    *splits = g.splits;
    return hipGetLastError();
}

hipError_t launch_gemv16_fold(const float *part, int S, int M, int N, const float *bias, void *Y, int ldy, int epi,
                              hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (!part || S < 1 || !Y || (epi != EPI_GELU_H2 && ldy < N) || (epi == EPI_GELU_H2 && N % 32)) return hipErrorInvalidValue;
    const dim3 grid((M * N + 255) / 256), block(256);
    switch (epi) {
    case EPI_NONE: hipLaunchKernelGGL(k_gemv16_fold<EPI_NONE>, grid, block, 0, st, part, S, M, N, bias, Y, ldy); break;
    case EPI_RESIDUAL:
        hipLaunchKernelGGL(k_gemv16_fold<EPI_RESIDUAL>, grid, block, 0, st, part, S, M, N, bias, Y, ldy);
        break;
    case EPI_GELU: hipLaunchKernelGGL(k_gemv16_fold<EPI_GELU>, grid, block, 0, st, part, S, M, N, bias, Y, ldy); break;
    case EPI_GELU_H2:
        hipLaunchKernelGGL(k_gemv16_fold<EPI_GELU_H2>, grid, block, 0, st, part, S, M, N, bias, Y, ldy);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv16(const DevMatrix &W, const unsigned short *X, int M, const float *bias, void *Y, int ldy,
                         int epi, const PartialBuf *pb, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (!gemv16_applies(W, AF_H2, M, epi) || !X || !Y || (epi != EPI_GELU_H2 && ldy < W.N) ||
        (epi == EPI_GELU_H2 && W.N % 32))
        return hipErrorInvalidValue;
    const Gemv16Grid g = gemv16_grid(W.N, W.K);
    // the path depends on the shape only: split when the partial sums fit the cap
    const size_t need = (size_t)g.splits * M * W.N;
    if (g.splits > 1 && need <= GEMV16_SPLIT_MAX_FLOATS) {
        if (!pb || !pb->part || pb->floats < need) return hipErrorInvalidValue;
        launch_any(W, X, M, nullptr, nullptr, 0, EPI_NONE, pb->part, g.splits, g.kw, st);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        return launch_gemv16_fold(pb->part, g.splits, M, W.N, bias, Y, ldy, epi, st);
    }
    launch_any(W, X, M, bias, Y, ldy, epi, nullptr, 1, g.kw, st);  // one split: the whole K per workgroup
    return hipGetLastError();
}

}  // namespace cih
