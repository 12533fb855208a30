// Kernels of the few-token forward (at most GEMV_MAX_M tokens in the batch),
// which consume the split-K partial sums of the f16-MFMA GEMV (k_gemv16)
// themselves instead of a separate reduction:
//
//   k_rln       residual + LayerNorm: x += bias + (sum of the splits of the
//               previous projection), then out = LN(x) (the projection's
//               residual epilogue and layer_norm, lib.rs:2556-2562)
//   k_attn_few  the QKV splits + bias, RoPE, scores, softmax and P.V of one
//               (sequence, head) in FP32 (attention of lib.rs:5206-5301 without
//               a probability export)
//
// Partial sums are added in split order (fold_splits), so results do not
// depend on scheduling.
#include <algorithm>
#include <cmath>

#include "head_wo.h"
#include "kernels.h"
#include "x3.h"

namespace cih {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int FEW_THREADS = 256;
constexpr int RLN_MAX_THREADS = 1024;

}  // namespace

// One workgroup per row; thread t owns column quads t, t + blockDim, ... (Q of
// them), so that every partial sum of a row is requested at once.  part (may
// be null): [S][rows][d] partial sums of the projection whose residual is
// added, with bias pb (x + (sum + bias), the split GEMM's reduction order).
// The row's mean and variance are then formed by wave 0 exactly as
// k_layernorm4 forms them (lane l sums quads l, l + 64, ... in order, then a
// butterfly), so the output does not depend on which kernel normalised it.
template <int Q, int OF>
__global__ __launch_bounds__(RLN_MAX_THREADS) void k_rln(float *__restrict__ x, const float *__restrict__ part, int S,
                                                         const float *__restrict__ pb, const float *__restrict__ w,
                                                         const float *__restrict__ b, void *__restrict__ out,
                                                         int rows, int d, int *__restrict__ flag) {
    __shared__ f32x4 xs[Q * RLN_MAX_THREADS];
    __shared__ float stat[2];
    const int row = blockIdx.x, n4 = d >> 2, nt = blockDim.x;
    f32x4 *xr = reinterpret_cast<f32x4 *>(x + (size_t)row * d);
    f32x4 v[Q], g[Q], be[Q];
#pragma unroll
    for (int i = 0; i < Q; i++) {
        const int c = min((int)threadIdx.x + nt * i, n4 - 1);  // past the row: re-read, masked below
        v[i] = xr[c];
        g[i] = reinterpret_cast<const f32x4 *>(w)[c];
        be[i] = reinterpret_cast<const f32x4 *>(b)[c];
    }
    if (part) {
        const size_t stride = (size_t)rows * d;
#pragma unroll
        for (int i = 0; i < Q; i++) {
            const int c = min((int)threadIdx.x + nt * i, n4 - 1);
            const f32x4 acc = fold_splits4(part + (size_t)row * d + 4 * c, S, stride);
            const f32x4 bb = reinterpret_cast<const f32x4 *>(pb)[c];
            v[i] = v[i] + (acc + bb);
            if ((int)threadIdx.x + nt * i < n4) xr[c] = v[i];
        }
    }
#pragma unroll
    for (int i = 0; i < Q; i++)
        if ((int)threadIdx.x + nt * i < n4) xs[threadIdx.x + nt * i] = v[i];
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        float mean, var;
        row_stats64(xs, n4, d, lane, mean, var);
        if (lane == 0) {
            stat[0] = mean;
            stat[1] = 1.0f / sqrtf(var + 1e-5f);
            if (flag && !(__builtin_isfinite(mean) && __builtin_isfinite(var))) atomicOr(flag, FLAG_NONFINITE);
        }
    }
    __syncthreads();
    const float mean = stat[0], inv = stat[1];
#pragma unroll
    for (int i = 0; i < Q; i++) {
        const int c = threadIdx.x + nt * i;
        if (c >= n4) break;
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            y[e] = g[i][e] * (v[i][e] - mean) * inv + be[i][e];
            flag_limb_range(flag, y[e]);
        }
        if constexpr (OF == AF_H2)
            h2_store4(reinterpret_cast<unsigned short *>(out), row, 4 * c, d, make_float4(y.x, y.y, y.z, y.w));
        else
            reinterpret_cast<f32x4 *>(out)[(size_t)row * n4 + c] = y;
    }
}

// The same for many rows: one wave per row, four rows per workgroup, lane l
// owning column quads l, l + 64, ... (PER of them) as k_layernorm4 does; the
// fold, the mean and variance sums and their order are k_rln's, so both give
// the same bits.  The splits are folded 8 at a time and the LayerNorm's
// weights read after the row's statistics, so that the kernel keeps a few
// waves per SIMD at d = 2560 (PER 10: 256 -> ~100 VGPRs).
template <int PER, int OF>
__global__ __launch_bounds__(256) void k_rln4(float *__restrict__ x, const float *__restrict__ part, int S,
                                              const float *__restrict__ pb, const float *__restrict__ w,
                                              const float *__restrict__ b, void *__restrict__ out, int rows, int d,
                                              int *__restrict__ flag) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int n4 = d >> 2;
    f32x4 *xr = reinterpret_cast<f32x4 *>(x + (size_t)row * d);
    f32x4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) v[i] = xr[min(lane + 64 * i, n4 - 1)];  // past the row: re-read, masked below
    if (part) {
        const size_t stride = (size_t)rows * d;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int c = min(lane + 64 * i, n4 - 1);
            const f32x4 acc = fold_splits4<8>(part + (size_t)row * d + 4 * c, S, stride);
            const f32x4 bb = reinterpret_cast<const f32x4 *>(pb)[c];
            v[i] = v[i] + (acc + bb);
            if (lane + 64 * i < n4) xr[c] = v[i];
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++)
        if (lane + 64 * i < n4) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    const float mean = s / (float)d;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const f32x4 t = v[i] - mean;
        if (lane + 64 * i < n4) q += (t.x * t.x + t.y * t.y) + (t.z * t.z + t.w * t.w);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o);
    const float var = q / (float)d;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    if (flag && lane == 0 && !(__builtin_isfinite(mean) && __builtin_isfinite(var))) atomicOr(flag, FLAG_NONFINITE);
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = lane + 64 * i;
        if (c >= n4) break;
        const f32x4 g = reinterpret_cast<const f32x4 *>(w)[c], be = reinterpret_cast<const f32x4 *>(b)[c];
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            y[e] = g[e] * (v[i][e] - mean) * inv + be[e];
            flag_limb_range(flag, y[e]);
        }
        if constexpr (OF == AF_H2)
            h2_store4(reinterpret_cast<unsigned short *>(out), row, 4 * c, d, make_float4(y.x, y.y, y.z, y.w));
        else
            reinterpret_cast<f32x4 *>(out)[(size_t)row * n4 + c] = y;
    }
}

template <int OF>
static hipError_t launch_rln_t(float *x, const float *part, int S, const float *pbias, const float *w, const float *b,
                               void *out, int rows, int d, int *flag, hipStream_t st) {
    const int n4 = d / 4;
    // many rows: one wave each, four rows per workgroup (the few-row form
    // spreads a row over up to 1024 threads: faster below ~1024 rows)
    if (rows >= 1024 && n4 <= 640) {
        const int per = (n4 + 63) / 64;
        const dim3 grid4((rows + 3) / 4), blk4(256);
#define CIH_RLN4(P) hipLaunchKernelGGL((k_rln4<P, OF>), grid4, blk4, 0, st, x, part, S, pbias, w, b, out, rows, d, flag)
        if (per <= 2) CIH_RLN4(2);
        else if (per == 3) CIH_RLN4(3);
        else if (per == 4) CIH_RLN4(4);
        else if (per == 5) CIH_RLN4(5);
        else CIH_RLN4(10);
#undef CIH_RLN4
        return hipGetLastError();
    }
    const int q = (n4 + RLN_MAX_THREADS - 1) / RLN_MAX_THREADS;
    const int nt = (n4 + q - 1) / q;
    const dim3 grid(rows), blk((nt + 63) / 64 * 64);
#define CIH_RLN(QV) hipLaunchKernelGGL((k_rln<QV, OF>), grid, blk, 0, st, x, part, S, pbias, w, b, out, rows, d, flag)
    if (q <= 1) CIH_RLN(1);
    else if (q <= 2) CIH_RLN(2);
    else return hipErrorInvalidValue;
#undef CIH_RLN
    return hipGetLastError();
}

hipError_t launch_residual_layernorm(float *x, const float *part, int S, const float *pbias, const float *w,
                                     const float *b, void *out, int out_fmt, int rows, int d, hipStream_t st,
                                     int *flag) {
    if (rows <= 0) return hipSuccess;
    if (d % 32 || d > 8 * RLN_MAX_THREADS || (part && (S < 1 || !pbias)) || (out_fmt != AF_H2 && out_fmt != AF_F32))
        return hipErrorInvalidValue;
    return out_fmt == AF_H2 ? launch_rln_t<AF_H2>(x, part, S, pbias, w, b, out, rows, d, flag, st)
                            : launch_rln_t<AF_F32>(x, part, S, pbias, w, b, out, rows, d, flag, st);
}

// One workgroup per (sequence, head), n <= GEMV_MAX_M tokens.  q, k, v of the
// head: the QKV splits in order + bias (part: [S][T][3d]); RoPE (apply_rope,
// lib.rs:3533-3552, products rounded one by one); scores (q . k) / sqrt(hd),
// softmax (lib.rs:3500-3504: max, exp(s - max), * 1/sum; the row's max and
// sum over a shuffle tree) and out = P V, all FP32; out in H2 limbs (the Wo
// GEMV's operand) or FP32.  A thread takes one item of the head's columns of
// all T rows (nothing waits for the sequence's offset before the loads): a
// q or k dim-quad pair (4j..4j+3 and its RoPE partners + hd/2), rotated in
// registers, or a v quad; every split is requested at once, four floats per
// load, with the bias.
constexpr int ATTF_THREADS = 512;
template <int OF>
__global__ __launch_bounds__(ATTF_THREADS) void k_attn_few(const float *__restrict__ part, int S, int T,
                                                           const float *__restrict__ bias, int d, int hd,
                                                           const int *__restrict__ cu, const int *__restrict__ lens,
                                                           int S_max, const float *__restrict__ rc,
                                                           const float *__restrict__ rs, float inv_scale,
                                                           void *__restrict__ out) {
    constexpr int RW = FEW_MAX_HD + 4;  // padded rows: the 8 key rows of a score read hit distinct banks
    __shared__ float qkv[3][GEMV_MAX_M][RW];
    __shared__ float p[GEMV_MAX_M][GEMV_MAX_M];
    const int b = blockIdx.x, h = blockIdx.y;
    const int half = hd / 2, hq = hd / 4, pq = hd / 8;  // quads per row, pairs per row
    const size_t stride = (size_t)T * 3 * d;
    const int len = lens[b], r0 = cu[b];
    // items: [0, 2 T pq) q/k pairs (which, row, pair), then T hq v quads
    const int nqk = 2 * T * pq, nitem = nqk + T * hq;
    const int it = min((int)threadIdx.x, nitem - 1);  // past the end: re-read, unused
    const bool pair = it < nqk;
    int which, r, j;  // j: first dim of the (lower) quad
    if (pair) {
        which = it / (T * pq);
        const int rem = it - which * T * pq;
        r = rem / pq;
        j = 4 * (rem - r * pq);
    } else {
        which = 2;
        const int rem = it - nqk;
        r = rem / hq;
        j = 4 * (rem - r * hq);
    }
    const float *src = part + (size_t)r * 3 * d + which * d + h * hd + j;
    const int up = pair ? half : 0;  // the partner quad
    fold4_t a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < S; s0 += FOLD_CHUNK) {
        fold4_t v0[FOLD_CHUNK], v1[FOLD_CHUNK];
#pragma unroll
        for (int u = 0; u < FOLD_CHUNK; u++) {
            const bool in = s0 + u < S;
            v0[u] = in ? *reinterpret_cast<const fold4_t *>(src + (size_t)(s0 + u) * stride) : fold4_t{0.0f, 0.0f, 0.0f, 0.0f};
            v1[u] = in && pair ? *reinterpret_cast<const fold4_t *>(src + up + (size_t)(s0 + u) * stride)
                               : fold4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < FOLD_CHUNK; u++) {
            a0 += v0[u];
            a1 += v1[u];
        }
    }
    const float *bp = bias + which * d + h * hd + j;
    a0 += *reinterpret_cast<const fold4_t *>(bp);
    if (pair) a1 += *reinterpret_cast<const fold4_t *>(bp + up);
    const int n = min(len, GEMV_MAX_M), pos = r - r0;
    if (pair && pos >= 0 && pos < n) {
        const fold4_t c = *reinterpret_cast<const fold4_t *>(rc + (size_t)pos * half + j);
        const fold4_t sn = *reinterpret_cast<const fold4_t *>(rs + (size_t)pos * half + j);
        fold4_t lo, hi;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            lo[t] = __fsub_rn(__fmul_rn(a0[t], c[t]), __fmul_rn(a1[t], sn[t]));
            hi[t] = __fadd_rn(__fmul_rn(a1[t], c[t]), __fmul_rn(a0[t], sn[t]));
        }
        a0 = lo;
        a1 = hi;
    }
    if ((int)threadIdx.x < nitem) {
        *reinterpret_cast<fold4_t *>(&qkv[which][r][j]) = a0;
        if (pair) *reinterpret_cast<fold4_t *>(&qkv[which][r][j + half]) = a1;
    }
    if (n <= 0) return;  // uniform: no barrier follows for this workgroup
    __syncthreads();
    // scores and softmax: lane 8 i + j of wave 0 holds (query i, key j); a
    // row's lanes meet through shuffles
    if (threadIdx.x < 64) {
        const int i = threadIdx.x >> 3, j = threadIdx.x & 7;
        const bool live = i < n && j < n;
        const f32x4 *qr = reinterpret_cast<const f32x4 *>(qkv[0][r0 + min(i, n - 1)]);
        const f32x4 *kr = reinterpret_cast<const f32x4 *>(qkv[1][r0 + min(j, n - 1)]);
        float a = 0.0f;
#pragma unroll 8
        for (int k = 0; k < hq; k++) {
            const f32x4 x = qr[k], y = kr[k];
            a = fmaf(x.x, y.x, a);
            a = fmaf(x.y, y.y, a);
            a = fmaf(x.z, y.z, a);
            a = fmaf(x.w, y.w, a);
        }
        const float sc = live ? a * inv_scale : -INFINITY;
        float mx = sc;
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float e = live ? expf(sc - mx) : 0.0f;
        float sum = e;
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) sum += __shfl_xor(sum, o);
        p[i][j] = e * (1.0f / sum);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < n * hd; e += ATTF_THREADS) {
        const int i = e / hd, j = e - i * hd;
        float a = 0.0f;
#pragma unroll
        for (int t = 0; t < GEMV_MAX_M; t++)
            if (t < n) a = fmaf(p[i][t], qkv[2][r0 + t][j], a);
        if constexpr (OF == AF_H2) h2_store(static_cast<unsigned short *>(out), r0 + i, h * hd + j, d, a);
        else static_cast<float *>(out)[(size_t)(r0 + i) * d + h * hd + j] = a;
    }
}

// k_attn_few followed by this head's share of the output projection Wo
// (Q8_0 / Q4_0, k-block-major), for head sizes that are whole 32-wide
// blocks: workgroup (sequence b, head h, column chunk z) forms the head's
// output o (n tokens x hd, FP32, in LDS) as k_attn_few does, splits it into
// f16 limbs as the GEMV's operand (A row = token + 8 limb, lane l holds
// A[l % 16][8 (l / 16) ..]) and multiplies it by Wo's k-blocks of the head
// for columns [z ncols, (z + 1) ncols) on v_mfma_f32_16x16x32_f16, each
// block's sum times its scale, as k_gemv16 does.  opart [H][T][N]: the head
// is the split, which the residual LayerNorm after it adds (with bo).
template <int WF>
__global__ __launch_bounds__(ATTF_THREADS) void k_attn_few_wo(const float *__restrict__ part, int S, int T,
                                                              const float *__restrict__ bias, int d, int hd,
                                                              const int *__restrict__ cu, const int *__restrict__ lens,
                                                              const float *__restrict__ rc,
                                                              const float *__restrict__ rs, float inv_scale,
                                                              const unsigned char *__restrict__ Wq,
                                                              const float *__restrict__ Wsc, int N, int ncols,
                                                              float *__restrict__ opart) {
    constexpr int RW = FEW_MAX_HD + 4;
    __shared__ float qkv[3][GEMV_MAX_M][RW];
    __shared__ float p[GEMV_MAX_M][GEMV_MAX_M];
    const int b = blockIdx.x, h = blockIdx.y;
    const int half = hd / 2, hq = hd / 4, pq = hd / 8;
    const size_t stride = (size_t)T * 3 * d;
    const int len = lens[b], r0 = cu[b];
    // q, k, v of the head, folded, with RoPE (as k_attn_few)
    const int nqk = 2 * T * pq, nitem = nqk + T * hq;
    const int it = min((int)threadIdx.x, nitem - 1);
    const bool pair = it < nqk;
    int which, r, j;
    if (pair) {
        which = it / (T * pq);
        const int rem = it - which * T * pq;
        r = rem / pq;
        j = 4 * (rem - r * pq);
    } else {
        which = 2;
        const int rem = it - nqk;
        r = rem / hq;
        j = 4 * (rem - r * hq);
    }
    // this workgroup's Wo columns and the head's k-blocks: weights and scales
    // requested first (they depend on nothing this layer computes), so their
    // latency runs under the fold's and the attention's
    const int nkb = hd / 32, c0 = (int)blockIdx.z * ncols, c1 = min(c0 + ncols, N);
    HeadWo<WF, 1> wo;
    wo.load(Wq, Wsc, N, h * nkb, nkb, c0, c1);
    // the QKV projection's splits in chunks of 10 (its GEMV leaves at most 10
    // for d <= 2560; the additions stay in split order), so that the weights
    // above fit beside them in registers
    constexpr int WO_FOLD = 10;
    const float *src = part + (size_t)r * 3 * d + which * d + h * hd + j;
    const int up = pair ? half : 0;
    fold4_t a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < S; s0 += WO_FOLD) {
        fold4_t v0[WO_FOLD], v1[WO_FOLD];
#pragma unroll
        for (int u = 0; u < WO_FOLD; u++) {
            const bool in = s0 + u < S;
            v0[u] = in ? *reinterpret_cast<const fold4_t *>(src + (size_t)(s0 + u) * stride) : fold4_t{0.0f, 0.0f, 0.0f, 0.0f};
            v1[u] = in && pair ? *reinterpret_cast<const fold4_t *>(src + up + (size_t)(s0 + u) * stride)
                               : fold4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < WO_FOLD; u++) {
            a0 += v0[u];
            a1 += v1[u];
        }
    }
    const float *bp = bias + which * d + h * hd + j;
    a0 += *reinterpret_cast<const fold4_t *>(bp);
    if (pair) a1 += *reinterpret_cast<const fold4_t *>(bp + up);
    const int n = min(len, GEMV_MAX_M), pos = r - r0;
    if (pair && pos >= 0 && pos < n) {
        const fold4_t c = *reinterpret_cast<const fold4_t *>(rc + (size_t)pos * half + j);
        const fold4_t sn = *reinterpret_cast<const fold4_t *>(rs + (size_t)pos * half + j);
        fold4_t lo, hi;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            lo[t] = __fsub_rn(__fmul_rn(a0[t], c[t]), __fmul_rn(a1[t], sn[t]));
            hi[t] = __fadd_rn(__fmul_rn(a1[t], c[t]), __fmul_rn(a0[t], sn[t]));
        }
        a0 = lo;
        a1 = hi;
    }
    if ((int)threadIdx.x < nitem) {
        *reinterpret_cast<fold4_t *>(&qkv[which][r][j]) = a0;
        if (pair) *reinterpret_cast<fold4_t *>(&qkv[which][r][j + half]) = a1;
    }
    if (n <= 0) return;  // uniform: no barrier follows for this workgroup
    __syncthreads();
    // scores and softmax (as k_attn_few)
    if (threadIdx.x < 64) {
        const int i = threadIdx.x >> 3, jj = threadIdx.x & 7;
        const bool live = i < n && jj < n;
        const f32x4 *qr = reinterpret_cast<const f32x4 *>(qkv[0][r0 + min(i, n - 1)]);
        const f32x4 *kr = reinterpret_cast<const f32x4 *>(qkv[1][r0 + min(jj, n - 1)]);
        float a = 0.0f;
#pragma unroll 8
        for (int k = 0; k < hq; k++) {
            const f32x4 x = qr[k], y = kr[k];
            a = fmaf(x.x, y.x, a);
            a = fmaf(x.y, y.y, a);
            a = fmaf(x.z, y.z, a);
            a = fmaf(x.w, y.w, a);
        }
        const float sc = live ? a * inv_scale : -INFINITY;
        float mx = sc;
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float e = live ? expf(sc - mx) : 0.0f;
        float sum = e;
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) sum += __shfl_xor(sum, o);
        p[i][jj] = e * (1.0f / sum);
    }
    __syncthreads();
    // o = P v into the q rows of this sequence (q is no longer read)
    for (int e = threadIdx.x; e < n * hd; e += ATTF_THREADS) {
        const int i = e / hd, jj = e - i * hd;
        float a = 0.0f;
#pragma unroll
        for (int t = 0; t < GEMV_MAX_M; t++)
            if (t < n) a = fmaf(p[i][t], qkv[2][r0 + t][jj], a);
        qkv[0][r0 + i][jj] = a;
    }
    __syncthreads();
    wo.run(qkv[0][r0], RW, n, nkb, N, c0, c1, opart + ((size_t)h * T + r0) * N);
}

hipError_t launch_attention_few_wo(const float *part, int S, int T, const float *bias, const DevMatrix &Wo, int d,
                                   int H, const SeqMeta &sm, const float *rope_c, const float *rope_s, float *opart,
                                   size_t opart_floats, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    const int hd = H > 0 ? d / H : 0;
    if (T > GEMV_MAX_M || !part || S < 1 || !bias || hd <= 0 || hd * H != d || hd % 32 || hd > FEW_MAX_HD ||
        (Wo.fmt != WF_Q8 && Wo.fmt != WF_Q4) || Wo.K != d || Wo.N % 16 || !opart ||
        (size_t)H * T * Wo.N > opart_floats)
        return hipErrorInvalidValue;
    const float inv_scale = 1.0f / sqrtf((float)hd);
    // 128 columns per workgroup (8 waves x 16 columns, one pass; measured at
    // 650M, B=1, L=8: 1.207 ms per forward, 1.221 with 256, 1.252 with 512,
    // 1.248 with attention and Wo apart)
    const int ncols = 128, nz = (Wo.N + ncols - 1) / ncols;
    const dim3 grid(sm.B, H, nz), blk(ATTF_THREADS);
    const unsigned char *wq = static_cast<const unsigned char *>(Wo.q);
    if (Wo.fmt == WF_Q8)
        hipLaunchKernelGGL(k_attn_few_wo<WF_Q8>, grid, blk, 0, st, part, S, T, bias, d, hd, sm.cu, sm.lens, rope_c,
                           rope_s, inv_scale, wq, Wo.sc, Wo.N, ncols, opart);
    else
        hipLaunchKernelGGL(k_attn_few_wo<WF_Q4>, grid, blk, 0, st, part, S, T, bias, d, hd, sm.cu, sm.lens, rope_c,
                           rope_s, inv_scale, wq, Wo.sc, Wo.N, ncols, opart);
    return hipGetLastError();
}

hipError_t launch_attention_few(const float *part, int S, int T, const float *bias, int d, int H, const SeqMeta &sm,
                                const float *rope_c, const float *rope_s, void *out, int out_fmt, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    const int hd = H > 0 ? d / H : 0;
    if (T > GEMV_MAX_M || !part || S < 1 || !bias || hd <= 0 || hd * H != d || hd % 8 || hd > FEW_MAX_HD ||
        (out_fmt == AF_H2 && d % 32) || (out_fmt != AF_H2 && out_fmt != AF_F32))
        return hipErrorInvalidValue;
    const float inv_scale = 1.0f / sqrtf((float)hd);
    const dim3 grid(sm.B, H), blk(ATTF_THREADS);
    if (out_fmt == AF_H2)
        hipLaunchKernelGGL(k_attn_few<AF_H2>, grid, blk, 0, st, part, S, T, bias, d, hd, sm.cu, sm.lens, sm.S_max,
                           rope_c, rope_s, inv_scale, out);
    else
        hipLaunchKernelGGL(k_attn_few<AF_F32>, grid, blk, 0, st, part, S, T, bias, d, hd, sm.cu, sm.lens, sm.S_max,
                           rope_c, rope_s, inv_scale, out);
    return hipGetLastError();
}

}  // namespace cih
