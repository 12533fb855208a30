// Memory-bound kernels of the forward: embedding, LayerNorm, last-layer head
// mean, contact-map (APC) statistics and finalisation, output scatter.
#include "kernels.h"

namespace cih {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Embedding + token-dropout rescale (codon-infer src/lib.rs:5117-5131; Q8
// 5461-5479; Q4 5820-5833).  scale = 0.88 / (1 - mask_count/len) for the
// sequence's own length; <mask> (id 32) rows are zero.  The Q8 embedding is
// dequantized as q*d first and then scaled, as the reference does.
// One workgroup per (position, sequence); the mask count is recomputed per
// row from the sequence's tokens (len <= a few thousand ints).
__global__ __launch_bounds__(256) void k_embed(const int *__restrict__ tokens, const int *__restrict__ cu,
                                               const int *__restrict__ lens, int S_max, int fmt,
                                               const void *__restrict__ eq, const float *__restrict__ esc, int d,
                                               int V, float *__restrict__ x, int *__restrict__ flag) {
    const int s = blockIdx.x, b = blockIdx.y;
    const int len = lens[b];
    if (s >= len) return;
    const int *tk = tokens + (size_t)b * S_max;
    __shared__ int cnt[4];
    int c = 0;
    for (int i = threadIdx.x; i < len; i += 256) c += tk[i] == 32;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
    if ((threadIdx.x & 63) == 0) cnt[threadIdx.x >> 6] = c;
    __syncthreads();
    const int mask_count = cnt[0] + cnt[1] + cnt[2] + cnt[3];
    const float ratio = (float)mask_count / (float)len;
    const float scale = ratio >= 1.0f ? 0.0f : (1.0f - 0.12f) / (1.0f - ratio);
    // ids outside [0, V) cannot occur on host-pointer calls (validated
    // there); on device-pointer calls such an id sets FLAG_BAD_TOKEN, which
    // the host turns into CIH_ERR_TOKEN, and is clamped so that no read
    // leaves the table.
    const int t0 = tk[s], t = min(max(t0, 0), V - 1);
    if (t0 != t && flag && threadIdx.x == 0) atomicOr(flag, FLAG_BAD_TOKEN);
    float *xr = x + (size_t)(cu[b] + s) * d;
    for (int i = threadIdx.x; i < d; i += 256) {
        float v = 0.0f;
        if (t != 32) {
            const size_t blk = (size_t)(i >> 5) * V + t;  // k-block-major [d/32][V][32]
            float e;
            if (fmt == WF_Q8)
                e = (float)reinterpret_cast<const signed char *>(eq)[blk * 32 + (i & 31)] * esc[blk];
            else
                e = reinterpret_cast<const float *>(eq)[blk * 32 + (i & 31)];
            v = e * scale;
        }
        xr[i] = v;
    }
}

hipError_t launch_embed(const int *tokens, SeqMeta sm, int emb_fmt, const void *emb_q, const float *emb_sc, int d,
                        int V, float *x, hipStream_t st, int *flag) {
    hipLaunchKernelGGL(k_embed, dim3(sm.S_max, sm.B), dim3(256), 0, st, tokens, sm.cu, sm.lens, sm.S_max, emb_fmt,
                       emb_q, emb_sc, d, V, x, flag);
    return hipGetLastError();
}

// layer_norm (lib.rs:2556-2562): mean, variance of (x - mean), 1/sqrt(var +
// 1e-5), out = w * (x - mean) * inv + b.  One wave per row.
template <int PER, int OF>
__global__ __launch_bounds__(256) void k_layernorm(const float *__restrict__ x, const float *__restrict__ w,
                                                   const float *__restrict__ b, void *__restrict__ out, int rows,
                                                   int d, int *__restrict__ flag) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + (size_t)row * d;
    // gamma and beta are requested with the row, so their latency overlaps the reductions
    float v[PER], g[PER], be[PER];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = lane + 64 * i;
        v[i] = c < d ? xr[c] : 0.0f;
        g[i] = c < d ? w[c] : 0.0f;
        be[i] = c < d ? b[c] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < PER; i++) s += v[i];
    const float mean = wave_sum(s) / (float)d;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = lane + 64 * i;
        const float t = v[i] - mean;
        q += c < d ? t * t : 0.0f;
    }
    const float var = wave_sum(q) / (float)d;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    if (flag && lane == 0 && !(__builtin_isfinite(mean) && __builtin_isfinite(var))) atomicOr(flag, FLAG_NONFINITE);
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = lane + 64 * i;
        if (c < d) {
            const float y = g[i] * (v[i] - mean) * inv + be[i];
            flag_limb_range(flag, y);
            if constexpr (OF == AF_X3)
                x3_store(reinterpret_cast<unsigned short *>(out), row, c, d, y);
            else if constexpr (OF == AF_H2)
                h2_store(reinterpret_cast<unsigned short *>(out), row, c, d, y);
            else
                reinterpret_cast<float *>(out)[(size_t)row * d + c] = y;
        }
    }
}

// The same with four consecutive columns per lane (d % 4 == 0): 16-byte
// loads, and 8-byte stores per limb.
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <int PER, int OF>
__global__ __launch_bounds__(256) void k_layernorm4(const float *__restrict__ x, const float *__restrict__ w,
                                                    const float *__restrict__ b, void *__restrict__ out, int rows,
                                                    int d, int *__restrict__ flag) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(x + (size_t)row * d);
    const f32x4 *wr = reinterpret_cast<const f32x4 *>(w), *br = reinterpret_cast<const f32x4 *>(b);
    const int n4 = d >> 2;
    f32x4 v[PER], g[PER], be[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = min(lane + 64 * i, n4 - 1);  // lanes past the row re-read its last quad, masked below
        v[i] = xr[c];
        g[i] = wr[c];
        be[i] = br[c];
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++)
        if (lane + 64 * i < n4) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    const float mean = wave_sum(s) / (float)d;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const f32x4 t = v[i] - mean;
        if (lane + 64 * i < n4) q += (t.x * t.x + t.y * t.y) + (t.z * t.z + t.w * t.w);
    }
    const float var = wave_sum(q) / (float)d;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    if (flag && lane == 0 && !(__builtin_isfinite(mean) && __builtin_isfinite(var))) atomicOr(flag, FLAG_NONFINITE);
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = lane + 64 * i;
        if (c < n4) {
            f32x4 y;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                y[e] = g[i][e] * (v[i][e] - mean) * inv + be[i][e];
                flag_limb_range(flag, y[e]);
            }
            const float4 yy = make_float4(y.x, y.y, y.z, y.w);
            if constexpr (OF == AF_X3)
                x3_store4(reinterpret_cast<unsigned short *>(out), row, 4 * c, d, yy);
            else if constexpr (OF == AF_H2)
                h2_store4(reinterpret_cast<unsigned short *>(out), row, 4 * c, d, yy);
            else
                reinterpret_cast<f32x4 *>(out)[(size_t)row * n4 + c] = y;
        }
    }
}

template <int OF>
static hipError_t launch_ln_t(const float *x, const float *w, const float *b, void *out, int rows, int d,
                              int *flag, hipStream_t st) {
    const dim3 grid((rows + 3) / 4), blk(256);
    if (d % 4 == 0) {
        const int per4 = (d / 4 + 63) / 64;
        if (per4 <= 2) hipLaunchKernelGGL((k_layernorm4<2, OF>), grid, blk, 0, st, x, w, b, out, rows, d, flag);
        else if (per4 <= 5) hipLaunchKernelGGL((k_layernorm4<5, OF>), grid, blk, 0, st, x, w, b, out, rows, d, flag);
        else if (per4 <= 10) hipLaunchKernelGGL((k_layernorm4<10, OF>), grid, blk, 0, st, x, w, b, out, rows, d, flag);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    const int per = (d + 63) / 64;
    if (per <= 5) hipLaunchKernelGGL((k_layernorm<5, OF>), grid, blk, 0, st, x, w, b, out, rows, d, flag);
    else if (per <= 10) hipLaunchKernelGGL((k_layernorm<10, OF>), grid, blk, 0, st, x, w, b, out, rows, d, flag);
    else if (per <= 20) hipLaunchKernelGGL((k_layernorm<20, OF>), grid, blk, 0, st, x, w, b, out, rows, d, flag);
    else if (per <= 40) hipLaunchKernelGGL((k_layernorm<40, OF>), grid, blk, 0, st, x, w, b, out, rows, d, flag);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_layernorm(const float *x, const float *w, const float *b, void *out, int out_fmt, int rows, int d,
                            hipStream_t st, int *flag) {
    if (rows <= 0) return hipSuccess;
    if (out_fmt == AF_X3) return d % 32 ? hipErrorInvalidValue : launch_ln_t<AF_X3>(x, w, b, out, rows, d, flag, st);
    if (out_fmt == AF_H2) return d % 32 ? hipErrorInvalidValue : launch_ln_t<AF_H2>(x, w, b, out, rows, d, flag, st);
    return launch_ln_t<AF_F32>(x, w, b, out, rows, d, flag, st);
}

// final_layer_att (lib.rs:5201-5204, 5256-5261): acc = 0; acc += P_h * (1/H)
// in ascending h.
__global__ __launch_bounds__(256) void k_head_mean(const float *__restrict__ P, long long pb, long long ph, int H,
                                                   const int *__restrict__ lens, int S_max,
                                                   float *__restrict__ fa) {
    const int p = blockIdx.x, b = blockIdx.y;
    const int len = lens[b];
    if (p >= len) return;
    const float hw = 1.0f / (float)H;
    for (int t = threadIdx.x; t < len; t += 256) {
        float acc = 0.0f;
        for (int h = 0; h < H; h++) acc += P[b * pb + h * ph + (size_t)p * S_max + t] * hw;
        fa[((size_t)b * S_max + p) * S_max + t] = acc;
    }
}

// The same sums with four keys per thread and every head's load issued
// before the first addition (HM >= H heads, loads past H predicated off); the
// additions stay in ascending h, so the bits are k_head_mean's.  Needs P, the
// strides and S_max 16-byte aligned.
template <int HM>
__global__ __launch_bounds__(128) void k_head_mean4(const float *__restrict__ P, long long pb, long long ph, int H,
                                                    const int *__restrict__ lens, int S_max,
                                                    float *__restrict__ fa) {
    const int p = blockIdx.x, b = blockIdx.y;
    const int len = lens[b];
    if (p >= len) return;
    const float hw = 1.0f / (float)H;
    const float *src = P + b * pb + (size_t)p * S_max;
    float *dst = fa + ((size_t)b * S_max + p) * S_max;
    for (int t = threadIdx.x * 4; t < len; t += 512) {
        float4 v[HM];
#pragma unroll
        for (int h = 0; h < HM; h++)
            v[h] = h < H ? *reinterpret_cast<const float4 *>(src + h * ph + t) : make_float4(0.f, 0.f, 0.f, 0.f);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int h = 0; h < HM; h++) {
            if (h < H) {
                acc[0] += v[h].x * hw;
                acc[1] += v[h].y * hw;
                acc[2] += v[h].z * hw;
                acc[3] += v[h].w * hw;
            }
        }
        if (t + 4 <= len) {
            *reinterpret_cast<float4 *>(dst + t) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (t + e < len) dst[t + e] = acc[e];
        }
    }
}

hipError_t launch_head_mean(const float *P, int64_t pb, int64_t ph, int H, SeqMeta sm, float *final_att,
                            hipStream_t st) {
    const bool al = ((uintptr_t)P & 15) == 0 && ((uintptr_t)final_att & 15) == 0 && ((pb | ph | sm.S_max) & 3) == 0;
    if (al && H <= 20)
        hipLaunchKernelGGL(k_head_mean4<20>, dim3(sm.S_max, sm.B), dim3(128), 0, st, P, (long long)pb, (long long)ph,
                           H, sm.lens, sm.S_max, final_att);
    else if (al && H <= 40)
        hipLaunchKernelGGL(k_head_mean4<40>, dim3(sm.S_max, sm.B), dim3(128), 0, st, P, (long long)pb, (long long)ph,
                           H, sm.lens, sm.S_max, final_att);
    else
        hipLaunchKernelGGL(k_head_mean, dim3(sm.S_max, sm.B), dim3(256), 0, st, P, (long long)pb, (long long)ph, H,
                           sm.lens, sm.S_max, final_att);
    return hipGetLastError();
}

// ---- contacts: accumulate_head_apc (lib.rs:5036-5076) restated over a batch.
// For a head with weight w and residue block A (rows/cols 1..n of P):
//   s_ij = A_ij + A_ji, r_i = sum_j s_ij, T = sum_i r_i,
//   logit_ij += w * (s_ij - (r_i / T) * r_j)
// Summed over heads: logit = M + M^T - sum_h (w_h / T_h) r_h r_h^T with
// M = sum_h w_h A_h, and r_i = (row sum of A)_i + (column sum of A)_i.  The
// attention kernel supplies the row sums; k_apc_tile reads each map once,
// accumulating M and per-32-row column partial sums, which k_apc_r adds in
// order.  M: [B][n_max][n_max], r: [L*H][B][n_max], n_max = S_max - 2.
constexpr int APC_ROWS = 32;  // map rows per workgroup of k_apc_tile
constexpr int APC_HMAX = 40;  // most heads of any preset (3B)

// HM >= nz heads per pass with branch-free loads (heads past nz repeat head
// nz - 1 with weight 0 and are not written), two map rows per step, so a
// thread has 2 * HM loads in flight.
template <int HM>
__global__ __launch_bounds__(256) void k_apc_tile(const float *__restrict__ P, long long pb, long long ph, int H,
                                                  int l, const float *__restrict__ w, const int *__restrict__ heads,
                                                  int nz, const int *__restrict__ lens, int S_max,
                                                  float *__restrict__ M, float *__restrict__ colpart, int B) {
    const int tile = blockIdx.x, b = blockIdx.z;
    const int n = lens[b] - 2, n_max = S_max - 2, ntiles = (n_max + APC_ROWS - 1) / APC_ROWS;
    const int j = blockIdx.y * 256 + threadIdx.x;  // residue column
    const int i0 = tile * APC_ROWS;
    if (j >= n || i0 >= n) return;
    const int i1 = min(i0 + APC_ROWS, n);
    long long off[HM];
    float wk[HM], cs[HM];
#pragma unroll
    for (int k = 0; k < HM; k++) {
        const int h = heads[min(k, nz - 1)];
        off[k] = h * ph;
        wk[k] = k < nz ? w[l * H + h] : 0.0f;
        cs[k] = 0.0f;
    }
    const float *P0 = P + b * pb + S_max + 1 + j;  // row i + 1, column j + 1
    float *M0 = M + (size_t)b * n_max * n_max + j;
    int i = i0;
    for (; i + 2 <= i1; i += 2) {
        const float *r0 = P0 + (size_t)i * S_max, *r1 = r0 + S_max;
        float a0[HM], a1[HM];
#pragma unroll
        for (int k = 0; k < HM; k++) {
            a0[k] = r0[off[k]];
            a1[k] = r1[off[k]];
        }
        float acc0 = M0[(size_t)i * n_max], acc1 = M0[(size_t)(i + 1) * n_max];
#pragma unroll
        for (int k = 0; k < HM; k++) {
            acc0 += wk[k] * a0[k];
            cs[k] += a0[k];
        }
#pragma unroll
        for (int k = 0; k < HM; k++) {
            acc1 += wk[k] * a1[k];
            cs[k] += a1[k];
        }
        M0[(size_t)i * n_max] = acc0;
        M0[(size_t)(i + 1) * n_max] = acc1;
    }
    if (i < i1) {
        const float *r0 = P0 + (size_t)i * S_max;
        float acc0 = M0[(size_t)i * n_max];
#pragma unroll
        for (int k = 0; k < HM; k++) {
            const float a = r0[off[k]];
            acc0 += wk[k] * a;
            cs[k] += a;
        }
        M0[(size_t)i * n_max] = acc0;
    }
#pragma unroll
    for (int k = 0; k < HM; k++)
        if (k < nz) colpart[(((size_t)b * H + heads[k]) * ntiles + tile) * n_max + j] = cs[k];
}

// r[l*H + h][b][i] = rowsum[b][h][i+1] + column partials of i in tile order
__global__ __launch_bounds__(256) void k_apc_r(const float *__restrict__ rowsum, const float *__restrict__ colpart,
                                               int H, int l, const int *__restrict__ heads,
                                               const int *__restrict__ lens, int S_max, float *__restrict__ r,
                                               int B) {
    const int b = blockIdx.z, h = heads[blockIdx.y];
    const int n = lens[b] - 2, n_max = S_max - 2, ntiles = (n_max + APC_ROWS - 1) / APC_ROWS;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float c = 0.0f;
    const int nt = (n + APC_ROWS - 1) / APC_ROWS;
    for (int t = 0; t < nt; t++) c += colpart[(((size_t)b * H + h) * ntiles + t) * n_max + i];
    r[((size_t)(l * H + h) * B + b) * n_max + i] = rowsum[((size_t)b * H + h) * S_max + i + 1] + c;
}

hipError_t launch_apc_layer(const float *P, int64_t pb, int64_t ph, int H, int l, const float *w_dev,
                            const int *heads_dev, int n_heads_nz, SeqMeta sm, const float *rowsum, float *colpart,
                            float *M, float *r, hipStream_t st) {
    if (n_heads_nz <= 0 || sm.S_max < 3) return hipSuccess;
    if (n_heads_nz > APC_HMAX || H > APC_HMAX) return hipErrorInvalidValue;
    const int n_max = sm.S_max - 2;
    const dim3 tg((n_max + APC_ROWS - 1) / APC_ROWS, (n_max + 255) / 256, sm.B);
    if (n_heads_nz <= 20)
        hipLaunchKernelGGL(k_apc_tile<20>, tg, dim3(256), 0, st, P, (long long)pb, (long long)ph, H, l, w_dev, heads_dev,
                           n_heads_nz, sm.lens, sm.S_max, M, colpart, sm.B);
    else
        hipLaunchKernelGGL(k_apc_tile<APC_HMAX>, tg, dim3(256), 0, st, P, (long long)pb, (long long)ph, H, l, w_dev,
                           heads_dev, n_heads_nz, sm.lens, sm.S_max, M, colpart, sm.B);
    hipLaunchKernelGGL(k_apc_r, dim3((n_max + 255) / 256, n_heads_nz, sm.B), dim3(256), 0, st, rowsum, colpart, H, l,
                       heads_dev, sm.lens, sm.S_max, r, sm.B);
    return hipGetLastError();
}

// coef[lh][b] = w_lh / T_lh (0 when |T| <= 1e-12 or w == 0), T = sum_i r_i
__global__ __launch_bounds__(256) void k_apc_coef(const float *__restrict__ r, const float *__restrict__ w,
                                                  const int *__restrict__ lens, int S_max, int B,
                                                  float *__restrict__ coef) {
    const int lh = blockIdx.x, b = blockIdx.y;
    const int n = lens[b] - 2, n_max = S_max - 2;
    __shared__ float red[4];
    float s = 0.0f;
    if (w[lh] != 0.0f)
        for (int i = threadIdx.x; i < n; i += 256) s += r[((size_t)lh * B + b) * n_max + i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float T = red[0] + red[1] + red[2] + red[3];
        coef[(size_t)lh * B + b] = (w[lh] != 0.0f && fabsf(T) > 1e-12f) ? w[lh] * (1.0f / T) : 0.0f;
    }
}

// A 64 x 64 block of contacts per workgroup, 4 x 4 per thread (rows
// i0 + 4ty + m, columns j0 + 4tx + k); the r vectors of 64 layer-heads at a
// time are staged in LDS, where a thread's four rows and four columns are one
// 16-byte read each.  Per output the arithmetic is the one-thread-per-output
// form: corr = fma(c, r_i * r_j, corr) in layer-head order, skipping c == 0.
constexpr int APC_FT = 64, APC_FL = 64;
__global__ __launch_bounds__(256) void k_apc_final(const float *__restrict__ M, const float *__restrict__ r,
                                                   const float *__restrict__ coef, int LH, const int *__restrict__ lens,
                                                   int S_max, int B, float bias, float *__restrict__ out,
                                                   int n_stride) {
    const int b = blockIdx.z, i0 = blockIdx.y * APC_FT, j0 = blockIdx.x * APC_FT;
    const int n = lens[b] - 2, n_max = S_max - 2;
    if (i0 >= n || j0 >= n) return;
    __shared__ __attribute__((aligned(16))) float ri[APC_FL][APC_FT], rj[APC_FL][APC_FT];
    __shared__ float cs[APC_FL];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    float corr[4][4];
#pragma unroll
    for (int m = 0; m < 4; m++)
#pragma unroll
        for (int k = 0; k < 4; k++) corr[m][k] = 0.0f;
    for (int lh0 = 0; lh0 < LH; lh0 += APC_FL) {
        __syncthreads();
        for (int e = tid; e < APC_FL * APC_FT; e += 256) {
            const int lh = lh0 + e / APC_FT, x = e % APC_FT;
            const float *rr = r + ((size_t)lh * B + b) * n_max;
            const bool in = lh < LH;
            ri[e / APC_FT][x] = in && i0 + x < n ? rr[i0 + x] : 0.0f;
            rj[e / APC_FT][x] = in && j0 + x < n ? rr[j0 + x] : 0.0f;
        }
        if (tid < APC_FL) cs[tid] = lh0 + tid < LH ? coef[(size_t)(lh0 + tid) * B + b] : 0.0f;
        __syncthreads();
        const int nl = min(APC_FL, LH - lh0);
        for (int t = 0; t < nl; t++) {
            const float c = cs[t];
            if (c == 0.0f) continue;
            const float4 a = *reinterpret_cast<const float4 *>(&ri[t][4 * ty]);
            const float4 q = *reinterpret_cast<const float4 *>(&rj[t][4 * tx]);
            const float av[4] = {a.x, a.y, a.z, a.w}, qv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int k = 0; k < 4; k++) corr[m][k] = fmaf(c, av[m] * qv[k], corr[m][k]);  // r_i r_j first: symmetric
        }
    }
    const float *Mb = M + (size_t)b * n_max * n_max;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const int i = i0 + 4 * ty + m;
        if (i >= n) continue;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int j = j0 + 4 * tx + k;
            if (j >= n) continue;
            const float logit = Mb[(size_t)i * n_max + j] + Mb[(size_t)j * n_max + i] - corr[m][k];
            out[((size_t)b * n_stride + i) * n_stride + j] = 1.0f / (1.0f + expf(-(logit + bias)));
        }
    }
}

hipError_t launch_apc_finalize(const float *M, const float *r, float *coef, const float *w_dev, int LH, SeqMeta sm,
                               float bias, float *contacts, int n_stride, hipStream_t st) {
    if (sm.S_max < 3) return hipSuccess;
    const int n_max = sm.S_max - 2;
    hipLaunchKernelGGL(k_apc_coef, dim3(LH, sm.B), dim3(256), 0, st, r, w_dev, sm.lens, sm.S_max, sm.B, coef);
    const int nt = (n_max + APC_FT - 1) / APC_FT;
    hipLaunchKernelGGL(k_apc_final, dim3(nt, nt, sm.B), dim3(256), 0, st, M, r, coef, LH, sm.lens, sm.S_max, sm.B, bias,
                       contacts, n_stride);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_scatter_rows(const float *__restrict__ src, int width,
                                                      const int *__restrict__ cu, const int *__restrict__ lens,
                                                      int S_max, float *__restrict__ dst, long long bstride) {
    const int s = blockIdx.x, b = blockIdx.y;
    if (s >= lens[b]) return;
    const float *sr = src + (size_t)(cu[b] + s) * width;
    float *dr = dst + b * bstride + (size_t)s * width;
    for (int i = threadIdx.x; i < width; i += 256) dr[i] = sr[i];
}

hipError_t launch_scatter_rows(const float *src, int width, SeqMeta sm, float *dst, int64_t dst_b_stride,
                               hipStream_t st) {
    hipLaunchKernelGGL(k_scatter_rows, dim3(sm.S_max, sm.B), dim3(256), 0, st, src, width, sm.cu, sm.lens, sm.S_max,
                       dst, (long long)dst_b_stride);
    return hipGetLastError();
}

// One thread per scored position: log_softmax_canonical (lib.rs:4426-4441),
// Shannon entropy over ids 4..=23 with p = exp(lp) counted when p > 1e-12,
// deltas lp[aa] - lp[wt] in CANONICAL_AAS order (benchmark.rs:702-707),
// 0 for the wild-type column (pipeline.rs:152-172).
__global__ __launch_bounds__(64) void k_dms_score(const float *__restrict__ logits, int V, const int *__restrict__ meta,
                                                  int count, float *__restrict__ out) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (i >= count) return;
    const float *lg = logits + (size_t)meta[2 * i] * V;
    const int wt = meta[2 * i + 1];
    float m = -INFINITY;
    for (int t = 4; t <= 23; t++) m = fmaxf(m, lg[t]);
    float s = 0.0f;
    for (int t = 4; t <= 23; t++) s += expf(lg[t] - m);
    const float lse = m + logf(s);
    float h = 0.0f;
    for (int t = 4; t <= 23; t++) {
        const float lp = lg[t] - lse;
        const float p = expf(lp);
        if (p > 1e-12f) h -= p * lp;
    }
    constexpr int tok[20] = {5, 23, 13, 9, 18, 6, 21, 12, 15, 4, 20, 17, 14, 16, 10, 8, 11, 7, 22, 19};
    // lp of a non-canonical wild-type token is -inf in the reference's table
    const float lw = (wt >= 4 && wt <= 23) ? lg[wt] - lse : -INFINITY;
    float *o = out + (size_t)i * 21;
    for (int c = 0; c < 20; c++) o[c] = tok[c] == wt ? 0.0f : (lg[tok[c]] - lse) - lw;
    o[20] = h;
}

hipError_t launch_dms_score(const float *logits, int V, const int *meta, int count, float *out, hipStream_t st) {
    if (count <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_dms_score, dim3((count + 63) / 64), dim3(64), 0, st, logits, V, meta, count, out);
    return hipGetLastError();
}

}  // namespace cih
