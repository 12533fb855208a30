// Autoregressive decoding against a per-slot KV cache: rotary embedding of
// the new rows' Q and K with their K/V written into the cache, and causal
// attention of each new row over its slot's positions 0..pos.  Replaces the
// cache write and attention_head_avx1 of forward / forward_q8 / forward_q4
// (codon-infer src/lib.rs:3616-3663, 3438-3483).
#include <math.h>

#include "kernels.h"

namespace cih {

namespace {

constexpr int DEC_THREADS = 256;

// apply_rope (lib.rs:3533-3552) on row r's Q (in place) and K (into the
// cache at the row's position); V is copied to the cache.  Products and sums
// are rounded one by one as the reference computes them (no fused multiply-add).
__global__ __launch_bounds__(DEC_THREADS) void k_rope_kv(float *__restrict__ qkv, int d, int hd,
                                                         const int *__restrict__ rows, const float *__restrict__ rc,
                                                         const float *__restrict__ rs, float *__restrict__ kc,
                                                         float *__restrict__ vc, int64_t slot_stride) {
    const int r = blockIdx.x;
    const int slot = rows[2 * r], pos = rows[2 * r + 1];
    const int half = hd / 2;
    float *q = qkv + (size_t)r * 3 * d;
    const float *k = q + d, *v = q + 2 * d;
    float *kd = kc + slot * slot_stride + (size_t)pos * d;
    float *vd = vc + slot * slot_stride + (size_t)pos * d;
    const float *c = rc + (size_t)pos * half, *s = rs + (size_t)pos * half;
    for (int i = threadIdx.x; i < d / 2; i += DEC_THREADS) {
        const int h = i / half, j = i - h * half;
        const int i0 = h * hd + j, i1 = i0 + half;
        const float cj = c[j], sj = s[j];
        const float q0 = q[i0], q1 = q[i1], k0 = k[i0], k1 = k[i1];
        q[i0] = __fsub_rn(__fmul_rn(q0, cj), __fmul_rn(q1, sj));
        q[i1] = __fadd_rn(__fmul_rn(q1, cj), __fmul_rn(q0, sj));
        kd[i0] = __fsub_rn(__fmul_rn(k0, cj), __fmul_rn(k1, sj));
        kd[i1] = __fadd_rn(__fmul_rn(k1, cj), __fmul_rn(k0, sj));
    }
    for (int i = threadIdx.x; i < d; i += DEC_THREADS) vd[i] = v[i];
}

__device__ __forceinline__ float block_reduce(float v, float *scratch, bool is_max) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float u = __shfl_xor(v, o);
        v = is_max ? fmaxf(v, u) : v + u;
    }
    const int w = threadIdx.x >> 6;
    __syncthreads();  // scratch free from the previous reduction
    if ((threadIdx.x & 63) == 0) scratch[w] = v;
    __syncthreads();
    float r = scratch[0];
#pragma unroll
    for (int i = 1; i < DEC_THREADS / 64; i++) r = is_max ? fmaxf(r, scratch[i]) : r + scratch[i];
    return r;
}

// One workgroup per (row, head).  Scores s_t = (q . k_t) / sqrt(hd) for
// t = 0..pos (a thread per key), softmax as softmax() (lib.rs:3500-3504:
// max, exp(s - max), 1 / sum, p = e * (1/sum)), then out = sum_t p_t v_t with
// G = 256 / HD key groups of HD lanes (a group reads whole V rows) whose
// partial sums are added in group order.
template <int HD>
__global__ __launch_bounds__(DEC_THREADS) void k_decode_attention(const float *__restrict__ qkv, int d,
                                                                  const int *__restrict__ rows,
                                                                  const float *__restrict__ kc,
                                                                  const float *__restrict__ vc, int64_t slot_stride,
                                                                  float inv_scale, float *__restrict__ out) {
    constexpr int G = DEC_THREADS / HD;
    extern __shared__ float sm[];
    float *qs = sm;                 // [HD]
    float *part = qs + HD;          // [G][HD]
    float *red = part + G * HD;     // [4]
    float *p = red + 4;             // [pos + 1]
    const int r = blockIdx.x, h = blockIdx.y;
    const int slot = rows[2 * r], pos = rows[2 * r + 1];
    const float *q = qkv + (size_t)r * 3 * d + h * HD;
    const float *K = kc + slot * slot_stride + h * HD;
    const float *V = vc + slot * slot_stride + h * HD;
    if (threadIdx.x < HD) qs[threadIdx.x] = q[threadIdx.x];
    __syncthreads();
    float mx = -INFINITY;
    for (int t = threadIdx.x; t <= pos; t += DEC_THREADS) {
        const float4 *kr = reinterpret_cast<const float4 *>(K + (size_t)t * d);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < HD / 4; i++) {
            const float4 kv = kr[i];
            acc = fmaf(qs[4 * i], kv.x, acc);
            acc = fmaf(qs[4 * i + 1], kv.y, acc);
            acc = fmaf(qs[4 * i + 2], kv.z, acc);
            acc = fmaf(qs[4 * i + 3], kv.w, acc);
        }
        const float sc = acc * inv_scale;
        p[t] = sc;
        mx = fmaxf(mx, sc);
    }
    mx = block_reduce(mx, red, true);
    float sum = 0.0f;
    for (int t = threadIdx.x; t <= pos; t += DEC_THREADS) {
        const float e = expf(p[t] - mx);
        p[t] = e;
        sum += e;
    }
    sum = block_reduce(sum, red, false);
    const float inv = 1.0f / sum;
    __syncthreads();
    const int g = threadIdx.x / HD, i = threadIdx.x - g * HD;
    if (g < G) {
        float acc = 0.0f;
        for (int t = g; t <= pos; t += G) acc = fmaf(p[t] * inv, V[(size_t)t * d + i], acc);
        part[g * HD + i] = acc;
    }
    __syncthreads();
    if (threadIdx.x < HD) {
        float o = part[threadIdx.x];
#pragma unroll
        for (int j = 1; j < G; j++) o += part[j * HD + threadIdx.x];
        out[(size_t)r * d + h * HD + threadIdx.x] = o;
    }
}

}  // namespace

size_t decode_attention_lds(int hd, int max_len) {
    return sizeof(float) * ((size_t)hd + DEC_THREADS + 4 + (size_t)max_len);
}

hipError_t launch_rope_kv(float *qkv, int d, int hd, const int *rows, int n, const float *rope_c, const float *rope_s,
                          float *kc, float *vc, int64_t slot_stride, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope_kv, dim3(n), dim3(DEC_THREADS), 0, st, qkv, d, hd, rows, rope_c, rope_s, kc, vc,
                       slot_stride);
    return hipGetLastError();
}

hipError_t launch_decode_attention(const float *qkv, int d, int H, const int *rows, int n, int max_len,
                                   const float *kc, const float *vc, int64_t slot_stride, float *out,
                                   hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int hd = d / H;
    const float inv_scale = 1.0f / sqrtf((float)hd);
    const size_t lds = decode_attention_lds(hd, max_len);
    const dim3 grid(n, H), block(DEC_THREADS);
    switch (hd) {
    case 16: hipLaunchKernelGGL(k_decode_attention<16>, grid, block, lds, st, qkv, d, rows, kc, vc, slot_stride, inv_scale, out); break;
    case 24: hipLaunchKernelGGL(k_decode_attention<24>, grid, block, lds, st, qkv, d, rows, kc, vc, slot_stride, inv_scale, out); break;
    case 32: hipLaunchKernelGGL(k_decode_attention<32>, grid, block, lds, st, qkv, d, rows, kc, vc, slot_stride, inv_scale, out); break;
    case 64: hipLaunchKernelGGL(k_decode_attention<64>, grid, block, lds, st, qkv, d, rows, kc, vc, slot_stride, inv_scale, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace cih
