// Weight residency kernels: the reference's row-major tensors, already copied
// to device memory unchanged, become the k-block-major device matrices (see
// kernels.h), and FP32 matrices are quantized to Q8_0 / Q4_0 on the way.
// Sources are only 4-byte aligned (the fields of a weight file follow each
// other without padding), so every read is a dword.
#include <math.h>

#include "kernels.h"

namespace cih {

namespace {

constexpr int LOAD_THREADS = 256;

__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *(const uint32_t *)p; }

// One packed block per thread: scale to sc, quants to qs (QB = 32 Q8_0, 16 Q4_0).
template <int QB>
__global__ __launch_bounds__(LOAD_THREADS) void k_repack_blocks(const uint8_t *__restrict__ src, int N, int KB,
                                                                uint8_t *__restrict__ qs, float *__restrict__ sc,
                                                                int Ntot, int n_off) {
    const int64_t total = (int64_t)N * KB;
    for (int64_t i = blockIdx.x * (int64_t)LOAD_THREADS + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * LOAD_THREADS) {
        const int64_t n = i / KB;
        const int kb = (int)(i - n * KB);
        const uint8_t *b = src + i * (QB + 4);
        const size_t o = (size_t)kb * Ntot + n_off + n;
        sc[o] = __uint_as_float(ld32(b));
        uint32_t *d = (uint32_t *)(qs + o * QB);
#pragma unroll
        for (int j = 0; j < QB / 4; j++) d[j] = ld32(b + 4 + 4 * j);
    }
}

// FP32 [N][K] -> [K/32][Ntot][32], one element per thread.
__global__ __launch_bounds__(LOAD_THREADS) void k_repack_f32(const float *__restrict__ src, int N, int K,
                                                             float *__restrict__ dst, int Ntot, int n_off) {
    const int64_t total = (int64_t)N * K;
    for (int64_t i = blockIdx.x * (int64_t)LOAD_THREADS + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * LOAD_THREADS) {
        const int64_t n = i / K;
        const int k = (int)(i - n * K);
        dst[((size_t)(k >> 5) * Ntot + n_off + n) * 32 + (k & 31)] = src[i];
    }
}

// BlockQ8_0::quantize (lib.rs:648-660): d = absmax / 127, id = d == 0 ? 0 :
// 1 / d, q = clamp(round(x * id), -127, 127) with round half away from zero;
// NaN quantizes to 0.  Division and rounding are IEEE-exact on the GPU, so
// the blocks equal the host quantizer's bit for bit.
__device__ __forceinline__ void quant_q8(const float *v, float &d_out, uint32_t *q) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fabsf(v[j]) > amax ? fabsf(v[j]) : amax;
    const float d = amax / 127.0f;
    const float id = d == 0.0f ? 0.0f : 1.0f / d;
    d_out = d;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float r = roundf(v[4 * w + b] * id);
            const int qi = isnan(r) ? 0 : (int)(r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r));
            word |= (uint32_t)(qi & 0xFF) << (8 * b);
        }
        q[w] = word;
    }
}

// BlockQ4_0::quantize (lib.rs:1054-1071): mx = the first element of largest
// |x| (signed), d = mx / -8, q = clamp(round(x * id) + 8, 0, 15) (NaN -> 8,
// Rust's saturating float -> i32 cast), byte j = q_j | q_{j+16} << 4.
__device__ __forceinline__ int q4_code(float x, float id) {
    const float r = roundf(x * id);
    return isnan(r) ? 8 : (int)(r < -8.0f ? -8.0f : (r > 7.0f ? 7.0f : r)) + 8;
}

__device__ __forceinline__ void quant_q4(const float *v, float &d_out, uint32_t *q) {
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++)
        if (fabsf(v[j]) > fabsf(mx)) mx = v[j];
    const float d = mx == 0.0f ? 0.0f : mx / -8.0f;
    const float id = d == 0.0f ? 0.0f : 1.0f / d;
    d_out = d;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int j = 4 * w + b;
            word |= (uint32_t)(q4_code(v[j], id) | (q4_code(v[j + 16], id) << 4)) << (8 * b);
        }
        q[w] = word;
    }
}

// FP32 [N][K] -> quantized k-block-major rows, one 32-value block per thread.
template <int WF>
__global__ __launch_bounds__(LOAD_THREADS) void k_quantize_rows(const float *__restrict__ src, int N, int KB,
                                                                uint8_t *__restrict__ qs, float *__restrict__ sc,
                                                                int Ntot, int n_off) {
    constexpr int QB = WF == WF_Q8 ? 32 : 16;
    const int64_t total = (int64_t)N * KB;
    for (int64_t i = blockIdx.x * (int64_t)LOAD_THREADS + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * LOAD_THREADS) {
        const int64_t n = i / KB;
        const int kb = (int)(i - n * KB);
        const float *x = src + i * 32;  // row n, block kb: n * K + kb * 32
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; j++) v[j] = x[j];
        float d;
        uint32_t q[QB / 4];
        if constexpr (WF == WF_Q8) quant_q8(v, d, q);
        else quant_q4(v, d, q);
        const size_t o = (size_t)kb * Ntot + n_off + n;
        sc[o] = d;
        uint32_t *dq = (uint32_t *)(qs + o * QB);
#pragma unroll
        for (int j = 0; j < QB / 4; j++) dq[j] = q[j];
    }
}

__global__ __launch_bounds__(LOAD_THREADS) void k_copy_segments(const uint8_t *__restrict__ src,
                                                                uint8_t *__restrict__ dst,
                                                                const CopySeg *__restrict__ segs) {
    const CopySeg s = segs[blockIdx.x];
    const float *a = (const float *)(src + s.src);
    float *b = (float *)(dst + s.dst);
    for (int64_t i = threadIdx.x; i < s.n; i += LOAD_THREADS) b[i] = a[i];
}

unsigned grid_for(int64_t items) {
    const int64_t g = (items + LOAD_THREADS - 1) / LOAD_THREADS;
    return (unsigned)(g < 65536 ? (g > 0 ? g : 1) : 65536);
}

}  // namespace

hipError_t launch_load_matrix(const uint8_t *src, int src_fmt, int N, const DevMatrix &dst, int n_off, hipStream_t st) {
    const int K = dst.K, KB = K / 32;
    if (N <= 0 || K <= 0 || K % 32 || n_off < 0 || n_off + N > dst.N) return hipErrorInvalidValue;
    uint8_t *qs = (uint8_t *)dst.q;
    float *sc = (float *)dst.sc;
    const int64_t blocks = (int64_t)N * KB;
    if (src_fmt == dst.fmt) {
        if (src_fmt == WF_F32)
            hipLaunchKernelGGL(k_repack_f32, dim3(grid_for((int64_t)N * K)), dim3(LOAD_THREADS), 0, st,
                               (const float *)src, N, K, (float *)qs, dst.N, n_off);
        else if (src_fmt == WF_Q8)
            hipLaunchKernelGGL(k_repack_blocks<32>, dim3(grid_for(blocks)), dim3(LOAD_THREADS), 0, st, src, N, KB,
                               qs, sc, dst.N, n_off);
        else
            hipLaunchKernelGGL(k_repack_blocks<16>, dim3(grid_for(blocks)), dim3(LOAD_THREADS), 0, st, src, N, KB,
                               qs, sc, dst.N, n_off);
    } else if (src_fmt == WF_F32 && dst.fmt == WF_Q8) {
        hipLaunchKernelGGL(k_quantize_rows<WF_Q8>, dim3(grid_for(blocks)), dim3(LOAD_THREADS), 0, st,
                           (const float *)src, N, KB, qs, sc, dst.N, n_off);
    } else if (src_fmt == WF_F32 && dst.fmt == WF_Q4) {
        hipLaunchKernelGGL(k_quantize_rows<WF_Q4>, dim3(grid_for(blocks)), dim3(LOAD_THREADS), 0, st,
                           (const float *)src, N, KB, qs, sc, dst.N, n_off);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_copy_segments(const uint8_t *src, uint8_t *dst, const CopySeg *segs, int count, hipStream_t st) {
    if (count <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_copy_segments, dim3(count), dim3(LOAD_THREADS), 0, st, src, dst, segs);
    return hipGetLastError();
}

}  // namespace cih
