// Autoregressive decoding against a per-slot KV cache: rotary embedding of
// the new rows' Q and K with their K/V written into the cache, and causal
// attention of each new row over its slot's positions 0..pos.  Replaces the
// cache write and attention_head_avx1 of forward / forward_q8 / forward_q4
// (codon-infer src/lib.rs:3616-3663, 3438-3483).
#include <math.h>

#include "head_wo.h"
#include "kernels.h"
#include "x3.h"

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

constexpr int ATT_THREADS = 512;  // 8 waves per (row, head)

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
    for (int i = 1; i < ATT_THREADS / 64; i++) r = is_max ? fmaxf(r, scratch[i]) : r + scratch[i];
    return r;
}

// One workgroup per (row, head).  Scores s_t = (q . k_t) / sqrt(hd) for
// t = 0..pos (a thread per key), softmax as softmax() (lib.rs:3500-3504:
// max, exp(s - max), 1 / sum), then out = sum_t p_t v_t with G = 512 / HD
// key groups of HD lanes (a group reads whole V rows, four rows in flight)
// whose partial sums are added in group order.
//
// FUSED (each slot at most once in the launch): the workgroup also applies
// RoPE to its head's Q and K, writes K and V at pos into the cache for later
// steps, and takes key pos from LDS rather than from the cache, so no
// workgroup reads what another one writes.  Otherwise k_rope_kv has run.
//
// WOF (WF_Q8 / WF_Q4; 0: none): instead of storing the head's output, the
// workgroup multiplies it by the head's k-blocks of Wo (HeadWo) for columns
// [z 128 WP, (z + 1) 128 WP), z = blockIdx.z, into wo_part + (h n + r) N:
// the heads are the projection's splits.  Its weights are requested before
// the attention, which each column chunk repeats (only chunk 0 writes the
// cache).  WP = 1 for one row, 2 for two (650M Q4_0: one stream 929 -> 940
// tokens/s with 128 columns, two streams 1,728 with 256 against 1,532).
template <int HD, bool FUSED, int OF, int WOF = 0, int WP = 2>
__global__ __launch_bounds__(ATT_THREADS) void k_decode_attention(const float *__restrict__ qkv,
                                                                  const float *__restrict__ part, int splits,
                                                                  const float *__restrict__ bias, int d,
                                                                  const int *__restrict__ rows,
                                                                  const float *__restrict__ rc,
                                                                  const float *__restrict__ rs, float *__restrict__ kc,
                                                                  float *__restrict__ vc, int64_t slot_stride,
                                                                  float inv_scale, float *__restrict__ out,
                                                                  const unsigned char *__restrict__ wo_q = nullptr,
                                                                  const float *__restrict__ wo_sc = nullptr,
                                                                  int wo_n = 0) {
    constexpr int G = ATT_THREADS / HD;
    constexpr int HALF = HD / 2;
    extern __shared__ float sm[];
    float *qs = sm;                        // [HD] rotated query
    float *kcur = qs + HD, *vcur = kcur + HD;  // [HD] key and value at pos (FUSED)
    float *gsum = vcur + HD;               // [G][HD] per-group partial outputs
    float *red = gsum + ATT_THREADS;       // [8]
    float *p = red + 8;                    // [pos + 1]
    const int r = blockIdx.x, h = blockIdx.y;
    const int slot = rows[2 * r], pos = rows[2 * r + 1];
    float *K = kc + slot * slot_stride + h * HD;
    float *V = vc + slot * slot_stride + h * HD;
    const int t = threadIdx.x;
    const int n_cached = FUSED ? pos : pos + 1;  // keys read from the cache
    constexpr int NKB = HD / 32;
    HeadWo<WOF ? WOF : WF_Q8, WP> wo;
    const int wc0 = (int)blockIdx.z * 128 * WP, wc1 = min(wc0 + 128 * WP, wo_n);
    if constexpr (WOF != 0) wo.load(wo_q, wo_sc, wo_n, h * NKB, NKB, wc0, wc1);
    const bool cache_writer = WOF == 0 || blockIdx.z == 0;
    // This thread's first key row is requested before anything waits, so its
    // latency overlaps the gather, the rotation and the barriers.
    float4 kfirst[HD / 4];
    if (t < n_cached) {
        const float4 *kr = reinterpret_cast<const float4 *>(K + (size_t)t * d);
#pragma unroll
        for (int i = 0; i < HD / 4; i++) kfirst[i] = kr[i];
    }
    // likewise the first four V rows of this lane's group (P.V below)
    const int g = t / HD, i = t - g * HD;
    float vfirst[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (g < G) {
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (g + u * G < n_cached) vfirst[u] = V[(size_t)(g + u * G) * d + i];
    }
    if constexpr (FUSED) {
        float c = 0.0f, s = 0.0f;
        if (t < HALF) {
            c = rc[(size_t)pos * HALF + t];
            s = rs[(size_t)pos * HALF + t];
        }
        // this head's q, k, v: the row of qkv, or the GEMV's partial sums
        // (eight interleaved sums over the splits) + bias
        if (t < 3 * HD) {
            const int which = t / HD, col = which * d + h * HD + (t - which * HD);
            float v;
            if (part) {
                const size_t stride = (size_t)gridDim.x * 3 * d;
                const float *pp = part + (size_t)r * 3 * d + col;
                float a[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
                int y = 0;
                for (; y + 8 <= splits; y += 8) {
#pragma unroll
                    for (int u = 0; u < 8; u++) a[u] += pp[(y + u) * stride];
                }
                for (int u = 0; y < splits; y++, u++) a[u] += pp[y * stride];
                v = (((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]))) + bias[col];
            } else {
                v = qkv[(size_t)r * 3 * d + col];
            }
            qs[t] = v;  // qs | kcur | vcur are contiguous
        }
        __syncthreads();
        // apply_rope (lib.rs:3533-3552) for this head, products rounded one by one
        if (t < HALF) {
            const float q0 = qs[t], q1 = qs[t + HALF], k0 = kcur[t], k1 = kcur[t + HALF];
            qs[t] = __fsub_rn(__fmul_rn(q0, c), __fmul_rn(q1, s));
            qs[t + HALF] = __fadd_rn(__fmul_rn(q1, c), __fmul_rn(q0, s));
            const float r0 = __fsub_rn(__fmul_rn(k0, c), __fmul_rn(k1, s));
            const float r1 = __fadd_rn(__fmul_rn(k1, c), __fmul_rn(k0, s));
            kcur[t] = r0;
            kcur[t + HALF] = r1;
            if (cache_writer) {
                K[(size_t)pos * d + t] = r0;
                K[(size_t)pos * d + t + HALF] = r1;
            }
        } else if (t >= 64 && t < 64 + HD && cache_writer) {
            V[(size_t)pos * d + t - 64] = vcur[t - 64];
        }
    } else {
        const float *q = qkv + (size_t)r * 3 * d + h * HD;
        if (t < HD) qs[t] = q[t];
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int j = t; j <= pos; j += ATT_THREADS) {
        float acc = 0.0f;
        if (j < n_cached) {
            float4 kv4[HD / 4];
            if (j == t) {
#pragma unroll
                for (int i = 0; i < HD / 4; i++) kv4[i] = kfirst[i];
            } else {
                const float4 *kr = reinterpret_cast<const float4 *>(K + (size_t)j * d);
#pragma unroll
                for (int i = 0; i < HD / 4; i++) kv4[i] = kr[i];
            }
#pragma unroll
            for (int i = 0; i < HD / 4; i++) {
                acc = fmaf(qs[4 * i], kv4[i].x, acc);
                acc = fmaf(qs[4 * i + 1], kv4[i].y, acc);
                acc = fmaf(qs[4 * i + 2], kv4[i].z, acc);
                acc = fmaf(qs[4 * i + 3], kv4[i].w, acc);
            }
        } else {
#pragma unroll
            for (int i = 0; i < HD; i++) acc = fmaf(qs[i], kcur[i], acc);
        }
        const float sc = acc * inv_scale;
        p[j] = sc;
        mx = fmaxf(mx, sc);
    }
    mx = block_reduce(mx, red, true);
    float sum = 0.0f;
    for (int j = t; j <= pos; j += ATT_THREADS) {
        const float e = expf(p[j] - mx);
        p[j] = e;
        sum += e;
    }
    sum = block_reduce(sum, red, false);
    const float inv = 1.0f / sum;
    __syncthreads();
    if (g < G) {
        const float *vi = V + i;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        // rows g, g+G, g+2G, g+3G from the registers, then four at a time
        if (g < n_cached) a0 = p[g] * inv * vfirst[0];
        if (g + G < n_cached) a1 = p[g + G] * inv * vfirst[1];
        if (g + 2 * G < n_cached) a2 = p[g + 2 * G] * inv * vfirst[2];
        if (g + 3 * G < n_cached) a3 = p[g + 3 * G] * inv * vfirst[3];
        int j = g + 4 * G;
        for (; j + 3 * G < n_cached; j += 4 * G) {
            const float v0 = vi[(size_t)j * d], v1 = vi[(size_t)(j + G) * d];
            const float v2 = vi[(size_t)(j + 2 * G) * d], v3 = vi[(size_t)(j + 3 * G) * d];
            a0 = fmaf(p[j] * inv, v0, a0);
            a1 = fmaf(p[j + G] * inv, v1, a1);
            a2 = fmaf(p[j + 2 * G] * inv, v2, a2);
            a3 = fmaf(p[j + 3 * G] * inv, v3, a3);
        }
        for (; j < n_cached; j += G) a0 = fmaf(p[j] * inv, vi[(size_t)j * d], a0);
        if (FUSED && pos >= g && (pos - g) % G == 0) a0 = fmaf(p[pos] * inv, vcur[i], a0);
        gsum[g * HD + i] = (a0 + a1) + (a2 + a3);
    }
    __syncthreads();
    if (t < HD) {
        float o = gsum[t];
#pragma unroll
        for (int k = 1; k < G; k++) o += gsum[k * HD + t];
        if constexpr (WOF != 0) qs[t] = o;  // the query is no longer read
        else if constexpr (OF == AF_H2) h2_store(reinterpret_cast<unsigned short *>(out), r, h * HD + t, d, o);
        else out[(size_t)r * d + h * HD + t] = o;
    }
    if constexpr (WOF != 0) {
        static_assert(HD % 32 == 0, "heads of whole 32-wide blocks");
        __syncthreads();
        wo.run(qs, HD, 1, NKB, wo_n, wc0, wc1, out + ((size_t)h * gridDim.x + r) * wo_n);
    }
}

}  // namespace

size_t decode_attention_lds(int hd, int max_len) {
    return sizeof(float) * (3 * (size_t)hd + ATT_THREADS + 8 + (size_t)max_len);
}

hipError_t launch_rope_kv(float *qkv, int d, int hd, const int *rows, int n, const float *rope_c, const float *rope_s,
                          float *kc, float *vc, int64_t slot_stride, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope_kv, dim3(n), dim3(DEC_THREADS), 0, st, qkv, d, hd, rows, rope_c, rope_s, kc, vc,
                       slot_stride);
    return hipGetLastError();
}

template <bool FUSED>
static hipError_t launch_att(const float *qkv, const float *part, int splits, const float *bias, int d, int H,
                             const int *rows, int n, int max_len, const float *rc, const float *rs, float *kc,
                             float *vc, int64_t slot_stride, float *out, int out_fmt, hipStream_t st) {
    const int hd = d / H;
    const float inv_scale = 1.0f / sqrtf((float)hd);
    const size_t lds = decode_attention_lds(hd, max_len);
    const dim3 grid(n, H), block(ATT_THREADS);
    if (out_fmt != AF_F32 && (out_fmt != AF_H2 || d % 32)) return hipErrorInvalidValue;
#define CIH_ATT_CASE(HDV)                                                                                           \
    case HDV:                                                                                                      \
        if (out_fmt == AF_H2)                                                                                      \
            hipLaunchKernelGGL((k_decode_attention<HDV, FUSED, AF_H2>), grid, block, lds, st, qkv, part, splits,   \
                               bias, d, rows, rc, rs, kc, vc, slot_stride, inv_scale, out);                        \
        else                                                                                                       \
            hipLaunchKernelGGL((k_decode_attention<HDV, FUSED, AF_F32>), grid, block, lds, st, qkv, part, splits,  \
                               bias, d, rows, rc, rs, kc, vc, slot_stride, inv_scale, out);                        \
        break;
    switch (hd) {
        CIH_ATT_CASE(16)
        CIH_ATT_CASE(24)
        CIH_ATT_CASE(32)
        CIH_ATT_CASE(64)
    default: return hipErrorInvalidValue;
    }
#undef CIH_ATT_CASE
    return hipGetLastError();
}

hipError_t launch_decode_attention(const float *qkv, int d, int H, const int *rows, int n, int max_len,
                                   const float *kc, const float *vc, int64_t slot_stride, float *out,
                                   hipStream_t st, int out_fmt) {
    if (n <= 0) return hipSuccess;
    return launch_att<false>(qkv, nullptr, 0, nullptr, d, H, rows, n, max_len, nullptr, nullptr,
                             const_cast<float *>(kc), const_cast<float *>(vc), slot_stride, out, out_fmt, st);
}

hipError_t launch_decode_attention_fused_wo(float *qkv, const float *part, int splits, const float *bias, int d, int H,
                                            const int *rows, int n, int max_len, const float *rope_c,
                                            const float *rope_s, float *kc, float *vc, int64_t slot_stride,
                                            const DevMatrix &Wo, float *wo_part, size_t wo_part_floats,
                                            hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int hd = H > 0 ? d / H : 0;
    if ((part && (!bias || splits < 1)) || hd * H != d || (hd != 32 && hd != 64) ||
        (Wo.fmt != WF_Q8 && Wo.fmt != WF_Q4) || Wo.K != d || Wo.N % 16 || !wo_part ||
        (size_t)H * n * Wo.N > wo_part_floats)
        return hipErrorInvalidValue;
    const float inv_scale = 1.0f / sqrtf((float)hd);
    const size_t lds = decode_attention_lds(hd, max_len);
    const int wp = n == 1 ? 1 : 2;  // Wo columns per workgroup: 128 wp
    const dim3 grid(n, H, (Wo.N + 128 * wp - 1) / (128 * wp)), block(ATT_THREADS);
    const unsigned char *wq = static_cast<const unsigned char *>(Wo.q);
#define CIH_ATT_WO(HDV, WFV)                                                                                          \
    if (wp == 1)                                                                                                      \
        hipLaunchKernelGGL((k_decode_attention<HDV, true, AF_F32, WFV, 1>), grid, block, lds, st, qkv, part, splits,  \
                           bias, d, rows, rope_c, rope_s, kc, vc, slot_stride, inv_scale, wo_part, wq, Wo.sc, Wo.N);  \
    else                                                                                                              \
        hipLaunchKernelGGL((k_decode_attention<HDV, true, AF_F32, WFV, 2>), grid, block, lds, st, qkv, part, splits,  \
                           bias, d, rows, rope_c, rope_s, kc, vc, slot_stride, inv_scale, wo_part, wq, Wo.sc, Wo.N)
    if (hd == 64 && Wo.fmt == WF_Q8) {
        CIH_ATT_WO(64, WF_Q8);
    } else if (hd == 64) {
        CIH_ATT_WO(64, WF_Q4);
    } else if (Wo.fmt == WF_Q8) {
        CIH_ATT_WO(32, WF_Q8);
    } else {
        CIH_ATT_WO(32, WF_Q4);
    }
#undef CIH_ATT_WO
    return hipGetLastError();
}

hipError_t launch_decode_attention_fused(float *qkv, const float *part, int splits, const float *bias, int d, int H,
                                         const int *rows, int n, int max_len, const float *rope_c,
                                         const float *rope_s, float *kc, float *vc, int64_t slot_stride, float *out,
                                         hipStream_t st, int out_fmt) {
    if (n <= 0) return hipSuccess;
    if (part && (!bias || splits < 1)) return hipErrorInvalidValue;
    return launch_att<true>(qkv, part, splits, bias, d, H, rows, n, max_len, rope_c, rope_s, kc, vc, slot_stride, out,
                            out_fmt, st);
}

}  // namespace cih
