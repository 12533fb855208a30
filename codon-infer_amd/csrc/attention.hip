// Bidirectional rotary multi-head attention for gfx950 (FP32 MFMA).
//
// Replaces the per-head, per-query loops of forward_bidirectional*
// (codon-infer src/lib.rs:5206-5301; Q8 5558-5653; Q4 ~5905-6005) together
// with apply_rope (3533-3552), softmax (3500-3504) and the dot/axpy
// micro-kernels (3292-3434):
//   s_t = (q_p . k_t) * (1/sqrt(hd)) over every key t of the same sequence,
//   P = softmax(s), o_p = sum_t P_pt v_t.
// Sequences are packed back to back (row cu[b] + position); keys past a
// sequence's length are masked, so each sequence sees exactly the keys the
// reference's unpadded call sees.
//
// One workgroup = (query block, head, sequence), 32 queries per wave: 4
// waves x 32 (k_attention_h also 8 waves x 32 = 256 queries on large batches,
// which halves the staging of each key tile per query).  Scores are computed transposed, S^T = K Q^T, with
// v_mfma_f32_32x32x2_f32 so that each lane holds one query column and 16
// keys: the softmax reductions are lane-local plus one swap between the two
// lane halves, and the probabilities feed the P.V MFMA (O^T = V^T P^T) as the
// B operand straight from the accumulator registers: register s of lane
// (j, half) holds key 8*(s/4) + 4*half + s%4, which is the k index that lane
// supplies at step s.
// When probabilities are requested (attention maps, contacts, last-layer
// map): two passes over the keys — pass 1 keeps a running max/sum per lane,
// pass 2 recomputes the scores, forms p = exp(s - max) * (1/sum) as the
// reference does (k_attention_h: base 2, on scores pre-scaled by log2(e)),
// stores P and accumulates P.V.  Otherwise one pass with
// an online softmax (P.V accumulated unnormalised, divided by the sum once).
// RoPE is applied while staging K into LDS and Q into registers, from the
// host-built cos/sin tables (the reference's f32 powf/cos/sin values).
//
// Two kernels share this structure:
//   k_attention   : FP32 MFMA (v_mfma_f32_32x32x2_f32), CIH_ATT=fp32;
//   k_attention_h : f16 MFMA (v_mfma_f32_32x32x16_f16) on two-limb operands
//                   (x = hi + lo, hi = f16(x), lo = f16(x - hi)); each product
//                   is taken as hi*hi + hi*lo + lo*hi (the dropped lo*lo term
//                   and the split are ~2^-22 relative), accumulated in FP32.
//                   The 16-wide k-chunks of the MFMA need the probabilities'
//                   key order permuted: register 8c + e of a lane in half h
//                   holds key 16c + 8(e/4) + 4h + e%4, and V is read from LDS
//                   in that order.  The default.
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "kernels.h"
#include "kv_image.h"

namespace cih {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));


// Stores a lane's 16 probabilities (keys k0 + 8g + e, g = 0..3, e = 0..3) of
// one query row: 16-byte stores where a group is whole and aligned.
__device__ __forceinline__ void store_p(float *Prow, const float (&p)[16], int k0, int len) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int key = k0 + 8 * g;
        float *dst = Prow + key;
        if (key + 3 < len && ((uintptr_t)dst & 15) == 0) {
            *reinterpret_cast<float4 *>(dst) = make_float4(p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (key + e < len) dst[e] = p[4 * g + e];
        }
    }
}

// One 32-key tile of the one-pass f16-limb kernels (staged and image), the
// same arithmetic in both.  Per lane (query column, in both lane halves): m
// the base-2 exponent offset, l the running sum, oacc the P V accumulators.
// scores(acc, c0) leaves c0 + the tile's base-2 scores (the query is
// pre-scaled) in acc; it is called with c0 = -m, so acc holds the exponents
// themselves.  m moves, lazily, only when a score exceeds it by more than 8
// (and at the first tile): then the accumulators are rescaled and the tile's
// exponents shifted.  Register 8c + e of lane half hh holds key
// kt0 + 16c + 8(e/4) + 4hh + e%4; keys from kend on are masked (MASKED).
template <int DT, bool MASKED, class Scores, class PV>
__device__ __forceinline__ void online_tile(float &m, float &l, f32x16 (&oacc)[DT], int kt0, int kend, int hh,
                                            Scores &&scores, PV &&pv) {
    const bool first = m == -INFINITY;
    const float mc = first ? 0.0f : m;
    f32x16 acc;
    scores(acc, -mc);
    float sv[16];
    float tmax = -INFINITY;
#pragma unroll
    for (int q = 0; q < 16; q++) {
        float v = acc[q];
        if constexpr (MASKED) {
            const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
            v = key < kend ? v : -INFINITY;
        }
        sv[q] = v;
        tmax = fmaxf(tmax, v);
    }
    // key kt0 (< kend) sits in half 0, so the combined tile max is finite
    const float tm = fmaxf(tmax, __shfl_xor(tmax, 32));
    const bool need = first || tm > 8.0f;
    if (__ballot(need)) {
        const float mn = need ? tm + mc : m;
        const float corr = __builtin_amdgcn_exp2f(m - mn);
        l *= corr;
        m = mn;
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int q = 0; q < 16; q++) oacc[t][q] *= corr;
        const float sh = need ? mn - mc : 0.0f;
#pragma unroll
        for (int q = 0; q < 16; q++) sv[q] -= sh;
    }
    float p[16], sum = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; q++) {
        p[q] = __builtin_amdgcn_exp2f(sv[q]);
        sum += p[q];
    }
    l += sum;
    pv(p);
}

// Sum of the lane's probabilities whose keys are residues (1 <= key <= len - 2).
__device__ __forceinline__ float residue_sum(const float (&p)[16], int k0, int len) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; q++) {
        const int key = k0 + 8 * (q >> 2) + (q & 3);
        if (key >= 1 && key <= len - 2) s += p[q];
    }
    return s;
}

// residue_sum over the 32-key tile from kt0: when every key of the tile is a
// residue (1 <= kt0, kt0 + 31 <= len - 2) the masks are all true and the
// plain sum in the same order gives the same value.
__device__ __forceinline__ float tile_residue_sum(const float (&p)[16], int kt0, int hh, int len) {
    if (kt0 >= 1 && kt0 + 33 <= len) {
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 16; q++) s += p[q];
        return s;
    }
    return residue_sum(p, kt0 + 4 * hh, len);
}

// store_p for a whole tile (kt0 + 32 <= len) of a 16-byte aligned row: four
// unconditional 16-byte stores
__device__ __forceinline__ void store_p_whole(float *Prow, const float (&p)[16], int k0) {
#pragma unroll
    for (int g = 0; g < 4; g++)
        *reinterpret_cast<float4 *>(Prow + k0 + 8 * g) = make_float4(p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3]);
}

// rowsum[b][h][qi] for residue queries: the two lane halves hold disjoint keys.
__device__ __forceinline__ void write_rowsum(float *rowsum, float rs, int b, int h, int H, int S_max, int qi, int len,
                                             int hh) {
    if (!rowsum) return;
    rs += __shfl_xor(rs, 32);
    if (hh == 0 && qi >= 1 && qi <= len - 2) rowsum[((size_t)b * H + h) * S_max + qi] = rs;
}

template <int HD, bool ONEPASS>
__global__ __launch_bounds__(256) void k_attention(const float *__restrict__ qkv, int d, const int *__restrict__ cu,
                                                   const int *__restrict__ lens, int S_max,
                                                   const float *__restrict__ rc, const float *__restrict__ rsn,
                                                   void *__restrict__ out, int out_fmt, float *__restrict__ P,
                                                   long long pb, long long ph, float inv_scale,
                                                   float *__restrict__ rowsum) {
    constexpr int HALF = HD / 2;
    constexpr int VW = HD < 32 ? 32 : HD;  // V tile width, zero padded for small heads
    constexpr int DT = VW / 32;            // 32-wide output tiles
    constexpr int K_LD = HD + 4;
    constexpr int V_LD = VW + 4;
    __shared__ __attribute__((aligned(16))) float Ks[32 * K_LD];
    __shared__ __attribute__((aligned(16))) float Vs[32 * V_LD];

    const int b = blockIdx.z, h = blockIdx.y;
    const int len = lens[b], base = cu[b];
    const int qblk = blockIdx.x * 128;
    if (qblk >= len) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 31, hh = lane >> 5;
    const size_t ld = (size_t)3 * d;
    const float *Qg = qkv + h * HD;
    const float *Kg = qkv + d + h * HD;
    const float *Vg = qkv + 2 * d + h * HD;

    const int qi = qblk + wave * 32 + li;
    const int qc = min(qi, len - 1);
    float qr[HALF];
    {
        const float *qrow = Qg + (size_t)(base + qc) * ld;
        const float *cs = rc + (size_t)qc * HALF, *sn = rsn + (size_t)qc * HALF;
#pragma unroll
        for (int s = 0; s < HALF; s++) {
            const float q0 = qrow[s], q1 = qrow[s + HALF];
            qr[s] = hh == 0 ? q0 * cs[s] - q1 * sn[s] : q1 * cs[s] + q0 * sn[s];
        }
    }

    auto load_k = [&](int kt0) {
        for (int idx = tid; idx < 32 * HALF; idx += 256) {
            const int key = idx / HALF, c = idx % HALF;
            const int kk = min(kt0 + key, len - 1);
            const float *krow = Kg + (size_t)(base + kk) * ld;
            const float k0 = krow[c], k1 = krow[c + HALF];
            const float cs = rc[(size_t)kk * HALF + c], sn = rsn[(size_t)kk * HALF + c];
            Ks[key * K_LD + c] = k0 * cs - k1 * sn;
            Ks[key * K_LD + c + HALF] = k1 * cs + k0 * sn;
        }
    };
    auto load_v = [&](int kt0) {
        for (int idx = tid; idx < 32 * VW; idx += 256) {
            const int key = idx / VW, c = idx % VW;
            const int kk = min(kt0 + key, len - 1);
            Vs[key * V_LD + c] = c < HD ? Vg[(size_t)(base + kk) * ld + c] : 0.0f;
        }
    };
    auto scores = [&](f32x16 &acc) {
#pragma unroll
        for (int q = 0; q < 16; q++) acc[q] = 0.0f;
        const float *kr = &Ks[li * K_LD + hh * HALF];
#pragma unroll
        for (int s4 = 0; s4 < HALF / 4; s4++) {
            const float4 k4 = *reinterpret_cast<const float4 *>(kr + 4 * s4);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.x, qr[4 * s4 + 0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.y, qr[4 * s4 + 1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.z, qr[4 * s4 + 2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.w, qr[4 * s4 + 3], acc, 0, 0, 0);
        }
    };

    if constexpr (ONEPASS) {
        // ---- no probabilities requested: one pass with online softmax.
        // The tile max is combined across the two lane halves so that both
        // halves scale their P.V contributions by the same running max; the
        // output is divided by the sum of exponentials at the end.
        f32x16 oacc[DT];
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int q = 0; q < 16; q++) oacc[t][q] = 0.0f;
        float m = -INFINITY, l = 0.0f;
        for (int kt0 = 0; kt0 < len; kt0 += 32) {
            __syncthreads();
            load_k(kt0);
            load_v(kt0);
            __syncthreads();
            f32x16 acc;
            scores(acc);
            float sv[16];
            float tmax = -INFINITY;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
                sv[q] = key < len ? acc[q] * inv_scale : -INFINITY;
                tmax = fmaxf(tmax, sv[q]);
            }
            // key kt0 (< len) sits in half 0, so the combined tile max is finite
            const float mn = fmaxf(m, fmaxf(tmax, __shfl_xor(tmax, 32)));
            const float corr = expf(m - mn);
            float p[16], sum = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                p[q] = expf(sv[q] - mn);
                sum += p[q];
            }
            l = l * corr + sum;
            m = mn;
#pragma unroll
            for (int t = 0; t < DT; t++) {
#pragma unroll
                for (int q = 0; q < 16; q++) oacc[t][q] *= corr;
#pragma unroll
                for (int s2 = 0; s2 < 16; s2++) {
                    const float v = Vs[(8 * (s2 >> 2) + 4 * hh + (s2 & 3)) * V_LD + t * 32 + li];
                    oacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(v, p[s2], oacc[t], 0, 0, 0);
                }
            }
        }
        const float inv_sum = 1.0f / (l + __shfl_xor(l, 32));
        if (qi < len) {
#pragma unroll
            for (int t = 0; t < DT; t++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int dd = t * 32 + 8 * g + 4 * hh;
                    if (dd >= HD) continue;
                    const float4 v = make_float4(oacc[t][4 * g] * inv_sum, oacc[t][4 * g + 1] * inv_sum,
                                                 oacc[t][4 * g + 2] * inv_sum, oacc[t][4 * g + 3] * inv_sum);
                    if (out_fmt == AF_X3)
                        x3_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
                    else if (out_fmt == AF_H2)
                        h2_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
                    else
                        *reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + (size_t)(base + qi) * d +
                                                    h * HD + dd) = v;
                }
        }
        return;
    }

    // ---- pass 1: running max / sum of exp per lane (16 keys per tile)
    float m = -INFINITY, l = 0.0f;
    for (int kt0 = 0; kt0 < len; kt0 += 32) {
        __syncthreads();
        load_k(kt0);
        __syncthreads();
        f32x16 acc;
        scores(acc);
        float sv[16];
        float tmax = -INFINITY;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
            sv[q] = key < len ? acc[q] * inv_scale : -INFINITY;
            tmax = fmaxf(tmax, sv[q]);
        }
        const float mn = fmaxf(m, tmax);
        if (mn != -INFINITY) {
            float sum = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; q++) sum += expf(sv[q] - mn);
            l = l * expf(m - mn) + sum;
            m = mn;
        }
    }
    const float mo = __shfl_xor(m, 32), lo = __shfl_xor(l, 32);
    const float mx = fmaxf(m, mo);
    const float tot = l * expf(m - mx) + lo * expf(mo - mx);
    const float inv_sum = 1.0f / tot;

    // ---- pass 2: normalized probabilities, optional export, P.V
    f32x16 oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
        for (int q = 0; q < 16; q++) oacc[t][q] = 0.0f;
    float *Prow = (P && qi < len) ? P + b * pb + h * ph + (size_t)qi * S_max : nullptr;
    float rs = 0.0f;  // sum of this query's probabilities over residue keys (contacts)
    for (int kt0 = 0; kt0 < len; kt0 += 32) {
        __syncthreads();
        load_k(kt0);
        load_v(kt0);
        __syncthreads();
        f32x16 acc;
        scores(acc);
        float p[16];
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
            p[q] = key < len ? expf(acc[q] * inv_scale - mx) * inv_sum : 0.0f;
        }
        if (Prow) store_p(Prow, p, kt0 + 4 * hh, len);
        if (rowsum) rs += residue_sum(p, kt0 + 4 * hh, len);
#pragma unroll
        for (int t = 0; t < DT; t++) {
#pragma unroll
            for (int s = 0; s < 16; s++) {
                const float v = Vs[(8 * (s >> 2) + 4 * hh + (s & 3)) * V_LD + t * 32 + li];
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(v, p[s], oacc[t], 0, 0, 0);
            }
        }
    }
    write_rowsum(rowsum, rs, b, h, gridDim.y, S_max, qi, len, hh);
    if (qi < len) {
        // lane holds output dims dd = t*32 + 8*(q/4) + 4*half + q%4: groups of 4
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int dd = t * 32 + 8 * g + 4 * hh;
                if (dd >= HD) continue;
                const float4 v = make_float4(oacc[t][4 * g], oacc[t][4 * g + 1], oacc[t][4 * g + 2], oacc[t][4 * g + 3]);
                if (out_fmt == AF_X3)
                    x3_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
                else if (out_fmt == AF_H2)
                    h2_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
                else
                    *reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + (size_t)(base + qi) * d + h * HD + dd) = v;
            }
    }
}

// hi/lo f16 limbs of 8 floats
__device__ __forceinline__ void split8(const float *v, f16x8 &hi, f16x8 &lo) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
        hi[e] = (_Float16)v[e];
        lo[e] = (_Float16)(v[e] - (float)hi[e]);
    }
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void split8_mix(const float *v, f16x8 &hi, f16x8 &lo) {
    uint4 h, l;
    h.x = split_pair(v[0], v[1], l.x);
    h.y = split_pair(v[2], v[3], l.y);
    h.z = split_pair(v[4], v[5], l.z);
    h.w = split_pair(v[6], v[7], l.w);
    hi = __builtin_bit_cast(f16x8, h);
    lo = __builtin_bit_cast(f16x8, l);
}

// Work items: (sequence, head, query block) tasks, task = (b * H + h) * nq + qb,
// one workgroup each for the first nfull; every later task is split into
// nsplit ranges of whole 32-key tiles (one workgroup each, ONEPASS only)
// that leave their unnormalized output, running max and sum in part for
// k_attention_merge.
template <int HD, bool ONEPASS, int NTH = 256>
__global__ __launch_bounds__(NTH, ONEPASS || HD <= 32 ? 4 : 2) void k_attention_h(const float *__restrict__ qkv, int d, const int *__restrict__ cu,
                                                     const int *__restrict__ lens, int S_max,
                                                     const float *__restrict__ rc, const float *__restrict__ rsn,
                                                     void *__restrict__ out, int out_fmt, float *__restrict__ P,
                                                     long long pb, long long ph, float inv_scale,
                                                     float *__restrict__ rowsum, int H, int nq, int nfull, int nsplit,
                                                     float *__restrict__ part) {
    // no FMA contraction: the staged and the image kernel round alike
#pragma clang fp contract(off)
    constexpr int HALF = HD / 2;
    constexpr int HDP = (HD + 15) / 16 * 16;  // dims padded to whole 16-wide k-chunks
    constexpr int NC = HDP / 16;
    constexpr int VW = HD < 32 ? 32 : HD;     // output tile rows (dims), zero padded for small heads
    constexpr int DT = VW / 32;
    constexpr int K_LD = HDP + 8;             // f16 per LDS key row (16-byte aligned, padded)
    constexpr int V_LD = 32 + 8;              // f16 per LDS dim row of the transposed V tile
    constexpr int NBUF = ONEPASS ? 1 : 2;     // the export kernel double-buffers its tiles
    constexpr int KBUF = 32 * K_LD, VBUF = VW * V_LD;
    __shared__ __attribute__((aligned(16))) _Float16 Kh[NBUF * KBUF], Kl[NBUF * KBUF];
    __shared__ __attribute__((aligned(16))) _Float16 Vh[NBUF * VBUF], Vl[NBUF * VBUF];
    int cur = 0;  // LDS buffer the current tile is read from

    int task = blockIdx.x, ks = 0, ns = 1;
    if (task >= nfull) {
        const int t = task - nfull;
        task = nfull + t / nsplit;
        ks = t % nsplit;
        ns = nsplit;
    }
    const int qb = task % nq, h = (task / nq) % H, b = task / nq / H;
    const int len = lens[b], base = cu[b];
    const int qblk = qb * (NTH / 2);  // 32 queries per wave
    if (qblk >= len) return;
    // keys [kbeg, kend) of this workgroup: part ks of ns of the sequence's 32-key tiles
    const int ntile = (len + 31) / 32, per = (ntile + ns - 1) / ns;
    const int kbeg = min(ks * per, ntile) * 32, kend = min((ks + 1) * per * 32, len);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 31, hh = lane >> 5;
    const size_t ld = (size_t)3 * d;
    const float *Qg = qkv + h * HD;
    const float *Kg = qkv + d + h * HD;
    const float *Vg = qkv + 2 * d + h * HD;

    // padding dims (HD..HDP of K, HD..VW of V) stay zero for every tile
    if constexpr (HDP > HD)
        for (int idx = tid; idx < NBUF * 32 * (HDP - HD); idx += NTH) {
            const int key = idx / (HDP - HD), c = HD + idx % (HDP - HD);  // key spans the buffers
            Kh[key * K_LD + c] = (_Float16)0.0f;
            Kl[key * K_LD + c] = (_Float16)0.0f;
        }
    if constexpr (VW > HD)
        for (int idx = tid; idx < NBUF * (VW - HD) * 32; idx += NTH) {
            const int bf = idx / ((VW - HD) * 32), r = idx % ((VW - HD) * 32);
            const int c = HD + r / 32, key = r % 32;
            Vh[bf * VBUF + c * V_LD + key] = (_Float16)0.0f;
            Vl[bf * VBUF + c * V_LD + key] = (_Float16)0.0f;
        }

    // rotated query dims 16c + 8hh + e of this lane's query, as f16 limbs,
    // pre-scaled by log2(e) / sqrt(hd): the scores come out of the MFMAs in
    // base-2 units
    const float sl2 = inv_scale * 1.44269504088896340736f;
    const int qi = qblk + wave * 32 + li;
    const int qc = min(qi, len - 1);
    f16x8 qh[NC], ql[NC];
    {
        const float *qrow = Qg + (size_t)(base + qc) * ld;
        const float *cs = rc + (size_t)qc * HALF, *sn = rsn + (size_t)qc * HALF;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int dim = 16 * c + 8 * hh + e;
                float r = 0.0f;
                if (dim < HALF) r = rot_lo(qrow[dim], qrow[dim + HALF], cs[dim], sn[dim]);
                else if (dim < HD) r = rot_hi(qrow[dim], qrow[dim - HALF], cs[dim - HALF], sn[dim - HALF]);
                v[e] = opaque(r * sl2);
            }
            split8(v, qh[c], ql[c]);
        }
    }

    // K tile: a thread rotates 4 consecutive pair-dims (c..c+3 with c+HALF..) of one key
    auto load_k = [&](int kt0) {
        constexpr int G = HALF / 4;
        for (int idx = tid; idx < 32 * G; idx += NTH) {
            const int key = idx / G, c = 4 * (idx % G);
            const int kk = min(kt0 + key, len - 1);
            const float *krow = Kg + (size_t)(base + kk) * ld;
            const float4 k0 = *reinterpret_cast<const float4 *>(krow + c);
            const float4 k1 = *reinterpret_cast<const float4 *>(krow + c + HALF);
            const float4 cs = *reinterpret_cast<const float4 *>(rc + (size_t)kk * HALF + c);
            const float4 sn = *reinterpret_cast<const float4 *>(rsn + (size_t)kk * HALF + c);
            const float r0[4] = {rot_lo(k0.x, k1.x, cs.x, sn.x), rot_lo(k0.y, k1.y, cs.y, sn.y),
                                 rot_lo(k0.z, k1.z, cs.z, sn.z), rot_lo(k0.w, k1.w, cs.w, sn.w)};
            const float r1[4] = {rot_hi(k1.x, k0.x, cs.x, sn.x), rot_hi(k1.y, k0.y, cs.y, sn.y),
                                 rot_hi(k1.z, k0.z, cs.z, sn.z), rot_hi(k1.w, k0.w, cs.w, sn.w)};
            f16x4 h0, l0, h1, l1;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                h0[e] = (_Float16)r0[e];
                l0[e] = (_Float16)(r0[e] - (float)h0[e]);
                h1[e] = (_Float16)r1[e];
                l1[e] = (_Float16)(r1[e] - (float)h1[e]);
            }
            *reinterpret_cast<f16x4 *>(&Kh[key * K_LD + c]) = h0;
            *reinterpret_cast<f16x4 *>(&Kl[key * K_LD + c]) = l0;
            *reinterpret_cast<f16x4 *>(&Kh[key * K_LD + c + HALF]) = h1;
            *reinterpret_cast<f16x4 *>(&Kl[key * K_LD + c + HALF]) = l1;
        }
    };
    // V tile, transposed: a thread takes 4 consecutive keys of one dim (coalesced over dims)
    auto load_v = [&](int kt0) {
        for (int idx = tid; idx < 8 * HD; idx += NTH) {
            const int c = idx % HD, kg = 4 * (idx / HD);
            f16x4 hv, lv;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int kk = min(kt0 + kg + e, len - 1);
                const float v = Vg[(size_t)(base + kk) * ld + c];
                hv[e] = (_Float16)v;
                lv[e] = (_Float16)(v - (float)hv[e]);
            }
            // 4-key groups 0, 1, 2, 3 of each 16-key chunk stored as 0, 2, 1, 3, so
            // the keys one lane half feeds an MFMA are 8 consecutive f16
            const int pos = (kg & ~15) | ((kg & 4) << 1) | ((kg & 8) >> 1);
            *reinterpret_cast<f16x4 *>(&Vh[c * V_LD + pos]) = hv;
            *reinterpret_cast<f16x4 *>(&Vl[c * V_LD + pos]) = lv;
        }
    };
    // S^T tile (32 keys x 32 queries) + c0: A = K rows (keys), B = Q columns (queries)
    auto scores = [&](f32x16 &acc, float c0) {
#pragma unroll
        for (int q = 0; q < 16; q++) acc[q] = c0;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const f16x8 kh = *reinterpret_cast<const f16x8 *>(&Kh[cur * KBUF + li * K_LD + 16 * c + 8 * hh]);
            const f16x8 kl = *reinterpret_cast<const f16x8 *>(&Kl[cur * KBUF + li * K_LD + 16 * c + 8 * hh]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[c], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, ql[c], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[c], acc, 0, 0, 0);
        }
    };
    // O^T += V^T P^T over the tile's 32 keys: B = this lane's 16 probabilities
    // (register 8c + e = key 16c + 8(e/4) + 4hh + e%4), A = V^T read in that key order
    auto pv = [&](f32x16 (&oacc)[DT], const float (&p)[16]) {
        f16x8 phi[2], plo[2];
        split8_mix(p, phi[0], plo[0]);
        split8_mix(p + 8, phi[1], plo[1]);
#pragma unroll
        for (int t = 0; t < DT; t++) {
            const int row = cur * VBUF + (t * 32 + li) * V_LD;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const f16x8 vh = *reinterpret_cast<const f16x8 *>(&Vh[row + 16 * c + 8 * hh]);
                const f16x8 vl = *reinterpret_cast<const f16x8 *>(&Vl[row + 16 * c + 8 * hh]);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, phi[c], oacc[t], 0, 0, 0);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, plo[c], oacc[t], 0, 0, 0);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl, phi[c], oacc[t], 0, 0, 0);
            }
        }
    };

    f32x16 oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
        for (int q = 0; q < 16; q++) oacc[t][q] = 0.0f;
    float out_scale;
    if constexpr (ONEPASS) {
        // One pass, online softmax (see k_attention) in base 2: the query is
        // pre-scaled by log2(e) / sqrt(hd) so every exponential is one
        // v_exp_f32, and the MFMAs start from -m, so their results are the
        // exponents themselves.  Whole tiles skip the key mask.  The exponent
        // offset m follows the running max lazily (it moves only when a score
        // exceeds it by more than 8, so p <= 256), which leaves the
        // accumulators unscaled on most tiles; o / l is unchanged.
        float m = -INFINITY, l = 0.0f;
        auto tile = [&](int kt0, auto masked) {
            __syncthreads();
            load_k(kt0);
            load_v(kt0);
            __syncthreads();
            online_tile<DT, decltype(masked)::value>(m, l, oacc, kt0, kend, hh,
                                                     [&](f32x16 &acc, float c0) { scores(acc, c0); },
                                                     [&](const float (&p)[16]) { pv(oacc, p); });
        };
        int kt0 = kbeg;
        for (; kt0 + 32 <= kend; kt0 += 32) tile(kt0, std::false_type{});
        if (kt0 < kend) tile(kt0, std::true_type{});
        const float lt = l + __shfl_xor(l, 32);
        if (ns > 1) {
            // split task: unnormalized output, running max (base 2) and sum
            if (qi < len) {
                float *pr = part + ((size_t)(blockIdx.x - nfull) * (NTH / 2) + wave * 32 + li) * (HD + 2);
#pragma unroll
                for (int t = 0; t < DT; t++)
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const int dd = t * 32 + 8 * g + 4 * hh;
                        if (dd >= HD) continue;
                        *reinterpret_cast<float2 *>(pr + dd) = make_float2(oacc[t][4 * g], oacc[t][4 * g + 1]);
                        *reinterpret_cast<float2 *>(pr + dd + 2) = make_float2(oacc[t][4 * g + 2], oacc[t][4 * g + 3]);
                    }
                if (hh == 0) *reinterpret_cast<float2 *>(pr + HD) = make_float2(m, lt);
            }
            return;
        }
        out_scale = 1.0f / lt;
    } else {
        // Two passes over the keys (the exported probabilities are final, so
        // the row max and sum come first), base-2 exponentials of the
        // pre-scaled scores.  With one 32-query wave per SIMD slot and few
        // waves, a tile's global loads are the critical path: they go to
        // registers one tile ahead (fetch) and into LDS as f16 limbs after the
        // barrier (stage), so tile t+1 is in flight while tile t is computed.
        constexpr int KG = HALF / 4, KI = (32 * KG + NTH - 1) / NTH, VI = (8 * HD + NTH - 1) / NTH;
        f32x4 kr[KI][4], vr[VI];
        auto fetch = [&](int kt0, bool with_v) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < KI; i++) {
                const int idx = tid + i * NTH;
                if (idx < 32 * KG) {
                    const int key = idx / KG, c = 4 * (idx % KG);
                    const int kk = min(kt0 + key, len - 1);
                    const float *krow = Kg + (size_t)(base + kk) * ld;
                    kr[i][0] = *reinterpret_cast<const f32x4 *>(krow + c);
                    kr[i][1] = *reinterpret_cast<const f32x4 *>(krow + c + HALF);
                    kr[i][2] = *reinterpret_cast<const f32x4 *>(rc + (size_t)kk * HALF + c);
                    kr[i][3] = *reinterpret_cast<const f32x4 *>(rsn + (size_t)kk * HALF + c);
                }
            }
            if (!with_v) return;
#pragma unroll
            for (int i = 0; i < VI; i++) {
                const int idx = tid + i * NTH;
                if (idx < 8 * HD) {
                    const int c = idx % HD, kg = 4 * (idx / HD);
#pragma unroll
                    for (int e = 0; e < 4; e++) vr[i][e] = Vg[(size_t)(base + min(kt0 + kg + e, len - 1)) * ld + c];
                }
            }
        };
        auto stage = [&](bool with_v, int bf) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < KI; i++) {
                const int idx = tid + i * NTH;
                if (idx < 32 * KG) {
                    const int key = idx / KG, c = 4 * (idx % KG);
                    const f32x4 k0 = kr[i][0], k1 = kr[i][1], cs = kr[i][2], sn = kr[i][3];
                    f16x4 h0, l0, h1, l1;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float r0 = rot_lo(k0[e], k1[e], cs[e], sn[e]);
                        const float r1 = rot_hi(k1[e], k0[e], cs[e], sn[e]);
                        h0[e] = (_Float16)r0;
                        l0[e] = (_Float16)(r0 - (float)h0[e]);
                        h1[e] = (_Float16)r1;
                        l1[e] = (_Float16)(r1 - (float)h1[e]);
                    }
                    *reinterpret_cast<f16x4 *>(&Kh[bf * KBUF + key * K_LD + c]) = h0;
                    *reinterpret_cast<f16x4 *>(&Kl[bf * KBUF + key * K_LD + c]) = l0;
                    *reinterpret_cast<f16x4 *>(&Kh[bf * KBUF + key * K_LD + c + HALF]) = h1;
                    *reinterpret_cast<f16x4 *>(&Kl[bf * KBUF + key * K_LD + c + HALF]) = l1;
                }
            }
            if (!with_v) return;
#pragma unroll
            for (int i = 0; i < VI; i++) {
                const int idx = tid + i * NTH;
                if (idx < 8 * HD) {
                    const int c = idx % HD, kg = 4 * (idx / HD);
                    f16x4 hv, lv;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        hv[e] = (_Float16)vr[i][e];
                        lv[e] = (_Float16)(vr[i][e] - (float)hv[e]);
                    }
                    const int pos = (kg & ~15) | ((kg & 4) << 1) | ((kg & 8) >> 1);  // as in load_v
                    *reinterpret_cast<f16x4 *>(&Vh[bf * VBUF + c * V_LD + pos]) = hv;
                    *reinterpret_cast<f16x4 *>(&Vl[bf * VBUF + c * V_LD + pos]) = lv;
                }
            }
        };
        // One barrier per tile: tile t + 1 is staged into the other buffer
        // right after the barrier that ends every wave's reads of tile t - 1
        // there, then tile t + 2 is fetched and tile t computed.
        auto sweep = [&](bool with_v, auto body) __attribute__((always_inline)) {
            fetch(0, with_v);
            __syncthreads();  // the previous sweep's reads of buffer 0 are done
            stage(with_v, 0);
            if (32 < len) fetch(32, with_v);
            for (int kt0 = 0, t = 0; kt0 < len; kt0 += 32, t++) {
                __syncthreads();
                cur = t & 1;
                if (kt0 + 32 < len) {
                    stage(with_v, cur ^ 1);
                    if (kt0 + 64 < len) fetch(kt0 + 64, with_v);
                }
                body(kt0);
            }
        };
        // pass 1: running max / sum of exp per lane
        float m = -INFINITY, l = 0.0f;
        sweep(false, [&](int kt0) __attribute__((always_inline)) {
            f32x16 acc;
            scores(acc, 0.0f);
            float sv[16];
            float tmax = -INFINITY;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
                sv[q] = key < len ? acc[q] : -INFINITY;
                tmax = fmaxf(tmax, sv[q]);
            }
            const float mn = fmaxf(m, tmax);
            if (mn != -INFINITY) {
                float sum = 0.0f;
#pragma unroll
                for (int q = 0; q < 16; q++) sum += __builtin_amdgcn_exp2f(sv[q] - mn);
                l = l * __builtin_amdgcn_exp2f(m - mn) + sum;
                m = mn;
            }
        });
        const float mo = __shfl_xor(m, 32), lo = __shfl_xor(l, 32);
        const float mx = fmaxf(m, mo);
        const float inv_sum = 1.0f / (l * __builtin_amdgcn_exp2f(m - mx) + lo * __builtin_amdgcn_exp2f(mo - mx));
        // pass 2: normalized probabilities, optional export, P.V
        float *Prow = (P && qi < len) ? P + b * pb + h * ph + (size_t)qi * S_max : nullptr;
        float rs = 0.0f;  // sum of this query's probabilities over residue keys (contacts)
        sweep(true, [&](int kt0) __attribute__((always_inline)) {
            f32x16 acc;
            scores(acc, 0.0f);
            float p[16];
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
                p[q] = key < len ? __builtin_amdgcn_exp2f(acc[q] - mx) * inv_sum : 0.0f;
            }
            if (Prow) store_p(Prow, p, kt0 + 4 * hh, len);
            if (rowsum) rs += tile_residue_sum(p, kt0, hh, len);
            pv(oacc, p);
        });
        write_rowsum(rowsum, rs, b, h, H, S_max, qi, len, hh);
        out_scale = 1.0f;
    }
    if (qi < len) {
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int dd = t * 32 + 8 * g + 4 * hh;
                if (dd >= HD) continue;
                const float4 v = make_float4(oacc[t][4 * g] * out_scale, oacc[t][4 * g + 1] * out_scale,
                                             oacc[t][4 * g + 2] * out_scale, oacc[t][4 * g + 3] * out_scale);
                if (out_fmt == AF_X3)
                    x3_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
                else if (out_fmt == AF_H2)
                    h2_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
                else
                    *reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + (size_t)(base + qi) * d + h * HD +
                                                dd) = v;
            }
    }
}

// Attention for batches whose 32-query tasks do not cover the compute units
// (one sequence of a few hundred residues): one workgroup per (sequence,
// head, 32 queries) task, KS waves on the same 32 queries, wave w over the
// 32-key tiles w, w + KS, ...  Each wave stages its tiles (RoPE, limbs, V
// transposed, as k_attention_h stages them) in its own LDS, so the waves
// meet only to combine:
//  * with the export (ONEPASS false): pass 1's running maxima and sums (per
//    wave and lane) give each query's maximum M and sum L = sum 2^(m_s - M)
//    l_s in wave order; pass 2 stores the probabilities exp2(s - M) / L and
//    the waves' P.V accumulators are added in wave order;
//  * without (ONEPASS): each wave runs the one-pass online softmax over its
//    tiles (online_tile, as k_attention_h), and the waves' results combine
//    as key ranges do in k_attention_merge: O = sum 2^(m_s - M) o_s /
//    sum 2^(m_s - M) l_s, in wave order.
// Per query the arithmetic is k_attention_h's, with the softmax and P.V sums
// regrouped by wave: agreement to rounding, not bit for bit.
template <int HD, int KS, bool ONEPASS>
__global__ __launch_bounds__(64 * KS) void k_attention_xs(const float *__restrict__ qkv, int d,
                                                          const int *__restrict__ cu, const int *__restrict__ lens,
                                                          int S_max, const float *__restrict__ rc,
                                                          const float *__restrict__ rsn, void *__restrict__ out,
                                                          int out_fmt, float *__restrict__ P, long long pb,
                                                          long long ph, float inv_scale, float *__restrict__ rowsum,
                                                          int H, int nq) {
#pragma clang fp contract(off)
    constexpr int HALF = HD / 2;
    constexpr int HDP = (HD + 15) / 16 * 16;
    constexpr int NC = HDP / 16;
    constexpr int VW = HD < 32 ? 32 : HD;
    constexpr int DT = VW / 32;
    constexpr int K_LD = HDP + 8, V_LD = 32 + 8;
    constexpr int KBUF = 32 * K_LD, VBUF = VW * V_LD;
    // [Kh | Kl | Vh | Vl] of every wave; after pass 2 the same bytes hold the
    // waves' P.V accumulators
    constexpr int STAGE_BYTES = KS * (2 * KBUF + 2 * VBUF) * 2, OX_BYTES = KS * DT * 16 * 64 * 4;
    __shared__ __attribute__((aligned(16))) unsigned char sm[STAGE_BYTES > OX_BYTES ? STAGE_BYTES : OX_BYTES];
    __shared__ float red[KS][3][64];  // per wave and lane: running max, sum, residue sum
    static_assert((STAGE_BYTES > OX_BYTES ? STAGE_BYTES : OX_BYTES) + KS * 3 * 64 * 4 <= 160 * 1024, "LDS");

    const int task = blockIdx.x, qb = task % nq, h = (task / nq) % H, b = task / nq / H;
    const int len = lens[b], base = cu[b];
    const int qblk = qb * 32;
    if (qblk >= len) return;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 31, hh = lane >> 5;
    const size_t ld = (size_t)3 * d;
    const float *Qg = qkv + h * HD;
    const float *Kg = qkv + d + h * HD;
    const float *Vg = qkv + 2 * d + h * HD;
    _Float16 *const Kh = reinterpret_cast<_Float16 *>(sm) + w * KBUF;
    _Float16 *const Kl = reinterpret_cast<_Float16 *>(sm) + KS * KBUF + w * KBUF;
    _Float16 *const Vh = reinterpret_cast<_Float16 *>(sm) + 2 * KS * KBUF + w * VBUF;
    _Float16 *const Vl = reinterpret_cast<_Float16 *>(sm) + 2 * KS * KBUF + KS * VBUF + w * VBUF;
    // A wave's LDS operations complete in order; this keeps the compiler from
    // moving this wave's LDS accesses across the point.
    auto wave_sync = [&]() __attribute__((always_inline)) { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); };

    // padding dims (HD..HDP of K, HD..VW of V) stay zero for every tile
    if constexpr (HDP > HD)
        for (int idx = lane; idx < 32 * (HDP - HD); idx += 64) {
            const int key = idx / (HDP - HD), c = HD + idx % (HDP - HD);
            Kh[key * K_LD + c] = (_Float16)0.0f;
            Kl[key * K_LD + c] = (_Float16)0.0f;
        }
    if constexpr (VW > HD)
        for (int idx = lane; idx < (VW - HD) * 32; idx += 64) {
            const int c = HD + idx / 32, key = idx % 32;
            Vh[c * V_LD + key] = (_Float16)0.0f;
            Vl[c * V_LD + key] = (_Float16)0.0f;
        }

    // rotated query dims 16c + 8hh + e of this lane's query, as f16 limbs
    const float sl2 = inv_scale * 1.44269504088896340736f;
    const int qi = qblk + li;
    const int qc = min(qi, len - 1);
    f16x8 qh[NC], ql[NC];
    {
        const float *qrow = Qg + (size_t)(base + qc) * ld;
        const float *cs = rc + (size_t)qc * HALF, *sn = rsn + (size_t)qc * HALF;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int dim = 16 * c + 8 * hh + e;
                float r = 0.0f;
                if (dim < HALF) r = rot_lo(qrow[dim], qrow[dim + HALF], cs[dim], sn[dim]);
                else if (dim < HD) r = rot_hi(qrow[dim], qrow[dim - HALF], cs[dim - HALF], sn[dim - HALF]);
                v[e] = opaque(r * sl2);  // pre-scaled, as in k_attention_h
            }
            split8(v, qh[c], ql[c]);
        }
    }

    // K tile: a lane rotates 4 consecutive pair-dims (c..c+3 with c+HALF..) of one key
    auto load_k = [&](int kt0) __attribute__((always_inline)) {
        constexpr int G = HALF / 4;
#pragma unroll
        for (int i = 0; i < (32 * G + 63) / 64; i++) {
            const int idx = lane + 64 * i;
            if (32 * G % 64 != 0 && idx >= 32 * G) break;
            const int key = idx / G, c = 4 * (idx % G);
            const int kk = min(kt0 + key, len - 1);
            const float *krow = Kg + (size_t)(base + kk) * ld;
            const float4 k0 = *reinterpret_cast<const float4 *>(krow + c);
            const float4 k1 = *reinterpret_cast<const float4 *>(krow + c + HALF);
            const float4 cs = *reinterpret_cast<const float4 *>(rc + (size_t)kk * HALF + c);
            const float4 sn = *reinterpret_cast<const float4 *>(rsn + (size_t)kk * HALF + c);
            const float r0[4] = {rot_lo(k0.x, k1.x, cs.x, sn.x), rot_lo(k0.y, k1.y, cs.y, sn.y),
                                 rot_lo(k0.z, k1.z, cs.z, sn.z), rot_lo(k0.w, k1.w, cs.w, sn.w)};
            const float r1[4] = {rot_hi(k1.x, k0.x, cs.x, sn.x), rot_hi(k1.y, k0.y, cs.y, sn.y),
                                 rot_hi(k1.z, k0.z, cs.z, sn.z), rot_hi(k1.w, k0.w, cs.w, sn.w)};
            f16x4 h0, l0, h1, l1;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                h0[e] = (_Float16)r0[e];
                l0[e] = (_Float16)(r0[e] - (float)h0[e]);
                h1[e] = (_Float16)r1[e];
                l1[e] = (_Float16)(r1[e] - (float)h1[e]);
            }
            *reinterpret_cast<f16x4 *>(&Kh[key * K_LD + c]) = h0;
            *reinterpret_cast<f16x4 *>(&Kl[key * K_LD + c]) = l0;
            *reinterpret_cast<f16x4 *>(&Kh[key * K_LD + c + HALF]) = h1;
            *reinterpret_cast<f16x4 *>(&Kl[key * K_LD + c + HALF]) = l1;
        }
    };
    // V tile, transposed: a lane takes 4 consecutive keys of one dim
    auto load_v = [&](int kt0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < (8 * HD + 63) / 64; i++) {
            const int idx = lane + 64 * i;
            if (8 * HD % 64 != 0 && idx >= 8 * HD) break;
            const int c = idx % HD, kg = 4 * (idx / HD);
            f16x4 hv, lv;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int kk = min(kt0 + kg + e, len - 1);
                const float v = Vg[(size_t)(base + kk) * ld + c];
                hv[e] = (_Float16)v;
                lv[e] = (_Float16)(v - (float)hv[e]);
            }
            const int pos = (kg & ~15) | ((kg & 4) << 1) | ((kg & 8) >> 1);  // as in k_attention_h
            *reinterpret_cast<f16x4 *>(&Vh[c * V_LD + pos]) = hv;
            *reinterpret_cast<f16x4 *>(&Vl[c * V_LD + pos]) = lv;
        }
    };
    auto scores = [&](f32x16 &acc, float c0) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 16; q++) acc[q] = c0;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const f16x8 kh = *reinterpret_cast<const f16x8 *>(&Kh[li * K_LD + 16 * c + 8 * hh]);
            const f16x8 kl = *reinterpret_cast<const f16x8 *>(&Kl[li * K_LD + 16 * c + 8 * hh]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[c], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, ql[c], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[c], acc, 0, 0, 0);
        }
    };
    auto pv = [&](f32x16 (&oacc)[DT], const float (&p)[16]) __attribute__((always_inline)) {
        f16x8 phi[2], plo[2];
        split8_mix(p, phi[0], plo[0]);
        split8_mix(p + 8, phi[1], plo[1]);
#pragma unroll
        for (int t = 0; t < DT; t++) {
            const int row = (t * 32 + li) * V_LD;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const f16x8 vh = *reinterpret_cast<const f16x8 *>(&Vh[row + 16 * c + 8 * hh]);
                const f16x8 vl = *reinterpret_cast<const f16x8 *>(&Vl[row + 16 * c + 8 * hh]);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, phi[c], oacc[t], 0, 0, 0);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, plo[c], oacc[t], 0, 0, 0);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl, phi[c], oacc[t], 0, 0, 0);
            }
        }
    };

    const int ntile = (len + 31) / 32;
    float *ox = reinterpret_cast<float *>(sm);
    // The waves' P.V accumulators (scaled by f) added in wave order and stored
    // for this lane's query, times out_scale; every wave must have written ox.
    auto finish = [&](float out_scale) __attribute__((always_inline)) {
        if (qi >= len) return;
        // output dims t 32 + 8 g + 4 hh + {0..3}: registers 4 g + {0..3} of tile t
#pragma unroll 1
        for (int tg = 0; tg < 4 * DT; tg++) {
            const int t = tg >> 2, g = tg & 3;
            const int dd = t * 32 + 8 * g + 4 * hh;
            if (dd >= HD) continue;
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int q = 4 * g + e;
                o[e] = ox[(t * 16 + q) * 64 + lane];
#pragma unroll
                for (int s = 1; s < KS; s++) o[e] += ox[((s * DT + t) * 16 + q) * 64 + lane];
            }
            const float4 v = make_float4(o[0] * out_scale, o[1] * out_scale, o[2] * out_scale, o[3] * out_scale);
            if (out_fmt == AF_X3)
                x3_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
            else if (out_fmt == AF_H2)
                h2_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
            else
                *reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + (size_t)(base + qi) * d + h * HD + dd) =
                    v;
        }
    };
    if constexpr (ONEPASS) {
        f32x16 oacc[DT];
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int q = 0; q < 16; q++) oacc[t][q] = 0.0f;
        float m = -INFINITY, l = 0.0f;
        auto tile = [&](int kt0, auto masked) __attribute__((always_inline)) {
            online_tile<DT, decltype(masked)::value>(m, l, oacc, kt0, len, hh,
                                                     [&](f32x16 &acc, float c0) { scores(acc, c0); },
                                                     [&](const float (&p)[16]) { pv(oacc, p); });
        };
        for (int t = w; t < ntile; t += KS) {
            const int kt0 = t * 32;
            wave_sync();
            load_k(kt0);
            load_v(kt0);
            wave_sync();
            if (kt0 + 32 <= len) tile(kt0, std::false_type{});
            else tile(kt0, std::true_type{});
        }
        const float lt = l + __shfl_xor(l, 32);  // both lane halves share m
        red[w][0][lane] = m;
        red[w][1][lane] = lt;
        __syncthreads();  // every wave is done with its stages
        float M = -INFINITY;
#pragma unroll
        for (int s = 0; s < KS; s++) M = fmaxf(M, red[s][0][lane]);
        float L = 0.0f;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const float ms = red[s][0][lane];
            if (ms != -INFINITY) L += __builtin_amdgcn_exp2f(ms - M) * red[s][1][lane];
        }
        const float f = m != -INFINITY ? __builtin_amdgcn_exp2f(m - M) : 0.0f;
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int q = 0; q < 16; q++) ox[((w * DT + t) * 16 + q) * 64 + lane] = f * oacc[t][q];
        __syncthreads();
        if (w == 0) finish(1.0f / L);
        return;
    } else {
        // pass 1: running max / sum of exp per lane over this wave's tiles
        float m = -INFINITY, l = 0.0f;
        for (int t = w; t < ntile; t += KS) {
            const int kt0 = t * 32;
            wave_sync();
            load_k(kt0);
            wave_sync();
            f32x16 acc;
            scores(acc, 0.0f);
            float sv[16];
            float tmax = -INFINITY;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
                sv[q] = key < len ? acc[q] : -INFINITY;
                tmax = fmaxf(tmax, sv[q]);
            }
            const float mn = fmaxf(m, tmax);
            if (mn != -INFINITY) {
                float sum = 0.0f;
#pragma unroll
                for (int q = 0; q < 16; q++) sum += __builtin_amdgcn_exp2f(sv[q] - mn);
                l = l * __builtin_amdgcn_exp2f(m - mn) + sum;
                m = mn;
            }
        }
        red[w][0][lane] = m;
        red[w][1][lane] = l;
        __syncthreads();
        // this query's max and sum over all waves and both lane halves (key 0,
        // in wave 0's half 0, makes M finite)
        float M = -INFINITY;
#pragma unroll
        for (int s = 0; s < KS; s++) M = fmaxf(M, fmaxf(red[s][0][li], red[s][0][li + 32]));
        float L = 0.0f;
#pragma unroll
        for (int s = 0; s < KS; s++)
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const float ms = red[s][0][li + 32 * hf];
                if (ms != -INFINITY) L += red[s][1][li + 32 * hf] * __builtin_amdgcn_exp2f(ms - M);
            }
        const float inv_sum = 1.0f / L;

        // pass 2: normalized probabilities, export, P.V
        f32x16 oacc[DT];
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int q = 0; q < 16; q++) oacc[t][q] = 0.0f;
        float *Prow = (P && qi < len) ? P + b * pb + h * ph + (size_t)qi * S_max : nullptr;
        float rs = 0.0f;
        for (int t = w; t < ntile; t += KS) {
            const int kt0 = t * 32;
            wave_sync();
            load_k(kt0);
            load_v(kt0);
            wave_sync();
            f32x16 acc;
            scores(acc, 0.0f);
            float p[16];
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
                p[q] = key < len ? __builtin_amdgcn_exp2f(acc[q] - M) * inv_sum : 0.0f;
            }
            if (Prow) store_p(Prow, p, kt0 + 4 * hh, len);
            if (rowsum) rs += tile_residue_sum(p, kt0, hh, len);
            pv(oacc, p);
        }
        red[w][2][lane] = rs;
        __syncthreads();  // every wave is done with its stages
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int q = 0; q < 16; q++) ox[((w * DT + t) * 16 + q) * 64 + lane] = oacc[t][q];
        __syncthreads();
        if (w != 0) return;
        float rsum = red[0][2][lane];
#pragma unroll
        for (int s = 1; s < KS; s++) rsum += red[s][2][lane];
        write_rowsum(rowsum, rsum, b, h, H, S_max, qi, len, hh);
        finish(1.0f);
    }
}

// Combines the nsplit partial results of each split task (k_attention_h):
// O = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s with M = max_s m_s (the
// running maxima are in base-2 units).  One thread per (task, query, 4 dims).
template <int HD>
__global__ __launch_bounds__(256) void k_attention_merge(const float *__restrict__ part, int ntask, int nsplit,
                                                         int nfull, int H, int nq, int QB, const int *__restrict__ cu,
                                                         const int *__restrict__ lens, int d, void *__restrict__ out,
                                                         int out_fmt) {
    constexpr int G = HD / 4;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)ntask * QB * G) return;
    const int st = (int)(i / ((long)QB * G)), rem = (int)(i % ((long)QB * G)), q = rem / G, c = 4 * (rem % G);
    const int task = nfull + st, qb = task % nq, h = (task / nq) % H, b = task / nq / H;
    const int qi = qb * QB + q;
    if (qi >= lens[b]) return;
    const float *p0 = part + ((size_t)st * nsplit * QB + q) * (HD + 2);
    const size_t step = (size_t)QB * (HD + 2);
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, p0[s * step + HD]);
    float L = 0.0f, o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f;
    for (int s = 0; s < nsplit; s++) {
        const float *ps = p0 + s * step;
        const float w = __builtin_amdgcn_exp2f(ps[HD] - M);  // an empty range: m = -inf, w = 0
        L += w * ps[HD + 1];
        o0 += w * ps[c];
        o1 += w * ps[c + 1];
        o2 += w * ps[c + 2];
        o3 += w * ps[c + 3];
    }
    const float inv = 1.0f / L;
    const float4 v = make_float4(o0 * inv, o1 * inv, o2 * inv, o3 * inv);
    const size_t row = (size_t)cu[b] + qi;
    if (out_fmt == AF_X3)
        x3_store4(reinterpret_cast<unsigned short *>(out), row, h * HD + c, d, v);
    else if (out_fmt == AF_H2)
        h2_store4(reinterpret_cast<unsigned short *>(out), row, h * HD + c, d, v);
    else
        *reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + row * d + h * HD + c) = v;
}

// 16 bytes global -> LDS by the load unit: lane l writes LDS bytes
// [lds_base + 16 l, +16).  Issued from inline assembly so that the compiler,
// which cannot see these LDS writes, does not wait for them at every LDS read
// (the kernels wait with explicit vmcnt counts before their barriers).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; listing it keeps values out of it here
__device__ __forceinline__ void dma16(const void *g, unsigned lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_base), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop

// Attention over K/V tile images (kv_image.h): the same tasks, key split,
// arithmetic and outputs as k_attention_h, but a key tile is staged by a flat
// copy of its image (global_load_lds, issued one tile ahead into the other of
// two LDS stages) instead of being rotated, split and transposed here; one
// barrier per tile.  The one-pass softmax keeps its exponent offset m until
// a score exceeds it by more than 8 (base-2 units), so the accumulators are
// rescaled rarely and p <= 256 (the normalisation is unchanged: o / l with o
// and l under the same offset).
template <int HD, bool ONEPASS, int NTH>
__global__ __launch_bounds__(NTH, ONEPASS || HD <= 32 ? 4 : 2) void k_attention_img(
    const float *__restrict__ qkv, int d, const int *__restrict__ cu, const int *__restrict__ lens, int S_max,
    const int *__restrict__ tb, const unsigned char *__restrict__ img, const float *__restrict__ rc,
    const float *__restrict__ rsn, void *__restrict__ out, int out_fmt, float *__restrict__ P, long long pb,
    long long ph, float inv_scale, float *__restrict__ rowsum, int H, int nq, int nfull, int nsplit,
    float *__restrict__ part, int xcd_pairs) {
    // no FMA contraction: the staged and the image kernel round alike
#pragma clang fp contract(off)
    using I = KvImg<HD>;
    constexpr int HALF = I::HALF, HDP = I::HDP, NC = HDP / 16, VW = I::VW, DT = VW / 32, TB = I::TB;
    constexpr int NWV = NTH / 64;
    constexpr int NJ = TB / 1024, JPW = (NJ + NWV - 1) / NWV;             // whole tile
    constexpr int NJK = I::VOFF / 1024, JPWK = (NJK + NWV - 1) / NWV;     // K rows only
    __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * TB];

    int task = blockIdx.x, ks = 0, ns = 1;
    if (task >= nfull) {
        const int t = task - nfull;
        task = nfull + t / nsplit;
        ks = t % nsplit;
        ns = nsplit;
    } else if (xcd_pairs) {
        // Workgroups go to the 8 XCDs in turn (id % 8); the nq query blocks
        // of one (sequence, head) read the same K/V images, so they are given
        // ids 8 apart: one XCD, whose L2 then serves the image to the others.
        // Ids in groups of 8 nq: block qb of head pair p = 8 g + r at 8 nq g + 8 qb + r.
        const int g = task / (8 * nq), r = task % (8 * nq);
        task = (8 * g + r % 8) * nq + r / 8;
    }
    const int qb = task % nq, h = (task / nq) % H, b = task / nq / H;
    const int len = lens[b], base = cu[b];
    const int qblk = qb * (NTH / 2);
    if (qblk >= len) return;
    const int ntile_all = (len + 31) / 32, per = (ntile_all + ns - 1) / ns;
    const int t0 = min(ks * per, ntile_all), t1 = min((ks + 1) * per, ntile_all);  // tiles [t0, t1)
    const int kend = min(t1 * 32, len);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 31, hh = lane >> 5;
    const size_t ld = (size_t)3 * d;
    const float sl2 = inv_scale * 1.44269504088896340736f;

    // rotated query dims 16c + 8hh + e of this lane's query, as f16 limbs
    // (pre-scaled by log2(e) / sqrt(hd) in the one-pass kernel, as in k_attention_h)
    const int qi = qblk + wave * 32 + li;
    const int qc = min(qi, len - 1);
    f16x8 qh[NC], ql[NC];
    {
        const float *qrow = qkv + (size_t)(base + qc) * ld + h * HD;
        const float *cs = rc + (size_t)qc * HALF, *sn = rsn + (size_t)qc * HALF;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int dim = 16 * c + 8 * hh + e;
                float r = 0.0f;
                if (dim < HALF) r = rot_lo(qrow[dim], qrow[dim + HALF], cs[dim], sn[dim]);
                else if (dim < HD) r = rot_hi(qrow[dim], qrow[dim - HALF], cs[dim - HALF], sn[dim - HALF]);
                v[e] = opaque(r * sl2);
            }
            split8_mix(v, qh[c], ql[c]);
        }
    }

    // image of key tile t (absolute within the sequence) of this head
    const unsigned char *himg = img + ((size_t)tb[b] * H + h) * TB;
    const unsigned lds0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)lds);
    // Copies tile t into stage stg: instruction j (1 KiB) is issued by wave j % NWV.
    auto dma = [&](int t, int stg, auto with_v) __attribute__((always_inline)) {
        constexpr int nj = decltype(with_v)::value ? NJ : NJK, jpw = decltype(with_v)::value ? JPW : JPWK;
        const unsigned char *src = himg + (size_t)t * H * TB + lane * 16;
#pragma unroll
        for (int i = 0; i < jpw; i++) {
            const int j = i * NWV + wave;
            if (j < nj) dma16(src + j * 1024, __builtin_amdgcn_readfirstlane(lds0 + stg * TB + j * 1024));
        }
    };
    // S^T tile (32 keys x 32 queries) + c0 from stage st
    auto scores = [&](const unsigned char *st, f32x16 &acc, float c0) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 16; q++) acc[q] = c0;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int dim = 16 * c + 8 * hh;
            const f16x8 kh = *reinterpret_cast<const f16x8 *>(st + li * I::KRP + I::kchunk(li, I::klc(dim, 0)) * 16);
            const f16x8 kl = *reinterpret_cast<const f16x8 *>(st + li * I::KRP + I::kchunk(li, I::klc(dim, 1)) * 16);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[c], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, ql[c], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[c], acc, 0, 0, 0);
        }
    };
    // O^T += V^T P^T: register 8c + e of lane half hh holds key 16c + 8(e/4) + 4hh + e%4
    auto pv = [&](const unsigned char *st, f32x16 (&oacc)[DT], const float (&p)[16]) __attribute__((always_inline)) {
        f16x8 phi[2], plo[2];
        split8_mix(p, phi[0], plo[0]);
        split8_mix(p + 8, phi[1], plo[1]);
#pragma unroll
        for (int t = 0; t < DT; t++) {
            const int row = t * 32 + li;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const unsigned char *vr = st + I::VOFF + row * 128;
                const f16x8 vh = *reinterpret_cast<const f16x8 *>(vr + I::vchunk(row, 2 * c + hh) * 16);
                const f16x8 vl = *reinterpret_cast<const f16x8 *>(vr + I::vchunk(row, 4 + 2 * c + hh) * 16);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, phi[c], oacc[t], 0, 0, 0);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, plo[c], oacc[t], 0, 0, 0);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl, phi[c], oacc[t], 0, 0, 0);
            }
        }
    };
    // One sweep over tiles [t0, t1): tile t + 1 is copied while tile t is
    // computed.  Before the barrier a wave waits for its own copies of tile
    // t; after it, every wave's copies have landed and every wave is done
    // with the stage tile t + 1 goes to.
    // Whole tiles run in one loop, a partial last tile after it (one inlined
    // copy of the body per loop keeps the register allocation of each).
    auto sweep = [&](auto with_v, auto body) __attribute__((always_inline)) {
        __syncthreads();  // a previous sweep's reads of the stages are done
        if (t0 < t1) dma(t0, 0, with_v);
        auto step = [&](int t, auto masked) __attribute__((always_inline)) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (t + 1 < t1) dma(t + 1, (t - t0 + 1) & 1, with_v);
            body(lds + ((t - t0) & 1) * TB, t * 32, masked);
        };
        const int tw = t1 > t0 && kend < t1 * 32 ? t1 - 1 : t1;  // past the whole tiles (an empty range: t1)
        for (int t = t0; t < tw; t++) step(t, std::false_type{});
        if (tw < t1) step(tw, std::true_type{});
    };

    f32x16 oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
        for (int q = 0; q < 16; q++) oacc[t][q] = 0.0f;
    float out_scale;
    if constexpr (ONEPASS) {
        float m = -INFINITY, l = 0.0f;
        sweep(std::true_type{}, [&](const unsigned char *st, int kt0, auto masked) __attribute__((always_inline)) {
            online_tile<DT, decltype(masked)::value>(
                m, l, oacc, kt0, kend, hh, [&](f32x16 &acc, float c0) { scores(st, acc, c0); },
                [&](const float (&p)[16]) { pv(st, oacc, p); });
        });
        const float lt = l + __shfl_xor(l, 32);
        if (ns > 1) {
            // split task: unnormalized output, exponent offset (base 2) and sum
            if (qi < len) {
                float *pr = part + ((size_t)(blockIdx.x - nfull) * (NTH / 2) + wave * 32 + li) * (HD + 2);
#pragma unroll
                for (int t = 0; t < DT; t++)
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const int dd = t * 32 + 8 * g + 4 * hh;
                        if (dd >= HD) continue;
                        *reinterpret_cast<float2 *>(pr + dd) = make_float2(oacc[t][4 * g], oacc[t][4 * g + 1]);
                        *reinterpret_cast<float2 *>(pr + dd + 2) = make_float2(oacc[t][4 * g + 2], oacc[t][4 * g + 3]);
                    }
                if (hh == 0) *reinterpret_cast<float2 *>(pr + HD) = make_float2(m, lt);
            }
            return;
        }
        out_scale = 1.0f / lt;
    } else {
        // pass 1 (K limbs only): running max / sum of exp per lane
        float m = -INFINITY, l = 0.0f;
        sweep(std::false_type{}, [&](const unsigned char *st, int kt0, auto masked) __attribute__((always_inline)) {
            constexpr bool MASKED = decltype(masked)::value;  // whole tiles: every key is < len
            f32x16 acc;
            scores(st, acc, 0.0f);
            float sv[16];
            float tmax = -INFINITY;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
                sv[q] = !MASKED || key < len ? acc[q] : -INFINITY;
                tmax = fmaxf(tmax, sv[q]);
            }
            const float mn = fmaxf(m, tmax);
            if (mn != -INFINITY) {
                float sum = 0.0f;
#pragma unroll
                for (int q = 0; q < 16; q++) sum += __builtin_amdgcn_exp2f(sv[q] - mn);
                l = l * __builtin_amdgcn_exp2f(m - mn) + sum;
                m = mn;
            }
        });
        const float mo = __shfl_xor(m, 32), lo = __shfl_xor(l, 32);
        const float mx = fmaxf(m, mo);
        const float inv_sum = 1.0f / (l * __builtin_amdgcn_exp2f(m - mx) + lo * __builtin_amdgcn_exp2f(mo - mx));
        // pass 2: normalized probabilities, optional export, P.V
        float *Prow = (P && qi < len) ? P + b * pb + h * ph + (size_t)qi * S_max : nullptr;
        const bool p_al = P && ((uintptr_t)P & 15) == 0 && ((pb | ph | (long long)S_max) & 3) == 0;
        float rs = 0.0f;
        sweep(std::true_type{}, [&](const unsigned char *st, int kt0, auto masked) __attribute__((always_inline)) {
            constexpr bool MASKED = decltype(masked)::value;  // whole tiles: every key is < len
            f32x16 acc;
            scores(st, acc, 0.0f);
            float p[16];
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int key = kt0 + 8 * (q >> 2) + 4 * hh + (q & 3);
                p[q] = !MASKED || key < len ? __builtin_amdgcn_exp2f(acc[q] - mx) * inv_sum : 0.0f;
            }
            if (Prow) {
                if (!MASKED && p_al) store_p_whole(Prow, p, kt0 + 4 * hh);
                else store_p(Prow, p, kt0 + 4 * hh, len);
            }
            if (rowsum) rs += tile_residue_sum(p, kt0, hh, len);
            pv(st, oacc, p);
        });
        write_rowsum(rowsum, rs, b, h, H, S_max, qi, len, hh);
        out_scale = 1.0f;
    }
    if (qi < len) {
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int dd = t * 32 + 8 * g + 4 * hh;
                if (dd >= HD) continue;
                const float4 v = make_float4(oacc[t][4 * g] * out_scale, oacc[t][4 * g + 1] * out_scale,
                                             oacc[t][4 * g + 2] * out_scale, oacc[t][4 * g + 3] * out_scale);
                if (out_fmt == AF_X3)
                    x3_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
                else if (out_fmt == AF_H2)
                    h2_store4(reinterpret_cast<unsigned short *>(out), base + qi, h * HD + dd, d, v);
                else
                    *reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + (size_t)(base + qi) * d + h * HD +
                                                dd) = v;
            }
    }
}

// Per-forward set-up of the tile images, one workgroup per (sequence b,
// head h): tb[b] = sum of ceil(len / 32) over the sequences before b; pk =
// 32 tb[b] + position and pos = position for its tokens, and the tile-row
// table ti (head 0's workgroup); the padding keys (positions len..) of the
// last tile are zeroed in head h's image, both limbs — the K rows as whole
// 16-byte stores (they are contiguous), the V positions one by one — so that
// masked keys multiply zeros whatever an earlier batch left there.
template <int HD>
__global__ __launch_bounds__(256) void k_kv_setup(const int *__restrict__ cu, const int *__restrict__ lens, int H,
                                                  int *__restrict__ tb, int *__restrict__ pk, int *__restrict__ pos,
                                                  int *__restrict__ ti, unsigned char *__restrict__ img) {
    using I = KvImg<HD>;
    const int b = blockIdx.x, h = blockIdx.y;
    __shared__ int s_first;
    if (threadIdx.x == 0) {
        int f = 0;
        for (int i = 0; i < b; i++) f += (lens[i] + 31) / 32;
        s_first = f;
        if (h == 0) tb[b] = f;
    }
    __syncthreads();
    const int first = s_first, len = lens[b], base = cu[b];
    if (h == 0) {
        for (int t = threadIdx.x; t < len; t += 256) {
            pk[base + t] = first * 32 + t;
            pos[base + t] = t;
        }
        for (int t = threadIdx.x; t < (len + 31) / 32; t += 256)
            *reinterpret_cast<int4 *>(ti + 4 * (first + t)) = make_int4(base + 32 * t, min(32, len - 32 * t), 32 * t, b);
    }
    const int pad = (32 - len % 32) % 32;
    if (pad == 0 || len == 0) return;
    const int last = first + (len - 1) / 32, k0 = len % 32;
    unsigned char *t = img + ((size_t)last * H + h) * I::TB;
    // K rows k0..31: bytes [k0 KRP, 32 KRP) of the image
    for (int i = threadIdx.x; i < pad * I::KRP / 16; i += 256)
        *reinterpret_cast<uint4 *>(t + k0 * I::KRP + 16 * i) = make_uint4(0u, 0u, 0u, 0u);
    // V: (limb, dim row, padding key)
    for (int i = threadIdx.x; i < 2 * I::VW * pad; i += 256) {
        const int limb = i / (I::VW * pad), r = i % (I::VW * pad), dim = r / pad, key = k0 + r % pad;
        *reinterpret_cast<_Float16 *>(t + I::voff(key, dim, limb)) = (_Float16)0.0f;
    }
}

// Tile images from FP32 Q|K|V rows, for projections that did not write them
// in their epilogue (GEMV, the register-staged GEMMs, FP32 weights, head size
// 24): the same rotation and split as the LDS GEMM's QKV epilogue, so both
// give the same bytes.  One wave per (tile row, head): lane k < 32 rotates
// key k's K row and writes its 16-byte chunks (8 dims of one limb); lane
// 32 + k splits key k's V row into LDS at its V^T position, and after a
// barrier the wave writes the V^T chunks (8 key positions of one dim and
// limb).  Padding keys are left to k_kv_setup, padding dims are zero from
// the allocation.
template <int HD>
__global__ __launch_bounds__(64) void k_kv_prep(const float *__restrict__ qkv, int d, const int *__restrict__ ti,
                                                const float *__restrict__ rc, const float *__restrict__ rsn,
                                                unsigned char *__restrict__ img, int H) {
    using I = KvImg<HD>;
    constexpr int HALF = HD / 2, NG = HD / 8;  // 8-dim groups of a row
    __shared__ __attribute__((aligned(16))) unsigned short vt[2][HD][32];  // [limb][dim][position]
    const int tr = blockIdx.x / H, h = blockIdx.x % H;
    const int4 info = *reinterpret_cast<const int4 *>(ti + 4 * tr);  // first packed row, keys, first position
    const int kt0 = info.z, nk = info.y;
    const size_t ld = (size_t)3 * d;
    const float *base = qkv + (size_t)info.x * ld + h * HD;
    unsigned char *t = img + ((size_t)tr * H + h) * I::TB;
    const int lane = threadIdx.x, key = lane & 31;
    auto pack8 = [](const unsigned short (&v)[8]) __attribute__((always_inline)) {
        return make_uint4(v[0] | (unsigned)v[1] << 16, v[2] | (unsigned)v[3] << 16, v[4] | (unsigned)v[5] << 16,
                          v[6] | (unsigned)v[7] << 16);
    };
    if (lane < 32) {
        if (key < nk) {
            const float *k = base + (size_t)key * ld + d;
            const float *c = rc + (size_t)(kt0 + key) * HALF, *sn = rsn + (size_t)(kt0 + key) * HALF;
            float x[HD], cs[HALF], ss[HALF];
#pragma unroll
            for (int j = 0; j < HD; j += 4)
                *reinterpret_cast<float4 *>(&x[j]) = *reinterpret_cast<const float4 *>(k + j);
#pragma unroll
            for (int j = 0; j < HALF; j += 4) {
                *reinterpret_cast<float4 *>(&cs[j]) = *reinterpret_cast<const float4 *>(c + j);
                *reinterpret_cast<float4 *>(&ss[j]) = *reinterpret_cast<const float4 *>(sn + j);
            }
#pragma unroll
            for (int g = 0; g < NG; g++) {
                unsigned short h8[8], l8[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int j = 8 * g + e;
                    const float r = j < HALF ? rot_lo(x[j], x[j + HALF], cs[j], ss[j])
                                             : rot_hi(x[j], x[j - HALF], cs[j - HALF], ss[j - HALF]);
                    const _Float16 rh = (_Float16)r, rl = (_Float16)(r - (float)rh);
                    h8[e] = __builtin_bit_cast(unsigned short, rh);
                    l8[e] = __builtin_bit_cast(unsigned short, rl);
                }
                *reinterpret_cast<uint4 *>(t + I::koff(key, 8 * g, 0)) = pack8(h8);
                *reinterpret_cast<uint4 *>(t + I::koff(key, 8 * g, 1)) = pack8(l8);
            }
        }
    } else {
        // key's V row into LDS at position vpos(key); keys past the tile's end are zero
        const int p = I::vpos(key);
        float x[HD];
#pragma unroll
        for (int j = 0; j < HD; j += 4)
            *reinterpret_cast<float4 *>(&x[j]) = key < nk ? *reinterpret_cast<const float4 *>(base + (size_t)key * ld + 2 * d + j)
                                                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int j = 0; j < HD; j++) {
            const _Float16 vh = (_Float16)x[j], vl = (_Float16)(x[j] - (float)vh);
            vt[0][j][p] = __builtin_bit_cast(unsigned short, vh);
            vt[1][j][p] = __builtin_bit_cast(unsigned short, vl);
        }
    }
    __syncthreads();
    // V^T chunks: (limb, dim, positions 8q .. 8q + 7)
    for (int i = lane; i < 2 * HD * 4; i += 64) {
        const int limb = i / (HD * 4), r = (i >> 2) % HD, q = i & 3;
        *reinterpret_cast<uint4 *>(t + I::voff(I::vpos(8 * q), r, limb)) =
            *reinterpret_cast<const uint4 *>(&vt[limb][r][8 * q]);
    }
}

// Rows of partial results the key split may use: one row per query of a
// workgroup slot, two rounds of 256-query (or four of 128-query) slots.
size_t attention_part_floats(int hd) { return (size_t)device_cus() * 512 * (hd + 2); }

hipError_t launch_attention(const float *qkv, int d, int H, SeqMeta sm, const float *rope_cos, const float *rope_sin,
                            void *out, int out_fmt, float *P, int64_t pb, int64_t ph, float *rowsum, float *part,
                            size_t part_floats, hipStream_t st) {
    if (rowsum && !P) return hipErrorInvalidValue;
    if ((out_fmt == AF_X3 || out_fmt == AF_H2) && d % 32) return hipErrorInvalidValue;
    const int hd = d / H;
    const float inv_scale = 1.0f / sqrtf((float)hd);
    const char *e = getenv("CIH_ATT");
    const bool fp32 = (e && !strcmp(e, "fp32")) || full_range_mode();
    // f16-limb kernel: 256 queries per workgroup (8 waves) halve the K/V tile
    // staging per query when that still leaves two workgroups per CU, else 128
    // (more workgroups for short batches).  CIH_ATT_QB=128|256 forces one.
    const char *qe = getenv("CIH_ATT_QB");
    bool wide = (long)((sm.S_max + 255) / 256) * H * sm.B >= 512;
    if (qe && !strcmp(qe, "128")) wide = false;
    if (qe && !strcmp(qe, "256")) wide = true;
    int QB = wide ? 256 : 128;
    // With a probability export there is no key split: batches whose 128-query
    // tasks do not cover the compute units take 64- or 32-query workgroups
    // (the per-query arithmetic does not depend on the block: same bits).
    if (P && !fp32 && !wide && !qe) {
        const long t128 = (long)((sm.S_max + 127) / 128) * H * sm.B;
        if (t128 < device_cus()) QB = t128 * 2 < device_cus() ? 32 : 64;
    }
    const int nq = (sm.S_max + QB - 1) / QB;
    const int tasks = sm.B * H * nq;
    // Key split (no probability export): when the tasks do not fill one round
    // of the 'slots' workgroups resident at once (two of 256 or four of 128
    // queries per CU), each is cut into nsplit key ranges (at least two
    // 32-key tiles each) so that they do (a single 402-token sequence: 80
    // tasks in six ranges, attention 41 -> 27 us per layer).  Splitting only
    // the tasks past the last whole round of a larger batch measured no gain
    // (the headline batch: 640 tasks on 512 slots, 3.85 vs 3.82 ms per
    // forward): the parts repeat the query staging and add the merge.  Nor
    // did counting only the tasks that hold queries in a ragged batch (35M
    // B=8, lengths 128-510: 460 of 640 tasks, two ranges each): attention
    // 0.37 -> 0.51 ms per forward, as two workgroups per CU already keep
    // this issue-bound kernel busy.
    // CIH_ATT_SPLIT=0 or CIH_SPLITK=0 turn it off.
    int nfull = tasks, nsplit = 1;
    const char *se = getenv("CIH_ATT_SPLIT"), *ke = getenv("CIH_SPLITK");
    const bool split_ok = !P && !fp32 && part && !(se && !strcmp(se, "0")) && !(ke && !strcmp(ke, "0"));
    const int slots = 2 * device_cus() * (wide ? 1 : 2);
    if (split_ok && tasks < slots) {
        const int full = 0, rest = tasks;
        int ns = std::min(slots / rest, (sm.S_max + 31) / 32 / 2);
        while (ns > 1 && (size_t)rest * ns * QB * (hd + 2) > part_floats) ns--;
        if (ns > 1) {
            nfull = full;
            nsplit = ns;
        }
    }
    const int grid = nfull + (tasks - nfull) * nsplit;
    // When even 32-query tasks fit one round of one workgroup per CU, the 8
    // waves of each 32-query task split its keys instead (k_attention_xs);
    // the switches of the key split turn it off.
    const int nq32 = (sm.S_max + 31) / 32, t32 = sm.B * H * nq32;
    const bool xsplit = !fp32 && attention_wave_split(sm.B, sm.S_max, H);
#define CIH_ATT_K(KER, HDV, ONE)                                                                                \
    hipLaunchKernelGGL((KER<HDV, ONE>), dim3((sm.S_max + 127) / 128, H, sm.B), dim3(256), 0, st, qkv, d, sm.cu, \
                       sm.lens, sm.S_max, rope_cos, rope_sin, out, out_fmt, P, (long long)pb, (long long)ph,     \
                       inv_scale, rowsum)
#define CIH_ATT_H(HDV, ONE, NTH)                                                                                 \
    hipLaunchKernelGGL((k_attention_h<HDV, ONE, NTH>), dim3(grid), dim3(NTH), 0, st, qkv, d, sm.cu, sm.lens,     \
                       sm.S_max, rope_cos, rope_sin, out, out_fmt, P, (long long)pb, (long long)ph, inv_scale, rowsum, \
                       H, nq, nfull, nsplit, part)
#define CIH_ATT(HDV)                                                                                           \
    if (xsplit && P)                                                                                            \
        hipLaunchKernelGGL((k_attention_xs<HDV, 8, false>), dim3(t32), dim3(512), 0, st, qkv, d, sm.cu, sm.lens, \
                           sm.S_max, rope_cos, rope_sin, out, out_fmt, P, (long long)pb, (long long)ph, inv_scale, \
                           rowsum, H, nq32);                                                                    \
    else if (xsplit)                                                                                            \
        hipLaunchKernelGGL((k_attention_xs<HDV, 8, true>), dim3(t32), dim3(512), 0, st, qkv, d, sm.cu, sm.lens,  \
                           sm.S_max, rope_cos, rope_sin, out, out_fmt, P, (long long)pb, (long long)ph, inv_scale, \
                           rowsum, H, nq32);                                                                    \
    else if (fp32 && P) CIH_ATT_K(k_attention, HDV, false);                                                     \
    else if (fp32) CIH_ATT_K(k_attention, HDV, true);                                                           \
    else if (P && wide) CIH_ATT_H(HDV, false, 512);                                                             \
    else if (P && QB == 32) CIH_ATT_H(HDV, false, 64);                                                          \
    else if (P && QB == 64) CIH_ATT_H(HDV, false, 128);                                                         \
    else if (P) CIH_ATT_H(HDV, false, 256);                                                                     \
    else if (wide) CIH_ATT_H(HDV, true, 512);                                                                   \
    else CIH_ATT_H(HDV, true, 256);                                                                             \
    if (nsplit > 1 && !xsplit) {                                                                                \
        const long n = (long)(tasks - nfull) * QB * (HDV / 4);                                                  \
        hipLaunchKernelGGL((k_attention_merge<HDV>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, \
                           tasks - nfull, nsplit, nfull, H, nq, QB, sm.cu, sm.lens, d, out, out_fmt);           \
    }
    switch (hd) {
    case 16: CIH_ATT(16) break;
    case 24: CIH_ATT(24) break;
    case 32: CIH_ATT(32) break;
    case 64: CIH_ATT(64) break;
    default: return hipErrorInvalidValue;
    }
#undef CIH_ATT
#undef CIH_ATT_H
#undef CIH_ATT_K
    return hipGetLastError();
}

bool attention_img_supported(int hd) { return hd == 16 || hd == 24 || hd == 32 || hd == 64; }

bool attention_wave_split(int B, int S_max, int H) {
    const char *se = getenv("CIH_ATT_SPLIT"), *ke = getenv("CIH_SPLITK");
    const long t32 = (long)B * H * ((S_max + 31) / 32);
    return t32 <= device_cus() && !(se && !strcmp(se, "0")) && !(ke && !strcmp(ke, "0"));
}

size_t kv_image_bytes(int hd) {
    switch (hd) {
    case 16: return KvImg<16>::TB;
    case 24: return KvImg<24>::TB;
    case 32: return KvImg<32>::TB;
    case 64: return KvImg<64>::TB;
    default: return 0;
    }
}

hipError_t launch_kv_setup(SeqMeta sm, int hd, int H, int *tb, int *pk, int *pos, int *ti, unsigned char *img,
                           hipStream_t st) {
    if (sm.B <= 0) return hipSuccess;
#define CIH_KVS(HDV)                                                                                               \
    hipLaunchKernelGGL((k_kv_setup<HDV>), dim3(sm.B, H), dim3(256), 0, st, sm.cu, sm.lens, H, tb, pk, pos, ti, img)
    switch (hd) {
    case 16: CIH_KVS(16); break;
    case 24: CIH_KVS(24); break;
    case 32: CIH_KVS(32); break;
    case 64: CIH_KVS(64); break;
    default: return hipErrorInvalidValue;
    }
#undef CIH_KVS
    return hipGetLastError();
}

hipError_t launch_kv_prep(const float *qkv, int d, int H, const int *ti, int tile_rows, const float *rope_cos,
                          const float *rope_sin, unsigned char *img, hipStream_t st) {
    if (tile_rows <= 0) return hipSuccess;
    const unsigned grid = (unsigned)tile_rows * H;
#define CIH_KVP(HDV)                                                                                              \
    hipLaunchKernelGGL((k_kv_prep<HDV>), dim3(grid), dim3(64), 0, st, qkv, d, ti, rope_cos, rope_sin, img, H)
    switch (d / H) {
    case 16: CIH_KVP(16); break;
    case 24: CIH_KVP(24); break;
    case 32: CIH_KVP(32); break;
    case 64: CIH_KVP(64); break;
    default: return hipErrorInvalidValue;
    }
#undef CIH_KVP
    return hipGetLastError();
}

hipError_t launch_attention_img(const float *qkv, int d, int H, SeqMeta sm, const int *tb, const unsigned char *img,
                                const float *rope_cos, const float *rope_sin, void *out, int out_fmt, float *P,
                                int64_t pb, int64_t ph, float *rowsum, float *part, size_t part_floats, hipStream_t st) {
    if (rowsum && !P) return hipErrorInvalidValue;
    if ((out_fmt == AF_X3 || out_fmt == AF_H2) && d % 32) return hipErrorInvalidValue;
    const int hd = d / H;
    if (!attention_img_supported(hd) || d != hd * H) return hipErrorInvalidValue;
    const float inv_scale = 1.0f / sqrtf((float)hd);
    // query blocks and key split as in launch_attention
    const char *qe = getenv("CIH_ATT_QB");
    bool wide = (long)((sm.S_max + 255) / 256) * H * sm.B >= 512;
    if (qe && !strcmp(qe, "128")) wide = false;
    if (qe && !strcmp(qe, "256")) wide = true;
    const int QB = wide ? 256 : 128, nq = (sm.S_max + QB - 1) / QB;
    const int tasks = sm.B * H * nq;
    int nfull = tasks, nsplit = 1;
    const char *se = getenv("CIH_ATT_SPLIT"), *ke = getenv("CIH_SPLITK");
    const bool split_ok = !P && part && !(se && !strcmp(se, "0")) && !(ke && !strcmp(ke, "0"));
    const int slots = 2 * device_cus() * (wide ? 1 : 2);
    if (split_ok && tasks < slots) {
        int ns = std::min(slots / tasks, (sm.S_max + 31) / 32 / 2);
        while (ns > 1 && (size_t)tasks * ns * QB * (hd + 2) > part_floats) ns--;
        if (ns > 1) {
            nfull = 0;
            nsplit = ns;
        }
    }
    const int grid = nfull + (tasks - nfull) * nsplit;
    // the query blocks of a head on one XCD: unsplit grids of whole groups of 8 heads
    const char *xe = getenv("CIH_ATT_XCD");
    const int xcd_pairs = nq > 1 && nfull == tasks && (sm.B * H) % 8 == 0 && !(xe && !strcmp(xe, "0"));
#define CIH_ATI(HDV, ONE, NTH)                                                                                   \
    hipLaunchKernelGGL((k_attention_img<HDV, ONE, NTH>), dim3(grid), dim3(NTH), 0, st, qkv, d, sm.cu, sm.lens,    \
                       sm.S_max, tb, img, rope_cos, rope_sin, out, out_fmt, P, (long long)pb, (long long)ph,      \
                       inv_scale, rowsum, H, nq, nfull, nsplit, part, xcd_pairs)
#define CIH_ATI_HD(HDV)                                                                                          \
    if (P && wide) CIH_ATI(HDV, false, 512);                                                                      \
    else if (P) CIH_ATI(HDV, false, 256);                                                                         \
    else if (wide) CIH_ATI(HDV, true, 512);                                                                       \
    else CIH_ATI(HDV, true, 256);                                                                                 \
    if (nsplit > 1) {                                                                                             \
        const long n = (long)(tasks - nfull) * QB * (HDV / 4);                                                    \
        hipLaunchKernelGGL((k_attention_merge<HDV>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part,   \
                           tasks - nfull, nsplit, nfull, H, nq, QB, sm.cu, sm.lens, d, out, out_fmt);             \
    }
    switch (hd) {
    case 16: CIH_ATI_HD(16) break;
    case 24: CIH_ATI_HD(24) break;
    case 32: CIH_ATI_HD(32) break;
    case 64: CIH_ATI_HD(64) break;
    default: return hipErrorInvalidValue;
    }
#undef CIH_ATI_HD
#undef CIH_ATI
    return hipGetLastError();
}

}  // namespace cih
