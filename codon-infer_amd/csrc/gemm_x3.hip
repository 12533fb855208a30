// Quantized GEMM on 16-bit MFMA with exact integer weights:
//   Y = epi(X * W^T + b),  W in Q8_0 / Q4_0 blocks of 32.
//
// Same result as matmul_tiled_q8/q4_parallel (codon-infer src/lib.rs:4870,
// 4937) to FP32 rounding, several times the FP32-MFMA rate:
//   * The block's quants q (|q| <= 127, or -8..7 for Q4_0) are exact in bf16
//     and in f16.
//   * Each FP32 activation is split into limbs whose sum carries (nearly) all
//     of its 24 significant bits:
//       LIMB_F16X2 (default): x = h0 + h1, h0 = f16(x), h1 = f16(x - h0):
//         22-23 bits; relative error <= 2^-22, absolute <= 2^-25 (f16
//         subnormals, which the f16 MFMA keeps); |x| must stay below 65520;
//       LIMB_BF16X3: x = b0 + b1 + b2 (b0 = bf16(x), b1 = bf16(x - b0),
//         b2 = bf16(x - b0 - b1)): 24 bits, full FP32 range.
//   Activations arrive as FP32 (split while staging) or already split by
//   their producer (AF_H2 for f16 limbs, AF_X3 for bf16 limbs: x3.h).
//   * Every limb x q product is exact in the MFMA's FP32 accumulator, so per
//     32-element block tmp = sum_k (limbs)_k q_k is the FP32 dot product of
//     the block, and acc += d * tmp applies the block scale in FP32.
// The reference forms w = q*d first and then sums w*x (lib.rs:4687, 4724-4741,
// 4476-4492); this is the same sum regrouped per block, with FP32 rounding.
//
// Tiling: 256 threads = 4 waves (2x2), workgroup tile BM x BN, BK = 32 = one
// block.  v_mfma_f32_32x32x16_{f16,bf16}: lane (i = lane%32, half = lane/32) feeds
// the 8 elements 16*kh + 8*half + e of k-half kh.  For Q4_0 that is the low
// nibbles (kh = 0) and high nibbles (kh = 1) of bytes 8*half..8*half+7: the
// reference's packing.  The activation split and the integer-to-bf16
// conversion happen once per workgroup while staging into LDS; two LDS stages
// alternate (one barrier per block) and the block after next is fetched into
// registers during the current block's MFMAs.
#include <algorithm>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kernels.h"
#include "x3.h"

namespace cih {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
// staging registers as a plain vector type (the struct-with-union uint4 kept
// the prefetch arrays in scratch memory)
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

enum Limb { LIMB_BF16X3 = 0, LIMB_F16X2 = 1 };
template <int LIMB> struct LimbT;
template <> struct LimbT<LIMB_BF16X3> { using V = bf16x8; static constexpr int NL = 3, AROW = 104; };
template <> struct LimbT<LIMB_F16X2> { using V = f16x8; static constexpr int NL = 2, AROW = 72; };

constexpr int XL = 40;    // 16-bit values per LDS column of B (32 + 8 pad): conflict-free 16-byte reads
// A rows in LDS: NL limbs x 32 + 8 pad (208 B / 144 B)

__device__ __forceinline__ unsigned pack_bf16(float lo, float hi) {
    // round-to-nearest-even f32 -> bf16 for both halves
    __bf16 a = (__bf16)lo, b = (__bf16)hi;
    return (unsigned)__builtin_bit_cast(unsigned short, a) | ((unsigned)__builtin_bit_cast(unsigned short, b) << 16);
}
// bf16 of two floats that are exact in bf16 (small integers): the high halves
__device__ __forceinline__ unsigned pack_exact(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}
__device__ __forceinline__ float bf16_lo(unsigned p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(unsigned p) { return __uint_as_float(p & 0xFFFF0000u); }

// x0..x3 -> three limbs, each as two packed bf16 dwords
__device__ __forceinline__ void split4(float4 x, uint2 &l0, uint2 &l1, uint2 &l2) {
    l0.x = pack_bf16(x.x, x.y);
    l0.y = pack_bf16(x.z, x.w);
    float r0 = x.x - bf16_lo(l0.x), r1 = x.y - bf16_hi(l0.x), r2 = x.z - bf16_lo(l0.y), r3 = x.w - bf16_hi(l0.y);
    l1.x = pack_bf16(r0, r1);
    l1.y = pack_bf16(r2, r3);
    r0 -= bf16_lo(l1.x); r1 -= bf16_hi(l1.x); r2 -= bf16_lo(l1.y); r3 -= bf16_hi(l1.y);
    l2.x = pack_bf16(r0, r1);
    l2.y = pack_bf16(r2, r3);
}

// two f16 (round to nearest even) packed low | high << 16
__device__ __forceinline__ unsigned pack_f16(float lo, float hi) {
    const _Float16 a = (_Float16)lo, b = (_Float16)hi;
    return (unsigned)__builtin_bit_cast(unsigned short, a) | ((unsigned)__builtin_bit_cast(unsigned short, b) << 16);
}
__device__ __forceinline__ float f16_lo(unsigned p) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(p & 0xFFFFu));
}
__device__ __forceinline__ float f16_hi(unsigned p) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(p >> 16)); }

// x0..x3 -> two f16 limbs, each as two packed dwords
__device__ __forceinline__ void split4_f16(float4 x, uint2 &l0, uint2 &l1) {
    l0.x = pack_f16(x.x, x.y);
    l0.y = pack_f16(x.z, x.w);
    l1.x = pack_f16(x.x - f16_lo(l0.x), x.y - f16_hi(l0.x));
    l1.y = pack_f16(x.z - f16_lo(l0.y), x.w - f16_hi(l0.y));
}

// packed f16 pair minus (1152, 1152) / (1032, 1032); exact for the integer-valued inputs here
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned sub_f16x2(unsigned p, _Float16 c) {
    const f16x2 v = __builtin_bit_cast(f16x2, p) - f16x2{c, c};
    return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ unsigned sub1152(unsigned p) { return sub_f16x2(p, (_Float16)1152.0f); }
__device__ __forceinline__ unsigned sub1032(unsigned p) { return sub_f16x2(p, (_Float16)1032.0f); }

// 16-bit packing of two small integers (exact in both formats)
template <int LIMB>
__device__ __forceinline__ unsigned pack_int(float lo, float hi) {
    if constexpr (LIMB == LIMB_F16X2) return pack_f16(lo, hi);
    else return pack_exact(lo, hi);
}

template <int WF, int EPI, int BM, int BN, int AF, int LIMB, bool SPLIT>
__global__ __launch_bounds__(256, 2) void k_gemm_x3(const void *__restrict__ Xv, int ldx,
                                                    const void *__restrict__ Wq, const float *__restrict__ Wsc,
                                                    const float *__restrict__ bias, void *__restrict__ Yv, int ldy,
                                                    int M, int N, int K, int kps, float *__restrict__ part) {
    constexpr int MT = BM / 64, NT = BN / 64;
    // A tile per k-block: FP32 -> BM*8 float4 (split here); X3 -> BM*12, H2 -> BM*8 16-byte chunks (copied)
    constexpr int A_LOADS = AF == AF_X3 ? BM * 12 / 256 : BM / 32;
    constexpr bool PAIR = WF == WF_F16P;             // f16 quants, K doubled: weight block kb meets A block kb mod KB
    static_assert(!PAIR || LIMB == LIMB_F16X2, "pair weights with f16 limbs only");
    constexpr int B_ITEMS = BN * (PAIR ? 4 : 2);     // (column, quarter or half of the block's bytes)
    constexpr int B_LOADS = (B_ITEMS + 255) / 256;
    constexpr int QB = WF == WF_Q8 ? 32 : (PAIR ? 64 : 16);  // quant bytes per block
    constexpr int NL = LimbT<LIMB>::NL, AROW = LimbT<LIMB>::AROW;
    using V8 = typename LimbT<LIMB>::V;
    static_assert(AF == AF_F32 || (AF == AF_X3) == (LIMB == LIMB_BF16X3), "activation format / limb type mismatch");
    static_assert(EPI != EPI_GELU_H2 || LIMB == LIMB_F16X2, "f16-limb epilogue with f16 limbs only");
    // two LDS stages: block kb+1 is stored while block kb is multiplied (one barrier per block)
    __shared__ __attribute__((aligned(16))) unsigned short Al2[2][BM * AROW];
    __shared__ __attribute__((aligned(16))) unsigned short Bl2[2][BN * XL];
    __shared__ float Ss2[2][BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 31, hh = lane >> 5;
    const int nM = (M + BM - 1) / BM, nN = (N + BN - 1) / BN;
    int mt, nt;
    tile_xcd(blockIdx.x, nM * nN, nM, nN, mt, nt);
    const int m0 = mt * BM, n0 = nt * BN;
    const int KB = K / 32, KBW = PAIR ? 2 * KB : KB;  // activation / weight k-blocks

    // two register stages: block kb+2 is in flight while block kb is multiplied
    u32x4 ra[2][A_LOADS];
    u32x4 rb[2][B_LOADS];  // Q8: 16 bytes (elements 16*part..+15); Q4: 8 bytes in .x/.y
    float rs[2];

    // Every load is unconditional: rows past M and columns past N read the
    // last row / column instead (their outputs are never stored), so the
    // compiler can count outstanding loads and keep the newer stage in
    // flight while the older one is waited for.
    auto gload = [&](int kbw, u32x4 (&a)[A_LOADS], u32x4 (&b)[B_LOADS], float &sc) __attribute__((always_inline)) {
        const int kb = PAIR && kbw >= KB ? kbw - KB : kbw;  // the activation block
#pragma unroll
        for (int i = 0; i < A_LOADS; i++) {
            if constexpr (AF == AF_X3) {
                const int c = tid + 256 * i, row = c / 12, part = c % 12;
                const int gr = min(m0 + row, M - 1);
                a[i] = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const unsigned short *>(Xv) +
                                                        ((size_t)gr * KB + kb) * 96 + part * 8);
            } else if constexpr (AF == AF_H2) {
                const int row = (tid >> 3) + 32 * i, part = tid & 7;
                const int gr = min(m0 + row, M - 1);
                a[i] = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const unsigned short *>(Xv) +
                                                        ((size_t)gr * KB + kb) * 64 + part * 8);
            } else {
                const int row = (tid >> 3) + 32 * i, c4 = tid & 7;
                const int gr = min(m0 + row, M - 1);
                a[i] = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const float *>(Xv) + (size_t)gr * ldx +
                                                        kb * 32 + c4 * 4);
            }
        }
#pragma unroll
        for (int i = 0; i < B_LOADS; i++) {
            const int idx = tid + 256 * i, col = PAIR ? idx >> 2 : idx >> 1, part = PAIR ? idx & 3 : idx & 1;
            const int gc = min(n0 + min(col, BN - 1), N - 1);
            const unsigned char *src = reinterpret_cast<const unsigned char *>(Wq) + ((size_t)kbw * N + gc) * QB;
            if constexpr (WF == WF_Q8 || PAIR) {
                b[i] = *reinterpret_cast<const u32x4 *>(src + part * 16);
            } else {
                const uint2 h = *reinterpret_cast<const uint2 *>(src + part * 8);
                b[i] = u32x4{h.x, h.y, 0u, 0u};
            }
        }
        sc = Wsc[(size_t)kbw * N + min(n0 + min(tid, BN - 1), N - 1)];
    };

    auto sstore = [&](int stg, const u32x4 (&a)[A_LOADS], const u32x4 (&b)[B_LOADS], float sc) __attribute__((always_inline)) {
        unsigned short *Al = Al2[stg], *Bl = Bl2[stg];
        float *Ss = Ss2[stg];
#pragma unroll
        for (int i = 0; i < A_LOADS; i++) {
            if constexpr (AF == AF_X3) {
                // chunk part p of a row = bf16 elements 8p..8p+7 of [limb0|limb1|limb2]
                const int c = tid + 256 * i, row = c / 12, part = c % 12;
                *reinterpret_cast<u32x4 *>(&Al[row * AROW + part * 8]) = a[i];
            } else if constexpr (AF == AF_H2) {
                // chunk part p of a row = f16 elements 8p..8p+7 of [hi|lo]
                const int row = (tid >> 3) + 32 * i, part = tid & 7;
                *reinterpret_cast<u32x4 *>(&Al[row * AROW + part * 8]) = a[i];
            } else {
                const int row = (tid >> 3) + 32 * i, c4 = tid & 7;
                const float4 xv = make_float4(__uint_as_float(a[i].x), __uint_as_float(a[i].y),
                                              __uint_as_float(a[i].z), __uint_as_float(a[i].w));
                if constexpr (LIMB == LIMB_F16X2) {
                    uint2 l0, l1;
                    split4_f16(xv, l0, l1);
                    *reinterpret_cast<uint2 *>(&Al[row * AROW + c4 * 4]) = l0;
                    *reinterpret_cast<uint2 *>(&Al[row * AROW + 32 + c4 * 4]) = l1;
                } else {
                    uint2 l0, l1, l2;
                    split4(xv, l0, l1, l2);
                    *reinterpret_cast<uint2 *>(&Al[row * AROW + c4 * 4]) = l0;
                    *reinterpret_cast<uint2 *>(&Al[row * AROW + 32 + c4 * 4]) = l1;
                    *reinterpret_cast<uint2 *>(&Al[row * AROW + 64 + c4 * 4]) = l2;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < B_LOADS; i++) {
            const int idx = tid + 256 * i, col = PAIR ? idx >> 2 : idx >> 1, part = PAIR ? idx & 3 : idx & 1;
            if (idx >= B_ITEMS) continue;
            const unsigned w[4] = {b[i].x, b[i].y, b[i].z, b[i].w};
            if constexpr (PAIR) {
                // 8 f16 quants = elements 8*part .. 8*part+7
                *reinterpret_cast<u32x4 *>(&Bl[col * XL + part * 8]) = b[i];
            } else if constexpr (WF == WF_Q8 && LIMB == LIMB_F16X2) {
                // 16 int8 = elements 16*part .. 16*part+15.  Biased byte u = q + 128 placed
                // under the f16 exponent of 1024 reads as 1024 + u; subtracting 1152 leaves q.
                unsigned o[8];
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const unsigned u = w[p] ^ 0x80808080u;
                    o[2 * p] = sub1152(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
                    o[2 * p + 1] = sub1152(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
                }
                *reinterpret_cast<u32x4 *>(&Bl[col * XL + part * 16]) = u32x4{o[0], o[1], o[2], o[3]};
                *reinterpret_cast<u32x4 *>(&Bl[col * XL + part * 16 + 8]) = u32x4{o[4], o[5], o[6], o[7]};
            } else if constexpr (WF == WF_Q8) {
                // 16 int8 = elements 16*part .. 16*part+15, exact in bf16
                unsigned o[8];
#pragma unroll
                for (int p = 0; p < 8; p++) {
                    const unsigned word = w[p >> 1];
                    const int sh = (p & 1) * 16;
                    o[p] = pack_int<LIMB>((float)(signed char)((word >> sh) & 0xFF),
                                          (float)(signed char)((word >> (sh + 8)) & 0xFF));
                }
                *reinterpret_cast<u32x4 *>(&Bl[col * XL + part * 16]) = u32x4{o[0], o[1], o[2], o[3]};
                *reinterpret_cast<u32x4 *>(&Bl[col * XL + part * 16 + 8]) = u32x4{o[4], o[5], o[6], o[7]};
            } else if constexpr (LIMB == LIMB_F16X2) {
                // 8 bytes = elements 8*part+e (low nibble) and 16+8*part+e (high nibble);
                // nibble n under the f16 exponent of 1024 reads as 1024 + n, minus 1032 = n - 8
                unsigned lo[4], hi[4];
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    const unsigned nl = w[p] & 0x0F0F0F0Fu, nh = (w[p] >> 4) & 0x0F0F0F0Fu;
                    lo[2 * p] = sub1032(__builtin_amdgcn_perm(0x64646464u, nl, 0x04010400u));
                    lo[2 * p + 1] = sub1032(__builtin_amdgcn_perm(0x64646464u, nl, 0x04030402u));
                    hi[2 * p] = sub1032(__builtin_amdgcn_perm(0x64646464u, nh, 0x04010400u));
                    hi[2 * p + 1] = sub1032(__builtin_amdgcn_perm(0x64646464u, nh, 0x04030402u));
                }
                *reinterpret_cast<u32x4 *>(&Bl[col * XL + part * 8]) = u32x4{lo[0], lo[1], lo[2], lo[3]};
                *reinterpret_cast<u32x4 *>(&Bl[col * XL + 16 + part * 8]) = u32x4{hi[0], hi[1], hi[2], hi[3]};
            } else {
                // 8 bytes = elements 8*part+e (low nibble) and 16+8*part+e (high nibble)
                unsigned lo[4], hi[4];
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const unsigned word = w[p >> 1];
                    const int sh = (p & 1) * 16;
                    const unsigned b0 = (word >> sh) & 0xFF, b1 = (word >> (sh + 8)) & 0xFF;
                    lo[p] = pack_int<LIMB>((float)((int)(b0 & 0xF) - 8), (float)((int)(b1 & 0xF) - 8));
                    hi[p] = pack_int<LIMB>((float)((int)(b0 >> 4) - 8), (float)((int)(b1 >> 4) - 8));
                }
                *reinterpret_cast<u32x4 *>(&Bl[col * XL + part * 8]) = u32x4{lo[0], lo[1], lo[2], lo[3]};
                *reinterpret_cast<u32x4 *>(&Bl[col * XL + 16 + part * 8]) = u32x4{hi[0], hi[1], hi[2], hi[3]};
            }
        }
        if (tid < BN) Ss[tid] = sc;
    };

    f32x16 acc[MT][NT];
#pragma unroll
    for (int r = 0; r < MT; r++)
#pragma unroll
        for (int c = 0; c < NT; c++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[r][c][q] = 0.0f;

    auto compute = [&](int stg) __attribute__((always_inline)) {
        const unsigned short *Al = Al2[stg], *Bl = Bl2[stg];
        const float *Ss = Ss2[stg];
        // A operands of this wave's rows for both k-halves and all limbs.  Lane
        // (li, hh) of k-half kh holds k = 16 hh + 8 kh + e of the block (B the
        // same k): the LDS-staged kernel then reads a column's 16 quant bytes of
        // both halves in one access.  Every f16-limb GEMM assigns k this way, so
        // each MFMA sums the same products and their results agree bit for bit.
        V8 a[2][NL][MT];
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int l = 0; l < NL; l++)
#pragma unroll
                for (int r = 0; r < MT; r++)
                    a[kh][l][r] = *reinterpret_cast<const V8 *>(
                        &Al[(wm * (BM / 2) + r * 32 + li) * AROW + l * 32 + hh * 16 + kh * 8]);
#pragma unroll
        for (int c = 0; c < NT; c++) {
            const int col = wn * (BN / 2) + c * 32 + li;
            f32x16 tmp[MT];
#pragma unroll
            for (int kh = 0; kh < 2; kh++) {
                const V8 b = *reinterpret_cast<const V8 *>(&Bl[col * XL + hh * 16 + kh * 8]);
#pragma unroll
                for (int l = 0; l < NL; l++)
#pragma unroll
                    for (int r = 0; r < MT; r++) {
                        f32x16 c;
                        if (kh == 0 && l == 0) {
#pragma unroll
                            for (int q = 0; q < 16; q++) c[q] = 0.0f;
                        } else {
                            c = tmp[r];
                        }
                        if constexpr (LIMB == LIMB_F16X2)
                            tmp[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[kh][l][r], b, c, 0, 0, 0);
                        else
                            tmp[r] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[kh][l][r], b, c, 0, 0, 0);
                    }
            }
            const float d = Ss[col];
#pragma unroll
            for (int r = 0; r < MT; r++)
#pragma unroll
                for (int q = 0; q < 16; q++) acc[r][c][q] += d * tmp[r][q];
        }
    };

    // k-blocks [kb0, kend) of this split (all of K without split-K)
    const int kb0 = SPLIT ? (int)blockIdx.y * kps : 0, kend = SPLIT ? min(KBW, kb0 + kps) : KBW;
    // Prefetches past the last block re-read the last block (unused), so every
    // path issues the same loads and the waits count only the older stage.
    gload(kb0, ra[0], rb[0], rs[0]);
    gload(min(kb0 + 1, kend - 1), ra[1], rb[1], rs[1]);
    for (int kb = kb0; kb < kend; kb += 2) {
        // Stage 0 was last read by compute(kb - 2); every wave finished that before the
        // previous iteration's barrier, so one barrier per block suffices.
        sstore(0, ra[0], rb[0], rs[0]);
        __syncthreads();
        gload(min(kb + 2, kend - 1), ra[0], rb[0], rs[0]);
        compute(0);
        if (kb + 1 >= kend) break;
        sstore(1, ra[1], rb[1], rs[1]);
        __syncthreads();
        gload(min(kb + 3, kend - 1), ra[1], rb[1], rs[1]);
        compute(1);
    }

    if (SPLIT && part) {  // split-K: raw partial sums, bias and epilogue in k_splitk_reduce
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

    // Epilogue: every output value is formed before the first store (bias and
    // residual reads share one wait, and no store follows a pending load,
    // which would make the compiler wait for each earlier store at every
    // bounds branch); tiles inside the matrix store without bounds branches.
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
                    res[c][r][q] = reinterpret_cast<const float *>(Yv)[(size_t)row * ldy + col];
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
                if constexpr (EPI == EPI_GELU_X3 || EPI == EPI_GELU_H2 || EPI == EPI_GELU) v = gelu_as(v);
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
                    if constexpr (EPI == EPI_GELU_X3)
                        x3_store(reinterpret_cast<unsigned short *>(Yv), row, col, N, acc[r][c][q]);
                    else if constexpr (EPI == EPI_GELU_H2)
                        h2_store(reinterpret_cast<unsigned short *>(Yv), row, col, N, acc[r][c][q]);
                    else
                        reinterpret_cast<float *>(Yv)[(size_t)row * ldy + col] = acc[r][c][q];
                }
        }
    };
    if (m0 + BM <= M && n0 + BN <= N)
        store(false);
    else
        store(true);
}

// Y = epi(sum over splits of part[s] + bias), splits in order
__global__ __launch_bounds__(256) void k_splitk_reduce(const float *__restrict__ part, int S, int M, int N,
                                                       const float *__restrict__ bias, void *__restrict__ Yv, int ldy,
                                                       int epi) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= M * N) return;
    const int row = i / N, col = i - row * N;
    const size_t MN = (size_t)M * N;
    float v = part[i];
    for (int s = 1; s < S; s++) v += part[s * MN + i];
    v += bias ? bias[col] : 0.0f;
    if (epi == EPI_GELU_X3) {
        x3_store(reinterpret_cast<unsigned short *>(Yv), row, col, N, gelu_as(v));
    } else if (epi == EPI_GELU_H2) {
        h2_store(reinterpret_cast<unsigned short *>(Yv), row, col, N, gelu_as(v));
    } else {
        float *dst = reinterpret_cast<float *>(Yv) + (size_t)row * ldy + col;
        if (epi == EPI_GELU) v = gelu_as(v);
        if (epi == EPI_RESIDUAL) v += *dst;
        *dst = v;
    }
}

hipError_t launch_splitk_reduce(const float *part, int S, int M, int N, const float *bias, void *Y, int ldy, int epi,
                                hipStream_t st) {
    hipLaunchKernelGGL(k_splitk_reduce, dim3((M * N + 255) / 256), dim3(256), 0, st, part, S, M, N, bias, Y, ldy, epi);
    return hipGetLastError();
}

template <int WF, int EPI, int BM, int BN, int AF, int LIMB>
static hipError_t launch_x3_t(const DevMatrix &W, const void *X, int ldx, const float *bias, void *Y, int ldy, int M,
                              const PartialBuf *pb, hipStream_t st, int *defer) {
    const int nM = (M + BM - 1) / BM, nN = (W.N + BN - 1) / BN, KB = W.K / 32 * (WF == WF_F16P ? 2 : 1);
    // Split K when the tiles alone leave the GPU mostly idle: up to ~1024
    // workgroups, at least 4 k-blocks per split, partials within pb.  Only
    // the 64x64 tile (the one chosen for small problems) is built with it.
    constexpr bool SPLIT = BM == 64 && BN == 64;
    int S = 1, kps = KB;
    const char *e = getenv("CIH_SPLITK");
    const long wgs = (long)nM * nN;
    if (SPLIT && pb && pb->part && !(e && !strcmp(e, "0")) && wgs < 512 && KB >= 8) {
        S = (int)std::min<long>(1024 / wgs, KB / 4);
        while (S > 1 && (size_t)S * M * W.N > pb->floats) S--;
        if (S > 1) {
            kps = (KB + S - 1) / S;
            S = (KB + kps - 1) / kps;
        }
    }
    float *part = S > 1 ? pb->part : nullptr;
    hipLaunchKernelGGL((k_gemm_x3<WF, EPI, BM, BN, AF, LIMB, SPLIT>), dim3(nM * nN, S), dim3(256), 0, st, X, ldx, W.q, W.sc,
                       bias, Y, ldy, M, W.N, W.K, kps, part);
    if (defer) *defer = S > 1 ? S : 0;  // the caller adds the splits (and bias, epilogue) itself
    else if (S > 1)
        hipLaunchKernelGGL(k_splitk_reduce, dim3((M * W.N + 255) / 256), dim3(256), 0, st, part, S, M, W.N, bias, Y,
                           ldy, EPI);
    return hipGetLastError();
}

// Tile shape: the largest of 128x128, 128x64, 64x128, 64x64 that still gives
// at least 1024 workgroups (two rounds of two per CU), else 64x64.
// CIH_GEMM_TILE=<BM>x<BN> forces one.
static void pick_tile(int M, int N, int &bm, int &bn) {
    const char *e = getenv("CIH_GEMM_TILE");
    if (e && sscanf(e, "%dx%d", &bm, &bn) == 2 && (bm == 64 || bm == 128) && (bn == 64 || bn == 128)) return;
    auto wgs = [&](int tm, int tn) { return (long)((M + tm - 1) / tm) * ((N + tn - 1) / tn); };
    const long target = 1024;
    if (M > 64 && N > 64 && wgs(128, 128) >= target) bm = 128, bn = 128;
    else if (M > 64 && wgs(128, 64) >= target) bm = 128, bn = 64;
    else if (N > 64 && wgs(64, 128) >= target) bm = 64, bn = 128;
    else bm = 64, bn = 64;
}

template <int WF, int EPI, int AF, int LIMB>
static hipError_t launch_x3_shape(const DevMatrix &W, const void *X, int ldx, const float *bias, void *Y, int ldy,
                                  int M, const PartialBuf *pb, hipStream_t st, int *defer) {
    int bm, bn;
    pick_tile(M, W.N, bm, bn);
    if (defer) *defer = 0;
    if (bm == 128 && bn == 128) return launch_x3_t<WF, EPI, 128, 128, AF, LIMB>(W, X, ldx, bias, Y, ldy, M, pb, st, defer);
    if (bm == 128) return launch_x3_t<WF, EPI, 128, 64, AF, LIMB>(W, X, ldx, bias, Y, ldy, M, pb, st, defer);
    if (bn == 128) return launch_x3_t<WF, EPI, 64, 128, AF, LIMB>(W, X, ldx, bias, Y, ldy, M, pb, st, defer);
    return launch_x3_t<WF, EPI, 64, 64, AF, LIMB>(W, X, ldx, bias, Y, ldy, M, pb, st, defer);
}

template <int WF, int AF, int LIMB>
static hipError_t launch_x3_epi(const DevMatrix &W, const void *X, int ldx, const float *bias, void *Y, int ldy,
                                int M, int epi, const PartialBuf *pb, hipStream_t st, int *defer) {
    switch (epi) {
    case EPI_GELU: return launch_x3_shape<WF, EPI_GELU, AF, LIMB>(W, X, ldx, bias, Y, ldy, M, pb, st, defer);
    case EPI_GELU_X3: return launch_x3_shape<WF, EPI_GELU_X3, AF, LIMB>(W, X, ldx, bias, Y, ldy, M, pb, st, defer);
    case EPI_GELU_H2:
        if constexpr (LIMB == LIMB_F16X2) return launch_x3_shape<WF, EPI_GELU_H2, AF, LIMB>(W, X, ldx, bias, Y, ldy, M, pb, st, defer);
        return hipErrorInvalidValue;
    case EPI_RESIDUAL: return launch_x3_shape<WF, EPI_RESIDUAL, AF, LIMB>(W, X, ldx, bias, Y, ldy, M, pb, st, defer);
    default: return launch_x3_shape<WF, EPI_NONE, AF, LIMB>(W, X, ldx, bias, Y, ldy, M, pb, st, defer);
    }
}

// Pair copy of an FP32 k-block-major matrix, one thread per (k-block, column):
// d = 2^(e - 14) for the block's largest magnitude m in [2^e, 2^(e+1)), so
// w / d (exact) is below 2^15; hi = f16(w / d), lo = f16(w / d - hi).
__global__ __launch_bounds__(256) void k_pair_f16(const float *__restrict__ w, int N, int KB,
                                                  unsigned short *__restrict__ p16, float *__restrict__ psc) {
    const size_t blk = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= (size_t)KB * N) return;
    const float4 *src = reinterpret_cast<const float4 *>(w + blk * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) *reinterpret_cast<float4 *>(&v[4 * i]) = src[i];
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) mx = fmaxf(mx, fabsf(v[i]));
    const int e = mx > 0.0f && __builtin_isfinite(mx) ? max(ilogbf(mx) - 14, -126) : 0;
    unsigned hi[16], lo[16];
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        const float x0 = ldexpf(v[i], -e), x1 = ldexpf(v[i + 1], -e);
        const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
        const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
        hi[i / 2] = __builtin_bit_cast(unsigned short, h0) | (unsigned)__builtin_bit_cast(unsigned short, h1) << 16;
        lo[i / 2] = __builtin_bit_cast(unsigned short, l0) | (unsigned)__builtin_bit_cast(unsigned short, l1) << 16;
    }
    u32x4 *dh = reinterpret_cast<u32x4 *>(p16 + blk * 32);
    u32x4 *dl = reinterpret_cast<u32x4 *>(p16 + ((size_t)KB * N + blk) * 32);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        dh[i] = u32x4{hi[4 * i], hi[4 * i + 1], hi[4 * i + 2], hi[4 * i + 3]};
        dl[i] = u32x4{lo[4 * i], lo[4 * i + 1], lo[4 * i + 2], lo[4 * i + 3]};
    }
    const float d = ldexpf(1.0f, e);
    psc[blk] = d;
    psc[(size_t)KB * N + blk] = d;
}

hipError_t launch_pair_f16(const DevMatrix &W, unsigned short *p16, float *psc, hipStream_t st) {
    if (W.fmt != WF_F32 || W.K % 32 || !W.q || !p16 || !psc) return hipErrorInvalidValue;
    const size_t blocks = (size_t)(W.K / 32) * W.N;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_pair_f16, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, st,
                       static_cast<const float *>(W.q), W.N, W.K / 32, p16, psc);
    return hipGetLastError();
}

hipError_t launch_gemm_x3(const DevMatrix &W, const void *X, int ldx, int a_fmt, const float *bias, void *Y, int ldy,
                          int M, int epi, const PartialBuf *pb, hipStream_t st, int *defer) {
    if (defer) *defer = 0;
    if (M <= 0) return hipSuccess;
    if (W.K % 32 != 0 || (a_fmt == AF_F32 && ldx % 4 != 0)) return hipErrorInvalidValue;
    if ((epi == EPI_GELU_X3 || epi == EPI_GELU_H2) && W.N % 32 != 0) return hipErrorInvalidValue;
    // f16 limbs with the f16 copy of the quants, 64 rows and more: the LDS
    // kernel's tile (and split) for the shape.  An FP32 matrix's pair copy
    // (W.q: [2K/32][N][32] f16) goes the same way as an f16 matrix of 2K
    // whose block kb meets activation block kb mod K/32.
    DevMatrix pv;
    const DevMatrix *lw = &W;
    if (W.fmt == WF_F16P && a_fmt == AF_H2) {
        pv = W;
        pv.K = 2 * W.K;
        pv.kx = W.K;
        pv.q16 = static_cast<const unsigned short *>(W.q);
        lw = &pv;
    }
    if (LdsPlan p; gemm_lds_plan(*lw, a_fmt, M, epi, defer && pb && pb->part ? pb->floats : 0, p)) {
        const hipError_t e = launch_gemm_lds_plan(*lw, X, bias, Y, ldy, M, epi, p, pb, st);
        if (e == hipSuccess && defer && p.splits > 1) *defer = p.splits;
        return e;
    }
    if (gemm_lds_applies(W, a_fmt, M, epi)) return launch_gemm_lds(W, X, bias, Y, ldy, M, epi, st);
    // a caller that adds the splits itself: the LDS kernel split over K
    if (defer && pb && gemm_lds_split_applies(W, a_fmt, M, epi)) {
        int S = 0;
        const hipError_t e = launch_gemm_lds_split(W, X, M, *pb, &S, st);
        if (e != hipSuccess || S > 1) {
            *defer = S;
            return e;
        }
    }
    // FP32 activations: f16 two-limb split unless CIH_LIMBS=bf16x3
    const char *lv = getenv("CIH_LIMBS");
    const bool bf16 = (lv && !strcmp(lv, "bf16x3")) || full_range_mode();
    if (W.fmt == WF_F16P) {
        if (a_fmt == AF_H2) return launch_x3_epi<WF_F16P, AF_H2, LIMB_F16X2>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
        if (a_fmt == AF_F32 && !bf16)
            return launch_x3_epi<WF_F16P, AF_F32, LIMB_F16X2>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
        return hipErrorInvalidValue;
    }
    if (a_fmt == AF_H2) {
        if (W.fmt == WF_Q8) return launch_x3_epi<WF_Q8, AF_H2, LIMB_F16X2>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
        if (W.fmt == WF_Q4) return launch_x3_epi<WF_Q4, AF_H2, LIMB_F16X2>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
    } else if (a_fmt == AF_X3) {
        if (W.fmt == WF_Q8) return launch_x3_epi<WF_Q8, AF_X3, LIMB_BF16X3>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
        if (W.fmt == WF_Q4) return launch_x3_epi<WF_Q4, AF_X3, LIMB_BF16X3>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
    } else if (bf16) {
        if (W.fmt == WF_Q8) return launch_x3_epi<WF_Q8, AF_F32, LIMB_BF16X3>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
        if (W.fmt == WF_Q4) return launch_x3_epi<WF_Q4, AF_F32, LIMB_BF16X3>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
    } else {
        if (W.fmt == WF_Q8) return launch_x3_epi<WF_Q8, AF_F32, LIMB_F16X2>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
        if (W.fmt == WF_Q4) return launch_x3_epi<WF_Q4, AF_F32, LIMB_F16X2>(W, X, ldx, bias, Y, ldy, M, epi, pb, st, defer);
    }
    return hipErrorInvalidValue;
}

}  // namespace cih
