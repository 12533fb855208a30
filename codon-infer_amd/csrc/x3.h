// Limb activation formats shared by the producers (LayerNorm, attention
// output, FC1's GELU epilogue) and the quantized GEMM, which then stages
// activations into LDS without converting them.
//
// "H2": two f16 limbs, 4 bytes/element (the size of FP32).  A row of K values
// is K/32 chunks of 64 f16:
//   chunk kb = [hi[32] | lo[32]]  for elements kb*32 .. kb*32+31
// with hi = f16(x), lo = f16(x - hi) (round to nearest even).
//
// "X3": three bf16 limbs, 6 bytes/element:
// A row of K FP32 values is stored as K/32 chunks of 96 bf16:
//   chunk kb = [limb0[32] | limb1[32] | limb2[32]]  for elements kb*32 .. kb*32+31
// with x = limb0 + limb1 + limb2, limb0 = bf16(x), limb1 = bf16(x - limb0),
// limb2 = bf16(x - limb0 - limb1) (round to nearest even): 24 significant
// bits, so the split reproduces x to below FP32 rounding.  6 bytes/element.
#pragma once
#include <hip/hip_runtime.h>

namespace cih {

enum AFmt { AF_F32 = 0, AF_X3 = 1, AF_H2 = 2 };

// The limbs split the FP32 value x as stored.  Without this (empty) operand
// barrier the backend may fold the multiply that produced x into the first
// limb's conversion (v_fma_mixlo_f16 rounds the exact product straight to
// f16) or into the residual subtraction, depending on the code around the
// call, and two kernels computing the same x would hand off different limbs.
__device__ __forceinline__ void limb_source(float &x) { asm("" : "+v"(x)); }

__device__ __forceinline__ unsigned short bf16_bits(float x) {
    return __builtin_bit_cast(unsigned short, (__bf16)x);
}
__device__ __forceinline__ float bf16_val(unsigned short b) { return __uint_as_float((unsigned)b << 16); }

// element index of (row, col) limb l in an X3 matrix with K columns
__device__ __forceinline__ size_t x3_index(size_t row, int col, int K, int l) {
    return (row * (size_t)(K / 32) + (col >> 5)) * 96 + l * 32 + (col & 31);
}

__device__ __forceinline__ void x3_store(unsigned short *base, size_t row, int col, int K, float x) {
    limb_source(x);
    const unsigned short a = bf16_bits(x);
    const float r1 = x - bf16_val(a);
    const unsigned short b = bf16_bits(r1);
    const unsigned short c = bf16_bits(r1 - bf16_val(b));
    const size_t i = x3_index(row, col, K, 0);
    base[i] = a;
    base[i + 32] = b;
    base[i + 64] = c;
}

// four consecutive columns col..col+3 (col % 4 == 0) as 8-byte stores per limb
__device__ __forceinline__ void x3_store4(unsigned short *base, size_t row, int col, int K, float4 x) {
    float v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; e++) limb_source(v[e]);
    unsigned short l[3][4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        l[0][e] = bf16_bits(v[e]);
        const float r1 = v[e] - bf16_val(l[0][e]);
        l[1][e] = bf16_bits(r1);
        l[2][e] = bf16_bits(r1 - bf16_val(l[1][e]));
    }
    const size_t i = x3_index(row, col, K, 0);
#pragma unroll
    for (int k = 0; k < 3; k++)
        *reinterpret_cast<uint2 *>(base + i + 32 * k) =
            make_uint2((unsigned)l[k][0] | ((unsigned)l[k][1] << 16), (unsigned)l[k][2] | ((unsigned)l[k][3] << 16));
}

__device__ __forceinline__ unsigned short f16_bits(float x) { return __builtin_bit_cast(unsigned short, (_Float16)x); }
__device__ __forceinline__ float f16_val(unsigned short h) { return (float)__builtin_bit_cast(_Float16, h); }

// element index of (row, col) limb l in an H2 matrix with K columns
__device__ __forceinline__ size_t h2_index(size_t row, int col, int K, int l) {
    return (row * (size_t)(K / 32) + (col >> 5)) * 64 + l * 32 + (col & 31);
}

__device__ __forceinline__ void h2_store(unsigned short *base, size_t row, int col, int K, float x) {
    limb_source(x);
    const unsigned short a = f16_bits(x);
    const size_t i = h2_index(row, col, K, 0);
    base[i] = a;
    base[i + 32] = f16_bits(x - f16_val(a));
}

// four consecutive columns col..col+3 (col % 4 == 0) as 8-byte stores per limb
__device__ __forceinline__ void h2_store4(unsigned short *base, size_t row, int col, int K, float4 x) {
    float v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; e++) limb_source(v[e]);
    unsigned short l[2][4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        l[0][e] = f16_bits(v[e]);
        l[1][e] = f16_bits(v[e] - f16_val(l[0][e]));
    }
    const size_t i = h2_index(row, col, K, 0);
#pragma unroll
    for (int k = 0; k < 2; k++)
        *reinterpret_cast<uint2 *>(base + i + 32 * k) =
            make_uint2((unsigned)l[k][0] | ((unsigned)l[k][1] << 16), (unsigned)l[k][2] | ((unsigned)l[k][3] << 16));
}

// Quants as f16 MFMA operands.  A byte b under the f16 exponent of 1024 (bits
// 0x64bb) reads as 1024 + b; one packed f16 subtraction takes the offset off
// two values at once (exact: every value involved is an integer below 2048).
typedef _Float16 qh16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 qh16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned qu32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned qu32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned sub_pair(unsigned p, _Float16 c) {
    return __builtin_bit_cast(unsigned, __builtin_bit_cast(qh16x2_t, p) - qh16x2_t{c, c});
}

// 8 quants of one column as 8 f16 integers: Q8_0 (WF 1) 8 signed bytes, Q4_0
// (WF 2) the low (shift 0) or high (shift 4) nibbles of 8 bytes, minus 8.
template <int WF>
__device__ __forceinline__ qh16x8_t quants_f16(qu32x2_t w, int shift) {
    qu32x4_t o;
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const unsigned u = WF == 1 ? w[p] ^ 0x80808080u : (w[p] >> shift) & 0x0F0F0F0Fu;  // q + 128 / nibble
        const _Float16 off = WF == 1 ? (_Float16)1152.0f : (_Float16)1032.0f;
        o[2 * p] = sub_pair(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u), off);
        o[2 * p + 1] = sub_pair(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u), off);
    }
    return __builtin_bit_cast(qh16x8_t, o);
}

}  // namespace cih
