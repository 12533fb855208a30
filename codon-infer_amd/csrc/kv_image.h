// K/V tile images: the layout in which the QKV projection hands keys and
// values to attention.
//
// A sequence's keys are cut into 32-key tiles (the last one zero padded).
// Tile rows of all sequences are numbered back to back (sequence b owns rows
// tb[b] .. tb[b] + ceil(len_b / 32) - 1) and a token's padded key index is
// pk = 32 * tb[b] + position.  For each (tile row, head) there is one image of
// TB bytes, image index tile_row * H + h, holding f16 limbs (hi = f16(x),
// lo = f16(x - hi)):
//
//   K  32 key rows of KRP = 4 HDP bytes: per group of GS = min(32, HDP)
//      dims, [limb][GS dims] (rotated by RoPE; dims HD..HDP zero);
//   V  VW dim rows of 128 bytes: [limb][32 key positions] (V transposed;
//      dims past HD zero).
//
// The image is exactly the LDS image attention multiplies from, so staging a
// tile is a flat copy (global_load_lds).  Rows keep one head's 32 dims (K) or
// 32 keys (V) of both limbs in one 128-byte line, so that the projection's
// epilogue writes whole lines.  The 16-byte chunks of a row are XOR-swizzled
// for gfx950's LDS (64 banks of 4 bytes, a ds_read_b128 served 16 lanes at a
// time): the 16 lanes of an MFMA operand read (16 consecutive rows, one
// logical chunk) hit 16 distinct bank groups, and so do 8 consecutive rows on
// a 32-bank LDS.  Within a V row, key k sits at position k with bits 2 and 3
// swapped: the keys lane half hh feeds the P.V MFMA for 16-key chunk c are
// 16c + 4hh + {0..3} and 16c + 8 + 4hh + {0..3}, which this order makes the
// eight consecutive positions 16c + 8hh + {0..7}; the same holds for the rows
// a GEMM lane holds in its accumulator, so a lane's 16 values of a V column
// are whole 8-position chunks.
#pragma once
#include <hip/hip_runtime.h>

namespace cih {

// RoPE of a dim pair (apply_rope, lib.rs:3533-3552) with one fixed rounding
// sequence, used by every kernel that rotates K or Q for the f16-limb
// attention (staged or from images), so that all of them give the same bits:
//   lower dim j:       fma(x_j, cos, -(x_{j+hd/2} sin))
//   upper dim j+hd/2:  fma(x_{j+hd/2}, cos, x_j sin)
// The result passes an empty asm so that the compiler cannot fuse the FMA with
// a following f16 conversion (v_fma_mix rounds once, from the exact value, and
// so can round a tie differently from f16(f32 result)).
__device__ __forceinline__ float opaque(float r) {
    asm("" : "+v"(r));
    return r;
}
__device__ __forceinline__ float rot_lo(float x, float xp, float c, float s) { return opaque(__builtin_fmaf(x, c, -(xp * s))); }
__device__ __forceinline__ float rot_hi(float x, float xp, float c, float s) { return opaque(__builtin_fmaf(x, c, xp * s)); }

// hi = f16(v), lo = f16(v - hi) for a pair of floats, packed two f16 to a
// register: one v_cvt_pk_f16_f32 and two v_fma_mix (lo = f16(fma(hi, -1, v));
// v - hi is exact in FP32, so this is the same single rounding as f16(v - hi),
// subnormal limbs included).  The limbs travel as packed 32-bit values: the
// mix instructions write register halves the compiler cannot see as vector
// elements.
__device__ __forceinline__ unsigned split_pair(float v0, float v1, unsigned &lo) {
    _Float16 __attribute__((ext_vector_type(2))) h;
    h[0] = (_Float16)v0;
    h[1] = (_Float16)v1;
    const unsigned hb = __builtin_bit_cast(unsigned, h);
    asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, -1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=&v"(lo)
        : "v"(hb), "v"(v0), "v"(v1));
    return hb;
}
template <int HD> struct KvImg {
    static constexpr int HALF = HD / 2;
    static constexpr int HDP = (HD + 15) / 16 * 16;  // K dims padded to whole 16-wide MFMA k-chunks
    static constexpr int VW = HD < 32 ? 32 : HD;     // V^T rows: whole 32-row MFMA tiles
    static constexpr int GS = HDP < 32 ? HDP : 32;   // dims per K group
    static constexpr int KRP = 4 * HDP;              // bytes per K row (both limbs)
    static constexpr int KC = KRP / 16;              // 16-byte chunks per K row
    static constexpr int VOFF = 32 * KRP;            // V rows start here
    static constexpr int TB = VOFF + 128 * VW;       // bytes of one image
    static_assert(TB % 1024 == 0, "an image is whole 1 KiB load instructions");

    // logical chunk of (dim, limb) in a K row
    __host__ __device__ static constexpr int klc(int dim, int limb) {
        return (dim / GS) * (2 * GS / 8) + limb * (GS / 8) + (dim % GS) / 8;
    }
    // physical chunk of logical chunk c in K row (key) r
    __host__ __device__ static constexpr int kchunk(int r, int c) {
        return KC == 16 ? c ^ (r & 15) : (KC == 8 ? c ^ ((r ^ (r >> 1)) & 7) : c ^ ((r ^ (r >> 2)) & 3));
    }
    // physical chunk of logical chunk c (limb * 4 + position / 8) in V row (dim) r
    __host__ __device__ static constexpr int vchunk(int r, int c) { return c ^ ((r ^ (r >> 1)) & 7); }
    // position of key k in a V row
    __host__ __device__ static constexpr int vpos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }
    // byte offsets of element (key, dim) of a limb
    __host__ __device__ static constexpr int koff(int key, int dim, int limb) {
        return key * KRP + kchunk(key, klc(dim, limb)) * 16 + (dim & 7) * 2;
    }
    __host__ __device__ static constexpr int voff(int key, int dim, int limb) {
        return VOFF + dim * 128 + vchunk(dim, limb * 4 + vpos(key) / 8) * 16 + (vpos(key) & 7) * 2;
    }
};

}  // namespace cih
