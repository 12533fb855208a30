// Quantized GEMM with operands staged global -> LDS by the load unit:
//   Y = epi(X * W^T + b),  X in f16 limbs (AF_H2), W in Q8_0 / Q4_0 blocks of 32.
//
// Arithmetic is that of k_gemm_x3 with LIMB_F16X2 (gemm_x3.hip), operation
// for operation: per 32-wide block, tmp = sum over both limbs and both
// k-halves of limb x quant on v_mfma_f32_32x32x16_f16 (exact products, FP32
// accumulation in the same order), then acc += d * tmp.  Results are
// bit-identical to that kernel; it replaces matmul_tiled_q8/q4_parallel
// (codon-infer src/lib.rs:4870, 4937) on the large bidirectional batches.
//
// What differs is the data movement:
//   * the quants come from W.q16, an f16 copy made when the model is loaded,
//     so no conversion runs in the loop and both operands are plain copies
//     (a model loaded without the copy: the quants themselves, 1 or 0.5 bytes
//     per weight, converted on the LDS -> register path);
//   * every k-block of A (BM rows x 128 B: 32 hi + 32 lo f16) and of W.q16
//     (BN columns x 64 B) plus its BN scales is fetched with
//     global_load_lds_dword{,x4}: the load unit writes LDS directly, nothing
//     passes through registers;
//   * three LDS stages: while block kb is multiplied, blocks kb+1 and kb+2
//     are in flight; one barrier per block;
//   * LDS layouts are swizzled for gfx950's LDS (64 banks of 4 bytes, a
//     ds_read_b128 served 16 lanes at a time): 16-byte chunk c of A row r sits
//     at chunk c ^ ((r >> 1) & 7), chunk c of W column n at c ^ ((n >> 2) & 3),
//     so the 16 lanes of each MFMA operand read hit 16 distinct bank groups.
//
// Workgroup tiles (BM x BN, waves x wave tile): 128 x 320 (8 x 32 x 160) and
// 128 x 256 (8 x 64 x 64), one workgroup per CU; 128 x 160 (4 x 32 x 160);
// 128 x 128 (4 x 64 x 64, two per CU); and, for problems too small to fill
// the device with those, 64 x 128 (4 x 32 x 64, three per CU) and 64 x 64
// (4 x 32 x 32, four per CU), read from the f16 copy only.  Every tile sums the same products in the same
// order, so the tile never changes a result.  The 64 x 64 tile can also run
// on 2 or 4 groups of its 4 waves (KW; 64 x 128: 2), which take alternate k-blocks
// through stages of their own and add their sums at the end: the k-sum
// regrouped, as a k-split regroups it.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "kernels.h"
#include "kv_image.h"
#include "x3.h"

namespace cih {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_ptr_t;
typedef __attribute__((address_space(1))) void glb_ptr_t;

// Workgroup tile: WM x WN waves, each owning RT x CT MFMA tiles of 32 x 32.
// A block of A (BM rows x 128 B) and of W.q16 (BN columns x 64 B) is LA and
// LB load instructions of 1 KiB; instruction j goes to wave j % NW.  When NW
// does not divide them, the waves with fewer real loads repeat their first
// one (same source, same LDS bytes), so every wave issues NI loads per block
// and the wait counts are the same in all waves.
template <int RT, int CT, int WM, int WN, int BPC = 64> struct LdsTile {
    static constexpr int BM = WM * RT * 32, BN = WN * CT * 32, NW = WM * WN, THREADS = 64 * NW;
    // BPC: bytes of W per column and block (64: the f16 copy; 32: Q8_0 quants; 16: Q4_0)
    static constexpr int SA = BM * 128, SB = (BN * BPC + 1023) / 1024 * 1024, SS = BN * 4, STAGE = SA + SB + SS;
    static constexpr int LA = SA / 1024, LB = SB / 1024;
    static constexpr int NA = (LA + NW - 1) / NW, NB = (LB + NW - 1) / NW;
    static constexpr int SL = BN / NW;      // scales per wave and block (4-byte loads)
    static constexpr int NI = NA + NB + 1;  // load instructions per wave and block
    static constexpr int OCC = THREADS >= 512 ? 1 : 512 / THREADS;  // workgroups per CU
    static constexpr int WPE = NW / 4 * OCC;  // waves per SIMD (HIP's second launch bound)
    // KW groups of NW waves on one tile, each group with its own three
    // stages: waves per SIMD when as many such workgroups as fit the LDS share a CU
    static constexpr int wpe(int kw) { return kw == 1 ? WPE : NW * kw / 4 * (160 * 1024 / (kw * 3 * STAGE + 1024)); }
    static_assert(SA % 1024 == 0 && LA >= NW, "loads");
    static_assert(BN % NW == 0 && SL <= 64 && OCC * 3 * STAGE <= 160 * 1024, "tile");
};

// f(integral_constant<int, I>) for each I of the sequence, in order
template <int... Is, class F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, Is...>, F &&f) {
    (f(std::integral_constant<int, Is>{}), ...);
}

// Epilogue of the QKV projection when attention reads K/V tile images
// (kv_image.h).  acc holds v = x.W^T + b; lane (li, hh) of wave (wm, wn) has
// column n0 + (wn CT + c) 32 + li and rows m0 + (wm RT + r) 32 + 8g + 4hh + e
// (register q = 4g + e).  Q columns ([0, d)) are stored as FP32 like
// EPI_NONE.  A K column (dim j of head h) is rotated with its partner dim
// j +- HD/2 by rot_lo / rot_hi (kv_image.h), as attention's prep kernel
// rotates, and split into f16 limbs (hi = f16(r), lo = f16(r - hi)); a V
// column is split.  The partner is the neighbouring column tile (hd 64;
// through LDS when the two tiles belong to different waves) or lane
// li ^ HD/2 (hd 32, 16).  Each 32 x 32 tile of limbs is rearranged in a
// wave-private LDS patch into the image's 128-byte lines (a key's 32 dims of
// both limbs, or a dim's 32 keys of both limbs) and stored a whole line per 8
// lanes.  V goes this way when the 32 rows are exactly one key tile, element
// by element otherwise (a sequence starting inside the 32 rows).
constexpr int QKV_PP = 144;  // bytes per patch row: 128 + 16 (spreads the rows over the banks)

// LDS bytes qkv_epilogue uses from the start of the kernel's LDS: the hd-64
// partner exchange (odd CT) and one patch of 32 rows per wave.  The rows'
// prefetched key indices and RoPE rows lie past both this and the stages.
template <int HD, int RT, int CT, int WM, int WN> constexpr int qkv_epilogue_lds() {
    return (HD == 64 && CT % 2 == 1 ? 2 * WM * RT * 16 * 64 * 4 : 0) + WM * WN * 32 * QKV_PP;
}

template <int HD, int RT, int CT, int WM, int WN, bool PREF>
__device__ __forceinline__ void qkv_epilogue(f32x16 (&acc)[RT][CT], unsigned char *lds, const unsigned char *pre,
                                             int m0, int n0, int wm, int wn, int lane, int M, int N,
                                             float *__restrict__ Y, int ldy, const QkvOut &qo) {
    using I = KvImg<HD>;
    constexpr int HALF = HD / 2, BM = WM * RT * 32;
    // per-row data: from the LDS copy (PREF: [BM] pk, [BM] pos, [2][BM][HALF] cos / sin) or from memory
    const int *s_pk = reinterpret_cast<const int *>(pre);
    const float *s_rope = reinterpret_cast<const float *>(pre + BM * 8);
    auto pk_of = [&](int row) __attribute__((always_inline)) { return PREF ? s_pk[row - m0] : qo.pk[row]; };
    static_assert(HD != 64 || CT % 2 == 0 || WN == 2, "hd-64 column pairs: within a wave or across two waves");
    const int li = lane & 31, hh = lane >> 5, d = qo.d;
    // hd 64 with an odd number of column tiles per wave: wave wn = 0 holds dims
    // 0..31 of the head its last tile starts, wave 1 dims 32..63 in its first
    float xpart[RT][16];
    if constexpr (HD == 64 && CT % 2 == 1) {
        float *xch = reinterpret_cast<float *>(lds);
        const int mine = wn == 0 ? CT - 1 : 0;
        const int col0 = n0 + (wn * CT + mine) * 32;
        const bool kcol = col0 >= d && col0 < 2 * d;
        __syncthreads();  // every wave is done with the operand stages
        if (kcol)
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int q = 0; q < 16; q++)
                    xch[(((wn * WM + wm) * RT + r) * 16 + q) * 64 + lane] = wn == 0 ? acc[r][CT - 1][q] : acc[r][0][q];
        __syncthreads();
        if (kcol)
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int q = 0; q < 16; q++) xpart[r][q] = xch[((((1 - wn) * WM + wm) * RT + r) * 16 + q) * 64 + lane];
    }
    const bool has_k = n0 + (wn * CT + CT) * 32 > d && n0 + wn * CT * 32 < 2 * d;  // this wave has K columns
    constexpr int PP = QKV_PP;
    if constexpr (!(HD == 64 && CT % 2 == 1)) __syncthreads();  // every wave is done with the operand stages
    unsigned char *patch = lds + (HD == 64 && CT % 2 == 1 ? 2 * WM * RT * 16 * 64 * 4 : 0) + (wm * WN + wn) * 32 * PP;
    // P = parity of wn CT: hd-64 partner tiles are compile-time indices (ct ^ 1)
    auto tiles = [&](auto P) __attribute__((always_inline)) {
        constexpr int PAR = decltype(P)::value;
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const int row0 = m0 + (wm * RT + r) * 32;
            // this lane's rows: padded key index and position
            int pk[16], pos[16];
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int row = row0 + 8 * (q >> 2) + 4 * hh + (q & 3);
                pk[q] = row < M ? pk_of(row) : -1;
                pos[q] = PREF || !(row < M && has_k) ? 0 : qo.pos[row];
            }
            // the 32 rows are one whole key tile (slots 0..31 in order)
            const bool tile_rows = row0 + 31 < M && (pk_of(row0) & 31) == 0 && pk_of(row0 + 31) == pk_of(row0) + 31;
            static_for(std::make_integer_sequence<int, CT>{}, [&](auto C) __attribute__((always_inline)) {
                constexpr int c = decltype(C)::value;
                const int ct = wn * CT + c;  // column tile within the workgroup
                const int col0 = n0 + ct * 32, col = col0 + li;
                if (col0 >= N) return;
                if (col0 < d) {  // Q: FP32 rows
#pragma unroll
                    for (int q = 0; q < 16; q++) {
                        const int row = row0 + 8 * (q >> 2) + 4 * hh + (q & 3);
                        if (row < M) Y[(size_t)row * ldy + col] = acc[r][c][q];
                    }
                    return;
                }
                const bool is_k = col0 < 2 * d;
                const int hc = col - (is_k ? d : 2 * d);
                const int h = hc / HD, j = hc % HD;
                float v[16];
#pragma unroll
                for (int q = 0; q < 16; q++) v[q] = acc[r][c][q];
                if (is_k) {
                    // fma(k_j, cos, -+(k_partner sin)): rot_lo below HD/2, rot_hi above, same rounding
                    const int jj = j < HALF ? j : j - HALF;
                    const float sgn = j < HALF ? -1.0f : 1.0f;
                    constexpr int pc = ((c + PAR) ^ 1) - PAR;  // partner tile in this wave, if in [0, CT)
#pragma unroll
                    for (int q = 0; q < 16; q++) {
                        float vp;
                        if constexpr (HD == 64) {
                            if constexpr (pc < 0 || pc >= CT) vp = xpart[r][q];
                            else vp = acc[r][pc][q];
                        } else {
                            vp = __shfl_xor(v[q], HALF);
                        }
                        float cs, sn;
                        if constexpr (PREF) {
                            const int rw = (wm * RT + r) * 32 + 8 * (q >> 2) + 4 * hh + (q & 3);
                            cs = s_rope[rw * HALF + jj];
                            sn = s_rope[(BM + rw) * HALF + jj];
                        } else {
                            const size_t t = (size_t)pos[q] * HALF + jj;
                            cs = qo.rc[t];
                            sn = qo.rs[t];
                        }
                        v[q] = opaque(__builtin_fmaf(v[q], cs, sgn * (vp * sn)));
                    }
                }
                // limbs, two rows to a register (registers q, q + 1)
                unsigned hi2[8], lo2[8];
#pragma unroll
                for (int i = 0; i < 8; i++) hi2[i] = split_pair(v[2 * i], v[2 * i + 1], lo2[i]);
                // Whole 128-byte image lines go out through the wave's patch (rows of
                // PP bytes: [limb][32] f16 and 16 bytes of padding), 8 lanes per line.
                unsigned char *pb = reinterpret_cast<unsigned char *>(patch);
                // A wave's LDS operations complete in order; the compiler only must not
                // move patch accesses across this point (a memory fence would also wait
                // for the global stores in flight).
                auto wave_sync = [&]() __attribute__((always_inline)) {
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                };
                if (is_k) {
                    // patch row = key row of the tile: [limb][32 tile dims]
#pragma unroll
                    for (int q = 0; q < 16; q++) {
                        const int rl = 8 * (q >> 2) + 4 * hh + (q & 3);
                        *reinterpret_cast<unsigned short *>(pb + rl * PP + li * 2) =
                            (unsigned short)(hi2[q >> 1] >> (16 * (q & 1)));
                        *reinterpret_cast<unsigned short *>(pb + rl * PP + 64 + li * 2) =
                            (unsigned short)(lo2[q >> 1] >> (16 * (q & 1)));
                    }
                    wave_sync();
#pragma unroll
                    for (int it = 0; it < 4; it++) {
                        const int rl = it * 8 + (lane >> 3), q = lane & 7, row = row0 + rl;
                        if (row >= M) continue;
                        const int p = pk_of(row), slot = p & 31;
                        unsigned char *base = qo.img + (size_t)(p >> 5) * qo.H * I::TB + slot * I::KRP;
                        int hdx, src, dst;  // head within the tile's first, patch chunk, line byte offset
                        if constexpr (HD == 64) {
                            // tile = group g of one head; physical chunk (g*8 + ls) ^ (slot & 15)
                            const int g = ((col0 - d) % 64) / 32, ls = q ^ (slot & 7);
                            hdx = 0;
                            src = (ls >> 2) * 64 + (ls & 3) * 16;
                            dst = ((g ^ ((slot >> 3) & 1)) * 8 + q) * 16;
                        } else if constexpr (HD == 32) {
                            const int ls = q ^ ((slot ^ (slot >> 1)) & 7);
                            hdx = 0;
                            src = (ls >> 2) * 64 + (ls & 3) * 16;
                            dst = q * 16;
                        } else {
                            // two heads of 16 dims: 4 chunks each, [limb][2 chunks]
                            hdx = q >> 2;
                            const int ls = (q & 3) ^ ((slot ^ (slot >> 2)) & 3);
                            src = (ls >> 1) * 64 + hdx * 32 + (ls & 1) * 16;
                            dst = (q & 3) * 16;
                        }
                        const int hk = (col0 - d) / HD + hdx;
                        *reinterpret_cast<uint4 *>(base + (size_t)hk * I::TB + dst) =
                            *reinterpret_cast<const uint4 *>(pb + rl * PP + src);
                    }
                    wave_sync();
                    return;
                }
                if (tile_rows) {
                    // patch row = dim of the tile: [limb][32 key positions]; a lane's keys
                    // 8g + 4hh + {0..3} are positions vpos(8g + 4hh) + {0..3}
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const int off = li * PP + I::vpos(8 * g + 4 * hh) * 2;
                        *reinterpret_cast<uint2 *>(pb + off) = make_uint2(hi2[2 * g], hi2[2 * g + 1]);
                        *reinterpret_cast<uint2 *>(pb + off + 64) = make_uint2(lo2[2 * g], lo2[2 * g + 1]);
                    }
                    wave_sync();
                    unsigned char *tb0 = qo.img + (size_t)(pk_of(row0) >> 5) * qo.H * I::TB + I::VOFF;
#pragma unroll
                    for (int it = 0; it < 4; it++) {
                        const int dl = it * 8 + (lane >> 3), q = lane & 7;
                        const int hc2 = col0 - 2 * d + dl, hv = hc2 / HD, jv = hc2 % HD;
                        const int ls = q ^ ((jv ^ (jv >> 1)) & 7);  // logical chunk: limb * 4 + position / 8
                        *reinterpret_cast<uint4 *>(tb0 + (size_t)hv * I::TB + jv * 128 + q * 16) =
                            *reinterpret_cast<const uint4 *>(pb + dl * PP + (ls >> 2) * 64 + (ls & 3) * 16);
                    }
                    wave_sync();
                    return;
                }
                // V rows of a tile that starts or ends a sequence: element by element
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    const int p = pk[q];
                    if (p < 0) continue;
                    unsigned char *t = qo.img + ((size_t)(p >> 5) * qo.H + h) * I::TB;
                    *reinterpret_cast<unsigned short *>(t + I::voff(p & 31, j, 0)) =
                        (unsigned short)(hi2[q >> 1] >> (16 * (q & 1)));
                    *reinterpret_cast<unsigned short *>(t + I::voff(p & 31, j, 1)) =
                        (unsigned short)(lo2[q >> 1] >> (16 * (q & 1)));
                }
            });
        }
    };
    if constexpr (HD == 64 && CT % 2 == 1) {
        if (wn & 1) tiles(std::integral_constant<int, 1>{});
        else tiles(std::integral_constant<int, 0>{});
    } else {
        tiles(std::integral_constant<int, 0>{});
    }
}

// a + b computed where it is written (inline asm): per-lane LDS offsets stay
// loop-invariant and the stage's base is added in the block, instead of an
// address per (stage, operand) being kept live across the k loop
__device__ __forceinline__ unsigned add_here(unsigned a, unsigned b) {
    unsigned r;
    asm volatile("v_add_u32 %0, %1, %2" : "=v"(r) : "s"(b), "v"(a));
    return r;
}

// WQ: 0 = W from the f16 copy (W.q16); WF_Q8 / WF_Q4 = W from its quants
// (W.q, a model loaded without the f16 copy), turned into f16 on the LDS ->
// register path: v_perm puts each byte (Q8_0: + 128; Q4_0: the lane's
// nibble) under the f16 exponent of 1024, a packed f16 subtraction removes
// the offset (1.25 VALU per weight).
//
// SPLIT: workgroup (tile, y) takes k-blocks [y kps, (y + 1) kps) and stores
// its raw sums (no bias, no epilogue) into part + y M N, row-major [M][N];
// the caller adds the splits in order (EPI_NONE only).
template <int EPI, int RT, int CT, int WM, int WN, int WQ, bool SPLIT = false, int SCH = 0, bool PERS = false,
          bool PX = false, int KW = 1>
__global__ __launch_bounds__((LdsTile<RT, CT, WM, WN>::THREADS * KW), (LdsTile<RT, CT, WM, WN>::wpe(KW))) void k_gemm_lds(
    const unsigned short *__restrict__ X, const unsigned char *__restrict__ WB, const float *__restrict__ Wsc,
    const float *__restrict__ bias, void *__restrict__ Yv, int ldy, int M, int N, int K, const QkvOut qo, int kps = 0,
    int kbx = 0) {
    static_assert(!SPLIT || EPI == EPI_NONE, "split partial sums carry no epilogue");
    constexpr int BPC = WQ == WF_Q8 ? 32 : (WQ == WF_Q4 ? 16 : 64);
    using T = LdsTile<RT, CT, WM, WN, BPC>;
    constexpr int BM = T::BM, BN = T::BN, NW = T::NW, SA = T::SA, SB = T::SB, STAGE = T::STAGE, NA = T::NA,
                  NB = T::NB, SL = T::SL;
    // QKV epilogue with one workgroup per CU: the rows' padded key indices,
    // positions and RoPE table rows are fetched into LDS behind the k loop
    constexpr bool QKV = EPI == EPI_QKV16 || EPI == EPI_QKV32 || EPI == EPI_QKV64;
    // KW > 1: KW groups of NW waves share the tile; group g takes k-blocks
    // kb0 + g, kb0 + g + KW, ... through three stages of its own, and the
    // groups' sums are added in group order at the end (through the stages)
    static_assert(KW == 1 || (RT == 1 && CT <= 2 && WQ == 0 && !PERS && !QKV), "k-groups: small tiles, f16 copy");
    static_assert((KW - 1) * NW * CT * 16 * 64 * 4 <= 3 * KW * STAGE, "group sums fit the stages");
    constexpr int NTH = T::THREADS * KW;
    constexpr int QHALF = EPI == EPI_QKV16 ? 8 : (EPI == EPI_QKV32 ? 16 : 32);
    constexpr bool PREF = QKV && T::OCC == 1;
    constexpr int XTRA = PREF ? BM * 8 + 2 * BM * QHALF * 4 : 0;
    constexpr int EL = QKV ? qkv_epilogue_lds<2 * QHALF, RT, CT, WM, WN>() : 0;
    constexpr int LOFF = 3 * KW * STAGE > EL ? 3 * KW * STAGE : EL;  // start of the prefetched rows
    // the tile's BN bias values, written 64 at a time (whole 256-byte rows)
    // (two buffers of it in the persistent form: the next tile's is fetched
    // while this tile's epilogue reads its own)
    constexpr int BOFF = LOFF + XTRA, BBYTES = (BN * 4 + 255) / 256 * 256, NBB = PERS ? 2 : 1;
    static_assert(!PERS || (!QKV && !SPLIT && WQ == 0), "persistent form: plain epilogues, f16 copy");
    static_assert(BOFF + NBB * BBYTES <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) unsigned char lds[BOFF + NBB * BBYTES];

    // the wave index is uniform: wave-derived offsets (LDS destinations) live in SGPRs
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // group grp and the wave lw within it (KW == 1: one group)
    const int grp = KW > 1 ? wave / NW : 0, lw = KW > 1 ? wave % NW : wave;
    const int wm = lw / WN, wn = lw % WN;
    const int goff = grp * 3 * STAGE;  // the group's stages
    const int li = lane & 31, hh = lane >> 5;
    const int nM = (M + BM - 1) / BM, nN = (N + BN - 1) / BN;
    int mt, nt;
    tile_xcd(blockIdx.x, nM * nN, nM, nN, mt, nt);
    int m0 = mt * BM, n0 = nt * BN;  // (the persistent form moves them to the next tile)
    const int KB = K / 32;
    // activation blocks of a row (PX: a pair copy, whose weight block kb
    // meets activation block kb mod kbx)
    const int KBX = PX ? kbx : KB;
    if (PX && (kbx <= 0 || 2 * kbx != KB)) return;  // (the host passes kbx = K / 64 with a pair copy)
    // k-blocks [kb0, kb1) of this workgroup
    const int kb0 = SPLIT ? (int)blockIdx.y * kps : 0, kb1 = SPLIT ? min(KB, kb0 + kps) : KB;
    if constexpr (SPLIT) {
        Yv = reinterpret_cast<float *>(Yv) + (size_t)blockIdx.y * M * N;
        ldy = N;
    }

    // Per-lane sources at k-block 0.  Load instruction j fills LDS bytes
    // [j * 1024, +1024) of its region, lane l the 16 bytes at l * 16: LDS
    // chunk p = 64 j + l holds the (row, chunk) whose swizzled position is p.
    // Rows past M and columns past N read the last row / column (never stored).
    // Sources as 32-bit byte offsets from wave-uniform bases (the tile's
    // first row of X, its first column of W and of the scales; the block
    // advances the bases in scalar registers): the loads take the scalar base
    // + 32-bit offset form, and no 64-bit address lives in vector registers.
    const unsigned char *xbase = reinterpret_cast<const unsigned char *>(X) + (size_t)m0 * KBX * 128;
    const unsigned char *wbase = WB + (size_t)n0 * BPC;
    const float *sbase = Wsc + n0;
    unsigned offA[NA];
    int dstA[NA];
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int j = i * NW + lw < T::LA ? i * NW + lw : lw;
        const int p = j * 64 + lane;
        const int row = p >> 3, chunk = (p & 7) ^ ((row >> 1) & 7);
        offA[i] = (unsigned)((min(m0 + row, M - 1) - m0) * KBX * 128 + chunk * 16);
        dstA[i] = j * 1024;
    }
    // W: chunk c of column n at c ^ ((n >> 2) & 3) (f16 copy, 4 chunks), at
    // c ^ ((n >> 3) & 1) (Q8_0, 2 chunks); Q4_0: one chunk.  Chunks past the
    // tile's columns (Q4_0 at 160 columns) fill padding nobody reads.
    unsigned offB[NB];
    int dstB[NB];
#pragma unroll
    for (int i = 0; i < NB; i++) {
        const int j = i * NW + lw < T::LB ? i * NW + lw : lw % T::LB;
        const int p = j * 64 + lane;
        int col, chunk;
        if constexpr (BPC == 64) {
            col = p >> 2;
            chunk = (p & 3) ^ ((col >> 2) & 3);
        } else if constexpr (BPC == 32) {
            col = p >> 1;
            chunk = (p & 1) ^ ((col >> 3) & 1);
        } else {
            col = min(p, BN - 1);
            chunk = 0;
        }
        offB[i] = (unsigned)((min(n0 + col, N - 1) - n0) * BPC + chunk * 16);
        dstB[i] = SA + j * 1024;
    }
    unsigned offS = (unsigned)(min(n0 + lw * SL + min(lane, SL - 1), N - 1) - n0) * 4;
    // the sources of tile t, as above (persistent form)
    auto set_tile = [&](int t) __attribute__((always_inline)) {
        int tm, tn;
        tile_xcd(t, nM * nN, nM, nN, tm, tn);
        m0 = tm * BM;
        n0 = tn * BN;
        xbase = reinterpret_cast<const unsigned char *>(X) + (size_t)m0 * KBX * 128;
        wbase = WB + (size_t)n0 * BPC;
        sbase = Wsc + n0;
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int j = i * NW + lw < T::LA ? i * NW + lw : lw;
            const int p = j * 64 + lane;
            const int row = p >> 3, chunk = (p & 7) ^ ((row >> 1) & 7);
            offA[i] = (unsigned)((min(m0 + row, M - 1) - m0) * KBX * 128 + chunk * 16);
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int j = i * NW + lw < T::LB ? i * NW + lw : lw % T::LB;
            const int p = j * 64 + lane;
            const int col = p >> 2, chunk = (p & 3) ^ ((col >> 2) & 3);
            offB[i] = (unsigned)((min(n0 + col, N - 1) - n0) * BPC + chunk * 16);
        }
        offS = (unsigned)(min(n0 + lw * SL + min(lane, SL - 1), N - 1) - n0) * 4;
    };
    // The tile's bias values go to LDS before the k loop (copied by the load
    // unit, ordered by the loop's first wait and barrier): the epilogue reads
    // them from LDS, so its stores follow no pending global load (a load
    // pending at a branch makes the compiler wait for every earlier store as
    // well) and no register holds them through the loop.
    float *s_bias = reinterpret_cast<float *>(lds + BOFF);
    auto load_bias = [&](int buf) __attribute__((always_inline)) {
        if (bias) {
            if (wave * 64 < BN)
                __builtin_amdgcn_global_load_lds((glb_ptr_t *)(bias + min(n0 + wave * 64 + lane, N - 1)),
                                                 (lds_ptr_t *)(lds + BOFF + buf * BBYTES + wave * 256), 4, 0, 0);
        } else if (buf == 0) {
            for (int i = tid; i < NBB * BBYTES / 4; i += NTH) s_bias[i] = 0.0f;
        }
    };
    load_bias(0);

    auto request = [&](int kb, int stg) __attribute__((always_inline)) {
        unsigned char *base = lds + goff + stg * STAGE;
        const unsigned char *xb = xbase + (size_t)(PX && kb >= KBX ? kb - KBX : kb) * 128, *wbk = wbase + (size_t)kb * N * BPC;
        const unsigned char *sbk = reinterpret_cast<const unsigned char *>(sbase + (size_t)kb * N);
#pragma unroll
        for (int i = 0; i < NA; i++)
            __builtin_amdgcn_global_load_lds((glb_ptr_t *)(xb + offA[i]), (lds_ptr_t *)(base + dstA[i]), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < NB; i++)
            __builtin_amdgcn_global_load_lds((glb_ptr_t *)(wbk + offB[i]), (lds_ptr_t *)(base + dstB[i]), 16, 0, 0);
        if (lane < SL)
            __builtin_amdgcn_global_load_lds((glb_ptr_t *)(sbk + offS), (lds_ptr_t *)(base + SA + SB + lw * SL * 4),
                                             4, 0, 0);
    };

    // Schedules with the same arithmetic (per 32 x 32 tile: tmp = both limbs
    // x both k-halves, then acc += d * tmp in block order):
    //  * RT >= 2: column tile after column tile, RT chains each; the last
    //    column tile's scaling is deferred under the next block's MFMAs (its
    //    FMAs would otherwise trail the block);
    //  * RT == 1: all CT chains interleaved (one chain per column tile would
    //    leave each MFMA waiting for its predecessor); a block's sums are
    //    scaled at the start of the next block, each column tile just before
    //    its chain restarts, so the FMAs run under the LDS reads and MFMAs
    //    of that block instead of trailing this one (same order of additions);
    //  * RT == 1, CT == 5 on the f16 copy (SCH 1): chains 0-2 as a triple,
    //    then chains 3-4 as a pair; the previous pair is scaled under the
    //    operand reads, the triple under the pair's MFMAs (below).
    f32x16 acc[RT][CT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[r][c][q] = 0.0f;
    constexpr int NT = RT >= 2 ? RT : CT;  // live chains
    f32x16 pend[RT >= 2 ? RT : 1];
    float dpend = 0.0f;
#pragma unroll
    for (int r = 0; r < (RT >= 2 ? RT : 1); r++)
#pragma unroll
        for (int q = 0; q < 16; q++) pend[r][q] = 0.0f;
    // RT == 1: the previous block's chains and scales (zero before the first)
    f32x16 tcar[RT >= 2 ? 1 : CT];
    float dcar[RT >= 2 ? 1 : CT];
#pragma unroll
    for (int c = 0; c < (RT >= 2 ? 1 : CT); c++) {
        dcar[c] = 0.0f;
#pragma unroll
        for (int q = 0; q < 16; q++) tcar[c][q] = 0.0f;
    }
    const int swA = (li >> 1) & 7, swB = (li >> 2) & 3;
    // B operands of column tile c, both k-halves
    auto read_b2 = [&](const unsigned char *base, int c, f16x8 (&b)[2]) __attribute__((always_inline)) {
        const int col = (wn * CT + c) * 32 + li;
        if constexpr (WQ == 0) {
#pragma unroll
            for (int kh = 0; kh < 2; kh++)
                b[kh] = *reinterpret_cast<const f16x8 *>(base + SA + col * 64 + (((hh * 2 + kh) ^ swB) << 4));
        } else {
            const qu32x4_t w = *reinterpret_cast<const qu32x4_t *>(
                base + SA + (BPC == 32 ? col * 32 + ((hh ^ ((li >> 3) & 1)) << 4) : col * 16));
#pragma unroll
            for (int kh = 0; kh < 2; kh++) b[kh] = quants_f16<WQ>(qu32x2_t{w[2 * kh], w[2 * kh + 1]}, 4 * hh);
        }
    };
    auto scale_of = [&](const unsigned char *base, int c) __attribute__((always_inline)) {
        return *reinterpret_cast<const float *>(base + SA + SB + ((wn * CT + c) * 32 + li) * 4);
    };
    auto mfma = [&](const f16x8 &x, const f16x8 &w, f32x16 &t, bool first) __attribute__((always_inline)) {
        f32x16 cc;
        if (first) {
#pragma unroll
            for (int q = 0; q < 16; q++) cc[q] = 0.0f;
        } else {
            cc = t;
        }
        t = __builtin_amdgcn_mfma_f32_32x32x16_f16(x, w, cc, 0, 0, 0);
    };
    // LDS read addresses: per-lane parts (loop-invariant) plus the stage's
    // base, added in the block (add_here), so the loop unrolled over the
    // three stages keeps one set of per-lane parts instead of one per stage
    const unsigned lds0 = (unsigned)(size_t)lds;
    auto at = [&](unsigned lane_part, int uniform) __attribute__((always_inline)) {
        return lds + (add_here(lane_part, lds0 + uniform) - lds0);
    };
    auto compute = [&](int stg) __attribute__((always_inline)) {
        const unsigned char *base = lds + goff + stg * STAGE;
        const int boff = goff + stg * STAGE + SA;  // the stage's B operands
        f16x8 a[2][2][RT];  // [k-half][limb][row tile]
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int l = 0; l < 2; l++)
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    const int row = (wm * RT + r) * 32 + li, chunk = l * 4 + hh * 2 + kh;
                    a[kh][l][r] = *reinterpret_cast<const f16x8 *>(
                        at((unsigned)(row * 128 + ((chunk ^ swA) << 4)), goff + stg * STAGE));
                }
        if constexpr (RT >= 2) {
#pragma unroll
            for (int c = 0; c < CT; c++) {
                f32x16 tmp[NT];
                if (c == CT - 1) {
                    // the previous block's last column tile, scaled while this block's MFMAs run
#pragma unroll
                    for (int r = 0; r < RT; r++)
#pragma unroll
                        for (int q = 0; q < 16; q++) acc[r][CT - 1][q] += dpend * pend[r][q];
                }
                f16x8 b[2];
                read_b2(base, c, b);
#pragma unroll
                for (int kh = 0; kh < 2; kh++) {
#pragma unroll
                    for (int l = 0; l < 2; l++)
#pragma unroll
                        for (int r = 0; r < RT; r++) mfma(a[kh][l][r], b[kh], tmp[r], kh == 0 && l == 0);
                }
                const float d = scale_of(base, c);
                if (c == CT - 1) {
#pragma unroll
                    for (int r = 0; r < RT; r++) pend[r] = tmp[r];
                    dpend = d;
                } else {
#pragma unroll
                    for (int r = 0; r < RT; r++)
#pragma unroll
                        for (int q = 0; q < 16; q++) acc[r][c][q] += d * tmp[r][q];
                }
            }
        } else if constexpr (SCH == 1 && CT == 5) {
            // Chains 0-2 as a triple, then chains 3-4 as a pair, each chain's
            // MFMAs in the same (k-half, limb) order as the default schedule.
            // The previous block's pair is scaled first, under the latency of
            // this block's operand reads; this block's triple is scaled under
            // the pair's MFMAs, so the scaling FMAs run beside MFMAs instead of
            // ahead of them.  The same additions in the same order.  The order
            // is written out and fenced (sched_barrier), and the pair's
            // operands are read once the triple's first k-half is issued.
            // B: one address per k-half (column tile c is 2048 bytes further)
            const unsigned char *bk[2] = {at((unsigned)((wn * CT * 32 + li) * 64 + (((hh * 2) ^ swB) << 4)), boff),
                                          at((unsigned)((wn * CT * 32 + li) * 64 + (((hh * 2 + 1) ^ swB) << 4)),
                                             boff)};
            auto rd_b = [&](int c, int kh) __attribute__((always_inline)) {
                return *reinterpret_cast<const f16x8 *>(bk[kh] + c * 2048);
            };
            auto fence = [&]() __attribute__((always_inline)) { __builtin_amdgcn_sched_barrier(0); };
            auto scale = [&](int c, float d, int q0, int q1) __attribute__((always_inline)) {
#pragma unroll
                for (int q = q0; q < q1; q++) acc[0][c][q] += d * tcar[c][q];
            };
            const f16x8 b00 = rd_b(0, 0), b10 = rd_b(1, 0), b20 = rd_b(2, 0);
            const f16x8 b01 = rd_b(0, 1), b11 = rd_b(1, 1), b21 = rd_b(2, 1);
            float dcur[CT];
            const unsigned char *sc = at((unsigned)((wn * CT * 32 + li) * 4), goff + stg * STAGE + SA + SB);
#pragma unroll
            for (int c = 0; c < CT; c++) dcur[c] = *reinterpret_cast<const float *>(sc + c * 128);
            fence();
            scale(3, dcar[3], 0, 16);
            scale(4, dcar[4], 0, 16);
            fence();
            mfma(a[0][0][0], b00, tcar[0], true);
            mfma(a[0][0][0], b10, tcar[1], true);
            mfma(a[0][0][0], b20, tcar[2], true);
            mfma(a[0][1][0], b00, tcar[0], false);
            mfma(a[0][1][0], b10, tcar[1], false);
            mfma(a[0][1][0], b20, tcar[2], false);
            fence();
            const f16x8 b30 = rd_b(3, 0), b40 = rd_b(4, 0), b31 = rd_b(3, 1), b41 = rd_b(4, 1);
            fence();
            mfma(a[1][0][0], b01, tcar[0], false);
            mfma(a[1][0][0], b11, tcar[1], false);
            mfma(a[1][0][0], b21, tcar[2], false);
            mfma(a[1][1][0], b01, tcar[0], false);
            mfma(a[1][1][0], b11, tcar[1], false);
            mfma(a[1][1][0], b21, tcar[2], false);
            fence();
            mfma(a[0][0][0], b30, tcar[3], true);
            scale(0, dcur[0], 0, 6);
            fence();
            mfma(a[0][0][0], b40, tcar[4], true);
            scale(0, dcur[0], 6, 12);
            fence();
            mfma(a[0][1][0], b30, tcar[3], false);
            scale(0, dcur[0], 12, 16);
            scale(1, dcur[1], 0, 2);
            fence();
            mfma(a[0][1][0], b40, tcar[4], false);
            scale(1, dcur[1], 2, 8);
            fence();
            mfma(a[1][0][0], b31, tcar[3], false);
            scale(1, dcur[1], 8, 14);
            fence();
            mfma(a[1][0][0], b41, tcar[4], false);
            scale(1, dcur[1], 14, 16);
            scale(2, dcur[2], 0, 4);
            fence();
            mfma(a[1][1][0], b31, tcar[3], false);
            scale(2, dcur[2], 4, 10);
            fence();
            mfma(a[1][1][0], b41, tcar[4], false);
            scale(2, dcur[2], 10, 16);
            dcar[3] = dcur[3];
            dcar[4] = dcur[4];
        } else {
            f16x8 b[CT][2];
#pragma unroll
            for (int c = 0; c < CT; c++) read_b2(base, c, b[c]);
#pragma unroll
            for (int c = 0; c < CT; c++) {
#pragma unroll
                for (int q = 0; q < 16; q++) acc[0][c][q] += dcar[c] * tcar[c][q];
                mfma(a[0][0][0], b[c][0], tcar[c], true);
            }
#pragma unroll
            for (int kh = 0; kh < 2; kh++) {
#pragma unroll
                for (int l = kh == 0 ? 1 : 0; l < 2; l++)
#pragma unroll
                    for (int c = 0; c < CT; c++) mfma(a[kh][l][0], b[c][kh], tcar[c], false);
            }
#pragma unroll
            for (int c = 0; c < CT; c++) dcar[c] = scale_of(base, c);
        }
    };

    // Before reading block kb: this wave's loads of kb have landed (those of
    // kb+1 may still be in flight: NI newer instructions), its own LDS reads
    // are done, and all waves meet.  After the barrier the stage of kb-1 is
    // free for kb+2.  The load unit's LDS writes are invisible to the
    // compiler, hence the explicit counts and the memory clobber.
    auto sync = [&]() __attribute__((always_inline)) {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(T::NI) : "memory");
    };
    if constexpr (PERS) {
        // Persistent workgroups (grid <= tiles, tiles strided by the grid;
        // the plain epilogues from the f16 copy): the stage ring runs on
        // across tiles, so the next tile's first two blocks and its bias are
        // fetched under this tile's last two blocks and its epilogue instead
        // of after a new workgroup's start.  Needs KB >= 3 (the bias buffer a
        // tile's epilogue reads is refilled two tiles later, after a barrier
        // of the tile between).  The same sums in the same order.
        auto finish = [&]() __attribute__((always_inline)) {
            if constexpr (RT >= 2) {
#pragma unroll
                for (int r = 0; r < RT; r++)
#pragma unroll
                    for (int q = 0; q < 16; q++) acc[r][CT - 1][q] += dpend * pend[r][q];
            } else {
                // (SCH 1 scales chains 0-2 inside each block; only the pair is pending)
#pragma unroll
                for (int c = (SCH == 1 && CT == 5) ? 3 : 0; c < CT; c++)
#pragma unroll
                    for (int q = 0; q < 16; q++) acc[0][c][q] += dcar[c] * tcar[c][q];
            }
        };
        auto epilogue = [&](const int em0, const int en0, const float *sb) __attribute__((always_inline)) {
            // Epilogue: every output value is formed before the first store (the
            // residual reads share one wait, and no store follows a pending load, which
            // would make the compiler wait for each earlier store at every bounds
            // branch); tiles inside the matrix store without bounds branches.
            float res[CT][RT][16];
            if constexpr (EPI == EPI_RESIDUAL) {
#pragma unroll
                for (int c = 0; c < CT; c++) {
                    const int col = min(en0 + (wn * CT + c) * 32 + li, N - 1);
#pragma unroll
                    for (int r = 0; r < RT; r++)
#pragma unroll
                        for (int q = 0; q < 16; q++) {
                            const int row = min(em0 + (wm * RT + r) * 32 + 8 * (q >> 2) + 4 * hh + (q & 3), M - 1);
                            res[c][r][q] = reinterpret_cast<const float *>(Yv)[(size_t)row * ldy + col];
                        }
                }
            }
            float bv[CT];
#pragma unroll
            for (int c = 0; c < CT; c++) bv[c] = sb[(wn * CT + c) * 32 + li];
#pragma unroll
            for (int c = 0; c < CT; c++)
#pragma unroll
                for (int r = 0; r < RT; r++)
#pragma unroll
                    for (int q = 0; q < 16; q++) {
                        float v = acc[r][c][q] + bv[c];
                        if constexpr (EPI == EPI_GELU_H2 || EPI == EPI_GELU) v = gelu_as(v);
                        if constexpr (EPI == EPI_RESIDUAL) v = res[c][r][q] + v;
                        acc[r][c][q] = v;
                    }
            auto store = [&](bool guard) __attribute__((always_inline)) {
#pragma unroll
                for (int c = 0; c < CT; c++) {
                    const int col = en0 + (wn * CT + c) * 32 + li;
                    if (guard && col >= N) continue;
#pragma unroll
                    for (int r = 0; r < RT; r++)
#pragma unroll
                        for (int q = 0; q < 16; q++) {
                            const int row = em0 + (wm * RT + r) * 32 + 8 * (q >> 2) + 4 * hh + (q & 3);
                            if (guard && row >= M) continue;
                            if constexpr (EPI == EPI_GELU_H2)
                                h2_store(reinterpret_cast<unsigned short *>(Yv), row, col, N, acc[r][c][q]);
                            else
                                reinterpret_cast<float *>(Yv)[(size_t)row * ldy + col] = acc[r][c][q];
                        }
                }
            };
            if (em0 + BM <= M && en0 + BN <= N)
                store(false);
            else
                store(true);
        };
        const int ntiles = nM * nN;
        int rt = blockIdx.x, rkb = 0, rbuf = 0;  // request cursor: tile, block, bias buffer
        bool rlive = true;
        // blocks in tile order across this workgroup's tiles; past its last
        // tile the requests re-read that tile's last block (stages nobody reads)
        auto issue = [&](int stgq) __attribute__((always_inline)) {
            request(rlive ? rkb : KB - 1, stgq);
            if (rlive && ++rkb == KB) {
                rkb = 0;
                rt += gridDim.x;
                if (rt < ntiles) {
                    set_tile(rt);
                    rbuf ^= 1;
                    load_bias(rbuf);
                } else {
                    rlive = false;
                }
            }
        };
        issue(0);
        issue(1);
        int stg = 0, buf = 0;
        for (int t = blockIdx.x; t < ntiles; t += gridDim.x) {
            int tm, tn;
            tile_xcd(t, ntiles, nM, nN, tm, tn);
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int c = 0; c < CT; c++)
#pragma unroll
                    for (int q = 0; q < 16; q++) acc[r][c][q] = 0.0f;
            dpend = 0.0f;
#pragma unroll
            for (int r = 0; r < (RT >= 2 ? RT : 1); r++)
#pragma unroll
                for (int q = 0; q < 16; q++) pend[r][q] = 0.0f;
#pragma unroll
            for (int c = 0; c < (RT >= 2 ? 1 : CT); c++) {
                dcar[c] = 0.0f;
#pragma unroll
                for (int q = 0; q < 16; q++) tcar[c][q] = 0.0f;
            }
            for (int kb = 0; kb < KB; kb++) {
                sync();
                issue(stg == 0 ? 2 : stg - 1);
                compute(stg);
                stg = stg == 2 ? 0 : stg + 1;
            }
            finish();
            epilogue(tm * BM, tn * BN, reinterpret_cast<const float *>(lds + BOFF + buf * BBYTES));
            buf ^= 1;
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }
    // Requests past the last block re-read it into a stage nobody reads again,
    // so every wave issues the same instructions and the counts hold.
    // KW > 1: group grp's step i is block kb0 + grp + KW i; every group runs
    // the same nit steps (the same barriers in every wave), and a step whose
    // block lies past kb1 requests the last block and computes nothing.
    const int nit = (kb1 - kb0 + KW - 1) / KW;
    auto gblk = [&](int i) __attribute__((always_inline)) { return min(kb0 + grp + KW * i, kb1 - 1); };
    if constexpr (KW > 1) {
        request(gblk(0), 0);
        request(gblk(1), 1);
    } else {
        request(kb0, 0);
        request(min(kb0 + 1, kb1 - 1), 1);
    }
    if constexpr (PREF) {
        int *s_pk = reinterpret_cast<int *>(lds + LOFF), *s_pos = s_pk + BM;
        if (tid < BM) {
            const int row = m0 + tid;
            s_pk[tid] = row < M ? qo.pk[row] : -1;
            s_pos[tid] = row < M ? qo.pos[row] : 0;
        }
        if (n0 < 2 * qo.d && n0 + BN > qo.d) {  // K columns: cos rows, then sin rows, [2][BM][QHALF]
            constexpr int CPRR = QHALF / 4, NCH = 2 * BM * CPRR, NJ = NCH / 64;
            static_assert(NCH % 64 == 0, "whole 1 KiB loads");
            for (int j = wave; j < NJ; j += NW) {
                const int c = j * 64 + lane, tbl = c / (BM * CPRR), rem = c % (BM * CPRR);
                const int row = min(m0 + rem / CPRR, M - 1);
                const float *src = (tbl ? qo.rs : qo.rc) + (size_t)qo.pos[row] * QHALF + (rem % CPRR) * 4;
                __builtin_amdgcn_global_load_lds((glb_ptr_t *)src, (lds_ptr_t *)(lds + LOFF + BM * 8 + j * 1024),
                                                 16, 0, 0);
            }
        }
    }
    if constexpr (KW > 1) {
        for (int i = 0;;) {
            const bool l0 = kb0 + grp + KW * i < kb1;
            sync();
            request(gblk(i + 2), 2);
            if (l0) compute(0);
            if (++i == nit) break;
            const bool l1 = kb0 + grp + KW * i < kb1;
            sync();
            request(gblk(i + 2), 0);
            if (l1) compute(1);
            if (++i == nit) break;
            const bool l2 = kb0 + grp + KW * i < kb1;
            sync();
            request(gblk(i + 2), 1);
            if (l2) compute(2);
            if (++i == nit) break;
        }
    } else {
        for (int kb = kb0;;) {
            sync();
            request(min(kb + 2, kb1 - 1), 2);
            compute(0);
            if (++kb == kb1) break;
            sync();
            request(min(kb + 2, kb1 - 1), 0);
            compute(1);
            if (++kb == kb1) break;
            sync();
            request(min(kb + 2, kb1 - 1), 1);
            compute(2);
            if (++kb == kb1) break;
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if constexpr (RT >= 2) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[r][CT - 1][q] += dpend * pend[r][q];
    } else {
        // (SCH 1 scales chains 0-2 inside each block; only the pair is pending)
#pragma unroll
        for (int c = (SCH == 1 && CT == 5) ? 3 : 0; c < CT; c++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[0][c][q] += dcar[c] * tcar[c][q];
    }
    if constexpr (KW > 1) {
        // The groups' sums, added in group order by group 0, through the
        // stages: after the first barrier every wave's copies have landed and
        // every wave is done reading the stages.
        float *red = reinterpret_cast<float *>(lds);
        __syncthreads();
        if (grp > 0) {
#pragma unroll
            for (int c = 0; c < CT; c++)
#pragma unroll
                for (int q = 0; q < 16; q++) red[((((grp - 1) * NW + lw) * CT + c) * 16 + q) * 64 + lane] = acc[0][c][q];
        }
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int g = 1; g < KW; g++)
#pragma unroll
            for (int c = 0; c < CT; c++)
#pragma unroll
                for (int q = 0; q < 16; q++) acc[0][c][q] += red[((((g - 1) * NW + lw) * CT + c) * 16 + q) * 64 + lane];
    }

    // Epilogue: every output value is formed before the first store (the
    // residual reads share one wait, and no store follows a pending load, which
    // would make the compiler wait for each earlier store at every bounds
    // branch); tiles inside the matrix store without bounds branches.
    float res[CT][RT][16];
    if constexpr (EPI == EPI_RESIDUAL) {
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const int col = min(n0 + (wn * CT + c) * 32 + li, N - 1);
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    const int row = min(m0 + (wm * RT + r) * 32 + 8 * (q >> 2) + 4 * hh + (q & 3), M - 1);
                    res[c][r][q] = reinterpret_cast<const float *>(Yv)[(size_t)row * ldy + col];
                }
        }
    }
    float bv[CT];
#pragma unroll
    for (int c = 0; c < CT; c++) bv[c] = s_bias[(wn * CT + c) * 32 + li];
#pragma unroll
    for (int c = 0; c < CT; c++)
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int q = 0; q < 16; q++) {
                float v = acc[r][c][q] + bv[c];
                if constexpr (EPI == EPI_GELU_H2 || EPI == EPI_GELU) v = gelu_as(v);
                if constexpr (EPI == EPI_RESIDUAL) v = res[c][r][q] + v;
                acc[r][c][q] = v;
            }
    if constexpr (EPI == EPI_QKV16 || EPI == EPI_QKV32 || EPI == EPI_QKV64) {
        qkv_epilogue<EPI == EPI_QKV16 ? 16 : (EPI == EPI_QKV32 ? 32 : 64), RT, CT, WM, WN, PREF>(
            acc, lds, lds + LOFF, m0, n0, wm, wn, lane, M, N, reinterpret_cast<float *>(Yv), ldy, qo);
        return;
    }
    auto store = [&](bool guard) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const int col = n0 + (wn * CT + c) * 32 + li;
            if (guard && col >= N) continue;
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    const int row = m0 + (wm * RT + r) * 32 + 8 * (q >> 2) + 4 * hh + (q & 3);
                    if (guard && row >= M) continue;
                    if constexpr (EPI == EPI_GELU_H2)
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

// q16[kb][n][j] = f16 of quant j of block (kb, n): Q8_0 bytes as signed
// integers; Q4_0 element j < 16 the low nibble of byte j, j >= 16 the high
// nibble of byte j - 16, minus 8 (the reference's nibble order).
template <int WF>
__global__ __launch_bounds__(256) void k_expand_f16(const unsigned char *__restrict__ q, unsigned short *__restrict__ q16,
                                                    int64_t blocks) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one element
    if (i >= blocks * 32) return;
    const int64_t blk = i >> 5;
    const int j = (int)(i & 31);
    int v;
    if constexpr (WF == WF_Q8) {
        v = (signed char)q[blk * 32 + j];
    } else {
        const unsigned b = q[blk * 16 + (j & 15)];
        v = (int)(j < 16 ? (b & 15u) : (b >> 4)) - 8;
    }
    q16[i] = __builtin_bit_cast(unsigned short, (_Float16)(float)v);
}

// Block order of the 32 x 160 wave tiles reading the f16 copy: 1 (default)
// the triple + pair order, 0 (CIH_GEMM_SCHED=0) all five chains interleaved.
// Both give the same bits.
int gemm_sched() {
    const char *e = getenv("CIH_GEMM_SCHED");
    return e ? atoi(e) : 1;
}

// The small tiles (RT == 1, CT <= 2: 64 x 64 and 64 x 128) read the f16
// copy only.
template <int RT, int CT> constexpr bool copy_only() { return RT == 1 && CT <= 2; }

// Workgroups of the persistent form for a launch of `tiles` tiles of KB
// blocks, 0 for one tile per workgroup: one per CU (a multiple of the 8
// XCDs, so that a workgroup's tiles stay on its XCD) when the tiles take
// more than one round.  CIH_GEMM_PERSIST=0: never; =force: 8 workgroups
// whenever the form applies (many tiles each, for tests).
int persist_grid(int tiles, int KB) {
    if (KB < 3) return 0;
    const char *e = getenv("CIH_GEMM_PERSIST");
    if (e && !strcmp(e, "0")) return 0;
    if (e && !strcmp(e, "force")) return std::min(tiles, 8);
    const int g = device_cus() / 8 * 8;
    return g > 0 && tiles > g ? g : 0;
}

template <int EPI, int RT, int CT, int WM, int WN, int KW = 1>
hipError_t launch_t(const DevMatrix &W, const void *X, const float *bias, void *Y, int ldy, int M, hipStream_t st,
                    const QkvOut &qo) {
    using T = LdsTile<RT, CT, WM, WN>;
    static_assert(KW == 1 || copy_only<RT, CT>(), "k-groups: the small tiles");
    const int tiles = ((M + T::BM - 1) / T::BM) * ((W.N + T::BN - 1) / T::BN);
    const unsigned short *Xh = reinterpret_cast<const unsigned short *>(X);
    const bool quants = !W.q16;
    const int kbx = W.kx / 32;
    // FP32 weights' pair copies (kbx): the small tiles and 128 x 320; the FP32
    // GELU epilogue (the LM head's dense layer) only with a pair copy
    constexpr bool PX320 = RT == 1 && CT == 5 && WM == 4 && WN == 2 && EPI < EPI_QKV16;
    if ((kbx && !copy_only<RT, CT>() && !PX320) || (EPI == EPI_GELU && (!kbx || quants))) return hipErrorInvalidValue;
    if constexpr (PX320) {
        if (kbx) {
            if (quants) return hipErrorInvalidValue;
            hipLaunchKernelGGL((k_gemm_lds<EPI, 1, 5, 4, 2, 0, false, 1, false, true>), dim3(tiles), dim3(T::THREADS), 0,
                               st, Xh, reinterpret_cast<const unsigned char *>(W.q16), W.sc, bias, Y, ldy, M, W.N, W.K,
                               qo, 0, kbx);
            return hipGetLastError();
        }
    }
    if constexpr (EPI == EPI_GELU && !copy_only<RT, CT>()) {
        return hipErrorInvalidValue;  // (rejected above)
    } else if constexpr (copy_only<RT, CT>()) {
        if (quants) return hipErrorInvalidValue;
        if (kbx)
            hipLaunchKernelGGL((k_gemm_lds<EPI, RT, CT, WM, WN, 0, false, 0, false, true, KW>), dim3(tiles),
                               dim3(T::THREADS * KW), 0, st, Xh, reinterpret_cast<const unsigned char *>(W.q16), W.sc,
                               bias, Y, ldy, M, W.N, W.K, qo, 0, kbx);
        else if constexpr (EPI != EPI_GELU)
            hipLaunchKernelGGL((k_gemm_lds<EPI, RT, CT, WM, WN, 0, false, 0, false, false, KW>), dim3(tiles),
                               dim3(T::THREADS * KW), 0, st, Xh, reinterpret_cast<const unsigned char *>(W.q16), W.sc,
                               bias, Y, ldy, M, W.N, W.K, qo);
    } else if (quants && W.fmt == WF_Q8)
        hipLaunchKernelGGL((k_gemm_lds<EPI, RT, CT, WM, WN, WF_Q8>), dim3(tiles), dim3(T::THREADS), 0, st, Xh,
                           static_cast<const unsigned char *>(W.q), W.sc, bias, Y, ldy, M, W.N, W.K, qo);
    else if (quants && W.fmt == WF_Q4)
        hipLaunchKernelGGL((k_gemm_lds<EPI, RT, CT, WM, WN, WF_Q4>), dim3(tiles), dim3(T::THREADS), 0, st, Xh,
                           static_cast<const unsigned char *>(W.q), W.sc, bias, Y, ldy, M, W.N, W.K, qo);
    else if (RT == 1 && CT == 5 && gemm_sched() == 1) {
        // 128 x 320 with a plain GELU or no epilogue over more than one round:
        // persistent workgroups (FC1 at 8192 tokens of ESM-2 650M, 4 rounds:
        // 290 -> 280 us in isolation; Wo and FC2 are one round, and the
        // residual form would spill)
        if constexpr (WM == 4 && WN == 2 && (EPI == EPI_GELU_H2 || EPI == EPI_NONE)) {
            if (const int g = persist_grid(tiles, W.K / 32)) {
                hipLaunchKernelGGL((k_gemm_lds<EPI, 1, 5, 4, 2, 0, false, 1, true>), dim3(g), dim3(T::THREADS), 0, st,
                                   Xh, reinterpret_cast<const unsigned char *>(W.q16), W.sc, bias, Y, ldy, M, W.N,
                                   W.K, qo, 0);
                return hipGetLastError();
            }
        }
        hipLaunchKernelGGL((k_gemm_lds<EPI, RT, CT, WM, WN, 0, false, (RT == 1 && CT == 5) ? 1 : 0>), dim3(tiles),
                           dim3(T::THREADS), 0, st, Xh, reinterpret_cast<const unsigned char *>(W.q16), W.sc, bias, Y,
                           ldy, M, W.N, W.K, qo, 0);
    }
    else
        hipLaunchKernelGGL((k_gemm_lds<EPI, RT, CT, WM, WN, 0>), dim3(tiles), dim3(T::THREADS), 0, st, Xh,
                           reinterpret_cast<const unsigned char *>(W.q16), W.sc, bias, Y, ldy, M, W.N, W.K, qo);
    return hipGetLastError();
}

// Split-K form: grid (tiles, S), raw partial sums into part.  128 x 128 tiles
// (4 waves) for every weight form; 64 x 128 and 64 x 64 from the f16 copy.
template <int RT, int CT, int WM, int WN, int KW = 1>
hipError_t launch_split_t(const DevMatrix &W, const void *X, int M, float *part, int S, int kps, hipStream_t st) {
    using T = LdsTile<RT, CT, WM, WN>;
    static_assert(KW == 1 || copy_only<RT, CT>(), "k-groups: the small tiles");
    const int tiles = ((M + T::BM - 1) / T::BM) * ((W.N + T::BN - 1) / T::BN);
    const unsigned short *Xh = reinterpret_cast<const unsigned short *>(X);
    const dim3 grid(tiles, S), block(T::THREADS * KW);
    const int kbx = W.kx / 32;
    if (kbx && !copy_only<RT, CT>()) return hipErrorInvalidValue;  // pair copies: the small tiles only
    if constexpr (copy_only<RT, CT>()) {
        if (!W.q16) return hipErrorInvalidValue;
        if (kbx)
            hipLaunchKernelGGL((k_gemm_lds<EPI_NONE, RT, CT, WM, WN, 0, true, 0, false, true, KW>), grid, block, 0, st,
                               Xh, reinterpret_cast<const unsigned char *>(W.q16), W.sc, nullptr, part, W.N, M, W.N,
                               W.K, QkvOut(), kps, kbx);
        else
            hipLaunchKernelGGL((k_gemm_lds<EPI_NONE, RT, CT, WM, WN, 0, true, 0, false, false, KW>), grid, block, 0, st,
                               Xh, reinterpret_cast<const unsigned char *>(W.q16), W.sc, nullptr, part, W.N, M, W.N,
                               W.K, QkvOut(), kps);
    } else if (!W.q16 && W.fmt == WF_Q8)
        hipLaunchKernelGGL((k_gemm_lds<EPI_NONE, RT, CT, WM, WN, WF_Q8, true>), grid, block, 0, st, Xh,
                           static_cast<const unsigned char *>(W.q), W.sc, nullptr, part, W.N, M, W.N, W.K, QkvOut(),
                           kps);
    else if (!W.q16)
        hipLaunchKernelGGL((k_gemm_lds<EPI_NONE, RT, CT, WM, WN, WF_Q4, true>), grid, block, 0, st, Xh,
                           static_cast<const unsigned char *>(W.q), W.sc, nullptr, part, W.N, M, W.N, W.K, QkvOut(),
                           kps);
    else
        hipLaunchKernelGGL((k_gemm_lds<EPI_NONE, RT, CT, WM, WN, 0, true>), grid, block, 0, st, Xh,
                           reinterpret_cast<const unsigned char *>(W.q16), W.sc, nullptr, part, W.N, M, W.N, W.K,
                           QkvOut(), kps);
    return hipGetLastError();
}

hipError_t launch_split(const DevMatrix &W, const void *X, int M, float *part, int S, int kps, int tile, int kw,
                        hipStream_t st) {
    if (tile == LDS_TILE_64x64) {
        if (kw == 4) return launch_split_t<1, 1, 2, 2, 4>(W, X, M, part, S, kps, st);
        if (kw == 2) return launch_split_t<1, 1, 2, 2, 2>(W, X, M, part, S, kps, st);
        return launch_split_t<1, 1, 2, 2>(W, X, M, part, S, kps, st);
    }
    if (tile == LDS_TILE_64x128) {
        if (kw == 2) return launch_split_t<1, 2, 2, 2, 2>(W, X, M, part, S, kps, st);
        return launch_split_t<1, 2, 2, 2>(W, X, M, part, S, kps, st);
    }
    return launch_split_t<2, 2, 2, 2>(W, X, M, part, S, kps, st);
}

// Tile choice for problems that fill the device with 128-row tiles, by a
// model of the time the rounds of workgroups take on the device's CUs.
// Candidates, in order of preference (fewest operand bytes per output
// first): 128 x 320 and 128 x 256 (8 waves, one workgroup per CU), 128 x 160
// (4 waves; two per CU with 1-byte quants, one with the f16 copy, whose
// three stages take 81 KiB: then it is left out) and 128 x 128 (4 waves,
// two per CU).  A full round costs the tile area times the workgroups
// sharing a CU; a last round that leaves a 4-wave workgroup alone on its CU
// runs it at about 1/1.4 of a CU's rate.  At M = 8192 this picks 128 x 320
// for every ESM-2 650M projection (QKV: 3 rounds instead of 3.75; N = 1280:
// one round instead of 1.25).
int tile_choice(int M, int N, bool copy) {
    const int cus = device_cus();
    const long mt = (M + 127) / 128;
    struct Cand {
        int tile, bn, per_cu;
    };
    const Cand cand[4] = {{LDS_TILE_128x320, 320, 1}, {LDS_TILE_128x256, 256, 1}, {LDS_TILE_128x160, 160, 2},
                          {LDS_TILE_128x128, 128, 2}};
    int best = LDS_TILE_128x128;
    double best_cost = 0;
    for (const Cand &c : cand) {
        if (copy && c.bn == 160) continue;
        const long tiles = mt * ((N + c.bn - 1) / c.bn), slots = (long)c.per_cu * cus;
        const double area = 128.0 * c.bn;
        const long full = tiles / slots, rest = tiles % slots;
        double cost = full * area * c.per_cu;
        if (rest) cost += (c.per_cu == 2 && rest <= cus) ? 1.4 * area : area * c.per_cu;
        if (best_cost == 0 || cost < best_cost) {
            best = c.tile;
            best_cost = cost;
        }
    }
    return best;
}

// CIH_GEMM_TILE_N (CIH_GEMM_TILE_N_GELU for the FC1 + GELU GEMM): 320, 256,
// 160, 128 (128-row tiles of that width), 64x128 or 64 (64 x 64); 0 when
// unset.
int tile_env(int epi) {
    const char *e = getenv("CIH_GEMM_TILE_N");
    if (const char *eg = getenv("CIH_GEMM_TILE_N_GELU"); eg && epi == EPI_GELU_H2) e = eg;
    if (!e) return 0;
    if (!strcmp(e, "64x128")) return LDS_TILE_64x128;
    switch (atoi(e)) {
    case 320: return LDS_TILE_128x320;
    case 256: return LDS_TILE_128x256;
    case 160: return LDS_TILE_128x160;
    case 64: return LDS_TILE_64x64;
    default: return LDS_TILE_128x128;
    }
}

// tile 0: CIH_GEMM_TILE_N, else the round model's choice.  The small tiles
// and 128 x 160 serve the plain epilogues only (in the QKV epilogue a
// workgroup's columns must hold whole heads); a small tile without the f16
// copy becomes 128 x 128.
template <int EPI>
hipError_t launch_epi(const DevMatrix &W, const void *X, const float *bias, void *Y, int ldy, int M, hipStream_t st,
                      const QkvOut &qo, int tile, int kw = 1) {
    if (!tile) tile = tile_env(EPI);
    if (!tile) tile = tile_choice(M, W.N, W.q16 != nullptr);
    if (tile == LDS_TILE_128x320) return launch_t<EPI, 1, 5, 4, 2>(W, X, bias, Y, ldy, M, st, qo);
    if (tile == LDS_TILE_128x256) return launch_t<EPI, 2, 2, 2, 4>(W, X, bias, Y, ldy, M, st, qo);
    if constexpr (EPI < EPI_QKV16) {
        if (tile == LDS_TILE_128x160) return launch_t<EPI, 1, 5, 4, 1>(W, X, bias, Y, ldy, M, st, qo);
        if (W.q16) {
            if (tile == LDS_TILE_64x128) {
                if (kw == 2) return launch_t<EPI, 1, 2, 2, 2, 2>(W, X, bias, Y, ldy, M, st, qo);
                return launch_t<EPI, 1, 2, 2, 2>(W, X, bias, Y, ldy, M, st, qo);
            }
            if (tile == LDS_TILE_64x64) {
                if (kw == 4) return launch_t<EPI, 1, 1, 2, 2, 4>(W, X, bias, Y, ldy, M, st, qo);
                if (kw == 2) return launch_t<EPI, 1, 1, 2, 2, 2>(W, X, bias, Y, ldy, M, st, qo);
                return launch_t<EPI, 1, 1, 2, 2>(W, X, bias, Y, ldy, M, st, qo);
            }
        }
    }
    return launch_t<EPI, 2, 2, 2, 2>(W, X, bias, Y, ldy, M, st, qo);
}

}  // namespace

int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
        else
            cus = 256;
    }
    return cus;
}

bool gemm_lds_applies(const DevMatrix &W, int a_fmt, int M, int epi) {
    if (a_fmt != AF_H2 || (W.fmt != WF_Q8 && W.fmt != WF_Q4) || W.K % 32 || M <= 0) return false;
    if (epi != EPI_NONE && epi != EPI_RESIDUAL && epi != EPI_GELU_H2) return false;
    const char *e = getenv("CIH_GEMM_LDS");
    if (e && !strcmp(e, "0")) return false;
    if (e && !strcmp(e, "force")) return true;
    return (long)((M + 127) / 128) * ((W.N + 127) / 128) >= 256;
}

bool gemm_lds_split_applies(const DevMatrix &W, int a_fmt, int M, int epi) {
    if (a_fmt != AF_H2 || (W.fmt != WF_Q8 && W.fmt != WF_Q4) || W.K % 32 || M <= 0 || W.N <= 0) return false;
    if (epi != EPI_NONE && epi != EPI_RESIDUAL) return false;
    const char *e = getenv("CIH_GEMM_LDS"), *ke = getenv("CIH_SPLITK");
    if ((e && !strcmp(e, "0")) || (ke && !strcmp(ke, "0"))) return false;
    // the splits cost their partial sums' traffic (S M N floats written here
    // and read by the caller's fold, 11-13 us per split projection on top of
    // the LayerNorm at 4096 x 640 and 2550 x 1280): only deep products over
    // many rows gain more than that (650M FC2, K = 5120, 2550 rows: 82 -> 56
    // us; K = 640 to 2560: no net gain; 402 rows: the register-staged split
    // is faster)
    const long tiles = (long)((M + 127) / 128) * ((W.N + 127) / 128);
    return tiles >= 32 && tiles < 256 && W.K >= 4096 && M >= 1024;
}

hipError_t launch_gemm_lds_split(const DevMatrix &W, const void *X, int M, const PartialBuf &pb, int *splits,
                                 hipStream_t st) {
    *splits = 0;
    if ((W.fmt != WF_Q8 && W.fmt != WF_Q4) || W.K % 32 || M <= 0 || W.N <= 0 || !pb.part) return hipErrorInvalidValue;
    // two 4-wave workgroups per CU: splits up to one round of them, at least
    // 4 k-blocks each, partial sums within pb
    const int KB = W.K / 32;
    const long tiles = (long)((M + 127) / 128) * ((W.N + 127) / 128);
    int S = (int)std::min<long>(2L * device_cus() / tiles, KB / 4);
    while (S > 1 && (size_t)S * M * W.N > pb.floats) S--;
    if (S < 2) return hipSuccess;
    const int kps = (KB + S - 1) / S;
    S = (KB + kps - 1) / kps;
    *splits = S;
    return launch_split(W, X, M, pb.part, S, kps, LDS_TILE_128x128, 1, st);
}

// Routing of the problems that do not fill the device with 128-row tiles,
// from a sweep of every tile and split over the ESM-2 8M-3B projections at
// 16-8192 tokens on MI355X (256 CUs; the thresholds scale with the CU
// count); below 64 rows the register-staged kernel stays.  One 4-wave workgroup per CU exposes the per-block barrier and
// operand-read latency to its lone wave per SIMD; smaller tiles put three or
// four workgroups on each CU and leave fewer CUs idle in the last round.  A
// split's partial sums cost the LayerNorm that adds them about S M N 4 bytes
// at 2 TB/s (3B, 2048 x 2560, 3 splits: 10.1 -> 41.6 us), so splits pay only
// where the unsplit GEMM leaves most of the device idle:
//   * residual projections with K >= 5120 (160 blocks) whose caller adds
//     splits, from 25 tiles of 128 x 128 on (fewer: the 64 x 64 rule
//     below): up to 100 such tiles, 64 x 128 tiles in 3 k-splits;
//     fewer 128 x 128 tiles than CUs, those in min(2 CUs / tiles, 3)
//     splits; else the round model's tile, unsplit;
//   * up to 5 CUs tiles of 64 x 64: that tile, residual projections split
//     into min(CUs / tiles, 6, blocks / 4) (5 -> 4); when the workgroups
//     (tiles x splits) leave each CU at most one, two groups of 4 waves share
//     each tile's k-blocks (below);
//   * else the round model's large tile (unchanged at the 650M 8192-token
//     shapes).
// ESM-2 35M at 2552 tokens (8 ragged sequences), against the register-staged
// kernel and 128 x 160 before: QKV 17.3 -> 14.4, Wo 8.9 -> 8.2, FC1 24.8 ->
// 20.1, FC2 20.8 -> 21.3 us, and Wo and FC2 no longer leave 3 splits each to
// the LayerNorm after them.
bool gemm_lds_plan(const DevMatrix &W, int a_fmt, int M, int epi, size_t part_floats, LdsPlan &p) {
    p = LdsPlan();
    if (a_fmt != AF_H2 || (W.fmt != WF_Q8 && W.fmt != WF_Q4 && W.fmt != WF_F16P) || !W.q16 || W.K % 32 || W.K <= 0 ||
        W.N <= 0 || W.kx % 32)
        return false;
    if (epi != EPI_NONE && epi != EPI_RESIDUAL && epi != EPI_GELU_H2 && !(epi == EPI_GELU && W.kx)) return false;
    if (M < 64) return false;  // fewer rows: the register-staged kernel (and its splits) is as fast or faster
    const char *le = getenv("CIH_GEMM_LDS"), *pe = getenv("CIH_GEMM_PLAN"), *ke = getenv("CIH_SPLITK");
    if (le || (pe && !strcmp(pe, "0"))) return false;  // CIH_GEMM_LDS=0 / force: the routes without the plan
    const long cus = device_cus();
    const long t64 = (long)((M + 63) / 64) * ((W.N + 63) / 64), t128 = (long)((M + 127) / 128) * ((W.N + 127) / 128);
    const int KB = W.K / 32;
    const bool can_split = epi == EPI_RESIDUAL && part_floats > 0 && !(ke && !strcmp(ke, "0"));
    int tile, S = 1;
    if (const int forced = tile_env(epi)) {
        tile = forced;
    } else if (can_split && KB >= 160 && t128 * 256 > 25 * cus) {
        if (t128 * 256 <= 100 * cus) {
            tile = LDS_TILE_64x128;
            S = 3;
        } else if (t128 < cus) {
            tile = LDS_TILE_128x128;
            S = (int)std::min<long>(2 * cus / t128, 3);
        } else {
            tile = tile_choice(M, W.N, true);
        }
    } else if (t64 <= 5 * cus) {
        tile = LDS_TILE_64x64;
        if (can_split) {
            S = (int)std::max<long>(1, std::min<long>({cus / t64, 6, KB / 4}));
            if (S == 5) S = 4;
        }
    } else {
        tile = tile_choice(M, W.N, true);
    }
    // a pair copy (W.kx): the 64-row tiles and 128 x 320 (the others keep the
    // register-staged pair path)
    if (W.kx && tile != LDS_TILE_64x64 && tile != LDS_TILE_64x128 && tile != LDS_TILE_128x320) return false;
    while (S > 1 && (size_t)S * M * W.N > part_floats) S--;
    if (S > 1) {
        p.kps = (KB + S - 1) / S;
        S = (KB + p.kps - 1) / p.kps;
    }
    p.tile = tile;
    p.splits = S;
    if (tile == LDS_TILE_64x128) {
        // the 64 x 128 tile (deep residual projections in 3 splits) likewise
        const long wg = (long)((M + 63) / 64) * ((W.N + 127) / 128) * S;
        int kw = wg <= cus && (S > 1 ? p.kps : KB) >= 4 ? 2 : 1;
        if (ke && !strcmp(ke, "0")) kw = 1;
        if (const char *we = getenv("CIH_GEMM_KW")) kw = atoi(we) >= 2 ? 2 : 1;
        p.kw = kw;
    }
    if (tile == LDS_TILE_64x64) {
        // Two groups of 4 waves on each 64 x 64 tile when the workgroups
        // leave each CU at most one (a lone 4-wave workgroup has one wave per
        // SIMD).  ESM-2 650M Q8_0 forwards, one sequence: L = 130 2.61 -> 2.26
        // ms, L = 66 2.40 -> 2.08, L = 402 4.06 -> 3.97; 150M B = 2 L = 100
        // 1.50 -> 1.41; 8M FP32 L = 256 0.377 -> 0.368.  More workgroups than
        // CUs (35M B = 8 ragged: Wo, FC2 at 328 tiles) gain nothing or lose:
        // a CU that runs two tiles moves the same operands through its LDS
        // either way.  Four groups: equal or slower everywhere.  The groups
        // regroup the k-sum as a split does, so CIH_SPLITK=0 keeps one group
        // (CIH_GEMM_KW=1, 2 or 4 sets the count).
        const long wg = t64 * S;
        const int kb = S > 1 ? p.kps : KB;
        int kw = wg <= cus && kb >= 4 ? 2 : 1;  // two blocks per group at least
        if (ke && !strcmp(ke, "0")) kw = 1;
        if (const char *we = getenv("CIH_GEMM_KW")) kw = atoi(we) == 4 ? 4 : (atoi(we) == 2 ? 2 : 1);
        p.kw = kw;
    }
    return true;
}

hipError_t launch_gemm_lds_plan(const DevMatrix &W, const void *X, const float *bias, void *Y, int ldy, int M, int epi,
                                const LdsPlan &p, const PartialBuf *pb, hipStream_t st) {
    if ((W.fmt != WF_Q8 && W.fmt != WF_Q4 && W.fmt != WF_F16P) || !W.q16 || W.K % 32 || W.K <= 0 || M <= 0 ||
        W.N <= 0 || !p.tile || W.kx % 32 || (W.kx && 2 * W.kx != W.K))
        return hipErrorInvalidValue;
    if (p.splits > 1) {
        if (epi != EPI_RESIDUAL || !pb || !pb->part || p.kps <= 0 || (size_t)p.splits * M * W.N > pb->floats ||
            (p.splits - 1) * p.kps >= W.K / 32)
            return hipErrorInvalidValue;
        return launch_split(W, X, M, pb->part, p.splits, p.kps, p.tile, p.kw, st);
    }
    if (epi == EPI_GELU_H2 && W.N % 32) return hipErrorInvalidValue;
    switch (epi) {
    case EPI_NONE: return launch_epi<EPI_NONE>(W, X, bias, Y, ldy, M, st, QkvOut(), p.tile, p.kw);
    case EPI_RESIDUAL: return launch_epi<EPI_RESIDUAL>(W, X, bias, Y, ldy, M, st, QkvOut(), p.tile, p.kw);
    case EPI_GELU_H2: return launch_epi<EPI_GELU_H2>(W, X, bias, Y, ldy, M, st, QkvOut(), p.tile, p.kw);
    case EPI_GELU: return launch_epi<EPI_GELU>(W, X, bias, Y, ldy, M, st, QkvOut(), p.tile, p.kw);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm_lds(const DevMatrix &W, const void *X, const float *bias, void *Y, int ldy, int M, int epi,
                           hipStream_t st, const QkvOut *qo) {
    if ((W.fmt != WF_Q8 && W.fmt != WF_Q4) || W.K % 32 || W.K <= 0 || M <= 0 || W.N <= 0) return hipErrorInvalidValue;
    if (epi == EPI_GELU_H2 && W.N % 32) return hipErrorInvalidValue;
    if (epi >= EPI_QKV16) {
        const int hd = epi == EPI_QKV16 ? 16 : (epi == EPI_QKV32 ? 32 : 64);
        if (!qo || !qo->img || !qo->pk || !qo->pos || qo->d <= 0 || qo->d % 32 || W.N != 3 * qo->d ||
            qo->d != qo->H * hd)
            return hipErrorInvalidValue;
    }
    switch (epi) {
    case EPI_NONE: return launch_epi<EPI_NONE>(W, X, bias, Y, ldy, M, st, QkvOut(), 0);
    case EPI_RESIDUAL: return launch_epi<EPI_RESIDUAL>(W, X, bias, Y, ldy, M, st, QkvOut(), 0);
    case EPI_GELU_H2: return launch_epi<EPI_GELU_H2>(W, X, bias, Y, ldy, M, st, QkvOut(), 0);
    case EPI_QKV16: return launch_epi<EPI_QKV16>(W, X, bias, Y, ldy, M, st, *qo, 0);
    case EPI_QKV32: return launch_epi<EPI_QKV32>(W, X, bias, Y, ldy, M, st, *qo, 0);
    case EPI_QKV64: return launch_epi<EPI_QKV64>(W, X, bias, Y, ldy, M, st, *qo, 0);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_expand_f16(const DevMatrix &W, unsigned short *q16, hipStream_t st) {
    if (W.fmt != WF_Q8 && W.fmt != WF_Q4) return hipErrorInvalidValue;
    const int64_t blocks = (int64_t)(W.K / 32) * W.N;
    if (blocks == 0) return hipSuccess;
    const unsigned grid = (unsigned)((blocks * 32 + 255) / 256);
    if (W.fmt == WF_Q8)
        hipLaunchKernelGGL(k_expand_f16<WF_Q8>, dim3(grid), dim3(256), 0, st,
                           reinterpret_cast<const unsigned char *>(W.q), q16, blocks);
    else
        hipLaunchKernelGGL(k_expand_f16<WF_Q4>, dim3(grid), dim3(256), 0, st,
                           reinterpret_cast<const unsigned char *>(W.q), q16, blocks);
    return hipGetLastError();
}

}  // namespace cih
