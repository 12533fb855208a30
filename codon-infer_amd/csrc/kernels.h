// Internal launch interface of the gfx950 kernels (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "x3.h"

namespace cih {

// Weight formats of the device-resident matrices.  All use a k-block-major
// layout so that one 32-wide k-block of BN consecutive output rows is a
// single contiguous span (coalesced loads for both the MFMA GEMM and GEMV):
//   F32: w  [K/32][N][32] float
//   Q8 : qs [K/32][N][32] int8,   sc [K/32][N] float
//   Q4 : qs [K/32][N][16] uint8,  sc [K/32][N] float   (reference nibble order)
// WF_F16P: FP32 weights as two f16 limbs per 32-wide block scale (the pair
// copy of an FP32 matrix, p16/psc below): block kb of K holds hi(w / d), block
// KB + kb lo(w / d), so the quantized GEMM multiplies [X | X] by [Whi | Wlo].
enum WFmt { WF_F32 = 0, WF_Q8 = 1, WF_Q4 = 2, WF_F16P = 3 };

// GEMM epilogue applied to v = acc + bias[n]; EPI_GELU_X3 / EPI_GELU_H2 write
// gelu(v) in the limb formats of x3.h (for the next quantized GEMM).
// EPI_QKV16/32/64 (LDS GEMM only): the QKV projection of heads of 16/32/64
// dims; Q columns go to Y as FP32, K (rotated) and V columns to the tile
// images of kv_image.h described by a QkvOut.
enum Epi {
    EPI_NONE = 0,
    EPI_GELU = 1,
    EPI_RESIDUAL = 2,
    EPI_GELU_X3 = 3,
    EPI_GELU_H2 = 4,
    EPI_QKV16 = 5,
    EPI_QKV32 = 6,
    EPI_QKV64 = 7
};

// Destination of the K/V columns of an EPI_QKV* projection.
struct QkvOut {
    const int *pk = nullptr;   // [T] padded key index of each packed token: 32 * tile row + slot
    const float *rc = nullptr; // RoPE cos / sin tables [max_len][hd/2]
    const float *rs = nullptr;
    const int *pos = nullptr;  // [T] position of each token in its sequence
    unsigned char *img = nullptr;
    int d = 0, H = 0;
};

// erf_f32 (src/lib.rs:3485-3491, Abramowitz & Stegun 7.1.26, |error| <= 1.5e-7)
// and gelu(x) = 0.5 x (1 + erf(x / sqrt 2)) (src/lib.rs:3493-3498).  Same
// polynomial; t = 1 / (1 + p|x|) by the hardware reciprocal (<= 1 ulp) and
// exp(-x^2) as 2^(-x^2 log2 e) by the hardware exponential instead of the
// correctly rounded division and libm exp: a few ulp of erf, against the
// approximation's own 1.5e-7.
__device__ __forceinline__ float erf_as(float x) {
    const float sign = x < 0.0f ? -1.0f : 1.0f;
    const float ax = fabsf(x);
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * ax);
    const float e = __builtin_amdgcn_exp2f(-ax * ax * 1.44269504088896340736f);
    const float y =
        1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) *
                   t * e;
    return sign * y;
}
__device__ __forceinline__ float gelu_as(float x) { return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752440f)); }

// Sum of S partial results p[0], p[stride], ... in split order (twenty loads
// in flight, then added one by one): the same bits whatever launched the
// splits.  fold_splits4: the same for four consecutive floats (16-byte loads).
constexpr int FOLD_CHUNK = 20;
__device__ __forceinline__ float fold_splits(const float *__restrict__ p, int S, size_t stride) {
    float acc = 0.0f;
    for (int s0 = 0; s0 < S; s0 += FOLD_CHUNK) {
        float v[FOLD_CHUNK];
#pragma unroll
        for (int u = 0; u < FOLD_CHUNK; u++) v[u] = s0 + u < S ? p[(size_t)(s0 + u) * stride] : 0.0f;
#pragma unroll
        for (int u = 0; u < FOLD_CHUNK; u++) acc += v[u];
    }
    return acc;
}
typedef float fold4_t __attribute__((ext_vector_type(4)));
// Mean and variance of one row of n4 quads held in LDS, formed by one wave:
// lane l sums quads l, l + 64, ... in order, then a butterfly (the
// reduction order of k_layernorm4, shared by every kernel that normalises a
// row of the residual stream so that all of them give the same bits).
__device__ __forceinline__ void row_stats64(const fold4_t *xs, int n4, int d, int lane, float &mean, float &var) {
    float s = 0.0f;
    for (int c = lane; c < n4; c += 64) s += (xs[c].x + xs[c].y) + (xs[c].z + xs[c].w);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    mean = s / (float)d;
    float q = 0.0f;
    for (int c = lane; c < n4; c += 64) {
        const fold4_t t = xs[c] - mean;
        q += (t.x * t.x + t.y * t.y) + (t.z * t.z + t.w * t.w);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o);
    var = q / (float)d;
}
// (CH loads in flight at a time: fewer registers for kernels that fold many
// column quads per lane; the additions stay in split order)
template <int CH = FOLD_CHUNK>
__device__ __forceinline__ fold4_t fold_splits4(const float *__restrict__ p, int S, size_t stride) {
    fold4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < S; s0 += CH) {
        fold4_t v[CH];
#pragma unroll
        for (int u = 0; u < CH; u++)
            v[u] = s0 + u < S ? *reinterpret_cast<const fold4_t *>(p + (size_t)(s0 + u) * stride)
                              : fold4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < CH; u++) acc += v[u];
    }
    return acc;
}

struct DevMatrix {
    int fmt = WF_F32;
    int N = 0, K = 0;          // out_dim, in_dim
    const void *q = nullptr;   // F32 values or packed quants
    const float *sc = nullptr; // per-block scales (quantized formats)
    // Optional copy of the quants as f16 integers, [K/32][N][32] (element
    // order of the block, Q4_0 nibbles already minus 8): the operand of the
    // LDS-staged GEMM.  Same values as q, so the same products.
    const unsigned short *q16 = nullptr;
    // Optional pair copy of an FP32 matrix: p16 [2K/32][N][32] f16 (blocks
    // 0..K/32-1: hi = f16(w / d), blocks K/32..: lo = f16(w / d - hi)), psc
    // [2K/32][N] the power-of-two block scales d (stored for both halves).
    // hi + lo keeps 22 significant bits of w; the f16-MFMA GEMM takes it
    // instead of FP32 MFMA (CIH_QGEMM=fp32 or full range: the FP32 kernel).
    const unsigned short *p16 = nullptr;
    const float *psc = nullptr;
    // Activation length when it differs from K: a pair copy handed to the
    // LDS-staged GEMM as an f16 matrix of K = 2 kx (weight block kb meets
    // activation block kb mod kx / 32); 0: the activations have K elements.
    int kx = 0;
};

// Workgroup -> output tile: consecutive workgroup ids go to the 8 XCDs in
// turn, so each XCD receives a contiguous range of tiles, ordered GROUP_M row
// tiles deep so that the tiles resident on one XCD share rows and columns in
// its L2.
__device__ __forceinline__ void tile_xcd(int bid, int total, int nM, int nN, int &mt, int &nt) {
    constexpr int XCD = 8, GROUP_M = 8;
    const int xcd = bid % XCD, local = bid / XCD;
    const int per = total / XCD, rem = total % XCD;
    const int id = (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
    const int in_group = GROUP_M * nN;
    const int g = id / in_group;
    const int first = g * GROUP_M;
    const int gsize = min(nM - first, GROUP_M);
    const int r = id % in_group;
    mt = first + r % gsize;
    nt = r / gsize;
}

// Y = epi(sum over s < S of part[s][M][N] + bias), splits in order (the
// reduction of the split-K GEMMs).
hipError_t launch_splitk_reduce(const float *part, int S, int M, int N, const float *bias, void *Y, int ldy, int epi,
                                hipStream_t st);

// Compute units of the current device (queried once; 256 if the query fails).
int device_cus();

// Device buffer for partial sums of k-split GEMMs and GEMVs (one stream uses
// it at a time).  A split-K GEMM needs at most SPLITK_PART_FLOATS floats.
struct PartialBuf {
    float *part = nullptr;
    size_t floats = 0;
};
constexpr size_t SPLITK_PART_FLOATS = (size_t)1024 * 64 * 64;

// Y[M][N] (row stride ldy) = epi(X[M][K] * W^T + bias).  X is FP32 with row
// stride ldx (a_fmt AF_F32) or in a limb format of x3.h (AF_X3 / AF_H2,
// quantized W only).  With pb, a GEMM too small to fill the GPU splits K
// (CIH_SPLITK=0 disables).  defer (may be null): a split GEMM of the f16-limb
// kernel leaves its [*defer][M][N] partial sums in pb for the caller to add
// (with bias and epilogue: the residual LayerNorm); *defer = 0 when the
// output was written.
hipError_t launch_gemm(const DevMatrix &W, const void *X, int ldx, int a_fmt, const float *bias, void *Y,
                       int ldy, int M, int epi, const PartialBuf *pb, hipStream_t st, int *defer = nullptr);

// Q8_0/Q4_0 GEMM on bf16 MFMA: exact integer weights, activations split
// into three bf16 limbs (FP32-equivalent products), block scale in FP32.
hipError_t launch_gemm_x3(const DevMatrix &W, const void *X, int ldx, int a_fmt, const float *bias, void *Y,
                          int ldy, int M, int epi, const PartialBuf *pb, hipStream_t st, int *defer = nullptr);

// Weight-streaming GEMV for M <= GEMV_MAX_M tokens (FP32 activations, epilogue
// EPI_NONE / EPI_GELU / EPI_RESIDUAL).  With several k-splits the partial sums
// go through pb ([splits][M][N] floats) and a second kernel.
constexpr int GEMV_MAX_M = 8;
// 64-column groups, k-splits, k-blocks per wave (a split is 4 waves x nb blocks)
struct GemvGrid { int cols = 0, splits = 0, nb = 0; };
GemvGrid gemv_grid(int N, int K);
size_t gemv_part_floats(int N, int K);  // partial-sum floats needed at M = GEMV_MAX_M
hipError_t launch_gemv(const DevMatrix &W, const float *X, int ldx, int M, const float *bias, float *Y, int ldy,
                       int epi, const PartialBuf &pb, hipStream_t st);
// The GEMV without its reduction: pb receives [*splits][M][N] partial sums
// (no bias) for a consumer that adds them itself.
hipError_t launch_gemv_partials(const DevMatrix &W, const float *X, int ldx, int M, const PartialBuf &pb, int *splits,
                                hipStream_t st);

// Few-token quantized GEMM on f16 MFMA: X (M <= GEMV_MAX_M rows) in H2 limbs
// ([M][K/32][64] f16), W Q8_0 / Q4_0 with N % 16 == 0; workgroups of 64
// columns and kw k-blocks, K split across `splits` workgroups.  CIH_GEMV16=0:
// gemv16_applies is false.
bool gemv16_applies(const DevMatrix &W, int a_fmt, int M, int epi);
struct Gemv16Grid { int kw = 0, splits = 0; };
constexpr size_t GEMV16_SPLIT_MAX_FLOATS = (size_t)1 << 21;
Gemv16Grid gemv16_grid(int N, int K);
// partial sums [*splits][M][N] (no bias) for a consumer that adds them in split order
hipError_t launch_gemv16_partials(const DevMatrix &W, const unsigned short *X, int M, float *part, size_t part_floats,
                                  int *splits, hipStream_t st);
// The residual LayerNorm of one row folded into the projection after it:
// x' = x + rbias + (sum of the rS splits of rpart, [rS][K]) is stored to xo
// (not x), and the activations are LayerNorm(x') with lnw, lnb, formed in
// every workgroup with k_rln's arithmetic (the same bits as k_rln followed by
// launch_gemv16_partials).  rpart == nullptr: x' = x.  K <= GEMV16_LN_MAX_K.
constexpr int GEMV16_LN_MAX_K = 2048;
struct LnIn {
    const float *x;
    float *xo;
    const float *w, *b;
};
hipError_t launch_gemv16_ln_partials(const DevMatrix &W, const float *x, float *xo, const float *rpart, int rS,
                                     const float *rbias, const float *lnw, const float *lnb, float *part,
                                     size_t part_floats, int *splits, hipStream_t st);
// the same with activations GELU(sum of the aS splits of apart + abias) formed
// while staging (apart: [aS][M][W.K], the FC1 projection's partial sums)
hipError_t launch_gemv16_gelu_partials(const DevMatrix &W, const float *apart, int aS, const float *abias, int M,
                                       float *part, size_t part_floats, int *splits, hipStream_t st);
// Y = epi(sum of the S splits of part + bias): EPI_NONE / EPI_RESIDUAL / EPI_GELU
// (FP32 Y, row stride ldy) or EPI_GELU_H2 (Y in H2 limbs, N columns)
hipError_t launch_gemv16_fold(const float *part, int S, int M, int N, const float *bias, void *Y, int ldy, int epi,
                              hipStream_t st);
// the whole GEMM: partials in pb and the fold, or (more than
// GEMV16_SPLIT_MAX_FLOATS partial sums) one workgroup per 64 columns over the
// whole K with the epilogue applied there
hipError_t launch_gemv16(const DevMatrix &W, const unsigned short *X, int M, const float *bias, void *Y, int ldy,
                         int epi, const PartialBuf *pb, hipStream_t st);
// FP32 [M][K] (16-byte aligned, K % 32 == 0) -> H2 limbs [M][K/32][64]
hipError_t launch_to_h2(const float *x, int M, int K, unsigned short *out, hipStream_t st);

// The same GEMM for activations in f16 limbs (AF_H2), with operands copied
// global -> LDS by the load unit (no staging registers), W read from W.q16
// or, without it, from the quants.  Epilogues EPI_NONE / EPI_RESIDUAL /
// EPI_GELU_H2 (and the QKV image epilogues).  With W.q16, launch_gemm_x3
// routes f16-limb calls of 64 rows and more by gemm_lds_plan (below);
// otherwise gemm_lds_applies says whether it routes a call here: the shape
// must give at least one full round of 128x128 tiles (smaller problems keep
// the split-K path).  CIH_GEMM_LDS=0 never, =force whenever the formats
// allow (tile: CIH_GEMM_TILE_N or the round model).
bool gemm_lds_applies(const DevMatrix &W, int a_fmt, int M, int epi);
hipError_t launch_gemm_lds(const DevMatrix &W, const void *X, const float *bias, void *Y, int ldy, int M, int epi,
                           hipStream_t st, const QkvOut *qo = nullptr);
// Split-K form for shapes whose 128 x 128 tiles do not fill one round (32 to
// 255 tiles; EPI_NONE / EPI_RESIDUAL, whose caller adds the splits): raw
// partial sums X * W^T over k-ranges into pb.part as [S][M][N], *splits = S
// (0: no split fits, nothing launched).
bool gemm_lds_split_applies(const DevMatrix &W, int a_fmt, int M, int epi);
hipError_t launch_gemm_lds_split(const DevMatrix &W, const void *X, int M, const PartialBuf &pb, int *splits,
                                 hipStream_t st);
// Workgroup tiles of the LDS-staged GEMM (BM x BN).
enum LdsTileId { LDS_TILE_128x128 = 1, LDS_TILE_128x160, LDS_TILE_128x256, LDS_TILE_128x320, LDS_TILE_64x128, LDS_TILE_64x64 };
// Tile and k-splits for an f16-limb GEMM with the f16 copy from 64 rows on
// (false: not such a GEMM, or CIH_GEMM_LDS / CIH_GEMM_PLAN=0 set).  Splits
// only for EPI_RESIDUAL with room for them (part_floats > 0; the caller
// adds them, as launch_gemm_lds_split's).  kw: groups of 4 waves that share
// a 64 x 64 tile's k-blocks (1, 2 or 4).
struct LdsPlan {
    int tile = 0, splits = 1, kps = 0, kw = 1;
};
bool gemm_lds_plan(const DevMatrix &W, int a_fmt, int M, int epi, size_t part_floats, LdsPlan &p);
// The planned GEMM: with p.splits > 1 the raw partial sums [p.splits][M][N]
// into pb->part (bias and epilogue left to the caller), else Y = epi(...).
hipError_t launch_gemm_lds_plan(const DevMatrix &W, const void *X, const float *bias, void *Y, int ldy, int M, int epi,
                                const LdsPlan &p, const PartialBuf *pb, hipStream_t st);
// W.q16 from W.q (quantized W, k-block-major), on stream st.
hipError_t launch_expand_f16(const DevMatrix &W, unsigned short *q16, hipStream_t st);
// The pair copy (p16, psc) of an FP32 matrix W, on stream st.
hipError_t launch_pair_f16(const DevMatrix &W, unsigned short *p16, float *psc, hipStream_t st);

// Dequantizes nblocks of a device matrix in k-block-major layout back to the
// reference's row-major [N][K] FP32 (test path).
hipError_t launch_dequant(const DevMatrix &W, float *out, hipStream_t st);

// Weight residency.  src: a [N][K] matrix in the reference's row-major
// layout (FP32 values, or packed 36-byte Q8_0 / 20-byte Q4_0 blocks; src_fmt
// a WFmt) in device memory, 4-byte aligned.  Writes rows [n_off, n_off + N)
// of dst (k-block-major, dst.K = K).  src_fmt == dst.fmt repacks the bytes
// unchanged; FP32 into Q8_0 / Q4_0 quantizes (bit-exact with the reference's
// quantizers).
hipError_t launch_load_matrix(const uint8_t *src, int src_fmt, int N, const DevMatrix &dst, int n_off, hipStream_t st);

// n floats from src + src_bytes to dst + dst_bytes, one workgroup per segment
// (segs in device memory).
struct CopySeg {
    int64_t src, dst, n;
};
hipError_t launch_copy_segments(const uint8_t *src, uint8_t *dst, const CopySeg *segs, int count, hipStream_t st);

struct SeqMeta {
    const int *cu;    // [B] first packed row of each sequence
    const int *lens;  // [B] tokens per sequence
    int B, S_max;
};

// Bits of a forward's device status word (one int, cleared before the
// forward, read after it).
constexpr int FLAG_BAD_TOKEN = 1;  // a token id outside [0, V) (device-pointer input)
// FLAG_NONFINITE: a LayerNorm row with a non-finite mean or variance, or (in a
// LayerNorm given the flag) an output the f16 limbs of the GEMM it feeds cannot
// hold: |y| >= 65520 rounds to an infinite hi limb.
constexpr int FLAG_NONFINITE = 2;

// Flags a LayerNorm output that is not finite or lies beyond the f16 limbs'
// range (no-op without a status word).
__device__ __forceinline__ void flag_limb_range(int *flag, float y) {
    if (flag && !(__builtin_fabsf(y) < 65520.0f)) atomicOr(flag, FLAG_NONFINITE);
}

// Few-token forward (few.hip).  x += pbias + (sum of the S splits of part,
// [S][rows][d]; part may be null), then out = LayerNorm(x) as FP32 or H2
// limbs; flag as launch_layernorm.
hipError_t launch_residual_layernorm(float *x, const float *part, int S, const float *pbias, const float *w,
                                     const float *b, void *out, int out_fmt, int rows, int d, hipStream_t st,
                                     int *flag = nullptr);
// Attention of T <= GEMV_MAX_M packed tokens from the QKV projection's splits
// (part [S][T][3d]) + bias: RoPE, softmax(q k / sqrt(hd)) v in FP32 per
// (sequence, head); out [T][d] in FP32 or H2 limbs.  hd % 8 == 0, <= FEW_MAX_HD.
constexpr int FEW_MAX_HD = 128;
hipError_t launch_attention_few(const float *part, int S, int T, const float *bias, int d, int H, const SeqMeta &sm,
                                const float *rope_c, const float *rope_s, void *out, int out_fmt, hipStream_t st);
// The same attention followed by each head's share of the output projection
// Wo (Q8_0 / Q4_0, K = d, hd a multiple of 32): partial sums per head into
// opart [H][T][Wo.N] (the caller adds the H splits and Wo's bias).
hipError_t launch_attention_few_wo(const float *part, int S, int T, const float *bias, const DevMatrix &Wo, int d,
                                   int H, const SeqMeta &sm, const float *rope_c, const float *rope_s, float *opart,
                                   size_t opart_floats, hipStream_t st);

// Full-range mode: quantized GEMMs take three bf16 limbs and attention the
// FP32-MFMA kernel, which cover the whole FP32 exponent range (the f16 limbs
// of the default path need |x| < 65504).  A forward whose residual stream
// turned non-finite is run again in it.  Thread-local; set by the host
// around that one forward.
bool full_range_mode();

// Embedding + token-dropout rescale, packed rows.  flag (may be null):
// FLAG_BAD_TOKEN is set for an id outside [0, V), which is clamped.
hipError_t launch_embed(const int *tokens, SeqMeta sm, int emb_fmt, const void *emb_q,
                        const float *emb_sc, int d, int V, float *x, hipStream_t st, int *flag = nullptr);

// out = LayerNorm(x) over rows of width d (eps 1e-5); out_fmt AF_F32, AF_X3
// or AF_H2.  flag (may be null): FLAG_NONFINITE is set when a row's mean or
// variance is not finite (the row holds an inf or NaN) or an output is not
// finite or reaches 65520 in magnitude (beyond the f16 limbs of the GEMM that
// reads it).
hipError_t launch_layernorm(const float *x, const float *w, const float *b, void *out, int out_fmt, int rows,
                            int d, hipStream_t st, int *flag = nullptr);

// Bidirectional rotary attention over packed Q|K|V rows.  When P != nullptr
// every softmax row is stored at P[b*pb + h*ph + q*S_max + k]; rowsum (with
// P) receives rowsum[b][h][q] = sum of row q over the residue keys 1..len-2,
// for residue queries.
// out: [T][d] FP32 (out_fmt AF_F32) or a limb format (AF_X3 / AF_H2).
// Without P, tasks that would leave workgroup slots idle are split over key
// ranges whose partial results (part, part_floats floats; nullptr: no split)
// a merge kernel combines; attention_part_floats(hd) floats always suffice.
hipError_t launch_attention(const float *qkv, int d, int H, SeqMeta sm, const float *rope_cos,
                            const float *rope_sin, void *out, int out_fmt, float *P, int64_t pb, int64_t ph,
                            float *rowsum, float *part, size_t part_floats, hipStream_t st);
size_t attention_part_floats(int hd);

// The same attention with K and V taken from the tile images of kv_image.h
// (written by an EPI_QKV* projection; Q still from qkv's Q columns).  tb: [B]
// first tile row of each sequence.  hd 16, 32 or 64.
hipError_t launch_attention_img(const float *qkv, int d, int H, SeqMeta sm, const int *tb, const unsigned char *img,
                                const float *rope_cos, const float *rope_sin, void *out, int out_fmt, float *P,
                                int64_t pb, int64_t ph, float *rowsum, float *part, size_t part_floats, hipStream_t st);

// Per-forward set-up of the tile images: tb[b] = first tile row of sequence
// b, pk / pos of every packed token, ti[tile row] = (first packed row, keys,
// first position, sequence), and the padding keys of each sequence's last
// tile zeroed in every head's image (so masked keys multiply finite zeros).
hipError_t launch_kv_setup(SeqMeta sm, int hd, int H, int *tb, int *pk, int *pos, int *ti, unsigned char *img,
                           hipStream_t st);
// Tile images from FP32 Q|K|V rows (any projection), tile_rows = sum over
// sequences of ceil(len / 32); after launch_kv_setup (reads its ti).  Same
// bytes as the EPI_QKV* epilogue.
hipError_t launch_kv_prep(const float *qkv, int d, int H, const int *ti, int tile_rows, const float *rope_cos,
                          const float *rope_sin, unsigned char *img, hipStream_t st);
bool attention_img_supported(int hd);
// Whether attention of B sequences (at most S_max tokens, H heads) runs each
// 32-query task on 8 waves that split its keys (k_attention_xs, staging K/V
// from FP32 rows): when those tasks fit one round of one workgroup per CU,
// unless CIH_ATT_SPLIT=0 or CIH_SPLITK=0.
bool attention_wave_split(int B, int S_max, int H);
size_t kv_image_bytes(int hd);  // bytes of one (tile row, head) image

// final_att[b][p][t] = sum_h P_h[p][t] * (1/H), h ascending
hipError_t launch_head_mean(const float *P, int64_t pb, int64_t ph, int H, SeqMeta sm, float *final_att,
                            hipStream_t st);

// Contacts (APC).  For layer l, heads with w != 0, one read of the maps:
//   M[b][i][j] += sum_h w_lh * P_lh[i+1][j+1]
//   r[l][h][b][i] = rowsum[b][h][i+1] + sum_j P_lh[j+1][i+1]   (residues only)
// rowsum comes from launch_attention; colpart: [B][H][ceil(n_max/32)][n_max] scratch.
hipError_t launch_apc_layer(const float *P, int64_t pb, int64_t ph, int H, int l, const float *w_dev,
                            const int *heads_dev, int n_heads_nz, SeqMeta sm, const float *rowsum, float *colpart,
                            float *M, float *r, hipStream_t st);
// contacts[b][i][j] = sigmoid(M_ij + M_ji - sum_lh (w_lh / T_lh) r_i r_j + bias)
// coef: [L*H][B] scratch for w_lh / T_lh.
hipError_t launch_apc_finalize(const float *M, const float *r, float *coef, const float *w_dev, int LH, SeqMeta sm,
                               float bias, float *contacts, int n_stride, hipStream_t st);

// DMS rows (pipeline.rs:152-172): for entry i, logits row meta[2i] of the
// packed [T][V] logits and wild-type token meta[2i+1] give out[i][0..19] =
// deltas in CANONICAL_AAS order and out[i][20] = entropy.
hipError_t launch_dms_score(const float *logits, int V, const int *meta, int count, float *out, hipStream_t st);

// Autoregressive decoding.  rows: [n][2] = (cache slot, position) per row of
// qkv [n][3d]; the K/V cache holds [slot][max_len][d] floats per layer
// (slot_stride floats between slots).  launch_rope_kv rotates Q in place
// and writes the rotated K and V at the row's position; afterwards
// launch_decode_attention writes out[n][d] = causal attention of each row
// over its slot's positions 0..pos.  A row may read positions written by
// other rows of the same launch pair.
hipError_t launch_rope_kv(float *qkv, int d, int hd, const int *rows, int n, const float *rope_c, const float *rope_s,
                          float *kc, float *vc, int64_t slot_stride, hipStream_t st);
hipError_t launch_decode_attention(const float *qkv, int d, int H, const int *rows, int n, int max_len,
                                   const float *kc, const float *vc, int64_t slot_stride, float *out,
                                   hipStream_t st, int out_fmt = AF_F32);
// Both steps in one launch when every slot appears at most once among the
// rows (one new token per sequence): each (row, head) workgroup rotates its
// head's Q and K, writes K and V at pos, and attends with key pos from LDS.
// With part != nullptr the rows' Q|K|V come as [splits][n][3d] GEMV partial
// sums (launch_gemv_partials, launch_gemv16_partials) plus bias; qkv is
// unused.  out_fmt: out as FP32 rows or H2 limbs.
hipError_t launch_decode_attention_fused(float *qkv, const float *part, int splits, const float *bias, int d, int H,
                                         const int *rows, int n, int max_len, const float *rope_c,
                                         const float *rope_s, float *kc, float *vc, int64_t slot_stride, float *out,
                                         hipStream_t st, int out_fmt = AF_F32);
// The same, each head's output multiplied by its k-blocks of Wo (Q8_0 /
// Q4_0, K = d, hd 32 or 64) instead of stored: partial sums per head into
// wo_part [H][n][Wo.N] (the caller adds the H splits and Wo's bias).
hipError_t launch_decode_attention_fused_wo(float *qkv, const float *part, int splits, const float *bias, int d, int H,
                                            const int *rows, int n, int max_len, const float *rope_c,
                                            const float *rope_s, float *kc, float *vc, int64_t slot_stride,
                                            const DevMatrix &Wo, float *wo_part, size_t wo_part_floats,
                                            hipStream_t st);
size_t decode_attention_lds(int hd, int max_len);  // dynamic LDS bytes per workgroup

// Copies packed rows [T][width] into padded [B][S_max][width] (valid rows only).
hipError_t launch_scatter_rows(const float *src, int width, SeqMeta sm, float *dst, int64_t dst_b_stride,
                               hipStream_t st);

}  // namespace cih
