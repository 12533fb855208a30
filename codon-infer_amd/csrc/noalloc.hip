// cih_matmul_tiled_noalloc: the tiled matmul of cih_matmul_tiled with every
// operand in device memory and its scratch memory in a fixed device array,
// for callers that cannot allocate (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// The scratch memory is the weight matrix repacked into the library's
// k-block-major layout and the partial sums of a k-split GEMM or GEMV.  It
// lives in `scratch`, a file-scope device array: each GPU the library runs
// on holds its own copy (NOALLOC_SCRATCH_BYTES) from the time this code is
// loaded on it until the process ends.  Host code reaches a device's copy
// only through the address hipGetSymbolAddress returns with that device
// current (the array's name is a host-side stand-in, not a device address).
#include <mutex>

#include "model.h"

namespace cih {
namespace {

constexpr size_t NOALLOC_WEIGHT_BYTES = (size_t)32 << 20;  // repacked quants + scales, or FP32 values
constexpr size_t NOALLOC_PART_BYTES = SPLITK_PART_FLOATS * sizeof(float);  // 16 MiB of partial sums
constexpr size_t NOALLOC_SCRATCH_BYTES = NOALLOC_WEIGHT_BYTES + NOALLOC_PART_BYTES;

__device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
unsigned char *g_ptr[MAX_DEVICES] = {};

// The current device's copy of `scratch`, looked up once per device.
int scratch_of_current_device(unsigned char **out) {
    int dev = -1;
    HIPCHK(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) return set_error(CIH_ERR_HIP, "device %d outside [0, %d)", dev, MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        // The first call on a device may come while the caller's stream is
        // being captured into a graph (in any capture mode): the one-time
        // lookup runs with this thread's capture mode relaxed, as a library's
        // lazy initialisation must, and the caller's mode is restored.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        HIPCHK(hipThreadExchangeStreamCaptureMode(&mode));
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        HIPCHK(hipThreadExchangeStreamCaptureMode(&mode));
        HIPCHK(e);
        if (!p) return set_error(CIH_ERR_HIP, "no device address for the scratch array");
        g_ptr[dev] = static_cast<unsigned char *>(p);
    }
    *out = g_ptr[dev];
    return 0;
}

}  // namespace
}  // namespace cih

using namespace cih;

extern "C" int cih_matmul_tiled_noalloc(int32_t dtype, float *out, const float *x, const void *w, const float *bias,
                                        int32_t in_dim, int32_t out_dim, int32_t seq_len, void *stream) {
    if (!out || !x || !w || !bias) return set_error(CIH_ERR_ARG, "null argument");
    if (in_dim <= 0 || out_dim <= 0 || seq_len < 0 || in_dim % 32)
        return set_error(CIH_ERR_SHAPE, "bad GEMM shape %d x %d x %d", seq_len, out_dim, in_dim);
    if (dtype != DT_FP32 && dtype != DT_Q8 && dtype != DT_Q4) return set_error(CIH_ERR_ARG, "bad dtype");
    if (reinterpret_cast<uintptr_t>(w) % 4 || reinterpret_cast<uintptr_t>(x) % 16)
        return set_error(CIH_ERR_ARG, "w must be 4-byte and x 16-byte aligned");
    if (seq_len == 0) return CIH_OK;
    // the repacked matrix: quants then (256-byte aligned) block scales
    const size_t blocks = (size_t)(in_dim / 32) * out_dim;
    const size_t qbytes = dtype == DT_FP32 ? blocks * 32 * 4 : blocks * (block_bytes(dtype) - 4);
    const size_t sc_off = (qbytes + 255) / 256 * 256;
    const size_t wbytes_needed = sc_off + (dtype == DT_FP32 ? 0 : blocks * 4);
    if (wbytes_needed > NOALLOC_WEIGHT_BYTES)
        return set_error(CIH_ERR_CAPACITY, "a %d x %d matrix needs %zu bytes of scratch, above the %zu available",
                         out_dim, in_dim, wbytes_needed, NOALLOC_WEIGHT_BYTES);
    // the partial sums the same call of cih_matmul_tiled would have
    PartialBuf pb;
    pb.floats = std::max(gemv_part_floats(out_dim, in_dim), SPLITK_PART_FLOATS);
    if (pb.floats * sizeof(float) > NOALLOC_PART_BYTES)
        return set_error(CIH_ERR_CAPACITY, "the GEMV of a %d x %d matrix needs %zu partial sums, above %zu", out_dim,
                         in_dim, pb.floats, NOALLOC_PART_BYTES / sizeof(float));
    unsigned char *base = nullptr;
    if (int rc = scratch_of_current_device(&base)) return rc;
    DevMatrix W;
    W.fmt = dtype == DT_FP32 ? WF_F32 : (dtype == DT_Q8 ? WF_Q8 : WF_Q4);
    W.N = out_dim;
    W.K = in_dim;
    W.q = base;
    W.sc = dtype == DT_FP32 ? nullptr : reinterpret_cast<const float *>(base + sc_off);
    pb.part = reinterpret_cast<float *>(base + NOALLOC_WEIGHT_BYTES);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool g16 = dtype != DT_FP32 && gemv16_applies(W, AF_H2, seq_len, EPI_NONE);
    if (g16 && (size_t)seq_len * in_dim * sizeof(float) > NOALLOC_PART_BYTES)
        return set_error(CIH_ERR_CAPACITY, "%d rows of %d limbs need more than the %zu bytes available", seq_len,
                         in_dim, NOALLOC_PART_BYTES);
    hipError_t e = launch_load_matrix(static_cast<const uint8_t *>(w), W.fmt, out_dim, W, 0, st);
    if (e == hipSuccess && g16) {
        // as cih_matmul_tiled: limbs in the partial-sum region, then the f16-MFMA GEMV
        unsigned short *xh = reinterpret_cast<unsigned short *>(pb.part);
        e = launch_to_h2(x, seq_len, in_dim, xh, st);
        PartialBuf rest{pb.part + (size_t)seq_len * in_dim, NOALLOC_PART_BYTES / sizeof(float) - (size_t)seq_len * in_dim};
        if (e == hipSuccess) e = launch_gemv16(W, xh, seq_len, bias, out, out_dim, EPI_NONE, &rest, st);
    } else if (e == hipSuccess) {
        e = use_gemv(seq_len, AF_F32, EPI_NONE)
                ? launch_gemv(W, x, in_dim, seq_len, bias, out, out_dim, EPI_NONE, pb, st)
                : launch_gemm(W, x, in_dim, AF_F32, bias, out, out_dim, seq_len, EPI_NONE, &pb, st);
    }
    if (e != hipSuccess) return set_error(CIH_ERR_HIP, "GEMM failed: %s", hipGetErrorString(e));
    return CIH_OK;
}
