"""cih_matmul_tiled_noalloc (device pointers, scratch in a fixed device array,
no allocation) against cih_matmul_tiled (host pointers, freshly allocated
scratch) through the C ABI: bit-identical outputs on two calls in a row, the
second one smaller, for FP32, Q8_0 and Q4_0 weights on the GEMV (a few rows),
the k-split GEMM and the unsplit GEMM; a matrix above the scratch capacity is
rejected with CIH_ERR_CAPACITY before anything runs."""
import ctypes

import numpy as np
import pytest

import codon_hip as ch
from codon_hip import _lib as C
from codon_hip.devmem import Hip

pytestmark = pytest.mark.gpu


def weights(rng, dtype, N, K):
    w = (rng.standard_normal(N * K) * 0.05).astype(np.float32)
    if dtype == ch.DTYPE_Q8_0:
        return ch.quantize_slice_to_q8(w)
    if dtype == ch.DTYPE_Q4_0:
        return ch.quantize_slice_to_q4(w)
    return w


def noalloc(hip, dtype, x, w, bias, K, N, M):
    """One call through the C ABI with device buffers; returns the output."""
    d_x, d_w, d_b, d_o = hip.malloc(x.nbytes), hip.malloc(w.nbytes), hip.malloc(bias.nbytes), hip.malloc(M * N * 4)
    try:
        hip.h2d(d_x, x)
        hip.h2d(d_w, w)
        hip.h2d(d_b, bias)
        hip.memset(d_o, 0xFF, M * N * 4)  # NaN pattern: every output must be written
        rc = C.lib().cih_matmul_tiled_noalloc(dtype, ctypes.c_void_p(d_o), ctypes.c_void_p(d_x), ctypes.c_void_p(d_w),
                                              ctypes.c_void_p(d_b), K, N, M, None)
        C.check(rc)
        hip.sync()
        out = np.empty((M, N), np.float32)
        hip.d2h(out, d_o)
        return out
    finally:
        for p in (d_x, d_w, d_b, d_o):
            hip.free(p)


@pytest.mark.parametrize("dtype", [ch.DTYPE_FP32, ch.DTYPE_Q8_0, ch.DTYPE_Q4_0])
@pytest.mark.parametrize("shapes", [((5, 1280, 1280), (3, 640, 640)),        # GEMV with k-splits, then smaller
                                    ((300, 1280, 5120), (40, 640, 1280)),    # unsplit GEMM, then k-split GEMM
                                    ((40, 2560, 1280), (8, 1280, 320))])     # k-split GEMM, then GEMV
def test_noalloc_matches_matmul_tiled(dtype, shapes):
    rng = np.random.default_rng(1000 + dtype)
    hip = Hip()
    for M, K, N in shapes:
        x = rng.standard_normal((M, K)).astype(np.float32)
        w = weights(rng, dtype, N, K)
        bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
        print(f"noalloc dtype={dtype} M={M} K={K} N={N}", flush=True)
        got = noalloc(hip, dtype, x, w, bias, K, N, M)
        ref = ch.matmul_tiled(dtype, x, w, bias, K, N)
        assert np.array_equal(got.view(np.uint32), np.asarray(ref, np.float32).reshape(M, N).view(np.uint32)), \
            (dtype, M, K, N, float(np.nanmax(np.abs(got - ref))))


def test_noalloc_rejects_oversized_matrix():
    """A 4096 x 4096 FP32 matrix (64 MiB repacked) exceeds the 32 MiB weight
    scratch: CIH_ERR_CAPACITY, checked before any device work."""
    hip = Hip()
    K = N = 4096
    d = hip.malloc(16)
    try:
        rc = C.lib().cih_matmul_tiled_noalloc(ch.DTYPE_FP32, ctypes.c_void_p(d), ctypes.c_void_p(d),
                                              ctypes.c_void_p(d), ctypes.c_void_p(d), K, N, 1, None)
        assert rc == -3, rc
        assert b"scratch" in C.lib().cih_last_error()
    finally:
        hip.free(d)
