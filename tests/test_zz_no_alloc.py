"""cih_matmul_tiled_noalloc (device pointers, scratch in a fixed device array,
no allocation) against cih_matmul_tiled (host pointers, freshly allocated
scratch) through the C ABI: bit-identical outputs on two calls in a row, the
second one smaller, for FP32, Q8_0 and Q4_0 weights on the GEMV (a few rows),
the k-split GEMM and the unsplit GEMM; a matrix above the scratch capacity is
rejected with CIH_ERR_CAPACITY before anything runs; and, in a fresh process,
calls captured into a HIP graph on a non-null stream in global capture mode
(the first call's scratch lookup inside the capture), replayed twice with
eager work in between, equal cih_matmul_tiled bit for bit."""
import ctypes
import os
import subprocess
import sys

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


CAPTURE_SCRIPT = r"""
import ctypes, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
import codon_hip as ch
from codon_hip import _lib as C
from codon_hip.devmem import Hip

hip = Hip()
L = hip.L
lib = C.lib()
stream = ctypes.c_void_p()
assert L.hipStreamCreate(ctypes.byref(stream)) == 0
rng = np.random.default_rng(77)
cases = []
for dtype, M, K, N in ((ch.DTYPE_Q8_0, 300, 1280, 1280), (ch.DTYPE_Q4_0, 5, 1280, 640), (ch.DTYPE_FP32, 40, 640, 1280)):
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.05).astype(np.float32)
    w = ch.quantize_slice_to_q8(w) if dtype == ch.DTYPE_Q8_0 else (ch.quantize_slice_to_q4(w) if dtype == ch.DTYPE_Q4_0 else w)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    ref = np.asarray(ch.matmul_tiled(dtype, x, w, b, K, N), np.float32).reshape(M, N)
    bufs = [hip.malloc(a.nbytes) for a in (x, w, b)] + [hip.malloc(M * N * 4)]
    for p, a in zip(bufs, (x, w, b)):
        hip.h2d(p, a)
    cases.append((dtype, M, K, N, bufs, ref))
graphs = []
for dtype, M, K, N, (dx, dw, db, do), ref in cases:
    print(f"capture dtype={dtype} M={M} K={K} N={N}", flush=True)
    assert L.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
    rc = lib.cih_matmul_tiled_noalloc(dtype, ctypes.c_void_p(do), ctypes.c_void_p(dx), ctypes.c_void_p(dw),
                                      ctypes.c_void_p(db), K, N, M, stream)
    g = ctypes.c_void_p()
    e = L.hipStreamEndCapture(stream, ctypes.byref(g))
    assert rc == 0, (rc, lib.cih_last_error())
    assert e == 0, e
    ex = ctypes.c_void_p()
    assert L.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0) == 0
    graphs.append(ex)
for rep in range(2):
    for (dtype, M, K, N, (dx, dw, db, do), ref), ex in zip(cases, graphs):
        hip.memset(do, 0xFF, M * N * 4)  # NaN pattern, outside the graph
        assert L.hipGraphLaunch(ex, stream) == 0
        assert L.hipStreamSynchronize(stream) == 0
        got = np.empty((M, N), np.float32)
        hip.d2h(got, do)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (rep, dtype, M, K, N)
        print(f"replay {rep} dtype={dtype} M={M}: bit-identical", flush=True)
    # eager work of the program between the replays, on the null stream
    dtype, M, K, N, (dx, dw, db, do), ref = cases[0]
    assert lib.cih_matmul_tiled_noalloc(dtype, ctypes.c_void_p(do), ctypes.c_void_p(dx), ctypes.c_void_p(dw),
                                        ctypes.c_void_p(db), K, N, M, None) == 0
    hip.sync()
print("capture ok", flush=True)
"""


def test_noalloc_inside_graph_capture():
    """The point of the entry point: callers under HIP graph capture.  In a
    fresh process (so the first call's scratch lookup happens inside the
    capture), three calls (Q8_0 GEMM, Q4_0 GEMV with k-splits, FP32 k-split
    GEMM) are each captured on a created stream in global capture mode, then
    every graph is replayed twice, with an eager call on the null stream in
    between; each replay equals cih_matmul_tiled bit for bit."""
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "codon-infer_amd")
    r = subprocess.run([sys.executable, "-u", "-c", CAPTURE_SCRIPT, pkg], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "capture ok" in r.stdout
