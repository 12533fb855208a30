"""GPU parity of the dequantizing GEMM, the weight-streaming GEMV (M <= 8
tokens) and the device block decode against the oracle (oracle/cpu_ref.c:
matmul_tiled_* restatement, lib.rs:4766-4961).

Tolerance (FP32 accumulate, different summation order): per element
|gpu - oracle| <= 2e-6 * sum_k |x_k w_k| + 1e-7.
"""
import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr

pytestmark = pytest.mark.gpu

SHAPES = [(1280, 1280), (5120, 1280), (1280, 5120), (480, 480), (1920, 480), (33, 320), (320, 1280), (96, 64)]
MS = [1, 7, 12, 64, 130, 512]


def _weights(dtype, N, K, rng):
    w = (rng.standard_normal(N * K, dtype=np.float32) * np.float32(0.02))
    if dtype == 0:
        return w, w
    q = cr.quantize_q8(w) if dtype == 1 else cr.quantize_q4(w)
    wd = cr.dequantize_q8(q) if dtype == 1 else cr.dequantize_q4(q)
    return q, wd


@pytest.mark.parametrize("path", ["f16x2", "f16x2-unsplit", "bf16x3", "fp32"])
@pytest.mark.parametrize("dtype", [0, 1, 2])
@pytest.mark.parametrize("N,K", SHAPES)
def test_gemm_matches_oracle(dtype, N, K, path, monkeypatch):
    """Every quantized GEMM kernel: the default 16-bit MFMA kernel with f16
    two-limb activations (split-K where the tiles alone would not fill the
    GPU; CIH_SPLITK=0 never splits), its bf16 three-limb form
    (CIH_LIMBS=bf16x3) and the FP32-MFMA kernel (CIH_QGEMM=fp32)."""
    monkeypatch.setenv("CIH_GEMV", "0")  # small M also through the MFMA kernels
    if path == "f16x2-unsplit":
        monkeypatch.setenv("CIH_SPLITK", "0")
    if path == "fp32":
        monkeypatch.setenv("CIH_QGEMM", "fp32")
    elif dtype == 0:
        pytest.skip("FP32 weights always use the FP32-MFMA kernel")
    if path == "bf16x3":
        monkeypatch.setenv("CIH_LIMBS", "bf16x3")
    rng = np.random.default_rng(N * 7 + K + dtype)
    w, wd = _weights(dtype, N, K, rng)
    bias = rng.standard_normal(N, dtype=np.float32) * np.float32(0.02)
    for M in MS:
        x = rng.standard_normal(M * K, dtype=np.float32)
        print(f"gemm {path} dtype={dtype} M={M} N={N} K={K}", flush=True)
        got = ch.matmul_tiled(dtype, x, w, bias, K, N)
        ref = cr.matmul_tiled(dtype, x, w, bias, K, N, num_threads=8)
        scale = np.abs(x.reshape(M, K)).astype(np.float64) @ np.abs(wd.reshape(N, K)).astype(np.float64).T
        err = np.abs(got.astype(np.float64) - ref)
        assert np.all(err <= 2e-6 * scale + 1e-7), (M, N, K, float(err.max()), float((err / (scale + 1e-30)).max()))


# (N, K) chosen to cover every GEMV grid shape: one split (K <= 128), one
# block per wave (1280x1280), two (1280x5120), four (5120x5120), a split with
# a partly filled last wave (K = 480), columns not a multiple of 64 (33, 1000);
# for the f16-MFMA GEMV: one wave with clamped blocks (K = 64), a partly
# filled last wave (K = 480), 16 waves (K = 5120), two rounds of 16 waves
# (K = 10240), columns not a multiple of 16 (33, FP32 GEMV instead).
GEMV_SHAPES = [(96, 64), (33, 320), (1280, 1280), (1280, 5120), (5120, 5120), (480, 480), (1000, 480), (3840, 1280),
               (64, 10240)]


@pytest.mark.parametrize("path", ["default", "fp32"])
@pytest.mark.parametrize("dtype", [0, 1, 2])
@pytest.mark.parametrize("N,K", GEMV_SHAPES)
def test_gemv_matches_oracle(dtype, N, K, path, monkeypatch):
    """At most 8 rows: quantized weights with N % 16 == 0 take the f16-MFMA
    GEMV on limbs (k_gemv16: one workgroup per 16 columns over the whole K),
    the others and CIH_GEMV16=0 the FP32 weight-streaming GEMV."""
    if path == "fp32":
        if dtype == 0:
            pytest.skip("FP32 weights always take the FP32 GEMV")
        monkeypatch.setenv("CIH_GEMV16", "0")
    rng = np.random.default_rng(N * 3 + K + dtype)
    w, wd = _weights(dtype, N, K, rng)
    bias = rng.standard_normal(N, dtype=np.float32) * np.float32(0.02)
    for M in range(1, 9):
        x = rng.standard_normal(M * K, dtype=np.float32)
        print(f"gemv {path} dtype={dtype} M={M} N={N} K={K}", flush=True)
        got = ch.matmul_tiled(dtype, x, w, bias, K, N)
        ref = cr.matmul_tiled(dtype, x, w, bias, K, N, num_threads=8)
        scale = np.abs(x.reshape(M, K)).astype(np.float64) @ np.abs(wd.reshape(N, K)).astype(np.float64).T
        err = np.abs(got.astype(np.float64) - ref)
        assert np.all(err <= 2e-6 * scale + 1e-7), (M, N, K, float(err.max()), float((err / (scale + 1e-30)).max()))
        # repeated calls give identical bits (split-K order does not depend on scheduling)
        assert np.array_equal(ch.matmul_tiled(dtype, x, w, bias, K, N).view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("tile", ["128x128", "128x64", "64x128", "64x64"])
@pytest.mark.parametrize("dtype", [1, 2])
def test_gemm_tile_shapes(tile, dtype, monkeypatch):
    """Every workgroup tile of the 16-bit-limb kernel (CIH_GEMM_TILE forces
    one), with row and column counts that end inside a tile."""
    monkeypatch.setenv("CIH_GEMV", "0")
    monkeypatch.setenv("CIH_GEMM_TILE", tile)
    rng = np.random.default_rng(31 + dtype)
    for N, K in [(1280, 1280), (200, 96), (33, 320)]:
        w, wd = _weights(dtype, N, K, rng)
        bias = rng.standard_normal(N, dtype=np.float32) * np.float32(0.02)
        for M in (130, 512, 9):
            x = rng.standard_normal(M * K, dtype=np.float32)
            print(f"tile {tile} dtype={dtype} M={M} N={N} K={K}", flush=True)
            got = ch.matmul_tiled(dtype, x, w, bias, K, N)
            ref = cr.matmul_tiled(dtype, x, w, bias, K, N, num_threads=8)
            scale = np.abs(x.reshape(M, K)).astype(np.float64) @ np.abs(wd.reshape(N, K)).astype(np.float64).T
            err = np.abs(got.astype(np.float64) - ref)
            assert np.all(err <= 2e-6 * scale + 1e-7), (M, N, K, float(err.max()))


@pytest.mark.parametrize("path", ["f16x2", "bf16x3"])
def test_gemm_activation_range(path, monkeypatch):
    """Activations spanning 1e-9 .. 3e4 (f16 subnormal to near its maximum):
    the limb split keeps the FP32-accumulate error bound."""
    monkeypatch.setenv("CIH_GEMV", "0")
    if path == "bf16x3":
        monkeypatch.setenv("CIH_LIMBS", "bf16x3")
    rng = np.random.default_rng(77)
    N, K, M = 256, 512, 96
    w, wd = _weights(1, N, K, rng)
    bias = np.zeros(N, np.float32)
    mag = np.float32(10.0) ** rng.uniform(-9, 4.5, M * K).astype(np.float32)
    x = (mag * np.sign(rng.standard_normal(M * K))).astype(np.float32)
    got = ch.matmul_tiled(1, x, w, bias, K, N)
    ref = cr.matmul_tiled(1, x, w, bias, K, N, num_threads=8)
    scale = np.abs(x.reshape(M, K)).astype(np.float64) @ np.abs(wd.reshape(N, K)).astype(np.float64).T
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 2e-6 * scale + 1e-7), float((err / (scale + 1e-30)).max())


@pytest.mark.parametrize("dtype", [1, 2])
def test_device_dequant_bit_exact(dtype):
    rng = np.random.default_rng(5 + dtype)
    x = rng.standard_normal(32 * 4099, dtype=np.float32) * np.float32(3.0)
    x[:32] = 0.0                                   # zero block
    x[32:64] = np.linspace(-8, 7, 32, dtype=np.float32)
    q = cr.quantize_q8(x) if dtype == 1 else cr.quantize_q4(x)
    ref = cr.dequantize_q8(q) if dtype == 1 else cr.dequantize_q4(q)
    got = ch.dequantize_on_device(dtype, q)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
