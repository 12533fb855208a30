"""Pins the CPU oracle (oracle/cpu_ref.c) before it is trusted as the checker.

Each check is a known answer from the reference's own tests
(src/lib.rs `mod tests`, `tests_q4_format`), a published number
(docs/benchmarks_v1.6.0.md), or a closed form / invariant that a plausible
slip (wrong rounding mode, transposed operand, dropped term, wrong sign)
would break.  No test retypes the oracle's formula.
"""
import math

import numpy as np
import pytest

import cpu_ref as cr


# ---------------------------------------------------------------- formats --

def test_q8_roundtrip_mse():
    """lib.rs:6834-6849: linspace(-1, 1, 32) round-trips with MSE < 0.02."""
    src = (np.arange(32, dtype=np.float32) / np.float32(31.0)) * np.float32(2.0) - np.float32(1.0)
    dst = cr.dequantize_q8(cr.quantize_q8(src))
    assert float(np.mean((src - dst) ** 2)) < 0.02


def test_q8_layout_and_round_half_away():
    """Block = {f32 d little-endian, i8 qs[32]}; absmax 127 gives d = 1 and
    halves round away from zero (2.5 -> 3, -2.5 -> -3, 0.5 -> 1), which a
    banker's-rounding slip (2, -2, 0) would fail."""
    src = np.zeros(32, np.float32)
    src[0] = 127.0
    src[1:7] = [2.5, -2.5, 0.5, -0.5, 126.5, -1.49]
    blk = cr.quantize_q8(src)
    assert blk.size == 36
    assert blk[:4].view(np.float32)[0] == np.float32(1.0)
    q = blk[4:].view(np.int8)
    assert list(q[:7]) == [127, 3, -3, 1, -1, 127, -1]
    # the largest magnitude always maps to +-127 and d = absmax / 127
    rng = np.random.default_rng(0)
    x = rng.standard_normal(32 * 64).astype(np.float32)
    b = cr.quantize_q8(x).reshape(64, 36)
    d = b[:, :4].copy().view(np.float32).ravel()
    amax = np.abs(x.reshape(64, 32)).max(1)
    assert np.array_equal(d, (amax / np.float32(127.0)).astype(np.float32))
    qs = b[:, 4:].view(np.int8)
    assert np.all(np.abs(qs).max(1) == 127)


def test_q8_zero_and_error_bound():
    assert np.array_equal(cr.quantize_q8(np.zeros(32, np.float32)), np.zeros(36, np.uint8))
    rng = np.random.default_rng(1)
    x = rng.standard_normal(32 * 256).astype(np.float32) * 5
    blocks = cr.quantize_q8(x)
    d = blocks.reshape(-1, 36)[:, :4].copy().view(np.float32).ravel()
    err = np.abs(cr.dequantize_q8(blocks) - x).reshape(-1, 32)
    assert np.all(err <= (d[:, None] / 2) * (1 + 1e-6) + 1e-7)


def test_q4_exact_nibble_packing():
    """lib.rs:7490-7517: src[j] = 8 - j, src[j+16] = j - 7 gives d = -1 and
    byte j = j | (15 - j) << 4, dequantizing exactly."""
    src = np.zeros(32, np.float32)
    for j in range(16):
        src[j] = 8 - j
        src[j + 16] = j - 7
    blk = cr.quantize_q4(src)
    assert blk.size == 20
    assert blk[:4].view(np.float32)[0] == np.float32(-1.0)
    assert list(blk[4:]) == [j | ((15 - j) << 4) for j in range(16)]
    assert np.array_equal(cr.dequantize_q4(blk), src)


def test_q4_zero_block():
    """lib.rs:7520-7531: zeros -> d = 0, every byte 0x88, dequantizes to 0."""
    blk = cr.quantize_q4(np.zeros(32, np.float32))
    assert blk[:4].view(np.float32)[0] == 0.0
    assert list(blk[4:]) == [0x88] * 16
    assert np.array_equal(cr.dequantize_q4(blk), np.zeros(32, np.float32))


def _q4_reference_vectors():
    """The vectors of test_q4_0_roundtrip_quantize_dequantize_bound (lib.rs:7440-7475)."""
    vecs = [np.array([-8.0 + i * (15.0 / 31.0) for i in range(32)], np.float32)]
    for sign, mult in ((-1, 11), (1, 7)):
        for scale in (0.05, 1.0, 2.5, 10.0):
            v = np.zeros(32, np.float32)
            v[0] = np.float32(8.0 * scale * sign)
            for i in range(1, 32):
                q_level = float((i % 16) - 8)
                noise = (((i * mult) % 9) - 4.0) / 10.0 * 0.45 * scale
                v[i] = np.float32(q_level * (scale if sign < 0 else -scale) + noise)
            vecs.append(v)
    return vecs


def test_q4_error_bound_reference_vectors():
    """lib.rs:7440-7487: |x - dequant(quant(x))| <= |d|/2 + 1e-5."""
    for v in _q4_reference_vectors():
        blk = cr.quantize_q4(v)
        d = abs(float(blk[:4].view(np.float32)[0]))
        assert np.all(np.abs(cr.dequantize_q4(blk) - v) <= d / 2 + 1e-5)


def test_q4_signed_max_and_nibble_order():
    """d = (signed first largest-|x| element) / -8, so that element maps to
    nibble 0; element j goes to the low nibble of byte j and element j+16 to
    the high nibble (a swapped order fails the comparison below)."""
    x = np.zeros(32, np.float32)
    x[20] = 4.0       # largest |x|, positive -> d = -0.5
    x[3] = -3.5
    x[5] = 1.0
    blk = cr.quantize_q4(x)
    assert blk[:4].view(np.float32)[0] == np.float32(-0.5)
    nib_lo = blk[4:] & 0xF
    nib_hi = blk[4:] >> 4
    assert nib_hi[4] == 0            # element 20 -> -8 -> nibble 0
    assert nib_lo[3] == 15           # -3.5 / -0.5 = 7 -> 15
    assert nib_lo[5] == 6            # 1.0 / -0.5 = -2 -> 6
    x2 = np.zeros(32, np.float32)
    x2[1], x2[7] = -2.0, 2.0         # tie in |x|: the first (index 1) sets the sign
    assert cr.quantize_q4(x2)[:4].view(np.float32)[0] == np.float32(0.25)


# -------------------------------------------------------------- tokenizer --

def test_tokenizer_known_answers():
    """lib.rs:6871, 6922-6924."""
    assert list(cr.tokenize("LA")) == [0, 4, 5, 2]
    assert list(cr.tokenize("M*C")) == [0, 20, 32, 23, 2]
    assert list(cr.tokenize("M<mask_1>C")) == [0, 20, 32, 23, 2]
    assert list(cr.tokenize("M<mask>C")) == [0, 20, 32, 23, 2]
    assert list(cr.tokenize("XBUZO.-")) == [0, 24, 25, 26, 27, 28, 29, 30, 2]
    assert list(cr.tokenize("a1J")) == [0, 3, 3, 3, 2]
    assert list(cr.tokenize("Aé")) == [0, 5, 3, 2]   # one id per Unicode scalar
    assert list(cr.tokenize("")) == [0, 2]


# ------------------------------------------------------- elementwise math --

def test_softmax_sums_to_one():
    """lib.rs:6868-6870 plus shift invariance and the closed form."""
    p = cr.softmax(np.array([1.0, 2.0, 3.0], np.float32))
    assert abs(float(p.sum()) - 1.0) < 1e-6
    e = np.exp(np.array([1.0, 2.0, 3.0]) - 3.0)
    assert np.allclose(p, e / e.sum(), rtol=1e-6)
    rng = np.random.default_rng(2)
    x = rng.standard_normal(300).astype(np.float32) * 10
    assert np.allclose(cr.softmax(x), cr.softmax(x + np.float32(50.0)), atol=1e-7)


def test_log_softmax_canonical():
    """lib.rs:6928-6936: normalizes over the 20 canonical ids only."""
    lp = cr.log_softmax_canonical(np.ones(33, np.float32))
    assert abs(float(np.exp(lp[4:24]).sum()) - 1.0) < 1e-5
    assert np.all(np.isneginf(lp[:4])) and np.all(np.isneginf(lp[24:]))
    rng = np.random.default_rng(3)
    x = rng.standard_normal(33).astype(np.float32)
    lp = cr.log_softmax_canonical(x)
    ref = x[4:24].astype(np.float64) - np.log(np.exp(x[4:24].astype(np.float64)).sum())
    assert np.allclose(lp[4:24], ref, atol=2e-6)


def test_erf_gelu_against_libm():
    """A&S 7.1.26 is within 1.5e-7 of erf (plus a few f32 ulps of evaluation
    error); it is odd; GELU follows 0.5 x (1 + erf(x/sqrt2))."""
    xs = np.linspace(-6, 6, 2001)
    err = max(abs(cr.erf(float(x)) - math.erf(float(np.float32(x)))) for x in xs)
    assert err < 5e-7
    assert abs(cr.erf(0.0)) < 1e-7 and cr.erf(-1.0) == -cr.erf(1.0)
    g = cr.gelu(xs.astype(np.float32))
    ref = 0.5 * xs * (1 + np.vectorize(math.erf)(xs / math.sqrt(2)))
    assert np.allclose(g, ref, atol=2e-6)


def test_layer_norm_invariants():
    """lib.rs:2556-2562 (stability test 6862-6864): with gamma 1, beta 0 the
    output has mean 0 and variance var/(var + eps); gamma/beta apply affinely."""
    out = cr.layer_norm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), np.zeros(4, np.float32))
    assert not np.isnan(out).any()
    rng = np.random.default_rng(4)
    x = rng.standard_normal(1280).astype(np.float32) * 3 + 1
    y = cr.layer_norm(x, np.ones(1280, np.float32), np.zeros(1280, np.float32)).astype(np.float64)
    var = float(np.var(x.astype(np.float64)))
    assert abs(y.mean()) < 1e-6 and abs(y.var() - var / (var + 1e-5)) < 1e-5
    w, b = rng.standard_normal(1280).astype(np.float32), rng.standard_normal(1280).astype(np.float32)
    assert np.allclose(cr.layer_norm(x, w, b), w * y + b, atol=1e-5)


def test_rope_tables_and_rotation():
    """lib.rs:2513-2522, 3533-3552: position 0 is the identity, each (j, j+hd/2)
    pair is rotated by pos * 10000^(-2j/hd), so pair norms are preserved."""
    hd, H = 64, 2
    c, s = cr.rope_tables(100, hd)
    pos = np.arange(100)[:, None]
    freq = 1.0 / 10000.0 ** (2 * np.arange(hd // 2) / hd)
    assert np.allclose(c, np.cos(pos * freq), atol=2e-5) and np.allclose(s, np.sin(pos * freq), atol=2e-5)
    rng = np.random.default_rng(5)
    q = rng.standard_normal(hd * H).astype(np.float32)
    k = rng.standard_normal(hd * H).astype(np.float32)
    q0, k0 = cr.apply_rope(q, k, c, s, 0, H)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    q7, _ = cr.apply_rope(q, k, c, s, 7, H)
    for h in range(H):
        a, b = q[h * hd:h * hd + hd // 2], q[h * hd + hd // 2:(h + 1) * hd]
        a2, b2 = q7[h * hd:h * hd + hd // 2], q7[h * hd + hd // 2:(h + 1) * hd]
        th = 7 * freq
        assert np.allclose(a2, a * np.cos(th) - b * np.sin(th), atol=1e-5)
        assert np.allclose(b2, b * np.cos(th) + a * np.sin(th), atol=1e-5)
    # relative-position property: <R_m q, R_n k> depends only on m - n
    qa, _ = cr.apply_rope(q, k, c, s, 10, H)
    _, ka = cr.apply_rope(q, k, c, s, 4, H)
    qb, _ = cr.apply_rope(q, k, c, s, 30, H)
    _, kb = cr.apply_rope(q, k, c, s, 24, H)
    assert abs(float(qa[:hd] @ ka[:hd]) - float(qb[:hd] @ kb[:hd])) < 1e-3


# ------------------------------------------------------------------- GEMM --

@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_matmul_against_float64(dtype):
    """Tiled GEMM = x @ W^T + b (not W @ x, not missing bias) against a float64
    product of the dequantized weights; thread count does not change bits
    (lib.rs:7803-7828); small out_dim takes the single-thread path."""
    rng = np.random.default_rng(6 + dtype)
    M, N, K = 13, 96, 480
    x = rng.standard_normal(M * K).astype(np.float32)
    w = rng.standard_normal(N * K).astype(np.float32) * np.float32(0.05)
    wq = w if dtype == 0 else (cr.quantize_q8(w) if dtype == 1 else cr.quantize_q4(w))
    wd = w if dtype == 0 else (cr.dequantize_q8(wq) if dtype == 1 else cr.dequantize_q4(wq))
    bias = rng.standard_normal(N).astype(np.float32)
    ref = x.reshape(M, K).astype(np.float64) @ wd.reshape(N, K).astype(np.float64).T + bias
    outs = [cr.matmul_tiled(dtype, x, wq, bias, K, N, num_threads=t) for t in (1, 2, 4, 8)]
    assert np.allclose(outs[0], ref, atol=1e-4, rtol=1e-5)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


# ------------------------------------------------------------- APC / metrics --

def test_apc_invariants_and_brute_force():
    """accumulate_head_apc (lib.rs:5036-5076): the correction has zero row
    sums, the result is symmetric, equals the float64 brute force, and a
    zero weight is skipped."""
    rng = np.random.default_rng(7)
    S = 23
    n = S - 2
    A = rng.random((S, S)).astype(np.float32)
    A /= A.sum(1, keepdims=True)
    cl = np.zeros((n, n), np.float32)
    cr.accumulate_head_apc(A.ravel(), cl, S, n, 1.0)
    a = A[1:-1, 1:-1].astype(np.float64)
    s = a + a.T
    r = s.sum(1)
    ref = s - np.outer(r, r) / r.sum()
    assert np.allclose(cl, ref, atol=1e-6)
    assert np.allclose(cl, cl.T, atol=1e-6)
    assert np.allclose(cl.sum(1), 0.0, atol=1e-5)
    before = cl.copy()
    cr.accumulate_head_apc(A.ravel(), cl, S, n, 0.0)
    assert np.array_equal(before, cl)


def test_metrics_known_answers():
    """lib.rs:6873-6887: top-1 match, KL of identical logits, ties -> last index."""
    a = np.array([10.0, 5.0, 1.0, 2.0, 8.0, 0.0], np.float32)
    b = np.array([23.0, 13.0, 5.0, 7.0, 19.0, 3.0], np.float32)
    assert cr.top1_match_rate(a, b, 3) == 1.0
    assert abs(cr.kl_divergence(a, a, 3)) < 1e-6
    t1 = np.array([1.0, 1.0, 0.0], np.float32)
    t2 = np.array([0.0, 1.0, 0.0], np.float32)
    assert cr.top1_match_rate(t1, t2, 3) == 1.0   # both argmax to index 1 (last of the tie)
    assert abs(cr.cosine_similarity(a, 2 * a) - 1.0) < 1e-6
    assert cr.rmse(a, a) == 0.0
