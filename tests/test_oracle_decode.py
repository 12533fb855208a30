"""The oracle's autoregressive path (forward / forward_q8 / forward_q4 with a
KV cache, SimpleRng, sample, generate_sequence*; src/lib.rs:3506-4233,
6538-6827), pinned without running the reference:

* SimpleRng: the first output for seed 1 worked by hand, the seed-0
  substitution, and Marsaglia's full-period criterion for the xorshift64
  triple (13, 7, 17) checked on its GF(2) matrix — a wrong shift or direction
  fails it;
* sample: argmax over the allowed ids with first-index ties, and the inverse
  CDF against a float64 recomputation for many seeds and temperatures;
* one token at position 0 is the bidirectional forward of a one-token
  sequence (same embedding scale, a single key): equal to the pinned
  bidirectional oracle within summation-order noise, in all three formats;
* positions 0..n-1 through the KV cache against a float64 causal transformer
  written from the mathematics (RoPE split-half, causal softmax, erf GELU);
* the reference's own tests: forward(20, 0) on the shipped 8M weights, FP32
  vs Q8_0 cosine > 0.995 and vs Q4_0 > 0.85 (lib.rs:7273-7353);
* the generation loop's limits: max_new_tokens, <eos>, prompt truncation.
"""
import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from ref64 import forward64


# ---- SimpleRng --------------------------------------------------------------

def test_rng_known_answers():
    # seed 1: x = 1; x ^= x << 13 -> 8193; x ^= x >> 7 -> 8193 ^ 64 = 8257;
    # x ^= x << 17 -> 8257 ^ (8257 * 131072) = 1082269761
    r = cr.SimpleRng(1)
    assert r.next_u32() == 1082269761
    # seed 0 is replaced by 0x123456789abcdef (lib.rs:3508)
    a, b = cr.SimpleRng(0), cr.SimpleRng(0x123456789ABCDEF)
    assert [a.next_u32() for _ in range(5)] == [b.next_u32() for _ in range(5)]
    # next_f32 = u32 / u32::MAX in f32: in [0, 1]
    r = cr.SimpleRng(99)
    f = np.array([r.next_f32() for _ in range(20000)])
    assert f.min() >= 0.0 and f.max() <= 1.0 and abs(f.mean() - 0.5) < 0.01


def _gf2_apply(images, v):
    out = 0
    i = 0
    while v:
        if v & 1:
            out ^= images[i]
        v >>= 1
        i += 1
    return out


def _gf2_compose(a, b):  # a after b
    return [_gf2_apply(a, x) for x in b]


def _gf2_pow(m, e):
    result = [1 << i for i in range(64)]
    base = m
    while e:
        if e & 1:
            result = _gf2_compose(base, result)
        base = _gf2_compose(base, base)
        e >>= 1
    return result


def test_rng_full_period_criterion():
    """Marsaglia (2003): xorshift64 with T = (I+L^a)(I+R^b)(I+L^c) has period
    2^64-1 iff T^(2^64-1) = I and T^((2^64-1)/p) != I for every prime p of
    2^64-1 = 3 * 5 * 17 * 257 * 641 * 65537 * 6700417.  T is read off the
    oracle's own step applied to the 64 basis states."""
    mask = (1 << 64) - 1
    images = []
    for i in range(64):
        r = cr.SimpleRng(1 << i)
        r.next_u32()
        images.append(r.state.value & mask)
    primes = [3, 5, 17, 257, 641, 65537, 6700417]
    order = (1 << 64) - 1
    assert np.prod([float(p) for p in primes]) == float(order) and all(order % p == 0 for p in primes)
    ident = [1 << i for i in range(64)]
    assert _gf2_pow(images, order) == ident
    for p in primes:
        assert _gf2_pow(images, order // p) != ident


# ---- sample -----------------------------------------------------------------

ALLOWED = [2] + list(range(4, 24))


def test_sample_greedy_masks_and_ties():
    rng = cr.SimpleRng(3)
    lg = np.full(33, -5.0, np.float32)
    lg[0], lg[1], lg[3], lg[24], lg[32] = 50, 40, 30, 20, 60    # disallowed ids never win
    lg[9] = 1.0
    lg[15] = 1.0                                                 # tie: the first index wins
    assert cr.sample(lg, 0.0, rng) == 9
    lg[2] = 2.0                                                  # <eos> is allowed
    assert cr.sample(lg, -1.0, rng) == 2
    before = rng.state.value
    cr.sample(lg, 0.0, rng)
    assert rng.state.value == before                             # greedy draws nothing


def test_sample_inverse_cdf_float64():
    rng0 = np.random.default_rng(11)
    checked = 0
    for seed in range(1, 400):
        T = [0.3, 0.7, 1.0, 1.6][seed % 4]
        lg = (rng0.standard_normal(33) * 2).astype(np.float32)
        r = cr.SimpleRng(seed)
        probe = cr.SimpleRng(seed)
        u = float(probe.next_f32())
        got = cr.sample(lg, T, r)
        assert r.state.value == probe.state.value                # exactly one draw
        z = np.full(33, -np.inf)
        z[ALLOWED] = lg[ALLOWED].astype(np.float64) / T
        p = np.exp(z - z.max())
        p /= p.sum()
        cum = np.cumsum(p)
        want = int(np.argmax(cum >= u)) if u <= cum[-1] else 4
        if np.min(np.abs(cum[ALLOWED] - u)) < 1e-5:
            continue                                             # too close to a boundary for f32 vs f64
        assert got == want, (seed, T, got, want, u)
        checked += 1
    assert checked > 350


# ---- the one-token forward ----------------------------------------------------

@pytest.fixture(scope="module")
def w8m_all(w8m_path):
    cfg = ch.EsmConfig.esm2_8m()
    w = ch.EsmWeights.from_grouped_canonical(w8m_path, cfg)
    return cfg, {"fp32": w, "q8": w.quantize_q8(), "q4": w.quantize_q4()}


@pytest.mark.parametrize("fmt", ["fp32", "q8", "q4"])
def test_position0_equals_one_token_bidirectional(w8m_all, fmt):
    cfg, ws = w8m_all
    w = ws[fmt]
    for tok in (0, 20, 32, 7):
        rs = cr.RunState(cfg, w, max_len=8, num_threads=4)
        ar = rs.step(tok, 0)
        bi = cr.forward(cfg, w, np.array([tok], np.int32), 4, final_att=False, hidden=False)["logits"][0]
        assert np.abs(ar - bi).max() <= 2e-5, (fmt, tok, np.abs(ar - bi).max())


def test_reference_cosines_at_position0(w8m_all):
    """test_forward_q8_cosine_similarity_8m / _q4_ (lib.rs:7273-7353)."""
    cfg, ws = w8m_all
    lg = {k: cr.RunState(cfg, w, max_len=4, num_threads=4).step(20, 0) for k, w in ws.items()}

    def cos(a, b):
        a, b = a[4:24].astype(np.float64), b[4:24].astype(np.float64)
        return float(a @ b / np.sqrt((a @ a) * (b @ b)))
    assert cos(lg["fp32"], lg["q8"]) > 0.995
    assert cos(lg["fp32"], lg["q4"]) > 0.85


def test_kv_cache_positions_against_float64_causal(w8m_all):
    cfg, ws = w8m_all
    w = ws["fp32"]
    toks = [0, 20, 5, 32, 11, 11, 23, 4, 17, 9, 30, 12]
    rs = cr.RunState(cfg, w, max_len=16, num_threads=4)
    steps = np.stack([rs.step(t, p) for p, t in enumerate(toks)])
    ref = forward64(cfg, w, toks, causal=True)["logits"]
    err = float(np.abs(steps - ref).max())
    print(f"AR oracle vs float64 causal, 12 positions: {err:.2e}")
    assert err <= 1e-4


def test_kv_cache_overwrite_and_revisit(w8m_all):
    """Stepping a position again overwrites its cache entries, as the
    reference's copy_from_slice does: p, p again gives the same logits, and a
    different token at p changes later positions consistently."""
    cfg, ws = w8m_all
    w = ws["q8"]
    a = cr.RunState(cfg, w, max_len=8, num_threads=4)
    for p, t in enumerate([0, 20, 7]):
        a.step(t, p)
    la = a.step(9, 3)
    b = cr.RunState(cfg, w, max_len=8, num_threads=4)
    for p, t in enumerate([0, 20, 11]):
        b.step(t, p)
    b.step(7, 2)                                                  # overwrite position 2
    lb = b.step(9, 3)
    assert np.array_equal(la, lb)


# ---- generation ----------------------------------------------------------------

def test_generation_loop_limits(w8m_all):
    cfg, ws = w8m_all
    w = ws["q8"]
    prompt = [0, 20, 5, 7]
    g = cr.generate(cfg, w, prompt, 0.0, 6, 0, max_seq_len=64, num_threads=4)
    assert g.size == 6 and all(t == 2 or 4 <= t <= 23 for t in g)
    # the loop is: sample from the last logits, step the sampled token
    rs = cr.RunState(cfg, w, max_len=64, num_threads=4)
    for p, t in enumerate(prompt):
        lg = rs.step(t, p)
    rng = cr.SimpleRng(0)
    manual = []
    for p in range(len(prompt), len(prompt) + 6):
        t = cr.sample(lg, 0.0, rng)
        if t == 2:
            break
        manual.append(t)
        lg = rs.step(t, p)
    assert list(g) == manual
    # limit = min(prompt + max_new, max_seq_len); a prompt at the limit generates nothing
    assert cr.generate(cfg, w, prompt, 0.0, 50, 0, max_seq_len=6, num_threads=4).size == 2
    assert cr.generate(cfg, w, list(range(4, 14)), 0.0, 5, 0, max_seq_len=8, num_threads=4).size == 0
    # sampled generation is reproducible from the seed and changes with it
    g1 = cr.generate(cfg, w, prompt, 4.0, 24, 5, max_seq_len=64, num_threads=4)
    g2 = cr.generate(cfg, w, prompt, 4.0, 24, 5, max_seq_len=64, num_threads=4)
    g3 = cr.generate(cfg, w, prompt, 4.0, 24, 6, max_seq_len=64, num_threads=4)
    assert np.array_equal(g1, g2) and not np.array_equal(g1, g3)


def test_generation_stops_at_eos():
    cfg = ch.EsmConfig(64, 128, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=4, bias_std=0.02)
    cls = np.array(w.classifier_weights, np.float32)
    cls[-cfg.vocab_size + 2] = 100.0                             # decoder bias of <eos>
    w.classifier_weights = cls
    assert cr.generate(cfg, w, [0, 5, 6], 0.0, 10, 0, max_seq_len=32).size == 0
    assert cr.generate(cfg, w, [0, 5, 6], 1.0, 10, 3, max_seq_len=32).size == 0
