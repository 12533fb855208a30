"""Pins the oracle's bidirectional forward (cr_forward: forward_bidirectional,
_q8, _q4, src/lib.rs:5097-6147) against an independent float64 ESM-2
(tests/ref64.py) at every head size the presets use (16, 24, 32, 64), for
FP32, Q8_0 and Q4_0 weights, with both LM-head forms (the full classifier,
lib.rs:5389-5426, and the tied-embedding decoder, 5427-5439 / Q8 5775-5787),
on every output: logits, hidden, every layer's hidden state and attention
maps, the last layer's head mean and the contact probabilities.  At head
dim 64 both of the reference's attention micro-kernels are pinned: the
AVX-512F one it runs on such hosts (lib.rs:3398-3434) and the 256-bit one.

Bounds (max abs vs float64; the oracle computes in float32):
  logits, hidden, layer hidden   1e-5   (a dropped bias, LN weight or RoPE term is >= 1e-3)
  attention maps, head mean      5e-7   (a wrong 1/sqrt(hd) or RoPE pairing is >= 1e-3)
  contacts                       5e-7
The measured errors are printed; they sit at float32 rounding (logits and
hidden 1e-7..2e-6, maps ~1e-8, contacts ~5e-8).
"""
import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from ref64 import forward64

TOL = {"logits": 1e-5, "hidden": 1e-5, "layer_hidden": 1e-5, "attn": 5e-7, "final_att": 5e-7, "contacts": 5e-7}


def model(hd, H, dtype, seed, L=2, tied=False):
    cfg = ch.EsmConfig(hd * H, 4 * hd * H, L, H)
    w = ch.EsmWeights.random(cfg, seed=seed, bias_std=0.02)
    rng = np.random.default_rng(seed)
    d = cfg.dim
    # LayerNorm weights away from (1, 0), so that each is exercised
    for g, b, n in (("ln_1_weight", "ln_1_bias", L * d), ("ln_2_weight", "ln_2_bias", L * d),
                    ("ln_f_weight", "ln_f_bias", d)):
        setattr(w, g, (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))
        setattr(w, b, (0.05 * rng.standard_normal(n)).astype(np.float32))
    cls = np.array(w.classifier_weights, np.float32)
    cls[:2 * d] = np.concatenate([1.0 + 0.1 * rng.standard_normal(d), 0.05 * rng.standard_normal(d)])
    w.classifier_weights = cls[:7] if tied else cls
    if dtype == 1:
        w = w.quantize_q8()
    elif dtype == 2:
        w = w.quantize_q4()
    cw = rng.standard_normal(L * H).astype(np.float32)
    cw[1::3] = 0.0  # zero-weight heads are skipped
    return cfg, w, (cw, np.float32(-0.3))


def tokens(rng, n, masks=()):
    t = np.concatenate([[0], 4 + rng.integers(0, 20, n), [2]]).astype(np.int32)
    for i in masks:
        t[i] = 32
    return t


def compare(cfg, w, toks, contact, tag):
    got = cr.forward(cfg, w, toks, 4, contacts=contact, attn=True, layer_hidden=True)
    ref = forward64(cfg, w, toks, contacts=contact)
    errs = {}
    for k in TOL:
        if k not in got or got[k].size == 0:
            assert k not in ref or ref[k].size == 0, (tag, k)
            continue
        errs[k] = float(np.abs(got[k].astype(np.float64) - ref[k]).max())
    print(tag, {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    for k, e in errs.items():
        assert e <= TOL[k], (tag, k, e)
    return got, ref


@pytest.mark.parametrize("dtype", [0, 1, 2])
@pytest.mark.parametrize("hd", [16, 24, 32, 64])
def test_bidirectional_forward_vs_float64(hd, dtype):
    rng = np.random.default_rng(hd * 7 + dtype)
    cfg, w, contact = model(hd, 4, dtype, seed=100 + hd + dtype)
    compare(cfg, w, tokens(rng, 37, masks=(5, 20)), contact, f"hd={hd} dtype={dtype}")


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_tied_decoder_vs_float64(dtype):
    """A classifier shorter than the LM head: logits = x . emb^T with no bias
    (the Q8_0 embedding dequantized, as matmul_tiled_q8_parallel reads it)."""
    rng = np.random.default_rng(300 + dtype)
    cfg, w, contact = model(32, 4, dtype, seed=300 + dtype, tied=True)
    compare(cfg, w, tokens(rng, 30, masks=(3,)), contact, f"tied dtype={dtype}")


@pytest.mark.parametrize("avx_only", [False, True])
def test_hd64_attention_micro_kernels(avx_only):
    """Head dim 64 through the AVX-512F dot/axpy (fused multiply-adds, the
    halving reduction) when the host has it, and through the 256-bit ones:
    both pinned to float64.  On an AVX-512F host the two paths round
    differently (which shows the dispatch is live) and agree to 2e-7."""
    rng = np.random.default_rng(64)
    cfg, w, contact = model(64, 4, 1, seed=640)
    toks = tokens(rng, 45, masks=(9,))
    has512 = cr.attention_uses_avx512(64)
    if not avx_only and not has512:
        pytest.skip("host without AVX-512F: the reference runs the 256-bit path here too")
    cr.set_attention_isa(avx_only)
    try:
        got, _ = compare(cfg, w, toks, contact, f"hd=64 {'avx' if avx_only else 'avx512'}")
        cr.set_attention_isa(not avx_only)
        other = cr.forward(cfg, w, toks, 4, contacts=contact, attn=True)
    finally:
        cr.set_attention_isa(False)
    e = float(np.abs(other["attn"] - got["attn"]).max())
    assert e <= 2e-7
    if has512:
        assert e > 0.0


def test_all_masked_and_short_sequences():
    """Edge cases of the embedding and the contact head: a sequence made only
    of <mask> (token-dropout scale 0, all embeddings zero), BOS+EOS alone (no
    residues, no contacts) and one residue."""
    cfg, w, contact = model(16, 4, 0, seed=5)
    for toks in (np.array([32, 32, 32], np.int32), np.array([0, 2], np.int32), np.array([0, 7, 2], np.int32)):
        compare(cfg, w, toks, contact, f"S={len(toks)}")


def test_float64_reference_catches_planted_mistakes():
    """The float64 model is sensitive to the mistakes it is meant to catch:
    the same inputs with a dropped bias, the contact weights' sign flipped, or
    a causal mask in place of bidirectional attention move the outputs far
    beyond the bounds."""
    rng = np.random.default_rng(1)
    cfg, w, contact = model(32, 4, 0, seed=11)
    toks = tokens(rng, 25)
    base = forward64(cfg, w, toks, contacts=contact)
    w2 = model(32, 4, 0, seed=11)[1]
    w2.bo = np.zeros_like(w2.bo)
    assert np.abs(forward64(cfg, w2, toks)["logits"] - base["logits"]).max() > 50 * TOL["logits"]
    flipped = forward64(cfg, w, toks, contacts=(-contact[0], contact[1]))
    assert np.abs(flipped["contacts"] - base["contacts"]).max() > 50 * TOL["contacts"]
    causal = forward64(cfg, w, toks, causal=True)
    assert np.abs(causal["attn"] - base["attn"]).max() > 50 * TOL["attn"]
