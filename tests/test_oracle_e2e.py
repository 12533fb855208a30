"""End-to-end pins of the oracle's forward on the shipped ESM-2 8M weights.

* docs/benchmarks_v1.6.0.md:61-62 — FP32, Q8_0 and Q4_0 all predict the
  unmasked test_peptidase.fasta peptide 39/39.
* docs/benchmarks_v1.6.0.md:19-20 — logits cosine vs HF 0.999995 (Q8_0) and
  0.998168 (Q4_0); the FP32 path equals HF to 1e-6, so the oracle's
  Q8/Q4-vs-FP32 cosines must reproduce those figures.
* lib.rs:7273-7353 — Q8 vs FP32 cosine > 0.995, Q4 > 0.85.
* lib.rs:6938-6983 — masked "MCMP*TTD" logits are finite with entropy > 0.1.
* tests/golden/hf_8m_peptide.npz — an independent implementation
  (transformers EsmForMaskedLM, built offline from a local config) on the
  same weights: logits, hidden state, all attention maps and contacts.
"""
import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from conftest import GOLDEN, PEPTIDE, decode


@pytest.fixture(scope="module")
def w8m(w8m_path):
    cfg = ch.EsmConfig.esm2_8m()
    return cfg, ch.EsmWeights.from_grouped_canonical(w8m_path, cfg)


def test_peptide_reconstruction_all_formats(w8m):
    cfg, w = w8m
    toks = cr.tokenize(PEPTIDE)
    r32 = cr.forward(cfg, w, toks, 4)["logits"]
    assert decode(r32.argmax(1)[1:-1]) == PEPTIDE
    r8 = cr.forward(cfg, w.quantize_q8(), toks, 4)["logits"]
    r4 = cr.forward(cfg, w.quantize_q4(), toks, 4)["logits"]
    assert decode(r8.argmax(1)[1:-1]) == PEPTIDE
    assert decode(r4.argmax(1)[1:-1]) == PEPTIDE
    c8, c4 = cr.cosine_similarity(r32, r8), cr.cosine_similarity(r32, r4)
    assert c8 > 0.995 and c4 > 0.85
    assert abs(c8 - 0.999995) < 2e-6, c8      # published Q8_0 logits cosine
    assert abs(c4 - 0.998168) < 2e-5, c4      # published Q4_0 logits cosine


def test_masked_inference_entropy(w8m):
    cfg, w = w8m
    toks = cr.tokenize("MCMP*TTD")
    lg = cr.forward(cfg, w, toks, 1)["logits"]
    assert np.isfinite(lg).all()
    lp = cr.log_softmax_canonical(lg[5])
    p = np.exp(lp[4:24])
    assert -(p * lp[4:24]).sum() > 0.1


def test_against_hf_fixture(w8m):
    cfg, w = w8m
    hf = np.load(f"{GOLDEN}/hf_8m_peptide.npz")
    cw, cb = cfg.contact_head_weights()
    for tag in ("peptide", "masked"):
        toks = hf[f"{tag}_tokens"]
        assert np.array_equal(toks, cr.tokenize(PEPTIDE if tag == "peptide" else "MCMP*TTD"))
        r = cr.forward(cfg, w, toks, 4, contacts=(cw, cb), attn=True)
        assert np.abs(r["logits"] - hf[f"{tag}_logits"]).max() < 1e-4
        assert np.abs(r["hidden"] - hf[f"{tag}_hidden"]).max() < 2e-5
        assert np.abs(r["attn"] - hf[f"{tag}_attn"]).max() < 1e-5
        assert np.abs(r["final_att"] - hf[f"{tag}_attn"][-1].mean(0)).max() < 1e-6
        assert np.abs(r["contacts"] - hf[f"{tag}_contacts"]).max() < 1e-5


def test_contacts_invariants(w8m):
    """Contact probabilities are symmetric and strictly inside (0, 1)
    (lib.rs:8535-8542)."""
    cfg, w = w8m
    cw, cb = cfg.contact_head_weights()
    toks = cr.tokenize(PEPTIDE)
    c = cr.forward(cfg, w, toks, 4, contacts=(cw, cb))["contacts"]
    assert np.all((c > 0) & (c < 1))
    assert np.allclose(c, c.T, atol=1e-6)
