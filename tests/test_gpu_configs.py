"""The five benchmark configurations at their full sizes.  Where the oracle
finishes in seconds it checks one or more sequences of the batch directly;
everywhere, size-independent properties: exported softmax rows sum to 1,
contact maps are symmetric probabilities, and the default kernels agree with
independent ones (FP32-MFMA attention and FP32-MFMA dequantizing GEMM)."""
import os
import sys

import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from test_gpu_forward import check_argmax

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

pytestmark = pytest.mark.gpu


def rand_tokens(rng, n):
    t = np.empty(n + 2, np.int32)
    t[0], t[-1] = 0, 2
    t[1:-1] = 4 + rng.integers(0, 20, n)
    return t


def test_config1_8m_fp32_maps(w8m_path):
    """8M FP32 (shipped weights), B=1, L=256, logits + all 6x20 maps."""
    rng = np.random.default_rng(1)
    cfg = ch.EsmConfig.esm2_8m()
    w = ch.EsmWeights.from_grouped_canonical(w8m_path, cfg)
    toks = rand_tokens(rng, 254)
    flags = ch.OUT_LOGITS | ch.OUT_ATTN
    m = ch.GpuModel(cfg, w, max_batch=1, max_len=256, outputs=flags)
    got = m.forward([toks], flags)
    ref = cr.forward(cfg, w, toks, 16, attn=True)
    assert np.abs(got["logits"][0] - ref["logits"]).max() <= 1e-3
    assert np.abs(got["attn"][0] - ref["attn"]).max() <= 1e-5
    assert np.abs(got["attn"][0].sum(-1) - 1.0).max() <= 1e-5
    m.close()


def test_config2_35m_q8_ragged():
    """35M Q8_0, B=8, lengths U[128, 510] padded to 512: every sequence vs the oracle."""
    rng = np.random.default_rng(2)
    cfg = ch.EsmConfig.esm2_35m()
    w = ch.EsmWeights.random(cfg, seed=35, bias_std=0.02).quantize_q8()
    seqs = [rand_tokens(rng, int(rng.integers(128, 511))) for _ in range(8)]
    m = ch.GpuModel(cfg, w, max_batch=8, max_len=512, outputs=ch.OUT_LOGITS | ch.OUT_HIDDEN)
    got = m.forward(seqs, ch.OUT_LOGITS | ch.OUT_HIDDEN)
    for b, t in enumerate(seqs):
        ref = cr.forward(cfg, w, t, 16, final_att=False)
        S = len(t)
        assert np.abs(got["logits"][b, :S] - ref["logits"]).max() <= 1e-3, b
        assert np.abs(got["hidden"][b, :S] - ref["hidden"]).max() <= 1e-3, b
    m.close()


def test_config3_150m_q4_contacts_maps(monkeypatch):
    """150M Q4_0, B=4, L=1024 (n=1022), all 30x20 maps exported + the official
    contact head: sequence 0 vs the oracle; all rows of all maps sum to 1;
    contacts symmetric in (0, 1); the FP32-MFMA attention kernel agrees."""
    rng = np.random.default_rng(3)
    cfg = ch.EsmConfig.esm2_150m()
    w = ch.EsmWeights.random(cfg, seed=150, bias_std=0.02).quantize_q4()
    contact = cfg.contact_head_weights()
    seqs = [rand_tokens(rng, 1022) for _ in range(4)]
    flags = ch.OUT_LOGITS | ch.OUT_CONTACTS | ch.OUT_ATTN
    m = ch.GpuModel(cfg, w, contact_head=contact, max_batch=4, max_len=1024, outputs=flags)
    got = m.forward(seqs, flags)
    ref = cr.forward(cfg, w, seqs[0], 16, contacts=contact, final_att=False)
    assert np.abs(got["logits"][0] - ref["logits"]).max() <= 1e-3
    assert np.abs(got["contacts"][0] - ref["contacts"]).max() <= 1e-4
    for b in range(4):
        a = got["attn"][b]
        assert np.abs(a.sum(-1, dtype=np.float64) - 1.0).max() <= 1e-5, b
        c = got["contacts"][b]
        assert np.array_equal(c, c.T) and c.min() > 0.0 and c.max() < 1.0
    del a
    monkeypatch.setenv("CIH_FORWARD_GRAPH", "0")
    monkeypatch.setenv("CIH_ATT", "fp32")
    alt = m.forward(seqs, ch.OUT_LOGITS | ch.OUT_CONTACTS)
    assert 0.0 < np.abs(alt["contacts"] - got["contacts"]).max() <= 1e-4
    assert np.abs(alt["logits"] - got["logits"]).max() <= 1e-3
    m.close()


def test_config5_3b_q4_long(monkeypatch):
    """3B Q4_0, B=1, L=2048 (attention-dominated).  The full-length logits
    against the oracle's: the oracle needs minutes at this length, so
    tests/golden/make_config5_fixture.py ran it once on the same seeded model
    and tokens and committed its logits.  Also a 62-residue sequence against
    the oracle run here, and at L=2048 the default kernels against the
    independent FP32-MFMA attention + FP32-MFMA GEMM (CIH_ATT=fp32,
    CIH_QGEMM=fp32)."""
    sys.path.insert(0, GOLDEN)
    from make_config5_fixture import model_and_tokens, weights_digest

    fx = np.load(os.path.join(GOLDEN, "config5_3b_q4_l2048.npz"))
    cfg, w, toks = model_and_tokens()
    assert np.array_equal(toks, fx["tokens"])
    assert weights_digest(w) == str(fx["weights_sha256"]), "the seeded 3B model differs from the fixture's"
    m = ch.GpuModel(cfg, w, max_batch=1, max_len=2048, outputs=ch.OUT_LOGITS)
    a = m.forward([toks])["logits"][0]
    e = float(np.abs(a.astype(np.float64) - fx["logits"]).max())
    print(f"3B Q4_0 L=2048 logits vs oracle: max abs {e:.2e}", flush=True)
    assert e <= 1e-3
    check_argmax(a, fx["logits"], "3B Q4_0 L=2048")
    rng = np.random.default_rng(5)
    short = rand_tokens(rng, 62)
    got = m.forward([short])["logits"][0]
    ref = cr.forward(cfg, w, short, 16, final_att=False, hidden=False)["logits"]
    assert np.abs(got - ref).max() <= 1e-3
    # kernel by kernel, so that no graph captured under the default switches
    # can stand in for the FP32-MFMA kernels; their results must differ in
    # rounding (identical logits would mean the same kernels ran twice)
    monkeypatch.setenv("CIH_FORWARD_GRAPH", "0")
    monkeypatch.setenv("CIH_ATT", "fp32")
    monkeypatch.setenv("CIH_QGEMM", "fp32")
    b = m.forward([toks])["logits"][0]
    diff = float(np.abs(a - b).max())
    print("3B L=2048 default vs FP32-MFMA kernels:", diff, flush=True)
    assert 0.0 < diff <= 1e-3
    m.close()
