"""GPU deep mutational scan (cih_dms) against the oracle's restatement of
run_pipeline_dms_with_mode (pipeline.rs:76-315) on the same model and
protein.  Tolerance: deltas and entropy within 2e-3 absolute (log-softmax
differences of logits that agree to 1e-3); the wild-type column exactly 0."""
import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from conftest import PEPTIDE

pytestmark = pytest.mark.gpu
TOL = 2e-3


def check(model, cfg, w, res, window, stride, mode, chunk, nthreads=8):
    got_d, got_e = model.dms(res, window, stride, mode, chunk)
    ref_d, ref_e = cr.dms(cfg, w, res, window, stride, "masked" if mode == ch.DMS_MASKED_MARGINAL else "wt",
                          nthreads, cfg.max_seq_len)
    ed, ee = float(np.abs(got_d - ref_d).max()), float(np.abs(got_e - ref_e).max())
    print(f"dms mode={mode} window={window} stride={stride} chunk={chunk}: deltas {ed:.2e} entropy {ee:.2e}",
          flush=True)
    assert ed <= TOL and ee <= TOL
    assert np.array_equal(got_d == 0.0, ref_d == 0.0)


@pytest.mark.parametrize("dtype", [1, 2])
def test_dms_random_model(dtype):
    rng = np.random.default_rng(40 + dtype)
    cfg = ch.EsmConfig(128, 512, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=40 + dtype, bias_std=0.02)
    w = w.quantize_q8() if dtype == 1 else w.quantize_q4()
    res = (4 + rng.integers(0, 20, 37)).astype(np.int32)
    m = ch.GpuModel(cfg, w, max_batch=8, max_len=40, outputs=ch.OUT_LOGITS)
    check(m, cfg, w, res, 0, 0, ch.DMS_MASKED_MARGINAL, 8)      # whole protein, 5 chunks (last one short)
    check(m, cfg, w, res, 16, 0, ch.DMS_MASKED_MARGINAL, 0)     # centred windows of 16
    check(m, cfg, w, res, 15, 0, ch.DMS_MASKED_MARGINAL, 3)     # odd window: cut windows at the end
    check(m, cfg, w, res, 0, 0, ch.DMS_WILDTYPE_MARGINAL, 0)    # one forward
    check(m, cfg, w, res, 16, 5, ch.DMS_WILDTYPE_MARGINAL, 0)   # sliding windows
    check(m, cfg, w, res, 16, 0, ch.DMS_WILDTYPE_MARGINAL, 0)   # default stride (window / 2)
    with pytest.raises(ch.CihError, match="CAPACITY"):
        m.dms(np.concatenate([res, res]), 0)                    # 74 residues need max_seq_len >= 76
    m.close()


def test_dms_8m_peptide(w8m_path):
    """Shipped 8M weights, the benchmark peptide, masked marginal in chunks of
    16, plus the row summary of the reference's DmsPositionRow."""
    cfg = ch.EsmConfig.esm2_8m()
    w = ch.EsmWeights.from_grouped_canonical(w8m_path, cfg).quantize_q8()
    res = ch.Tokenizer.encode(PEPTIDE)[1:-1]
    m = ch.GpuModel(cfg, w, max_batch=16, max_len=len(res) + 2, outputs=ch.OUT_LOGITS)
    check(m, cfg, w, res, 0, 0, ch.DMS_MASKED_MARGINAL, 16)
    rows, rate = ch.run_pipeline_dms(PEPTIDE, m, chunk=16)
    assert len(rows) == len(PEPTIDE) and rows[0].pos == 1 and rows[0].wt == PEPTIDE[0] and rate > 0
    m.close()


def test_config4_650m_q8_dms_full_shape():
    """Config 4 at its real shape: ESM-2 650M Q8_0, a seeded 400-residue
    protein, masked marginal over all 400 positions in chunks of 32 (12
    batched forwards of 32 masked copies of L = 402 and one of 16,
    pipeline.rs:76-315).  The oracle scores positions 0, 31, 32 (either side
    of the first chunk boundary), 200 and 399 (the last, in the short chunk);
    every row has its wild-type column exactly 0, finite deltas and an
    entropy in [0, ln 20]."""
    rng = np.random.default_rng(400)
    cfg = ch.EsmConfig.esm2_650m()
    w = ch.EsmWeights.random(cfg, seed=4000, bias_std=0.02).quantize_q8()
    res = (4 + rng.integers(0, 20, 400)).astype(np.int32)
    m = ch.GpuModel(cfg, w, max_batch=32, max_len=402, outputs=ch.OUT_LOGITS)
    print("650M Q8_0 DMS, 400 residues, chunks of 32", flush=True)
    got_d, got_e = m.dms(res, 0, 0, ch.DMS_MASKED_MARGINAL, 32)
    m.close()
    canon = "ACDEFGHIKLMNPQRSTVWY"
    aa = "LAGVSERTIDPKQNFYMHWC"  # token ids 4..23
    wt_col = np.array([canon.index(aa[t - 4]) for t in res])
    assert np.all(got_d[np.arange(400), wt_col] == 0.0)
    assert np.isfinite(got_d).all()
    assert np.all((got_e >= 0.0) & (got_e <= np.log(20.0) + 1e-5))
    _, wins = cr.dms_windows(400, 0, cfg.max_seq_len)
    for p in (0, 31, 32, 200, 399):
        ws, we = wins[p]
        toks = np.concatenate([[0], res[ws:we], [2]]).astype(np.int32)
        tp = p - ws + 1
        wt = int(toks[tp])
        toks[tp] = 32
        logits = cr.forward(cfg, w, toks, 16, final_att=False, hidden=False)["logits"]
        rd, re_ = cr.dms_score(logits[tp], wt)
        ed, ee = float(np.abs(got_d[p] - rd).max()), abs(float(got_e[p]) - re_)
        print(f"position {p}: deltas {ed:.2e} entropy {ee:.2e}", flush=True)
        assert ed <= TOL and ee <= TOL
