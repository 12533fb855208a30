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
