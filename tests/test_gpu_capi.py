"""The C caller of the ABI (codon-infer_amd/capi/pipeline.c, built with gcc
against include/codon_hip.h) running pipeline.rs's two call sequences on the
shipped ESM-2 8M weights, checked against the oracle:

* contacts (compute_pipeline_contacts_parallel, pipeline.rs:410-513): the
  contact map within 1e-4 of the oracle's; the top pairs are the highest
  pairs at the requested separation (each within 2e-4 of the oracle's k-th
  score, i.e. no pair the oracle ranks clearly lower), listed by descending
  score; the Cys-Cys enrichment recomputed from them;
* DMS (run_pipeline_dms_with_mode, pipeline.rs:76-315): deltas and entropy
  within 2e-3 of the oracle's scan, the wild-type column exactly 0, and the
  row means / categories of DmsPositionRow::new (export.rs:17-40) recomputed
  from the deltas the program printed.
"""
import os
import subprocess

import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from conftest import PEPTIDE, REPO

pytestmark = pytest.mark.gpu
DRIVER = os.path.join(REPO, "codon-infer_amd", "capi", "pipeline")
# a 60-residue sequence with six cysteines (contacts between them count in the enrichment)
CYS_SEQ = "MKTACLLVGCAAQPEYWGCRTSLNDKCVEFHGAIMTRQCPWSYNLAVGDCKETFRAGHLIS"


def run(*args):
    assert os.path.exists(DRIVER), "capi/pipeline not built (python codon-infer_amd/build.py)"
    r = subprocess.run([DRIVER, *map(str, args)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    return r.stdout.splitlines()


def select_top(probs, n, min_sep, top_l_factor, max_k):
    """The reference's pair selection on a map: scan order, stable sort by
    descending score, top_k = max_k or clamp(round(n * factor), 5, 50)."""
    pairs = [(i, j, float(probs[i, j])) for i in range(n) for j in range(i + min_sep, n)]
    order = sorted(range(len(pairs)), key=lambda t: -pairs[t][2])  # Python's sort is stable
    k = min(max_k, len(pairs)) if max_k else min(max(int(np.floor(n * top_l_factor + 0.5)), 5), 50, len(pairs))
    return [pairs[t] for t in order[:k]]


@pytest.mark.parametrize("seq,min_sep,factor,max_k", [(PEPTIDE, 6, 1.0, 0), (CYS_SEQ, 6, 0.5, 0),
                                                      (CYS_SEQ, 12, 1.0, 7)])
def test_capi_contacts_vs_oracle(w8m_path, tmp_path, seq, min_sep, factor, max_k):
    cfg = ch.EsmConfig.esm2_8m()
    cw, cb = cfg.contact_head_weights()
    head = str(tmp_path / "head.bin")
    np.concatenate([np.asarray(cw, np.float32), [np.float32(cb)]]).astype(np.float32).tofile(head)
    mapf = str(tmp_path / "map.bin")
    lines = run("contacts", w8m_path, head, seq, min_sep, factor, max_k, mapf)
    n = len(seq)
    got = np.fromfile(mapf, np.float32).reshape(n, n)
    w = ch.EsmWeights.from_grouped_canonical(w8m_path, cfg)
    ref = cr.forward(cfg, w, cr.tokenize(seq), 8, contacts=(cw, cb))["contacts"]
    err = float(np.abs(got - ref).max())
    print(f"contacts n={n}: max|map - oracle| = {err:.2e}", flush=True)
    assert err <= 1e-4
    kv = {ln.split()[0]: ln.split()[1:] for ln in lines if not ln.startswith("top ")}
    tops = [ln.split() for ln in lines if ln.startswith("top ")]
    assert int(kv["n"][0]) == n and int(kv["top_k"][0]) == len(tops)
    assert int(kv["n_cys"][0]) == seq.count("C")
    expect = select_top(ref, n, min_sep, factor, max_k)
    assert len(tops) == len(expect)
    kth = expect[-1][2]
    scores = [float(t[5]) for t in tops]
    assert scores == sorted(scores, reverse=True)
    for t in tops:
        i, j = int(t[1]), int(t[3])
        assert j - i >= min_sep and t[2] == seq[i] and t[4] == seq[j]
        assert np.float32(float(t[5])) == got[i, j]
        assert ref[i, j] >= kth - 2e-4, (i, j, ref[i, j], kth)
    # Cys-Cys enrichment from the printed pairs (pipeline.rs:485-502)
    cands = [(i, j) for i in range(n) for j in range(i + min_sep, n)]
    bg = sum(seq[i] == "C" and seq[j] == "C" for i, j in cands) / len(cands)
    top_d = sum(int(t[6]) for t in tops) / len(tops)
    enrich = top_d / bg if bg > 0 else 1.0
    assert abs(float(kv["cys_enrichment"][0]) - enrich) <= 1e-5 * max(1.0, enrich)


@pytest.mark.parametrize("window,stride,mode,chunk", [(0, 0, 0, 16), (20, 0, 0, 7), (16, 5, 1, 0), (0, 0, 1, 0)])
def test_capi_dms_vs_oracle(w8m_path, window, stride, mode, chunk):
    cfg = ch.EsmConfig.esm2_8m()
    lines = run("dms", w8m_path, PEPTIDE, window, stride, mode, chunk)
    rows = [ln.split() for ln in lines if ln.startswith("row ")]
    n = len(PEPTIDE)
    assert len(rows) == n
    deltas = np.array([[float(v) for v in r[6:26]] for r in rows], np.float32)
    ent = np.array([float(r[4]) for r in rows], np.float32)
    w = ch.EsmWeights.from_grouped_canonical(w8m_path, cfg)
    res = cr.tokenize(PEPTIDE)[1:-1]
    rd, re_ = cr.dms(cfg, w, res, window, stride, "masked" if mode == 0 else "wt", 8, cfg.max_seq_len)
    ed, ee = float(np.abs(deltas - rd).max()), float(np.abs(ent - re_).max())
    print(f"dms window={window} stride={stride} mode={mode} chunk={chunk}: deltas {ed:.2e} entropy {ee:.2e}",
          flush=True)
    assert ed <= 2e-3 and ee <= 2e-3
    canon = "ACDEFGHIKLMNPQRSTVWY"
    catalytic = 0
    for p, r in enumerate(rows):
        assert int(r[1]) == p + 1 and r[2] == PEPTIDE[p]
        assert deltas[p, canon.index(PEPTIDE[p])] == 0.0
        nz = deltas[p][deltas[p] != 0.0]
        s = np.float32(0.0)
        for v in nz:
            s = np.float32(s + v)
        mean = np.float32(s / np.float32(19.0))
        assert np.float32(float(r[3])) == mean
        cat = "catalytic" if mean <= np.float32(-3.8) else ("core" if mean <= np.float32(-2.2) else "tolerated")
        assert r[5] == cat
        catalytic += cat == "catalytic"
    kv = {ln.split()[0]: ln.split()[1:] for ln in lines if not ln.startswith("row ")}
    assert int(kv["catalytic_sites"][0]) == catalytic and float(kv["muts_per_sec"][0]) > 0
