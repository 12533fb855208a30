"""The oracle's restatement of the deep mutational scan (pipeline.rs:76-315):
scoring of one row against float64 closed forms, the window arithmetic
against the reference's branches worked by hand, and the row summary
(export.rs DmsPositionRow::new)."""
import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr


def test_uniform_logits():
    d, h = cr.dms_score(np.zeros(33, np.float32), 5)
    assert np.all(d == 0.0)
    assert abs(h - np.log(20.0)) < 1e-6


def test_score_matches_float64():
    rng = np.random.default_rng(0)
    tok = [5, 23, 13, 9, 18, 6, 21, 12, 15, 4, 20, 17, 14, 16, 10, 8, 11, 7, 22, 19]
    assert list(ch.Tokenizer.encode(cr.CANONICAL_AAS)[1:-1]) == tok  # column order = CANONICAL_AAS
    for trial in range(50):
        logits = (rng.standard_normal(33) * 4).astype(np.float32)
        wt = int(rng.integers(4, 24))
        d, h = cr.dms_score(logits, wt)
        l64 = logits.astype(np.float64)
        m = l64[4:24].max()
        lse = m + np.log(np.exp(l64[4:24] - m).sum())
        lp = l64 - lse
        p = np.exp(lp[4:24])
        h64 = -(p * lp[4:24])[p > 1e-12].sum()
        ref = np.array([0.0 if t == wt else lp[t] - lp[wt] for t in tok])
        assert np.abs(d - ref).max() < 2e-5
        assert abs(h - h64) < 2e-5
        assert d[tok.index(wt)] == 0.0  # exactly zero, not a rounded difference


def test_noncanonical_wildtype_is_infinite():
    d, _ = cr.dms_score(np.zeros(33, np.float32), 3)  # <unk>: lp = -inf in the reference's table
    assert np.all(np.isposinf(d))


def test_masked_windows_by_hand():
    # n = 10, window 4 (half 2): p < 2 -> 0; p + 2 > 10 -> 6; else p - 2 (pipeline.rs:111-118)
    aw, w = cr.dms_windows(10, 4, 1024)
    assert aw == 4
    assert [a for a, _ in w] == [0, 0, 0, 1, 2, 3, 4, 5, 6, 6]
    assert all(b == a + 4 for a, b in w)
    # odd window: the comparison is strict (p + half > n), so p = 7 of n = 9
    # keeps the centred start 5 and its window is cut at n to 4 residues
    aw, w = cr.dms_windows(9, 5, 1024)
    assert [a for a, _ in w] == [0, 0, 0, 1, 2, 3, 4, 5, 4]
    assert w[7] == (5, 9) and w[8] == (4, 9)
    # whole protein when it fits or window == 0; max_seq_len caps it
    assert cr.dms_windows(30, 0, 1024)[0] == 30 and cr.dms_windows(30, 40, 1024)[0] == 30
    assert cr.dms_windows(30, 0, 16)[0] == 16


@pytest.mark.parametrize("n,window,stride", [(10, 4, 0), (10, 4, 3), (37, 16, 5), (37, 16, 16), (12, 0, 0)])
def test_wildtype_windows_cover_once(n, window, stride):
    seen = np.zeros(n, int)
    for ws, we, c0, c1 in cr.dms_wt_windows(n, window, stride, 1024):
        assert ws <= c0 <= c1 <= we <= n and we - ws <= (window or n)
        seen[c0:c1] += 1
    assert np.all(seen == 1)


def test_row_summary():
    d = np.zeros(20, np.float32)
    d[:19] = -4.0
    r = ch.DmsPositionRow(3, "A", d, 1.5)
    assert r.mean_delta_logp == np.float32(-4.0) and r.category.startswith("Catalytic")
    d[:19] = -3.0
    assert ch.DmsPositionRow(3, "A", d, 1.5).category == "Conserved Structural Core"
    assert ch.DmsPositionRow(3, "A", np.zeros(20, np.float32), 0.0).category == "Tolerated Variable"
