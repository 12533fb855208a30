"""K/V tile images (csrc/kv_image.h): attention reading keys and values that
the QKV projection's epilogue (LDS GEMM, EPI_QKV*) or the prep kernel (other
projection paths) laid out as f16 limbs, against attention staging them from
the FP32 Q|K|V rows itself (CIH_ATT_IMG=0), and against the oracle.

Both paths rotate with the same rounding (rot_lo / rot_hi), split into the
same limbs and run the same arithmetic in the same order, so the maps and
outputs must be bit-identical (which is what keeps a sequence's results
independent of the batch it runs in: large batches take the image path, small
ones the staged one); against the oracle, the tolerances of test_gpu_forward.
Batches cover each head size with a ragged batch large enough for the LDS
GEMM (the epilogue writes the images: sequences start inside 32-row GEMM
tiles, so both the whole-line and the element-wise V stores run; head size
24, which has no epilogue form, takes the prep kernel there), a small batch,
the prep kernel (CIH_ATT_IMG=prep: images from FP32 rows at any size) and
every layer's maps (the two-pass export kernel).  The key splits are off
(CIH_ATT_SPLIT=0): batches small enough for attention's split over waves
stage K/V themselves under every setting, and the split regroups sums
(test_gpu_forward covers it).
"""
import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from test_gpu_forward import rand_tokens

pytestmark = pytest.mark.gpu

FLAGS = ch.OUT_LOGITS | ch.OUT_HIDDEN


def run_paths(monkeypatch, cfg, w, seqs, flags):
    """Outputs of the default path, the staged path (CIH_ATT_IMG=0), the prep
    kernel's images (CIH_ATT_IMG=prep) and the default path again."""
    monkeypatch.setenv("CIH_FORWARD_GRAPH", "0")
    monkeypatch.setenv("CIH_ATT_SPLIT", "0")
    m = ch.GpuModel(cfg, w, max_batch=len(seqs), max_len=max(len(s) for s in seqs), outputs=flags)
    out = {"default": m.forward(seqs, flags)}
    for tag, v in (("staged", "0"), ("prep", "prep")):
        monkeypatch.setenv("CIH_ATT_IMG", v)
        out[tag] = m.forward(seqs, flags)
    monkeypatch.delenv("CIH_ATT_IMG")
    out["again"] = m.forward(seqs, flags)
    m.close()
    return out


@pytest.mark.parametrize("hd,n_seq,lo,hi", [(64, 6, 190, 420), (32, 9, 250, 420), (24, 9, 250, 420),
                                             (16, 13, 300, 420), (64, 2, 20, 90), (32, 3, 5, 40), (24, 2, 10, 60),
                                             (16, 2, 1, 33)])
def test_image_vs_staged(monkeypatch, hd, n_seq, lo, hi):
    d = 20 * hd
    cfg = ch.EsmConfig(d, 4 * d, 2, 20)
    rng = np.random.default_rng(hd * 100 + n_seq)
    w = ch.EsmWeights.random(cfg, seed=hd + n_seq, bias_std=0.02).quantize_q8()
    seqs = [rand_tokens(rng, int(rng.integers(lo, hi))) for _ in range(n_seq)]
    print(f"hd {hd}: {n_seq} sequences, {sum(len(s) for s in seqs)} tokens", flush=True)
    out = run_paths(monkeypatch, cfg, w, seqs, FLAGS)
    for name in ("logits", "hidden"):
        for tag in ("staged", "prep", "again"):
            e = float(np.abs(out["default"][name] - out[tag][name]).max())
            print(f"  {name}: max |default - {tag}| = {e:.2e}", flush=True)
            assert np.array_equal(out["default"][name], out[tag][name]), (name, tag, e)
    img = out["default"]
    b = n_seq - 1
    S = len(seqs[b])
    ref = cr.forward(cfg, w, seqs[b], 16, final_att=False)
    e = float(np.abs(img["logits"][b, :S].astype(np.float64) - ref["logits"]).max())
    print(f"  logits vs oracle (sequence {b}): {e:.2e}", flush=True)
    assert e <= 1e-3


@pytest.mark.parametrize("hd", [64, 32, 24, 16])
def test_image_maps_vs_staged(monkeypatch, hd):
    """Every layer's attention maps and the final-layer mean: the two-pass
    export kernel on images (prep kernel) bit-identical to its staged twin,
    and one sequence's maps against the oracle."""
    d = 20 * hd
    cfg = ch.EsmConfig(d, 4 * d, 2, 20)
    rng = np.random.default_rng(7 + hd)
    w = ch.EsmWeights.random(cfg, seed=70 + hd, bias_std=0.02).quantize_q8()
    seqs = [rand_tokens(rng, int(rng.integers(100, 300))) for _ in range(4)]
    flags = FLAGS | ch.OUT_ATTN | ch.OUT_FINAL_ATT
    out = run_paths(monkeypatch, cfg, w, seqs, flags)
    for name in ("attn", "final_att"):
        for tag in ("staged", "prep"):
            e = float(np.abs(out["default"][name] - out[tag][name]).max())
            print(f"hd {hd} {name}: max |default - {tag}| = {e:.2e}", flush=True)
            assert np.array_equal(out["default"][name], out[tag][name]), (name, tag, e)
    img = out["default"]
    S = len(seqs[0])
    ref = cr.forward(cfg, w, seqs[0], 16, attn=True)
    e = float(np.abs(img["attn"][0, :, :, :S, :S] - ref["attn"]).max())
    print(f"hd {hd} maps vs oracle: {e:.2e}", flush=True)
    assert e <= 1e-5


def test_graph_replay_with_another_tile_count(monkeypatch):
    """Two batches with the same size, longest sequence and token count but
    a different number of 32-key tiles (lengths 34, 31, 31: 4 tiles; 34, 34,
    28: 5 tiles).  The prep kernel runs one wave per tile and head, so the
    second batch must not replay the first one's captured forward: its
    outputs equal a forward launched without graphs."""
    monkeypatch.setenv("CIH_ATT_IMG", "prep")
    monkeypatch.setenv("CIH_ATT_SPLIT", "0")
    cfg = ch.EsmConfig(96, 384, 2, 4)  # head size 24
    w = ch.EsmWeights.random(cfg, seed=24, bias_std=0.02).quantize_q8()
    rng = np.random.default_rng(24)
    first = [rand_tokens(rng, n) for n in (32, 29, 29)]
    second = [rand_tokens(rng, n) for n in (32, 32, 26)]
    assert sum(map(len, first)) == sum(map(len, second)) == 96
    m = ch.GpuModel(cfg, w, max_batch=3, max_len=34, outputs=FLAGS)
    m.forward(first, FLAGS)
    got = m.forward(second, FLAGS)
    monkeypatch.setenv("CIH_FORWARD_GRAPH", "0")
    ref = m.forward(second, FLAGS)
    m.close()
    print("second batch after the first: outputs of the graph path equal a forward without graphs", flush=True)
    for name in ("logits", "hidden"):
        for i, s in enumerate(second):
            assert np.array_equal(got[name][i][:len(s)], ref[name][i][:len(s)]), (name, i)
