"""The LDS-staged quantized GEMM (csrc/gemm_lds.hip: operands loaded global ->
LDS by the load unit, quants read from an f16 copy made at model load, or,
in a model loaded without that copy, the quants themselves converted on the
LDS -> register path) against the register-staged GEMM (csrc/gemm_x3.hip) it
replaces on large batches.  All three compute matmul_tiled_q8/q4_parallel
(src/lib.rs:4870, 4937) with the same operations in the same order, so whole
forwards must agree bit for bit: a wrong swizzle, load count, stage
rotation, k assignment or f16 expansion changes the result.

A model built with CIH_GEMM_F16=0 has no f16 copy; CIH_GEMM_LDS=0 keeps every
GEMM on the register-staged kernel, CIH_GEMM_LDS=force sends every eligible
GEMM (activations in f16 limbs) to the LDS-staged one.  CIH_SPLITK=0 keeps
the register-staged kernel from splitting K on small shapes (a split sums
the blocks in another order).
"""
import numpy as np
import pytest

import codon_hip as ch

pytestmark = pytest.mark.gpu

FLAGS = ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_CONTACTS


def rand_tokens(rng, n):
    t = np.empty(n + 2, np.int32)
    t[0], t[-1] = 0, 2
    t[1:-1] = 4 + rng.integers(0, 20, n)
    return t


def two_models(monkeypatch, cfg, w, cw, max_batch, max_len):
    monkeypatch.setenv("CIH_GEMM_F16", "0")
    ref = ch.GpuModel(cfg, w, contact_head=(cw, 0.2), max_batch=max_batch, max_len=max_len, outputs=FLAGS)
    monkeypatch.delenv("CIH_GEMM_F16")
    lds = ch.GpuModel(cfg, w, contact_head=(cw, 0.2), max_batch=max_batch, max_len=max_len, outputs=FLAGS)
    return ref, lds


def assert_same(got, ref, seqs, what):
    for i, s in enumerate(seqs):
        n = len(s)
        for k in ("logits", "hidden", "contacts"):
            g, r = got[k][i], ref[k][i]
            g, r = (g[:n - 2, :n - 2], r[:n - 2, :n - 2]) if k == "contacts" else (g[:n], r[:n])
            assert np.array_equal(g, r), (what, i, k, float(np.abs(g - r).max()))


@pytest.mark.parametrize("tile", ["model", "128", "160", "256", "320", "64x128", "64"])
@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_forced_lds_gemm_is_bit_identical(fmt, tile, monkeypatch):
    """Ragged shapes: token count 687 and projection widths 576 / 192 / 768
    are not multiples of any tile (128 x 128, 128 x 160, 128 x 256,
    128 x 320, 64 x 128 and 64 x 64, forced through CIH_GEMM_TILE_N, or the
    round model's choice), FC2 has K = 768.  The two small tiles read the f16
    copy only: the model without it takes 128 x 128 for them."""
    if tile != "model":
        monkeypatch.setenv("CIH_GEMM_TILE_N", tile)
    rng = np.random.default_rng(11)
    cfg = ch.EsmConfig(192, 768, 2, 3)
    w = ch.EsmWeights.random(cfg, seed=11, bias_std=0.02)
    w = w.quantize_q8() if fmt == "q8" else w.quantize_q4()
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.1).astype(np.float32)
    seqs = [rand_tokens(rng, 298), rand_tokens(rng, 255), rand_tokens(rng, 128)]
    ref, lds = two_models(monkeypatch, cfg, w, cw, 3, 300)
    monkeypatch.setenv("CIH_SPLITK", "0")
    monkeypatch.setenv("CIH_GEMM_LDS", "0")
    a = ref.forward(seqs, FLAGS)
    monkeypatch.setenv("CIH_GEMM_LDS", "force")
    b = lds.forward(seqs, FLAGS)
    c = ref.forward(seqs, FLAGS)
    print(f"{fmt} tile {tile}: forced LDS GEMM forwards (f16 copy, quants) equal the register-staged one", flush=True)
    assert_same(b, a, seqs, fmt + " f16 copy")
    assert_same(c, a, seqs, fmt + " quants")
    ref.close()
    lds.close()


def test_650m_headline_batch_is_bit_identical(monkeypatch):
    """ESM-2 650M Q8_0, 16 sequences of 510 residues (8192 tokens): the
    default tile choice (128 x 320 for every projection, K = 1280 and
    5120)."""
    rng = np.random.default_rng(650)
    cfg = ch.EsmConfig.esm2_650m()
    w = ch.EsmWeights.random(cfg, seed=650, bias_std=0.02).quantize_q8()
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.05).astype(np.float32)
    seqs = [rand_tokens(rng, 510) for _ in range(16)]
    ref, lds = two_models(monkeypatch, cfg, w, cw, 16, 512)
    monkeypatch.setenv("CIH_GEMM_LDS", "0")
    a = ref.forward(seqs, FLAGS)
    monkeypatch.delenv("CIH_GEMM_LDS")
    b = lds.forward(seqs, FLAGS)
    c = ref.forward(seqs, FLAGS)
    print("650M B=16 L=512: LDS GEMM forwards (f16 copy, quants) equal the register-staged one", flush=True)
    assert_same(b, a, seqs, "650M f16 copy")
    assert_same(c, a, seqs, "650M quants")
    ref.close()
    lds.close()


@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_planned_routing_is_bit_identical(fmt, monkeypatch):
    """The default route of f16-limb GEMMs from 64 rows on (gemm_lds_plan:
    64 x 64 tiles here, 687 and 273 tokens) gives the register-staged
    kernel's bits with every split off, as does the route without the plan
    (CIH_GEMM_PLAN=0)."""
    rng = np.random.default_rng(13)
    cfg = ch.EsmConfig(192, 768, 2, 3)
    w = ch.EsmWeights.random(cfg, seed=13, bias_std=0.02)
    w = w.quantize_q8() if fmt == "q8" else w.quantize_q4()
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.1).astype(np.float32)
    m = ch.GpuModel(cfg, w, contact_head=(cw, 0.2), max_batch=3, max_len=300, outputs=FLAGS)
    monkeypatch.setenv("CIH_SPLITK", "0")
    for lens in ((298, 255, 128), (150, 117)):
        seqs = [rand_tokens(rng, n) for n in lens]
        monkeypatch.setenv("CIH_GEMM_LDS", "0")
        a = m.forward(seqs, FLAGS)
        monkeypatch.delenv("CIH_GEMM_LDS")
        b = m.forward(seqs, FLAGS)
        monkeypatch.setenv("CIH_GEMM_PLAN", "0")
        c = m.forward(seqs, FLAGS)
        monkeypatch.delenv("CIH_GEMM_PLAN")
        print(f"{fmt} {sum(lens) + 2 * len(lens)} tokens: planned and unplanned routes equal the register-staged one",
              flush=True)
        assert_same(b, a, seqs, fmt + " planned")
        assert_same(c, a, seqs, fmt + " unplanned")
    m.close()


@pytest.mark.parametrize("dims", [(192, 768, 3), (96, 384, 4)])
def test_persistent_workgroups_are_bit_identical(dims, monkeypatch):
    """The persistent form of the 128 x 320 tile (FC1 + GELU, and the plain
    QKV projection of head size 24, which has no image epilogue): 8
    workgroups stride over all tiles (CIH_GEMM_PERSIST=force), each running
    the stage ring on from one tile into the next, and the forwards equal
    the register-staged kernel's bit for bit."""
    d, f, H = dims
    rng = np.random.default_rng(17)
    cfg = ch.EsmConfig(d, f, 2, H)
    w = ch.EsmWeights.random(cfg, seed=17, bias_std=0.02).quantize_q8()
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.1).astype(np.float32)
    seqs = [rand_tokens(rng, 298), rand_tokens(rng, 255), rand_tokens(rng, 128)]
    m = ch.GpuModel(cfg, w, contact_head=(cw, 0.2), max_batch=3, max_len=300, outputs=FLAGS)
    monkeypatch.setenv("CIH_SPLITK", "0")
    monkeypatch.setenv("CIH_GEMM_LDS", "0")
    a = m.forward(seqs, FLAGS)
    monkeypatch.setenv("CIH_GEMM_LDS", "force")
    monkeypatch.setenv("CIH_GEMM_TILE_N", "320")
    monkeypatch.setenv("CIH_GEMM_PERSIST", "force")
    b = m.forward(seqs, FLAGS)
    monkeypatch.setenv("CIH_GEMM_PERSIST", "0")
    c = m.forward(seqs, FLAGS)
    print(f"d={d}: persistent and one-tile workgroups equal the register-staged forward", flush=True)
    assert_same(b, a, seqs, "persistent")
    assert_same(c, a, seqs, "one tile per workgroup")
    m.close()


def test_fp32_pair_copy_is_bit_identical(monkeypatch):
    """FP32 weights run as f16 pair copies (an f16 matrix of 2K whose block
    kb meets activation block kb mod K/32) with the activations handed over
    as f16 limbs; from 64 rows on they take the LDS GEMM's planned tiles,
    and the forward equals the register-staged kernel's pair path bit for
    bit, with limbs or with FP32 activations split inside it (CIH_ACT=f32;
    splits off; ESM-2 8M widths)."""
    rng = np.random.default_rng(19)
    cfg = ch.EsmConfig(320, 1280, 2, 20)
    w = ch.EsmWeights.random(cfg, seed=19, bias_std=0.02)
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.1).astype(np.float32)
    m = ch.GpuModel(cfg, w, contact_head=(cw, 0.2), max_batch=2, max_len=300, outputs=FLAGS)
    monkeypatch.setenv("CIH_SPLITK", "0")
    for lens in ((298, 120), (70,)):
        seqs = [rand_tokens(rng, n) for n in lens]
        monkeypatch.setenv("CIH_GEMM_LDS", "0")
        a = m.forward(seqs, FLAGS)
        monkeypatch.setenv("CIH_ACT", "f32")  # FP32 hand-off, split inside the register-staged GEMM
        c = m.forward(seqs, FLAGS)
        monkeypatch.delenv("CIH_ACT")
        monkeypatch.delenv("CIH_GEMM_LDS")
        b = m.forward(seqs, FLAGS)
        print(f"FP32 pair copy, {sum(lens) + 2 * len(lens)} tokens: LDS GEMM equals the register-staged one", flush=True)
        assert_same(b, a, seqs, "fp32 pair")
        assert_same(c, a, seqs, "fp32 hand-off")
    m.close()


def assert_close(got, ref, seqs, what, tol=2e-5):
    for i, s in enumerate(seqs):
        n = len(s)
        for k in ("logits", "hidden", "contacts"):
            g, r = got[k][i], ref[k][i]
            g, r = (g[:n - 2, :n - 2], r[:n - 2, :n - 2]) if k == "contacts" else (g[:n], r[:n])
            e = float(np.abs(g.astype(np.float64) - r).max())
            assert e <= tol * max(1.0, float(np.abs(r).max())), (what, i, k, e)


@pytest.mark.parametrize("kw", ["2", "4"])
@pytest.mark.parametrize("case", ["q8", "q4", "f32", "q8-d480", "q8-deep"])
def test_k_groups_match_one_group(case, kw, monkeypatch):
    """Groups of 4 waves sharing a 64 x 64 tile's k-blocks (group g takes
    blocks kb0 + g, kb0 + g + KW, ...; the groups' sums are added in group
    order): the k-sum is regrouped, so the forward agrees with one group to
    2e-5 of the largest value, not bit for bit, with the residual k-splits
    off and on, from the f16 copy of the quants and from FP32 pair copies.
    d = 480 gives Wo 15 k-blocks, which 2 and 4 groups do not divide (a
    group's last step computes nothing); d = 640 with K = 5120 at 704 tokens
    puts FC2 on 64 x 128 tiles in 3 splits (which take 2 groups for either
    count)."""
    rng = np.random.default_rng(23)
    d, f, H = {"f32": (320, 1280, 20), "q8-d480": (480, 1920, 20), "q8-deep": (640, 5120, 20)}.get(case, (192, 768, 3))
    cfg = ch.EsmConfig(d, f, 2, H)
    w = ch.EsmWeights.random(cfg, seed=23, bias_std=0.02)
    if case != "f32":
        w = w.quantize_q4() if case == "q4" else w.quantize_q8()
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.1).astype(np.float32)
    lens = (298, 255, 128) if d == 192 else ((300, 400) if d == 640 else (298, 200))
    seqs = [rand_tokens(rng, n) for n in lens]
    m = ch.GpuModel(cfg, w, contact_head=(cw, 0.2), max_batch=3, max_len=402, outputs=FLAGS)
    monkeypatch.setenv("CIH_SPLITK", "0")
    monkeypatch.setenv("CIH_GEMM_KW", "1")
    a = m.forward(seqs, FLAGS)
    monkeypatch.setenv("CIH_GEMM_KW", kw)
    b = m.forward(seqs, FLAGS)
    monkeypatch.delenv("CIH_SPLITK")
    c = m.forward(seqs, FLAGS)
    print(f"{case}, {sum(lens) + 2 * len(lens)} tokens: {kw} k-groups agree with one group, splits off and on",
          flush=True)
    assert_close(b, a, seqs, case + " groups")
    assert_close(c, a, seqs, case + " groups + splits")
    m.close()


@pytest.mark.parametrize("case", ["8m-fp32", "650m-width-q8"])
def test_lm_head_limb_handoff_is_bit_identical(case, monkeypatch):
    """Without a hidden-state export the final LayerNorm hands the LM head's
    dense layer (FP32 weights through their pair copy) f16 limbs instead of
    FP32 rows; the GEMM made the same split itself, so with every k-split off
    (CIH_SPLITK=0: the register-staged kernel splits the FP32-row form at
    small batches) the logits equal the FP32 hand-off's (a forward that also
    exports the hidden state) bit for bit, on the LDS-staged kernel and on
    the register-staged one (CIH_GEMM_LDS=0).  d = 320 FP32 at 422 tokens:
    the 64 x 64 tiles; d = 1280 at 4608 tokens: 128 x 320 tiles with the pair
    copy's wrap."""
    rng = np.random.default_rng(29)
    if case == "8m-fp32":
        cfg = ch.EsmConfig(320, 1280, 2, 20)
        w = ch.EsmWeights.random(cfg, seed=29, bias_std=0.02)
        lens = (298, 120)
    else:
        cfg = ch.EsmConfig(1280, 5120, 2, 20)
        w = ch.EsmWeights.random(cfg, seed=29, bias_std=0.02).quantize_q8()
        lens = (510,) * 9
    seqs = [rand_tokens(rng, n) for n in lens]
    both = ch.OUT_LOGITS | ch.OUT_HIDDEN
    m = ch.GpuModel(cfg, w, max_batch=len(seqs), max_len=max(len(s) for s in seqs), outputs=both)
    monkeypatch.setenv("CIH_SPLITK", "0")
    a = m.forward(seqs, ch.OUT_LOGITS)
    b = m.forward(seqs, both)
    monkeypatch.setenv("CIH_GEMM_LDS", "0")
    c = m.forward(seqs, ch.OUT_LOGITS)
    m.close()
    print(f"{case}, {sum(len(s) for s in seqs)} tokens: LM head on limbs equals the FP32 hand-off", flush=True)
    for i, s in enumerate(seqs):
        n = len(s)
        assert np.array_equal(a["logits"][i, :n], b["logits"][i, :n]), (case, i)
        assert np.array_equal(c["logits"][i, :n], b["logits"][i, :n]), (case, i)
