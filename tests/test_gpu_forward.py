"""GPU parity of the full batched forward (cih_forward) against the oracle run
one unpadded sequence at a time (forward_bidirectional / _q8 / _q4,
src/lib.rs:5078-6147).

Tolerances (FP32 accumulate throughout):
  logits        max |gpu - oracle| <= 1e-3
  hidden        max |gpu - oracle| <= 1e-3
  attention P   max |gpu - oracle| <= 1e-5
  final_att     max |gpu - oracle| <= 1e-5
  contacts      max |gpu - oracle| <= 1e-4
  argmax        identical wherever the oracle's top-1/top-2 margin exceeds
                twice the measured max |logit error| of that sequence (where
                the argmax provably cannot change); at least 90% of the
                positions must be compared, and the count is printed
"""
import ctypes

import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from conftest import PEPTIDE, decode

pytestmark = pytest.mark.gpu

ALL = ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_FINAL_ATT | ch.OUT_CONTACTS | ch.OUT_ATTN | ch.OUT_LAYER_HIDDEN
TOL = {"logits": 1e-3, "hidden": 1e-3, "attn": 1e-5, "final_att": 1e-5, "contacts": 1e-4, "layer_hidden": 1e-3}


def rand_tokens(rng, n):
    t = np.empty(n + 2, np.int32)
    t[0], t[-1] = 0, 2
    t[1:-1] = 4 + rng.integers(0, 20, n)
    return t


def quantized(w, dtype):
    return w if dtype == 0 else (w.quantize_q8() if dtype == 1 else w.quantize_q4())


def check_argmax(got_logits, ref_logits, tag):
    """Argmax over all 33 ids (ties to the last index, as compute_top1_match_rate,
    lib.rs:2300-2315) identical wherever the oracle's top-1/top-2 gap exceeds
    twice the observed max logit error: a perturbation of at most e per logit
    cannot reorder two logits more than 2e apart."""
    e = float(np.abs(got_logits.astype(np.float64) - ref_logits).max())
    top2 = np.sort(ref_logits, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2.0 * e
    last = lambda a: a.shape[1] - 1 - a[:, ::-1].argmax(1)  # noqa: E731
    print(f"argmax {tag}: {int(clear.sum())}/{clear.size} positions compared (margin {2 * e:.1e})", flush=True)
    assert clear.mean() >= 0.9, (tag, int(clear.sum()), clear.size)
    assert np.array_equal(last(got_logits)[clear], last(ref_logits)[clear]), tag


def check_batch(cfg, w, seqs, flags, contact=None, nthreads=8):
    model = ch.GpuModel(cfg, w, contact_head=contact, max_batch=len(seqs), max_len=max(len(s) for s in seqs),
                        outputs=flags)
    got = model.forward(seqs, flags)
    worst = {}
    for b, toks in enumerate(seqs):
        S = len(toks)
        ref = cr.forward(cfg, w, toks, nthreads, contacts=contact if flags & ch.OUT_CONTACTS else None,
                         attn=bool(flags & ch.OUT_ATTN), layer_hidden=bool(flags & ch.OUT_LAYER_HIDDEN))
        n = S - 2
        pairs = [("logits", got["logits"][b, :S], ref["logits"])]
        if flags & ch.OUT_HIDDEN:
            pairs.append(("hidden", got["hidden"][b, :S], ref["hidden"]))
        if flags & ch.OUT_FINAL_ATT:
            pairs.append(("final_att", got["final_att"][b, :S, :S], ref["final_att"]))
        if flags & ch.OUT_CONTACTS and n > 0:
            pairs.append(("contacts", got["contacts"][b, :n, :n], ref["contacts"]))
        if flags & ch.OUT_ATTN:
            pairs.append(("attn", got["attn"][b, :, :, :S, :S], ref["attn"]))
        if flags & ch.OUT_LAYER_HIDDEN:
            pairs.append(("layer_hidden", got["layer_hidden"][b, :, :S], ref["layer_hidden"]))
        for name, g, r in pairs:
            e = float(np.abs(g.astype(np.float64) - r).max())
            worst[name] = max(worst.get(name, 0.0), e)
            assert e <= TOL[name], (name, b, S, e)
        check_argmax(got["logits"][b, :S], ref["logits"], f"seq {b} (S={S})")
    print("worst abs errors:", {k: f"{v:.2e}" for k, v in worst.items()}, flush=True)
    model.close()
    return got


@pytest.mark.parametrize("act", ["h2", "f32", "x3"])
@pytest.mark.parametrize("hd,H", [(16, 4), (24, 4), (32, 2), (64, 2)])
@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_forward_small_configs(hd, H, dtype, act, monkeypatch):
    """Every head size, every weight format, ragged batch crossing the 32-key
    and 128-query tile edges, all outputs including contacts and maps; every
    activation hand-off to the quantized GEMMs (h2: two f16 limbs written by
    the producers, the default; f32: FP32 split in the GEMM, CIH_ACT=f32;
    x3: three bf16 limbs written by the producers, CIH_ACT=x3)."""
    if act != "h2" and dtype == 0:
        pytest.skip("FP32 weights always hand over FP32")
    if act != "h2":
        monkeypatch.setenv("CIH_ACT", act)
    rng = np.random.default_rng(hd * 10 + dtype)
    d = hd * H
    cfg = ch.EsmConfig(d, 4 * d, 2, H)
    w = quantized(ch.EsmWeights.random(cfg, seed=hd + dtype, bias_std=0.02), dtype)
    cw = rng.standard_normal(cfg.n_layers * H).astype(np.float32)
    cw[::3] = 0.0
    seqs = [rand_tokens(rng, n) for n in (3, 35, 70, 128, 1)]
    seqs[1][5] = 32  # a <mask> changes the embedding scale of that sequence only
    print(f"small config hd={hd} H={H} dtype={dtype}", flush=True)
    check_batch(cfg, w, seqs, ALL, contact=(cw, np.float32(-0.5)))


def test_contacts_forty_heads():
    """Contacts with more than 20 weighted heads per layer (the 3B and 15B
    head count, 40): the map reader's 40-head pass, with a few zero-weight
    heads (skipped as in the reference) so the nonzero count is 34 per layer."""
    rng = np.random.default_rng(4040)
    cfg = ch.EsmConfig(640, 1280, 2, 40)
    w = ch.EsmWeights.random(cfg, seed=4040, bias_std=0.02).quantize_q8()
    cw = rng.standard_normal(cfg.n_layers * 40).astype(np.float32)
    cw[::7] = 0.0
    seqs = [rand_tokens(rng, n) for n in (97, 40, 130)]
    check_batch(cfg, w, seqs, ALL, contact=(cw, np.float32(0.1)))


@pytest.mark.parametrize("hd,H", [(16, 4), (24, 4), (32, 2), (64, 2)])
def test_forward_fp32_attention_kernel(hd, H, monkeypatch):
    """The FP32-MFMA attention kernel (CIH_ATT=fp32), kept for A/B runs, on
    the same ragged batch and outputs as the default f16-limb kernel."""
    monkeypatch.setenv("CIH_ATT", "fp32")
    rng = np.random.default_rng(hd * 10 + 7)
    d = hd * H
    cfg = ch.EsmConfig(d, 4 * d, 2, H)
    w = ch.EsmWeights.random(cfg, seed=hd + 7, bias_std=0.02).quantize_q8()
    cw = rng.standard_normal(cfg.n_layers * H).astype(np.float32)
    seqs = [rand_tokens(rng, n) for n in (3, 35, 70, 128, 1)]
    check_batch(cfg, w, seqs, ALL, contact=(cw, np.float32(-0.5)))


def test_forward_8m_peptide(w8m_path):
    """Shipped 8M weights: every format reproduces the published prediction
    (docs/benchmarks_v1.6.0.md:61-62) and matches the oracle within tolerance."""
    cfg = ch.EsmConfig.esm2_8m()
    w = ch.EsmWeights.from_grouped_canonical(w8m_path, cfg)
    toks = ch.Tokenizer.encode(PEPTIDE)
    masked = ch.Tokenizer.encode("MCMP*TTD")
    for dtype in (0, 1, 2):
        print(f"8M peptide dtype={dtype}", flush=True)
        got = check_batch(cfg, quantized(w, dtype), [toks, masked], ALL, contact=cfg.contact_head_weights())
        assert decode(got["logits"][0, 1:len(toks) - 1].argmax(1)) == PEPTIDE


@pytest.mark.parametrize("splitk", ["0", "1"])
def test_forward_batch_invariance(splitk, monkeypatch):
    """A sequence's outputs do not depend on its batch neighbours: bit-identical
    alone and inside a ragged batch while every GEMM runs unsplit
    (CIH_SPLITK=0); with split-K (the default for GEMMs too small to fill the
    GPU) the k-summation is regrouped, so alone and batched agree to 1e-5."""
    monkeypatch.setenv("CIH_SPLITK", splitk)
    rng = np.random.default_rng(3)
    cfg = ch.EsmConfig(128, 512, 2, 2)
    w = ch.EsmWeights.random(cfg, seed=9, bias_std=0.02).quantize_q8()
    seqs = [rand_tokens(rng, n) for n in (50, 200, 17)]
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN
    m = ch.GpuModel(cfg, w, max_batch=3, max_len=202, outputs=flags)
    batch = m.forward(seqs, flags)
    for b, s in enumerate(seqs):
        alone = m.forward([s], flags)
        S = len(s)
        for name in ("logits", "hidden"):
            if splitk == "0":
                assert np.array_equal(alone[name][0, :S], batch[name][b, :S]), name
            else:
                assert np.abs(alone[name][0, :S] - batch[name][b, :S]).max() <= 1e-5, name
    m.close()


@pytest.mark.parametrize("arch,dtype,B,lo,hi", [("35M", 1, 4, 20, 130), ("150M", 2, 2, 60, 100)])
def test_forward_preset_archs(arch, dtype, B, lo, hi):
    """Preset ESM-2 shapes (35M Q8_0 ragged, 150M Q4_0 with contacts) at
    oracle-friendly lengths."""
    rng = np.random.default_rng(11)
    cfg = ch.EsmConfig.by_name(arch)
    w = quantized(ch.EsmWeights.random(cfg, seed=1, bias_std=0.02), dtype)
    seqs = [rand_tokens(rng, int(rng.integers(lo, hi))) for _ in range(B)]
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_FINAL_ATT | ch.OUT_CONTACTS
    print(f"preset {arch} dtype={dtype}", flush=True)
    check_batch(cfg, w, seqs, flags, contact=cfg.contact_head_weights())


@pytest.mark.parametrize("lens", [(300, 220), (300, 400), (650, 650, 650, 650)])
def test_planned_splits_vs_oracle(lens):
    """d = 640 with FC2 K = 5120 over two layers, Q8_0: the planned k-splits
    of the residual projections, which leave their partial sums to the
    LayerNorm after them.  524 tokens: Wo and FC2 on 64 x 64 tiles in 2
    splits, each tile's k-blocks shared by two groups of 4 waves (180
    workgroups); 704 tokens: FC2 on 64 x 128 tiles in 3 splits, also on two
    wave groups; 2608 tokens: Wo unsplit, FC2 on 128 x 128 tiles in 3."""
    rng = np.random.default_rng(21)
    cfg = ch.EsmConfig(640, 5120, 2, 20)
    w = ch.EsmWeights.random(cfg, seed=21, bias_std=0.02).quantize_q8()
    seqs = [rand_tokens(rng, n) for n in lens]
    print(f"planned splits, {sum(lens) + 2 * len(lens)} tokens", flush=True)
    check_batch(cfg, w, seqs, ch.OUT_LOGITS | ch.OUT_HIDDEN, nthreads=16)


def test_forward_650m_q8_short():
    """The headline architecture (650M, Q8_0) on two short sequences, then on
    six residues alone (8 tokens: every linear layer on the GEMV path)."""
    rng = np.random.default_rng(12)
    cfg = ch.EsmConfig.esm2_650m()
    w = ch.EsmWeights.random(cfg, seed=2, bias_std=0.02).quantize_q8()
    seqs = [rand_tokens(rng, 62), rand_tokens(rng, 40)]
    print("650M Q8 short", flush=True)
    check_batch(cfg, w, seqs, ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_FINAL_ATT, nthreads=16)
    print("650M Q8 GEMV path (T = 8)", flush=True)
    check_batch(cfg, w, [rand_tokens(rng, 6)], ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_FINAL_ATT, nthreads=16)


def test_forward_headline_shape(monkeypatch):
    """The benchmark workload itself (650M Q8_0, B=16, L=512: the largest GEMM
    tiles and the f16-limb hand-off at full size).  One sequence of the batch
    against the oracle; with every split off (CIH_SPLITK=0: the LM head's
    33-wide decoder GEMM splits K by default even here), another sequence is
    bit-identical alone and inside the batch, and the default batch agrees
    with the unsplit one to 1e-5."""
    rng = np.random.default_rng(650)
    cfg = ch.EsmConfig.esm2_650m()
    w = ch.EsmWeights.random(cfg, seed=650, bias_std=0.02).quantize_q8()
    seqs = [rand_tokens(rng, 510) for _ in range(16)]
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN
    m = ch.GpuModel(cfg, w, max_batch=16, max_len=512, outputs=flags)
    print("650M Q8 B=16 L=512", flush=True)
    got = m.forward(seqs, flags)
    ref = cr.forward(cfg, w, seqs[0], 16, final_att=False)
    for name in ("logits", "hidden"):
        e = float(np.abs(got[name][0].astype(np.float64) - ref[name]).max())
        print(name, f"{e:.2e}", flush=True)
        assert e <= TOL[name], (name, e)
    check_argmax(got["logits"][0], ref["logits"], "650M Q8 headline seq 0")
    monkeypatch.setenv("CIH_SPLITK", "0")
    monkeypatch.setenv("CIH_FORWARD_GRAPH", "0")  # a replayed graph keeps the splits it was captured with
    unsplit = m.forward(seqs, flags)
    assert float(np.abs(unsplit["logits"] - got["logits"]).max()) <= 1e-5
    alone = m.forward([seqs[5]], flags)
    assert np.array_equal(alone["logits"][0], unsplit["logits"][5])
    m.close()


@pytest.mark.parametrize("gemv", ["on", "fp32", "off"])
@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_forward_few_tokens(dtype, gemv, monkeypatch):
    """Batches of at most 8 tokens in total run every layer projection on
    the few-token f16-MFMA GEMV with limb hand-off (quantized weights), or
    on the FP32 weight-streaming GEMV (FP32 weights; CIH_GEMV16=0), or on
    the MFMA GEMMs (CIH_GEMV=0); all outputs, with a <mask>, a sequence with
    no residues (BOS, EOS) and contacts."""
    if gemv == "off":
        monkeypatch.setenv("CIH_GEMV", "0")
    if gemv == "fp32":
        if dtype == 0:
            pytest.skip("FP32 weights always take the FP32 GEMV")
        monkeypatch.setenv("CIH_GEMV16", "0")
    rng = np.random.default_rng(21 + dtype)
    cfg = ch.EsmConfig(128, 512, 2, 4)
    w = quantized(ch.EsmWeights.random(cfg, seed=5 + dtype, bias_std=0.02), dtype)
    cw = rng.standard_normal(cfg.n_layers * cfg.n_heads).astype(np.float32)
    for lens in ([2], [1, 2], [0, 1, 1], [6]):  # at most 8 tokens per batch
        seqs = [rand_tokens(rng, n) for n in lens]
        if len(seqs[0]) > 3:
            seqs[0][2] = 32
        print(f"few tokens dtype={dtype} gemv={gemv} residues={lens}", flush=True)
        check_batch(cfg, w, seqs, ALL, contact=(cw, np.float32(0.25)))


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("hd", [32, 64])
def test_few_tokens_attention_with_wo(dtype, hd, monkeypatch):
    """Few tokens without maps and head sizes of whole 32-wide blocks: the
    8-token attention also applies each head's share of Wo (k_attn_few_wo,
    the heads as the projection's splits).  Logits and hidden state against
    the oracle, and against attention and Wo run apart (CIH_FEW_WO=0) to
    1e-5."""
    rng = np.random.default_rng(hd + dtype)
    cfg = ch.EsmConfig(4 * hd, 16 * hd, 2, 4)
    w = quantized(ch.EsmWeights.random(cfg, seed=hd + 10 * dtype, bias_std=0.02), dtype)
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN
    for lens in ([2], [1, 2], [0, 1, 1], [6]):  # at most 8 tokens per batch
        seqs = [rand_tokens(rng, n) for n in lens]
        print(f"attention + Wo hd={hd} dtype={dtype} residues={lens}", flush=True)
        monkeypatch.delenv("CIH_FEW_WO", raising=False)
        fused = check_batch(cfg, w, seqs, flags)
        monkeypatch.setenv("CIH_FEW_WO", "0")
        apart = check_batch(cfg, w, seqs, flags)
        for k in ("logits", "hidden"):
            for b, t in enumerate(seqs):
                e = float(np.abs(fused[k][b, :len(t)] - apart[k][b, :len(t)]).max())
                assert e <= 1e-5, (k, b, e)


@pytest.mark.parametrize("T", [8, 40])
def test_forward_graph_replays_match_eager(T, monkeypatch):
    """Forwards of a shape seen before replay a captured graph (keyed by
    batch, padded length, token count, 32-key tile count and outputs).
    Different lengths with the same token count reuse one graph; every
    replay, with eager forwards and host syncs in between, equals the
    kernel-by-kernel run bit for bit."""
    rng = np.random.default_rng(T)
    cfg = ch.EsmConfig(128, 512, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=T, bias_std=0.02).quantize_q8()
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.1).astype(np.float32)
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_CONTACTS | ch.OUT_FINAL_ATT
    half = T // 2
    splits = [(half + 1, T - half - 1), (half, T - half), (half - 1, T - half + 1), (half, T - half)]
    S_max = T - half + 1
    mg = ch.GpuModel(cfg, w, contact_head=(cw, 0.3), max_batch=2, max_len=S_max, outputs=flags)
    me = ch.GpuModel(cfg, w, contact_head=(cw, 0.3), max_batch=2, max_len=S_max, outputs=flags)
    for a, b in splits:
        seqs = [rand_tokens(rng, a - 2), rand_tokens(rng, b - 2)]
        monkeypatch.setenv("CIH_FORWARD_GRAPH", "1")
        got = mg.forward(seqs, flags)
        monkeypatch.setenv("CIH_FORWARD_GRAPH", "0")
        ref = me.forward(seqs, flags)
        for k in ("logits", "hidden", "contacts", "final_att"):
            for i, s in enumerate(seqs):
                n = len(s)
                g, r = got[k][i], ref[k][i]
                g, r = (g[:n - 2, :n - 2], r[:n - 2, :n - 2]) if k == "contacts" else \
                       ((g[:n, :n], r[:n, :n]) if k == "final_att" else (g[:n], r[:n]))
                assert np.array_equal(g, r), (T, a, b, k)
    mg.close()
    me.close()


@pytest.mark.parametrize("path", ["staged", "prep", "epilogue"])
def test_forward_graph_replays_ragged_lengths(path, monkeypatch):
    """Ragged batches of one size, longest sequence and token count whose
    lengths differ in 32-key tiles and in 128- and 256-query blocks, one
    after another through the graph path, each equal bit for bit to a
    forward launched kernel by kernel: attention staging K/V itself (head
    size 32), K/V images from the prep kernel (head size 24), and images
    from the QKV projection's LDS GEMM epilogue (head size 64, d = 1280)."""
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_FINAL_ATT
    if path == "staged":
        cfg, L, rest = ch.EsmConfig(128, 512, 2, 4), 200, [(99, 60, 41), (96, 64, 40), (130, 35, 35), (97, 66, 37)]
    elif path == "prep":
        monkeypatch.setenv("CIH_ATT_IMG", "prep")
        monkeypatch.setenv("CIH_ATT_SPLIT", "0")
        cfg, L, rest = ch.EsmConfig(96, 384, 2, 4), 150, [(96, 64, 34), (97, 64, 33), (128, 32, 34), (65, 65, 64)]
    else:
        cfg, L, rest = ch.EsmConfig(1280, 5120, 2, 20), 510, [(384, 288, 208), (400, 257, 223), (256, 256, 368),
                                                              (500, 190, 190)]
    rng = np.random.default_rng(len(path))
    w = ch.EsmWeights.random(cfg, seed=len(path), bias_std=0.02).quantize_q8()
    mg = ch.GpuModel(cfg, w, max_batch=4, max_len=L, outputs=flags)
    me = ch.GpuModel(cfg, w, max_batch=4, max_len=L, outputs=flags)
    for lens in rest:
        assert max(lens) <= L and sum(lens) == sum(rest[0])
        seqs = [rand_tokens(rng, L - 2)] + [rand_tokens(rng, n - 2) for n in lens]
        monkeypatch.setenv("CIH_FORWARD_GRAPH", "1")
        got = mg.forward(seqs, flags)
        monkeypatch.setenv("CIH_FORWARD_GRAPH", "0")
        ref = me.forward(seqs, flags)
        print(path, "lengths", [len(t) for t in seqs], flush=True)
        for k in ("logits", "hidden", "final_att"):
            for i, t in enumerate(seqs):
                n = len(t)
                g, r = (got[k][i][:n, :n], ref[k][i][:n, :n]) if k == "final_att" else (got[k][i][:n], ref[k][i][:n])
                assert np.array_equal(g, r), (path, lens, k, i)
    mg.close()
    me.close()


def test_host_outputs_leave_padding_untouched():
    """Host-pointer outputs of a ragged batch (every kind) are written inside
    each sequence's rows, columns and maps only: buffers filled with a
    sentinel keep it in the padding, and hold the same values as a forward
    into zeroed buffers everywhere else (the copies run through pinned
    staging in whole padded rows, of which only the kept part is copied)."""
    from codon_hip import _lib as C
    rng = np.random.default_rng(12)
    cfg = ch.EsmConfig(64, 256, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=12, bias_std=0.02).quantize_q8()
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.1).astype(np.float32)
    flags = (ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_FINAL_ATT | ch.OUT_CONTACTS | ch.OUT_ATTN |
             ch.OUT_LAYER_HIDDEN)
    seqs = [rand_tokens(rng, n) for n in (28, 59, 3)]
    m = ch.GpuModel(cfg, w, contact_head=(cw, 0.3), max_batch=3, max_len=61, outputs=flags)
    ref = m.forward(seqs, flags)
    B, S = len(seqs), max(len(t) for t in seqs)
    lens = np.array([len(t) for t in seqs], np.int32)
    toks = np.zeros((B, S), np.int32)
    for b, t in enumerate(seqs):
        toks[b, :len(t)] = t
    d, V, L, H, n = cfg.dim, cfg.vocab_size, cfg.n_layers, cfg.n_heads, S - 2
    SENT = np.float32(12345.0)
    got = {"logits": (B, S, V), "hidden": (B, S, d), "final_att": (B, S, S), "contacts": (B, n, n),
           "attn": (B, L, H, S, S), "layer_hidden": (B, L, S, d)}
    got = {k: np.full(shape, SENT, np.float32) for k, shape in got.items()}
    o = C.Outputs()
    for k, a in got.items():
        setattr(o, k, a.ctypes.data)
    C.check(C.lib().cih_forward(m._h, toks.ctypes.data, lens.ctypes.data, B, S, flags, ctypes.byref(o)))
    m.close()
    print("sentinel-filled host outputs: written regions equal, padding untouched", flush=True)
    for b, t in enumerate(seqs):
        nb, nc = len(t), max(len(t) - 2, 0)
        inside = {"logits": (np.s_[b, :nb], np.s_[b, nb:]), "hidden": (np.s_[b, :nb], np.s_[b, nb:]),
                  "layer_hidden": (np.s_[b, :, :nb], np.s_[b, :, nb:])}
        for k, (ins, pad) in inside.items():
            assert np.array_equal(got[k][ins], ref[k][ins]), (k, b)
            assert np.all(got[k][pad] == SENT), (k, b)
        for k, m_ in (("final_att", nb), ("contacts", nc), ("attn", nb)):
            a, r = got[k][b], ref[k][b]
            assert np.array_equal(a[..., :m_, :m_], r[..., :m_, :m_]), (k, b)
            assert np.all(a[..., m_:, :] == SENT) and np.all(a[..., :m_, m_:] == SENT), (k, b)


def test_tied_embedding_decoder():
    """A classifier shorter than the LM head selects logits = x . emb^T
    (lib.rs:5427-5439, Q8: 5775-5787)."""
    rng = np.random.default_rng(4)
    cfg = ch.EsmConfig(64, 256, 2, 4)
    for dtype in (0, 1, 2):
        w = quantized(ch.EsmWeights.random(cfg, seed=4, bias_std=0.02), dtype)
        w.classifier_weights = w.classifier_weights[:10]
        check_batch(cfg, w, [rand_tokens(rng, 30)], ch.OUT_LOGITS | ch.OUT_HIDDEN)


def test_forward_errors():
    cfg = ch.EsmConfig(64, 256, 1, 4)
    w = ch.EsmWeights.random(cfg, seed=0)
    m = ch.GpuModel(cfg, w, max_batch=2, max_len=16, outputs=ch.OUT_LOGITS)
    with pytest.raises(ch.CihError, match="CAPACITY"):
        m.forward([np.zeros(20, np.int32)])
    with pytest.raises(ch.CihError, match="CAPACITY"):
        m.forward([np.zeros(5, np.int32)], ch.OUT_LOGITS | ch.OUT_HIDDEN)
    with pytest.raises(ch.CihError, match="TOKEN"):
        m.forward([np.array([0, 40, 2], np.int32)])
    with pytest.raises(ch.CihError, match="CONTACTS|ARG"):
        m.reserve(1, 1030, ch.OUT_CONTACTS)
    m.close()


@pytest.mark.parametrize("with_maps", [False, True])
def test_attention_query_block_size_is_invisible(with_maps, monkeypatch):
    """256 queries per attention workgroup (chosen on large batches) and 128
    give the same bits: each query's scores, softmax and P.V do not depend on
    the block it is computed in."""
    rng = np.random.default_rng(31)
    cfg = ch.EsmConfig(128, 512, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=31, bias_std=0.02).quantize_q8()
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.1).astype(np.float32)
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN | (ch.OUT_CONTACTS | ch.OUT_FINAL_ATT if with_maps else 0)
    seqs = [rand_tokens(rng, n) for n in (298, 97, 255, 30)]
    monkeypatch.setenv("CIH_ATT_SPLIT", "0")  # the key split (tested below) depends on the block size
    res = {}
    for qb in ("128", "256"):
        monkeypatch.setenv("CIH_ATT_QB", qb)
        m = ch.GpuModel(cfg, w, contact_head=(cw, 0.3), max_batch=4, max_len=300, outputs=flags)
        res[qb] = m.forward(seqs, flags)
        m.close()
    keys = ("logits", "hidden") + (("contacts", "final_att") if with_maps else ())
    for k in keys:
        for i, s in enumerate(seqs):
            n = len(s)
            a, b = res["128"][k][i], res["256"][k][i]
            a, b = (a[:n - 2, :n - 2], b[:n - 2, :n - 2]) if k == "contacts" else \
                   ((a[:n, :n], b[:n, :n]) if k == "final_att" else (a[:n], b[:n]))
            assert np.array_equal(a, b), (with_maps, k, i)


@pytest.mark.parametrize("case", ["one", "three", "short"])
def test_attention_key_split(case, monkeypatch):
    """Attention tasks (sequence, head, query block) that do not fill one round
    of workgroup slots run as key ranges whose partial softmax results a merge
    kernel combines: one 402-token sequence (80 tasks of 128 queries, six
    ranges), or three ragged sequences; a 252-token sequence (160 tasks of 32
    queries, at most one workgroup per CU) runs each 32-query task on 8
    waves that split its keys (k_attention_xs, one pass).  The forward agrees
    with the unsplit one (CIH_ATT_SPLIT=0) to 1e-5 and with the oracle to the
    stated tolerances."""
    rng = np.random.default_rng(77)
    cfg = ch.EsmConfig(320, 1280, 2, 20)
    lens = {"one": [400], "three": [300, 61, 190], "short": [250]}[case]
    seqs = [rand_tokens(rng, n) for n in lens]
    w = ch.EsmWeights.random(cfg, seed=77, bias_std=0.02).quantize_q8()
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN
    res = {}
    for sp in ("0", "1"):
        monkeypatch.setenv("CIH_ATT_SPLIT", sp)
        m = ch.GpuModel(cfg, w, max_batch=len(seqs), max_len=max(len(t) for t in seqs), outputs=flags)
        res[sp] = m.forward(seqs, flags)
        m.close()
    for i, t in enumerate(seqs):
        n = len(t)
        for k in ("logits", "hidden"):
            e = float(np.abs(res["1"][k][i, :n] - res["0"][k][i, :n]).max())
            assert e <= 1e-5, (case, i, k, e)
    ref = cr.forward(cfg, w, seqs[-1], 4, final_att=False)
    n = len(seqs[-1])
    for k in ("logits", "hidden"):
        e = float(np.abs(res["1"][k][-1, :n].astype(np.float64) - ref[k]).max())
        print(case, k, f"{e:.2e}", flush=True)
        assert e <= TOL[k], (case, k, e)


@pytest.mark.parametrize("maps", [True, False])
@pytest.mark.parametrize("hd", [16, 24, 32, 64])
@pytest.mark.parametrize("case", ["one", "two"])
def test_attention_wave_key_split(hd, case, maps, monkeypatch):
    """Batches whose 32-query tasks fit one round of one workgroup per CU run
    each task on 8 waves that split its keys (k_attention_xs; with the
    probability export, or the one-pass kernel): one 256-token sequence (8
    tiles, one per wave) or two ragged ones (partial tiles, waves without a
    tile).  Every output agrees with the unsplit kernels (CIH_ATT_SPLIT=0) to
    1e-5; the maps of the last sequence agree with the oracle to 1e-5, or
    its logits to the stated tolerance."""
    rng = np.random.default_rng(hd + (0 if case == "one" else 500))
    d = 20 * hd
    cfg = ch.EsmConfig(d, 4 * d, 2, 20)
    lens = [254] if case == "one" else [61, 140]
    seqs = [rand_tokens(rng, n) for n in lens]
    w = ch.EsmWeights.random(cfg, seed=hd, bias_std=0.02).quantize_q8()
    cw = (rng.standard_normal(cfg.n_layers * cfg.n_heads) * 0.1).astype(np.float32)
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN | ((ch.OUT_ATTN | ch.OUT_FINAL_ATT | ch.OUT_CONTACTS) if maps else 0)
    keys = ("logits", "hidden") + (("attn", "final_att", "contacts") if maps else ())
    res = {}
    for sp in ("0", "1"):
        monkeypatch.setenv("CIH_ATT_SPLIT", sp)
        m = ch.GpuModel(cfg, w, contact_head=(cw, 0.3), max_batch=len(seqs), max_len=max(len(t) for t in seqs),
                        outputs=flags)
        res[sp] = m.forward(seqs, flags)
        m.close()
    for i, t in enumerate(seqs):
        n = len(t)
        for k in keys:
            a, b = res["1"][k][i], res["0"][k][i]
            if k == "attn":
                a, b = a[:, :, :n, :n], b[:, :, :n, :n]
            elif k == "final_att":
                a, b = a[:n, :n], b[:n, :n]
            elif k == "contacts":
                a, b = a[:n - 2, :n - 2], b[:n - 2, :n - 2]
            else:
                a, b = a[:n], b[:n]
            e = float(np.abs(a - b).max())
            assert e <= 1e-5, (hd, case, i, k, e)
    n = len(seqs[-1])
    if maps:
        ref = cr.forward(cfg, w, seqs[-1], 16, attn=True)
        e = float(np.abs(res["1"]["attn"][-1, :, :, :n, :n] - ref["attn"]).max())
        print(f"hd {hd} {case}: maps vs oracle {e:.2e}", flush=True)
        assert e <= 1e-5
    else:
        ref = cr.forward(cfg, w, seqs[-1], 16, final_att=False)
        e = float(np.abs(res["1"]["logits"][-1, :n].astype(np.float64) - ref["logits"]).max())
        print(f"hd {hd} {case}: logits vs oracle {e:.2e}", flush=True)
        assert e <= TOL["logits"]


def test_device_io_token_validation():
    """With CIH_IO_DEVICE the token ids are checked on the device: an id
    outside [0, vocab) returns CIH_ERR_TOKEN (as the host path does) instead
    of being computed with a clamped id; the next valid forward on the same
    workspace (and the same captured graph) succeeds and matches the host
    path."""
    from codon_hip.devmem import Hip
    rng = np.random.default_rng(90)
    cfg = ch.EsmConfig(128, 512, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=90, bias_std=0.02).quantize_q8()
    S, B = 40, 2
    flags = ch.OUT_LOGITS
    m = ch.GpuModel(cfg, w, max_batch=B, max_len=S, outputs=flags | ch.IO_DEVICE)
    hip = Hip()
    d_tok, d_log = hip.malloc(B * S * 4), hip.malloc(B * S * cfg.vocab_size * 4)
    seqs = [rand_tokens(rng, S - 2), rand_tokens(rng, 25)]
    toks = np.zeros((B, S), np.int32)
    for b, s in enumerate(seqs):
        toks[b, :len(s)] = s
    lens = [len(s) for s in seqs]
    try:
        for bad in (40, -1, 33):
            t = toks.copy()
            t[1, 7] = bad
            hip.h2d(d_tok, t)
            with pytest.raises(ch.CihError, match="TOKEN"):
                m.forward_device(d_tok, lens, S, flags, {"logits": d_log})
        hip.h2d(d_tok, toks)
        for _ in range(2):
            m.forward_device(d_tok, lens, S, flags, {"logits": d_log})
            got = np.zeros((B, S, cfg.vocab_size), np.float32)
            hip.d2h(got, d_log)
            m2 = ch.GpuModel(cfg, w, max_batch=B, max_len=S, outputs=flags)
            ref = m2.forward(seqs, flags)
            m2.close()
            for b in range(B):
                assert np.array_equal(got[b, :lens[b]], ref["logits"][b, :lens[b]])
    finally:
        hip.free(d_tok)
        hip.free(d_log)
        m.close()


@pytest.mark.parametrize("dtype", [1, 2])
def test_limb_overflow_runs_full_range(dtype):
    """An activation the f16 limbs cannot hold: layer 0's LN1 output is
    ~7e4 in one column (bias 7e4) whose Q, K and V weights are zero, so the
    reference's result does not depend on it, while the f16 hi limb is inf
    and inf * 0 = NaN in the MFMA.  The forward detects the non-finite
    residual and runs again with the full-range kernels: results match the
    oracle at the usual tolerances, with the default f16-limb hand-off and
    with the FP32 one (CIH_ACT=f32, split inside the GEMM)."""
    rng = np.random.default_rng(91 + dtype)
    cfg = ch.EsmConfig(128, 512, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=91, bias_std=0.02)
    d, c = cfg.dim, 37
    b1 = np.array(w.ln_1_bias, np.float32)
    b1[c] = 7.0e4
    w.ln_1_bias = b1
    for name in ("wq", "wk", "wv"):
        a = np.array(getattr(w, name), np.float32).reshape(cfg.n_layers, d, d)
        a[0, :, c] = 0.0
        setattr(w, name, a.ravel())
    w = quantized(w, dtype)
    seqs = [rand_tokens(rng, n) for n in (60, 33)]
    check_batch(cfg, w, seqs, ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_FINAL_ATT)


@pytest.mark.parametrize("where", ["final_ln", "lm_head_ln"])
def test_lm_head_input_beyond_limbs_runs_full_range(where):
    """A LayerNorm output the f16 limbs of the LM head's GEMMs cannot hold:
    column 37 of the final LayerNorm (bias 7e4; the dense weights of that
    column zero) or of the LM head's own LayerNorm (bias 7e4; the decoder's
    weights of that column zero) is ~7e4, so the reference's logits do not
    depend on it, while a hi limb of f16(7e4) = inf gives inf * 0 = NaN.
    The LayerNorm flags the value, the forward runs again with the FP32-MFMA
    LM head and the logits match the oracle."""
    rng = np.random.default_rng(95)
    cfg = ch.EsmConfig(128, 512, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=95, bias_std=0.02)
    d, V, c = cfg.dim, cfg.vocab_size, 37
    cw = np.array(w.classifier_weights, np.float32)  # [ln_w d, ln_b d, dense_w d*d, dense_b d, dec_w V*d, dec_b V]
    if where == "final_ln":
        fb = np.array(w.ln_f_bias, np.float32)
        fb[c] = 7.0e4
        w.ln_f_bias = fb
        cw[2 * d:2 * d + d * d].reshape(d, d)[:, c] = 0.0
    else:
        cw[d + c] = 7.0e4
        cw[3 * d + d * d:3 * d + d * d + V * d].reshape(V, d)[:, c] = 0.0
    w.classifier_weights = cw
    w = w.quantize_q8()
    seqs = [rand_tokens(rng, n) for n in (60, 33)]
    # logits only: a hidden state of ~7e4 carries 1-ulp (0.0078) differences
    # whenever the rounding of the small part differs
    check_batch(cfg, w, seqs, ch.OUT_LOGITS)


def test_graph_key_follows_kernel_switches(monkeypatch):
    """A captured forward is keyed by the kernel switches read while it was
    enqueued: with graphs on, CIH_ATT=fp32 after a default forward of the same
    shape runs the FP32-MFMA attention (rounding differs), and unsetting it
    replays the default graph bit for bit."""
    rng = np.random.default_rng(92)
    cfg = ch.EsmConfig(128, 512, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=92, bias_std=0.02).quantize_q8()
    seqs = [rand_tokens(rng, 70), rand_tokens(rng, 50)]
    flags = ch.OUT_LOGITS | ch.OUT_HIDDEN
    monkeypatch.setenv("CIH_FORWARD_GRAPH", "1")
    m = ch.GpuModel(cfg, w, max_batch=2, max_len=72, outputs=flags)
    a = m.forward(seqs, flags)
    monkeypatch.setenv("CIH_ATT", "fp32")
    b = m.forward(seqs, flags)
    monkeypatch.delenv("CIH_ATT")
    c = m.forward(seqs, flags)
    m.close()
    diff = float(np.abs(a["hidden"] - b["hidden"]).max())
    assert 0.0 < diff <= 1e-3, diff
    assert np.array_equal(a["hidden"], c["hidden"]) and np.array_equal(a["logits"], c["logits"])
