"""GPU autoregressive decoding (cih_decode / cih_generate) against the
oracle's forward_step / generate (forward, forward_q8, forward_q4 with a KV
cache and generate_sequence*, src/lib.rs:3554-4233, 6538-6827).

Tolerance: logits within 1e-3 absolute at every step (observed ~1e-5);
generated token ids identical (greedy and seeded sampling).  Rows of one
call that take the GEMV (at most 8) are computed independently of each
other, so a stream decoded alone or next to others is bit-identical.
"""
import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def w8m_all(w8m_path):
    cfg = ch.EsmConfig.esm2_8m()
    w = ch.EsmWeights.from_grouped_canonical(w8m_path, cfg)
    return cfg, {"fp32": w, "q8": w.quantize_q8(), "q4": w.quantize_q4()}


def report(what, got, ref):
    err = float(np.abs(got - ref).max())
    print(f"{what}: max|dlogit| = {err:.2e}", flush=True)
    assert err <= TOL, (what, err)


@pytest.mark.parametrize("fmt", ["fp32", "q8", "q4"])
def test_steps_match_oracle(w8m_all, fmt):
    cfg, ws = w8m_all
    w = ws[fmt]
    toks = [0, 20, 5, 32, 11, 11, 23, 4, 17, 9, 30, 12]
    m = ch.GpuModel(cfg, w, max_batch=1, max_len=16)
    dec = ch.GpuDecoder(m, n_slots=2, max_len=64, max_rows=16)
    rs = cr.RunState(cfg, w, max_len=64, num_threads=8)
    for p, t in enumerate(toks):
        got = dec.decode([1], [t], [p])[0]
        report(f"{fmt} step {p}", got, rs.step(t, p))
    # the whole prompt in one call (12 rows: the MFMA GEMM path)
    dec.reset()
    rows = dec.decode(np.zeros(len(toks)), toks, np.arange(len(toks)))
    rs2 = cr.RunState(cfg, w, max_len=64, num_threads=8)
    ref = np.stack([rs2.step(t, p) for p, t in enumerate(toks)])
    report(f"{fmt} prefill of 12 rows", rows, ref)
    dec.close()
    m.close()


def test_slots_are_independent_and_batch_invariant(w8m_all):
    cfg, ws = w8m_all
    w = ws["q8"]
    m = ch.GpuModel(cfg, w, max_batch=1, max_len=16)
    prompts = [[0, 20, 5, 7], [0, 11, 12], [0, 4, 4, 4, 4, 9]]
    # every slot alone, one position per call
    alone = []
    for s, pr in enumerate(prompts):
        dec = ch.GpuDecoder(m, n_slots=3, max_len=32, max_rows=8)
        alone.append(np.stack([dec.decode([s], [t], [p])[0] for p, t in enumerate(pr)]))
        dec.close()
    # all slots together, interleaved, one position of each live slot per call
    dec = ch.GpuDecoder(m, n_slots=3, max_len=32, max_rows=8)
    together = [[] for _ in prompts]
    for p in range(max(map(len, prompts))):
        live = [s for s, pr in enumerate(prompts) if p < len(pr)]
        lg = dec.decode(live, [prompts[s][p] for s in live], [p] * len(live))
        for j, s in enumerate(live):
            together[s].append(lg[j])
    for s, pr in enumerate(prompts):
        assert np.array_equal(alone[s], np.stack(together[s])), s
        rs = cr.RunState(cfg, w, max_len=32, num_threads=8)
        report(f"slot {s}", alone[s], np.stack([rs.step(t, p) for p, t in enumerate(pr)]))
    dec.close()
    m.close()


def test_graph_replays_match_eager(w8m_all, monkeypatch):
    """Decode steps replay a captured graph; every replay, with eager prefill
    calls and host syncs in between, equals the kernel-by-kernel run."""
    cfg, ws = w8m_all
    m = ch.GpuModel(cfg, ws["q4"], max_batch=1, max_len=16)
    d_graph = ch.GpuDecoder(m, n_slots=2, max_len=64, max_rows=16)
    d_eager = ch.GpuDecoder(m, n_slots=2, max_len=64, max_rows=16)
    prompt = [0, 20, 5, 7, 9, 11, 4, 4, 13, 6]                   # 10 rows: eager in both
    for dec in (d_graph, d_eager):
        monkeypatch.setenv("CIH_DECODE_GRAPH", "1" if dec is d_graph else "0")
        dec.decode(np.zeros(10), prompt, np.arange(10))
        dec.decode(np.ones(4), prompt[:4], np.arange(4))
    rng = np.random.default_rng(2)
    p1 = 4                                                       # next position of slot 1
    for step in range(20):
        t = (4 + rng.integers(0, 20, 3)).astype(np.int32)
        if step % 3 == 2:                                        # two rows of slot 1: the unfused kernels
            rows = ([0, 1, 1], t, [10 + step, p1, p1 + 1])
            p1 += 2
        else:                                                    # one row per slot: the fused kernel
            rows = ([0, 1], t[:2], [10 + step, p1])
            p1 += 1
        monkeypatch.setenv("CIH_DECODE_GRAPH", "1")
        a = d_graph.decode(*rows)
        monkeypatch.setenv("CIH_DECODE_GRAPH", "0")
        b = d_eager.decode(*rows)
        assert np.array_equal(a, b), step
    d_graph.close()
    d_eager.close()
    m.close()


def test_row_validation(w8m_all):
    cfg, ws = w8m_all
    m = ch.GpuModel(cfg, ws["q8"], max_batch=1, max_len=16)
    dec = ch.GpuDecoder(m, n_slots=2, max_len=16, max_rows=4)
    with pytest.raises(ch.CihError, match="continue"):
        dec.decode([0], [5], [3])                                # slot 0 has nothing yet
    dec.decode([0, 0], [0, 5], [0, 1])
    with pytest.raises(ch.CihError, match="continue"):
        dec.decode([0, 0], [5, 6], [2, 4])                       # a gap inside one call
    dec.decode([0], [7], [1])                                    # rewriting a position is allowed
    with pytest.raises(ch.CihError):
        dec.decode([2], [5], [0])                                # no slot 2
    with pytest.raises(ch.CihError):
        dec.decode([1], [40], [0])                               # token outside the vocabulary
    with pytest.raises(ch.CihError):
        dec.decode([1] * 5, [5] * 5, list(range(5)))             # more rows than reserved
    with pytest.raises(ch.CihError):
        dec.decode([1], [5], [16])                               # beyond max_len
    dec.close()
    m.close()


@pytest.mark.parametrize("fmt,temperature,seed", [("q8", 0.0, 0), ("q8", 1.0, 7), ("fp32", 4.0, 3),
                                                  ("q4", 1.0, 11)])
def test_generate_matches_oracle(w8m_all, fmt, temperature, seed):
    cfg, ws = w8m_all
    w = ws[fmt]
    m = ch.GpuModel(cfg, w, max_batch=1, max_len=16)
    dec = ch.GpuDecoder(m, n_slots=4, max_len=128, max_rows=32)
    prompts = [ch.prompt_tokens("MKTAYIAKQR"), ch.prompt_tokens(""), ch.prompt_tokens("GSHMLEDPVA" * 2)]
    got, pre, gen = dec.generate(prompts, temperature, 40, [seed, seed + 1, seed + 2], max_seq_len=128)
    for i, pr in enumerate(prompts):
        ref = cr.generate(cfg, w, pr, temperature, 40, seed + i, max_seq_len=128, num_threads=8)
        print(f"{fmt} T={temperature} stream {i}: {got[i].size} tokens, oracle {ref.size}", flush=True)
        assert np.array_equal(got[i], ref), (i, got[i], ref)
    # each stream alone gives the same tokens
    for i, pr in enumerate(prompts):
        solo, _, _ = dec.generate([pr], temperature, 40, [seed + i], slots=[3], max_seq_len=128)
        assert np.array_equal(solo[0], got[i])
    dec.close()
    m.close()


def test_generate_sequence_mirror(w8m_all):
    cfg, ws = w8m_all
    m = ch.GpuModel(cfg, ws["q8"], max_batch=1, max_len=16)
    dec = ch.GpuDecoder(m, n_slots=1, max_len=cfg.max_seq_len, max_rows=16)
    g = ch.generate_sequence("MKV", dec, temperature=0.0, max_new_tokens=12, seed=0)
    ref = cr.generate(cfg, ws["q8"], ch.prompt_tokens("MKV"), 0.0, 12, 0, num_threads=8)
    assert g.tokens_generated == ref.size and g.full_sequence.startswith("MKV")
    assert g.generated_suffix == "".join(ch.Tokenizer.decode(t) for t in ref)
    assert g.throughput_tps > 0
    dec.close()
    m.close()


def test_650m_q8_decode_steps():
    cfg = ch.EsmConfig.esm2_650m()
    w = ch.EsmWeights.random(cfg, seed=650, bias_std=0.02).quantize_q8()
    m = ch.GpuModel(cfg, w, max_batch=1, max_len=16)
    dec = ch.GpuDecoder(m, n_slots=1, max_len=64, max_rows=8)
    rs = cr.RunState(cfg, w, max_len=64, num_threads=16)
    for p, t in enumerate([0, 20, 15, 7, 32, 9]):
        report(f"650M q8 step {p}", dec.decode([0], [t], [p])[0], rs.step(t, p))
    dec.close()
    m.close()


@pytest.mark.gpu
@pytest.mark.parametrize("d,heads,fmt", [(256, 4, "q4"), (128, 4, "q8"), (64, 4, "q8"), (480, 20, "q8"),
                                          (1280, 20, "q4"), (2048, 32, "q8")])
def test_decode_layernorm_in_gemv(d, heads, fmt, monkeypatch):
    """One stream: the residual LayerNorms run inside the QKV and FC1 GEMVs
    (every workgroup normalises the row; the residual alternates between two
    buffers).  Rows of one to two quads per thread, partial waves (d = 480:
    120 quads), the largest row taken (2048).  Same bits as the separate
    residual LayerNorm kernel (CIH_DECODE_LN=0) at every step, and steps
    against the oracle."""
    cfg = ch.EsmConfig(d, 4 * d, 2 if d > 256 else 3, heads)
    w = ch.EsmWeights.random(cfg, seed=100 + d, bias_std=0.02)
    w = w.quantize_q8() if fmt == "q8" else w.quantize_q4()
    toks = [0, 20, 15, 7, 32, 9, 11]
    got = {}
    for env in ("1", "0"):
        monkeypatch.setenv("CIH_DECODE_LN", env)
        m = ch.GpuModel(cfg, w, max_batch=1, max_len=16)
        dec = ch.GpuDecoder(m, n_slots=1, max_len=32, max_rows=8)
        got[env] = [dec.decode([0], [t], [p])[0].copy() for p, t in enumerate(toks)]
        dec.close()
        m.close()
    for p in range(len(toks)):
        assert np.array_equal(got["1"][p], got["0"][p]), (p, float(np.abs(got["1"][p] - got["0"][p]).max()))
    rs = cr.RunState(cfg, w, max_len=32, num_threads=8)
    for p, t in enumerate(toks):
        report(f"d {d} {fmt} step {p}", got["1"][p], rs.step(t, p))


@pytest.mark.parametrize("hd,fmt,streams", [(64, "q4", 2), (32, "q8", 2), (64, "q8", 1), (32, "q4", 1)])
def test_decode_attention_with_wo(hd, fmt, streams, monkeypatch):
    """Head sizes 32 and 64 with quantized weights: each (row, head, column
    chunk) workgroup of the decode attention also applies the head's share of
    Wo (the heads as the projection's splits; 128 columns per workgroup for
    one row, 256 for two).  Steps against the oracle, and against attention
    and Wo run apart (CIH_FEW_WO=0) to 1e-5."""
    cfg = ch.EsmConfig(4 * hd, 16 * hd, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=hd, bias_std=0.02)
    w = w.quantize_q8() if fmt == "q8" else w.quantize_q4()
    toks = [[0, 20, 15, 7, 32, 9], [0, 5, 11, 24, 6, 13]][:streams]
    sl = list(range(streams))
    got = {}
    for env in ("1", "0"):
        monkeypatch.setenv("CIH_FEW_WO", env)
        m = ch.GpuModel(cfg, w, max_batch=1, max_len=16)
        dec = ch.GpuDecoder(m, n_slots=2, max_len=32, max_rows=8)
        got[env] = [dec.decode(sl, list(col), [p] * streams) for p, col in enumerate(zip(*toks))]
        dec.close()
        m.close()
    for p in range(len(toks[0])):
        for s in range(streams):
            e = float(np.abs(got["1"][p][s] - got["0"][p][s]).max())
            assert e <= 1e-5, (p, s, e)
    for s in range(streams):
        rs = cr.RunState(cfg, w, max_len=32, num_threads=8)
        for p, t in enumerate(toks[s]):
            report(f"hd {hd} {fmt} stream {s} step {p}", got["1"][p][s], rs.step(t, p))


def overflow_model(where, seed):
    """A model whose reference results do not depend on one activation column
    that the f16 limbs cannot hold (~7e4, past f16's 65504): layer 0's LN1
    column 37 (Q, K, V weights of that column zero) or the LM head's
    LayerNorm column 37 (decoder weights of that column zero)."""
    cfg = ch.EsmConfig(128, 512, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=seed, bias_std=0.02)
    d, V, c = cfg.dim, cfg.vocab_size, 37
    if where == "ln1":
        b1 = np.array(w.ln_1_bias, np.float32)
        b1[c] = 7.0e4
        w.ln_1_bias = b1
        for name in ("wq", "wk", "wv"):
            a = np.array(getattr(w, name), np.float32).reshape(cfg.n_layers, d, d)
            a[0, :, c] = 0.0
            setattr(w, name, a.ravel())
    else:
        cw = np.array(w.classifier_weights, np.float32)
        cw[d + c] = 7.0e4
        cw[3 * d + d * d:3 * d + d * d + V * d].reshape(V, d)[:, c] = 0.0
        w.classifier_weights = cw
    return cfg, w.quantize_q8()


@pytest.mark.parametrize("rows", [1, 2])
def test_limb_overflow_decode_steps_run_full_range(rows):
    """Decode analogue of test_limb_overflow_runs_full_range: every step of
    one stream (LayerNorms inside the QKV and FC1 GEMVs, attention with Wo,
    replayed graph) or of two streams overflows the f16 limbs in layer 0; the
    NaN reaches the final LayerNorm, the step runs again in full range,
    rewriting the same cache positions, and every step and the steps after
    it match the oracle."""
    cfg, w = overflow_model("ln1", 96)
    m = ch.GpuModel(cfg, w, max_batch=1, max_len=16)
    dec = ch.GpuDecoder(m, n_slots=rows, max_len=32, max_rows=16)
    refs = [cr.RunState(cfg, w, max_len=32, num_threads=4) for _ in range(rows)]
    for p in range(8):
        toks = [0 if p == 0 else 4 + (7 * p + 3 * s) % 20 for s in range(rows)]
        got = dec.decode(list(range(rows)), toks, [p] * rows)
        for s in range(rows):
            report(f"rows {rows} slot {s} step {p}", got[s], refs[s].step(toks[s], p))
    dec.close()
    m.close()


def test_lm_head_input_beyond_limbs_in_prefill():
    """A 12-row prefill (the MFMA GEMMs, f16 limbs) whose LM-head LayerNorm
    writes ~7e4: flagged, the rows run again in full range (FP32-MFMA LM
    head) and match the oracle; the one-row steps after it (FP32 GEMV LM
    head, no limbs) too."""
    cfg, w = overflow_model("lm_head", 97)
    m = ch.GpuModel(cfg, w, max_batch=1, max_len=16)
    dec = ch.GpuDecoder(m, n_slots=1, max_len=32, max_rows=16)
    rs = cr.RunState(cfg, w, max_len=32, num_threads=4)
    toks = [0, 20, 5, 32, 11, 11, 23, 4, 17, 9, 30, 12]
    rows = dec.decode(np.zeros(len(toks)), toks, np.arange(len(toks)))
    report("prefill of 12 rows", rows, np.stack([rs.step(t, p) for p, t in enumerate(toks)]))
    for p in range(len(toks), len(toks) + 3):
        report(f"step {p}", dec.decode([0], [7], [p])[0], rs.step(7, p))
    dec.close()
    m.close()
