"""GPU model residency: weight files loaded straight to the device and FP32
weights quantized there.

* The device quantizer equals the oracle's quantizers (quantize_slice_to_q8
  / _q4, lib.rs:670-673, 1085-1088, pinned against the reference's
  known-answer tests) and the host one byte for byte, including zero blocks,
  NaN, infinities, subnormals, values near 1e37, exact .5 ties and
  equal-magnitude maxima of opposite sign.
* The shipped ESM-2 8M weights file (grouped_canonical_v1), loaded through
  cih_model_create_from_file as FP32 and quantized to Q8_0 / Q4_0 on the
  device, agrees with the oracle's forward of the same weights (logits
  <= 1e-3, last-layer map <= 1e-5, contacts <= 1e-4) and reconstructs the
  published 39/39 peptide (docs/benchmarks_v1.6.0.md:61-62).
* A model loaded from a file (CODQ Q8_0 / Q4_0 / FP32, headerless
  grouped_canonical_v1, sequential_hf) produces bit-identical logits and
  hidden states to the same weights handed over as host tensors, and an FP32
  file loaded with quantize_to equals the host-quantized weights: identical
  device matrices are the only way the same kernels give identical outputs.
"""
import os

import numpy as np
import pytest

import codon_hip as ch
import cpu_ref as cr
from conftest import PEPTIDE, decode

pytestmark = pytest.mark.gpu
FLAGS = ch.OUT_LOGITS | ch.OUT_HIDDEN


def special_blocks():
    """Blocks of 32 that exercise the quantizers' edge cases."""
    b = []
    b.append(np.zeros(32, np.float32))                                   # d = 0
    t = np.zeros(32, np.float32)
    t[0] = 127.0
    t[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]           # Q8 ties at d = 1
    b.append(t)
    t = np.zeros(32, np.float32)
    t[3] = -8.0
    t[4:12] = [0.5, -0.5, 1.5, -1.5, 6.5, -6.5, 7.5, -7.5]              # Q4 ties at d = 1
    b.append(t)
    t = np.linspace(-1, 1, 32).astype(np.float32)
    t[5], t[20] = 3.0, -3.0                                              # first of equal |max| wins
    b.append(t)
    t = np.linspace(-1, 1, 32).astype(np.float32)
    t[2] = np.nan
    b.append(t)
    t = np.linspace(-1, 1, 32).astype(np.float32)
    t[7] = np.inf
    b.append(t)
    t = np.linspace(-1, 1, 32).astype(np.float32)
    t[9] = -np.inf
    b.append(t)
    b.append(np.full(32, 1e-42, np.float32))                             # subnormal block
    b.append((np.arange(32, dtype=np.float32) - 16) * np.float32(1e37))  # near the top of the range
    return np.concatenate(b)


@pytest.mark.parametrize("dtype", [ch.DTYPE_Q8_0, ch.DTYPE_Q4_0])
def test_device_quantizer_bit_exact(dtype):
    rng = np.random.default_rng(7 + dtype)
    x = np.concatenate([special_blocks(), rng.standard_normal(32 * 40000).astype(np.float32) * 0.05,
                        rng.standard_normal(32 * 1000).astype(np.float32) * 1e4])
    oracle = cr.quantize_q8(x) if dtype == ch.DTYPE_Q8_0 else cr.quantize_q4(x)
    host = ch.quantize_slice_to_q8(x) if dtype == ch.DTYPE_Q8_0 else ch.quantize_slice_to_q4(x)
    dev = ch.quantize_on_device(dtype, x)
    bb = 36 if dtype == ch.DTYPE_Q8_0 else 20
    for name, ref in (("oracle", oracle), ("host", host)):
        bad = np.nonzero((ref.reshape(-1, bb) != dev.reshape(-1, bb)).any(axis=1))[0]
        print(f"dtype {dtype}: {x.size // 32} blocks, {bad.size} differ from the {name} quantizer", flush=True)
        assert bad.size == 0, (name, bad[:10])


def write_grouped(path, w, header_cfg=None):
    """grouped_canonical_v1 FP32 (lib.rs:369-395), optionally behind a CODQ header."""
    if header_cfg is not None:
        ch.save_codq(path, header_cfg, w)
        return
    with open(path, "wb") as f:
        for k in ch.model.FIELDS:
            f.write(np.ascontiguousarray(getattr(w, k), np.float32).tobytes())


def write_sequential_hf(path, cfg, w, seed=0):
    """sequential_hf (lib.rs:396-499): per-layer tensors, rotary inv_freq and a
    contact head the loader skips, the LM head in HF order."""
    d, F, L, V, H = cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.vocab_size, cfg.n_heads
    rng = np.random.default_rng(seed)
    f32 = lambda a: np.ascontiguousarray(a, np.float32).tobytes()  # noqa: E731
    cls = np.asarray(w.classifier_weights, np.float32)
    lm_lnw, lm_lnb = cls[:d], cls[d:2 * d]
    dense_w, dense_b = cls[2 * d:2 * d + d * d], cls[2 * d + d * d:3 * d + d * d]
    dec_w, dec_b = cls[3 * d + d * d:3 * d + d * d + V * d], cls[3 * d + d * d + V * d:]
    with open(path, "wb") as f:
        f.write(f32(w.token_embedding_table))
        f.write(f32(rng.standard_normal((d // H) // 2)))
        per = lambda name, n: np.asarray(getattr(w, name), np.float32).reshape(L, n)  # noqa: E731
        order = [("wq", d * d), ("bq", d), ("wk", d * d), ("bk", d), ("wv", d * d), ("bv", d), ("wo", d * d),
                 ("bo", d), ("ln_1_weight", d), ("ln_1_bias", d), ("fc1_weight", F * d), ("fc1_bias", F),
                 ("fc2_weight", d * F), ("fc2_bias", d), ("ln_2_weight", d), ("ln_2_bias", d)]
        stacks = {name: per(name, n) for name, n in order}
        for l in range(L):
            for name, _ in order:
                f.write(f32(stacks[name][l]))
        f.write(f32(w.ln_f_weight))
        f.write(f32(w.ln_f_bias))
        f.write(f32(rng.standard_normal(L * H + 1)))
        for a in (dec_b, dense_w, dense_b, lm_lnw, lm_lnb, dec_w):
            f.write(f32(a))


def seqs_for(rng, lens):
    return [np.concatenate([[0], 4 + rng.integers(0, 20, n), [2]]).astype(np.int32) for n in lens]


def assert_same_outputs(m_file, m_host, seqs, what):
    a, b = m_file.forward(seqs, FLAGS), m_host.forward(seqs, FLAGS)
    for k in ("logits", "hidden"):
        diff = float(np.abs(a[k] - b[k]).max())
        print(f"{what}: {k} max|diff| = {diff:.3e}", flush=True)
        assert np.array_equal(a[k], b[k]), (what, k, diff)


@pytest.fixture(scope="module")
def w8m():
    cfg = ch.EsmConfig.esm2_8m()
    return cfg, ch.EsmWeights.random(cfg, seed=81, bias_std=0.02)


@pytest.mark.parametrize("kind", ["codq_q8", "codq_q4", "codq_fp32", "grouped_fp32", "sequential_hf"])
def test_file_load_equals_host_create(tmp_path, w8m, kind):
    cfg, w = w8m
    rng = np.random.default_rng(3)
    seqs = seqs_for(rng, (17, 60, 5))
    path = str(tmp_path / f"m.{kind}")
    if kind == "codq_q8":
        w = w.quantize_q8()
        ch.save_codq(path, cfg, w)
    elif kind == "codq_q4":
        w = w.quantize_q4()
        ch.save_codq(path, cfg, w)
    elif kind == "codq_fp32":
        write_grouped(path, w, header_cfg=cfg)
    elif kind == "grouped_fp32":
        write_grouped(path, w)
    else:
        write_sequential_hf(path, cfg, w)
    print(f"{kind}: {os.path.getsize(path)} bytes", flush=True)
    m_file = ch.GpuModel.from_file(path, max_batch=3, max_len=62, outputs=FLAGS)
    m_host = ch.GpuModel(cfg, w, max_batch=3, max_len=62, outputs=FLAGS)
    assert m_file.dtype == w.dtype
    assert_same_outputs(m_file, m_host, seqs, kind)
    m_file.close()
    m_host.close()


@pytest.mark.parametrize("model,dtype", [("8M", ch.DTYPE_Q8_0), ("8M", ch.DTYPE_Q4_0), ("35M", ch.DTYPE_Q4_0)])
def test_quantize_to_on_device_equals_host_quantizer(tmp_path, model, dtype):
    cfg = ch.EsmConfig.by_name(model)
    w = ch.EsmWeights.random(cfg, seed=90 + dtype, bias_std=0.02)
    path = str(tmp_path / "m.fp32")
    write_grouped(path, w)
    wq = w.quantize_q8() if dtype == ch.DTYPE_Q8_0 else w.quantize_q4()
    rng = np.random.default_rng(5)
    seqs = seqs_for(rng, (33, 9))
    m_file = ch.GpuModel.from_file(path, quantize_to=dtype, max_batch=2, max_len=35, outputs=FLAGS)
    m_host = ch.GpuModel(cfg, wq, max_batch=2, max_len=35, outputs=FLAGS)
    assert m_file.dtype == dtype
    assert_same_outputs(m_file, m_host, seqs, f"{model} fp32 file -> dtype {dtype}")
    m_file.close()
    m_host.close()


def test_load_without_lm_head(tmp_path):
    """A quantized file whose classifier is shorter than the LM head loads
    with the tied-embedding decoder, like host tensors with the same short
    classifier."""
    cfg = ch.EsmConfig.esm2_8m()
    w = ch.EsmWeights.random(cfg, seed=12, bias_std=0.02).quantize_q8()
    w.classifier_weights = np.zeros(0, np.float32)
    path = str(tmp_path / "nohead.q8")
    ch.save_codq(path, cfg, w)
    seqs = seqs_for(np.random.default_rng(1), (20,))
    m_file = ch.GpuModel.from_file(path, max_batch=1, max_len=22, outputs=FLAGS)
    m_host = ch.GpuModel(cfg, w, max_batch=1, max_len=22, outputs=FLAGS)
    assert_same_outputs(m_file, m_host, seqs, "no LM head")
    m_file.close()
    m_host.close()


@pytest.mark.parametrize("quantize_to", [-1, ch.DTYPE_Q8_0, ch.DTYPE_Q4_0])
def test_shipped_8m_file_vs_oracle(w8m_path, quantize_to):
    cfg = ch.EsmConfig.esm2_8m()
    w = ch.EsmWeights.from_grouped_canonical(w8m_path, cfg)
    if quantize_to == ch.DTYPE_Q8_0:
        w = w.quantize_q8()
    elif quantize_to == ch.DTYPE_Q4_0:
        w = w.quantize_q4()
    contact = cfg.contact_head_weights()
    flags = ch.OUT_LOGITS | ch.OUT_FINAL_ATT | ch.OUT_CONTACTS
    m = ch.GpuModel.from_file(w8m_path, quantize_to=quantize_to, contact_head=contact, max_batch=2, max_len=64,
                              outputs=flags)
    assert m.dtype == (ch.DTYPE_FP32 if quantize_to < 0 else quantize_to)
    toks = ch.Tokenizer.encode(PEPTIDE)
    other = np.concatenate([[0], 4 + np.random.default_rng(8).integers(0, 20, 60), [2]]).astype(np.int32)
    got = m.forward([toks, other], flags)
    m.close()
    for b, t in enumerate((toks, other)):
        S = len(t)
        ref = cr.forward(cfg, w, t, 8, contacts=contact)
        el = float(np.abs(got["logits"][b, :S] - ref["logits"]).max())
        ea = float(np.abs(got["final_att"][b, :S, :S] - ref["final_att"]).max())
        ec = float(np.abs(got["contacts"][b, :S - 2, :S - 2] - ref["contacts"]).max())
        print(f"8M file quantize_to={quantize_to} seq {b}: logits {el:.2e} final_att {ea:.2e} contacts {ec:.2e}",
              flush=True)
        assert el <= 1e-3 and ea <= 1e-5 and ec <= 1e-4
    assert decode(got["logits"][0, 1:len(toks) - 1].argmax(1)) == PEPTIDE
