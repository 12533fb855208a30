"""Writes config5_3b_q4_l2048.npz: the oracle's logits for ESM-2 3B Q4_0 on
one 2048-token sequence (BOS + 2046 residues + EOS), the long-sequence
configuration whose oracle forward takes minutes (36 layers, d = 2560, 40
heads of 64; the reference's serial attention at S = 2048 is most of it).

The model and tokens are the ones tests/test_gpu_configs.py builds:
  * weights: EsmWeights.random(esm2_3b, seed=3000, bias_std=0.02), quantized
    to Q4_0 in-tree (numpy's seeded generator, so the same on every machine
    with this image);
  * tokens: 4 + default_rng(2048).integers(0, 20, 2046) between BOS (0) and
    EOS (2).
Stored: tokens [2048] int32, logits [2048, 33] float32, and the SHA-256 of
the packed Q4_0 layer matrices (wq, wk, wv, wo, fc1, fc2 of all layers) so a
test can tell whether it rebuilt the same model.

The oracle's results do not depend on its thread count (each output row of a
GEMM is summed by one thread in the reference's order), so any number of
threads writes the same fixture.  Run from the repo root:
    python tests/golden/make_config5_fixture.py [threads]
"""
import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "codon-infer_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

OUT = os.path.join(HERE, "config5_3b_q4_l2048.npz")


def model_and_tokens():
    import codon_hip as ch
    cfg = ch.EsmConfig.esm2_3b()
    w = ch.EsmWeights.random(cfg, seed=3000, bias_std=0.02).quantize_q4()
    rng = np.random.default_rng(2048)
    toks = np.empty(2048, np.int32)
    toks[0], toks[-1] = 0, 2
    toks[1:-1] = 4 + rng.integers(0, 20, 2046)
    return cfg, w, toks


def weights_digest(w):
    h = hashlib.sha256()
    for name in ("wq", "wk", "wv", "wo", "fc1_weight", "fc2_weight"):
        h.update(np.ascontiguousarray(getattr(w, name)).tobytes())
    return h.hexdigest()


def main():
    import cpu_ref as cr
    threads = int(sys.argv[1]) if len(sys.argv) > 1 else (os.cpu_count() or 1)
    t0 = time.time()
    cfg, w, toks = model_and_tokens()
    print(f"model ready in {time.time() - t0:.0f} s; oracle forward with {threads} threads ...", flush=True)
    t1 = time.time()
    ref = cr.forward(cfg, w, toks, threads, final_att=False, hidden=False)
    print(f"oracle forward {time.time() - t1:.0f} s", flush=True)
    np.savez_compressed(OUT, tokens=toks, logits=ref["logits"].astype(np.float32),
                        weights_sha256=np.array(weights_digest(w)))
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
