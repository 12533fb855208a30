"""Long sequences against the oracle: more than 32 key tiles per sequence,
RoPE positions past 1024 (the reference's analytic tables,
src/lib.rs:2513-2522, at every position of a 2048-token state), the
attention loop at S = 2048 (lib.rs:5206-5301; Q8 5558-5653; Q4 ~5905-6005),
at every head size ESM-2 uses.  The long-sequence configuration itself (3B
Q4_0 at 2048 tokens, lib.rs:5800-6147) is compared with the oracle at full
length in test_gpu_configs.py.

Tolerances as in test_gpu_forward.py: logits and hidden states <= 1e-3,
attention maps and final_att <= 1e-5, argmax identical wherever the
oracle's top-1/top-2 margin exceeds twice the measured logit error.
Contacts are not requested here: the reference refuses them past 1024
residues (lib.rs:5046), as cih_forward does (CIH_ERR_CONTACTS).
"""
import numpy as np
import pytest

import codon_hip as ch
from test_gpu_forward import check_batch, rand_tokens

pytestmark = pytest.mark.gpu

LONG = ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_FINAL_ATT | ch.OUT_ATTN | ch.OUT_LAYER_HIDDEN


@pytest.mark.parametrize("hd,dtype", [(16, 1), (24, 2), (32, 0), (64, 1)])
def test_long_sequences_every_head_size(hd, dtype):
    """d = 4 hd, 4 heads, 2 layers: one 2048-token sequence alone (4 heads x
    64 key tiles fit one round of the compute units: attention splits each
    task's keys over 8 waves), then a ragged
    pair of 2048 and 1500 tokens (3548 tokens: K/V tile images from the prep
    kernel); all outputs including every layer's maps."""
    rng = np.random.default_rng(2048 + hd)
    cfg = ch.EsmConfig(4 * hd, 16 * hd, 2, 4)
    w = ch.EsmWeights.random(cfg, seed=hd, bias_std=0.02)
    w = w if dtype == 0 else (w.quantize_q8() if dtype == 1 else w.quantize_q4())
    long = rand_tokens(rng, 2046)
    long[777] = 32  # a <mask> (token-dropout rescale of this sequence)
    print(f"hd={hd} dtype={dtype}: one sequence of 2048", flush=True)
    check_batch(cfg, w, [long], LONG)
    print(f"hd={hd} dtype={dtype}: ragged 2048 + 1500", flush=True)
    check_batch(cfg, w, [long, rand_tokens(rng, 1498)], LONG)


def test_long_sequences_qkv_image_epilogue():
    """ESM-2 650M width (d = 1280, 20 heads of 64), 2 layers, Q8_0: a ragged
    pair of 2048 and 1500 tokens is large enough for the LDS-staged QKV
    projection, whose epilogue rotates K with the RoPE rows of positions up
    to 2047 and writes the K/V tile images; logits, hidden states, every
    layer's hidden state and final_att (the 2x20 maps of 2048^2 are left to
    the narrow models above)."""
    rng = np.random.default_rng(1280)
    cfg = ch.EsmConfig(1280, 5120, 2, 20)
    w = ch.EsmWeights.random(cfg, seed=1280, bias_std=0.02).quantize_q8()
    seqs = [rand_tokens(rng, 2046), rand_tokens(rng, 1498)]
    check_batch(cfg, w, seqs, ch.OUT_LOGITS | ch.OUT_HIDDEN | ch.OUT_FINAL_ATT | ch.OUT_LAYER_HIDDEN)

