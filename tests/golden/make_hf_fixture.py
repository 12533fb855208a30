"""Writes hf_8m_peptide.npz: an independent FP32 cross-check of the ESM-2 8M
forward, computed with HuggingFace transformers' EsmForMaskedLM built from a
local config (no download) and loaded with the shipped 8M weights
(esm2_8m_weights.bin, grouped_canonical_v1 layout).

Runs only in the build container (it needs the weights file and
transformers); the output is a small committed fixture.  Inputs:
  * test_peptidase.fasta's 39-residue peptide, unmasked;
  * "MCMP*TTD" with one <mask> (the reference's masked-inference test input,
    src/lib.rs:6938-6983).
Stored per input: tokens, logits [S,33], last hidden state after
emb_layer_norm_after [S,320], all attention probabilities [6,20,S,S] and the
contact map [S-2,S-2] (contact head set from the 8M regression weights).
Known deviation: HF GELU uses exact erf, the reference the A&S 7.1.26
polynomial (|error| <= 1.5e-7).
"""
import json
import os
import sys

import numpy as np
import torch
from transformers import EsmConfig, EsmForMaskedLM

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
PEPTIDE = "AQVGDSGGPMLCNGQLQGVTSWGYVCAQPEYPGVYTEVS"
AA = {c: i + 4 for i, c in enumerate("LAGVSERTIDPKQNFYMHWC")}


def encode(s):
    return [0] + [32 if c == "*" else AA[c] for c in s] + [2]


def load_state(path):
    d, F, L, V = 320, 1280, 6, 33
    raw = np.fromfile(path, dtype="<f4")
    assert raw.size * 4 == 30_091_652
    off = 0

    def take(n, shape):
        nonlocal off
        a = raw[off:off + n].reshape(shape)
        off += n
        return torch.from_numpy(a.copy())

    emb = take(V * d, (V, d))
    t = {}
    for name, n, shape in [("ln1w", L * d, (L, d)), ("ln1b", L * d, (L, d)), ("wq", L * d * d, (L, d, d)),
                           ("bq", L * d, (L, d)), ("wk", L * d * d, (L, d, d)), ("bk", L * d, (L, d)),
                           ("wv", L * d * d, (L, d, d)), ("bv", L * d, (L, d)), ("wo", L * d * d, (L, d, d)),
                           ("bo", L * d, (L, d)), ("ln2w", L * d, (L, d)), ("ln2b", L * d, (L, d)),
                           ("fc1", L * F * d, (L, F, d)), ("fc1b", L * F, (L, F)), ("fc2", L * d * F, (L, d, F)),
                           ("fc2b", L * d, (L, d)), ("lnfw", d, (d,)), ("lnfb", d, (d,))]:
        t[name] = take(n, shape)
    lm_lnw, lm_lnb = take(d, (d,)), take(d, (d,))
    dense_w, dense_b = take(d * d, (d, d)), take(d, (d,))
    dec_w, dec_b = take(V * d, (V, d)), take(V, (V,))
    assert off == raw.size
    sd = {"esm.embeddings.word_embeddings.weight": emb,
          "esm.encoder.emb_layer_norm_after.weight": t["lnfw"], "esm.encoder.emb_layer_norm_after.bias": t["lnfb"],
          "lm_head.bias": dec_b, "lm_head.dense.weight": dense_w, "lm_head.dense.bias": dense_b,
          "lm_head.layer_norm.weight": lm_lnw, "lm_head.layer_norm.bias": lm_lnb, "lm_head.decoder.weight": dec_w}
    for l in range(L):
        p = f"esm.encoder.layer.{l}."
        sd.update({p + "attention.self.query.weight": t["wq"][l], p + "attention.self.query.bias": t["bq"][l],
                   p + "attention.self.key.weight": t["wk"][l], p + "attention.self.key.bias": t["bk"][l],
                   p + "attention.self.value.weight": t["wv"][l], p + "attention.self.value.bias": t["bv"][l],
                   p + "attention.output.dense.weight": t["wo"][l], p + "attention.output.dense.bias": t["bo"][l],
                   p + "attention.LayerNorm.weight": t["ln1w"][l], p + "attention.LayerNorm.bias": t["ln1b"][l],
                   p + "intermediate.dense.weight": t["fc1"][l], p + "intermediate.dense.bias": t["fc1b"][l],
                   p + "output.dense.weight": t["fc2"][l], p + "output.dense.bias": t["fc2b"][l],
                   p + "LayerNorm.weight": t["ln2w"][l], p + "LayerNorm.bias": t["ln2b"][l]})
    return sd


def main():
    wpath = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/esm2_8m_weights.bin"
    with open(os.path.join(REPO, "codon-infer_amd", "codon_hip", "data", "contact_heads.json")) as f:
        ch = json.load(f)["8M"]
    cfg = EsmConfig(vocab_size=33, hidden_size=320, num_hidden_layers=6, num_attention_heads=20,
                    intermediate_size=1280, position_embedding_type="rotary", token_dropout=True,
                    emb_layer_norm_before=False, mask_token_id=32, pad_token_id=1, layer_norm_eps=1e-5,
                    max_position_embeddings=1026, hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0,
                    hidden_act="gelu")
    cfg._attn_implementation = "eager"
    m = EsmForMaskedLM(cfg).eval()
    sd = load_state(wpath)
    sd["esm.contact_head.regression.weight"] = torch.tensor(ch["weight"], dtype=torch.float32).reshape(1, -1)
    sd["esm.contact_head.regression.bias"] = torch.tensor([ch["bias"]], dtype=torch.float32)
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("inv_freq" in k for k in missing), missing
    out = {}
    for tag, seq in (("peptide", PEPTIDE), ("masked", "MCMP*TTD")):
        ids = torch.tensor([encode(seq)])
        with torch.no_grad():
            r = m(input_ids=ids, attention_mask=torch.ones_like(ids), output_attentions=True,
                  output_hidden_states=True)
            contacts = m.esm.predict_contacts(ids, attention_mask=torch.ones_like(ids))
        out[f"{tag}_tokens"] = ids[0].numpy().astype(np.int32)
        out[f"{tag}_logits"] = r.logits[0].numpy()
        out[f"{tag}_hidden"] = r.hidden_states[-1][0].numpy()
        out[f"{tag}_attn"] = torch.stack(r.attentions, 0)[:, 0].numpy()
        out[f"{tag}_contacts"] = contacts[0].numpy()
    dst = os.path.join(HERE, "hf_8m_peptide.npz")
    np.savez(dst, **out)
    print("wrote", dst, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
