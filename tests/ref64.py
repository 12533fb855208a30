"""Float64 ESM-2 written from the mathematics (test infrastructure): the
bidirectional encoder forward, its causal twin (token i attends to 0..i, the
autoregressive path), every attention map, the last layer's head mean, the
contact head (symmetrize, APC, logistic regression), and the LM head or the
tied-embedding decoder.

It shares no code with the oracle and uses none of its summation orders:
numpy float64 matrix products, exact erf, softmax over all keys.  Weights
are the float32 values the reference multiplies with: FP32 tensors as they
are, Q8_0 / Q4_0 matrices as the dequantized (q as f32) * d.  It pins the
oracle to within FP32 rounding at every head size and weight format; what it
cannot pin is the oracle's exact bit pattern (summation order).
"""
import math

import numpy as np

import cpu_ref as cr

MATRICES = ("wq", "wk", "wv", "wo", "fc1_weight", "fc2_weight")


def _erf(x):
    return np.vectorize(math.erf, otypes=[np.float64])(x)


def dense_weights(cfg, w):
    """float64 copies of every tensor; quantized matrices dequantized with the
    reference's (q as f32) * d (the oracle's dequantizers are pinned bit-exact
    to the reference's known-answer tests)."""
    dt = int(w.dtype)
    out = {}
    for name in ("token_embedding_table", "ln_1_weight", "ln_1_bias", "bq", "bk", "bv", "bo", "ln_2_weight",
                 "ln_2_bias", "fc1_bias", "fc2_bias", "ln_f_weight", "ln_f_bias", "classifier_weights") + MATRICES:
        a = np.asarray(getattr(w, name))
        quant = (name in MATRICES and dt != 0) or (name == "token_embedding_table" and dt == 1)
        if quant:
            a = cr.dequantize_q8(a) if (dt == 1 or name == "token_embedding_table") else cr.dequantize_q4(a)
        out[name] = np.asarray(a, np.float32).astype(np.float64)
    return out


def _ln(v, g, b):
    mu = v.mean(-1, keepdims=True)
    var = ((v - mu) ** 2).mean(-1, keepdims=True)
    return g * (v - mu) / np.sqrt(var + 1e-5) + b


def _gelu(v):
    return 0.5 * v * (1.0 + _erf(v / np.sqrt(2.0)))


def forward64(cfg, w, tokens, causal=False, contacts=None):
    """One sequence.  Returns float64 arrays: logits [S][V], hidden [S][d]
    (after LN_f), layer_hidden [L][S][d], attn [L][H][S][S], final_att [S][S]
    and, with contacts = (w [L*H], b), contacts [n][n] for the n = S - 2
    residues."""
    d, F, L, H, V = cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.n_heads, cfg.vocab_size
    hd = d // H
    W = dense_weights(cfg, w)
    tokens = np.asarray(tokens)
    S = len(tokens)
    emb = W["token_embedding_table"].reshape(V, d)
    if causal:
        scale = np.float64(np.float32(0.88))  # every step is a one-token sequence
    else:
        # token dropout: 0.88 / (1 - masked fraction), the float32 value
        ratio = np.float32(np.sum(tokens == 32)) / np.float32(S)
        scale = 0.0 if ratio >= 1.0 else np.float64(np.float32(np.float32(1.0 - 0.12) / (np.float32(1.0) - ratio)))
    x = np.stack([np.zeros(d) if t == 32 else emb[t] * scale for t in tokens])

    half = hd // 2
    freq = 1.0 / 10000.0 ** (np.arange(half) * 2 / hd)
    ang = np.arange(S)[:, None] * freq[None, :]
    c, s = np.cos(ang), np.sin(ang)

    def rope(t):
        t = t.reshape(S, H, hd)
        a, b = t[..., :half], t[..., half:]
        return np.concatenate([a * c[:, None] - b * s[:, None], b * c[:, None] + a * s[:, None]], -1)

    def mat(name, l, o, i):
        return W[name].reshape(L, o, i)[l]

    def vec(name, l, o):
        return W[name].reshape(L, o)[l]

    mask = np.tril(np.ones((S, S), bool)) if causal else np.ones((S, S), bool)
    attn = np.zeros((L, H, S, S))
    layer_hidden = np.zeros((L, S, d))
    for l in range(L):
        h = _ln(x, vec("ln_1_weight", l, d), vec("ln_1_bias", l, d))
        q = rope(h @ mat("wq", l, d, d).T + vec("bq", l, d))
        k = rope(h @ mat("wk", l, d, d).T + vec("bk", l, d))
        v = (h @ mat("wv", l, d, d).T + vec("bv", l, d)).reshape(S, H, hd)
        sc = np.einsum("qhe,khe->hqk", q, k) / np.sqrt(hd)
        sc = np.where(mask[None], sc, -np.inf)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        attn[l] = p
        o = np.einsum("hqk,khe->qhe", p, v).reshape(S, d)
        x = x + o @ mat("wo", l, d, d).T + vec("bo", l, d)
        h = _ln(x, vec("ln_2_weight", l, d), vec("ln_2_bias", l, d))
        h = _gelu(h @ mat("fc1_weight", l, F, d).T + vec("fc1_bias", l, F))
        x = x + h @ mat("fc2_weight", l, d, F).T + vec("fc2_bias", l, d)
        layer_hidden[l] = x
    x = _ln(x, W["ln_f_weight"], W["ln_f_bias"])
    cw = W["classifier_weights"]
    if cw.size >= 3 * d + d * d + V * d + V:
        lnw, lnb = cw[:d], cw[d:2 * d]
        dw, db = cw[2 * d:2 * d + d * d].reshape(d, d), cw[2 * d + d * d:3 * d + d * d]
        decw = cw[3 * d + d * d:3 * d + d * d + V * d].reshape(V, d)
        decb = cw[3 * d + d * d + V * d:3 * d + d * d + V * d + V]
        logits = _ln(_gelu(x @ dw.T + db), lnw, lnb) @ decw.T + decb
    else:
        logits = x @ emb.T  # tied embedding decoder, no bias
    res = {"logits": logits, "hidden": x, "layer_hidden": layer_hidden, "attn": attn,
           "final_att": attn[L - 1].mean(0)}
    n = S - 2
    if contacts is not None and n > 0:
        wl, b = np.asarray(contacts[0], np.float64), float(contacts[1])
        z = np.zeros((n, n))
        for l in range(L):
            for hh in range(H):
                if wl[l * H + hh] == 0.0:
                    continue
                P = attn[l, hh, 1:S - 1, 1:S - 1]
                sym = P + P.T
                r = sym.sum(1)
                tot = r.sum()
                z += wl[l * H + hh] * (sym - np.outer(r, r) / tot if abs(tot) > 1e-12 else sym)
        res["contacts"] = 1.0 / (1.0 + np.exp(-(z + b)))
    return res
