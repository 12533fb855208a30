"""ctypes wrapper over oracle/_build/libcpu_ref.so.

TEST INFRASTRUCTURE ONLY: the CPU oracle that the HIP path is checked
against, and the timed CPU baseline of bench.py.  Only tests/, the smoke
check and bench.py's cpu_baseline leg import this module.

Weights are passed as any object carrying the reference's field names
(`EsmWeights` / `EsmWeightsQ8` / `EsmWeightsQ4`, src/lib.rs:299-307,
675-687, 1113-1125) as numpy arrays: float32 for FP32 tensors, uint8 block
bytes (36 B per Q8_0 block, 20 B per Q4_0 block) for quantized matrices.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libcpu_ref.so")

FP32, Q8_0, Q4_0 = 0, 1, 2
_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u8p = ctypes.POINTER(ctypes.c_uint8)


class _Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("dim", "hidden_dim", "n_layers", "n_heads", "vocab_size")]


class _Weights(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("token_embedding_table", ctypes.c_void_p),
        ("ln_1_weight", ctypes.c_void_p), ("ln_1_bias", ctypes.c_void_p),
        ("wq", ctypes.c_void_p), ("bq", ctypes.c_void_p),
        ("wk", ctypes.c_void_p), ("bk", ctypes.c_void_p),
        ("wv", ctypes.c_void_p), ("bv", ctypes.c_void_p),
        ("wo", ctypes.c_void_p), ("bo", ctypes.c_void_p),
        ("ln_2_weight", ctypes.c_void_p), ("ln_2_bias", ctypes.c_void_p),
        ("fc1_weight", ctypes.c_void_p), ("fc1_bias", ctypes.c_void_p),
        ("fc2_weight", ctypes.c_void_p), ("fc2_bias", ctypes.c_void_p),
        ("ln_f_weight", ctypes.c_void_p), ("ln_f_bias", ctypes.c_void_p),
        ("classifier_weights", ctypes.c_void_p), ("classifier_len", ctypes.c_int64),
    ]


class _Outputs(ctypes.Structure):
    _fields_ = [
        ("logits", ctypes.c_void_p), ("hidden", ctypes.c_void_p), ("final_att", ctypes.c_void_p),
        ("contacts", ctypes.c_void_p), ("attn", ctypes.c_void_p), ("layer_hidden", ctypes.c_void_p),
        ("contact_w", ctypes.c_void_p), ("contact_b", ctypes.c_float),
    ]


class _RunState(ctypes.Structure):
    _fields_ = [("max_len", ctypes.c_int32), ("key_cache", _f32p), ("value_cache", _f32p),
                ("rope_cos", _f32p), ("rope_sin", _f32p), ("logits", _f32p)]


WEIGHT_FIELDS = [
    "token_embedding_table", "ln_1_weight", "ln_1_bias", "wq", "bq", "wk", "bk", "wv", "bv",
    "wo", "bo", "ln_2_weight", "ln_2_bias", "fc1_weight", "fc1_bias", "fc2_weight", "fc2_bias",
    "ln_f_weight", "ln_f_bias", "classifier_weights",
]

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        L.cr_quantize_q8.argtypes = [_f32p, ctypes.c_int64, _u8p]
        L.cr_quantize_q4.argtypes = [_f32p, ctypes.c_int64, _u8p]
        L.cr_dequantize_q8.argtypes = [_u8p, ctypes.c_int64, _f32p]
        L.cr_dequantize_q4.argtypes = [_u8p, ctypes.c_int64, _f32p]
        L.cr_tokenize.argtypes = [ctypes.c_char_p, _i32p, ctypes.c_int32]
        L.cr_tokenize.restype = ctypes.c_int32
        L.cr_layer_norm.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int32]
        L.cr_erf.argtypes = [ctypes.c_float]
        L.cr_erf.restype = ctypes.c_float
        L.cr_gelu.argtypes = [_f32p, _f32p, ctypes.c_int64]
        L.cr_softmax.argtypes = [_f32p, ctypes.c_int32]
        L.cr_rope_tables.argtypes = [ctypes.c_int32, ctypes.c_int32, _f32p, _f32p]
        L.cr_apply_rope.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.cr_log_softmax_canonical.argtypes = [_f32p, _f32p]
        L.cr_dms_score.argtypes = [_f32p, ctypes.c_int32, _f32p, _f32p]
        L.cr_accumulate_head_apc.argtypes = [_f32p, _f32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_float]
        L.cr_matmul_tiled.argtypes = [ctypes.c_int32, _f32p, _f32p, ctypes.c_void_p, _f32p,
                                      ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.cr_forward.argtypes = [ctypes.POINTER(_Config), ctypes.POINTER(_Weights), _i32p,
                                 ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(_Outputs)]
        L.cr_forward.restype = ctypes.c_int32
        L.cr_matmul_vec.argtypes = [ctypes.c_int32, _f32p, _f32p, ctypes.c_void_p, _f32p,
                                    ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.cr_run_state_new.argtypes = [ctypes.POINTER(_Config), ctypes.c_int32]
        L.cr_run_state_new.restype = ctypes.POINTER(_RunState)
        L.cr_run_state_free.argtypes = [ctypes.POINTER(_RunState)]
        L.cr_forward_step.argtypes = [ctypes.POINTER(_Config), ctypes.POINTER(_Weights), ctypes.c_int32,
                                      ctypes.c_int32, ctypes.POINTER(_RunState), ctypes.c_int32]
        L.cr_forward_step.restype = ctypes.c_int32
        L.cr_rng_seed.argtypes = [ctypes.c_uint64]
        L.cr_rng_seed.restype = ctypes.c_uint64
        L.cr_rng_next_u32.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.cr_rng_next_u32.restype = ctypes.c_uint32
        L.cr_rng_next_f32.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.cr_rng_next_f32.restype = ctypes.c_float
        L.cr_sample.argtypes = [_f32p, ctypes.c_int32, ctypes.c_float, ctypes.POINTER(ctypes.c_uint64)]
        L.cr_sample.restype = ctypes.c_int32
        L.cr_generate.argtypes = [ctypes.POINTER(_Config), ctypes.POINTER(_Weights), _i32p, ctypes.c_int32,
                                  ctypes.c_float, ctypes.c_int32, ctypes.c_uint64, ctypes.c_int32, ctypes.c_int32,
                                  _i32p, ctypes.c_int32]
        L.cr_generate.restype = ctypes.c_int32
        L.cr_set_attention_isa.argtypes = [ctypes.c_int32]
        L.cr_attention_uses_avx512.argtypes = [ctypes.c_int32]
        L.cr_attention_uses_avx512.restype = ctypes.c_int32
        for name in ("cr_cosine_similarity", "cr_rmse"):
            getattr(L, name).argtypes = [_f32p, _f32p, ctypes.c_int64]
            getattr(L, name).restype = ctypes.c_float
        for name in ("cr_top1_match_rate", "cr_kl_divergence"):
            getattr(L, name).argtypes = [_f32p, _f32p, ctypes.c_int64, ctypes.c_int32]
            getattr(L, name).restype = ctypes.c_float
        _lib = L
    return _lib


def _f(a):
    return a.ctypes.data_as(_f32p)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def quantize_q8(src):
    src = _c32(src).ravel()
    assert src.size % 32 == 0
    out = np.empty(src.size // 32 * 36, np.uint8)
    lib().cr_quantize_q8(_f(src), src.size, out.ctypes.data_as(_u8p))
    return out


def quantize_q4(src):
    src = _c32(src).ravel()
    assert src.size % 32 == 0
    out = np.empty(src.size // 32 * 20, np.uint8)
    lib().cr_quantize_q4(_f(src), src.size, out.ctypes.data_as(_u8p))
    return out


def dequantize_q8(blocks):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    nb = blocks.size // 36
    out = np.empty(nb * 32, np.float32)
    lib().cr_dequantize_q8(blocks.ctypes.data_as(_u8p), nb, _f(out))
    return out


def dequantize_q4(blocks):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    nb = blocks.size // 20
    out = np.empty(nb * 32, np.float32)
    lib().cr_dequantize_q4(blocks.ctypes.data_as(_u8p), nb, _f(out))
    return out


def tokenize(text):
    cap = len(text.encode()) + 2
    out = np.empty(cap, np.int32)
    n = lib().cr_tokenize(text.encode(), out.ctypes.data_as(_i32p), cap)
    assert n >= 0
    return out[:n].copy()


def layer_norm(x, w, b):
    x, w, b = _c32(x), _c32(w), _c32(b)
    out = np.empty_like(x)
    lib().cr_layer_norm(_f(out), _f(x), _f(w), _f(b), x.size)
    return out


def erf(x):
    return lib().cr_erf(float(x))


def gelu(x):
    x = _c32(x)
    out = np.empty_like(x)
    lib().cr_gelu(_f(out), _f(x), x.size)
    return out


def softmax(x):
    x = _c32(x).copy()
    lib().cr_softmax(_f(x), x.size)
    return x


def rope_tables(max_len, head_dim):
    c = np.empty(max_len * (head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().cr_rope_tables(max_len, head_dim, _f(c), _f(s))
    return c.reshape(max_len, head_dim // 2), s.reshape(max_len, head_dim // 2)


def apply_rope(q, k, cos_t, sin_t, pos, n_heads):
    q, k = _c32(q).copy(), _c32(k).copy()
    cos_t, sin_t = _c32(cos_t), _c32(sin_t)
    lib().cr_apply_rope(_f(q), _f(k), _f(cos_t), _f(sin_t), pos, q.size, n_heads)
    return q, k


def log_softmax_canonical(logits):
    logits = _c32(logits)
    out = np.empty(33, np.float32)
    lib().cr_log_softmax_canonical(_f(logits), _f(out))
    return out


CANONICAL_AAS = "ACDEFGHIKLMNPQRSTVWY"  # benchmark.rs:702-707 column order


def dms_score(logits33, wt_tok):
    """(deltas[20], entropy) of one DMS row from 33 logits (pipeline.rs:152-172)."""
    logits33 = np.ascontiguousarray(logits33, np.float32)
    deltas = np.empty(20, np.float32)
    ent = np.empty(1, np.float32)
    lib().cr_dms_score(_f(logits33), int(wt_tok), _f(deltas), _f(ent))
    return deltas, float(ent[0])


def dms_windows(n, window, max_seq_len):
    """Window of every position for the masked-marginal scan (pipeline.rs:87-122):
    returns actual_window and a list of (w_start, w_end) per position."""
    aw = min(n, max_seq_len) if (n <= window or window == 0) else min(window, max_seq_len)
    half = aw // 2
    out = []
    for p in range(n):
        if p < half:
            ws = 0
        elif p + half > n:
            ws = max(n - aw, 0)
        else:
            ws = p - half
        out.append((ws, min(ws + aw, n)))
    return aw, out


def dms_wt_windows(n, window, stride, max_seq_len):
    """Forwards of the wild-type-marginal scan (pipeline.rs:196-265): a list of
    (w_start, w_end, first_scored, end_scored)."""
    aw = min(n, max_seq_len) if (n <= window or window == 0) else min(window, max_seq_len)
    if n <= aw:
        return [(0, n, 0, n)]
    step = stride if 0 < stride <= aw else max(aw // 2, 1)
    out, covered, ws = [], 0, 0
    while covered < n:
        we = min(ws + aw, n)
        out.append((ws, we, covered, we))
        covered = we
        if we >= n:
            break
        ws = min(ws + step, max(n - aw, 0))
    return out


def dms(cfg, weights, residue_tokens, window=0, stride=0, mode="masked", num_threads=1, max_seq_len=1024):
    """run_pipeline_dms_with_mode (pipeline.rs:76-280) on one protein given as
    residue token ids: returns deltas [n][20] and entropy [n]."""
    res = np.asarray(residue_tokens, np.int32)
    n = res.size
    deltas = np.zeros((n, 20), np.float32)
    ent = np.zeros(n, np.float32)
    if mode == "masked":
        _, wins = dms_windows(n, window, max_seq_len)
        for p, (ws, we) in enumerate(wins):
            toks = np.concatenate([[0], res[ws:we], [2]]).astype(np.int32)
            tp = p - ws + 1
            wt = int(toks[tp])
            toks[tp] = 32
            logits = forward(cfg, weights, toks, num_threads, final_att=False, hidden=False)["logits"]
            deltas[p], ent[p] = dms_score(logits[tp], wt)
    else:
        for ws, we, c0, c1 in dms_wt_windows(n, window, stride, max_seq_len):
            toks = np.concatenate([[0], res[ws:we], [2]]).astype(np.int32)
            logits = forward(cfg, weights, toks, num_threads, final_att=False, hidden=False)["logits"]
            for p in range(c0, c1):
                tp = p - ws + 1
                deltas[p], ent[p] = dms_score(logits[tp], int(toks[tp]))
    return deltas, ent


def accumulate_head_apc(head_att, contact_logits, seq_len, n_res, w_lh):
    head_att = _c32(head_att)
    assert contact_logits.dtype == np.float32 and contact_logits.flags.c_contiguous
    lib().cr_accumulate_head_apc(_f(head_att), _f(contact_logits), seq_len, n_res, float(w_lh))


def matmul_tiled(dtype, x, w, bias, in_dim, out_dim, num_threads=1):
    """matmul_tiled_{fp32,q8,q4}_parallel (src/lib.rs:4803, 4870, 4937)."""
    x = _c32(x)
    seq_len = x.size // in_dim
    w = np.ascontiguousarray(w)
    bias = _c32(bias)
    out = np.empty((seq_len, out_dim), np.float32)
    lib().cr_matmul_tiled(dtype, _f(out), _f(x), w.ctypes.data, _f(bias), in_dim, out_dim, seq_len, num_threads)
    return out


def _cfg_weights(cfg, weights):
    c = _Config(cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.n_heads, cfg.vocab_size)
    keep = []
    wc = _Weights()
    wc.dtype = int(weights.dtype)
    for name in WEIGHT_FIELDS:
        arr = np.ascontiguousarray(getattr(weights, name))
        keep.append(arr)
        setattr(wc, name, arr.ctypes.data)
    wc.classifier_len = int(np.asarray(weights.classifier_weights).size)
    return c, wc, keep


def matmul_vec(dtype, x, w, bias, in_dim, out_dim, num_threads=1):
    """matmul_parallel / matmul_q8_parallel / matmul_q4_parallel
    (src/lib.rs:2860, 3027, 3265): one token."""
    x = _c32(x)
    w = np.ascontiguousarray(w)
    bias = _c32(bias)
    out = np.empty(out_dim, np.float32)
    lib().cr_matmul_vec(dtype, _f(out), _f(x), w.ctypes.data, _f(bias), in_dim, out_dim, num_threads)
    return out


class RunState:
    """RunState (src/lib.rs:2459-2486) with forward / forward_q8 / forward_q4
    (3554, 3741, 4016) as step(): one token at one position against the KV
    cache.  The K/V caches are views [L][max_len][d]."""

    def __init__(self, cfg, weights, max_len=1024, num_threads=1):
        self.cfg, self.nt = cfg, num_threads
        self._c, self._w, self._keep = _cfg_weights(cfg, weights)
        self._s = lib().cr_run_state_new(ctypes.byref(self._c), max_len)
        self.max_len = max_len

    def step(self, token, pos):
        rc = lib().cr_forward_step(ctypes.byref(self._c), ctypes.byref(self._w), int(token), int(pos), self._s,
                                   self.nt)
        if rc != 0:
            raise RuntimeError(f"cr_forward_step failed with code {rc}")
        return np.ctypeslib.as_array(self._s.contents.logits, (self.cfg.vocab_size,)).copy()

    def cache(self):
        shp = (self.cfg.n_layers, self.max_len, self.cfg.dim)
        return (np.ctypeslib.as_array(self._s.contents.key_cache, shp),
                np.ctypeslib.as_array(self._s.contents.value_cache, shp))

    def __del__(self):
        if getattr(self, "_s", None):
            lib().cr_run_state_free(self._s)
            self._s = None


class SimpleRng:
    """SimpleRng (src/lib.rs:3506-3511) over the C restatement."""

    def __init__(self, seed):
        self.state = ctypes.c_uint64(lib().cr_rng_seed(seed))

    def next_u32(self):
        return lib().cr_rng_next_u32(ctypes.byref(self.state))

    def next_f32(self):
        return lib().cr_rng_next_f32(ctypes.byref(self.state))


def sample(logits, temperature, rng):
    """sample (src/lib.rs:3513-3530); rng: SimpleRng (advanced when T > 0)."""
    lg = _c32(logits).copy()
    return lib().cr_sample(_f(lg), lg.size, float(temperature), ctypes.byref(rng.state))


def generate(cfg, weights, prompt_tokens, temperature=0.0, max_new_tokens=None, seed=0, max_seq_len=1024,
             num_threads=1):
    """generate_sequence* (src/lib.rs:6551-6827) from the prompt's token ids
    (Tokenizer::encode minus the trailing <eos>): the generated token ids."""
    c, wc, keep = _cfg_weights(cfg, weights)
    prompt = np.ascontiguousarray(prompt_tokens, np.int32)
    cap = max_seq_len
    out = np.zeros(cap, np.int32)
    n = lib().cr_generate(ctypes.byref(c), ctypes.byref(wc), prompt.ctypes.data_as(_i32p), prompt.size,
                          float(temperature), -1 if max_new_tokens is None else int(max_new_tokens), seed,
                          max_seq_len, num_threads, out.ctypes.data_as(_i32p), cap)
    if n < 0:
        raise RuntimeError(f"cr_generate failed with code {n}")
    return out[:n].copy()


def set_attention_isa(avx_only):
    """Force the reference's 256-bit attention dot/axpy (True) or let head_dim
    64 take its AVX-512F path when the host has it (False, the default)."""
    lib().cr_set_attention_isa(1 if avx_only else 0)


def attention_uses_avx512(head_dim):
    return bool(lib().cr_attention_uses_avx512(head_dim))


def forward(cfg, weights, tokens, num_threads=1, contacts=None, attn=False, layer_hidden=False,
            final_att=True, hidden=True):
    """One forward_bidirectional_* call on one unpadded sequence.

    cfg: object with dim, hidden_dim, n_layers, n_heads, vocab_size.
    contacts: None, or (contact_w [L*H] float32, contact_b float) to compute
    contact probabilities.  Returns a dict of numpy arrays.
    """
    tokens = np.ascontiguousarray(tokens, np.int32)
    S = tokens.size
    d, L, H, V = cfg.dim, cfg.n_layers, cfg.n_heads, cfg.vocab_size
    c = _Config(cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.n_heads, cfg.vocab_size)
    keep = []
    wc = _Weights()
    wc.dtype = int(weights.dtype)
    for name in WEIGHT_FIELDS:
        arr = np.ascontiguousarray(getattr(weights, name))
        keep.append(arr)
        setattr(wc, name, arr.ctypes.data)
    wc.classifier_len = int(np.asarray(weights.classifier_weights).size)
    res = {"logits": np.zeros((S, V), np.float32)}
    if hidden:
        res["hidden"] = np.zeros((S, d), np.float32)
    if final_att:
        res["final_att"] = np.zeros((S, S), np.float32)
    n = max(S - 2, 0)
    if contacts is not None:
        res["contacts"] = np.zeros((n, n), np.float32)
        cw = _c32(contacts[0])
        keep.append(cw)
    if attn:
        res["attn"] = np.zeros((L, H, S, S), np.float32)
    if layer_hidden:
        res["layer_hidden"] = np.zeros((L, S, d), np.float32)
    o = _Outputs()
    for k2 in ("logits", "hidden", "final_att", "contacts", "attn", "layer_hidden"):
        setattr(o, k2, res[k2].ctypes.data if k2 in res else None)
    if contacts is not None:
        o.contact_w = cw.ctypes.data
        o.contact_b = float(contacts[1])
    rc = lib().cr_forward(ctypes.byref(c), ctypes.byref(wc), tokens.ctypes.data_as(_i32p), S,
                          num_threads, ctypes.byref(o))
    if rc != 0:
        raise RuntimeError(f"cr_forward failed with code {rc}")
    return res


def cosine_similarity(a, b):
    a, b = _c32(a).ravel(), _c32(b).ravel()
    return lib().cr_cosine_similarity(_f(a), _f(b), min(a.size, b.size))


def rmse(a, b):
    a, b = _c32(a).ravel(), _c32(b).ravel()
    return lib().cr_rmse(_f(a), _f(b), min(a.size, b.size))


def top1_match_rate(a, b, vocab=33):
    a, b = _c32(a).ravel(), _c32(b).ravel()
    return lib().cr_top1_match_rate(_f(a), _f(b), min(a.size, b.size), vocab)


def kl_divergence(a, b, vocab=33):
    a, b = _c32(a).ravel(), _c32(b).ravel()
    return lib().cr_kl_divergence(_f(a), _f(b), min(a.size, b.size), vocab)
