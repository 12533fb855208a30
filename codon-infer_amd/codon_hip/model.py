"""Host-side mirror of codon-infer's model-load / forward / logits /
attention-map API over the gfx950 library.

Names and argument meanings follow the reference crate (src/lib.rs):
`EsmConfig` (76-150), `EsmWeights` / `EsmWeightsQ8` / `EsmWeightsQ4`
(299-307, 675-687, 1113-1125) with `quantize_q8` / `quantize_q4`
(559-607), `BidirectionalRunState` (2488-2544), `Tokenizer` (6509-6531),
`log_softmax_canonical` (4426-4441) and the `forward_bidirectional*`
family (5078-6147).  The forward itself always runs on the GPU through
libcodon_hip.so.
"""
import concurrent.futures
import ctypes
import json
import os
from dataclasses import dataclass

import numpy as np

from . import _lib as C

_DATA = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data")

# CODQ arch ids (lib.rs:878-882)
ARCH_IDS = {"8M": 0, "35M": 1, "150M": 2, "650M": 3, "3B": 4}


@dataclass(frozen=True)
class EsmConfig:
    dim: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    vocab_size: int = 33
    max_seq_len: int = 1024
    arch: str = "custom"

    @classmethod
    def esm2_8m(cls):
        return cls(320, 1280, 6, 20, arch="8M")

    @classmethod
    def esm2_35m(cls):
        return cls(480, 1920, 12, 20, arch="35M")

    @classmethod
    def esm2_150m(cls):
        return cls(640, 2560, 30, 20, arch="150M")

    @classmethod
    def esm2_650m(cls):
        return cls(1280, 5120, 33, 20, arch="650M")

    @classmethod
    def esm2_3b(cls):
        return cls(2560, 10240, 36, 40, arch="3B")

    @classmethod
    def by_name(cls, name):
        return {"8M": cls.esm2_8m, "35M": cls.esm2_35m, "150M": cls.esm2_150m, "650M": cls.esm2_650m,
                "3B": cls.esm2_3b}[name]()

    def head_dim(self):
        return self.dim // self.n_heads

    def lm_head_floats(self):
        d, V = self.dim, self.vocab_size
        return 3 * d + d * d + V * d + V

    def grouped_canonical_floats(self):
        d, F, L, V = self.dim, self.hidden_dim, self.n_layers, self.vocab_size
        return V * d + L * (4 * d * d + 9 * d + 2 * d * F + F) + 2 * d + self.lm_head_floats()

    def contact_head_weights(self):
        """Official (weight[L*H], bias) for the preset architectures (lib.rs:154-177)."""
        with open(os.path.join(_DATA, "contact_heads.json")) as f:
            ch = json.load(f)[self.arch]
        w = np.asarray(ch["weight"], dtype=np.float32)
        assert w.size == self.n_layers * self.n_heads
        return w, np.float32(ch["bias"])

    def _c(self):
        return C.Config(self.dim, self.hidden_dim, self.n_layers, self.n_heads, self.vocab_size, self.max_seq_len)


FIELDS = ["token_embedding_table", "ln_1_weight", "ln_1_bias", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
          "ln_2_weight", "ln_2_bias", "fc1_weight", "fc1_bias", "fc2_weight", "fc2_bias", "ln_f_weight",
          "ln_f_bias", "classifier_weights"]
MATRICES = ["wq", "wk", "wv", "wo", "fc1_weight", "fc2_weight"]


def save_codq(path, cfg, weights):
    """EsmWeights{Q8,Q4}::save_to_file_with_header (lib.rs:716-742,
    1128-1154): the 64-byte CODQ header (magic, version 1, dtype, arch id,
    n_layers, dim, hidden_dim, vocab_size, 32 zero bytes), then every field in
    EsmWeights order (FP32 floats or the packed 36/20-byte blocks)."""
    import struct
    hdr = b"CODQ" + struct.pack("<7I", 1, weights.dtype, ARCH_IDS[cfg.arch], cfg.n_layers, cfg.dim, cfg.hidden_dim,
                                cfg.vocab_size) + bytes(32)
    with open(path, "wb") as f:
        f.write(hdr)
        for k in FIELDS:
            f.write(np.ascontiguousarray(getattr(weights, k)).tobytes())


def quantize_slice_to_q8(src):
    """quantize_slice_to_q8 (lib.rs:670-673): packed 36-byte blocks as uint8."""
    src = np.ascontiguousarray(src, np.float32).ravel()
    out = np.empty(src.size // 32 * 36, np.uint8)
    C.check(C.lib().cih_quantize_q8(src.ctypes.data, src.size, out.ctypes.data))
    return out


def quantize_slice_to_q4(src):
    """quantize_slice_to_q4 (lib.rs:1085-1088): packed 20-byte blocks as uint8."""
    src = np.ascontiguousarray(src, np.float32).ravel()
    out = np.empty(src.size // 32 * 20, np.uint8)
    C.check(C.lib().cih_quantize_q4(src.ctypes.data, src.size, out.ctypes.data))
    return out


def dequantize_blocks(dtype, blocks):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    bb = 36 if dtype == C.DTYPE_Q8_0 else 20
    nb = blocks.size // bb
    out = np.empty(nb * 32, np.float32)
    fn = C.lib().cih_dequantize_q8 if dtype == C.DTYPE_Q8_0 else C.lib().cih_dequantize_q4
    C.check(fn(blocks.ctypes.data, nb, out.ctypes.data))
    return out


def _normal(n, std, seed, stream, chunk=1 << 22):
    """N(0, std) float32 samples; chunk c of tensor `stream` is drawn from
    default_rng([seed, stream, c]), so the result does not depend on the
    number of threads that fill it."""
    out = np.empty(n, np.float32)
    nch = (n + chunk - 1) // chunk

    def fill(c):
        sl = out[c * chunk:min(n, (c + 1) * chunk)]
        np.random.default_rng([seed, stream, c]).standard_normal(sl.size, dtype=np.float32, out=sl)
        sl *= np.float32(std)

    if nch == 1:
        fill(0)
    else:
        with concurrent.futures.ThreadPoolExecutor(min(16, os.cpu_count() or 1)) as ex:
            list(ex.map(fill, range(nch)))
    return out


class _Weights:
    dtype = C.DTYPE_FP32

    def __init__(self, **tensors):
        for k in FIELDS:
            setattr(self, k, tensors[k])

    def _host(self):
        hw = C.HostWeights()
        keep = []
        for k in FIELDS:
            a = np.ascontiguousarray(getattr(self, k))
            keep.append(a)
            setattr(hw, k, a.ctypes.data)
        hw.classifier_len = int(np.asarray(self.classifier_weights).size)
        return hw, keep


class EsmWeights(_Weights):
    """FP32 weights (EsmWeights, lib.rs:299-307): flat float32 arrays."""

    dtype = C.DTYPE_FP32

    @classmethod
    def from_grouped_canonical(cls, path, cfg):
        """grouped_canonical_v1 FP32 file (lib.rs:369-395)."""
        raw = np.fromfile(path, dtype="<f4")
        if raw.size != cfg.grouped_canonical_floats():
            raise ValueError(f"{path}: {raw.size} floats, expected {cfg.grouped_canonical_floats()}")
        d, F, L, V = cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.vocab_size
        sizes = [V * d, L * d, L * d, L * d * d, L * d, L * d * d, L * d, L * d * d, L * d, L * d * d, L * d, L * d,
                 L * d, L * F * d, L * F, L * d * F, L * d, d, d, cfg.lm_head_floats()]
        t, off = {}, 0
        for k, n in zip(FIELDS, sizes):
            t[k] = raw[off:off + n]
            off += n
        return cls(**t)

    @classmethod
    def random(cls, cfg, seed=0, std=0.02, bias_std=0.0):
        """Seeded N(0, std) weights of the given architecture; LayerNorm gamma 1,
        beta 0; biases N(0, bias_std) (0 by default, the HF init)."""
        d, F, L, V = cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.vocab_size
        counter = [0]

        def nrm(n, s):
            counter[0] += 1
            if s == 0:
                return np.zeros(n, np.float32)
            return _normal(n, s, seed, counter[0])

        ones = lambda n: np.ones(n, np.float32)  # noqa: E731
        zeros = lambda n: np.zeros(n, np.float32)  # noqa: E731
        t = dict(token_embedding_table=nrm(V * d, std), ln_1_weight=ones(L * d), ln_1_bias=zeros(L * d),
                 wq=nrm(L * d * d, std), bq=nrm(L * d, bias_std), wk=nrm(L * d * d, std), bk=nrm(L * d, bias_std),
                 wv=nrm(L * d * d, std), bv=nrm(L * d, bias_std), wo=nrm(L * d * d, std), bo=nrm(L * d, bias_std),
                 ln_2_weight=ones(L * d), ln_2_bias=zeros(L * d), fc1_weight=nrm(L * F * d, std),
                 fc1_bias=nrm(L * F, bias_std), fc2_weight=nrm(L * d * F, std), fc2_bias=nrm(L * d, bias_std),
                 ln_f_weight=ones(d), ln_f_bias=zeros(d))
        cls_w = np.concatenate([ones(d), zeros(d), nrm(d * d, std), nrm(d, bias_std), nrm(V * d, std),
                                nrm(V, bias_std)])
        t["classifier_weights"] = cls_w
        return cls(**t)

    def quantize_q8(self):
        """EsmWeights::quantize_q8 (lib.rs:559-582): matrices and the token embedding to Q8_0."""
        t = {k: getattr(self, k) for k in FIELDS}
        for k in MATRICES + ["token_embedding_table"]:
            t[k] = quantize_slice_to_q8(t[k])
        return EsmWeightsQ8(**t)

    def quantize_q4(self):
        """EsmWeights::quantize_q4 (lib.rs:584-607): matrices to Q4_0, embedding stays FP32."""
        t = {k: getattr(self, k) for k in FIELDS}
        for k in MATRICES:
            t[k] = quantize_slice_to_q4(t[k])
        return EsmWeightsQ4(**t)


class EsmWeightsQ8(_Weights):
    dtype = C.DTYPE_Q8_0


class EsmWeightsQ4(_Weights):
    dtype = C.DTYPE_Q4_0


class Tokenizer:
    @staticmethod
    def encode(text):
        """Tokenizer::encode (lib.rs:6511-6521)."""
        cap = len(text.encode()) + 2
        out = np.empty(cap, np.int32)
        n = C.check(C.lib().cih_tokenize(text.encode(), out.ctypes.data, cap))
        return out[:n].copy()

    _DECODE = dict(zip(range(4, 31), "LAGVSERTIDPKQNFYMHWCXBUZO.-"))
    _DECODE[32] = "*"

    @staticmethod
    def decode(token_id):
        """Tokenizer::decode (lib.rs:6523-6530): the residue letter or None."""
        return Tokenizer._DECODE.get(int(token_id))


def log_softmax_canonical(logits):
    """log_softmax_canonical (lib.rs:4426-4441) over one 33-logit row."""
    logits = np.ascontiguousarray(logits, np.float32)
    out = np.empty(33, np.float32)
    C.check(C.lib().cih_log_softmax_canonical(logits.ctypes.data, out.ctypes.data))
    return out


def matmul_tiled(dtype, x, w, bias, in_dim, out_dim):
    """matmul_tiled_{fp32,q8,q4}_parallel (lib.rs:4803, 4870, 4937) on the GPU."""
    x = np.ascontiguousarray(x, np.float32)
    seq_len = x.size // in_dim
    w = np.ascontiguousarray(w)
    bias = np.ascontiguousarray(bias, np.float32)
    out = np.empty((seq_len, out_dim), np.float32)
    C.check(C.lib().cih_matmul_tiled(dtype, out.ctypes.data, x.ctypes.data, w.ctypes.data, bias.ctypes.data,
                                     in_dim, out_dim, seq_len))
    return out


def dequantize_on_device(dtype, blocks):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    nb = blocks.size // (36 if dtype == C.DTYPE_Q8_0 else 20)
    out = np.empty(nb * 32, np.float32)
    C.check(C.lib().cih_dequantize_device(dtype, blocks.ctypes.data, nb, out.ctypes.data))
    return out


def quantize_on_device(dtype, src):
    """quantize_slice_to_q8 / _q4 (lib.rs:670-673, 1085-1088) run by the
    loader's GPU kernel: packed blocks as uint8."""
    src = np.ascontiguousarray(src, np.float32).ravel()
    out = np.empty(src.size // 32 * (36 if dtype == C.DTYPE_Q8_0 else 20), np.uint8)
    C.check(C.lib().cih_quantize_device(dtype, src.ctypes.data, src.size, out.ctypes.data))
    return out


class GpuModel:
    """Device-resident ESM-2 (one HIP stream).  Replaces the reference's
    weights + BidirectionalRunState pair for the GPU path."""

    def __init__(self, cfg, weights, contact_head=None, max_batch=1, max_len=None, outputs=C.OUT_LOGITS,
                 path=None, quantize_to=-1):
        self.cfg = cfg
        self._h = ctypes.c_void_p()
        cw, cb = (None, 0.0) if contact_head is None else contact_head
        if cw is not None:
            cw = np.ascontiguousarray(cw, np.float32)
        cw_ptr = cw.ctypes.data if cw is not None else None
        if path is not None:
            C.check(C.lib().cih_model_create_from_file(path.encode(), quantize_to, cw_ptr, float(cb),
                                                       ctypes.byref(self._h)))
            c = C.Config()
            dt = ctypes.c_int32()
            C.check(C.lib().cih_model_config(self._h, ctypes.byref(c), ctypes.byref(dt)))
            self.cfg = EsmConfig(c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.vocab_size, c.max_seq_len)
            self.dtype = dt.value
        else:
            hw, keep = weights._host()
            cc = cfg._c()
            C.check(C.lib().cih_model_create(ctypes.byref(cc), weights.dtype, ctypes.byref(hw), cw_ptr, float(cb),
                                             ctypes.byref(self._h)))
            del keep
            self.dtype = weights.dtype
        self.reserved = None
        self.reserve(max_batch, max_len or 1024, outputs)

    @classmethod
    def from_file(cls, path, quantize_to=-1, contact_head=None, **kw):
        return cls(None, None, contact_head=contact_head, path=path, quantize_to=quantize_to, **kw)

    def reserve(self, max_batch, max_len, outputs):
        C.check(C.lib().cih_model_reserve(self._h, max_batch, max_len, outputs))
        self.reserved = (max_batch, max_len, outputs)

    def close(self):
        if self._h:
            C.lib().cih_model_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, seqs, outputs=C.OUT_LOGITS):
        """Batched forward of a list of token arrays (each one reference call).
        Returns padded float32 arrays keyed by output name plus 'lens'."""
        B = len(seqs)
        lens = np.array([len(s) for s in seqs], np.int32)
        S = int(lens.max())
        toks = np.zeros((B, S), np.int32)
        for b, s in enumerate(seqs):
            toks[b, :len(s)] = s
        cfg = self.cfg
        d, V, L, H = cfg.dim, cfg.vocab_size, cfg.n_layers, cfg.n_heads
        n = max(S - 2, 0)
        res = {"lens": lens}
        shapes = {C.OUT_LOGITS: ("logits", (B, S, V)), C.OUT_HIDDEN: ("hidden", (B, S, d)),
                  C.OUT_FINAL_ATT: ("final_att", (B, S, S)), C.OUT_CONTACTS: ("contacts", (B, n, n)),
                  C.OUT_ATTN: ("attn", (B, L, H, S, S)), C.OUT_LAYER_HIDDEN: ("layer_hidden", (B, L, S, d))}
        o = C.Outputs()
        for flag, (name, shape) in shapes.items():
            if outputs & flag:
                res[name] = np.zeros(shape, np.float32)
                setattr(o, name, res[name].ctypes.data)
        C.check(C.lib().cih_forward(self._h, toks.ctypes.data, lens.ctypes.data, B, S, outputs, ctypes.byref(o)))
        return res

    def forward_device(self, tokens_ptr, lens, S_max, outputs, out_ptrs):
        """Device-pointer forward: tokens_ptr is a device int32 [B][S_max]
        buffer, out_ptrs maps output names to device float32 pointers."""
        lens = np.ascontiguousarray(lens, np.int32)
        o = C.Outputs()
        for k, v in out_ptrs.items():
            setattr(o, k, v)
        C.check(C.lib().cih_forward(self._h, ctypes.c_void_p(tokens_ptr), lens.ctypes.data, lens.size, S_max,
                                    outputs | C.IO_DEVICE, ctypes.byref(o)))

    def dms(self, residues, window=0, stride=0, mode=C.DMS_MASKED_MARGINAL, chunk=0):
        """In-silico deep mutational scan of one protein (cih_dms; the
        reference's run_pipeline_dms_with_mode, pipeline.rs:76-280).
        residues: token ids of the residues (no BOS/EOS).  Returns
        (deltas [n][20] in CANONICAL_AAS order, entropy [n])."""
        res = np.ascontiguousarray(residues, np.int32)
        n = res.size
        deltas = np.zeros((n, 20), np.float32)
        ent = np.zeros(n, np.float32)
        C.check(C.lib().cih_dms(self._h, res.ctypes.data, n, window, stride, mode, chunk, deltas.ctypes.data,
                                ent.ctypes.data))
        return deltas, ent

    def profile(self, enable=True):
        C.check(C.lib().cih_profile_enable(self._h, int(enable)))

    def profile_read(self, kc):
        s = C.KernelStats()
        C.check(C.lib().cih_profile_read(self._h, kc, ctypes.byref(s)))
        return {"launches": s.launches, "total_ms": s.total_ms, "flops": s.flops, "bytes": s.bytes}


class BidirectionalRunState:
    """Output surface of one forward (BidirectionalRunState, lib.rs:2488-2508)."""

    def __init__(self, config, max_len):
        self.max_len = max_len
        self.compute_contacts = True  # the reference's default (lib.rs:2539)
        self.logits = np.zeros(max_len * config.vocab_size, np.float32)
        self.x = np.zeros(max_len * config.dim, np.float32)
        self.final_layer_att = np.zeros(max_len * max_len, np.float32)
        self.contact_probs = np.zeros(max_len * max_len, np.float32)


def forward_bidirectional_gpu(tokens, config, model, state, on_layer=None):
    """One unpadded sequence through the GPU forward, filling `state` like
    forward_bidirectional / _q8 / _q4 do (lib.rs:5078-6147): logits, x (after
    the final LayerNorm), final_layer_att and, when state.compute_contacts,
    contact_probs.  on_layer(l, x) is called after each layer as in
    forward_bidirectional_parallel_ext (5097)."""
    tokens = np.ascontiguousarray(tokens, np.int32)
    S = tokens.size
    if S > state.max_len:
        raise ValueError(f"Sequence length {S} exceeds max_len {state.max_len}")
    flags = C.OUT_LOGITS | C.OUT_HIDDEN | C.OUT_FINAL_ATT
    if state.compute_contacts and S > 2:
        flags |= C.OUT_CONTACTS
    if on_layer is not None:
        flags |= C.OUT_LAYER_HIDDEN
    r = model.forward([tokens], flags)
    V, d = config.vocab_size, config.dim
    state.logits[:S * V] = r["logits"][0].ravel()
    state.x[:S * d] = r["hidden"][0].ravel()
    state.final_layer_att[:S * S] = r["final_att"][0].ravel()
    if flags & C.OUT_CONTACTS:
        n = S - 2
        state.contact_probs[:n * n] = r["contacts"][0].ravel()
    if on_layer is not None:
        for l in range(config.n_layers):
            on_layer(l, r["layer_hidden"][0, l].ravel())


# The reference's per-format entry points all dispatch to the same device forward.
forward_bidirectional = forward_bidirectional_gpu


def forward_bidirectional_q8(tokens, config, model, state, num_threads=1):
    forward_bidirectional_gpu(tokens, config, model, state)


def forward_bidirectional_q4(tokens, config, model, state, num_threads=1):
    forward_bidirectional_gpu(tokens, config, model, state)


CANONICAL_AAS = "ACDEFGHIKLMNPQRSTVWY"  # benchmark.rs:702-707 column order


class DmsPositionRow:
    """One scanned position (export.rs DmsPositionRow::new): mean of the 19
    non-zero deltas and the tolerance category."""

    def __init__(self, pos, wt, deltas, entropy):
        self.pos, self.wt = pos, wt
        self.deltas = np.asarray(deltas, np.float32)
        nz = self.deltas[self.deltas != 0.0]
        self.mean_delta_logp = np.float32(np.float32(nz.sum(dtype=np.float32)) / np.float32(19.0))
        self.entropy = float(entropy)
        if self.mean_delta_logp <= -3.8:
            self.category = "Catalytic / Strictly Intolerant"
        elif self.mean_delta_logp <= -2.2:
            self.category = "Conserved Structural Core"
        else:
            self.category = "Tolerated Variable"


def run_pipeline_dms(sequence, model, window_size=0, stride=0, mode=C.DMS_MASKED_MARGINAL, chunk=0):
    """run_pipeline_dms_with_mode (pipeline.rs:76-315) on the GPU model:
    returns the rows and mutations per second."""
    import time
    toks = Tokenizer.encode(sequence)[1:-1]
    t0 = time.perf_counter()
    deltas, ent = model.dms(toks, window_size, stride, mode, chunk)
    el = time.perf_counter() - t0
    rows = [DmsPositionRow(p + 1, sequence[p], deltas[p], ent[p]) for p in range(len(sequence))]
    return rows, (len(sequence) * 20 / el if el > 0 else 0.0)



class GenerationMetrics:
    """GenerationMetrics (lib.rs:6533-6536)."""

    def __init__(self, full_sequence, generated_suffix, tokens_generated, prefill_ms, generation_ms):
        self.full_sequence, self.generated_suffix = full_sequence, generated_suffix
        self.tokens_generated, self.prefill_ms, self.generation_ms = tokens_generated, prefill_ms, generation_ms
        self.throughput_tps = tokens_generated / (generation_ms / 1e3) if generation_ms > 0 else 0.0


class GpuDecoder:
    """RunState (lib.rs:2459-2486) on the GPU for n_slots sequences: per-slot
    KV caches, forward_* for batches of rows (decode), and the
    generate_sequence* loop (generate)."""

    def __init__(self, model, n_slots=1, max_len=None, max_rows=64):
        self.model = model
        self.max_len = max_len or model.cfg.max_seq_len
        self._h = ctypes.c_void_p()
        C.check(C.lib().cih_decoder_create(model._h, n_slots, self.max_len, max_rows, ctypes.byref(self._h)))
        self.n_slots, self.max_rows = n_slots, max_rows

    def close(self):
        if self._h:
            C.lib().cih_decoder_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self, slot=-1):
        C.check(C.lib().cih_decoder_reset(self._h, slot))

    def decode(self, slots, tokens, pos):
        """forward / forward_q8 / forward_q4 (lib.rs:3554-4233) for rows
        (slot, token, position): logits [n][vocab]."""
        slots = np.ascontiguousarray(slots, np.int32)
        tokens = np.ascontiguousarray(tokens, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        n = slots.size
        out = np.empty((n, self.model.cfg.vocab_size), np.float32)
        C.check(C.lib().cih_decode(self._h, slots.ctypes.data, tokens.ctypes.data, pos.ctypes.data, n,
                                   out.ctypes.data))
        return out

    def generate(self, prompts, temperature=0.0, max_new_tokens=None, seeds=None, slots=None, max_seq_len=0):
        """generate_sequence* (lib.rs:6551-6827) for a list of prompt id
        arrays: returns (list of generated id arrays, prefill_ms, generation_ms)."""
        n = len(prompts)
        slots = np.arange(n, dtype=np.int32) if slots is None else np.ascontiguousarray(slots, np.int32)
        seeds = np.zeros(n, np.uint64) if seeds is None else np.ascontiguousarray(seeds, np.uint64)
        flat = np.concatenate([np.asarray(p, np.int32) for p in prompts]).astype(np.int32)
        offs = np.zeros(n + 1, np.int32)
        offs[1:] = np.cumsum([len(p) for p in prompts])
        cap = self.max_len
        out = np.zeros((n, cap), np.int32)
        cnt = np.zeros(n, np.int32)
        pre, gen = ctypes.c_double(), ctypes.c_double()
        C.check(C.lib().cih_generate(self._h, n, slots.ctypes.data, flat.ctypes.data, offs.ctypes.data,
                                     float(temperature), -1 if max_new_tokens is None else int(max_new_tokens),
                                     seeds.ctypes.data, int(max_seq_len), out.ctypes.data, cap, cnt.ctypes.data,
                                     ctypes.byref(pre), ctypes.byref(gen)))
        return [out[i, :cnt[i]].copy() for i in range(n)], pre.value, gen.value


def prompt_tokens(prompt):
    """The ids generate_sequence* feeds (lib.rs:6563-6567): encode, drop the
    trailing <eos>, [0] if nothing is left."""
    t = list(Tokenizer.encode(prompt)[:-1])
    return np.asarray(t or [0], np.int32)


def generate_sequence(prompt, decoder, temperature=0.0, max_new_tokens=None, seed=0, slot=0):
    """generate_sequence / _q8 / _q4 (lib.rs:6538-6827) on the GPU decoder."""
    toks, pre, gen = decoder.generate([prompt_tokens(prompt)], temperature, max_new_tokens, [seed], [slot],
                                      decoder.model.cfg.max_seq_len)
    suffix = "".join(c for c in (Tokenizer.decode(t) for t in toks[0]) if c is not None)
    return GenerationMetrics(prompt + suffix, suffix, int(toks[0].size), pre, gen)
