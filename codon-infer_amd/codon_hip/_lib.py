"""ctypes binding of libcodon_hip.so (the C ABI in include/codon_hip.h).

The library is loaded from this package directory only; if it is missing the
import fails loudly — there is no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcodon_hip.so")

CIH_OK = 0
STATUS = {
    -1: "CIH_ERR_ARG", -2: "CIH_ERR_SHAPE", -3: "CIH_ERR_CAPACITY", -4: "CIH_ERR_CONTACTS",
    -5: "CIH_ERR_HIP", -6: "CIH_ERR_IO", -7: "CIH_ERR_FORMAT", -8: "CIH_ERR_TOKEN",
}
DTYPE_FP32, DTYPE_Q8_0, DTYPE_Q4_0 = 0, 1, 2

OUT_LOGITS = 1 << 0
OUT_HIDDEN = 1 << 1
OUT_FINAL_ATT = 1 << 2
OUT_CONTACTS = 1 << 3
OUT_ATTN = 1 << 4
OUT_LAYER_HIDDEN = 1 << 5
IO_DEVICE = 1 << 16

KC_GEMM_QUANT, KC_GEMM_FP32, KC_ATTENTION, KC_OTHER = 0, 1, 2, 3

EXPORTED = [
    "cih_model_create", "cih_model_create_from_file", "cih_model_reserve", "cih_model_config",
    "cih_model_destroy", "cih_forward", "cih_matmul_tiled", "cih_dequantize_device", "cih_quantize_device", "cih_quantize_q8",
    "cih_quantize_q4", "cih_dequantize_q8", "cih_dequantize_q4", "cih_tokenize", "cih_log_softmax_canonical",
    "cih_profile_enable", "cih_profile_read", "cih_last_error", "cih_abi_version", "cih_dms",
    "cih_decoder_create", "cih_decoder_destroy", "cih_decoder_reset", "cih_decode", "cih_generate",
    "cih_matmul_tiled_noalloc",
]

DMS_MASKED_MARGINAL, DMS_WILDTYPE_MARGINAL = 0, 1


class CihError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code


class Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("dim", "hidden_dim", "n_layers", "n_heads", "vocab_size", "max_seq_len")]


class HostWeights(ctypes.Structure):
    _fields_ = [
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


class Outputs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("logits", "hidden", "final_att", "contacts", "attn", "layer_hidden")]


class KernelStats(ctypes.Structure):
    _fields_ = [("launches", ctypes.c_int64), ("total_ms", ctypes.c_double), ("flops", ctypes.c_double),
                ("bytes", ctypes.c_double)]


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libcodon_hip.so not built at {LIB_PATH}; run `python codon-infer_amd/build.py`")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    pmodel = ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "cih_model_create": [ctypes.POINTER(Config), i32, ctypes.POINTER(HostWeights), vp, f32, pmodel],
        "cih_model_create_from_file": [ctypes.c_char_p, i32, vp, f32, pmodel],
        "cih_model_reserve": [vp, i32, i32, ctypes.c_uint32],
        "cih_model_config": [vp, ctypes.POINTER(Config), ctypes.POINTER(i32)],
        "cih_model_destroy": [vp],
        "cih_forward": [vp, vp, vp, i32, i32, ctypes.c_uint32, ctypes.POINTER(Outputs)],
        "cih_dms": [vp, vp, i32, i32, i32, i32, i32, vp, vp],
        "cih_decoder_create": [vp, i32, i32, i32, pmodel],
        "cih_decoder_destroy": [vp],
        "cih_decoder_reset": [vp, i32],
        "cih_decode": [vp, vp, vp, vp, i32, vp],
        "cih_generate": [vp, i32, vp, vp, vp, f32, i32, vp, i32, vp, i32, vp, ctypes.POINTER(ctypes.c_double),
                         ctypes.POINTER(ctypes.c_double)],
        "cih_matmul_tiled": [i32, vp, vp, vp, vp, i32, i32, i32],
        "cih_matmul_tiled_noalloc": [i32, vp, vp, vp, vp, i32, i32, i32, vp],
        "cih_dequantize_device": [i32, vp, i64, vp],
        "cih_quantize_device": [i32, vp, i64, vp],
        "cih_quantize_q8": [vp, i64, vp],
        "cih_quantize_q4": [vp, i64, vp],
        "cih_dequantize_q8": [vp, i64, vp],
        "cih_dequantize_q4": [vp, i64, vp],
        "cih_tokenize": [ctypes.c_char_p, vp, i32],
        "cih_log_softmax_canonical": [vp, vp],
        "cih_profile_enable": [vp, i32],
        "cih_profile_read": [vp, i32, ctypes.POINTER(KernelStats)],
        "cih_last_error": [],
        "cih_abi_version": [],
    }
    for name, args in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    L.cih_last_error.restype = ctypes.c_char_p
    _lib = L
    return L


def check(rc):
    """Raises CihError for a negative status; returns rc otherwise."""
    if rc < 0:
        raise CihError(rc, lib().cih_last_error().decode(errors="replace"))
    return rc
