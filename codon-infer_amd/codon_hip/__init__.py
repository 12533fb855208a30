"""codon_hip — MI355X (gfx950) ESM-2 bidirectional encoder behind a C ABI.

Host-side mirror of codon-infer's model-load / forward / logits /
attention-map API, its deep mutational scan and its autoregressive
decoding.  All compute runs in libcodon_hip.so (HIP kernels);
importing fails if the library has not been built.
"""
from . import _lib
from ._lib import (CihError, DMS_MASKED_MARGINAL, DMS_WILDTYPE_MARGINAL, DTYPE_FP32, DTYPE_Q4_0, DTYPE_Q8_0,
                   IO_DEVICE, KC_ATTENTION, KC_GEMM_FP32,
                   KC_GEMM_QUANT, KC_OTHER, OUT_ATTN, OUT_CONTACTS, OUT_FINAL_ATT, OUT_HIDDEN, OUT_LAYER_HIDDEN,
                   OUT_LOGITS)
from .model import (CANONICAL_AAS, BidirectionalRunState, DmsPositionRow, EsmConfig, EsmWeights, EsmWeightsQ4,
                    EsmWeightsQ8, GenerationMetrics, GpuDecoder, GpuModel, Tokenizer, dequantize_blocks,
                    dequantize_on_device, forward_bidirectional, forward_bidirectional_gpu, forward_bidirectional_q4,
                    forward_bidirectional_q8, generate_sequence, log_softmax_canonical, matmul_tiled, prompt_tokens,
                    quantize_on_device, quantize_slice_to_q4, quantize_slice_to_q8, run_pipeline_dms, save_codq)

_lib.lib()  # load now: no silent fallback

__all__ = [n for n in dir() if not n.startswith("_")]
