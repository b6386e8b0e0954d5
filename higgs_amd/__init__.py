"""higgs_amd -- MI355X (gfx950) HIP kernels for the per-layer ops of
panbanda/higgs' higgs-models (RMSNorm variants, RoPE variants, SwiGLU/GeGLU,
the Qwen3-Next gated norm, the 4-bit QuantizedEmbedding gather, the fused
residual-add + RMSNorm and embedding + RMSNorm forms, the 4-bit
quantized_matmul / gather_qmm projections and the GatedDeltaNet recurrence),
exposed
through the C ABI in include/higgs_hip.h and mirrored here for Python callers.
"""
from ._lib import ACT_GELU_TANH, ACT_SILU, HgkError, LIB_PATH, lib  # noqa: F401
from .ops import (OpSequence, QuantizedEmbedding, add_rms_norm, gated_rms_norm, gelu_approximate_mul,  # noqa: F401
                  fused_gate_up_swiglu, gather_qmm, gather_qmm_swiglu, gated_delta,
                  gated_delta_gated_norm, gdn_qk_norm_weights,
                  llama3_rope_freqs, qk_norm_rope, quantized_matmul, rms_norm, rope,
                  rope_inv_freq, silu_mul, swiglu)
