"""MI355X-native FP8 paged-attention hot path for nano-vLLM.

Public surface (drop-in for the reference's functions of the same names):
  nanovllm_amd.kernels.fp8_attention: fp8_decode_attention, fp8_prefill_attention
  nanovllm_amd.kernels.fp8_linear:    fp8_block_linear, BLOCK_SIZE
  nanovllm_amd.layers.attention:      store_kvcache
  nanovllm_amd.layers.qk_norm_rope:   qk_norm_rope_store (fused q/k RMSNorm + RoPE + FP8 KV store)
  nanovllm_amd.utils.context:         Context, get_context, set_context, reset_context
  nanovllm_amd.engine.metadata:       host-side slot mapping / cu_seqlens / block tables
  nanovllm_amd.engine.graph:          pure-decode HIP-graph capture and replay
  nanovllm_amd.ops:                   the same calls as dispatcher operators (torch.ops.nvamd.store_kvcache,
                                      torch.ops.nvamd.decode, torch.ops.nvamd.prefill)
"""
from .kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention  # noqa: F401
from .kernels.fp8_linear import fp8_block_linear  # noqa: F401
from .layers.attention import store_kvcache  # noqa: F401
from . import ops  # noqa: F401  (registers torch.ops.nvamd.*)
