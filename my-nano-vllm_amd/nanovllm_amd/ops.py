"""The attention path as operators of torch's dispatcher.

``torch.ops.nvamd.store_kvcache``, ``torch.ops.nvamd.decode`` and
``torch.ops.nvamd.prefill`` carry the schemas a ``TORCH_LIBRARY`` block would
declare for the reference's three calls (store: attention.py:33-40; decode:
fp8_attention.py:173-207; prefill: fp8_attention.py:314-353):

    store_kvcache(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor slot_mapping) -> ()
    decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, Tensor context_lens, float scale) -> Tensor
    prefill(Tensor q, Tensor k, Tensor v, Tensor? block_tables, Tensor cu_q, Tensor cu_k, SymInt max_q,
            SymInt max_k, float scale) -> Tensor

Their CUDA (ROCm) kernels are the same C-ABI calls as the Python functions of
``nanovllm_amd.kernels.fp8_attention`` and ``nanovllm_amd.layers.attention``;
their fake implementations give torch.compile and FakeTensor tracing the
output shapes without running anything.  There is no CPU kernel: a call on
CPU tensors raises.
"""
from typing import Optional

import torch

from .kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention
from .layers.attention import store_kvcache as _store_kvcache


@torch.library.custom_op("nvamd::store_kvcache", mutates_args=("k_cache", "v_cache"), device_types="cuda")
def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    _store_kvcache(key, value, k_cache, v_cache, slot_mapping)


@store_kvcache.register_fake
def _(key, value, k_cache, v_cache, slot_mapping):
    return None


@torch.library.custom_op("nvamd::decode", mutates_args=(), device_types="cuda")
def decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
           context_lens: torch.Tensor, scale: float) -> torch.Tensor:
    return fp8_decode_attention(q, k_cache, v_cache, block_tables, context_lens, scale)


@decode.register_fake
def _(q, k_cache, v_cache, block_tables, context_lens, scale):
    return torch.empty_like(q)


@torch.library.custom_op("nvamd::prefill", mutates_args=(), device_types="cuda")
def prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_tables: Optional[torch.Tensor],
            cu_q: torch.Tensor, cu_k: torch.Tensor, max_q: int, max_k: int, scale: float) -> torch.Tensor:
    return fp8_prefill_attention(q, k, v, block_tables=block_tables, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                                 max_seqlen_q=max_q, max_seqlen_k=max_k, softmax_scale=scale)


@prefill.register_fake
def _(q, k, v, block_tables, cu_q, cu_k, max_q, max_k, scale):
    return torch.empty_like(q)
