"""FP8 KV store and the attention layer, mirroring nanovllm/layers/attention.py.

``store_kvcache`` keeps the reference's name, signature and assertions
(attention.py:33-40) and launches the gfx950 store/quantise kernel instead of
``store_kvcache_kernel``.  ``Attention`` restates the layer's FP8 path
(attention.py:42-126): write the new K/V into the paged FP8 cache, run decode
on the rows before ``split_pt`` and varlen prefill on the rest, concatenate.
The bf16 (flash-attn) branch of the reference is outside this package: a
non-FP8 cache raises ``NotImplementedError``.
"""
import torch
from torch import nn

from .. import _native
from ..kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention
from ..utils.context import get_context


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor):
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    lib = _native.load()
    for t, name in ((key, "key"), (value, "value"), (k_cache, "k_cache"), (v_cache, "v_cache"),
                    (slot_mapping, "slot_mapping")):
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a ROCm GPU (got {t.device})")
    if key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
        raise ValueError("key/value must be bf16")
    if k_cache.dtype != torch.float8_e4m3fn or v_cache.dtype != torch.float8_e4m3fn:
        raise ValueError("k_cache/v_cache must be float8_e4m3fn")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache must be contiguous")
    if tuple(value.shape) != tuple(key.shape):
        raise ValueError("key and value shapes differ")
    if slot_mapping.dtype != torch.int32:
        slot_mapping = slot_mapping.to(torch.int32)
    slot_mapping = slot_mapping.contiguous()
    num_slots = k_cache.numel() // D
    status = lib.nvamd_store_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(), N, num_heads, head_dim,
        num_slots, torch.cuda.current_stream(key.device).cuda_stream)
    _native.check(status, "store_kvcache")


class Attention(nn.Module):

    def __init__(self, num_heads, head_dim, scale):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        # bound to the model runner's per-layer cache views (kv_cache[0/1, layer])
        self.k_cache = self.v_cache = torch.tensor([])

    def forward(self, q, k, v):
        context = get_context()
        split_pt = context.split_pt
        if self.k_cache.numel() > 0:
            store_kvcache(k, v, self.k_cache, self.v_cache, context.slot_mapping)

        block_tables = context.block_tables
        if block_tables is not None:
            d_block_tables = block_tables[:split_pt]
            p_block_tables = block_tables[split_pt:]
            if d_block_tables.numel() == 0:
                d_block_tables = None
            if p_block_tables.numel() == 0:
                p_block_tables = None
        else:
            d_block_tables = p_block_tables = None

        q_d = q[:split_pt]
        q_p = q[split_pt:]
        if p_block_tables is not None:
            k_p, v_p = self.k_cache, self.v_cache
        else:
            k_p, v_p = k[split_pt:], v[split_pt:]

        outs = []
        if len(q_d) > 0:
            outs.append(self._decode_attention(q_d, self.k_cache, self.v_cache, d_block_tables,
                                               context.context_lens))
        if len(q_p) > 0:
            outs.append(self._prefill_attention(q_p, k_p, v_p,
                                                max_seqlen_q=context.max_seqlen_q,
                                                cu_seqlens_q=context.cu_seqlens_q,
                                                max_seqlen_k=context.max_seqlen_k,
                                                cu_seqlens_k=context.cu_seqlens_k,
                                                block_tables=p_block_tables))
        return outs[0] if len(outs) == 1 else torch.cat(outs, 0)

    def _decode_attention(self, q, k, v, block_tables, context_lens):
        if k.dtype != torch.float8_e4m3fn:
            raise NotImplementedError("nanovllm_amd implements the FP8 KV-cache path only")
        return fp8_decode_attention(q, k, v, block_tables, context_lens, self.scale)

    def _prefill_attention(self, q, k, v, max_seqlen_q, max_seqlen_k, cu_seqlens_q, cu_seqlens_k,
                           block_tables):
        if k.dtype != torch.float8_e4m3fn:
            raise NotImplementedError("nanovllm_amd implements the FP8 KV-cache path only")
        return fp8_prefill_attention(q, k, v, max_seqlen_q=max_seqlen_q, cu_seqlens_q=cu_seqlens_q,
                                     max_seqlen_k=max_seqlen_k, cu_seqlens_k=cu_seqlens_k,
                                     softmax_scale=self.scale, block_tables=block_tables)
