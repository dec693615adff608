"""The reference's FP8 ``Attention`` layer, restated over this package's kernels (TEST HARNESS).

nanovllm/layers/attention.py:42-126 is the caller of the drop-in functions:
write the new K/V into the paged FP8 cache (``store_kvcache``), run decode on
the rows before ``split_pt`` and varlen prefill on the rest, concatenate.
In a deployment the reference keeps its own layer and imports the functions
of ``nanovllm_amd``; this copy lets the tests drive the kernels the way the
layer does (graph capture, the random-init Qwen3 greedy check).  The bf16
(flash-attn) branch of the reference is not restated: a non-FP8 cache raises
``NotImplementedError``.
"""
import torch
from torch import nn

from nanovllm_amd.kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention
from nanovllm_amd.layers.attention import store_kvcache
from nanovllm_amd.utils.context import get_context


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
