"""FP8 KV store, the drop-in for ``store_kvcache`` in nanovllm/layers/attention.py.

``store_kvcache`` keeps the reference's name, signature and assertions
(attention.py:33-40) and calls the C++ operator torch.ops.nvamd.store_kvcache
(csrc/torch_ops.cpp: dtype and device checks, then the gfx950
store/quantise kernel through the C ABI) instead of ``store_kvcache_kernel``.
key/value may be bf16 or fp16.  The reference's ``Attention`` layer
(attention.py:42-126) stays the caller: it imports this function and the two
attention functions of ``nanovllm_amd.kernels.fp8_attention`` unchanged.
"""
from .. import _native

_store_op = None


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    global _store_op
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    if _store_op is None:
        _store_op = _native.load_ops().store_kvcache.default
    _store_op(key, value, k_cache, v_cache, slot_mapping)
