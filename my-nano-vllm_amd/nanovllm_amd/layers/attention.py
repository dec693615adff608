"""FP8 KV store, the drop-in for ``store_kvcache`` in nanovllm/layers/attention.py.

``store_kvcache`` keeps the reference's name, signature and assertions
(attention.py:33-40) and launches the gfx950 store/quantise kernel instead of
``store_kvcache_kernel``.  The reference's ``Attention`` layer (attention.py:42-126)
stays the caller: it imports this function and the two attention functions of
``nanovllm_amd.kernels.fp8_attention`` unchanged.
"""
import torch

from .. import _native


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
    if key.dtype not in (torch.bfloat16, torch.float16) or value.dtype != key.dtype:
        raise ValueError(f"key/value must both be bf16 or both fp16 (got {key.dtype}, {value.dtype})")
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
        num_slots, 1 if key.dtype == torch.float16 else 0, torch.cuda.current_stream(key.device).cuda_stream)
    _native.check(status, "store_kvcache")
