"""Fused q/k RMSNorm + rotary embedding + FP8 KV store (one attention layer).

Replaces, in nano-vLLM's Qwen3 attention (nanovllm/models/qwen3.py:99-112),
the steps between the QKV projection and the attention call::

    q, k, v = qkv.split([q_size, kv_size, kv_size], dim=-1)       # qwen3.py:103
    q = self.q_norm(q); k = self.k_norm(k)                        # qwen3.py:107-109
    q, k = self.rotary_emb(positions, q, k)                       # qwen3.py:110
    store_kvcache(k, v, k_cache, v_cache, slot_mapping)           # attention.py:61-62 (inside self.attn)

with one gfx950 kernel that reads each head row of ``qkv`` once, returns
the normalised, rotated q (bf16) and writes k and v straight into the FP8
cache.  The attention call that follows then skips its own store.  The
arithmetic keeps the reference's rounding points (fp32 math, bf16 after the
normalisation, after the weight product and after the rotation).

Before the runner allocates the cache (its warm-up runs first,
model_runner.py:35-36) the layer's caches are empty ``torch.tensor([])``:
then nothing is stored, ``slot_mapping`` is ignored, and the caller asks for
k as well (``return_k=True``), which the contiguous prefill path needs
beside v.
"""
import torch

from .. import _native


def _check(t, name, dtype, device):
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.device != device:
        raise ValueError(f"{name} must be a tensor on {device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")


def qk_norm_rope_store(positions: torch.Tensor, qkv: torch.Tensor, q_norm_weight: torch.Tensor,
                       k_norm_weight: torch.Tensor, eps: float, cos_sin_cache: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                       num_heads: int, num_kv_heads: int, head_dim: int = 128, return_k: bool = False):
    """
    Args:
        positions: [N] int (token positions, indexes cos_sin_cache)
        qkv: [N, (num_heads + 2 * num_kv_heads) * head_dim] bf16, unit column stride
        q_norm_weight, k_norm_weight: [head_dim] bf16 (RMSNorm weights)
        eps: RMSNorm epsilon
        cos_sin_cache: [max_position, head_dim] or [max_position, 1, head_dim] fp32
            (RotaryEmbedding.cos_sin_cache)
        k_cache, v_cache: [num_blocks, block_size, num_kv_heads, head_dim] FP8 E4M3FN,
            or both empty (numel() == 0) or None: no store
        slot_mapping: [N] int32; -1 stores nothing for that token (ignored
            without a cache)
    Returns:
        q: [N, num_heads, head_dim] bf16 = RoPE(RMSNorm(q)); with return_k
        also k: [N, num_kv_heads, head_dim] bf16 = RoPE(RMSNorm(k)).
    """
    lib = _native.load()
    dev = qkv.device
    _check(qkv, "qkv", torch.bfloat16, dev)
    n = qkv.shape[0]
    if qkv.dim() != 2 or qkv.shape[1] != (num_heads + 2 * num_kv_heads) * head_dim or qkv.stride(1) != 1:
        raise ValueError("qkv must be [N, (num_heads + 2 * num_kv_heads) * head_dim] with unit column stride")
    for t, name in ((q_norm_weight, "q_norm_weight"), (k_norm_weight, "k_norm_weight")):
        _check(t, name, torch.bfloat16, dev)
        if t.numel() != head_dim:
            raise ValueError(f"{name} must have head_dim elements")
    _check(cos_sin_cache, "cos_sin_cache", torch.float32, dev)
    cs = cos_sin_cache.reshape(cos_sin_cache.shape[0], -1).contiguous()
    if cs.shape[1] != head_dim:
        raise ValueError("cos_sin_cache rows must hold head_dim values (cos then sin)")
    no_cache = [c is None or c.numel() == 0 for c in (k_cache, v_cache)]
    if no_cache[0] != no_cache[1]:
        raise ValueError("k_cache and v_cache must both be allocated or both be empty")
    has_cache = not no_cache[0]
    if has_cache:
        _check(k_cache, "k_cache", torch.float8_e4m3fn, dev)
        _check(v_cache, "v_cache", torch.float8_e4m3fn, dev)
        if v_cache.shape != k_cache.shape or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("k_cache/v_cache must be contiguous and of one shape")
        if k_cache.shape[-2] * k_cache.shape[-1] != num_kv_heads * head_dim:
            raise ValueError("cache rows do not hold num_kv_heads * head_dim values")
    pos = positions.to(device=dev, dtype=torch.int64).contiguous()
    if pos.numel() != n:
        raise ValueError("positions need one entry per token")
    if has_cache:
        slots = slot_mapping.to(device=dev, dtype=torch.int32).contiguous()
        if slots.numel() != n:
            raise ValueError("slot_mapping needs one entry per token")
    wq, wk = q_norm_weight.contiguous(), k_norm_weight.contiguous()  # held until the launch is enqueued
    q = torch.empty(n, num_heads, head_dim, dtype=torch.bfloat16, device=dev)
    k = torch.empty(n, num_kv_heads, head_dim, dtype=torch.bfloat16, device=dev) if return_k else None
    if has_cache:
        num_slots = k_cache.numel() // (num_kv_heads * head_dim)
        kc, vc, sl = k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr()
    else:
        num_slots, kc, vc, sl = 0, None, None, None
    status = lib.nvamd_qk_norm_rope_store(
        qkv.data_ptr(), qkv.stride(0), pos.data_ptr(), wq.data_ptr(), wk.data_ptr(), float(eps), cs.data_ptr(),
        cs.shape[0], q.data_ptr(), k.data_ptr() if k is not None else None, kc, vc, sl, n,
        num_heads, num_kv_heads, head_dim, num_slots, torch.cuda.current_stream(dev).cuda_stream)
    _native.check(status, "qk_norm_rope_store")
    return (q, k) if return_k else q
