"""Oracle: q/k RMSNorm + RoPE + FP8 KV store of one attention layer (TEST INFRASTRUCTURE ONLY).

Restates, on the CPU with torch, the steps between the QKV projection and the
attention call of nano-vLLM's Qwen3 layer:

* split of the fused projection output into q, k, v views
  (nanovllm/models/qwen3.py:103-106);
* q_norm / k_norm: RMSNorm per head over head_dim (nanovllm/layers/layernorm.py:16-25,
  called at qwen3.py:107-109): ``x.float()``, ``var = mean(x^2)``,
  ``x * rsqrt(var + eps)``, rounded to the input dtype (bf16), then multiplied
  by the bf16 weight (a bf16 product, i.e. rounded again);
* rotary embedding, neox style over the full head (nanovllm/layers/rotary_embedding.py:6-14,
  40-50, applied at qwen3.py:110): with cos/sin the fp32 halves of
  ``cos_sin_cache[position]``, ``y1 = x1*cos - x2*sin``, ``y2 = x2*cos + x1*sin``
  computed in fp32 from the bf16 inputs, rounded to bf16;
* the store of the rotated k and the unmodified v into the FP8 cache
  (nanovllm/layers/attention.py:61-62, restated by ``oracle.fp8.store_kvcache``).

``rope_cache`` builds the reference's cos/sin table (rotary_embedding.py:26-33).

The reference's RMSNorm and RoPE run under ``@torch.compile``
(layernorm.py:16, rotary_embedding.py:37).  Its source rounds the
normalised row to bf16 before the weight product (``x.to(orig_dtype).mul_
(self.weight)``), which eager mode executes as written; inductor, with its
default ``emulate_precision_casts = False``, may fuse the downcast and the
following upcast away and round once, after the product.  ``fused_norm``
selects that single-rounding form (RoPE has no intermediate rounding in
either mode: fp32 math, one cast at the end).

Pinned by tests/test_oracle_qk_norm_rope.py: RMSNorm against torch's own
``rms_norm`` in float64 and the constant-vector closed form; RoPE against a
complex multiplication in float64, position 0 as the identity and the
preservation of each rotated pair's norm; the store by the FP8 oracle.
"""
import torch

from . import fp8 as _fp8


def rope_cache(head_dim, max_position, base):
    """float32 [max_position, head_dim]: cos of the head_dim/2 frequencies, then sin
    (rotary_embedding.py:26-33)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    angles = torch.outer(torch.arange(max_position, dtype=torch.float), inv_freq)
    return torch.cat((angles.cos(), angles.sin()), dim=-1)


def rms_norm_bf16(x, weight, eps, fused_norm=False):
    """x: bf16 [..., D]; weight: bf16 [D] -> bf16 [..., D] (layernorm.py:16-25);
    fused_norm: one rounding after the weight product instead of two."""
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    y = xf * torch.rsqrt(var + eps)
    if not fused_norm:
        y = y.to(torch.bfloat16).float()
    return (y * weight.float()).to(torch.bfloat16)


def rope_bf16(x, positions, cache):
    """x: bf16 [N, H, D]; positions: int [N]; cache: float32 [max_pos, D]
    -> bf16 [N, H, D] (rotary_embedding.py:6-14, 45-50)."""
    half = x.shape[-1] // 2
    cs = cache[positions.long()].unsqueeze(1)          # [N, 1, D]
    cos, sin = cs[..., :half], cs[..., half:]
    x1, x2 = x.float()[..., :half], x.float()[..., half:]
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(torch.bfloat16)


def qk_norm_rope_store(qkv, num_heads, num_kv_heads, head_dim, positions, q_weight, k_weight, eps, cache,
                       k_cache, v_cache, slot_mapping, fused_norm=False):
    """qkv: bf16 [N, (Hq + 2 Hkv) * D]; k_cache/v_cache: uint8 [P, bs, Hkv, D]
    written in place (rows with slot -1 skipped).  Returns (q, k): bf16
    [N, Hq, D] and [N, Hkv, D] after RMSNorm and RoPE."""
    n = qkv.shape[0]
    q_size, kv_size = num_heads * head_dim, num_kv_heads * head_dim
    q = qkv[:, :q_size].reshape(n, num_heads, head_dim)
    k = qkv[:, q_size:q_size + kv_size].reshape(n, num_kv_heads, head_dim)
    v = qkv[:, q_size + kv_size:q_size + 2 * kv_size].reshape(n, num_kv_heads, head_dim)
    q = rope_bf16(rms_norm_bf16(q, q_weight, eps, fused_norm), positions, cache)
    k = rope_bf16(rms_norm_bf16(k, k_weight, eps, fused_norm), positions, cache)
    _fp8.store_kvcache(k, v, k_cache, v_cache, slot_mapping)
    return q, k
