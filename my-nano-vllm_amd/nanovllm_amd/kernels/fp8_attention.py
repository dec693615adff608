"""Drop-in replacement for nanovllm/kernels/fp8_attention.py on MI355X (gfx950).

Same function names, parameter names, defaults and return values as the
reference (fp8_decode_attention: fp8_attention.py:173-207,
fp8_prefill_attention: fp8_attention.py:314-353), so
nanovllm/layers/attention.py can import them unchanged.  Each call is one
dispatcher call of the C++ operator torch.ops.nvamd.decode / prefill
(csrc/torch_ops.cpp): it validates the tensors (ValueError on bad
arguments), allocates the output (and, when the kernels need one, a
workspace) from torch's caching allocator, and enqueues hand-written HIP
kernels on torch's current stream through the C ABI in
include/nvamd_fp8_attention.h.  Nothing synchronises, so the calls can be
captured in a HIP graph (torch.cuda.CUDAGraph).

q may be bf16 or fp16 (the output has q's dtype, as empty_like(q) in the
reference).  There is no Triton and no CPU fallback: tensors must live on a
ROCm GPU and the native libraries must be built, otherwise the call raises.
"""
from .. import _native

_decode_op = None
_prefill_op = None


def _ops():
    global _decode_op, _prefill_op
    ops = _native.load_ops()
    _decode_op, _prefill_op = ops.decode.default, ops.prefill.default


def fp8_decode_attention(
    q, k_cache, v_cache, block_tables, context_lens, softmax_scale,
):
    """
    Args:
        q: [batch_size, num_heads, head_dim] bf16 or fp16
        k_cache: [num_blocks, block_size, num_kv_heads, head_dim] (FP8 E4M3FN)
        v_cache: same as k_cache
        block_tables: [batch_size, max_num_blocks] int32
        context_lens: [batch_size] int32
        softmax_scale: attention scaling factor (1/sqrt(head_dim))

    Returns:
        [batch_size, num_heads, head_dim] attention output of q's dtype
        (rows with context_lens == 0 are zero).
    """
    if _decode_op is None:
        _ops()
    return _decode_op(q, k_cache, v_cache, block_tables, context_lens, float(softmax_scale))


def fp8_prefill_attention(
    q, k, v, block_tables, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
):
    """Varlen causal (chunked) prefill with FP8 K/V.

    Args:
        q: [num_tokens, num_heads, head_dim] bf16 or fp16 (the output's dtype)
        k, v: paged caches [num_blocks, block_size, num_kv_heads, head_dim]
              when block_tables is given, else contiguous [num_kv_tokens,
              num_kv_heads, head_dim]; FP8 E4M3FN
        block_tables: [num_seqs, max_num_blocks] int32 or None
        cu_seqlens_q, cu_seqlens_k: [num_seqs + 1] int32 prefix sums
        max_seqlen_q: longest query length (host int)
        max_seqlen_k: longest key length (host int; accepted, not needed)
        softmax_scale: attention scaling factor

    Query row i of sequence s attends to keys j <= i + (Lk - Lq).
    """
    if _prefill_op is None:
        _ops()
    return _prefill_op(q, k, v, block_tables, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), int(max_seqlen_k),
                       float(softmax_scale))
