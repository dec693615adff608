"""Drop-in replacement for nanovllm/kernels/fp8_attention.py on MI355X (gfx950).

Same function names, parameter names, defaults and return values as the
reference (fp8_decode_attention: fp8_attention.py:173-207,
fp8_prefill_attention: fp8_attention.py:314-353), so
nanovllm/layers/attention.py can import them unchanged.  Each call
validates its tensors, allocates the output (and, when the split-KV path
needs one, a workspace) from torch's caching allocator, and enqueues
hand-written HIP kernels on torch's current stream through the C ABI in
include/nvamd_fp8_attention.h.  Nothing synchronises, so the calls can be
captured in a HIP graph (torch.cuda.CUDAGraph).

There is no Triton and no CPU fallback: tensors must live on a ROCm GPU and
the native library must be built, otherwise the call raises.
"""
import torch

from .. import _native

_FP8 = torch.float8_e4m3fn
# element type codes of the C ABI (NVAMD_DTYPE_BF16 / NVAMD_DTYPE_F16)
_QO_DTYPES = {torch.bfloat16: 0, torch.float16: 1}


def _require(cond, msg):
    if not cond:
        raise ValueError(msg)


def _dev_tensor(t, name, dtype=None):
    _require(isinstance(t, torch.Tensor), f"{name} must be a torch.Tensor")
    _require(t.is_cuda, f"{name} must be on a ROCm GPU (got {t.device})")
    if dtype is not None:
        _require(t.dtype == dtype, f"{name} must be {dtype} (got {t.dtype})")


def _qo_dtype(q):
    _require(q.dtype in _QO_DTYPES, f"q must be bfloat16 or float16 (got {q.dtype})")
    return _QO_DTYPES[q.dtype]


def _int32(t, name):
    _dev_tensor(t, name)
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _stream_ptr(device):
    return torch.cuda.current_stream(device).cuda_stream


def _workspace(nbytes, device):
    if nbytes <= 0:
        return None, 0
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device), int(nbytes)


def fp8_decode_attention(
    q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
    block_tables: torch.Tensor, context_lens: torch.Tensor, softmax_scale: float,
) -> torch.Tensor:
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
    lib = _native.load()
    _dev_tensor(q, "q")
    qo_dtype = _qo_dtype(q)
    _dev_tensor(k_cache, "k_cache", _FP8)
    _dev_tensor(v_cache, "v_cache", _FP8)
    _require(q.dim() == 3, "q must be [batch, num_heads, head_dim]")
    _require(k_cache.dim() == 4 and v_cache.shape == k_cache.shape,
             "k_cache/v_cache must be [num_blocks, block_size, num_kv_heads, head_dim]")
    num_heads = q.shape[1]
    num_blocks, block_size, num_kv_heads, head_dim = k_cache.shape
    _require(q.shape[2] == head_dim, "q head_dim does not match the cache")
    block_tables = _int32(block_tables, "block_tables")
    context_lens = _int32(context_lens, "context_lens")
    batch_size, max_num_blocks = block_tables.shape
    _require(q.shape[0] >= batch_size and context_lens.numel() >= batch_size,
             "q and context_lens need at least block_tables.shape[0] rows")
    q = q.contiguous()
    k_cache = k_cache.contiguous()
    v_cache = v_cache.contiguous()

    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if batch_size == 0:
        return out
    ws_bytes = lib.nvamd_decode_workspace_bytes(batch_size, num_heads, num_kv_heads,
                                                max_num_blocks, block_size, 0)
    ws, ws_bytes = _workspace(ws_bytes, q.device)
    status = lib.nvamd_fp8_decode_attention(
        out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        block_tables.data_ptr(), context_lens.data_ptr(),
        batch_size, num_heads, num_kv_heads, head_dim, num_blocks, block_size, max_num_blocks,
        float(softmax_scale), 0, ws.data_ptr() if ws is not None else None, ws_bytes, qo_dtype,
        _stream_ptr(q.device))
    _native.check(status, "fp8_decode_attention")
    return out


def fp8_prefill_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    block_tables: torch.Tensor, cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float,
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
    lib = _native.load()
    _dev_tensor(q, "q")
    qo_dtype = _qo_dtype(q)
    _dev_tensor(k, "k", _FP8)
    _dev_tensor(v, "v", _FP8)
    _require(q.dim() == 3, "q must be [num_tokens, num_heads, head_dim]")
    num_tokens, num_heads, head_dim = q.shape
    cu_seqlens_q = _int32(cu_seqlens_q, "cu_seqlens_q")
    cu_seqlens_k = _int32(cu_seqlens_k, "cu_seqlens_k")
    num_seqs = cu_seqlens_q.shape[0] - 1
    _require(cu_seqlens_k.shape[0] == num_seqs + 1, "cu_seqlens_k must have num_seqs + 1 entries")
    if block_tables is None:
        _require(k.dim() == 3 and v.shape == k.shape, "contiguous k/v must be [num_kv_tokens, num_kv_heads, head_dim]")
        num_kv_heads = k.shape[1]
        num_kv_rows, block_size, max_num_blocks = k.shape[0], 0, 0
        kv_cap = num_kv_rows
        bt_ptr = None
    else:
        _require(k.dim() == 4 and v.shape == k.shape,
                 "paged k/v must be [num_blocks, block_size, num_kv_heads, head_dim]")
        block_tables = _int32(block_tables, "block_tables")
        _require(block_tables.shape[0] >= num_seqs, "block_tables needs a row per sequence")
        num_blocks, block_size, num_kv_heads, _ = k.shape
        num_kv_rows = num_blocks * block_size
        max_num_blocks = block_tables.shape[1]
        kv_cap = max_num_blocks * block_size
        bt_ptr = block_tables.data_ptr()
    _require(k.shape[-1] == head_dim, "k head_dim does not match q")
    q = q.contiguous()
    k = k.contiguous()
    v = v.contiguous()

    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if num_tokens == 0 or num_seqs <= 0:
        return out
    max_seqlen_q = int(max_seqlen_q)
    ws_bytes = lib.nvamd_prefill_workspace_bytes(num_tokens, num_seqs, num_heads, num_kv_heads,
                                                 kv_cap, max_seqlen_q, block_size, 0)
    ws, ws_bytes = _workspace(ws_bytes, q.device)
    status = lib.nvamd_fp8_prefill_attention(
        out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), bt_ptr,
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(),
        num_tokens, num_seqs, num_heads, num_kv_heads, head_dim, num_kv_rows, block_size,
        max_num_blocks, max_seqlen_q, int(max_seqlen_k), float(softmax_scale), 0,
        ws.data_ptr() if ws is not None else None, ws_bytes, qo_dtype, _stream_ptr(q.device))
    _native.check(status, "fp8_prefill_attention")
    return out
