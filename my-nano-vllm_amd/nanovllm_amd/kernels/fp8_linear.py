"""Drop-in replacement for nanovllm/kernels/fp8_linear.py on MI355X (gfx950).

``fp8_block_linear(x, weight, weight_scale)`` keeps the reference's name,
arguments, assertions and return value (fp8_linear.py:93-139), so
nanovllm/layers/linear.py (LinearBase.apply_linear, :56-62) can import it
unchanged.  As in the reference it runs two kernels: the per-token,
per-128-column dynamic activation quantisation (``nvamd_fp8_act_quant``) and
the 128 x 128 block-scaled FP8 GEMM (``nvamd_fp8_block_gemm``), both
hand-written HIP behind the C ABI in include/nvamd_fp8_linear.h, enqueued on
torch's current stream.  The quantised activations and their scales are
allocated from torch's caching allocator, like the reference's.

There is no Triton and no CPU fallback: tensors must live on a ROCm GPU and
the native library must be built, otherwise the call raises.
"""
import torch

from .. import _native

# compressed-tensors FP8_BLOCK block size (fp8_linear.py:8)
BLOCK_SIZE = 128

_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1}


def fp8_block_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
) -> torch.Tensor:
    """
    Block-scaled FP8 linear layer: y = x @ weight.T
    Args:
        x: [M, K] bf16 / fp16 activations
        weight: [N, K] FP8 E4M3 weights
        weight_scale: [N/128, K/128] bf16 per-block weight scales
    Returns:
        [M, N], with x's dtype and device
    """
    M, K = x.shape
    N = weight.shape[0]
    Nc, Kc = weight_scale.shape
    assert weight.dtype == torch.float8_e4m3fn
    assert N == Nc * BLOCK_SIZE and K == Kc * BLOCK_SIZE
    for t, name in ((x, "x"), (weight, "weight"), (weight_scale, "weight_scale")):
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a ROCm GPU (got {t.device})")
    if x.dtype not in _DTYPE_CODE:
        raise ValueError(f"x must be bf16 or fp16 (got {x.dtype})")
    if weight_scale.dtype != torch.bfloat16:
        weight_scale = weight_scale.to(torch.bfloat16)
    if x.stride(1) != 1 or x.stride(0) % 8 != 0 or x.data_ptr() % 16 != 0:
        x = x.contiguous()
    if weight.stride(1) != 1 or weight.stride(0) % 16 != 0 or weight.data_ptr() % 16 != 0:
        weight = weight.contiguous()
    weight_scale = weight_scale.contiguous()
    lib = _native.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream

    # (1) dynamic activation quantisation
    xq = torch.empty((M, K), device=x.device, dtype=torch.float8_e4m3fn)
    x_scale = torch.empty((M, Kc), device=x.device, dtype=torch.bfloat16)
    _native.check(lib.nvamd_fp8_act_quant(x.data_ptr(), x.stride(0), _DTYPE_CODE[x.dtype], xq.data_ptr(),
                                          x_scale.data_ptr(), M, K, stream), "fp8_act_quant")

    # (2) block-scaled FP8 GEMM
    out = torch.empty((M, N), device=x.device, dtype=x.dtype)
    _native.check(lib.nvamd_fp8_block_gemm(xq.data_ptr(), x_scale.data_ptr(), weight.data_ptr(), weight.stride(0),
                                           weight_scale.data_ptr(), out.data_ptr(), out.stride(0),
                                           _DTYPE_CODE[x.dtype], M, N, K, stream), "fp8_block_gemm")
    return out
