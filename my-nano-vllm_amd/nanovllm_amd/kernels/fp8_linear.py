"""Drop-in replacement for nanovllm/kernels/fp8_linear.py on MI355X (gfx950).

``fp8_block_linear(x, weight, weight_scale)`` keeps the reference's name,
arguments, assertions and return value (fp8_linear.py:93-139), so
nanovllm/layers/linear.py (LinearBase.apply_linear, :56-62) can import it
unchanged.  It is one dispatcher call of the C++ operator
torch.ops.nvamd.fp8_block_linear (csrc/torch_ops.cpp), which runs the
reference's two steps as two hand-written HIP kernels behind the C ABI in
include/nvamd_fp8_linear.h, enqueued on torch's current stream: the
per-token, per-128-column dynamic activation quantisation
(``nvamd_fp8_act_quant``) and the 128 x 128 block-scaled FP8 GEMM
(``nvamd_fp8_block_gemm``).  The quantised activations and their scales are
allocated from torch's caching allocator, like the reference's.

There is no Triton and no CPU fallback: tensors must live on a ROCm GPU and
the native libraries must be built, otherwise the call raises.
"""
import torch

from .. import _native

# compressed-tensors FP8_BLOCK block size (fp8_linear.py:8)
BLOCK_SIZE = 128

_linear_op = None


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
    global _linear_op
    M, K = x.shape
    N = weight.shape[0]
    Nc, Kc = weight_scale.shape
    assert weight.dtype == torch.float8_e4m3fn
    assert N == Nc * BLOCK_SIZE and K == Kc * BLOCK_SIZE
    if _linear_op is None:
        _linear_op = _native.load_ops().fp8_block_linear.default
    return _linear_op(x, weight, weight_scale)
