"""Oracle: FP8 block-scaled linear layer (TEST INFRASTRUCTURE ONLY).

Restates on the CPU the two kernels behind ``fp8_block_linear``
(nanovllm/kernels/fp8_linear.py:93-139), the linear layer of FP8 checkpoints
(nanovllm/layers/linear.py:56-62):

* ``act_quant`` -- fp8_dyn_quant_kernel (fp8_linear.py:11-31, launched at
  :116-123).  Per token m and 128-column group g of x (bf16 or fp16, read as
  fp32): ``amax = max |x|``; ``scale = amax / 448`` (fp32), replaced by 1 when
  it is not > 0 (an all-zero group); ``xq = E4M3FN(clamp(x / scale, -448,
  448))``; the scale is stored as bf16 (``x_scale`` is allocated bf16 at
  :118).  The GEMM then uses that bf16 scale, not the fp32 one ``xq`` was
  divided by, exactly as the reference does.
* ``block_gemm`` -- fp8_block_gemm_kernel (fp8_linear.py:34-71, launched at
  :125-138).  ``out[m, n] = sum_kc partial[m, n, kc] * (sx[m, kc] * sw[n // 128,
  kc])`` with ``partial`` the fp32 dot product of one 128-wide K block
  (``tl.dot(..., out_dtype=fp32)``), the scale product in fp32 and the sum over
  K blocks accumulated in fp32 in increasing kc (:56-66); the result is
  rounded to the output dtype (x's dtype, :128) at the store (:68-71).

Rounding points restated:
  * divisions are IEEE fp32 (correctly rounded);
  * fp32 -> E4M3FN is round-to-nearest-even after the clamp (the NVIDIA
    lowering converts with ``cvt.rn.satfinite``); fp32 -> bf16 / fp16 is
    round-to-nearest-even (``oracle.fp8.e4m3_encode``, ``f32_to_bf16_bits``,
    numpy's float16 cast);
  * a 128-wide partial is computed exactly (float64: every product of two
    E4M3FN values is exact and 128 of them sum exactly in 53 bits) and
    rounded once to fp32 -- the tensor-core dot product's own summation order
    is not specified by the reference, so implementations may differ from
    this in the last bits of a partial.

Where an NVIDIA run of the reference can differ from this restatement: Triton
lowers fp32 ``/`` to PTX ``div.full.f32`` (within 2 ulp, not correctly
rounded), so an ``xq`` byte can differ where x / scale lies within 2 ulp of a
midpoint between two E4M3FN values.  NaN inputs are outside the contract.

Pinned by tests/test_oracle_fp8_linear.py: the reference's exhaustive bf16 ->
E4M3FN table on groups whose scale is exactly 1; torch's own CPU casts
(float32 -> float8_e4m3fn, -> bfloat16, -> float16); the closed forms of the
amax element (+-448), zero and constant groups; the E4M3 error bound of
dequantised values; and, for the GEMM, torch float64 matmuls of the
dequantised operands, an all-exact integer case that must match bit for bit,
and the locality of every (weight block, K block) scale.
"""
import numpy as np

from . import fp8 as _fp8

BLOCK = 128
FP8_MAX = np.float32(448.0)


def f32_to_bf16_bits(x):
    """float32 values -> uint16 bf16 bit patterns, round to nearest even (finite inputs)."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def to_f32(x):
    """torch bf16 / fp16 tensor, or uint16 bf16 bit patterns -> float32 numpy array (exact)."""
    if hasattr(x, "dtype") and str(x.dtype) in ("torch.bfloat16", "torch.float16"):
        import torch
        return x.detach().cpu().to(torch.float32).numpy()
    a = np.asarray(x)
    if a.dtype == np.uint16:
        return _fp8.bf16_bits_to_f32(a)
    return a.astype(np.float32)


def act_quant(x):
    """Per-token, per-128-group dynamic quantisation (fp8_linear.py:11-31).

    x: [M, K] bf16 / fp16 (torch) or float32 values exactly representable in
    the input dtype, K % 128 == 0.  Returns (xq: uint8 [M, K] E4M3FN codes,
    x_scale: uint16 [M, K / 128] bf16 bit patterns, scale32: float32
    [M, K / 128], the unrounded scale x was divided by)."""
    xf = to_f32(x)
    M, K = xf.shape
    assert K % BLOCK == 0
    g = xf.reshape(M, K // BLOCK, BLOCK)
    amax = np.abs(g).max(axis=-1)                          # exact
    scale = (amax / FP8_MAX).astype(np.float32)            # IEEE fp32 division
    scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    y = (g / scale[..., None]).astype(np.float32)          # IEEE fp32 division
    y = np.clip(y, -FP8_MAX, FP8_MAX)
    xq = _fp8.e4m3_encode(y).reshape(M, K)
    return xq, f32_to_bf16_bits(scale), scale


def block_gemm(xq, x_scale, w, w_scale, out_dtype="bf16"):
    """Block-scaled FP8 GEMM (fp8_linear.py:34-71).

    xq: uint8 [M, K] codes; x_scale: uint16 [M, K/128] bf16 bits; w: uint8
    [N, K] codes; w_scale: uint16 [N/128, K/128] bf16 bits.  Returns the
    output as uint16 bit patterns [M, N] of out_dtype ("bf16" or "fp16") and
    the fp32 accumulator [M, N]."""
    xq = np.asarray(xq, dtype=np.uint8)
    w = np.asarray(w, dtype=np.uint8)
    M, K = xq.shape
    N = w.shape[0]
    Kc = K // BLOCK
    assert w.shape[1] == K and N % BLOCK == 0 and K % BLOCK == 0
    table = _fp8.dequant_table().astype(np.float64)
    xv = table[xq].reshape(M, Kc, BLOCK)
    wv = table[w].reshape(N, Kc, BLOCK)
    sx = _fp8.bf16_bits_to_f32(np.asarray(x_scale, dtype=np.uint16))          # [M, Kc]
    sw = _fp8.bf16_bits_to_f32(np.asarray(w_scale, dtype=np.uint16))          # [Nc, Kc]
    sw_n = np.repeat(sw, BLOCK, axis=0)                                        # [N, Kc]
    acc = np.zeros((M, N), dtype=np.float32)
    for kc in range(Kc):
        partial = (xv[:, kc, :] @ wv[:, kc, :].T).astype(np.float32)          # exact sum, one rounding
        s = (sx[:, kc][:, None] * sw_n[:, kc][None, :]).astype(np.float32)    # exact: bf16 x bf16
        acc = (acc + (partial * s).astype(np.float32)).astype(np.float32)
    if out_dtype == "bf16":
        return f32_to_bf16_bits(acc), acc
    return acc.astype(np.float16).view(np.uint16), acc


def block_linear(x, w, w_scale):
    """fp8_block_linear (fp8_linear.py:93-139): x [M, K] bf16/fp16 (torch),
    w uint8 [N, K] codes, w_scale uint16 [N/128, K/128] bf16 bits -> output
    bit patterns [M, N] in x's dtype."""
    xq, x_scale, _ = act_quant(x)
    out_dtype = "fp16" if str(getattr(x, "dtype", "")) == "torch.float16" else "bf16"
    return block_gemm(xq, x_scale, w, w_scale, out_dtype)[0]
