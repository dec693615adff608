/*
 * C ABI of the MI355X (gfx950) FP8 block-scaled linear layer.
 *
 * These entry points replace the two Triton launches of nano-vLLM's
 * fp8_block_linear (nanovllm/kernels/fp8_linear.py:93-139, called from
 * LinearBase.apply_linear, nanovllm/layers/linear.py:56-62); the Python
 * function that wraps them keeps the reference's name and signature:
 *
 *   nvamd_fp8_act_quant   <- fp8_dyn_quant_kernel[(M, Kc)]   nanovllm/kernels/fp8_linear.py:119-123
 *                            (kernel fp8_linear.py:11-31)
 *   nvamd_fp8_block_gemm  <- fp8_block_gemm_kernel[grid]     nanovllm/kernels/fp8_linear.py:130-138
 *                            (kernel fp8_linear.py:34-71)
 *
 * Conventions are those of nvamd_fp8_attention.h: device pointers, work
 * enqueued on `stream` (no allocation, no synchronisation, capturable into a
 * HIP graph), NVAMD_OK or an NVAMD_ERR_* code with nvamd_last_error().
 * Weights use the compressed-tensors FP8_BLOCK layout of the reference:
 * E4M3FN [N, K] with one bf16 scale per 128 x 128 block, [N/128, K/128].
 */
#ifndef NVAMD_FP8_LINEAR_H_
#define NVAMD_FP8_LINEAR_H_

#include <stdint.h>

#include "nvamd_fp8_attention.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Per-token, per-128-column dynamic quantisation of the activations.
 * Replaces fp8_dyn_quant_kernel (nanovllm/kernels/fp8_linear.py:11-31).
 *
 * x: [M, K] of x_dtype (NVAMD_DTYPE_BF16 or NVAMD_DTYPE_F16), row stride
 *   x_stride0 elements (a multiple of 8), 16-byte aligned; K % 128 == 0.
 * xq: E4M3FN [M, K] contiguous, 8-byte aligned.
 * x_scale: bf16 [M, K/128] contiguous.
 * For each token m and group g: scale = max|x[m, 128g : 128g + 128]| / 448
 * (IEEE fp32 division; 1 when not > 0), xq = E4M3FN(clamp(x / scale, +-448))
 * (IEEE division, round to nearest even), x_scale = bf16(scale) (RNE).
 */
int32_t nvamd_fp8_act_quant(const void* x, int64_t x_stride0, int32_t x_dtype, void* xq, void* x_scale,
                            int64_t M, int64_t K, void* stream);

/*
 * Block-scaled FP8 GEMM, out = (xq . x_scale) x (weight . weight_scale)^T.
 * Replaces fp8_block_gemm_kernel (nanovllm/kernels/fp8_linear.py:34-71).
 *
 * xq: E4M3FN [M, K] contiguous; x_scale: bf16 [M, K/128] contiguous (as
 *   written by nvamd_fp8_act_quant).
 * weight: E4M3FN [N, K], row stride weight_stride0 bytes (a multiple of 16);
 *   weight_scale: bf16 [N/128, K/128] contiguous.  N % 128 == 0, K % 128 == 0.
 * out: [M, N] of out_dtype, row stride out_stride0 elements (a multiple of 4).
 * out[m, n] = sum over 128-wide K blocks kc of P[m, n, kc] * (x_scale[m, kc] *
 *   weight_scale[n/128, kc]), P the fp32 dot product of the block, fp32
 *   accumulation, rounded to out_dtype (RNE).
 * Pointers 16-byte aligned (out 8).  K is limited by the LDS that holds a
 * tile's scales: NVAMD_ERR_UNSUPPORTED beyond it (K <= 32768 always fits).
 *
 * workspace (16-byte aligned, contents ignored; NULL with workspace_bytes 0
 * allowed): M <= 256 tokens take a kernel that streams each weight row once
 * and may split K over workgroups; it then writes fp32 partial sums there and
 * adds them in split order (repeated calls are bit-identical).  With less
 * than nvamd_fp8_block_gemm_workspace_bytes(M, N, K) bytes, K is split only
 * as far as the workspace holds.  The reference's launch has no workspace: its
 * grid tiles (M, N) only (fp8_linear.py:125-138).
 */
int32_t nvamd_fp8_block_gemm(const void* xq, const void* x_scale, const void* weight, int64_t weight_stride0,
                             const void* weight_scale, void* out, int64_t out_stride0, int32_t out_dtype, int64_t M,
                             int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes nvamd_fp8_block_gemm uses for an M x N x K product on the
 * current device (0: none). */
int64_t nvamd_fp8_block_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);

#ifdef __cplusplus
}
#endif

#endif /* NVAMD_FP8_LINEAR_H_ */
