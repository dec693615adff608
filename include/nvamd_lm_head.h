/*
 * C ABI of the MI355X (gfx950) LM-head row selection and sampler.
 *
 * These entry points replace the step after the attention path in nano-vLLM:
 *
 *   nvamd_select_logit_rows <- the row selection of ParallelLMHead.forward
 *                              nanovllm/layers/embed_head.py:56-72 (index_select of the kept rows)
 *   nvamd_sample            <- Sampler.forward           nanovllm/layers/sampler.py:7-12
 *
 * Conventions are those of nvamd_fp8_attention.h: device pointers, work
 * enqueued on `stream` (no allocation, no synchronisation), NVAMD_OK or an
 * NVAMD_ERR_* code with nvamd_last_error().
 */
#ifndef NVAMD_LM_HEAD_H_
#define NVAMD_LM_HEAD_H_

#include <stdint.h>

#include "nvamd_fp8_attention.h"

#ifdef __cplusplus
extern "C" {
#endif

#define NVAMD_LOGITS_BF16 0
#define NVAMD_LOGITS_F16 1
#define NVAMD_LOGITS_F32 2

/*
 * Rows of the hidden states that the LM head needs (embed_head.py:56-72).
 * x: [x_rows, hidden] of elem_bytes-wide elements, row stride x_stride0
 *   elements: the num_plain plain-decode rows, then the varlen rows (the
 *   num_spec_seqs speculative sequences' rows first, then one or more rows
 *   per prefill sequence).
 * cu_seqlens_q: int32 [num_spec_seqs + num_prefill_seqs + 1] of the varlen
 *   sequences; num_spec_rows = cu_seqlens_q[num_spec_seqs] (the caller knows
 *   it from scheduling; passing it avoids reading it back from the GPU).
 * out: [num_plain + num_spec_rows + num_prefill_seqs, hidden], row stride
 *   out_stride0 elements: rows 0 .. num_plain + num_spec_rows - 1 of x, then
 *   the last row of each prefill sequence, num_plain +
 *   cu_seqlens_q[num_spec_seqs + 1 + i] - 1.
 * hidden * elem_bytes must be a multiple of 16 and the row starts 16-byte
 * aligned.
 */
int32_t nvamd_select_logit_rows(const void* x, int64_t x_stride0, int64_t x_rows, int32_t hidden, int32_t elem_bytes,
                                const int32_t* cu_seqlens_q, int32_t num_plain, int32_t num_spec_seqs,
                                int32_t num_spec_rows, int32_t num_prefill_seqs, void* out, int64_t out_stride0,
                                void* stream);

/* Workspace needed by nvamd_sample for `rows` rows of `vocab` logits
 * (partial results of the workgroups that share a row; no initialisation
 * needed). */
int64_t nvamd_sample_workspace_bytes(int64_t rows, int64_t vocab);

/*
 * Temperature sampling (sampler.py:7-12): for each row r, y = logits[r] /
 * temperatures[r], p = softmax(y), token = argmax_v p_v / max(E_v, 1e-10)
 * (the first index on ties), E ~ Exp(1).  Computed as the equal argmax of
 * logits[r][v] log2(e) / temperatures[r] - log2(max(E_v, 1e-10)) (the
 * softmax's max and sum do not depend on v), so two candidates whose scores
 * agree to a few ulps may be ordered differently from an fp32 softmax.  With
 * noise != NULL, E is read from it (fp32 [rows, vocab], row stride vocab).
 * Otherwise the noise is drawn in the kernel from Philox4x32-10 with key
 * (seed mod 2^32, seed >> 32), each draw x giving E = -ln(((x >> 8) + 1)
 * 2^-24), top down by groups of 16 tokens (an exact reformulation of one
 * Exp(1) per token, by the Gumbel-max property; the token distribution is
 * softmax(logits / T) either way): group g = tokens [16g, 16g + 16) draws its
 * maximum score M_g = log2(sum_v 2^(c z_v)) - log2(max(E_g, 1e-10)), c =
 * log2(e) / T, with E_g from counter (2^31 + 64 (g / 256) + g % 64, r, offset
 * mod 2^32, offset >> 32) word (g / 64) % 4; the first group with the largest
 * M_g wins, and in it the first token with the largest c z_v - log2(max(E_v,
 * 1e-10)), E_v from counter (v / 4, r, offset mod 2^32, offset >> 32) word
 * v % 4.  logits: [rows, vocab] of logits_dtype (NVAMD_LOGITS_*), row stride
 * stride0 elements; temperatures: fp32 [rows], > 0; out: int64 [rows];
 * workspace: 16-byte aligned, nvamd_sample_workspace_bytes(rows, vocab)
 * bytes.  vocab < 2^31 - 4098 (NVAMD_ERR_UNSUPPORTED beyond).
 */
int32_t nvamd_sample(const void* logits, int32_t logits_dtype, int64_t stride0, int64_t rows, int64_t vocab,
                     const float* temperatures, const float* noise, uint64_t seed, uint64_t offset, int64_t* out,
                     void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NVAMD_LM_HEAD_H_ */
