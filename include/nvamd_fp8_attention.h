/*
 * C ABI of the MI355X (gfx950) FP8 paged-attention kernels.
 *
 * These entry points replace the three Triton launches of nano-vLLM's FP8
 * attention path; the Python functions that wrap them keep the reference's
 * names and signatures:
 *
 *   nvamd_store_kvcache          <- store_kvcache_kernel[(N,)]            nanovllm/layers/attention.py:40
 *                                   (wrapper store_kvcache,                nanovllm/layers/attention.py:33-40)
 *   nvamd_fp8_decode_attention   <- fp8_paged_attention_decode_kernel[grid] nanovllm/kernels/fp8_attention.py:196-206
 *                                   (wrapper fp8_decode_attention,         nanovllm/kernels/fp8_attention.py:173-207)
 *   nvamd_fp8_prefill_attention  <- fp8_paged_attention_prefill_kernel[grid] nanovllm/kernels/fp8_attention.py:341-352
 *                                   (wrapper fp8_prefill_attention,        nanovllm/kernels/fp8_attention.py:314-353)
 *   nvamd_qk_norm_rope_store     <- q_norm, k_norm, rotary_emb, store_kvcache  nanovllm/models/qwen3.py:107-110,
 *                                   nanovllm/layers/attention.py:61-62
 *   nvamd_build_attention_metadata <- ModelRunner.prepare_block_tables / prepare_prefill / prepare_decode /
 *                                   prepare_sequence               nanovllm/engine/model_runner.py:133-220
 *
 * Conventions
 *   - All pointers are device pointers (HIP), except where noted.  No call
 *     allocates memory or synchronises; every kernel is enqueued on `stream`
 *     (a hipStream_t, NULL = default stream), so the calls may be captured
 *     into a HIP graph.
 *   - bf16 / fp16 tensors are passed as raw 16-bit storage, their type named
 *     by a dtype argument (NVAMD_DTYPE_BF16 or NVAMD_DTYPE_F16; the
 *     reference's Triton kernels take the type of the tensors they are
 *     given); FP8 tensors hold OCP E4M3FN bytes (torch.float8_e4m3fn).
 *     Integer metadata is int32.
 *   - head_dim must be 128 for the attention kernels; block_size must be a
 *     positive multiple of 16 (the reference's kvcache_block_size rule,
 *     nanovllm/config.py:30).
 *   - Return value: NVAMD_OK (0) or an NVAMD_ERR_* code; nvamd_last_error()
 *     then describes the failure (thread-local, valid until the next call
 *     on the same thread).
 *   - Workspace: decode and prefill need `*_workspace_bytes()` bytes of
 *     device memory for split-KV partial results (0 when no split happens).
 *     Its contents need no initialisation and are scratch after the call.
 *     nvamd_fp8_decode_attention_noalloc uses a library-held array instead.
 */
#ifndef NVAMD_FP8_ATTENTION_H_
#define NVAMD_FP8_ATTENTION_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NVAMD_OK 0
#define NVAMD_ERR_INVALID_ARGUMENT 1
#define NVAMD_ERR_UNSUPPORTED 2
#define NVAMD_ERR_WORKSPACE 3
#define NVAMD_ERR_LAUNCH 4

/* Element types of 16-bit float tensors. */
#define NVAMD_DTYPE_BF16 0
#define NVAMD_DTYPE_F16 1

/* ABI version of this header and nvamd_fp8_linear.h (bumped on any signature change). */
#define NVAMD_ABI_VERSION 7
int32_t nvamd_abi_version(void);

/* Description of the last error on the calling thread ("" if none). */
const char* nvamd_last_error(void);

/*
 * FP8 KV-cache store / quantise.  Replaces store_kvcache_kernel
 * (nanovllm/layers/attention.py:11-31, launched at :40).
 *
 * key/value: kv_dtype (bf16 or fp16), num_tokens rows of num_kv_heads*head_dim
 *   contiguous elements (strides (key_stride0, head_dim, 1)), row stride in
 *   elements.
 * k_cache/v_cache: E4M3FN [num_slots, num_kv_heads*head_dim] contiguous
 *   (num_slots = num_blocks*block_size).
 * slot_mapping: int32[num_tokens]; -1 skips the row (attention.py:24).
 *   Slots outside [0, num_slots) are not written.
 * Rounding: nearest-even to E4M3FN, |x| > 448 saturates to +-448, NaN -> NaN.
 */
int32_t nvamd_store_kvcache(const void* key, int64_t key_stride0,
                            const void* value, int64_t value_stride0,
                            void* k_cache, void* v_cache,
                            const int32_t* slot_mapping, int64_t num_tokens,
                            int32_t num_kv_heads, int32_t head_dim, int64_t num_slots,
                            int32_t kv_dtype, void* stream);

/*
 * Fused q/k RMSNorm + rotary embedding + FP8 KV store of one attention
 * layer.  Replaces, between the QKV projection and the attention call, the
 * q_norm / k_norm RMSNorm (nanovllm/models/qwen3.py:107-109,
 * nanovllm/layers/layernorm.py:16-25), the rotary embedding (qwen3.py:110,
 * nanovllm/layers/rotary_embedding.py:40-50) and the KV store
 * (nanovllm/layers/attention.py:61-62).
 *
 * qkv: bf16 [num_tokens, (num_heads + 2 num_kv_heads) * head_dim], row
 *   stride qkv_stride0 elements (the projection output; q, k, v columns).
 * positions: int64 [num_tokens]; values outside [0, max_position) read the
 *   nearest row of the table.
 * q_norm_weight / k_norm_weight: bf16 [head_dim].
 * cos_sin_cache: fp32 [max_position, head_dim] (cos of the head_dim/2
 *   frequencies, then sin; the reference's cos_sin_cache without its unit dim).
 * q_out: bf16 [num_tokens, num_heads, head_dim] = RoPE(RMSNorm(q)).
 * k_out: bf16 [num_tokens, num_kv_heads, head_dim] = RoPE(RMSNorm(k)), or NULL.
 * k_cache / v_cache, slot_mapping, num_slots: as nvamd_store_kvcache; the
 *   cache receives E4M3FN(RoPE(RMSNorm(k))) and E4M3FN(v).  num_slots == 0
 *   (no cache allocated yet: the runner's warm-up, model_runner.py:35-36)
 *   stores nothing, and the three pointers may then be NULL.
 * head_dim must be 128; num_heads + 2 * num_kv_heads at most 128; tensors
 * 16-byte aligned (caches 8).
 */
int32_t nvamd_qk_norm_rope_store(const void* qkv, int64_t qkv_stride0, const int64_t* positions,
                                 const void* q_norm_weight, const void* k_norm_weight, float eps,
                                 const float* cos_sin_cache, int64_t max_position, void* q_out, void* k_out,
                                 void* k_cache, void* v_cache, const int32_t* slot_mapping, int64_t num_tokens,
                                 int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int64_t num_slots,
                                 void* stream);

/*
 * One engine step's attention metadata, built on the GPU.  Replaces the
 * host loops and per-tensor copies of ModelRunner.prepare_sequence
 * (nanovllm/engine/model_runner.py:203-220 with prepare_decode :188-201,
 * prepare_prefill :144-186 and prepare_block_tables :133-142).
 *
 * packed (device, 16-byte aligned, packed_ints int32 entries): num_seqs
 *   descriptors {num_tokens, num_cached_tokens, num_scheduled_tokens,
 *   table_len} in the reference's row order -- the num_plain plain decode
 *   sequences (num_scheduled_tokens == 1) first, then speculative ones, then
 *   prefill chunks -- followed by the sequences' block tables back to back.
 * Outputs, in that order of sequences:
 *   positions int64 [num_tokens]: len - 1 for plain decode rows, num_cached
 *     .. num_cached + num_scheduled - 1 for varlen rows;
 *   slot_mapping int32 [num_slots]: block_table[-1] * block_size +
 *     last_block_num_tokens - 1 for plain decode rows, block_table[p /
 *     block_size] * block_size + p % block_size for each varlen position p
 *     (none for a sequence with an empty table, as in the reference's warm-up);
 *   context_lens int32 [num_plain];
 *   cu_seqlens_q / cu_seqlens_k int32 [num_seqs - num_plain + 1] (prefix sums
 *     of num_scheduled and of num_cached + num_scheduled);
 *   block_tables int32 [num_table_rows, max_table_len]: the non-empty
 *     tables, padded with -1.
 * num_tokens, num_slots and num_table_rows are the output sizes the
 * descriptors imply (the caller computes them to allocate the outputs);
 * writes beyond them are dropped.  num_seqs <= 2048.
 */
int32_t nvamd_build_attention_metadata(const int32_t* packed, int64_t packed_ints, int32_t num_seqs,
                                       int32_t num_plain, int32_t block_size, int64_t num_tokens,
                                       int64_t num_slots, int32_t num_table_rows, int32_t max_table_len,
                                       int64_t* positions, int32_t* slot_mapping, int32_t* context_lens,
                                       int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int32_t* block_tables,
                                       void* stream);

/* Workspace needed by nvamd_fp8_decode_attention for these static shapes
 * (part_tokens = 0 selects the library's partition size). */
int64_t nvamd_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                     int32_t max_num_blocks, int32_t block_size,
                                     int32_t part_tokens);

/*
 * Paged decode, one query token per sequence.  Replaces
 * fp8_paged_attention_decode_kernel (nanovllm/kernels/fp8_attention.py:88-171,
 * launched at :196-206).
 *
 * out, q: qo_dtype (bf16 or fp16) [batch, num_heads, head_dim] contiguous (q
 *   may have more rows; only the first `batch` are used, as in the reference
 *   where batch comes from block_tables.shape[0]).  out has q's type
 *   (empty_like(q), fp8_attention.py:193).
 * k_cache/v_cache: E4M3FN [num_blocks, block_size, num_kv_heads, head_dim].
 * block_tables: int32 [batch, max_num_blocks] row-major; entries past
 *   ceil(context_lens[b]/block_size) are never read.
 * context_lens: int32 [batch].  A row with context 0 is written as zeros
 *   (the reference produces NaN there).
 * out = fp16(softmax(scale * q.K^T) . V), fp32 accumulation, stored as fp16,
 *   or for bf16 as bf16(fp16(.)) (the reference casts to fp16, :169).
 * part_tokens: split-KV partition length (multiple of 256, at most
 *   63 blocks) or 0 = automatic.
 */
int32_t nvamd_fp8_decode_attention(void* out, const void* q,
                                   const void* k_cache, const void* v_cache,
                                   const int32_t* block_tables, const int32_t* context_lens,
                                   int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_dim, int64_t num_blocks, int32_t block_size,
                                   int32_t max_num_blocks, float softmax_scale,
                                   int32_t part_tokens, void* workspace, int64_t workspace_bytes,
                                   int32_t qo_dtype, void* stream);

/*
 * Paged decode that allocates nothing and takes no workspace.  This entry
 * point has no counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture that must not
 * allocate, tight serving loops, harnesses that forbid hipMalloc).
 *
 * Same arguments, semantics and kernels as nvamd_fp8_decode_attention with
 * part_tokens = 0 (the library's partitioning), except that the scratch those
 * kernels use (the balanced kernel's stage prefix and cut-pair partials, or
 * the split-KV partials) lives in a device array the library holds on every
 * GPU it runs on, NVAMD_NOALLOC_SCRATCH_BYTES (32 MiB) per GPU until the
 * process ends.  Shapes whose workspace (nvamd_decode_workspace_bytes with
 * part_tokens = 0) exceeds it are rejected with NVAMD_ERR_WORKSPACE before
 * anything is launched.  The scratch needs no initialisation and keeps the
 * last call's contents; all calls on one GPU share it, so calls that
 * overlap on one GPU (different streams, not ordered) race.
 */
#define NVAMD_NOALLOC_SCRATCH_BYTES (32ll << 20)
int32_t nvamd_fp8_decode_attention_noalloc(void* out, const void* q,
                                           const void* k_cache, const void* v_cache,
                                           const int32_t* block_tables, const int32_t* context_lens,
                                           int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                           int32_t head_dim, int64_t num_blocks, int32_t block_size,
                                           int32_t max_num_blocks, float softmax_scale, int32_t qo_dtype,
                                           void* stream);

/* Workspace needed by nvamd_fp8_prefill_attention.  kv_cap is the static
 * upper bound of keys per sequence: max_num_blocks*block_size for the paged
 * layout, the number of K/V rows for the contiguous layout.  block_size is
 * the paged cache's block size, 0 for the contiguous layout. */
int64_t nvamd_prefill_workspace_bytes(int64_t num_tokens, int32_t num_seqs, int32_t num_heads,
                                      int32_t num_kv_heads, int64_t kv_cap,
                                      int32_t max_seqlen_q, int32_t block_size,
                                      int32_t part_tokens);

/*
 * Varlen causal prefill (chunked prefill over cached context and
 * speculative-decode verification rows).  Replaces
 * fp8_paged_attention_prefill_kernel (nanovllm/kernels/fp8_attention.py:209-312,
 * launched at :341-352).
 *
 * q, out: qo_dtype (bf16 or fp16) [num_tokens, num_heads, head_dim]
 *   contiguous; out rounded as for decode.
 * Paged layout (block_tables != NULL): k/v are E4M3FN caches
 *   [num_kv_rows/block_size, block_size, num_kv_heads, head_dim] and
 *   block_tables is int32 [num_seqs, max_num_blocks].
 * Contiguous layout (block_tables == NULL): k/v are E4M3FN
 *   [num_kv_rows, num_kv_heads, head_dim]; sequence s owns rows
 *   [cu_seqlens_k[s], cu_seqlens_k[s+1]).
 * cu_seqlens_q/k: int32 [num_seqs+1].  Query row i of sequence s attends to
 *   keys j <= i + (Lk - Lq) (bottom-right aligned causal mask).
 * max_seqlen_q bounds Lq (host value, as in the reference's grid);
 *   max_seqlen_k is accepted for signature parity and not needed.
 * Short-query sequences (Lq * num_heads/num_kv_heads <= 32, e.g. speculative
 * decode verification) run on a decode kernel: the balanced (stream-K) one
 * for the paged layout when decode would use it (part_tokens = 0,
 * num_kv_heads % 4 == 0), else the split-KV one; longer ones on the MFMA
 * prefill kernel.
 */
int32_t nvamd_fp8_prefill_attention(void* out, const void* q, const void* k, const void* v,
                                    const int32_t* block_tables,
                                    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                    int64_t num_tokens, int32_t num_seqs, int32_t num_heads,
                                    int32_t num_kv_heads, int32_t head_dim, int64_t num_kv_rows,
                                    int32_t block_size, int32_t max_num_blocks,
                                    int32_t max_seqlen_q, int32_t max_seqlen_k,
                                    float softmax_scale, int32_t part_tokens,
                                    void* workspace, int64_t workspace_bytes, int32_t qo_dtype,
                                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NVAMD_FP8_ATTENTION_H_ */
