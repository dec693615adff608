// Kernel parameter blocks and launchers shared by the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nvamd {

// Paged decode / short-query attention (split-KV).
struct MqParams {
  const uint16_t* q;            // bf16 or fp16 (out_f16) [q_rows, Hq, 128]
  const uint8_t* k;             // FP8: paged [P, bs, Hkv, 128] or contiguous [Nk, Hkv, 128]
  const uint8_t* v;
  const int32_t* block_tables;  // [num_seqs, bt_stride]; nullptr = contiguous layout
  int64_t bt_stride;
  const int32_t* context_lens;  // decode mode: [num_seqs]
  const int32_t* cu_q;          // varlen mode: [num_seqs + 1] (nullptr in decode mode)
  const int32_t* cu_k;
  uint16_t* out;                // [q_rows, Hq, 128], the type of q
  float* part_acc;              // [q_rows * Hq, max_parts, 128]
  float* part_ml;               // [q_rows * Hq, max_parts, 2]
  int64_t q_rows;               // rows of q / out
  int64_t kv_rows;              // K/V token rows addressable (P*bs or Nk)
  int num_seqs;
  int Hq, Hkv, G;
  int block_size;
  int part_tokens, max_parts;
  int mq_max_q;                 // varlen mode: only sequences with 1 <= Lq <= mq_max_q
  float scale_log2;
  int out_f16;                  // q and out are fp16 (else bf16)
  // Balanced decode (stream-K over KV stages), see decode_sk_kernel.
  float* sk_part;               // [sk_wgs, 2, sk_heads, sk_cols, kSkSlotFloats] partials (see kSkSlotFloats)
  int32_t* sk_prefix;           // [num_seqs + 1] stages per kv-head group before each sequence
  int sk_wgs;                   // persistent workgroups
  int sk_heads;                 // kv heads per workgroup (4 or 8; one wave each)
  int sk_cols;                  // query columns per kv head: G (decode) or G * mq_max_q (varlen)
};

// Balanced decode: 16-token stages.
constexpr int kSkStageTokens = 16;
// A cut pair's partial per query column: acc / l as fp16[128] (a weighted
// mean of V rows, |.| <= 448, so fp16 holds it to 2^-11 relative; the
// output is rounded to fp16 anyway), then m and l as fp32, 2 pad: 68 floats.
constexpr int kSkSlotFloats = 68;
constexpr int kSkSlotMl = 64;  // float offset of (m, l) in a slot
constexpr int kSkMaxSeqs = 6136;    // the stage prefix and lengths (2 * num_seqs + 1 ints) fit the 48 KiB LDS ring

// Waves per prefill workgroup: each owns 32 query rows of one head.
constexpr int kPrefillWaves = 8;

// Varlen causal prefill (long query blocks).
struct PrefillParams {
  const uint16_t* q;
  const uint8_t* k;
  const uint8_t* v;
  const int32_t* block_tables;
  int64_t bt_stride;
  const int32_t* cu_q;
  const int32_t* cu_k;
  uint16_t* out;
  int64_t q_rows;
  int64_t kv_rows;
  int num_seqs;
  int Hq, Hkv, G;
  int GW;         // query heads per workgroup
  int BM;         // query tokens per workgroup (32 * kPrefillWaves / GW)
  int n_hgroups;  // G / GW
  int n_mblocks;  // ceil(max_seqlen_q / BM)
  int block_size;      // a multiple of 16 (paged layout)
  uint32_t blk_magic;  // ceil(2^31 / (block_size / 16)): block of key kv = umulhi(2 * (kv >> 4), blk_magic)
  int mq_max_q;   // sequences with Lq <= mq_max_q are left to the short-query kernel
  float scale_log2;
  int out_f16;    // q and out are fp16 (else bf16)
  // Work list and split key ranges (see prefill_schedule): a call with fewer
  // items than a round of workgroups splits its long items' tiles into
  // pieces whose partial results the item's last piece merges.
  int n_records;        // work-list records: max(num_seqs * n_mblocks, 2 * slots_per_group)
  int slots_per_group;  // workgroups a kv-head group gets in one round: CUs / (Hkv * n_hgroups), >= 1
  int* counters;        // [slots_per_group][Hkv * n_hgroups] arrivals per split item and group, then the
                        // last round's claim counter and {claim_from, total_units} (see prefill_schedule)
  uint32_t* part;       // [2 * slots_per_group][Hkv * n_hgroups][kPrefillPartDwords][64 * kPrefillWaves]
};

// Partial result of one lane of a piece of a split item: its 64 accumulators
// normalised and rounded to fp16 (32 dwords), then m and l.
constexpr int kPrefillPartDwords = 34;
// Most pieces one item is split into.
constexpr int kPrefillMaxPieces = 8;

// Fused q/k RMSNorm + rotary embedding + FP8 KV store (qk_norm_rope.hip).
struct QkNormRopeParams {
  const uint16_t* qkv;        // bf16 [num_tokens, (Hq + 2 Hkv) * 128], row stride qkv_stride elements
  int64_t qkv_stride;
  const int64_t* positions;   // [num_tokens]
  const uint16_t* q_weight;   // bf16 [128]
  const uint16_t* k_weight;   // bf16 [128]
  const float* cos_sin;       // fp32 [max_position, 128]: cos of the 64 frequencies, then sin
  int64_t max_position;
  const int32_t* slot_mapping;  // [num_tokens]; -1 stores nothing
  uint8_t* k_cache;           // E4M3FN [num_slots, Hkv * 128]
  uint8_t* v_cache;
  int64_t num_slots;
  uint16_t* q_out;            // bf16 [num_tokens, Hq, 128]
  uint16_t* k_out;            // bf16 [num_tokens, Hkv, 128] or nullptr
  int64_t num_tokens;
  int Hq, Hkv;
  float eps;
};

hipError_t launch_qk_norm_rope_store(const QkNormRopeParams& p, hipStream_t stream);

// On-device attention metadata (see attn_metadata.hip).
constexpr int kMetaMaxSeqs = 2048;
struct AttnMetaParams {
  const int32_t* packed;  // int32 [num_seqs, 4] descriptors, then the block tables back to back
  int64_t packed_ints;    // int32 entries in packed
  int num_seqs, num_plain, block_size, max_table_len;
  int64_t cap_tokens, cap_slots, cap_rows;  // output sizes (writes beyond them are dropped)
  int64_t* positions;
  int32_t* slot_mapping;
  int32_t* context_lens;
  int32_t* cu_seqlens_q;
  int32_t* cu_seqlens_k;
  int32_t* block_tables;
};
hipError_t launch_build_metadata(const AttnMetaParams& p, int64_t units, hipStream_t stream);

// LM-head row selection and the sampler (see lm_head.hip).
hipError_t launch_select_rows(const void* x, int64_t x_stride_bytes, int64_t x_rows, int row_bytes,
                              const int32_t* cu_seqlens_q, int split_pt, int num_spec_rows, int num_spec_seqs,
                              int64_t out_rows, void* out, int64_t out_stride_bytes, hipStream_t stream);
// sampling with the caller's noise matrix (parts workgroups per row) ...
hipError_t launch_sample_noise(const void* logits, int dtype, int64_t stride, int64_t rows, int64_t vocab,
                               const float* temperatures, const float* noise, int64_t* out, float* part_score,
                               int64_t* part_index, int parts, hipStream_t stream);
// ... or with in-kernel noise, drawn top down by groups of 16 tokens (one
// task per 4,096-token quad of a row: sample_quads(vocab) per row)
int sample_quads(int64_t vocab);
hipError_t launch_sample_group(const void* logits, int dtype, int64_t stride, int64_t rows, int64_t vocab,
                               const float* temperatures, uint64_t seed, uint64_t offset, int64_t* out,
                               float* task_score, int* task_group, hipStream_t stream);

// FP8 block-scaled linear (128 x 128 weight blocks, 128-wide activation groups).
struct Fp8GemmParams {
  const uint8_t* xq;        // E4M3FN [M, K], row stride K
  const uint16_t* x_scale;  // bf16 [M, K / 128]
  const uint8_t* w;         // E4M3FN [N, K], row stride w_stride (bytes)
  const uint16_t* w_scale;  // bf16 [N / 128, K / 128]
  uint16_t* out;            // bf16 or fp16 [M, N], row stride out_stride (elements)
  int64_t w_stride, out_stride;
  int64_t M;
  int N, K, Kc;
};

hipError_t launch_fp8_act_quant(const void* x, int64_t x_stride, bool f16_in, void* xq, void* x_scale, int64_t M,
                                int64_t K, hipStream_t stream);
// Tile configuration for an M x N x K GEMM on `cus` CUs (-1: none fits lds_limit).
int fp8_gemm_pick_config(int64_t M, int64_t N, int Kc, int cus, int64_t lds_limit);
int64_t fp8_gemm_lds_bytes(int config, int Kc);
hipError_t launch_fp8_block_gemm(const Fp8GemmParams& p, int config, bool f16_out, hipStream_t stream);
// Small-M GEMM (M <= kSkinnyMaxM): cw compute waves of 16 features, mf
// 16-token fragments, K split into `splits` ranges of kper blocks (cw == 0:
// no plan; splits > 1 needs splits * M * N fp32 partials).
constexpr int64_t kSkinnyMaxM = 256;
struct SkinnyPlan {
  int cw = 0, mf = 0, splits = 1, kper = 0;
};
SkinnyPlan fp8_skinny_plan(int64_t M, int64_t N, int Kc, int cus, int64_t workspace_bytes, int64_t lds_limit);
int64_t fp8_skinny_workspace_bytes(int64_t M, int64_t N, int Kc, int cus, int64_t lds_limit);
hipError_t launch_fp8_skinny_gemm(const Fp8GemmParams& p, const SkinnyPlan& plan, bool f16_out, float* part,
                                  hipStream_t stream);

hipError_t launch_kv_store(const void* key, int64_t key_stride, const void* value,
                           int64_t value_stride, void* k_cache, void* v_cache,
                           const int32_t* slot_mapping, int64_t num_tokens, int row_elems,
                           int64_t num_slots, bool vec, bool f16, hipStream_t stream);

hipError_t launch_paged_mq(const MqParams& p, int ncb, hipStream_t stream);
// Persistent workgroups the balanced decode kernel keeps resident per CU.
int decode_sk_wgs_per_cu(int ncb, int hg, int G, bool varlen);
// pp/items: a prefill call's work list, written by one more workgroup (nullptr: none)
hipError_t launch_decode_sk(const MqParams& p, int ncb, bool merge, const PrefillParams* pp, void* items,
                            hipStream_t stream);


// Short-query (split-KV) pass of a prefill call whose extra workgroup writes
// the prefill work list to `items` (prefill_schedule_bytes(pp) bytes).
hipError_t launch_prefill_short(const MqParams& p, int ncb, const PrefillParams& pp, void* items, hipStream_t stream);

// The prefill kernel over the work list `schedule` (one workgroup per work
// unit); with `merge`, extra workgroups also merge the short-query pass's
// partitions (mq).
hipError_t launch_varlen_prefill(const PrefillParams& p, const void* schedule, const MqParams& mq, bool merge,
                                 hipStream_t stream);

}  // namespace nvamd
