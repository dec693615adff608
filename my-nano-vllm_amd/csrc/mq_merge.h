// Log-sum-exp merge of split-KV partitions (shared by the short-query /
// decode passes and the prefill kernel, which merges the short-query rows of
// a prefill call in extra workgroups instead of a launch of its own).
#pragma once

#include "fp8_common.h"
#include "kernels.h"

namespace nvamd {

// Keys a sequence can address: at most max_parts partitions and, for the
// paged layout, at most the block-table width (the reference's loop bound).
__device__ __forceinline__ int key_capacity(const MqParams& p) {
  int64_t cap = (int64_t)p.max_parts * p.part_tokens;
  if (p.block_tables != nullptr) cap = min(cap, p.bt_stride * (int64_t)p.block_size);
  return (int)min(cap, (int64_t)0x7fffffff);
}

// Log-sum-exp merge of the partitions of one (query row, head) by one wave.
__device__ __forceinline__ void merge_partitions(const MqParams& p, int64_t rh, int Lk, int lane) {
  Lk = min(Lk, key_capacity(p));
  if (Lk <= 0) return;
  const int n_parts = (Lk + p.part_tokens - 1) / p.part_tokens;
  if (n_parts <= 1) return;

  const float* ml = p.part_ml + 2 * rh * p.max_parts;
  float M = -INFINITY;
  for (int q = lane; q < n_parts; q += 64) M = fmaxf(M, ml[2 * q]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, shfl_xor_f32(M, off));
  const float Ms = (M == -INFINITY) ? 0.f : M;
  float L = 0.f;
  for (int q = lane; q < n_parts; q += 64) L += ml[2 * q + 1] * fast_exp2(ml[2 * q] - Ms);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) L += shfl_xor_f32(L, off);

  const float* pa = p.part_acc + rh * p.max_parts * kHeadDim + 2 * lane;
  float o0 = 0.f, o1 = 0.f;
  for (int q = 0; q < n_parts; ++q) {
    const float w = fast_exp2(ml[2 * q] - Ms);
    const f32x2 a = *reinterpret_cast<const f32x2*>(pa + (int64_t)q * kHeadDim);
    o0 += w * a.x;
    o1 += w * a.y;
  }
  const float inv = (L > 0.f) ? 1.0f / L : 0.f;
  const uint32_t w = out_round_bf16_bits(o0 * inv) | (out_round_bf16_bits(o1 * inv) << 16);
  *reinterpret_cast<uint32_t*>(p.out + rh * kHeadDim + 2 * lane) = w;
}

// Varlen mode: the merges of sequence `seq` (only short-query sequences, the
// ones the split-KV kernel served, have partitions), by `n_waves` waves.
__device__ __forceinline__ void merge_varlen_seq(const MqParams& p, int seq, int wave, int n_waves, int lane) {
  const int row0 = p.cu_q[seq];
  const int Lq = p.cu_q[seq + 1] - row0;
  if (Lq <= 0 || Lq > p.mq_max_q) return;
  const int Lk = p.cu_k[seq + 1] - p.cu_k[seq];
  for (int idx = wave; idx < Lq * p.Hq; idx += n_waves) {
    const int64_t row = (int64_t)row0 + idx / p.Hq;
    if (row >= p.q_rows) break;
    merge_partitions(p, row * p.Hq + idx % p.Hq, Lk, lane);
  }
}

}  // namespace nvamd
