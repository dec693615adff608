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
// Lane l of a 64-partition chunk holds partition l's (m, l) and its weight;
// each lane holds two output dims.  The partial accumulators are loaded eight
// partitions at a time, all issued before any is used (indices clamped to the
// last partition, weights zero past it), so a merge of up to eight
// partitions is one memory round trip after the (m, l) loads, not one per
// partition.
__device__ __forceinline__ void merge_partitions(const MqParams& p, int64_t rh, int Lk, int lane) {
  Lk = min(Lk, key_capacity(p));
  if (Lk <= 0) return;
  const int n_parts = (Lk + p.part_tokens - 1) / p.part_tokens;
  if (n_parts <= 1) return;

  const float* ml = p.part_ml + 2 * rh * p.max_parts;
  const float* pa = p.part_acc + rh * p.max_parts * kHeadDim + 2 * lane;
  float M = -INFINITY;
  for (int c = 0; c < n_parts; c += 64) {
    const int qn = min(64, n_parts - c);
    const float m = ml[2 * (c + min(lane, qn - 1))];
    M = fmaxf(M, lane < qn ? m : -INFINITY);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, shfl_xor_f32(M, off));
  const float Ms = (M == -INFINITY) ? 0.f : M;

  float L = 0.f, o0 = 0.f, o1 = 0.f;
  for (int c = 0; c < n_parts; c += 64) {
    const int qn = min(64, n_parts - c);
    const f32x2 v = *reinterpret_cast<const f32x2*>(ml + 2 * (c + min(lane, qn - 1)));
    const float w = (lane < qn) ? fast_exp2(v.x - Ms) : 0.f;
    L += (lane < qn) ? v.y * w : 0.f;
    for (int q0 = 0; q0 < qn; q0 += 8) {
      f32x2 a[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        a[j] = *reinterpret_cast<const f32x2*>(pa + (int64_t)(c + min(q0 + j, qn - 1)) * kHeadDim);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float wj = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), min(q0 + j, 63)));
        const float wk = (q0 + j < qn) ? wj : 0.f;
        o0 += wk * a[j].x;
        o1 += wk * a[j].y;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) L += shfl_xor_f32(L, off);
  const float inv = (L > 0.f) ? 1.0f / L : 0.f;
  const uint32_t w = out_round_bf16_bits(o0 * inv) | (out_round_bf16_bits(o1 * inv) << 16);
  *reinterpret_cast<uint32_t*>(p.out + rh * kHeadDim + 2 * lane) = w;
}

// Varlen mode: merges of sequence `seq` (only short-query sequences, the
// ones the split-KV kernel served, have partitions), one (row, head) per
// wave: this wave merges index `idx` of the sequence's Lq * Hq (row, head)
// pairs.  Launches give every pair a wave of its own, since a merge is a
// chain of dependent memory round trips.
__device__ __forceinline__ void merge_varlen_one(const MqParams& p, int seq, int idx, int lane) {
  const int row0 = p.cu_q[seq];
  const int Lq = p.cu_q[seq + 1] - row0;
  if (Lq <= 0 || Lq > p.mq_max_q || idx >= Lq * p.Hq) return;
  const int64_t row = (int64_t)row0 + idx / p.Hq;
  if (row >= p.q_rows) return;
  merge_partitions(p, row * p.Hq + idx % p.Hq, p.cu_k[seq + 1] - p.cu_k[seq], lane);
}

// Slices of `n_waves` (row, head) pairs per sequence: workgroups a varlen
// merge launch needs per sequence.
__host__ __device__ __forceinline__ int merge_slices(const MqParams& p, int n_waves) {
  return (p.mq_max_q * p.Hq + n_waves - 1) / n_waves;
}

}  // namespace nvamd
