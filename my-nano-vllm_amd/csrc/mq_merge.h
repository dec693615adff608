// Log-sum-exp merges of split-KV partitions and of the balanced kernel's cut
// pairs (shared by the merge launches and the prefill kernel, which merges
// the short-query rows of a prefill call in extra workgroups instead of a
// launch of its own).
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
  M = wave_max_f32(M);  // DPP and row swaps: no LDS round trip
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
  L = wave_sum_f32(L);
  const float inv = (L > 0.f) ? 1.0f / L : 0.f;
  const bool f16 = p.out_f16 != 0;
  const uint32_t w = out_bits_rt(o0 * inv, f16) | (out_bits_rt(o1 * inv, f16) << 16);
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

// ---- balanced (stream-K) kernel: merge of a pair cut across workgroups ----

// Stream-K ranges of the balanced decode kernel.  Workgroup w gets a share
// of the T stages proportional to its weight: a for even w, kSkPairWeight - a
// for odd w.  Workgroups are dealt to the 8 XCDs round-robin, so even
// workgroups run on even-numbered XCDs; on MI355X those stream this kernel's
// KV bytes 5-10% faster than the odd-numbered ones when every CU is loading
// at full rate (per-workgroup wall-clock timestamps, on several boxes), and
// equal shares then leave the even XCDs idle at the end.  Decode runs at
// that rate and takes a = kSkEvenWeight; the short-query rows of a varlen
// call do not, and take equal shares.  The split is fixed, so results do
// not depend on timing.  With C(w) = the weight of workgroups 0 .. w-1,
// workgroup w owns stages [T C(w) / C(W), T C(w+1) / C(W)).
constexpr int kSkPairWeight = 64, kSkEvenWeight = 33;

__device__ __forceinline__ int sk_even_weight(const MqParams& p) {
  return p.cu_q == nullptr ? kSkEvenWeight : kSkPairWeight / 2;
}

// C(w) in the integer type U (uint32_t when T * C(W) + T < 2^32, see
// sk_fits32, else uint64_t: a 64-bit division is a long instruction
// sequence, so each caller picks the type once and does all its range
// arithmetic in it).
template <typename U>
__device__ __forceinline__ U sk_cum_weight(U w, U a) {
  return (w >> 1) * (U)kSkPairWeight + (w & 1) * a;
}

__device__ __forceinline__ bool sk_fits32(int64_t T, int W, int a) {
  return (T * (sk_cum_weight<uint64_t>((uint64_t)W, (uint64_t)a) + 1)) >> 32 == 0;
}

// First stage of workgroup w's range.
template <typename U>
__device__ __forceinline__ U sk_range_start(U w, U T, U W, U a) {
  return T * sk_cum_weight<U>(w, a) / sk_cum_weight<U>(W, a);
}

// Workgroup holding stage x (0 <= x < T): the last w with T C(w) / C(W) <= x,
// i.e. with C(w) <= ceil((x + 1) C(W) / T) - 1.
template <typename U>
__device__ __forceinline__ int sk_owner(U x, U T, U W, U a) {
  const U cmax = ((x + 1) * sk_cum_weight<U>(W, a) + T - 1) / T - 1;
  const U k = cmax / (U)kSkPairWeight, r = cmax % (U)kSkPairWeight;
  const U w = 2 * k + (r >= a ? 1 : 0);
  return (int)(w < W - 1 ? w : W - 1);
}

// Owners of a pair's first (stage P) and last (P + n - 1) stages, and
// whether the pair starts after the first owner's range does (then it is
// that workgroup's last pair: slot 1).
template <typename U>
__device__ __forceinline__ void sk_pair_owners(U P, U n, U T, U W, U a, int& wf, int& wl, int& slot_f) {
  wf = sk_owner<U>(P, T, W, a);
  wl = sk_owner<U>(P + n - 1, T, W, a);
  slot_f = sk_range_start<U>((U)wf, T, W, a) < P ? 1 : 0;
}

// Merges the partials of one (query row, head) whose pair was cut across
// workgroups, or zero-fills it when its context is empty; one wave: row
// idx / Hq of sequence b (the only row in decode), head idx % Hq.  Lane i
// reads (m, l) of the i-th contributing workgroup, the wave reduces them,
// then every lane accumulates 2 dims over the contributions.
__device__ __forceinline__ void sk_merge_one(const MqParams& p, int b, int idx, int lane) {
  if (b >= p.num_seqs || idx >= p.mq_max_q * p.Hq) return;
  const int qr = idx / p.Hq, hq = idx - qr * p.Hq;
  int64_t q0 = b;
  if (p.cu_q != nullptr) {  // varlen: short-query sequences only
    q0 = p.cu_q[b];
    const int lq = p.cu_q[b + 1] - (int)q0;
    if (lq <= 0 || lq > p.mq_max_q || qr >= lq || q0 + qr >= p.q_rows) return;
  }
  const int G = p.G, HG = p.sk_heads, NHG = p.Hkv / HG;
  const int kvh = hq / G, col = qr * G + (hq - kvh * G);
  const int hg = kvh / HG, hh = kvh - hg * HG;
  // the pair's stage count and position come from the prefix the main pass
  // wrote (loads independent of each other and of cu_q: one round trip)
  const int pre_b = p.sk_prefix[b];
  const int n = p.sk_prefix[b + 1] - pre_b;
  uint32_t* out = reinterpret_cast<uint32_t*>(p.out + ((q0 + qr) * p.Hq + hq) * kHeadDim);
  if (n == 0) {
    // Empty context (graph padding rows): the reference yields NaN here; write 0.
    out[lane] = 0u;
    return;
  }
  const int W = p.sk_wgs;
  const int64_t T = (int64_t)NHG * p.sk_prefix[p.num_seqs];
  const int64_t P = (int64_t)NHG * pre_b + (int64_t)hg * n;
  // owners of the pair's first and last stages, and wf's slot (below); in
  // 32-bit arithmetic when T * (W + 1) < 2^32 (every product below is then
  // below 2^32), since a 64-bit division is a long instruction sequence and
  // this pass runs one per wave
  const int a = sk_even_weight(p);
  int wf, wl, slot_f;
  if (sk_fits32(T, W, a)) sk_pair_owners<uint32_t>((uint32_t)P, (uint32_t)n, (uint32_t)T, (uint32_t)W, (uint32_t)a, wf, wl, slot_f);
  else sk_pair_owners<uint64_t>((uint64_t)P, (uint64_t)n, (uint64_t)T, (uint64_t)W, (uint64_t)a, wf, wl, slot_f);
  if (wf == wl) return;  // finished by its workgroup
  // Workgroups in (wf, wl] start inside the pair, so it is their first pair
  // (slot 0); wf holds it in slot 0 if its range starts at P, else in slot 1
  // (its last pair).  With T >= W no range is empty; otherwise workgroups
  // with empty ranges wrote nothing and are skipped.  (64-bit divisions are
  // long instruction sequences: one per contributor made this pass
  // instruction-bound when pairs are cut many times.)  Slot s of workgroup w
  // for (hh, col) is at base + (2w + s) * wstride.
  const bool may_be_empty = T < W;
  const float* base = p.sk_part + (int64_t)(hh * p.sk_cols + col) * kSkSlotFloats;
  const int64_t wstride = (int64_t)HG * p.sk_cols * kSkSlotFloats;
  // Contributors in chunks of 16 (one DPP row): all of a chunk's loads
  // (lane j < 16 reads (m, l) of contributor j, every lane its 2 dims of
  // each) are issued before any is used, so a chunk costs one memory round
  // trip (speculative rows' pairs have up to ~14 contributors).
  constexpr int kChunk = 16;
  float M = -INFINITY, Lsum = 0.f, o0 = 0.f, o1 = 0.f;
  for (int w0 = wf; w0 <= wl; w0 += kChunk) {
    const int cnt = min(kChunk, wl - w0 + 1);
    float mi = -INFINITY, li = 0.f;
    uint32_t skip = 0;  // bit j: contributor j has an empty range (only when T < W)
    if (may_be_empty) {
#pragma nounroll
      for (int j = 0; j < cnt; ++j)
        if (sk_range_start<uint32_t>(w0 + j, (uint32_t)T, W, a) ==  // T < W: T * C(W) < 2^32
            sk_range_start<uint32_t>(w0 + j + 1, (uint32_t)T, W, a))
          skip |= 1u << j;
    }
    uint32_t a[kChunk];  // dims 2 lane, 2 lane + 1 of contributor j's acc / l (fp16)
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      a[j] = 0u;
      if (j < cnt && !((skip >> j) & 1u)) {
        const int w = w0 + j;
        const float* ps = base + (int64_t)(2 * w + (w == wf ? slot_f : 0)) * wstride;
        a[j] = reinterpret_cast<const uint32_t*>(ps)[lane];
        if (lane == j) {
          mi = ps[kSkSlotMl];
          li = ps[kSkSlotMl + 1];
        }
      }
    }
    // lanes 0..15 hold the chunk's values (the rest -inf and 0): DPP inside
    // the first row, then lane 0's result read by every lane
    const float Mp = readlane_f32(row16_max(mi), 0);
    const float Mn = fmaxf(M, Mp);
    const float Ms = (Mn == -INFINITY) ? 0.f : Mn;
    const float sc = (M == -INFINITY) ? 0.f : fast_exp2(M - Ms);
    Lsum *= sc;
    o0 *= sc;
    o1 *= sc;
    M = Mn;
    const float wi = (mi == -INFINITY) ? 0.f : fast_exp2(mi - Ms);
    const float lw = li * wi;
    Lsum += readlane_f32(row16_sum(lw), 0);
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {  // weight of a normalised partial: w_j * l_j
      const float wk = readlane_f32(lw, j);
      const f16x2 h = __builtin_bit_cast(f16x2, a[j]);
      o0 += wk * (float)h.x;
      o1 += wk * (float)h.y;
    }
  }
  const float inv = (Lsum > 0.f) ? 1.0f / Lsum : 0.f;
  const bool f16 = p.out_f16 != 0;
  out[lane] = out_bits_rt(o0 * inv, f16) | (out_bits_rt(o1 * inv, f16) << 16);
}

// Decode (one query row per sequence) with G <= 4 query heads per kv head:
// the merge of one (sequence, kv head) by one wave, 16 lanes per query head
// (8 dims each), so a wave covers the kv head's G heads with the same two
// memory round trips (the pair's prefix, then every contributor's partial) as
// sk_merge_one takes for one head, and the launch has a quarter of the waves.
// Every lane loads each contributor's (m, l) itself (the 16 lanes of a head
// share the address), so no cross-lane exchange is needed; the contributors
// are added in workgroup order.
__device__ __forceinline__ void sk_merge_heads(const MqParams& p, int b, int kvh, int lane) {
  const int G = p.G, HG = p.sk_heads, NHG = p.Hkv / HG;
  const int sub = lane >> 4, d8 = lane & 15;  // query head kvh * G + sub, dims 8 d8 .. 8 d8 + 7
  const int hg = kvh / HG, hh = kvh - hg * HG;
  const int pre_b = p.sk_prefix[b];
  const int n = p.sk_prefix[b + 1] - pre_b;
  u32x4* out = reinterpret_cast<u32x4*>(p.out + ((int64_t)b * p.Hq + kvh * G + sub) * kHeadDim + 8 * d8);
  if (n == 0) {
    // Empty context (graph padding rows): the reference yields NaN here; write 0.
    if (sub < G) *out = u32x4{0u, 0u, 0u, 0u};
    return;
  }
  const int W = p.sk_wgs;
  const int64_t T = (int64_t)NHG * p.sk_prefix[p.num_seqs];
  const int64_t P = (int64_t)NHG * pre_b + (int64_t)hg * n;
  const int a = sk_even_weight(p);
  int wf, wl, slot_f;
  if (sk_fits32(T, W, a)) sk_pair_owners<uint32_t>((uint32_t)P, (uint32_t)n, (uint32_t)T, (uint32_t)W, (uint32_t)a, wf, wl, slot_f);
  else sk_pair_owners<uint64_t>((uint64_t)P, (uint64_t)n, (uint64_t)T, (uint64_t)W, (uint64_t)a, wf, wl, slot_f);
  if (wf == wl) return;  // finished by its workgroup
  // slot s of workgroup w for (hh, col) at base + (2w + s) * wstride (as in sk_merge_one)
  const int col = min(sub, G - 1);
  const float* base = p.sk_part + (int64_t)(hh * p.sk_cols + col) * kSkSlotFloats;
  const int64_t wstride = (int64_t)HG * p.sk_cols * kSkSlotFloats;
  const bool may_be_empty = T < W;  // then workgroups with empty ranges wrote nothing
  float M = -INFINITY, L = 0.f, o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;
  for (int w0 = wf; w0 <= wl; w0 += 8) {
    const int cnt = min(8, wl - w0 + 1);
    uint32_t use = (1u << cnt) - 1u;  // bit j: contributor w0 + j wrote a partial
    if (may_be_empty) {
#pragma nounroll
      for (int j = 0; j < cnt; ++j)
        if (sk_range_start<uint32_t>(w0 + j, (uint32_t)T, W, a) ==  // T < W: T * C(W) < 2^32
            sk_range_start<uint32_t>(w0 + j + 1, (uint32_t)T, W, a))
          use &= ~(1u << j);
    }
    u32x4 h[8];
    f32x2 ml[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // all of the chunk's loads before any is used: one round trip
      // a contributor without a partial reads wl's instead (its weight is zero
      // and the skipped slot may hold anything, NaN included)
      const int w = ((use >> j) & 1u) ? w0 + j : wl;
      const float* ps = base + (int64_t)(2 * w + (w == wf ? slot_f : 0)) * wstride;
      h[j] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(ps) + 8 * d8);
      ml[j] = *reinterpret_cast<const f32x2*>(ps + kSkSlotMl);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = ((use >> j) & 1u) ? fmaxf(mx, ml[j].x) : mx;
    const float Mn = fmaxf(M, mx);
    const float Ms = (Mn == -INFINITY) ? 0.f : Mn;
    const float sc = (M == -INFINITY) ? 0.f : fast_exp2(M - Ms);
    L *= sc;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] *= sc;
    M = Mn;
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // weight of a normalised partial: w_j * l_j
      const bool u = ((use >> j) & 1u) && ml[j].x != -INFINITY;
      const float wk = u ? fast_exp2(ml[j].x - Ms) * ml[j].y : 0.f;
      L += wk;
      const uint32_t hw[4] = {h[j].x, h[j].y, h[j].z, h[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h2 = __builtin_bit_cast(f16x2, hw[e]);
        o[2 * e] += wk * (float)h2.x;
        o[2 * e + 1] += wk * (float)h2.y;
      }
    }
  }
  if (sub >= G) return;
  const float inv = (L > 0.f) ? 1.0f / L : 0.f;
  const bool f16 = p.out_f16 != 0;
  u32x4 v;
  v.x = out_bits_rt(o[0] * inv, f16) | (out_bits_rt(o[1] * inv, f16) << 16);
  v.y = out_bits_rt(o[2] * inv, f16) | (out_bits_rt(o[3] * inv, f16) << 16);
  v.z = out_bits_rt(o[4] * inv, f16) | (out_bits_rt(o[5] * inv, f16) << 16);
  v.w = out_bits_rt(o[6] * inv, f16) | (out_bits_rt(o[7] * inv, f16) << 16);
  *out = v;
}

}  // namespace nvamd
