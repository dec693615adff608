// Work items of the varlen prefill kernel and the device pass that orders
// them (shared by the prefill kernel and the short-query launch that writes
// the work list before it).
#pragma once

#include "fp8_common.h"
#include "kernels.h"

namespace nvamd {

constexpr int kPrefillTile = 64;     // kv tokens per prefill tile
constexpr int kCostBuckets = 1024;   // schedule sort resolution (tiles)

struct ItemGeom {
  int q_start, Lq, k_start, Lk, c;
};

// One entry of the prefill work list: a (sequence, m-block) item with its
// geometry resolved, so that a workgroup needs a single load to start it.
// seq < 0 marks a slot past the last item.
// head = {seq, mb, q_start, Lq}, tail = {k_start, Lk, n_tiles, 0}.
struct PrefillItem {
  int4 head, tail;
};

__device__ __forceinline__ ItemGeom item_geom(const PrefillParams& p, int seq) {
  ItemGeom g;
  g.q_start = p.cu_q[seq];
  g.Lq = p.cu_q[seq + 1] - g.q_start;
  g.k_start = p.cu_k[seq];
  g.Lk = p.cu_k[seq + 1] - g.k_start;
  g.c = g.Lk - g.Lq;
  return g;
}

// KV tiles item (seq, mb) visits: keys visible to the block's last row,
// bounded by the block table.
__device__ __forceinline__ int item_tiles(const PrefillParams& p, const ItemGeom& g, int mb) {
  int kv_hi = min(g.Lk, g.c + mb * p.BM + p.BM);
  if (p.block_tables != nullptr) kv_hi = (int)min((int64_t)kv_hi, p.bt_stride * (int64_t)p.block_size);
  return max(0, (kv_hi + kPrefillTile - 1) / kPrefillTile);
}

__device__ __forceinline__ bool item_valid(const PrefillParams& p, const ItemGeom& g, int mb) {
  return g.Lq > p.mq_max_q && mb * p.BM < g.Lq;
}

// Work list of the prefill kernel: one workgroup (256 threads or more; the
// first 256 do the work, the rest only take part in the barriers) writes the
// (seq, m-block) items in decreasing tile count (counting sort), followed by
// records with seq = -1 for slots without an item.  Run as an extra
// workgroup of the launch that precedes the prefill kernel.
__device__ __forceinline__ void prefill_schedule(const PrefillParams& p, PrefillItem* __restrict__ items,
                                                 int n_items_max) {
  __shared__ int hist[kCostBuckets];
  __shared__ int warp_tot[4];
  const int tid = threadIdx.x;
  const bool worker = tid < 256;
  const int lane = tid & 63, wave = tid >> 6;
  if (worker)
    for (int b = tid; b < kCostBuckets; b += 256) hist[b] = 0;
  __syncthreads();
  if (worker)
    for (int idx = tid; idx < n_items_max; idx += 256) {
      const int seq = idx / p.n_mblocks, mb = idx - seq * p.n_mblocks;
      const ItemGeom g = item_geom(p, seq);
      if (!item_valid(p, g, mb)) continue;
      atomicAdd(&hist[min(item_tiles(p, g, mb), kCostBuckets - 1)], 1);
    }
  __syncthreads();
  // Exclusive scan in decreasing cost order: thread t owns buckets
  // [1023 - 4t - 3, 1023 - 4t] (walked from high cost to low).
  int local[4] = {0, 0, 0, 0}, sum = 0, incl = 0;
  if (worker) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      local[j] = hist[kCostBuckets - 1 - (4 * tid + j)];
      sum += local[j];
    }
    incl = sum;  // inclusive scan of per-thread sums over the wave
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    if (lane == 63) warp_tot[wave] = incl;
  }
  __syncthreads();
  int total = 0, run = 0;
  if (worker) {
    int base = 0;
    for (int w = 0; w < wave; ++w) base += warp_tot[w];
    total = warp_tot[0] + warp_tot[1] + warp_tot[2] + warp_tot[3];
    run = base + incl - sum;
  }
  __syncthreads();
  if (worker) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      hist[kCostBuckets - 1 - (4 * tid + j)] = run;
      run += local[j];
    }
  }
  __syncthreads();
  if (!worker) return;
  for (int idx = tid; idx < n_items_max; idx += 256) {
    const int seq = idx / p.n_mblocks, mb = idx - seq * p.n_mblocks;
    const ItemGeom g = item_geom(p, seq);
    if (!item_valid(p, g, mb)) continue;
    const int tiles = item_tiles(p, g, mb);
    const int pos = atomicAdd(&hist[min(tiles, kCostBuckets - 1)], 1);
    items[pos] = PrefillItem{make_int4(seq, mb, g.q_start, g.Lq), make_int4(g.k_start, g.Lk, tiles, 0)};
  }
  for (int pos = total + tid; pos < n_items_max; pos += 256)
    items[pos] = PrefillItem{make_int4(-1, 0, 0, 0), make_int4(0, 0, 0, 0)};
}

}  // namespace nvamd
