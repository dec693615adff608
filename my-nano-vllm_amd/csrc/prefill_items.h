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

// One entry of the prefill work list: a piece of a (sequence, m-block)
// item, its geometry resolved so that a workgroup needs a single load to
// start it.  seq < 0 marks a slot past the last piece.
// head = {seq, mb, q_start, Lq}, tail = {k_start, Lk, t_lo, t_hi}: tiles
// [t_lo, t_hi) of the item; split = {piece, pieces, slot, counter}: piece
// `piece` of `pieces` (1: the whole item), the partial slot of its piece 0
// (its piece j writes slot + j) and its arrival counter.
struct PrefillItem {
  int4 head, tail, split;
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

// Host-side check of the work-list geometry a schedule pass writes.
inline bool schedule_params_ok(const PrefillParams& p) {
  const int64_t n_items_max = (int64_t)p.num_seqs * p.n_mblocks;
  return n_items_max <= 0x7fffffff && p.n_records >= n_items_max && p.n_records >= 2 * p.slots_per_group &&
         p.slots_per_group >= 1 && p.counters != nullptr && p.part != nullptr;
}

// Pieces item of n tiles is split into when its call splits (piece_tiles
// > 0): about n / piece_tiles, at least 2 tiles each, at most
// kPrefillMaxPieces.
__device__ __forceinline__ int item_pieces(int n, int piece_tiles) {
  if (piece_tiles <= 0 || n < 4) return 1;
  return max(1, min(min((n + piece_tiles - 1) / piece_tiles, n / 2), kPrefillMaxPieces));
}

// Tiles [lo, hi) of piece j of k over n tiles (sizes differ by at most 1).
__device__ __forceinline__ int piece_lo(int n, int k, int j) { return j * n / k; }

// Inclusive scans of N values over the 256 worker threads (4 waves; waves
// past them get the workers' totals as their base), with one barrier: the
// wave totals alternate between two halves of warp_tot (2 x 4 x N ints), so
// a scan's totals are not overwritten before every wave has read them (the
// scan two calls later writes them again only after the barrier of the scan
// between, which every wave reaches after its reads).  `parity` is the
// caller's alternation state, the same in every thread.
constexpr int kScanMaxValues = 4;
template <int N>
__device__ __forceinline__ void block_incl_scan_n(int (&x)[N], int* warp_tot, int& parity, int (&total)[N]) {
  static_assert(N <= kScanMaxValues, "warp_tot holds kScanMaxValues values per wave");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int incl[N];
#pragma unroll
  for (int i = 0; i < N; ++i) incl[i] = wave_incl_scan(x[i]);
  int* buf = warp_tot + 4 * kScanMaxValues * parity;
  parity ^= 1;
  if (tid < 256 && lane == 63) {
#pragma unroll
    for (int i = 0; i < N; ++i) buf[4 * i + wave] = incl[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    int base = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (w < wave) base += buf[4 * i + w];
    total[i] = buf[4 * i] + buf[4 * i + 1] + buf[4 * i + 2] + buf[4 * i + 3];
    x[i] = base + incl[i];
  }
}

__device__ __forceinline__ int2 block_incl_scan2(int2 x, int* warp_tot, int& parity, int2& total) {
  int v[2] = {x.x, x.y}, t[2];
  block_incl_scan_n(v, warp_tot, parity, t);
  total = make_int2(t[0], t[1]);
  return make_int2(v[0], v[1]);
}

__device__ __forceinline__ int block_incl_scan(int x, int* warp_tot, int& parity, int& total) {
  int2 t;
  const int2 r = block_incl_scan2(make_int2(x, 0), warp_tot, parity, t);
  total = t.x;
  return r.x;
}

// Work list of the prefill kernel, written by one workgroup (256 threads or
// more; the first 256 do the work, the rest only take part in the
// barriers) run as an extra workgroup of the launch that precedes the
// prefill kernel.
//
// Items are the valid (sequence, m-block) pairs.  When there are fewer
// than a round of workgroups' worth of them (V < slots_per_group per
// kv-head group), long items are split into pieces of about T / slots_per_group
// tiles (T = all items' tiles), lengthened until the pieces fit one round,
// so the pieces fill the machine and the longest one is short; a split
// item gets consecutive partial slots and an arrival counter (zeroed here,
// so the prefill kernel, the next launch, starts from zero).  The pieces
// are written in decreasing tile count (counting sort), followed by records
// with seq = -1 up to n_records.  Each thread keeps the geometry of its
// first kSchedCached candidates in registers, so the passes over the items
// read the sequence lengths from memory once.  `lds` is the caller's LDS,
// at least kScheduleLdsInts ints (the workgroup that runs the schedule uses
// no other LDS, so the caller lends it its own buffer).
constexpr int kSchedCached = 4;
constexpr int kScheduleLdsInts = kCostBuckets + 8 * kScanMaxValues;

__device__ __forceinline__ void prefill_schedule(const PrefillParams& p, PrefillItem* __restrict__ items, int* lds) {
  int* hist = lds;                    // [kCostBuckets]
  int* warp_tot = lds + kCostBuckets;  // [8 * kScanMaxValues]
  int parity = 0;                      // block_incl_scan2's alternation
  const int tid = threadIdx.x;
  const bool worker = tid < 256;
  const int n_items_max = p.num_seqs * p.n_mblocks;
  const int n_groups = p.Hkv * p.n_hgroups;
  if (worker) {
    for (int b = tid; b < kCostBuckets; b += 256) hist[b] = 0;
    for (int c = tid; c <= p.slots_per_group * n_groups; c += 256) p.counters[c] = 0;  // + the claim counter
  }
  // candidate idx: its geometry and tile count (-1: not a valid item)
  auto candidate = [&](int idx, ItemGeom& g) {
    const int seq = idx / p.n_mblocks, mb = idx - seq * p.n_mblocks;
    g = item_geom(p, seq);
    return item_valid(p, g, mb) ? item_tiles(p, g, mb) : -1;
  };
  ItemGeom cg[kSchedCached];
  int ct[kSchedCached];
#pragma unroll
  for (int i = 0; i < kSchedCached; ++i) {
    const int idx = tid + 256 * i;
    cg[i] = ItemGeom{};
    ct[i] = (worker && idx < n_items_max) ? candidate(idx, cg[i]) : -1;
  }
  // f(tiles, geometry, idx) for this thread's valid candidates: the cached
  // ones (static indices, so they stay in registers), then the rest
  auto each_item = [&](auto&& f) {
    if (!worker) return;
#pragma unroll
    for (int i = 0; i < kSchedCached; ++i)
      if (ct[i] >= 0) f(ct[i], cg[i], tid + 256 * i);
    for (int idx = tid + 256 * kSchedCached; idx < n_items_max; idx += 256) {
      ItemGeom g;
      const int n = candidate(idx, g);
      if (n >= 0) f(n, g, idx);
    }
  };
  // valid items and their tiles
  int v = 0, tt = 0;
  each_item([&](int n, const ItemGeom&, int) {
    ++v;
    tt += n;
  });
  int2 vt;
  block_incl_scan2(make_int2(v, tt), warp_tot, parity, vt);
  const int n_valid = vt.x, n_tiles_all = vt.y;
  const bool split = n_valid > 0 && n_valid < p.slots_per_group;
  // piece length: from T / slots_per_group up (by a quarter, at least 1 tile,
  // at most 16 times), until the pieces fit one round; four lengths are
  // counted per scan
  int piece_tiles = split ? max(2, (n_tiles_all + p.slots_per_group - 1) / p.slots_per_group) : 0;
  for (int iter = 0; split && iter < 16; iter += 4) {
    int cand[4], np[4] = {0, 0, 0, 0}, tot[4];
    cand[0] = piece_tiles;
#pragma unroll
    for (int i = 1; i < 4; ++i) cand[i] = cand[i - 1] + max(1, cand[i - 1] / 4);
    each_item([&](int n, const ItemGeom&, int) {
#pragma unroll
      for (int i = 0; i < 4; ++i) np[i] += item_pieces(n, cand[i]);
    });
    block_incl_scan_n(np, warp_tot, parity, tot);
    int fit = 4;
#pragma unroll
    for (int i = 3; i >= 0; --i)
      if (tot[i] <= p.slots_per_group) fit = i;
    if (fit < 4) {
      piece_tiles = cand[fit];
      break;
    }
    piece_tiles = cand[3] + max(1, cand[3] / 4);
  }
  // histogram of piece sizes
  each_item([&](int n, const ItemGeom&, int) {
    const int k = item_pieces(n, piece_tiles);
    for (int j = 0; j < k; ++j)
      atomicAdd(&hist[min(piece_lo(n, k, j + 1) - piece_lo(n, k, j), kCostBuckets - 1)], 1);
  });
  __syncthreads();
  // Exclusive scan in decreasing cost order: thread t owns buckets
  // [1023 - 4t - 3, 1023 - 4t] (walked from high cost to low).
  int local[4] = {0, 0, 0, 0}, sum = 0;
  if (worker) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      local[j] = hist[kCostBuckets - 1 - (4 * tid + j)];
      sum += local[j];
    }
  }
  int total = 0;
  const int incl = block_incl_scan(sum, warp_tot, parity, total);
  if (worker) {
    int run = incl - sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      hist[kCostBuckets - 1 - (4 * tid + j)] = run;
      run += local[j];
    }
  }
  __syncthreads();
  // Scatter the pieces; split items take partial slots and counters in item
  // order (a scan over the candidates, 256 at a time: round i covers
  // candidates [256 i, 256 i + 256)).
  int slot_carry = 0, cnt_carry = 0;
  auto scatter_round = [&](int n, const ItemGeom& g, int idx) {
    const int k = n >= 0 ? item_pieces(n, piece_tiles) : 0;
    const int ks = k > 1 ? k : 0;
    int2 tot;
    const int2 inc = block_incl_scan2(make_int2(ks, ks > 0 ? 1 : 0), warp_tot, parity, tot);
    const int slot0 = slot_carry + inc.x - ks;
    const int cnt0 = cnt_carry + inc.y - (ks > 0 ? 1 : 0);
    slot_carry += tot.x;
    cnt_carry += tot.y;
    const int seq = idx / p.n_mblocks, mb = idx - seq * p.n_mblocks;
    for (int j = 0; j < k; ++j) {
      const int lo = piece_lo(n, k, j), hi = piece_lo(n, k, j + 1);
      const int pos = atomicAdd(&hist[min(hi - lo, kCostBuckets - 1)], 1);
      items[pos] = PrefillItem{make_int4(seq, mb, g.q_start, g.Lq), make_int4(g.k_start, g.Lk, lo, hi),
                               make_int4(j, k, k > 1 ? slot0 : -1, k > 1 ? cnt0 : -1)};
    }
  };
#pragma unroll
  for (int i = 0; i < kSchedCached; ++i)
    if (256 * i < n_items_max) scatter_round(worker ? ct[i] : -1, cg[i], tid + 256 * i);
  for (int base = 256 * kSchedCached; base < n_items_max; base += 256) {
    const int idx = base + tid;
    ItemGeom g{};
    const int n = (worker && idx < n_items_max) ? candidate(idx, g) : -1;
    scatter_round(n, g, idx);
  }
  if (worker)
    for (int pos = total + tid; pos < p.n_records; pos += 256)
      items[pos] = PrefillItem{make_int4(-1, 0, 0, 0), make_int4(0, 0, 0, 0), make_int4(0, 1, -1, -1)};
  // The last round of workgroups claims its units (record, group) in the
  // order the workgroups start: a workgroup goes to XCD blockIdx % 8 however
  // busy that XCD is, and the XCDs run at different rates, so the XCDs that
  // reach the last round first take its longest units.
  if (tid == 0) {
    const int round = p.slots_per_group * n_groups, units = total * n_groups;
    p.counters[round + 1] = units > round ? units - round : units;  // claim_from
    p.counters[round + 2] = units;                                   // total_units
  }
}

}  // namespace nvamd
