// FP8 varlen causal (chunked) prefill for gfx950, paged and contiguous KV.
//
// Replaces fp8_paged_attention_prefill_kernel (nanovllm/kernels/fp8_attention.py:209-312).
// Sequence s owns query rows [cu_q[s], cu_q[s+1]) and Lk = cu_k[s+1]-cu_k[s]
// keys; query row i sees key j iff j <= i + (Lk - Lq) (bottom-right aligned
// causal mask, fp8_attention.py:237,267,297).  Keys come from the paged
// cache through block_tables[s], or from contiguous K/V rows
// [cu_k[s], cu_k[s+1]) when block_tables is NULL (fp8_attention.py:254-278).
//
// Work item = (sequence, m-block of BM query tokens) x (kv head, group of GW
// query heads sharing it).  A workgroup is 4 waves = 128 query rows = GW
// heads x BM tokens; wave w owns 32 rows: head (w % GW), tokens
// [m0 + 32*(w / GW), +32).  prefill_schedule_kernel first orders the items
// by decreasing number of KV tiles (a counting sort on the device), and the
// grid walks that list with the kv-head group varying fastest, so the
// longest items start first and short ones fill the tail.
//
// K/V stream in 64-token tiles.  Each thread loads its share of an FP8 tile
// into registers two tiles ahead (bounded raw buffer loads: rows past the
// sequence read as zero, so every iteration issues the same loads and the
// compiler's wait counts stay exact), converts it to bf16 (exact) and
// stages it in one of two LDS buffers -- K as [token][dim], V transposed as
// [dim][token] -- while the waves compute the other buffer.  One barrier
// per tile.  Each K load instruction fetches whole 128-byte rows (8 lanes
// per row), each V load instruction 4 whole rows.
//
// Per tile a wave computes with v_mfma_f32_32x32x16_bf16 (fp32 accumulate):
//     S^T[kv][q] = K[kv][:] . Q[q][:]          2 row blocks x 8 k-steps
//     O^T[d][q] += V^T[d][kv] . P^T[kv][q]     4 dim blocks x 4 k-steps
// Lane l (h = l / 32) holds query column l % 32; in the S^T result it holds
// kv tokens (i%4) + 8(i/4) + 4h of each 32-token row block, so the PV
// operand for k-step ks is simply p[ks/2][8(ks%2) .. +8) once V^T is stored
// with bits 2 and 3 of the token index swapped inside each 16-token step.
// The V^T rows XOR their 16-byte chunks with bits 5..6 of the dim index and
// the V staging lanes are arranged so the transposing stores, the K stores
// and the MFMA operand reads are all free of LDS bank conflicts.  The causal
// mask is applied in registers only on tiles that cross the diagonal (or
// the end of the sequence); tiles wholly above a wave's rows are skipped.
// The kernel is register-budgeted for two waves per SIMD.
#include "fp8_common.h"
#include "kernels.h"

namespace nvamd {

namespace {

constexpr int kBN = 64;                       // kv tokens per tile
constexpr int kKPitch = kHeadDim + 8;         // bf16 per K row in LDS (272 B)
constexpr int kVPitch = kBN + 8;              // bf16 per V^T row in LDS (144 B)
constexpr int kKElems = kBN * kKPitch;        // 8704
constexpr int kVElems = kHeadDim * kVPitch;   // 9216
constexpr int kBufElems = kKElems + kVElems;  // 17920 bf16 = 35840 B per buffer
constexpr int kBtWindow = 64;                 // block-table entries held in one register
constexpr int kCostBuckets = 1024;            // schedule sort resolution (tiles)

struct TileRegs {
  u32x4 k[2];   // 16 B of K rows (tid/8) and (tid/8 + 32): bytes [16*(tid%8), +16)
  u32x2 v[4];   // 8 B (dims [8*(tid%16), +8)) of tokens 4*(tid/16) + e
};

// position of token t (0..63) inside the transposed V tile before the chunk
// swizzle: bits 2 and 3 swapped (the P^T operand layout).
__device__ __forceinline__ int v_pos(int t) {
  const int b2 = (t >> 2) & 1, b3 = (t >> 3) & 1;
  return (t & ~12) | (b2 << 3) | (b3 << 2);
}

// Chunk swizzle of V^T row `dim`: XOR of the column (in bf16) with 16 *
// bits 5..6 of the dim.  It is constant across the 32 rows one MFMA operand
// read touches (those rows are conflict-free as they are: 144-byte pitch),
// and separates the dim blocks a staging store group writes.  Keeps 8-element
// chunks intact.
__device__ __forceinline__ int v_swz(int dim) { return ((dim >> 5) & 3) << 4; }

// One 8-byte LDS store, kept as its own instruction (the compiler would pair
// adjacent rows into ds_write2_b64, whose two halves collide in the banks).
// Completion is waited for explicitly before the barrier that publishes it.
__device__ __forceinline__ void lds_store8(const uint16_t* p, u32x2 v) {
  const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint16_t*)p;
  asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(v));
}

// s_waitcnt lgkmcnt(0): every LDS access of this wave has completed.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xc07f); }

struct ItemGeom {
  int q_start, Lq, k_start, Lk, c;
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
  return max(0, (kv_hi + kBN - 1) / kBN);
}

__device__ __forceinline__ bool item_valid(const PrefillParams& p, const ItemGeom& g, int mb) {
  return g.Lq > p.mq_max_q && mb * p.BM < g.Lq;
}

}  // namespace

// ---------------------------------------------------------------------------
// Schedule: one workgroup writes the (seq, m-block) items in decreasing tile
// count (counting sort), followed by (-1, -1) for slots without an item.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_schedule_kernel(PrefillParams p, int2* __restrict__ items,
                                                               int n_items_max) {
  __shared__ int hist[kCostBuckets];
  __shared__ int warp_tot[4];
  const int tid = threadIdx.x;
  for (int b = tid; b < kCostBuckets; b += 256) hist[b] = 0;
  __syncthreads();
  for (int idx = tid; idx < n_items_max; idx += 256) {
    const int seq = idx / p.n_mblocks, mb = idx - seq * p.n_mblocks;
    const ItemGeom g = item_geom(p, seq);
    if (!item_valid(p, g, mb)) continue;
    atomicAdd(&hist[min(item_tiles(p, g, mb), kCostBuckets - 1)], 1);
  }
  __syncthreads();
  // Exclusive scan in decreasing cost order: thread t owns buckets
  // [1023 - 4t - 3, 1023 - 4t] (walked from high cost to low).
  int local[4], sum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    local[j] = hist[kCostBuckets - 1 - (4 * tid + j)];
    sum += local[j];
  }
  int incl = sum;  // inclusive scan of per-thread sums over the wave
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) warp_tot[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += warp_tot[w];
  const int total = warp_tot[0] + warp_tot[1] + warp_tot[2] + warp_tot[3];
  int run = base + incl - sum;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    hist[kCostBuckets - 1 - (4 * tid + j)] = run;
    run += local[j];
  }
  __syncthreads();
  for (int idx = tid; idx < n_items_max; idx += 256) {
    const int seq = idx / p.n_mblocks, mb = idx - seq * p.n_mblocks;
    const ItemGeom g = item_geom(p, seq);
    if (!item_valid(p, g, mb)) continue;
    const int pos = atomicAdd(&hist[min(item_tiles(p, g, mb), kCostBuckets - 1)], 1);
    items[pos] = make_int2(seq, mb);
  }
  for (int pos = total + tid; pos < n_items_max; pos += 256) items[pos] = make_int2(-1, -1);
}

// ---------------------------------------------------------------------------
// Main kernel
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void varlen_prefill_kernel(PrefillParams p, const int2* __restrict__ items) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kBufElems];

  // blockIdx.x = item * n_groups + group: the kv-head group varies fastest.
  const int n_groups = p.Hkv * p.n_hgroups;
  const int item = (int)(blockIdx.x / (unsigned)n_groups);
  const int grp = (int)blockIdx.x - item * n_groups;
  const int2 it = items[item];
  if (it.x < 0) return;
  const int seq = it.x, mb = it.y;
  const int g = grp / p.n_hgroups;
  const int hg = grp - g * p.n_hgroups;
  const ItemGeom geo = item_geom(p, seq);
  const int Lq = geo.Lq, Lk = geo.Lk, c = geo.c;
  const int m0 = mb * p.BM;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_uniform(tid >> 6);
  const int h = lane >> 5, col = lane & 31;
  const int hw = wave % p.GW, tw = wave / p.GW;
  const int head = g * p.G + hg * p.GW + hw;
  const int m0w = m0 + 32 * tw;          // first query token of this wave
  const int tq = m0w + col;              // this lane's query token

  // ---- Q operand (B of S^T): dims 16ks + 8h + [0,8) --------------------------
  bf16x8 qop[8];
  {
    const int64_t row = (int64_t)geo.q_start + tq;
    const bool valid = tq < Lq && row < p.q_rows;
    const uint16_t* qp = p.q + (row * p.Hq + head) * kHeadDim + 8 * h;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      u32x4 a = {0u, 0u, 0u, 0u};
      if (valid) a = *reinterpret_cast<const u32x4*>(qp + 16 * ks);
      qop[ks] = as_bf16x8(a);
    }
  }

  f32x16 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const int n_tiles = item_tiles(p, geo, mb);
  const bool paged = p.block_tables != nullptr;
  const int64_t rs = (int64_t)p.Hkv * kHeadDim;  // bytes between token rows

  // ---- per-thread load / staging geometry ------------------------------------
  // K: thread t loads and stages 16 fp8 of rows t/8 and t/8 + 32.
  // V: thread t loads dims [8*dg, +8) of tokens 4*tg + e.  Inside each
  // 16-lane group the lanes span 4 dim blocks (bits 5..6 of the dim, which
  // pick the chunk swizzle) x 4 token groups, so the group's transposing
  // stores (one dim row, 4 tokens each) land on 16 distinct bank pairs;
  // each load instruction still covers 4 whole rows.
  const int k_row = tid >> 3;                       // K rows k_row and k_row + 32
  const int k_byte = 16 * (tid & 7);
  const int v_q = tid & 15, v_g = (tid >> 4) & 3;
  const int v_tg = (v_q & 3) + 4 * (tid >> 6);                          // tokens 4*v_tg + e
  const int v_byte = 8 * (4 * (v_q >> 2) + (v_g & 1) + 2 * (v_g >> 1));  // dims [v_byte, +8)
  const uint32_t k_off0 = (uint32_t)(k_row * rs + k_byte);
  const uint32_t k_off1 = (uint32_t)((k_row + 32) * rs + k_byte);
  const uint32_t v_off = (uint32_t)(4 * v_tg * rs + v_byte);
  const uint32_t urs = (uint32_t)rs;

  // Block-table window: lane l holds entry win_base + l (paged layout).
  int bt_lane = 0, win_base = 0;

  // Issues the loads of tile t into tr.  Tiles past the item (or with an
  // invalid block) get zero-length descriptors: the loads read nothing.
  auto load_tile = [&](int t, TileRegs& tr) {
    const int kv0 = t * kBN;
    int nvalid = (t < n_tiles) ? min(kBN, Lk - kv0) : 0;
    int64_t row0 = 0;
    if (paged) {
      const int bi = kv0 / p.block_size;
      const int blk = __builtin_amdgcn_readlane(bt_lane, min(max(bi - win_base, 0), kBtWindow - 1));
      row0 = (int64_t)blk * p.block_size + (kv0 - bi * p.block_size);
      if (blk < 0 || row0 + kBN > p.kv_rows) nvalid = 0;
    } else {
      row0 = (int64_t)geo.k_start + kv0;
      if (row0 < 0 || row0 + max(nvalid, 0) > p.kv_rows) nvalid = 0;
    }
    nvalid = max(nvalid, 0);
    if (nvalid == 0) row0 = 0;
    const int64_t base = (row0 * p.Hkv + g) * kHeadDim;
    const uint32_t nbytes = (uint32_t)(nvalid * rs);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + base, nbytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.v + base, nbytes);
    tr.k[0] = buf_load16(rk, k_off0);
    tr.k[1] = buf_load16(rk, k_off1);
#pragma unroll
    for (int e = 0; e < 4; ++e) tr.v[e] = buf_load8(rv, v_off + (uint32_t)e * urs);
  };

  // Converts tile registers to bf16 and writes LDS buffer `b`.
  auto stage_tile = [&](const TileRegs& tr, int b) {
    uint16_t* kb = lds + b * kBufElems;
    uint16_t* vb = kb + kKElems;
    // Lanes 4..7 of each row store their high 16 bytes first, so each
    // store instruction's 8-lane groups cover all banks of the row.
    const bool swap_halves = (tid & 4) != 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const u32x4 w = tr.k[i];
      u32x4 lo, hi;
      lo.x = fp8x2_to_bf16x2<false>(w.x); lo.y = fp8x2_to_bf16x2<true>(w.x);
      lo.z = fp8x2_to_bf16x2<false>(w.y); lo.w = fp8x2_to_bf16x2<true>(w.y);
      hi.x = fp8x2_to_bf16x2<false>(w.z); hi.y = fp8x2_to_bf16x2<true>(w.z);
      hi.z = fp8x2_to_bf16x2<false>(w.w); hi.w = fp8x2_to_bf16x2<true>(w.w);
      uint16_t* kd = kb + (k_row + 32 * i) * kKPitch + k_byte;
      const u32x4 first = swap_halves ? hi : lo, second = swap_halves ? lo : hi;
      *reinterpret_cast<u32x4*>(kd + (swap_halves ? 8 : 0)) = first;
      *reinterpret_cast<u32x4*>(kd + (swap_halves ? 0 : 8)) = second;
    }
    // V: transpose 4 tokens x 8 dims; one 8-byte store (4 tokens) per dim.
    const int pos = v_pos(4 * v_tg);  // tokens 4tg..4tg+3 stay contiguous
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t a = half ? tr.v[0].y : tr.v[0].x;
      const uint32_t bb = half ? tr.v[1].y : tr.v[1].x;
      const uint32_t cc = half ? tr.v[2].y : tr.v[2].x;
      const uint32_t d = half ? tr.v[3].y : tr.v[3].x;
      const uint32_t x01 = __builtin_amdgcn_perm(a, bb, 0x01050004u);   // [a0 b0 a1 b1]
      const uint32_t y01 = __builtin_amdgcn_perm(cc, d, 0x01050004u);   // [c0 d0 c1 d1]
      const uint32_t x23 = __builtin_amdgcn_perm(a, bb, 0x03070206u);   // [a2 b2 a3 b3]
      const uint32_t y23 = __builtin_amdgcn_perm(cc, d, 0x03070206u);   // [c2 d2 c3 d3]
      const uint32_t tt[4] = {__builtin_amdgcn_perm(x01, y01, 0x01000504u),   // [a0 b0 c0 d0]
                              __builtin_amdgcn_perm(x01, y01, 0x03020706u),   // [a1 b1 c1 d1]
                              __builtin_amdgcn_perm(x23, y23, 0x01000504u),   // [a2 b2 c2 d2]
                              __builtin_amdgcn_perm(x23, y23, 0x03020706u)};  // [a3 b3 c3 d3]
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int dim = v_byte + 4 * half + e;
        lds_store8(vb + dim * kVPitch + (pos ^ v_swz(dim)), fp8x4_to_bf16x4(tt[e]));
      }
    }
  };

  // Attention over tile t (LDS buffer b) for this wave's 32 rows.
  auto compute_tile = [&](int t, int b) {
    const int kv0 = t * kBN;
    if (kv0 > c + m0w + 31) return;  // wholly above this wave's causal diagonal
    const bool need_mask = (kv0 + kBN - 1 > c + m0w) || (kv0 + kBN > Lk);
    const uint16_t* kb = lds + b * kBufElems;
    const uint16_t* vb = kb + kKElems;

    // ---- S^T = K . Q^T ------------------------------------------------------
    // The two row blocks' MFMA chains are interleaved (step i: k-step i/2 of
    // row block i%2) and each K operand is read from LDS four steps before
    // its MFMA, so the LDS latency hides behind the MFMAs in flight.
    f32x16 s[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[rb][i] = 0.f;
    {
      const uint16_t* kr = kb + col * kKPitch + 8 * h;
      auto kaddr = [&](int i) { return kr + (i & 1) * 32 * kKPitch + 16 * (i >> 1); };
      u32x4 pre[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pre[i] = *reinterpret_cast<const u32x4*>(kaddr(i));
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const u32x4 cur = pre[i & 3];
        if (i + 4 < 16) pre[i & 3] = *reinterpret_cast<const u32x4*>(kaddr(i + 4));
        s[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(cur), qop[i >> 1], s[i & 1], 0, 0, 0);
      }
      // Keep that order through scheduling: 4 LDS reads, then MFMA / read
      // pairs, then the last 4 MFMAs.
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < 12; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }

    // ---- online softmax (row = query column of this lane) -----------------
    // The maximum is taken over raw scores (scale > 0), the exponent is
    // exp2(s * scale_log2 - m) with m in log2 units.
    if (need_mask) {
      const int lim = c + tq;  // last visible key
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int j = kv0 + 32 * rb + (i & 3) + 8 * (i >> 2) + 4 * h;
          s[rb][i] = (j <= lim && j < Lk) ? s[rb][i] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[rb][i]);
    mx = fmaxf(mx, shfl_xor_f32(mx, 32)) * p.scale_log2;
    // Lazy rescale (see kLazyRescaleLog2).
    const bool grow = mx > m_run + kLazyRescaleLog2;
    if (wave_any(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = grow ? fast_exp2(m_run - m_new) : 1.f;
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
    }
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
    float ps = 0.f;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e = fast_exp2(__builtin_fmaf(s[rb][i], p.scale_log2, -m_use));
        s[rb][i] = e;
        ps += e;
      }
    l_run += ps;

    // ---- O^T += V^T . P^T -----------------------------------------------------
    // MFMA i = (k-step i/4, dim block i%4); each V^T operand is read from LDS
    // four MFMAs ahead (same scheme as S^T).
    {
      auto vaddr = [&](int i) {
        const int ks = i >> 2, d = 32 * (i & 3) + col;
        return vb + d * kVPitch + ((16 * ks + 8 * h) ^ v_swz(d));
      };
      u32x4 pre[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pre[i] = *reinterpret_cast<const u32x4*>(vaddr(i));
      bf16x8 pop;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int ks = i >> 2;
        if ((i & 3) == 0) {
          const int rb = ks >> 1, base = 8 * (ks & 1);
          pop = as_bf16x8(pack_bf16x2(s[rb][base + 0], s[rb][base + 1]),
                          pack_bf16x2(s[rb][base + 2], s[rb][base + 3]),
                          pack_bf16x2(s[rb][base + 4], s[rb][base + 5]),
                          pack_bf16x2(s[rb][base + 6], s[rb][base + 7]));
        }
        const u32x4 cur = pre[i & 3];
        if (i + 4 < 16) pre[i & 3] = *reinterpret_cast<const u32x4*>(vaddr(i + 4));
        acc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(cur), pop, acc[i & 3], 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < 12; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
  };

  // ---- tile loop, one block-table window at a time -----------------------------
  // Within a window: tile t is computed from buffer t%2 while tile t+1 is
  // staged into the other buffer and tile t+2 is loading into registers.
  // The loop runs whole pairs of tiles and leaves only through its latch (a
  // phantom last tile is skipped by a uniform branch), so every path into
  // the loop head has the same loads in flight.
  const int win_tiles = paged ? kBtWindow * p.block_size / kBN : n_tiles;
  for (int t0 = 0; t0 < n_tiles; t0 += win_tiles) {
    const int t1 = min(n_tiles, t0 + win_tiles);
    if (paged) {
      win_base = (t0 * kBN) / p.block_size;
      const int bi = min(win_base + lane, (int)p.bt_stride - 1);
      bt_lane = p.block_tables[(int64_t)seq * p.bt_stride + bi];
    }
    TileRegs ra, rb;
    load_tile(t0, ra);
    load_tile(t0 + 1 < t1 ? t0 + 1 : n_tiles, rb);
    stage_tile(ra, 0);
    wait_lds();
    __syncthreads();
    for (int t = t0; t < t1; t += 2) {
      load_tile(t + 2 < t1 ? t + 2 : n_tiles, ra);
      compute_tile(t, 0);
      stage_tile(rb, 1);
      wait_lds();
      __syncthreads();
      load_tile(t + 3 < t1 ? t + 3 : n_tiles, rb);
      if (t + 1 < t1) compute_tile(t + 1, 1);
      stage_tile(ra, 0);
      wait_lds();
      __syncthreads();
    }
  }

  // ---- normalise and store ----------------------------------------------------
  l_run += shfl_xor_f32(l_run, 32);
  const int64_t row = (int64_t)geo.q_start + tq;
  if (tq < Lq && row < p.q_rows) {
    const float inv = (l_run > 0.f) ? 1.0f / l_run : 0.f;
    uint16_t* op = p.out + (row * p.Hq + head) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int b4 = 0; b4 < 4; ++b4) {
        const int d = 32 * db + 8 * b4 + 4 * h;
        u32x2 w;
        w.x = out_round_bf16_bits(acc[db][4 * b4 + 0] * inv) | (out_round_bf16_bits(acc[db][4 * b4 + 1] * inv) << 16);
        w.y = out_round_bf16_bits(acc[db][4 * b4 + 2] * inv) | (out_round_bf16_bits(acc[db][4 * b4 + 3] * inv) << 16);
        *reinterpret_cast<u32x2*>(op + d) = w;
      }
    }
  }
}

int64_t prefill_schedule_bytes(const PrefillParams& p) {
  return (int64_t)p.num_seqs * p.n_mblocks * (int64_t)sizeof(int2);
}

hipError_t launch_varlen_prefill(const PrefillParams& p, void* schedule, hipStream_t stream) {
  if (p.num_seqs == 0 || p.n_mblocks == 0) return hipSuccess;
  const int64_t n_items_max = (int64_t)p.num_seqs * p.n_mblocks;
  const int64_t n_blocks = n_items_max * p.Hkv * p.n_hgroups;
  if (n_blocks > 0x7fffffff || schedule == nullptr) return hipErrorInvalidValue;
  int2* items = static_cast<int2*>(schedule);
  hipLaunchKernelGGL(prefill_schedule_kernel, dim3(1), dim3(256), 0, stream, p, items, (int)n_items_max);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(varlen_prefill_kernel, dim3((unsigned)n_blocks), dim3(256), 0, stream, p,
                     (const int2*)items);
  return hipGetLastError();
}

}  // namespace nvamd
