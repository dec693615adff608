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
// query heads sharing it).  A workgroup is 8 waves = 256 query rows = GW
// heads x BM tokens; wave w owns 32 rows: head (w % GW), tokens
// [m0 + 32*(w / GW), +32).  The short-query launch before this kernel
// orders the items by decreasing number of KV tiles (a counting sort on the
// device, prefill_schedule), and the grid walks that list with the kv-head
// group varying fastest, so the longest items start first and short ones
// fill the tail.  Workgroups past the items merge the short-query rows'
// split-KV partitions.
//
// K/V stream in 64-token tiles, K one tile ahead of V.  Waves 0..3 load and
// stage K tiles, waves 4..7 V tiles: each thread loads its share of an FP8
// tile into registers two steps ahead (bounded raw buffer loads: rows past
// the sequence read as zero, so every iteration issues the same loads and
// the compiler's wait counts stay exact), converts it to bf16 (exact) and
// stages it in one of two LDS buffers -- K as [token][dim], V transposed as
// [dim][token] -- while the waves compute the other buffer.  One barrier
// per tile.  Each K load instruction fetches 8 rows (8 lanes per row), each
// V load instruction 4 whole rows.
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
// Step t of a wave runs the softmax of S_t with the MFMAs of S_{t+1}
// interleaved between its exponentials, then O += P_t V_t.  The kernel is
// register-budgeted for two waves per SIMD (one workgroup per CU).
#include "fp8_common.h"
#include "kernels.h"
#include "mq_merge.h"
#include "prefill_items.h"

namespace nvamd {

namespace {

constexpr int kBN = kPrefillTile;             // kv tokens per tile
constexpr int kKPitch = kHeadDim + 8;         // bf16 per K row in LDS (272 B)
constexpr int kVPitch = kBN + 8;              // bf16 per V^T row in LDS (144 B)
constexpr int kKElems = kBN * kKPitch;        // 8704
constexpr int kVElems = kHeadDim * kVPitch;   // 9216
constexpr int kBufElems = kKElems + kVElems;  // 17920 bf16 = 35840 B per K + V pair
constexpr int kBtWindow = 64;                 // block-table entries held in one register

// One staging thread's share of a K or V tile (see the staging geometry in
// the kernel): K rows s/8 (r[0], r[1]) and s/8 + 32 (r[2], r[3]), bytes
// [16*(s%8), +16) of each, as two 8-byte halves in store order; or 8 fp8
// (one dim group) of each of 4 tokens.
struct TileRegs {
  u32x2 r[4];
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

// One 8-byte LDS store to p + OFF bytes, kept as its own instruction (the
// compiler would pair adjacent rows into ds_write2_b64, whose two halves
// collide in the banks).  Completion is waited for explicitly before the
// barrier that publishes it.
template <int OFF>
__device__ __forceinline__ void lds_store8(const uint16_t* p, u32x2 v) {
  static_assert(OFF >= 0 && OFF < 65536, "ds_write_b64 offset is 16 bits");
  const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint16_t*)p;
  asm volatile("ds_write_b64 %0, %1 offset:%2" ::"v"(a), "v"(v), "i"(OFF));
}

// s_waitcnt lgkmcnt(0): every LDS access of this wave has completed.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xc07f); }

}  // namespace

// ---------------------------------------------------------------------------
// Main kernel
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64 * kPrefillWaves, 1) void varlen_prefill_kernel(PrefillParams p,
                                                                              const int2* __restrict__ items,
                                                                              MqParams mq, int n_main) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kBufElems];

  // Workgroups past the items merge the split-KV partitions of the
  // short-query sequences (one sequence each), which the launch before this
  // one computed.
  if ((int)blockIdx.x >= n_main) {
    merge_varlen_seq(mq, (int)blockIdx.x - n_main, wave_uniform(threadIdx.x >> 6), kPrefillWaves, threadIdx.x & 63);
    return;
  }

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
  // Waves 0..3 load and stage K tiles, waves 4..7 V tiles; s = tid % 256.
  // K: thread s loads and stages 16 fp8 of rows s/8 and s/8 + 32.
  // V: thread s loads dims [8*dg, +8) of tokens 4*tg + e.  Inside each
  // 16-lane group the lanes span 4 dim blocks (bits 5..6 of the dim, which
  // pick the chunk swizzle) x 4 token groups, so the group's transposing
  // stores (one dim row, 4 tokens each) land on 16 distinct bank pairs;
  // each load instruction still covers 4 whole rows.
  const bool k_role = wave < 4;
  // The V waves stage twice the vector work of the K waves (the transpose)
  // and, being younger, lose the SIMD's issue arbitration to them, so they
  // reach each barrier last; a higher wave priority evens that out.
  if (!k_role) __builtin_amdgcn_s_setprio(1);
  const int stid = tid & 255;
  const int k_row = stid >> 3;                      // K rows k_row and k_row + 32
  const int k_byte = 16 * (stid & 7);
  const int v_q = stid & 15, v_g = (stid >> 4) & 3;
  const int v_tg = (v_q & 3) + 4 * (stid >> 6);                         // tokens 4*v_tg + e
  const int v_byte = 8 * (4 * (v_q >> 2) + (v_g & 1) + 2 * (v_g >> 1));  // dims [v_byte, +8)
  // Lanes 4..7 of each K row store (and so load) their high 8 fp8 first,
  // so each store instruction's 8-lane groups cover all banks of the row.
  const int k_first = (stid & 4) ? 8 : 0;
  const uint32_t k_off0 = (uint32_t)(k_row * rs + k_byte + k_first);
  const uint32_t k_off1 = (uint32_t)((k_row + 32) * rs + k_byte + k_first);
  const uint32_t v_off = (uint32_t)(4 * v_tg * rs + v_byte);
  const uint32_t urs = (uint32_t)rs;

  // Block-table window: lane l holds entry win_base + l (paged layout).
  int bt_lane = 0, win_base = 0;

  // Buffer descriptor of tile t of this wave's role (K or V).  Tiles past
  // the item (or with an invalid block) get zero-length descriptors: their
  // loads read nothing.
  auto tile_rsrc = [&](int t) {
    const int kv0 = t * kBN;
    int nvalid = (t < n_tiles) ? min(kBN, Lk - kv0) : 0;
    int64_t row0 = 0;
    if (paged) {
      // block index and offset: shift and mask for power-of-two block sizes
      // (a runtime division costs dozens of instructions per tile)
      const int bi = (p.bs_shift >= 0) ? (kv0 >> p.bs_shift) : kv0 / p.block_size;
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
    return make_rsrc((k_role ? p.k : p.v) + base, nbytes);
  };
  // Loads this thread's share of tile t of its role: K tile t (K waves) or
  // V tile tv (V waves).
  auto load = [&](int t, int tv, TileRegs& r) {
    const __amdgpu_buffer_rsrc_t rs_ = tile_rsrc(k_role ? t : tv);
    if (k_role) {
      r.r[0] = buf_load8(rs_, k_off0);
      r.r[1] = buf_load8(rs_, k_off0 ^ 8u);
      r.r[2] = buf_load8(rs_, k_off1);
      r.r[3] = buf_load8(rs_, k_off1 ^ 8u);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) r.r[e] = buf_load8(rs_, v_off + (uint32_t)e * urs);
    }
  };

  // Converts a K tile share to bf16 and writes it to K buffer kb.
  const int k_lds[2] = {k_row * kKPitch + k_byte + k_first, k_row * kKPitch + k_byte + (k_first ^ 8)};
  auto stage_k = [&](const TileRegs& kr, uint16_t* kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x2 w = kr.r[i];
      u32x4 o;
      o.x = fp8x2_to_bf16x2<false>(w.x); o.y = fp8x2_to_bf16x2<true>(w.x);
      o.z = fp8x2_to_bf16x2<false>(w.y); o.w = fp8x2_to_bf16x2<true>(w.y);
      *reinterpret_cast<u32x4*>(kb + k_lds[i & 1] + (i >> 1) * 32 * kKPitch) = o;
    }
  };
  // Transposes a V tile share (4 tokens x 8 dims) to bf16 and writes it to
  // V^T buffer vb: one 8-byte store (4 tokens) per dim.
  // Dims v_byte..v_byte+7 share one chunk swizzle (v_byte is a multiple of
  // 8), so the 8 stores are one address plus constant offsets.
  const int v_lds = v_byte * kVPitch + (v_pos(4 * v_tg) ^ v_swz(v_byte));  // tokens 4tg..4tg+3 stay contiguous
  auto stage_v = [&](const TileRegs& vr, uint16_t* vb) {
    uint16_t* vd = vb + v_lds;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t a = half ? vr.r[0].y : vr.r[0].x;
      const uint32_t bb = half ? vr.r[1].y : vr.r[1].x;
      const uint32_t cc = half ? vr.r[2].y : vr.r[2].x;
      const uint32_t d = half ? vr.r[3].y : vr.r[3].x;
      const uint32_t x01 = __builtin_amdgcn_perm(a, bb, 0x01050004u);   // [a0 b0 a1 b1]
      const uint32_t y01 = __builtin_amdgcn_perm(cc, d, 0x01050004u);   // [c0 d0 c1 d1]
      const uint32_t x23 = __builtin_amdgcn_perm(a, bb, 0x03070206u);   // [a2 b2 a3 b3]
      const uint32_t y23 = __builtin_amdgcn_perm(cc, d, 0x03070206u);   // [c2 d2 c3 d3]
      const uint32_t tt[4] = {__builtin_amdgcn_perm(x01, y01, 0x01000504u),   // [a0 b0 c0 d0]
                              __builtin_amdgcn_perm(x01, y01, 0x03020706u),   // [a1 b1 c1 d1]
                              __builtin_amdgcn_perm(x23, y23, 0x01000504u),   // [a2 b2 c2 d2]
                              __builtin_amdgcn_perm(x23, y23, 0x03020706u)};  // [a3 b3 c3 d3]
      constexpr int kRow = 2 * kVPitch;  // bytes per V^T row
      if (half == 0) {
        lds_store8<0 * kRow>(vd, fp8x4_to_bf16x4(tt[0]));
        lds_store8<1 * kRow>(vd, fp8x4_to_bf16x4(tt[1]));
        lds_store8<2 * kRow>(vd, fp8x4_to_bf16x4(tt[2]));
        lds_store8<3 * kRow>(vd, fp8x4_to_bf16x4(tt[3]));
      } else {
        lds_store8<4 * kRow>(vd, fp8x4_to_bf16x4(tt[0]));
        lds_store8<5 * kRow>(vd, fp8x4_to_bf16x4(tt[1]));
        lds_store8<6 * kRow>(vd, fp8x4_to_bf16x4(tt[2]));
        lds_store8<7 * kRow>(vd, fp8x4_to_bf16x4(tt[3]));
      }
    }
  };

  // S^T = K . Q^T of one tile (K buffer kb).  The two row blocks' MFMA
  // chains are interleaved (step i: k-step i/2 of row block i%2); each K
  // operand is read from LDS four steps before its MFMA.  after(i) runs
  // behind MFMA i: vector work of another tile that fills the matrix pipe's
  // shadow.
  auto qk_mfma = [&](const uint16_t* kb, f32x16 (&s)[2], auto&& after) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[rb][i] = 0.f;
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
      after(i);
    }
  };

  // O^T += V^T . P^T for one tile (V^T in buffer vb): MFMA i = (k-step i/4,
  // dim block i%4); each V^T operand is read four MFMAs ahead.
  auto pv = [&](const bf16x8 (&pp)[4], const uint16_t* vb) {
    auto vaddr = [&](int i) {
      const int ks = i >> 2, d = 32 * (i & 3) + col;
      return vb + d * kVPitch + ((16 * ks + 8 * h) ^ v_swz(d));
    };
    u32x4 pre[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pre[i] = *reinterpret_cast<const u32x4*>(vaddr(i));
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u32x4 cur = pre[i & 3];
      if (i + 4 < 16) pre[i & 3] = *reinterpret_cast<const u32x4*>(vaddr(i + 4));
      acc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(cur), pp[i >> 2], acc[i & 3], 0, 0, 0);
    }
    // keep the reads four MFMAs ahead (the scheduler would otherwise sink
    // them next to their MFMAs to save registers)
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i < 12) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  };

  // One pipeline step for tile t of this wave: softmax of S_t (already in
  // s_cur), O^T += V^T . P^T from V buffer vb, and S_{t+1} = K . Q^T from K
  // buffer kb_next into s_next.  The S_{t+1} MFMAs are issued between the
  // exponentials of tile t, so the matrix and vector pipes work on different
  // tiles at the same time.  `loads` issues the step's global loads after the
  // exponentials, where S_t is dead and the registers they fill are free;
  // every wave issues them, since the whole workgroup stages each tile.
  auto step = [&](int t, bool run, f32x16 (&s_cur)[2], f32x16 (&s_next)[2], const uint16_t* kb_next,
                  const uint16_t* vb, auto&& loads) {
    const int kv0 = t * kBN;
    // not run, or tile t (and every later one) above this wave's diagonal:
    // nothing but the loads
    const bool active = run && kv0 <= c + m0w + 31;
    bf16x8 pop[4];
    if (active) {
    if ((kv0 + kBN - 1 > c + m0w) || (kv0 + kBN > Lk)) {
      // key kv0 + 4h + off is visible iff off < rem (keys up to c + tq, below Lk)
      const int rem = min(c + tq + 1, Lk) - kv0 - 4 * h;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int off = 32 * rb + (i & 3) + 8 * (i >> 2);
          s_cur[rb][i] = (off < rem) ? s_cur[rb][i] : -INFINITY;
        }
    }
    // The maximum is taken over raw scores (scale > 0); exponents are
    // exp2(s * scale_log2 - m) with m in log2 units.
    float mx = -INFINITY;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s_cur[rb][i]);
    {  // the other half of the column (lane l ^ 32) through v_permlane32_swap, no LDS round trip
      const uint32_t u = __builtin_bit_cast(uint32_t, mx);
      const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      const uint32_t s0 = sw[0], s1 = sw[1];
      mx = fmaxf(__builtin_bit_cast(float, s0), __builtin_bit_cast(float, s1)) * p.scale_log2;
    }
    const bool grow = mx > m_run + kLazyRescaleLog2;  // lazy rescale (see kLazyRescaleLog2)
    if (wave_any(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = grow ? fast_exp2(m_run - m_new) : 1.f;
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
    }
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run;

    // exponentials of tile t, two behind each S_{t+1} MFMA: element n of
    // S_t is s_cur[n / 16][n % 16]; word i of the P^T operands holds
    // elements 2i and 2i + 1.  The row sum adds the bf16 weights the PV
    // MFMAs use, two per v_dot2_f32_bf16 (against 1.0, 1.0).
    uint32_t pw[16];
    float ps = 0.f;
    qk_mfma(kb_next, s_next, [&](int i) {
      const int rb = i >> 3, n = (2 * i) & 15;
      const float e0 = fast_exp2(__builtin_fmaf(s_cur[rb][n], p.scale_log2, -m_use));
      const float e1 = fast_exp2(__builtin_fmaf(s_cur[rb][n + 1], p.scale_log2, -m_use));
      pw[i] = pack_bf16x2(e0, e1);
      ps = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pw[i]), __builtin_bit_cast(bf16x2, 0x3f803f80u),
                                           ps, false);
    });
    l_run += ps;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) pop[ks] = as_bf16x8(pw[4 * ks], pw[4 * ks + 1], pw[4 * ks + 2], pw[4 * ks + 3]);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i < 12) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x402, 7, 0);
    }
    }
    __builtin_amdgcn_sched_barrier(0);
    loads();
    __builtin_amdgcn_sched_barrier(0);
    if (active) pv(pop, vb);
  };

  // ---- tile loop, one block-table window at a time -----------------------------
  // K runs one tile ahead of V.  Step t reads S_{t+1}'s K from K buffer
  // (t+1)%2 and V_t from V buffer t%2, while K_{t+2} is staged into K buffer
  // t%2 and V_{t+1} into V buffer (t+1)%2 from registers loaded one step
  // earlier; the loads issued in step t fetch K_{t+3} and V_{t+2}.  One
  // barrier per step.  The loop runs whole pairs of steps and leaves only
  // through its latch; loads past the window read nothing, and steps past it
  // are skipped by uniform branches, so every path into the loop head has the
  // same loads in flight.
  uint16_t* kbuf0 = lds;
  uint16_t* kbuf1 = lds + kKElems;
  uint16_t* vbuf0 = lds + 2 * kKElems;
  uint16_t* vbuf1 = vbuf0 + kVElems;
  const int win_tiles = paged ? kBtWindow * p.block_size / kBN : n_tiles;
  for (int t0 = 0; t0 < n_tiles; t0 += win_tiles) {
    const int t1 = min(n_tiles, t0 + win_tiles);
    if (paged) {
      win_base = (t0 * kBN) / p.block_size;
      const int bi = min(win_base + lane, (int)p.bt_stride - 1);
      bt_lane = p.block_tables[(int64_t)seq * p.bt_stride + bi];
    }
    auto in_win = [&](int t) { return t < t1 ? t : n_tiles; };
    TileRegs ra, rb;
    load(t0, t0, ra);
    if (k_role) {
      load(in_win(t0 + 1), 0, rb);
      stage_k(ra, kbuf0);
      stage_k(rb, kbuf1);
    } else {
      stage_v(ra, vbuf0);
    }
    load(in_win(t0 + 2), in_win(t0 + 1), ra);
    wait_lds();
    __syncthreads();
    f32x16 sa[2], sb[2];
    qk_mfma(kbuf0, sa, [](int) {});
    for (int t = t0; t < t1; t += 2) {
      step(t, true, sa, sb, kbuf1, vbuf0, [&] { load(in_win(t + 3), in_win(t + 2), rb); });
      if (k_role) stage_k(ra, kbuf0);
      else stage_v(ra, vbuf1);
      wait_lds();
      __syncthreads();
      // past the window's last tile: no step, but the loads keep the same
      // count in flight at the loop head
      step(t + 1, t + 1 < t1, sb, sa, kbuf0, vbuf1, [&] { load(in_win(t + 4), in_win(t + 3), ra); });
      if (k_role) stage_k(rb, kbuf1);
      else stage_v(rb, vbuf0);
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

hipError_t launch_varlen_prefill(const PrefillParams& p, const void* schedule, const MqParams& mq, bool merge,
                                 hipStream_t stream) {
  if (p.num_seqs == 0 || p.n_mblocks == 0) return hipSuccess;
  const int64_t n_items_max = (int64_t)p.num_seqs * p.n_mblocks;
  const int64_t n_blocks = n_items_max * p.Hkv * p.n_hgroups;
  const int64_t n_merge = merge ? mq.num_seqs : 0;
  if (n_blocks + n_merge > 0x7fffffff || schedule == nullptr) return hipErrorInvalidValue;
  hipLaunchKernelGGL(varlen_prefill_kernel, dim3((unsigned)(n_blocks + n_merge)), dim3(64 * kPrefillWaves), 0, stream,
                     p, static_cast<const int2*>(schedule), mq, (int)n_blocks);
  return hipGetLastError();
}

}  // namespace nvamd
