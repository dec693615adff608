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
// tile into registers a step ahead (bounded raw buffer loads: rows past the
// sequence read as zero, so every iteration issues the same loads and the
// compiler's wait counts stay exact), converts it exactly -- K to bf16 (to
// fp16 for fp16 queries), V to fp16 -- and stages it in one of two LDS buffers, K as [token][dim], V
// transposed as [dim][token].  One barrier per tile.  Each K load
// instruction fetches 8 rows (8 lanes per row), each V load instruction 4
// whole rows.
//
// Per tile a wave computes (fp32 accumulate)
//     S^T[kv][q] = K[kv][:] . Q[q][:]          v_mfma_f32_32x32x16_bf16 (_f16), 2 row blocks x 8 k-steps
//     O^T[d][q] += V^T[d][kv] . P^T[kv][q]     v_mfma_f32_32x32x16_f16,  4 dim blocks x 4 k-steps
// The softmax weights P are rounded to fp16 (11-bit significand; the lazy
// rescale keeps them <= 2^8), V is exact in fp16.  Lane l (h = l / 32) holds
// query column l % 32; in the S^T result it holds kv tokens (i%4) + 8(i/4) +
// 4h of each 32-token row block, so the PV operand for k-step ks is simply
// p[ks/2][8(ks%2) .. +8) once V^T is stored with bits 2 and 3 of the token
// index swapped inside each 16-token step.  The V^T rows XOR their 16-byte
// chunks with bits 5..6 of the dim index and the V staging lanes are
// arranged so the transposing stores, the K stores and the MFMA operand
// reads are all free of LDS bank conflicts.  The causal mask is applied in
// registers only on tiles that cross the diagonal (or the end of the
// sequence); tiles wholly above a wave's rows only load and stage.  Step t
// of a wave is two stretches of 16 MFMAs with the vector work spread
// between them (part A: S_{t+1} and most of S_t's exponentials; part B:
// O += P_t V_t, S_{t+1}'s maximum, the loads and the staging).  The kernel
// is register-budgeted for two waves per SIMD (one workgroup per CU).
#include <type_traits>

#include "fp8_common.h"
#include "kernels.h"
#include "lds_dma.h"
#include "mq_merge.h"
#include "prefill_items.h"

namespace nvamd {

namespace {

constexpr int kBN = kPrefillTile;             // kv tokens per tile
constexpr int kKPitch = kHeadDim + 8;         // bf16 per K row in LDS (272 B)
constexpr int kVPitch = kBN + 8;              // fp16 per V^T row in LDS (144 B)
constexpr int kKElems = kBN * kKPitch;        // 8704
constexpr int kVElems = kHeadDim * kVPitch;   // 9216
constexpr int kBufElems = kKElems + kVElems;  // 17920 16-bit = 35840 B per K + V pair
constexpr int kQRowBytes = kHeadDim * 2;      // bytes per bf16 Q row (in a wave's LDS slice too)
constexpr int kQSliceBytes = 32 * kQRowBytes + 256;  // a wave's 32 Q rows + 64 block-table entries
constexpr int kBtWindow = 64;                 // block-table entries held in one register
constexpr int kLead = 4;                      // MFMA operands are read from LDS this many MFMAs ahead
// A tile's row sum of fp16 weights above this moves the reference maximum
// (every weight is then at most this, far below the fp16 maximum 65504).
constexpr float kRowSumLimit = 16384.0f;

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

// Chunk swizzle of V^T row `dim`: XOR of the column (in 16-bit elements) with 16 *
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

// Pins a value to this point of the instruction stream: the compiler would
// otherwise sink a computation into the block of its only use, out of the
// stretch of MFMAs it is placed between.
template <typename T>
__device__ __forceinline__ void pin(T& v) { asm volatile("" : "+v"(v)); }

}  // namespace

// ---------------------------------------------------------------------------
// Main kernel
// ---------------------------------------------------------------------------
template <bool PAGED, bool SMALL_BLOCKS, bool F16>
__global__ __launch_bounds__(64 * kPrefillWaves, 1) void varlen_prefill_kernel(PrefillParams p,
                                                                              const PrefillItem* __restrict__ items,
                                                                              MqParams mq, int n_main) {
  using QT = QkType<F16>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kBufElems];

  // Workgroups past the items merge the split-KV partitions of the
  // short-query sequences, which the launch before this one computed: one
  // (row, head) pair per wave.
  if ((int)blockIdx.x >= n_main) {
    const int slices = merge_slices(mq, kPrefillWaves);
    const int m = (int)blockIdx.x - n_main, seq = m / slices;
    const int idx = (m - seq * slices) * kPrefillWaves + (int)(threadIdx.x >> 6);
    if (mq.sk_part != nullptr) sk_merge_one(mq, seq, idx, threadIdx.x & 63);  // balanced-kernel partials
    else merge_varlen_one(mq, seq, idx, threadIdx.x & 63);                    // split-KV partitions
    return;
  }

  // Unit blockIdx.x = record * n_groups + group (the kv-head group varies
  // fastest); the last round's workgroups claim theirs in the order they
  // start (the schedule pass zeroed the counter and wrote the bounds).  The
  // bounds are scalar loads beside the record's, so a workgroup that does not
  // claim waits for neither longer than for its record.
  const int n_groups = p.Hkv * p.n_hgroups;
  int unit = (int)blockIdx.x;
  int item = (int)((unsigned)unit / (unsigned)n_groups);
  // one record load gives the piece and its geometry
  int4 rec_a = items[item].head, rec_b = items[item].tail, rec_c = items[item].split;
  {
    int* claim = p.counters + p.slots_per_group * n_groups;
    const auto* bounds = (const __attribute__((address_space(4))) int*)(claim + 1);
    const int claim_from = bounds[0], total_units = bounds[1];
    // the bounds and the record are loaded together (the record is reloaded
    // only by a workgroup that claims)
    asm volatile("" ::"s"(claim_from), "s"(total_units), "s"(rec_a.x), "s"(rec_a.y), "s"(rec_a.z), "s"(rec_a.w),
                 "s"(rec_b.x), "s"(rec_b.y), "s"(rec_b.z), "s"(rec_b.w), "s"(rec_c.x), "s"(rec_c.y), "s"(rec_c.z),
                 "s"(rec_c.w));
    if (unit >= claim_from && unit < total_units) {
      __shared__ int s_unit;
      if (threadIdx.x == 0)
        s_unit = claim_from + __hip_atomic_fetch_add(claim, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      unit = s_unit;
      item = (int)((unsigned)unit / (unsigned)n_groups);
      rec_a = items[item].head;
      rec_b = items[item].tail;
      rec_c = items[item].split;
    }
  }
  const int grp = unit - item * n_groups;
  const int seq = wave_uniform(rec_a.x);
  if (seq < 0) return;
  const int mb = wave_uniform(rec_a.y), q_start = wave_uniform(rec_a.z), Lq = wave_uniform(rec_a.w);
  const int k_start = wave_uniform(rec_b.x), Lk = wave_uniform(rec_b.y);
  const int t_lo = wave_uniform(rec_b.z), n_tiles = wave_uniform(rec_b.w);  // this piece: tiles [t_lo, n_tiles)
  const int piece = wave_uniform(rec_c.x), n_pieces = wave_uniform(rec_c.y);
  const int part_slot = wave_uniform(rec_c.z), counter = wave_uniform(rec_c.w);
  const int c = Lk - Lq;
  const int g = grp / p.n_hgroups;
  const int hg = grp - g * p.n_hgroups;
  const int m0 = mb * p.BM;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_uniform(tid >> 6);
  const int h = lane >> 5, col = lane & 31;
  const int hw = wave % p.GW, tw = wave / p.GW;
  const int head = g * p.G + hg * p.GW + hw;
  const int m0w = m0 + 32 * tw;          // first query token of this wave
  const int tq = m0w + col;              // this lane's query token

  // ---- Q operand (B of S^T): dims 16ks + 8h + [0,8) of query row col.
  // Loaded whole rows at a time (16 lanes x 16 bytes per 256-byte row, 4 rows
  // per instruction) straight into the wave's own LDS slice, then read back
  // in the operand layout: loaded in that layout directly, each instruction
  // would touch 32 rows 8 KiB apart for 32 bytes of each.  Chunk c of row r
  // sits in slot c ^ (r % 16) of the row, so the 16 lanes of an operand read
  // hit 16 different slots.  A wave reads back only what it loaded.  Rows
  // past the sequence (or past q) read as zero through a bounded buffer
  // descriptor, no branches.
  // The start of a workgroup is a chain of loads: the first block-table
  // window's entries go out first (to LDS, beside the wave's Q rows), then
  // Q; the tile loop waits for the window only (loads complete in order, so
  // vmcnt(8) leaves the 8 Q loads in flight) and issues the first tile
  // loads before it waits for Q, so Q's loads overlap both round trips.
  // Both are direct-to-LDS loads, which the compiler's wait counts do not
  // see: every wait for them is explicit.
  const int win_tiles = PAGED ? kBtWindow * p.block_size / kBN : max(n_tiles, 1);
  __shared__ __attribute__((aligned(16))) uint8_t q_lds[kPrefillWaves * kQSliceBytes];
  const uint8_t* qs = q_lds + wave * kQSliceBytes;
  const uint8_t* bt_first = qs + 32 * kQRowBytes;  // the first window's entries, one dword per lane
  if constexpr (PAGED) {
    const int bi = min(t_lo / win_tiles * kBtWindow + lane, (int)p.bt_stride - 1);
    dma_load4_keep(rsrc_words(p.block_tables + (int64_t)seq * p.bt_stride, (uint32_t)p.bt_stride * 4u),
                   (uint32_t)bi * 4u, lds_addr(bt_first));
  }
  {
    const int64_t row = (int64_t)q_start + m0w;
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(min(Lq - m0w, 32), p.q_rows - row));
    const uint32_t row_bytes = (uint32_t)(p.Hq * kHeadDim * 2);
    const u32x4 qr =
        rsrc_words(p.q + (row * p.Hq + head) * kHeadDim, rows == 0 ? 0u : (rows - 1) * row_bytes + kQRowBytes);
    const int r0 = lane >> 4, slot = lane & 15;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 4 * j + r0;
      dma_load16_keep(qr, (uint32_t)r * row_bytes + 16 * (slot ^ (r & 15)), lds_addr(qs + 4 * j * kQRowBytes));
    }
  }
  typename QT::V8 qop[8];
  auto q_to_operands = [&] {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the Q loads (and every later load) have landed
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      qop[ks] = QT::from_bits(*reinterpret_cast<const u32x4*>(qs + col * kQRowBytes + 16 * ((2 * ks + h) ^ (col & 15))));
  };

  f32x16 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  // Online softmax state: reference maximum (log2 units), the maximum the
  // exponentials of the current tile use, running row sum, and the row sum
  // of the next tile's weights computed so far.
  float m_run = -INFINITY, m_use = 0.f, l_run = 0.f, ps_pend = 0.f;

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
  const uint32_t urs = (uint32_t)rs;
  // With SMALL_BLOCKS (block_size % 64 != 0, a tile may span several
  // blocks) a wave's load instructions, which cover 8 consecutive tile rows
  // (K: rows kg0 + [0, 8) and kg0 + 32 + [0, 8)) or 16 (V: rows vg0 +
  // [0, 16)) that lie in one block whenever block_size % 16 == 0, get a
  // descriptor per row group, and the lanes' offsets are relative to its
  // first row; otherwise one descriptor covers the tile.
  const int kg0 = SMALL_BLOCKS ? 8 * (stid >> 6) : 0, vg0 = SMALL_BLOCKS ? 16 * (stid >> 6) : 0;
  const uint32_t k_rel = (uint32_t)((k_row - kg0) * rs + k_byte + k_first);
  const uint32_t k_rel_hi = SMALL_BLOCKS ? k_rel : (uint32_t)((k_row + 32) * rs + k_byte + k_first);
  const uint32_t v_rel = (uint32_t)(4 * (v_tg - vg0 / 4) * rs + v_byte);

  // Block-table window (paged layout): lane l holds the byte offset in the
  // cache of kv head g's slice of block entry win_base + l, as two dwords
  // (-1 when the entry is not a usable block), computed once per window so
  // that a descriptor takes a few scalar instructions.
  uint32_t blk_lo = 0, blk_hi = 0;
  int win_base = 0;

  // Buffer descriptor of rows [r0, r0 + nrows) of tile t.  Rows past the
  // item's keys (or in an invalid block, or of tiles past the item) are
  // outside the descriptor's range: their loads read zeros.
  auto group_rsrc = [&](int t, int r0, int nrows) {
    const int kv = t * kBN + r0;
    int nvalid = (t < n_tiles) ? min(nrows, Lk - kv) : 0;
    int64_t base = 0;
    if constexpr (PAGED) {
      // block of key kv by a multiply with the reciprocal of the block size
      // in 16-token units (exact for kv < 2^35 / block_size, which the host
      // checks; a division would be dozens of instructions and a branch)
      const int bi = (int)__umulhi((uint32_t)(kv >> 4) << 1, p.blk_magic);
      const int l = min(max(bi - win_base, 0), kBtWindow - 1);
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)blk_lo, l);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)blk_hi, l);
      const int64_t boff = (int64_t)(((uint64_t)hi << 32) | lo);
      if (boff < 0) nvalid = 0;
      base = boff + (int64_t)((uint32_t)(kv - bi * p.block_size) * urs);
    } else {
      const int64_t row0 = (int64_t)k_start + kv;
      if (row0 < 0 || row0 + max(nvalid, 0) > p.kv_rows) nvalid = 0;
      base = (row0 * p.Hkv + g) * kHeadDim;
    }
    nvalid = max(nvalid, 0);
    if (nvalid == 0) base = 0;
    const uint32_t nbytes = (uint32_t)(nvalid * rs);
    return make_rsrc((k_role ? p.k : p.v) + base, nbytes);
  };
  // Loads this thread's share of tile t of its role: K tile t (K waves) or
  // V tile tv (V waves).  The role is a compile-time constant (std::true_type
  // for K) so that no branch splits the code the loads are scheduled into.
  auto load = [&](auto role, int t, int tv, TileRegs& r) {
    constexpr bool kRole = decltype(role)::value;
    if constexpr (kRole) {
      const __amdgpu_buffer_rsrc_t lo = SMALL_BLOCKS ? group_rsrc(t, kg0, 8) : group_rsrc(t, 0, kBN);
      const __amdgpu_buffer_rsrc_t hi = SMALL_BLOCKS ? group_rsrc(t, kg0 + 32, 8) : lo;
      r.r[0] = buf_load8(lo, k_rel);
      r.r[1] = buf_load8(lo, k_rel ^ 8u);
      r.r[2] = buf_load8(hi, k_rel_hi);
      r.r[3] = buf_load8(hi, k_rel_hi ^ 8u);
    } else {
      const __amdgpu_buffer_rsrc_t rv = SMALL_BLOCKS ? group_rsrc(tv, vg0, 16) : group_rsrc(tv, 0, kBN);
#pragma unroll
      for (int e = 0; e < 4; ++e) r.r[e] = buf_load8(rv, v_rel + (uint32_t)e * urs);
    }
  };

  // Converts a K tile share to bf16 (fp16 with F16) and writes it to K buffer kb, in four
  // quarters (one 16-byte store each) that can be spread over a stretch of
  // MFMAs.
  const int k_lds[2] = {k_row * kKPitch + k_byte + k_first, k_row * kKPitch + k_byte + (k_first ^ 8)};
  auto stage_k_q = [&](const TileRegs& kr, uint16_t* kb, int i) {
    const u32x2 w = kr.r[i];
    u32x4 o;
    o.x = QT::template k2<false>(w.x); o.y = QT::template k2<true>(w.x);
    o.z = QT::template k2<false>(w.y); o.w = QT::template k2<true>(w.y);
    *reinterpret_cast<u32x4*>(kb + k_lds[i & 1] + (i >> 1) * 32 * kKPitch) = o;
  };
  auto stage_k = [&](const TileRegs& kr, uint16_t* kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) stage_k_q(kr, kb, i);
  };
  // Transposes a V tile share (4 tokens x 8 dims) to fp16 and writes it to
  // V^T buffer vb: one 8-byte store (4 tokens) per dim, in four quarters of
  // two dims each.  Dims v_byte..v_byte+7 share one chunk swizzle (v_byte is
  // a multiple of 8), so the 8 stores are one address plus constant offsets.
  const int v_lds = v_byte * kVPitch + (v_pos(4 * v_tg) ^ v_swz(v_byte));  // tokens 4tg..4tg+3 stay contiguous
  // quarter q: dims 2q and 2q + 1 of the share (bytes of the low or high
  // dword of each token's 8 fp8 for q < 2 or q >= 2)
  auto stage_v_q = [&](const TileRegs& vr, uint16_t* vb, auto qc) {
    constexpr int q = decltype(qc)::value;
    constexpr int half = q >> 1;
    uint16_t* vd = vb + v_lds;
    const uint32_t a = half ? vr.r[0].y : vr.r[0].x;
    const uint32_t bb = half ? vr.r[1].y : vr.r[1].x;
    const uint32_t cc = half ? vr.r[2].y : vr.r[2].x;
    const uint32_t d = half ? vr.r[3].y : vr.r[3].x;
    constexpr uint32_t kSel = (q & 1) ? 0x03070206u : 0x01050004u;  // bytes 2,3 or 0,1 of each token
    const uint32_t x = __builtin_amdgcn_perm(a, bb, kSel);    // [a_j b_j a_j+1 b_j+1]
    const uint32_t y = __builtin_amdgcn_perm(cc, d, kSel);    // [c_j d_j c_j+1 d_j+1]
    const uint32_t t0 = __builtin_amdgcn_perm(x, y, 0x01000504u);  // [a_j b_j c_j d_j]
    const uint32_t t1 = __builtin_amdgcn_perm(x, y, 0x03020706u);  // [a_j+1 b_j+1 c_j+1 d_j+1]
    constexpr int kRow = 2 * kVPitch;  // bytes per V^T row
    lds_store8<(2 * q) * kRow>(vd, fp8x4_to_f16x4(t0));
    lds_store8<(2 * q + 1) * kRow>(vd, fp8x4_to_f16x4(t1));
  };
  auto stage_v = [&](const TileRegs& vr, uint16_t* vb) {
    stage_v_q(vr, vb, std::integral_constant<int, 0>{});
    stage_v_q(vr, vb, std::integral_constant<int, 1>{});
    stage_v_q(vr, vb, std::integral_constant<int, 2>{});
    stage_v_q(vr, vb, std::integral_constant<int, 3>{});
  };
  auto stage = [&](auto role, const TileRegs& r, uint16_t* kb, uint16_t* vb) {
    if constexpr (decltype(role)::value) stage_k(r, kb);
    else stage_v(r, vb);
  };
  // quarter qc (an integral_constant) of the staging
  auto stage_q = [&](auto role, const TileRegs& r, uint16_t* kb, uint16_t* vb, auto qc) {
    if constexpr (decltype(role)::value) stage_k_q(r, kb, decltype(qc)::value);
    else stage_v_q(r, vb, qc);
  };

  // ---- softmax pieces -----------------------------------------------------------
  // Element n of an S^T tile is s[n / 16][n % 16]; lane (h, col) holds kv
  // token 32*(n/16) + (n%4) + 8*((n%16)/4) + 4h of query column col.
  // Word i of the P^T operands holds the weights of elements 2i and 2i + 1;
  // the row sum adds the fp16 weights the PV MFMAs use, two per
  // v_dot2_f32_f16 (against 1.0, 1.0).
  const f16x2 ones = __builtin_bit_cast(f16x2, 0x3c003c00u);
  auto exp_pair = [&](const f32x16 (&s)[2], int i, uint32_t (&pw)[16], float& ps) {
    const int rb = i >> 3, n = (2 * i) & 15;
    const float e0 = fast_exp2(__builtin_fmaf(s[rb][n], p.scale_log2, -m_use));
    const float e1 = fast_exp2(__builtin_fmaf(s[rb][n + 1], p.scale_log2, -m_use));
    pw[i] = pack_f16x2(e0, e1);
    ps = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pw[i]), ones, ps, false);
  };
  // Causal / length mask of tile t in registers (only tiles that cross the
  // diagonal or the end of the keys, and tiles past the window, which are
  // wholly masked): key kv0 + 4h + off is visible iff off < rem.
  auto mask_tile = [&](int t, int t_end, f32x16 (&s)[2]) {
    const int kv0 = t * kBN;
    if ((kv0 + kBN - 1 > c + m0w) || (kv0 + kBN > Lk) || t >= t_end) {
      const int rem = (t >= t_end) ? 0 : min(c + tq + 1, Lk) - kv0 - 4 * h;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int off = 32 * rb + (i & 3) + 8 * (i >> 2);
          s[rb][i] = (off < rem) ? s[rb][i] : -INFINITY;
        }
    }
  };
  // Row maximum of tile s in pieces: elements 8q..8q+7, then the running
  // maximum is moved from the maximum of the pieces (raw scores; the scale
  // is positive) on the lanes where it exceeds the reference.  Used on the
  // first tile of a block-table window and when a tile's weights grow past
  // kRowSumLimit.  The update scales the row sum and returns whether any
  // lane moved; alpha is the factor for the accumulators.
  auto max8 = [&](const f32x16 (&s)[2], int q) {
    const int rb = q >> 1, o = 8 * (q & 1);
    float m = fmaxf(s[rb][o], s[rb][o + 1]);
#pragma unroll
    for (int j = 2; j < 8; ++j) m = fmaxf(m, s[rb][o + j]);
    return m;
  };
  auto update_max_from = [&](float mx, float& alpha) {
    {  // the other half of the column (lane l ^ 32) through v_permlane32_swap, no LDS round trip
      const uint32_t u = __builtin_bit_cast(uint32_t, mx);
      const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      const uint32_t s0 = sw[0], s1 = sw[1];
      mx = fmaxf(__builtin_bit_cast(float, s0), __builtin_bit_cast(float, s1)) * p.scale_log2;
    }
    const bool grow = mx > m_run;
    alpha = grow ? fast_exp2(m_run - mx) : 1.f;
    m_run = grow ? mx : m_run;
    m_use = (m_run == -INFINITY) ? 0.f : m_run;
    l_run *= alpha;
    return wave_any(grow);
  };
  auto update_max = [&](const f32x16 (&s)[2], float& alpha) {
    return update_max_from(fmaxf(fmaxf(max8(s, 0), max8(s, 1)), fmaxf(max8(s, 2), max8(s, 3))), alpha);
  };
  auto rescale_acc = [&](float alpha) {
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[db] *= alpha;
  };

  // ---- the two halves of a pipeline step --------------------------------------
  // Step t of a wave (tile t visible to it): part A computes S_{t+1} = K_{t+1}
  // Q^T from K buffer kb with the exponentials of S_t's words 4..15 between
  // its MFMAs; part B computes O^T += V_t^T P_t^T from V buffer vb with, between
  // its MFMAs, the row maximum of S_{t+1}, the step's global loads, the staging
  // of the tiles loaded one step earlier and the exponentials of S_{t+1}'s
  // words 0..3.  Every MFMA of the step thus has a share of the vector work
  // behind it.  Operands are read from LDS four MFMAs ahead.
  auto vaddr = [&](const uint16_t* vb, int i) {  // V^T operand of PV MFMA i (k-step i/4, dim block i%4)
    const int ks = i >> 2, d = 32 * (i & 3) + col;
    return vb + d * kVPitch + ((16 * ks + 8 * h) ^ v_swz(d));
  };
  // Part A also reads part B's first four V^T operands (from vb) behind its
  // last MFMAs.
  auto part_a = [&](const uint16_t* kb, const uint16_t* vb, const f32x16 (&s_cur)[2], f32x16 (&s_next)[2],
                    uint32_t (&pw)[16], u32x4 (&vpre)[kLead]) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s_next[rb][i] = 0.f;
    const uint16_t* kr = kb + col * kKPitch + 8 * h;
    auto kaddr = [&](int i) { return kr + (i & 1) * 32 * kKPitch + 16 * (i >> 1); };
    u32x4 pre[kLead];
#pragma unroll
    for (int i = 0; i < kLead; ++i) pre[i] = *reinterpret_cast<const u32x4*>(kaddr(i));
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u32x4 cur = pre[i % kLead];
      if (i + kLead < 16) pre[i % kLead] = *reinterpret_cast<const u32x4*>(kaddr(i + kLead));
      else vpre[i + kLead - 16] = *reinterpret_cast<const u32x4*>(vaddr(vb, i + kLead - 16));
      s_next[i & 1] = QT::mfma32(QT::from_bits(cur), qop[i >> 1], s_next[i & 1]);
      if (i < 12) exp_pair(s_cur, 4 + i, pw, ps_pend);
    }
    // the first exponentials run while the first K operands are in flight
    __builtin_amdgcn_sched_group_barrier(0x100, kLead, 0);
    __builtin_amdgcn_sched_group_barrier(0x402, 6, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (i < 11) __builtin_amdgcn_sched_group_barrier(0x402, 6, 0);
    }
#pragma unroll
    for (int i = 4; i < 16; ++i) pin(pw[i]);
#pragma unroll
    for (int i = 0; i < kLead; ++i) pin(vpre[i]);
    pin(ps_pend);
  };

  // Part B places its work by hand, one segment per MFMA (sched_barrier
  // fences): the loads, the staging in four quarters, and S_{t+1}'s words
  // 0..3, one per segment.  S_{t+1} is exponentiated against the current
  // reference maximum without taking its row maximum first; the step checks
  // the resulting row sum instead (see full_step).
  auto part_b = [&](const uint16_t* vb, u32x4 (&vpre)[kLead], const uint32_t (&pw)[16], const f32x16 (&s_next)[2],
                    uint32_t (&pw_next)[16], auto&& loads, auto&& stage_quarter) {
    f16x8 pop[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) pop[ks] = as_f16x8(pw[4 * ks], pw[4 * ks + 1], pw[4 * ks + 2], pw[4 * ks + 3]);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u32x4 cur = vpre[i % kLead];
      if (i + kLead < 16) vpre[i % kLead] = *reinterpret_cast<const u32x4*>(vaddr(vb, i + kLead));
      acc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(cur), pop[i >> 2], acc[i & 3], 0, 0, 0);
      if (i == 0) loads();
      if (i == 3) stage_quarter(std::integral_constant<int, 0>{});
      if (i == 5) stage_quarter(std::integral_constant<int, 1>{});
      if (i == 7) stage_quarter(std::integral_constant<int, 2>{});
      if (i == 9) stage_quarter(std::integral_constant<int, 3>{});
      if (i == 10) ps_pend = 0.f;
      if (i >= 10 && i < 14) exp_pair(s_next, i - 10, pw_next, ps_pend);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) pin(pw_next[j]);
    pin(ps_pend);
  };

  // The weights of a tile are exp2(s * scale - m_use) with m_use the running
  // reference maximum, so they stay bounded as long as no score exceeds it
  // by much.  A lane's row sum of the tile's fp16 weights (ps_pend) above
  // kRowSumLimit (or infinite: an fp16 overflow) means some score did: the
  // reference maximum then moves to the row maximum of the tile, the
  // accumulators and row sum are rescaled, and the tile's 16 words are
  // computed again.  Rare (at most once per growth of the maximum by more
  // than log2(kRowSumLimit / 32)); every weight used is <= kRowSumLimit.
  auto check_tile = [&](const f32x16 (&s)[2], uint32_t (&pw)[16]) {
    if (wave_any(!(ps_pend <= kRowSumLimit))) {
      float alpha;
      if (update_max(s, alpha)) rescale_acc(alpha);
      ps_pend = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) exp_pair(s, j, pw, ps_pend);
    }
    l_run += ps_pend;
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
  // Window w holds the blocks of tiles [w * win_tiles, (w + 1) * win_tiles);
  // a piece starts inside one and ends inside one.
  // The tile loop, specialised for the wave's role (K or V staging).
  auto tile_loop = [&](auto role) {
  int t0 = t_lo, t1 = 0;
  auto in_win = [&](int t) { return t < t1 ? t : n_tiles; };
  TileRegs ra, rb;
  // Start of t0's window: its block offsets, the first tiles loaded and
  // staged, the next step's load issued.  The piece's first window is its
  // own copy (kFirst), placed before the loop: there the only loads in
  // flight are the direct-to-LDS block-table and Q loads, and the wait for
  // the table entries leaves the Q loads in flight (inside the loop the
  // compiler's waits would also cover loads of the previous window).
  auto window_start = [&](auto first) {
    constexpr bool kFirst = decltype(first)::value;
    const int win = t0 / win_tiles;
    t1 = min(n_tiles, (win + 1) * win_tiles);
    if constexpr (PAGED) {
      win_base = win * kBtWindow;
      int blk;
      if constexpr (kFirst) {
        // the entries were loaded before the 8 Q loads
        asm volatile("s_waitcnt vmcnt(8)\n\tds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                     : "=v"(blk)
                     : "v"(lds_addr(bt_first) + 4u * (uint32_t)lane)
                     : "memory");
      } else {
        blk = p.block_tables[(int64_t)seq * p.bt_stride + min(win_base + lane, (int)p.bt_stride - 1)];
      }
      const int64_t row = (int64_t)blk * p.block_size;
      const int64_t off = (blk >= 0 && row + p.block_size <= p.kv_rows) ? (row * p.Hkv + g) * kHeadDim : -1;
      blk_lo = (uint32_t)off;
      blk_hi = (uint32_t)((uint64_t)off >> 32);
    }
    load(role, t0, t0, ra);
    if constexpr (decltype(role)::value) load(role, in_win(t0 + 1), 0, rb);
    if constexpr (kFirst) q_to_operands();
    if constexpr (decltype(role)::value) {
      stage_k(ra, kbuf0);
      stage_k(rb, kbuf1);
    } else {
      stage_v(ra, vbuf0);
    }
    load(role, in_win(t0 + 2), in_win(t0 + 1), ra);
    wait_lds();
    __syncthreads();
  };
  if (t0 >= n_tiles) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no direct-to-LDS load outlives the wave
    return;
  }
  window_start(std::true_type{});
  for (;;) {
    // Prologue: S_{t0}, its maximum and the exponentials of its words 0..3.
    f32x16 sa[2], sb[2];
    uint32_t pa[16], pb[16];
    {
#pragma unroll
      for (int rb_ = 0; rb_ < 2; ++rb_)
#pragma unroll
        for (int i = 0; i < 16; ++i) sa[rb_][i] = 0.f;
      const uint16_t* kr = kbuf0 + col * kKPitch + 8 * h;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        sa[i & 1] = QT::mfma32(
            QT::from_bits(*reinterpret_cast<const u32x4*>(kr + (i & 1) * 32 * kKPitch + 16 * (i >> 1))), qop[i >> 1],
            sa[i & 1]);
      mask_tile(t0, t1, sa);
      float alpha;
      if (update_max(sa, alpha)) rescale_acc(alpha);
      ps_pend = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) exp_pair(sa, j, pa, ps_pend);
    }
    // K buffer 0 is restaged during the first step: every wave's reads of it
    // above must be done first.
    __syncthreads();

    // A step of tile t visible to this wave, and a step of a tile past it
    // (tiles above the wave's diagonal, and past the window, whose steps only
    // load and stage for the other waves).  Visibility is monotone in t, so
    // the visible steps run first; each step ends with the one barrier.
    auto full_step = [&](int t, f32x16 (&s_cur)[2], f32x16 (&s_next)[2], uint32_t (&pw)[16], uint32_t (&pw_next)[16],
                         const uint16_t* kb_next, const uint16_t* vb, TileRegs& stage_regs, uint16_t* stage_kb,
                         uint16_t* stage_vb, TileRegs& load_regs) {
      u32x4 vpre[kLead];
      part_a(kb_next, vb, s_cur, s_next, pw, vpre);
      check_tile(s_cur, pw);
      mask_tile(t + 1, t1, s_next);
      part_b(vb, vpre, pw, s_next, pw_next, [&] { load(role, in_win(t + 3), in_win(t + 2), load_regs); },
             [&](auto qc) { stage_q(role, stage_regs, stage_kb, stage_vb, qc); });
      wait_lds();
      __syncthreads();
    };
    auto idle_step = [&](int t, TileRegs& stage_regs, uint16_t* stage_kb, uint16_t* stage_vb, TileRegs& load_regs) {
      load(role, in_win(t + 3), in_win(t + 2), load_regs);
      stage(role, stage_regs, stage_kb, stage_vb);
      wait_lds();
      __syncthreads();
    };
    // Steps at an even offset from t0 compute S into sb from K buffer 1, read V
    // buffer 0, stage ra into K buffer 0 / V buffer 1 and load into rb; odd
    // steps swap every pair.
    const int t_vis = max(t0, min(t1, (c + m0w + 31) / kBN + 1));
    int t = t0;
    for (; t + 1 < t_vis; t += 2) {
      full_step(t, sa, sb, pa, pb, kbuf1, vbuf0, ra, kbuf0, vbuf1, rb);
      full_step(t + 1, sb, sa, pb, pa, kbuf0, vbuf1, rb, kbuf1, vbuf0, ra);
    }
    if (t < t_vis) {
      full_step(t, sa, sb, pa, pb, kbuf1, vbuf0, ra, kbuf0, vbuf1, rb);
      ++t;
      if (t < t1) {
        idle_step(t, rb, kbuf1, vbuf0, ra);
        ++t;
      }
    }
    for (; t < t1; t += 2) {
      idle_step(t, ra, kbuf0, vbuf1, rb);
      if (t + 1 < t1) idle_step(t + 1, rb, kbuf1, vbuf0, ra);
    }
    t0 = t1;
    if (t0 >= n_tiles) break;
    window_start(std::false_type{});
  }
  };
  if (k_role) tile_loop(std::true_type{});
  else tile_loop(std::false_type{});

  // ---- normalise and store ----------------------------------------------------
  l_run = swap32_pair(l_run, true);  // + lane l ^ 32 (row swap, no LDS round trip)
  if (n_pieces > 1) {
    // A piece of a split item: write this lane's partial (accumulators
    // normalised, fp16; m, l) to the piece's slot; the item's last piece to
    // arrive merges all pieces, in piece order, and stores the output.  The
    // partials are written and read with agent-coherent buffer accesses
    // (sc1: coherent across the XCDs' L2 caches without writing back or
    // invalidating them), and each wave's stores have completed before the
    // arrival is counted.
    constexpr int kLanes = 64 * kPrefillWaves;
    constexpr int kSc1 = 16;  // cache-policy bit sc1 of a buffer access
    const uint32_t slot_bytes = (uint32_t)(kPrefillPartDwords * kLanes * 4);
    const uint32_t piece_stride = (uint32_t)n_groups * slot_bytes;
    const __amdgpu_buffer_rsrc_t pr =
        make_rsrc(p.part + ((int64_t)part_slot * n_groups + grp) * (kPrefillPartDwords * kLanes),
                  (uint32_t)n_pieces * piece_stride);
    {
      const float inv = (l_run > 0.f) ? 1.0f / l_run : 0.f;
      const uint32_t mine = (uint32_t)piece * piece_stride;
#pragma unroll
      for (int w4 = 0; w4 < 8; ++w4) {  // dwords 4 w4 .. 4 w4 + 3: accumulators 8 w4 .. 8 w4 + 7
        const int db = w4 >> 1, i0 = 8 * (w4 & 1);
        const u32x4 hv = {pack_f16x2(acc[db][i0 + 0] * inv, acc[db][i0 + 1] * inv),
                          pack_f16x2(acc[db][i0 + 2] * inv, acc[db][i0 + 3] * inv),
                          pack_f16x2(acc[db][i0 + 4] * inv, acc[db][i0 + 5] * inv),
                          pack_f16x2(acc[db][i0 + 6] * inv, acc[db][i0 + 7] * inv)};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, hv), pr,
                                               (int)(mine + 16u * (uint32_t)(w4 * kLanes + tid)), 0, kSc1);
      }
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, f32x2{m_run, l_run}), pr,
                                            (int)(mine + 32u * 4u * kLanes + 8u * (uint32_t)tid), 0, kSc1);
    }
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores have completed
    __syncthreads();
    if (tid == 0) {
      const int arrived = __hip_atomic_fetch_add(p.counters + (int64_t)counter * n_groups + grp, 1, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
      s_last = (arrived == n_pieces - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    // (m, l) of every piece in one round trip, the first pieces' accumulators
    // in flight behind them, then each piece added while later ones load.
    // The merge is instantiated per piece count and unrolled, so that every
    // load is unconditional, exactly the item's pieces are read, and each wait
    // counts exactly the loads issued after the ones it needs.
    auto ml_off = [&](int j) { return (int)((uint32_t)j * piece_stride + 32u * 4u * kLanes + 8u * (uint32_t)tid); };
    auto acc_off = [&](int j, int w4) { return (int)((uint32_t)j * piece_stride + 16u * (uint32_t)(w4 * kLanes + tid)); };
    auto load_piece = [&](u32x4 (&dst)[8], int j) {
#pragma unroll
      for (int w4 = 0; w4 < 8; ++w4)
        dst[w4] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, acc_off(j, w4), 0, kSc1));
    };
    float L = 0.f;
    auto merge_pieces = [&](auto n_const) {
      constexpr int N = decltype(n_const)::value;
      constexpr int R = N < 3 ? N : 3;  // pieces whose accumulators are in flight (32 VGPRs each)
      f32x2 ml[N];
#pragma unroll
      for (int j = 0; j < N; ++j)
        ml[j] = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(pr, ml_off(j), 0, kSc1));
      u32x4 ring[R][8];
#pragma unroll
      for (int j = 0; j < R; ++j) load_piece(ring[j], j);
      float M = -INFINITY;
#pragma unroll
      for (int j = 0; j < N; ++j) M = fmaxf(M, ml[j].x);
      const float Ms = (M == -INFINITY) ? 0.f : M;
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] = f32x16{};
#pragma unroll
      for (int j = 0; j < N; ++j) {
        u32x4 cur[8];
#pragma unroll
        for (int w4 = 0; w4 < 8; ++w4) cur[w4] = ring[j % R][w4];
        if (j + R < N) load_piece(ring[j % R], j + R);
        const float wj = (ml[j].x == -INFINITY) ? 0.f : ml[j].y * fast_exp2(ml[j].x - Ms);
        L += wj;
#pragma unroll
        for (int w4 = 0; w4 < 8; ++w4) {
          const u32x4 hv = cur[w4];
          const int db = w4 >> 1, i0 = 8 * (w4 & 1);
          const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f16x2 h2 = __builtin_bit_cast(f16x2, hw[e]);
            acc[db][i0 + 2 * e] += wj * (float)h2.x;
            acc[db][i0 + 2 * e + 1] += wj * (float)h2.y;
          }
        }
      }
    };
    static_assert(kPrefillMaxPieces == 8, "one merge instance per piece count 2 .. 8");
    switch (n_pieces) {  // 2 <= n_pieces <= kPrefillMaxPieces (the schedule's bound)
      case 2: merge_pieces(std::integral_constant<int, 2>{}); break;
      case 3: merge_pieces(std::integral_constant<int, 3>{}); break;
      case 4: merge_pieces(std::integral_constant<int, 4>{}); break;
      case 5: merge_pieces(std::integral_constant<int, 5>{}); break;
      case 6: merge_pieces(std::integral_constant<int, 6>{}); break;
      case 7: merge_pieces(std::integral_constant<int, 7>{}); break;
      default: merge_pieces(std::integral_constant<int, 8>{}); break;
    }
    l_run = L;
  }
  // Output through LDS: a lane holds 4-dim pieces of its query row, so
  // storing from registers writes 16 bytes into each of 32 rows 8 KiB apart
  // per instruction.  Each wave writes its 32 x 128 bf16 rows to a region of
  // its own (the tile buffers: every wave passed the last step's barrier, so
  // no wave reads them any more), then stores whole rows: 16 lanes per row,
  // 4 rows per instruction.  A wave reads back only what it wrote, and its
  // LDS accesses complete in order, so no barrier is needed.
  {
    constexpr int kOPitch = kHeadDim + 8;  // bf16 per row in LDS (272 B)
    uint16_t* ob = lds + wave * 32 * kOPitch;
    const float inv = (l_run > 0.f) ? 1.0f / l_run : 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int b4 = 0; b4 < 4; ++b4) {
        const int d = 32 * db + 8 * b4 + 4 * h;
        u32x2 w;
        w.x = QT::out_bits(acc[db][4 * b4 + 0] * inv) | (QT::out_bits(acc[db][4 * b4 + 1] * inv) << 16);
        w.y = QT::out_bits(acc[db][4 * b4 + 2] * inv) | (QT::out_bits(acc[db][4 * b4 + 3] * inv) << 16);
        *reinterpret_cast<u32x2*>(ob + col * kOPitch + d) = w;
      }
    }
    const int chunk = lane & 15;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 4 * j + (lane >> 4);  // row of the wave's 32
      const u32x4 v = *reinterpret_cast<const u32x4*>(ob + r * kOPitch + 8 * chunk);
      const int tr = m0w + r;
      const int64_t grow = (int64_t)q_start + tr;
      if (tr < Lq && grow < p.q_rows)
        *reinterpret_cast<u32x4*>(p.out + (grow * p.Hq + head) * kHeadDim + 8 * chunk) = v;
    }
  }
}

static_assert(sizeof(PrefillItem) == 48, "the host sizes the work list with 48-byte records");

hipError_t launch_varlen_prefill(const PrefillParams& p, const void* schedule, const MqParams& mq, bool merge,
                                 hipStream_t stream) {
  if (p.num_seqs == 0 || p.n_mblocks == 0) return hipSuccess;
  if (p.n_records < (int64_t)p.num_seqs * p.n_mblocks || p.slots_per_group < 1 || p.counters == nullptr ||
      p.part == nullptr)
    return hipErrorInvalidValue;
  const int64_t n_blocks = (int64_t)p.n_records * p.Hkv * p.n_hgroups;
  const int64_t n_merge = merge ? (int64_t)mq.num_seqs * merge_slices(mq, kPrefillWaves) : 0;
  if (n_blocks + n_merge > 0x7fffffff || schedule == nullptr) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(n_blocks + n_merge)), block(64 * kPrefillWaves);
  const PrefillItem* items = static_cast<const PrefillItem*>(schedule);
  const int layout = p.block_tables == nullptr ? 0 : (p.block_size % kBN == 0 ? 1 : 2);
  switch (2 * layout + (p.out_f16 ? 1 : 0)) {
#define NVAMD_VP_CASE(c, PAGED, SMALL, F16)                                                                   \
  case c:                                                                                                     \
    hipLaunchKernelGGL((varlen_prefill_kernel<PAGED, SMALL, F16>), grid, block, 0, stream, p, items, mq,      \
                       (int)n_blocks);                                                                        \
    break;
    NVAMD_VP_CASE(0, false, false, false)
    NVAMD_VP_CASE(1, false, false, true)
    NVAMD_VP_CASE(2, true, false, false)
    NVAMD_VP_CASE(3, true, false, true)
    NVAMD_VP_CASE(4, true, true, false)
    NVAMD_VP_CASE(5, true, true, true)
#undef NVAMD_VP_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace nvamd
