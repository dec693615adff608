// FP8 paged decode / multi-query attention for gfx950 (split-KV + reduce).
//
// Replaces fp8_paged_attention_decode_kernel (nanovllm/kernels/fp8_attention.py:88-171)
// and serves the short-query (speculative decode, Lq = 1 + drafts) sequences
// that the reference routes through fp8_paged_attention_prefill_kernel
// (fp8_attention.py:209-312 via nanovllm/layers/attention.py:74-93).
//
// Work item = (sequence, kv head, KV partition).  One 256-thread workgroup
// (4 waves) owns one item and packs every query row that reads this kv head
// -- the G = Hq/Hkv heads times Lq query tokens -- as the 16-wide column
// block(s) of its MFMAs, so each KV byte is fetched from HBM once.
//
// Per 16-token chunk a wave computes, in fp32 accumulators:
//     S^T[token][col] = K[token][:] . Q[col][:]      4 x v_mfma_f32_16x16x32_bf16 per column block
//     O^T[dim][col]  += V^T[dim][token] . P^T[token][col]   8 x v_mfma_f32_16x16x16_f16
// The FP8 cache bytes are converted exactly, K to bf16 and V to fp16, with
// v_cvt_scalef32_pk_{bf16,f16}_fp8 (scale 1.0).  fp16 queries (F16) take
// v_mfma_f32_16x16x32_f16 for S with K converted to fp16.  The softmax weights P are
// rounded to fp16 (11-bit significand; the lazy rescale keeps them below
// 2^8), and the row sum adds those rounded weights, so numerator and
// denominator use the same P.
//
// Lane layouts (lane = 16*gam + r, gam in 0..3, r in 0..15):
//   K operand : lane loads 2x16 B of token row r, bytes [16gam + 64h, +16);
//               MFMA c = 2h+hh uses its 8 bytes [8hh, +8) as k-slots 8gam..8gam+7.
//   Q operand : the same dims of query column (16cb + r).
//   S^T result: lane holds tokens 4gam + i (i < 4) for column r -- which is
//               exactly the k-slot layout of the 16x16x16 B operand, so P^T
//               needs no data movement.
//   V operand : lane loads 8 B (dims [8r, +8)) of tokens 4gam..4gam+3; a byte
//               transpose (v_perm_b32) builds MFMA i's row r = dim 8r+i.
//   O^T result: lane holds dims 32gam + 8k + i (k < 4) of column r in MFMA i.
// Every K load instruction reads 64 contiguous bytes of 16 rows and every V
// load instruction reads 4 whole 128-byte rows.  Loads are raw buffer loads
// whose descriptor bounds the chunk's valid rows (rows past the end read 0).
// Three chunks are in flight per wave (triple-buffered registers).
//
// Online softmax works in the log2 domain (exp2 with log2(e) folded into the
// scale); row maxima are reduced across the 4 lane groups with the gfx950
// v_permlane16_swap / v_permlane32_swap exchanges (no LDS traffic).  At the end of a partition the 4 waves are merged through LDS.
// A sequence that fits in one partition is normalised and written directly;
// otherwise the partition writes (m, l, acc) and mq_reduce_kernel merges the
// partitions with the log-sum-exp identity.
#include <atomic>

#include "fp8_common.h"
#include "kernels.h"
#include "mq_merge.h"
#include "prefill_items.h"
#include "lds_dma.h"

namespace nvamd {

namespace {

constexpr int kChunk = 16;
constexpr int kWaves = 4;
constexpr int kPitch = kHeadDim + 4;  // LDS row pitch in floats (conflict-free 16 B writes)

struct ChunkRegs {
  u32x4 k[2];   // K row r, bytes [16gam + 64h, +16)
  u32x2 v[4];   // V rows 4gam + e, bytes [8r, +8)
};

__device__ __forceinline__ void load_chunk(ChunkRegs& cr, __amdgpu_buffer_rsrc_t rk,
                                           __amdgpu_buffer_rsrc_t rv, uint32_t k_off,
                                           uint32_t v_off, uint32_t rs) {
  cr.k[0] = buf_load16(rk, k_off);
  cr.k[1] = buf_load16(rk, k_off + 64u);
#pragma unroll
  for (int e = 0; e < 4; ++e) cr.v[e] = buf_load8(rv, v_off + (uint32_t)e * rs);
}

// 8 fp8 bytes (two dwords) -> 8 bf16 (or fp16 with F16) as four dwords (exact).
template <bool F16>
__device__ __forceinline__ u32x4 fp8x8_to(uint32_t lo, uint32_t hi) {
  using QT = QkType<F16>;
  return u32x4{QT::template k2<false>(lo), QT::template k2<true>(lo), QT::template k2<false>(hi),
               QT::template k2<true>(hi)};
}

__device__ __forceinline__ f16x4 as_f16x4(uint32_t a, uint32_t b) {
  u32x2 t = {a, b};
  return __builtin_bit_cast(f16x4, t);
}

// Two E4M3FN bytes held in the low (HI=false) or high (HI=true) 16 bits of w
// -> two fp16 packed in one dword.  Exact.
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_f16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
}

// max over the 4 lanes {l, l^16, l^32, l^48} (the lane groups holding one
// column), with the gfx950 row-swap exchanges: permlane16/32_swap(x, x)
// leaves each lane holding {x[l], x[l^16]} (resp. x[l^32]) across its two
// results.  The results are copied to scalars before the bit cast:
// __builtin_bit_cast of an ext-vector element lvalue reads element 0.
__device__ __forceinline__ float pair_max(uint32_t lo, uint32_t hi) {
  return fmaxf(__builtin_bit_cast(float, lo), __builtin_bit_cast(float, hi));
}

__device__ __forceinline__ float col_max(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t a0 = a[0], a1 = a[1];
  const uint32_t w = __builtin_bit_cast(uint32_t, pair_max(a0, a1));
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  const uint32_t b0 = b[0], b1 = b[1];
  return pair_max(b0, b1);
}

template <int NCB, bool F16>
__device__ __forceinline__ void attend_chunk(const ChunkRegs& cr, const typename QkType<F16>::V8 (&qop)[NCB][4],
                                             const int (&col_limit)[NCB], int tok0, bool need_mask,
                                             float scale_log2, int gam, float (&m)[NCB],
                                             float (&lsum)[NCB], f32x4 (&acc)[NCB][8]) {
  // ---- S^T = K . Q^T -------------------------------------------------------
  using QT = QkType<F16>;
  typename QT::V8 kop[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    kop[2 * h + 0] = QT::from_bits(fp8x8_to<F16>(cr.k[h].x, cr.k[h].y));
    kop[2 * h + 1] = QT::from_bits(fp8x8_to<F16>(cr.k[h].z, cr.k[h].w));
  }
  f32x4 s[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) a = QT::mfma16(kop[c], qop[cb][c], a);
    s[cb] = a;
  }

  // ---- V^T operands: byte transpose of the 4 token rows, exact fp16 ---------
  f16x4 vop[8];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const uint32_t x0 = half ? cr.v[0].y : cr.v[0].x;
    const uint32_t x1 = half ? cr.v[1].y : cr.v[1].x;
    const uint32_t x2 = half ? cr.v[2].y : cr.v[2].x;
    const uint32_t x3 = half ? cr.v[3].y : cr.v[3].x;
    const uint32_t a01 = __builtin_amdgcn_perm(x0, x1, 0x01050004u);  // [t0d0 t1d0 t0d1 t1d1]
    const uint32_t b01 = __builtin_amdgcn_perm(x0, x1, 0x03070206u);  // [t0d2 t1d2 t0d3 t1d3]
    const uint32_t a23 = __builtin_amdgcn_perm(x2, x3, 0x01050004u);
    const uint32_t b23 = __builtin_amdgcn_perm(x2, x3, 0x03070206u);
    vop[4 * half + 0] = as_f16x4(fp8x2_to_f16x2<false>(a01), fp8x2_to_f16x2<false>(a23));
    vop[4 * half + 1] = as_f16x4(fp8x2_to_f16x2<true>(a01), fp8x2_to_f16x2<true>(a23));
    vop[4 * half + 2] = as_f16x4(fp8x2_to_f16x2<false>(b01), fp8x2_to_f16x2<false>(b23));
    vop[4 * half + 3] = as_f16x4(fp8x2_to_f16x2<true>(b01), fp8x2_to_f16x2<true>(b23));
  }

  // ---- online softmax + O^T += V^T . P^T -----------------------------------
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = s[cb][i] * scale_log2;
    if (need_mask) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (tok0 + 4 * gam + i < col_limit[cb]) ? v[i] : -INFINITY;
    }
    const float mx = col_max(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
    // Lazy rescale: move the reference max only when a score exceeds it by
    // more than 2**kLazyRescaleLog2 (always on a column's first valid chunk).
    const bool grow = mx > m[cb] + kLazyRescaleLog2;
    if (wave_any(grow)) {
      const float m_new = grow ? mx : m[cb];
      const float alpha = grow ? fast_exp2(m[cb] - m_new) : 1.f;
      m[cb] = m_new;
      lsum[cb] *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[cb][i] *= alpha;
    }
    const float m_use = (m[cb] == -INFINITY) ? 0.f : m[cb];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = fast_exp2(v[i] - m_use);
    const uint32_t p01 = pack_f16x2(v[0], v[1]), p23 = pack_f16x2(v[2], v[3]);
    // row sum of the fp16 weights the MFMAs use (v_dot2_f32_f16 against 1.0, 1.0)
    const f16x2 ones = __builtin_bit_cast(f16x2, 0x3c003c00u);
    lsum[cb] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p01), ones, lsum[cb], false);
    lsum[cb] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p23), ones, lsum[cb], false);
    const f16x4 pop = as_f16x4(p01, p23);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      acc[cb][i] = __builtin_amdgcn_mfma_f32_16x16x16f16(vop[i], pop, acc[cb][i], 0, 0, 0);
  }
}

struct SeqGeom {
  int row0, Lq, Lk, kv_row0;  // kv_row0: first K/V row of the sequence (contiguous layout)
  bool active;
};


__device__ __forceinline__ SeqGeom seq_geom(const MqParams& p, int seq) {
  SeqGeom sg;
  if (p.cu_q != nullptr) {
    sg.row0 = p.cu_q[seq];
    sg.Lq = p.cu_q[seq + 1] - sg.row0;
    sg.kv_row0 = p.cu_k[seq];
    sg.Lk = p.cu_k[seq + 1] - sg.kv_row0;
    sg.active = sg.Lq > 0 && sg.Lq <= p.mq_max_q;
  } else {
    sg.row0 = seq;
    sg.Lq = 1;
    sg.kv_row0 = 0;
    sg.Lk = p.context_lens[seq];
    sg.active = true;
  }
  sg.Lk = min(sg.Lk, key_capacity(p));
  return sg;
}

template <bool F16>
__device__ __forceinline__ void store_out_row8(uint16_t* __restrict__ dst, const float* o, float inv) {
  using QT = QkType<F16>;
  u32x4 w;
  w.x = QT::out_bits(o[0] * inv) | (QT::out_bits(o[1] * inv) << 16);
  w.y = QT::out_bits(o[2] * inv) | (QT::out_bits(o[3] * inv) << 16);
  w.z = QT::out_bits(o[4] * inv) | (QT::out_bits(o[5] * inv) << 16);
  w.w = QT::out_bits(o[6] * inv) | (QT::out_bits(o[7] * inv) << 16);
  *reinterpret_cast<u32x4*>(dst) = w;
}

// ---------------------------------------------------------------------------
// LDS staging of the KV stream
// ---------------------------------------------------------------------------
// A workgroup owns HG kv heads (HG = 2 when Hkv is even, else 1), so every
// token row it reads is a contiguous HG*128-byte slice of the cache row.  K
// and V move HBM -> LDS with direct-to-LDS buffer loads (no VGPRs are held
// while a load is in flight): one stage = kTS tokens of K then of V, 8 KiB
// each, every load instruction fetching 1 KiB of whole 128-byte lines.  A
// ring of kStages stages keeps two stages in flight while one is computed.
//
// The stage image in LDS is row-major [kTS rows][HG*128 bytes] with the
// 16-byte granules of each row XOR-swizzled by (row & 7), so the operand
// reads below (16 rows at one column, or 16 lanes along one row) hit
// distinct banks.  The swizzle is applied on the fetch side: lane l of a load
// instruction always lands at LDS offset 16*l and fetches the global granule
// that belongs there.
template <int HG>
struct Stage {
  static constexpr int kTS = 64 / HG;              // tokens per stage
  static constexpr int kRowBytes = HG * kHeadDim;  // bytes of one token row in LDS
  static constexpr int kHalf = kTS * kRowBytes;    // K (or V) bytes per stage: 8 KiB
  static constexpr int kBytes = 2 * kHalf;         // 16 KiB
  static constexpr int kRowsPerLoad = 8 / HG;      // token rows per 1 KiB load instruction
  static constexpr int kLanesPerRow = 8 * HG;      // 16-byte granules per row
  static constexpr int kWavesPerHead = kWaves / HG;
};
constexpr int kStages = 3;
constexpr int kRingBytes = kStages * 16384;

// Makes the compiler wait here for the loads that produced x (an empty asm
// that reads it), so no load of x is still counted as pending inside the
// main loop, where the compiler would otherwise wait for every load in flight.
template <typename T>
__device__ __forceinline__ void consume(const T& x) { asm volatile("" ::"v"(x)); }
__device__ __forceinline__ void consume_i32(int x) { asm volatile("" ::"v"(x)); }

__device__ __forceinline__ u32x4 lds_read16(const uint8_t* a) { return *reinterpret_cast<const u32x4*>(a); }
__device__ __forceinline__ u32x2 lds_read8(const uint8_t* a) { return *reinterpret_cast<const u32x2*>(a); }

}  // namespace

// Work item (partition `part`, kv head group `hg`: heads hg*HG .. hg*HG+HG-1,
// sequence `seq`) of the split-KV kernel.
template <int NCB, int HG, bool F16>
__device__ __forceinline__ void mq_attn(const MqParams& p, const int part, const int hg, const int seq) {
  using S = Stage<HG>;
  using QT = QkType<F16>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kRingBytes];
  const uint32_t lds_smem = wave_uniform((int)lds_addr(smem));

  const SeqGeom sg = seq_geom(p, seq);
  if (!sg.active) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_uniform(tid >> 6);
  const int gam = lane >> 4, r = lane & 15;
  const int G = p.G;
  const int hh = wave / S::kWavesPerHead;        // head of this wave within the group
  const int cw = wave % S::kWavesPerHead;        // its 16-token chunk within each stage
  const int g = hg * HG + hh;                    // kv head of this wave

  const int kv_begin = part * p.part_tokens;
  if (sg.Lk <= 0) {
    // Empty context (graph padding rows): the reference yields NaN here; write 0.
    if (part == 0) {
      for (int idx = tid; idx < sg.Lq * HG * G * (kHeadDim / 8); idx += 256) {
        const int col = idx / (kHeadDim / 8), d8 = idx % (kHeadDim / 8);
        const int qi = col / (HG * G), gh = col - qi * (HG * G);
        const int64_t row = sg.row0 + qi;
        if (row >= p.q_rows) continue;
        u32x4 z = {0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(p.out + (row * p.Hq + hg * HG * G + gh) * kHeadDim + 8 * d8) = z;
      }
    }
    return;
  }
  if (kv_begin >= sg.Lk) return;
  const int kv_end = min(sg.Lk, kv_begin + p.part_tokens);
  const int n_parts = (sg.Lk + p.part_tokens - 1) / p.part_tokens;

  // ---- query operands ------------------------------------------------------
  typename QT::V8 qop[NCB][4];
  int col_limit[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int col = 16 * cb + r;
    const int qi = col / G, gh = col - qi * G;
    const int64_t row = sg.row0 + qi;
    const bool valid = qi < sg.Lq && row < p.q_rows;
    col_limit[cb] = valid ? (sg.Lk - sg.Lq + qi + 1) : 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
      if (valid) {
        const uint16_t* qp = p.q + (row * p.Hq + g * G + gh) * kHeadDim + 16 * gam + 64 * h;
        a = *reinterpret_cast<const u32x4*>(qp);
        b = *reinterpret_cast<const u32x4*>(qp + 8);
      }
      qop[cb][2 * h + 0] = QT::from_bits(a);
      qop[cb][2 * h + 1] = QT::from_bits(b);
    }
  }

  float m[NCB], lsum[NCB];
  f32x4 acc[NCB][8];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    m[cb] = -INFINITY;
    lsum[cb] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[cb][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int64_t rs = (int64_t)p.Hkv * kHeadDim;  // bytes between consecutive token rows
  const int n_st = (kv_end - kv_begin + S::kTS - 1) / S::kTS;  // stages of this partition
  // Masking is needed only on chunks that reach past the smallest visible
  // limit of any column (or past the partition end, whose rows read as 0).
  const int mask_from = min(kv_end, sg.Lk - sg.Lq + 1);
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) col_limit[cb] = min(col_limit[cb], kv_end);

  // ---- fetch side: this wave's two K and two V load instructions per stage --
  // Instruction j (= 2*wave + i) covers stage rows [j*kRowsPerLoad, +kRowsPerLoad);
  // lane l fetches row j*kRowsPerLoad + l/kLanesPerRow, granule
  // (l % kLanesPerRow) ^ (row & 7), and lands at LDS offset j*1024 + 16*l.
  // The wave's rows [wr0, wr0 + kWaveRows) get a descriptor of their own
  // (offsets relative to row wr0): they start at a multiple of kWaveRows
  // (8 or 16) from the partition start, so they lie in one KV block
  // whenever block_size % 16 == 0, even when a stage spans several blocks.
  constexpr int kWaveRows = 2 * S::kRowsPerLoad;
  const int wr0 = wave * kWaveRows;
  uint32_t fetch_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = (2 * wave + i) * S::kRowsPerLoad + lane / S::kLanesPerRow;
    const int gran = (lane % S::kLanesPerRow) ^ (row & 7);
    fetch_off[i] = (uint32_t)(row - wr0) * (uint32_t)rs + 16u * (uint32_t)gran;
  }

  // Cursor of the wave's rows (paged layout): block index w_bi (relative to
  // the partition's first block) and row offset w_off in it.  The
  // partition's block-table entries are loaded once, lane l holding entry
  // first_bi + l (a partition spans at most kMaxPartBlocks blocks, enforced
  // by the host), and read in the loop with v_readlane, so the loop issues
  // no memory reads besides the stages.  Table indices are clamped into the
  // row: entries past the partition are never dereferenced (their stages
  // get zero-length descriptors).
  const bool paged = p.block_tables != nullptr;
  int ld_tok = kv_begin + wr0;  // the wave's first row of the next stage
  int w_bi = 0, w_off = 0, bt_lane = 0;
  if (paged) {
    const int first_bi = kv_begin / p.block_size;
    w_off = kv_begin + wr0 - first_bi * p.block_size;
    while (w_off >= p.block_size) {
      w_off -= p.block_size;
      ++w_bi;
    }
    const int bi = min(first_bi + lane, (int)p.bt_stride - 1);
    bt_lane = p.block_tables[(int64_t)seq * p.bt_stride + bi];
  }
  auto cur_block = [&]() -> int { return __builtin_amdgcn_readlane(bt_lane, min(w_bi, 63)); };

  // Issues this wave's share of the cursor's stage into ring slot `slot`
  // and advances the cursor.  Rows past the partition (or an invalid block)
  // get a zero-length descriptor: the loads are still issued, so every
  // iteration has the same loads in flight, but they read nothing and write
  // zeros.
  auto issue_stage = [&](int slot) {
    int nvalid = max(0, min(kWaveRows, kv_end - ld_tok));
    int64_t row;
    if (paged) {
      const int blk = cur_block();
      row = (int64_t)blk * p.block_size + w_off;
      if (blk < 0 || row + kWaveRows > p.kv_rows) nvalid = 0;
    } else {
      row = (int64_t)sg.kv_row0 + ld_tok;
      if (row < 0 || row + nvalid > p.kv_rows) nvalid = 0;
    }
    if (nvalid == 0) row = 0;
    const int64_t base = (row * p.Hkv + hg * HG) * kHeadDim;
    const uint32_t nbytes = (uint32_t)(nvalid * rs);
    const u32x4 rk = rsrc_words(p.k + base, nbytes);
    const u32x4 rv = rsrc_words(p.v + base, nbytes);
    const uint32_t dst = lds_smem + (uint32_t)(slot * S::kBytes + (2 * wave) * 1024);
    dma_load16(rk, fetch_off[0], dst);
    dma_load16(rk, fetch_off[1], dst + 1024u);
    dma_load16(rv, fetch_off[0], dst + (uint32_t)S::kHalf);
    dma_load16(rv, fetch_off[1], dst + (uint32_t)S::kHalf + 1024u);
    ld_tok += S::kTS;
    w_off += S::kTS;
    while (w_off >= p.block_size) {  // at most kTS / 16 blocks per stage
      w_off -= p.block_size;
      ++w_bi;
    }
  };

  // ---- read side: this wave's operands of one stage --------------------------
  // K: row 16cw + r, logical granules 8hh + gam and 8hh + 4 + gam.
  // V: rows 16cw + 4gam + e, bytes [8r, +8) of head hh.
  uint32_t k_rd[2], v_rd[4];
  {
    const int row = 16 * cw + r;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      k_rd[i] = (uint32_t)(row * S::kRowBytes + 16 * ((8 * hh + 4 * i + gam) ^ (row & 7)));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rv = 16 * cw + 4 * gam + e;
      v_rd[e] = (uint32_t)(S::kHalf + rv * S::kRowBytes + 16 * ((8 * hh + (r >> 1)) ^ (rv & 7)) + 8 * (r & 1));
    }
  }

  // ---- main loop: one stage per iteration, two more in flight --------------
  issue_stage(0);
  issue_stage(1);
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int c = 0; c < 4; ++c) consume(qop[cb][c]);
  consume_i32(bt_lane);
  int tok0 = kv_begin + 16 * cw;
  for (int s = 0; s < n_st; ++s) {
    wait_vmcnt<4>();   // this wave's loads of stage s have landed (stage s+1's 4 may not)
    lds_barrier();     // ... and every wave's; slot (s+2)%3 is no longer being read
    issue_stage((s + 2) % kStages);
    const uint8_t* sl = smem + (s % kStages) * S::kBytes;
    ChunkRegs cr;
    cr.k[0] = lds_read16(sl + k_rd[0]);
    cr.k[1] = lds_read16(sl + k_rd[1]);
#pragma unroll
    for (int e = 0; e < 4; ++e) cr.v[e] = lds_read8(sl + v_rd[e]);
    attend_chunk<NCB, F16>(cr, qop, col_limit, tok0, tok0 + kChunk > mask_from, p.scale_log2, gam, m, lsum,
                           acc);
    tok0 += S::kTS;
  }

  // ---- merge the waves of each head ------------------------------------------
  wait_vmcnt<0>();     // the ring is reused below: no load may still be landing
  lds_barrier();
  float* sm_o = reinterpret_cast<float*>(smem);                      // [4 waves][16][kPitch]
  float* sm_ml = sm_o + kWaves * 16 * kPitch;                         // [4 waves][NCB*16][2]
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    lsum[cb] = swap32_pair(swap16_pair(lsum[cb], true), true);  // once per partition: + lanes l ^ 16, then l ^ 32
    if (gam == 0) {
      sm_ml[(wave * NCB * 16 + 16 * cb + r) * 2 + 0] = m[cb];
      sm_ml[(wave * NCB * 16 + 16 * cb + r) * 2 + 1] = lsum[cb];
    }
  }
  lds_barrier();

  const int c16 = (tid >> 4) & 15;   // output column within the block
  const int d0 = 8 * (tid & 15);     // 8 output dims
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    {
      const int col = 16 * cb + r;
      float M = -INFINITY;
#pragma unroll
      for (int k = 0; k < S::kWavesPerHead; ++k)
        M = fmaxf(M, sm_ml[((hh * S::kWavesPerHead + k) * NCB * 16 + col) * 2]);
      const float Ms = (M == -INFINITY) ? 0.f : M;
      const float sc = fast_exp2(m[cb] - Ms);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float* dst = sm_o + (wave * 16 + r) * kPitch + 32 * gam + 8 * k;
        f32x4 lo = {acc[cb][0][k] * sc, acc[cb][1][k] * sc, acc[cb][2][k] * sc, acc[cb][3][k] * sc};
        f32x4 hi = {acc[cb][4][k] * sc, acc[cb][5][k] * sc, acc[cb][6][k] * sc, acc[cb][7][k] * sc};
        *reinterpret_cast<f32x4*>(dst) = lo;
        *reinterpret_cast<f32x4*>(dst + 4) = hi;
      }
    }
    lds_barrier();
    // 256 threads: 16 columns x 16 dim-octets, repeated for each head of the group.
#pragma unroll
    for (int oh = 0; oh < HG; ++oh) {
      const int col = 16 * cb + c16;
      const int qi = col / G, gh = col - qi * G;
      const int64_t row = sg.row0 + qi;
      if (qi < sg.Lq && row < p.q_rows) {
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < S::kWavesPerHead; ++k)
          M = fmaxf(M, sm_ml[((oh * S::kWavesPerHead + k) * NCB * 16 + col) * 2]);
        const float Ms = (M == -INFINITY) ? 0.f : M;
        float L = 0.f;
#pragma unroll
        for (int k = 0; k < S::kWavesPerHead; ++k) {
          const float* e = sm_ml + ((oh * S::kWavesPerHead + k) * NCB * 16 + col) * 2;
          L += e[1] * fast_exp2(e[0] - Ms);
        }
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float t = 0.f;
#pragma unroll
          for (int k = 0; k < S::kWavesPerHead; ++k)
            t += sm_o[((oh * S::kWavesPerHead + k) * 16 + c16) * kPitch + d0 + e];
          o[e] = t;
        }
        const int64_t rh = row * p.Hq + (hg * HG + oh) * G + gh;
        if (n_parts == 1) {
          const float inv = (L > 0.f) ? 1.0f / L : 0.f;
          store_out_row8<F16>(p.out + rh * kHeadDim + d0, o, inv);
        } else {
          const int64_t pi = rh * p.max_parts + part;
          float* pa = p.part_acc + pi * kHeadDim + d0;
          *reinterpret_cast<f32x4*>(pa) = f32x4{o[0], o[1], o[2], o[3]};
          *reinterpret_cast<f32x4*>(pa + 4) = f32x4{o[4], o[5], o[6], o[7]};
          if (d0 == 0) {
            p.part_ml[2 * pi + 0] = M;
            p.part_ml[2 * pi + 1] = L;
          }
        }
      }
    }
    lds_barrier();
  }
}

template <int NCB, int HG, bool F16>
__global__ __launch_bounds__(256) void paged_mq_attn_kernel(MqParams p) {
  mq_attn<NCB, HG, F16>(p, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Short-query pass of a prefill call, with one more z-slice whose first
// workgroup writes the prefill kernel's work list (the prefill kernel is the
// next launch on the stream).
template <int NCB, int HG, bool F16>
__global__ __launch_bounds__(256) void prefill_short_kernel(MqParams p, PrefillParams pp, PrefillItem* items) {
  if ((int)blockIdx.z == p.num_seqs) {
    __shared__ int sched_lds[kScheduleLdsInts];
    if (blockIdx.x == 0 && blockIdx.y == 0) prefill_schedule(pp, items, sched_lds);
    return;
  }
  mq_attn<NCB, HG, F16>(p, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Decode mode: one wave per (sequence, head).
__global__ __launch_bounds__(256) void mq_reduce_kernel(MqParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t rh = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (rh >= (int64_t)p.num_seqs * p.Hq) return;
  merge_partitions(p, rh, p.context_lens[rh / p.Hq], lane);
}

// Varlen mode: workgroup (sequence, slice), one (row, head) per wave.
__global__ __launch_bounds__(256) void mq_reduce_varlen_kernel(MqParams p) {
  const int slices = merge_slices(p, 4);
  const int seq = (int)blockIdx.x / slices, slice = (int)blockIdx.x - seq * slices;
  merge_varlen_one(p, seq, slice * 4 + (int)(threadIdx.x >> 6), threadIdx.x & 63);
}

// ---------------------------------------------------------------------------
// Balanced decode: stream-K over KV stages
// ---------------------------------------------------------------------------
// Pure decode (one query row per sequence) with Hkv % 4 == 0, and the
// short-query sequences of a paged varlen call (speculative-decode rows:
// the Lq * G <= 32 query rows of a kv head are its MFMA columns, each with
// its causal key limit; other sequences take no stages).  A pair =
// (sequence b, group hg of HG kv heads; HG = 8 for decode when Hkv % 8 == 0, else 4);
// its n_b = ceil(L_b / 16) stages of 16 tokens are laid end to end in
// (b, hg) order, T stages in all.  Workgroup w of a persistent grid of W
// (as many as stay resident) streams a fixed share of about T/W stages
// (sk_range_start: in decode a little more on the faster even-numbered
// XCDs), so the work
// per workgroup does not depend on the context lengths; the uneven
// per-sequence workgroups of paged_mq_attn_kernel leave the machine half
// idle at the end of a batch.  Wave i owns kv head HG*hg + i and all
// 16 tokens of each stage (a 128-byte slice of each token row; with HG = 8
// a stage row is a whole 1 KiB cache row), so no cross-wave merge is
// needed.  A pair inside one range is finished by its workgroup; a pair cut
// by range boundaries leaves (acc, m, l) per workgroup in the workspace
// (slot 0: the range's first pair, slot 1: its last) and
// decode_sk_merge_kernel combines them.  Block-table entries and context
// lengths are scalar loads and, with QL, the queries arrive in LDS with the
// first stage of each pair, so pair boundaries do not drain the pipeline.

// Wave-uniform read through the scalar data cache (constant address space:
// the tables are not written while the kernel runs).
__device__ __forceinline__ int sload_i32(const int32_t* base, int64_t i) {
  return ((const __attribute__((address_space(4))) int32_t*)base)[i];
}


__device__ __forceinline__ int sk_capacity(const MqParams& p) {
  return (int)min(p.bt_stride * (int64_t)p.block_size, (int64_t)0x7fffffff);
}

__device__ __forceinline__ int sk_stages(int L) { return L > 0 ? (L + kSkStageTokens - 1) / kSkStageTokens : 0; }

// Keys of sequence b in the stage space: its context (decode) or, in varlen
// mode, its key count when it is a short-query sequence (1 <= Lq <=
// mq_max_q); the other sequences take no stages.  SCALAR reads the tables
// through the scalar data cache (b wave-uniform).
template <bool SCALAR>
__device__ __forceinline__ int sk_seq_len(const MqParams& p, int b, int cap) {
  auto rd = [&](const int32_t* t, int i) { return SCALAR ? sload_i32(t, i) : t[i]; };
  if (p.cu_q == nullptr) return min(rd(p.context_lens, b), cap);
  const int lq = rd(p.cu_q, b + 1) - rd(p.cu_q, b);
  if (lq <= 0 || lq > p.mq_max_q) return 0;
  return max(0, min(rd(p.cu_k, b + 1) - rd(p.cu_k, b), cap));
}

// Stage of the balanced kernel: 16 token rows of HG*128 bytes (K, then V),
// fetched by 64*HG lanes as 2*HG 1 KiB direct-to-LDS loads per half.  With
// QL the slot also has room for the queries of the HG kv heads (G <=
// kSkQMaxG), loaded with the first stage of each pair.
constexpr int kSkQMaxG = 8;
constexpr int kSkDepth = 3;            // stages per ring, at most
constexpr int kSkLdsBytes = 160 * 1024;  // LDS per CU
template <int HG, bool QL>
struct SkStage {
  static constexpr int kTS = kSkStageTokens;
  static constexpr int kRowBytes = HG * kHeadDim;
  static constexpr int kHalf = kTS * kRowBytes;      // 8 KiB (HG 4) or 16 KiB (HG 8)
  static constexpr int kBytes = 2 * kHalf;
  static constexpr int kQBytes = QL ? HG * kSkQMaxG * kHeadDim * 2 : 0;
  static constexpr int kSlot = kBytes + kQBytes;
  static constexpr int kRowsPerLoad = 8 / HG;
  static constexpr int kLanesPerRow = 8 * HG;
  // stages in the ring (kDepth - 1 in flight): kSkDepth, or fewer if the LDS cannot hold them
  static constexpr int kDepth = kSkDepth * kSlot <= kSkLdsBytes ? kSkDepth : kSkLdsBytes / kSlot;
  static_assert(kDepth >= 3, "ring of at least three stages");
  static constexpr int kRing = kDepth * kSlot;
};

// Granule swizzle of stage row r (0..15): granule g of the row sits at
// position g ^ sk_swz(r).  Rows are 512 or 1024 bytes, so every row starts on
// the same LDS banks and the swizzle alone spreads the reads.  A K read takes
// granules {c, c + 1} (or {c + 2, c + 3}) of rows 0..15 in 32 lanes:
// sk_swz(r) >> 1 == r, so the 32 positions are distinct mod 32 granules
// (512 bytes), and sk_swz(r) & 15 is a permutation of 0..15, so each 16-lane
// half is distinct mod 16 too.  A V read takes rows e, e+4, e+8, e+12 (8
// bytes of one granule column each): their swizzles differ in bits 3..4, so
// the four rows sit on four different 128-byte lines of a 512-byte window.
// Bits 0..2 permute within a 128-byte line and bits 3..4 move whole lines, so
// each 8-lane group of a fetch still reads one whole 128-byte line.
// (r & 7) put 32 lanes of a K read on 8 positions: a 4-way bank conflict.
__device__ __forceinline__ int sk_swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1) | ((r & 8) << 1); }

// A prefill call with long sequences launches one workgroup more (index
// sk_wgs, resident beside the sk_wgs stream-K workgroups) that writes the
// prefill kernel's work list (items != nullptr).
template <int NCB, int HG, bool QL, bool F16>
__global__ __launch_bounds__(64 * HG) void decode_sk_kernel(MqParams p, PrefillParams pp, PrefillItem* items) {
  using S = SkStage<HG, QL>;
  using QT = QkType<F16>;
  static_assert(HG == 4 || HG == 8, "4 or 8 kv heads per workgroup");
  static_assert(!QL || NCB == 1, "queries through LDS for G <= 8 only");
  constexpr int kRingBytes = S::kRing;
  static_assert(kRingBytes >= 4 * kScheduleLdsInts, "the schedule borrows the ring");
  __shared__ __attribute__((aligned(16))) uint8_t smem[kRingBytes];
  if (items != nullptr && (int)blockIdx.x == p.sk_wgs) {
    prefill_schedule(pp, items, reinterpret_cast<int*>(smem));
    return;
  }
  const uint32_t lds_smem = wave_uniform((int)lds_addr(smem));
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_uniform(tid >> 6);
  const int gam = lane >> 4, r = lane & 15;
  const int G = p.G;
  const int NHG = p.Hkv / HG;
  const int B = p.num_seqs;
  const int W = p.sk_wgs;
  const int w = blockIdx.x;
  constexpr int kThreads = 64 * HG;
  const int cap = sk_capacity(p);

  // ---- stage prefix over the sequences, built in the (still idle) ring -------
  int* pre = reinterpret_cast<int*>(smem);                 // pre[b] = sum of n_b' for b' < b
  int* lens = pre + (B + 1);                               // lens[b] = L_b (clamped)
  int* wtot = pre + (kRingBytes / 4 - 8);                  // per-wave totals of a chunk (HG <= 8)
  if (tid == 0) pre[0] = 0;
  int carry = 0;
  for (int base = 0; base < B; base += kThreads) {
    const int b = base + tid;
    const int L = (b < B) ? sk_seq_len<false>(p, b, cap) : 0;
    if (b < B) lens[b] = L;
    const int n = sk_stages(L);
    const int incl = wave_incl_scan(n);  // DPP row shifts and readlane, no LDS round trip
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
    int wb = carry;
    for (int k = 0; k < wave; ++k) wb += wtot[k];
    if (b < B) pre[b + 1] = wb + incl;
#pragma unroll
    for (int k = 0; k < HG; ++k) carry += wtot[k];
    __syncthreads();
  }
  const int64_t T = (int64_t)NHG * carry;
  if (w == 0)
    for (int b = tid; b <= B; b += kThreads) p.sk_prefix[b] = pre[b];
  // this workgroup's share of the stages (sk_range_start)
  int64_t start, end;
  {
    const int a = sk_even_weight(p);
    if (sk_fits32(T, W, a)) {
      start = sk_range_start<uint32_t>(w, (uint32_t)T, W, a);
      end = sk_range_start<uint32_t>(w + 1, (uint32_t)T, W, a);
    } else {
      start = (int64_t)sk_range_start<uint64_t>(w, T, W, a);
      end = (int64_t)sk_range_start<uint64_t>(w + 1, T, W, a);
    }
  }
  if (start >= end) return;
  // first pair: the last sequence b0 with NHG * pre[b0] <= start
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int64_t)NHG * pre[mid] <= start) lo = mid;
    else hi = mid - 1;
  }
  const int b0 = lo;
  const int n0 = pre[b0 + 1] - pre[b0];
  const int64_t rem = start - (int64_t)NHG * pre[b0];
  const int hg0 = (rem >> 32) == 0 ? (int)((uint32_t)rem / (uint32_t)n0) : (int)(rem / n0);
  const int o0 = (int)(rem - (int64_t)hg0 * n0);
  const int n_w = (int)(end - start);
  const int L0 = lens[b0];
  // varlen: the first pair's query rows, read here so that the read overlaps
  // the block-table reads of the first stage
  int q0_first = b0, lq_first = 1;
  if (p.cu_q != nullptr) {
    q0_first = sload_i32(p.cu_q, b0);
    lq_first = sload_i32(p.cu_q, b0 + 1) - q0_first;
  }
  __syncthreads();  // the prefix is read; the ring is about to be filled

  const int64_t rs = (int64_t)p.Hkv * kHeadDim;  // bytes between token rows

  // ---- fetch side: 1 KiB loads of whole HG*128-byte row slices, swizzled by row
  uint32_t fetch_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = (2 * wave + i) * S::kRowsPerLoad + lane / S::kLanesPerRow;
    const int gran = (lane % S::kLanesPerRow) ^ sk_swz(row);
    fetch_off[i] = (uint32_t)row * (uint32_t)rs + 16u * (uint32_t)gran;
  }

  // Issue cursor: pair (ib, ihg), stage io of in_ in it, sequence length
  // iL; block ibi of the sequence holds the stage at row offset ioff, and
  // blk_cur / blk_nxt are the table entries of blocks ibi and ibi + 1 (the
  // next one is read a block ahead).  Table entries and context lengths are
  // scalar loads, so they never wait for the stage loads in flight.
  int ib = b0, ihg = hg0, io = o0, in_ = n0;
  int iL = L0;
  int ibi = 0, ioff = 0, blk_cur = 0, blk_nxt = 0;
  auto seek_block = [&]() {  // block entries for stage io of sequence ib
    const int tok = io * kSkStageTokens;
    ibi = tok / p.block_size;
    ioff = tok - ibi * p.block_size;
    const int64_t row0 = (int64_t)ib * p.bt_stride;
    blk_cur = sload_i32(p.block_tables, row0 + ibi);
    blk_nxt = sload_i32(p.block_tables, row0 + min(ibi + 1, (int)p.bt_stride - 1));
  };
  // next pair with stages (only called while stages remain in the range)
  auto next_pair = [&](int& b, int& hg, int& n, int& L) {
    if (++hg == NHG) {
      hg = 0;
      do {
        ++b;
        L = (b < B) ? sk_seq_len<true>(p, b, cap) : 0;
        n = sk_stages(L);
      } while (n == 0 && b < B - 1);
    }
  };
  int issued = 0;
  bool q_due = true;  // the next stage issued is the first of a pair in this range
  auto issue_stage = [&](int slot) {
    int nvalid = 0;
    int64_t row = 0;
    const bool live = issued < n_w;
    if (live) {
      nvalid = min(kSkStageTokens, iL - io * kSkStageTokens);
      row = (int64_t)blk_cur * p.block_size + ioff;
      if (blk_cur < 0 || row + kSkStageTokens > p.kv_rows) nvalid = 0;
      if (QL && q_due) {
        // the pair's queries (HG*G rows of 256 bytes, contiguous) into the
        // slot's query area, before the stage: its wait covers them
        const int n_q = HG * G * kHeadDim * 2 / 1024;  // 1 KiB loads (2G)
        const u32x4 rq = rsrc_words(p.q + ((int64_t)ib * p.Hq + (int64_t)ihg * HG * G) * kHeadDim,
                                    (uint32_t)(n_q * 1024));
        const uint32_t qdst = lds_smem + (uint32_t)(slot * S::kSlot + S::kBytes);
        for (int j = wave; j < n_q; j += HG) dma_load16(rq, 1024u * j + 16u * lane, qdst + 1024u * j);
      }
      q_due = false;
    }
    if (nvalid <= 0) {
      nvalid = 0;
      row = 0;
    }
    const int64_t base = (row * p.Hkv + ihg * HG) * kHeadDim;
    const uint32_t nbytes = (uint32_t)(nvalid * rs);
    const u32x4 rk = rsrc_words(p.k + base, nbytes);
    const u32x4 rv = rsrc_words(p.v + base, nbytes);
    const uint32_t dst = lds_smem + (uint32_t)(slot * S::kSlot + (2 * wave) * 1024);
    dma_load16(rk, fetch_off[0], dst);
    dma_load16(rk, fetch_off[1], dst + 1024u);
    dma_load16(rv, fetch_off[0], dst + (uint32_t)S::kHalf);
    dma_load16(rv, fetch_off[1], dst + (uint32_t)S::kHalf + 1024u);
    if (live) {
      ++issued;
      if (++io == in_) {
        if (issued < n_w) {
          next_pair(ib, ihg, in_, iL);
          io = 0;
          seek_block();
          q_due = true;
        }
      } else if ((ioff += kSkStageTokens) == p.block_size) {
        ioff = 0;
        ++ibi;
        blk_cur = blk_nxt;
        blk_nxt = sload_i32(p.block_tables, (int64_t)ib * p.bt_stride + min(ibi + 1, (int)p.bt_stride - 1));
      }
    }
  };

  // ---- read side: head `wave`, token row r of the stage ------------------------
  uint32_t k_rd[2], v_rd[4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
    k_rd[i] = (uint32_t)(r * S::kRowBytes + 16 * ((8 * wave + 4 * i + gam) ^ sk_swz(r)));
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int rv = 4 * gam + e;
    v_rd[e] = (uint32_t)(S::kHalf + rv * S::kRowBytes + 16 * ((8 * wave + (r >> 1)) ^ sk_swz(rv)) + 8 * (r & 1));
  }

  // ---- compute cursor: pair (cb_s, chg), stage co of cn, length cL -------------
  int cb_s = b0, chg = hg0, co = o0, cn = n0;
  int cL = L0;
  bool first_seg = true;
  int seg_o0 = o0;
  typename QT::V8 qop[NCB][4];
  int col_limit[NCB];
  int64_t col_row[NCB];  // output / query element offset of the lane's column, -1 if unused
  int mask_from = 0;     // first key position that some column of the pair cannot see
  float m[NCB], lsum[NCB];
  f32x4 acc[NCB][8];
  // New pair: reset the softmax state; the queries are read here from
  // global memory (!QL: the wait drains the stages in flight) or, with QL,
  // from the query area of the pair's first stage once it has landed.
  // Column c of kv head kvh is query row c / G (of the sequence's Lq rows;
  // Lq = 1 in decode) of head kvh * G + c % G, and sees the keys before
  // L - Lq + 1 + c / G (causal within the new rows).
  bool q_from_lds = false;
  auto begin_pair = [&]() {
    const int kvh = chg * HG + wave;
    int64_t q0 = cb_s;
    int lq = 1;
    if (p.cu_q != nullptr) {
      if (cb_s == b0) {  // read in the prologue
        q0 = q0_first;
        lq = lq_first;
      } else {
        q0 = sload_i32(p.cu_q, cb_s);
        lq = sload_i32(p.cu_q, cb_s + 1) - (int)q0;
      }
    }
    mask_from = cL - lq + 1;
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const int col = 16 * cb + r;
      const int qr = col / G, j = col - qr * G;
      const bool valid = qr < lq && q0 + qr < p.q_rows;
      col_limit[cb] = valid ? cL - lq + 1 + qr : 0;
      col_row[cb] = valid ? ((q0 + qr) * p.Hq + kvh * G + j) * kHeadDim : -1;
      if (!QL) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
          if (valid) {
            const uint16_t* qp = p.q + col_row[cb] + 16 * gam + 64 * h;
            a = *reinterpret_cast<const u32x4*>(qp);
            b = *reinterpret_cast<const u32x4*>(qp + 8);
          }
          qop[cb][2 * h + 0] = QT::from_bits(a);
          qop[cb][2 * h + 1] = QT::from_bits(b);
        }
      }
      m[cb] = -INFINITY;
      lsum[cb] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[cb][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (!QL) {
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int c = 0; c < 4; ++c) consume(qop[cb][c]);
    }
    q_from_lds = QL;
  };
  // QL: query row (wave * G + col) of the slot's query area, dims 16gam + 64h + 8j.
  auto read_q = [&](const uint8_t* slot_base) {
    const uint8_t* qa = slot_base + S::kBytes;
    const int col = r;  // NCB == 1
    const bool valid = col < G;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        u32x4 a = {0u, 0u, 0u, 0u};
        if (valid) a = lds_read16(qa + (wave * G + col) * (kHeadDim * 2) + (16 * gam + 64 * h + 8 * j) * 2);
        qop[0][2 * h + j] = QT::from_bits(a);
      }
  };
  // Writes the output of a pair finished here, or the partial of a cut pair.
  auto end_segment = [&](bool full) {
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      lsum[cb] = swap32_pair(swap16_pair(lsum[cb], true), true);  // + lanes l ^ 16, then l ^ 32
      const int col = 16 * cb + r;
      if (col_row[cb] < 0) continue;
      if (full) {
        const float inv = (lsum[cb] > 0.f) ? 1.0f / lsum[cb] : 0.f;
        uint16_t* op = p.out + col_row[cb] + 32 * gam;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float o[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = acc[cb][i][k];
          store_out_row8<F16>(op + 8 * k, o, inv);
        }
      } else {
        const int slot = first_seg ? 0 : 1;
        float* ps = p.sk_part + ((((int64_t)w * 2 + slot) * HG + wave) * p.sk_cols + col) * kSkSlotFloats;
        const float inv = (lsum[cb] > 0.f) ? 1.0f / lsum[cb] : 0.f;  // normalised: fp16 holds it
        uint16_t* ph = reinterpret_cast<uint16_t*>(ps);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const u32x4 h8 = {pack_f16x2(acc[cb][0][k] * inv, acc[cb][1][k] * inv),
                            pack_f16x2(acc[cb][2][k] * inv, acc[cb][3][k] * inv),
                            pack_f16x2(acc[cb][4][k] * inv, acc[cb][5][k] * inv),
                            pack_f16x2(acc[cb][6][k] * inv, acc[cb][7][k] * inv)};
          *reinterpret_cast<u32x4*>(ph + 32 * gam + 8 * k) = h8;
        }
        if (gam == 0) {
          ps[kSkSlotMl] = m[cb];
          ps[kSkSlotMl + 1] = lsum[cb];
        }
      }
    }
  };

  constexpr int D = S::kDepth;
  seek_block();
#pragma unroll
  for (int i = 0; i < D - 1; ++i) issue_stage(i);
  begin_pair();  // after the first stages are issued: a global query load overlaps them
  for (int s = 0; s < n_w; ++s) {
    wait_vmcnt<4 * (D - 2)>();  // this wave's loads of stage s have landed (the 4 of each later stage may not)
    lds_barrier();              // ... and every wave's; slot (s-1)%D is no longer being read
    issue_stage((s + D - 1) % D);
    const uint8_t* sl = smem + (s % D) * S::kSlot;
    if (QL && q_from_lds) {
      read_q(sl);
      q_from_lds = false;
    }
    ChunkRegs cr;
    cr.k[0] = lds_read16(sl + k_rd[0]);
    cr.k[1] = lds_read16(sl + k_rd[1]);
#pragma unroll
    for (int e = 0; e < 4; ++e) cr.v[e] = lds_read8(sl + v_rd[e]);
    const int tok0 = co * kSkStageTokens;
    attend_chunk<NCB, F16>(cr, qop, col_limit, tok0, tok0 + kSkStageTokens > mask_from, p.scale_log2, gam, m, lsum,
                           acc);
    if (++co == cn || s == n_w - 1) {
      end_segment(seg_o0 == 0 && co == cn);
      if (s < n_w - 1) {
        next_pair(cb_s, chg, cn, cL);
        co = 0;
        seg_o0 = 0;
        first_seg = false;
        begin_pair();
      }
    }
  }
  wait_vmcnt<0>();  // nothing may land in LDS after the workgroup exits
}

// One wave per (sequence, query row, head): wave -> (sequence b, index of
// its mq_max_q * Hq (row, head) pairs); decode has one row per sequence
// (mq_max_q = 1).
__global__ __launch_bounds__(256) void decode_sk_merge_kernel(MqParams p) {
  // 32-bit indices: the launch checks num_seqs * mq_max_q * Hq < 2^31
  const int gw = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  const int per_seq = p.mq_max_q * p.Hq;
  if (gw >= p.num_seqs * per_seq) return;
  const int b = gw / per_seq;
  sk_merge_one(p, b, gw - b * per_seq, threadIdx.x & 63);
}

// Decode with G <= 4: one wave per (sequence, kv head), its G heads at once.
__global__ __launch_bounds__(256) void decode_sk_merge_heads_kernel(MqParams p) {
  // 32-bit indices: the launch checks num_seqs * Hkv < 2^31
  const int gw = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (gw >= p.num_seqs * p.Hkv) return;
  const int b = gw / p.Hkv;
  sk_merge_heads(p, b, gw - b * p.Hkv, threadIdx.x & 63);
}

namespace {
template <int NCB, int HG, bool QL>
int sk_occupancy() {
  static std::atomic<int> cached{0};  // the kernel's occupancy does not change
  int n = cached.load(std::memory_order_relaxed);
  if (n > 0) return n;
  // the fp16 instances use the same registers and LDS (the workspace size,
  // which depends on the grid, does not depend on the query type)
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_sk_kernel<NCB, HG, QL, false>, 64 * HG, 0) !=
          hipSuccess ||
      n <= 0)
    return 1;  // no device: not cached
  cached.store(n, std::memory_order_relaxed);
  return n;
}

// Instantiation: 0 = <1,4,-> 1 = <2,4,-> 2 = <1,8,QL> 3 = <1,8,-> 4 = <2,8,->
// (queries through LDS only for decode: one query row per sequence)
int sk_variant(int ncb, int hg, int G, bool varlen) {
  if (hg == 4) return ncb == 1 ? 0 : 1;
  if (ncb == 2) return 4;
  return (G <= kSkQMaxG && !varlen) ? 2 : 3;
}
}  // namespace

int decode_sk_wgs_per_cu(int ncb, int hg, int G, bool varlen) {
  switch (sk_variant(ncb, hg, G, varlen)) {
    case 0: return sk_occupancy<1, 4, false>();
    case 1: return sk_occupancy<2, 4, false>();
    case 2: return sk_occupancy<1, 8, true>();
    case 3: return sk_occupancy<1, 8, false>();
    default: return sk_occupancy<2, 8, false>();
  }
}

hipError_t launch_decode_sk(const MqParams& p, int ncb, bool merge, const PrefillParams* pp, void* items,
                            hipStream_t stream) {
  if (p.num_seqs == 0) return hipSuccess;
  const int hg = p.sk_heads;
  const bool varlen = p.cu_q != nullptr;
  if ((hg != 4 && hg != 8) || p.Hkv % hg != 0 || p.num_seqs > kSkMaxSeqs || p.sk_wgs <= 0 ||
      (ncb != 1 && ncb != 2) || p.mq_max_q < 1 || p.G * p.mq_max_q > 16 * ncb || p.sk_cols < p.G * p.mq_max_q ||
      (varlen && p.cu_k == nullptr) || (!varlen && (p.mq_max_q != 1 || p.context_lens == nullptr)))
    return hipErrorInvalidValue;
  const int64_t merge_waves = (int64_t)p.num_seqs * p.mq_max_q * p.Hq;  // one per (row, head)
  if (merge_waves + 3 > 0x7fffffff) return hipErrorInvalidValue;
  const int64_t merge_wgs = (merge_waves + 3) / 4;
  // the work list of a prefill call: one more workgroup
  PrefillParams ppv{};
  PrefillItem* it = nullptr;
  if (items != nullptr) {
    if (pp == nullptr || !varlen || !schedule_params_ok(*pp)) return hipErrorInvalidValue;
    ppv = *pp;
    it = static_cast<PrefillItem*>(items);
  }
  const dim3 grid((unsigned)p.sk_wgs + (it != nullptr ? 1u : 0u)), block((unsigned)(64 * hg));
  switch (2 * sk_variant(ncb, hg, p.G, varlen) + (p.out_f16 ? 1 : 0)) {
#define NVAMD_SK_CASE(c, NCB, HG, QL, F16)                                                                   \
  case c: hipLaunchKernelGGL((decode_sk_kernel<NCB, HG, QL, F16>), grid, block, 0, stream, p, ppv, it); break;
    NVAMD_SK_CASE(0, 1, 4, false, false)
    NVAMD_SK_CASE(1, 1, 4, false, true)
    NVAMD_SK_CASE(2, 2, 4, false, false)
    NVAMD_SK_CASE(3, 2, 4, false, true)
    NVAMD_SK_CASE(4, 1, 8, true, false)
    NVAMD_SK_CASE(5, 1, 8, true, true)
    NVAMD_SK_CASE(6, 1, 8, false, false)
    NVAMD_SK_CASE(7, 1, 8, false, true)
    NVAMD_SK_CASE(8, 2, 8, false, false)
    NVAMD_SK_CASE(9, 2, 8, false, true)
#undef NVAMD_SK_CASE
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (!merge) return hipSuccess;  // the caller's next launch merges
  if (!varlen && p.G <= 4)
    hipLaunchKernelGGL(decode_sk_merge_heads_kernel, dim3((unsigned)(((int64_t)p.num_seqs * p.Hkv + 3) / 4)),
                       dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(decode_sk_merge_kernel, dim3((unsigned)merge_wgs), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_prefill_short(const MqParams& p, int ncb, const PrefillParams& pp, void* items,
                                hipStream_t stream) {
  if (p.num_seqs == 0 || items == nullptr || !schedule_params_ok(pp)) return hipErrorInvalidValue;
  const int hg = (p.Hkv % 2 == 0) ? 2 : 1;  // kv heads per workgroup
  const dim3 grid((unsigned)p.max_parts, (unsigned)(p.Hkv / hg), (unsigned)p.num_seqs + 1u);
  PrefillItem* it = static_cast<PrefillItem*>(items);
  if (ncb != 1 && ncb != 2) return hipErrorInvalidValue;
  switch (4 * (ncb - 1) + 2 * (hg - 1) + (p.out_f16 ? 1 : 0)) {
#define NVAMD_PS_CASE(c, NCB, HG, F16)                                                                        \
  case c: hipLaunchKernelGGL((prefill_short_kernel<NCB, HG, F16>), grid, dim3(256), 0, stream, p, pp, it); break;
    NVAMD_PS_CASE(0, 1, 1, false)
    NVAMD_PS_CASE(1, 1, 1, true)
    NVAMD_PS_CASE(2, 1, 2, false)
    NVAMD_PS_CASE(3, 1, 2, true)
    NVAMD_PS_CASE(4, 2, 1, false)
    NVAMD_PS_CASE(5, 2, 1, true)
    NVAMD_PS_CASE(6, 2, 2, false)
    NVAMD_PS_CASE(7, 2, 2, true)
#undef NVAMD_PS_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_paged_mq(const MqParams& p, int ncb, hipStream_t stream) {
  if (p.num_seqs == 0) return hipSuccess;
  const int hg = (p.Hkv % 2 == 0) ? 2 : 1;  // kv heads per workgroup
  const dim3 grid((unsigned)p.max_parts, (unsigned)(p.Hkv / hg), (unsigned)p.num_seqs);
  if (ncb != 1 && ncb != 2) return hipErrorInvalidValue;
  switch (4 * (ncb - 1) + 2 * (hg - 1) + (p.out_f16 ? 1 : 0)) {
#define NVAMD_MQ_CASE(c, NCB, HG, F16)                                                                   \
  case c: hipLaunchKernelGGL((paged_mq_attn_kernel<NCB, HG, F16>), grid, dim3(256), 0, stream, p); break;
    NVAMD_MQ_CASE(0, 1, 1, false)
    NVAMD_MQ_CASE(1, 1, 1, true)
    NVAMD_MQ_CASE(2, 1, 2, false)
    NVAMD_MQ_CASE(3, 1, 2, true)
    NVAMD_MQ_CASE(4, 2, 1, false)
    NVAMD_MQ_CASE(5, 2, 1, true)
    NVAMD_MQ_CASE(6, 2, 2, false)
    NVAMD_MQ_CASE(7, 2, 2, true)
#undef NVAMD_MQ_CASE
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.max_parts > 1) {
    if (p.cu_q != nullptr) {
      const int64_t wgs = (int64_t)p.num_seqs * merge_slices(p, 4);
      if (wgs > 0x7fffffff) return hipErrorInvalidValue;
      hipLaunchKernelGGL(mq_reduce_varlen_kernel, dim3((unsigned)wgs), dim3(256), 0, stream, p);
    } else {
      const int64_t waves = (int64_t)p.num_seqs * p.Hq;
      hipLaunchKernelGGL(mq_reduce_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, p);
    }
    e = hipGetLastError();
  }
  return e;
}

}  // namespace nvamd
