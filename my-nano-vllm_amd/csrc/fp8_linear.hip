// FP8 block-scaled linear layer for gfx950: dynamic activation quantisation
// and the 128 x 128 block-scaled FP8 GEMM.
//
// Replaces the two Triton kernels of nanovllm/kernels/fp8_linear.py:
//   act_quant_kernel   <- fp8_dyn_quant_kernel  (fp8_linear.py:11-31, launched at :116-123)
//   block_gemm_kernel  <- fp8_block_gemm_kernel (fp8_linear.py:34-71, launched at :125-138)
//
// Quantisation: one 16-lane group per (token m, 128-column group g), the
// token from the workgroup's index; lane j loads 8 consecutive values (one
// 16-byte load).  amax over the group by
// DPP row exchanges; scale = amax / 448 (IEEE fp32 division), 1 when not
// > 0; xq = E4M3FN(clamp(x / scale)) (IEEE division, RNE); the scale is stored
// as bf16 (RNE), x_scale[m, g].  Purely HBM-bound: 2 B read + 1 B written per
// element.
//
// GEMM: out[m, n] = sum_kc P[m, n, kc] * (sx[m, kc] * sw[n / 128, kc]), with
// P the fp32 dot product of one 128-wide K block.  A workgroup computes the
// transposed tile out^T[BN features x BM tokens] as D = W . X^T on
// v_mfma_scale_f32_16x16x128_f8f6f4 (E4M3 operands, unit E8M0 scales): one
// MFMA per 16 x 16 output fragment per K block, so P of a K block is one MFMA
// result, and the lane holding D[n][m] (column m = lane % 16) needs one
// activation scale per fragment column and one weight scale per 128
// features: acc += P * (sx * sw), one FMA per output per K block.  W and X
// tiles ([rows x 128 B] per K block) are staged through LDS by direct-to-LDS
// 16-byte loads, rows' 16-byte granules XOR-swizzled by row so that the
// fragment reads (16 rows, 32 B per lane) are bank-conflict free.  Two stage
// buffers and one barrier per K block: the barrier that publishes stage kc
// also retires stage kc - 1, so stage kc + 1 is issued into its buffer right
// after it and loads while stage kc is computed.  A stage also holds, per
// token row, the x_scale dword with the row's scale for the K block (one
// direct-to-LDS dword load per 64 rows); the weight scales of the tile's
// feature blocks ([kWBlocks x Kc]) are loaded to LDS once.
// A lane feeds the MFMA the bytes of K-chunk lane / 16 (32 bytes) of its row
// in both operands, so any assignment of K positions to (lane, byte) that
// the hardware uses for A it also uses for B, and the sum over K is exact
// up to the MFMA's own fp32 accumulation.
#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>

#include "fp8_common.h"
#include "kernels.h"
#include "lds_dma.h"

namespace nvamd {

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int kFp8Block = 128;  // the reference's BLOCK_SIZE (fp8_linear.py:8)

// ---------------------------------------------------------------------------
// Dynamic activation quantisation
// ---------------------------------------------------------------------------
template <bool F16_IN>
__device__ __forceinline__ float in_to_f32(uint32_t bits16) {
  if constexpr (F16_IN) return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  return bf16_bits_to_f32(bits16);
}

// Grid (M, ceil(Kc / 16)): workgroup (m, y) quantises groups 16 y .. 16 y + 15
// of token m, one 16-lane group each, so no lane divides.
template <bool F16_IN>
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                        uint8_t* __restrict__ xq, uint16_t* __restrict__ x_scale,
                                                        int64_t M, int Kc) {
  const int64_t m = blockIdx.x;
  const int g = 16 * (int)blockIdx.y + (int)(threadIdx.x >> 4);  // 128-column group of the token
  const int j = (int)(threadIdx.x & 15);
  if (g >= Kc) return;  // whole 16-lane groups
  const u32x4 w = *reinterpret_cast<const u32x4*>(x + m * x_stride + (int64_t)g * kFp8Block + 8 * j);
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = in_to_f32<F16_IN>(d[i] & 0xFFFFu);
    v[2 * i + 1] = in_to_f32<F16_IN>(d[i] >> 16);
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, __builtin_fabsf(v[i]));
  amax = row16_max(amax);  // the group's 16 lanes are one DPP row
  float scale = amax / 448.0f;  // correctly rounded fp32 division
  scale = scale > 0.f ? scale : 1.0f;
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = v[i] / scale;  // clamp and RNE in f32x4_to_fp8x4
  *reinterpret_cast<u32x2*>(xq + m * ((int64_t)Kc * kFp8Block) + (int64_t)g * kFp8Block + 8 * j) =
      u32x2{f32x4_to_fp8x4(y[0], y[1], y[2], y[3]), f32x4_to_fp8x4(y[4], y[5], y[6], y[7])};
  if (j == 0) x_scale[m * Kc + g] = (uint16_t)(pack_bf16x2(scale, 0.f) & 0xFFFFu);
}

// ---------------------------------------------------------------------------
// Block-scaled GEMM
// ---------------------------------------------------------------------------
// Tile shape: WN x WM waves, each TN x TM fragments of 16 x 16 (features x
// tokens): BN = 16 TN WN features, BM = 16 TM WM tokens per workgroup; a ring
// of S stages (S - 1 K blocks in flight while one is computed).
template <int WN, int WM, int TN, int TM, int S = 2>
struct GemmTile {
  static constexpr int kWaves = WN * WM;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kStages = S;
  static constexpr int BN = 16 * TN * WN;
  static constexpr int BM = 16 * TM * WM;
  static constexpr int kWBytes = BN * kFp8Block;   // one K block of the weight tile
  static constexpr int kXBytes = BM * kFp8Block;   // one K block of the activation tile
  static constexpr int kSxLoads = (BM + 63) / 64;   // dword loads (64 rows each) of a K block's activation scales
  static constexpr int kSxBytes = 256 * kSxLoads;
  static constexpr int kStage = kWBytes + kXBytes + kSxBytes;
  static constexpr int kWLoads = kWBytes / 1024 / kWaves;  // 1 KiB loads per wave per stage
  static constexpr int kXLoads = kXBytes / 1024 / kWaves;
  static constexpr int kLoads = kWLoads + kXLoads;
  // A tile whose width neither divides nor is a multiple of the 128-row
  // weight block (96) can straddle two blocks: its fragments then take their
  // scales one by one.
  static constexpr bool kStraddle = kFp8Block % BN != 0 && BN % kFp8Block != 0;
  static constexpr int kWBlocks = (BN + kFp8Block - 1) / kFp8Block + (kStraddle ? 1 : 0);  // weight-scale rows spanned
  static_assert(kWBytes % (1024 * kWaves) == 0 && kXBytes % (1024 * kWaves) == 0, "whole loads per wave");
  static_assert(BN <= kFp8Block || BN % kFp8Block == 0, "tiles wider than a block are whole blocks");
  static_assert(kFp8Block % 16 == 0, "a fragment never straddles two weight blocks");
  static_assert(kWaves >= kSxLoads, "one scale load per wave");
  static_assert(S >= 2, "a ring of at least two stages");
};

template <int WN, int WM, int TN, int TM, int S = 2>
constexpr int64_t gemm_scale_offset() { return (int64_t)S * GemmTile<WN, WM, TN, TM, S>::kStage; }

__host__ __device__ constexpr int64_t round_up_1k(int64_t b) { return (b + 1023) & ~(int64_t)1023; }

// LDS bytes of a launch: S stages (weight tile, activation tile, and per
// token row the dword of x_scale that holds its scale for the K block), then
// the weight scales [kWBlocks, Kc] (bf16, from up to 7 elements earlier,
// rounded up to whole 1 KiB loads).
template <int WN, int WM, int TN, int TM, int S = 2>
int64_t gemm_lds_bytes(int Kc) {
  using T = GemmTile<WN, WM, TN, TM, S>;
  return (int64_t)S * T::kStage + round_up_1k(((int64_t)T::kWBlocks * Kc + 8) * 2);
}

// Granule swizzle of a staged 128-byte row r: granule g sits at position
// g ^ frag_swz(r).  A fragment read takes one granule from each of 16 rows
// (the same g); a 16-byte read of row r at position p covers banks
// 4p + 32 (r & 1) .. + 3, so the 16 rows hit 16 distinct bank groups when the
// even rows, and the odd rows, take 8 distinct positions: (r >> 1) & 7.
// ((r & 7) would put rows r and r + 8 on the same banks.)
__device__ __forceinline__ int frag_swz(int r) { return (r >> 1) & 7; }

// 32 swizzled fragment bytes -> MFMA operand: row r (16 rows), lane group
// q = lane / 16 takes granules q and q + 4 of the row's 128 bytes.  Both
// operands of an MFMA are read this way, so their K positions pair up
// whatever the hardware's lane layout.  Measured (SQ_LDS_BANK_CONFLICT): with
// granules 2q and 2q + 1 every 16-byte read took a 2-way bank conflict
// (4 extra cycles per read), with q and q + 4 none.  That fits an LDS that
// serves such a read 32 lanes (two lane groups) at a time with rows r and
// r + 4 on the same banks: positions q ^ s and (q + 1) ^ s are distinct for
// the swizzles s of rows r, r + 4, r + 8, r + 12 (4 values two apart), while
// 2q ^ s and (2q + 2) ^ s collide.
__device__ __forceinline__ i32x8 read_frag(const uint8_t* rows, int r, int q) {
  const uint8_t* row = rows + r * kFp8Block;
  const u32x4 a = *reinterpret_cast<const u32x4*>(row + 16 * (q ^ frag_swz(r)));
  const u32x4 b = *reinterpret_cast<const u32x4*>(row + 16 * ((q + 4) ^ frag_swz(r)));
  return i32x8{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

template <int WN, int WM, int TN, int TM, int S, bool F16_OUT>
__global__ __launch_bounds__(64 * WN * WM) void block_gemm_kernel(Fp8GemmParams p) {
  using T = GemmTile<WN, WM, TN, TM, S>;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const uint32_t lds0 = wave_uniform((int)lds_addr(smem));
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_uniform(tid >> 6);
  const int wn = wave % WN, wm = wave / WN;
  const int n0 = (int)blockIdx.x * T::BN;
  const int64_t m0 = (int64_t)blockIdx.y * T::BM;
  const int Kc = p.Kc;
  const int rows_x = (int)min((int64_t)T::BM, p.M - m0);  // valid token rows of the tile

  // descriptors: rows past the matrix (tokens >= M) read as zeros
  const u32x4 rw = rsrc_words(p.w + (int64_t)n0 * p.w_stride, (uint32_t)((int64_t)T::BN * p.w_stride));
  const u32x4 rx = rsrc_words(p.xq + m0 * ((int64_t)Kc * kFp8Block), (uint32_t)((int64_t)rows_x * Kc * kFp8Block));
  // scale descriptors end on a whole dword: the bounds check drops a dword
  // that is only partly in range, and an aligned dword never crosses a page
  const int64_t sx_bytes = ((int64_t)rows_x * Kc * 2 + 3) & ~(int64_t)3;
  const u32x4 rsx = rsrc_words(p.x_scale + m0 * Kc, (uint32_t)sx_bytes);
  // weight scales from a 16-byte aligned element (sw_shift elements before the tile's first)
  const int64_t sw_first = (int64_t)(n0 / kFp8Block) * Kc;
  const int sw_shift = (int)(sw_first & 7);
  // kWBlocks rows, or to the array's end (a straddling tile's second row may
  // not exist: the last tile need not straddle)
  const int64_t sw_elems = min((int64_t)T::kWBlocks * Kc + sw_shift, (int64_t)(p.N / kFp8Block) * Kc - (sw_first - sw_shift));
  const u32x4 rsw = rsrc_words(p.w_scale + (sw_first - sw_shift), (uint32_t)((sw_elems * 2 + 3) & ~3ll));

  // fetch offsets: load i of this wave covers tile rows 8 (wave + kWaves i) ..
  // + 7; lane l -> row + l / 8, LDS granule position l % 8, global granule
  // (l % 8) ^ frag_swz(row)
  const int fr = lane >> 3, fp = lane & 7;
  auto w_off = [&](int i, int kc) {
    const int r = 8 * (wave + T::kWaves * i) + fr;
    return (uint32_t)((int64_t)r * p.w_stride + kc * kFp8Block + 16 * (fp ^ frag_swz(r)));
  };
  auto x_off = [&](int i, int kc) {
    const int r = 8 * (wave + T::kWaves * i) + fr;
    return (uint32_t)((int64_t)r * Kc * kFp8Block + kc * kFp8Block + 16 * (fp ^ frag_swz(r)));
  };
  // wave w < kSxLoads: token rows 64 w + lane, the dword holding x_scale[row][kc]
  const uint32_t sx_row_off = (uint32_t)((64 * wave + lane) * Kc) * 2u;
  auto issue_stage = [&](int kc, int buf) {
    const uint32_t base = lds0 + (uint32_t)(buf * T::kStage);
#pragma unroll
    for (int i = 0; i < T::kWLoads; ++i) {
      // a ring tile (S > 2) covers all the tokens, so its weight bytes are
      // read once: non-temporal, leaving the L2 to the activation rows every
      // workgroup of the XCD reads
      if constexpr (S > 2) dma_load16(rw, w_off(i, kc), base + (uint32_t)(1024 * (wave + T::kWaves * i)));
      else dma_load16_keep(rw, w_off(i, kc), base + (uint32_t)(1024 * (wave + T::kWaves * i)));
    }
#pragma unroll
    for (int i = 0; i < T::kXLoads; ++i)
      dma_load16_keep(rx, x_off(i, kc), base + (uint32_t)(T::kWBytes + 1024 * (wave + T::kWaves * i)));
    if (wave < T::kSxLoads)
      dma_load4_keep(rsx, (sx_row_off + 2u * kc) & ~3u, base + (uint32_t)(T::kWBytes + T::kXBytes + 256 * wave));
  };

  // weight scales [kWBlocks x Kc], loaded once
  const uint32_t sw_lds = lds0 + (uint32_t)gemm_scale_offset<WN, WM, TN, TM, S>();
  for (int i = wave; i < (int)(round_up_1k(((int64_t)T::kWBlocks * Kc + 8) * 2) / 1024); i += T::kWaves)
    dma_load16_keep(rsw, 1024u * i + 16u * lane, sw_lds + 1024u * i);
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < Kc) issue_stage(st, st);

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int q = lane >> 4, r16 = lane & 15;
  const uint16_t* sw_rows = reinterpret_cast<const uint16_t*>(smem + gemm_scale_offset<WN, WM, TN, TM, S>());
  // weight block (row of sw_rows) of the wave's fragments: one for the whole
  // wave, or one per fragment when the tile can straddle two blocks
  const int wblk = T::BN <= kFp8Block ? 0 : (wn * TN * 16) / kFp8Block;
  int fblk[TN];
#pragma unroll
  for (int i = 0; i < TN; ++i) fblk[i] = (n0 % kFp8Block + (wn * TN + i) * 16) / kFp8Block;
  // loads of one stage by this wave (waves below kSxLoads issue one more: the
  // wait below is then stricter than needed for them)
  constexpr int kStageLoads = T::kWLoads + T::kXLoads;

  for (int kc = 0; kc < Kc; ++kc) {
    // one barrier per K block: past it, every wave's loads of stage kc have
    // landed and every wave is done reading buffer (kc - 1) % S (stage
    // kc - 1), which then receives stage kc + S - 1 while stage kc is computed
    // (this wave's loads of stage kc, and of the scales, are done when at most
    // the later stages' loads are outstanding; near the end fewer are issued)
    if (kc + S - 2 < Kc) wait_vmcnt<(S - 2) * kStageLoads>();
    else wait_vmcnt<0>();
    lds_barrier();
    if (kc + S - 1 < Kc) issue_stage(kc + S - 1, (kc + S - 1) % S);
    const uint8_t* st = smem + (kc % S) * T::kStage;
    const uint8_t* wrows = st + (wn * TN * 16) * kFp8Block;
    const uint8_t* xrows = st + T::kWBytes + (wm * TM * 16) * kFp8Block;
    const uint32_t* sx_dw = reinterpret_cast<const uint32_t*>(st + T::kWBytes + T::kXBytes);
    const float sw = bf16_bits_to_f32(sw_rows[sw_shift + wblk * Kc + kc]);
    float sx[TM];
    i32x8 b[TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int row = wm * TM * 16 + 16 * j + r16;
      const uint32_t d = sx_dw[row];
      sx[j] = bf16_bits_to_f32((row * Kc + kc) & 1 ? d >> 16 : d & 0xFFFFu);
      b[j] = read_frag(xrows + 16 * j * kFp8Block, r16, q);
    }
    float s[TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) s[j] = sx[j] * sw;  // exact (two bf16 values)
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const i32x8 a = read_frag(wrows + 16 * i * kFp8Block, r16, q);
      float swi = sw;
      if constexpr (T::kStraddle) swi = bf16_bits_to_f32(sw_rows[sw_shift + fblk[i] * Kc + kc]);
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const f32x4 part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            a, b[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
        const float sij = T::kStraddle ? sx[j] * swi : s[j];  // exact
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][j][e] = __builtin_fmaf(part[e], sij, acc[i][j][e]);
      }
    }
  }

  // out[m][n]: lane holds D[4 (lane / 16) + e][lane % 16] of each fragment,
  // i.e. token m = column, features n .. n + 3 (8 contiguous output bytes)
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int64_t m = m0 + wm * TM * 16 + 16 * j + r16;
    if (m >= p.M) continue;
    uint16_t* orow = p.out + m * p.out_stride + n0 + wn * TN * 16 + 4 * q;
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const f32x4 v = acc[i][j];
      const u32x2 o = F16_OUT ? u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])}
                              : u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      *reinterpret_cast<u32x2*>(orow + 16 * i) = o;
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny GEMM (M <= 256 tokens): the weights stream once, into registers
// ---------------------------------------------------------------------------
// With few tokens the weights are nearly all of the bytes (Qwen3-8B gate/up
// at 192 tokens: 100.7 MB of weights, 0.8 MB of activations), and a tile grid
// over (features, tokens) re-reads them per token tile, reads each row 128
// bytes at a time (one K block per stage) and waits for every stage at a
// barrier.  Here a workgroup owns BN = 16 CW features, all tokens (16 MF rows)
// and a range of K blocks, on CW compute waves and LW loader waves:
//  - compute wave w owns features n0 + 16 w .. + 15 and loads its weight rows
//    straight into registers, four K blocks (512 bytes of each row) per batch,
//    two batches in flight; its only vector-memory loads are these, so the
//    compiler's wait counts for them are exact and no barrier waits for them;
//  - the loader waves stage the activation rows of a K block and, per token
//    row, the x_scale dword of the block (direct-to-LDS loads) in a ring of
//    kStages stages, one barrier per K block;
//  - per K block a compute wave runs MF MFMAs (its weight fragment against
//    each 16-token fragment) and the block-scale FMAs.
// A lane feeds the MFMA granules q and q + 4 (q = lane / 16) of its row in
// both operands, so the K positions pair up whatever the hardware's lane
// layout, and each weight load instruction reads 64 contiguous bytes of 16
// rows.  With one K range (splits = 1) the workgroup rounds and stores the
// output; otherwise it stores fp32 partial sums to the workspace, [split][M][N],
// and skinny_reduce_kernel adds them in split order (bit-identical on repeat).
constexpr int kSkinnyBatch = 4;  // K blocks per weight batch

template <int CW, int MF>
struct Skinny {
  static constexpr int LW = MF >= 12 ? 2 : 1;            // loader waves
  static constexpr int kWaves = CW + LW;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int BN = 16 * CW;
  static constexpr int kRows = 16 * MF;                  // token rows of a stage
  static constexpr int kXBytes = kRows * kFp8Block;      // activation rows of one K block
  static constexpr int kXLoads = kXBytes / 1024;         // 1 KiB loads, 8 rows each
  static constexpr int kSxLoads = (kRows + 63) / 64;     // dword loads, 64 rows each
  static constexpr int kStage = kXBytes + 256 * kSxLoads;
  // loader l issues activation loads l, l + LW, ... and, if l == 0, the scale loads
  static constexpr int kLoads0 = (kXLoads + LW - 1) / LW + kSxLoads;
  static constexpr int kLoads1 = kXLoads / LW;
  // stages in the ring: kStages - 1 in flight per loader within vmcnt's 63
  static constexpr int kStages = 1 + 63 / kLoads0 < 4 ? 1 + 63 / kLoads0 : 4;
  static_assert(kXLoads % LW == 0, "activation loads split evenly over the loaders");
  static_assert(kStages >= 2, "at least one stage in flight");
  static_assert(BN <= kFp8Block && kFp8Block % BN == 0, "a workgroup's features lie in one weight block");
};

// LDS bytes of a skinny launch: the ring, then the weight scales of the
// workgroup's K range (bf16, from up to 7 elements earlier, whole 1 KiB loads).
template <int CW, int MF>
int64_t skinny_lds_bytes(int kper) {
  using T = Skinny<CW, MF>;
  return (int64_t)T::kStages * T::kStage + round_up_1k(((int64_t)kper + 8) * 2);
}

template <int CW, int MF, bool PARTIAL>
__global__ __launch_bounds__((64 * Skinny<CW, MF>::kWaves)) void skinny_gemm_kernel(Fp8GemmParams p, int kper,
                                                                                 float* __restrict__ part,
                                                                                 int f16_out) {
  using T = Skinny<CW, MF>;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const uint32_t lds0 = wave_uniform((int)lds_addr(smem));
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_uniform(tid >> 6);
  const int n0 = (int)blockIdx.x * T::BN;
  const int split = (int)blockIdx.y;
  const int Kc = p.Kc;
  const int kc0 = split * kper, kc1 = min(Kc, kc0 + kper);
  const int nk = kc1 - kc0;  // >= 1: the launch has no empty splits
  const int64_t sw_first = (int64_t)(n0 / kFp8Block) * Kc + kc0;
  const int sw_shift = (int)(sw_first & 7);
  const uint32_t sw_off = (uint32_t)(T::kStages * T::kStage);
  const uint16_t* sw_lds = reinterpret_cast<const uint16_t*>(smem + sw_off) + sw_shift;

  if (wave >= CW) {
    // ---- loader waves ------------------------------------------------------
    const int l = wave - CW;
    const u32x4 rx = rsrc_words(p.xq, (uint32_t)(p.M * p.K));
    const u32x4 rsx = rsrc_words(p.x_scale, (uint32_t)((p.M * Kc * 2 + 3) & ~3ll));
    if (l == 0) {
      const u32x4 rsw = rsrc_words(p.w_scale + (sw_first - sw_shift), (uint32_t)(((int64_t)nk + sw_shift) * 2 + 3) & ~3u);
      for (int i = 0; i < (int)(round_up_1k(((int64_t)kper + 8) * 2) / 1024); ++i)
        dma_load16_keep(rsw, 1024u * i + 16u * lane, lds0 + sw_off + 1024u * i);
    }
    const int fr = lane >> 3, fp = lane & 7;
    // Stage kc into slot s.  Stages past the range are issued too (their
    // bytes are never read), so every wait below counts the same loads.
    auto issue_stage = [&](int kc, int s) {
      const uint32_t base = lds0 + (uint32_t)(s * T::kStage);
#pragma unroll
      for (int i0 = 0; i0 < T::kXLoads; i0 += T::LW) {
        const int i = i0 + l;
        const int r = 8 * i + fr;
        dma_load16_keep(rx, (uint32_t)r * (uint32_t)p.K + (uint32_t)kc * kFp8Block + 16u * (uint32_t)(fp ^ frag_swz(r)),
                        base + 1024u * i);
      }
      if (l == 0) {
#pragma unroll
        for (int i = 0; i < T::kSxLoads; ++i) {
          const int r = 64 * i + lane;
          dma_load4_keep(rsx, ((uint32_t)(r * Kc + kc) * 2u) & ~3u, base + (uint32_t)(T::kXBytes + 256 * i));
        }
      }
    };
#pragma unroll
    for (int t = 0; t < T::kStages - 1; ++t) issue_stage(kc0 + t, t);
    const int nk_pad = (nk + 2 * kSkinnyBatch - 1) / (2 * kSkinnyBatch) * (2 * kSkinnyBatch);  // the compute rounds
    for (int k = 0; k < nk_pad; ++k) {
      // stage k has landed once at most the kStages - 2 later stages are in flight
      if (l == 0) wait_vmcnt<(T::kStages - 2) * T::kLoads0>();
      else wait_vmcnt<(T::kStages - 2) * T::kLoads1>();
      lds_barrier();  // publishes stage k; every compute wave is done with stage k - 1
      issue_stage(kc0 + k + T::kStages - 1, (k + T::kStages - 1) % T::kStages);
    }
    wait_vmcnt<0>();  // nothing may land in LDS after the workgroup exits
    return;
  }

  // ---- compute waves -------------------------------------------------------
  const int q = lane >> 4, r16 = lane & 15;
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(p.w + (int64_t)(n0 + 16 * wave) * p.w_stride, (uint32_t)(16 * p.w_stride));
  const uint32_t w_row = (uint32_t)r16 * (uint32_t)p.w_stride + 16u * (uint32_t)q;
  u32x4 wr[2][kSkinnyBatch][2];  // two batches of kSkinnyBatch K blocks, granules q and q + 4
  // Batch b <- K blocks kc .. kc + 3; blocks past the range re-read its last
  // block (unconditional loads keep the compiler's wait counts exact).
  auto load_batch = [&](int b, int kc) {
#pragma unroll
    for (int u = 0; u < kSkinnyBatch; ++u) {
      const uint32_t off = w_row + (uint32_t)min(kc + u, kc1 - 1) * kFp8Block;
      wr[b][u][0] = buf_load16(rw, off);
      wr[b][u][1] = buf_load16(rw, off + 64u);
      // issued in block order everywhere (the prologue too), so the compiler's
      // count of younger loads is the same on every path into the loop
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  f32x4 acc[MF];
#pragma unroll
  for (int j = 0; j < MF; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  load_batch(0, kc0);
  load_batch(1, kc0 + kSkinnyBatch);

  // The loop body is straight-line over 2 kSkinnyBatch blocks (branches in
  // it make the compiler drain every load in flight): blocks k >= nk of the
  // last round use the range's last weight block and the next activation
  // stages with a zero scale, which adds +0 (every operand is finite).
  for (int k0 = 0; k0 < nk; k0 += 2 * kSkinnyBatch) {
#pragma unroll
    for (int t = 0; t < 2 * kSkinnyBatch; ++t) {
      const int k = k0 + t;
      lds_barrier();  // stage k is in LDS
      const uint8_t* st = smem + (k % T::kStages) * T::kStage;
      const uint32_t* sx_dw = reinterpret_cast<const uint32_t*>(st + T::kXBytes);
      float sw = bf16_bits_to_f32(sw_lds[min(k, nk - 1)]);
      asm volatile("" : "+v"(sw));  // read in every block (no branch around it)
      sw = k < nk ? sw : 0.f;
      const u32x4 lo = wr[t / kSkinnyBatch][t % kSkinnyBatch][0], hi = wr[t / kSkinnyBatch][t % kSkinnyBatch][1];
      const i32x8 a = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      const int kc = kc0 + k;
#pragma unroll
      for (int j = 0; j < MF; ++j) {
        const int row = 16 * j + r16;
        const uint32_t d = sx_dw[row];
        const float s = bf16_bits_to_f32((row * Kc + kc) & 1 ? d >> 16 : d & 0xFFFFu) * sw;  // exact
        const i32x8 b = read_frag(st + 16 * j * kFp8Block, r16, q);
        const f32x4 pr = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0,
                                                                          127, 0, 127);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[j][e] = __builtin_fmaf(pr[e], s, acc[j][e]);
      }
      // The block's MFMAs stay before the next barrier (the compiler would
      // sink them all to the end of the unrolled body, every block's operands
      // live at once) and the refill after the batch's last use.
#pragma unroll
      for (int j = 0; j < MF; ++j) asm volatile("" : "+v"(acc[j]));
      __builtin_amdgcn_sched_barrier(0);
      if (t % kSkinnyBatch == kSkinnyBatch - 1)
        load_batch(t / kSkinnyBatch, kc0 + k0 + t + 1 + kSkinnyBatch);  // refill the batch just used
    }
  }

  // lane holds D[4q + e][r16] of fragment j: token 16 j + r16, features
  // n0 + 16 wave + 4q .. + 3
  const int nf = n0 + 16 * wave + 4 * q;
#pragma unroll
  for (int j = 0; j < MF; ++j) {
    const int64_t m = 16 * j + r16;
    if (m >= p.M) continue;
    const f32x4 v = acc[j];
    if (PARTIAL) {
      *reinterpret_cast<f32x4*>(part + ((int64_t)split * p.M + m) * p.N + nf) = v;
    } else {
      const u32x2 o = f16_out ? u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])}
                              : u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      *reinterpret_cast<u32x2*>(p.out + m * p.out_stride + nf) = o;
    }
  }
}

// out[m, n .. n + 3] = round(sum over splits s, in order, of part[s][m][n .. n + 3]);
// one thread per four outputs.
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ part, int splits, int64_t M,
                                                            int N, uint16_t* __restrict__ out, int64_t out_stride,
                                                            int f16_out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = N / 4;
  if (i >= M * per_row) return;
  const int64_t m = i / per_row;
  const int n = (int)(i - m * per_row) * 4;
  const int64_t plane = M * N;
  const float* src = part + m * N + n;
  f32x4 v = *reinterpret_cast<const f32x4*>(src);
  for (int s = 1; s < splits; ++s) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(src + s * plane);
    v = f32x4{v[0] + t[0], v[1] + t[1], v[2] + t[2], v[3] + t[3]};
  }
  const u32x2 o = f16_out ? u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])}
                          : u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  *reinterpret_cast<u32x2*>(out + m * out_stride + n) = o;
}

// Tile configurations, largest first: (WN, WM, TN, TM) -> BN x BM.
//   0: 2 x 4 waves, 8 x 4 fragments -> 256 features x 256 tokens (one
//      workgroup of 8 waves per CU: a K block is ~1 us of MFMA work, about
//      the latency of the next block's loads, which the second buffer hides)
//   1: 2 x 2 waves, 4 x 2 fragments -> 128 x 64
//   2: 4 x 1 waves, 2 x 2 fragments -> 128 x 32
//   3: 2 x 1 waves, 2 x 1 fragments ->  64 x 16
// (A 256 x 128 tile on 4 waves was slower than 1 at every size measured:
// with one wave per SIMD neither the loads nor the FMAs overlap the MFMAs.)
// and, outside that order, for 64 < M <= 192 tokens:
//   4: 2 x 6 waves, 3 x 2 fragments -> 96 x 192 (all the tokens), a ring of 4
//      stages: a K block of 192 tokens is ~0.1 us of MFMA work per CU, so
//      with one stage in flight every block waits a full load round trip;
//      three stages in flight keep the weight stream going, and with N / 96
//      tiles (a multiple of the CUs for Qwen3-8B gate/up) each weight byte is
//      read once.
constexpr int kGemmConfigs = 5;
constexpr int kGemmOrdered = 4;  // configurations 0 .. 3 form the size order
constexpr int kGemmBN[kGemmConfigs] = {256, 128, 128, 64, 96};
constexpr int kGemmBM[kGemmConfigs] = {256, 64, 32, 16, 192};

int64_t config_lds_bytes(int c, int Kc) {
  switch (c) {
    case 0: return gemm_lds_bytes<2, 4, 8, 4>(Kc);
    case 1: return gemm_lds_bytes<2, 2, 4, 2>(Kc);
    case 2: return gemm_lds_bytes<4, 1, 2, 2>(Kc);
    case 3: return gemm_lds_bytes<2, 1, 2, 1>(Kc);
    default: return gemm_lds_bytes<2, 6, 3, 2, 4>(Kc);
  }
}

template <int WN, int WM, int TN, int TM, int S, bool F16_OUT>
hipError_t launch_config(const Fp8GemmParams& p, int64_t lds, hipStream_t stream) {
  using T = GemmTile<WN, WM, TN, TM, S>;
  auto kern = block_gemm_kernel<WN, WM, TN, TM, S, F16_OUT>;
  static std::atomic<int64_t> lds_set{0};  // largest dynamic LDS size granted so far
  if (lds > lds_set.load(std::memory_order_relaxed)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    lds_set.store(lds, std::memory_order_relaxed);
  }
  const dim3 grid((unsigned)(p.N / T::BN), (unsigned)((p.M + T::BM - 1) / T::BM));
  hipLaunchKernelGGL(kern, grid, dim3(T::kThreads), (size_t)lds, stream, p);
  return hipGetLastError();
}

template <int CW, int MF, bool PARTIAL>
hipError_t launch_skinny_kernel(const Fp8GemmParams& p, int splits, int kper, bool f16_out, float* part,
                                hipStream_t stream) {
  using T = Skinny<CW, MF>;
  auto kern = skinny_gemm_kernel<CW, MF, PARTIAL>;
  const int64_t lds = skinny_lds_bytes<CW, MF>(kper);
  static std::atomic<int64_t> lds_set{0};  // largest dynamic LDS size granted so far
  if (lds > lds_set.load(std::memory_order_relaxed)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    lds_set.store(lds, std::memory_order_relaxed);
  }
  const dim3 grid((unsigned)(p.N / T::BN), (unsigned)splits);
  hipLaunchKernelGGL(kern, grid, dim3(T::kThreads), (size_t)lds, stream, p, kper, part, f16_out ? 1 : 0);
  return hipGetLastError();
}

template <int CW, int MF>
hipError_t launch_skinny_t(const Fp8GemmParams& p, int splits, int kper, bool f16_out, float* part,
                           hipStream_t stream) {
  if (splits == 1) return launch_skinny_kernel<CW, MF, false>(p, 1, kper, f16_out, nullptr, stream);
  hipError_t e = launch_skinny_kernel<CW, MF, true>(p, splits, kper, f16_out, part, stream);
  if (e != hipSuccess) return e;
  const int64_t threads = p.M * (p.N / 4);
  hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, part,
                     splits, p.M, p.N, p.out, p.out_stride, f16_out ? 1 : 0);
  return hipGetLastError();
}

// Instances: CW 8 only up to MF 12 (beyond it 10 waves leave too few registers).
constexpr bool skinny_has(int cw, int mf) { return cw != 8 || mf <= 12; }

template <int CW>
hipError_t launch_skinny_cw(const Fp8GemmParams& p, int mf, int splits, int kper, bool f16_out, float* part,
                            hipStream_t stream) {
  switch (mf) {
    case 1: return launch_skinny_t<CW, 1>(p, splits, kper, f16_out, part, stream);
    case 2: return launch_skinny_t<CW, 2>(p, splits, kper, f16_out, part, stream);
    case 4: return launch_skinny_t<CW, 4>(p, splits, kper, f16_out, part, stream);
    case 8: return launch_skinny_t<CW, 8>(p, splits, kper, f16_out, part, stream);
    default:
      if constexpr (skinny_has(CW, 12)) {
        if (mf == 12) return launch_skinny_t<CW, 12>(p, splits, kper, f16_out, part, stream);
        if (mf == 16) return launch_skinny_t<CW, 16>(p, splits, kper, f16_out, part, stream);
      }
      return hipErrorInvalidValue;
  }
}

int64_t skinny_lds(int cw, int mf, int kper) {
  // the ring does not depend on CW
  (void)cw;
  switch (mf) {
    case 1: return skinny_lds_bytes<2, 1>(kper);
    case 2: return skinny_lds_bytes<2, 2>(kper);
    case 4: return skinny_lds_bytes<2, 4>(kper);
    case 8: return skinny_lds_bytes<2, 8>(kper);
    case 12: return skinny_lds_bytes<2, 12>(kper);
    default: return skinny_lds_bytes<2, 16>(kper);
  }
}

}  // namespace

SkinnyPlan fp8_skinny_plan(int64_t M, int64_t N, int Kc, int cus, int64_t workspace_bytes, int64_t lds_limit) {
  SkinnyPlan best;
  if (M < 1 || M > kSkinnyMaxM || N % 128 != 0 || Kc < 1 || (int64_t)Kc * kFp8Block >= (1 << 24) || cus < 1)
    return best;
  // A tile grid that covers the CUs keeps them busier (measured at 192
  // tokens: gate/up, 576 tiles of 128 x 64, 41.8 us against 50 us here); the
  // small-M kernel is for grids that would leave CUs idle (qkv 144 tiles:
  // 27.3 -> 24.3 us; down 96 tiles: 63.7 -> 35.3 us, weights streamed from
  // HBM).
  if ((N / 128) * ((M + 63) / 64) >= cus) return best;
  const int mf = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : M <= 128 ? 8 : M <= 192 ? 12 : 16;
  // Estimated time (us): a workgroup's K blocks are latency-bound, about
  // 0.40 + 0.19 CW us each at 192 tokens (less with fewer token fragments),
  // one round of workgroups per CU; a split adds the partial sums' HBM writes
  // and reads and the reduce launch (about 3 us + 2 x bytes / 5 TB/s).
  double best_t = 0.0;
  for (int cw : {8, 4, 2}) {
    if (!skinny_has(cw, mf)) continue;
    for (int s : {1, 2, 3, 4, 6, 8}) {
      if (s > Kc) break;
      const int kper = (Kc + s - 1) / s;
      const int splits = (Kc + kper - 1) / kper;
      if (splits != s) continue;
      const double part_bytes = splits > 1 ? (double)splits * M * N * 4 : 0.0;
      if (part_bytes > (double)workspace_bytes) continue;
      if (skinny_lds(cw, mf, kper) > lds_limit) continue;
      const double wgs = (double)(N / (16 * cw)) * splits;
      const double rounds = std::ceil(wgs / cus);
      const int nk_pad = (kper + 2 * kSkinnyBatch - 1) / (2 * kSkinnyBatch) * (2 * kSkinnyBatch);
      double t = rounds * nk_pad * (0.40 + 0.19 * cw) * (0.4 + 0.6 * mf / 12.0);
      if (splits > 1) t += 3.0 + 2.0 * part_bytes / 5.0e6;
      if (best.cw == 0 || t < best_t) {
        best_t = t;
        best = SkinnyPlan{cw, mf, splits, kper};
      }
    }
  }
  return best;
}

int64_t fp8_skinny_workspace_bytes(int64_t M, int64_t N, int Kc, int cus, int64_t lds_limit) {
  const SkinnyPlan pl = fp8_skinny_plan(M, N, Kc, cus, INT64_MAX, lds_limit);
  return pl.cw > 0 && pl.splits > 1 ? (int64_t)pl.splits * M * N * 4 : 0;
}

hipError_t launch_fp8_skinny_gemm(const Fp8GemmParams& p, const SkinnyPlan& plan, bool f16_out, float* part,
                                  hipStream_t stream) {
  if (p.M == 0) return hipSuccess;
  if (plan.cw == 0 || !skinny_has(plan.cw, plan.mf) || p.M > 16 * plan.mf || p.N % (16 * plan.cw) != 0 || plan.splits < 1 ||
      (plan.splits > 1 && part == nullptr) || (int64_t)(plan.splits - 1) * plan.kper >= p.Kc ||
      (int64_t)plan.splits * plan.kper < p.Kc)
    return hipErrorInvalidValue;
  switch (plan.cw) {
    case 8: return launch_skinny_cw<8>(p, plan.mf, plan.splits, plan.kper, f16_out, part, stream);
    case 4: return launch_skinny_cw<4>(p, plan.mf, plan.splits, plan.kper, f16_out, part, stream);
    case 2: return launch_skinny_cw<2>(p, plan.mf, plan.splits, plan.kper, f16_out, part, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fp8_act_quant(const void* x, int64_t x_stride, bool f16_in, void* xq, void* x_scale, int64_t M,
                                int64_t K, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const int64_t ys = (K / kFp8Block + 15) / 16;
  if (M > 0x7fffffff || ys > 0xffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)M, (unsigned)ys);
  if (f16_in)
    hipLaunchKernelGGL(act_quant_kernel<true>, grid, dim3(256), 0, stream, (const uint16_t*)x, x_stride, (uint8_t*)xq,
                       (uint16_t*)x_scale, M, (int)(K / kFp8Block));
  else
    hipLaunchKernelGGL(act_quant_kernel<false>, grid, dim3(256), 0, stream, (const uint16_t*)x, x_stride,
                       (uint8_t*)xq, (uint16_t*)x_scale, M, (int)(K / kFp8Block));
  return hipGetLastError();
}

int fp8_gemm_pick_config(int64_t M, int64_t N, int Kc, int cus, int64_t lds_limit) {
  // 64 < M <= 192 with whole 96-feature tiles covering the CUs: the deep-ring
  // tile over all the tokens
  if (M > 64 && M <= kGemmBM[4] && N % kGemmBN[4] == 0 && N / kGemmBN[4] >= cus &&
      config_lds_bytes(4, Kc) <= lds_limit)
    return 4;
  // the largest tile whose grid still covers the CUs and whose LDS fits;
  // otherwise the smallest tile that fits
  int best = -1;
  for (int c = 0; c < kGemmOrdered; ++c) {
    if (N % kGemmBN[c] != 0 || config_lds_bytes(c, Kc) > lds_limit) continue;
    best = c;
    if ((N / kGemmBN[c]) * ((M + kGemmBM[c] - 1) / kGemmBM[c]) >= cus) return c;
  }
  return best;
}

int64_t fp8_gemm_lds_bytes(int config, int Kc) { return config_lds_bytes(config, Kc); }

hipError_t launch_fp8_block_gemm(const Fp8GemmParams& p, int config, bool f16_out, hipStream_t stream) {
  if (p.M == 0) return hipSuccess;
  if (config < 0 || config >= kGemmConfigs || p.N % kGemmBN[config] != 0 || (p.M + kGemmBM[config] - 1) / kGemmBM[config] > 0xffff)
    return hipErrorInvalidValue;
  const int64_t lds = config_lds_bytes(config, p.Kc);
  switch (config * 2 + (f16_out ? 1 : 0)) {
    case 0: return launch_config<2, 4, 8, 4, 2, false>(p, lds, stream);
    case 1: return launch_config<2, 4, 8, 4, 2, true>(p, lds, stream);
    case 2: return launch_config<2, 2, 4, 2, 2, false>(p, lds, stream);
    case 3: return launch_config<2, 2, 4, 2, 2, true>(p, lds, stream);
    case 4: return launch_config<4, 1, 2, 2, 2, false>(p, lds, stream);
    case 5: return launch_config<4, 1, 2, 2, 2, true>(p, lds, stream);
    case 6: return launch_config<2, 1, 2, 1, 2, false>(p, lds, stream);
    case 7: return launch_config<2, 1, 2, 1, 2, true>(p, lds, stream);
    case 8: return launch_config<2, 6, 3, 2, 4, false>(p, lds, stream);
    default: return launch_config<2, 6, 3, 2, 4, true>(p, lds, stream);
  }
}

}  // namespace nvamd
