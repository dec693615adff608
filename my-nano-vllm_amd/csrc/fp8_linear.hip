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
// cross-lane exchange; scale = amax / 448 (IEEE fp32 division), 1 when not
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
#include <atomic>

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
#pragma unroll
  for (int s = 1; s < 16; s <<= 1) amax = fmaxf(amax, shfl_xor_f32(amax, s));
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
// tokens): BN = 16 TN WN features, BM = 16 TM WM tokens per workgroup.
template <int WN, int WM, int TN, int TM>
struct GemmTile {
  static constexpr int kWaves = WN * WM;
  static constexpr int kThreads = 64 * kWaves;
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
  static constexpr int kWBlocks = (BN + kFp8Block - 1) / kFp8Block;  // weight-scale rows spanned
  static_assert(kWBytes % (1024 * kWaves) == 0 && kXBytes % (1024 * kWaves) == 0, "whole loads per wave");
  static_assert(BN <= kFp8Block || BN % kFp8Block == 0, "a fragment never straddles two weight blocks");
  static_assert(kWaves >= kSxLoads, "one scale load per wave");
};

template <int WN, int WM, int TN, int TM>
constexpr int64_t gemm_scale_offset() { return 2 * GemmTile<WN, WM, TN, TM>::kStage; }

__host__ __device__ constexpr int64_t round_up_1k(int64_t b) { return (b + 1023) & ~(int64_t)1023; }

// LDS bytes of a launch: two stages (weight tile, activation tile, and per
// token row the dword of x_scale that holds its scale for the K block), then
// the weight scales [kWBlocks, Kc] (bf16, from up to 7 elements earlier,
// rounded up to whole 1 KiB loads).
template <int WN, int WM, int TN, int TM>
int64_t gemm_lds_bytes(int Kc) {
  using T = GemmTile<WN, WM, TN, TM>;
  return 2 * T::kStage + round_up_1k(((int64_t)T::kWBlocks * Kc + 8) * 2);
}

// 8 swizzled fragment bytes -> MFMA operand: row r (16 rows), K-chunk q =
// lane / 16 (32 bytes = granules 2q, 2q + 1 at positions (2q) ^ (r & 7),
// (2q + 1) ^ (r & 7) of the row's 128 bytes).
__device__ __forceinline__ i32x8 read_frag(const uint8_t* rows, int r, int q) {
  const uint8_t* row = rows + r * kFp8Block;
  const u32x4 a = *reinterpret_cast<const u32x4*>(row + 16 * ((2 * q) ^ (r & 7)));
  const u32x4 b = *reinterpret_cast<const u32x4*>(row + 16 * ((2 * q + 1) ^ (r & 7)));
  return i32x8{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

template <int WN, int WM, int TN, int TM, bool F16_OUT>
__global__ __launch_bounds__(64 * WN * WM) void block_gemm_kernel(Fp8GemmParams p) {
  using T = GemmTile<WN, WM, TN, TM>;
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
  const u32x4 rsw =
      rsrc_words(p.w_scale + (sw_first - sw_shift), (uint32_t)((((int64_t)T::kWBlocks * Kc + sw_shift) * 2 + 3) & ~3ll));

  // fetch offsets: load i of this wave covers tile rows 8 (wave + kWaves i) ..
  // + 7; lane l -> row + l / 8, LDS granule position l % 8, global granule
  // (l % 8) ^ (row & 7)
  const int fr = lane >> 3, fp = lane & 7;
  auto w_off = [&](int i, int kc) {
    const int r = 8 * (wave + T::kWaves * i) + fr;
    return (uint32_t)((int64_t)r * p.w_stride + kc * kFp8Block + 16 * (fp ^ (r & 7)));
  };
  auto x_off = [&](int i, int kc) {
    const int r = 8 * (wave + T::kWaves * i) + fr;
    return (uint32_t)((int64_t)r * Kc * kFp8Block + kc * kFp8Block + 16 * (fp ^ (r & 7)));
  };
  // wave w < kSxLoads: token rows 64 w + lane, the dword holding x_scale[row][kc]
  const uint32_t sx_row_off = (uint32_t)((64 * wave + lane) * Kc) * 2u;
  auto issue_stage = [&](int kc, int buf) {
    const uint32_t base = lds0 + (uint32_t)(buf * T::kStage);
#pragma unroll
    for (int i = 0; i < T::kWLoads; ++i)
      dma_load16_keep(rw, w_off(i, kc), base + (uint32_t)(1024 * (wave + T::kWaves * i)));
#pragma unroll
    for (int i = 0; i < T::kXLoads; ++i)
      dma_load16_keep(rx, x_off(i, kc), base + (uint32_t)(T::kWBytes + 1024 * (wave + T::kWaves * i)));
    if (wave < T::kSxLoads)
      dma_load4_keep(rsx, (sx_row_off + 2u * kc) & ~3u, base + (uint32_t)(T::kWBytes + T::kXBytes + 256 * wave));
  };

  // weight scales [kWBlocks x Kc], loaded once
  const uint32_t sw_lds = lds0 + (uint32_t)gemm_scale_offset<WN, WM, TN, TM>();
  for (int i = wave; i < (int)(round_up_1k(((int64_t)T::kWBlocks * Kc + 8) * 2) / 1024); i += T::kWaves)
    dma_load16_keep(rsw, 1024u * i + 16u * lane, sw_lds + 1024u * i);
  issue_stage(0, 0);

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int q = lane >> 4, r16 = lane & 15;
  const uint16_t* sw_rows = reinterpret_cast<const uint16_t*>(smem + gemm_scale_offset<WN, WM, TN, TM>());
  const int wblk = T::BN <= kFp8Block ? 0 : (wn * TN * 16) / kFp8Block;  // the wave's weight block in the tile

  for (int kc = 0; kc < Kc; ++kc) {
    // one barrier per K block: past it, every wave's loads of stage kc have
    // landed and every wave is done reading buffer (kc + 1) & 1 (stage kc - 1),
    // which then receives stage kc + 1 while stage kc is computed
    wait_vmcnt<0>();  // this wave's loads of stage kc (and of the scales)
    lds_barrier();
    if (kc + 1 < Kc) issue_stage(kc + 1, (kc + 1) & 1);
    const uint8_t* st = smem + (kc & 1) * T::kStage;
    const uint8_t* wrows = st + (wn * TN * 16) * kFp8Block;
    const uint8_t* xrows = st + T::kWBytes + (wm * TM * 16) * kFp8Block;
    const uint32_t* sx_dw = reinterpret_cast<const uint32_t*>(st + T::kWBytes + T::kXBytes);
    const float sw = bf16_bits_to_f32(sw_rows[sw_shift + wblk * Kc + kc]);
    float s[TM];
    i32x8 b[TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int row = wm * TM * 16 + 16 * j + r16;
      const uint32_t d = sx_dw[row];
      s[j] = bf16_bits_to_f32((row * Kc + kc) & 1 ? d >> 16 : d & 0xFFFFu) * sw;  // exact
      b[j] = read_frag(xrows + 16 * j * kFp8Block, r16, q);
    }
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const i32x8 a = read_frag(wrows + 16 * i * kFp8Block, r16, q);
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const f32x4 part = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            a, b[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][j][e] = __builtin_fmaf(part[e], s[j], acc[i][j][e]);
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

// Tile configurations, largest first: (WN, WM, TN, TM) -> BN x BM.
//   0: 2 x 4 waves, 8 x 4 fragments -> 256 features x 256 tokens (one
//      workgroup of 8 waves per CU: a K block is ~1 us of MFMA work, about
//      the latency of the next block's loads, which the second buffer hides)
//   1: 2 x 2 waves, 4 x 2 fragments -> 128 x 64
//   2: 4 x 1 waves, 2 x 2 fragments -> 128 x 32
//   3: 2 x 1 waves, 2 x 1 fragments ->  64 x 16
// (A 256 x 128 tile on 4 waves was slower than 1 at every size measured:
// with one wave per SIMD neither the loads nor the FMAs overlap the MFMAs.)
constexpr int kGemmConfigs = 4;
constexpr int kGemmBN[kGemmConfigs] = {256, 128, 128, 64};
constexpr int kGemmBM[kGemmConfigs] = {256, 64, 32, 16};

int64_t config_lds_bytes(int c, int Kc) {
  switch (c) {
    case 0: return gemm_lds_bytes<2, 4, 8, 4>(Kc);
    case 1: return gemm_lds_bytes<2, 2, 4, 2>(Kc);
    case 2: return gemm_lds_bytes<4, 1, 2, 2>(Kc);
    default: return gemm_lds_bytes<2, 1, 2, 1>(Kc);
  }
}

template <int WN, int WM, int TN, int TM, bool F16_OUT>
hipError_t launch_config(const Fp8GemmParams& p, int64_t lds, hipStream_t stream) {
  using T = GemmTile<WN, WM, TN, TM>;
  auto kern = block_gemm_kernel<WN, WM, TN, TM, F16_OUT>;
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

}  // namespace

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
  // the largest tile whose grid still covers the CUs and whose LDS fits;
  // otherwise the smallest tile that fits
  int best = -1;
  for (int c = 0; c < kGemmConfigs; ++c) {
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
    case 0: return launch_config<2, 4, 8, 4, false>(p, lds, stream);
    case 1: return launch_config<2, 4, 8, 4, true>(p, lds, stream);
    case 2: return launch_config<2, 2, 4, 2, false>(p, lds, stream);
    case 3: return launch_config<2, 2, 4, 2, true>(p, lds, stream);
    case 4: return launch_config<4, 1, 2, 2, false>(p, lds, stream);
    case 5: return launch_config<4, 1, 2, 2, true>(p, lds, stream);
    case 6: return launch_config<2, 1, 2, 1, false>(p, lds, stream);
    default: return launch_config<2, 1, 2, 1, true>(p, lds, stream);
  }
}

}  // namespace nvamd
