// Shared device helpers for the gfx950 FP8 paged-attention kernels.
//
// Numerical contract (nanovllm/layers/attention.py:27-31 and
// nanovllm/kernels/fp8_attention.py:147-150,169,311):
//   * KV values are stored as OCP FP8 E4M3FN with scale 1, rounded to nearest
//     even; magnitudes beyond 448 saturate to +-448, NaN stays NaN.
//   * FP8 -> bf16 is exact (every E4M3FN value is a bf16 value), so the MFMA
//     operands carry the cache values unchanged.
//   * Outputs are written as bf16(fp16(x)) for bf16 queries, the reference's
//     double rounding, and as fp16(x) for fp16 queries (out = empty_like(q)).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nvamd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// the vector types of the raw buffer load/store builtins
typedef unsigned int v4u32_t __attribute__((ext_vector_type(4)));
typedef unsigned int v2u32_t __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 128;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// FP8 <-> wider types
// ---------------------------------------------------------------------------

// Two E4M3FN bytes held in the low (HI=false) or high (HI=true) 16 bits of w
// -> two bf16 packed in one dword (element 0 = lower byte).  Exact.
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
  bf16x2 r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
  return __builtin_bit_cast(uint32_t, r);
}

// Four E4M3FN bytes -> bf16 x4 as two dwords.
__device__ __forceinline__ u32x2 fp8x4_to_bf16x4(uint32_t w) {
  u32x2 r;
  r.x = fp8x2_to_bf16x2<false>(w);
  r.y = fp8x2_to_bf16x2<true>(w);
  return r;
}

// Four E4M3FN bytes -> fp16 x4 as two dwords.  Exact: every E4M3FN value
// (|x| <= 448, subnormals down to 2^-9) is an fp16 value.
__device__ __forceinline__ u32x2 fp8x4_to_f16x4(uint32_t w) {
  u32x2 r;
  r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
  r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
  return r;
}

// Saturating clamp applied before the hardware RNE conversion: |x| > 448
// (including inf) -> +-448; NaN passes through unchanged.
__device__ __forceinline__ float e4m3_satfinite(float x) {
  const float ax = __builtin_fabsf(x);
  return (ax > 448.0f) ? __builtin_copysignf(448.0f, x) : x;
}

// Four floats -> four E4M3FN bytes (RNE, satfinite) in one dword.
__device__ __forceinline__ uint32_t f32x4_to_fp8x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_satfinite(a), e4m3_satfinite(b), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_satfinite(c), e4m3_satfinite(d), w, true);
  return (uint32_t)w;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// Two fp32 -> two bf16 (round to nearest even) in one dword: v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Two fp32 -> two fp16 (round to nearest even) in one dword: v_cvt_pk_f16_f32.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

__device__ __forceinline__ f16x8 as_f16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 t = {a, b, c, d};
  return __builtin_bit_cast(f16x8, t);
}

__device__ __forceinline__ f16x8 as_f16x8(u32x4 t) { return __builtin_bit_cast(f16x8, t); }

// 2**x with the bare v_exp_f32 (inputs here are <= 0 or -inf; tiny results
// may flush to zero, which is harmless for softmax weights).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Online softmax keeps a reference maximum per row and only rescales the
// accumulators when a new score exceeds it by more than this many powers of
// two; in between, weights exp2(s - m_ref) stay below 2**8.
constexpr float kLazyRescaleLog2 = 8.0f;

__device__ __forceinline__ bool wave_any(bool pred) {
  return __builtin_amdgcn_ballot_w64(pred) != 0;
}

// The reference stores fp16(acc / l) into a bf16 tensor: fp32 -> fp16 (RNE)
// -> bf16 (RNE).  Returns the bf16 bits.
__device__ __forceinline__ uint32_t out_round_bf16_bits(float x) {
  const _Float16 h = (_Float16)x;
  const float hf = (float)h;
  uint32_t u = __builtin_bit_cast(uint32_t, hf);
  if ((u & 0x7F800000u) == 0x7F800000u) return u >> 16;  // inf / NaN keep their class
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// fp16 output (q and out fp16, empty_like(q) in the reference): fp32 -> fp16
// (RNE) only.  Returns the fp16 bits.
__device__ __forceinline__ uint32_t out_round_f16_bits(float x) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// ---------------------------------------------------------------------------
// The query / output element type of the attention kernels
// ---------------------------------------------------------------------------
// F16 = false: bf16 q, S = K . Q^T on the bf16 MFMAs with K converted to bf16;
// out = bf16(fp16(x)).  F16 = true: fp16 q, the fp16 MFMAs with K converted to
// fp16; out = fp16(x).  Both conversions of the FP8 cache are exact, so in
// either case S is the fp32-accumulated product of the exact q and K values.
template <bool F16>
struct QkType;

template <>
struct QkType<false> {
  using V8 = bf16x8;
  static __device__ __forceinline__ V8 from_bits(u32x4 t) { return __builtin_bit_cast(bf16x8, t); }
  template <bool HI>
  static __device__ __forceinline__ uint32_t k2(uint32_t w) {  // two E4M3FN bytes -> two elements
    return fp8x2_to_bf16x2<HI>(w);
  }
  static __device__ __forceinline__ f32x4 mfma16(V8 a, V8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t out_bits(float x) { return out_round_bf16_bits(x); }
};

template <>
struct QkType<true> {
  using V8 = f16x8;
  static __device__ __forceinline__ V8 from_bits(u32x4 t) { return __builtin_bit_cast(f16x8, t); }
  template <bool HI>
  static __device__ __forceinline__ uint32_t k2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
  static __device__ __forceinline__ f32x4 mfma16(V8 a, V8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t out_bits(float x) { return out_round_f16_bits(x); }
};

// Output rounding chosen at run time (merge passes shared by both types).
__device__ __forceinline__ uint32_t out_bits_rt(float x, bool f16) {
  return f16 ? out_round_f16_bits(x) : out_round_bf16_bits(x);
}

// ---------------------------------------------------------------------------
// Wave-level helpers (wave64)
// ---------------------------------------------------------------------------

__device__ __forceinline__ float shfl_xor_f32(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// Cross-lane moves inside a 16-lane DPP row: rotations by 8 and 4 and
// swaps within quads, all VALU (no LDS round trip as with __shfl_xor).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppRor8 = 0x128, kDppRor4 = 0x124, kDppXor2 = 0x4E, kDppXor1 = 0xB1;

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, dpp_u32<CTRL>(__builtin_bit_cast(uint32_t, v)));
}

// sum / maximum over the 16 lanes of a row, in every lane
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<kDppRor8>(x);  // lanes i, i + 8
  x += dpp_f32<kDppRor4>(x);  // + i + 4, i + 12
  x += dpp_f32<kDppXor2>(x);  // + the other pair of the quad
  return x + dpp_f32<kDppXor1>(x);
}
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_f32<kDppRor8>(x));
  x = fmaxf(x, dpp_f32<kDppRor4>(x));
  x = fmaxf(x, dpp_f32<kDppXor2>(x));
  return fmaxf(x, dpp_f32<kDppXor1>(x));
}

// max / sum over the 64 lanes of a wave, in every lane: DPP inside each row,
// then the gfx950 row swaps (permlane16/32_swap(x, x) leave a lane holding
// x[l] and x[l ^ 16], resp. x[l ^ 32], in its two results).
__device__ __forceinline__ float swap16_pair(float x, bool sum) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float a0 = __builtin_bit_cast(float, (uint32_t)a[0]), a1 = __builtin_bit_cast(float, (uint32_t)a[1]);
  return sum ? a0 + a1 : fmaxf(a0, a1);
}
__device__ __forceinline__ float swap32_pair(float x, bool sum) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float a0 = __builtin_bit_cast(float, (uint32_t)a[0]), a1 = __builtin_bit_cast(float, (uint32_t)a[1]);
  return sum ? a0 + a1 : fmaxf(a0, a1);
}
__device__ __forceinline__ float wave_max_f32(float x) { return swap32_pair(swap16_pair(row16_max(x), false), false); }
__device__ __forceinline__ float wave_sum_f32(float x) { return swap32_pair(swap16_pair(row16_sum(x), true), true); }

// lane j's value, in every lane (j wave-uniform)
__device__ __forceinline__ float readlane_f32(float x, int j) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), j));
}

// Inclusive prefix sum over the 64 lanes of a wave: inside each row of 16
// lanes by DPP row shifts (a lane whose source is before its row's start
// adds 0), then the totals of the rows before it (lanes 15, 31, 47) through
// readlane.  No LDS round trip.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  const int row = (int)(threadIdx.x & 63) >> 4;
  const int t0 = __builtin_amdgcn_readlane(x, 15), t1 = __builtin_amdgcn_readlane(x, 31);
  const int t2 = __builtin_amdgcn_readlane(x, 47);
  return x + (row >= 1 ? t0 : 0) + (row >= 2 ? t1 : 0) + (row >= 3 ? t2 : 0);
}

__device__ __forceinline__ int wave_uniform(int v) {
  return __builtin_amdgcn_readfirstlane(v);
}

// ---------------------------------------------------------------------------
// Raw buffer loads: the descriptor's num_records bounds every access, and
// bytes at or past it read as zero (no exec-masked branches around loads).
// All offsets go in the VGPR offset (soffset = 0) so the range check sees them.
// ---------------------------------------------------------------------------

constexpr int kBufferRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_bytes,
                                           kBufferRsrcWord3);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

__device__ __forceinline__ u32x2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

// bf16x8 from four packed dwords.
__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 t = {a, b, c, d};
  return __builtin_bit_cast(bf16x8, t);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 t) {
  return __builtin_bit_cast(bf16x8, t);
}

}  // namespace nvamd
