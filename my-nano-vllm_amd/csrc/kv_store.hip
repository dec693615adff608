// FP8 E4M3FN KV-cache store / quantise for gfx950.
//
// Replaces store_kvcache_kernel (nanovllm/layers/attention.py:11-31): for
// every token i with slot_mapping[i] != -1, the D = Hkv*head_dim bf16 (or fp16)
// values of key[i] and value[i] are rounded to E4M3FN and written to
// cache[slot*D : slot*D + D].  Both 16-bit types widen to fp32 exactly, so the
// one RNE, saturating fp32 -> E4M3FN conversion rounds the value itself.
//
// Design: purely HBM-bound (2 B read + 1 B written per element).  A lane
// converts 16 consecutive elements of one row at a time: two 16-byte loads,
// eight v_cvt_pk_fp8_f32 and one 16-byte store, so a wave moves 1 KiB of
// bf16 per load instruction.  Lanes of a wave cover consecutive 16-element
// chunks of the same row (K row, then the V row), so every load/store
// instruction is fully coalesced.  Rows of a multiple of 32 elements take the
// two-chunk kernel (twice the loads in flight per lane); a conversion-free
// copy with its access pattern moves the 8,192-token, 8-KV-head store only
// ~2% faster.  Cache offsets are 64-bit (the reference's int32 slot*D wraps
// once slot*D >= 2**31).
#include "fp8_common.h"
#include "kernels.h"

namespace nvamd {

// One 16-bit element (bf16, or fp16 with F16) -> fp32, exact.
template <bool F16>
__device__ __forceinline__ float h16_to_f32(uint32_t bits16) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  else return bf16_bits_to_f32(bits16);
}

// Four 16-bit elements (two dwords) -> four E4M3FN bytes (RNE, satfinite).
template <bool F16>
__device__ __forceinline__ uint32_t quantize4(uint32_t lo, uint32_t hi) {
  return f32x4_to_fp8x4(h16_to_f32<F16>(lo & 0xFFFFu), h16_to_f32<F16>(lo >> 16), h16_to_f32<F16>(hi & 0xFFFFu),
                        h16_to_f32<F16>(hi >> 16));
}

// 16 elements (two dwords x 4) -> 16 E4M3FN bytes (RNE, satfinite)
template <bool F16>
__device__ __forceinline__ u32x4 quantize16(u32x4 a, u32x4 b) {
  u32x4 o;
  o.x = quantize4<F16>(a.x, a.y);
  o.y = quantize4<F16>(a.z, a.w);
  o.z = quantize4<F16>(b.x, b.y);
  o.w = quantize4<F16>(b.z, b.w);
  return o;
}

// Rows of 32-element multiples (every Qwen3 shape: D = Hkv * 128) with
// 32-bit indexing: a lane owns two 16-element chunks of one K or V row, half
// a row apart, and issues all four 16-byte loads before converting, so a
// lane has twice the bytes in flight of a one-chunk lane and half the
// index arithmetic per byte.  Row r of the launch is token r / 2, K (even)
// or V (odd).
template <bool F16>
__global__ __launch_bounds__(256) void kv_store_fp8_pair_kernel(
    const uint16_t* __restrict__ key, int64_t key_stride, const uint16_t* __restrict__ value, int64_t value_stride,
    uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache, const int32_t* __restrict__ slot_mapping,
    int num_tokens, int row_elems, int64_t num_slots) {
  const int lanes_per_row = row_elems / 32;
  const int gid = (int)blockIdx.x * 256 + (int)threadIdx.x;
  const int r = gid / lanes_per_row, c0 = gid - r * lanes_per_row;
  if (r >= 2 * num_tokens) return;
  const int tok = r >> 1;
  const bool is_v = r & 1;
  const int32_t slot = slot_mapping[tok];
  if (slot < 0 || (int64_t)slot >= num_slots) return;  // -1: padding row (attention.py:24)
  const uint16_t* src = is_v ? value + (int64_t)tok * value_stride : key + (int64_t)tok * key_stride;
  uint8_t* dst = (is_v ? v_cache : k_cache) + (int64_t)slot * row_elems;
  u32x4 a[2], b[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = 16 * (c0 + j * lanes_per_row);
    a[j] = *reinterpret_cast<const u32x4*>(src + e);
    b[j] = *reinterpret_cast<const u32x4*>(src + e + 8);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
    *reinterpret_cast<u32x4*>(dst + 16 * (c0 + j * lanes_per_row)) = quantize16<F16>(a[j], b[j]);
}

// VEC: rows are 16-byte aligned and D % 16 == 0 (the normal case: K/V are
// views of the fused qkv projection); otherwise one element per lane-step.
template <bool VEC, bool F16>
__global__ __launch_bounds__(256) void kv_store_fp8_kernel(
    const uint16_t* __restrict__ key, int64_t key_stride,
    const uint16_t* __restrict__ value, int64_t value_stride,
    uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
    const int32_t* __restrict__ slot_mapping, int64_t num_tokens, int row_elems,
    int64_t num_slots) {
  const int per_lane = VEC ? 16 : 1;
  const int64_t chunks_per_row = row_elems / per_lane;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = num_tokens * 2 * chunks_per_row;
  if (idx >= total) return;
  const int64_t tok = idx / (2 * chunks_per_row);
  const int64_t rem = idx - tok * 2 * chunks_per_row;
  const bool is_v = rem >= chunks_per_row;
  const int64_t ch = is_v ? rem - chunks_per_row : rem;

  const int32_t slot = slot_mapping[tok];
  if (slot < 0 || (int64_t)slot >= num_slots) return;  // -1: padding row (attention.py:24)

  const uint16_t* src = (is_v ? value + tok * value_stride : key + tok * key_stride) + ch * per_lane;
  uint8_t* dst = (is_v ? v_cache : k_cache) + (int64_t)slot * row_elems + ch * per_lane;

  if constexpr (VEC) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(src);
    const u32x4 b = *reinterpret_cast<const u32x4*>(src + 8);
    *reinterpret_cast<u32x4*>(dst) = quantize16<F16>(a, b);
  } else {
    const float f = h16_to_f32<F16>(*src);
    const int w = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_satfinite(f), 0.0f, 0, false);
    *dst = (uint8_t)(w & 0xFF);
  }
}

namespace {

template <bool F16>
hipError_t launch_kv_store_t(const void* key, int64_t key_stride, const void* value, int64_t value_stride,
                             void* k_cache, void* v_cache, const int32_t* slot_mapping, int64_t num_tokens,
                             int row_elems, int64_t num_slots, bool vec, hipStream_t stream) {
  if (vec && row_elems % 32 == 0 && num_tokens * 2 * (row_elems / 32) + 255 < 0x7fffffff) {
    const int64_t threads = num_tokens * 2 * (row_elems / 32);
    hipLaunchKernelGGL(kv_store_fp8_pair_kernel<F16>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                       (const uint16_t*)key, key_stride, (const uint16_t*)value, value_stride, (uint8_t*)k_cache,
                       (uint8_t*)v_cache, slot_mapping, (int)num_tokens, row_elems, num_slots);
    return hipGetLastError();
  }
  const int per_lane = vec ? 16 : 1;
  const int64_t total = num_tokens * 2 * (row_elems / per_lane);
  const int64_t blocks = (total + 255) / 256;
  if (vec) {
    hipLaunchKernelGGL((kv_store_fp8_kernel<true, F16>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       (const uint16_t*)key, key_stride, (const uint16_t*)value, value_stride,
                       (uint8_t*)k_cache, (uint8_t*)v_cache, slot_mapping, num_tokens, row_elems,
                       num_slots);
  } else {
    hipLaunchKernelGGL((kv_store_fp8_kernel<false, F16>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       (const uint16_t*)key, key_stride, (const uint16_t*)value, value_stride,
                       (uint8_t*)k_cache, (uint8_t*)v_cache, slot_mapping, num_tokens, row_elems,
                       num_slots);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_kv_store(const void* key, int64_t key_stride, const void* value,
                           int64_t value_stride, void* k_cache, void* v_cache,
                           const int32_t* slot_mapping, int64_t num_tokens, int row_elems,
                           int64_t num_slots, bool vec, bool f16, hipStream_t stream) {
  if (num_tokens == 0) return hipSuccess;
  return f16 ? launch_kv_store_t<true>(key, key_stride, value, value_stride, k_cache, v_cache, slot_mapping,
                                       num_tokens, row_elems, num_slots, vec, stream)
             : launch_kv_store_t<false>(key, key_stride, value, value_stride, k_cache, v_cache, slot_mapping,
                                        num_tokens, row_elems, num_slots, vec, stream);
}

}  // namespace nvamd
