// Fused q/k RMSNorm + rotary embedding + FP8 KV store for gfx950.
//
// Replaces, for one attention layer, the steps between the QKV projection
// and the attention call: the q/k RMSNorm (nanovllm/models/qwen3.py:107-109,
// nanovllm/layers/layernorm.py:16-25), the neox rotary embedding
// (qwen3.py:110, nanovllm/layers/rotary_embedding.py:6-14,40-50) and the
// store of k and v into the FP8 cache (nanovllm/layers/attention.py:61-62,
// store_kvcache_kernel :11-31).  The reference reads the bf16 projection
// output three times and writes the normalised and rotated q and k back to
// HBM before the store reads k again; here each head row of the projection
// output is read once and q leaves as bf16, k and v as FP8 cache bytes.
//
// Layout: the projection output is [N, (Hq + 2 Hkv) * 128] bf16 with row
// stride qkv_stride elements; a 16-lane group owns one 128-dim head row
// (lane j: dims 8j .. 8j + 7, one 16-byte load), so a wave covers 4 head
// rows of one token and every access is a whole 16-byte granule of
// contiguous rows.
//
// Arithmetic, with the reference's rounding points:
//   RMSNorm:  y = bf16(x * rsqrt(mean(x^2) + eps)) in fp32, then
//             z = bf16(y * w) (a bf16 product with the bf16 weight);
//   RoPE:     out[i]      = bf16(z[i] cos_i - z[i + 64] sin_i),
//             out[i + 64] = bf16(z[i + 64] cos_i + z[i] sin_i), i < 64, fp32 math,
//             cos/sin from the fp32 cos_sin_cache row of the token's position;
//             lane j (< 8) and lane j + 8 hold the two halves and swap them
//             with one DPP row rotation;
//   store:    k (after RoPE) and v (as projected) rounded to E4M3FN (RNE,
//             satfinite), written to slot_mapping[token] unless it is -1.
// The sum of squares is reduced in a different order from the reference
// and rsqrt is the hardware's, so an output can differ from it by one bf16
// ulp where the fp32 value sits at a rounding boundary.
#include "fp8_common.h"
#include "kernels.h"

namespace nvamd {

namespace {

constexpr int kLanesPerRow = kHeadDim / 8;  // 16

// 8 floats -> 8 bf16 (RNE) in four dwords
__device__ __forceinline__ u32x4 pack8_bf16(const float (&v)[8]) {
  return u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
}

__device__ __forceinline__ void unpack8_bf16(u32x4 w, float (&v)[8]) {
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_bits_to_f32(d[i] & 0xFFFFu);
    v[2 * i + 1] = bf16_bits_to_f32(d[i] >> 16);
  }
}

// 8 bf16 values (as floats) -> 8 E4M3FN bytes in two dwords
__device__ __forceinline__ u32x2 to_fp8x8(const float (&v)[8]) {
  return u32x2{f32x4_to_fp8x4(v[0], v[1], v[2], v[3]), f32x4_to_fp8x4(v[4], v[5], v[6], v[7])};
}

// lane j of the row <- lane j ^ 8 (the other half of the head dims)
__device__ __forceinline__ u32x4 swap_halves(u32x4 w) {
  return u32x4{dpp_u32<kDppRor8>(w.x), dpp_u32<kDppRor8>(w.y), dpp_u32<kDppRor8>(w.z), dpp_u32<kDppRor8>(w.w)};
}

}  // namespace

// One workgroup per token: 16-lane group g takes head rows g, g + 16, g + 32,
// ... of the token, so the token's position and slot are uniform scalar
// loads, no lane divides, and the cos / sin of the position and both norm
// weights are loaded once per lane for all of its rows (they are reused
// from the caches, but each load instruction costs address-unit time).
constexpr int kRowsPerPass = 256 / kLanesPerRow;  // 16 head rows per pass of the workgroup
constexpr int kMaxPasses = 8;                      // rows of a token: at most 128 (checked at launch)

// NP passes: ceil((Hq + 2 Hkv) / 16) (3 for Qwen3-8B's 32 + 2 x 8 rows)
template <int NP>
__global__ __launch_bounds__(256) void qk_norm_rope_store_kernel(QkNormRopeParams p) {
  const int rows_per_token = p.Hq + 2 * p.Hkv;
  const int64_t tok = blockIdx.x;
  const int g = (int)(threadIdx.x >> 4);
  const int j = (int)(threadIdx.x & 15);
  // num_slots == 0: no cache yet (the runner's warm-up), nothing is stored and
  // slot_mapping may be null
  const int32_t slot = p.num_slots > 0 ? p.slot_mapping[tok] : -1;
  const bool store = slot >= 0 && (int64_t)slot < p.num_slots;
  const int64_t cache_row = (int64_t)slot * p.Hkv * kHeadDim;
  int64_t pos = p.positions[tok];
  pos = pos < 0 ? 0 : (pos >= p.max_position ? p.max_position - 1 : pos);  // no read outside the table
  const uint16_t* xrow = p.qkv + tok * p.qkv_stride + 8 * j;

  // this lane's rows: all loads first
  u32x4 xr[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int r = g + kRowsPerPass * i;
    xr[i] = r < rows_per_token ? *reinterpret_cast<const u32x4*>(xrow + (int64_t)r * kHeadDim) : u32x4{0u, 0u, 0u, 0u};
  }
  // lanes j and j ^ 8 hold dims i and i + 64 of the same frequencies
  const float* cs = p.cos_sin + pos * kHeadDim + 8 * (j & 7);
  const f32x4 c0 = *reinterpret_cast<const f32x4*>(cs), c1 = *reinterpret_cast<const f32x4*>(cs + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(cs + kHeadDim / 2);
  const f32x4 s1 = *reinterpret_cast<const f32x4*>(cs + kHeadDim / 2 + 4);
  const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  float wq[8], wk[8];
  unpack8_bf16(*reinterpret_cast<const u32x4*>(p.q_weight + 8 * j), wq);
  unpack8_bf16(*reinterpret_cast<const u32x4*>(p.k_weight + 8 * j), wk);
  const float sgn = (j < 8) ? -1.f : 1.f;  // first half: z cos - other sin; second: z cos + other sin

#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int r = g + kRowsPerPass * i;  // uniform in a 16-lane group, so the exchanges below stay in live lanes
    if (r >= rows_per_token) break;
    float x[8];
    unpack8_bf16(xr[i], x);
    if (r >= p.Hq + p.Hkv) {  // v: stored as projected
      if (store) *reinterpret_cast<u32x2*>(p.v_cache + cache_row + (int64_t)(r - p.Hq - p.Hkv) * kHeadDim + 8 * j) = to_fp8x8(x);
      continue;
    }
    const bool is_q = r < p.Hq;
    // RMSNorm over the row's 128 dims (the 16 lanes of the group)
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(x[e], x[e], ss);
    ss = row16_sum(ss);
    const float rs = __builtin_amdgcn_rsqf(ss * (1.0f / kHeadDim) + p.eps);
    float z[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = bf16_bits_to_f32(pack_bf16x2(x[e] * rs, 0.f) & 0xFFFFu);
      z[e] = bf16_bits_to_f32(pack_bf16x2(y * (is_q ? wq[e] : wk[e]), 0.f) & 0xFFFFu);
    }
    // RoPE
    const u32x4 zp = pack8_bf16(z);  // exact: z is bf16
    float other[8];
    unpack8_bf16(swap_halves(zp), other);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = bf16_bits_to_f32(pack_bf16x2(z[e] * cv[e] + sgn * (other[e] * sv[e]), 0.f) & 0xFFFFu);
    const u32x4 out = pack8_bf16(o);
    if (is_q) {
      *reinterpret_cast<u32x4*>(p.q_out + (tok * p.Hq + r) * kHeadDim + 8 * j) = out;
      continue;
    }
    const int hk = r - p.Hq;
    if (p.k_out != nullptr) *reinterpret_cast<u32x4*>(p.k_out + (tok * p.Hkv + hk) * kHeadDim + 8 * j) = out;
    if (store) *reinterpret_cast<u32x2*>(p.k_cache + cache_row + (int64_t)hk * kHeadDim + 8 * j) = to_fp8x8(o);
  }
}

hipError_t launch_qk_norm_rope_store(const QkNormRopeParams& p, hipStream_t stream) {
  if (p.num_tokens == 0) return hipSuccess;
  if (p.num_tokens > 0x7fffffff || p.Hq + 2 * p.Hkv > kRowsPerPass * kMaxPasses) return hipErrorInvalidValue;
  const dim3 grid((unsigned)p.num_tokens), block(256);
  switch ((p.Hq + 2 * p.Hkv + kRowsPerPass - 1) / kRowsPerPass) {
    case 1: hipLaunchKernelGGL(qk_norm_rope_store_kernel<1>, grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL(qk_norm_rope_store_kernel<2>, grid, block, 0, stream, p); break;
    case 3: hipLaunchKernelGGL(qk_norm_rope_store_kernel<3>, grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL(qk_norm_rope_store_kernel<4>, grid, block, 0, stream, p); break;
    case 5: hipLaunchKernelGGL(qk_norm_rope_store_kernel<5>, grid, block, 0, stream, p); break;
    case 6: hipLaunchKernelGGL(qk_norm_rope_store_kernel<6>, grid, block, 0, stream, p); break;
    case 7: hipLaunchKernelGGL(qk_norm_rope_store_kernel<7>, grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL(qk_norm_rope_store_kernel<8>, grid, block, 0, stream, p); break;
  }
  return hipGetLastError();
}

}  // namespace nvamd
