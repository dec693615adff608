// LM-head row selection and the sampler for gfx950.
//
// select_rows_kernel <- the row selection of ParallelLMHead.forward
//   (nanovllm/layers/embed_head.py:56-72): the hidden states of the plain
//   decode rows and of every speculative row are a prefix of x and are
//   copied as they are; each remaining varlen (prefill) sequence contributes
//   its last row, split_pt + cu_seqlens_q[nspec + 1 + i] - 1.  The number of
//   speculative rows (cu_seqlens_q[nspec]) comes from the host, which
//   scheduled them, instead of a device-to-host read.  16-byte copies.
//
// sample_part_kernel + sample_pick_kernel <- Sampler.forward
//   (nanovllm/layers/sampler.py:7-12), token = argmax_v softmax(z / T)_v /
//   max(E_v, 1e-10), the first index on ties.  The softmax's max and sum are
//   the same for every v of a row and exp and log are increasing, so that
//   argmax is the argmax of z_v log2(e) / T - log2(max(E_v, 1e-10)): one sweep
//   of the logits (read once, no fp32 copy of [rows, vocab]) with two
//   hardware log2 per element; rounding can only decide between candidates
//   whose scores agree to within a few ulps.  Each row is split into `parts`
//   workgroups (355 rows would leave most CUs one row and some two); the
//   pick kernel takes the best part in part order.  E is the caller's noise
//   matrix or, without one, Exp(1) samples -ln(u) drawn in the kernel from
//   Philox4x32-10 (Salmon et al., SC'11), u = ((x >> 8) + 1) 2^-24, counter
//   (v / 4, row, offset) and key seed for elements v .. v + 3.
#include "fp8_common.h"
#include "kernels.h"

namespace nvamd {

namespace {

constexpr int kSampleThreads = 512;

// Workgroup r copies output row r: its source row from the prefix rule
// (uniform scalar loads), then the row's 16-byte chunks, strided over the
// 256 lanes.
__global__ __launch_bounds__(256) void select_rows_kernel(const uint8_t* __restrict__ x, int64_t x_stride_bytes,
                                                          int64_t x_rows, int row_bytes,
                                                          const int32_t* __restrict__ cu_seqlens_q, int split_pt,
                                                          int num_spec_rows, int num_spec_seqs, int64_t out_rows,
                                                          uint8_t* __restrict__ out, int64_t out_stride_bytes) {
  const int64_t r = blockIdx.x;
  const int64_t prefix = (int64_t)split_pt + num_spec_rows;
  const int64_t src = r < prefix ? r : split_pt + (int64_t)cu_seqlens_q[num_spec_seqs + 1 + (r - prefix)] - 1;
  if (src < 0 || src >= x_rows) return;
  const u32x4* in = reinterpret_cast<const u32x4*>(x + src * x_stride_bytes);
  u32x4* o = reinterpret_cast<u32x4*>(out + r * out_stride_bytes);
  for (int c = (int)threadIdx.x; c < row_bytes / 16; c += 256) o[c] = in[c];
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11).
__device__ __forceinline__ u32x4 philox4x32_10(u32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint64_t p0 = (uint64_t)c.x * 0xD2511F53u, p1 = (uint64_t)c.z * 0xCD9E8D57u;
    c = u32x4{(uint32_t)(p1 >> 32) ^ c.y ^ k0, (uint32_t)p1, (uint32_t)(p0 >> 32) ^ c.w ^ k1, (uint32_t)p0};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

// (value, index): larger value wins, the smaller index on equal values
__device__ __forceinline__ void better(float& bv, int64_t& bi, float v, int64_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

template <int DT>  // 0 bf16, 1 fp16, 2 fp32
__device__ __forceinline__ void load4(const void* row, int64_t v, float (&z)[4]) {
  if constexpr (DT == 2) {
    const f32x4 w = *reinterpret_cast<const f32x4*>(static_cast<const float*>(row) + v);
    z[0] = w.x, z[1] = w.y, z[2] = w.z, z[3] = w.w;
  } else {
    const u32x2 w = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(row) + v);
    const uint32_t h[4] = {w.x & 0xFFFFu, w.x >> 16, w.y & 0xFFFFu, w.y >> 16};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      z[i] = DT == 0 ? bf16_bits_to_f32(h[i]) : (float)__builtin_bit_cast(_Float16, (uint16_t)h[i]);
  }
}

template <int DT>
__device__ __forceinline__ float load1(const void* row, int64_t v) {
  if constexpr (DT == 0) return bf16_bits_to_f32(static_cast<const uint16_t*>(row)[v]);
  else if constexpr (DT == 1) return (float)static_cast<const _Float16*>(row)[v];
  else return static_cast<const float*>(row)[v];
}

// Part `part` of row `row`: Philox blocks [j0, j1) (elements 4j .. 4j + 3).
// score_v = z_v * log2(e) / T - log2(max(E_v, 1e-10)); the row's argmax of
// score equals the reference's argmax of softmax(z / T)_v / max(E_v, 1e-10)
// (the softmax's max and sum are the same for every v, and exp and log are
// increasing), so one sweep of the logits suffices.  A lane visits its
// elements in increasing index order, so a strict > keeps the first index
// of a tie; the index order decides ties only across lanes and parts.
// Indices are 32-bit (vocab < 2^31, checked at launch).
template <int DT, bool VEC>
__global__ __launch_bounds__(kSampleThreads) void sample_part_kernel(
    const void* __restrict__ logits, int64_t stride, int64_t vocab64, const float* __restrict__ temperatures,
    const float* __restrict__ noise, uint64_t seed, uint64_t offset, int parts, float* __restrict__ part_score,
    int64_t* __restrict__ part_index) {
  __shared__ float bval[kSampleThreads / 64];
  __shared__ int bidx[kSampleThreads / 64];
  const int vocab = (int)vocab64;
  const int64_t row = blockIdx.x / parts;
  const int part = (int)(blockIdx.x - row * parts);
  const int tid = threadIdx.x;
  const void* lr = static_cast<const uint8_t*>(logits) + row * stride * (DT == 2 ? 4 : 2);
  const float* nr = noise != nullptr ? noise + row * vocab64 : nullptr;
  const float c1 = 1.4426950408889634f / temperatures[row];
  const int nb = (vocab + 3) / 4, nb_full = vocab / 4;  // Philox blocks; those with 4 elements in the row
  const int j0 = (int)((int64_t)nb * part / parts), j1 = (int)((int64_t)nb * (part + 1) / parts);
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  const uint32_t off_lo = (uint32_t)offset, off_hi = (uint32_t)(offset >> 32);
  float bv = -INFINITY;
  int bi = vocab;
  for (int j = j0 + tid; j < j1; j += kSampleThreads) {
    const int v0 = 4 * j;
    const bool full = j < nb_full;
    float z[4];
    if (VEC && full) {
      load4<DT>(lr, v0, z);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) z[i] = v0 + i < vocab ? load1<DT>(lr, v0 + i) : -INFINITY;
    }
    float e[4];
    if (nr != nullptr) {
      if (full) {
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = nr[v0 + i];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = v0 + i < vocab ? nr[v0 + i] : 1.f;
      }
    } else {
      const u32x4 x = philox4x32_10(u32x4{(uint32_t)j, (uint32_t)row, off_lo, off_hi}, k0, k1);
      const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)  // E = -ln(u) = -log2(u) ln 2
        e[i] = -__builtin_amdgcn_logf((float)((xs[i] >> 8) + 1u) * 0x1p-24f) * 0.6931471805599453f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // past the row: z = -inf, never above bv
      const float sc = z[i] * c1 - __builtin_amdgcn_logf(fmaxf(e[i], 1e-10f));
      const bool up = sc > bv;
      bv = up ? sc : bv;
      bi = up ? v0 + i : bi;
    }
  }
  // (value, index): larger value wins, the smaller index on equal values
  auto better32 = [](float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  };
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) better32(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
  const int w = tid >> 6;
  if ((tid & 63) == 0) {
    bval[w] = bv;
    bidx[w] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int i = 1; i < kSampleThreads / 64; ++i) better32(bv, bi, bval[i], bidx[i]);
    part_score[blockIdx.x] = bv;
    part_index[blockIdx.x] = bi;
  }
}

__global__ __launch_bounds__(256) void sample_pick_kernel(const float* __restrict__ part_score,
                                                          const int64_t* __restrict__ part_index, int64_t rows,
                                                          int parts, int64_t vocab, int64_t* __restrict__ out) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (row >= rows) return;
  float bv = -INFINITY;
  int64_t bi = vocab;
  for (int p = 0; p < parts; ++p) better(bv, bi, part_score[row * parts + p], part_index[row * parts + p]);
  out[row] = bi < vocab ? bi : 0;
}

}  // namespace

hipError_t launch_select_rows(const void* x, int64_t x_stride_bytes, int64_t x_rows, int row_bytes,
                              const int32_t* cu_seqlens_q, int split_pt, int num_spec_rows, int num_spec_seqs,
                              int64_t out_rows, void* out, int64_t out_stride_bytes, hipStream_t stream) {
  if (out_rows == 0) return hipSuccess;
  if (out_rows > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(select_rows_kernel, dim3((unsigned)out_rows), dim3(256), 0, stream, (const uint8_t*)x,
                     x_stride_bytes, x_rows, row_bytes, cu_seqlens_q, split_pt, num_spec_rows, num_spec_seqs,
                     out_rows, (uint8_t*)out, out_stride_bytes);
  return hipGetLastError();
}

hipError_t launch_sample(const void* logits, int dtype, int64_t stride, int64_t rows, int64_t vocab,
                         const float* temperatures, const float* noise, uint64_t seed, uint64_t offset, int64_t* out,
                         float* part_score, int64_t* part_index, int parts, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  if (parts < 1 || rows * parts > 0x7fffffff || vocab >= 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(rows * parts)), block(kSampleThreads);
  // vector loads need every row start aligned to 4 elements
  const bool vec = (stride % 4 == 0) && ((uintptr_t)logits % (dtype == 2 ? 16 : 8) == 0);
  switch (dtype * 2 + (vec ? 1 : 0)) {
#define NVAMD_SAMPLE_CASE(c, DT, V)                                                                             \
  case c:                                                                                                       \
    hipLaunchKernelGGL((sample_part_kernel<DT, V>), grid, block, 0, stream, logits, stride, vocab, temperatures, \
                       noise, seed, offset, parts, part_score, part_index);                                      \
    break;
    NVAMD_SAMPLE_CASE(0, 0, false)
    NVAMD_SAMPLE_CASE(1, 0, true)
    NVAMD_SAMPLE_CASE(2, 1, false)
    NVAMD_SAMPLE_CASE(3, 1, true)
    NVAMD_SAMPLE_CASE(4, 2, false)
    default:
      hipLaunchKernelGGL((sample_part_kernel<2, true>), grid, block, 0, stream, logits, stride, vocab, temperatures,
                         noise, seed, offset, parts, part_score, part_index);
      break;
#undef NVAMD_SAMPLE_CASE
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sample_pick_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, part_score,
                     part_index, rows, parts, vocab, out);
  return hipGetLastError();
}

}  // namespace nvamd
