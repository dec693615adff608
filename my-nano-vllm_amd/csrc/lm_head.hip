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
// Sampler.forward (nanovllm/layers/sampler.py:7-12): token = argmax_v
// softmax(z / T)_v / max(E_v, 1e-10), the first index on ties, E_v ~ Exp(1).
// The softmax's max and sum are the same for every v of a row and exp and log
// are increasing, so that argmax is the argmax of the Gumbel-max score
// z_v c1 - log2(max(E_v, 1e-10)), c1 = log2(e) / T: one sweep of the logits
// (read once, no fp32 copy of [rows, vocab]); rounding can only decide
// between candidates whose scores agree to within a few ulps.
//
// sample_part_kernel + sample_pick_kernel: E is the caller's noise matrix.
//   Each row is split into `parts` workgroups; the pick kernel takes the best
//   part in part order.
//
// sample_group_kernel + sample_group_pick_kernel: E drawn in the kernel,
//   from Philox4x32-10 (Salmon et al., SC'11), u = ((x >> 8) + 1) 2^-24,
//   E = -ln u.  Drawing and ranking one E per token costs two 64-bit-product
//   rounds per token pair and two log2 per token, 3-4x the time the logits
//   take to stream.  The draw is taken top down instead (the Gumbel-max
//   property: the maximum of z_v c1 + G_v over a set of tokens, G_v =
//   -log2(E_v), is itself a Gumbel variable located at log2 sum_v 2^(z_v c1),
//   and independent of which token attains it):
//   * the row's tokens form groups of 16, [16g, 16g + 16);
//   * group g's maximum is drawn directly: M_g = log2(sum_v 2^(z_v c1)) -
//     log2(max(E_g, 1e-10)), E_g from Philox counter (2^31 + 64 (g / 256) +
//     g % 64, row, offset) word (g / 64) % 4 (the group stream: counters
//     disjoint from the token stream's);
//   * the winning group is the argmax of M_g (the first on ties), and the
//     token inside it the argmax of z_v c1 - log2(max(E_v, 1e-10)) with E_v
//     from the token stream, counter (v / 4, row, offset) word v % 4.
//   So every token costs one exp2 and a sixteenth of a log2, and a lane's
//   four groups of a 4,096-token quad share one Philox call.  The token
//   distribution is exactly softmax(z / T), as with one E per token.
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

// (value, index): larger value wins, the smaller index on equal values
__device__ __forceinline__ void better_i32(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

// Best (value, index) over the wave, in every lane.  The order is total, so
// any reduction order gives the same winner: DPP inside each 16-lane row,
// then the gfx950 row swaps (no LDS round trip).
template <int CTRL>
__device__ __forceinline__ void best_dpp(float& v, int& i) {
  better_i32(v, i, dpp_f32<CTRL>(v), (int)dpp_u32<CTRL>((uint32_t)i));
}
__device__ __forceinline__ void best_swap(float& v, int& i, bool swap32) {
  const uint32_t uv = __builtin_bit_cast(uint32_t, v), ui = (uint32_t)i;
  const auto a = swap32 ? __builtin_amdgcn_permlane32_swap(uv, uv, false, false)
                        : __builtin_amdgcn_permlane16_swap(uv, uv, false, false);
  const auto b = swap32 ? __builtin_amdgcn_permlane32_swap(ui, ui, false, false)
                        : __builtin_amdgcn_permlane16_swap(ui, ui, false, false);
  const uint32_t a0 = a[0], a1 = a[1], b0 = b[0], b1 = b[1];
  float v0 = __builtin_bit_cast(float, a0);
  int i0 = (int)b0;
  better_i32(v0, i0, __builtin_bit_cast(float, a1), (int)b1);
  v = v0;
  i = i0;
}
__device__ __forceinline__ void wave_best(float& v, int& i) {
  best_dpp<kDppRor8>(v, i);
  best_dpp<kDppRor4>(v, i);
  best_dpp<kDppXor2>(v, i);
  best_dpp<kDppXor1>(v, i);
  best_swap(v, i, false);
  best_swap(v, i, true);
}

// Part `part` of row `row` with the caller's noise: 4-element blocks [j0, j1)
// (elements 4j .. 4j + 3).  score_v = z_v * log2(e) / T - log2(max(E_v,
// 1e-10)); the row's argmax of score equals the reference's argmax of
// softmax(z / T)_v / max(E_v, 1e-10) (the softmax's max and sum are the same
// for every v, and exp and log are increasing), so one sweep of the logits
// suffices.  A lane visits its elements in increasing index order, so a
// strict > keeps the first index of a tie; the index order decides ties only
// across lanes and parts.  Indices are 32-bit (vocab < 2^31, checked at
// launch).
template <int DT, bool VEC>
__global__ __launch_bounds__(kSampleThreads) void sample_part_kernel(
    const void* __restrict__ logits, int64_t stride, int64_t vocab64, const float* __restrict__ temperatures,
    const float* __restrict__ noise, int parts, float* __restrict__ part_score, int64_t* __restrict__ part_index) {
  __shared__ float bval[kSampleThreads / 64];
  __shared__ int bidx[kSampleThreads / 64];
  const int vocab = (int)vocab64;
  const int64_t row = blockIdx.x / parts;
  const int part = (int)(blockIdx.x - row * parts);
  const int tid = threadIdx.x;
  const void* lr = static_cast<const uint8_t*>(logits) + row * stride * (DT == 2 ? 4 : 2);
  const float* nr = noise + row * vocab64;
  const float c1 = 1.4426950408889634f / temperatures[row];
  const int nb = (vocab + 3) / 4, nb_full = vocab / 4;  // 4-element blocks; those with 4 elements in the row
  const int j0 = (int)((int64_t)nb * part / parts), j1 = (int)((int64_t)nb * (part + 1) / parts);
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
    if (full) {
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = nr[v0 + i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = v0 + i < vocab ? nr[v0 + i] : 1.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // past the row: z = -inf, never above bv
      const float sc = z[i] * c1 - __builtin_amdgcn_logf(fmaxf(e[i], 1e-10f));
      const bool up = sc > bv;
      bv = up ? sc : bv;
      bi = up ? v0 + i : bi;
    }
  }
  wave_best(bv, bi);
  const int w = tid >> 6;
  if ((tid & 63) == 0) {
    bval[w] = bv;
    bidx[w] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int i = 1; i < kSampleThreads / 64; ++i) better_i32(bv, bi, bval[i], bidx[i]);
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

// ---- in-kernel noise: top-down group draw --------------------------------------
constexpr int kGroupTok = 16;                   // tokens per group (one lane)
constexpr int kQuadTok = 4 * 64 * kGroupTok;    // 4,096: the four windows whose groups share a Philox call
constexpr uint32_t kGroupCounter = 0x80000000u;  // group-stream counters start here (token-stream ones < 2^29)

// The 16 logits of the group starting at t0 (-inf past the row).
template <int DT, bool VEC>
__device__ __forceinline__ void load_group(const void* row, int t0, int vocab, float (&z)[kGroupTok]) {
  if (VEC && t0 + kGroupTok <= vocab) {
#pragma unroll
    for (int i = 0; i < kGroupTok; i += 4) load4<DT>(row, t0 + i, *reinterpret_cast<float(*)[4]>(&z[i]));
  } else {
#pragma unroll
    for (int i = 0; i < kGroupTok; ++i) z[i] = t0 + i < vocab ? load1<DT>(row, t0 + i) : -INFINITY;
  }
}

// E = -ln(u), u = ((x >> 8) + 1) 2^-24 in (0, 1]; then -log2(max(E, 1e-10)).
__device__ __forceinline__ float gumbel_log2(uint32_t x) {
  const float e = -__builtin_amdgcn_logf((float)((x >> 8) + 1u) * 0x1p-24f) * 0.6931471805599453f;
  return -__builtin_amdgcn_logf(fmaxf(e, 1e-10f));
}

// One wave per (row, quad): lane l takes group 64k + l of each of the quad's
// four 1,024-token windows k (16 consecutive tokens, so each load
// instruction of the wave reads 1 KiB contiguous) and draws its four group
// maxima from one Philox call.  Writes the quad's best (M_g, g).
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void sample_group_kernel(const void* __restrict__ logits, int64_t stride,
                                                           int vocab, const float* __restrict__ temperatures,
                                                           uint64_t seed, uint64_t offset, int nq, int64_t tasks,
                                                           float* __restrict__ task_score,
                                                           int* __restrict__ task_group) {
  const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (task >= tasks) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int64_t row = task / nq;
  const int q = (int)(task - row * nq);
  const void* lr = static_cast<const uint8_t*>(logits) + row * stride * (DT == 2 ? 4 : 2);
  const float c1 = 1.4426950408889634f / temperatures[row];
  float z[4][kGroupTok];
#pragma unroll
  for (int k = 0; k < 4; ++k) load_group<DT, VEC>(lr, q * kQuadTok + k * 64 * kGroupTok + lane * kGroupTok, vocab, z[k]);
  const u32x4 x = philox4x32_10(u32x4{kGroupCounter + (uint32_t)(64 * q + lane), (uint32_t)row, (uint32_t)offset,
                                      (uint32_t)(offset >> 32)},
                                (uint32_t)seed, (uint32_t)(seed >> 32));
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
  float bm = -INFINITY;
  int bg = 0x7fffffff;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < kGroupTok; ++i) {
      z[k][i] *= c1;
      mx = fmaxf(mx, z[k][i]);
    }
    float sum = 0.f;  // in token order
#pragma unroll
    for (int i = 0; i < kGroupTok; ++i) sum += __builtin_amdgcn_exp2f(z[k][i] - mx);
    const float m = (mx == -INFINITY) ? -INFINITY : (mx + __builtin_amdgcn_logf(sum)) + gumbel_log2(xs[k]);
    const int g = (4 * q + k) * 64 + lane;
    if (m > bm) {  // groups in increasing order: a strict > keeps the first on ties
      bm = m;
      bg = g;
    }
  }
  wave_best(bm, bg);
  if (lane == 0) {
    task_score[task] = bm;
    task_group[task] = bg;
  }
}

// One wave per row: the best group over the row's quads, then the best token
// of that group on the token stream.
template <int DT>
__global__ __launch_bounds__(256) void sample_group_pick_kernel(const void* __restrict__ logits, int64_t stride,
                                                                int vocab, const float* __restrict__ temperatures,
                                                                uint64_t seed, uint64_t offset, int nq, int64_t rows,
                                                                const float* __restrict__ task_score,
                                                                const int* __restrict__ task_group,
                                                                int64_t* __restrict__ out) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  float bm = -INFINITY;
  int bg = 0x7fffffff;
  for (int q = lane; q < nq; q += 64) better_i32(bm, bg, task_score[row * nq + q], task_group[row * nq + q]);
  wave_best(bm, bg);
  const void* lr = static_cast<const uint8_t*>(logits) + row * stride * (DT == 2 ? 4 : 2);
  const int v = bg * kGroupTok + (lane & (kGroupTok - 1));
  float sc = -INFINITY;
  if (bm != -INFINITY && lane < kGroupTok && v < vocab) {
    const float c1 = 1.4426950408889634f / temperatures[row];
    const u32x4 x = philox4x32_10(u32x4{(uint32_t)(v >> 2), (uint32_t)row, (uint32_t)offset,
                                        (uint32_t)(offset >> 32)},
                                  (uint32_t)seed, (uint32_t)(seed >> 32));
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
    sc = load1<DT>(lr, v) * c1 + gumbel_log2(xs[v & 3]);
  }
  int bv = lane < kGroupTok ? v : 0x7fffffff;
  wave_best(sc, bv);
  if (lane == 0) out[row] = (sc != -INFINITY && bv < vocab) ? bv : 0;
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

int sample_quads(int64_t vocab) { return (int)((vocab + kQuadTok - 1) / kQuadTok); }

hipError_t launch_sample_group(const void* logits, int dtype, int64_t stride, int64_t rows, int64_t vocab,
                               const float* temperatures, uint64_t seed, uint64_t offset, int64_t* out,
                               float* task_score, int* task_group, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  const int nq = sample_quads(vocab);
  const int64_t tasks = rows * nq;
  if (vocab >= 0x7fffffff - kQuadTok || (tasks + 3) / 4 > 0x7fffffff || (rows + 3) / 4 > 0x7fffffff)
    return hipErrorInvalidValue;
  const bool vec = (stride % 4 == 0) && ((uintptr_t)logits % (dtype == 2 ? 16 : 8) == 0);
  const dim3 grid((unsigned)((tasks + 3) / 4)), block(256);
  switch (dtype * 2 + (vec ? 1 : 0)) {
#define NVAMD_GROUP_CASE(c, DT, V)                                                                               \
  case c:                                                                                                        \
    hipLaunchKernelGGL((sample_group_kernel<DT, V>), grid, block, 0, stream, logits, stride, (int)vocab,          \
                       temperatures, seed, offset, nq, tasks, task_score, task_group);                           \
    break;
    NVAMD_GROUP_CASE(0, 0, false)
    NVAMD_GROUP_CASE(1, 0, true)
    NVAMD_GROUP_CASE(2, 1, false)
    NVAMD_GROUP_CASE(3, 1, true)
    NVAMD_GROUP_CASE(4, 2, false)
    NVAMD_GROUP_CASE(5, 2, true)
#undef NVAMD_GROUP_CASE
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 pgrid((unsigned)((rows + 3) / 4));
  switch (dtype) {
    case 0: hipLaunchKernelGGL((sample_group_pick_kernel<0>), pgrid, block, 0, stream, logits, stride, (int)vocab,
                               temperatures, seed, offset, nq, rows, task_score, task_group, out); break;
    case 1: hipLaunchKernelGGL((sample_group_pick_kernel<1>), pgrid, block, 0, stream, logits, stride, (int)vocab,
                               temperatures, seed, offset, nq, rows, task_score, task_group, out); break;
    default: hipLaunchKernelGGL((sample_group_pick_kernel<2>), pgrid, block, 0, stream, logits, stride, (int)vocab,
                                temperatures, seed, offset, nq, rows, task_score, task_group, out); break;
  }
  return hipGetLastError();
}

hipError_t launch_sample_noise(const void* logits, int dtype, int64_t stride, int64_t rows, int64_t vocab,
                               const float* temperatures, const float* noise, int64_t* out, float* part_score,
                               int64_t* part_index, int parts, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  if (parts < 1 || rows * parts > 0x7fffffff || vocab >= 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(rows * parts)), block(kSampleThreads);
  // vector loads need every row start aligned to 4 elements
  const bool vec = (stride % 4 == 0) && ((uintptr_t)logits % (dtype == 2 ? 16 : 8) == 0);
  switch (dtype * 2 + (vec ? 1 : 0)) {
#define NVAMD_SAMPLE_CASE(c, DT, V)                                                                             \
  case c:                                                                                                       \
    hipLaunchKernelGGL((sample_part_kernel<DT, V>), grid, block, 0, stream, logits, stride, vocab, temperatures, \
                       noise, parts, part_score, part_index);                                                    \
    break;
    NVAMD_SAMPLE_CASE(0, 0, false)
    NVAMD_SAMPLE_CASE(1, 0, true)
    NVAMD_SAMPLE_CASE(2, 1, false)
    NVAMD_SAMPLE_CASE(3, 1, true)
    NVAMD_SAMPLE_CASE(4, 2, false)
    default:
      hipLaunchKernelGGL((sample_part_kernel<2, true>), grid, block, 0, stream, logits, stride, vocab, temperatures,
                         noise, parts, part_score, part_index);
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
