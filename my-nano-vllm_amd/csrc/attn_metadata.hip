// On-device attention metadata for one engine step (gfx950).
//
// Builds, from one small per-step upload, the tensors nano-vLLM's
// ModelRunner builds on the host with per-token Python loops and copies to
// the GPU one by one (nanovllm/engine/model_runner.py:133-220):
//   positions     int64 [T]   plain decode: len - 1 (:196); varlen: num_cached .. + num_scheduled (:163)
//   slot_mapping  int32 [S]   plain decode: block_table[-1] * bs + last_block_num_tokens - 1 (:198);
//                             varlen: the block walk of :172-182, i.e. block_table[p / bs] * bs + p % bs
//                             for each scheduled position p; none for a sequence without a table (:170)
//   context_lens  int32 [n_plain]                      (:197)
//   cu_seqlens_q / _k int32 [n_varlen + 1]             (:166-167)
//   block_tables  int32 [rows with a table, max_len]   padded with -1 (:133-142)
// in the reference's row order: plain decode sequences, then speculative
// ones, then prefill chunks (:203-216).
//
// Input (device): `packed` = int32 [num_seqs, 4] descriptors {num_tokens,
// num_cached_tokens, num_scheduled_tokens, table_len}, in that order, then the
// sequences' block tables back to back (sum of table_len entries).  Every
// workgroup loads the descriptors into LDS once and scans them in one pass
// (token offsets, slot offsets, output table rows, key-length prefix, table
// offsets: per-thread chunk sums, a shuffle scan per wave, one exchange
// between the waves), then walks
// a grid-stride range of output units -- tokens, table entries, context
// lengths, cu_seqlens entries -- locating each unit's sequence by binary
// search.  Offsets are 64-bit; slot values are computed in 64 bits and
// stored as int32 like the reference's int32 tensor.  Writes are bounded by
// the caller's output sizes and reads by the upload's length; a scheduled
// position past a sequence's table (where the reference's Python raises)
// gets slot -1, and negative descriptor fields read as 0.
#include <algorithm>

#include "fp8_common.h"
#include "kernels.h"

namespace nvamd {

namespace {

constexpr int kMetaThreads = 256;

// Last s in [0, n) with a[s] <= x (a nondecreasing, a[0] <= x).
__device__ __forceinline__ int last_le(const int* a, int n, int64_t x) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

__global__ __launch_bounds__(kMetaThreads) void build_metadata_kernel(AttnMetaParams p) {
  __shared__ int4 dsc[kMetaMaxSeqs];          // the descriptors, negatives read as 0
  __shared__ int pos_off[kMetaMaxSeqs + 1];   // first token (query row) of each sequence
  __shared__ int slot_off[kMetaMaxSeqs + 1];  // first slot_mapping entry
  __shared__ int trow[kMetaMaxSeqs + 1];      // output block-table row (sequences with a table)
  __shared__ int kpre[kMetaMaxSeqs + 1];      // varlen key-length prefix (cu_seqlens_k)
  __shared__ int toff[kMetaMaxSeqs + 1];      // offset of the sequence's table in the upload
  __shared__ int wave_tot[kMetaThreads / 64][5];
  const int n = p.num_seqs, np_ = p.num_plain;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int4* desc = reinterpret_cast<const int4*>(p.packed);
  const int* tables = p.packed + 4 * (int64_t)n;
  const int64_t n_table_ints = p.packed_ints - 4 * (int64_t)n;  // table entries the upload holds
  for (int q = tid; q < n; q += kMetaThreads) {
    const int4 v = desc[q];
    dsc[q] = int4{max(v.x, 0), max(v.y, 0), max(v.z, 0), max(v.w, 0)};
  }
  __syncthreads();
  auto d = [&](int q) { return dsc[q]; };  // {num_tokens, num_cached, num_scheduled, table_len}
  // table entry c of the table at offset o: -1 past the upload
  auto entry = [&](int64_t o, int64_t c) { return o + c < n_table_ints ? tables[o + c] : -1; };
  // The five exclusive prefixes over the sequences in one pass: each thread
  // sums a chunk of sequences, the chunk sums are scanned across the wave
  // with shuffles and across the waves through LDS, then each thread writes
  // its chunk's prefixes.
  auto terms = [&](int q, int (&t)[5]) {
    const int4 v = d(q);
    const bool plain = q < np_;
    t[0] = plain ? 1 : v.z;                          // query rows
    t[1] = plain ? 1 : (v.w > 0 ? v.z : 0);          // slot_mapping entries
    t[2] = v.w > 0 ? 1 : 0;                          // output table rows
    t[3] = plain ? 0 : v.y + v.z;                    // varlen key lengths
    t[4] = v.w;                                      // table entries in the upload
  };
  const int chunk = (n + kMetaThreads - 1) / kMetaThreads;
  const int q0 = min(n, tid * chunk), q1 = min(n, q0 + chunk);
  int sum[5] = {0, 0, 0, 0, 0};
  for (int q = q0; q < q1; ++q) {
    int t[5];
    terms(q, t);
#pragma unroll
    for (int k = 0; k < 5; ++k) sum[k] += t[k];
  }
  int incl[5];
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    incl[k] = wave_incl_scan(sum[k]);
    if (lane == 63) wave_tot[wave][k] = incl[k];
  }
  __syncthreads();
  int run[5], total[5];
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kMetaThreads / 64; ++w) {
      before += w < wave ? wave_tot[w][k] : 0;
      all += wave_tot[w][k];
    }
    run[k] = before + incl[k] - sum[k];
    total[k] = all;
  }
  int* const outs[5] = {pos_off, slot_off, trow, kpre, toff};
  for (int q = q0; q < q1; ++q) {
    int t[5];
    terms(q, t);
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      outs[k][q] = run[k];
      run[k] += t[k];
    }
  }
  if (tid == 0) {
#pragma unroll
    for (int k = 0; k < 5; ++k) outs[k][n] = total[k];
  }
  __syncthreads();

  const int64_t T = pos_off[n], W = p.max_table_len, R = trow[n];
  const int n_var = n - np_;
  const int64_t u_tables = T, u_ctx = T + R * W, u_cu = u_ctx + np_;
  const int64_t U = u_cu + (n_var > 0 ? n_var + 1 : 0);
  const int64_t bs = p.block_size;
  for (int64_t u = (int64_t)blockIdx.x * kMetaThreads + threadIdx.x; u < U; u += (int64_t)gridDim.x * kMetaThreads) {
    if (u < u_tables) {  // one token
      const int s = last_le(pos_off, n, u);
      const int4 ds = d(s);
      if (u >= p.cap_tokens) continue;
      if (s < np_) {
        const int64_t len = ds.x;
        const int64_t nb = (len + bs - 1) / bs;
        p.positions[u] = len - 1;
        // a plain decode row always owns one slot entry; without a block table
        // (which the reference's loops cannot handle) it is -1, so the store skips it
        if (slot_off[s] < p.cap_slots)
          p.slot_mapping[slot_off[s]] =
              ds.w > 0 ? (int32_t)(entry(toff[s], ds.w - 1) * bs + (len - (nb - 1) * bs) - 1) : -1;
      } else {
        const int64_t i = u - pos_off[s], pos = (int64_t)ds.y + i;
        p.positions[u] = pos;
        const int64_t blk = pos / bs;
        if (ds.w > 0 && slot_off[s] + i < p.cap_slots)
          p.slot_mapping[slot_off[s] + i] = blk < ds.w ? (int32_t)(entry(toff[s], blk) * bs + pos % bs) : -1;
      }
    } else if (u < u_ctx) {  // one padded block-table entry
      const int64_t e = u - u_tables;
      const int r = (int)(e / W), c = (int)(e - (int64_t)r * W);
      // the sequence whose table is output row r: first s with trow[s + 1] > r
      int lo = 0, hi = n - 1;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (trow[mid + 1] > r) hi = mid;
        else lo = mid + 1;
      }
      if (r < p.cap_rows) p.block_tables[e] = c < d(lo).w ? entry(toff[lo], c) : -1;
    } else if (u < u_cu) {  // context length of a plain decode sequence
      const int s = (int)(u - u_ctx);
      p.context_lens[s] = d(s).x;
    } else {  // cu_seqlens entry v of the varlen sequences
      const int v = (int)(u - u_cu);
      p.cu_seqlens_q[v] = pos_off[np_ + v] - np_;
      p.cu_seqlens_k[v] = kpre[np_ + v];
    }
  }
}

}  // namespace

hipError_t launch_build_metadata(const AttnMetaParams& p, int64_t units, hipStream_t stream) {
  if (p.num_seqs <= 0) return hipSuccess;
  if (p.num_seqs > kMetaMaxSeqs) return hipErrorInvalidValue;
  // one unit per lane (each unit is a chain of dependent loads); every
  // workgroup first loads and scans all descriptors, which is short
  const int64_t wgs = std::max<int64_t>(1, std::min<int64_t>(1024, (units + kMetaThreads - 1) / kMetaThreads));
  hipLaunchKernelGGL(build_metadata_kernel, dim3((unsigned)wgs), dim3(kMetaThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace nvamd
