// FP8 varlen causal (chunked) prefill for gfx950, paged and contiguous KV.
//
// Replaces fp8_paged_attention_prefill_kernel (nanovllm/kernels/fp8_attention.py:209-312).
// Sequence s owns query rows [cu_q[s], cu_q[s+1]) and Lk = cu_k[s+1]-cu_k[s]
// keys; query row i sees key j iff j <= i + (Lk - Lq) (bottom-right aligned
// causal mask, fp8_attention.py:237,267,297).  Keys come from the paged
// cache through block_tables[s], or from contiguous K/V rows
// [cu_k[s], cu_k[s+1]) when block_tables is NULL (fp8_attention.py:254-278).
//
// Workgroup = 4 waves = 128 query rows = GW query heads (all sharing one kv
// head, GQA) x BM = 128/GW query tokens.  Wave w owns 32 rows: head
// (w % GW), tokens [m0 + 32*(w / GW), +32).  K/V are streamed in 64-token
// tiles: the workgroup loads each FP8 tile from HBM once, converts it to
// bf16 (exact) and stages it in LDS -- K as [token][dim], V transposed as
// [dim][token] -- so every wave reads its MFMA operands with 16-byte LDS
// reads.  The next tile's global loads are issued before the current tile
// is computed.
//
// Per tile a wave computes with v_mfma_f32_32x32x16_bf16 (fp32 accumulate):
//     S^T[kv][q] = K[kv][:] . Q[q][:]          2 row blocks x 8 k-steps
//     O^T[d][q] += V^T[d][kv] . P^T[kv][q]     4 dim blocks x 4 k-steps
// Lane l (h = l / 32) holds query column l % 32; in the S^T result it holds
// kv tokens (i%4) + 8(i/4) + 4h of each 32-token row block, so the PV
// operand for k-step ks is simply p[ks/2][8(ks%2) .. +8) once V^T is stored
// with bits 2 and 3 of the token index swapped inside each 16-token step.
// The causal mask is applied in registers only on tiles that cross the
// diagonal (or the end of the sequence); tiles wholly above a wave's rows
// are skipped.
#include "fp8_common.h"
#include "kernels.h"

namespace nvamd {

namespace {

constexpr int kBN = 64;                   // kv tokens per tile
constexpr int kKPitch = kHeadDim + 8;     // bf16 elements per K row in LDS (272 B)
constexpr int kVPitch = kBN + 8;          // bf16 elements per V^T row in LDS (144 B)

struct TileRegs {
  u32x4 k[2];   // 32 fp8 of one K row
  u32x2 v[4];   // 8 fp8 (dims [8c, +8)) of 4 consecutive tokens
};

// position of token t (0..63) inside the transposed V tile
__device__ __forceinline__ int v_pos(int t) {
  const int b2 = (t >> 2) & 1, b3 = (t >> 3) & 1;
  return (t & ~12) | (b2 << 3) | (b3 << 2);
}

}  // namespace

__global__ __launch_bounds__(256) void varlen_prefill_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kBN * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[kHeadDim * kVPitch];

  const int mb = p.n_mblocks - 1 - (int)blockIdx.x;  // longest causal rows first
  const int seq = blockIdx.y;
  const int g = blockIdx.z / p.n_hgroups;
  const int hg = blockIdx.z - g * p.n_hgroups;

  const int q_start = p.cu_q[seq];
  const int Lq = p.cu_q[seq + 1] - q_start;
  if (Lq <= p.mq_max_q) return;          // short queries: multi-query kernel
  const int m0 = mb * p.BM;
  if (m0 >= Lq) return;
  const int k_start = p.cu_k[seq];
  const int Lk = p.cu_k[seq + 1] - k_start;
  const int c = Lk - Lq;                 // cached context before the chunk

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_uniform(tid >> 6);
  const int h = lane >> 5, col = lane & 31;
  const int hw = wave % p.GW, tw = wave / p.GW;
  const int head = g * p.G + hg * p.GW + hw;
  const int m0w = m0 + 32 * tw;          // first query token of this wave
  const int tq = m0w + col;              // this lane's query token

  // ---- Q operand (B of S^T): dims 16ks + 8h + [0,8) --------------------------
  bf16x8 qop[8];
  {
    const int64_t row = (int64_t)q_start + tq;
    const bool valid = tq < Lq && row < p.q_rows;
    const uint16_t* qp = p.q + (row * p.Hq + head) * kHeadDim + 8 * h;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      u32x4 a = {0u, 0u, 0u, 0u};
      if (valid) a = *reinterpret_cast<const u32x4*>(qp + 16 * ks);
      qop[ks] = as_bf16x8(a);
    }
  }

  f32x16 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  int kv_hi = min(Lk, c + m0 + p.BM);        // keys visible to the last row of the block
  if (p.block_tables != nullptr)             // the block table bounds the addressable keys
    kv_hi = (int)min((int64_t)kv_hi, p.bt_stride * (int64_t)p.block_size);
  const int n_tiles = (kv_hi + kBN - 1) / kBN;

  // staging assignment
  const int sk_tok = tid >> 2, sk_off = (tid & 3) * 32;        // K: 32 B of one row
  const int sv_tg = tid >> 4, sv_d0 = (tid & 15) * 8;          // V: 4 tokens x 8 dims

  auto tile_row0 = [&](int kv0, int64_t& row0) -> bool {
    if (p.block_tables != nullptr) {
      const int bi = kv0 / p.block_size;
      if (bi >= p.bt_stride) return false;
      const int blk = wave_uniform(p.block_tables[(int64_t)seq * p.bt_stride + bi]);
      row0 = (int64_t)blk * p.block_size + (kv0 % p.block_size);
      return blk >= 0 && row0 + kBN <= p.kv_rows;
    }
    row0 = (int64_t)k_start + kv0;
    return row0 >= 0 && row0 + min(kBN, Lk - kv0) <= p.kv_rows;
  };

  auto load_tile = [&](int kv0, TileRegs& tr) {
    int64_t row0;
    const bool ok = tile_row0(kv0, row0);
    const int nvalid = ok ? min(kBN, Lk - kv0) : 0;
    {
      u32x4 z = {0u, 0u, 0u, 0u};
      tr.k[0] = z;
      tr.k[1] = z;
      if (sk_tok < nvalid) {
        const uint8_t* kp = p.k + ((row0 + sk_tok) * p.Hkv + g) * kHeadDim + sk_off;
        tr.k[0] = *reinterpret_cast<const u32x4*>(kp);
        tr.k[1] = *reinterpret_cast<const u32x4*>(kp + 16);
      }
    }
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int t = 4 * sv_tg + x;
      u32x2 z = {0u, 0u};
      if (t < nvalid) z = *reinterpret_cast<const u32x2*>(p.v + ((row0 + t) * p.Hkv + g) * kHeadDim + sv_d0);
      tr.v[x] = z;
    }
  };

  auto stage_tile = [&](const TileRegs& tr) {
    // K row: 32 fp8 -> 32 bf16 (64 B) at k_lds[sk_tok][sk_off ..]
    uint16_t* kd = k_lds + sk_tok * kKPitch + sk_off;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const u32x4 w = tr.k[q];
      u32x4 lo, hi;
      lo.x = fp8x2_to_bf16x2<false>(w.x); lo.y = fp8x2_to_bf16x2<true>(w.x);
      lo.z = fp8x2_to_bf16x2<false>(w.y); lo.w = fp8x2_to_bf16x2<true>(w.y);
      hi.x = fp8x2_to_bf16x2<false>(w.z); hi.y = fp8x2_to_bf16x2<true>(w.z);
      hi.z = fp8x2_to_bf16x2<false>(w.w); hi.w = fp8x2_to_bf16x2<true>(w.w);
      *reinterpret_cast<u32x4*>(kd + 16 * q) = lo;
      *reinterpret_cast<u32x4*>(kd + 16 * q + 8) = hi;
    }
    // V: transpose 4 tokens x 8 dims; write dim rows of 4 tokens (8 B) each
    const int pos = v_pos(4 * sv_tg);  // tokens 4tg..4tg+3 stay contiguous
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t a = half ? tr.v[0].y : tr.v[0].x;
      const uint32_t b = half ? tr.v[1].y : tr.v[1].x;
      const uint32_t cc = half ? tr.v[2].y : tr.v[2].x;
      const uint32_t d = half ? tr.v[3].y : tr.v[3].x;
      const uint32_t x01 = __builtin_amdgcn_perm(a, b, 0x01050004u);   // [a0 b0 a1 b1]
      const uint32_t y01 = __builtin_amdgcn_perm(cc, d, 0x01050004u);  // [c0 d0 c1 d1]
      const uint32_t x23 = __builtin_amdgcn_perm(a, b, 0x03070206u);   // [a2 b2 a3 b3]
      const uint32_t y23 = __builtin_amdgcn_perm(cc, d, 0x03070206u);  // [c2 d2 c3 d3]
      const uint32_t t0 = __builtin_amdgcn_perm(x01, y01, 0x01000504u); // [a0 b0 c0 d0]
      const uint32_t t1 = __builtin_amdgcn_perm(x01, y01, 0x03020706u); // [a1 b1 c1 d1]
      const uint32_t t2 = __builtin_amdgcn_perm(x23, y23, 0x01000504u); // [a2 b2 c2 d2]
      const uint32_t t3 = __builtin_amdgcn_perm(x23, y23, 0x03020706u); // [a3 b3 c3 d3]
      const uint32_t tt[4] = {t0, t1, t2, t3};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int dim = sv_d0 + 4 * half + e;
        *reinterpret_cast<u32x2*>(v_lds + dim * kVPitch + pos) = fp8x4_to_bf16x4(tt[e]);
      }
    }
  };

  TileRegs tr;
  if (n_tiles > 0) load_tile(0, tr);

  for (int t = 0; t < n_tiles; ++t) {
    const int kv0 = t * kBN;
    __syncthreads();          // previous tile fully consumed
    stage_tile(tr);
    __syncthreads();
    if (t + 1 < n_tiles) load_tile(kv0 + kBN, tr);

    // Tile wholly above this wave's causal diagonal: nothing to do.
    if (kv0 > c + m0w + 31) continue;
    const bool need_mask = (kv0 + kBN - 1 > c + m0w) || (kv0 + kBN > Lk);

    // ---- S^T = K . Q^T ----------------------------------------------------------
    f32x16 s[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      f32x16 a;
#pragma unroll
      for (int i = 0; i < 16; ++i) a[i] = 0.f;
      const uint16_t* kr = k_lds + (32 * rb + col) * kKPitch + 8 * h;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const bf16x8 kop = as_bf16x8(*reinterpret_cast<const u32x4*>(kr + 16 * ks));
        a = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, qop[ks], a, 0, 0, 0);
      }
      s[rb] = a;
    }

    // ---- online softmax (row = query column of this lane) -----------------------
    float mx = -INFINITY;
    const int lim = c + tq;  // last visible key
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float sv = s[rb][i] * p.scale_log2;
        if (need_mask) {
          const int j = kv0 + 32 * rb + (i & 3) + 8 * (i >> 2) + 4 * h;
          sv = (j <= lim && j < Lk) ? sv : -INFINITY;
        }
        s[rb][i] = sv;
        mx = fmaxf(mx, sv);
      }
    }
    mx = fmaxf(mx, shfl_xor_f32(mx, 32));
    // Lazy rescale (see kLazyRescaleLog2).
    const bool grow = mx > m_run + kLazyRescaleLog2;
    if (wave_any(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = grow ? fast_exp2(m_run - m_new) : 1.f;
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
    }
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
    float ps = 0.f;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e = fast_exp2(s[rb][i] - m_use);
        s[rb][i] = e;
        ps += e;
      }
    }
    l_run += ps;

    // ---- O^T += V^T . P^T ---------------------------------------------------------
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int rb = ks >> 1, base = 8 * (ks & 1);
      const bf16x8 pop = as_bf16x8(pack_bf16x2(s[rb][base + 0], s[rb][base + 1]),
                                   pack_bf16x2(s[rb][base + 2], s[rb][base + 3]),
                                   pack_bf16x2(s[rb][base + 4], s[rb][base + 5]),
                                   pack_bf16x2(s[rb][base + 6], s[rb][base + 7]));
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x8 vop = as_bf16x8(
            *reinterpret_cast<const u32x4*>(v_lds + (32 * db + col) * kVPitch + 16 * ks + 8 * h));
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop, pop, acc[db], 0, 0, 0);
      }
    }
  }

  // ---- normalise and store ----------------------------------------------------------
  l_run += shfl_xor_f32(l_run, 32);
  const int64_t row = (int64_t)q_start + tq;
  if (tq < Lq && row < p.q_rows) {
    const float inv = (l_run > 0.f) ? 1.0f / l_run : 0.f;
    uint16_t* op = p.out + (row * p.Hq + head) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int b4 = 0; b4 < 4; ++b4) {
        const int d = 32 * db + 8 * b4 + 4 * h;
        u32x2 w;
        w.x = out_round_bf16_bits(acc[db][4 * b4 + 0] * inv) | (out_round_bf16_bits(acc[db][4 * b4 + 1] * inv) << 16);
        w.y = out_round_bf16_bits(acc[db][4 * b4 + 2] * inv) | (out_round_bf16_bits(acc[db][4 * b4 + 3] * inv) << 16);
        *reinterpret_cast<u32x2*>(op + d) = w;
      }
    }
  }
}

hipError_t launch_varlen_prefill(const PrefillParams& p, hipStream_t stream) {
  if (p.num_seqs == 0 || p.n_mblocks == 0) return hipSuccess;
  const dim3 grid((unsigned)p.n_mblocks, (unsigned)p.num_seqs, (unsigned)(p.Hkv * p.n_hgroups));
  hipLaunchKernelGGL(varlen_prefill_kernel, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace nvamd
