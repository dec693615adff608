// Direct-to-LDS staging helpers shared by the gfx950 kernels: LDS byte
// addresses, raw buffer descriptors, 16-byte buffer loads that land in LDS,
// explicit vmcnt waits and an LDS-only workgroup barrier.
#pragma once

#include "fp8_common.h"

namespace nvamd {

typedef __attribute__((address_space(3))) const uint8_t* lds_cptr_t;

// LDS byte address (the M0 operand of a direct-to-LDS load) of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(lds_cptr_t)p;
}

// Raw buffer descriptor as four dwords (base, stride 0, num_records, word 3).
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t num_bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xFFFFu, num_bytes, (uint32_t)kBufferRsrcWord3};
}

// Direct-to-LDS 16-byte load: lane l's 16 bytes at byte offset voff of the
// buffer land at LDS address lds + 16*l; offsets at or past num_records
// write zeros.  Issued as inline asm so that the compiler's wait-count
// insertion does not treat the pending LDS write as a hazard on every later
// LDS access (it would wait for all loads in flight); completion is tracked
// explicitly with wait_vmcnt + lds_barrier.  s_nop: one wait state between
// the M0 write and the LDS-DMA instruction that reads it.  The statement is
// volatile, so it stays ordered with the barrier and s_waitcnt intrinsics;
// no memory clobber is declared so the compiler can keep the block-table
// reads on the scalar path (no kernel code stores to the cache or tables).
// The M0 write needs no clobber: this code uses M0 only for these loads.
// dma_load16 is non-temporal (nt), for streams whose bytes are read once
// per call: streaming the decode KV cache past the caches' normal retention
// measured 10-12% faster (its cache lines are never reused).
// dma_load16_keep uses the default policy, for tiles other workgroups re-read.
__device__ __forceinline__ void dma_load16(u32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen nt lds"
      :
      : "s"(lds), "v"(voff), "s"(rsrc));
}

__device__ __forceinline__ void dma_load16_keep(u32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds), "v"(voff), "s"(rsrc));
}

// Direct-to-LDS 4-byte load: lane l's dword at byte offset voff lands at LDS
// address lds + 4*l (default cache policy; same conventions as above).
__device__ __forceinline__ void dma_load4_keep(u32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, 0 offen lds"
      :
      : "s"(lds), "v"(voff), "s"(rsrc));
}

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt left unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier that orders LDS only: loads to VGPRs or LDS that are still
// in flight stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace nvamd
