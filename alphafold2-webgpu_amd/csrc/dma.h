// Direct global -> LDS loads for gfx950 (buffer_load_dword{,x4} ... lds).
//
// Each lane of a wave-level instruction loads `size` bytes from its own byte
// offset into a raw buffer resource; the data lands in LDS at
// M0 + size * lane, M0 being the wave-uniform destination passed in. Loads at
// offsets at or beyond the resource's byte count return zeros, which is how
// the kernels zero-fill ragged tiles: an offset of kOutOfRange is always
// beyond.
//
// The loads are issued from inline assembly, so the compiler does not track
// them: it would otherwise drain every in-flight load (s_waitcnt vmcnt(0))
// before LDS accesses it cannot prove disjoint from the DMA's destination.
// They count in vmcnt like any vector-memory instruction, in issue order;
// a kernel waits for one with wait_vmcnt<N>(), N being the number of
// vector-memory instructions the wave issued after it. Untracked loads only
// make the compiler's own vmcnt waits stricter, never looser, since every
// vector-memory instruction completes in order.
//
// M0 is an input operand of each statement ("{m0}"): the compiler writes it
// itself right before the statement and knows what M0 holds afterwards, so
// it never assumes a value of its own survived there.
#pragma once

#include "internal.h"

namespace afhip {

typedef int int32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kOutOfRange = 0x80000000u;

// 16 bytes per lane into LDS [lds, lds + 1024). `lds` must be wave-uniform;
// readfirstlane puts it in a scalar register even where the compiler cannot
// prove that. The s_nop covers the one wait state between writing M0 and
// its use.
__device__ __forceinline__ void dma16(int32x4_t rsrc, uint32_t lds, uint32_t voffset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voffset), "s"(rsrc), "{m0}"(m0)
               : "memory");
}

// dma16 with a wave-uniform byte offset added to every lane's (soffset).
__device__ __forceinline__ void dma16_so(int32x4_t rsrc, uint32_t lds, uint32_t voffset, uint32_t soffset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soffset);
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voffset), "s"(rsrc), "s"(so),
               "{m0}"(m0)
               : "memory");
}

// dma4 with a wave-uniform byte offset added to every lane's (soffset).
__device__ __forceinline__ void dma4_so(int32x4_t rsrc, uint32_t lds, uint32_t voffset, uint32_t soffset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soffset);
  asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voffset), "s"(rsrc), "s"(so),
               "{m0}"(m0)
               : "memory");
}

// dma16 when `enable` (wave-uniform) is nonzero. The test and the skip are
// inside the statement, so a caller's straight-line code stays one basic
// block the compiler can schedule MFMAs and VALU work across.
__device__ __forceinline__ void dma16_if(int32x4_t rsrc, uint32_t lds, uint32_t voffset, int enable) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  const int on = __builtin_amdgcn_readfirstlane(enable);
  asm volatile(
      "s_cmp_eq_u32 %2, 0\n\ts_cbranch_scc1 1f\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds\n1:" ::"v"(voffset), "s"(rsrc), "s"(on), "{m0}"(m0)
      : "memory", "scc");
}

// 4 bytes per lane into LDS [lds, lds + 256).
__device__ __forceinline__ void dma4(int32x4_t rsrc, uint32_t lds, uint32_t voffset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voffset), "s"(rsrc), "{m0}"(m0)
               : "memory");
}

// Raw buffer resource (stride 0) over `bytes` bytes from `base`.
__device__ __forceinline__ int32x4_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  int32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left at their maxima), issued as
// the builtin so the compiler's own wait insertion sees it.
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt holds at most 63 outstanding instructions");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
  asm volatile("" ::: "memory");
}

// s_barrier with compiler fences on both sides, without the release/acquire
// waits __syncthreads() adds: callers wait for their own loads explicitly.
// gfx950 does not drain LDS traffic at a barrier by itself, so a barrier
// that publishes this wave's LDS stores first waits for them (lds = true).
template <bool lds = true> __device__ __forceinline__ void block_barrier() {
  if (lds) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  else asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace afhip
