// HBM -> LDS DMA helpers shared by the GEMM and router kernels (gfx950).
#pragma once

#include "common.h"

namespace moe {

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// s_waitcnt with only the LDS/scalar counter constrained, to zero.
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char_t;

// One 1 KiB LDS DMA: 64 lanes x 16 bytes from `rsrc` + voffset into LDS at
// M0 (lane-ordered).  Issued from inline assembly so that the compiler does
// not add its own (conservative) waits for the asynchronous LDS write: the
// kernel waits for each k-tile with an explicit vmcnt and a barrier.
// The descriptor is passed as four scalar words (base, base high, byte size,
// format flags: the same words __builtin_amdgcn_make_buffer_rsrc builds).
// The compiler's hazard recognizer does not look inside the asm, so the asm
// supplies the wait states itself: 5 cover a VALU write of the descriptor
// SGPRs (v_readfirstlane, or a v_readlane restoring spilled SGPRs) right
// before the load, and the 1 needed after the write of M0.
__device__ __forceinline__ void dma16(u32x4_t rsrc, uint32_t voffset, uint32_t lds_addr) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voffset), "s"(rsrc), "{m0}"(lds_addr)
               : "memory");
}

__device__ __forceinline__ u32x4_t rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(base);
  const uint32_t w0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t w1 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32)) & 0xffffu;
  const uint32_t w2 = __builtin_amdgcn_readfirstlane(bytes);
  return u32x4_t{w0, w1, w2, 0x00020000u};
}

__device__ __forceinline__ uint32_t lds_address(const char* p) {
  // The generic -> LDS address-space cast yields the 32-bit LDS byte address.
  return (uint32_t)(uintptr_t)(const lds_char_t*)p;
}

}  // namespace moe
