// Direct global -> LDS copies (global_load_lds) and explicit vmcnt waits,
// shared by the kernels that stream operands into LDS.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qc {

// Waits until at most N vector-memory loads of this wave are outstanding
// (they retire in issue order).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Waits until at most min(n, MAXN) loads are outstanding; n must fold to a
// constant (an unrolled loop index), leaving one s_waitcnt.
template <int MAXN>
__device__ __forceinline__ void wait_vmcnt_le(int n) {
  if constexpr (MAXN <= 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= MAXN) wait_vmcnt<MAXN>();
    else wait_vmcnt_le<MAXN - 1>(n);
  }
}

// The helpers below load M0 (the LDS base of global_load_lds) and list it as
// clobbered; clang warns for any clobber of M0 as a reserved register,
// which is the intent here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"

// global_load_lds_dwordx4 from a wave-uniform base (scalar registers) plus a
// per-lane byte offset, to LDS byte lds + 16 * lane (lds wave-uniform, in
// M0).  Written as inline assembly so the compiler, which cannot see that
// the ring slots read next are not the ones being filled, adds no waits of
// its own: the kernels wait for these loads explicitly (wait_vmcnt) before
// any read of the data and before the workgroup ends.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, const void* lds) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));  // LDS offset
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(base), "s"(m0)
      : "memory", "m0");
}

// Same with a per-lane 64-bit address (used only for a short last stage).
__device__ __forceinline__ void dma16_addr(const void* addr, const void* lds) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(addr), "s"(m0)
      : "memory", "m0");
}
// One dword per lane from a wave-uniform base plus a per-lane byte offset to
// LDS byte lds + 4 * lane.
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, const void* lds) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %0, %1"
      :
      : "v"(voff), "s"(base), "s"(m0)
      : "memory", "m0");
}
#pragma clang diagnostic pop

}  // namespace qc
