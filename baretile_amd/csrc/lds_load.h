// Loads straight into LDS (`buffer_load ... lds`) and the waits for them, shared by the kernels that stage their
// operands that way (matmul.hip's streaming and GEMM kernels, attention.hip's prefill).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace bt {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// A buffer resource as four dwords, for inline assembly: base, stride 0, `bytes` records, the same flags as buffer().
__device__ __forceinline__ i32x4 buffer_words(const void *base, uint32_t bytes) {
  const uint64_t p = (uint64_t)(uintptr_t)base;
  return i32x4{(int)(uint32_t)p, (int)(uint32_t)(p >> 32) & 0xFFFF, (int)bytes, 0x00020000};
}

// 16 bytes a lane from the buffer at voff into LDS at lds + 16 * lane: one wave writes 1 KB. Issued as assembly so
// that the compiler, which can't tell which LDS bytes such a load writes, doesn't wait for every one of them before
// each LDS read; the kernel waits for them itself (wait_vm). Loads complete in order, so the compiler's own waits
// on other loads stay correct (at worst they wait for these too).
// The resource is wave-uniform; readfirstlane hands it to the assembly in scalar registers even where the compiler
// would otherwise keep a copy in vector registers.
__device__ __forceinline__ i32x4 uniform_words(const i32x4 &w) {
  return i32x4{__builtin_amdgcn_readfirstlane(w.x), __builtin_amdgcn_readfirstlane(w.y),
               __builtin_amdgcn_readfirstlane(w.z), __builtin_amdgcn_readfirstlane(w.w)};
}
__device__ __forceinline__ void lds_load16(const i32x4 &rsrc, uint32_t voff, const void *lds) {
  const uint32_t at = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(uniform_words(rsrc)), "s"(at)
               : "memory", "m0");
}

// 4 bytes a lane from the buffer at voff into LDS at lds + 4 * lane, as lds_load16.
__device__ __forceinline__ void lds_load4(const i32x4 &rsrc, uint32_t voff, const void *lds) {
  const uint32_t at = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(uniform_words(rsrc)), "s"(at)
               : "memory", "m0");
}

// Waits until at most N vector memory loads of this wave are outstanding. Assembly too: the compiler would drop a
// wait for loads it doesn't know of.
template <int N> __device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

}  // namespace bt
