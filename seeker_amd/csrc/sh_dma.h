// Direct global -> LDS loads for double-buffered staging.
//
// One wave's load writes lane l's element at lds + size * l (global_load_lds).
// They are issued as inline asm, not through __builtin_amdgcn_global_load_lds:
// the compiler treats the builtin as an LDS write it cannot place, so before
// every LDS read it waits for all loads in flight (s_waitcnt vmcnt(0)),
// including the next stage's prefetch, and no load overlaps the compute. A
// kernel using these waits for its own stages (s_waitcnt vmcnt) before the
// barrier that publishes a buffer, and for all of them before it ends. The
// compiler cannot count these loads, so its own waits for other loads only
// come out stricter than needed, never looser.
//
// M0 is set here without the compiler's knowledge (clang warns that a
// reserved register is clobbered). A kernel may use these helpers only if
// nothing else in it uses M0: its direct LDS loads all go through here, and
// it has no other M0 user (LDS-direct loads, s_sendmsg, GWS, movrel); checked
// in the gfx950 assembly of the kernels that include this header.
#pragma once
#include <cstdint>

__device__ __forceinline__ uint32_t sh_lds_addr(const void* lds) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane.
__device__ __forceinline__ void sh_dma16(const void* src, const void* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(sh_lds_addr(lds))
               : "memory", "m0");
}
// 4 bytes per lane.
__device__ __forceinline__ void sh_dma4(const void* src, const void* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(sh_lds_addr(lds))
               : "memory", "m0");
}
// The same with the non-temporal hint, for streams read once (weights).
__device__ __forceinline__ void sh_dma16_nt(const void* src, const void* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(sh_lds_addr(lds))
               : "memory", "m0");
}
__device__ __forceinline__ void sh_dma4_nt(const void* src, const void* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off nt" ::"v"(src), "s"(sh_lds_addr(lds))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Waits until at most N of this wave's vector-memory loads are in flight.
template <int N>
__device__ __forceinline__ void sh_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
