// Hand-off of data between workgroups of one kernel (gfx950).
//
// The L2 caches of the eight XCDs are not coherent with each other for
// ordinary loads and stores, so data one workgroup writes for another goes
// through these agent-coherent accesses, and the protocol is:
//
//   producer: data stores with sh_st_coh16 / sh_st_coh4 (sc1: agent scope, written
//             through past its XCD's L2), then s_waitcnt vmcnt(0) (on gfx9
//             family parts stores count in vmcnt: the wait ends when they
//             are performed at agent scope), then a relaxed agent-scope
//             atomic on the counter or flag;
//   consumer: reads the counter or flag with an agent-scope atomic, and
//             only after its value is known (a control dependency: the
//             loads are issued after the atomic returns) loads the data with
//             sh_ld_coh16 / sh_ld_coh4 (sc1: served at agent scope, never
//             from a stale L2 line).
//
// This is the part of the HIP memory model's agent-scope release / acquire
// that such data needs. The compiler's own release on gfx950 first writes
// back the whole L2 (buffer_wbl2) so that ORDINARY stores become visible, and
// its acquire invalidates the L2 (buffer_inv) so that ORDINARY loads miss;
// here the data itself is stored and loaded at agent scope, so neither is
// needed, and both are expensive (GEMVs whose last-workgroup reductions used
// release / acquire fences ran 3x slower). Only data passed through these
// helpers may cross workgroups this way.
//
// The loads are not tracked by the compiler: their results pass through
// sh_coh_wait (an asm statement holding s_waitcnt vmcnt(0), the values as
// "+v" operands) before any use.
#pragma once
#include <cstdint>

typedef float sh_f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void sh_st_coh16(void* p, sh_f4v v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void sh_st_coh4(void* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ sh_f4v sh_ld_coh16(const void* p) {
  sh_f4v v;
  asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t sh_ld_coh4(const void* p) {
  uint32_t v;
  asm volatile("global_load_dword %0, %1, off sc1" : "=v"(v) : "v"(p) : "memory");
  return v;
}
template <class T>
__device__ __forceinline__ void sh_coh_wait(T& v) {
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(v) : : "memory");
}
// every store of this wave performed (at agent scope for sh_st_coh16)
__device__ __forceinline__ void sh_stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// A pair of doubles as four f32 lanes (bit copies) and back.
__device__ __forceinline__ sh_f4v sh_pack_d2(double x, double y) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  const f2v a = __builtin_bit_cast(f2v, x), b = __builtin_bit_cast(f2v, y);
  return sh_f4v{a[0], a[1], b[0], b[1]};
}
__device__ __forceinline__ void sh_unpack_d2(sh_f4v v, double& x, double& y) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  x = __builtin_bit_cast(double, f2v{v[0], v[1]});
  y = __builtin_bit_cast(double, f2v{v[2], v[3]});
}
