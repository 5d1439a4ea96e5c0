// mfma_common.hpp -- shared pieces of the matrix-core GEMM kernels
// (q4k_gemm.hip, proj_gemm.hip): operand vector types, explicit wait counts,
// a barrier without the release fence, and LDS reads the compiler's
// wait-count pass does not track.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rt_device.hpp"

namespace rt {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
// Native vectors for staging registers: HIP's uint4 is a union-wrapped struct
// whose copies become memcpys, which LLVM turns back into global reloads.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

// s_waitcnt with only a vector-memory bound (expcnt / lgkmcnt left open), gfx9 encoding.
template <int N>
RT_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// s_waitcnt lgkmcnt(0) alone (vmcnt 63 and expcnt 7 mean "no wait").
RT_DEV void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }
// Workgroup barrier that keeps memory operations on their side of it in the
// compiler (s_barrier alone is a no-memory intrinsic) without the release
// fence's wait for every outstanding load.
RT_DEV void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS reads the compiler does not see as LDS reads.  Its wait insertion
// cannot tell which ring slot an in-flight global_load_lds targets once the
// loop back-edge merges its state, and would drain every copy (vmcnt(0))
// before the first read of each block.  The kernel orders the copies itself
// (explicit vmcnt + barrier per chunk) and waits for these reads with
// lds_wait, whose register operands keep every consumer after the wait.
RT_DEV u32x4 lds_read16(const void *p) {
  u32x4 v;
  const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a));
  return v;
}
RT_DEV void lds_wait(u32x4 &a, u32x4 &b, u32x4 &c, u32x4 &d) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}


}  // namespace rt
