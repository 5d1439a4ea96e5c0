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


// Stores a wave's C tile from v_mfma_f32_32x32x16 accumulators: four row
// tiles of 32 rows by NT column tiles of 32 columns, register r of tile (i, j)
// being C[row0 + 32i + 8(r/4) + 4(lane/32) + r%4][col0 + 32j + lane%32],
// scaled by 2^(ea[row] + ecol[j]).  One 32-row slice at a time goes through
// `stage` (32 x (32NT + 8) floats of LDS that only this wave uses; the pitch
// puts the two row groups of a 4-byte write on disjoint banks) and leaves as
// whole rows in 16-byte lanes, so no store waits on a load and every store
// instruction writes full row pieces.
template <int NT>
RT_DEV void store_c_tile(const floatx16 (&acc)[4][NT], float *stage, float *c, int M, int N, int row0, int col0,
                         const int *ea, const int (&ecol)[NT]) {
  constexpr int P = 32 * NT + 8, F4 = 8 * NT, RPI = 64 / F4;
  const int lane = (int)(threadIdx.x & 63), g = lane >> 5, l32 = lane & 31;
  const bool vec = (N & 3) == 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int er[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) er[r] = ea[min(row0 + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3), M - 1)];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        stage[(8 * (r >> 2) + 4 * g + (r & 3)) * P + 32 * j + l32] =
            __builtin_amdgcn_ldexpf(acc[i][j][r], er[r] + ecol[j]);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < 32 / RPI; ++q) {
      const int rl = q * RPI + lane / F4, f = lane % F4;
      const int row = row0 + 32 * i + rl, col = col0 + 4 * f;
      const float4 v = *reinterpret_cast<const float4 *>(stage + rl * P + 4 * f);
      if (row < M) {
        float *dst = c + (size_t)row * N + col;
        if (vec && col + 4 <= N) {
          *reinterpret_cast<float4 *>(dst) = v;
        } else {
          if (col < N) dst[0] = v.x;
          if (col + 1 < N) dst[1] = v.y;
          if (col + 2 < N) dst[2] = v.z;
          if (col + 3 < N) dst[3] = v.w;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

}  // namespace rt
