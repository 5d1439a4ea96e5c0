// q4k_gemm_dev.hpp -- device pieces shared by the Q4_K GEMM kernels
// (q4k_gemm.hip, q4k_gemm_wide.hip): the K chunk, the dequantisation step
// into an MFMA B operand, and the matrix set of a one-launch projection set.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_common.hpp"
#include "rt_device.hpp"

namespace rt {

constexpr int kBK = 64;  // K per pipeline stage = one Q4_K chunk (32 qs bytes, 2 sub-blocks)

// ---------------------------------------------------------------------------
// Matrix-core kernels.  Both use v_mfma_f32_32x32x16_f16 (lane l: A row / B
// column l%32, k group g = l/32, 8 halves each) and the same K order inside a
// 64-wide chunk (A and B agree on it, so the sum is unchanged):
//   lane group g holds qs bytes [16g, 16g+16) of the chunk's 32; k-step t
//   (0..3) covers chunk-local k = 16g + 8(t&1) + 32(t>>1) + [0, 8): t < 2 are
//   the low nibbles (sub-block 2c), t >= 2 the high nibbles of the same
//   bytes (sub-block 2c+1).
// A (and in the eight-wave kernel the packed W bytes) reaches LDS by
// global_load_lds_dwordx4 (no VGPRs, no ds_write); each ring slot is its own
// __shared__ variable.  Every lane dequantises the qs bytes of its own column
// straight into the MFMA B operand, so no dequantised weight is written back
// to LDS.
// ---------------------------------------------------------------------------
// Eight f16 weights of one k-step from two qs words (low or high nibbles).
// v_perm builds halves 1024+q (low nibbles) or 1024+16q (high nibbles), and
// each v_fma_mix computes f16(s*h - c) from them in f32 with one rounding.
// The eight v_fma_mix sit in one asm block that ends with two wait states:
// the compiler's hazard recognizer cannot tell that an asm block is VALU
// work, so it would not separate it from an MFMA that reads its result
// (a VALU write followed by an MFMA read of that VGPR needs two wait states).
template <bool HIGH>
RT_DEV half8 dq_step(uint32_t w0, uint32_t w1, float s, float negc) {
  const uint32_t mask = HIGH ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
  const uint32_t a = w0 & mask, b = w1 & mask;
  const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
  const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
  const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
  const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
  uint32_t r0, r1, r2, r3;
  asm("v_fma_mixlo_f16 %0, %8, %4, %9 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %0, %8, %4, %9 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %1, %8, %5, %9 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %1, %8, %5, %9 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %2, %8, %6, %9 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %2, %8, %6, %9 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %3, %8, %7, %9 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %3, %8, %7, %9 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "s_nop 1"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(p0), "v"(p1), "v"(p2), "v"(p3), "v"(s), "v"(negc));
  const u32x4 r = {r0, r1, r2, r3};
  return __builtin_bit_cast(half8, r);
}

// Up to three matrices sharing A (q|k|v, gate|up) in one launch: their
// 256-column tiles are numbered one after another (tn0), and a workgroup
// takes the matrix its column tile falls in.
struct HMats {
  const uint8_t *w[3];
  const int *ew[3];
  float *c[3];
  int n[3];
  int tn0[3];  // first column tile of each matrix
  int count;
};

// The 256 x 256-tile kernel (q4k_gemm_wide.hip) on prepared operands:
// tiles_n column tiles of 256 over the matrices of `mats`, K split ksplit
// ways (1 <= ksplit <= K/256); with ksplit > 1 the matrix's c receives
// ksplit partial products of M x N, one after another.
hipError_t launch_q4k_gemm_wide(const _Float16 *a16, const int *ea, const HMats &mats, int M, int K, int tiles_n,
                                int ksplit, hipStream_t s);

}  // namespace rt
