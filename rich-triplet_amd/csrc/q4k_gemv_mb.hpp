// q4k_gemv_mb.hpp -- batched Q4_K GEMV (M <= 8 rows) on the int8 matrix
// cores: shared declarations (kernels in q4k_gemv_mb.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rt {

// One weight matrix of a batched GEMV launch: y[m][n] = sum_k A[m][k] w[n][k].
struct MbMat {
  const uint8_t *w;  // Q4_K blocks [n][k/256]
  float *y;          // [M][n]
  int n;
  int row_blocks;    // filled by the launcher
  int part_off;      // filled by the launcher
};

struct MbArgs {
  MbMat mat[3];
  int nmat;
  const int8_t *dig;   // staged activation digits
  const float *stats;  // staged {delta, sum_lo, sum_hi, 0} per (chunk, row)
  int m, k, ksplit, ntot;
  float *part;         // [ksplit][8][ntot] partial sums when ksplit > 1
};

constexpr int kMbMaxRows = 8;

// Device bytes of the staged activations of up to 8 rows of length k.
size_t mb_stage_bytes(int k);
// K slices the launcher uses for n_total output rows, and the partial-sum bytes.
int mb_ksplit(int n_total, int k);
size_t mb_part_bytes(int n_total, int k);
// Stage x[m][k] (row stride k, m <= 8, k % 256 == 0) into `stage`.
hipError_t launch_mb_stage(const float *x, int m, int k, void *stage, hipStream_t s);
// Batched GEMV over up to three matrices sharing the staged activations
// (e.g. q|k|v or gate|up); part holds mb_part_bytes(sum of n, k) bytes.
hipError_t launch_q4k_gemv_mb(const MbMat *mats, int nmat, int m, int k, const void *stage, float *part,
                              hipStream_t s);

}  // namespace rt
