// q4k_gemv_mb.hpp -- batched Q4_K GEMV (M <= 8 rows) on the int8 matrix
// cores: shared declarations (kernels in q4k_gemv_mb.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "rt_device.hpp"

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

// The matrix of a launch that workgroup column rb falls in, and rb within it.
// Constant indices only: every row_blocks and pointer is read from the kernel
// arguments at once and then selected (a loop over them makes a chain of
// dependent scalar loads ahead of the workgroup's first memory loads).
RT_DEV MbMat mb_pick(const MbArgs &p, int &rb) {
  const int c1 = p.mat[0].row_blocks, c2 = c1 + p.mat[1].row_blocks;
  const bool in1 = p.nmat > 1 && rb >= c1, in2 = p.nmat > 2 && rb >= c2;
  rb -= in2 ? c2 : (in1 ? c1 : 0);
  MbMat m;
  m.w = in2 ? p.mat[2].w : (in1 ? p.mat[1].w : p.mat[0].w);
  m.y = in2 ? p.mat[2].y : (in1 ? p.mat[1].y : p.mat[0].y);
  m.n = in2 ? p.mat[2].n : (in1 ? p.mat[1].n : p.mat[0].n);
  m.row_blocks = in2 ? p.mat[2].row_blocks : (in1 ? p.mat[1].row_blocks : p.mat[0].row_blocks);
  m.part_off = in2 ? p.mat[2].part_off : (in1 ? p.mat[1].part_off : p.mat[0].part_off);
  return m;
}

// A [rows][cols] f32 operand that may be split-K partial sums: element (t, i)
// = sum over z < ks of p[z*slice_stride + t*row_stride + col_off + i], added
// in slice order (col_off, row_stride, slice_stride and i multiples of 4 for
// the float4 read).
struct RowsIn {
  const float *p;
  int ks;
  size_t slice_stride;
  int row_stride, col_off;
};
__host__ __device__ inline RowsIn rows_plain(const float *p, int cols) { return RowsIn{p, 1, 0, cols, 0}; }

// Slices are loaded sixteen at a time (the last group at clamped, in-bounds
// slices that are not added), all sixteen in flight, then added in slice
// order: one round trip for the ten slices of a k = 2560 GEMV.
__device__ __forceinline__ float4 rows_in4(const RowsIn &r, int t, int i) {
  const float *b = r.p + (size_t)t * r.row_stride + r.col_off + i;
  float4 s = *reinterpret_cast<const float4 *>(b);
  for (int z = 1; z < r.ks; z += 16) {
    float4 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = *reinterpret_cast<const float4 *>(b + (size_t)min(z + u, r.ks - 1) * r.slice_stride);
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (z + u < r.ks) s.x += v[u].x, s.y += v[u].y, s.z += v[u].z, s.w += v[u].w;
  }
  return s;
}
// rows_in4 for at most four slices (the prefill GEMMs' split-K partials,
// each read once: nontemporal loads), without the sixteen-slice batch.
__device__ __forceinline__ float4 rows_in4_few(const RowsIn &r, int t, int i) {
  const float *b = r.p + (size_t)t * r.row_stride + r.col_off + i;
  float4 v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint4 q = ld_nt16(b + (size_t)min(u, r.ks - 1) * r.slice_stride);
    v[u] = make_float4(__uint_as_float(q.x), __uint_as_float(q.y), __uint_as_float(q.z), __uint_as_float(q.w));
  }
  float4 s = v[0];
#pragma unroll
  for (int u = 1; u < 4; ++u)
    if (u < r.ks) s.x += v[u].x, s.y += v[u].y, s.z += v[u].z, s.w += v[u].w;
  return s;
}
__device__ __forceinline__ float2 rows_in2(const RowsIn &r, int t, int i) {  // i even
  const float *b = r.p + (size_t)t * r.row_stride + r.col_off + i;
  float2 s = *reinterpret_cast<const float2 *>(b);
  for (int z = 1; z < r.ks; z += 16) {
    float2 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = *reinterpret_cast<const float2 *>(b + (size_t)min(z + u, r.ks - 1) * r.slice_stride);
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (z + u < r.ks) s.x += v[u].x, s.y += v[u].y;
  }
  return s;
}
__device__ __forceinline__ float rows_in1(const RowsIn &r, int t, int i) {
  const float *b = r.p + (size_t)t * r.row_stride + r.col_off + i;
  float s = *b;
  for (int z = 1; z < r.ks; z += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = b[(size_t)min(z + u, r.ks - 1) * r.slice_stride];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (z + u < r.ks) s += v[u];
  }
  return s;
}

// Device bytes of the staged activations of up to 8 rows of length k.
size_t mb_stage_bytes(int k);
// K slices the launcher uses for n_total output rows, and the partial-sum bytes.
int mb_ksplit(int n_total, int k);
size_t mb_part_bytes(int n_total, int k);
// Staged statistics of a stage buffer for rows of length k.
__host__ __device__ inline float *mb_stats(void *stage, int k) {
  return reinterpret_cast<float *>(static_cast<int8_t *>(stage) + (size_t)(k / 64) * 8 * 128);
}
// Stage x[m][k] (row stride k, m <= 8, k % 256 == 0) into `stage`.
hipError_t launch_mb_stage(const float *x, int m, int k, void *stage, hipStream_t s);
// Batched GEMV over up to three matrices sharing the staged activations
// (e.g. q|k|v or gate|up); part holds mb_part_bytes(sum of n, k) bytes.
// With `views`, split-K partial sums are left in `part` and views[i] reads
// matrix i's result (the consumer adds the slices); without, a reduction
// kernel writes every matrix's y.
hipError_t launch_q4k_gemv_mb(const MbMat *mats, int nmat, int m, int k, const void *stage, float *part,
                              hipStream_t s, RowsIn *views = nullptr);
// y of every matrix of p from its split-K partial sums (slice order).
hipError_t launch_mb_reduce(const MbArgs &p, hipStream_t s);
// One matrix of n rows (an lm_head): y[m][n] from the staged activations,
// the whole row per workgroup where K allows; part holds
// mb_head_part_bytes(n, k) bytes (0 for k of 2 or 10 super-blocks).
size_t mb_head_part_bytes(int n, int k);
hipError_t launch_q4k_gemv_mb_head(const uint8_t *w, float *y, int n, int m, int k, const void *stage, float *part,
                                   hipStream_t s);

// The same batched GEMV for Q8_0 and Q6_K weights (planar layout, from the
// staged digits) and BF16 weights (from the f32 rows x[m][k] themselves),
// kquant_mb.hip.  k: a multiple of 256 for Q6_K, of 64 for Q8_0 and BF16.
bool kquant_mb_supported(int fmt, int k);
int kquant_mb_ksplit(int k);
size_t kquant_mb_part_bytes(int n_total, int k);
hipError_t launch_kquant_gemv_mb(int fmt, const MbMat *mats, int nmat, int m, int k, const void *stage,
                                 const float *x, float *part, hipStream_t s, RowsIn *views = nullptr);

// ---------------------------------------------------------------------------
// Staging of a batched-GEMV input (device).  Each 64-element chunk of each
// row is scaled to integers X = rint(x * s), s = 32639 / 2^e with
// max |x| < 2^e (so |X| <= 32639), and written as two balanced signed bytes
// X = 256*x1 + x0 (x0, x1 in -128..127).  The rounding is one FMA,
// x*s + (1.5*2^23 + 128), whose low 16 mantissa bits are X + 128.  Per
// (chunk, row): {delta = 2^e/32639, sum of x over each 32-element half}.
//   layout: dig[(chunk*8 + row)*2 + digit][64] bytes, stats[chunk*8 + row][4]
// ---------------------------------------------------------------------------
struct MbScale {
  float s, delta;
};
__device__ __forceinline__ MbScale mb_scale(uint32_t max_abs_bits) {
  // max < 2^e, e = biased exponent - 126; s = 32639 * 2^-e stays a normal
  // float for e >= -111 (smaller chunks lose digits instead of overflowing)
  const int e = max((int)(max_abs_bits >> 23) - 126, -111);
  return {__uint_as_float(__float_as_uint(32639.0f) - ((uint32_t)e << 23)),
          __uint_as_float(__float_as_uint(1.0f / 32639.0f) + ((uint32_t)e << 23))};
}
constexpr float kMbMagic = 12583040.0f;  // 1.5*2^23 + 128

// Digits of one float4 (elements 4q..4q+3 of chunk c of `row`); the 16 lanes
// of a chunk (q = 0..15) are consecutive lanes of a wave and all run this
// (the chunk maximum is a DPP reduction); only lanes with `store` write.
__device__ __forceinline__ void mb_stage4(int8_t *dig, float *stats, int row, int c, int q, float4 v, bool store) {
  const uint32_t ax = __float_as_uint(v.x) & 0x7FFFFFFFu, ay = __float_as_uint(v.y) & 0x7FFFFFFFu;
  const uint32_t az = __float_as_uint(v.z) & 0x7FFFFFFFu, aw = __float_as_uint(v.w) & 0x7FFFFFFFu;
  uint32_t mb = max(max(ax, ay), max(az, aw));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0xB1, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x4E, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x141, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x140, 0xF, 0xF, false));
  const MbScale sc = mb_scale(mb);
  const uint32_t b0 = __float_as_uint(fmaf(v.x, sc.s, kMbMagic)), b1 = __float_as_uint(fmaf(v.y, sc.s, kMbMagic));
  const uint32_t b2 = __float_as_uint(fmaf(v.z, sc.s, kMbMagic)), b3 = __float_as_uint(fmaf(v.w, sc.s, kMbMagic));
  const uint32_t p01 = __builtin_amdgcn_perm(b1, b0, 0x05010400u);  // b0.0 b1.0 b0.1 b1.1
  const uint32_t p23 = __builtin_amdgcn_perm(b3, b2, 0x05010400u);
  const uint32_t d0 = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;  // (X+128 mod 256) - 128
  const uint32_t d1 = __builtin_amdgcn_perm(p23, p01, 0x07060302u);                // floor((X+128)/256)
  float sum = (v.x + v.y) + (v.z + v.w);
  sum += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(sum), 0xB1, 0xF, 0xF, false));
  sum += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(sum), 0x4E, 0xF, 0xF, false));
  sum += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(sum), 0x141, 0xF, 0xF, false));
  if (store) {
    int8_t *base = dig + ((size_t)c * 8 + row) * 128;
    *reinterpret_cast<uint32_t *>(base + 4 * q) = d0;
    *reinterpret_cast<uint32_t *>(base + 64 + 4 * q) = d1;
    float *st = stats + ((size_t)c * 8 + row) * 4;
    if (q == 0) {
      st[0] = sc.delta;
      st[1] = sum;
    }
    if (q == 8) st[2] = sum;
  }
}

// The same for one element per lane: element `lane` (0..63) of chunk c, one
// chunk per wave (every lane of the wave runs this).
__device__ __forceinline__ void mb_stage1(int8_t *dig, float *stats, int row, int c, float x) {
  const int lane = (int)(threadIdx.x & 63);
  uint32_t mb = __float_as_uint(x) & 0x7FFFFFFFu;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, o));
  const MbScale sc = mb_scale(mb);
  const uint32_t b = __float_as_uint(fmaf(x, sc.s, kMbMagic));
  int8_t *base = dig + ((size_t)c * 8 + row) * 128;
  base[lane] = (int8_t)((b & 0xFFu) ^ 0x80u);
  base[64 + lane] = (int8_t)((b >> 8) & 0xFFu);
  float sum = x;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) sum += __shfl_xor(sum, o);  // 32 lanes = one sub-block
  float *st = stats + ((size_t)c * 8 + row) * 4;
  if (lane == 0) {
    st[0] = sc.delta;
    st[1] = sum;
  }
  if (lane == 32) st[2] = sum;
}


}  // namespace rt
