// proj_gemm.hip -- the GEMM of a projection that is not Q4_K (Q6_K, Q8_0 or
// BF16 kept in their device layouts), for prefill rows.
//
// The reference runs these weights as BF16 after widening them at load
// (transformer4.rs:1233-1242) and multiplies on the CPU in f32
// (MatBf16::matmul_by_t, autograd2.rs:757-852).  Here each row of W is
// widened to f16 with a power-of-two scale 2^-ew[n] (max |w'| in
// [2^14, 2^15), exact for BF16, Q8_0 and Q6_K codes times their f16 scales up
// to f16 rounding), A gets the same treatment per row (k_gemm_prep), and
// k_gemm_f16w multiplies on v_mfma_f32_32x32x16_f16 with the scales
// restored in the epilogue, as the Q4_K GEMM does.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/rt_hip.h"
#include "rt_device.hpp"
#include "rt_kernels.hpp"

namespace rt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Element e of row n of a projection in format FMT (decode_*_to_f32 values).
template <int FMT>
RT_DEV float proj_value(const uint8_t *__restrict__ W, int N, int K, int n, int e) {
#pragma clang fp contract(off)
  if constexpr (FMT == RT_LINEAR_BF16) {
    return bf16_lo((uint32_t) reinterpret_cast<const uint16_t *>(W)[(size_t)n * K + e]);
  } else if constexpr (FMT == RT_LINEAR_Q8_0) {
    const size_t i = (size_t)n * K + e;
    const uint16_t *D = reinterpret_cast<const uint16_t *>(W + (size_t)N * K);
    return half_bits_to_f32(D[i / 32]) * (float)(int8_t)W[i];
  } else {  // RT_LINEAR_Q6K, planar
    const size_t nbt = (size_t)N * (K / 256), blk = (size_t)n * (K / 256) + e / 256;
    const int i = e & 255, j = i >> 7, h = i & 127, m = h >> 5, l = h & 31;
    const uint8_t ql = W[blk * 128 + 64 * j + 32 * (m & 1) + l];
    const uint8_t qh = W[nbt * 128 + blk * 64 + 32 * j + l];
    const int q = (int)(((m < 2 ? ql & 15 : ql >> 4)) | (((qh >> (2 * m)) & 3) << 4)) - 32;
    const float d = half_bits_to_f32(reinterpret_cast<const uint16_t *>(W + nbt * 208)[blk]);
    const float s = d * (float)(int8_t)W[nbt * 192 + blk * 16 + 8 * j + (l >> 4) + 2 * m];
    return s * (float)q;
  }
}

// One row per workgroup: bound, exponent, then the scaled f16 row.
template <int FMT>
__global__ __launch_bounds__(256) void k_rows_to_f16(const uint8_t *__restrict__ W, int N, int K,
                                                     _Float16 *__restrict__ w16, int *__restrict__ ew) {
  __shared__ float red[4];
  const int n = (int)blockIdx.x;
  float amax = 0.f;
  for (int e = threadIdx.x; e < K; e += 256) amax = fmaxf(amax, fabsf(proj_value<FMT>(W, N, K, n, e)));
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const int ex = f16_exponent_for(amax);
  if (threadIdx.x == 0) ew[n] = ex;
  for (int e = threadIdx.x; e < K; e += 256)
    w16[(size_t)n * K + e] = (_Float16)__builtin_amdgcn_ldexpf(proj_value<FMT>(W, N, K, n, e), -ex);
}

// C[M][N] = 2^(ea[m]+ew[n]) * sum_k a16[m][k] w16[n][k].  128 x 128 tile per
// workgroup, four waves of 64 x 64 (2 x 2 v_mfma_f32_32x32x16_f16 tiles),
// K in steps of 32 through double-buffered LDS with the next step's global
// loads in registers during the MFMAs.  Lane l: A row / B column l%32,
// halves 8*(l/32) + [0, 8) of a 16-wide k step.
constexpr int kFP = 40;  // LDS row pitch in halves (32 + 8): rows 80 B apart
__global__ __launch_bounds__(256) void k_gemm_f16w(const _Float16 *__restrict__ a16, const int *__restrict__ ea,
                                                   const _Float16 *__restrict__ w16, const int *__restrict__ ew,
                                                   float *__restrict__ c, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) _Float16 as[2][128 * kFP], bs[2][128 * kFP];
  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, g = lane >> 5;
  const int m0 = (int)blockIdx.y * 128, n0 = (int)blockIdx.x * 128;
  // global -> LDS copy: thread t moves 32 B of row t/2 (halves 16*(t%2) .. +16)
  const int cr = tid >> 1, ch = 16 * (tid & 1);
  const _Float16 *ga = a16 + (size_t)min(m0 + cr, M - 1) * K + ch;
  const _Float16 *gb = w16 + (size_t)min(n0 + cr, N - 1) * K + ch;
  uint4 ra[2], rb[2];
  auto gload = [&](int k0) __attribute__((always_inline)) {
    ra[0] = *reinterpret_cast<const uint4 *>(ga + k0);
    ra[1] = *reinterpret_cast<const uint4 *>(ga + k0 + 8);
    rb[0] = *reinterpret_cast<const uint4 *>(gb + k0);
    rb[1] = *reinterpret_cast<const uint4 *>(gb + k0 + 8);
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
    *reinterpret_cast<uint4 *>(&as[buf][cr * kFP + ch]) = ra[0];
    *reinterpret_cast<uint4 *>(&as[buf][cr * kFP + ch + 8]) = ra[1];
    *reinterpret_cast<uint4 *>(&bs[buf][cr * kFP + ch]) = rb[0];
    *reinterpret_cast<uint4 *>(&bs[buf][cr * kFP + ch + 8]) = rb[1];
  };
  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{};
  const int nk = K / 32;
  gload(0);
  sstore(0);
  __syncthreads();
#pragma unroll 1
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(32 * (kt + 1));
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      half8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        af[i] = *reinterpret_cast<const half8 *>(&as[buf][(64 * wm + 32 * i + l32) * kFP + 16 * ks + 8 * g]);
        bf[i] = *reinterpret_cast<const half8 *>(&bs[buf][(64 * wn + 32 * i + l32) * kFP + 16 * ks + 8 * g]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }
  // register r of tile (i, j): C[64wm + 32i + 8(r/4) + 4g + r%4][64wn + 32j + l32]
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + 64 * wn + 32 * j + l32;
    if (col >= N) continue;
    const int ec = ew[col];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
        if (row < M) c[(size_t)row * N + col] = __builtin_amdgcn_ldexpf(acc[i][j][r], ea[row] + ec);
      }
  }
}

}  // namespace

size_t proj_gemm_workspace_bytes(int M, int N, int K) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  return r256((size_t)M * K * 2) + r256((size_t)M * 4) + r256((size_t)N * K * 2) + r256((size_t)N * 4);
}

hipError_t launch_proj_gemm(const float *a, int fmt, const void *w, float *c, int M, int N, int K, void *ws,
                            hipStream_t s) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  char *p = static_cast<char *>(ws);
  _Float16 *a16 = reinterpret_cast<_Float16 *>(p);
  p += r256((size_t)M * K * 2);
  int *ea = reinterpret_cast<int *>(p);
  p += r256((size_t)M * 4);
  _Float16 *w16 = reinterpret_cast<_Float16 *>(p);
  p += r256((size_t)N * K * 2);
  int *ew = reinterpret_cast<int *>(p);
  const uint8_t *wb = static_cast<const uint8_t *>(w);
  switch (fmt) {
    case RT_LINEAR_Q6K: hipLaunchKernelGGL(k_rows_to_f16<RT_LINEAR_Q6K>, dim3(N), dim3(256), 0, s, wb, N, K, w16, ew); break;
    case RT_LINEAR_Q8_0: hipLaunchKernelGGL(k_rows_to_f16<RT_LINEAR_Q8_0>, dim3(N), dim3(256), 0, s, wb, N, K, w16, ew); break;
    case RT_LINEAR_BF16: hipLaunchKernelGGL(k_rows_to_f16<RT_LINEAR_BF16>, dim3(N), dim3(256), 0, s, wb, N, K, w16, ew); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = launch_gemm_prep_a(a, M, K, a16, ea, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_gemm_f16w, dim3((N + 127) / 128, (M + 127) / 128), dim3(256), 0, s, a16, ea, w16, ew, c, M, N,
                     K);
  return hipGetLastError();
}

}  // namespace rt
