// bf16_kernels.hip -- BF16 GEMV (the lm_head shape K=2560, N=262144, and any
// K up to 16384 for BF16 projections).
//
// y[N] = W[N,K] (bf16, row-major) . x[K] (f32), f32 accumulation.
// One wave per row: lane l reads 16-byte pieces l, l+64, ... of the row, so
// every load instruction moves 1 KB of contiguous weights; the lane's 8*CPL
// activations stay in registers for all rows the wave visits.
#include <algorithm>

#include "rt_device.hpp"
#include "rt_kernels.hpp"

namespace rt {

template <int CPL>
struct Bf16X {
  float v[CPL][8];
};

template <int CPL>
RT_DEV void load_bf16_x(const float *__restrict__ x, int lane, Bf16X<CPL> &xr) {
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const float4 *p = reinterpret_cast<const float4 *>(x + (size_t)(i * 64 + lane) * 8);
    const float4 a = p[0], b = p[1];
    xr.v[i][0] = a.x; xr.v[i][1] = a.y; xr.v[i][2] = a.z; xr.v[i][3] = a.w;
    xr.v[i][4] = b.x; xr.v[i][5] = b.y; xr.v[i][6] = b.z; xr.v[i][7] = b.w;
  }
}

template <int CPL>
RT_DEV float bf16_piece_dot(const uint4 w, const float *xv) {
  float a = bf16_lo(w.x) * xv[0];
  float b = bf16_hi(w.x) * xv[1];
  a += bf16_lo(w.y) * xv[2];
  b += bf16_hi(w.y) * xv[3];
  a += bf16_lo(w.z) * xv[4];
  b += bf16_hi(w.z) * xv[5];
  a += bf16_lo(w.w) * xv[6];
  b += bf16_hi(w.w) * xv[7];
  return a + b;
}

// Rows [r0, r0+U) of W against resident x; returns nothing, lane 0 stores.
template <int CPL, int U>
RT_DEV void bf16_rows(const uint16_t *__restrict__ W, const Bf16X<CPL> &xr, int r0, int N, int lane,
                      float *__restrict__ y) {
  constexpr int K = CPL * 512;
  uint4 wv[U][CPL];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int r = r0 + u;
    const uint4 *rp = reinterpret_cast<const uint4 *>(W + (size_t)(r < N ? r : 0) * K);
#pragma unroll
    for (int i = 0; i < CPL; ++i) wv[u][i] = ld_nt16(rp + i * 64 + lane);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) acc += bf16_piece_dot<CPL>(wv[u][i], xr.v[i]);
    acc = wave_sum(acc);
    if (lane == 0 && r0 + u < N) y[r0 + u] = acc;
  }
}

template <int CPL, int U>
__global__ __launch_bounds__(256) void k_bf16_gemv(const uint16_t *__restrict__ W, const float *__restrict__ x,
                                                   float *__restrict__ y, int N) {
  const int lane = threadIdx.x & 63;
  const int wave = (int)((blockIdx.x * 256u + threadIdx.x) >> 6);
  const int nwaves = (int)(gridDim.x * 4u);
  Bf16X<CPL> xr;
  load_bf16_x<CPL>(x, lane, xr);
  for (int r0 = wave * U; r0 < N; r0 += nwaves * U) bf16_rows<CPL, U>(W, xr, r0, N, lane, y);
}

// Any K (multiple of 8): one wave per row, activations read through the cache.
__global__ __launch_bounds__(256) void k_bf16_gemv_generic(const uint16_t *__restrict__ W, const float *__restrict__ x,
                                                           float *__restrict__ y, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
  if (row >= N) return;
  const int pieces = K / 8;
  const uint4 *rp = reinterpret_cast<const uint4 *>(W + (size_t)row * K);
  float acc = 0.f;
  for (int p = lane; p < pieces; p += 64) {
    const float4 *xp = reinterpret_cast<const float4 *>(x + (size_t)p * 8);
    const float4 a = xp[0], b = xp[1];
    const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    acc += bf16_piece_dot<1>(rp[p], xv);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

// K up to 16384 (multiple of 8), x staged in LDS once per workgroup: each
// wave takes U rows at a time and keeps 4 pieces of each in flight.
template <int U>
__global__ __launch_bounds__(256) void k_bf16_gemv_lds(const uint16_t *__restrict__ W, const float *__restrict__ x,
                                                       float *__restrict__ y, int N, int K) {
  __shared__ __attribute__((aligned(16))) float xs[16384];
  for (int i = threadIdx.x; i < K / 4; i += 256)
    reinterpret_cast<float4 *>(xs)[i] = reinterpret_cast<const float4 *>(x)[i];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = (int)((blockIdx.x * 256u + threadIdx.x) >> 6), nwaves = (int)(gridDim.x * 4u);
  const int pieces = K / 8;
  for (int r0 = wave * U; r0 < N; r0 += nwaves * U) {
    const uint4 *rp[U];
#pragma unroll
    for (int u = 0; u < U; ++u) rp[u] = reinterpret_cast<const uint4 *>(W + (size_t)min(r0 + u, N - 1) * K);
    float acc[U] = {};
    for (int p0 = lane; p0 < pieces; p0 += 256) {
      uint4 wv[U][4];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[u][j] = p0 + 64 * j < pieces ? rp[u][p0 + 64 * j] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int p = min(p0 + 64 * j, pieces - 1);
        const float4 a = reinterpret_cast<const float4 *>(xs)[2 * p], b = reinterpret_cast<const float4 *>(xs)[2 * p + 1];
        const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] += bf16_piece_dot<1>(wv[u][j], xv);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float v = wave_sum(acc[u]);
      if (lane == 0 && r0 + u < N) y[r0 + u] = v;
    }
  }
}

hipError_t launch_bf16_gemv(const uint16_t *W, const float *x, float *y, int N, int K, hipStream_t s) {
  if (K == 2560) {
    constexpr int U = 2;
    const int waves_needed = (N + U - 1) / U;
    int grid = (waves_needed + 3) / 4;
    if (grid > 256 * 32) grid = 256 * 32;  // 262144 rows: 8192 workgroups (measured 4% over 2048)
    hipLaunchKernelGGL((k_bf16_gemv<5, U>), dim3(grid), dim3(256), 0, s, W, x, y, N);
    return hipGetLastError();
  }
  if (K <= 16384) {
    constexpr int U = 2;
    const unsigned grid = (unsigned)std::min((N + 4 * U - 1) / (4 * U), 256 * 4);
    hipLaunchKernelGGL(k_bf16_gemv_lds<U>, dim3(grid), dim3(256), 0, s, W, x, y, N, K);
    return hipGetLastError();
  }
  const unsigned grid = (unsigned)((N + 3) / 4);
  hipLaunchKernelGGL(k_bf16_gemv_generic, dim3(grid), dim3(256), 0, s, W, x, y, N, K);
  return hipGetLastError();
}

}  // namespace rt
