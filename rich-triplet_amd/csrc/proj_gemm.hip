// proj_gemm.hip -- the GEMM of a projection that is not Q4_K (Q6_K, Q8_0,
// BF16 kept in their device layouts, or f32), for prefill rows, and the f32
// weight GEMV of a few rows.
//
// The reference runs these weights as BF16 after widening them at load
// (transformer4.rs:1233-1242) and multiplies on the CPU in f32
// (MatBf16::matmul_by_t, autograd2.rs:757-852).  Here each row of W is
// widened to f16 with a power-of-two scale 2^-ew[n] (max |w'| in
// [2^14, 2^15), exact for BF16, Q8_0 and Q6_K codes times their f16 scales up
// to f16 rounding), A gets the same treatment per row (k_gemm_prep), and
// k_gemm_f16_t256 multiplies on v_mfma_f32_32x32x16_f16 with the scales
// restored in the epilogue, as the Q4_K GEMM does.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/rt_hip.h"
#include "kquant_layout.hpp"
#include "mfma_common.hpp"
#include "rt_device.hpp"
#include "rt_kernels.hpp"

namespace rt {
namespace {

// Element e of row n of a projection in format FMT (decode_*_to_f32 values).
template <int FMT>
RT_DEV float proj_value(const uint8_t *__restrict__ W, int N, int K, int n, int e) {
#pragma clang fp contract(off)
  if constexpr (FMT == RT_LINEAR_BF16) {
    return bf16_lo((uint32_t) reinterpret_cast<const uint16_t *>(W)[(size_t)n * K + e]);
  } else if constexpr (FMT == RT_LINEAR_F32) {
    return reinterpret_cast<const float *>(W)[(size_t)n * K + e];
  } else if constexpr (FMT == RT_LINEAR_Q8_0) {
    return q8_0_value(W, (size_t)N * K, (size_t)n * K + e);
  } else {  // RT_LINEAR_Q6K, planar
    return q6k_value(q6k_planes(W, (size_t)N * (K / 256)), (size_t)n * (K / 256) + e / 256, e & 255);
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

// C[M][N] = 2^(ea[m]+ew[n]) * sum_k a16[m][k] w16[n][k] on
// v_mfma_f32_32x32x16_f16.  C tile 256 x 256 per workgroup of four waves
// (2 x 2), each wave 128 x 128 = 4 x 4 MFMA tiles with its 256 accumulator
// registers in AGPRs (one wave per SIMD issues MFMAs back to back).
//   Operands: K moves in stages of 64 through two LDS slots per operand,
//   filled by global_load_lds_dwordx4 (no VGPRs), each copy instruction
//   moving whole 128-B row pieces.  A slot row is 128 B (8 segments of 8
//   halves) and holds logical segment s at physical segment
//   s ^ ((row >> 1) & 7), so the 16 lanes served together by a ds_read_b128
//   (16 consecutive rows) hit 16 distinct bank groups.  Lane l of an MFMA
//   reads row l%32 of its 32-row tile; k-step t of a stage is logical
//   segment 2t + l/32.
//   Schedule per stage: each k-step's MFMAs run while the next k-step's
//   fragments are read; before the last k-step's MFMAs, the barrier that
//   publishes the next stage (and frees this slot), the refill of this slot
//   two stages ahead, and the next stage's first fragment reads.
//   Epilogue: store_c_tile (32-row slices staged in LDS, 16-byte stores).
//   Measured on the config-4 shapes (4608 x 9216 x 3072): loads and LDS reads
//   alone take about 60% of the kernel's time; the two-slot ring keeps one
//   stage in flight, which is what bounds the overlap with the MFMAs.
constexpr int kFTile = 256, kFK = 64;
constexpr int kFSlot = kFTile * kFK * 2;  // 32 KB per operand per stage

__global__ __launch_bounds__(256) void k_gemm_f16_t256(const _Float16 *__restrict__ a16, const int *__restrict__ ea,
                                                       const _Float16 *__restrict__ w16, const int *__restrict__ ew,
                                                       float *__restrict__ c, int M, int N, int K, int tiles_m,
                                                       int tiles_n, int ksplit) {
  // [A slot 0 | A slot 1 | B slot 0 | B slot 1]; the epilogue reuses the start
  __shared__ __attribute__((aligned(1024))) uint8_t lds[4 * kFSlot];
  auto slot_a = [&](int i) __attribute__((always_inline)) { return lds + i * kFSlot; };
  auto slot_b = [&](int i) __attribute__((always_inline)) { return lds + (2 + i) * kFSlot; };
  const int tid = (int)threadIdx.x, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // Workgroup b runs on XCD b % 8: give each XCD a contiguous run of tiles,
  // walked in groups of eight tile rows so neighbours share A and W in L2.
  const int ntiles = tiles_m * tiles_n, per_xcd = (ntiles + 7) / 8;
  const int bid = (int)blockIdx.x;
  const int tile = ntiles % 8 == 0 ? (bid & 7) * per_xcd + (bid >> 3) : bid;
  const int group = tile / (8 * tiles_n), in_group = tile % (8 * tiles_n);
  const int gm = min(8, tiles_m - group * 8);
  const int m0 = (group * 8 + in_group % gm) * kFTile, n0 = (in_group / gm) * kFTile;
  // Split-K: blockIdx.y = s takes stages [s*nk/ksplit, (s+1)*nk/ksplit) and,
  // with ksplit > 1, writes its scaled partial tile to c + s*M*N.
  const int nk_all = K / kFK, split = (int)blockIdx.y;
  const int kb = split * nk_all / ksplit, nk = (split + 1) * nk_all / ksplit - kb;  // nk >= 1 (host)
  if (ksplit > 1) c += (size_t)split * M * N;

  // Copies: wave w moves rows [64w, 64w+64) of both operands, eight 1 KB
  // instructions each; lane -> row 8*(8w+i) + lane/8, physical segment lane%8.
  const _Float16 *a_src[8], *b_src[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 64 * wave + 8 * i + (lane >> 3);
    const int seg = (lane & 7) ^ ((r >> 1) & 7);
    a_src[i] = a16 + (size_t)min(m0 + r, M - 1) * K + 8 * seg;
    b_src[i] = w16 + (size_t)min(n0 + r, N - 1) * K + 8 * seg;
  }
  auto issue = [&](int kt, int slot) __attribute__((always_inline)) {  // kt: stage of this split
    uint8_t *da = slot_a(slot), *db = slot_b(slot);
    kt += kb;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_global_load_lds((gvoid *)(a_src[i] + (size_t)kt * kFK), (lvoid *)(da + (8 * wave + i) * 1024),
                                       16, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_global_load_lds((gvoid *)(b_src[i] + (size_t)kt * kFK), (lvoid *)(db + (8 * wave + i) * 1024),
                                       16, 0, 0);
  };
  int ra[4], rb[4];  // this lane's fragment rows
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ra[i] = 128 * wm + 32 * i + l32;
    rb[i] = 128 * wn + 32 * i + l32;
  }
  auto frag_off = [&](int r, int s) __attribute__((always_inline)) { return r * 128 + 16 * (s ^ ((r >> 1) & 7)); };
  auto read = [&](int slot, int s, u32x4 (&af)[4], u32x4 (&bf)[4]) __attribute__((always_inline)) {
    const uint8_t *pa = slot_a(slot), *pb = slot_b(slot);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      af[i] = lds_read16(pa + frag_off(ra[i], s));
      bf[i] = lds_read16(pb + frag_off(rb[i], s));
    }
  };
  auto await = [&](u32x4 (&af)[4], u32x4 (&bf)[4]) __attribute__((always_inline)) {
    lds_wait(af[0], af[1], af[2], af[3]);
    lds_wait(bf[0], bf[1], bf[2], bf[3]);
  };
  floatx16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx16{};
  auto mfma16 = [&](const u32x4 (&af)[4], const u32x4 (&bf)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, af[i]),
                                                            __builtin_bit_cast(half8, bf[j]), acc[i][j], 0, 0, 0);
  };

  issue(0, 0);
  if (nk > 1) issue(1, 1);
  u32x4 a0[4], b0[4], a1[4], b1[4];
  if (nk > 1) wait_vmcnt<16>();  // stage 0 landed, stage 1 may be in flight
  else wait_vmcnt<0>();
  wg_barrier();
  read(0, g, a0, b0);
  await(a0, b0);
  auto step = [&](int kt, int slot) __attribute__((always_inline)) {
    read(slot, 2 + g, a1, b1);
    mfma16(a0, b0);
    await(a1, b1);
    read(slot, 4 + g, a0, b0);
    mfma16(a1, b1);
    await(a0, b0);
    read(slot, 6 + g, a1, b1);
    mfma16(a0, b0);
    await(a1, b1);
    if (kt + 1 < nk) {
      wait_vmcnt<0>();  // stage kt+1, the only one in flight, has landed
      wg_barrier();     // everywhere, and this slot is read out everywhere
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 2 < nk) issue(kt + 2, slot);
      __builtin_amdgcn_sched_barrier(0);
      read(slot ^ 1, g, a0, b0);
    }
    mfma16(a1, b1);
    if (kt + 1 < nk) await(a0, b0);
  };
  int kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    step(kt, 0);
    step(kt + 1, 1);
  }
  if (kt < nk) step(kt, 0);

  // Epilogue: the wave's 128 x 128 tile through LDS in 32-row slices (17 KB
  // per wave at the start of the free slots), 16-byte stores.
  int ec[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) ec[j] = ew[min(n0 + rb[j], N - 1)];
  wg_barrier();  // the slots are free: every wave's last fragments are read
  store_c_tile<4>(acc, reinterpret_cast<float *>(lds) + wave * 32 * (32 * 4 + 8), c, M, N, m0 + 128 * wm,
                  n0 + 128 * wn, ea, ec);
}

// ---------------------------------------------------------------------------
// f32 weights with a few activation rows (QLinear's f32 branch, x.matmul_bt(W),
// qlinear.rs:102-106, for M <= 8 per launch row group): each wave owns four
// weight rows and streams them once for the MR activation rows of its group
// (blockIdx.y), 16-byte loads along K; per output a lane-strided f32 sum, then
// the wave's DPP sum.  With a bias, out = sum + bias[n], the one f32 add of
// add_bias_rows (qlinear.rs:49-60).
// ---------------------------------------------------------------------------
template <int MR>
__global__ __launch_bounds__(256) void k_f32_gemv_rows(const float *__restrict__ W, const float *__restrict__ a,
                                                       const float *__restrict__ bias, float *__restrict__ c, int M,
                                                       int N, int K) {
  constexpr int RW = 4;
  const int lane = (int)threadIdx.x & 63;
  const int n0 = (int)((blockIdx.x * 256u + threadIdx.x) >> 6) * RW;
  const int m0 = (int)blockIdx.y * 8;
  if (n0 >= N) return;  // whole waves
  const int K4 = K / 4;
  const float4 *w4 = reinterpret_cast<const float4 *>(W);
  const float4 *a4 = reinterpret_cast<const float4 *>(a) + (size_t)m0 * K4;
  float acc[RW][MR];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int i = 0; i < MR; ++i) acc[r][i] = 0.f;
#pragma unroll 2
  for (int k4 = lane; k4 < K4; k4 += 64) {
    float4 w[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) w[r] = w4[(size_t)min(n0 + r, N - 1) * K4 + k4];
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      const float4 x = a4[(size_t)min(i, M - 1 - m0) * K4 + k4];  // rows past M re-read row M-1, unstored
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        acc[r][i] = fmaf(w[r].x, x.x, acc[r][i]);
        acc[r][i] = fmaf(w[r].y, x.y, acc[r][i]);
        acc[r][i] = fmaf(w[r].z, x.z, acc[r][i]);
        acc[r][i] = fmaf(w[r].w, x.w, acc[r][i]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      const float v = wave_sum(acc[r][i]);
      if (lane == 0 && n0 + r < N && m0 + i < M) c[(size_t)(m0 + i) * N + n0 + r] = bias ? v + bias[n0 + r] : v;
    }
}

// The same for BF16 weights (MatBf16::matmul_by_t, autograd2.rs:757-852, of a
// few rows): 16-byte loads of eight weights, each widened exactly.
template <int MR>
__global__ __launch_bounds__(256) void k_bf16_gemv_rows(const uint16_t *__restrict__ W, const float *__restrict__ a,
                                                        const float *__restrict__ bias, float *__restrict__ c, int M,
                                                        int N, int K) {
  constexpr int RW = 4;
  const int lane = (int)threadIdx.x & 63;
  const int n0 = (int)((blockIdx.x * 256u + threadIdx.x) >> 6) * RW;
  const int m0 = (int)blockIdx.y * 8;
  if (n0 >= N) return;
  const int K8 = K / 8;
  const uint4 *w8 = reinterpret_cast<const uint4 *>(W);
  const float4 *a4 = reinterpret_cast<const float4 *>(a) + (size_t)m0 * (K / 4);
  float acc[RW][MR];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int i = 0; i < MR; ++i) acc[r][i] = 0.f;
#pragma unroll 2
  for (int k8 = lane; k8 < K8; k8 += 64) {
    float wf[RW][8];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const uint4 q = w8[(size_t)min(n0 + r, N - 1) * K8 + k8];
      const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) wf[r][2 * j] = bf16_lo(u[j]), wf[r][2 * j + 1] = bf16_hi(u[j]);
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      const float4 *xr = a4 + (size_t)min(i, M - 1 - m0) * (K / 4) + 2 * k8;
      const float4 x0 = xr[0], x1 = xr[1];
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[r][i] = fmaf(wf[r][j], xv[j], acc[r][i]);
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      const float v = wave_sum(acc[r][i]);
      if (lane == 0 && n0 + r < N && m0 + i < M) c[(size_t)(m0 + i) * N + n0 + r] = bias ? v + bias[n0 + r] : v;
    }
}

// add_bias_rows (qlinear.rs:49-60): c[r][j] += bias[j].
__global__ __launch_bounds__(256) void k_add_bias_rows(float *__restrict__ c, const float *__restrict__ bias,
                                                       size_t total, int N) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256)
    c[i] += bias[i % (size_t)N];
}

}  // namespace

hipError_t launch_f32_gemv_rows(const float *w, const float *a, const float *bias, float *c, int M, int N, int K,
                                hipStream_t s) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 4 != 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 7) / 8));
  const int mr = std::min(M, 8);  // rows of the last group are bounded by M inside
  switch (mr) {
    case 1: hipLaunchKernelGGL(k_f32_gemv_rows<1>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
    case 2: hipLaunchKernelGGL(k_f32_gemv_rows<2>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
    case 3: hipLaunchKernelGGL(k_f32_gemv_rows<3>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
    case 4: hipLaunchKernelGGL(k_f32_gemv_rows<4>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
    default: hipLaunchKernelGGL(k_f32_gemv_rows<8>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
  }
  return hipGetLastError();
}

hipError_t launch_bf16_gemv_rows(const uint16_t *w, const float *a, const float *bias, float *c, int M, int N, int K,
                                 hipStream_t s) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 8 != 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 7) / 8));
  switch (std::min(M, 8)) {
    case 1: hipLaunchKernelGGL(k_bf16_gemv_rows<1>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
    case 2: hipLaunchKernelGGL(k_bf16_gemv_rows<2>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
    case 3: hipLaunchKernelGGL(k_bf16_gemv_rows<3>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
    case 4: hipLaunchKernelGGL(k_bf16_gemv_rows<4>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
    default: hipLaunchKernelGGL(k_bf16_gemv_rows<8>, grid, dim3(256), 0, s, w, a, bias, c, M, N, K); break;
  }
  return hipGetLastError();
}

hipError_t launch_add_bias_rows(float *c, const float *bias, int M, int N, hipStream_t s) {
  const size_t total = (size_t)M * N;
  const unsigned grid = (unsigned)std::min<size_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(k_add_bias_rows, dim3(grid), dim3(256), 0, s, c, bias, total, N);
  return hipGetLastError();
}

// Split-K count: enough workgroups to cover the 256 CUs when the output has
// few 256 x 256 tiles (M = 512, N = 2560: 20 tiles), at least 8 stages
// (K = 512) per split.
static int proj_ksplit(int M, int N, int K) {
  const int ntiles = ((M + kFTile - 1) / kFTile) * ((N + kFTile - 1) / kFTile);
  return std::max(1, std::min(256 / ntiles, (K / kFK) / 8));
}

size_t proj_gemm_workspace_bytes(int M, int N, int K) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  const int ks = proj_ksplit(M, N, K);
  return r256((size_t)M * K * 2) + r256((size_t)M * 4) + r256((size_t)N * K * 2) + r256((size_t)N * 4) +
         (ks > 1 ? (size_t)ks * M * N * 4 : 0);
}

size_t proj_gemm_prepped_ws_bytes(int M, int N, int K) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  return proj_gemm_workspace_bytes(M, N, K) - r256((size_t)M * K * 2) - r256((size_t)M * 4);
}

hipError_t launch_proj_gemm_prepped(const _Float16 *a16, const int *ea, int fmt, const void *w, float *c, int M,
                                    int N, int K, void *ws, hipStream_t s) {
  if (M <= 0 || N <= 0 || K <= 0 || K % kFK != 0) return hipErrorInvalidValue;  // K moves in stages of 64
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  char *p = static_cast<char *>(ws);
  _Float16 *w16 = reinterpret_cast<_Float16 *>(p);
  p += r256((size_t)N * K * 2);
  int *ew = reinterpret_cast<int *>(p);
  p += r256((size_t)N * 4);
  const uint8_t *wb = static_cast<const uint8_t *>(w);
  switch (fmt) {
    case RT_LINEAR_Q6K:
      hipLaunchKernelGGL(k_rows_to_f16<RT_LINEAR_Q6K>, dim3(N), dim3(256), 0, s, wb, N, K, w16, ew);
      break;
    case RT_LINEAR_Q8_0:
      hipLaunchKernelGGL(k_rows_to_f16<RT_LINEAR_Q8_0>, dim3(N), dim3(256), 0, s, wb, N, K, w16, ew);
      break;
    case RT_LINEAR_BF16:
      hipLaunchKernelGGL(k_rows_to_f16<RT_LINEAR_BF16>, dim3(N), dim3(256), 0, s, wb, N, K, w16, ew);
      break;
    case RT_LINEAR_F32:
      hipLaunchKernelGGL(k_rows_to_f16<RT_LINEAR_F32>, dim3(N), dim3(256), 0, s, wb, N, K, w16, ew);
      break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int tiles_m = (M + kFTile - 1) / kFTile, tiles_n = (N + kFTile - 1) / kFTile;
  const int ks = proj_ksplit(M, N, K);
  float *out = ks > 1 ? reinterpret_cast<float *>(p) : c;
  hipLaunchKernelGGL(k_gemm_f16_t256, dim3(tiles_m * tiles_n, ks), dim3(256), 0, s, a16, ea, w16, ew, out, M, N, K,
                     tiles_m, tiles_n, ks);
  e = hipGetLastError();
  if (e == hipSuccess && ks > 1) e = launch_gemm_splitk_sum(out, c, (size_t)M * N, ks, s);
  return e;
}

hipError_t launch_proj_gemm(const float *a, int fmt, const void *w, float *c, int M, int N, int K, void *ws,
                            hipStream_t s) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  char *p = static_cast<char *>(ws);
  _Float16 *a16 = reinterpret_cast<_Float16 *>(p);
  int *ea = reinterpret_cast<int *>(p + r256((size_t)M * K * 2));
  hipError_t e = launch_gemm_prep_a(a, M, K, a16, ea, s);
  if (e != hipSuccess) return e;
  return launch_proj_gemm_prepped(a16, ea, fmt, w, c, M, N, K, p + r256((size_t)M * K * 2) + r256((size_t)M * 4), s);
}

}  // namespace rt
