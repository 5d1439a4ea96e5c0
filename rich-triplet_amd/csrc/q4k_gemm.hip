// q4k_gemm.hip -- Q4_K GEMM on gfx950 matrix cores:  C[m][n] = sum_k A[m][k] * W[n][k].
//
// Replaces Q4KMat::matmul_q4k_t / matmul_q4k_t_exact (autograd2.rs:1437-1625,
// dequantise a band of rows to f32 and sgemm it) and the FLUX GPU path
// flux_dequant_q4k + flux_gemm_bt (metal_flux.rs:108-190, dequantise the whole
// weight to bfloat scratch, then a 64x64 simdgroup GEMM).  Here the weight
// stays packed in HBM (144-byte super-blocks) and each workgroup dequantises
// only the 64-column chunk it is about to multiply, into LDS.
//
// Arithmetic: v_mfma_f32_16x16x32_f16, f32 accumulation.
//   Weights rounded to bf16 (8-bit significand, what the reference's GPU path
//   does) land ~1.6e-3 rel-L2 away from the f32 CPU result at K=2560; rounded
//   to f16 (11-bit significand) they land ~2e-4 away.  bf16 activations are
//   exact in f16.  f16 has a narrow exponent range, so k_gemm_prep gives every
//   A row and every W row a power-of-two scale:
//       a'[m][k] = a[m][k] * 2^-ea[m],   max|a'| in [2^14, 2^15)
//       w'[n][k] = w[n][k] * 2^-ew[n],   bound|w'| in [2^14, 2^15)
//   and the epilogue multiplies by 2^(ea[m]+ew[n]), which is exact.
//
// Dequantisation of one weight: w = (d*sv)*q - (dmin*mv) (autograd2.rs:1359-1363).
// v_perm builds the f16 bit pattern 0x64qq = 1024 + q from a nibble, and one
// v_fma_mix computes s*(1024+q) - (m + 1024*s) in f32 with a single rounding
// to f16: two VALU operations per weight.
#include <hip/hip_runtime.h>

#include "rt_device.hpp"
#include "rt_kernels.hpp"

namespace rt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
// Native vectors for staging registers: HIP's uint4 is a union-wrapped struct
// whose copies become memcpys, which LLVM turns back into global reloads.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;          // K per pipeline stage = one Q4_K chunk (32 qs bytes, 2 sub-blocks)
constexpr int kPitch = kBK + 8;  // halves per LDS row: 144 bytes keeps 8 consecutive rows on distinct banks

// ---------------------------------------------------------------------------
// Prep: A -> f16 with a per-row exponent; W row exponents from block headers.
// Workgroups [0, M) take one A row each, the rest 256 W rows each.
// ---------------------------------------------------------------------------
RT_DEV int f16_exponent_for(float bound) {
  // 2^-e * bound in [2^14, 2^15); 0 for zero / non-finite bounds (those propagate).
  if (!(bound > 0.f) || !__builtin_isfinite(bound)) return 0;
  int E;
  (void)frexpf(bound, &E);  // bound = f * 2^E, f in [0.5, 1)
  return E - 15;
}

template <typename TA>
RT_DEV void load8(const TA *p, float v[8]);
template <>
RT_DEV void load8<uint16_t>(const uint16_t *p, float v[8]) {
  const uint4 u = *reinterpret_cast<const uint4 *>(p);
  v[0] = bf16_lo(u.x), v[1] = bf16_hi(u.x), v[2] = bf16_lo(u.y), v[3] = bf16_hi(u.y);
  v[4] = bf16_lo(u.z), v[5] = bf16_hi(u.z), v[6] = bf16_lo(u.w), v[7] = bf16_hi(u.w);
}
template <>
RT_DEV void load8<float>(const float *p, float v[8]) {
  const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
  v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

RT_DEV uint32_t half_bits(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }


template <typename TA>
__global__ __launch_bounds__(256) void k_gemm_prep(const TA *__restrict__ a, _Float16 *__restrict__ a16,
                                                   int *__restrict__ ea, const uint8_t *__restrict__ w,
                                                   int *__restrict__ ew, int M, int N, int K) {
  __shared__ float red[4];
  const int b = (int)blockIdx.x;
  if (b < M) {
    const TA *row = a + (size_t)b * K;
    float amax = 0.f;
    for (int g = threadIdx.x; g < K / 8; g += 256) {
      float v[8];
      load8<TA>(row + g * 8, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // A NaN anywhere makes the row NaN in the product too; keep it visible.
    const int e = f16_exponent_for(amax);
    if (threadIdx.x == 0) ea[b] = e;
    _Float16 *out = a16 + (size_t)b * K;
    for (int g = threadIdx.x; g < K / 8; g += 256) {
      float v[8];
      load8<TA>(row + g * 8, v);
      uint32_t ow[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ow[i] = half_bits((_Float16)__builtin_amdgcn_ldexpf(v[2 * i], -e)) |
                (half_bits((_Float16)__builtin_amdgcn_ldexpf(v[2 * i + 1], -e)) << 16);
      *reinterpret_cast<uint4 *>(out + g * 8) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
  } else {
    const int n = (b - M) * 256 + (int)threadIdx.x;
    if (n >= N) return;
    const int kb = K / 256;
    const uint8_t *blk = w + (size_t)n * kb * kQ4KBlockBytes;
    float bound = 0.f;  // |w| <= max(15*63*|d|, 63*|dmin|)
    for (int i = 0; i < kb; ++i) {
      const uint32_t h = *reinterpret_cast<const uint32_t *>(blk + (size_t)i * kQ4KBlockBytes);
      bound = fmaxf(bound, fmaxf(945.f * fabsf(half_bits_to_f32(h & 0xFFFFu)), 63.f * fabsf(half_bits_to_f32(h >> 16))));
    }
    ew[n] = f16_exponent_for(bound);
  }
}

// ---------------------------------------------------------------------------
// Main kernel.  256 threads = WGM x WGN waves; the workgroup owns a BM x BN
// tile of C and walks K in 64-wide stages, double-buffered in LDS:
//   registers <- global (stage s+1)  |  MFMA on LDS buffer s%2
//   dequantise registers -> LDS buffer (s+1)%2;  one barrier per stage.
// Loads are unconditional at clamped indices (rows past M / N repeat the last
// row; their results are never stored) so the loop has no branches.
// ---------------------------------------------------------------------------
template <int BM, int BN, int WGM, int WGN>
struct GemmTile {
  static_assert(WGM * WGN == 4, "four waves");
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int TI = WM / 16, TJ = WN / 16;
  static_assert(TI * 16 == WM && TJ * 16 == WN, "wave tile must be a multiple of 16");
  static constexpr int A_LOADS = BM * (kBK / 8) / 256;  // 16-byte A loads per thread per stage
  static constexpr int B_ITEMS = BN * 2 / 256;          // (row, 16-byte half of the chunk) items per thread
  static_assert(A_LOADS * 256 == BM * (kBK / 8) && B_ITEMS * 256 == BN * 2, "tile / thread mismatch");
};

// Two weights from one v_perm result: halves hold 1024+q (or 1024+16q).
RT_DEV uint32_t dq_pair(uint32_t p, float s, float negc) {
  const _Float16 h0 = __builtin_bit_cast(_Float16, (uint16_t)(p & 0xFFFFu));
  const _Float16 h1 = __builtin_bit_cast(_Float16, (uint16_t)(p >> 16));
  const _Float16 r0 = (_Float16)__builtin_fmaf(s, (float)h0, negc);
  const _Float16 r1 = (_Float16)__builtin_fmaf(s, (float)h1, negc);
  return half_bits(r0) | (half_bits(r1) << 16);
}

template <int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(256) void k_q4k_gemm(const _Float16 *__restrict__ a16, const int *__restrict__ ea,
                                                  const uint8_t *__restrict__ w, const int *__restrict__ ew,
                                                  float *__restrict__ c, int M, int N, int K, int tiles_n) {
  using T = GemmTile<BM, BN, WGM, WGN>;
  __shared__ __attribute__((aligned(16))) _Float16 lds_a[2][BM * kPitch];
  __shared__ __attribute__((aligned(16))) _Float16 lds_b[2][BN * kPitch];

  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int m0 = ((int)blockIdx.x / tiles_n) * BM, n0 = ((int)blockIdx.x % tiles_n) * BN;
  const int kb = K / 256, nstages = K / kBK;

  // Per-thread load slots (fixed for the whole K loop).
  const _Float16 *a_src[T::A_LOADS];
  int a_dst[T::A_LOADS];
#pragma unroll
  for (int i = 0; i < T::A_LOADS; ++i) {
    const int idx = tid + 256 * i, r = idx >> 3, c8 = idx & 7;
    a_src[i] = a16 + (size_t)min(m0 + r, M - 1) * K + c8 * 8;
    a_dst[i] = r * kPitch + c8 * 8;
  }
  const uint8_t *b_row[T::B_ITEMS];
  int b_half[T::B_ITEMS], b_dst[T::B_ITEMS];
  float b_pow[T::B_ITEMS];
#pragma unroll
  for (int j = 0; j < T::B_ITEMS; ++j) {
    const int item = tid + 256 * j, r = item >> 1, h = item & 1, n = min(n0 + r, N - 1);
    b_row[j] = w + (size_t)n * kb * kQ4KBlockBytes;
    b_half[j] = h;
    b_dst[j] = r * kPitch + h * 16;
    b_pow[j] = __builtin_amdgcn_ldexpf(1.0f, -ew[n]);
  }

  u32x4 ra[T::A_LOADS], rh[T::B_ITEMS], rq[T::B_ITEMS];
  auto load_stage = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < T::A_LOADS; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(a_src[i] + s * kBK);
#pragma unroll
    for (int j = 0; j < T::B_ITEMS; ++j) {
      const uint8_t *blk = b_row[j] + (size_t)(s >> 2) * kQ4KBlockBytes;
      rh[j] = *reinterpret_cast<const u32x4 *>(blk);
      rq[j] = *reinterpret_cast<const u32x4 *>(blk + 16 + (s & 3) * 32 + b_half[j] * 16);
    }
  };
  auto store_stage = [&](int s, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < T::A_LOADS; ++i) *reinterpret_cast<u32x4 *>(&lds_a[buf][a_dst[i]]) = ra[i];
    const int chunk = s & 3;
#pragma unroll
    for (int j = 0; j < T::B_ITEMS; ++j) {
      const float d = half_bits_to_f32(rh[j][0] & 0xFFFFu), dmin = half_bits_to_f32(rh[j][0] >> 16);
      uint32_t sv0, mv0, sv1, mv1;
      q4k_scale_min(rh[j][1], rh[j][2], rh[j][3], 2 * chunk, sv0, mv0);
      q4k_scale_min(rh[j][1], rh[j][2], rh[j][3], 2 * chunk + 1, sv1, mv1);
      // low nibbles (sub-block 2c): halves are 1024+q;  high (2c+1): 1024+16q.
      const float s0 = d * (float)sv0 * b_pow[j], mn0 = dmin * (float)mv0 * b_pow[j];
      const float s1 = d * (float)sv1 * b_pow[j], mn1 = dmin * (float)mv1 * b_pow[j];
      const float neg0 = -(mn0 + 1024.f * s0), neg1 = -(mn1 + 64.f * s1), s1q = s1 * 0.0625f;
      uint32_t lo[8], hi[8];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t qw = rq[j][t], ql = qw & 0x0F0F0F0Fu, qh = qw & 0xF0F0F0F0u;
        lo[2 * t] = dq_pair(__builtin_amdgcn_perm(0x64646464u, ql, 0x04010400u), s0, neg0);
        lo[2 * t + 1] = dq_pair(__builtin_amdgcn_perm(0x64646464u, ql, 0x04030402u), s0, neg0);
        hi[2 * t] = dq_pair(__builtin_amdgcn_perm(0x64646464u, qh, 0x04010400u), s1q, neg1);
        hi[2 * t + 1] = dq_pair(__builtin_amdgcn_perm(0x64646464u, qh, 0x04030402u), s1q, neg1);
      }
      u32x4 *dl = reinterpret_cast<u32x4 *>(&lds_b[buf][b_dst[j]]);
      u32x4 *dh = reinterpret_cast<u32x4 *>(&lds_b[buf][b_dst[j] + 32]);
      dl[0] = u32x4{lo[0], lo[1], lo[2], lo[3]};
      dl[1] = u32x4{lo[4], lo[5], lo[6], lo[7]};
      dh[0] = u32x4{hi[0], hi[1], hi[2], hi[3]};
      dh[1] = u32x4{hi[4], hi[5], hi[6], hi[7]};
    }
  };

  floatx4 acc[T::TI][T::TJ];
#pragma unroll
  for (int i = 0; i < T::TI; ++i)
#pragma unroll
    for (int j = 0; j < T::TJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int frag_row = lane & 15, frag_k = 8 * (lane >> 4);
  load_stage(0);
  store_stage(0, 0);
  __syncthreads();
  for (int s = 0; s < nstages; ++s) {
    const int buf = s & 1;
    load_stage(min(s + 1, nstages - 1));
    // Keep the next stage's loads ahead of the MFMAs so their latency overlaps
    // the matrix work (the scheduler would otherwise sink them to their use).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      half8 af[T::TI], bf[T::TJ];
#pragma unroll
      for (int i = 0; i < T::TI; ++i)
        af[i] = *reinterpret_cast<const half8 *>(
            &lds_a[buf][(wm * T::WM + 16 * i + frag_row) * kPitch + 32 * sub + frag_k]);
#pragma unroll
      for (int j = 0; j < T::TJ; ++j)
        bf[j] = *reinterpret_cast<const half8 *>(
            &lds_b[buf][(wn * T::WN + 16 * j + frag_row) * kPitch + 32 * sub + frag_k]);
#pragma unroll
      for (int i = 0; i < T::TI; ++i)
#pragma unroll
        for (int j = 0; j < T::TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // Unconditional: on the last stage this refills the idle buffer, which is
    // never read again.  A conditional store lets the compiler sink the loads
    // above into the branch, after the MFMAs.
    store_stage(s + 1, buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds C[4*(lane/16)+r][lane%16] of every 16x16 tile.
  int ecol[T::TJ];
#pragma unroll
  for (int j = 0; j < T::TJ; ++j) {
    const int col = n0 + wn * T::WN + 16 * j + frag_row;
    ecol[j] = col < N ? ew[col] : 0;
  }
#pragma unroll
  for (int i = 0; i < T::TI; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + wm * T::WM + 16 * i + 4 * (lane >> 4) + r;
      if (row >= M) continue;
      const int er = ea[row];
      float *crow = c + (size_t)row * N;
#pragma unroll
      for (int j = 0; j < T::TJ; ++j) {
        const int col = n0 + wn * T::WN + 16 * j + frag_row;
        if (col < N) crow[col] = __builtin_amdgcn_ldexpf(acc[i][j][r], er + ecol[j]);
      }
    }
  }
}

template <int BM, int BN, int WGM, int WGN>
hipError_t launch_tile(const _Float16 *a16, const int *ea, const uint8_t *w, const int *ew, float *c, int M, int N,
                       int K, hipStream_t s) {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  hipLaunchKernelGGL((k_q4k_gemm<BM, BN, WGM, WGN>), dim3(tiles_m * tiles_n), dim3(256), 0, s, a16, ea, w, ew, c, M,
                     N, K, tiles_n);
  return hipGetLastError();
}

}  // namespace

size_t q4k_gemm_workspace_bytes(int M, int N, int K) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  return r256((size_t)M * K * 2) + r256((size_t)M * 4) + r256((size_t)N * 4);
}

hipError_t launch_q4k_gemm(const void *a, bool a_bf16, const void *w, float *c, int M, int N, int K, void *ws,
                           hipStream_t s) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  char *p = static_cast<char *>(ws);
  _Float16 *a16 = reinterpret_cast<_Float16 *>(p);
  int *ea = reinterpret_cast<int *>(p + r256((size_t)M * K * 2));
  int *ew = reinterpret_cast<int *>(p + r256((size_t)M * K * 2) + r256((size_t)M * 4));
  const uint8_t *wb = static_cast<const uint8_t *>(w);
  const int prep_blocks = M + (N + 255) / 256;
  if (a_bf16)
    hipLaunchKernelGGL((k_gemm_prep<uint16_t>), dim3(prep_blocks), dim3(256), 0, s,
                       static_cast<const uint16_t *>(a), a16, ea, wb, ew, M, N, K);
  else
    hipLaunchKernelGGL((k_gemm_prep<float>), dim3(prep_blocks), dim3(256), 0, s, static_cast<const float *>(a), a16,
                       ea, wb, ew, M, N, K);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_tile<128, 128, 2, 2>(a16, ea, wb, ew, c, M, N, K, s);
}

}  // namespace rt
