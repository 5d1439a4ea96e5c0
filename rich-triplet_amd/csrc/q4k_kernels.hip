// q4k_kernels.hip -- Q4_K super-block dequantisation and the bandwidth-bound
// Q4_K GEMV for gfx950.
//
// Weight layout (unchanged from GGUF, uploaded verbatim): row-major [N, K]
// with K/256 consecutive 144-byte super-blocks per row:
//   [0,2) f16 d   [2,4) f16 dmin   [4,16) 6-bit scale/min pairs   [16,144) nibbles
// Chunk c (0..3) owns nibble bytes [32c, 32c+32): low nibbles are elements
// 64c+0..31 (sub-block 2c), high nibbles are 64c+32..63 (sub-block 2c+1).
#include "rt_device.hpp"
#include "q4k_gemv.hpp"
#include "rt_kernels.hpp"

namespace rt {

// ---------------------------------------------------------------------------
// Dequantisation (bit-exact with the reference's scalar CPU path:
//   w = (d*sv)*q - (dmin*mv), each product and the difference rounded in f32).
// One thread per (block, 16 nibble bytes) -> 32 outputs.
// ---------------------------------------------------------------------------
template <bool BF16>
__global__ __launch_bounds__(256) void k_q4k_dequant(const uint8_t *__restrict__ blocks, size_t n_blocks,
                                                     void *__restrict__ out) {
#pragma clang fp contract(off)
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t g = tid >> 3;  // block
  if (g >= n_blocks) return;
  const int piece = (int)(tid & 7);  // 16-byte piece of the 128 nibble bytes
  const int c = piece >> 1, h = piece & 1;
  const uint8_t *bp = blocks + g * kQ4KBlockBytes;
  const uint4 hd = *reinterpret_cast<const uint4 *>(bp);
  const uint4 qv = *reinterpret_cast<const uint4 *>(bp + 16 + 16 * piece);
  const float d = half_bits_to_f32(hd.x & 0xFFFFu);
  const float dm = half_bits_to_f32(hd.x >> 16);
  uint32_t sv1, mv1, sv2, mv2;
  q4k_scale_min(hd.y, hd.z, hd.w, 2 * c, sv1, mv1);
  q4k_scale_min(hd.y, hd.z, hd.w, 2 * c + 1, sv2, mv2);
  const float scale1 = d * (float)sv1, min1 = dm * (float)mv1;
  const float scale2 = d * (float)sv2, min2 = dm * (float)mv2;
  const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
  float lo[16], hi[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t byte = (w[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    lo[i] = scale1 * (float)(byte & 15u) - min1;
    hi[i] = scale2 * (float)(byte >> 4) - min2;
  }
  const size_t e0 = g * kQ4KBlockElems + 64 * c + 16 * h;  // first low-nibble element
  if (!BF16) {
    float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + e0);
    float4 *o2 = reinterpret_cast<float4 *>(static_cast<float *>(out) + e0 + 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] = make_float4(lo[4 * i], lo[4 * i + 1], lo[4 * i + 2], lo[4 * i + 3]);
      o2[i] = make_float4(hi[4 * i], hi[4 * i + 1], hi[4 * i + 2], hi[4 * i + 3]);
    }
  } else {
    uint4 *o = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + e0);
    uint4 *o2 = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + e0 + 32);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint32_t a[4], b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a[j] = (uint32_t)f32_to_bf16_bits(lo[8 * i + 2 * j]) | ((uint32_t)f32_to_bf16_bits(lo[8 * i + 2 * j + 1]) << 16);
        b[j] = (uint32_t)f32_to_bf16_bits(hi[8 * i + 2 * j]) | ((uint32_t)f32_to_bf16_bits(hi[8 * i + 2 * j + 1]) << 16);
      }
      o[i] = make_uint4(a[0], a[1], a[2], a[3]);
      o2[i] = make_uint4(b[0], b[1], b[2], b[3]);
    }
  }
}

// ---------------------------------------------------------------------------
// Standalone GEMV: y[N] = W[N,K] . x[K]
// ---------------------------------------------------------------------------
template <int NB, int T, int ITERS>
__global__ __launch_bounds__(T) void k_q4k_gemv_cr(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                   float *__restrict__ y, int N) {
  using Tile = Q4KTile<NB, T, ITERS>;
  __shared__ __attribute__((aligned(16))) float xl[NB * 4 * kXPitch];
  __shared__ float red[Tile::ROWS * NB];
  Tile tile;
  const int row0 = (int)blockIdx.x * Tile::ROWS;
  const size_t row_bytes = (size_t)NB * kQ4KBlockBytes;
  XRegs<NB * 256, T> xr;
  x_load<NB * 256, T>(x, xr);
  tile.load([&](int rl) -> const uint8_t * {
    const int r = row0 + rl;
    return r < N ? W + (size_t)r * row_bytes : nullptr;
  }, W);
  x_store<NB * 256, T>(xr, xl);
  __syncthreads();
  ChunkX cx;
  chunkx_from_lds(xl, tile.slot, cx);
  tile.compute(cx, red);
  __syncthreads();
  for (int i = threadIdx.x; i < Tile::ROWS; i += T) {
    const int r = row0 + i;
    if (r < N) y[r] = reduce_row<NB>(red, i);
  }
}


// Digit-staged activations, all ITERS row-iterations of a workgroup in flight:
// rows [row0, row0 + ROWS) of W.
template <int NB, int T, int ITERS>
RT_DEV void gemv_dig_tile(const uint8_t *__restrict__ W, const float *__restrict__ x, float *__restrict__ y, int N,
                          int row0) {
  using Tile = Q4KTile<NB, T, ITERS>;
  __shared__ __attribute__((aligned(16))) uint32_t dl[NB * 4 * kDPitch];
  __shared__ float red[Tile::ROWS * NB];
  Tile tile;
  const size_t row_bytes = (size_t)NB * kQ4KBlockBytes;
  XRegs<NB * 256, T> xr;
  x_load<NB * 256, T>(x, xr);
  // With a 40 KB activation vector every wave's activation loads go out
  // before any weight load of the workgroup, so they do not queue behind
  // the first waves' weight stream (smaller vectors do better without the
  // barrier)
  if constexpr (NB >= 40) __syncthreads();
  tile.load([&](int rl) -> const uint8_t * {
    const int r = row0 + rl;
    return r < N ? W + (size_t)r * row_bytes : nullptr;
  }, W);
  x_store_digits<NB * 256, T>(xr, dl);
  __syncthreads();
  ChunkD cx;
  chunkd_from_lds(dl, tile.slot, cx);
  tile.compute_digits(cx, red);
  __syncthreads();
  for (int i = threadIdx.x; i < Tile::ROWS; i += T) {
    const int r = row0 + i;
    if (r < N) y[r] = reduce_row<NB>(red, i);
  }
}

template <int NB, int T, int ITERS>
__global__ __launch_bounds__(T) void k_q4k_gemv_dig(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                    float *__restrict__ y, int N) {
  gemv_dig_tile<NB, T, ITERS>(W, x, y, N, (int)blockIdx.x * Q4KTile<NB, T, ITERS>::ROWS);
}

// Several matrices sharing x in one launch: workgroup b takes a row tile of
// matrix i with tile0[i] <= b < tile0[i+1] (every matrix covers whole tiles;
// rows past its end are masked).
struct GemvMats {
  const uint8_t *w[kGemvMaxMats];
  float *y[kGemvMaxMats];
  int n[kGemvMaxMats];
  int tile0[kGemvMaxMats + 1];
  int count;
};

// The matrix is picked with constant indices only (every bound and pointer is
// read from the kernel arguments at once, then selected): a loop over
// tile0[i] makes a chain of dependent scalar loads that holds back the first
// activation and weight loads by about 0.25 us.
template <int NB, int T, int ITERS>
__global__ __launch_bounds__(T) void k_q4k_gemv_dig_multi(GemvMats m, const float *__restrict__ x) {
  const int b = (int)blockIdx.x;
  const uint8_t *w = m.w[0];
  float *y = m.y[0];
  int n = m.n[0], t0 = 0;
#pragma unroll
  for (int j = 1; j < kGemvMaxMats; ++j) {
    const bool in = j < m.count && b >= m.tile0[j];
    w = in ? m.w[j] : w;
    y = in ? m.y[j] : y;
    n = in ? m.n[j] : n;
    t0 = in ? m.tile0[j] : t0;
  }
  gemv_dig_tile<NB, T, ITERS>(w, x, y, n, (b - t0) * Q4KTile<NB, T, ITERS>::ROWS);
}

// Any K (multiple of 256): one wave per row, lanes stride over the row's chunks.
__global__ __launch_bounds__(256) void k_q4k_gemv_generic(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                          float *__restrict__ y, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
  if (row >= N) return;
  const int nb = K / kQ4KBlockElems, nchunks = nb * 4;
  float acc = 0.f;
  const uint32_t mlo = opaque_u32(0x0F0F0F0Fu), mhi = opaque_u32(0xF0F0F0F0u);
  for (int ci = lane; ci < nchunks; ci += 64) {
    const int b = ci >> 2, c = ci & 3;
    const uint8_t *bp = W + ((size_t)row * nb + b) * kQ4KBlockBytes;
    const uint4 hd = *reinterpret_cast<const uint4 *>(bp);
    const uint4 qa = *reinterpret_cast<const uint4 *>(bp + 16 + 32 * c);
    const uint4 qb = *reinterpret_cast<const uint4 *>(bp + 32 + 32 * c);
    ChunkX xr;
    const float4 *xp = reinterpret_cast<const float4 *>(x + ci * 64);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = xp[i], u = xp[8 + i];
      xr.lo[4 * i] = v.x; xr.lo[4 * i + 1] = v.y; xr.lo[4 * i + 2] = v.z; xr.lo[4 * i + 3] = v.w;
      xr.hi[4 * i] = u.x; xr.hi[4 * i + 1] = u.y; xr.hi[4 * i + 2] = u.z; xr.hi[4 * i + 3] = u.w;
    }
    float a = 0.f, bsum = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) { a += xr.lo[i]; bsum += xr.hi[i]; }
    xr.sum_lo = a;
    xr.sum_hi = bsum;
    acc += q4k_chunk_dot(hd, qa, qb, c, xr, mlo, mhi);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
hipError_t launch_q4k_dequant(const void *blocks, size_t n_blocks, void *out, bool bf16, hipStream_t s) {
  if (n_blocks == 0) return hipSuccess;
  const size_t threads = n_blocks * 8;
  const unsigned grid = (unsigned)((threads + 255) / 256);
  if (bf16)
    hipLaunchKernelGGL((k_q4k_dequant<true>), dim3(grid), dim3(256), 0, s, (const uint8_t *)blocks, n_blocks, out);
  else
    hipLaunchKernelGGL((k_q4k_dequant<false>), dim3(grid), dim3(256), 0, s, (const uint8_t *)blocks, n_blocks, out);
  return hipGetLastError();
}


template <int NB, int T, int ITERS>
static hipError_t launch_cr(const void *W, const float *x, float *y, int N, hipStream_t s) {
  constexpr int ROWS = Q4KTile<NB, T, ITERS>::ROWS;
  const unsigned grid = (unsigned)((N + ROWS - 1) / ROWS);
  hipLaunchKernelGGL((k_q4k_gemv_cr<NB, T, ITERS>), dim3(grid), dim3(T), 0, s, (const uint8_t *)W, x, y, N);
  return hipGetLastError();
}

// Row-iterations per workgroup: enough rows per workgroup to amortise the
// activation staging, while keeping >= ~320 workgroups for 256 CUs.
template <int NB, int T>
static hipError_t launch_cr_auto(const void *W, const float *x, float *y, int N, hipStream_t s) {
  constexpr int RPI = T / (NB * 4);
  if (N >= 320 * 4 * RPI) return launch_cr<NB, T, 4>(W, x, y, N, s);
  if (N >= 320 * 2 * RPI) return launch_cr<NB, T, 2>(W, x, y, N, s);
  return launch_cr<NB, T, 1>(W, x, y, N, s);
}

hipError_t launch_q4k_gemv_generic(const void *W, const float *x, float *y, int N, int K, hipStream_t s) {
  const unsigned grid = (unsigned)((N + 3) / 4);
  hipLaunchKernelGGL(k_q4k_gemv_generic, dim3(grid), dim3(256), 0, s, (const uint8_t *)W, x, y, N, K);
  return hipGetLastError();
}

template <int NB, int T, int ITERS>
static hipError_t launch_dig(const void *W, const float *x, float *y, int N, hipStream_t s) {
  constexpr int ROWS = Q4KTile<NB, T, ITERS>::ROWS;
  const unsigned grid = (unsigned)((N + ROWS - 1) / ROWS);
  hipLaunchKernelGGL((k_q4k_gemv_dig<NB, T, ITERS>), dim3(grid), dim3(T), 0, s, (const uint8_t *)W, x, y, N);
  return hipGetLastError();
}

// Kernel choice per shape, from measurements on MI355X (graph-launched, cold
// weights, 34 distinct matrices back to back).  The Gemma-3 shapes use
// digit-staged activations with workgroup sizes that trade activation staging
// (once per workgroup) against parallelism: K=2560 with 8 rows per workgroup
// up to 8k rows, 48 rows (960 threads, two row-iterations) up to 12k, 32 rows
// beyond; K=2048 with 16 rows; K=10240 with 6 rows (960 threads).  Other K's
// use the f32-staged tile.
template <int NB, int T, int ITERS>
static hipError_t launch_dig_multi(const void *const *w, float *const *y, const int *n, int count, const float *x,
                                   hipStream_t s) {
  constexpr int ROWS = Q4KTile<NB, T, ITERS>::ROWS;
  GemvMats m{};
  m.count = count;
  m.tile0[0] = 0;
  for (int i = 0; i < count; ++i) {
    m.w[i] = static_cast<const uint8_t *>(w[i]);
    m.y[i] = y[i];
    m.n[i] = n[i];
    m.tile0[i + 1] = m.tile0[i] + (n[i] + ROWS - 1) / ROWS;
  }
  hipLaunchKernelGGL((k_q4k_gemv_dig_multi<NB, T, ITERS>), dim3(m.tile0[count]), dim3(T), 0, s, m, x);
  return hipGetLastError();
}

// Matrices sharing x in one launch (q|k|v, gate|up): the fixed cost of a
// launch (about 2 us from the previous kernel's end to this one's first
// weights) is paid once for all of them.  Tiles for K=2560 from measurements
// of the combined row count; other K's run one launch per matrix.
hipError_t launch_q4k_gemv_multi(const void *const *w, float *const *y, const int *n, int count, const float *x,
                                 int K, hipStream_t s) {
  if (count < 1 || count > kGemvMaxMats) return hipErrorInvalidValue;
  if (K == 2560) {
    int total = 0;
    for (int i = 0; i < count; ++i) total += n[i];
    if (total > 12288) return launch_dig_multi<10, 320, 2>(w, y, n, count, x, s);
    if (total >= 8192) return launch_dig_multi<10, 960, 2>(w, y, n, count, x, s);
    return launch_dig_multi<10, 640, 1>(w, y, n, count, x, s);
  }
  for (int i = 0; i < count; ++i) {
    const hipError_t e = launch_q4k_gemv(w[i], x, y[i], n[i], K, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_q4k_gemv(const void *W, const float *x, float *y, int N, int K, hipStream_t s) {
  switch (K / kQ4KBlockElems) {
    case 1: return launch_cr_auto<1, 256>(W, x, y, N, s);
    case 2: return launch_cr_auto<2, 256>(W, x, y, N, s);
    case 4: return launch_cr_auto<4, 256>(W, x, y, N, s);
    case 8: return launch_dig<8, 512, 1>(W, x, y, N, s);
    case 10:
      if (N > 12288) return launch_dig<10, 640, 2>(W, x, y, N, s);
      if (N >= 8192) return launch_dig<10, 960, 2>(W, x, y, N, s);
      return launch_dig<10, 320, 1>(W, x, y, N, s);
    case 16: return launch_cr_auto<16, 256>(W, x, y, N, s);
    case 40: return launch_dig<40, 960, 2>(W, x, y, N, s);
    default: break;
  }
  return launch_q4k_gemv_generic(W, x, y, N, K, s);
}

}  // namespace rt
