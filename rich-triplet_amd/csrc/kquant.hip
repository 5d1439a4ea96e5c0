// kquant.hip -- Q6_K and Q8_0 weights kept packed in HBM: repacking, exact
// dequantisation and the decode GEMV y = W x.
//
// The reference widens both types to f32 and then BF16 at load
// (load_linear_from_gguf, transformer4.rs:1233-1242, via decode_q6k_to_f32
// gguf_loader.rs:482-549 and decode_q8_0_to_f32 628-650), so its GPU GEMV
// streams 16 bits per weight.  Here Q6_K stays at 6.5625 bits and Q8_0 at
// 8.5: 2.4x and 1.9x fewer bytes for the same matrix.
//
// Device layout (planar, filled by rt_q6k_repack / rt_q8_0_repack from the
// GGUF blocks).  GGUF interleaves fields inside 210-byte (Q6_K) and 34-byte
// (Q8_0) blocks, which leaves most fields 2-byte aligned; each field gets its
// own plane so every lane load is an aligned 16-byte load:
//   Q6_K [N][K], nb = K/256 blocks per row, nbt = N*nb:
//     QL [nbt][128] low nibbles | QH [nbt][64] high bit pairs |
//     SC [nbt][16] int8 sub-block scales | D [nbt] f16 block scales
//   Q8_0 [N][K], nb = K/32:
//     QS [N][K] int8 | D [N*nb] f16
// Both are exactly as many bytes as the GGUF tensor.
//
// GEMV arithmetic: the activation vector is staged once per workgroup as
// 16-bit integer digits per 64-element chunk (stage_digits_store:
// X = rint(x * 2^sh) = 256*x1 + x0), and the weight codes multiply the digits
// in exact integer dot products:
//   Q6_K  q = ql | qh << 4 in 0..63, w = d * sc * (q - 32):
//         per 16-element sub-block  T = sum X q - 32 sum X  (|T| < 2^24, exact)
//   Q8_0  q in -128..127, w = d * q:  with q' = q ^ 0x80 = q + 128 (unsigned),
//         sum x0 q = sum x0 q' - 128 sum x0, so both digits use v_dot4 forms
//         with matching signedness.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>

#include "q4k_gemv.hpp"
#include "rt_device.hpp"
#include "kquant_layout.hpp"
#include "kquant_tile.hpp"
#include "rt_kernels.hpp"

namespace rt {
namespace {


// ---------------------------------------------------------------------------
// Dequantisation (bit-exact with decode_q6k_to_f32 / decode_q8_0_to_f32:
// s = d * sc in f32, then s * q)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_q6k_dequant(const uint8_t *__restrict__ w, size_t nbt,
                                                     float *__restrict__ out) {
#pragma clang fp contract(off)
  const Q6KPlanes P = q6k_planes(w, nbt);
  const size_t total = nbt * 256;
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (size_t)gridDim.x * 256)
    out[e] = q6k_value(P, e >> 8, (int)(e & 255));
}

__global__ __launch_bounds__(256) void k_q8_0_dequant(const uint8_t *__restrict__ w, size_t n_elem,
                                                      float *__restrict__ out) {
#pragma clang fp contract(off)
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n_elem; e += (size_t)gridDim.x * 256)
    out[e] = q8_0_value(w, n_elem, e);
}

// ---------------------------------------------------------------------------
// Q6_K GEMV: the activation vector staged as digits once per workgroup, then
// the Q6KTile of ROWS rows (kquant_tile.hpp).
// ---------------------------------------------------------------------------
template <int NB, int T, int ITERS>
__global__ __launch_bounds__(T) void k_q6k_gemv(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                float *__restrict__ y, int n) {
  using Tile = Q6KTile<NB, T, ITERS>;
  constexpr int K = NB * 256;
  __shared__ __attribute__((aligned(16))) uint32_t dl[K / 64 * kDPitch];
  __shared__ float red[Tile::ROWS * NB];
  const int row0 = (int)blockIdx.x * Tile::ROWS;
  XRegs<K, T> xr;
  x_load<K, T>(x, xr);
  Tile tile;
  tile.load(q6k_planes(W, (size_t)n * NB), row0, n);
  x_store_digits<K, T>(xr, dl);
  __syncthreads();
  tile.compute(dl, red);
  __syncthreads();
  for (int i = (int)threadIdx.x; i < Tile::ROWS; i += T)
    if (row0 + i < n) y[row0 + i] = reduce_row<NB>(red, i);
}

// ---------------------------------------------------------------------------
// Q8_0 GEMV: the activation vector staged as digits once per workgroup, then
// the Q8Tile of ROWS rows (kquant_tile.hpp).
// ---------------------------------------------------------------------------
template <int NB32, int T, int ITERS>
__global__ __launch_bounds__(T) void k_q8_0_gemv(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                 float *__restrict__ y, int n) {
  using Tile = Q8Tile<NB32, T, ITERS>;
  constexpr int K = NB32 * kQ8Block;
  __shared__ __attribute__((aligned(16))) uint32_t dl[K / 64 * kDPitch];
  __shared__ float red[Tile::ROWS * Tile::RED];
  const uint16_t *D = reinterpret_cast<const uint16_t *>(W + (size_t)n * K);
  const int row0 = (int)blockIdx.x * Tile::ROWS;
  XRegs<K, T> xr;
  x_load<K, T>(x, xr);
  Tile tile;
  // rows past n read row n - 1 and are never stored
  tile.load([&](int rl) { return W + (size_t)min(row0 + rl, n - 1) * K; },
            [&](int rl) { return D + (size_t)min(row0 + rl, n - 1) * NB32; });
  x_store_digits<K, T>(xr, dl);
  __syncthreads();
  tile.compute(dl, red);
  __syncthreads();
  for (int i = (int)threadIdx.x; i < Tile::ROWS; i += T)
    if (row0 + i < n) y[row0 + i] = Tile::reduce(red, i);
}

// ---------------------------------------------------------------------------
// Generic fallbacks (any K that is a whole number of blocks): one wave per
// row, f32 arithmetic on activations read from global memory.
__global__ __launch_bounds__(256) void k_q6k_gemv_generic(const uint8_t *__restrict__ W,
                                                          const float *__restrict__ x, float *__restrict__ y, int n,
                                                          int nb) {
  const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  if (row >= n) return;
  const Q6KPlanes P = q6k_planes(W, (size_t)n * nb);
  float acc = 0.f;
  for (int e = lane; e < nb * 256; e += 64) {
    const size_t blk = (size_t)row * nb + (e >> 8);
    const int i = e & 255, j = i >> 7, h = i & 127, m = h >> 5, l = h & 31;
    const uint8_t ql = P.ql[blk * 128 + 64 * j + 32 * (m & 1) + l];
    const uint8_t qh = P.qh[blk * 64 + 32 * j + l];
    const int q = (int)(((m < 2 ? ql & 15 : ql >> 4)) | (((qh >> (2 * m)) & 3) << 4)) - 32;
    const float w = half_bits_to_f32(P.d[blk]) * (float)(int8_t)P.sc[blk * 16 + 8 * j + (l >> 4) + 2 * m];
    acc = fmaf(w * (float)q, x[e], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

__global__ __launch_bounds__(256) void k_q8_0_gemv_generic(const uint8_t *__restrict__ W,
                                                           const float *__restrict__ x, float *__restrict__ y, int n,
                                                           int k) {
  const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  if (row >= n) return;
  const uint16_t *D = reinterpret_cast<const uint16_t *>(W + (size_t)n * k);
  const int8_t *q = reinterpret_cast<const int8_t *>(W) + (size_t)row * k;
  float acc = 0.f;
  for (int e = lane; e < k; e += 64)
    acc = fmaf(half_bits_to_f32(D[((size_t)row * k + e) / kQ8Block]) * (float)q[e], x[e], acc);
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

template <int NB, int T, int ITERS>
hipError_t launch_q6k(const void *W, const float *x, float *y, int n, hipStream_t s) {
  constexpr int ROWS = T / (4 * NB) * ITERS;
  hipLaunchKernelGGL((k_q6k_gemv<NB, T, ITERS>), dim3((n + ROWS - 1) / ROWS), dim3(T), 0, s,
                     static_cast<const uint8_t *>(W), x, y, n);
  return hipGetLastError();
}

template <int NB32, int T, int ITERS>
hipError_t launch_q8(const void *W, const float *x, float *y, int n, hipStream_t s) {
  constexpr int ROWS = T / NB32 * ITERS;
  hipLaunchKernelGGL((k_q8_0_gemv<NB32, T, ITERS>), dim3((n + ROWS - 1) / ROWS), dim3(T), 0, s,
                     static_cast<const uint8_t *>(W), x, y, n);
  return hipGetLastError();
}

}  // namespace

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
void q6k_repack_host(const uint8_t *src, size_t n_blocks, uint8_t *dst) {
  uint8_t *ql = dst, *qh = dst + n_blocks * 128, *sc = dst + n_blocks * 192, *d = dst + n_blocks * 208;
  for (size_t b = 0; b < n_blocks; ++b) {
    const uint8_t *bp = src + b * kQ6KBlockBytes;
    std::memcpy(ql + b * 128, bp, 128);
    std::memcpy(qh + b * 64, bp + 128, 64);
    std::memcpy(sc + b * 16, bp + 192, 16);
    std::memcpy(d + b * 2, bp + 208, 2);
  }
}

void q8_0_repack_host(const uint8_t *src, size_t n_blocks, uint8_t *dst) {
  uint8_t *qs = dst, *d = dst + n_blocks * kQ8Block;
  for (size_t b = 0; b < n_blocks; ++b) {
    const uint8_t *bp = src + b * kQ8BlockBytes;
    std::memcpy(d + b * 2, bp, 2);
    std::memcpy(qs + b * kQ8Block, bp + 2, kQ8Block);
  }
}

hipError_t launch_q6k_dequant(const void *w, size_t n_blocks, float *out, hipStream_t s) {
  const unsigned grid = (unsigned)std::min<size_t>(n_blocks, 65536);
  hipLaunchKernelGGL(k_q6k_dequant, dim3(grid), dim3(256), 0, s, static_cast<const uint8_t *>(w), n_blocks, out);
  return hipGetLastError();
}

hipError_t launch_q8_0_dequant(const void *w, size_t n_elem, float *out, hipStream_t s) {
  const unsigned grid = (unsigned)std::min<size_t>((n_elem + 255) / 256, 65536);
  hipLaunchKernelGGL(k_q8_0_dequant, dim3(grid), dim3(256), 0, s, static_cast<const uint8_t *>(w), n_elem, out);
  return hipGetLastError();
}

hipError_t launch_q6k_gemv(const void *W, const float *x, float *y, int N, int K, hipStream_t s) {
  switch (K) {
    case 2048: return launch_q6k<8, 256, 1>(W, x, y, N, s);
    case 2560: return N >= 4096 ? launch_q6k<10, 320, 2>(W, x, y, N, s) : launch_q6k<10, 320, 1>(W, x, y, N, s);
    // 12 rows per workgroup (214 for 2560 rows): 8.1-8.2 us at 2560x10240
    // against 8.4-10.7 us for 4 to 18 rows (34 distinct matrices in a graph)
    case 10240: return launch_q6k<40, 960, 2>(W, x, y, N, s);
    default:
      hipLaunchKernelGGL(k_q6k_gemv_generic, dim3((N + 3) / 4), dim3(256), 0, s, static_cast<const uint8_t *>(W),
                         x, y, N, K / 256);
      return hipGetLastError();
  }
}

hipError_t launch_q8_0_gemv(const void *W, const float *x, float *y, int N, int K, hipStream_t s) {
  switch (K) {
    case 2048: return launch_q8<64, 256, 1>(W, x, y, N, s);
    case 2560: return N >= 4096 ? launch_q8<80, 320, 2>(W, x, y, N, s) : launch_q8<80, 320, 1>(W, x, y, N, s);
    // 6 rows per workgroup (427 for 2560 rows): 8.6 us at 2560x10240 against
    // 8.8-11.1 us for 2 to 9 rows (34 distinct matrices in a graph)
    case 10240: return launch_q8<320, 960, 2>(W, x, y, N, s);
    default:
      hipLaunchKernelGGL(k_q8_0_gemv_generic, dim3((N + 3) / 4), dim3(256), 0, s, static_cast<const uint8_t *>(W),
                         x, y, N, K);
      return hipGetLastError();
  }
}

}  // namespace rt
