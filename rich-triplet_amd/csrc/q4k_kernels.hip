// q4k_kernels.hip -- Q4_K super-block dequantisation and the bandwidth-bound
// Q4_K GEMV for gfx950.
//
// Weight layout (unchanged from GGUF, uploaded verbatim): row-major [N, K]
// with K/256 consecutive 144-byte super-blocks per row:
//   [0,2) f16 d   [2,4) f16 dmin   [4,16) 6-bit scale/min pairs   [16,144) nibbles
// Chunk c (0..3) owns nibble bytes [32c, 32c+32): low nibbles are elements
// 64c+0..31 (sub-block 2c), high nibbles are 64c+32..63 (sub-block 2c+1).
#include "rt_device.hpp"
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
// GEMV building block: one lane owns one 64-element chunk of a row (32 nibble
// bytes + its super-block header) and keeps the matching 64 activations in
// registers for every row it visits ("column resident").
// ---------------------------------------------------------------------------
struct ChunkX {
  float lo[32], hi[32];
  float sum_lo, sum_hi;
};

// Dot of one chunk against resident activations, using the reference's
// integer trick: scale*sum(q*a) - min*sum(a) per sub-block.  High nibbles are
// converted as 16*q straight from the byte (exact), and 1/16 folds into scale.
RT_DEV float q4k_chunk_dot(const uint4 hd, const uint4 qa, const uint4 qb, int c, const ChunkX &x, uint32_t mlo,
                           uint32_t mhi) {
  const float d = half_bits_to_f32(hd.x & 0xFFFFu);
  const float dm = half_bits_to_f32(hd.x >> 16);
  uint32_t sv1, mv1, sv2, mv2;
  q4k_scale_min(hd.y, hd.z, hd.w, 2 * c, sv1, mv1);
  q4k_scale_min(hd.y, hd.z, hd.w, 2 * c + 1, sv2, mv2);
  const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  float dl0 = 0.f, dl1 = 0.f, dh0 = 0.f, dh1 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = w[i] & mlo;
    const uint32_t hi = w[i] & mhi;
    dl0 += ubyte0(lo) * x.lo[4 * i + 0];
    dl1 += ubyte1(lo) * x.lo[4 * i + 1];
    dl0 += ubyte2(lo) * x.lo[4 * i + 2];
    dl1 += ubyte3(lo) * x.lo[4 * i + 3];
    dh0 += ubyte0(hi) * x.hi[4 * i + 0];
    dh1 += ubyte1(hi) * x.hi[4 * i + 1];
    dh0 += ubyte2(hi) * x.hi[4 * i + 2];
    dh1 += ubyte3(hi) * x.hi[4 * i + 3];
  }
  const float scale1 = d * (float)sv1, min1 = dm * (float)mv1;
  const float scale2 = d * (float)sv2 * 0.0625f, min2 = dm * (float)mv2;
  return scale1 * (dl0 + dl1) - min1 * x.sum_lo + scale2 * (dh0 + dh1) - min2 * x.sum_hi;
}

RT_DEV void load_chunk_x(const float *__restrict__ xs, ChunkX &x) {
  const float4 *p = reinterpret_cast<const float4 *>(xs);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 v = p[i];
    x.lo[4 * i] = v.x; x.lo[4 * i + 1] = v.y; x.lo[4 * i + 2] = v.z; x.lo[4 * i + 3] = v.w;
    const float4 u = p[8 + i];
    x.hi[4 * i] = u.x; x.hi[4 * i + 1] = u.y; x.hi[4 * i + 2] = u.z; x.hi[4 * i + 3] = u.w;
  }
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) { a += x.lo[i]; b += x.hi[i]; }
  x.sum_lo = a;
  x.sum_hi = b;
}

// Column-resident GEMV over rows [row0, row0 + rows) of one weight matrix.
// T threads = RPI rows x S chunk slots; per-block partials land in `red`
// (rows x NB floats) and are summed per row in block order at the end.
template <int NB, int T, int U>
RT_DEV void q4k_colres_rows(const uint8_t *__restrict__ W, const ChunkX &x, int row0, int rows, int n_rows,
                            float *red) {
  constexpr int S = NB * 4;
  constexpr int RPI = T / S;
  static_assert(T % S == 0 && T % 64 == 0, "tile must cover whole rows and waves");
  const int t = threadIdx.x;
  const int slot = t % S, rsub = t / S;
  const int b = slot >> 2, c = slot & 3;
  const int iters = (rows + RPI - 1) / RPI;
  const uint32_t mlo = opaque_u32(0x0F0F0F0Fu), mhi = opaque_u32(0xF0F0F0F0u);
  for (int it = 0; it < iters; it += U) {
    uint4 hd[U], qa[U], qb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int rl = (it + u) * RPI + rsub;
      const int r = row0 + rl;
      if (it + u < iters && rl < rows && r < n_rows) {
        const uint8_t *bp = W + ((size_t)r * NB + b) * kQ4KBlockBytes;
        hd[u] = *reinterpret_cast<const uint4 *>(bp);
        qa[u] = *reinterpret_cast<const uint4 *>(bp + 16 + 32 * c);
        qb[u] = *reinterpret_cast<const uint4 *>(bp + 32 + 32 * c);
      } else {
        hd[u] = make_uint4(0, 0, 0, 0);
        qa[u] = qb[u] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float p = q4k_chunk_dot(hd[u], qa[u], qb[u], c, x, mlo, mhi);
      p = quad_sum(p);
      const int rl = (it + u) * RPI + rsub;
      if (c == 0 && it + u < iters && rl < rows) red[rl * NB + b] = p;
    }
  }
}

template <int NB>
RT_DEV float reduce_row(const float *red, int rl) {
  float s = 0.f;
#pragma unroll
  for (int b = 0; b < NB; ++b) s += red[rl * NB + b];
  return s;
}

template <int NB, int T, int U>
__global__ __launch_bounds__(T) void k_q4k_gemv_cr(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                   float *__restrict__ y, int N, int rows_per_wg) {
  extern __shared__ float red[];
  constexpr int S = NB * 4;
  const int slot = threadIdx.x % S;
  ChunkX xr;
  load_chunk_x(x + slot * 64, xr);
  const int row0 = blockIdx.x * rows_per_wg;
  q4k_colres_rows<NB, T, U>(W, xr, row0, rows_per_wg, N, red);
  __syncthreads();
  for (int i = threadIdx.x; i < rows_per_wg; i += T) {
    const int r = row0 + i;
    if (r < N) y[r] = reduce_row<NB>(red, i);
  }
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
    load_chunk_x(x + ci * 64, xr);
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

template <int NB, int T, int U>
static hipError_t launch_cr(const void *W, const float *x, float *y, int N, int rows_per_wg, hipStream_t s) {
  const unsigned grid = (unsigned)((N + rows_per_wg - 1) / rows_per_wg);
  const size_t lds = (size_t)rows_per_wg * NB * sizeof(float);
  hipLaunchKernelGGL((k_q4k_gemv_cr<NB, T, U>), dim3(grid), dim3(T), lds, s, (const uint8_t *)W, x, y, N,
                     rows_per_wg);
  return hipGetLastError();
}

int q4k_gemv_rows_per_wg(int N, int K) {
  // Aim for >= 2 workgroups per CU (256 CUs) while keeping whole iterations.
  const int nb = K / kQ4KBlockElems;
  int rpi;
  switch (nb) {
    case 8: rpi = 256 / 32; break;
    case 10: rpi = 320 / 40; break;
    case 40: rpi = 320 / 160; break;
    default: return 0;
  }
  int rows = rpi;
  while (rows < 64 && (N + 2 * rows - 1) / (2 * rows) >= 512) rows *= 2;
  return rows;
}

hipError_t launch_q4k_gemv(const void *W, const float *x, float *y, int N, int K, hipStream_t s) {
  const int nb = K / kQ4KBlockElems;
  const int rows = q4k_gemv_rows_per_wg(N, K);
  switch (nb) {
    case 8: return launch_cr<8, 256, 2>(W, x, y, N, rows, s);
    case 10: return launch_cr<10, 320, 2>(W, x, y, N, rows, s);
    case 40: return launch_cr<40, 320, 2>(W, x, y, N, rows, s);
    default: break;
  }
  const unsigned grid = (unsigned)((N + 3) / 4);
  hipLaunchKernelGGL(k_q4k_gemv_generic, dim3(grid), dim3(256), 0, s, (const uint8_t *)W, x, y, N, K);
  return hipGetLastError();
}

hipError_t launch_q4k_gemv_generic(const void *W, const float *x, float *y, int N, int K, hipStream_t s) {
  const unsigned grid = (unsigned)((N + 3) / 4);
  hipLaunchKernelGGL(k_q4k_gemv_generic, dim3(grid), dim3(256), 0, s, (const uint8_t *)W, x, y, N, K);
  return hipGetLastError();
}

}  // namespace rt
