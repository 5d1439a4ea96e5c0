// q4k_gemv_mb.hip -- batched Q4_K GEMV, C[m][n] = sum_k A[m][k] W[n][k] for
// M <= 8 activation rows, on the int8 matrix cores (v_mfma_i32_16x16x64_i8).
//
// Replaces gemv_q4k_t_batch (metal_decode.rs:459-521), the GEMV of the
// speculative verify batch: one pass over the weights for all M rows, where
// the reference's kernel runs its per-row float loop M times per block.
//
// Activations (k_mb_stage).  Each 64-element chunk of each row is scaled to
// integers X = rint(x * s), s = 32639 / 2^e with max |x| < 2^e, so
// |X| <= 32639, and written as two balanced signed bytes X = 256*x1 + x0
// (x0, x1 in -128..127).  The rounding is one FMA, x*s + (1.5*2^23 + 128):
// the low 16 mantissa bits of the sum are X + 128.  Per (chunk, row) the
// stage keeps delta = 2^e / 32639 and the f32 sums of x over the chunk's two
// 32-element sub-blocks (the min term of the integer trick).
//   layout: dig[(chunk*8 + row)*2 + digit][64] bytes, stats[chunk*8 + row]
//   = {delta, sum_lo, sum_hi, 0}; rows M..7 are zero.
//
// Product.  Lane l of a wave (j = l%16, g = l/16) is A row j = (row m = j/2,
// digit d = j%2) and B column j = (weight row r = j/2, sub-block half
// h = j%2); byte i of its operands is element 16g + i of the chunk.  A holds
// digit d of row m; B holds the 4-bit codes of weight row r where the element
// lies in half h (elements 0..31: low nibbles of qs[0..32), sub-block 2c;
// 32..63: high nibbles, sub-block 2c+1) and zero elsewhere.  So
//   C[(m,d)][(r,h)] = sum over sub-block 2c+h of q * x_d     (exact int32)
// and lane (j, g) receives rows 4g..4g+3 of C: rows m = 2g, 2g+1, both
// digits, for its (r, h).  The epilogue applies the scales:
//   acc[m] += d*sv*delta_m * (256 C1 + C0) - dmin*mv * sum_m(sub-block)
// and lanes (r, 0) and (r, 1) add their halves at the end.  A wave owns 16
// weight rows (two B operands against one A), a workgroup 64 rows and a
// slice of one or two super-blocks; with several slices each writes partial
// sums that k_mb_reduce adds in slice order.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "q4k_gemv_mb.hpp"
#include "rt_device.hpp"

namespace rt {
namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_mb_stage(const float *__restrict__ x, int m, int k,
                                                  int8_t *__restrict__ dig, float *__restrict__ stats) {
  const int nchunk = k / 64;
  const int ci = (int)blockIdx.x * 16 + (int)(threadIdx.x >> 4), q = (int)(threadIdx.x & 15);
  const int row = (int)blockIdx.y;  // 0..7; rows m..7 are staged as zeros
  const int c = min(ci, nchunk - 1);
  const float4 v = row < m ? *reinterpret_cast<const float4 *>(x + (size_t)row * k + 64 * c + 4 * q)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
  mb_stage4(dig, stats, row, c, q, v, ci < nchunk);
}

template <int SB>
__global__ __launch_bounds__(256) void k_q4k_gemv_mb(MbArgs p) {
  // A workgroup: 64 rows (16 per wave, two B operands of 8 rows) times a
  // slice of SB super-blocks.  The slice's activation digits and stats are
  // copied to LDS once; every weight load of the slice is issued before the
  // first MFMA, so the many small workgroups hide each other's latency.
  constexpr int CH = 4 * SB;  // chunks in the slice
  __shared__ __attribute__((aligned(16))) int8_t a_lds[CH * 1024];
  __shared__ __attribute__((aligned(16))) float4 st_lds[CH * 8];
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int j = lane & 15, g = lane >> 4, r = j >> 1, h = j & 1;
  int rb = (int)blockIdx.x, mi = 0;
  while (mi + 1 < p.nmat && rb >= p.mat[mi].row_blocks) rb -= p.mat[mi++].row_blocks;
  const MbMat &M = p.mat[mi];
  const int nb = p.k / 256, slice = (int)blockIdx.y;
  const int sb0 = slice * SB;  // the launcher makes SB divide nb
  const size_t row_bytes = (size_t)nb * kQ4KBlockBytes;
  int row[2];
  const uint8_t *wp[2];
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    row[gi] = rb * 64 + wave * 16 + 8 * gi + r;
    wp[gi] = M.w + (size_t)min(row[gi], M.n - 1) * row_bytes + (size_t)sb0 * kQ4KBlockBytes;
  }
  const bool carries = (g >> 1) == h;  // this lane's k-slots lie in sub-block half h
  const int qoff = 16 + 16 * (g & 1);
  // weights of the whole slice
  uint4 hd[2][SB], qw[2][SB][4];
#pragma unroll
  for (int gi = 0; gi < 2; ++gi)
#pragma unroll
    for (int b = 0; b < SB; ++b) {
      hd[gi][b] = *reinterpret_cast<const uint4 *>(wp[gi] + b * kQ4KBlockBytes);
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
        qw[gi][b][cc] = carries ? *reinterpret_cast<const uint4 *>(wp[gi] + b * kQ4KBlockBytes + qoff + 32 * cc)
                                : make_uint4(0u, 0u, 0u, 0u);
    }
  // activations of the slice: CH KB of digits, CH*8 stats
  {
    const uint4 *src = reinterpret_cast<const uint4 *>(p.dig + (size_t)sb0 * 4 * 1024);
    uint4 *dst = reinterpret_cast<uint4 *>(a_lds);
#pragma unroll
    for (int i = (int)threadIdx.x; i < CH * 64; i += 256) dst[i] = src[i];
    const float4 *ssrc = reinterpret_cast<const float4 *>(p.stats) + (size_t)sb0 * 4 * 8;
    for (int i = (int)threadIdx.x; i < CH * 8; i += 256) st_lds[i] = ssrc[i];
  }
  __syncthreads();
  const uint32_t m4 = opaque_u32(0x0F0F0F0Fu);
  float acc[2][2] = {};
#pragma unroll
  for (int b = 0; b < SB; ++b) {
    float dsv[2][4], dmv[2][4];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const float d = half_bits_to_f32(hd[gi][b].x & 0xFFFFu), dm = half_bits_to_f32(hd[gi][b].x >> 16);
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        uint32_t sv, mv;
        q4k_scale_min(hd[gi][b].y, hd[gi][b].z, hd[gi][b].w, 2 * cc + h, sv, mv);
        dsv[gi][cc] = d * (float)sv;
        dmv[gi][cc] = dm * (float)mv;
      }
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int c = 4 * b + cc;
      const i32x4_t A = *reinterpret_cast<const i32x4_t *>(a_lds + c * 1024 + j * 64 + 16 * g);
      const float4 st0 = st_lds[c * 8 + 2 * g], st1 = st_lds[c * 8 + 2 * g + 1];  // rows 2g, 2g+1
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const uint4 q = qw[gi][b][cc];
        const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
        i32x4_t B;
#pragma unroll
        for (int t = 0; t < 4; ++t) B[t] = (int)((h ? w4[t] >> 4 : w4[t]) & m4);
        const i32x4_t C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, i32x4_t{0, 0, 0, 0}, 0, 0, 0);
        const float s0 = (float)(C[0] + 256 * C[1]), s1 = (float)(C[2] + 256 * C[3]);  // exact: < 2^24
        acc[gi][0] = fmaf(dsv[gi][cc] * st0.x, s0, fmaf(-dmv[gi][cc], h ? st0.z : st0.y, acc[gi][0]));
        acc[gi][1] = fmaf(dsv[gi][cc] * st1.x, s1, fmaf(-dmv[gi][cc], h ? st1.z : st1.y, acc[gi][1]));
      }
    }
  }
  // add the two sub-block halves (lanes j and j^1), then rows 2g, 2g+1 out
#pragma unroll
  for (int gi = 0; gi < 2; ++gi)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[gi][t] += dpp<0xB1>(acc[gi][t]);
  if (h == 0) {
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      if (row[gi] >= M.n) continue;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int m = 2 * g + t;
        if (m >= p.m) continue;
        if (p.ksplit == 1)
          M.y[(size_t)m * M.n + row[gi]] = acc[gi][t];
        else
          p.part[((size_t)slice * 8 + m) * p.ntot + M.part_off + row[gi]] = acc[gi][t];
      }
    }
  }
}

// y_mat[m][n] = sum over slices of the partials (slice order: deterministic).
__global__ __launch_bounds__(256) void k_mb_reduce(MbArgs p) {
  const size_t total = (size_t)p.m * p.ntot;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const int m = (int)(i / p.ntot), col = (int)(i % p.ntot);
    float s = 0.f;
    for (int sl = 0; sl < p.ksplit; ++sl) s += p.part[((size_t)sl * 8 + m) * p.ntot + col];
    int mi = 0;
    while (mi + 1 < p.nmat && col >= p.mat[mi + 1].part_off) ++mi;
    const MbMat &M = p.mat[mi];
    M.y[(size_t)m * M.n + (col - M.part_off)] = s;
  }
}

}  // namespace

size_t mb_stage_bytes(int k) { return (size_t)(k / 64) * 8 * (128 + 16); }

// Super-blocks per K slice: two where they divide the row, else one.
static int mb_slice_sb(int k) { return (k / 256) % 2 == 0 ? 2 : 1; }

int mb_ksplit(int n_total, int k) {
  (void)n_total;
  return (k / 256) / mb_slice_sb(k);
}

size_t mb_part_bytes(int n_total, int k) {
  const int ks = mb_ksplit(n_total, k);
  return ks > 1 ? (size_t)ks * 8 * n_total * 4 : 0;
}

hipError_t launch_mb_stage(const float *x, int m, int k, void *stage, hipStream_t s) {
  int8_t *dig = static_cast<int8_t *>(stage);
  float *stats = mb_stats(stage, k);
  hipLaunchKernelGGL(k_mb_stage, dim3((k / 64 + 15) / 16, 8), dim3(256), 0, s, x, m, k, dig, stats);
  return hipGetLastError();
}

hipError_t launch_q4k_gemv_mb(const MbMat *mats, int nmat, int m, int k, const void *stage, float *part,
                              hipStream_t s, RowsIn *views) {
  MbArgs p{};
  p.nmat = nmat;
  int ntot = 0, blocks = 0;
  for (int i = 0; i < nmat; ++i) {
    p.mat[i] = mats[i];
    p.mat[i].row_blocks = (mats[i].n + 63) / 64;
    p.mat[i].part_off = ntot;
    ntot += mats[i].n;
    blocks += p.mat[i].row_blocks;
  }
  p.dig = static_cast<const int8_t *>(stage);
  p.stats = reinterpret_cast<const float *>(p.dig + (size_t)(k / 64) * 8 * 128);
  p.m = m;
  p.k = k;
  p.ntot = ntot;
  p.ksplit = mb_ksplit(ntot, k);
  p.part = part;
  if (mb_slice_sb(k) == 2)
    hipLaunchKernelGGL(k_q4k_gemv_mb<2>, dim3(blocks, p.ksplit), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(k_q4k_gemv_mb<1>, dim3(blocks, p.ksplit), dim3(256), 0, s, p);
  hipError_t e = hipGetLastError();
  if (views)
    for (int i = 0; i < nmat; ++i)
      views[i] = p.ksplit == 1 ? rows_plain(mats[i].y, mats[i].n)
                               : RowsIn{part, p.ksplit, (size_t)8 * ntot, ntot, p.mat[i].part_off};
  if (e != hipSuccess || p.ksplit == 1 || views) return e;
  const size_t total = (size_t)m * ntot;
  hipLaunchKernelGGL(k_mb_reduce, dim3((unsigned)std::min<size_t>((total + 255) / 256, 2048)), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace rt
