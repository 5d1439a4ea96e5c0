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
// slice of K (whole super-blocks); slices beyond one write partial sums that
// k_mb_reduce adds in slice order.
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
  const int row = (int)blockIdx.y;  // 0..7
  const int c = min(ci, nchunk - 1);
  const float4 v = row < m ? *reinterpret_cast<const float4 *>(x + (size_t)row * k + 64 * c + 4 * q)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
  const uint32_t ax = f32_bits(v.x) & 0x7FFFFFFFu, ay = f32_bits(v.y) & 0x7FFFFFFFu;
  const uint32_t az = f32_bits(v.z) & 0x7FFFFFFFu, aw = f32_bits(v.w) & 0x7FFFFFFFu;
  uint32_t mb = max(max(ax, ay), max(az, aw));
  mb = max(mb, dpp_u32<0xB1>(mb));
  mb = max(mb, dpp_u32<0x4E>(mb));
  mb = max(mb, dpp_u32<0x141>(mb));
  mb = max(mb, dpp_u32<0x140>(mb));
  // max < 2^e, e = biased exponent - 126; s = 32639 * 2^-e stays a normal
  // float for e >= -111 (smaller chunks lose digits instead of overflowing)
  const int e = max((int)(mb >> 23) - 126, -111);
  const float s = bits_f32(f32_bits(32639.0f) - ((uint32_t)e << 23));
  const float delta = bits_f32(f32_bits(1.0f / 32639.0f) + ((uint32_t)e << 23));
  const float magic = 12583040.0f;  // 1.5*2^23 + 128
  const uint32_t b0 = f32_bits(fmaf(v.x, s, magic)), b1 = f32_bits(fmaf(v.y, s, magic));
  const uint32_t b2 = f32_bits(fmaf(v.z, s, magic)), b3 = f32_bits(fmaf(v.w, s, magic));
  const uint32_t p01 = __builtin_amdgcn_perm(b1, b0, 0x05010400u);  // b0.0 b1.0 b0.1 b1.1
  const uint32_t p23 = __builtin_amdgcn_perm(b3, b2, 0x05010400u);
  const uint32_t d0 = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;  // (X+128 mod 256) - 128
  const uint32_t d1 = __builtin_amdgcn_perm(p23, p01, 0x07060302u);                // floor((X+128)/256)
  float sum = (v.x + v.y) + (v.z + v.w);
  sum += dpp<0xB1>(sum);
  sum += dpp<0x4E>(sum);
  sum += dpp<0x141>(sum);  // 8 lanes = one 32-element sub-block
  if (ci < nchunk) {
    int8_t *base = dig + ((size_t)c * 8 + row) * 128;
    *reinterpret_cast<uint32_t *>(base + 4 * q) = d0;
    *reinterpret_cast<uint32_t *>(base + 64 + 4 * q) = d1;
    float *st = stats + ((size_t)c * 8 + row) * 4;
    if (q == 0) {
      st[0] = delta;
      st[1] = sum;
      st[3] = 0.f;
    }
    if (q == 8) st[2] = sum;
  }
}

template <int RPW>
__global__ __launch_bounds__(256) void k_q4k_gemv_mb(MbArgs p) {
  constexpr int NG = RPW / 8;  // B operands (8-row groups) per wave
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int j = lane & 15, g = lane >> 4, r = j >> 1, h = j & 1;
  // matrix of this row block
  int rb = (int)blockIdx.x, mi = 0;
  while (mi + 1 < p.nmat && rb >= p.mat[mi].row_blocks) rb -= p.mat[mi++].row_blocks;
  const MbMat &M = p.mat[mi];
  const int nb = p.k / 256, slice = (int)blockIdx.y;
  const int sb0 = slice * nb / p.ksplit, sb1 = (slice + 1) * nb / p.ksplit;
  const size_t row_bytes = (size_t)nb * kQ4KBlockBytes;
  int row[NG];
  const uint8_t *wrow[NG];
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    row[gi] = rb * 4 * RPW + wave * RPW + 8 * gi + r;
    wrow[gi] = M.w + (size_t)min(row[gi], M.n - 1) * row_bytes;  // rows past n: masked at the store
  }
  const bool carries = (g >> 1) == h;  // this lane's k-slots lie in sub-block half h
  const int qoff = 16 * (g & 1);
  const uint32_t m4 = opaque_u32(0x0F0F0F0Fu);
  float acc[NG][2] = {};
  const int8_t *dig = p.dig + j * 64 + 16 * g;  // row m = j/2, digit j%2
  const float4 *stats = reinterpret_cast<const float4 *>(p.stats) + 2 * g;

#pragma unroll 1
  for (int sb = sb0; sb < sb1; ++sb) {
    uint4 hd[NG];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) hd[gi] = *reinterpret_cast<const uint4 *>(wrow[gi] + (size_t)sb * kQ4KBlockBytes);
    float dsv[NG][4], dmv[NG][4];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      const float d = half_bits_to_f32(hd[gi].x & 0xFFFFu), dm = half_bits_to_f32(hd[gi].x >> 16);
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        uint32_t sv, mv;
        q4k_scale_min(hd[gi].y, hd[gi].z, hd[gi].w, 2 * cc + h, sv, mv);
        dsv[gi][cc] = d * (float)sv;
        dmv[gi][cc] = dm * (float)mv;
      }
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int c = sb * 4 + cc;
      const i32x4_t A = *reinterpret_cast<const i32x4_t *>(dig + (size_t)c * 1024);
      const float4 st0 = stats[(size_t)c * 8], st1 = stats[(size_t)c * 8 + 1];  // rows 2g, 2g+1
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        const uint4 qw = *reinterpret_cast<const uint4 *>(wrow[gi] + (size_t)sb * kQ4KBlockBytes + 16 + 32 * cc + qoff);
        const uint32_t w4[4] = {qw.x, qw.y, qw.z, qw.w};
        i32x4_t B;
#pragma unroll
        for (int t = 0; t < 4; ++t) B[t] = carries ? (int)((h ? w4[t] >> 4 : w4[t]) & m4) : 0;
        const i32x4_t C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, i32x4_t{0, 0, 0, 0}, 0, 0, 0);
        const float s0 = (float)(C[0] + 256 * C[1]), s1 = (float)(C[2] + 256 * C[3]);  // exact: < 2^24
        acc[gi][0] = fmaf(dsv[gi][cc] * st0.x, s0, fmaf(-dmv[gi][cc], h ? st0.z : st0.y, acc[gi][0]));
        acc[gi][1] = fmaf(dsv[gi][cc] * st1.x, s1, fmaf(-dmv[gi][cc], h ? st1.z : st1.y, acc[gi][1]));
      }
    }
  }
  // add the two sub-block halves (lanes j and j^1), then rows 2g, 2g+1 out
#pragma unroll
  for (int gi = 0; gi < NG; ++gi)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[gi][t] += dpp<0xB1>(acc[gi][t]);
  if (h == 0) {
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
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

int mb_ksplit(int n_total, int k) {
  // enough workgroups of 64 rows to cover the CUs, slices of whole super-blocks
  const int blocks = (n_total + 63) / 64, nb = k / 256;
  int ks = 1;
  while (blocks * ks < 256 && ks * 2 <= nb) ks *= 2;
  return ks;
}

size_t mb_part_bytes(int n_total, int k) {
  const int ks = mb_ksplit(n_total, k);
  return ks > 1 ? (size_t)ks * 8 * n_total * 4 : 0;
}

hipError_t launch_mb_stage(const float *x, int m, int k, void *stage, hipStream_t s) {
  int8_t *dig = static_cast<int8_t *>(stage);
  float *stats = reinterpret_cast<float *>(dig + (size_t)(k / 64) * 8 * 128);
  hipLaunchKernelGGL(k_mb_stage, dim3((k / 64 + 15) / 16, 8), dim3(256), 0, s, x, m, k, dig, stats);
  return hipGetLastError();
}

hipError_t launch_q4k_gemv_mb(const MbMat *mats, int nmat, int m, int k, const void *stage, float *part,
                              hipStream_t s) {
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
  hipLaunchKernelGGL(k_q4k_gemv_mb<16>, dim3(blocks, p.ksplit), dim3(256), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ksplit == 1) return e;
  const size_t total = (size_t)m * ntot;
  hipLaunchKernelGGL(k_mb_reduce, dim3((unsigned)std::min<size_t>((total + 255) / 256, 2048)), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace rt
