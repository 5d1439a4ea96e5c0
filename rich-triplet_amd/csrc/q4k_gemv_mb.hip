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
// Product (v_mfma_i32_16x16x32_i8, one MFMA per 32-element sub-block).  Lane
// l of a wave (j = l%16, g = l/16) holds k-slots 8g..8g+7 of A row j =
// (activation row m = j/2, digit d = j%2) and of B column j = weight row j of
// the wave's 16.  A sub-block's 32 codes are the low (even sub-block) or high
// (odd) nibbles of its chunk's 32 bytes, so one 8-byte load of bytes
// 8g..8g+7 feeds both sub-blocks of a chunk and no B lane is padding:
//   C[(m,d)][j] = sum over the sub-block of q * x_d     (exact int32)
// Lane (j, g) receives rows 4g..4g+3 of C: rows m = 2g, 2g+1, both digits,
// for weight row j, and applies the scales:
//   acc[m] += d*sv*delta_m * (256 C1 + C0) - dmin*mv * sum_m(sub-block)
// A workgroup is four waves of 16 rows (64 rows) over a slice of KS
// super-blocks; its activation slice is copied to LDS once.  With several
// slices each writes partial sums that k_mb_reduce (or the consumer) adds in
// slice order.  Many small workgroups at full occupancy overlap one
// workgroup's arithmetic with the others' loads.
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

typedef long i64_t;

template <int KS>
__global__ __launch_bounds__(256) void k_q4k_gemv_mb(MbArgs p) {
  constexpr int CH = 4 * KS;            // chunks in the slice
  constexpr int NA = CH * 64 + CH * 8;  // 16-byte pieces of digits + stats
  constexpr int AV = (NA + 255) / 256;
  __shared__ __attribute__((aligned(16))) int8_t a_lds[CH * 1024];
  __shared__ __attribute__((aligned(16))) float4 st_lds[CH * 8];
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int j = lane & 15, g = lane >> 4;
  int rb = (int)blockIdx.x;
  const MbMat M = mb_pick(p, rb);
  const int nb = p.k / 256, slice = (int)blockIdx.y;
  const int sb0 = slice * KS;  // the launcher makes KS divide nb
  // The slice's activations first (clamped, unconditional loads), so their
  // wait leaves every weight load in flight.
  uint4 av[AV];
  {
    const uint4 *dsrc = reinterpret_cast<const uint4 *>(p.dig + (size_t)sb0 * 4 * 1024);
    const uint4 *ssrc = reinterpret_cast<const uint4 *>(p.stats) + (size_t)sb0 * 4 * 8;
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int idx = min((int)threadIdx.x + 256 * i, NA - 1);
      av[i] = idx < CH * 64 ? dsrc[idx] : ssrc[idx - CH * 64];
    }
  }
  const int row = rb * 64 + wave * 16 + j;
  const uint8_t *wp = M.w + (size_t)min(row, M.n - 1) * ((size_t)nb * kQ4KBlockBytes) + (size_t)sb0 * kQ4KBlockBytes;
  uint4 hd[KS];
  uint2 qw[KS][4];
#pragma unroll
  for (int b = 0; b < KS; ++b) {
    hd[b] = *reinterpret_cast<const uint4 *>(wp + b * kQ4KBlockBytes);
#pragma unroll
    for (int c = 0; c < 4; ++c) qw[b][c] = *reinterpret_cast<const uint2 *>(wp + b * kQ4KBlockBytes + 16 + 32 * c + 8 * g);
  }
#pragma unroll
  for (int i = 0; i < AV; ++i) {
    const int idx = (int)threadIdx.x + 256 * i;
    if (idx < CH * 64) reinterpret_cast<uint4 *>(a_lds)[idx] = av[i];
    else if (idx < NA) reinterpret_cast<uint4 *>(st_lds)[idx - CH * 64] = av[i];
  }
  __syncthreads();
  const uint32_t m4 = opaque_u32(0x0F0F0F0Fu);
  float acc[2] = {};
#pragma unroll
  for (int b = 0; b < KS; ++b) {
    const float d = half_bits_to_f32(hd[b].x & 0xFFFFu), dm = half_bits_to_f32(hd[b].x >> 16);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int ci = 4 * b + c;
      const float4 st0 = st_lds[ci * 8 + 2 * g], st1 = st_lds[ci * 8 + 2 * g + 1];  // rows 2g, 2g+1
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const i64_t A = *reinterpret_cast<const i64_t *>(a_lds + ci * 1024 + j * 64 + 32 * h + 8 * g);
        uint32_t sv, mv;
        q4k_scale_min(hd[b].y, hd[b].z, hd[b].w, 2 * c + h, sv, mv);
        const float sc = d * (float)sv, mn = dm * (float)mv;
        const uint32_t b0 = (h ? qw[b][c].x >> 4 : qw[b][c].x) & m4, b1 = (h ? qw[b][c].y >> 4 : qw[b][c].y) & m4;
        const i64_t B = (i64_t)(((uint64_t)b1 << 32) | b0);
        const i32x4_t C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, i32x4_t{0, 0, 0, 0}, 0, 0, 0);
        const float s0 = (float)(C[0] + 256 * C[1]), s1 = (float)(C[2] + 256 * C[3]);  // exact: < 2^24
        acc[0] = fmaf(sc * st0.x, s0, fmaf(-mn, h ? st0.z : st0.y, acc[0]));
        acc[1] = fmaf(sc * st1.x, s1, fmaf(-mn, h ? st1.z : st1.y, acc[1]));
        // Keeps each sub-block's scaling beside its MFMA: sunk into the store
        // branch, it holds every MFMA result live and halves the occupancy.
        asm volatile("" : "+v"(acc[0]), "+v"(acc[1]));
      }
    }
  }
  if (row >= M.n) return;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int m = 2 * g + t;
    if (m >= p.m) continue;
    if (p.ksplit == 1)
      M.y[(size_t)m * M.n + row] = acc[t];
    else
      p.part[((size_t)slice * 8 + m) * p.ntot + M.part_off + row] = acc[t];
  }
}

// y_mat[m][n] = sum over slices of the partials (slice order: deterministic).
__global__ __launch_bounds__(256) void k_mb_reduce(MbArgs p) {
  const size_t total = (size_t)p.m * p.ntot;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const int m = (int)(i / p.ntot), col = (int)(i % p.ntot);
    float s = 0.f;
    for (int sl = 0; sl < p.ksplit; ++sl) s += p.part[((size_t)sl * 8 + m) * p.ntot + col];
    const bool in1 = p.nmat > 1 && col >= p.mat[1].part_off, in2 = p.nmat > 2 && col >= p.mat[2].part_off;
    const MbMat M = in2 ? p.mat[2] : (in1 ? p.mat[1] : p.mat[0]);
    M.y[(size_t)m * M.n + (col - M.part_off)] = s;
  }
}

}  // namespace

size_t mb_stage_bytes(int k) { return (size_t)(k / 64) * 8 * (128 + 16); }

// Super-blocks per K slice.  One for rows up to 8192: the smallest
// workgroups overlap best, and the partial sums they leave (32 bytes per row
// and super-block, against 144 of weights) cost less than two-block slices'
// longer workgroups.  Four for longer rows (the FFN down projection), whose
// 40 one-block slices would leave its consumer, a row norm on one workgroup
// per row, too many partials to add.
static int mb_slice_sb(int k) { return k >= 8192 && (k / 256) % 4 == 0 ? 4 : 1; }

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
  if (mb_slice_sb(k) == 4)
    hipLaunchKernelGGL(k_q4k_gemv_mb<4>, dim3(blocks, p.ksplit), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(k_q4k_gemv_mb<1>, dim3(blocks, p.ksplit), dim3(256), 0, s, p);
  hipError_t e = hipGetLastError();
  if (views)
    for (int i = 0; i < nmat; ++i)
      views[i] = p.ksplit == 1 ? rows_plain(mats[i].y, mats[i].n)
                               : RowsIn{part, p.ksplit, (size_t)8 * ntot, ntot, p.mat[i].part_off};
  if (e != hipSuccess || p.ksplit == 1 || views) return e;
  return launch_mb_reduce(p, s);
}

// One matrix of many rows (an lm_head over the vocabulary): for K of 2 or 10
// super-blocks the whole row is one slice (no partial sums, no reduction;
// the rows alone give thousands of workgroups), other K take the split path.
static bool mb_head_whole_row(int k) { return k / 256 == 2 || k / 256 == 10; }

size_t mb_head_part_bytes(int n, int k) { return mb_head_whole_row(k) ? 0 : mb_part_bytes(n, k); }

hipError_t launch_q4k_gemv_mb_head(const uint8_t *w, float *y, int n, int m, int k, const void *stage, float *part,
                                   hipStream_t s) {
  if (!mb_head_whole_row(k)) {
    const MbMat mat{w, y, n, 0, 0};
    return launch_q4k_gemv_mb(&mat, 1, m, k, stage, part, s);
  }
  MbArgs p{};
  p.nmat = 1;
  p.mat[0] = MbMat{w, y, n, (n + 63) / 64, 0};
  p.dig = static_cast<const int8_t *>(stage);
  p.stats = reinterpret_cast<const float *>(p.dig + (size_t)(k / 64) * 8 * 128);
  p.m = m;
  p.k = k;
  p.ntot = n;
  p.ksplit = 1;
  if (k / 256 == 10)
    hipLaunchKernelGGL(k_q4k_gemv_mb<10>, dim3(p.mat[0].row_blocks, 1), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(k_q4k_gemv_mb<2>, dim3(p.mat[0].row_blocks, 1), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_mb_reduce(const MbArgs &p, hipStream_t s) {
  const size_t total = (size_t)p.m * p.ntot;
  hipLaunchKernelGGL(k_mb_reduce, dim3((unsigned)std::min<size_t>((total + 255) / 256, 2048)), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace rt
