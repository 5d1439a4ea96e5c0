// kquant_mb.hip -- batched GEMVs, C[m][n] = sum_k A[m][k] W[n][k] for M <= 8
// activation rows, for the projection formats other than Q4_K: Q8_0, Q6_K
// (both kept packed, planar layout of kquant.hip) and BF16.
//
// Replaces gemv_bf16_t_batch (metal_decode.rs:527-558), the GEMV that
// encode_layer_batch (2184-2240) sends every BF16 projection of the
// speculative verify batch to, and the same batch for the Q6_K / Q8_0 weights
// the reference widens to BF16 at load (transformer4.rs:1233-1242): one pass
// over the weights for all M rows.
//
// Work split (as the Q4_K kernel, q4k_gemv_mb.hip): a workgroup is four waves
// of 16 weight rows over one K slice; lane l (j = l%16, g = l/16) holds
// k-slots 8g..8g+7 of A row j and of B column j (weight row j of the wave's
// 16), and receives C rows 4g..4g+3.  Slices leave partial sums
// [slice][8][ntot] that the consumer (or k_mb_reduce) adds in slice order.
//
// Q8_0 and Q6_K read the activations as the staged 16-bit digits of the Q4_K
// kernel (X = 256*x1 + x0 per 64-element chunk, scale delta per chunk and row;
// A row j = token j/2, digit j%2) and multiply the signed weight codes on
// v_mfma_i32_16x16x32_i8 in exact integer arithmetic:
//   Q8_0  one MFMA per 32-element block, codes q in -128..127 as they are:
//         acc += d * delta * (C_x0 + 256 C_x1)
//   Q6_K  per 32-element window two MFMAs, each with the codes q - 32 of one
//         16-element sub-block (the other half of B zero), so each sub-block
//         keeps its own int8 scale sc:
//         acc += d * delta * (sc_lo * S_lo + sc_hi * S_hi),  S = C_x0 + 256 C_x1
//         (|S| < 16 * 32767 * 32 < 2^24: exact in f32)
// BF16 reads the f32 rows themselves: each workgroup splits its slice into
// bf16 parts hi = bf16(x), lo = bf16(x - hi) in LDS (A row j = token j/2,
// part j%2) and multiplies the weights as they are on
// v_mfma_f32_16x16x32_bf16; y = C_hi + C_lo (x to about 2^-17).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/rt_hip.h"
#include "kquant_layout.hpp"
#include "q4k_gemv_mb.hpp"
#include "rt_device.hpp"

namespace rt {
namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef long i64_t;


// The slice's staged digits and statistics (chunks c0 .. c0+CH-1) into LDS;
// the loads are issued by load_stage before the weight loads, the stores by
// store_stage after them.
template <int CH>
struct StageSlice {
  static constexpr int NA = CH * 64 + CH * 8;  // 16-byte pieces: digits, then stats
  static constexpr int AV = (NA + 255) / 256;
  uint4 av[AV];
  __device__ __forceinline__ void load(const MbArgs &p, int c0) {
    const uint4 *dsrc = reinterpret_cast<const uint4 *>(p.dig + (size_t)c0 * 1024);
    const uint4 *ssrc = reinterpret_cast<const uint4 *>(p.stats) + (size_t)c0 * 8;
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int idx = min((int)threadIdx.x + 256 * i, NA - 1);
      av[i] = idx < CH * 64 ? dsrc[idx] : ssrc[idx - CH * 64];
    }
  }
  __device__ __forceinline__ void store(int8_t *a_lds, float4 *st_lds) const {
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int idx = (int)threadIdx.x + 256 * i;
      if (idx < CH * 64) reinterpret_cast<uint4 *>(a_lds)[idx] = av[i];
      else if (idx < NA) reinterpret_cast<uint4 *>(st_lds)[idx - CH * 64] = av[i];
    }
  }
};

__device__ __forceinline__ void mb_store(const MbArgs &p, const MbMat &M, int row, int slice, int g, const float *acc) {
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

// ---------------------------------------------------------------------------
// Q8_0: slice of CH chunks = 2*CH blocks of 32.
// ---------------------------------------------------------------------------
template <int CH>
__global__ __launch_bounds__(256) void k_q8_0_gemv_mb(MbArgs p) {
  __shared__ __attribute__((aligned(16))) int8_t a_lds[CH * 1024];
  __shared__ __attribute__((aligned(16))) float4 st_lds[CH * 8];
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int j = lane & 15, g = lane >> 4;
  int rb = (int)blockIdx.x;
  const MbMat M = mb_pick(p, rb);
  const int slice = (int)blockIdx.y, c0 = slice * CH;
  StageSlice<CH> sa;
  sa.load(p, c0);
  const int row = rb * 64 + wave * 16 + j;
  const size_t r = (size_t)min(row, M.n - 1);
  const uint16_t *D = reinterpret_cast<const uint16_t *>(M.w + (size_t)M.n * p.k);
  const uint8_t *qp = M.w + r * p.k + (size_t)c0 * 64 + 8 * g;
  uint2 qv[2 * CH];
  uint32_t dv[2 * CH];
#pragma unroll
  for (int b = 0; b < 2 * CH; ++b) {
    qv[b] = *reinterpret_cast<const uint2 *>(qp + 32 * b);
    dv[b] = D[r * (p.k / kQ8Block) + 2 * c0 + b];
  }
  sa.store(a_lds, st_lds);
  __syncthreads();
  float acc[2] = {0.f, 0.f};
#pragma unroll
  for (int b = 0; b < 2 * CH; ++b) {
    const int ci = b >> 1, h = b & 1;
    const i64_t A = *reinterpret_cast<const i64_t *>(a_lds + ci * 1024 + j * 64 + 32 * h + 8 * g);
    const i64_t B = (i64_t)(((uint64_t)qv[b].y << 32) | qv[b].x);
    const i32x4_t C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, i32x4_t{0, 0, 0, 0}, 0, 0, 0);
    const float d = half_bits_to_f32(dv[b]);
    const float4 st0 = st_lds[ci * 8 + 2 * g], st1 = st_lds[ci * 8 + 2 * g + 1];  // tokens 2g, 2g+1
    acc[0] = fmaf(d * st0.x, (float)(C[0] + 256 * C[1]), acc[0]);
    acc[1] = fmaf(d * st1.x, (float)(C[2] + 256 * C[3]), acc[1]);
    asm volatile("" : "+v"(acc[0]), "+v"(acc[1]));  // scaling beside its MFMA (see q4k_gemv_mb.hip)
  }
  mb_store(p, M, row, slice, g, acc);
}

// ---------------------------------------------------------------------------
// Q6_K: slice of SB super-blocks.  Window w (elements 32w..32w+31 of a
// super-block) is half h = w%2 of chunk w/2; its codes are the low (w%4 < 2)
// or high nibbles of ql[64*(w/4) + 32*(w%2) + l] with bit pair w%4 of
// qh[32*(w/4) + l], l = 0..31; lane g takes l = 8g..8g+7, whose sub-block
// is the window's first (g < 2) or second (scale sc[8*(w/4) + 2*(w%4) + {0, 1}]).
// ---------------------------------------------------------------------------
template <int SB>
__global__ __launch_bounds__(256) void k_q6k_gemv_mb(MbArgs p) {
  constexpr int CH = 4 * SB;
  __shared__ __attribute__((aligned(16))) int8_t a_lds[CH * 1024];
  __shared__ __attribute__((aligned(16))) float4 st_lds[CH * 8];
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int j = lane & 15, g = lane >> 4;
  int rb = (int)blockIdx.x;
  const MbMat M = mb_pick(p, rb);
  const int nb = p.k / 256, slice = (int)blockIdx.y, sb0 = slice * SB;
  StageSlice<CH> sa;
  sa.load(p, sb0 * 4);
  const int row = rb * 64 + wave * 16 + j;
  const Q6KPlanes P = q6k_planes(M.w, (size_t)M.n * nb);
  const size_t blk0 = (size_t)min(row, M.n - 1) * nb + sb0;
  uint2 ql[SB][2][2], qh[SB][2];
  uint4 sc[SB];
  uint32_t dv[SB];
#pragma unroll
  for (int b = 0; b < SB; ++b) {
    const size_t blk = blk0 + b;
#pragma unroll
    for (int ip = 0; ip < 2; ++ip) {
#pragma unroll
      for (int o = 0; o < 2; ++o) ql[b][ip][o] = *reinterpret_cast<const uint2 *>(P.ql + blk * 128 + 64 * ip + 32 * o + 8 * g);
      qh[b][ip] = *reinterpret_cast<const uint2 *>(P.qh + blk * 64 + 32 * ip + 8 * g);
    }
    sc[b] = *reinterpret_cast<const uint4 *>(P.sc + blk * 16);
    dv[b] = P.d[blk];
  }
  sa.store(a_lds, st_lds);
  __syncthreads();
  const uint32_t m4 = opaque_u32(0x0F0F0F0Fu), m2 = opaque_u32(0x03030303u);
  const uint32_t set = opaque_u32(0x80808080u), off = opaque_u32(0x20202020u);
  // q - 32 per byte for codes q in 0..63: ((q | 0x80) - 0x20) ^ 0x80, no borrow across bytes
  auto code = [&](uint32_t lw, uint32_t hw, int w) -> uint32_t {
    const int qq = w & 3;
    const uint32_t q = ((qq < 2 ? lw : lw >> 4) & m4) | (((hw >> (2 * qq)) & m2) << 4);
    return ((q | set) - off) ^ set;
  };
  float acc[2] = {0.f, 0.f};
#pragma unroll
  for (int b = 0; b < SB; ++b) {
    const float d = half_bits_to_f32(dv[b]);
    const uint32_t scw[4] = {sc[b].x, sc[b].y, sc[b].z, sc[b].w};
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const int ip = w >> 2, ci = 4 * b + (w >> 1), h = w & 1;
      const uint2 lw = ql[b][ip][w & 1], hw = qh[b][ip];
      const uint32_t c0 = code(lw.x, hw.x, w), c1 = code(lw.y, hw.y, w);
      const i64_t B = (i64_t)(((uint64_t)c1 << 32) | c0);
      const i64_t Blo = g < 2 ? B : 0, Bhi = g < 2 ? 0 : B;
      const i64_t A = *reinterpret_cast<const i64_t *>(a_lds + ci * 1024 + j * 64 + 32 * h + 8 * g);
      const i32x4_t Cl = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, Blo, i32x4_t{0, 0, 0, 0}, 0, 0, 0);
      const i32x4_t Ch = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, Bhi, i32x4_t{0, 0, 0, 0}, 0, 0, 0);
      const int si = 8 * ip + 2 * (w & 3);  // scale of the window's first sub-block; si + 1 the second
      const float sl = (float)(int)__builtin_amdgcn_sbfe(scw[si >> 2], 8 * (si & 3), 8);
      const float sh = (float)(int)__builtin_amdgcn_sbfe(scw[(si + 1) >> 2], 8 * ((si + 1) & 3), 8);
      const float4 st0 = st_lds[ci * 8 + 2 * g], st1 = st_lds[ci * 8 + 2 * g + 1];
      const float t0 = fmaf(sh, (float)(Ch[0] + 256 * Ch[1]), sl * (float)(Cl[0] + 256 * Cl[1]));
      const float t1 = fmaf(sh, (float)(Ch[2] + 256 * Ch[3]), sl * (float)(Cl[2] + 256 * Cl[3]));
      acc[0] = fmaf(d * st0.x, t0, acc[0]);
      acc[1] = fmaf(d * st1.x, t1, acc[1]);
      asm volatile("" : "+v"(acc[0]), "+v"(acc[1]));
    }
  }
  mb_store(p, M, row, slice, g, acc);
}

// ---------------------------------------------------------------------------
// BF16: slice of CH chunks; x rows (f32, row stride k) split into bf16 hi/lo
// in LDS as [window][16 A rows][32], the 8-element groups XOR-swizzled by
// (row >> 2) so a 16-lane read of one group column hits distinct banks.
// ---------------------------------------------------------------------------
template <int CH>
__global__ __launch_bounds__(256) void k_bf16_gemv_mb(MbArgs p, const float *__restrict__ x) {
  constexpr int NW = 2 * CH;  // 32-element windows in the slice
  __shared__ __attribute__((aligned(16))) uint16_t xa[NW * 16 * 32];
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int j = lane & 15, g = lane >> 4;
  int rb = (int)blockIdx.x;
  const MbMat M = mb_pick(p, rb);
  const int slice = (int)blockIdx.y, e0 = slice * CH * 64;
  // x: 8 rows x 64*CH elements, one float4 per thread per step
  constexpr int XV = (8 * CH * 16 + 255) / 256;
  float4 xv[XV];
#pragma unroll
  for (int i = 0; i < XV; ++i) {
    const int idx = (int)threadIdx.x + 256 * i, m = idx / (CH * 16), c4 = idx % (CH * 16);
    xv[i] = (idx < 8 * CH * 16 && m < p.m) ? *reinterpret_cast<const float4 *>(x + (size_t)m * p.k + e0 + 4 * c4)
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int row = rb * 64 + wave * 16 + j;
  const uint16_t *wp = reinterpret_cast<const uint16_t *>(M.w) + (size_t)min(row, M.n - 1) * p.k + e0 + 8 * g;
  uint4 wv[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) wv[w] = *reinterpret_cast<const uint4 *>(wp + 32 * w);
#pragma unroll
  for (int i = 0; i < XV; ++i) {
    const int idx = (int)threadIdx.x + 256 * i;
    if (idx < 8 * CH * 16) {
      const int m = idx / (CH * 16), e = 4 * (idx % (CH * 16));  // element e..e+3 of the slice
      const int w = e >> 5, k = e & 31, grp = k >> 3;
      const float v[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) {
        const int ar = 2 * m + pt;
        uint16_t *dst = xa + (w * 16 + ar) * 32 + 8 * (grp ^ ((ar >> 2) & 3)) + (k & 7);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint16_t hi = f32_to_bf16_bits(v[q]);
          dst[q] = pt ? f32_to_bf16_bits(v[q] - bf16_lo((uint32_t)hi)) : hi;
        }
      }
    }
  }
  __syncthreads();
  const int aoff = j * 32 + 8 * (g ^ ((j >> 2) & 3));
  f32x4_t C = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const uint4 af = *reinterpret_cast<const uint4 *>(xa + w * 512 + aoff);
    C = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af), __builtin_bit_cast(bf16x8_t, wv[w]),
                                                C, 0, 0, 0);
  }
  const float acc[2] = {C[0] + C[1], C[2] + C[3]};
  mb_store(p, M, row, slice, g, acc);
}

// Chunks per K slice: the Q4_K kernel's slices (one super-block, four for
// rows of 8192 and more) where k is a whole number of super-blocks, so the
// consumers see the same slice counts; otherwise (Q8_0 and BF16 rows of
// 64-element chunks) the largest of 4, 2, 1 chunks that divides the row.
int slice_chunks(int k) {
  if (k % 256 == 0) return (k >= 8192 && (k / 256) % 4 == 0) ? 16 : 4;
  const int nc = k / 64;
  return nc % 4 == 0 ? 4 : nc % 2 == 0 ? 2 : 1;
}

template <int CH>
void launch_q8_ch(const MbArgs &p, int blocks, hipStream_t s) {
  hipLaunchKernelGGL(k_q8_0_gemv_mb<CH>, dim3(blocks, p.ksplit), dim3(256), 0, s, p);
}
template <int CH>
void launch_bf16_ch(const MbArgs &p, int blocks, const float *x, hipStream_t s) {
  hipLaunchKernelGGL(k_bf16_gemv_mb<CH>, dim3(blocks, p.ksplit), dim3(256), 0, s, p, x);
}

}  // namespace

bool kquant_mb_supported(int fmt, int k) {
  if (k <= 0 || k % 64 != 0) return false;
  switch (fmt) {
    case RT_LINEAR_Q6K: return k % 256 == 0;
    case RT_LINEAR_Q8_0:
    case RT_LINEAR_BF16: return true;
    default: return false;
  }
}

int kquant_mb_ksplit(int k) { return (k / 64) / slice_chunks(k); }

size_t kquant_mb_part_bytes(int n_total, int k) {
  const int ks = kquant_mb_ksplit(k);
  return ks > 1 ? (size_t)ks * 8 * n_total * 4 : 0;
}

hipError_t launch_kquant_gemv_mb(int fmt, const MbMat *mats, int nmat, int m, int k, const void *stage,
                                 const float *x, float *part, hipStream_t s, RowsIn *views) {
  if (!kquant_mb_supported(fmt, k) || nmat < 1 || nmat > 3 || m < 1 || m > kMbMaxRows) return hipErrorInvalidValue;
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
  p.stats = stage ? mb_stats(const_cast<void *>(stage), k) : nullptr;
  p.m = m;
  p.k = k;
  p.ntot = ntot;
  p.ksplit = kquant_mb_ksplit(k);
  p.part = part;
  const int ch = slice_chunks(k);
  switch (fmt) {
    case RT_LINEAR_Q8_0:
      if (ch == 16) launch_q8_ch<16>(p, blocks, s);
      else if (ch == 4) launch_q8_ch<4>(p, blocks, s);
      else if (ch == 2) launch_q8_ch<2>(p, blocks, s);
      else launch_q8_ch<1>(p, blocks, s);
      break;
    case RT_LINEAR_Q6K:
      if (ch == 16) hipLaunchKernelGGL(k_q6k_gemv_mb<4>, dim3(blocks, p.ksplit), dim3(256), 0, s, p);
      else hipLaunchKernelGGL(k_q6k_gemv_mb<1>, dim3(blocks, p.ksplit), dim3(256), 0, s, p);
      break;
    default:
      if (ch == 16) launch_bf16_ch<16>(p, blocks, x, s);
      else if (ch == 4) launch_bf16_ch<4>(p, blocks, x, s);
      else if (ch == 2) launch_bf16_ch<2>(p, blocks, x, s);
      else launch_bf16_ch<1>(p, blocks, x, s);
      break;
  }
  hipError_t e = hipGetLastError();
  if (views)
    for (int i = 0; i < nmat; ++i)
      views[i] = p.ksplit == 1 ? rows_plain(mats[i].y, mats[i].n)
                               : RowsIn{part, p.ksplit, (size_t)8 * ntot, ntot, p.mat[i].part_off};
  if (e != hipSuccess || p.ksplit == 1 || views) return e;
  return launch_mb_reduce(p, s);
}

}  // namespace rt
