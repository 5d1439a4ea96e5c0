// q4k_gemm.hip -- Q4_K GEMM on gfx950 matrix cores:  C[m][n] = sum_k A[m][k] * W[n][k].
//
// Replaces Q4KMat::matmul_q4k_t / matmul_q4k_t_exact (autograd2.rs:1437-1625,
// dequantise a band of rows to f32 and sgemm it) and the FLUX GPU path
// flux_dequant_q4k + flux_gemm_bt (metal_flux.rs:108-190, dequantise the whole
// weight to bfloat scratch, then a 64x64 simdgroup GEMM).  Here the weight
// stays packed in HBM (144-byte super-blocks): the packed bytes of the chunk
// about to be multiplied reach each lane (through LDS in the eight-wave
// kernel, straight into VGPRs in the half-block kernel) and every lane
// dequantises its own column into registers.
//
// Arithmetic: v_mfma_f32_32x32x16_f16, f32 accumulation.
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
// to f16: 1.5 VALU operations per weight.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "gemma3_math.hpp"
#include "mfma_common.hpp"
#include "q4k_gemm_dev.hpp"
#include "rt_device.hpp"
#include "rt_kernels.hpp"

namespace rt {
namespace {


// ---------------------------------------------------------------------------
// Prep: A -> f16 with a per-row exponent; W row exponents from block headers.
// Workgroups [0, M) take one A row each, the rest four W rows each.
// ---------------------------------------------------------------------------
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


// Row exponent of W row n (one wave, one block header per lane: a strided
// walk by a single thread is latency-bound at K = 12288).
RT_DEV void prep_w_row(const uint8_t *__restrict__ w, int *__restrict__ ew, int n, int K, int lane) {
  const int kb = K / 256;
  const uint8_t *row = w + (size_t)n * kb * kQ4KBlockBytes;
  float bound = 0.f;  // |w| <= max(15*63*|d|, 63*|dmin|)
  for (int i = lane; i < kb; i += 64) {
    const uint32_t h = *reinterpret_cast<const uint32_t *>(row + (size_t)i * kQ4KBlockBytes);
    bound = fmaxf(bound, fmaxf(945.f * fabsf(half_bits_to_f32(h & 0xFFFFu)), 63.f * fabsf(half_bits_to_f32(h >> 16))));
  }
  bound = wave_max(bound);
  if (lane == 0) ew[n] = f16_exponent_for(bound);
}

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
    // one wave per W row
    const int n = (b - M) * 4 + (int)(threadIdx.x >> 6);
    if (n < N) prep_w_row(w, ew, n, K, threadIdx.x & 63);
  }
}

// ---------------------------------------------------------------------------
// Eight-wave kernel, 64-wide K per barrier: C tile (128*WGM) x 256, waves
// WGM (M) x 8/WGM (N), two waves per SIMD.  Wave tile 128 x (256*WGM/8) as
// 4 x NT tiles of v_mfma_f32_32x32x16_f16; per barrier each wave issues
// 4 k-steps x 4 x NT MFMAs.
// Operands reach LDS by global_load_lds_dwordx4 two chunks ahead, in a ring
// of three slots (the chunk loop is unrolled by three so the slot is a
// compile-time constant; one __shared__ variable per slot):
//   A slot: BM rows x 8 x 16-byte segments; physical segment = logical ^
//           ((row >> 1) & 7), so the 16 rows served together (16 lanes of a
//           16-byte read per cycle, 64 banks) hit 16 distinct bank groups.
//   W slot: [part][column] 16-byte pieces for 256 columns: part 0 = qs bytes
//           0..15 of the chunk, part 1 = qs bytes 16..31, part 2 = header,
//           part 3 = a second copy of the header that nothing reads: it makes
//           every wave issue the same two W copies, so the kernel has no
//           wave-dependent branch and one vmcnt bound.
// ---------------------------------------------------------------------------
constexpr int kW8bSlotW = 4 * 256 * 16;  // 16 KB

// Split-K: blockIdx.y = s takes chunks [s*nchunks/ksplit, (s+1)*nchunks/ksplit)
// and, when ksplit > 1, writes its scaled partial tile to c + s*M*N for
// k_gemm_splitk_sum.
template <int WGM>
__global__ __launch_bounds__(512) void k_q4k_gemm_w8b(const _Float16 *__restrict__ a16, const int *__restrict__ ea,
                                                      const uint8_t *__restrict__ w, const int *__restrict__ ew,
                                                      float *__restrict__ c, int M, int N, int K, int tiles_m,
                                                      int tiles_n, int ksplit) {
  constexpr int BM = 128 * WGM, WN = 8 / WGM, NT = 256 / WN / 32;
  constexpr int IA = BM / 64;            // A copies per wave per chunk (BM rows x 128 B / 1 KB / 8 waves)
  constexpr int SLOT_A = BM * 128;       // bytes
  __shared__ __attribute__((aligned(1024))) uint8_t sa0[SLOT_A], sa1[SLOT_A], sa2[SLOT_A];
  __shared__ __attribute__((aligned(1024))) uint8_t sw0[kW8bSlotW], sw1[kW8bSlotW], sw2[kW8bSlotW];
  auto slotA = [&](int i) __attribute__((always_inline)) { return i == 0 ? sa0 : (i == 1 ? sa1 : sa2); };
  auto slotW = [&](int i) __attribute__((always_inline)) { return i == 0 ? sw0 : (i == 1 ? sw1 : sw2); };

  const int tid = (int)threadIdx.x, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, kept in an SGPR
  const int wm = wave / WN, wn = wave % WN;
  const int ntiles = tiles_m * tiles_n, per_xcd = (ntiles + 7) / 8;
  const int bid = (int)blockIdx.x;
  int tile = (bid & 7) * per_xcd + (bid >> 3);
  if (ntiles % 8 != 0) tile = bid;
  const int group = tile / (4 * tiles_n), in_group = tile % (4 * tiles_n);
  const int gm = min(4, tiles_m - group * 4);
  const int tm = group * 4 + in_group % gm, tn = in_group / gm;
  const int m0 = tm * BM, n0 = tn * 256;
  const int nblocks = K / 256, nchunks = K / kBK;
  const size_t row_bytes = (size_t)nblocks * kQ4KBlockBytes;
  const int split = (int)blockIdx.y;
  const int kc0 = split * nchunks / ksplit, kc1 = (split + 1) * nchunks / ksplit;  // >= 1 chunk (host: ksplit <= nchunks)
  const int nloc = kc1 - kc0;
  if (ksplit > 1) c += (size_t)split * M * N;

  // A copy i of this wave: slot rows 8*(IA*wave+i) + [0,8); lane -> row
  // r = 8*(IA*wave+i) + lane/8, physical segment lane%8, logical segment
  // (lane%8) ^ ((r >> 1) & 7).
  const _Float16 *a_src[IA];
#pragma unroll
  for (int i = 0; i < IA; ++i) {
    const int r = 8 * (IA * wave + i) + (lane >> 3);
    a_src[i] = a16 + (size_t)min(m0 + r, M - 1) * K + 8 * ((lane & 7) ^ ((r >> 1) & 7));
  }
  // W copies: waves 0-3 load parts 0 and 1 (qs), waves 4-7 parts 2 and 3
  // (header twice), for columns 64*(wave%4) + lane.
  const uint8_t *w_src = w + (size_t)min(n0 + 64 * (wave & 3) + lane, N - 1) * row_bytes;
  const int w_part0 = 2 * (wave >> 2);
  const int w_off0 = wave < 4 ? 0 : -1;  // qs byte offset of part 0 / 1; -1 selects the header

  auto issue = [&](int kc, int slot) __attribute__((always_inline)) {
    uint8_t *da = slotA(slot), *dw = slotW(slot);
#pragma unroll
    for (int i = 0; i < IA; ++i)
      __builtin_amdgcn_global_load_lds((gvoid *)(a_src[i] + (size_t)kc * kBK), (lvoid *)(da + (IA * wave + i) * 1024),
                                       16, 0, 0);
    const uint8_t *blk = w_src + (size_t)(kc >> 2) * kQ4KBlockBytes;
    const uint8_t *p0 = w_off0 < 0 ? blk : blk + 16 + 32 * (kc & 3);
    const uint8_t *p1 = w_off0 < 0 ? blk : p0 + 16;
    const int cw = 64 * (wave & 3) * 16;
    __builtin_amdgcn_global_load_lds((gvoid *)p0, (lvoid *)(dw + w_part0 * 4096 + cw), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((gvoid *)p1, (lvoid *)(dw + (w_part0 + 1) * 4096 + cw), 16, 0, 0);
  };

  int colw[NT];
  float bpw[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    colw[j] = (256 / WN) * wn + 32 * j + l32;
    bpw[j] = __builtin_amdgcn_ldexpf(g ? 0.0625f : 1.0f, -ew[min(n0 + colw[j], N - 1)]);
  }

  floatx16 acc[4][NT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = floatx16{};

  issue(kc0, 0);
  issue(min(kc0 + 1, kc1 - 1), 1);
  wait_vmcnt<0>();
  wg_barrier();

  // One chunk (local index lc, absolute kc): compute from ring slot `slot`,
  // prefetch chunk kc+2 into slot (slot+2)%3.
  auto chunk = [&](int lc, int slot) __attribute__((always_inline)) {
    const int kc = kc0 + lc;
    if (lc > 0) {
      // chunk kc's copies have landed everywhere; chunk kc+1's may stay in flight
      wait_vmcnt<IA + 2>();
      wait_lgkmcnt0();
      wg_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
    issue(min(kc + 2, kc1 - 1), slot == 0 ? 2 : slot - 1);
    __builtin_amdgcn_sched_barrier(0);

    const uint8_t *pa = slotA(slot), *pw = slotW(slot);
    auto read_a = [&](int t, u32x4 (&af)[4]) __attribute__((always_inline)) {
      const int seg = 2 * g + (t & 1) + 4 * (t >> 1);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 128 * wm + 32 * i + l32;
        af[i] = lds_read16(pa + rr * 128 + 16 * (seg ^ ((rr >> 1) & 7)));
      }
    };
    u32x4 qv[NT], hw[NT], af[4], afn[4];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      qv[j] = lds_read16(pw + g * 4096 + 16 * colw[j]);
      hw[j] = lds_read16(pw + 2 * 4096 + 16 * colw[j]);
    }
    read_a(0, afn);
    if constexpr (NT == 2)
      lds_wait(qv[0], qv[1], hw[0], hw[1]);
    else
      lds_wait(qv[0], hw[0], afn[0], afn[1]);
    const int cc = kc & 3;
    float sc_lo[NT], sc_hi[NT], nc_lo[NT], nc_hi[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const float d = half_bits_to_f32(hw[j][0] & 0xFFFFu), dmin = half_bits_to_f32(hw[j][0] >> 16);
      uint32_t sv, mv;
      q4k_scale_min(hw[j][1], hw[j][2], hw[j][3], 2 * cc + g, sv, mv);
      const float sfac = d * (float)sv * bpw[j];
      const float mn = dmin * (float)mv * (bpw[j] * (g ? 16.f : 1.f));
      const float ncv = -(mn + 1024.f * sfac);
      const auto s2 = __builtin_amdgcn_permlane32_swap(f32_bits(sfac), f32_bits(sfac), false, false);
      const auto n2 = __builtin_amdgcn_permlane32_swap(f32_bits(ncv), f32_bits(ncv), false, false);
      sc_lo[j] = bits_f32(s2[0]), sc_hi[j] = bits_f32(s2[1]);
      nc_lo[j] = bits_f32(n2[0]), nc_hi[j] = bits_f32(n2[1]);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      half8 bf[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const uint32_t w0 = qv[j][2 * (t & 1)], w1 = qv[j][2 * (t & 1) + 1];
        bf[j] = t < 2 ? dq_step<false>(w0, w1, sc_lo[j], nc_lo[j]) : dq_step<true>(w0, w1, sc_hi[j], nc_hi[j]);
      }
      lds_wait(afn[0], afn[1], afn[2], afn[3]);
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = afn[i];
      if (t < 3) read_a(t + 1, afn);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, af[i]), bf[j], acc[i][j], 0, 0, 0);
    }
  };

  int lc = 0;
  for (; lc + 3 <= nloc; lc += 3) {
    chunk(lc, 0);
    chunk(lc + 1, 1);
    chunk(lc + 2, 2);
  }
  if (lc < nloc) chunk(lc, 0);
  if (lc + 1 < nloc) chunk(lc + 1, 1);

  // Epilogue: the wave's 128 x 32NT tile through LDS (the ring is free once
  // every wave has passed the barrier; wave w stages in slot array w % 6,
  // at 8 KB for waves 6 and 7).
  int ecol[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) ecol[j] = ew[min(n0 + colw[j], N - 1)];
  wg_barrier();
  static_assert(32 * (32 * NT + 8) * 4 <= 8192 && SLOT_A >= 16384, "staging slice fits in half a slot");
  const int ws = wave % 6;
  uint8_t *sbase = ws == 0 ? sa0 : ws == 1 ? sa1 : ws == 2 ? sa2 : ws == 3 ? sw0 : ws == 4 ? sw1 : sw2;
  float *stage = reinterpret_cast<float *>(sbase + (wave / 6) * 8192);
  store_c_tile<NT>(acc, stage, c, M, N, m0 + 128 * wm, n0 + (256 / WN) * wn, ea, ecol);
}

// ---------------------------------------------------------------------------
// Half-block kernel: C tile 128 x 256, four waves side by side in N (wave
// tile 128 x 64 = 4 x 2 tiles of v_mfma_f32_32x32x16_f16), two workgroups
// per CU so one workgroup's barrier and LDS waits overlap the other's MFMAs.
//   A (f16): one 64-wide chunk per copy (128 rows x 128 B) by
//            global_load_lds into a ring of four LDS slots, two chunks ahead.
//            Row segments XOR-swizzled by (row >> 1) & 7.
//   W (Q4_K): straight into VGPRs, also two chunks ahead.  A wave uses only
//            its own 64 columns, so W has no reason to pass through LDS: per
//            chunk a lane loads the 16 qs bytes of its column and k group
//            (a ring of four register sets indexed by the chunk's place in
//            its block; the loop over blocks is unrolled by four), and per
//            block the 16-byte header.
// Split-K as in the eight-wave kernel, by whole super-blocks: blockIdx.y = s
// takes blocks [s*nblocks/ksplit, (s+1)*nblocks/ksplit).
// Up to three matrices sharing A (q|k|v, gate|up) run as one launch: their
// 256-column tiles are numbered one after another (HMats::tn0), and a
// workgroup takes the matrix its column tile falls in.
// GELU: the gate and up matrices of an FFN (mats.w[0], mats.w[1], N rows
// each) in one tile of 128 rows x 128 columns of both: a wave's column tile
// j = 0 is 32 gate columns and j = 1 the same 32 up columns, so the lane
// that holds g[m][n] also holds u[m][n], and the epilogue stores
// h = gelu_tanh(g) * u (Gemma3Mlp::forward, transformer4.rs:328-334) to
// mats.c[0] instead of g and u.  No K split.
// ---------------------------------------------------------------------------
constexpr int kHSlotA = 128 * 128;       // bytes

// The GELU epilogue: each staged value is gelu_tanh(g) * u of the wave's gate
// (acc[i][0]) and up (acc[i][1]) accumulators, each scaled by
// 2^(ea[row] + ew of its matrix) as store_c_tile scales them, and h goes out
// as the next GEMM's A operand: f16 scaled by 2^-eh[row] with eh[row] =
// f16_exponent_for(2 * a_nrm2[row] * gu_bound).  By Cauchy-Schwarz
// |g| <= |a| |w_gate|, |u| <= |a| |w_up| and |gelu_tanh(g)| <= |g|, so
// |h| <= |a|^2 max_n |w_gate,n| |w_up,n|: a_nrm2 = |a|^2 of the row of A (f32,
// before its f16 rounding) and gu_bound that maximum; the factor 2 covers
// the f16 operands and the f32 sums.  No value overflows, and f16 rounding is
// relative, so h rounds as with the exponent of its exact row maximum except
// for elements below 2^-14 of the scale.
RT_DEV void store_gelu_tile(const floatx16 (&acc)[4][2], float *stage, _Float16 *h16, int *eh, int M, int N,
                            int row0, int col0, const int *ea, const int (&ecol)[2], const float *a_nrm2,
                            float gu_bound) {
  constexpr int P = 40, F4 = 8, RPI = 8;
  const int lane = (int)(threadIdx.x & 63), g = lane >> 5, l32 = lane & 31;
  const bool vec = (N & 3) == 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int er[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) er[r] = ea[min(row0 + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3), M - 1)];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float gv = __builtin_amdgcn_ldexpf(acc[i][0][r], er[r] + ecol[0]);
      const float uv = __builtin_amdgcn_ldexpf(acc[i][1][r], er[r] + ecol[1]);
      stage[(8 * (r >> 2) + 4 * g + (r & 3)) * P + l32] = mul_nc(gelu_tanh(gv), uv);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < 32 / RPI; ++q) {
      const int rl = q * RPI + lane / F4, f = lane % F4;
      const int row = row0 + 32 * i + rl, col = col0 + 4 * f;
      const float4 v = *reinterpret_cast<const float4 *>(stage + rl * P + 4 * f);
      if (row < M) {
        const int e = f16_exponent_for(2.0f * a_nrm2[row] * gu_bound);
        if (col == 0) eh[row] = e;
        _Float16 *dst = h16 + (size_t)row * N + col;
        if (vec && col + 4 <= N) {
          *reinterpret_cast<uint2 *>(dst) = f16x4_scaled(v, e);
        } else {
          const float x[4] = {v.x, v.y, v.z, v.w};
          for (int k = 0; k < 4; ++k)
            if (col + k < N) dst[k] = (_Float16)__builtin_amdgcn_ldexpf(x[k], -e);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// |W row n|_2 of a Q4_K weight [N][K] over its dequantised values (one wave
// per row, f32 sums): the GELU GEMM's bound on |h| is built from them.
__global__ __launch_bounds__(256) void k_q4k_row_norms(const uint8_t *__restrict__ w, float *__restrict__ nrm, int N,
                                                       int K) {
  const int n = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  if (n >= N) return;  // whole waves
  const int kb = K / 256;
  const uint8_t *row = w + (size_t)n * kb * kQ4KBlockBytes;
  float ss = 0.f;
  for (int i = lane; i < kb; i += 64) {
    const uint8_t *blk = row + (size_t)i * kQ4KBlockBytes;
    const uint32_t *hw = reinterpret_cast<const uint32_t *>(blk);
    const float d = half_bits_to_f32(hw[0] & 0xFFFFu), dmin = half_bits_to_f32(hw[0] >> 16);
    for (int j = 0; j < 8; ++j) {  // sub-block j: the low (even j) or high nibbles of qs[32*(j/2), +32)
      uint32_t sv, mv;
      q4k_scale_min(hw[1], hw[2], hw[3], j, sv, mv);
      const float sc = d * (float)sv, mn = dmin * (float)mv;
      const uint8_t *qs = blk + 16 + 32 * (j >> 1);
      for (int b = 0; b < 32; ++b) {
        const float v = sc * (float)((j & 1) ? (qs[b] >> 4) : (qs[b] & 15)) - mn;
        ss += v * v;
      }
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) nrm[n] = sqrtf(ss);
}

// The W row exponents of every matrix of a set in one launch: wave r takes
// row r of the matrices' rows laid end to end.
__global__ __launch_bounds__(256) void k_gemm_prep_w_multi(HMats mats, int K) {
  int r = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), i = 0;
  while (i + 1 < mats.count && r >= mats.n[i]) r -= mats.n[i++];  // wave-uniform
  if (r < mats.n[i]) prep_w_row(mats.w[i], const_cast<int *>(mats.ew[i]), r, K, threadIdx.x & 63);
}

// GELU mode's output: h16 [M][N] f16 and its row exponents eh [M]; a_nrm2 and
// gu_bound as store_gelu_tile uses them.
struct GeluOut {
  _Float16 *h16;
  int *eh;
  const float *a_nrm2;
  float gu_bound;
};

// QKV mode: the per-head RMSNorm (gamma g_q for matrix 0, g_k for matrix 1)
// and NeoX RoPE of row m with cos | sin at cs + m*cs_stride (+ head_dim),
// applied before the store; matrix 2 (v) is stored as computed.
struct QkRope {
  const float *cs;
  int cs_stride;
  const float *g_q, *g_k;
  float eps;
};

enum HMode { kHPlain = 0, kHGelu = 1, kHQkv = 2 };

template <int MODE>
__global__ __launch_bounds__(256, 2) void k_q4k_gemm_h(const _Float16 *__restrict__ a16, const int *__restrict__ ea,
                                                       HMats mats, int M, int K, int tiles_m, int tiles_n,
                                                       int ksplit, GeluOut go = {}, QkRope qr = {}) {
  constexpr bool GELU = MODE == kHGelu, QKV = MODE == kHQkv;
  __shared__ __attribute__((aligned(1024))) uint8_t sa0[kHSlotA], sa1[kHSlotA], sa2[kHSlotA], sa3[kHSlotA];

  const int tid = (int)threadIdx.x, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ntiles = tiles_m * tiles_n, per_xcd = (ntiles + 7) / 8;
  const int bid = (int)blockIdx.x;
  int tile = (bid & 7) * per_xcd + (bid >> 3);
  if (ntiles % 8 != 0) tile = bid;
  const int group = tile / (4 * tiles_n), in_group = tile % (4 * tiles_n);
  const int gm = min(4, tiles_m - group * 4);
  const int tm = group * 4 + in_group % gm, tn = in_group / gm;
  int mi = 0;
  if (!GELU)
    while (mi + 1 < mats.count && tn >= mats.tn0[mi + 1]) ++mi;  // workgroup-uniform
  float *__restrict__ c = mats.c[mi];
  const int N = mats.n[mi];
  const int m0 = tm * 128, n0 = GELU ? tn * 128 : (tn - mats.tn0[mi]) * 256;
  const int nblocks = K / 256;
  const size_t row_bytes = (size_t)nblocks * kQ4KBlockBytes;
  const int split = (int)blockIdx.y;
  const int b0 = split * nblocks / ksplit, b1 = (split + 1) * nblocks / ksplit;  // >= 1 block (host: ksplit <= nblocks)
  const int klast = 4 * b1 - 1;                                                   // last chunk of this split
  if (ksplit > 1) c += (size_t)split * M * N;

  // Addresses are a workgroup-uniform base (SGPRs) plus a 32-bit lane
  // offset within the tile (at most 128 rows of A, 256 rows of W), which
  // keeps one VGPR per stream.
  // A copy i (0..3) of this wave: rows 8*(4*wave+i) + [0,8); lane -> row
  // r = 8*(4*wave+i) + lane/8, physical segment lane%8, logical segment
  // (lane%8) ^ ((r >> 1) & 7).
  const uint8_t *a_base = reinterpret_cast<const uint8_t *>(a16 + (size_t)m0 * K);
  uint32_t a_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * (4 * wave + i) + (lane >> 3);
    a_off[i] = (uint32_t)((min(m0 + r, M - 1) - m0) * K + 8 * ((lane & 7) ^ ((r >> 1) & 7))) * 2u;
  }
  auto issue_a = [&](int kc, uint8_t *slot) __attribute__((always_inline)) {
    const uint8_t *base = a_base + (size_t)kc * (kBK * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds((gvoid *)(base + a_off[i]), (lvoid *)(slot + (4 * wave + i) * 1024), 16, 0, 0);
  };
  // W: column tile j (0, 1) of this wave, lane -> column colw[j] of matrix
  // wm[j], k group g -> qs bytes [16g, 16g+16) of each chunk's 32.
  int colw[2], ewc[2];
  float bpw[2];
  const uint8_t *w_base[2];
  uint32_t w_off[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int wm = GELU ? j : mi;
    colw[j] = GELU ? 32 * wave + l32 : QKV ? 32 * wave + 128 * j + l32 : 64 * wave + 32 * j + l32;
    const int n = min(n0 + colw[j], N - 1);
    ewc[j] = mats.ew[wm][n];
    bpw[j] = __builtin_amdgcn_ldexpf(g ? 0.0625f : 1.0f, -ewc[j]);
    w_base[j] = mats.w[wm] + (size_t)n0 * row_bytes;
    w_off[j] = (uint32_t)(n - n0) * (uint32_t)row_bytes;
  }
  auto load_qs = [&](int kc, u32x4 (&q)[2]) __attribute__((always_inline)) {
    const size_t koff = (size_t)(kc >> 2) * kQ4KBlockBytes + 16 + 32 * (kc & 3);
#pragma unroll
    for (int j = 0; j < 2; ++j) q[j] = *reinterpret_cast<const u32x4 *>(w_base[j] + koff + (w_off[j] + 16u * g));
  };
  auto load_hdr = [&](int blk, u32x4 (&h)[2]) __attribute__((always_inline)) {
    const size_t koff = (size_t)blk * kQ4KBlockBytes;
#pragma unroll
    for (int j = 0; j < 2; ++j) h[j] = *reinterpret_cast<const u32x4 *>(w_base[j] + koff + w_off[j]);
  };

  floatx16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{};

  // Loads issued per chunk k, in this order: qs of chunk k+2 (2), at the
  // second chunk of a block the next block's headers (2), then the A copies
  // of chunk k+2 (4), one after each k-step's LDS reads (spread over the
  // chunk, the copies cost 4-7% less time than issued together).  Past the
  // split's last chunk they repeat the last one, so every chunk issues the
  // same count.  The prologue issues what chunks 4*b0-2 and 4*b0-1 would
  // have.
  u32x4 qs0[2], qs1[2], qs2[2], qs3[2], hnext[2], hcur[2];
  load_qs(4 * b0, qs0);
  load_hdr(b0, hnext);
  issue_a(4 * b0, sa0);
  load_qs(min(4 * b0 + 1, klast), qs1);
  issue_a(min(4 * b0 + 1, klast), sa1);

  for (int b = b0; b < b1; ++b) {
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int kc = 4 * b + cc;
      const uint8_t *pa = cc == 0 ? sa0 : cc == 1 ? sa1 : cc == 2 ? sa2 : sa3;
      // Chunk kc's A copies were issued two chunks ago; the 6 loads issued
      // one chunk ago (8 after a block's second chunk) may stay in flight.
      // The barrier then shows every wave's copies, and the slot the copies
      // below overwrite was last read two chunks ago.  (The compiler's own
      // waits cover the W registers.)
      __builtin_amdgcn_sched_barrier(0);
      if (cc == 2)
        wait_vmcnt<8>();
      else
        wait_vmcnt<6>();
      wg_barrier();
      __builtin_amdgcn_sched_barrier(0);
      const int kn = min(kc + 2, klast);
      {
        u32x4(&qn)[2] = cc == 0 ? qs2 : cc == 1 ? qs3 : cc == 2 ? qs0 : qs1;
        load_qs(kn, qn);
        if (cc == 1) load_hdr(min(b + 1, b1 - 1), hnext);
      }
      __builtin_amdgcn_sched_barrier(0);
      uint8_t *slot_n = cc == 0 ? sa2 : cc == 1 ? sa3 : cc == 2 ? sa0 : sa1;
      const uint8_t *a_next = a_base + (size_t)kn * (kBK * 2);
      if (cc == 0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) hcur[j] = hnext[j];
      }
      const u32x4(&qw)[2] = cc == 0 ? qs0 : cc == 1 ? qs1 : cc == 2 ? qs2 : qs3;

      auto read_a = [&](int t, u32x4 (&af)[4]) __attribute__((always_inline)) {
        const int seg = 2 * g + (t & 1) + 4 * (t >> 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rr = 32 * i + l32;
          af[i] = lds_read16(pa + rr * 128 + 16 * (seg ^ ((rr >> 1) & 7)));
        }
      };
      u32x4 af[4], afn[4];
      read_a(0, afn);
      float sc_lo[2], sc_hi[2], nc_lo[2], nc_hi[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float d = half_bits_to_f32(hcur[j][0] & 0xFFFFu), dmin = half_bits_to_f32(hcur[j][0] >> 16);
        uint32_t sv, mv;
        q4k_scale_min(hcur[j][1], hcur[j][2], hcur[j][3], 2 * cc + g, sv, mv);
        const float sfac = d * (float)sv * bpw[j];
        const float mn = dmin * (float)mv * (bpw[j] * (g ? 16.f : 1.f));
        const float ncv = -(mn + 1024.f * sfac);
        const auto s2 = __builtin_amdgcn_permlane32_swap(f32_bits(sfac), f32_bits(sfac), false, false);
        const auto n2 = __builtin_amdgcn_permlane32_swap(f32_bits(ncv), f32_bits(ncv), false, false);
        sc_lo[j] = bits_f32(s2[0]), sc_hi[j] = bits_f32(s2[1]);
        nc_lo[j] = bits_f32(n2[0]), nc_hi[j] = bits_f32(n2[1]);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        half8 bf[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t w0 = qw[j][2 * (t & 1)], w1 = qw[j][2 * (t & 1) + 1];
          bf[j] = t < 2 ? dq_step<false>(w0, w1, sc_lo[j], nc_lo[j]) : dq_step<true>(w0, w1, sc_hi[j], nc_hi[j]);
        }
        lds_wait(afn[0], afn[1], afn[2], afn[3]);
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = afn[i];
        if (t < 3) read_a(t + 1, afn);
        __builtin_amdgcn_global_load_lds((gvoid *)(a_next + a_off[t]), (lvoid *)(slot_n + (4 * wave + t) * 1024), 16,
                                         0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, af[i]), bf[j], acc[i][j], 0,
                                                               0, 0);
      }
    }
  }

  // Epilogue: the wave's 128 x 64 tile through LDS, wave w staging in slot w
  // once the tail's repeated copies have landed and every wave has passed
  // the barrier.
  int ecol[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) ecol[j] = ewc[j];
  wait_vmcnt<0>();
  wg_barrier();
  static_assert(32 * 72 * 4 <= kHSlotA, "staging slice fits in a slot");
  uint8_t *sbase = wave == 0 ? sa0 : wave == 1 ? sa1 : wave == 2 ? sa2 : sa3;
  if constexpr (GELU) {
    store_gelu_tile(acc, reinterpret_cast<float *>(sbase), go.h16, go.eh, M, N, m0, n0 + 32 * wave, ea, ecol,
                    go.a_nrm2, go.gu_bound);
  } else if constexpr (QKV) {
    // The tile is one head (256 columns) of 128 rows; lane (g, l32) of wave w
    // holds columns c = 32w + l32 (j = 0) and c + 128 (j = 1), the RoPE pair.
    // One 32-row MFMA tile (i) at a time, so its accumulators are free once
    // it is stored.
    float *stage = reinterpret_cast<float *>(sbase);
    // each wave's sums of squares of the tile's rows: the last 2 KB of slot 3
    // (the staging slices use the first 9 KB of each slot)
    float(*wsum)[128] = reinterpret_cast<float(*)[128]>(sa3 + kHSlotA - 2048);
    const int colp[2] = {n0 + 32 * wave, n0 + 128 + 32 * wave};
    const int cl = 32 * wave + l32;  // the pair's column within the head
    const float *gam = mi == 0 ? qr.g_q : qr.g_k;
    const float g0 = mi < 2 ? 1.0f + gam[cl] : 0.f, g1 = mi < 2 ? 1.0f + gam[cl + 128] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_sched_barrier(0);
      floatx16 v0, v1;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int er = ea[min(m0 + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3), M - 1)];
        v0[r] = __builtin_amdgcn_ldexpf(acc[i][0][r], er + ecol[0]);
        v1[r] = __builtin_amdgcn_ldexpf(acc[i][1][r], er + ecol[1]);
      }
      if (mi < 2) {  // workgroup-uniform
        // sums of squares of the 32 rows: this wave's 64 columns through its
        // LDS slot ([row][l32], 16-byte groups swizzled by the row), two
        // lanes per row, then the four waves' sums through wsum
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int R = 8 * (r >> 2) + 4 * g + (r & 3);
          stage[R * 32 + ((((l32 >> 2) ^ R) & 7) << 2) + (l32 & 3)] = v0[r] * v0[r] + v1[r] * v1[r];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        {
          const int R = lane >> 1;
          float t = 0.f;
#pragma unroll
          for (int m4 = 4 * (lane & 1); m4 < 4 * (lane & 1) + 4; ++m4) {
            const float4 x = *reinterpret_cast<const float4 *>(stage + R * 32 + (((m4 ^ R) & 7) << 2));
            t += (x.x + x.y) + (x.z + x.w);
          }
          t += __shfl_xor(t, 1);
          if ((lane & 1) == 0) wsum[wave][32 * i + R] = t;
        }
        wg_barrier();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
#pragma clang fp contract(off)
          const int R = 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
          const float ss = (wsum[0][R] + wsum[1][R]) + (wsum[2][R] + wsum[3][R]);
          const float rinv = rms_inv_from_sumsq(ss, 1.0f / 256.0f, qr.eps);
          const int co = min(m0 + R, M - 1) * qr.cs_stride + cl;  // 32-bit offset from the uniform base
          const float cv = qr.cs[co], sv = qr.cs[co + 128];
          const float a0 = (v0[r] * rinv) * g0, a1 = (v1[r] * rinv) * g1;
          v0[r] = a0 * cv - a1 * sv;
          v1[r] = a0 * sv + a1 * cv;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      // stage and store the tile's 32 rows x (32 + 32) columns
      constexpr int P = 72;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        stage[(8 * (r >> 2) + 4 * g + (r & 3)) * P + l32] = v0[r];
        stage[(8 * (r >> 2) + 4 * g + (r & 3)) * P + 32 + l32] = v1[r];
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int rl = q * 4 + lane / 16, f = lane % 16;
        const int row = m0 + 32 * i + rl, cc = colp[f >> 3] + 4 * (f & 7);
        const float4 x = *reinterpret_cast<const float4 *>(stage + rl * P + 4 * f);
        if (row < M) *reinterpret_cast<float4 *>(c + (size_t)row * N + cc) = x;
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  } else {
    store_c_tile<2>(acc, reinterpret_cast<float *>(sbase), c, M, N, m0, n0 + 64 * wave, ea, ecol);
  }
}

}  // namespace

// Sums the split-K partial tiles in split order (deterministic):
// c[i] = sum_s part[s*mn + i].
__global__ __launch_bounds__(256) void k_gemm_splitk_sum(const float *__restrict__ part, float *__restrict__ c,
                                                         size_t mn, int ksplit) {
  const size_t n4 = mn / 4;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    float4 acc = reinterpret_cast<const float4 *>(part)[i];
    for (int s = 1; s < ksplit; ++s) {
      const float4 v = reinterpret_cast<const float4 *>(part + (size_t)s * mn)[i];
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    reinterpret_cast<float4 *>(c)[i] = acc;
  }
  for (size_t i = n4 * 4 + (size_t)blockIdx.x * 256 + threadIdx.x; i < mn; i += (size_t)gridDim.x * 256) {
    float acc = part[i];
    for (int s = 1; s < ksplit; ++s) acc += part[(size_t)s * mn + i];
    c[i] = acc;
  }
}

// Which matrix-core kernel takes an M x N output, and how many ways K is
// split (blockIdx.y; a split of ks writes ks partial products of M x N).
// Tiles are 128 x 256 (th) for the eight-wave and half-block kernels and
// 256 x 256 (tw) for the wide one.
//   w8b:   up to 1024 rows and th < 512; the eight-wave kernel, one
//          workgroup per CU, fills the chip better with few tiles
//          (512x10240, 160 tiles: 54.9 us against 61.6 us for the
//          half-block kernel).  K splits into enough workgroups to cover the
//          256 CUs (a prefill's down projection, M=512 N=2560: 40 tiles),
//          keeping at least 16 chunks (K=1024) per split.
//   wide:  a single matrix of more than 1024 rows with 128 < tw <= 256: one
//          round of one workgroup per CU, where the half-block kernel runs
//          two on most CUs.  4608x3072x12288 (216 tiles): 349 us against
//          377 us; 4096x2560x10240 split 3 ways: 230 against 235 us.
//   half:  the rest (and every set of matrices sharing A); two workgroups per
//          CU.  4608x12288x3072 (864 wide tiles, 3.4 rounds): 375 us against
//          425 us for the wide kernel, whose last round runs 96 workgroups
//          on 256 CUs; with tw <= 128 its 128-row tiles, one workgroup per
//          CU, spread the work over twice as many CUs.
// Above 1024 rows K takes the split that minimises a time model fitted to
// MI355X measurements:
//   rounds/ks of c us per K element, plus (2*ks+1)*M*N*4 bytes of partial
//   tiles at 5 TB/s;
//   wide:  rounds = ceil(tw*ks/256), c = 0.036;
//   half:  rounds = ceil(th*ks/512), x0.75 when at most 256 workgroups run
//          (one per CU), c = 0.032.
// 4096x2560 outputs (160 wide tiles) split K=10240 three ways: 2 rounds of a
// third instead of 1 round of the whole K on 160 of the 256 CUs.
enum class GemmKind { w8b, half, wide };
struct GemmPlan {
  GemmKind kind;
  int ks;
};
static GemmKind gemm_kind(int M, int tiles_n, bool single) {
  const int th = ((M + 127) / 128) * tiles_n, tw = ((M + 255) / 256) * tiles_n;
  if (single && M > 1024 && tw > 128 && tw <= 256) return GemmKind::wide;
  return M > 1024 || th >= 512 ? GemmKind::half : GemmKind::w8b;
}

static GemmPlan gemm_plan(int M, int N, int K) {
  const int tiles_n = (N + 255) / 256;
  const GemmKind kind = gemm_kind(M, tiles_n, true);
  if (kind == GemmKind::w8b) {
    const int by_cus = 256 / (((M + 127) / 128) * tiles_n), by_k = (K / kBK) / 16;
    return {kind, max(1, min(by_cus, by_k))};
  }
  if (M <= 1024) return {kind, 1};
  const bool wide = kind == GemmKind::wide;
  const int ntiles = wide ? ((M + 255) / 256) * tiles_n : ((M + 127) / 128) * tiles_n;
  auto est_us = [&](int ks) {
    const int wgs = ntiles * ks;
    const double rounds = wide ? (double)((wgs + 255) / 256) : (double)((wgs + 511) / 512) * (wgs <= 256 ? 0.75 : 1.0);
    const double partial = ks > 1 ? (2.0 * ks + 1.0) * M * N * 4.0 / 5e6 : 0.0;
    return rounds / ks * K * (wide ? 0.036 : 0.032) + partial;
  };
  int best = 1;
  for (int ks = 2; ks <= 4 && ks <= K / 256; ++ks)
    if (est_us(ks) < est_us(best)) best = ks;
  return {kind, best};
}

hipError_t launch_gemm_splitk_sum(const float *part, float *c, size_t mn, int ksplit, hipStream_t s) {
  const unsigned grid = (unsigned)std::min<size_t>((mn / 4 + 255) / 256 + 1, 2048);
  hipLaunchKernelGGL(k_gemm_splitk_sum, dim3(grid), dim3(256), 0, s, part, c, mn, ksplit);
  return hipGetLastError();
}

hipError_t launch_gemm_prep_a(const float *a, int M, int K, _Float16 *a16, int *ea, hipStream_t s) {
  hipLaunchKernelGGL((k_gemm_prep<float>), dim3(M), dim3(256), 0, s, a, a16, ea, nullptr, nullptr, M, 0, K);
  return hipGetLastError();
}

size_t q4k_gemm_workspace_bytes(int M, int N, int K) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  const int ks = gemm_plan(M, N, K).ks;
  return r256((size_t)M * K * 2) + r256((size_t)M * 4) + r256((size_t)N * 4) +
         (ks > 1 ? r256((size_t)ks * M * N * 4) : 0);
}

// The matrix-core launch on prepared operands; `part` holds the split-K
// partials when the shape splits K.
static hipError_t q4k_gemm_core(const _Float16 *a16, const int *ea, const uint8_t *wb, const int *ew, float *part,
                                float *c, int M, int N, int K, hipStream_t s, GemmLeft *left = nullptr) {
  const int tiles_m = (M + 127) / 128, tiles_n = (N + 255) / 256;
  const GemmPlan plan = gemm_plan(M, N, K);
  const GemmKind kind = plan.kind;
  const int ks = plan.ks;
  float *out = ks > 1 ? part : c;
  hipError_t e = hipSuccess;
  if (kind == GemmKind::wide) {
    e = launch_q4k_gemm_wide(a16, ea, HMats{{wb}, {ew}, {out}, {N}, {0}, 1}, M, K, tiles_n, ks, s);
  } else {
    if (kind == GemmKind::w8b)
      hipLaunchKernelGGL(k_q4k_gemm_w8b<1>, dim3(tiles_m * tiles_n, ks), dim3(512), 0, s, a16, ea, wb, ew, out, M,
                         N, K, tiles_m, tiles_n, ks);
    else
      hipLaunchKernelGGL(k_q4k_gemm_h<kHPlain>, dim3(tiles_m * tiles_n, ks), dim3(256), 0, s, a16, ea,
                         HMats{{wb}, {ew}, {out}, {N}, {0}, 1}, M, K, tiles_m, tiles_n, ks);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  if (left) {
    *left = GemmLeft{out, ks};
    return hipSuccess;
  }
  return ks > 1 ? launch_gemm_splitk_sum(part, c, (size_t)M * N, ks, s) : hipSuccess;
}

hipError_t launch_q4k_gemm(const void *a, bool a_bf16, const void *w, float *c, int M, int N, int K, void *ws,
                           hipStream_t s) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  char *p = static_cast<char *>(ws);
  _Float16 *a16 = reinterpret_cast<_Float16 *>(p);
  int *ea = reinterpret_cast<int *>(p + r256((size_t)M * K * 2));
  int *ew = reinterpret_cast<int *>(p + r256((size_t)M * K * 2) + r256((size_t)M * 4));
  float *part = reinterpret_cast<float *>(p + r256((size_t)M * K * 2) + r256((size_t)M * 4) + r256((size_t)N * 4));
  const uint8_t *wb = static_cast<const uint8_t *>(w);
  const int prep_blocks = M + (N + 3) / 4;
  if (a_bf16)
    hipLaunchKernelGGL((k_gemm_prep<uint16_t>), dim3(prep_blocks), dim3(256), 0, s,
                       static_cast<const uint16_t *>(a), a16, ea, wb, ew, M, N, K);
  else
    hipLaunchKernelGGL((k_gemm_prep<float>), dim3(prep_blocks), dim3(256), 0, s, static_cast<const float *>(a), a16,
                       ea, wb, ew, M, N, K);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return q4k_gemm_core(a16, ea, wb, ew, part, c, M, N, K, s);
}

size_t q4k_gemm_prepped_ws_bytes(int M, int N, int K) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  return q4k_gemm_workspace_bytes(M, N, K) - r256((size_t)M * K * 2) - r256((size_t)M * 4);
}

hipError_t launch_q4k_row_exponents(const void *w, int N, int K, int *ew, hipStream_t s) {
  // W rows only (no A rows: M = 0 in the prep's indexing)
  hipLaunchKernelGGL((k_gemm_prep<float>), dim3((N + 3) / 4), dim3(256), 0, s, nullptr, nullptr, nullptr,
                     static_cast<const uint8_t *>(w), ew, 0, N, K);
  return hipGetLastError();
}

hipError_t launch_q4k_gemm_prepped(const _Float16 *a16, const int *ea, const void *w, float *c, int M, int N, int K,
                                   void *ws, hipStream_t s, GemmLeft *left, const int *ew_pre) {
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  char *p = static_cast<char *>(ws);
  float *part = reinterpret_cast<float *>(p + r256((size_t)N * 4));
  const uint8_t *wb = static_cast<const uint8_t *>(w);
  const int *ew = ew_pre;
  if (!ew) {
    int *ewp = reinterpret_cast<int *>(p);
    hipError_t e = launch_q4k_row_exponents(wb, N, K, ewp, s);
    if (e != hipSuccess) return e;
    ew = ewp;
  }
  return q4k_gemm_core(a16, ea, wb, ew, part, c, M, N, K, s, left);
}

bool q4k_gemm_multi_ok(int M, int count, const int *n) {
  if (count < 1 || count > 3) return false;
  int tiles_n = 0;
  for (int i = 0; i < count; ++i) tiles_n += (n[i] + 255) / 256;
  return gemm_kind(M, tiles_n, false) == GemmKind::half;
}

bool q4k_gemm_gelu_ok(int M, int N) {
  const int n[2] = {N, N};
  return q4k_gemm_multi_ok(M, 2, n);
}

hipError_t launch_q4k_gemm_gelu_prepped(const _Float16 *a16, const int *ea, const float *a_nrm2, const void *w_gate,
                                        const void *w_up, const int *ew_gate, const int *ew_up, float gu_bound,
                                        _Float16 *h16, int *eh, int M, int N, int K, hipStream_t s) {
  if (!q4k_gemm_gelu_ok(M, N) || K % 256 != 0 || N <= 0 || !ew_gate || !ew_up || !a_nrm2 || !(gu_bound >= 0.f))
    return hipErrorInvalidValue;
  HMats mats{};
  mats.w[0] = static_cast<const uint8_t *>(w_gate);
  mats.w[1] = static_cast<const uint8_t *>(w_up);
  mats.ew[0] = ew_gate;
  mats.ew[1] = ew_up;
  mats.n[0] = mats.n[1] = N;
  mats.count = 2;
  const int tiles_m = (M + 127) / 128, tiles_n = (N + 127) / 128;
  hipLaunchKernelGGL(k_q4k_gemm_h<kHGelu>, dim3(tiles_m * tiles_n), dim3(256), 0, s, a16, ea, mats, M, K, tiles_m,
                     tiles_n, 1, GeluOut{h16, eh, a_nrm2, gu_bound});
  return hipGetLastError();
}

bool q4k_gemm_qkv_ok(int M, int QD, int KVD, int head_dim) {
  const int n[3] = {QD, KVD, KVD};
  return head_dim == 256 && QD % 256 == 0 && KVD % 256 == 0 && q4k_gemm_multi_ok(M, 3, n);
}

hipError_t launch_q4k_gemm_qkv_prepped(const _Float16 *a16, const int *ea, const void *const *w, const int *const *ew,
                                       float *q_out, float *k_rows, float *v_rows, int M, int QD, int KVD, int K,
                                       const float *cs, int cs_stride, const float *g_q, const float *g_k, float eps,
                                       hipStream_t s) {
  if (!q4k_gemm_qkv_ok(M, QD, KVD, 256) || K % 256 != 0) return hipErrorInvalidValue;
  HMats mats{};
  float *out[3] = {q_out, k_rows, v_rows};
  const int n[3] = {QD, KVD, KVD};
  int tiles_n = 0;
  for (int i = 0; i < 3; ++i) {
    if (!w[i] || !ew[i]) return hipErrorInvalidValue;
    mats.w[i] = static_cast<const uint8_t *>(w[i]);
    mats.ew[i] = ew[i];
    mats.c[i] = out[i];
    mats.n[i] = n[i];
    mats.tn0[i] = tiles_n;
    tiles_n += n[i] / 256;
  }
  mats.count = 3;
  const int tiles_m = (M + 127) / 128;
  hipLaunchKernelGGL(k_q4k_gemm_h<kHQkv>, dim3(tiles_m * tiles_n), dim3(256), 0, s, a16, ea, mats, M, K, tiles_m,
                     tiles_n, 1, GeluOut{}, QkRope{cs, cs_stride, g_q, g_k, eps});
  return hipGetLastError();
}

hipError_t launch_q4k_row_norms(const void *w, int N, int K, float *nrm, hipStream_t s) {
  hipLaunchKernelGGL(k_q4k_row_norms, dim3((N + 3) / 4), dim3(256), 0, s, static_cast<const uint8_t *>(w), nrm, N, K);
  return hipGetLastError();
}

hipError_t launch_q4k_gemm_multi_prepped(const _Float16 *a16, const int *ea, int count, const void *const *w,
                                         float *const *c, const int *n, void *const *ws, int M, int K,
                                         hipStream_t s, const int *const *ew_pre) {
  if (!q4k_gemm_multi_ok(M, count, n) || K % 256 != 0) return hipErrorInvalidValue;
  HMats mats{};
  int tiles_n = 0, rows = 0;
  bool all_pre = ew_pre != nullptr;
  for (int i = 0; i < count; ++i) {
    if (n[i] <= 0) return hipErrorInvalidValue;
    all_pre = all_pre && ew_pre[i];
  }
  for (int i = 0; i < count; ++i) {
    mats.w[i] = static_cast<const uint8_t *>(w[i]);
    mats.ew[i] = all_pre ? ew_pre[i] : static_cast<const int *>(ws[i]);
    mats.c[i] = c[i];
    mats.n[i] = n[i];
    mats.tn0[i] = tiles_n;
    tiles_n += (n[i] + 255) / 256;
    rows += n[i];
  }
  mats.count = count;
  if (!all_pre) {
    hipLaunchKernelGGL(k_gemm_prep_w_multi, dim3((rows + 3) / 4), dim3(256), 0, s, mats, K);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int tiles_m = (M + 127) / 128;
  hipLaunchKernelGGL(k_q4k_gemm_h<kHPlain>, dim3(tiles_m * tiles_n), dim3(256), 0, s, a16, ea, mats, M, K, tiles_m, tiles_n,
                     1);
  return hipGetLastError();
}

}  // namespace rt
