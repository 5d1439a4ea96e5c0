// q4k_gemm_wide.hip -- the Q4_K GEMM on 256 x 256 C tiles: four waves of
// 256 x 64, one workgroup per CU, accumulators in AGPRs.
//
// Same operands, dequantisation, K order and epilogue as the kernels of
// q4k_gemm.hip: for the same K split its results are bit-identical to
// theirs.  What changes is the wave tile: each dequantised B fragment feeds
// eight 32-row MFMA tiles instead of four, so the dequantisation costs half
// as much VALU work per MFMA.  The host takes this kernel where its tiles fit
// one round of the CUs (q4k_gemm.hip, gemm_plan).  The 256 x 4 x 16
// accumulator registers per lane fill the AGPR file, so this file is built
// without the VGPR-form MFMA option of q4k_gemm.hip.
//
// Pipeline: a ring of three LDS slots, two chunks ahead.  Per chunk a slot
// holds A (256 rows x 64 k of f16, 32 KB, 16-byte segments XOR-swizzled by
// (row >> 1) & 7) and the chunk's W bytes (256 columns x 48 B: the block
// header and the chunk's 32 qs bytes, 12 KB), copied by global_load_lds
// (8 A and 3 W copies per wave).  The copies of chunk kc+2 are issued one
// to three after each k-step's LDS reads rather than together at the chunk
// start; the chunk-start wait and barrier are unchanged.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "mfma_common.hpp"
#include "q4k_gemm_dev.hpp"
#include "rt_device.hpp"

namespace rt {
namespace {

constexpr int kWSlotA = 256 * 128;  // bytes
constexpr int kWSlotW = 256 * 48;   // bytes
constexpr int kWCopies = 11;        // copies per wave per chunk: 8 A, 3 W

// Split-K: blockIdx.y = s takes chunks [s*nchunks/ksplit, (s+1)*nchunks/ksplit)
// and, when ksplit > 1, writes its scaled partial tile to c + s*M*N.
__global__ __launch_bounds__(256, 1) void k_q4k_gemm_wide(const _Float16 *__restrict__ a16,
                                                          const int *__restrict__ ea, HMats mats, int M, int K,
                                                          int tiles_m, int tiles_n, int ksplit) {
  __shared__ __attribute__((aligned(1024))) uint8_t sa0[kWSlotA], sa1[kWSlotA], sa2[kWSlotA];
  __shared__ __attribute__((aligned(1024))) uint8_t sw0[kWSlotW], sw1[kWSlotW], sw2[kWSlotW];
  auto slotA = [&](int i) __attribute__((always_inline)) { return i == 0 ? sa0 : (i == 1 ? sa1 : sa2); };
  auto slotW = [&](int i) __attribute__((always_inline)) { return i == 0 ? sw0 : (i == 1 ? sw1 : sw2); };

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
  while (mi + 1 < mats.count && tn >= mats.tn0[mi + 1]) ++mi;  // wave-uniform
  const uint8_t *__restrict__ w = mats.w[mi];
  const int *__restrict__ ew = mats.ew[mi];
  float *__restrict__ c = mats.c[mi];
  const int N = mats.n[mi];
  const int m0 = tm * 256, n0 = (tn - mats.tn0[mi]) * 256;
  const int nblocks = K / 256, nchunks = K / kBK;
  const size_t row_bytes = (size_t)nblocks * kQ4KBlockBytes;
  const int split = (int)blockIdx.y;
  const int kc0 = split * nchunks / ksplit, kc1 = (split + 1) * nchunks / ksplit;  // >= 1 chunk (host)
  const int nloc = kc1 - kc0;
  if (ksplit > 1) c += (size_t)split * M * N;

  // A copy i (0..7) of this wave: slot rows 8*(8*wave+i) + [0,8); lane ->
  // row r = 8*(8*wave+i) + lane/8, physical segment lane%8, logical segment
  // (lane%8) ^ ((r >> 1) & 7).  Addresses: a workgroup-uniform base plus a
  // 32-bit lane offset within the 256-row tile.
  const uint8_t *a_base = reinterpret_cast<const uint8_t *>(a16 + (size_t)m0 * K);
  uint32_t a_off[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 8 * (8 * wave + i) + (lane >> 3);
    a_off[i] = (uint32_t)((min(m0 + r, M - 1) - m0) * K + 8 * ((lane & 7) ^ ((r >> 1) & 7))) * 2u;
  }
  // W copy i (0..2): piece p = 64*(3*wave+i) + lane of the slot, column p/3,
  // part p%3 (0 = block header, 1 and 2 = qs bytes 0..15 and 16..31 of the
  // chunk), 48 contiguous LDS bytes per column.
  const uint8_t *w_base = w + (size_t)n0 * row_bytes;
  uint32_t w_off[3];
  int w_part[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int p = 64 * (3 * wave + i) + lane, col = p / 3;
    w_part[i] = p - 3 * col;
    w_off[i] = (uint32_t)(min(n0 + col, N - 1) - n0) * (uint32_t)row_bytes;
  }
  // copy q (0..10) of chunk kc into slot `slot`: A copies 0..7, then W copies
  auto issue_one = [&](int kc, int slot, int q) __attribute__((always_inline)) {
    if (q < 8) {
      __builtin_amdgcn_global_load_lds((gvoid *)(a_base + (size_t)kc * (kBK * 2) + a_off[q]),
                                       (lvoid *)(slotA(slot) + (8 * wave + q) * 1024), 16, 0, 0);
    } else {
      const int i = q - 8;
      const int off = w_part[i] == 0 ? 0 : 16 * w_part[i] + 32 * (kc & 3);
      __builtin_amdgcn_global_load_lds((gvoid *)(w_base + (size_t)(kc >> 2) * kQ4KBlockBytes + w_off[i] + off),
                                       (lvoid *)(slotW(slot) + (3 * wave + i) * 1024), 16, 0, 0);
    }
  };

  int colw[2], ewc[2];
  float bpw[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    colw[j] = 64 * wave + 32 * j + l32;
    ewc[j] = ew[min(n0 + colw[j], N - 1)];
    bpw[j] = __builtin_amdgcn_ldexpf(g ? 0.0625f : 1.0f, -ewc[j]);
  }
  floatx16 acc[2][4][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[h][i][j] = floatx16{};

#pragma unroll
  for (int q = 0; q < kWCopies; ++q) issue_one(kc0, 0, q);
#pragma unroll
  for (int q = 0; q < kWCopies; ++q) issue_one(min(kc0 + 1, kc1 - 1), 1, q);
  wait_vmcnt<0>();
  wg_barrier();

  // One chunk (local index lc): compute from ring slot `slot`, and copy
  // chunk kc+2 (past the split's end: its last chunk again, so every chunk
  // issues the same count) into slot (slot+2)%3, whose chunk every wave
  // finished before this chunk's barrier.
  auto chunk = [&](int lc, int slot) __attribute__((always_inline)) {
    const int kc = kc0 + lc;
    if (lc > 0) {
      // chunk kc's copies have landed everywhere; chunk kc+1's may stay in flight
      wait_vmcnt<kWCopies>();
      wait_lgkmcnt0();
      wg_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
    const int kn = min(kc + 2, kc1 - 1), sn = slot == 0 ? 2 : slot - 1;
    const uint8_t *pa = slotA(slot), *pw = slotW(slot);
    auto read_a = [&](int t, u32x4 (&af)[8]) __attribute__((always_inline)) {
      const int seg = 2 * g + (t & 1) + 4 * (t >> 1);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int rr = 32 * i + l32;
        af[i] = lds_read16(pa + rr * 128 + 16 * (seg ^ ((rr >> 1) & 7)));
      }
    };
    u32x4 hw[2], qv[2], af[8], afn[8];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      hw[j] = lds_read16(pw + 48 * colw[j]);
      qv[j] = lds_read16(pw + 48 * colw[j] + 16 + 16 * g);
    }
    read_a(0, afn);
    lds_wait(hw[0], hw[1], qv[0], qv[1]);
    const int cc = kc & 3;
    float sc_lo[2], sc_hi[2], nc_lo[2], nc_hi[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
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
      half8 bf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t w0 = qv[j][2 * (t & 1)], w1 = qv[j][2 * (t & 1) + 1];
        bf[j] = t < 2 ? dq_step<false>(w0, w1, sc_lo[j], nc_lo[j]) : dq_step<true>(w0, w1, sc_hi[j], nc_hi[j]);
      }
      lds_wait(afn[0], afn[1], afn[2], afn[3]);
      lds_wait(afn[4], afn[5], afn[6], afn[7]);
#pragma unroll
      for (int i = 0; i < 8; ++i) af[i] = afn[i];
      if (t < 3) read_a(t + 1, afn);
#pragma unroll
      for (int q = 3 * t; q < (t < 3 ? 3 * t + 3 : kWCopies); ++q) issue_one(kn, sn, q);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i >> 2][i & 3][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, af[i]), bf[j],
                                                                         acc[i >> 2][i & 3][j], 0, 0, 0);
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

  // Epilogue: the wave's 256 x 64 tile in two 128-row halves through LDS,
  // wave w staging in slot array w once the tail's repeated copies have
  // landed and every wave has passed the barrier.
  wait_vmcnt<0>();
  wg_barrier();
  static_assert(32 * 72 * 4 <= kWSlotW && kWSlotW <= kWSlotA, "staging slice fits in a slot");
  uint8_t *sbase = wave == 0 ? sa0 : wave == 1 ? sa1 : wave == 2 ? sa2 : sw0;
#pragma unroll
  for (int h = 0; h < 2; ++h)
    store_c_tile<2>(acc[h], reinterpret_cast<float *>(sbase), c, M, N, m0 + 128 * h, n0 + 64 * wave, ea, ewc);
}

}  // namespace

hipError_t launch_q4k_gemm_wide(const _Float16 *a16, const int *ea, const HMats &mats, int M, int K, int tiles_n,
                                int ksplit, hipStream_t s) {
  const int tiles_m = (M + 255) / 256;
  hipLaunchKernelGGL(k_q4k_gemm_wide, dim3(tiles_m * tiles_n, ksplit), dim3(256), 0, s, a16, ea, mats, M, K, tiles_m,
                     tiles_n, ksplit);
  return hipGetLastError();
}

}  // namespace rt
