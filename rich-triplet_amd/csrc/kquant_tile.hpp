// kquant_tile.hpp -- the Q6_K and Q8_0 GEMV tiles on staged activation
// digits, shared by the stand-alone GEMVs (kquant.hip) and the decode step's
// fused launches (decode_kernels.hip): a Q6_K v projection beside Q4_K q and
// k rows, and the q|k|v and gate|up sets of a Q8_0 model, each on the input
// its own prologue normalises and stages.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kquant_layout.hpp"
#include "q4k_gemv.hpp"
#include "rt_device.hpp"

namespace rt {

// Slot s = threadIdx % S (S = 4*NB) of a row: block b = s/4, half
// j = (s/2)%2, a = s%2.  The slot owns l in [16a, 16a+16) of its half, i.e.
// the four 16-element sub-blocks 2m + a (m = 0..3) at elements
// 128j + 32m + 16a + [0, 16): ql[16a..] (m = 0, 2: low / high nibbles),
// ql[32+16a..] (m = 1, 3) and qh[16a..] (bit pair m), three 16-byte loads.
// A workgroup of T threads covers RPI = T/S rows per iteration, ROWS in all;
// per (row, block) the slot sums go to red[row * NB + block].
template <int NB, int T, int ITERS>
struct Q6KTile {
  static constexpr int S = 4 * NB, RPI = T / S, ROWS = RPI * ITERS;
  static_assert(T % S == 0 && T % 64 == 0, "a tile covers whole rows and whole waves");
  uint4 qa[ITERS], qb[ITERS], qh[ITERS];
  uint2 sc[ITERS];
  uint32_t dd[ITERS];

  RT_DEV static int slot() { return (int)threadIdx.x % S; }
  RT_DEV static int rsub() { return (int)threadIdx.x / S; }

  // Issues the weight loads of rows row0 .. row0 + ROWS - 1 of a matrix of n
  // rows (rows past n read row n - 1 and are never stored).
  RT_DEV void load(const Q6KPlanes &P, int row0, int n) {
    const int s = slot(), b = s >> 2, j = (s >> 1) & 1, a = s & 1;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const size_t blk = (size_t)min(row0 + it * RPI + rsub(), n - 1) * NB + b;
      qa[it] = *reinterpret_cast<const uint4 *>(P.ql + blk * 128 + 64 * j + 16 * a);
      qb[it] = *reinterpret_cast<const uint4 *>(P.ql + blk * 128 + 64 * j + 32 + 16 * a);
      qh[it] = *reinterpret_cast<const uint4 *>(P.qh + blk * 64 + 32 * j + 16 * a);
      sc[it] = *reinterpret_cast<const uint2 *>(P.sc + blk * 16 + 8 * j);
      dd[it] = P.d[blk];
    }
  }

  // Exact integer dot products of the codes against the staged digits in dl
  // (stage_digits_store layout), scaled per sub-block; red[ROWS * NB].
  RT_DEV void compute(const uint32_t *dl, float *red) const {
    const int s = slot(), b = s >> 2, j = (s >> 1) & 1, a = s & 1;
    // this slot's activation digits and 32 * sum(X) of each sub-block
    uint32_t x0[4][4];
    int x1[4][4], xs32[4];
    float delta[2];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t *p = dl + (4 * b + 2 * j + (m >> 1)) * kDPitch + 8 * (m & 1) + 4 * a;
      const uint4 u0 = *reinterpret_cast<const uint4 *>(p), u1 = *reinterpret_cast<const uint4 *>(p + 16);
      x0[m][0] = u0.x; x0[m][1] = u0.y; x0[m][2] = u0.z; x0[m][3] = u0.w;
      x1[m][0] = (int)u1.x; x1[m][1] = (int)u1.y; x1[m][2] = (int)u1.z; x1[m][3] = (int)u1.w;
      uint32_t s0 = 0;
      int s1 = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        s0 = __builtin_amdgcn_udot4(x0[m][k], 0x01010101u, s0, false);
        s1 = __builtin_amdgcn_sdot4(x1[m][k], 0x01010101, s1, false);
      }
      xs32[m] = 32 * ((int)s0 + 256 * s1);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) delta[h] = __uint_as_float(dl[(4 * b + 2 * j + h) * kDPitch + 32]);

    const uint32_t m4 = opaque_u32(0x0F0F0F0Fu), m2 = opaque_u32(0x30303030u);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const uint32_t lo[4] = {qa[it].x, qa[it].y, qa[it].z, qa[it].w};
      const uint32_t hi[4] = {qb[it].x, qb[it].y, qb[it].z, qb[it].w};
      const uint32_t hb[4] = {qh[it].x, qh[it].y, qh[it].z, qh[it].w};
      const uint32_t scw = a ? (sc[it].x >> 8) | (sc[it].y << 24) : sc[it].x;  // sc[a], sc[a+2] in bytes 0, 2
      const uint32_t scw2 = a ? sc[it].y >> 8 : sc[it].y;                        // sc[a+4], sc[a+6]
      float acc[2] = {0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        uint32_t s0 = 0;
        int s1 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t src = (m & 1) ? hi[k] : lo[k];
          const uint32_t nib = (m < 2 ? src : src >> 4) & m4;
          const int sh = 2 * m;  // bit pair m of qh moved to bits 4..5
          const uint32_t q = nib | ((sh <= 4 ? hb[k] << (4 - sh) : hb[k] >> (sh - 4)) & m2);
          s0 = __builtin_amdgcn_udot4(q, x0[m][k], s0, false);
          s1 = __builtin_amdgcn_sdot4((int)q, x1[m][k], s1, false);
        }
        const int t = (int)s0 + 256 * s1 - xs32[m];  // sum X (q - 32), exact
        const uint32_t word = m < 2 ? scw : scw2;
        const float scf = (float)(int)__builtin_amdgcn_sbfe(word, 16 * (m & 1), 8);
        acc[m >> 1] = fmaf(scf, (float)t, acc[m >> 1]);
      }
      float p = half_bits_to_f32(dd[it]) * fmaf(acc[1], delta[1], acc[0] * delta[0]);
      p = quad_sum(p);
      if ((s & 3) == 0) red[(it * RPI + rsub()) * NB + b] = p;
    }
  }
};

// Q8_0 tile on staged digits.  Slot s = threadIdx % S (S = NB32, the
// 32-element blocks of a row) owns block s of RPI = T/S rows per iteration:
// its 32 code bytes (two 16-byte loads) and its f16 scale.  q is signed; with
// q' = q ^ 0x80 = q + 128 unsigned, sum x0 q = sum x0 q' - 128 sum x0, so both
// digits run on v_dot4 forms of matching signedness.  Per (row, 64-element
// chunk) the pair of block sums goes to red[row * RED + chunk].
template <int NB32, int T, int ITERS>
struct Q8Tile {
  static constexpr int S = NB32, RPI = T / S, ROWS = RPI * ITERS, RED = (NB32 + 1) / 2;
  static_assert(T % S == 0 && T % 64 == 0 && S % 2 == 0, "a tile covers whole rows and whole waves");
  uint4 qa[ITERS], qb[ITERS];
  uint32_t dd[ITERS];

  RT_DEV static int slot() { return (int)threadIdx.x % S; }
  RT_DEV static int rsub() { return (int)threadIdx.x / S; }

  // rowq(rl) / rowd(rl): the code bytes and the f16 scales of tile row rl.
  template <typename RowQ, typename RowD>
  RT_DEV void load(RowQ rowq, RowD rowd) {
    const int s = slot();
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int rl = it * RPI + rsub();
      const uint8_t *p = rowq(rl) + 32 * s;
      qa[it] = *reinterpret_cast<const uint4 *>(p);
      qb[it] = *reinterpret_cast<const uint4 *>(p + 16);
      dd[it] = rowd(rl)[s];
    }
  }

  RT_DEV void compute(const uint32_t *dl, float *red) const {
    const int s = slot();
    uint32_t x0[8];
    int x1[8];
    const uint32_t *px = dl + (s >> 1) * kDPitch + 8 * (s & 1);
    uint32_t sx0 = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x0[k] = px[k];
      x1[k] = (int)px[16 + k];
      sx0 = __builtin_amdgcn_udot4(x0[k], 0x01010101u, sx0, false);
    }
    const int corr = 128 * (int)sx0;
    const float delta = __uint_as_float(dl[(s >> 1) * kDPitch + 32]);
    const uint32_t flip = opaque_u32(0x80808080u);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const uint32_t w[8] = {qa[it].x, qa[it].y, qa[it].z, qa[it].w, qb[it].x, qb[it].y, qb[it].z, qb[it].w};
      uint32_t s0 = 0;
      int s1 = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        s0 = __builtin_amdgcn_udot4(w[k] ^ flip, x0[k], s0, false);
        s1 = __builtin_amdgcn_sdot4((int)w[k], x1[k], s1, false);
      }
      // sum X q = (sum x0 q' - 128 sum x0) + 256 sum x1 q; |.| < 2^31
      const int t = (int)(s0 - (uint32_t)corr) + 256 * s1;
      float p = half_bits_to_f32(dd[it]) * delta * (float)t;
      p += dpp<0xB1>(p);  // pair of blocks = one 64-element chunk
      if ((s & 1) == 0) red[(it * RPI + rsub()) * RED + (s >> 1)] = p;
    }
  }

  // y of tile row rl from its chunk sums (chunk order)
  RT_DEV static float reduce(const float *red, int rl) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < RED; ++c) acc += red[rl * RED + c];
    return acc;
  }
};

}  // namespace rt
