// kquant_layout.hpp -- the planar device layouts of Q6_K and Q8_0 weights and
// the decode of one element (bit-exact with decode_q6k_to_f32 /
// decode_q8_0_to_f32, gguf_loader.rs:482-549 and 628-650: s = d * sc in f32,
// then s * q).
//   Q6_K, nbt blocks of 256: ql [nbt][128] | qh [nbt][64] | sc [nbt][16] | d [nbt] f16
//   Q8_0, n elements:        q [n] int8 | d [n/32] f16
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "rt_device.hpp"

namespace rt {

constexpr int kQ6KBlockBytes = 210;
constexpr int kQ8Block = 32, kQ8BlockBytes = 34;

struct Q6KPlanes {
  const uint8_t *ql, *qh;
  const uint8_t *sc;
  const uint16_t *d;
};

__host__ __device__ inline Q6KPlanes q6k_planes(const void *w, size_t nbt) {
  const uint8_t *p = static_cast<const uint8_t *>(w);
  return {p, p + nbt * 128, p + nbt * 192, reinterpret_cast<const uint16_t *>(p + nbt * 208)};
}

// Element i (0..255) of block blk: half j = i/128, h = i%128, quarter m = h/32,
// l = h%32; 6-bit code = ql nibble (low for m < 2) | qh bit pair m << 4, minus 32.
RT_DEV float q6k_value(const Q6KPlanes &P, size_t blk, int i) {
#pragma clang fp contract(off)
  const int j = i >> 7, h = i & 127, m = h >> 5, l = h & 31;
  const uint8_t ql = P.ql[blk * 128 + 64 * j + 32 * (m & 1) + l];
  const uint8_t qh = P.qh[blk * 64 + 32 * j + l];
  const int q = (int)(((m < 2 ? ql & 15 : ql >> 4)) | (((qh >> (2 * m)) & 3) << 4)) - 32;
  const float d = half_bits_to_f32(P.d[blk]);
  const float s = d * (float)(int8_t)P.sc[blk * 16 + 8 * j + (l >> 4) + 2 * m];
  return s * (float)q;
}

// Element e of a planar Q8_0 tensor of n_elem elements.
RT_DEV float q8_0_value(const uint8_t *w, size_t n_elem, size_t e) {
#pragma clang fp contract(off)
  const uint16_t *D = reinterpret_cast<const uint16_t *>(w + n_elem);
  return half_bits_to_f32(D[e / kQ8Block]) * (float)(int8_t)w[e];
}

}  // namespace rt
