// q4k_gemv.hpp -- device building blocks of the Q4_K GEMV (standalone and
// fused into the decode-step kernels).
//
// Work split ("column resident"): a workgroup of T threads owns ROWS
// consecutive output rows.  Thread t owns chunk slot s = t % S (S = 4*NB
// 64-element chunks per row: super-block b = s/4, chunk c = s%4) and visits
// rows rsub, rsub+RPI, ... (rsub = t / S, RPI = T / S).  Per row it loads the
// 16-byte super-block header and its 32 nibble bytes (three 16-byte loads, the
// four chunk lanes of a block read one contiguous 144-byte block), and keeps
// the matching 64 activations in registers for all rows it visits.  The
// activations are staged once per workgroup through LDS.
//
// Every load of the ITERS row-iterations is issued before any arithmetic so a
// workgroup has all of its weights in flight at once.
#pragma once

#include "rt_device.hpp"

namespace rt {

// LDS layout of a staged activation vector: chunk slot s occupies floats
// [s*kXPitch, s*kXPitch + 64), followed by the sums of its low and high
// halves (the per-sub-block sum(a) of the integer trick) at +64 and +65.
// The pitch of 68 floats keeps slots 16-byte aligned and puts the eight lanes
// of a ds_read_b128 phase on distinct banks.
constexpr int kXPitch = 68;
RT_DEV int xlds_index(int e) { return (e >> 6) * kXPitch + (e & 63); }

struct ChunkX {
  float lo[32], hi[32];
  float sum_lo, sum_hi;
};

RT_DEV void chunkx_from_lds(const float *xl, int slot, ChunkX &x) {
  const float4 *p = reinterpret_cast<const float4 *>(xl + slot * kXPitch);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 v = p[i];
    x.lo[4 * i] = v.x; x.lo[4 * i + 1] = v.y; x.lo[4 * i + 2] = v.z; x.lo[4 * i + 3] = v.w;
    const float4 u = p[8 + i];
    x.hi[4 * i] = u.x; x.hi[4 * i + 1] = u.y; x.hi[4 * i + 2] = u.z; x.hi[4 * i + 3] = u.w;
  }
  const float4 sums = p[16];
  x.sum_lo = sums.x;
  x.sum_hi = sums.y;
}

// Store one float4 of the staged vector (element 4f..4f+3) and, from the 16
// lanes that hold one chunk, the sums of its two 32-element halves.  Lanes
// f..f+15 of a chunk must be consecutive lanes of one wave (f = tid + i*T with
// T a multiple of 16).
RT_DEV void stage_x_store(float *xl, int f, float4 v) {
  *reinterpret_cast<float4 *>(xl + xlds_index(4 * f)) = v;
  float s = (v.x + v.y) + (v.z + v.w);
  s += dpp<0xB1>(s);   // quad
  s += dpp<0x4E>(s);
  s += dpp<0x141>(s);  // half row: 8 lanes = 32 elements
  const int sub = f & 15;
  if (sub == 0) xl[(f >> 4) * kXPitch + 64] = s;
  if (sub == 8) xl[(f >> 4) * kXPitch + 65] = s;
}

// Activation staging in two halves so the global loads of x can be issued
// before the weight loads (x_load) and consumed after them (x_store): the
// s_waitcnt for x then leaves every weight load in flight.
template <int K, int T>
struct XRegs {
  static constexpr int PER = (K / 4 + T - 1) / T;
  float4 v[PER];
};

template <int K, int T>
RT_DEV void x_load(const float *__restrict__ x, XRegs<K, T> &r) {
  static_assert(T % 16 == 0 && (K / 4) % 16 == 0, "chunk lanes must be whole DPP rows");
#pragma unroll
  for (int i = 0; i < XRegs<K, T>::PER; ++i) {
    const int f = min((int)threadIdx.x + i * T, K / 4 - 1);  // clamped, unconditional 16-byte load
    r.v[i] = reinterpret_cast<const float4 *>(x)[f];
  }
}

template <int K, int T>
RT_DEV void x_store(const XRegs<K, T> &r, float *xl) {
#pragma unroll
  for (int i = 0; i < XRegs<K, T>::PER; ++i) {
    const int f = threadIdx.x + i * T;
    if (f < K / 4) stage_x_store(xl, f, r.v[i]);
  }
}

// Dot of one 64-element chunk against resident activations with the
// reference's integer trick, per sub-block: scale*sum(q*a) - min*sum(a)
// (autograd2.rs:1671-1698).  High nibbles are converted as 16*q straight from
// the byte (exact) and the 1/16 folds into the scale.
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


// ---------------------------------------------------------------------------
// Integer-digit variant of the chunk dot.  Each 64-element activation chunk is
// scaled by a power of two to 16-bit integers X = rint(x * 2^sh) (sh = 15 - e
// with the chunk's max |x| < 2^e; the one value that can round to 2^15 is
// clamped to 2^15 - 1), written as two bytes, X = 256*x1 + x0 (x0 in 0..255,
// x1 in -128..127).  The nibble-by-digit products then run on v_dot4_u32_u8
// (x0) and v_dot4_i32_i8 (x1) in exact integer arithmetic:
//   sum_k q_k X_k = d0 + 256 d1,  d_i = sum_k q_k x_i,k,
// and d0 + 256 d1 (< 2^24 over 32 elements) converts to f32 exactly.  The only
// roundings are X (half a unit of 2^-15 of the chunk's bound 2^e) and the final
// f32 combine: about 3e-5 rel-L2 on N(0,1) activations.
// Staging costs about five lane-ops per element: the rounding is one FMA,
// x * 2^sh + 1.5*2^23, whose low 16 mantissa bits are X in two's complement,
// and four byte permutes pack the digits of four elements.
// ---------------------------------------------------------------------------
constexpr int kDPitch = 36;  // dwords per slot: 2 digits x 16 dwords, delta, sum_lo, sum_hi, pad

struct ChunkD {
  uint32_t d0[16];
  int32_t d1[16];
  float delta, sum_lo, sum_hi;
};

// Stage one float4 (elements 4f..4f+3) as digits; the 16 lanes of a chunk
// (consecutive lanes of one wave) agree on the chunk's power-of-two scale.
RT_DEV void stage_digits_store(uint32_t *dl, int f, float4 v) {
  // max |x| over the chunk on the bit patterns (monotone for |x|, no NaN
  // canonicalisation between the DPP steps)
  const uint32_t ax = f32_bits(v.x) & 0x7FFFFFFFu, ay = f32_bits(v.y) & 0x7FFFFFFFu;
  const uint32_t az = f32_bits(v.z) & 0x7FFFFFFFu, aw = f32_bits(v.w) & 0x7FFFFFFFu;
  uint32_t mb = max(max(ax, ay), max(az, aw));
  mb = max(mb, dpp_u32<0xB1>(mb));
  mb = max(mb, dpp_u32<0x4E>(mb));
  mb = max(mb, dpp_u32<0x141>(mb));
  mb = max(mb, dpp_u32<0x140>(mb));
  // max < 2^e with e = biased exponent - 126; sh = 15 - e keeps |X| <= 2^15.
  // 2^sh must be a normal float: chunks with max |x| below 2^-111 lose
  // precision (their digits shrink toward zero) instead of overflowing.
  const int sh = min(141 - (int)(mb >> 23), 126);
  const float scale = __int_as_float((127 + sh) << 23);
  const float magic = 12582912.0f;  // 1.5 * 2^23: the sum's low mantissa bits hold rint(x * 2^sh)
  constexpr uint32_t top = 0x4B400000u + 32767u;  // bits of magic + (2^15 - 1)
  const uint32_t b0 = min(__float_as_uint(fmaf(v.x, scale, magic)), top);
  const uint32_t b1 = min(__float_as_uint(fmaf(v.y, scale, magic)), top);
  const uint32_t b2 = min(__float_as_uint(fmaf(v.z, scale, magic)), top);
  const uint32_t b3 = min(__float_as_uint(fmaf(v.w, scale, magic)), top);
  const uint32_t p01 = __builtin_amdgcn_perm(b1, b0, 0x05010400u);  // b0.0 b1.0 b0.1 b1.1
  const uint32_t p23 = __builtin_amdgcn_perm(b3, b2, 0x05010400u);  // b2.0 b3.0 b2.1 b3.1
  const int slot = f >> 4, sub = f & 15;
  uint32_t *base = dl + slot * kDPitch;
  base[sub] = __builtin_amdgcn_perm(p23, p01, 0x05040100u);       // low bytes:  x0 of 4 elements
  base[16 + sub] = __builtin_amdgcn_perm(p23, p01, 0x07060302u);  // high bytes: x1 of 4 elements
  float s = (v.x + v.y) + (v.z + v.w);
  s += dpp<0xB1>(s);
  s += dpp<0x4E>(s);
  s += dpp<0x141>(s);  // 8 lanes = 32 elements
  if (sub == 0) {
    reinterpret_cast<float *>(base)[32] = __int_as_float((127 - sh) << 23);  // 2^-sh
    reinterpret_cast<float *>(base)[33] = s;
  }
  if (sub == 8) reinterpret_cast<float *>(base)[34] = s;
}

template <int K, int T>
RT_DEV void x_store_digits(const XRegs<K, T> &r, uint32_t *dl) {
#pragma unroll
  for (int i = 0; i < XRegs<K, T>::PER; ++i) {
    const int f = threadIdx.x + i * T;
    if (f < K / 4) stage_digits_store(dl, f, r.v[i]);
  }
}

RT_DEV void chunkd_from_lds(const uint32_t *dl, int slot, ChunkD &x) {
  const uint4 *p = reinterpret_cast<const uint4 *>(dl + slot * kDPitch);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 a = p[i], b = p[4 + i];
    x.d0[4 * i] = a.x; x.d0[4 * i + 1] = a.y; x.d0[4 * i + 2] = a.z; x.d0[4 * i + 3] = a.w;
    x.d1[4 * i] = (int)b.x; x.d1[4 * i + 1] = (int)b.y; x.d1[4 * i + 2] = (int)b.z; x.d1[4 * i + 3] = (int)b.w;
  }
  const float4 f = reinterpret_cast<const float4 *>(dl + slot * kDPitch)[8];
  x.delta = f.x;
  x.sum_lo = f.y;
  x.sum_hi = f.z;
}

// Scales and mins of sub-blocks 2c and 2c+1 (get_scale_min_k4 of the
// reference, quants.rs) as two bytes each: svp = sv(2c) | sv(2c+1) << 8,
// mvp likewise.  The two sub-blocks share one byte pair of each scale word.
RT_DEV void q4k_scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, int c, uint32_t &svp, uint32_t &mvp) {
  const int sh = (c & 1) * 16;
  const uint32_t a = __builtin_amdgcn_ubfe(s0, sh, 16);  // sc[j], sc[j+1]          (j = 2c mod 4)
  const uint32_t b = __builtin_amdgcn_ubfe(s1, sh, 16);  // sc[j+4], sc[j+5]
  const uint32_t d = __builtin_amdgcn_ubfe(s2, sh, 16);  // sc[j+8], sc[j+9]
  // both layouts, then a select (lanes of one wave hold different c)
  const uint32_t sv_lo = a & 0x3F3Fu, mv_lo = b & 0x3F3Fu;
  const uint32_t sv_hi = (d & 0x0F0Fu) | ((a >> 2) & 0x3030u);
  const uint32_t mv_hi = ((d >> 4) & 0x0F0Fu) | ((b >> 2) & 0x3030u);
  svp = c < 2 ? sv_lo : sv_hi;
  mvp = c < 2 ? mv_lo : mv_hi;
}

// f32 combine of one chunk's exact integer sums (low digit l0/h0, high digit
// l1/h1 of the low and high 32-element halves) with the block's scales.
RT_DEV float q4k_digits_combine(const uint4 hd, int c, uint32_t l0, int l1, uint32_t h0, int h1, float delta,
                                float sum_lo, float sum_hi) {
  const float d = half_bits_to_f32(hd.x & 0xFFFFu);
  const float dm = half_bits_to_f32(hd.x >> 16);
  uint32_t svp, mvp;
  q4k_scale_min_pair(hd.y, hd.z, hd.w, c, svp, mvp);
  const float dot_lo = fmaf((float)l1, 256.0f, (float)l0);  // exact: |value| < 2^24
  const float dot_hi = fmaf((float)h1, 256.0f, (float)h0);
  const float sv1 = (float)(svp & 0xFFu), sv2 = (float)(svp >> 8);
  const float mv1 = (float)(mvp & 0xFFu), mv2 = (float)(mvp >> 8);
  const float qsum = fmaf(sv2, dot_hi, sv1 * dot_lo);
  const float msum = fmaf(mv2, sum_hi, mv1 * sum_lo);
  return fmaf(d * delta, qsum, -(dm * msum));
}

RT_DEV float q4k_chunk_dot_digits(const uint4 hd, const uint4 qa, const uint4 qb, int c, const ChunkD &x,
                                  uint32_t m4) {
  const float d = half_bits_to_f32(hd.x & 0xFFFFu);
  const float dm = half_bits_to_f32(hd.x >> 16);
  uint32_t svp, mvp;
  q4k_scale_min_pair(hd.y, hd.z, hd.w, c, svp, mvp);
  const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  uint32_t l0 = 0, h0 = 0;
  int l1 = 0, h1 = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = w[i] & m4;         // nibbles of elements 4i..4i+3 (low half of the chunk)
    const uint32_t hi = (w[i] >> 4) & m4;  // elements 32+4i..32+4i+3
    l0 = __builtin_amdgcn_udot4(lo, x.d0[i], l0, false);
    l1 = __builtin_amdgcn_sdot4((int)lo, x.d1[i], l1, false);
    h0 = __builtin_amdgcn_udot4(hi, x.d0[8 + i], h0, false);
    h1 = __builtin_amdgcn_sdot4((int)hi, x.d1[8 + i], h1, false);
  }
  const float dot_lo = fmaf((float)l1, 256.0f, (float)l0);  // exact: |value| < 2^24
  const float dot_hi = fmaf((float)h1, 256.0f, (float)h0);
  const float sv1 = (float)(svp & 0xFFu), sv2 = (float)(svp >> 8);
  const float mv1 = (float)(mvp & 0xFFu), mv2 = (float)(mvp >> 8);
  const float qsum = fmaf(sv2, dot_hi, sv1 * dot_lo);
  const float msum = fmaf(mv2, x.sum_hi, mv1 * x.sum_lo);
  return fmaf(d * x.delta, qsum, -(dm * msum));
}

template <int NB, int T, int ITERS>
struct Q4KTile {
  static constexpr int S = NB * 4;
  static constexpr int RPI = T / S;
  static constexpr int ROWS = RPI * ITERS;
  static constexpr int kThreads = T, kIters = ITERS;
  static_assert(T % S == 0 && T % 64 == 0, "a tile covers whole rows and whole waves");

  int slot, rsub, b, c;
  bool valid[ITERS];
  uint4 hd[ITERS], qa[ITERS], qb[ITERS];

  RT_DEV Q4KTile() {
    slot = (int)threadIdx.x % S;
    rsub = (int)threadIdx.x / S;
    b = slot >> 2;
    c = slot & 3;
  }

  // rowptr(rl) -> start of local row rl's blocks, or nullptr past the end.
  // The loads themselves are unconditional (a row past the end re-reads
  // `fallback`, a valid row, and is masked out of the result): branch-free
  // loads let the compiler wait for exactly the loads an iteration needs.
  template <class RowPtr>
  RT_DEV void load(RowPtr rowptr, const uint8_t *fallback) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const uint8_t *row = rowptr(it * RPI + rsub);
      valid[it] = row != nullptr;
      const uint8_t *bp = (row ? row : fallback) + (size_t)b * kQ4KBlockBytes;
      hd[it] = *reinterpret_cast<const uint4 *>(bp);
      qa[it] = *reinterpret_cast<const uint4 *>(bp + 16 + 32 * c);
      qb[it] = *reinterpret_cast<const uint4 *>(bp + 32 + 32 * c);
    }
  }

  // Same with digit-staged activations.
  RT_DEV void compute_digits(const ChunkD &x, float *red) {
    const uint32_t m4 = opaque_u32(0x0F0F0F0Fu);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      float p = q4k_chunk_dot_digits(hd[it], qa[it], qb[it], c, x, m4);
      p = quad_sum(p);
      if (c == 0 && valid[it]) red[(it * RPI + rsub) * NB + b] = p;
    }
  }

  // compute_digits with the digit words read from LDS four at a time and
  // applied to every iteration's nibbles before the next four: 16 digit
  // registers live instead of 35, for tiles with several iterations.
  RT_DEV void compute_digits_lds(const uint32_t *dl, float *red) {
    const uint32_t m4 = opaque_u32(0x0F0F0F0Fu);
    const uint32_t *base = dl + slot * kDPitch;
    uint32_t l0[ITERS], h0[ITERS];
    int l1[ITERS], h1[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) l0[it] = h0[it] = 0u, l1[it] = h1[it] = 0;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const uint4 a0 = *reinterpret_cast<const uint4 *>(base + 4 * g);       // x0 of low-half words 4g..4g+3
      const uint4 b0 = *reinterpret_cast<const uint4 *>(base + 8 + 4 * g);   // x0 of high-half words
      const uint4 a1 = *reinterpret_cast<const uint4 *>(base + 16 + 4 * g);  // x1 of low-half words
      const uint4 b1 = *reinterpret_cast<const uint4 *>(base + 24 + 4 * g);  // x1 of high-half words
      const uint32_t A0[4] = {a0.x, a0.y, a0.z, a0.w}, B0[4] = {b0.x, b0.y, b0.z, b0.w};
      const uint32_t A1[4] = {a1.x, a1.y, a1.z, a1.w}, B1[4] = {b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        const uint4 q = g ? qb[it] : qa[it];
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t lo = w[j] & m4, hi = (w[j] >> 4) & m4;
          l0[it] = __builtin_amdgcn_udot4(lo, A0[j], l0[it], false);
          l1[it] = __builtin_amdgcn_sdot4((int)lo, (int)A1[j], l1[it], false);
          h0[it] = __builtin_amdgcn_udot4(hi, B0[j], h0[it], false);
          h1[it] = __builtin_amdgcn_sdot4((int)hi, (int)B1[j], h1[it], false);
        }
      }
    }
    const float4 f = *reinterpret_cast<const float4 *>(base + 32);  // delta, sum_lo, sum_hi
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      float p = q4k_digits_combine(hd[it], c, l0[it], l1[it], h0[it], h1[it], f.x, f.y, f.z);
      p = quad_sum(p);
      if (c == 0 && valid[it]) red[(it * RPI + rsub) * NB + b] = p;
    }
  }

  // Per-(row, super-block) partial sums into red[rl * NB + b].
  RT_DEV void compute(const ChunkX &x, float *red) {
    const uint32_t mlo = opaque_u32(0x0F0F0F0Fu), mhi = opaque_u32(0xF0F0F0F0u);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      float p = q4k_chunk_dot(hd[it], qa[it], qb[it], c, x, mlo, mhi);
      p = quad_sum(p);
      if (c == 0 && valid[it]) red[(it * RPI + rsub) * NB + b] = p;
    }
  }
};

// Sum of one row's NB block partials, in block order.
template <int NB>
RT_DEV float reduce_row(const float *red, int rl) {
  float s = 0.f;
#pragma unroll
  for (int b = 0; b < NB; ++b) s += red[rl * NB + b];
  return s;
}

}  // namespace rt
