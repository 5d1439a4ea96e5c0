// rt_device.hpp -- device-side helpers shared by every rich-triplet HIP kernel.
//
// gfx950 (CDNA4) only: wave64, DPP cross-lane adds, 16-byte vector loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define RT_DEV __device__ __forceinline__

namespace rt {

constexpr int kQ4KBlockBytes = 144;  // f16 d, f16 dmin, 12 B scales, 128 B nibbles
constexpr int kQ4KBlockElems = 256;

RT_DEV float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
RT_DEV uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

// IEEE half -> float.  v_cvt_f32_f16 is exact for every finite half,
// subnormals included (f16 denormals are preserved in the default FP mode).
RT_DEV float half_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// Nibble masks the compiler cannot see through.  With a literal mask the
// combiner folds `(w & 0x0F0F0F0F) >> 8 & 0xFF` into v_bfe_u32 and then needs a
// second instruction to convert; with an opaque mask every byte converts with
// one v_cvt_f32_ubyte{0..3}.
RT_DEV uint32_t opaque_u32(uint32_t v) {
  asm volatile("" : "+s"(v));
  return v;
}
// A 16-byte vector load of data a launch reads once (weights), with the
// nontemporal hint: streaming reads reach 8-10% more HBM bandwidth with it.
RT_DEV uint4 ld_nt16(const void *p) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load(static_cast<const v4u *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
RT_DEV float ubyte0(uint32_t v) { return (float)(v & 0xFFu); }
RT_DEV float ubyte1(uint32_t v) { return (float)((v >> 8) & 0xFFu); }
RT_DEV float ubyte2(uint32_t v) { return (float)((v >> 16) & 0xFFu); }
RT_DEV float ubyte3(uint32_t v) { return (float)(v >> 24); }

// Power-of-two exponent e with 2^-e * bound in [2^14, 2^15): values scaled by
// 2^-e fit f16 without overflow.  0 for zero / non-finite bounds (those propagate).
RT_DEV int f16_exponent_for(float bound) {
  if (!(bound > 0.f) || !__builtin_isfinite(bound)) return 0;
  int E;
  (void)frexpf(bound, &E);  // bound = f * 2^E, f in [0.5, 1)
  return E - 15;
}

RT_DEV float bf16_lo(uint32_t pair) { return bits_f32(pair << 16); }
RT_DEV float bf16_hi(uint32_t pair) { return bits_f32(pair & 0xFFFF0000u); }

// RNE float -> bf16 bits, NaN keeps a set quiet bit (same rule as the host).
RT_DEV uint16_t f32_to_bf16_bits(float v) {
  uint32_t b = f32_bits(v);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x0040u);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// Byte i (0..11) of the 12-byte scale field held in three dwords.
RT_DEV uint32_t sc_byte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
  uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
  return (w >> (8 * (i & 3))) & 0xFFu;
}

// 6-bit scale / min of sub-block j (0..7), Q4_K "get_scale_min_k4" packing:
//   j < 4 : sv = sc[j] & 63,                 mv = sc[j+4] & 63
//   j >= 4: sv = (sc[j+4] & 15) | (sc[j-4] >> 6) << 4,
//           mv = (sc[j+4] >> 4) | (sc[j]   >> 6) << 4
// Branch-free in j so lanes of one wave may ask for different sub-blocks.
RT_DEV void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, uint32_t &sv, uint32_t &mv) {
  // j < 4 path
  uint32_t a = (s0 >> (8 * (j & 3))) & 0xFFu;        // sc[j]      (j<4)
  uint32_t b = (s1 >> (8 * (j & 3))) & 0xFFu;        // sc[j+4]    (j<4) == sc[j] (j>=4)
  uint32_t c = (s2 >> (8 * (j & 3))) & 0xFFu;        // sc[j+4]    (j>=4)
  uint32_t sv_lo = a & 63u, mv_lo = b & 63u;
  uint32_t sv_hi = (c & 15u) | ((a >> 6) << 4);      // sc[j-4] == a for j>=4
  uint32_t mv_hi = (c >> 4) | ((b >> 6) << 4);       // sc[j]   == b for j>=4
  bool lo = j < 4;
  sv = lo ? sv_lo : sv_hi;
  mv = lo ? mv_lo : mv_hi;
}

// ---------------------------------------------------------------------------
// Cross-lane sums (DPP).  Masks follow the GCN/CDNA DPP control encoding.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF, bool BOUND = false>
RT_DEV float dpp(float v) {
  return bits_f32((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f32_bits(v), CTRL, ROW_MASK, BANK_MASK, BOUND));
}

template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF, bool BOUND = false>
RT_DEV uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, BANK_MASK, BOUND);
}

// Sum over aligned groups of 4 lanes; every lane of the group gets the sum.
RT_DEV float quad_sum(float v) {
  v += dpp<0xB1>(v);  // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);  // quad_perm [2,3,0,1]
  return v;
}

// Sum over aligned groups of 16 lanes (a DPP row); every lane gets the sum.
RT_DEV float row16_sum(float v) {
  v = quad_sum(v);
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return v;
}

// Sum over the whole wave64; the result is returned to every lane.
RT_DEV float wave_sum(float v) {
  v = row16_sum(v);
  v += dpp<0x142, 0xA>(v);  // row_bcast15 into rows 1 and 3
  v += dpp<0x143, 0xC>(v);  // row_bcast31 into rows 2 and 3
  return bits_f32((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(v), 63));
}

RT_DEV float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  // rows 0 and 2 receive 0 from the masked broadcast; combine with readlanes instead
  float r0 = bits_f32((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(v), 0));
  float r1 = bits_f32((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(v), 16));
  float r2 = bits_f32((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(v), 32));
  float r3 = bits_f32((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Block-wide sum for blockDim.x == NT (multiple of 64).  `red` needs NT/64 floats.
template <int NT>
RT_DEV float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red may still be read from a previous call
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) s += red[i];
  return s;
}

// block_sum into `red` that no earlier call in the kernel reads (a fresh
// array per reduction): the barrier that protects a reused array is not needed.
template <int NT>
RT_DEV float block_sum_fresh(float v, float *red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) s += red[i];
  return s;
}

template <int NT>
RT_DEV float block_max(float v, float *red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red may still be read from a previous call
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) m = fmaxf(m, red[i]);
  return m;
}

// Four values of a GEMM A row as f16 scaled by 2^-e (e = f16_exponent_for of
// the row's max |x|, the GEMM's A preparation), packed for one 8-byte store.
RT_DEV uint2 f16x4_scaled(float4 v, int e) {
  auto hb = [](float x, int ex) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)__builtin_amdgcn_ldexpf(x, -ex)); };
  return make_uint2(hb(v.x, e) | (hb(v.y, e) << 16), hb(v.z, e) | (hb(v.w, e) << 16));
}

// 0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3)))   (autograd2.rs:3082-3091)
// with tanh(y) = 1 - 2 / (e^(2y) + 1): e^(2y) = 2^(2y log2(e)) by v_exp_f32
// and the quotient by v_rcp_f32, about 1 ulp each: six VALU operations
// where a libm tanhf takes about forty.  Against the same expression on
// glibc's tanhf it differs by at most (|v| + |y|) 2^-23 over [-40, 40], and
// not at all where tanh saturates (|v| >= 6: e^(2y) overflows to +inf or
// falls below 2^-25, so t is exactly +1 or -1); +-inf and NaN behave as with
// tanhf.
RT_DEV float gelu_tanh(float v) {
  const float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  const float e2y = __builtin_amdgcn_exp2f(inner * 2.8853900817779268f);
  const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + e2y);
  return v * 0.5f * (1.0f + t);
}

}  // namespace rt
