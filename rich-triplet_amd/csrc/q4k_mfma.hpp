// q4k_mfma.hpp -- Q4_K GEMV building blocks on the int8 matrix cores
// (v_mfma_i32_16x16x64_i8).
//
// Replaces the reference's per-row dot of quants.rs / autograd2.rs:1671-1698
// (sum over sub-blocks of scale*sum(q*a) - min*sum(a)) for one decode token.
//
// Activations.  Each 64-element chunk (one Q4_K chunk: sub-blocks 2g, 2g+1 of
// a super-block) is scaled to integers X = rint(x * s), s = 32639 / 2^e with
// max |x| < 2^e, so |X| <= 32639, and written as two balanced signed bytes,
// X = 256*x1 + x0 (x0, x1 in -128..127).  The rounding is one FMA,
// x*s + (1.5*2^23 + 128): the low 16 mantissa bits of the sum are X + 128.
//
// Product.  A wave owns 16 rows.  Per super-block it issues four MFMAs
// (t = 0..3) into one 16x16 int32 accumulator C[m][n]:
//   B (weights): lane (n = l%16, g = l/16) holds row n's qs bytes
//     32g + 8t + [0,8) as 16 int8 nibbles: 8 low nibbles (sub-block 2g,
//     elements 8t..8t+7), then the 8 high nibbles (sub-block 2g+1).
//   A (activations): row m = 4c + 2h + d (chunk c, half h, digit d) is the
//     digit d of the matching elements where the k-slot belongs to chunk c and
//     half h, zero elsewhere.  Only lanes with (l%16)/4 == l/16 are non-zero;
//     they read their 16 bytes from LDS, the others keep zero registers.
// so that lane (n, g) receives in C[j] (j = 2h + d) the exact integer
// sum over sub-block 2g+h of q * x_d.  The epilogue applies that row's scales:
//   acc += d*delta*(sv_lo*(256 C1 + C0) + sv_hi*(256 C3 + C2))
//          - dmin*(mv_lo*sum_lo + mv_hi*sum_hi)
// with sum_lo/hi the f32 sums of x over the two sub-blocks.  About 0.9 VALU
// lane-ops per weight against 1.6 for the v_dot4 path.
#pragma once

#include "q4k_gemv.hpp"

namespace rt {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t mxu4 __attribute__((ext_vector_type(4)));

// LDS image of the staged activations: per super-block b, 1 KB of A-operand
// units [t][g][d] of 32 bytes ([0,8): digits of sub-block 2g, [8,24): zero,
// [24,32): digits of sub-block 2g+1; a lane of half h reads bytes 16h..16h+15),
// then per (b, g) a float4 {delta, sum_lo, sum_hi, 0}.
constexpr int kMxSBBytes = 1024;

// Stage one float4 (elements 4f..4f+3 of x).  The 16 lanes of a 64-element
// chunk are consecutive lanes of one wave (f = tid + i*T with T % 16 == 0).
// Every lane runs the arithmetic (the DPP steps keep the x loads ahead of the
// weight loads: convergent operations cannot sink into a branch); only lanes
// with `store` write.
RT_DEV void stage_mfma_x(uint8_t *xa, float4 *xs, int f, float4 v, bool store) {
  const uint32_t ax = f32_bits(v.x) & 0x7FFFFFFFu, ay = f32_bits(v.y) & 0x7FFFFFFFu;
  const uint32_t az = f32_bits(v.z) & 0x7FFFFFFFu, aw = f32_bits(v.w) & 0x7FFFFFFFu;
  uint32_t mb = max(max(ax, ay), max(az, aw));
  mb = max(mb, dpp_u32<0xB1>(mb));
  mb = max(mb, dpp_u32<0x4E>(mb));
  mb = max(mb, dpp_u32<0x141>(mb));
  mb = max(mb, dpp_u32<0x140>(mb));
  // max < 2^e, e = biased exponent - 126.  s = 32639 * 2^-e must stay a
  // normal float: chunks whose max |x| is below 2^-111 lose precision
  // (their digits shrink toward zero) instead of overflowing.
  const int e = max((int)(mb >> 23) - 126, -111);
  const float s = bits_f32(f32_bits(32639.0f) - ((uint32_t)e << 23));
  const float delta = bits_f32(f32_bits(1.0f / 32639.0f) + ((uint32_t)e << 23));
  const float magic = 12583040.0f;  // 1.5*2^23 + 128
  const uint32_t b0 = f32_bits(fmaf(v.x, s, magic)), b1 = f32_bits(fmaf(v.y, s, magic));
  const uint32_t b2 = f32_bits(fmaf(v.z, s, magic)), b3 = f32_bits(fmaf(v.w, s, magic));
  const uint32_t p01 = __builtin_amdgcn_perm(b1, b0, 0x05010400u);  // b0.0 b1.0 b0.1 b1.1
  const uint32_t p23 = __builtin_amdgcn_perm(b3, b2, 0x05010400u);
  const uint32_t d0 = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;  // x0 = (X+128 mod 256) - 128
  const uint32_t d1 = __builtin_amdgcn_perm(p23, p01, 0x07060302u);                // x1
  const int chunk = f >> 4, b = chunk >> 2, g = chunk & 3, q = f & 15;
  const int h = q >> 3, t = (q & 7) >> 1, iw = q & 1;
  uint8_t *unit = xa + b * kMxSBBytes + (t * 4 + g) * 64;  // digit 0 unit; digit 1 at +32
  const int off = h ? 24 + 4 * iw : 4 * iw;
  const int zoff = h ? 16 + 4 * iw : 8 + 4 * iw;
  float sum = (v.x + v.y) + (v.z + v.w);
  sum += dpp<0xB1>(sum);
  sum += dpp<0x4E>(sum);
  sum += dpp<0x141>(sum);  // 8 lanes = one 32-element sub-block
  if (store) {
    *reinterpret_cast<uint32_t *>(unit + off) = d0;
    *reinterpret_cast<uint32_t *>(unit + zoff) = 0u;
    *reinterpret_cast<uint32_t *>(unit + 32 + off) = d1;
    *reinterpret_cast<uint32_t *>(unit + 32 + zoff) = 0u;
    float *st = reinterpret_cast<float *>(xs + chunk);
    if (q == 0) {
      st[0] = delta;
      st[1] = sum;
    }
    if (q == 8) st[2] = sum;
  }
}

// Also zeroes the 16-byte pad that inactive lanes read as their A operand.
template <int K, int T>
RT_DEV void x_store_mfma(const XRegs<K, T> &r, uint8_t *xa, float4 *xs) {
#pragma unroll
  for (int i = 0; i < XRegs<K, T>::PER; ++i) {
    const int f = threadIdx.x + i * T;
    stage_mfma_x(xa, xs, min(f, K / 4 - 1), r.v[i], f < K / 4);
  }
  if (threadIdx.x == 0) *reinterpret_cast<float4 *>(xa + (K / 256) * kMxSBBytes) = make_float4(0.f, 0.f, 0.f, 0.f);
}

// Weights of one super-block for lane (n, g): its 16-byte header and the 32 qs
// bytes of chunk g.
struct MxBlock {
  mxu4 hd, qa, qb;
};

RT_DEV void mx_load(const uint8_t *__restrict__ blk, int g, MxBlock &w) {
  w.hd = *reinterpret_cast<const mxu4 *>(blk);
  w.qa = *reinterpret_cast<const mxu4 *>(blk + 16 + 32 * g);
  w.qb = *reinterpret_cast<const mxu4 *>(blk + 32 + 32 * g);
}

// One super-block of one 16-row group: four MFMAs and the scale epilogue.
// a_addr: LDS byte address of this lane's t = 0 A operand for the super-block
// (a_step = 256 between t's); inactive lanes pass the zero pad with step 0.
RT_DEV float mx_superblock(const MxBlock &w, const uint8_t *lds, int a_addr, int a_step, const float4 *xs_sb,
                           int g, float acc) {
  const uint32_t m4 = 0x0F0F0F0Fu;
  const uint32_t q[8] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w};
  i32x4_t A[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) A[t] = *reinterpret_cast<const i32x4_t *>(lds + a_addr + t * a_step);
  i32x4_t C = {0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t w0 = q[2 * t], w1 = q[2 * t + 1];
    const i32x4_t B = {(int)(w0 & m4), (int)(w1 & m4), (int)((w0 >> 4) & m4), (int)((w1 >> 4) & m4)};
    C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[t], B, C, 0, 0, 0);
  }
  const float4 xs = xs_sb[g];  // delta, sum_lo, sum_hi
  const float d = half_bits_to_f32(w.hd.x & 0xFFFFu);
  const float dm = half_bits_to_f32(w.hd.x >> 16);
  uint32_t svp, mvp;
  q4k_scale_min_pair(w.hd.y, w.hd.z, w.hd.w, g, svp, mvp);
  const float dot_lo = fmaf((float)C[1], 256.0f, (float)C[0]);  // exact: |value| < 2^24
  const float dot_hi = fmaf((float)C[3], 256.0f, (float)C[2]);
  const float sv1 = (float)(svp & 0xFFu), sv2 = (float)(svp >> 8);
  const float mv1 = (float)(mvp & 0xFFu), mv2 = (float)(mvp >> 8);
  const float qsum = fmaf(sv2, dot_hi, sv1 * dot_lo);
  const float msum = fmaf(mv2, xs.z, mv1 * xs.y);
  return fmaf(d * xs.x, qsum, fmaf(-dm, msum, acc));
}

// Byte offset of lane l's A operand inside a super-block image (t = 0), and
// whether the lane carries data: lane (m = l%16, g = l/16) is row m = 4c+2h+d
// of A and is non-zero only for c == g.
RT_DEV int mx_a_offset(int lane) {
  const int m = lane & 15, g = lane >> 4;
  return (g * 2 + (m & 1)) * 32 + ((m >> 1) & 1) * 16;
}
RT_DEV bool mx_active(int lane) { return ((lane & 15) >> 2) == (lane >> 4); }

// Sum over the four lane groups (lanes n, n+16, n+32, n+48).
RT_DEV float mx_group_sum(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

}  // namespace rt
