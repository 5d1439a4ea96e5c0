// gemma3_math.hpp -- the per-element arithmetic of a Gemma-3 block, shared by
// the decode-step kernels and the prefill kernels so both round identically.
#pragma once

#include "rt_device.hpp"

namespace rt {

// rms_norm_gemma3 (autograd2.rs:3477-3496):
//   rinv = 1/sqrt(sum(x^2) * (1/K) + eps);  out = (x * rinv) * (1 + gamma)
RT_DEV float rms_inv_from_sumsq(float ss, float inv_k, float eps) {
#pragma clang fp contract(off)
  return 1.0f / sqrtf(ss * inv_k + eps);
}

RT_DEV float4 norm4(float4 x, float rinv, float4 g) {
#pragma clang fp contract(off)
  return make_float4((x.x * rinv) * (1.0f + g.x), (x.y * rinv) * (1.0f + g.y), (x.z * rinv) * (1.0f + g.z),
                     (x.w * rinv) * (1.0f + g.w));
}

RT_DEV float4 add4(float4 a, float4 b) {
#pragma clang fp contract(off)
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

RT_DEV float mul_nc(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

RT_DEV float sumsq4(float4 v) { return v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w; }

// Per-head RMSNorm (apply_per_head_norm, transformer4.rs:2485-2508, gamma
// shared by the heads) followed by NeoX RoPE (apply_rope_at_offset,
// 2742-2772) of one head of D values, by one wave.  Lane owns pairs
// i = lane*P + p (p < P) with partners i + D/2, held in x0[p] / x1[p];
// cs[i] = cos and cs[D/2 + i] = sin of the pair's angle.  The source may be
// dst: every lane has read its own elements before it writes them.
template <int D>
RT_DEV void norm_rope_head_regs(float (&x0)[D / 128], float (&x1)[D / 128], const float *__restrict__ gamma,
                                const float *__restrict__ cs, float eps, float *dst) {
  constexpr int P = D / 128;
  const int lane = threadIdx.x & 63;
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < P; ++p) ss += x0[p] * x0[p] + x1[p] * x1[p];
  const float rinv = rms_inv_from_sumsq(wave_sum(ss), 1.0f / (float)D, eps);
#pragma unroll
  for (int p = 0; p < P; ++p) {
#pragma clang fp contract(off)
    const int i = lane * P + p;
    const float a0 = (x0[p] * rinv) * (1.0f + gamma[i]);
    const float a1 = (x1[p] * rinv) * (1.0f + gamma[i + D / 2]);
    const float c = cs[i], sn = cs[D / 2 + i];
    dst[i] = a0 * c - a1 * sn;
    dst[i + D / 2] = a0 * sn + a1 * c;
  }
}

// The same with element i from src(i).
template <int D, class Load>
RT_DEV void norm_rope_head_ld(Load src, const float *__restrict__ gamma, const float *__restrict__ cs, float eps,
                              float *dst) {
  constexpr int P = D / 128;
  const int lane = threadIdx.x & 63;
  float x0[P], x1[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int i = lane * P + p;
    x0[p] = src(i);
    x1[p] = src(i + D / 2);
  }
  norm_rope_head_regs<D>(x0, x1, gamma, cs, eps, dst);
}

template <int D>
RT_DEV void norm_rope_head(const float *src, const float *__restrict__ gamma, const float *__restrict__ cs,
                           float eps, float *dst) {
  norm_rope_head_ld<D>([&](int i) { return src[i]; }, gamma, cs, eps, dst);
}

}  // namespace rt
