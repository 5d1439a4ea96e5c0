// prefill.hip -- GPU prefill for the Gemma-3 decode context: every token of a
// prompt chunk goes through each layer at once (one row per token), filling
// the KV cache rows of the chunk and, for the last chunk, the logits of the
// last token.
//
// Replaces the reference's CPU prefill in generate_cached_streaming
// (transformer4.rs:2103-2139: Gemma3Block::forward_cached over the whole
// prompt, 1900-1964) and the copy of its KV cache to the device that follows
// (sync_kv_from_cpu, metal_decode.rs:1366-1396).  Per layer:
//   k_pf_norm        input RMSNorm (layer 0) / post-norm residual + next norm
//   Q4_K GEMM x3     q, k, v projections (q4k_gemm.hip, matrix cores)
//   k_pf_qk_rope     per-head q/k RMSNorm + NeoX RoPE; k and v into the cache
//   k_pf_attn        causal (windowed) attention on bf16 MFMA
//   Q4_K GEMM        o projection
//   k_pf_norm        residual + post-attention norm, pre-FFN norm
//   Q4_K GEMM x2     gate, up
//   k_pf_gelu_mul    gelu_tanh(gate) * up
//   Q4_K GEMM        down projection
// The per-element arithmetic (norms, RoPE, residuals, GELU) is the decode
// step's (gemma3_math.hpp); the projections are GEMMs instead of GEMVs.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/rt_hip.h"
#include "decode.hpp"
#include "gemma3_math.hpp"
#include "q4k_gemv_mb.hpp"
#include "rt_device.hpp"
#include "rt_kernels.hpp"

namespace rt {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Row kernels
// ---------------------------------------------------------------------------
// x[t] = bf16(E[token_t]) * sqrt(hidden)   (transformer4.rs:2106-2121)
__global__ __launch_bounds__(256) void k_pf_embed(const int *__restrict__ tokens, int tok_stride,
                                                  const uint16_t *__restrict__ E, float scale, float *__restrict__ x,
                                                  int H) {
  const uint16_t *row = E + (size_t)tokens[(size_t)blockIdx.x * tok_stride] * H;
  float *out = x + (size_t)blockIdx.x * H;
  for (int c = threadIdx.x; c < H; c += 256) out[c] = mul_nc(bf16_lo((uint32_t)row[c]), scale);
}

// One row per workgroup, H <= 4096 (H % 64 == 0).
//   RESID:  x = base + rms(add)(1 + g_add);  x_out = x;  xn = rms(x)(1 + g_out)
//   !RESID: x = add;                                     xn = rms(x)(1 + g_out)
// `add` may be split-K partial sums.  With st_dig, xn is also staged as the
// input of a batched GEMV; with a16, it is written as the next GEMM's A
// operand (f16 row scaled by 2^-ea[t], bit-identical to the GEMM's own
// preparation of the f32 row) instead of going through xn_out.  T = 1024 for
// a few rows (more loads in flight per row when `add` is a sum of many
// slices), 256 otherwise.  FEW: `add` holds at most four slices (the prefill
// GEMMs' split-K partials), read with rows_in4_few.
template <bool RESID, int T, bool FEW>
__global__ __launch_bounds__(T) void k_pf_norm(const float *__restrict__ base, RowsIn add,
                                                 const float *__restrict__ g_add, const float *__restrict__ g_out,
                                                 float *__restrict__ x_out, float *__restrict__ xn_out, int H,
                                                 float eps, int8_t *__restrict__ st_dig, _Float16 *__restrict__ a16,
                                                 int *__restrict__ ea, float *__restrict__ nrm2_out, int add_row0) {
  constexpr int PER = 1024 / T;
  __shared__ float red[T / 64];
  const int t = (int)blockIdx.x;
  const size_t off = (size_t)t * (H / 4);
  const int F4 = H / 4;
  const float inv_k = 1.0f / (float)H;
  float4 x[PER];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int f = threadIdx.x + i * T;
    x[i] = f < F4 && t >= add_row0 ? (FEW ? rows_in4_few(add, t, 4 * f) : rows_in4(add, t, 4 * f))
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
    ss += sumsq4(x[i]);
  }
  if constexpr (RESID) {
    const float ra = rms_inv_from_sumsq(block_sum<T>(ss, red), inv_k, eps);
    const float4 *b4 = reinterpret_cast<const float4 *>(base) + off;
    float4 *xo = reinterpret_cast<float4 *>(x_out) + off;
    ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int f = threadIdx.x + i * T;
      if (f < F4) {
        x[i] = add4(b4[f], norm4(x[i], ra, reinterpret_cast<const float4 *>(g_add)[f]));
        xo[f] = x[i];
        ss += sumsq4(x[i]);
      }
    }
  }
  const float rx = rms_inv_from_sumsq(block_sum<T>(ss, red), inv_k, eps);
  float4 *xn = reinterpret_cast<float4 *>(xn_out) + off;
  float *st_stats = st_dig ? mb_stats(st_dig, H) : nullptr;
  float amax = 0.f, nn = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int f = threadIdx.x + i * T;
    if (i * T >= F4) break;  // block-uniform
    const float4 v = norm4(x[i], rx, reinterpret_cast<const float4 *>(g_out)[min(f, F4 - 1)]);
    x[i] = v;
    if (f < F4) {
      if (xn_out) xn[f] = v;
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
      nn += sumsq4(v);
    }
    if (st_dig) mb_stage4(st_dig, st_stats, t, min(f, F4 - 1) >> 4, f & 15, v, f < F4);  // 16 lanes per chunk
  }
  if (nrm2_out) {  // |xn|^2 of the row (block-uniform)
    nn = block_sum<T>(nn, red);
    if (threadIdx.x == 0) nrm2_out[t] = nn;
  }
  if (a16) {
    const int e = f16_exponent_for(block_max<T>(amax, red));
    if (threadIdx.x == 0) ea[t] = e;
    uint2 *dst = reinterpret_cast<uint2 *>(a16 + (size_t)t * H);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int f = threadIdx.x + i * T;
      if (f < F4) dst[f] = f16x4_scaled(x[i], e);
    }
  }
}

template <bool RESID>
hipError_t launch_pf_norm(int n, hipStream_t st, const float *base, RowsIn add, const float *g_add,
                          const float *g_out, float *x_out, float *xn_out, int H, float eps, int8_t *st_dig,
                          _Float16 *a16 = nullptr, int *ea = nullptr, float *nrm2_out = nullptr, int add_row0 = 0) {
  // two to four slices: the prefill GEMMs' split-K partials (a 4096-row
  // prefill 34.51 ms against 35.29-35.48 with the sixteen-slice reader);
  // the verify's GEMV slices keep rows_in4
  const bool few = add.ks >= 2 && add.ks <= 4;
  auto go = [&](auto kern, int threads) {
    hipLaunchKernelGGL(kern, dim3(n), dim3(threads), 0, st, base, add, g_add, g_out, x_out, xn_out, H, eps, st_dig,
                       a16, ea, nrm2_out, add_row0);
  };
  if (n <= 64) {
    if (few) go(k_pf_norm<RESID, 1024, true>, 1024);
    else go(k_pf_norm<RESID, 1024, false>, 1024);
  } else {
    if (few) go(k_pf_norm<RESID, 256, true>, 256);
    else go(k_pf_norm<RESID, 256, false>, 256);
  }
  return hipGetLastError();
}

// One wave per (row, head): q heads in place, k heads into the cache row
// p0 + t (with the matching v row copied next to it), as the decode step's
// k_attn does for its single row (transformer4.rs:1912-1923).  Row t's
// cos/sin table starts at cs + t*cs_stride (+ head_dim for global layers);
// p0 comes from *p0_dev when that is set (graph replays).
template <int D>
__global__ __launch_bounds__(256) void k_pf_qk_rope(RowsIn q, RowsIn k, RowsIn v, float *q_out,
                                                    const float *__restrict__ g_q, const float *__restrict__ g_k,
                                                    const float *__restrict__ cs, int cs_stride, int cs_off,
                                                    float *__restrict__ kc, float *__restrict__ vc, int p0,
                                                    const int *__restrict__ p0_dev, int n, int nq, int nkv,
                                                    float eps) {
  const int heads = nq + nkv;
  // Waves past the last item compute item n*heads-1 again and store nothing;
  // the operands are picked by selects: no early exit or branch makes the
  // arguments load in rounds of their own before the first data loads.
  const int item_raw = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  const bool live = item_raw < n * heads;  // whole waves
  const int item = min(item_raw, n * heads - 1);
  const int t = item / heads, h = item % heads;
  const float *c = cs + (size_t)t * cs_stride + cs_off;
  const int lane = (int)(threadIdx.x & 63);
  auto head = [&](const RowsIn &r, int col, const float *g, float *dst) __attribute__((always_inline)) {
    if constexpr (D == 256) {
      // lane l: dims 4l .. 4l+3 in one 16-byte read of the (split-K)
      // projection output; after the norm, v_permlane32_swap gives every
      // lane the pair (dim p, dim p + 128), p = 4(l % 32) + e, and lane l
      // writes its own dims: a0 c - a1 s below 128, a0 s + a1 c above, as
      // norm_rope_head_regs computes them (sums of squares in another order)
      const float4 xv = rows_in4(r, t, col + 4 * lane);
      const float ss = xv.x * xv.x + xv.y * xv.y + xv.z * xv.z + xv.w * xv.w;
      const float rinv = rms_inv_from_sumsq(wave_sum(ss), 1.0f / (float)D, eps);
      const float4 gm = reinterpret_cast<const float4 *>(g)[lane];
      const int pl = lane & 31;
      const float4 cv = reinterpret_cast<const float4 *>(c)[pl], sv = reinterpret_cast<const float4 *>(c + D / 2)[pl];
      const float x[4] = {xv.x, xv.y, xv.z, xv.w}, gg[4] = {gm.x, gm.y, gm.z, gm.w};
      const float cc[4] = {cv.x, cv.y, cv.z, cv.w}, sn[4] = {sv.x, sv.y, sv.z, sv.w};
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
        const float a = (x[e] * rinv) * (1.0f + gg[e]);
        const auto sw = __builtin_amdgcn_permlane32_swap(f32_bits(a), f32_bits(a), false, false);
        const float a0 = bits_f32(sw[0]), a1 = bits_f32(sw[1]);
        o[e] = lane < 32 ? a0 * cc[e] - a1 * sn[e] : a0 * sn[e] + a1 * cc[e];
      }
      reinterpret_cast<float4 *>(dst)[lane] = make_float4(o[0], o[1], o[2], o[3]);
    } else {
      float x0[D / 128], x1[D / 128];
#pragma unroll
      for (int pp = 0; pp < D / 128; ++pp) {
        x0[pp] = rows_in1(r, t, col + lane * (D / 128) + pp);
        x1[pp] = rows_in1(r, t, col + D / 2 + lane * (D / 128) + pp);
      }
      norm_rope_head_regs<D>(x0, x1, g, c, eps, dst);
    }
  };
  const bool is_q = h < nq;
  const int kh = is_q ? 0 : h - nq;
  if constexpr (D == 256) {
    // the v row of a k head goes with it (q heads load one they do not store)
    const float4 vv = rows_in4(v, t, kh * D + 4 * lane);
    if (p0_dev) p0 = p0_dev[0];  // the step's first position, read after the data loads are out
    const size_t kdst = ((size_t)(p0 + t) * nkv + kh) * D;
    float *dst = is_q ? q_out + ((size_t)t * nq + h) * D : kc + kdst;
    if (!live) return;
    head(is_q ? q : k, is_q ? h * D : kh * D, is_q ? g_q : g_k, dst);
    if (!is_q) reinterpret_cast<float4 *>(vc + kdst)[lane] = vv;
  } else {
    if (!live) return;
    if (p0_dev) p0 = p0_dev[0];
    if (is_q) {
      head(q, h * D, g_q, q_out + ((size_t)t * nq + h) * D);
    } else {
      const size_t dst = ((size_t)(p0 + t) * nkv + kh) * D;
      head(k, kh * D, g_k, kc + dst);
      for (int i = 2 * lane; i < D; i += 128) *reinterpret_cast<float2 *>(vc + dst + i) = rows_in2(v, t, kh * D + i);
    }
  }
}

// h = gelu_tanh(g) * u  (Gemma3Mlp::forward, transformer4.rs:328-334) over
// n rows of F; g and u may be split-K partial sums, h may alias g (each
// element is read before it is written, by one thread).  With st_dig, h is
// also staged as the input of a batched GEMV.
__global__ __launch_bounds__(256) void k_pf_gelu_mul(RowsIn g, RowsIn u, float *h, int n, int F,
                                                     int8_t *__restrict__ st_dig) {
  const int f4 = F / 4;  // a multiple of 16: the 16 lanes of a chunk stay in one row
  const int n4 = n * f4;  // at most 8 rows of F <= 16384 (32-bit indices: no 64-bit division)
  // The first pass runs unconditionally at a clamped index (the launcher
  // sizes the grid for one pass), so every argument is read at the start;
  // lanes past n4 store nothing (whole 16-lane groups: n4 and f4 are
  // multiples of 16).
  int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
  do {
    const bool live = i < n4;
    const int ic = min(i, n4 - 1);
    const int t = ic / f4, c4 = ic - t * f4;
    const float4 a = rows_in4(g, t, 4 * c4), b = rows_in4(u, t, 4 * c4);
    const float4 r = make_float4(mul_nc(gelu_tanh(a.x), b.x), mul_nc(gelu_tanh(a.y), b.y),
                                 mul_nc(gelu_tanh(a.z), b.z), mul_nc(gelu_tanh(a.w), b.w));
    if (live) reinterpret_cast<float4 *>(h)[i] = r;
    // every lane runs the staging (its digits need the chunk's 16 lanes); it
    // writes only with st_dig set
    mb_stage4(st_dig, st_dig ? mb_stats(st_dig, F) : nullptr, t, c4 >> 4, c4 & 15, r, live && st_dig != nullptr);
    i += (int)gridDim.x * 256;
  } while (i < n4);
}

// The same product for the GEMM path, one row per workgroup of kGeluRowT
// threads (F <= 16384; 1024 threads measured 1% faster over a 4096-row
// prefill than 256): h goes straight out as the down GEMM's A operand (f16
// row, exponent ea[t]), bit-identical to preparing the f32 row.
constexpr int kGeluRowT = 1024;
__global__ __launch_bounds__(kGeluRowT) void k_pf_gelu_rows(RowsIn g, RowsIn u, int F, _Float16 *__restrict__ a16,
                                                      int *__restrict__ ea) {
  constexpr int MAXP = 16384 / 4 / kGeluRowT;
  __shared__ float red[kGeluRowT / 64];
  const int t = (int)blockIdx.x, f4 = F / 4;
  float4 r[MAXP];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < MAXP; ++i) {
    const int c4 = (int)threadIdx.x + kGeluRowT * i;
    if (c4 < f4) {
      const float4 a = rows_in4(g, t, 4 * c4), b = rows_in4(u, t, 4 * c4);
      r[i] = make_float4(mul_nc(gelu_tanh(a.x), b.x), mul_nc(gelu_tanh(a.y), b.y), mul_nc(gelu_tanh(a.z), b.z),
                         mul_nc(gelu_tanh(a.w), b.w));
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(r[i].x), fabsf(r[i].y)), fmaxf(fabsf(r[i].z), fabsf(r[i].w))));
    }
  }
  const int e = f16_exponent_for(block_max<kGeluRowT>(amax, red));
  if (threadIdx.x == 0) ea[t] = e;
  uint2 *dst = reinterpret_cast<uint2 *>(a16 + (size_t)t * F);
#pragma unroll
  for (int i = 0; i < MAXP; ++i) {
    const int c4 = (int)threadIdx.x + kGeluRowT * i;
    if (c4 < f4) dst[c4] = f16x4_scaled(r[i], e);
  }
}

// ---------------------------------------------------------------------------
// k_pf_attn: causal attention of a chunk of query rows against the f32 KV
// cache (gqa_attention_cached's prefill branch, transformer4.rs:2882-2940,
// and the per-row window of gqa_attention_windowed, 2661-2700).
//
// Query row t (absolute position r = p0 + t) sees keys
//   [lo(r), r],  lo(r) = max(lo_fixed, window ? r + 1 - window : 0),
// and an empty range gives a zero output row (the reference's rows that
// precede the window start).
//
// Matrix cores: v_mfma_f32_16x16x32_bf16 with every f32 operand x split into
// bf16 parts hi = bf16(x), lo = bf16(x - hi) (|x - hi - lo| <= 2^-16 |x|) and
// the products hi*hi + hi*lo + lo*hi accumulated in f32.
//   scores   S^T[key][col] = K . Q^T  (A = 16 keys x 32 dims from LDS,
//            B = this wave's 16 query columns, held in registers)
//   output   O^T[dim][col] += V^T . P^T (A = 16 dims x 32 keys from LDS,
//            B = the probabilities, taken from the lanes' own score registers)
// A query column is a (row, head) pair; the G heads that share a KV head sit
// in adjacent columns and share every K/V tile.  Lane (c = l%16, g = l/16)
// holds score rows 4g..4g+3 of each 16-key tile; the MFMA's k index 8g + i
// stands for key 4g + i (i < 4) or 16 + 4g + (i - 4) (i >= 4), for A and B
// alike, so the probabilities feed the second MFMA without leaving the lane.
// Softmax is online over stages of 32 keys (running max and sum per column).
// ---------------------------------------------------------------------------
constexpr int kPfKeys = 32;  // keys per LDS stage

struct PfAttnArgs {
  int p0, n, n_kv_heads;
  int lo_fixed, window;
  float scale;
  const int *p0_dev;  // when set, p0 = *p0_dev (graph replays)
  // Key split (few rows, long key ranges): workgroup z takes stages
  // [z*split_stages, (z+1)*split_stages) of its key range and writes the
  // unnormalised (max, sum, O) of each column for k_pf_attn_combine.
  int split_stages;   // 0: no split, the kernel writes the output itself
  float *part_ml;     // [splits][(n - row_base)*n_q_heads][2]
  float *part_o;      // [splits][(n - row_base)*n_q_heads][D]
  // Rows [row_base, n) are computed (rows below see no key and are zeroed by
  // the combine).
  int row_base = 0;
};

template <int D>
struct PfAttnSmem {
  static constexpr int KP = D + 8;        // K row pitch (bf16): rows 16 B apart in the bank space
  static constexpr int VP = kPfKeys + 4;  // V^T row pitch (bf16): 72 B
  uint16_t khi[kPfKeys * KP], klo[kPfKeys * KP];
  uint16_t vhi[D * VP], vlo[D * VP];
};

RT_DEV int pf_key_lo(const PfAttnArgs &p, int r) { return max(p.lo_fixed, p.window > 0 ? r - p.window + 1 : 0); }

// Two f32 -> packed bf16 hi parts (.x) and lo parts (.y), RNE (v_cvt_pk_bf16_f32).
RT_DEV uint2 split_pair(float a, float b) {
  const f32x2_t x = {a, b};
  const bf16x2_t h = __builtin_convertvector(x, bf16x2_t);
  const f32x2_t r = x - __builtin_convertvector(h, f32x2_t);
  return make_uint2(__builtin_bit_cast(uint32_t, h), __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2_t)));
}

// Eight f32 -> a bf16x8 hi fragment and lo fragment.
RT_DEV void split8(const float (&x)[8], u32x4_t &hi, u32x4_t &lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint2 v = split_pair(x[2 * i], x[2 * i + 1]);
    hi[i] = v.x;
    lo[i] = v.y;
  }
}

RT_DEV f32x4_t mfma3(u32x4_t ahi, u32x4_t alo, u32x4_t bhi, u32x4_t blo, f32x4_t acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, alo), __builtin_bit_cast(bf16x8_t, bhi),
                                                acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ahi), __builtin_bit_cast(bf16x8_t, blo),
                                                acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ahi), __builtin_bit_cast(bf16x8_t, bhi),
                                                 acc, 0, 0, 0);
}

template <int D, int G, int W>
__global__ __launch_bounds__(64 * W) void k_pf_attn(const float *__restrict__ q, const float *__restrict__ kc,
                                                    const float *__restrict__ vc, float *__restrict__ out,
                                                    PfAttnArgs p) {
  constexpr int NT = 64 * W;                  // threads: W waves of 16 columns share each K/V stage
  constexpr int NC = 16 * W;                  // columns per workgroup
  constexpr int KB = kPfKeys;
  constexpr int DS = D / 32;                  // k steps of the score MFMA
  constexpr int DT = D / 16;                  // 16-dim tiles of the output
  constexpr int KQ = D / 4;                   // float4 per cache row
  constexpr int K_ITEMS = KB * KQ / NT;       // K float4 per thread per stage
  constexpr int V_ITEMS = KB / 2 * KQ / NT;   // V key pairs x float4 per thread per stage
  static_assert(K_ITEMS >= 1 && V_ITEMS >= 1, "D too small");
  using S = PfAttnSmem<D>;
  __shared__ __attribute__((aligned(16))) S sm;

  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63), n16 = lane & 15, g = lane >> 4;
  const size_t qd = (size_t)p.n_kv_heads * G * D, kvd = (size_t)p.n_kv_heads * D;
  const int last_row = p.n - 1;
  const int nb = ((p.n - p.row_base) * G + NC - 1) / NC;  // row blocks of the launch
  // Workgroups are dealt to the eight XCDs in turn (linear id mod 8).  When
  // the KV heads divide the XCDs and the grid is whole rounds of them, the
  // workgroups of one XCD all take the same KV head, so its L2 holds one
  // head's K/V stages for every row block walking them.
  int kvh = (int)blockIdx.y, bx = (int)blockIdx.x;
  if (8 % p.n_kv_heads == 0 && ((int)gridDim.x * p.n_kv_heads) % 8 == 0) {
    const int lin = (int)(blockIdx.x + blockIdx.y * gridDim.x), xcd = lin & 7, slot = lin >> 3;
    const int per = 8 / p.n_kv_heads;  // XCDs per KV head
    kvh = xcd / per;
    bx = slot * per + xcd % per;
  }
  const int b = nb - 1 - bx;  // late rows (the longest key ranges) first
  const int col0 = p.row_base * G + b * NC;
  const int wt0 = (col0 + 16 * wave) / G;
  const bool wave_live = wt0 <= last_row;
  const int col = col0 + 16 * wave + n16;
  const int t = col / G;
  const bool col_ok = t <= last_row;
  const int hq = kvh * G + col % G;

  // this lane's query fragment: dims 32s + 8g + [0, 8) of column `col`
  // (loaded here, split into bf16 parts below)
  float4 qx0[DS], qx1[DS];
  {
    const float *qrow = q + (size_t)min(t, last_row) * qd + (size_t)hq * D + 8 * g;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      qx0[s] = *reinterpret_cast<const float4 *>(qrow + 32 * s);
      qx1[s] = *reinterpret_cast<const float4 *>(qrow + 32 * s + 4);
    }
  }

  // the step's first position (a load from the parameter block) is read
  // once the query loads, which do not depend on it, are out
  __builtin_amdgcn_sched_barrier(0);
  if (p.p0_dev) p.p0 = p.p0_dev[0];
  const int key_first = pf_key_lo(p, p.p0 + col0 / G) & ~(KB - 1);
  const int key_last = p.p0 + min(last_row, (col0 + NC - 1) / G);
  const int wkey_lo = pf_key_lo(p, p.p0 + wt0);
  const int wkey_hi = p.p0 + min(last_row, (col0 + 16 * wave + 15) / G);
  const int r = p.p0 + t;
  const int klo = pf_key_lo(p, r);
  u32x4_t qh[DS], ql[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s) {
    const float x[8] = {qx0[s].x, qx0[s].y, qx0[s].z, qx0[s].w, qx1[s].x, qx1[s].y, qx1[s].z, qx1[s].w};
    split8(x, qh[s], ql[s]);
  }

  // stage loads: rows clamped to key_last (keys past it are masked)
  float4 kr[K_ITEMS], vr[V_ITEMS][2];
  const float *kbase = kc + (size_t)kvh * D, *vbase = vc + (size_t)kvh * D;
  auto load_stage = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < K_ITEMS; ++i) {
      const int it = (int)threadIdx.x + NT * i, key = it / KQ, qq = it % KQ;
      kr[i] = *reinterpret_cast<const float4 *>(kbase + (size_t)min(k0 + key, key_last) * kvd + 4 * qq);
    }
#pragma unroll
    for (int i = 0; i < V_ITEMS; ++i) {
      const int it = (int)threadIdx.x + NT * i, pr = it / KQ, qq = it % KQ;
      vr[i][0] = *reinterpret_cast<const float4 *>(vbase + (size_t)min(k0 + 2 * pr, key_last) * kvd + 4 * qq);
      vr[i][1] = *reinterpret_cast<const float4 *>(vbase + (size_t)min(k0 + 2 * pr + 1, key_last) * kvd + 4 * qq);
    }
  };
  auto store_stage = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < K_ITEMS; ++i) {
      const int it = (int)threadIdx.x + NT * i, key = it / KQ, qq = it % KQ;
      const uint2 p0 = split_pair(kr[i].x, kr[i].y), p1 = split_pair(kr[i].z, kr[i].w);
      *reinterpret_cast<uint2 *>(&sm.khi[key * S::KP + 4 * qq]) = make_uint2(p0.x, p1.x);
      *reinterpret_cast<uint2 *>(&sm.klo[key * S::KP + 4 * qq]) = make_uint2(p0.y, p1.y);
    }
#pragma unroll
    for (int i = 0; i < V_ITEMS; ++i) {
      const int it = (int)threadIdx.x + NT * i, pr = it / KQ, qq = it % KQ;
      const float a[4] = {vr[i][0].x, vr[i][0].y, vr[i][0].z, vr[i][0].w};
      const float c[4] = {vr[i][1].x, vr[i][1].y, vr[i][1].z, vr[i][1].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint2 hl = split_pair(a[e], c[e]);
        *reinterpret_cast<uint32_t *>(&sm.vhi[(4 * qq + e) * S::VP + 2 * pr]) = hl.x;
        *reinterpret_cast<uint32_t *>(&sm.vlo[(4 * qq + e) * S::VP + 2 * pr]) = hl.y;
      }
    }
  };

  f32x4_t o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  int k_begin = key_first, k_end = key_last;
  if (p.split_stages) {
    // the last split runs to key_last, so the splits cover the block's keys
    // whatever span the host planned them for
    k_begin = key_first + (int)blockIdx.z * p.split_stages * KB;
    if ((int)blockIdx.z + 1 < (int)gridDim.z) k_end = min(key_last, k_begin + p.split_stages * KB - 1);
  }
  load_stage(k_begin);
#pragma unroll 1
  for (int k0 = k_begin; k0 <= k_end; k0 += KB) {
    __syncthreads();  // every wave is done with the previous stage
    store_stage();
    __syncthreads();
    if (k0 + KB <= k_end) load_stage(k0 + KB);  // lands during this stage's MFMAs
    if (!wave_live || k0 > wkey_hi || k0 + KB - 1 < wkey_lo) continue;  // wave-uniform

    f32x4_t sc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      const int ko = (16 * tt + n16) * S::KP + 8 * g;
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const u32x4_t ah = *reinterpret_cast<const u32x4_t *>(&sm.khi[ko + 32 * s]);
        const u32x4_t al = *reinterpret_cast<const u32x4_t *>(&sm.klo[ko + 32 * s]);
        acc = mfma3(ah, al, qh[s], ql[s], acc);
      }
      sc[tt] = acc;
    }
    // mask, scale (scores = (q.k) * scale, transformer4.rs:2897) and the running softmax
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = k0 + 16 * tt + 4 * g + j;
        const bool ok = col_ok && key <= r && key >= klo;
        sv[4 * tt + j] = ok ? sc[tt][j] * p.scale : -INFINITY;
        mx = fmaxf(mx, sv[4 * tt + j]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float mb = m_new == -INFINITY ? 0.f : m_new;  // a column with no key yet keeps zeros
    const float alpha = expf(m_run - mb);
    float pv[8], ps = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pv[i] = expf(sv[i] - mb);
      ps += pv[i];
    }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    u32x4_t ph, pl;
    split8(pv, ph, pl);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int vo = (16 * dt + n16) * S::VP + 4 * g;
      const uint2 h0 = *reinterpret_cast<const uint2 *>(&sm.vhi[vo]);
      const uint2 h1 = *reinterpret_cast<const uint2 *>(&sm.vhi[vo + 16]);
      const uint2 l0 = *reinterpret_cast<const uint2 *>(&sm.vlo[vo]);
      const uint2 l1 = *reinterpret_cast<const uint2 *>(&sm.vlo[vo + 16]);
      const u32x4_t ah = {h0.x, h0.y, h1.x, h1.y}, al = {l0.x, l0.y, l1.x, l1.y};
      o[dt] *= alpha;
      o[dt] = mfma3(ah, al, ph, pl, o[dt]);
    }
  }

  if (col_ok && p.split_stages) {
    // partial of this key split (an empty split leaves max -inf, sum 0, O 0)
    const int na = p.n - p.row_base;
    const size_t cidx =
        (size_t)blockIdx.z * na * p.n_kv_heads * G + (size_t)(t - p.row_base) * p.n_kv_heads * G + hq;
    if (g == 0) {
      p.part_ml[2 * cidx] = m_run;
      p.part_ml[2 * cidx + 1] = l_run;
    }
    float *po = p.part_o + cidx * D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<float4 *>(po + 16 * dt) = make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
  } else if (col_ok) {
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    float *orow = out + (size_t)t * qd + (size_t)hq * D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<float4 *>(orow + 16 * dt) =
          make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
  }
}

// Merge of the key splits of every (row, head) column:
//   out = sum_s O_s e^(m_s - M) / sum_s l_s e^(m_s - M),  M = max_s m_s
// (0 for a column with no key at all, as the reference's empty rows).
// Columns below col_base (rows that see no key) are written as zeros; the
// partials hold the columns from col_base on.
template <int D>
__global__ __launch_bounds__(D) void k_pf_attn_combine(const float *__restrict__ part_ml,
                                                       const float *__restrict__ part_o, float *__restrict__ out,
                                                       int ncols, int splits, int nq, int8_t *__restrict__ st_dig,
                                                       int col_base) {
  static_assert(D >= kPfMaxSplits, "one lane of wave 0 per split");
  __shared__ float w_lds[kPfMaxSplits];
  __shared__ float l_lds;
  const int col_out = (int)blockIdx.x, d = (int)threadIdx.x;
  if (col_out < col_base) {  // block-uniform
    out[(size_t)col_out * D + d] = 0.f;
    if (st_dig) mb_stage1(st_dig, mb_stats(st_dig, nq * D), col_out / nq, ((col_out % nq) * D + d) >> 6, 0.f);
    return;
  }
  const int col = col_out - col_base;
  ncols -= col_base;
  if (d < 64) {  // wave 0: split z = lane
    const bool live = d < splits;
    const float m = live ? part_ml[2 * ((size_t)d * ncols + col)] : -INFINITY;
    const float l = live ? part_ml[2 * ((size_t)d * ncols + col) + 1] : 0.f;
    const float M = wave_max(m);
    const float w = (m == -INFINITY) ? 0.f : expf(m - M);
    if (live) w_lds[d] = w;
    const float L = wave_sum(l * w);
    if (d == 0) l_lds = L;
  }
  __syncthreads();
  float O = 0.f;
#pragma unroll 8
  for (int z = 0; z < splits; ++z) O = fmaf(part_o[((size_t)z * ncols + col) * D + d], w_lds[z], O);
  const float L = l_lds;
  const float r = L > 0.f ? O / L : 0.f;
  out[(size_t)col_out * D + d] = r;
  if (st_dig) {  // element (col % nq)*D + d of row col / nq; one 64-element chunk per wave
    const int t = col_out / nq, e = (col_out % nq) * D + d;
    mb_stage1(st_dig, mb_stats(st_dig, nq * D), t, e >> 6, r);
  }
}

// The same merge for the GEMM path with D = 256, one workgroup per row
// (thread = dimension, the row's nq <= MAXH heads in turn): the merged row
// goes out as the o projection's A operand, f16 scaled by 2^-ea[t] (bit-
// identical to the GEMM's own preparation of the f32 row), instead of f32.
// Rows below row_base (no key) are zero rows; workgroup b takes row
// row_first + b (row_first = row_base: the zero rows are not written).
template <int MAXH>
__global__ __launch_bounds__(256) void k_pf_attn_combine_a16(const float *__restrict__ part_ml,
                                                           const float *__restrict__ part_o, int n, int nq,
                                                           int splits, int row_base, int row_first,
                                                           _Float16 *__restrict__ a16, int *__restrict__ ea) {
  constexpr int D = 256;
  __shared__ float w_lds[MAXH][kPfMaxSplits];
  __shared__ float l_lds[MAXH];
  __shared__ float red[4];
  const int t = row_first + (int)blockIdx.x, d = (int)threadIdx.x, wave = d >> 6, lane = d & 63;
  _Float16 *out = a16 + (size_t)t * nq * D;
  if (t < row_base) {  // block-uniform
    for (int h = 0; h < nq; ++h) out[h * D + d] = (_Float16)0.f;
    if (d == 0) ea[t] = 0;
    return;
  }
  const int ncols = (n - row_base) * nq, col0 = (t - row_base) * nq;
  // Up to 8 splits: every partial O of the row is loaded before the weights
  // are formed (one memory round trip per row instead of two).
  constexpr int ZP = 8;
  float po[MAXH][ZP];
  if (splits <= ZP) {  // block-uniform
#pragma unroll
    for (int h = 0; h < MAXH; ++h)
#pragma unroll
      for (int z = 0; z < ZP; ++z)
        po[h][z] = (h < nq && z < splits) ? part_o[((size_t)z * ncols + col0 + h) * D + d] : 0.f;
  }
  for (int h = wave; h < nq; h += 4) {  // wave-uniform: split z = lane
    const bool live = lane < splits;
    const size_t ci = (size_t)lane * ncols + col0 + h;
    const float m = live ? part_ml[2 * ci] : -INFINITY;
    const float l = live ? part_ml[2 * ci + 1] : 0.f;
    const float M = wave_max(m);
    const float w = (m == -INFINITY) ? 0.f : expf(m - M);
    if (live) w_lds[h][lane] = w;
    const float L = wave_sum(l * w);
    if (lane == 0) l_lds[h] = L;
  }
  __syncthreads();
  float r[MAXH];
  float amax = 0.f;
#pragma unroll
  for (int h = 0; h < MAXH; ++h) {
    r[h] = 0.f;
    if (h < nq) {  // block-uniform
      float O = 0.f;
      if (splits <= ZP) {
#pragma unroll
        for (int z = 0; z < ZP; ++z)
          if (z < splits) O = fmaf(po[h][z], w_lds[h][z], O);
      } else {
#pragma unroll 8
        for (int z = 0; z < splits; ++z) O = fmaf(part_o[((size_t)z * ncols + col0 + h) * D + d], w_lds[h][z], O);
      }
      const float L = l_lds[h];
      r[h] = L > 0.f ? O / L : 0.f;
      amax = fmaxf(amax, fabsf(r[h]));
    }
  }
  const int e = f16_exponent_for(block_max<256>(amax, red));
  if (d == 0) ea[t] = e;
#pragma unroll
  for (int h = 0; h < MAXH; ++h)
    if (h < nq) out[h * D + d] = (_Float16)__builtin_amdgcn_ldexpf(r[h], -e);
}

template <int D, int W>
hipError_t launch_pf_attn_w(int G, dim3 grid, hipStream_t st, const float *q, const float *kc, const float *vc,
                            float *out, const PfAttnArgs &p) {
  switch (G) {
    case 1: hipLaunchKernelGGL((k_pf_attn<D, 1, W>), grid, dim3(64 * W), 0, st, q, kc, vc, out, p); break;
    case 2: hipLaunchKernelGGL((k_pf_attn<D, 2, W>), grid, dim3(64 * W), 0, st, q, kc, vc, out, p); break;
    case 4: hipLaunchKernelGGL((k_pf_attn<D, 4, W>), grid, dim3(64 * W), 0, st, q, kc, vc, out, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// grid: (column blocks of 64, KV heads, key splits).  From 256 columns on,
// workgroups of eight waves take 128 columns each, which halves the K/V stage
// loads and bf16 splits per column.
// With a16 (the GEMM path, D = 256, at most 16 q heads) a key-split launch
// merges straight into the o projection's f16 A operand and sets *a16_row0
// to the first row it writes: p.row_base with skip_zero_rows (the rows below
// see no key, their A rows are left unwritten), else 0.
template <int D>
hipError_t launch_pf_attn(int G, dim3 grid, hipStream_t st, const float *q, const float *kc, const float *vc,
                          float *out, const PfAttnArgs &p, int8_t *st_dig, _Float16 *a16 = nullptr,
                          int *ea = nullptr, int *a16_row0 = nullptr, bool skip_zero_rows = false) {
  hipError_t e;
  const int na = p.n - p.row_base;
  if (na * G >= 256) {
    grid.x = (unsigned)((na * G + 127) / 128);
    e = launch_pf_attn_w<D, 8>(G, grid, st, q, kc, vc, out, p);
  } else {
    grid.x = (unsigned)((na * G + 63) / 64);
    e = launch_pf_attn_w<D, 4>(G, grid, st, q, kc, vc, out, p);
  }
  if (e != hipSuccess || !p.split_stages) return e;
  const int nq = p.n_kv_heads * G;
  if (D == 256 && a16 && !st_dig && nq <= 16) {
    const int row_first = skip_zero_rows ? p.row_base : 0;
    if (nq <= 8)
      hipLaunchKernelGGL(k_pf_attn_combine_a16<8>, dim3(p.n - row_first), dim3(256), 0, st, p.part_ml, p.part_o, p.n,
                         nq, (int)grid.z, p.row_base, row_first, a16, ea);
    else
      hipLaunchKernelGGL(k_pf_attn_combine_a16<16>, dim3(p.n - row_first), dim3(256), 0, st, p.part_ml, p.part_o,
                         p.n, nq, (int)grid.z, p.row_base, row_first, a16, ea);
    *a16_row0 = row_first;
    return hipGetLastError();
  }
  const int ncols = p.n * p.n_kv_heads * G;
  hipLaunchKernelGGL((k_pf_attn_combine<D>), dim3(ncols), dim3(D), 0, st, p.part_ml, p.part_o, out, ncols,
                     (int)grid.z, p.n_kv_heads * G, st_dig, p.row_base * p.n_kv_heads * G);
  return hipGetLastError();
}

}  // namespace

size_t prefill_gemm_workspace_bytes(const DecodeShape &s, int cap) {
  const int H = s.hidden, F = s.ffn, QD = s.n_q_heads * s.head_dim, KVD = s.n_kv_heads * s.head_dim;
  // The projection sets (K, then the rows of each matrix): the A part of the
  // largest K, then each matrix's own region, which may keep split-K
  // partials for the consumer.
  const int sets[4][4] = {{H, QD, KVD, KVD}, {QD, H, 0, 0}, {H, F, F, 0}, {F, H, 0, 0}};
  const int kmax = std::max({H, QD, F});
  auto r256 = [](size_t v) { return (v + 255) & ~size_t(255); };
  // A chunk may hold fewer rows than cap, and a smaller M may split K more
  // ways: take the largest requirement over every row count up to cap.
  size_t m = 0;
  for (int rows = 1; rows <= cap; ++rows)
    for (auto &st : sets) {
      const int K = st[0];
      size_t b = r256((size_t)rows * kmax * 2) + r256((size_t)rows * 4);
      for (int i = 1; i < 4 && st[i]; ++i)
        b += std::max(q4k_gemm_prepped_ws_bytes(rows, st[i], K), proj_gemm_prepped_ws_bytes(rows, st[i], K));
      m = std::max(m, b);
    }
  return m;
}

size_t rows_mb_stage_bytes(const DecodeShape &s) {
  return mb_stage_bytes(std::max({s.hidden, s.ffn, s.n_q_heads * s.head_dim}));
}

size_t rows_mb_part_bytes(const DecodeShape &s) {
  const int H = s.hidden, F = s.ffn, QD = s.n_q_heads * s.head_dim, KVD = s.n_kv_heads * s.head_dim;
  // a set split by format takes one region per launch: at most the larger
  // slice count of the two kernel families times the set's rows
  auto set = [](int n, int k) {
    return std::max(k % 256 == 0 ? mb_part_bytes(n, k) : (size_t)0, kquant_mb_part_bytes(n, k));
  };
  return std::max({set(QD + 2 * KVD, H), set(H, QD), set(2 * F, H), set(H, F)});
}

bool rows_mb_formats_ok(const DecodeShape &s, const int *fmt) {
  const int H = s.hidden, F = s.ffn, QD = s.n_q_heads * s.head_dim;
  const int kdim[7] = {H, H, H, QD, H, H, F};
  for (int i = 0; i < 7; ++i) {
    const bool ok = fmt[i] == RT_LINEAR_Q4K ? kdim[i] % 256 == 0 : kquant_mb_supported(fmt[i], kdim[i]);
    if (!ok) return false;
  }
  return true;
}

hipError_t enqueue_rows(const DecodeShape &s, const DecodeArgs &a, const LayerArgs *layers, const PrefillBuffers &b,
                        const RowsPlan &plan, hipStream_t st) {
  const int H = s.hidden, F = s.ffn, D = s.head_dim, nq = s.n_q_heads, nkv = s.n_kv_heads;
  const int QD = nq * D, KVD = nkv * D, G = nq / nkv, n = plan.n;
  hipError_t e = hipSuccess;
#define PF_CHECK(x)               \
  do {                            \
    x;                            \
    e = hipGetLastError();        \
    if (e != hipSuccess) return e; \
  } while (0)
#define PF_TRY(x)                 \
  do {                            \
    e = (x);                      \
    if (e != hipSuccess) return e; \
  } while (0)
  // Projections: the GEMM on plain inputs, or (plan.mb, n <= 8) the batched
  // GEMV.  On the batched path each producer kernel also stages its output
  // as the next GEMV's input (stage != null), and the GEMV leaves split-K
  // partial sums that the consumer adds while reading (views).
  int8_t *stage = plan.mb ? static_cast<int8_t *>(b.mb_stage) : nullptr;
  RowsIn vq, vk, vv, vo, vg, vu, vd;
  // The GEMM path's A operand (f16 rows + exponents) at the start of the
  // workspace, for rows of length K.
  auto r256 = [](size_t v) { return (v + 255) & ~size_t(255); };
  auto gemm_a16 = [&](int K) { return reinterpret_cast<_Float16 *>(b.ws); };
  auto gemm_ea = [&](int K) {
    return reinterpret_cast<int *>(static_cast<char *>(b.ws) + r256((size_t)n * K * 2));
  };
  const int kmax = std::max({H, QD, F});
  _Float16 *a16_h = plan.mb ? nullptr : gemm_a16(H);  // producers that write A directly
  int *ea_h = plan.mb ? nullptr : gemm_ea(H);
  float *xn_f32 = plan.mb ? b.xn : nullptr;
  auto proj = [&](const float *A, int K, std::initializer_list<int> fmts, std::initializer_list<MbMat> mats,
                  std::initializer_list<RowsIn *> views, std::initializer_list<const int *> ews,
                  _Float16 *a16_in = nullptr, int *ea_in = nullptr) {
    if (plan.mb) {
      // the set's Q4_K matrices in one launch, each other format in one
      // launch of its own (Q8_0 / Q6_K from the same staged digits, BF16 from
      // the f32 rows A), each with its own region of the partial sums
      float *part = b.mb_part;
      for (int fmt : {RT_LINEAR_Q4K, RT_LINEAR_Q6K, RT_LINEAR_Q8_0, RT_LINEAR_BF16}) {
        MbMat grp[3];
        RowsIn *gv[3];
        int cnt = 0, ntot = 0, i = 0;
        for (const MbMat &m : mats) {
          if (fmts.begin()[i] == fmt) grp[cnt] = m, gv[cnt++] = views.begin()[i], ntot += m.n;
          ++i;
        }
        if (!cnt) continue;
        RowsIn out[3];
        hipError_t r = fmt == RT_LINEAR_Q4K ? launch_q4k_gemv_mb(grp, cnt, n, K, b.mb_stage, part, st, out)
                                            : launch_kquant_gemv_mb(fmt, grp, cnt, n, K, b.mb_stage, A, part, st, out);
        if (r != hipSuccess) return r;
        for (int c = 0; c < cnt; ++c) *gv[c] = out[c];
        part += (fmt == RT_LINEAR_Q4K ? mb_part_bytes(ntot, K) : kquant_mb_part_bytes(ntot, K)) / sizeof(float);
      }
      return hipSuccess;
    }
    // A is prepared once for every matrix of the set (q|k|v, gate|up); the
    // norms and the gelu product write it themselves (A == nullptr), at
    // a16_in / ea_in when given
    _Float16 *a16 = a16_in ? a16_in : gemm_a16(K);
    int *ea = a16_in ? ea_in : gemm_ea(K);
    // The matrices' regions start after the A part of the largest K: the
    // producer of the next set's A (a norm, the gelu product) writes it
    // while it reads partials left here.
    char *rest = static_cast<char *>(b.ws) + r256((size_t)n * kmax * 2) + r256((size_t)n * 4);
    hipError_t r = A ? launch_gemm_prep_a(A, n, K, a16, ea, st) : hipSuccess;
    if (r != hipSuccess) return r;
    // A set of Q4_K matrices with enough rows or tiles for the half-block
    // kernel (long prompts, or a gate|up set from about 900 rows at 4B
    // widths): one matrix-core launch for the set (its tiles fill the CUs in
    // whole rounds), row exponents of each matrix at the start of its region
    bool all_q4k = true;
    int set_n[3] = {0, 0, 0}, ni = 0;
    for (int f : fmts) all_q4k = all_q4k && f == RT_LINEAR_Q4K;
    for (const MbMat &m : mats)
      if (ni < 3) set_n[ni++] = m.n;
    if (all_q4k && mats.size() > 1 && q4k_gemm_multi_ok(n, (int)mats.size(), set_n)) {
      const void *w[3];
      float *c[3];
      int nn[3];
      void *ew[3];
      int i = 0;
      char *reg = rest;
      for (const MbMat &m : mats) {
        w[i] = m.w, c[i] = m.y, nn[i] = m.n, ew[i] = reg;
        reg += q4k_gemm_prepped_ws_bytes(n, m.n, K);
        *views.begin()[i++] = rows_plain(m.y, m.n);
      }
      return launch_q4k_gemm_multi_prepped(a16, ea, i, w, c, nn, ew, n, K, st, ews.begin());
    }
    // each matrix in its own region; a split Q4_K GEMM leaves its partials
    // there and the consumer adds them while reading (views)
    int i = 0;
    for (const MbMat &m : mats) {
      const int fmt = fmts.begin()[i];
      RowsIn &v = *views.begin()[i++];
      if (fmt == RT_LINEAR_Q4K) {
        GemmLeft left{};
        r = launch_q4k_gemm_prepped(a16, ea, m.w, m.y, n, m.n, K, rest, st, &left, ews.begin()[i - 1]);
        v = left.ks > 1 ? RowsIn{left.part, left.ks, (size_t)n * m.n, m.n, 0} : rows_plain(m.y, m.n);
        rest += q4k_gemm_prepped_ws_bytes(n, m.n, K);
      } else {
        r = launch_proj_gemm_prepped(a16, ea, fmt, m.w, m.y, n, m.n, K, rest, st);
        v = rows_plain(m.y, m.n);
        rest += proj_gemm_prepped_ws_bytes(n, m.n, K);
      }
      if (r != hipSuccess) return r;
    }
    return hipSuccess;
  };
  if (plan.layer_begin == 0)
    PF_CHECK(hipLaunchKernelGGL(k_pf_embed, dim3(n), dim3(256), 0, st, plan.tokens, plan.tok_stride, a.embed,
                                a.embed_scale, b.hid, H));
  for (int li = plan.layer_begin; li < s.n_layers; ++li) {
    const LayerArgs &L = layers[li];
    const int cs_off = L.global ? D : 0;
    // (a tail run starts after its first layer's q|k|v step: q in b.q, K/V
    // in the cache)
    const bool qkv_step = !(plan.qkv_done && li == plan.layer_begin);
    if (li == 0 && qkv_step)
      PF_TRY(launch_pf_norm<false>(n, st, nullptr, rows_plain(b.hid, H), nullptr, L.g_in, nullptr, xn_f32, H, a.eps,
                                   stage, a16_h, ea_h));
    // q|k|v of a long prompt in Q4_K at head_dim 256: one launch whose
    // epilogue applies the q/k norms and RoPE and stores k and v straight into
    // the cache rows (no k_pf_qk_rope)
    const bool qkv_gemm = qkv_step && !plan.mb && !plan.p0_dev && L.fmt[kProjQ] == RT_LINEAR_Q4K &&
                          L.fmt[kProjK] == RT_LINEAR_Q4K && L.fmt[kProjV] == RT_LINEAR_Q4K && L.ew[kProjQ] &&
                          L.ew[kProjK] && L.ew[kProjV] && q4k_gemm_qkv_ok(n, QD, KVD, D);
    if (qkv_gemm) {
      const void *w3[3] = {L.wq, L.wk, L.wv};
      const int *ew3[3] = {L.ew[kProjQ], L.ew[kProjK], L.ew[kProjV]};
      PF_TRY(launch_q4k_gemm_qkv_prepped(gemm_a16(H), gemm_ea(H), w3, ew3, b.q, L.kc + (size_t)plan.p0 * KVD,
                                         L.vc + (size_t)plan.p0 * KVD, n, QD, KVD, H, plan.cs + cs_off,
                                         plan.cs_stride, L.g_q, L.g_k, a.eps, st));
    } else if (qkv_step) {
      PF_TRY(proj(plan.mb ? b.xn : nullptr, H, {L.fmt[kProjQ], L.fmt[kProjK], L.fmt[kProjV]},
                  {MbMat{L.wq, b.q, QD, 0, 0}, MbMat{L.wk, b.k, KVD, 0, 0}, MbMat{L.wv, b.v, KVD, 0, 0}},
                  {&vq, &vk, &vv}, {L.ew[kProjQ], L.ew[kProjK], L.ew[kProjV]}));
      const int items = n * (nq + nkv);
      if (D == 256)
        PF_CHECK(hipLaunchKernelGGL(k_pf_qk_rope<256>, dim3((items + 3) / 4), dim3(256), 0, st, vq, vk, vv, b.q,
                                    L.g_q, L.g_k, plan.cs, plan.cs_stride, cs_off, L.kc, L.vc, plan.p0, plan.p0_dev,
                                    n, nq, nkv, a.eps));
      else
        PF_CHECK(hipLaunchKernelGGL(k_pf_qk_rope<128>, dim3((items + 3) / 4), dim3(256), 0, st, vq, vk, vv, b.q,
                                    L.g_q, L.g_k, plan.cs, plan.cs_stride, cs_off, L.kc, L.vc, plan.p0, plan.p0_dev,
                                    n, nq, nkv, a.eps));
    }
    // The last layer's attention, o and FFN feed only the logits: a run that
    // needs no logits from these rows stops after the last K/V rows.
    if (plan.last_layer_kv_only && li == s.n_layers - 1) break;
    PfAttnArgs pa;
    pa.p0 = plan.p0;
    pa.p0_dev = plan.p0_dev;
    pa.n = n;
    pa.n_kv_heads = nkv;
    pa.lo_fixed = L.global ? 0 : plan.lo_fixed;
    pa.window = L.global ? 0 : plan.window;
    pa.scale = a.attn_scale;
    pa.split_stages = 0;
    pa.part_ml = b.attn_ml;
    pa.part_o = b.attn_o;
    // Rows before a fixed window start (the reference's prefill rule) see no
    // key: a key-split launch covers the rows from it on and its merge zeroes
    // the rest (row_base returns to 0 below when the keys are not split).
    if (!L.global && plan.lo_fixed > 0 && !plan.p0_dev && b.attn_ml)
      pa.row_base = std::min(std::max(plan.lo_fixed - plan.p0, 0), n - 1);
    int na = n - pa.row_base;
    dim3 agrid((na * G + 63) / 64, nkv);
    const bool causal = L.global || (plan.window <= 0 && plan.lo_fixed <= 0);
    if (agrid.x == 1 && b.attn_ml && n <= b.attn_rows) {
      // one row block: split the keys so about 256 workgroups share them
      const int span = causal ? plan.max_pos
                              : std::min(plan.max_pos, (plan.window > 0 ? plan.window : plan.max_pos) + n + 32);
      const int stages = (span + 31) / 32 + 1;
      pa.split_stages = (stages + kPfMaxSplits - 1) / kPfMaxSplits;
      agrid.z = (stages + pa.split_stages - 1) / pa.split_stages;
    } else if (!stage) {
      // Several row blocks with unequal key ranges (causal rows, the reference
      // window rule) or too few workgroups for the CUs (a short prompt): split
      // the keys as far as the partial buffers allow, so no workgroup walks
      // many more key stages than the average.
      const int splits_max = b.attn_ml ? std::min(kPfMaxSplits, b.attn_rows * kPfMaxSplits / na) : 0;
      // a row block of R rows walks at most window + R - 1 keys from a
      // 32-aligned start; R follows the launch's workgroup width
      const int rows_wg = ((na * G >= 256 ? 128 : 64) + G - 1) / G;
      const int span = causal ? plan.max_pos
                       : plan.window > 0 ? std::min(plan.max_pos, plan.window + rows_wg + 32)
                                         : std::max(plan.max_pos - plan.lo_fixed, 1);
      const int stages = (span + 31) / 32 + 1;
      // Causal rows: the last row block walks every key, the first one stage.
      if (splits_max >= 2 && (causal || plan.lo_fixed > 0 || (int)(agrid.x * agrid.y) < 512)) {
        pa.split_stages = std::max(4, (stages + splits_max - 1) / splits_max);
        agrid.z = (stages + pa.split_stages - 1) / pa.split_stages;
        if (agrid.z < 2) pa.split_stages = 0, agrid.z = 1;
      }
      if (!pa.split_stages) {
        pa.row_base = 0;  // the kernel writes the zero rows itself
        na = n;
        agrid.x = (na * G + 63) / 64;
      }
    }
    if (agrid.x == 1 || stage) pa.row_base = pa.split_stages ? pa.row_base : 0;
    if (stage && !pa.split_stages) return hipErrorInvalidValue;  // the batched path stages in the merge kernel
    // on the GEMM path a key-split merge writes the o projection's A itself
    // (rows that see no key have a zero attention row, so a zero o row: with
    // a Q4_K o the merge leaves them out, the o GEMM runs on the rows from
    // o_row0 on, and the norm below adds nothing for the rows before)
    int attn_row0 = -1;
    const bool o_q4k = L.fmt[kProjO] == RT_LINEAR_Q4K;
    if (D == 256)
      PF_TRY(launch_pf_attn<256>(G, agrid, st, b.q, L.kc, L.vc, b.attn, pa, stage, plan.mb ? nullptr : gemm_a16(QD),
                                 plan.mb ? nullptr : gemm_ea(QD), &attn_row0, o_q4k));
    else
      PF_TRY(launch_pf_attn<128>(G, agrid, st, b.q, L.kc, L.vc, b.attn, pa, stage));
    int o_row0 = 0;
    if (attn_row0 > 0) {
      o_row0 = attn_row0;
      const int m = n - o_row0;
      char *rest = static_cast<char *>(b.ws) + r256((size_t)n * kmax * 2) + r256((size_t)n * 4);
      GemmLeft left{};
      PF_TRY(launch_q4k_gemm_prepped(gemm_a16(QD) + (size_t)o_row0 * QD, gemm_ea(QD) + o_row0, L.wo,
                                     b.o + (size_t)o_row0 * H, m, H, QD, rest, st, &left, L.ew[kProjO]));
      // rows indexed from 0: the partial tiles of row t start (t - o_row0) rows in
      vo = left.ks > 1 ? RowsIn{left.part - (size_t)o_row0 * H, left.ks, (size_t)m * H, H, 0} : rows_plain(b.o, H);
    } else {
      PF_TRY(proj(attn_row0 >= 0 ? nullptr : b.attn, QD, {L.fmt[kProjO]}, {MbMat{L.wo, b.o, H, 0, 0}}, {&vo},
                  {L.ew[kProjO]}));
    }
    // gate|up: Q4_K pairs that would run as one set launch form h = gelu(g)*u
    // in the GEMM itself, written as the down GEMM's f16 A operand (rows in
    // b.g, exponents in b.u) with exponents from |xn|^2 of each row, which the
    // norm returns
    const bool gelu_gemm = !plan.mb && L.fmt[kProjGate] == RT_LINEAR_Q4K && L.fmt[kProjUp] == RT_LINEAR_Q4K &&
                           L.ew[kProjGate] && L.ew[kProjUp] && L.gu_bound > 0.f && q4k_gemm_gelu_ok(n, F);
    float *xn_nrm2 = b.nrm2;
    PF_TRY(launch_pf_norm<true>(n, st, b.hid, vo, L.g_post_attn, L.g_pre_ffn, b.x2, xn_f32, H, a.eps, stage, a16_h,
                                ea_h, gelu_gemm ? xn_nrm2 : nullptr, o_row0));
    _Float16 *h16 = reinterpret_cast<_Float16 *>(b.g);
    int *eh = reinterpret_cast<int *>(b.u);
    if (gelu_gemm) {
      PF_TRY(launch_q4k_gemm_gelu_prepped(gemm_a16(H), gemm_ea(H), xn_nrm2, L.wgate, L.wup, L.ew[kProjGate],
                                          L.ew[kProjUp], L.gu_bound, h16, eh, n, F, H, st));
    } else {
      PF_TRY(proj(plan.mb ? b.xn : nullptr, H, {L.fmt[kProjGate], L.fmt[kProjUp]},
                  {MbMat{L.wgate, b.g, F, 0, 0}, MbMat{L.wup, b.u, F, 0, 0}}, {&vg, &vu},
                  {L.ew[kProjGate], L.ew[kProjUp]}));
      if (plan.mb) {
        const size_t n4 = (size_t)n * F / 4;
        const unsigned eg = (unsigned)std::min<size_t>((n4 + 255) / 256, 4096);
        PF_CHECK(hipLaunchKernelGGL(k_pf_gelu_mul, dim3(eg), dim3(256), 0, st, vg, vu, b.g, n, F, stage));
      } else {
        PF_CHECK(
            hipLaunchKernelGGL(k_pf_gelu_rows, dim3(n), dim3(kGeluRowT), 0, st, vg, vu, F, gemm_a16(F), gemm_ea(F)));
      }
    }
    PF_TRY(proj(plan.mb ? b.g : nullptr, F, {L.fmt[kProjDown]}, {MbMat{L.wdown, b.dn, H, 0, 0}}, {&vd},
                {L.ew[kProjDown]}, gelu_gemm ? h16 : nullptr, gelu_gemm ? eh : nullptr));
    if (li + 1 < s.n_layers)
      PF_TRY(launch_pf_norm<true>(n, st, b.x2, vd, L.g_post_ffn, layers[li + 1].g_in, b.hid, xn_f32, H, a.eps,
                                  stage, a16_h, ea_h));
  }
  const LayerArgs &last = layers[s.n_layers - 1];
  if (plan.logits != RowsPlan::kNone) {
    // the final residual and final norm of every row (transformer4.rs:2131-2139,
    // 2370-2380), then the tied lm_head of the last row or of every row
    float *xn_out = plan.logits == RowsPlan::kEveryRow ? plan.xn_b : b.xn;
    PF_TRY(launch_pf_norm<true>(n, st, b.x2, vd, last.g_post_ffn, a.g_final,
                                b.hid, xn_out, H, a.eps, nullptr));
    if (plan.logits == RowsPlan::kEveryRow)
      PF_TRY(enqueue_lm_head_batch(s, a, plan.xn_b, plan.logits_b, n, st));
    else
      PF_TRY(enqueue_lm_head_batch(s, a, b.xn + (size_t)(n - 1) * H, a.logits, 1, st));
  }
#undef PF_CHECK
#undef PF_TRY
  return hipSuccess;
}

}  // namespace rt
