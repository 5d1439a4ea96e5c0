// decode_kernels.hip -- the fused kernels of one Gemma-3 decode step.
//
// Per layer six launches replace the reference's 21 dispatches
// (metal_decode.rs:1930-2024):
//   k_qkv      residual+post-FFN norm of the previous layer (or the embedding
//              row for layer 0), input RMSNorm, then one GEMV over the stacked
//              q|k|v rows;
//   k_attn     q/k per-head RMSNorm + NeoX RoPE, K/V append at `pos`, split-K
//              attention over the f32 cache (per-chunk softmax partials);
//   k_attn_combine  merge of the chunk partials into the attention output;
//   k_gemv     o projection;
//   k_gateup   residual + post-attention norm, pre-FFN norm, gate and up
//              GEMVs of the same rows (persistent tiles), gelu_tanh(gate)*up;
//   k_gemv     down projection.
// After the last layer k_lmhead applies the final residual, the final norm
// and the BF16 lm_head GEMV.  Token id and position are read from device
// memory so the whole step replays as one hipGraph.
#include <algorithm>
#include <vector>

#include "../../include/rt_hip.h"
#include "decode.hpp"
#include "gemma3_math.hpp"
#include "q4k_gemv.hpp"
#include "q4k_gemv_mb.hpp"
#include "kquant_tile.hpp"
#include "rt_device.hpp"
#include "rt_kernels.hpp"
#include "rt_capi_util.hpp"

namespace rt {

// ---------------------------------------------------------------------------
// Optional per-wave timeline of the decode step (built with RT_TRACE=1,
// `make -C rich-triplet_amd trace`; off in librt_hip.so, where every call
// below compiles to nothing).  Each traced kernel records, per wave, the
// 100 MHz real-time counter at entry, once its activation (or prologue)
// staging is done, once all its loads have landed (an explicit wait, which
// the traced build adds) and at exit.  Every launch of a kernel overwrites
// its slots, so after a step they hold the last layer's launches.
// ---------------------------------------------------------------------------
#ifndef RT_TRACE
#define RT_TRACE 0
#endif
constexpr bool kTrace = RT_TRACE != 0;
constexpr int kTraceKernels = 7, kTraceSlots = 8192;  // qkv, attn, merge, o, gateup, down, lm_head
enum TraceKernel { kTrQkv = 0, kTrAttn, kTrMerge, kTrO, kTrGateup, kTrDown, kTrHead };
__device__ unsigned long long g_trace[kTrace ? kTraceKernels : 1][kTrace ? kTraceSlots : 1][4];

struct Trace {
  unsigned long long t[3] = {0, 0, 0};
  RT_DEV void mark(int i) {
    if constexpr (kTrace) t[i] = __builtin_amdgcn_s_memrealtime();
  }
  // stamp 2: wait for every outstanding load of the wave first
  RT_DEV void mark_landed() {
    if constexpr (kTrace) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      t[2] = __builtin_amdgcn_s_memrealtime();
    }
  }
  RT_DEV void put(int kernel, int slot) const {
    if constexpr (kTrace) {
      const unsigned long long t3 = __builtin_amdgcn_s_memrealtime();
      if ((threadIdx.x & 63) == 0 && slot < kTraceSlots) {
        unsigned long long *p = g_trace[kernel][slot];
        p[0] = t[0], p[1] = t[1], p[2] = t[2], p[3] = t3;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Prologues: build the normalised activation vector in the LDS x layout.
// ---------------------------------------------------------------------------
enum class Pro { Embed, Resid };

// x = Embed: bf16(E[token]) * embed_scale        (transformer4.rs:2360-2368)
//     Resid: base + rms(add)*(1+g_add)           (post-norm residual, 1954-1964)
// then xn = rms(x)*(1+g_out) into LDS; workgroup 0 stores x to x_out.
// pro_load issues every global load of the prologue (call it before the
// weight loads); pro_finish does the arithmetic and the LDS stores.
template <int K, int T>
struct ProRegs {
  static constexpr int F4 = K / 4;
  static constexpr int PER = (F4 + T - 1) / T;
  float4 add[PER], base[PER], ga[PER], go[PER];
};

template <int K, int T, Pro MODE>
RT_DEV void pro_load(const DecodeArgs &a, const float *__restrict__ base, const float *__restrict__ add,
                     const float *__restrict__ g_add, const float *__restrict__ g_out, ProRegs<K, T> &r) {
  using R = ProRegs<K, T>;
  // Unconditional 16-byte loads at a clamped index (entries past the end are
  // never stored): branch-free loads keep their own s_waitcnt.
#pragma unroll
  for (int i = 0; i < R::PER; ++i) {
    const int f = min((int)threadIdx.x + i * T, R::F4 - 1);
    if constexpr (MODE == Pro::Embed) {
      const uint2 w = reinterpret_cast<const uint2 *>(a.embed + (size_t)a.params[0] * K)[f];
      r.add[i] = make_float4(mul_nc(bf16_lo(w.x), a.embed_scale), mul_nc(bf16_hi(w.x), a.embed_scale),
                             mul_nc(bf16_lo(w.y), a.embed_scale), mul_nc(bf16_hi(w.y), a.embed_scale));
    } else {
      r.add[i] = reinterpret_cast<const float4 *>(add)[f];
      r.base[i] = reinterpret_cast<const float4 *>(base)[f];
      r.ga[i] = reinterpret_cast<const float4 *>(g_add)[f];
    }
    r.go[i] = reinterpret_cast<const float4 *>(g_out)[f];
  }
}

// `red`: 2*T/64 floats of LDS, one half per reduction (no barrier between
// them protects a reused array).
template <int K, int T, Pro MODE, bool DIG = false>
RT_DEV void pro_finish(const DecodeArgs &a, ProRegs<K, T> &r, float *__restrict__ x_out, void *lds, float *red,
                       float *__restrict__ xn_out = nullptr) {
  using R = ProRegs<K, T>;
  const float inv_k = 1.0f / (float)K;
  float4 *x = r.add;  // Embed: the embedding row; Resid: overwritten with the residual sum
  auto live = [&](int i) { return (int)threadIdx.x + i * T < R::F4; };
  if constexpr (MODE == Pro::Resid) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < R::PER; ++i) ss += live(i) ? sumsq4(r.add[i]) : 0.f;
    const float ra = rms_inv_from_sumsq(block_sum_fresh<T>(ss, red + T / 64), inv_k, a.eps);
#pragma unroll
    for (int i = 0; i < R::PER; ++i) x[i] = add4(r.base[i], norm4(r.add[i], ra, r.ga[i]));
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < R::PER; ++i) ss += live(i) ? sumsq4(x[i]) : 0.f;
  const float rx = rms_inv_from_sumsq(block_sum_fresh<T>(ss, red), inv_k, a.eps);
#pragma unroll
  for (int i = 0; i < R::PER; ++i) {
    const int f = threadIdx.x + i * T;
    if (f < R::F4) {
      const float4 xn = norm4(x[i], rx, r.go[i]);
      if (blockIdx.x == 0) {
        if (x_out) reinterpret_cast<float4 *>(x_out)[f] = x[i];
        if (xn_out) reinterpret_cast<float4 *>(xn_out)[f] = xn;
      }
      if constexpr (DIG)
        stage_digits_store(static_cast<uint32_t *>(lds), f, xn);
      else
        stage_x_store(static_cast<float *>(lds), f, xn);
    }
  }
}

// ---------------------------------------------------------------------------
// k_qkv: [prologue] + GEMV over q|k|v rows (each workgroup inside one matrix).
// V6: v is Q6_K (planar), as in Q4_K_M files; its workgroups run the Q6_K
// tile on the same staged input, so the layer keeps one launch for q|k|v.
// ---------------------------------------------------------------------------
template <int NB, int T, int ITERS, Pro MODE, bool V6 = false>
__global__ __launch_bounds__(T) void k_qkv(DecodeArgs a, LayerArgs L, LayerArgs prev) {
  Trace tr;
  tr.mark(0);
  using Tile = Q4KTile<NB, T, ITERS>;
  using Tile6 = Q6KTile<NB, T, ITERS>;
  static_assert(Tile6::ROWS == Tile::ROWS, "both tiles cover the same rows per workgroup");
  constexpr int K = NB * 256;
  __shared__ __attribute__((aligned(16))) uint32_t dl[NB * 4 * kDPitch];
  __shared__ float red[Tile::ROWS * NB];
  __shared__ float bred[2 * (T / 64)];
  ProRegs<K, T> pr;
  pro_load<K, T, MODE>(a, a.x2, a.dn, prev.g_post_ffn, L.g_in, pr);
  // the matrix of this workgroup, picked by selects once the prologue loads
  // are out (branches here load their arguments in a round of their own)
  const int qd = a.n_q_heads * a.head_dim, kvd = a.n_kv_heads * a.head_dim;
  const int row0 = (int)blockIdx.x * Tile::ROWS;  // ROWS divides qd and kvd (checked on the host)
  const bool in_q = row0 < qd, in_k = !in_q && row0 < qd + kvd;
  const uint8_t *W = in_q ? L.wq : (in_k ? L.wk : L.wv);
  float *y = in_q ? a.q : (in_k ? a.k : a.v);
  const int r0 = row0 - (in_q ? 0 : (in_k ? qd : qd + kvd));
  const bool six = V6 && row0 >= qd + kvd;  // workgroup-uniform
  const size_t row_bytes = (size_t)NB * kQ4KBlockBytes;
  // every wave's prologue loads go out before any weight load of the
  // workgroup: they return ahead of the weight stream
  __syncthreads();
  Tile tile;
  Tile6 tile6;
  if (six)
    tile6.load(q6k_planes(L.wv, (size_t)kvd * NB), r0, kvd);
  else
    tile.load([&](int rl) -> const uint8_t * { return W + (size_t)(r0 + rl) * row_bytes; }, W);
  pro_finish<K, T, MODE, true>(a, pr, a.hid, dl, bred, a.xn);
  __syncthreads();
  tr.mark(1);
  tr.mark_landed();
  if (six) {
    tile6.compute(dl, red);
  } else {
    ChunkD cx;
    chunkd_from_lds(dl, tile.slot, cx);
    tile.compute_digits(cx, red);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < Tile::ROWS; i += T) y[r0 + i] = reduce_row<NB>(red, i);
  tr.put(kTrQkv, (int)blockIdx.x * (T / 64) + (int)(threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------
// Split projection sets (a projection that is not Q4_K): k_prologue forms the
// same x and normalised xn as the fused kernels' prologues, one workgroup,
// into global memory; the projections then run as plain GEMVs of their
// format, and k_gelu_mul_vec finishes a split gate/up pair.
// ---------------------------------------------------------------------------
template <int K, Pro MODE>
__global__ __launch_bounds__(256) void k_prologue(DecodeArgs a, const float *__restrict__ base,
                                                  const float *__restrict__ add, const float *__restrict__ g_add,
                                                  const float *__restrict__ g_out, float *__restrict__ x_out,
                                                  float *__restrict__ xn_out) {
  constexpr int T = 256;
  __shared__ float bred[2 * (T / 64)];
  ProRegs<K, T> pr;
  pro_load<K, T, MODE>(a, base, add, g_add, g_out, pr);
  using R = ProRegs<K, T>;
  const float inv_k = 1.0f / (float)K;
  auto live = [&](int i) { return (int)threadIdx.x + i * T < R::F4; };
  float4 *x = pr.add;
  if constexpr (MODE == Pro::Resid) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < R::PER; ++i) ss += live(i) ? sumsq4(pr.add[i]) : 0.f;
    const float ra = rms_inv_from_sumsq(block_sum<T>(ss, bred), inv_k, a.eps);
#pragma unroll
    for (int i = 0; i < R::PER; ++i) x[i] = add4(pr.base[i], norm4(pr.add[i], ra, pr.ga[i]));
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < R::PER; ++i) ss += live(i) ? sumsq4(x[i]) : 0.f;
  const float rx = rms_inv_from_sumsq(block_sum<T>(ss, bred), inv_k, a.eps);
#pragma unroll
  for (int i = 0; i < R::PER; ++i)
    if (live(i)) {
      const int f = threadIdx.x + i * T;
      reinterpret_cast<float4 *>(x_out)[f] = x[i];
      reinterpret_cast<float4 *>(xn_out)[f] = norm4(x[i], rx, pr.go[i]);
    }
}

// gelu_tanh of n values (the activation of the decode step and prefill).
__global__ __launch_bounds__(256) void k_gelu_tanh(const float *__restrict__ x, float *__restrict__ y, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) y[i] = gelu_tanh(x[i]);
}

hipError_t launch_gelu_tanh(const float *x, float *y, size_t n, hipStream_t s) {
  const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(k_gelu_tanh, dim3(grid), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_gelu_mul_vec(float *h, const float *__restrict__ u, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) h[i] = mul_nc(gelu_tanh(h[i]), u[i]);
}

// ---------------------------------------------------------------------------
// k_gateup: x2 = hid + rms(o)(1+g_pa); n2 = rms(x2)(1+g_pf); each workgroup
// then computes GR gate rows and the same GR up rows, walked as one list of
// 2*GR rows (gate first) in iterations of RPI rows, and stores
// h[j] = gelu_tanh(gate[j]) * up[j]  (transformer4.rs:328-334)
// ---------------------------------------------------------------------------
template <int NB, int T, int GR>
__global__ __launch_bounds__(T) void k_gateup(DecodeArgs a, LayerArgs L) {
  Trace tr;
  tr.mark(0);
  constexpr int RPI = T / (4 * NB);
  using Tile = Q4KTile<NB, T, (2 * GR + RPI - 1) / RPI>;
  constexpr int K = NB * 256;
  __shared__ __attribute__((aligned(16))) uint32_t dl[NB * 4 * kDPitch];
  __shared__ float red[Tile::ROWS * NB];
  __shared__ float bred[2 * (T / 64)];
  const size_t row_bytes = (size_t)NB * kQ4KBlockBytes;
  const int j0 = (int)blockIdx.x * GR;  // GR divides ffn (checked on the host)
  ProRegs<K, T> pr;
  pro_load<K, T, Pro::Resid>(a, a.hid, a.o, L.g_post_attn, L.g_pre_ffn, pr);
  // every wave's prologue loads go out before any weight load of the
  // workgroup: they return ahead of its weight stream
  __syncthreads();
  Tile tile;
  tile.load([&](int rl) -> const uint8_t * {
    return rl < GR ? L.wgate + (size_t)(j0 + rl) * row_bytes
                   : (rl < 2 * GR ? L.wup + (size_t)(j0 + rl - GR) * row_bytes : nullptr);
  }, L.wgate);
  pro_finish<K, T, Pro::Resid, true>(a, pr, a.x2, dl, bred);
  __syncthreads();
  tr.mark(1);
  tr.mark_landed();
  tile.compute_digits_lds(dl, red);
  __syncthreads();
  for (int i = threadIdx.x; i < GR; i += T) {
    const float g = reduce_row<NB>(red, i);
    const float u = reduce_row<NB>(red, GR + i);
    a.h[j0 + i] = mul_nc(gelu_tanh(g), u);
  }
  tr.put(kTrGateup, (int)blockIdx.x * (T / 64) + (int)(threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------
// The same two launches for a layer whose q, k, v (k_qkv8) or gate, up
// (k_gateup8) are Q8_0 (planar: codes [n][K] | f16 scales [n][K/32]), as in
// Q8_0 files: the prologue and the staged digits as above, then Q8Tile
// (kquant_tile.hpp) rows, 16 per workgroup at K = 2560 like the Q4_K tiles.
// ---------------------------------------------------------------------------
template <int NB32, int T, int ITERS, Pro MODE>
__global__ __launch_bounds__(T) void k_qkv8(DecodeArgs a, LayerArgs L, LayerArgs prev) {
  using Tile = Q8Tile<NB32, T, ITERS>;
  constexpr int K = NB32 * 32;
  __shared__ __attribute__((aligned(16))) uint32_t dl[K / 64 * kDPitch];
  __shared__ float red[Tile::ROWS * Tile::RED];
  __shared__ float bred[2 * (T / 64)];
  const int qd = a.n_q_heads * a.head_dim, kvd = a.n_kv_heads * a.head_dim;
  const int row0 = (int)blockIdx.x * Tile::ROWS;  // ROWS divides qd and kvd (checked on the host)
  const uint8_t *W;
  float *y;
  int r0, nrows;
  if (row0 < qd) {
    W = L.wq, y = a.q, r0 = row0, nrows = qd;
  } else if (row0 < qd + kvd) {
    W = L.wk, y = a.k, r0 = row0 - qd, nrows = kvd;
  } else {
    W = L.wv, y = a.v, r0 = row0 - qd - kvd, nrows = kvd;
  }
  const uint16_t *D = reinterpret_cast<const uint16_t *>(W + (size_t)nrows * K);
  ProRegs<K, T> pr;
  pro_load<K, T, MODE>(a, a.x2, a.dn, prev.g_post_ffn, L.g_in, pr);
  __syncthreads();
  Tile tile;
  tile.load([&](int rl) { return W + (size_t)(r0 + rl) * K; }, [&](int rl) { return D + (size_t)(r0 + rl) * NB32; });
  pro_finish<K, T, MODE, true>(a, pr, a.hid, dl, bred, a.xn);
  __syncthreads();
  tile.compute(dl, red);
  __syncthreads();
  for (int i = threadIdx.x; i < Tile::ROWS; i += T) y[r0 + i] = Tile::reduce(red, i);
}

template <int NB32, int T, int GR>
__global__ __launch_bounds__(T) void k_gateup8(DecodeArgs a, LayerArgs L, int ffn) {
  constexpr int RPI = T / NB32;
  using Tile = Q8Tile<NB32, T, (2 * GR + RPI - 1) / RPI>;
  constexpr int K = NB32 * 32;
  __shared__ __attribute__((aligned(16))) uint32_t dl[K / 64 * kDPitch];
  __shared__ float red[Tile::ROWS * Tile::RED];
  __shared__ float bred[2 * (T / 64)];
  const int j0 = (int)blockIdx.x * GR;  // GR divides ffn (checked on the host)
  const uint16_t *Dg = reinterpret_cast<const uint16_t *>(L.wgate + (size_t)ffn * K);
  const uint16_t *Du = reinterpret_cast<const uint16_t *>(L.wup + (size_t)ffn * K);
  ProRegs<K, T> pr;
  pro_load<K, T, Pro::Resid>(a, a.hid, a.o, L.g_post_attn, L.g_pre_ffn, pr);
  Tile tile;
  // tile rows [0, GR) are gate rows j0.., [GR, 2GR) the same up rows; slots
  // past 2GR re-read the last up row and are never stored
  tile.load([&](int rl) {
    return rl < GR ? L.wgate + (size_t)(j0 + rl) * K : L.wup + (size_t)(j0 + min(rl - GR, GR - 1)) * K;
  }, [&](int rl) {
    return rl < GR ? Dg + (size_t)(j0 + rl) * NB32 : Du + (size_t)(j0 + min(rl - GR, GR - 1)) * NB32;
  });
  pro_finish<K, T, Pro::Resid, true>(a, pr, a.x2, dl, bred);
  __syncthreads();
  tile.compute(dl, red);
  __syncthreads();
  for (int i = threadIdx.x; i < GR; i += T)
    a.h[j0 + i] = mul_nc(gelu_tanh(Tile::reduce(red, i)), Tile::reduce(red, GR + i));
}

// ---------------------------------------------------------------------------
// And for BF16 q, k, v (k_qkv16) or gate, up (k_gateup16), as in BF16 files:
// the prologue stages xn in LDS as f32 (k_lmhead's layout), then one wave per
// row as in the BF16 GEMV: lane l holds elements (64 i + l) * 8 .. + 8 of the
// row for i < CPL (K = 512 CPL), two rows' loads in flight per wave.
// ---------------------------------------------------------------------------
template <int CPL>
RT_DEV float bf16_dot_lane(const uint4 (&w)[CPL], const float (&xr)[CPL][8]) {
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    acc0 += bf16_lo(w[i].x) * xr[i][0];
    acc1 += bf16_hi(w[i].x) * xr[i][1];
    acc0 += bf16_lo(w[i].y) * xr[i][2];
    acc1 += bf16_hi(w[i].y) * xr[i][3];
    acc0 += bf16_lo(w[i].z) * xr[i][4];
    acc1 += bf16_hi(w[i].z) * xr[i][5];
    acc0 += bf16_lo(w[i].w) * xr[i][6];
    acc1 += bf16_hi(w[i].w) * xr[i][7];
  }
  return wave_sum(acc0 + acc1);
}

template <int CPL>
RT_DEV void bf16_x_from_lds(const float *xl, float (&xr)[CPL][8]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < CPL; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) xr[i][j] = xl[xlds_index((i * 64 + lane) * 8 + j)];
}

template <int CPL, Pro MODE>
__global__ __launch_bounds__(256) void k_qkv16(DecodeArgs a, LayerArgs L, LayerArgs prev) {
  constexpr int K = CPL * 512;
  __shared__ __attribute__((aligned(16))) float xl[K / 64 * kXPitch];
  __shared__ float bred[8];
  ProRegs<K, 256> pr;
  pro_load<K, 256, MODE>(a, a.x2, a.dn, prev.g_post_ffn, L.g_in, pr);
  pro_finish<K, 256, MODE>(a, pr, a.hid, xl, bred, a.xn);
  __syncthreads();
  float xr[CPL][8];
  bf16_x_from_lds<CPL>(xl, xr);
  const int lane = threadIdx.x & 63;
  const int qd = a.n_q_heads * a.head_dim, kvd = a.n_kv_heads * a.head_dim, total = qd + 2 * kvd;
  const int wave = (int)((blockIdx.x * 256u + threadIdx.x) >> 6), nwaves = (int)(gridDim.x * 4u);
  // rows r0, r0 + 1 of the stacked q|k|v (qd and kvd are even: a pair never
  // straddles two matrices)
  for (int r0 = 2 * wave; r0 < total; r0 += 2 * nwaves) {
    const uint16_t *W;
    float *y;
    int lr;
    if (r0 < qd) {
      W = reinterpret_cast<const uint16_t *>(L.wq), y = a.q, lr = r0;
    } else if (r0 < qd + kvd) {
      W = reinterpret_cast<const uint16_t *>(L.wk), y = a.k, lr = r0 - qd;
    } else {
      W = reinterpret_cast<const uint16_t *>(L.wv), y = a.v, lr = r0 - qd - kvd;
    }
    uint4 w0[CPL], w1[CPL];
    const uint4 *p0 = reinterpret_cast<const uint4 *>(W + (size_t)lr * K), *p1 = p0 + K / 8;
#pragma unroll
    for (int i = 0; i < CPL; ++i) w0[i] = ld_nt16(p0 + i * 64 + lane), w1[i] = ld_nt16(p1 + i * 64 + lane);
    const float d0 = bf16_dot_lane<CPL>(w0, xr), d1 = bf16_dot_lane<CPL>(w1, xr);
    if (lane == 0) y[lr] = d0, y[lr + 1] = d1;
  }
}

template <int CPL>
__global__ __launch_bounds__(256) void k_gateup16(DecodeArgs a, LayerArgs L, int ffn) {
  constexpr int K = CPL * 512;
  __shared__ __attribute__((aligned(16))) float xl[K / 64 * kXPitch];
  __shared__ float bred[8];
  ProRegs<K, 256> pr;
  pro_load<K, 256, Pro::Resid>(a, a.hid, a.o, L.g_post_attn, L.g_pre_ffn, pr);
  pro_finish<K, 256, Pro::Resid>(a, pr, a.x2, xl, bred);
  __syncthreads();
  float xr[CPL][8];
  bf16_x_from_lds<CPL>(xl, xr);
  const int lane = threadIdx.x & 63;
  const int wave = (int)((blockIdx.x * 256u + threadIdx.x) >> 6), nwaves = (int)(gridDim.x * 4u);
  const uint16_t *Wg = reinterpret_cast<const uint16_t *>(L.wgate), *Wu = reinterpret_cast<const uint16_t *>(L.wup);
  for (int j = wave; j < ffn; j += nwaves) {  // gate row j and up row j: h[j] = gelu(g) u
    uint4 wg[CPL], wu[CPL];
    const uint4 *pg = reinterpret_cast<const uint4 *>(Wg + (size_t)j * K);
    const uint4 *pu = reinterpret_cast<const uint4 *>(Wu + (size_t)j * K);
#pragma unroll
    for (int i = 0; i < CPL; ++i) wg[i] = ld_nt16(pg + i * 64 + lane), wu[i] = ld_nt16(pu + i * 64 + lane);
    const float g = bf16_dot_lane<CPL>(wg, xr), u = bf16_dot_lane<CPL>(wu, xr);
    if (lane == 0) a.h[j] = mul_nc(gelu_tanh(g), u);
  }
}

// ---------------------------------------------------------------------------
// k_gemv: plain GEMV with the activation vector read from global memory.
// ---------------------------------------------------------------------------
template <int NB, int T, int ITERS>
__global__ __launch_bounds__(T) void k_gemv(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                            float *__restrict__ y, int n) {
  Trace tr;
  tr.mark(0);
  using Tile = Q4KTile<NB, T, ITERS>;
  __shared__ __attribute__((aligned(16))) uint32_t dl[NB * 4 * kDPitch];
  __shared__ float red[Tile::ROWS * NB];
  const int row0 = (int)blockIdx.x * Tile::ROWS;
  const size_t row_bytes = (size_t)NB * kQ4KBlockBytes;
  XRegs<NB * 256, T> xr;
  x_load<NB * 256, T>(x, xr);
  // With a 40 KB activation vector every wave's activation loads go out
  // before any weight load of the workgroup, so they do not queue behind
  // the first waves' weight stream (smaller vectors do better without the
  // barrier)
  if constexpr (NB >= 40) __syncthreads();
  Tile tile;
  tile.load([&](int rl) -> const uint8_t * {
    return row0 + rl < n ? W + (size_t)(row0 + rl) * row_bytes : nullptr;
  }, W);
  x_store_digits<NB * 256, T>(xr, dl);
  __syncthreads();
  tr.mark(1);
  tr.mark_landed();
  ChunkD cx;
  chunkd_from_lds(dl, tile.slot, cx);
  tile.compute_digits(cx, red);
  __syncthreads();
  for (int i = threadIdx.x; i < Tile::ROWS; i += T)
    if (row0 + i < n) y[row0 + i] = reduce_row<NB>(red, i);
  tr.put(NB == 40 ? kTrDown : kTrO, (int)blockIdx.x * (T / 64) + (int)(threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------
// k_attn: one layer's attention for the token at `pos` (gqa_attention_cached's
// t_q == 1 branch, transformer4.rs:2806-2879).  Grid (key chunk, KV head);
// a workgroup of WAVES waves takes a chunk of up to KPW*WAVES keys and each
// wave walks its own KPW keys with a private softmax, so the key loop has no
// barrier.  A lane holds D/64 consecutive dimensions of every vector (q, K
// row, V row, output), so each K and V row is one coalesced wave load.
//   1. Every wave forms the per-head RMSNorm (gamma shared, 2485-2508) and
//      NeoX RoPE (2742-2772) of its G q heads itself, from the step's cos/sin
//      table; the wave whose keys hold `pos` also normalises and rotates k,
//      takes v, uses both for that key and writes them into cache row `pos`
//      (1813-1823).
//   2. s_c = (q . k_c) * scale per key (a wave sum), m = max s_c, p_c =
//      e^(s_c - m), l = sum p_c, o = sum p_c v_c over the wave's keys.
//   3. The waves' (m, l, o) merge through LDS into the chunk's partial
//      (rescaled by e^(m_w - M)); k_attn_combine then merges the chunks.
// ---------------------------------------------------------------------------
template <int D>
struct LaneRow {
  static constexpr int N = D / 64;  // dimensions per lane: lane l holds [N*l, N*l + N)
  float v[N];
  // N floats at row + N*idx (idx = lane for a whole row)
  RT_DEV void load(const float *__restrict__ row, int idx) {
    if constexpr (N == 4) {
      const float4 t = reinterpret_cast<const float4 *>(row)[idx];
      v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
    } else {
      const float2 t = reinterpret_cast<const float2 *>(row)[idx];
      v[0] = t.x, v[1] = t.y;
    }
  }
  RT_DEV void store(float *row, int idx) const {
    if constexpr (N == 4)
      reinterpret_cast<float4 *>(row)[idx] = make_float4(v[0], v[1], v[2], v[3]);
    else
      reinterpret_cast<float2 *>(row)[idx] = make_float2(v[0], v[1]);
  }
};

// Per-head RMSNorm and NeoX RoPE of one head held as a LaneRow (the
// arithmetic of norm_rope_head_regs): lanes 0..31 hold the pairs' first
// elements i < D/2, lanes 32..63 their partners i + D/2, exchanged across
// the halves.  cs/sn: the cos and sin of the lane's pairs (table entries
// N*(lane & 31) ..).
template <int D>
RT_DEV void norm_rope_lane(LaneRow<D> &x, const LaneRow<D> &g, const LaneRow<D> &cs, const LaneRow<D> &sn,
                           float eps) {
  constexpr int N = D / 64;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < N; ++j) ss += x.v[j] * x.v[j];
  const float rinv = rms_inv_from_sumsq(wave_sum(ss), 1.0f / (float)D, eps);
  const bool upper = (threadIdx.x & 63) >= 32;
#pragma unroll
  for (int j = 0; j < N; ++j) {
#pragma clang fp contract(off)
    const float a = (x.v[j] * rinv) * (1.0f + g.v[j]);
    const float b = __shfl_xor(a, 32);
    x.v[j] = upper ? b * sn.v[j] + a * cs.v[j] : a * cs.v[j] - b * sn.v[j];
  }
}

template <int D, int G, int KPW, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_attn(DecodeArgs a, LayerArgs L) {
  Trace tr;
  tr.mark(0);
  constexpr int N = D / 64, NT = 64 * WAVES;
  static_assert(D == 128 || D == 256, "head_dim 128 or 256");
  __shared__ float sm_ml[WAVES][G][2];
  __shared__ __attribute__((aligned(16))) float sm_o[WAVES][G][D];
  const int kvh = blockIdx.y, chunk = blockIdx.x, nchunk = gridDim.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kvd = a.n_kv_heads * D;

  // loads, in the order they are consumed (vector loads return in order):
  // q heads and the norm / RoPE inputs, then K rows, then V rows; rows past
  // the wave's keys re-read its last row (or row 0) and are masked.  The
  // first group does not depend on the step's position, so it goes out
  // before the position (a load from the parameter block) has landed.
  LaneRow<D> q[G], gq, cs, sn, kn, vn, gk;
#pragma unroll
  for (int g = 0; g < G; ++g) q[g].load(a.q + (size_t)(kvh * G + g) * D, lane);
  gq.load(L.g_q, lane);
  cs.load(L.rope_cs, lane & 31);
  sn.load(L.rope_cs + D / 2, lane & 31);
  kn.load(a.k + (size_t)kvh * D, lane);
  vn.load(a.v + (size_t)kvh * D, lane);
  gk.load(L.g_k, lane);
  __builtin_amdgcn_sched_barrier(0);
  const int pos = a.params[1];
  const int t_end = pos + 1;
  const int t_start = L.window > 0 ? max(0, t_end - L.window) : 0;
  const int csize = (t_end - t_start + nchunk - 1) / nchunk;  // <= KPW*WAVES: the host sizes nchunk
  const int c0 = t_start + chunk * csize, c1 = min(c0 + csize, t_end);
  const int kw = (csize + WAVES - 1) / WAVES;  // <= KPW
  const int w0 = c0 + wave * kw, w1 = min(w0 + kw, c1);
  const int nk = max(0, w1 - w0);  // wave-uniform
  const bool owner = w0 <= pos && pos < w1;
  const int last = max(w1 - 1, 0);
  LaneRow<D> kr[KPW], vr[KPW];
#pragma unroll
  for (int k = 0; k < KPW; ++k) kr[k].load(L.kc + (size_t)min(w0 + k, last) * kvd + (size_t)kvh * D, lane);
#pragma unroll
  for (int k = 0; k < KPW; ++k) vr[k].load(L.vc + (size_t)min(w0 + k, last) * kvd + (size_t)kvh * D, lane);
  __builtin_amdgcn_sched_barrier(0);

  // 1. q heads; the new key and value at `pos`
#pragma unroll
  for (int g = 0; g < G; ++g) norm_rope_lane<D>(q[g], gq, cs, sn, a.eps);
  if (owner) {
    norm_rope_lane<D>(kn, gk, cs, sn, a.eps);
    kn.store(L.kc + (size_t)pos * kvd + (size_t)kvh * D, lane);
    vn.store(L.vc + (size_t)pos * kvd + (size_t)kvh * D, lane);
#pragma unroll
    for (int k = 0; k < KPW; ++k)
      if (w0 + k == pos) kr[k] = kn, vr[k] = vn;
  }

  tr.mark(1);
  tr.mark_landed();
  // 2. scores, softmax and values of this wave's keys
  float m[G], l[G];
  LaneRow<D> o[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float s[KPW];
#pragma unroll
    for (int k = 0; k < KPW; ++k) {
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < N; ++j) d += q[g].v[j] * kr[k].v[j];
      s[k] = wave_sum(d) * a.attn_scale;
    }
    m[g] = -INFINITY;
#pragma unroll
    for (int k = 0; k < KPW; ++k)
      if (k < nk) m[g] = fmaxf(m[g], s[k]);
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j) o[g].v[j] = 0.f;
#pragma unroll
    for (int k = 0; k < KPW; ++k) {
      const float p = k < nk ? expf(s[k] - m[g]) : 0.f;
      l[g] += p;
#pragma unroll
      for (int j = 0; j < N; ++j) o[g].v[j] += p * vr[k].v[j];
    }
  }

  // 3. the waves' partials merged into the chunk's
#pragma unroll
  for (int g = 0; g < G; ++g) {
    o[g].store(&sm_o[wave][g][0], lane);
    if (lane == 0) sm_ml[wave][g][0] = m[g], sm_ml[wave][g][1] = l[g];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < G * D; e += NT) {
    const int g = e / D, d = e % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sm_ml[w][g][0]);
    float O = 0.f, Ls = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float mw = sm_ml[w][g][0];
      const float f = mw == -INFINITY ? 0.f : expf(mw - M);
      O = fmaf(sm_o[w][g][d], f, O);
      Ls = fmaf(sm_ml[w][g][1], f, Ls);
    }
    const size_t ci = (size_t)(kvh * G + g) * nchunk + chunk;
    a.part_o[ci * D + d] = O;
    if (d == 0) a.part_m[ci] = M, a.part_l[ci] = Ls;
  }
  tr.put(kTrAttn, ((int)blockIdx.x + (int)gridDim.x * (int)blockIdx.y) * WAVES + (int)(threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------
// k_attn_combine: merge the chunk partials of one q head and DW dimensions.
//   out[d] = sum_i o_i[d] e^(m_i - M) / sum_i l_i e^(m_i - M),  M = max_i m_i
// 256 threads = CG = 256/DW chunk groups x DW dimensions.  A thread loads the
// partials of up to R chunks at once (all loads in flight together), folds
// them into its running (M, L, O), and the CG groups merge through LDS; grid
// (n_q_heads, D/DW).
// ---------------------------------------------------------------------------
template <int D, int DW>
__global__ __launch_bounds__(256) void k_attn_combine(DecodeArgs a, int nchunk) {
  Trace tr;
  tr.mark(0);
  constexpr int CG = 256 / DW;
  constexpr int R = (80 + CG - 1) / CG;  // at least 80 chunks per batch
  static_assert(D % DW == 0 && 256 % DW == 0, "DW divides D and the workgroup");
  __shared__ float gm[CG], gl[CG];
  __shared__ float go[CG][DW];
  const int h = blockIdx.x, d0 = blockIdx.y * DW;
  const int cg = threadIdx.x / DW, dl = threadIdx.x % DW;
  const float *pm = a.part_m + (size_t)h * nchunk;
  const float *pl = a.part_l + (size_t)h * nchunk;
  const float *po = a.part_o + (size_t)h * nchunk * D + d0 + dl;
  float M = -INFINITY, Ls = 0.f, O = 0.f;
  // the first batch runs unconditionally (nchunk >= 1; the loads are clamped
  // and chunks past nchunk are masked), so the partial-buffer arguments are
  // read with the others at the start rather than inside a branch
  int base = cg;
  do {
    float mi[R], li[R], oi[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = min(base + CG * r, nchunk - 1);  // clamped, unconditional loads
      mi[r] = pm[i];
      li[r] = pl[i];
      oi[r] = po[(size_t)i * D];
    }
    float mb = M;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (base + CG * r < nchunk) mb = fmaxf(mb, mi[r]);  // empty chunks carry m = -inf, l = 0
    if (mb != -INFINITY) {
      const float sc = expf(M - mb);  // 0 while M is still -inf
      Ls *= sc;
      O *= sc;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float w = (base + CG * r < nchunk && mi[r] != -INFINITY) ? expf(mi[r] - mb) : 0.f;
        Ls = fmaf(li[r], w, Ls);
        O = fmaf(oi[r], w, O);
      }
      M = mb;
    }
    base += CG * R;
  } while (base < nchunk);
  tr.mark(1);
  tr.mark_landed();
  if (dl == 0) {
    gm[cg] = M;
    gl[cg] = Ls;
  }
  go[cg][dl] = O;
  __syncthreads();
  if (cg == 0) {
    float Mx = gm[0];
#pragma unroll
    for (int q = 1; q < CG; ++q) Mx = fmaxf(Mx, gm[q]);
    float Lt = 0.f, Ot = 0.f;
#pragma unroll
    for (int q = 0; q < CG; ++q) {
      const float w = gm[q] == -INFINITY ? 0.f : expf(gm[q] - Mx);
      Lt += gl[q] * w;
      Ot += go[q][dl] * w;
    }
    a.attn[(size_t)h * D + d0 + dl] = Ot / Lt;
  }
  tr.put(kTrMerge, ((int)blockIdx.x + (int)gridDim.x * (int)blockIdx.y) * 4 + (int)(threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------
// k_lmhead: x = x2 + rms(dn)(1+g_post_ffn_last); xn = rms(x)(1+g_final);
// logits = E(bf16 lm_head, the tied embedding by default) . xn
// (transformer4.rs:2380-2385)
// ---------------------------------------------------------------------------
template <int CPL>
__global__ __launch_bounds__(256) void k_lmhead(DecodeArgs a, LayerArgs last) {
  Trace tr;
  tr.mark(0);
  constexpr int K = CPL * 512;
  constexpr int U = 2;
  __shared__ __attribute__((aligned(16))) float xl[K / 64 * kXPitch];
  __shared__ float bred[8];
  ProRegs<K, 256> pr;
  pro_load<K, 256, Pro::Resid>(a, a.x2, a.dn, last.g_post_ffn, a.g_final, pr);
  pro_finish<K, 256, Pro::Resid>(a, pr, nullptr, xl, bred);
  __syncthreads();
  tr.mark(1);
  tr.t[2] = tr.t[1];
  const int lane = threadIdx.x & 63;
  float xr[CPL][8];
#pragma unroll
  for (int i = 0; i < CPL; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) xr[i][j] = xl[xlds_index((i * 64 + lane) * 8 + j)];
  const int wave = (int)((blockIdx.x * 256u + threadIdx.x) >> 6);
  const int nwaves = (int)(gridDim.x * 4u);
  const int N = a.vocab;
  for (int r0 = wave * U; r0 < N; r0 += nwaves * U) {
    uint4 wv[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = min(r0 + u, N - 1);
      const uint4 *rp = reinterpret_cast<const uint4 *>(a.lm_bf16 + (size_t)r * K);
#pragma unroll
      for (int i = 0; i < CPL; ++i) wv[u][i] = ld_nt16(rp + i * 64 + lane);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const uint4 w = wv[u][i];
        acc0 += bf16_lo(w.x) * xr[i][0];
        acc1 += bf16_hi(w.x) * xr[i][1];
        acc0 += bf16_lo(w.y) * xr[i][2];
        acc1 += bf16_hi(w.y) * xr[i][3];
        acc0 += bf16_lo(w.z) * xr[i][4];
        acc1 += bf16_hi(w.z) * xr[i][5];
        acc0 += bf16_lo(w.w) * xr[i][6];
        acc1 += bf16_hi(w.w) * xr[i][7];
      }
      const float acc = wave_sum(acc0 + acc1);
      if (lane == 0 && r0 + u < N) a.logits[r0 + u] = acc;
    }
  }
  tr.put(kTrHead, (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------
// k_final_norm: one token's x = x2 + rms(dn)(1+g_post_ffn_last) and
// xn = rms(x)(1+g_final) (transformer4.rs:2370-2380) into out[hidden]; the
// batched lm_head then reads every token's xn.
// ---------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(256) void k_final_norm(DecodeArgs a, LayerArgs last, float *__restrict__ out) {
  constexpr int T = 256;
  __shared__ float bred[2 * (T / 64)];
  ProRegs<K, T> pr;
  pro_load<K, T, Pro::Resid>(a, a.x2, a.dn, last.g_post_ffn, a.g_final, pr);
  using R = ProRegs<K, T>;
  const float inv_k = 1.0f / (float)K;
  auto live = [&](int i) { return (int)threadIdx.x + i * T < R::F4; };
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < R::PER; ++i) ss += live(i) ? sumsq4(pr.add[i]) : 0.f;
  const float ra = rms_inv_from_sumsq(block_sum<T>(ss, bred), inv_k, a.eps);
  float4 x[R::PER];
#pragma unroll
  for (int i = 0; i < R::PER; ++i) x[i] = add4(pr.base[i], norm4(pr.add[i], ra, pr.ga[i]));
  float sx = 0.f;
#pragma unroll
  for (int i = 0; i < R::PER; ++i) sx += live(i) ? sumsq4(x[i]) : 0.f;
  const float rx = rms_inv_from_sumsq(block_sum<T>(sx, bred), inv_k, a.eps);
#pragma unroll
  for (int i = 0; i < R::PER; ++i)
    if (live(i)) reinterpret_cast<float4 *>(out)[threadIdx.x + i * T] = norm4(x[i], rx, pr.go[i]);
}

// ---------------------------------------------------------------------------
// k_lmhead_batch: logits[v][r] = E[r] . xn[v] for v < M <= 8 on
// v_mfma_f32_16x16x32_bf16 (decode_step_batch's lm_head, metal_decode.rs:
// 2162-2172).  Each xn[v] is split into bf16 parts hi + lo (x - hi rounded
// again: 2^-17 relative), and A row 2v+p carries part p of vector v (rows of
// absent vectors are zero), so one pass over the 1.34 GB embedding serves
// every token.  B is 16 embedding rows as they are.  Lane (n = l%16,
// g = l/16) holds C rows 4g..4g+3: vectors 2g and 2g+1, both parts, of
// vocabulary row n.  A sits in LDS for the whole K: [segment][16][32] bf16
// with the 16-byte groups XOR-swizzled by (row >> 2) so a ds_read_b128 of 16
// lanes hits 64 distinct banks.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// One workgroup of 16 waves per CU (the staged A fills half the LDS), each
// wave with 16 segments of its 16 rows in flight: 2.671 against 2.697 ms per
// M = 8 verify call for 4 waves and 8 segments.
constexpr int kHeadBatchThreads = 1024, kHeadBatchGrid = 256;

// K (the hidden width, a multiple of 32) is a template constant for the
// fused-kernel shapes and a run-time value (K = 0) otherwise; the staged A
// takes K*32 bytes of dynamic LDS.
template <int KC>
__global__ __launch_bounds__(kHeadBatchThreads) void k_lmhead_batch(const uint16_t *__restrict__ E,
                                                                    const float *__restrict__ xn,
                                                                    float *__restrict__ logits, int N, int M, int Krt) {
  const int K = KC ? KC : Krt;
  const int SEG = K / 32;
  extern __shared__ __attribute__((aligned(16))) uint16_t xa[];
  // stage: element e of vector v -> hi, lo bf16 at A rows 2v, 2v+1
#pragma unroll 1
  for (int i = threadIdx.x; i < 8 * K; i += kHeadBatchThreads) {
    const int v = i / K, e = i % K;
    uint16_t hi = 0, lo = 0;
    if (v < M) {
      const float x = xn[(size_t)v * K + e];
      hi = f32_to_bf16_bits(x);
      lo = f32_to_bf16_bits(x - bf16_lo((uint32_t)hi));
    }
    const int seg = e >> 5, k = e & 31, grp = k >> 3;
    for (int p = 0; p < 2; ++p) {
      const int row = 2 * v + p;
      xa[(seg * 16 + row) * 32 + 8 * (grp ^ ((row >> 2) & 3)) + (k & 7)] = p ? lo : hi;
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const int aoff = n * 32 + 8 * (g ^ ((n >> 2) & 3));  // this lane's A fragment inside a segment
  const int wave = (int)((blockIdx.x * (unsigned)kHeadBatchThreads + threadIdx.x) >> 6);
  const int nwaves = (int)gridDim.x * (kHeadBatchThreads / 64);
  constexpr int B = 16;  // segments in flight per batch
#pragma unroll 1
  for (int r0 = wave * 16; r0 < N; r0 += nwaves * 16) {
    const uint16_t *row = E + (size_t)min(r0 + n, N - 1) * K + 8 * g;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    u32x4_t bw[B];
#pragma unroll
    for (int j = 0; j < B; ++j) bw[j] = *reinterpret_cast<const u32x4_t *>(row + 32 * min(j, SEG - 1));
#pragma unroll 1
    for (int s0 = 0; s0 < SEG; s0 += B) {
      u32x4_t bn[B];
      const int s1 = s0 + B < SEG ? s0 + B : s0;  // next batch (repeats the last one at the end)
#pragma unroll
      for (int j = 0; j < B; ++j) bn[j] = *reinterpret_cast<const u32x4_t *>(row + 32 * min(s1 + j, SEG - 1));
#pragma unroll
      for (int j = 0; j < B; ++j) {
        if (s0 + j >= SEG) break;  // a last batch of fewer than B segments (K % 256 != 0; wave-uniform)
        const u32x4_t af = *reinterpret_cast<const u32x4_t *>(xa + (s0 + j) * 512 + aoff);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af),
                                                      __builtin_bit_cast(bf16x8_t, bw[j]), acc, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < B; ++j) bw[j] = bn[j];
    }
    if (r0 + n < N) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int v = 2 * g + h;
        if (v < M) logits[(size_t)v * N + r0 + n] = acc[2 * h] + acc[2 * h + 1];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side step encoder
// ---------------------------------------------------------------------------
// q|k|v tiles (Q4_K rows, the Q6_K v beside them): hidden 2560 runs 320
// threads of two row iterations, hidden 512 one iteration of 256 threads
using QkvTileBig = Q4KTile<10, 320, 2>;
using QkvTileSmall = Q4KTile<2, 256, 1>;
// gate rows (and as many up rows) per k_gateup workgroup; k_gateup8 (Q8_0)
// takes 20 at hidden 2560
constexpr int kGateRowsBig = 40, kGateRowsSmall = 32, kGateRowsBig8 = 20;
static_assert(kGateRowsBig % kGateRowsBig8 == 0, "one divisibility check serves both gate/up tiles");

struct Launch {
  hipStream_t s;
  hipError_t err = hipSuccess;
  void check() {
    if (err == hipSuccess) err = hipGetLastError();
  }
};

template <int NB, int T, int ITERS>
static void launch_qkv(Launch &l, const DecodeArgs &a, const LayerArgs &L, const LayerArgs &prev, bool first,
                       int rows_total, bool v6 = false) {
  constexpr int ROWS = Q4KTile<NB, T, ITERS>::ROWS;
  const dim3 grid(rows_total / ROWS);
  if (v6) {
    if (first)
      hipLaunchKernelGGL((k_qkv<NB, T, ITERS, Pro::Embed, true>), grid, dim3(T), 0, l.s, a, L, prev);
    else
      hipLaunchKernelGGL((k_qkv<NB, T, ITERS, Pro::Resid, true>), grid, dim3(T), 0, l.s, a, L, prev);
  } else if (first) {
    hipLaunchKernelGGL((k_qkv<NB, T, ITERS, Pro::Embed>), grid, dim3(T), 0, l.s, a, L, prev);
  } else {
    hipLaunchKernelGGL((k_qkv<NB, T, ITERS, Pro::Resid>), grid, dim3(T), 0, l.s, a, L, prev);
  }
  l.check();
}

template <int NB32, int T, int ITERS>
static void launch_qkv8(Launch &l, const DecodeArgs &a, const LayerArgs &L, const LayerArgs &prev, bool first,
                        int rows_total) {
  constexpr int ROWS = Q8Tile<NB32, T, ITERS>::ROWS;
  const dim3 grid(rows_total / ROWS);
  if (first)
    hipLaunchKernelGGL((k_qkv8<NB32, T, ITERS, Pro::Embed>), grid, dim3(T), 0, l.s, a, L, prev);
  else
    hipLaunchKernelGGL((k_qkv8<NB32, T, ITERS, Pro::Resid>), grid, dim3(T), 0, l.s, a, L, prev);
  l.check();
}

template <int NB32, int T, int GR>
static void launch_gateup8(Launch &l, const DecodeArgs &a, const LayerArgs &L, int ffn) {
  hipLaunchKernelGGL((k_gateup8<NB32, T, GR>), dim3(ffn / GR), dim3(T), 0, l.s, a, L, ffn);
  l.check();
}

template <int CPL>
static void launch_qkv16(Launch &l, const DecodeArgs &a, const LayerArgs &L, const LayerArgs &prev, bool first,
                         int rows_total) {
  // at most two workgroups per CU, each paying the prologue once (a BF16
  // model's step: 2.211 ms at 512, 2.238 at 256, 2.213 at 1024)
  const dim3 grid((unsigned)std::min((rows_total / 2 + 3) / 4, 512));
  if (first)
    hipLaunchKernelGGL((k_qkv16<CPL, Pro::Embed>), grid, dim3(256), 0, l.s, a, L, prev);
  else
    hipLaunchKernelGGL((k_qkv16<CPL, Pro::Resid>), grid, dim3(256), 0, l.s, a, L, prev);
  l.check();
}

template <int CPL>
static void launch_gateup16(Launch &l, const DecodeArgs &a, const LayerArgs &L, int ffn) {
  hipLaunchKernelGGL((k_gateup16<CPL>), dim3((unsigned)std::min((ffn + 3) / 4, 512)), dim3(256), 0, l.s, a, L, ffn);
  l.check();
}

template <int NB, int T, int GR>
static void launch_gateup(Launch &l, const DecodeArgs &a, const LayerArgs &L, int ffn) {
  hipLaunchKernelGGL((k_gateup<NB, T, GR>), dim3(ffn / GR), dim3(T), 0, l.s, a, L);
  l.check();
}

template <int NB, int T, int ITERS>
static void launch_gemv(Launch &l, const uint8_t *W, const float *x, float *y, int n) {
  constexpr int ROWS = Q4KTile<NB, T, ITERS>::ROWS;
  hipLaunchKernelGGL((k_gemv<NB, T, ITERS>), dim3((n + ROWS - 1) / ROWS), dim3(T), 0, l.s, W, x, y, n);
  l.check();
}

// Shape dispatch.  Supported K's (in super-blocks): hidden 2 | 10, q*d 2 | 8,
// ffn 4 | 40; head_dim 128 | 256; group 1 | 2 | 4.  The host validates these
// and the divisibility of every row count before creating an engine.
bool decode_shape_supported(const DecodeShape &s, const char **why) {
  auto nb = [](int k) { return k / 256; };
  if (s.hidden % 512 != 0 || (nb(s.hidden) != 2 && nb(s.hidden) != 10)) return *why = "hidden must be 512 or 2560", false;
  const int qd = s.n_q_heads * s.head_dim, kvd = s.n_kv_heads * s.head_dim;
  if (qd % 256 != 0 || (nb(qd) != 2 && nb(qd) != 8)) return *why = "n_q_heads*head_dim must be 512 or 2048", false;
  if (s.ffn % 256 != 0 || (nb(s.ffn) != 4 && nb(s.ffn) != 40)) return *why = "ffn must be 1024 or 10240", false;
  if (s.head_dim != 128 && s.head_dim != 256) return *why = "head_dim must be 128 or 256", false;
  if (s.n_kv_heads <= 0 || s.n_q_heads % s.n_kv_heads != 0) return *why = "n_q_heads must be a multiple of n_kv_heads", false;
  const int g = s.n_q_heads / s.n_kv_heads;
  if (g != 1 && g != 2 && g != 4) return *why = "GQA group must be 1, 2 or 4", false;
  if (qd % 16 != 0 || kvd % 16 != 0) return *why = "q/kv widths must be multiples of 16", false;
  return true;
}

template <int D, int KPW, int WAVES>
static void launch_attn_kw(Launch &l, const DecodeArgs &a, const LayerArgs &L, int nchunk, int group) {
  const dim3 grid(nchunk, a.n_kv_heads), block(64 * WAVES);
  switch (group) {
    case 1: hipLaunchKernelGGL((k_attn<D, 1, KPW, WAVES>), grid, block, 0, l.s, a, L); break;
    case 2: hipLaunchKernelGGL((k_attn<D, 2, KPW, WAVES>), grid, block, 0, l.s, a, L); break;
    default: hipLaunchKernelGGL((k_attn<D, 4, KPW, WAVES>), grid, block, 0, l.s, a, L); break;
  }
}

template <int D>
static void launch_attn_d(Launch &l, const DecodeArgs &a, const LayerArgs &L, int nchunk, int group) {
  if (L.window > 0)
    launch_attn_kw<D, kAttnLocalKpw, kAttnLocalWaves>(l, a, L, nchunk, group);
  else
    launch_attn_kw<D, kAttnGlobalKpw, kAttnGlobalWaves>(l, a, L, nchunk, group);
  l.check();
  hipLaunchKernelGGL((k_attn_combine<D, kCombineDims>), dim3(a.n_q_heads, D / kCombineDims), dim3(256), 0, l.s, a,
                     nchunk);
  l.check();
}

// A projection that is not Q4_K: the plain GEMV of its format.
static void launch_proj(Launch &l, int fmt, const uint8_t *W, const float *x, float *y, int n, int k) {
  if (l.err != hipSuccess) return;
  switch (fmt) {
    case RT_LINEAR_Q6K: l.err = launch_q6k_gemv(W, x, y, n, k, l.s); break;
    case RT_LINEAR_Q8_0: l.err = launch_q8_0_gemv(W, x, y, n, k, l.s); break;
    case RT_LINEAR_BF16: l.err = launch_bf16_gemv(reinterpret_cast<const uint16_t *>(W), x, y, n, k, l.s); break;
    default: l.err = launch_q4k_gemv(W, x, y, n, k, l.s); break;
  }
}

template <Pro MODE>
static void launch_prologue(Launch &l, const DecodeShape &s, const DecodeArgs &a, const float *base, const float *add,
                            const float *g_add, const float *g_out, float *x_out) {
  if (s.hidden == 2560)
    hipLaunchKernelGGL((k_prologue<2560, MODE>), dim3(1), dim3(256), 0, l.s, a, base, add, g_add, g_out, x_out, a.xn);
  else
    hipLaunchKernelGGL((k_prologue<512, MODE>), dim3(1), dim3(256), 0, l.s, a, base, add, g_add, g_out, x_out, a.xn);
  l.check();
}

// The six launches of every layer (all-Q4_K projections); a projection of
// another format splits its set into a prologue and plain GEMVs.
static hipError_t enqueue_layers(const DecodeShape &s, const DecodeArgs &a, const LayerArgs *layers, hipStream_t stream) {
  Launch l{stream};
  const int qd = s.n_q_heads * s.head_dim, kvd = s.n_kv_heads * s.head_dim;
  const int group = s.n_q_heads / s.n_kv_heads;
  const bool big = s.hidden == 2560;
  for (int li = 0; li < s.n_layers && l.err == hipSuccess; ++li) {
    const LayerArgs &L = layers[li];
    const LayerArgs &P = layers[li > 0 ? li - 1 : 0];
    auto q4 = [&](int p) { return L.fmt[p] == RT_LINEAR_Q4K; };
    auto q8 = [&](int p) { return L.fmt[p] == RT_LINEAR_Q8_0; };
    auto b16 = [&](int p) { return L.fmt[p] == RT_LINEAR_BF16; };
    if (q4(kProjQ) && q4(kProjK)) {
      // fused prologue + GEMV over q|k|v rows (v in Q4_K or Q6_K); it also
      // leaves xn for a v of another format
      const bool v6 = L.fmt[kProjV] == RT_LINEAR_Q6K;
      const int qkv_rows = qd + kvd + (q4(kProjV) || v6 ? kvd : 0);
      if (big) launch_qkv<10, QkvTileBig::kThreads, QkvTileBig::kIters>(l, a, L, P, li == 0, qkv_rows, v6);
      else launch_qkv<2, QkvTileSmall::kThreads, QkvTileSmall::kIters>(l, a, L, P, li == 0, qkv_rows, v6);
      if (!q4(kProjV) && !v6) launch_proj(l, L.fmt[kProjV], L.wv, a.xn, a.v, kvd, s.hidden);
    } else if (q8(kProjQ) && q8(kProjK) && q8(kProjV)) {
      if (big) launch_qkv8<80, 640, 2>(l, a, L, P, li == 0, qd + 2 * kvd);
      else launch_qkv8<16, 256, 2>(l, a, L, P, li == 0, qd + 2 * kvd);
    } else if (b16(kProjQ) && b16(kProjK) && b16(kProjV)) {
      if (big) launch_qkv16<5>(l, a, L, P, li == 0, qd + 2 * kvd);
      else launch_qkv16<1>(l, a, L, P, li == 0, qd + 2 * kvd);
    } else {
      if (li == 0) launch_prologue<Pro::Embed>(l, s, a, nullptr, nullptr, nullptr, L.g_in, a.hid);
      else launch_prologue<Pro::Resid>(l, s, a, a.x2, a.dn, P.g_post_ffn, L.g_in, a.hid);
      launch_proj(l, L.fmt[kProjQ], L.wq, a.xn, a.q, qd, s.hidden);
      launch_proj(l, L.fmt[kProjK], L.wk, a.xn, a.k, kvd, s.hidden);
      launch_proj(l, L.fmt[kProjV], L.wv, a.xn, a.v, kvd, s.hidden);
    }
    const int nchunk = L.window > 0 ? s.nchunk_local : s.nchunk_global;
    if (s.head_dim == 256)
      launch_attn_d<256>(l, a, L, nchunk, group);
    else
      launch_attn_d<128>(l, a, L, nchunk, group);
    if (!q4(kProjO)) launch_proj(l, L.fmt[kProjO], L.wo, a.attn, a.o, s.hidden, qd);
    else if (qd == 2048) launch_gemv<8, 512, 1>(l, L.wo, a.attn, a.o, s.hidden);
    else launch_gemv<2, 256, 1>(l, L.wo, a.attn, a.o, s.hidden);
    if (q4(kProjGate) && q4(kProjUp)) {
      // 40 gate + 40 up rows per workgroup (five 16-row iterations): 256
      // workgroups, one per CU
      if (big) launch_gateup<10, 640, kGateRowsBig>(l, a, L, s.ffn);
      else launch_gateup<2, 256, kGateRowsSmall>(l, a, L, s.ffn);
    } else if (q8(kProjGate) && q8(kProjUp)) {
      if (big) launch_gateup8<80, 640, kGateRowsBig8>(l, a, L, s.ffn);
      else launch_gateup8<16, 256, kGateRowsSmall>(l, a, L, s.ffn);
    } else if (b16(kProjGate) && b16(kProjUp)) {
      if (big) launch_gateup16<5>(l, a, L, s.ffn);
      else launch_gateup16<1>(l, a, L, s.ffn);
    } else {
      launch_prologue<Pro::Resid>(l, s, a, a.hid, a.o, L.g_post_attn, L.g_pre_ffn, a.x2);
      launch_proj(l, L.fmt[kProjGate], L.wgate, a.xn, a.h, s.ffn, s.hidden);
      launch_proj(l, L.fmt[kProjUp], L.wup, a.xn, a.u, s.ffn, s.hidden);
      if (l.err == hipSuccess) {
        hipLaunchKernelGGL(k_gelu_mul_vec, dim3((s.ffn + 255) / 256), dim3(256), 0, l.s, a.h, a.u, s.ffn);
        l.check();
      }
    }
    if (!q4(kProjDown)) launch_proj(l, L.fmt[kProjDown], L.wdown, a.h, a.dn, s.hidden, s.ffn);
    else if (s.ffn == 10240) launch_gemv<40, 960, 2>(l, L.wdown, a.h, a.dn, s.hidden);
    else launch_gemv<4, 256, 1>(l, L.wdown, a.h, a.dn, s.hidden);
  }
  return l.err;
}

hipError_t enqueue_lm_head(const DecodeShape &s, const DecodeArgs &a, const LayerArgs &last, hipStream_t stream) {
  Launch l{stream};
  if (a.lm_q4k) {
    // a Q4_K lm_head (metal_decode.rs:1079-1107, dispatch_gemv 2053-2063):
    // the final norm into a.xn (free once the last layer is done), then the
    // single-token Q4_K GEMV over the vocabulary rows
    if (s.hidden == 2560)
      hipLaunchKernelGGL((k_final_norm<2560>), dim3(1), dim3(256), 0, l.s, a, last, a.xn);
    else
      hipLaunchKernelGGL((k_final_norm<512>), dim3(1), dim3(256), 0, l.s, a, last, a.xn);
    l.check();
    if (l.err == hipSuccess) l.err = launch_q4k_gemv(a.lm_q4k, a.xn, a.logits, s.vocab, s.hidden, l.s);
    return l.err;
  }
  // three workgroups per CU stay resident for the whole pass (grid-stride rows)
  const dim3 grid(768);
  if (s.hidden == 2560) hipLaunchKernelGGL((k_lmhead<5>), grid, dim3(256), 0, l.s, a, last);
  else hipLaunchKernelGGL((k_lmhead<1>), grid, dim3(256), 0, l.s, a, last);
  l.check();
  return l.err;
}

hipError_t enqueue_decode_step(const DecodeShape &s, const DecodeArgs &a, const LayerArgs *layers, hipStream_t stream) {
  hipError_t e = enqueue_layers(s, a, layers, stream);
  return e == hipSuccess ? enqueue_lm_head(s, a, layers[s.n_layers - 1], stream) : e;
}

hipError_t enqueue_decode_batch(const DecodeShape &s, const DecodeArgs &a, const LayerArgs *layers, int m,
                                float *xn, float *logits_b, hipStream_t stream) {
  Launch l{stream};
  const int slot = param_slot_floats(s.head_dim);
  std::vector<LayerArgs> ls(layers, layers + s.n_layers);
  for (int t = 0; t < m && l.err == hipSuccess; ++t) {
    DecodeArgs at = a;
    at.params = a.params + (size_t)t * slot;
    for (int li = 0; li < s.n_layers; ++li) ls[li].rope_cs = layers[li].rope_cs + (size_t)t * slot;
    l.err = enqueue_layers(s, at, ls.data(), stream);
    if (l.err != hipSuccess) break;
    if (s.hidden == 2560)
      hipLaunchKernelGGL((k_final_norm<2560>), dim3(1), dim3(256), 0, l.s, at, ls[s.n_layers - 1], xn + (size_t)t * 2560);
    else
      hipLaunchKernelGGL((k_final_norm<512>), dim3(1), dim3(256), 0, l.s, at, ls[s.n_layers - 1], xn + (size_t)t * 512);
    l.check();
  }
  return l.err == hipSuccess ? enqueue_lm_head_batch(s, a, xn, logits_b, m, stream) : l.err;
}

hipError_t prepare_lm_head_batch(int hidden) {
  if (hidden % 32 != 0 || hidden > kLmHeadMaxHidden) return hipErrorInvalidValue;
  const int bytes = hidden * 32;
  if (hidden == 2560) return hipFuncSetAttribute((const void *)k_lmhead_batch<2560>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (hidden == 512) return hipSuccess;
  return hipFuncSetAttribute((const void *)k_lmhead_batch<0>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

hipError_t enqueue_lm_head_batch(const DecodeShape &s, const DecodeArgs &a, const float *xn, float *logits_b, int m,
                                 hipStream_t stream) {
  Launch l{stream};
  if (a.lm_q4k) {
    // gemv_q4k_t_batch over the vocabulary (metal_decode.rs:2168-2172): the
    // m rows staged as digits once, the Q4_K head read once for all of them
    l.err = launch_mb_stage(xn, m, s.hidden, a.lm_stage, l.s);
    if (l.err == hipSuccess)
      l.err = launch_q4k_gemv_mb_head(a.lm_q4k, logits_b, s.vocab, m, s.hidden, a.lm_stage, a.lm_part, l.s);
    return l.err;
  }
  const size_t lds = (size_t)s.hidden * 32;
  if (s.hidden == 2560)
    hipLaunchKernelGGL((k_lmhead_batch<2560>), dim3(kHeadBatchGrid), dim3(kHeadBatchThreads), lds, l.s, a.lm_bf16, xn,
                       logits_b, s.vocab, m, 0);
  else if (s.hidden == 512)
    hipLaunchKernelGGL((k_lmhead_batch<512>), dim3(kHeadBatchGrid), dim3(kHeadBatchThreads), lds, l.s, a.lm_bf16, xn,
                       logits_b, s.vocab, m, 0);
  else
    hipLaunchKernelGGL((k_lmhead_batch<0>), dim3(kHeadBatchGrid), dim3(kHeadBatchThreads), lds, l.s, a.lm_bf16, xn,
                       logits_b, s.vocab, m, s.hidden);
  l.check();
  return l.err;
}

// Shapes the rows kernels serve: the decode step then runs as a one-row
// pass of enqueue_rows.  Their projections take any format the batched
// GEMVs take; a width that is not whole super-blocks (Gemma-3-1B's hidden
// 1152) leaves the projections that read it to Q8_0 and BF16.
bool decode_shape_generic(const DecodeShape &s, const char **why) {
  const int qd = s.n_q_heads * s.head_dim;
  if (s.hidden % 64 != 0 || s.hidden > kLmHeadMaxHidden)
    return *why = "hidden must be a multiple of 64 up to 4096", false;
  if (qd % 256 != 0) return *why = "n_q_heads*head_dim must be a multiple of 256", false;
  if (s.ffn % 256 != 0 || s.ffn > 16384) return *why = "ffn must be a multiple of 256 up to 16384", false;
  if (s.head_dim != 128 && s.head_dim != 256) return *why = "head_dim must be 128 or 256", false;
  if (s.n_kv_heads <= 0 || s.n_q_heads % s.n_kv_heads != 0) return *why = "n_q_heads must be a multiple of n_kv_heads", false;
  const int g = s.n_q_heads / s.n_kv_heads;
  if (g != 1 && g != 2 && g != 4) return *why = "GQA group must be 1, 2 or 4", false;
  return true;
}

// Row-count divisibility the launches above rely on.
static_assert(Q8Tile<80, 640, 2>::ROWS == QkvTileBig::ROWS && Q8Tile<16, 256, 2>::ROWS == QkvTileSmall::ROWS,
              "the Q8_0 q|k|v tiles cover the Q4_K tiles' rows, so one divisibility check serves both");

bool decode_rows_divisible(const DecodeShape &s, const char **why) {
  const int qd = s.n_q_heads * s.head_dim, kvd = s.n_kv_heads * s.head_dim;
  const bool big = s.hidden == 2560;
  const int qkv_rows_per_wg = big ? QkvTileBig::ROWS : QkvTileSmall::ROWS;
  if (qd % qkv_rows_per_wg || kvd % qkv_rows_per_wg) return *why = "q/kv rows must divide into workgroup tiles", false;
  const int gate_rows_per_wg = big ? kGateRowsBig : kGateRowsSmall;
  if (s.ffn % gate_rows_per_wg) return *why = "ffn rows must divide into gate/up tiles", false;
  return true;  // the o and down GEMVs bound their rows themselves
}

}  // namespace rt

extern "C" rt_status rt_trace_read(void *host_dst, size_t bytes, int32_t *kernels, int32_t *slots) {
  if (!rt::kTrace) return rt::set_error(RT_ESTATE, "rt_trace_read: this library is built without RT_TRACE (make trace)");
  if (kernels) *kernels = rt::kTraceKernels;
  if (slots) *slots = rt::kTraceSlots;
  if (!host_dst) return RT_OK;
  if (bytes != sizeof(rt::g_trace))
    return rt::set_error(RT_EINVAL, "rt_trace_read: bytes must be %zu", sizeof(rt::g_trace));
  return rt::hip_error(hipMemcpyFromSymbol(host_dst, HIP_SYMBOL(rt::g_trace), bytes, 0, hipMemcpyDeviceToHost),
                       "rt_trace_read");
}
