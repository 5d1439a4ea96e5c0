// decode_engine.hip -- the Gemma-3 decode context behind rt_decode_* (the
// MI355X counterpart of MetalDecodeContext, metal_decode.rs:754-829).
//
// Owns the device KV cache (f32, [max_seq, n_kv_heads*head_dim] per layer),
// the activation buffers and, unless the caller binds its own device
// pointers, the uploaded weights (Q4_K blocks copied verbatim).  A step is the
// kernel sequence of enqueue_decode_step(), captured once into a hipGraph and
// replayed; token id and position travel through a device buffer.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/rt_hip.h"
#include "decode.hpp"
#include "q4k_gemv_mb.hpp"
#include "rt_capi_util.hpp"
#include "rt_kernels.hpp"

using namespace rt;

struct rt_decode {
  rt_gemma3_config cfg{};
  DecodeShape shape{};
  int device = 0;
  hipStream_t stream = nullptr;
  // every hipMalloc of this context, with its size and what it holds
  enum Mem { kWeights, kKv, kActivation, kBatch, kPrefill, kMemKinds };
  struct Alloc {
    void *p;
    size_t bytes;
    int kind;
  };
  std::vector<Alloc> owned;
  size_t bound_weight_bytes[66] = {};    // weights bound by device pointer: per layer, [64] embedding + final norm, [65] lm_head
  std::vector<LayerArgs> layers;
  std::vector<char> layer_set;
  std::vector<void *> owned_layer[64];  // per-layer uploads (replaced on re-set)
  bool embed_set = false;
  void *embed_owned = nullptr, *final_owned = nullptr;
  int lm_fmt = 0;                        // lm_head: 0 the tied embedding, else RT_LINEAR_Q4K / RT_LINEAR_BF16
  std::vector<void *> lm_owned;          // its upload and (Q4_K) batched-head scratch
  DecodeArgs args{};
  int *params_dev = nullptr;             // kMaxBatch step parameter slots (kParamRopeLocal)
  int *params_host = nullptr;            // pinned
  size_t params_bytes = 0, slot_bytes = 0;
  float *xn_batch = nullptr, *logits_batch = nullptr;  // decode_step_batch: [kMaxBatch][hidden | vocab]
  hipGraphExec_t exec_batch[kMaxBatch + 1] = {};
  hipEvent_t params_copied = nullptr;
  bool params_pending = false;
  std::vector<float> rope_den_local, rope_den_global;  // theta^(2i/d), host powf
  hipGraphExec_t exec = nullptr;
  bool graph_enabled = true;
  bool graph_dirty = true;
  PrefillBuffers pf;                     // rt_decode_prefill scratch (grown on demand)
  PrefillBuffers vb;                     // decode_step_batch rows (kMaxBatch), allocated at create
  bool rows_mb = true;                   // every layer's formats served by the batched GEMVs (verify, short chunks)
  bool fused = true;                     // the fused single-token kernels serve this shape (else the rows path)
  int pf_chunk = 4096;                   // rows per prefill chunk (~180 KB of scratch per row at Gemma-3-4B)
  std::vector<void *> pf_owned;
  int *pf_tokens_host = nullptr;         // pinned staging: [pf.cap] tokens
  float *rope_cs = nullptr;              // [rope_rows][2][head_dim] cos/sin of positions 0 .. rope_rows-1
  int rope_rows = 0;
};

namespace {

rt_status dalloc(rt_decode *d, size_t bytes, void **out, int kind = rt_decode::kActivation) {
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return hip_error(e, "rt_decode hipMalloc");
  d->owned.push_back({p, bytes, kind});
  *out = p;
  return RT_OK;
}

void dfree(rt_decode *d, void *p) {
  if (!p) return;
  for (auto &q : d->owned)
    if (q.p == p) {
      (void)hipFree(q.p);
      q.p = nullptr;
      q.bytes = 0;
    }
}

void drop_graph(rt_decode *d) {
  if (d->exec) (void)hipGraphExecDestroy(d->exec);
  d->exec = nullptr;
  for (auto &x : d->exec_batch) {
    if (x) (void)hipGraphExecDestroy(x);
    x = nullptr;
  }
  d->graph_dirty = true;
}

bool is_global(const rt_gemma3_config &c, int layer) {
  // Config4::is_global_layer (transformer4.rs:141-143): layer % 6 == 5 for Gemma 3.
  return c.global_every > 0 && (layer % c.global_every) == c.global_every - 1;
}

}  // namespace

extern "C" {

rt_status rt_decode_create(const rt_gemma3_config *cfg, rt_decode **out) {
  if (!cfg || !out) return set_error(RT_EINVAL, "rt_decode_create: null pointer");
  *out = nullptr;
  const rt_gemma3_config &c = *cfg;
  if (c.n_layers <= 0 || c.n_layers > 64 || c.vocab <= 0 || c.max_seq <= 0 || c.max_seq > (1 << 22))
    return set_error(RT_EINVAL, "rt_decode_create: n_layers (1..64), vocab and max_seq must be positive");
  if (!(c.eps > 0.f) || c.global_every < 0 || c.sliding_window < 0)
    return set_error(RT_EINVAL, "rt_decode_create: eps must be > 0, global_every and sliding_window >= 0");
  DecodeShape s{};
  s.hidden = c.hidden;
  s.ffn = c.ffn;
  s.n_q_heads = c.n_q_heads;
  s.n_kv_heads = c.n_kv_heads;
  s.head_dim = c.head_dim;
  s.n_layers = c.n_layers;
  s.vocab = c.vocab;
  const char *why = "", *why_generic = "";
  if (c.hidden <= 0 || c.ffn <= 0 || c.n_q_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0)
    return set_error(RT_EINVAL, "rt_decode_create: hidden, ffn, heads and head_dim must be positive");
  // The fused single-token kernels where their templates cover the shape,
  // else every step through the rows kernels (projections in Q4_K only).
  const bool fused = decode_shape_supported(s, &why) && decode_rows_divisible(s, &why);
  if (!fused && !decode_shape_generic(s, &why_generic))
    return set_error(RT_EINVAL, "rt_decode_create: unsupported shape: %s (fused kernels), %s (rows kernels)", why,
                     why_generic);
  if (hipError_t pe = prepare_lm_head_batch(c.hidden); pe != hipSuccess)
    return hip_error(pe, "rt_decode_create: batched lm_head");
  const int window = c.sliding_window;
  const int local_span = window > 0 ? std::min(window, c.max_seq) : c.max_seq;
  constexpr int kLocalKeys = kAttnLocalKpw * kAttnLocalWaves, kGlobalKeys = kAttnGlobalKpw * kAttnGlobalWaves;
  s.nchunk_local = (local_span + kLocalKeys - 1) / kLocalKeys;
  s.nchunk_global = (c.max_seq + kGlobalKeys - 1) / kGlobalKeys;
  if (s.nchunk_global > kAttnMaxChunks || s.nchunk_local > kAttnMaxChunks)
    return set_error(RT_EINVAL, "rt_decode_create: max_seq %d exceeds %d", c.max_seq, kLocalKeys * kAttnMaxChunks);

  rt_decode *d = new rt_decode();
  d->cfg = c;
  d->shape = s;
  d->fused = fused;
  hipError_t e = hipGetDevice(&d->device);
  rt_status st = RT_OK;
#define TRY(x)                  \
  do {                          \
    st = (x);                   \
    if (st != RT_OK) goto fail; \
  } while (0)
#define TRYH(x, what)                          \
  do {                                         \
    e = (x);                                   \
    if (e != hipSuccess) {                     \
      st = hip_error(e, what);                 \
      goto fail;                               \
    }                                          \
  } while (0)
  {
    TRYH(e, "hipGetDevice");
    TRYH(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking), "hipStreamCreate");
    TRYH(hipEventCreateWithFlags(&d->params_copied, hipEventDisableTiming), "hipEventCreate");
    const size_t H = c.hidden, F = c.ffn, D = c.head_dim;
    const size_t QD = (size_t)c.n_q_heads * D, KVD = (size_t)c.n_kv_heads * D;
    const int nch = std::max(s.nchunk_local, s.nchunk_global);
    d->slot_bytes = (size_t)param_slot_floats((int)D) * sizeof(float);
    d->params_bytes = kMaxBatch * d->slot_bytes;
    TRYH(hipHostMalloc((void **)&d->params_host, d->params_bytes, hipHostMallocDefault), "hipHostMalloc");
    std::memset(d->params_host, 0, d->params_bytes);
    void *p;
    TRY(dalloc(d, d->params_bytes, &p)); d->params_dev = (int *)p;
    TRYH(hipMemset(d->params_dev, 0, d->params_bytes), "hipMemset");
    DecodeArgs &a = d->args;
    int kind = rt_decode::kActivation;  // what the next fbuf holds
    auto fbuf = [&](size_t n, float **dst) -> rt_status {
      void *q = nullptr;
      rt_status r = dalloc(d, std::max<size_t>(n, 4) * sizeof(float), &q, kind);
      if (r == RT_OK) {
        *dst = (float *)q;
        hipError_t z = hipMemset(q, 0, std::max<size_t>(n, 4) * sizeof(float));
        if (z != hipSuccess) r = hip_error(z, "hipMemset");
      }
      return r;
    };
    TRY(fbuf(H, &a.hid)); TRY(fbuf(H, &a.x2)); TRY(fbuf(QD, &a.q)); TRY(fbuf(KVD, &a.k)); TRY(fbuf(KVD, &a.v));
    TRY(fbuf(QD, &a.attn)); TRY(fbuf(H, &a.o)); TRY(fbuf(F, &a.h)); TRY(fbuf(H, &a.dn));
    TRY(fbuf(H, &a.xn)); TRY(fbuf(F, &a.u));
    TRY(fbuf((size_t)c.vocab, &a.logits));
    TRY(fbuf((size_t)c.n_q_heads * nch, &a.part_m)); TRY(fbuf((size_t)c.n_q_heads * nch, &a.part_l));
    TRY(fbuf((size_t)c.n_q_heads * nch * D, &a.part_o));
    kind = rt_decode::kBatch;
    TRY(fbuf((size_t)kMaxBatch * H, &d->xn_batch));
    TRY(fbuf((size_t)kMaxBatch * c.vocab, &d->logits_batch));
    {
      PrefillBuffers &vb = d->vb;
      const size_t R = kMaxBatch;
      TRY(fbuf(R * H, &vb.hid)); TRY(fbuf(R * H, &vb.x2)); TRY(fbuf(R * H, &vb.xn)); TRY(fbuf(R * H, &vb.o));
      TRY(fbuf(R * H, &vb.dn)); TRY(fbuf(R * QD, &vb.q)); TRY(fbuf(R * QD, &vb.attn)); TRY(fbuf(R * KVD, &vb.k));
      TRY(fbuf(R * KVD, &vb.v)); TRY(fbuf(R * F, &vb.g)); TRY(fbuf(R * F, &vb.u));
      void *q = nullptr;
      TRY(dalloc(d, rows_mb_stage_bytes(s), &q, kind)); vb.mb_stage = q;
      TRY(fbuf(rows_mb_part_bytes(s) / 4, &vb.mb_part));
      TRY(fbuf(attn_part_floats(s, kMaxBatch, false), &vb.attn_ml));
      TRY(fbuf(attn_part_floats(s, kMaxBatch, true), &vb.attn_o));
      vb.attn_rows = kMaxBatch;
      vb.cap = kMaxBatch;
    }
    a.params = d->params_dev;
    a.embed_scale = std::sqrt((float)c.hidden);   // transformer4.rs:2092
    a.eps = c.eps;
    a.attn_scale = c.attn_scale;
    a.vocab = c.vocab;
    a.n_q_heads = c.n_q_heads;
    a.n_kv_heads = c.n_kv_heads;
    a.head_dim = c.head_dim;
    // RoPE denominators theta^(2i/d), computed with the host libm exactly as
    // apply_rope_at_offset does (transformer4.rs:2755); each step turns them
    // into the cos/sin table of its position (rt_decode_step_async).
    d->rope_den_local.resize(D / 2);
    d->rope_den_global.resize(D / 2);
    for (size_t i = 0; i < D / 2; ++i) {
      const float ex = 2.0f * (float)i / (float)D;
      d->rope_den_local[i] = powf(c.rope_theta_local, ex);
      d->rope_den_global[i] = powf(c.rope_theta_global, ex);
    }
    const float *cs_dev = reinterpret_cast<const float *>(d->params_dev) + kParamRopeLocal;
    d->layers.resize(c.n_layers);
    d->layer_set.assign(c.n_layers, 0);
    for (int l = 0; l < c.n_layers; ++l) {
      LayerArgs &L = d->layers[l];
      std::memset(&L, 0, sizeof L);
      kind = rt_decode::kKv;
      TRY(fbuf((size_t)c.max_seq * KVD, &L.kc));
      TRY(fbuf((size_t)c.max_seq * KVD, &L.vc));
      const bool g = is_global(c, l);
      L.rope_cs = cs_dev + (g ? D : 0);
      L.window = g ? 0 : c.sliding_window;
      L.global = g ? 1 : 0;
      for (int &f : L.fmt) f = RT_LINEAR_Q4K;
    }
  }
#undef TRY
#undef TRYH
  *out = d;
  return RT_OK;
fail:
  rt_decode_destroy(d);
  return st;
}

rt_status rt_decode_destroy(rt_decode *d) {
  if (!d) return RT_OK;
  if (d->stream) (void)hipStreamSynchronize(d->stream);
  drop_graph(d);
  for (auto &a : d->owned)
    if (a.p) (void)hipFree(a.p);
  if (d->params_host) (void)hipHostFree(d->params_host);
  if (d->pf_tokens_host) (void)hipHostFree(d->pf_tokens_host);
  if (d->params_copied) (void)hipEventDestroy(d->params_copied);
  if (d->stream) (void)hipStreamDestroy(d->stream);
  delete d;
  return RT_OK;
}

static rt_status bind_buf(rt_decode *d, const void *src, size_t bytes, int32_t device_ptrs, std::vector<void *> &owned,
                      const void **dst, const char *what) {
  if (!src) return set_error(RT_EINVAL, "rt_decode: %s is null", what);
  if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0 && device_ptrs)
    return set_error(RT_EINVAL, "rt_decode: %s must be 16-byte aligned", what);
  if (device_ptrs) {
    *dst = src;
    return RT_OK;
  }
  void *p = nullptr;
  rt_status st = dalloc(d, bytes, &p, rt_decode::kWeights);
  if (st != RT_OK) return st;
  hipError_t e = hipMemcpy(p, src, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    dfree(d, p);
    return hip_error(e, what);
  }
  owned.push_back(p);
  *dst = p;
  return RT_OK;
}

// Bytes of a [rows][cols] projection in format fmt; 0 if cols does not suit it.
static size_t proj_bytes(int fmt, size_t rows, size_t cols) {
  switch (fmt) {
    case RT_LINEAR_Q4K: return cols % 256 ? 0 : rows * (cols / 256) * 144;
    case RT_LINEAR_Q6K: return cols % 256 ? 0 : rows * (cols / 256) * 210;
    case RT_LINEAR_Q8_0: return cols % 32 ? 0 : rows * (cols / 32) * 34;
    case RT_LINEAR_BF16: return cols % 8 ? 0 : rows * cols * 2;
    default: return 0;
  }
}

rt_status rt_decode_set_layer(rt_decode *d, int32_t layer, const rt_gemma3_layer *w, int32_t device_ptrs) {
  const int32_t all_q4k[7] = {RT_LINEAR_Q4K, RT_LINEAR_Q4K, RT_LINEAR_Q4K, RT_LINEAR_Q4K,
                              RT_LINEAR_Q4K, RT_LINEAR_Q4K, RT_LINEAR_Q4K};
  return rt_decode_set_layer_formats(d, layer, w, all_q4k, device_ptrs);
}

// max over n of |Wgate row n| |Wup row n| (dequantised Q4_K rows, F rows of
// K), rounded up by one part in 2^20; *out = 0 when the product is not finite.
static rt_status gate_up_bound(rt_decode *d, const uint8_t *wg, const uint8_t *wu, int F, int K, float *out) {
  void *p = nullptr;
  rt_status st = dalloc(d, (size_t)2 * F * sizeof(float), &p);
  if (st != RT_OK) return st;
  float *nrm = static_cast<float *>(p);
  hipError_t e = launch_q4k_row_norms(wg, F, K, nrm, d->stream);
  if (e == hipSuccess) e = launch_q4k_row_norms(wu, F, K, nrm + F, d->stream);
  std::vector<float> host((size_t)2 * F);
  if (e == hipSuccess) e = hipMemcpyAsync(host.data(), nrm, host.size() * sizeof(float), hipMemcpyDeviceToHost, d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  dfree(d, p);
  if (e != hipSuccess) return hip_error(e, "rt_decode_set_layer: gate/up row norms");
  double m = 0.0;
  for (int n = 0; n < F; ++n) m = std::max(m, (double)host[n] * (double)host[F + n]);
  *out = std::isfinite(m) && m < 1e37 ? (float)(m * (1.0 + 0x1p-20)) : 0.f;
  return RT_OK;
}

rt_status rt_decode_set_layer_formats(rt_decode *d, int32_t layer, const rt_gemma3_layer *w, const int32_t *formats,
                                      int32_t device_ptrs) {
  if (!d) return set_error(RT_EINVAL, "rt_decode_set_layer: null context");
  const rt_gemma3_config &c = d->cfg;
  if (layer < 0 || layer >= c.n_layers) return set_error(RT_EINVAL, "rt_decode_set_layer: layer %d out of range", layer);
  // Any failure from here on leaves the layer unset: its old uploads are
  // freed, the captured graphs dropped, and rt_decode_step answers RT_ESTATE
  // until the layer is set again.  Nothing is freed or uploaded before every
  // argument has been checked.
  auto unset = [&](rt_status st) {
    (void)hipStreamSynchronize(d->stream);
    for (void *q : d->owned_layer[layer]) dfree(d, q);
    d->owned_layer[layer].clear();
    d->layer_set[layer] = 0;
    d->bound_weight_bytes[layer] = 0;
    drop_graph(d);
    return st;
  };
  if (!w || !formats) return unset(set_error(RT_EINVAL, "rt_decode_set_layer: null pointer"));
  {
    const size_t H = c.hidden, F = c.ffn, QD = (size_t)c.n_q_heads * c.head_dim, KVD = (size_t)c.n_kv_heads * c.head_dim;
    const size_t shape[7][2] = {{QD, H}, {KVD, H}, {KVD, H}, {H, QD}, {F, H}, {F, H}, {H, F}};
    static const char *names[7] = {"q", "k", "v", "o", "gate", "up", "down"};
    for (int p = 0; p < 7; ++p)
      if (!proj_bytes(formats[p], shape[p][0], shape[p][1]))
        return unset(set_error(RT_EINVAL, "rt_decode_set_layer: projection %s has unsupported format %d", names[p],
                               formats[p]));
    if (!d->fused && !rows_mb_formats_ok(d->shape, formats))
      return unset(set_error(RT_EINVAL,
                             "rt_decode_set_layer: this shape runs on the rows kernels, whose batched GEMVs take "
                             "Q4_K, Q6_K (whole super-blocks), Q8_0 and BF16 projections"));
  }
  // Every pointer is checked before anything is freed or uploaded; the new
  // binding is built aside and replaces the old one only when it is whole.
  const void *srcs[13] = {w->q, w->k, w->v, w->o, w->gate, w->up, w->down, w->in_norm, w->post_attn_norm,
                          w->pre_ffn_norm, w->post_ffn_norm, w->q_norm, w->k_norm};
  static const char *src_names[13] = {"q", "k", "v", "o", "gate", "up", "down", "in_norm", "post_attn_norm",
                                      "pre_ffn_norm", "post_ffn_norm", "q_norm", "k_norm"};
  for (int i = 0; i < 13; ++i) {
    if (!srcs[i]) return unset(set_error(RT_EINVAL, "rt_decode_set_layer: %s is null", src_names[i]));
    if (device_ptrs && (reinterpret_cast<uintptr_t>(srcs[i]) & 15u) != 0)
      return unset(set_error(RT_EINVAL, "rt_decode_set_layer: %s must be 16-byte aligned", src_names[i]));
  }
  (void)hipStreamSynchronize(d->stream);
  const size_t H = c.hidden, F = c.ffn, D = c.head_dim;
  const size_t QD = (size_t)c.n_q_heads * D, KVD = (size_t)c.n_kv_heads * D;
  LayerArgs L = d->layers[layer];  // keeps the cache, RoPE table and window of the layer
  std::vector<void *> own;
  const void *p;
  rt_status st = RT_OK;
#define B(field, src, bytes, cast)                                  \
  if (st == RT_OK) {                                                \
    st = bind_buf(d, src, bytes, device_ptrs, own, &p, #field);     \
    if (st == RT_OK) L.field = (cast)p;                             \
  }
  B(wq, w->q, proj_bytes(formats[kProjQ], QD, H), const uint8_t *);
  B(wk, w->k, proj_bytes(formats[kProjK], KVD, H), const uint8_t *);
  B(wv, w->v, proj_bytes(formats[kProjV], KVD, H), const uint8_t *);
  B(wo, w->o, proj_bytes(formats[kProjO], H, QD), const uint8_t *);
  B(wgate, w->gate, proj_bytes(formats[kProjGate], F, H), const uint8_t *);
  B(wup, w->up, proj_bytes(formats[kProjUp], F, H), const uint8_t *);
  B(wdown, w->down, proj_bytes(formats[kProjDown], H, F), const uint8_t *);
  B(g_in, w->in_norm, H * 4, const float *);
  B(g_post_attn, w->post_attn_norm, H * 4, const float *);
  B(g_pre_ffn, w->pre_ffn_norm, H * 4, const float *);
  B(g_post_ffn, w->post_ffn_norm, H * 4, const float *);
  B(g_q, w->q_norm, D * 4, const float *);
  B(g_k, w->k_norm, D * 4, const float *);
#undef B
  // The prefill GEMM's row exponents of each Q4_K weight, computed once here
  // (a weight bound to the context must not change until it is bound again).
  {
    const int rows[7] = {(int)QD, (int)KVD, (int)KVD, (int)H, (int)F, (int)F, (int)H};
    const int cols[7] = {(int)H, (int)H, (int)H, (int)QD, (int)H, (int)H, (int)F};
    const uint8_t *wp[7] = {L.wq, L.wk, L.wv, L.wo, L.wgate, L.wup, L.wdown};
    for (int i = 0; i < 7; ++i) {
      L.ew[i] = nullptr;
      if (st != RT_OK || formats[i] != RT_LINEAR_Q4K) continue;
      void *q = nullptr;
      st = dalloc(d, (size_t)rows[i] * 4, &q, rt_decode::kWeights);
      if (st != RT_OK) break;
      own.push_back(q);
      hipError_t e = launch_q4k_row_exponents(wp[i], rows[i], cols[i], static_cast<int *>(q), d->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
      if (e != hipSuccess) st = hip_error(e, "rt_decode_set_layer: weight row exponents");
      L.ew[i] = static_cast<const int *>(q);
    }
  }
  // The prefill's GELU GEMM bounds h = gelu(g)*u of a row by
  // |xn|^2 max_n |Wgate row n| |Wup row n|: that maximum, once here.
  L.gu_bound = 0.f;
  if (st == RT_OK && formats[kProjGate] == RT_LINEAR_Q4K && formats[kProjUp] == RT_LINEAR_Q4K)
    st = gate_up_bound(d, L.wgate, L.wup, (int)F, (int)H, &L.gu_bound);
  if (st != RT_OK) {
    for (void *q : own) dfree(d, q);
    return unset(st);
  }
  for (void *q : d->owned_layer[layer]) dfree(d, q);  // replaced by the new binding
  d->owned_layer[layer].clear();
  drop_graph(d);
  for (int i = 0; i < 7; ++i) L.fmt[i] = formats[i];
  d->layers[layer] = L;
  d->owned_layer[layer] = std::move(own);
  d->bound_weight_bytes[layer] = 0;
  if (device_ptrs) {  // borrowed: counted in rt_decode_memory's weights all the same
    const size_t sh[7][2] = {{QD, H}, {KVD, H}, {KVD, H}, {H, QD}, {F, H}, {F, H}, {H, F}};
    size_t b = (4 * H + 2 * D) * 4;
    for (int i = 0; i < 7; ++i) b += proj_bytes(formats[i], sh[i][0], sh[i][1]);
    d->bound_weight_bytes[layer] = b;
  }
  d->rows_mb = true;
  for (const LayerArgs &X : d->layers) d->rows_mb = d->rows_mb && rows_mb_formats_ok(d->shape, X.fmt);
  d->layer_set[layer] = 1;
  return RT_OK;
}

rt_status rt_decode_set_embed(rt_decode *d, const uint16_t *embed, const float *final_norm, int32_t device_ptrs) {
  if (!d) return set_error(RT_EINVAL, "rt_decode_set_embed: null context");
  // as rt_decode_set_layer: a failure leaves the embedding unset
  (void)hipStreamSynchronize(d->stream);
  std::vector<void *> own;
  const void *pe = nullptr, *pf = nullptr;
  rt_status st = RT_OK;
  if (!embed || !final_norm) st = set_error(RT_EINVAL, "rt_decode_set_embed: %s is null", embed ? "final_norm" : "embed");
  if (st == RT_OK) st = bind_buf(d, embed, (size_t)d->cfg.vocab * d->cfg.hidden * 2, device_ptrs, own, &pe, "embed");
  if (st == RT_OK) st = bind_buf(d, final_norm, (size_t)d->cfg.hidden * 4, device_ptrs, own, &pf, "final_norm");
  dfree(d, d->embed_owned);
  dfree(d, d->final_owned);
  d->embed_owned = d->final_owned = nullptr;
  drop_graph(d);
  if (st != RT_OK) {
    for (void *q : own) dfree(d, q);
    d->embed_set = false;
    d->bound_weight_bytes[64] = 0;
    return st;
  }
  d->args.embed = (const uint16_t *)pe;
  if (d->lm_fmt == 0) d->args.lm_bf16 = d->args.embed;
  d->args.g_final = (const float *)pf;
  d->bound_weight_bytes[64] = device_ptrs ? (size_t)d->cfg.vocab * d->cfg.hidden * 2 + (size_t)d->cfg.hidden * 4 : 0;
  if (!device_ptrs) {
    d->embed_owned = (void *)pe;
    d->final_owned = (void *)pf;
  }
  d->embed_set = true;
  return RT_OK;
}

// The lm_head apart from the embedding (metal_decode.rs:1079-1107): a Q4_K
// head (the model's own, or the BF16 one requantised: feature q4k-lm-head)
// or an untied BF16 one; w == nullptr restores the tied embedding.
rt_status rt_decode_set_lm_head(rt_decode *d, int32_t fmt, const void *w, int32_t device_ptrs) {
  if (!d) return set_error(RT_EINVAL, "rt_decode_set_lm_head: null context");
  const size_t V = (size_t)d->cfg.vocab, H = (size_t)d->cfg.hidden;
  rt_status st = RT_OK;
  size_t bytes = 0;
  if (w) {
    if (fmt == RT_LINEAR_Q4K && H % 256 == 0) bytes = V * (H / 256) * 144;
    else if (fmt == RT_LINEAR_BF16) bytes = V * H * 2;
    else
      st = set_error(RT_EINVAL, "rt_decode_set_lm_head: format %d unsupported (RT_LINEAR_Q4K with hidden %% 256 == 0, "
                     "or RT_LINEAR_BF16)", fmt);
  }
  // the new head is built aside; any failure leaves the tied embedding
  (void)hipStreamSynchronize(d->stream);
  std::vector<void *> own;
  const void *pw = nullptr;
  void *stage = nullptr, *part = nullptr;
  if (st == RT_OK && w) st = bind_buf(d, w, bytes, device_ptrs, own, &pw, "lm_head");
  if (st == RT_OK && w && fmt == RT_LINEAR_Q4K) {
    st = dalloc(d, mb_stage_bytes((int)H), &stage, rt_decode::kBatch);
    if (st == RT_OK) own.push_back(stage);
    const size_t pb = mb_head_part_bytes((int)V, (int)H);
    if (st == RT_OK && pb) {
      st = dalloc(d, pb, &part, rt_decode::kBatch);
      if (st == RT_OK) own.push_back(part);
    }
  }
  for (void *q : d->lm_owned) dfree(d, q);
  d->lm_owned.clear();
  drop_graph(d);
  d->lm_fmt = 0;
  d->args.lm_q4k = nullptr;
  d->args.lm_stage = nullptr;
  d->args.lm_part = nullptr;
  d->args.lm_bf16 = d->args.embed;
  d->bound_weight_bytes[65] = 0;
  if (st != RT_OK) {
    for (void *q : own) dfree(d, q);
    return st;
  }
  if (!w) return RT_OK;
  d->lm_fmt = fmt;
  d->lm_owned = std::move(own);
  if (fmt == RT_LINEAR_Q4K) {
    d->args.lm_q4k = static_cast<const uint8_t *>(pw);
    d->args.lm_stage = stage;
    d->args.lm_part = static_cast<float *>(part);
  } else {
    d->args.lm_bf16 = static_cast<const uint16_t *>(pw);
  }
  if (device_ptrs) d->bound_weight_bytes[65] = bytes;
  return RT_OK;
}

// sync_kv_from_cpu (metal_decode.rs:1366-1396) for one layer: rows
// [0, seq_len) of K and V, each [seq_len, n_kv_heads*head_dim] f32.
rt_status rt_decode_sync_kv(rt_decode *d, int32_t layer, const float *k, const float *v, int32_t seq_len,
                            int32_t device_ptrs) {
  if (!d || !k || !v) return set_error(RT_EINVAL, "rt_decode_sync_kv: null pointer");
  if (layer < 0 || layer >= d->cfg.n_layers) return set_error(RT_EINVAL, "rt_decode_sync_kv: layer %d out of range", layer);
  if (seq_len < 0 || seq_len > d->cfg.max_seq)
    return set_error(RT_EINVAL, "rt_decode_sync_kv: seq_len %d outside [0, max_seq=%d]", seq_len, d->cfg.max_seq);
  const size_t bytes = (size_t)seq_len * d->cfg.n_kv_heads * d->cfg.head_dim * 4;
  const hipMemcpyKind kind = device_ptrs ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  hipError_t e = hipMemcpyAsync(d->layers[layer].kc, k, bytes, kind, d->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(d->layers[layer].vc, v, bytes, kind, d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  return hip_error(e, "rt_decode_sync_kv");
}

static rt_status check_ready(rt_decode *d, int32_t token, int32_t position) {
  if (!d) return set_error(RT_EINVAL, "rt_decode_step: null context");
  if (!d->embed_set) return set_error(RT_ESTATE, "rt_decode_step: embedding not set");
  for (int l = 0; l < d->cfg.n_layers; ++l)
    if (!d->layer_set[l]) return set_error(RT_ESTATE, "rt_decode_step: layer %d weights not set", l);
  if (token < 0 || token >= d->cfg.vocab)
    return set_error(RT_EINVAL, "rt_decode_step: token %d outside [0, vocab=%d)", token, d->cfg.vocab);
  if (position < 0 || position >= d->cfg.max_seq)
    return set_error(RT_EINVAL, "rt_decode_step: position %d outside [0, max_seq=%d)", position, d->cfg.max_seq);
  return RT_OK;
}

// Token id, position and the RoPE cos/sin tables of slot `slot`: angle =
// (pos*fs)/theta^(2i/d) in f32 with the host libm, as apply_rope_at_offset
// computes it (transformer4.rs:2742-2772).
static void fill_slot(rt_decode *d, int slot, int32_t token, int32_t position) {
  int *ip = reinterpret_cast<int *>(reinterpret_cast<char *>(d->params_host) + (size_t)slot * d->slot_bytes);
  ip[0] = token;
  ip[1] = position;
  const int D = d->cfg.head_dim, P = D / 2;
  float *cs = reinterpret_cast<float *>(ip) + kParamRopeLocal;
  for (int t = 0; t < 2; ++t, cs += D) {
    const float fs = t ? d->cfg.rope_fs_global : d->cfg.rope_fs_local;
    const float *den = t ? d->rope_den_global.data() : d->rope_den_local.data();
    const float pf = (float)position * fs;
    for (int i = 0; i < P; ++i) {
      const float ang = pf / den[i];
      cs[i] = cosf(ang);
      cs[P + i] = sinf(ang);
    }
  }
}

// Waits until the previous parameter copy has left the pinned buffer.
static rt_status params_ready(rt_decode *d) {
  if (!d->params_pending) return RT_OK;
  return hip_error(hipEventSynchronize(d->params_copied), "rt_decode_step");
}

static rt_status params_send(rt_decode *d, int slots) {
  hipError_t e = hipMemcpyAsync(d->params_dev, d->params_host, (size_t)slots * d->slot_bytes, hipMemcpyHostToDevice,
                                d->stream);
  if (e == hipSuccess) e = hipEventRecord(d->params_copied, d->stream);
  if (e != hipSuccess) return hip_error(e, "rt_decode_step params");
  d->params_pending = true;
  return RT_OK;
}

// m rows (m <= kMaxBatch) at the positions and tokens of the step parameter
// slots, each attending its own window as a decode step does, projections
// on the batched GEMV (every projection Q4_K).
static RowsPlan rows_plan_params(rt_decode *d, int m) {
  const int slot = param_slot_floats(d->cfg.head_dim);
  RowsPlan plan;
  plan.n = m;
  plan.p0_dev = d->params_dev + 1;
  plan.tokens = d->params_dev;
  plan.tok_stride = slot;
  plan.cs = reinterpret_cast<const float *>(d->params_dev) + kParamRopeLocal;
  plan.cs_stride = slot;
  plan.window = d->cfg.sliding_window;
  plan.max_pos = d->cfg.max_seq;
  plan.mb = true;
  return plan;
}

// Launch `enqueue` through a graph captured on first use (or eagerly when
// graphs are off).
extern "C++" template <class F>
static rt_status run_graph(rt_decode *d, hipGraphExec_t &exec, F enqueue, const char *what) {
  if (!d->graph_enabled) return hip_error(enqueue(), what);
  if (d->graph_dirty) drop_graph(d);
  if (!exec) {
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_error(e, "hipStreamBeginCapture");
    hipError_t le = enqueue();
    e = hipStreamEndCapture(d->stream, &g);
    if (le != hipSuccess) {
      if (g) (void)hipGraphDestroy(g);
      return hip_error(le, what);
    }
    if (e != hipSuccess) return hip_error(e, "hipStreamEndCapture");
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
      exec = nullptr;
      return hip_error(e, "hipGraphInstantiate");
    }
  }
  d->graph_dirty = false;
  return hip_error(hipGraphLaunch(exec, d->stream), "hipGraphLaunch");
}

rt_status rt_decode_step_async(rt_decode *d, int32_t token, int32_t position) {
  rt_status st = check_ready(d, token, position);
  if (st == RT_OK) st = params_ready(d);
  if (st != RT_OK) return st;
  fill_slot(d, 0, token, position);
  if ((st = params_send(d, 1)) != RT_OK) return st;
  if (!d->fused)  // one row through the rows kernels: batched GEMVs, row attention, lm_head
    return run_graph(d, d->exec, [&] {
      RowsPlan plan = rows_plan_params(d, 1);
      plan.logits = RowsPlan::kLastRow;
      return enqueue_rows(d->shape, d->args, d->layers.data(), d->vb, plan, d->stream);
    }, "rt_decode_step");
  return run_graph(d, d->exec, [&] { return enqueue_decode_step(d->shape, d->args, d->layers.data(), d->stream); },
                   "rt_decode_step");
}

// decode_step_batch (metal_decode.rs:2079-2179): m <= 8 tokens at positions
// start .. start+m-1.  Each token sees the keys of the ones before it, as in
// the reference (its K/V rows are appended before its attention); the
// logits of token i land in row i of the batch logits buffer.
rt_status rt_decode_step_batch_async(rt_decode *d, const int32_t *tokens, int32_t m, int32_t start_position) {
  if (!d || !tokens) return set_error(RT_EINVAL, "rt_decode_step_batch: null pointer");
  if (m < 1 || m > kMaxBatch) return set_error(RT_EINVAL, "rt_decode_step_batch: M=%d outside [1, %d]", m, kMaxBatch);
  for (int i = 0; i < m; ++i) {
    rt_status st = check_ready(d, tokens[i], start_position + i);
    if (st != RT_OK) return st;
  }
  rt_status st = params_ready(d);
  if (st != RT_OK) return st;
  for (int i = 0; i < m; ++i) fill_slot(d, i, tokens[i], start_position + i);
  if ((st = params_send(d, m)) != RT_OK) return st;
  return run_graph(d, d->exec_batch[m], [&] {
    if (!d->rows_mb)  // per-token layer kernels (any projection format)
      return enqueue_decode_batch(d->shape, d->args, d->layers.data(), m, d->xn_batch, d->logits_batch, d->stream);
    // all rows through each layer at once: batched GEMVs (one pass over the
    // weights), the causal row attention, a batched lm_head
    RowsPlan plan = rows_plan_params(d, m);
    plan.logits = RowsPlan::kEveryRow;
    plan.xn_b = d->xn_batch;
    plan.logits_b = d->logits_batch;
    return enqueue_rows(d->shape, d->args, d->layers.data(), d->vb, plan, d->stream);
  }, "rt_decode_step_batch");
}

rt_status rt_decode_step_batch(rt_decode *d, const int32_t *tokens, int32_t m, int32_t start_position,
                               float *logits_host) {
  rt_status st = rt_decode_step_batch_async(d, tokens, m, start_position);
  if (st != RT_OK) return st;
  hipError_t e = hipSuccess;
  if (logits_host)
    e = hipMemcpyAsync(logits_host, d->logits_batch, (size_t)m * d->cfg.vocab * 4, hipMemcpyDeviceToHost, d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  return hip_error(e, "rt_decode_step_batch");
}

rt_status rt_decode_logits_batch(rt_decode *d, float **logits_dev) {
  if (!d || !logits_dev) return set_error(RT_EINVAL, "rt_decode_logits_batch: null pointer");
  *logits_dev = d->logits_batch;
  return RT_OK;
}

rt_status rt_decode_step(rt_decode *d, int32_t token, int32_t position, float *logits_host) {
  rt_status st = rt_decode_step_async(d, token, position);
  if (st != RT_OK) return st;
  hipError_t e = hipSuccess;
  if (logits_host)
    e = hipMemcpyAsync(logits_host, d->args.logits, (size_t)d->cfg.vocab * 4, hipMemcpyDeviceToHost, d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  return hip_error(e, "rt_decode_step");
}

// ---------------------------------------------------------------------------
// Prefill
// ---------------------------------------------------------------------------
static rt_status prefill_reserve(rt_decode *d, int cap) {
  PrefillBuffers &b = d->pf;
  if (b.cap >= cap) return RT_OK;
  hipError_t e = hipStreamSynchronize(d->stream);
  if (e != hipSuccess) return hip_error(e, "rt_decode_prefill");
  for (void *p : d->pf_owned) dfree(d, p);
  d->pf_owned.clear();
  if (d->pf_tokens_host) (void)hipHostFree(d->pf_tokens_host);
  d->pf_tokens_host = nullptr;
  b = PrefillBuffers{};
  const rt_gemma3_config &c = d->cfg;
  const size_t H = c.hidden, F = c.ffn, D = c.head_dim, QD = (size_t)c.n_q_heads * D, KVD = (size_t)c.n_kv_heads * D;
  const size_t rows = (size_t)cap;
  auto get = [&](size_t bytes, void **dst) -> rt_status {
    rt_status st = dalloc(d, std::max<size_t>(bytes, 256), dst, rt_decode::kPrefill);
    if (st == RT_OK) d->pf_owned.push_back(*dst);
    return st;
  };
  rt_status st = RT_OK;
  void *p = nullptr;
#define PF_GET(field, type, count)                     \
  if ((st = get((count) * sizeof(type), &p)) != RT_OK) \
    return st;                                         \
  b.field = static_cast<type *>(p);
  PF_GET(tokens, int, rows);
  PF_GET(hid, float, rows * H);
  PF_GET(x2, float, rows * H);
  PF_GET(xn, float, rows * H);
  PF_GET(o, float, rows * H);
  PF_GET(dn, float, rows * H);
  PF_GET(q, float, rows * QD);
  PF_GET(attn, float, rows * QD);
  PF_GET(k, float, rows * KVD);
  PF_GET(v, float, rows * KVD);
  PF_GET(g, float, rows * F);
  PF_GET(u, float, rows * F);
  PF_GET(nrm2, float, rows);
#undef PF_GET
  if ((st = get(prefill_gemm_workspace_bytes(d->shape, cap), &b.ws)) != RT_OK) return st;
  if ((st = get(rows_mb_stage_bytes(d->shape), &b.mb_stage)) != RT_OK) return st;
  if ((st = get(rows_mb_part_bytes(d->shape), &p)) != RT_OK) return st;
  b.mb_part = static_cast<float *>(p);
  // key-split partials: 64 splits of 128 rows (two splits of a 4096-row
  // chunk's causal attention, eight of a 1024-row window; more splits
  // measured slower: the walk is bound by the K/V stage reads in aggregate)
  const int split_rows = std::min(cap, 128);
  if ((st = get(attn_part_floats(d->shape, split_rows, false) * 4, &p)) != RT_OK) return st;
  b.attn_ml = static_cast<float *>(p);
  if ((st = get(attn_part_floats(d->shape, split_rows, true) * 4, &p)) != RT_OK) return st;
  b.attn_o = static_cast<float *>(p);
  b.attn_rows = split_rows;
  e = hipHostMalloc((void **)&d->pf_tokens_host, rows * sizeof(int), hipHostMallocDefault);
  if (e != hipSuccess) return hip_error(e, "rt_decode_prefill hipHostMalloc");
  b.cap = cap;
  return RT_OK;
}

// The cos/sin tables of positions 0 .. `upto`-1 (rounded up to 4096, at most
// max_seq), local then global per row, with the host libm as fill_slot
// computes them for a decode step.  They depend on the position alone, so
// they are computed once (about 2 ms of host time per 4096 positions on 16
// threads) and every prefill reads its rows' slice; a prefill past the
// table's end computes it again, longer.
static rt_status prefill_rope_table(rt_decode *d, int upto) {
  if (d->rope_rows >= upto) return RT_OK;
  const int D = d->cfg.head_dim, P = D / 2, n = std::min(d->cfg.max_seq, (upto + 4095) / 4096 * 4096);
  std::vector<float> host((size_t)n * 2 * D);
  auto rows = [&](int t0, int t1) {
    for (int t = t0; t < t1; ++t) {
      float *cs = host.data() + (size_t)t * 2 * D;
      for (int k = 0; k < 2; ++k, cs += D) {
        const float fs = k ? d->cfg.rope_fs_global : d->cfg.rope_fs_local;
        const float *den = k ? d->rope_den_global.data() : d->rope_den_local.data();
        const float pf = (float)t * fs;
        for (int i = 0; i < P; ++i) {
          const float ang = pf / den[i];
          cs[i] = cosf(ang);
          cs[P + i] = sinf(ang);
        }
      }
    }
  };
  const int nt = std::max(1, std::min({16, (int)std::thread::hardware_concurrency(), n / 64}));
  if (nt == 1) {
    rows(0, n);
  } else {
    std::vector<std::thread> pool;
    const int per = (n + nt - 1) / nt;
    for (int i = 0; i < nt; ++i) pool.emplace_back(rows, std::min(n, i * per), std::min(n, (i + 1) * per));
    for (auto &th : pool) th.join();
  }
  hipError_t e = hipStreamSynchronize(d->stream);  // no queued prefill reads the old table
  if (e != hipSuccess) return hip_error(e, "rt_decode_prefill");
  if (d->rope_cs) dfree(d, d->rope_cs);
  d->rope_cs = nullptr;
  d->rope_rows = 0;
  void *p = nullptr;
  rt_status st = dalloc(d, host.size() * sizeof(float), &p, rt_decode::kPrefill);
  if (st != RT_OK) return st;
  e = hipMemcpy(p, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    dfree(d, p);
    return hip_error(e, "rt_decode_prefill position table");
  }
  d->rope_cs = static_cast<float *>(p);
  d->rope_rows = n;
  return RT_OK;
}

rt_status rt_decode_prefill(rt_decode *d, const int32_t *tokens, int32_t n, int32_t start_position, int32_t mode,
                            float *logits_host) {
  if (!d || !tokens) return set_error(RT_EINVAL, "rt_decode_prefill: null pointer");
  if (n < 1) return set_error(RT_EINVAL, "rt_decode_prefill: n=%d must be >= 1", n);
  if (mode != RT_PREFILL_REFERENCE && mode != RT_PREFILL_SLIDING)
    return set_error(RT_EINVAL, "rt_decode_prefill: unknown mode %d", mode);
  if (mode == RT_PREFILL_REFERENCE && start_position != 0)
    return set_error(RT_EINVAL, "rt_decode_prefill: RT_PREFILL_REFERENCE starts at position 0 (got %d)",
                     start_position);
  if (start_position < 0 || (int64_t)start_position + n > d->cfg.max_seq)
    return set_error(RT_EINVAL, "rt_decode_prefill: positions [%d, %lld) outside [0, max_seq=%d)", start_position,
                     (long long)start_position + n, d->cfg.max_seq);
  for (int i = 0; i < n; ++i) {
    rt_status st = check_ready(d, tokens[i], start_position + i);
    if (st != RT_OK) return st;
  }
  const int w = d->cfg.sliding_window;
  int lo_fixed = 0, window = 0;
  if (mode == RT_PREFILL_REFERENCE)
    lo_fixed = (w > 0 && n > w) ? n - w : 0;  // k_start = seq_len - window (transformer4.rs:1926-1929)
  else
    window = w;
  const int cap = std::min(n, d->pf_chunk);
  rt_status st = prefill_reserve(d, cap);
  if (st == RT_OK) st = prefill_rope_table(d, start_position + n);
  if (st != RT_OK) return st;
  const int D = d->cfg.head_dim;
  hipError_t e = hipSuccess;
  for (int c0 = 0; c0 < n && e == hipSuccess; c0 += cap) {
    const int cn = std::min(cap, n - c0);
    e = hipStreamSynchronize(d->stream);  // the staging buffers are free again
    if (e != hipSuccess) break;
    std::memcpy(d->pf_tokens_host, tokens + c0, (size_t)cn * sizeof(int));
    e = hipMemcpyAsync(d->pf.tokens, d->pf_tokens_host, (size_t)cn * sizeof(int), hipMemcpyHostToDevice, d->stream);
    if (e == hipSuccess) {
      RowsPlan plan;
      plan.n = cn;
      plan.p0 = start_position + c0;
      plan.tokens = d->pf.tokens;
      plan.cs = d->rope_cs + (size_t)(start_position + c0) * 2 * D;
      plan.cs_stride = 2 * D;
      plan.lo_fixed = lo_fixed;
      plan.window = window;
      plan.max_pos = start_position + c0 + cn;
      plan.mb = cn <= kMaxBatch && d->rows_mb;  // a few rows: one pass over the weights beats the GEMM's tiles
      const bool last_chunk = c0 + cn == n;
      if (cn == 1) {
        plan.logits = last_chunk ? RowsPlan::kLastRow : RowsPlan::kNone;
        e = enqueue_rows(d->shape, d->args, d->layers.data(), d->pf, plan, d->stream);
      } else {
        // The last layer's attention, o projection and FFN only feed the
        // logits: every row runs up to the last layer's K/V rows, and the
        // prompt's last row alone (if its logits are wanted) runs the rest.
        plan.logits = RowsPlan::kNone;
        plan.last_layer_kv_only = true;
        e = enqueue_rows(d->shape, d->args, d->layers.data(), d->pf, plan, d->stream);
        if (e == hipSuccess && last_chunk) {
          const size_t r = (size_t)cn - 1;
          const rt_gemma3_config &c = d->cfg;
          const size_t Hs = c.hidden, Fs = c.ffn, QDs = (size_t)c.n_q_heads * D, KVDs = (size_t)c.n_kv_heads * D;
          PrefillBuffers tb = d->pf;  // the buffers' rows from the last one on
          tb.tokens += r;
          tb.hid += r * Hs, tb.x2 += r * Hs, tb.xn += r * Hs, tb.o += r * Hs, tb.dn += r * Hs;
          tb.q += r * QDs, tb.attn += r * QDs, tb.k += r * KVDs, tb.v += r * KVDs;
          tb.g += r * Fs, tb.u += r * Fs, tb.nrm2 += r;
          RowsPlan tail = plan;
          tail.n = 1;
          tail.p0 = plan.p0 + (int)r;
          tail.tokens = tb.tokens;
          tail.cs = plan.cs + r * 2 * D;
          tail.mb = d->rows_mb;
          tail.logits = RowsPlan::kLastRow;
          tail.layer_begin = c.n_layers - 1;
          tail.qkv_done = true;
          tail.last_layer_kv_only = false;
          e = enqueue_rows(d->shape, d->args, d->layers.data(), tb, tail, d->stream);
        }
      }
    }
  }
  if (e == hipSuccess && logits_host)
    e = hipMemcpyAsync(logits_host, d->args.logits, (size_t)d->cfg.vocab * 4, hipMemcpyDeviceToHost, d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  return hip_error(e, "rt_decode_prefill");
}

rt_status rt_decode_set_prefill_chunk(rt_decode *d, int32_t rows) {
  if (!d) return set_error(RT_EINVAL, "rt_decode_set_prefill_chunk: null context");
  if (rows < 1) return set_error(RT_EINVAL, "rt_decode_set_prefill_chunk: rows=%d must be >= 1", rows);
  d->pf_chunk = rows;
  return RT_OK;
}

rt_status rt_decode_synchronize(rt_decode *d) {
  if (!d) return set_error(RT_EINVAL, "rt_decode_synchronize: null context");
  return hip_error(hipStreamSynchronize(d->stream), "rt_decode_synchronize");
}

rt_status rt_decode_set_graph(rt_decode *d, int32_t enabled) {
  if (!d) return set_error(RT_EINVAL, "rt_decode_set_graph: null context");
  (void)hipStreamSynchronize(d->stream);
  d->graph_enabled = enabled != 0;
  drop_graph(d);
  return RT_OK;
}

// Whether decode_step_batch runs every layer through the batched GEMVs (one
// pass over the weights for all rows) or falls back to per-token passes.
rt_status rt_decode_verify_batched(const rt_decode *d, int32_t *batched) {
  if (!d || !batched) return set_error(RT_EINVAL, "rt_decode_verify_batched: null pointer");
  *batched = d->rows_mb ? 1 : 0;
  return RT_OK;
}

// print_metal_memory (metal_decode.rs:1285-1354): the device memory of the
// context by what it holds.  Weights bound by device pointer count too, as
// the reference's uploads do; the prefill scratch appears once a prefill has
// sized it.
rt_status rt_decode_memory(const rt_decode *d, rt_decode_memory_info *out) {
  if (!d || !out) return set_error(RT_EINVAL, "rt_decode_memory: null pointer");
  uint64_t by[rt_decode::kMemKinds] = {};
  for (const auto &a : d->owned)
    if (a.p) by[a.kind] += a.bytes;
  for (size_t b : d->bound_weight_bytes) by[rt_decode::kWeights] += b;
  out->weights = by[rt_decode::kWeights];
  out->kv_cache = by[rt_decode::kKv];
  out->activation = by[rt_decode::kActivation];
  out->batch = by[rt_decode::kBatch];
  out->prefill = by[rt_decode::kPrefill];
  out->total = out->weights + out->kv_cache + out->activation + out->batch + out->prefill;
  return RT_OK;
}

rt_status rt_decode_logits(rt_decode *d, float **logits_dev) {
  if (!d || !logits_dev) return set_error(RT_EINVAL, "rt_decode_logits: null pointer");
  *logits_dev = d->args.logits;
  return RT_OK;
}

rt_status rt_decode_kv(rt_decode *d, int32_t layer, float **k_dev, float **v_dev) {
  if (!d || !k_dev || !v_dev) return set_error(RT_EINVAL, "rt_decode_kv: null pointer");
  if (layer < 0 || layer >= d->cfg.n_layers) return set_error(RT_EINVAL, "rt_decode_kv: layer %d out of range", layer);
  *k_dev = d->layers[layer].kc;
  *v_dev = d->layers[layer].vc;
  return RT_OK;
}

rt_status rt_decode_hidden(rt_decode *d, float **x2_dev, float **dn_dev) {
  if (!d || !x2_dev || !dn_dev) return set_error(RT_EINVAL, "rt_decode_hidden: null pointer");
  *x2_dev = d->args.x2;
  *dn_dev = d->args.dn;
  return RT_OK;
}

rt_status rt_decode_get_stream(rt_decode *d, void **stream) {
  if (!d || !stream) return set_error(RT_EINVAL, "rt_decode_get_stream: null pointer");
  *stream = d->stream;
  return RT_OK;
}

}  // extern "C"
