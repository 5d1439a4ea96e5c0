// capi.hip -- extern "C" boundary of librt_hip.so (declared in include/rt_hip.h).
//
// Validation happens here, before any kernel is launched: every shape the
// kernels assume (K multiple of 256 or 8, 16-byte alignment, non-null
// pointers, int32 row counts) is checked on the host and reported as
// RT_EINVAL instead of reaching the GPU.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>
#include <algorithm>

#include "../../include/rt_hip.h"
#include "rt_capi_util.hpp"
#include "q4k_gemv_mb.hpp"
#include "rt_kernels.hpp"

namespace rt {

static thread_local std::string g_last_error;

rt_status set_error(rt_status code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

rt_status hip_error(hipError_t e, const char *what) {
  if (e == hipSuccess) return RT_OK;
  if (e == hipErrorOutOfMemory) return set_error(RT_ENOMEM, "%s: %s", what, hipGetErrorString(e));
  return set_error(RT_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace rt

using namespace rt;

extern "C" {

const char *rt_last_error(void) { return g_last_error.c_str(); }

int32_t rt_abi_version(void) { return 1; }

rt_status rt_q4k_dequant_f32(const void *blocks, size_t n_blocks, float *out, void *stream) {
  if (n_blocks == 0) return RT_OK;
  if (!blocks || !out) return set_error(RT_EINVAL, "rt_q4k_dequant_f32: null pointer");
  if (!aligned16(blocks) || !aligned16(out)) return set_error(RT_EINVAL, "rt_q4k_dequant_f32: buffers must be 16-byte aligned");
  return hip_error(launch_q4k_dequant(blocks, n_blocks, out, false, (hipStream_t)stream), "rt_q4k_dequant_f32");
}

rt_status rt_q4k_dequant_bf16(const void *blocks, size_t n_blocks, uint16_t *out, void *stream) {
  if (n_blocks == 0) return RT_OK;
  if (!blocks || !out) return set_error(RT_EINVAL, "rt_q4k_dequant_bf16: null pointer");
  if (!aligned16(blocks) || !aligned16(out)) return set_error(RT_EINVAL, "rt_q4k_dequant_bf16: buffers must be 16-byte aligned");
  return hip_error(launch_q4k_dequant(blocks, n_blocks, out, true, (hipStream_t)stream), "rt_q4k_dequant_bf16");
}

rt_status check_gemv_shape(const char *who, const void *w, const float *x, const float *y, int64_t n, int64_t k,
                           int64_t kmult) {
  if (n <= 0 || k <= 0) return set_error(RT_EINVAL, "%s: n=%lld k=%lld must be positive", who, (long long)n, (long long)k);
  if (k % kmult != 0) return set_error(RT_EINVAL, "%s: k=%lld must be a multiple of %lld", who, (long long)k, (long long)kmult);
  if (n > INT32_MAX || k > INT32_MAX) return set_error(RT_EINVAL, "%s: n or k exceeds int32", who);
  if (!w || !x || !y) return set_error(RT_EINVAL, "%s: null pointer", who);
  if (!aligned16(w) || !aligned16(x)) return set_error(RT_EINVAL, "%s: w and x must be 16-byte aligned", who);
  return RT_OK;
}

rt_status rt_q4k_gemv(const void *w, const float *x, float *y, int64_t n, int64_t k, void *stream) {
  rt_status st = check_gemv_shape("rt_q4k_gemv", w, x, y, n, k, 256);
  if (st != RT_OK) return st;
  return hip_error(launch_q4k_gemv(w, x, y, (int)n, (int)k, (hipStream_t)stream), "rt_q4k_gemv");
}

// The q, k, v (or gate, up) GEMVs of one step share their input and are
// dispatched one by one by the reference (metal_decode.rs:1948-1954,
// 2001-2004); one launch covers them here.
rt_status rt_q4k_gemv_multi(const void *const *w, float *const *y, const int64_t *n, int32_t count, const float *x,
                            int64_t k, void *stream) {
  static const char *who = "rt_q4k_gemv_multi";
  if (!w || !y || !n) return set_error(RT_EINVAL, "%s: null array", who);
  if (count < 1 || count > kGemvMaxMats)
    return set_error(RT_EINVAL, "%s: count=%d outside [1, %d]", who, count, kGemvMaxMats);
  int ni[kGemvMaxMats];
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    rt_status st = check_gemv_shape(who, w[i], x, y[i], n[i], k, 256);
    if (st != RT_OK) return st;
    ni[i] = (int)n[i];
    total += n[i];
  }
  if (total > INT32_MAX) return set_error(RT_EINVAL, "%s: total rows exceed int32", who);
  return hip_error(launch_q4k_gemv_multi(w, y, ni, count, x, (int)k, (hipStream_t)stream), who);
}

rt_status rt_bf16_gemv(const uint16_t *w, const float *x, float *y, int64_t n, int64_t k, void *stream) {
  rt_status st = check_gemv_shape("rt_bf16_gemv", w, x, y, n, k, 8);
  if (st != RT_OK) return st;
  return hip_error(launch_bf16_gemv(w, x, y, (int)n, (int)k, (hipStream_t)stream), "rt_bf16_gemv");
}

// gelu_tanh (autograd2.rs:3082-3091) as the decode step and prefill apply it.
rt_status rt_gelu_tanh(const float *x, float *y, size_t n, void *stream) {
  if (n == 0) return RT_OK;
  if (!x || !y) return set_error(RT_EINVAL, "rt_gelu_tanh: null pointer");
  return hip_error(launch_gelu_tanh(x, y, n, (hipStream_t)stream), "rt_gelu_tanh");
}

rt_status rt_q6k_repack(const void *gguf_blocks, size_t n_blocks, void *dst) {
  if (n_blocks == 0) return RT_OK;
  if (!gguf_blocks || !dst) return set_error(RT_EINVAL, "rt_q6k_repack: null pointer");
  q6k_repack_host(static_cast<const uint8_t *>(gguf_blocks), n_blocks, static_cast<uint8_t *>(dst));
  return RT_OK;
}

rt_status rt_q8_0_repack(const void *gguf_blocks, size_t n_blocks, void *dst) {
  if (n_blocks == 0) return RT_OK;
  if (!gguf_blocks || !dst) return set_error(RT_EINVAL, "rt_q8_0_repack: null pointer");
  q8_0_repack_host(static_cast<const uint8_t *>(gguf_blocks), n_blocks, static_cast<uint8_t *>(dst));
  return RT_OK;
}

rt_status rt_q6k_dequant_f32(const void *w, size_t n_blocks, float *out, void *stream) {
  if (n_blocks == 0) return RT_OK;
  if (!w || !out) return set_error(RT_EINVAL, "rt_q6k_dequant_f32: null pointer");
  if (!aligned16(w)) return set_error(RT_EINVAL, "rt_q6k_dequant_f32: w must be 16-byte aligned");
  return hip_error(launch_q6k_dequant(w, n_blocks, out, (hipStream_t)stream), "rt_q6k_dequant_f32");
}

rt_status rt_q8_0_dequant_f32(const void *w, size_t n_elem, float *out, void *stream) {
  if (n_elem == 0) return RT_OK;
  if (!w || !out) return set_error(RT_EINVAL, "rt_q8_0_dequant_f32: null pointer");
  if (n_elem % 32 != 0) return set_error(RT_EINVAL, "rt_q8_0_dequant_f32: n_elem=%zu must be a multiple of 32", n_elem);
  if (!aligned16(w)) return set_error(RT_EINVAL, "rt_q8_0_dequant_f32: w must be 16-byte aligned");
  return hip_error(launch_q8_0_dequant(w, n_elem, out, (hipStream_t)stream), "rt_q8_0_dequant_f32");
}

rt_status rt_q6k_gemv(const void *w, const float *x, float *y, int64_t n, int64_t k, void *stream) {
  rt_status st = check_gemv_shape("rt_q6k_gemv", w, x, y, n, k, 256);
  if (st != RT_OK) return st;
  return hip_error(launch_q6k_gemv(w, x, y, (int)n, (int)k, (hipStream_t)stream), "rt_q6k_gemv");
}

rt_status rt_q8_0_gemv(const void *w, const float *x, float *y, int64_t n, int64_t k, void *stream) {
  rt_status st = check_gemv_shape("rt_q8_0_gemv", w, x, y, n, k, 32);
  if (st != RT_OK) return st;
  return hip_error(launch_q8_0_gemv(w, x, y, (int)n, (int)k, (hipStream_t)stream), "rt_q8_0_gemv");
}

}  // extern "C"

namespace {
rt_status gemm_workspace(size_t bytes, hipStream_t stream, void **out);

rt_status q4k_gemm_entry(const char *who, const void *a, bool a_bf16, const void *w, float *c, int64_t m, int64_t n,
                         int64_t k, void *stream) {
  if (m <= 0 || n <= 0 || k <= 0)
    return set_error(RT_EINVAL, "%s: m=%lld n=%lld k=%lld must be positive", who, (long long)m, (long long)n,
                     (long long)k);
  if (k % 256 != 0) return set_error(RT_EINVAL, "%s: k=%lld must be a multiple of 256", who, (long long)k);
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return set_error(RT_EINVAL, "%s: m, n or k exceeds int32", who);
  if (!a || !w || !c) return set_error(RT_EINVAL, "%s: null pointer", who);
  if (!aligned16(a) || !aligned16(w)) return set_error(RT_EINVAL, "%s: a and w must be 16-byte aligned", who);
  if ((reinterpret_cast<uintptr_t>(c) & 3u) != 0) return set_error(RT_EINVAL, "%s: c must be 4-byte aligned", who);
  void *ws = nullptr;
  rt_status st = gemm_workspace(q4k_gemm_workspace_bytes((int)m, (int)n, (int)k), (hipStream_t)stream, &ws);
  if (st != RT_OK) return st;
  return hip_error(launch_q4k_gemm(a, a_bf16, w, c, (int)m, (int)n, (int)k, ws, (hipStream_t)stream), who);
}
}  // namespace

extern "C" {

rt_status rt_q4k_gemm_bf16(const uint16_t *a, const void *w, float *c, int64_t m, int64_t n, int64_t k,
                           void *stream) {
  return q4k_gemm_entry("rt_q4k_gemm_bf16", a, true, w, c, m, n, k, stream);
}

rt_status rt_q4k_gemm_f32(const float *a, const void *w, float *c, int64_t m, int64_t n, int64_t k, void *stream) {
  return q4k_gemm_entry("rt_q4k_gemm_f32", a, false, w, c, m, n, k, stream);
}

// The matmul of QLinear::forward (qlinear.rs:82-111) for a weight of any
// format: Q4_K -> matmul_q4k_t_exact (the Q4_K GEMM); BF16, and Q6_K / Q8_0
// which the reference widens to BF16 -> MatBf16::matmul_by_t
// (autograd2.rs:757-852); F32 -> Mat::matmul_bt (autograd2.rs:378-429).  With
// a bias, add_bias_rows (qlinear.rs:49-60) follows.
static rt_status linear_forward(const char *who, int32_t fmt, const void *w, const float *bias, const float *a,
                                float *c, int64_t m, int64_t n, int64_t k, void *stream) {
  hipStream_t s = (hipStream_t)stream;
  if (fmt != RT_LINEAR_Q4K && fmt != RT_LINEAR_BF16 && fmt != RT_LINEAR_Q6K && fmt != RT_LINEAR_Q8_0 &&
      fmt != RT_LINEAR_F32)
    return set_error(RT_EINVAL, "%s: unsupported format %d", who, fmt);
  if (m <= 0 || n <= 0 || k <= 0)
    return set_error(RT_EINVAL, "%s: m=%lld n=%lld k=%lld must be positive", who, (long long)m, (long long)n,
                     (long long)k);
  // K granularity: Q4_K / Q6_K super-blocks, the f16 GEMM's 64-wide stages,
  // or (f32 weights) 16-byte row loads
  const bool few = m <= 8;  // f32 / bf16 weights: the row-group GEMV
  const int align = (fmt == RT_LINEAR_Q4K || fmt == RT_LINEAR_Q6K) ? 256
                    : fmt == RT_LINEAR_F32                         ? 4
                    : fmt == RT_LINEAR_BF16 && (few || k % 64)     ? 8
                                                                   : 64;
  if (k % align != 0) return set_error(RT_EINVAL, "%s: k=%lld must be a multiple of %d", who, (long long)k, align);
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return set_error(RT_EINVAL, "%s: m, n or k exceeds int32", who);
  if (!a || !w || !c) return set_error(RT_EINVAL, "%s: null pointer", who);
  if (!aligned16(a) || !aligned16(w)) return set_error(RT_EINVAL, "%s: a and w must be 16-byte aligned", who);
  if ((reinterpret_cast<uintptr_t>(c) & 3u) != 0) return set_error(RT_EINVAL, "%s: c must be 4-byte aligned", who);
  if (bias && (reinterpret_cast<uintptr_t>(bias) & 3u) != 0)
    return set_error(RT_EINVAL, "%s: bias must be 4-byte aligned", who);
  if (fmt == RT_LINEAR_Q4K) {
    rt_status st = q4k_gemm_entry(who, a, false, w, c, m, n, k, stream);
    if (st != RT_OK || !bias) return st;
    return hip_error(launch_add_bias_rows(c, bias, (int)m, (int)n, s), who);
  }
  // f32 / bf16 weights with a few rows, or a K the 64-wide GEMM stages do not
  // divide: the weights stream once per 8 rows, the bias add fused
  if (fmt == RT_LINEAR_F32 && (few || k % 64 != 0))
    return hip_error(launch_f32_gemv_rows(static_cast<const float *>(w), a, bias, c, (int)m, (int)n, (int)k, s), who);
  if (fmt == RT_LINEAR_BF16 && (few || k % 64 != 0))
    return hip_error(launch_bf16_gemv_rows(static_cast<const uint16_t *>(w), a, bias, c, (int)m, (int)n, (int)k, s),
                     who);
  void *ws = nullptr;
  rt_status st = gemm_workspace(proj_gemm_workspace_bytes((int)m, (int)n, (int)k), s, &ws);
  if (st != RT_OK) return st;
  hipError_t e = launch_proj_gemm(a, fmt, w, c, (int)m, (int)n, (int)k, ws, s);
  if (e == hipSuccess && bias) e = launch_add_bias_rows(c, bias, (int)m, (int)n, s);
  return hip_error(e, who);
}

rt_status rt_linear_gemm_f32(int32_t fmt, const void *w, const float *a, float *c, int64_t m, int64_t n, int64_t k,
                             void *stream) {
  return linear_forward("rt_linear_gemm_f32", fmt, w, nullptr, a, c, m, n, k, stream);
}

rt_status rt_qlinear_forward(int32_t fmt, const void *w, const float *bias, const float *x, float *out, int64_t m,
                             int64_t n, int64_t k, void *stream) {
  return linear_forward("rt_qlinear_forward", fmt, w, bias, x, out, m, n, k, stream);
}

// gemv_q4k_t_batch (metal_decode.rs:459-521): c[m][n] = a[m][k] . W[n][k]
// for m <= 8 rows, one pass over the weights.
rt_status rt_q4k_gemv_batch(const void *w, const float *a, float *c, int64_t m, int64_t n, int64_t k, void *stream) {
  rt_status st = check_gemv_shape("rt_q4k_gemv_batch", w, a, c, n, k, 256);
  if (st != RT_OK) return st;
  if (m < 1 || m > kMbMaxRows) return set_error(RT_EINVAL, "rt_q4k_gemv_batch: m=%lld outside [1, 8]", (long long)m);
  const size_t stage = (mb_stage_bytes((int)k) + 255) & ~size_t(255);
  void *ws = nullptr;
  st = gemm_workspace(stage + mb_part_bytes((int)n, (int)k), (hipStream_t)stream, &ws);
  if (st != RT_OK) return st;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = launch_mb_stage(a, (int)m, (int)k, ws, s);
  if (e == hipSuccess) {
    MbMat mat{static_cast<const uint8_t *>(w), c, (int)n, 0, 0};
    e = launch_q4k_gemv_mb(&mat, 1, (int)m, (int)k, ws, reinterpret_cast<float *>(static_cast<char *>(ws) + stage), s);
  }
  return hip_error(e, "rt_q4k_gemv_batch");
}

rt_status rt_linear_gemv_batch(int32_t fmt, const void *w, const float *a, float *c, int64_t m, int64_t n, int64_t k,
                               void *stream) {
  static const char *who = "rt_linear_gemv_batch";
  if (fmt == RT_LINEAR_Q4K) return rt_q4k_gemv_batch(w, a, c, m, n, k, stream);
  if (fmt != RT_LINEAR_Q6K && fmt != RT_LINEAR_Q8_0 && fmt != RT_LINEAR_BF16)
    return set_error(RT_EINVAL, "%s: format %d has no batched GEMV", who, fmt);
  rt_status st = check_gemv_shape(who, w, a, c, n, k, fmt == RT_LINEAR_Q6K ? 256 : 64);
  if (st != RT_OK) return st;
  if (m < 1 || m > kMbMaxRows) return set_error(RT_EINVAL, "%s: m=%lld outside [1, 8]", who, (long long)m);
  const size_t stage = fmt == RT_LINEAR_BF16 ? 0 : (mb_stage_bytes((int)k) + 255) & ~size_t(255);
  void *ws = nullptr;
  st = gemm_workspace(std::max<size_t>(stage + kquant_mb_part_bytes((int)n, (int)k), 256), (hipStream_t)stream, &ws);
  if (st != RT_OK) return st;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = stage ? launch_mb_stage(a, (int)m, (int)k, ws, s) : hipSuccess;
  if (e == hipSuccess) {
    MbMat mat{static_cast<const uint8_t *>(w), c, (int)n, 0, 0};
    e = launch_kquant_gemv_mb(fmt, &mat, 1, (int)m, (int)k, stage ? ws : nullptr, a,
                              reinterpret_cast<float *>(static_cast<char *>(ws) + stage), s);
  }
  return hip_error(e, who);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free batched GEMV.  Its workspace (staged activation digits and
// split-K partial sums) is a fixed device array, `scratch`, one copy per GPU
// the library runs on, held until the process ends.  The host side never
// passes the array's name to a kernel: the first call on a device looks up
// that device's copy with hipGetSymbolAddress and keeps the address.
// Every call on one GPU shares its array; calls that overlap on one GPU
// (different streams, or host threads) race on it.  The stage is fully
// written by the staging kernel and every partial by the GEMV before it is
// read, so nothing has to start at zero.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
constexpr int kNoAllocMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
void *g_scratch_ptr[kNoAllocMaxDevices] = {};

rt_status scratch_address(const char *who, void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_error(e, who);
  if (dev < 0 || dev >= kNoAllocMaxDevices) return set_error(RT_EINVAL, "%s: device %d beyond %d", who, dev, kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
    if (!p) return set_error(RT_EHIP, "%s: hipGetSymbolAddress returned null", who);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return RT_OK;
}
}  // namespace

extern "C" {

size_t rt_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

rt_status rt_q4k_gemv_batch_noalloc(const void *w, const float *a, float *c, int64_t m, int64_t n, int64_t k,
                                    void *stream) {
  static const char *who = "rt_q4k_gemv_batch_noalloc";
  rt_status st = check_gemv_shape(who, w, a, c, n, k, 256);
  if (st != RT_OK) return st;
  if (m < 1 || m > kMbMaxRows) return set_error(RT_EINVAL, "%s: m=%lld outside [1, 8]", who, (long long)m);
  const size_t stage = (mb_stage_bytes((int)k) + 255) & ~size_t(255);
  const size_t need = stage + mb_part_bytes((int)n, (int)k);
  if (need > kNoAllocScratchBytes)
    return set_error(RT_EINVAL, "%s: n=%lld k=%lld needs %zu bytes of workspace, more than the fixed %zu", who,
                     (long long)n, (long long)k, need, kNoAllocScratchBytes);
  void *ws = nullptr;
  st = scratch_address(who, &ws);
  if (st != RT_OK) return st;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = launch_mb_stage(a, (int)m, (int)k, ws, s);
  if (e == hipSuccess) {
    MbMat mat{static_cast<const uint8_t *>(w), c, (int)n, 0, 0};
    e = launch_q4k_gemv_mb(&mat, 1, (int)m, (int)k, ws, reinterpret_cast<float *>(static_cast<char *>(ws) + stage), s);
  }
  return hip_error(e, who);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Host-pointer drop-ins with a weight cache keyed by (host pointer, bytes).
// ---------------------------------------------------------------------------
namespace {

struct CacheKey {
  int device;
  const void *ptr;
  size_t bytes;
  bool operator<(const CacheKey &o) const {
    if (device != o.device) return device < o.device;
    if (ptr != o.ptr) return ptr < o.ptr;
    return bytes < o.bytes;
  }
};

std::mutex g_cache_mu;
std::map<CacheKey, void *> g_weight_cache;

rt_status cached_upload(const void *host, size_t bytes, void **dev_out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_error(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_cache_mu);
  CacheKey key{dev, host, bytes};
  auto it = g_weight_cache.find(key);
  if (it != g_weight_cache.end()) {
    *dev_out = it->second;
    return RT_OK;
  }
  void *d = nullptr;
  e = hipMalloc(&d, bytes);
  if (e != hipSuccess) return hip_error(e, "weight upload hipMalloc");
  e = hipMemcpy(d, host, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    return hip_error(e, "weight upload hipMemcpy");
  }
  g_weight_cache[key] = d;
  *dev_out = d;
  return RT_OK;
}

// Per-call activation/output staging (the reference's scratch_act / output buffers).
struct Staging {
  void *buf = nullptr;
  size_t cap = 0;
};
thread_local Staging g_stage;

rt_status stage(size_t bytes, void **out) {
  if (g_stage.cap < bytes) {
    if (g_stage.buf) (void)hipFree(g_stage.buf);
    g_stage.buf = nullptr;
    g_stage.cap = 0;
    hipError_t e = hipMalloc(&g_stage.buf, bytes);
    if (e != hipSuccess) return hip_error(e, "staging hipMalloc");
    g_stage.cap = bytes;
  }
  *out = g_stage.buf;
  return RT_OK;
}

// GEMM / batched-GEMV workspace (A in f16 plus row exponents, staged digits,
// split-K partials), one per (host thread, device, stream), so calls queued
// on different streams never share one.  It grows on demand, by at least
// doubling, but never while its stream is being captured into a graph (such a
// call returns RT_ESTATE: run it once uncaptured first).  A buffer it
// outgrows is kept, not freed: a graph captured earlier may still read it.
struct GemmWorkspace {
  void *buf = nullptr;
  size_t cap = 0;
  std::vector<void *> retired;
  size_t retired_bytes = 0;
};
thread_local std::map<std::pair<int, hipStream_t>, GemmWorkspace> g_gemm_ws;

rt_status gemm_workspace(size_t bytes, hipStream_t stream, void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_error(e, "hipGetDevice");
  GemmWorkspace &w = g_gemm_ws[{dev, stream}];
  if (w.cap < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return hip_error(e, "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone)
      return set_error(RT_ESTATE,
                       "workspace must grow to %zu bytes while its stream is being captured; make the same call once "
                       "outside capture first",
                       bytes);
    const size_t grow = std::max(bytes, 2 * w.cap);
    void *nb = nullptr;
    e = hipMalloc(&nb, grow);
    if (e != hipSuccess) return hip_error(e, "gemm workspace hipMalloc");
    if (w.buf) w.retired.push_back(w.buf), w.retired_bytes += w.cap;
    w.buf = nb;
    w.cap = grow;
  }
  *out = w.buf;
  return RT_OK;
}

template <typename LaunchFn>
rt_status host_gemv(const char *who, const float *a, size_t k, const void *w_host, size_t w_bytes, size_t rows,
                    float *out, LaunchFn launch) {
  void *wdev = nullptr, *buf = nullptr;
  rt_status st = cached_upload(w_host, w_bytes, &wdev);
  if (st != RT_OK) return st;
  const size_t xbytes = (k * sizeof(float) + 255) & ~size_t(255);
  st = stage(xbytes + rows * sizeof(float), &buf);
  if (st != RT_OK) return st;
  float *xd = static_cast<float *>(buf);
  float *yd = reinterpret_cast<float *>(static_cast<char *>(buf) + xbytes);
  hipError_t e = hipMemcpy(xd, a, k * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_error(e, who);
  e = launch(wdev, xd, yd);
  if (e != hipSuccess) return hip_error(e, who);
  e = hipMemcpy(out, yd, rows * sizeof(float), hipMemcpyDeviceToHost);
  return hip_error(e, who);
}

}  // namespace

extern "C" {

rt_status rt_gemv_q4k_t(const float *a, size_t k, const uint8_t *blocks, size_t rows, float *out) {
  if (!a || !blocks || !out) return set_error(RT_EINVAL, "rt_gemv_q4k_t: null pointer");
  if (k == 0 || rows == 0 || k % 256 != 0 || k > INT32_MAX || rows > INT32_MAX)
    return set_error(RT_EINVAL, "rt_gemv_q4k_t: k=%zu rows=%zu (k must be a positive multiple of 256)", k, rows);
  const size_t bytes = rows * (k / 256) * 144;
  return host_gemv("rt_gemv_q4k_t", a, k, blocks, bytes, rows, out, [&](void *w, float *x, float *y) {
    return launch_q4k_gemv(w, x, y, (int)rows, (int)k, nullptr);
  });
}

rt_status rt_gemv_bf16_t(const float *a, size_t k, const uint16_t *w, size_t rows, float *out) {
  if (!a || !w || !out) return set_error(RT_EINVAL, "rt_gemv_bf16_t: null pointer");
  if (k == 0 || rows == 0 || k % 8 != 0 || k > INT32_MAX || rows > INT32_MAX)
    return set_error(RT_EINVAL, "rt_gemv_bf16_t: k=%zu rows=%zu (k must be a positive multiple of 8)", k, rows);
  const size_t bytes = rows * k * 2;
  return host_gemv("rt_gemv_bf16_t", a, k, w, bytes, rows, out, [&](void *wd, float *x, float *y) {
    return launch_bf16_gemv(static_cast<const uint16_t *>(wd), x, y, (int)rows, (int)k, nullptr);
  });
}

rt_status rt_matmul_q4k_t(const float *a, size_t m, size_t k, const uint8_t *blocks, size_t rows, float *out) {
  if (!a || !blocks || !out) return set_error(RT_EINVAL, "rt_matmul_q4k_t: null pointer");
  if (m == 0 || k == 0 || rows == 0 || k % 256 != 0 || k > INT32_MAX || rows > INT32_MAX || m > INT32_MAX)
    return set_error(RT_EINVAL, "rt_matmul_q4k_t: m=%zu k=%zu rows=%zu (k must be a positive multiple of 256)", m, k,
                     rows);
  if (m == 1) return rt_gemv_q4k_t(a, k, blocks, rows, out);
  void *wdev = nullptr, *buf = nullptr, *ws = nullptr;
  const size_t wbytes = rows * (k / 256) * 144;
  rt_status st = cached_upload(blocks, wbytes, &wdev);
  if (st != RT_OK) return st;
  const size_t abytes = (m * k * sizeof(float) + 255) & ~size_t(255);
  st = stage(abytes + m * rows * sizeof(float), &buf);
  if (st != RT_OK) return st;
  st = gemm_workspace(q4k_gemm_workspace_bytes((int)m, (int)rows, (int)k), nullptr, &ws);
  if (st != RT_OK) return st;
  float *ad = static_cast<float *>(buf);
  float *cd = reinterpret_cast<float *>(static_cast<char *>(buf) + abytes);
  hipError_t e = hipMemcpy(ad, a, m * k * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_error(e, "rt_matmul_q4k_t");
  e = launch_q4k_gemm(ad, false, wdev, cd, (int)m, (int)rows, (int)k, ws, nullptr);
  if (e != hipSuccess) return hip_error(e, "rt_matmul_q4k_t");
  e = hipMemcpy(out, cd, m * rows * sizeof(float), hipMemcpyDeviceToHost);
  return hip_error(e, "rt_matmul_q4k_t");
}

// Host drop-in for QLinear::forward (qlinear.rs:82-111) on the formats a
// QLinear holds (Q4_K, BF16, F32): the weight is uploaded once and cached by
// (host pointer, bytes) like rt_gemv_q4k_t's; x, the bias and the output are
// staged per call; synchronous.
rt_status rt_qlinear_forward_host(int32_t fmt, const void *w, size_t w_bytes, const float *bias, const float *x,
                                  float *out, int64_t m, int64_t n, int64_t k) {
  static const char *who = "rt_qlinear_forward_host";
  if (!w || !x || !out) return set_error(RT_EINVAL, "%s: null pointer", who);
  if (fmt != RT_LINEAR_Q4K && fmt != RT_LINEAR_BF16 && fmt != RT_LINEAR_F32)
    return set_error(RT_EINVAL, "%s: format %d (a QLinear holds Q4_K, BF16 or F32)", who, fmt);
  if (m <= 0 || n <= 0 || k <= 0 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
    return set_error(RT_EINVAL, "%s: m=%lld n=%lld k=%lld", who, (long long)m, (long long)n, (long long)k);
  size_t need = 0;
  switch (fmt) {
    case RT_LINEAR_Q4K: need = k % 256 ? 0 : (size_t)n * (size_t)(k / 256) * 144; break;
    case RT_LINEAR_BF16: need = (size_t)n * (size_t)k * 2; break;
    case RT_LINEAR_F32: need = (size_t)n * (size_t)k * 4; break;
    default: return set_error(RT_EINVAL, "%s: format %d (a QLinear holds Q4_K, BF16 or F32)", who, fmt);
  }
  if (need == 0 || w_bytes != need)
    return set_error(RT_EINVAL, "%s: weight of %zu bytes, format %d [%lld, %lld] needs %zu", who, w_bytes, fmt,
                     (long long)n, (long long)k, need);
  void *wdev = nullptr, *buf = nullptr;
  rt_status st = cached_upload(w, w_bytes, &wdev);
  if (st != RT_OK) return st;
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  const size_t xb = r256((size_t)m * k * 4), ob = r256((size_t)m * n * 4), bb = bias ? r256((size_t)n * 4) : 0;
  st = stage(xb + ob + bb, &buf);
  if (st != RT_OK) return st;
  float *xd = static_cast<float *>(buf);
  float *od = reinterpret_cast<float *>(static_cast<char *>(buf) + xb);
  float *bd = bias ? reinterpret_cast<float *>(static_cast<char *>(buf) + xb + ob) : nullptr;
  hipError_t e = hipMemcpy(xd, x, (size_t)m * k * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess && bias) e = hipMemcpy(bd, bias, (size_t)n * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_error(e, who);
  st = rt_qlinear_forward(fmt, wdev, bd, xd, od, m, n, k, nullptr);
  if (st != RT_OK) return st;
  return hip_error(hipMemcpy(out, od, (size_t)m * n * 4, hipMemcpyDeviceToHost), who);
}

rt_status rt_gemm_workspace_release(void *stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_error(e, "hipGetDevice");
  auto it = g_gemm_ws.find({dev, (hipStream_t)stream});
  if (it == g_gemm_ws.end()) return RT_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing((hipStream_t)stream, &cs);
  if (e != hipSuccess) return hip_error(e, "hipStreamIsCapturing");
  if (cs != hipStreamCaptureStatusNone)
    return set_error(RT_ESTATE, "rt_gemm_workspace_release: the stream is being captured");
  // queued calls on the stream may still read the buffers
  e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return hip_error(e, "rt_gemm_workspace_release: hipStreamSynchronize");
  for (void *q : it->second.retired) e = hipFree(q) == hipSuccess ? e : hipErrorInvalidValue;
  if (it->second.buf && hipFree(it->second.buf) != hipSuccess) e = hipErrorInvalidValue;
  g_gemm_ws.erase(it);
  return hip_error(e, "rt_gemm_workspace_release: hipFree");
}

size_t rt_gemm_workspace_held(void *stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  auto it = g_gemm_ws.find({dev, (hipStream_t)stream});
  return it == g_gemm_ws.end() ? 0 : it->second.cap + it->second.retired_bytes;
}

rt_status rt_weight_cache_clear(void) {
  std::lock_guard<std::mutex> lk(g_cache_mu);
  for (auto &kv : g_weight_cache) (void)hipFree(kv.second);
  g_weight_cache.clear();
  return RT_OK;
}

}  // extern "C"
