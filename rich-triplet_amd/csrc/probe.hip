// probe.hip -- measurement kernels behind bench.py's floors: a plain
// streaming read (the same bytes as a GEMV read with 16-byte loads, no
// arithmetic, nothing written: the checksum is stored only if it equals a
// constant the data cannot produce in practice, which keeps the loads alive)
// and an empty kernel (the cost of a launch in a graph with nothing in it).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/rt_hip.h"
#include "rt_capi_util.hpp"
#include "rt_device.hpp"

namespace {

// A 16-byte load, with the nontemporal hint when NT.
template <bool NT>
__device__ __forceinline__ uint4 ld16(const uint4 *p) {
  if constexpr (NT) return rt::ld_nt16(p);
  else return *p;
}

// Strided: thread i reads 16-byte words i, i + nth, i + 2 nth, ... in
// batches of U, and the next batch's loads are issued before the current
// batch is folded, so each thread always has loads in flight.
template <int U, bool NT>
__global__ __launch_bounds__(256) void k_stream_read(const uint4 *__restrict__ p, size_t n16, uint32_t *sink) {
  const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, nth = (size_t)gridDim.x * 256;
  uint32_t acc = 0;
  uint4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = ld16<NT>(p + std::min(tid + u * nth, n16 - 1));
  for (size_t i = tid; i < n16; i += nth * U) {
    uint4 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = ld16<NT>(p + std::min(i + (U + u) * nth, n16 - 1));
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = w[u];
  }
  if (acc == 0x9E3779B9u && tid == 0) sink[0] = acc;
}

// Blocked: workgroup b reads its own contiguous slice, 256 x U words per batch.
template <int U, bool NT>
__global__ __launch_bounds__(256) void k_stream_read_blk(const uint4 *__restrict__ p, size_t n16, uint32_t *sink) {
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t b0 = (size_t)blockIdx.x * per, b1 = std::min(b0 + per, n16);
  uint32_t acc = 0;
  for (size_t i = b0 + threadIdx.x; i < b1; i += 256 * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ld16<NT>(p + std::min(i + u * 256, b1 - 1));
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u && threadIdx.x == 0) sink[0] = acc;
}

__global__ void k_empty() {}

}  // namespace

extern "C" rt_status rt_stream_read_cfg(const void *buf, size_t bytes, void *sink, void *stream, int kind, int grid) {
  if (bytes == 0) return RT_OK;
  if (!buf || !sink) return rt::set_error(RT_EINVAL, "rt_stream_read: null pointer");
  if (bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(buf) & 15u) != 0)
    return rt::set_error(RT_EINVAL, "rt_stream_read: bytes and buf must be multiples of 16");
  if (kind < 0 || kind > 3 || grid < 0 || grid > 65536)
    return rt::set_error(RT_EINVAL, "rt_stream_read_cfg: kind must be 0..3 and grid 0..65536");
  const size_t n16 = bytes / 16;
  // grid 0: one batch per thread for reads up to 32 MB (single-launch
  // GEMV sizes), 512 workgroups looping beyond
  const unsigned g = grid > 0 ? (unsigned)grid
                              : (unsigned)std::max<size_t>(1, std::min<size_t>((n16 + 1023) / 1024, 512));
  hipStream_t s = (hipStream_t)stream;
  const uint4 *p = static_cast<const uint4 *>(buf);
  uint32_t *k = static_cast<uint32_t *>(sink);
  switch (kind) {
    case 0: hipLaunchKernelGGL((k_stream_read<4, false>), dim3(g), dim3(256), 0, s, p, n16, k); break;
    case 1: hipLaunchKernelGGL((k_stream_read_blk<8, false>), dim3(g), dim3(256), 0, s, p, n16, k); break;
    case 2: hipLaunchKernelGGL((k_stream_read<4, true>), dim3(g), dim3(256), 0, s, p, n16, k); break;
    default: hipLaunchKernelGGL((k_stream_read_blk<8, true>), dim3(g), dim3(256), 0, s, p, n16, k); break;
  }
  return rt::hip_error(hipGetLastError(), "rt_stream_read");
}

extern "C" rt_status rt_stream_read(const void *buf, size_t bytes, void *sink, void *stream) {
  return rt_stream_read_cfg(buf, bytes, sink, stream, 0, 0);
}

extern "C" rt_status rt_empty_launch(int grid, int threads, void *stream) {
  if (grid < 1 || grid > 65536 || threads < 1 || threads > 1024)
    return rt::set_error(RT_EINVAL, "rt_empty_launch: grid 1..65536, threads 1..1024");
  hipLaunchKernelGGL(k_empty, dim3(grid), dim3(threads), 0, (hipStream_t)stream);
  return rt::hip_error(hipGetLastError(), "rt_empty_launch");
}
