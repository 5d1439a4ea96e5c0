// probe.hip -- the streaming-read floor that bench.py sets each GEMV's
// bandwidth against: the same bytes read with 16-byte loads, no arithmetic,
// nothing written (the checksum is stored only if it equals a constant the
// data cannot produce in practice, which keeps the loads alive).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/rt_hip.h"
#include "rt_capi_util.hpp"

namespace {

__global__ __launch_bounds__(256) void k_stream_read(const uint4 *__restrict__ p, size_t n16, uint32_t *sink) {
  constexpr int U = 8;
  const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, nth = (size_t)gridDim.x * 256;
  uint32_t acc = 0;
  for (size_t i = tid; i < n16; i += nth * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = p[std::min(i + u * nth, n16 - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u && tid == 0) sink[0] = acc;
}

}  // namespace

extern "C" rt_status rt_stream_read(const void *buf, size_t bytes, void *sink, void *stream) {
  if (bytes == 0) return RT_OK;
  if (!buf || !sink) return rt::set_error(RT_EINVAL, "rt_stream_read: null pointer");
  if (bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(buf) & 15u) != 0)
    return rt::set_error(RT_EINVAL, "rt_stream_read: bytes and buf must be multiples of 16");
  const size_t n16 = bytes / 16;
  const unsigned grid = (unsigned)std::max<size_t>(1, std::min<size_t>((n16 + 2047) / 2048, 2048));
  hipLaunchKernelGGL(k_stream_read, dim3(grid), dim3(256), 0, (hipStream_t)stream, static_cast<const uint4 *>(buf),
                     n16, static_cast<uint32_t *>(sink));
  return rt::hip_error(hipGetLastError(), "rt_stream_read");
}
