// Measurement kernels: a plain streaming read of a buffer, the reference point the
// decode GEMVs are measured against (the fastest a launch of that many bytes can
// read them), in the configurations the sweep in bench.py tries.
#include <hip/hip_runtime.h>

#include "lb_device.h"
#include "lb_internal.h"

namespace lbk {

// Workgroup w reads the 16-byte units [w * per_wg, (w + 1) * per_wg) of the buffer,
// thread t the units t, t + T, ... of that range, U loads in flight per iteration
// (all issued before the first is used). Units past the buffer read 0 through the
// descriptor. The XOR of everything read is stored only if it equals a constant, so
// no load can be dropped and the kernel writes (almost surely) nothing; `sink` is
// one dword.
template <int T, int U>
__global__ __launch_bounds__(T) void stream_read_kernel(const uint8_t *src, uint32_t bytes, uint32_t per_wg,
                                                        uint32_t *sink) {
  const uint32_t first = blockIdx.x * per_wg;
  if (first * 16ull >= bytes) return;
  const uint32_t units = min(per_wg, (uint32_t)((bytes - first * 16ull) / 16));
  const Rsrc r = make_rsrc(src + (size_t)first * 16, units * 16);
  uint4 acc = make_uint4(0, 0, 0, 0);
  for (uint32_t base = 0; base < units; base += T * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = ld_b128(r, (base + u * T + threadIdx.x) * 16);
#pragma unroll
    for (int u = 0; u < U; u++) {
      acc.x ^= v[u].x;
      acc.y ^= v[u].y;
      acc.z ^= v[u].z;
      acc.w ^= v[u].w;
    }
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[0] = acc.x;
}

template <int T>
static hipError_t launch_read_t(const void *src, uint32_t bytes, int wgs, int loads, uint32_t *sink, hipStream_t s) {
  const uint32_t n16 = bytes / 16;
  const uint32_t per_wg = (n16 + wgs - 1) / wgs;
  const auto *p = static_cast<const uint8_t *>(src);
  switch (loads) {
    case 1: hipLaunchKernelGGL((stream_read_kernel<T, 1>), dim3(wgs), dim3(T), 0, s, p, bytes, per_wg, sink); break;
    case 2: hipLaunchKernelGGL((stream_read_kernel<T, 2>), dim3(wgs), dim3(T), 0, s, p, bytes, per_wg, sink); break;
    case 4: hipLaunchKernelGGL((stream_read_kernel<T, 4>), dim3(wgs), dim3(T), 0, s, p, bytes, per_wg, sink); break;
    case 8: hipLaunchKernelGGL((stream_read_kernel<T, 8>), dim3(wgs), dim3(T), 0, s, p, bytes, per_wg, sink); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_stream_read(const void *src, size_t bytes, int workgroups, int threads, int loads, uint32_t *sink,
                              hipStream_t s) {
  if (bytes == 0 || bytes % 16 || bytes > 0xFFFFFFF0u || workgroups <= 0 || workgroups > 65536)
    return hipErrorInvalidValue;
  if (threads == 256) return launch_read_t<256>(src, (uint32_t)bytes, workgroups, loads, sink, s);
  if (threads == 512) return launch_read_t<512>(src, (uint32_t)bytes, workgroups, loads, sink, s);
  return hipErrorInvalidValue;
}

}  // namespace lbk
