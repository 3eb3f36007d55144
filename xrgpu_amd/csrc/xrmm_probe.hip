// Read-bandwidth probe: the plain HBM stream that bounds the decode GEMVs.
//
// k_stream_read reads a buffer once with 16-byte non-temporal loads (the
// decode kernels' access width and cache policy) and writes nothing but one
// word in the practically impossible case that the XOR of everything it read
// equals a fixed constant, which keeps the loads live. Each lane issues its U
// loads back to back (stride 256 chunks, so every wave load instruction reads
// 1 KB of contiguous bytes) and then retires, like a one-shot decode GEMV.
// Timing it on the decode workload's byte count gives the achievable read rate
// that a decode kernel's time is compared with.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/xrmm.h"
#include "xrmm_internal.h"

namespace xrmm {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void k_stream_read(const u32x4_t* __restrict__ src, uint64_t n16, uint32_t* sink) {
  const uint64_t base = static_cast<uint64_t>(blockIdx.x) * 256u * U + threadIdx.x;
  u32x4_t v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint64_t i = base + 256u * u;
    v[u] = i < n16 ? __builtin_nontemporal_load(src + i) : u32x4_t{0u, 0u, 0u, 0u};
  }
  u32x4_t acc = v[0];
#pragma unroll
  for (int u = 1; u < U; ++u) acc ^= v[u];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[0] = 1u;
}

template <int U>
hipError_t launch_read(const void* src, uint64_t n16, uint32_t* sink, hipStream_t st) {
  const uint64_t per = 256u * U;
  const uint64_t grid = (n16 + per - 1) / per;
  if (grid > 0x7FFFFFFFu) return hipErrorInvalidValue;
  hipLaunchKernelGGL((k_stream_read<U>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, st,
                     static_cast<const u32x4_t*>(src), n16, sink);
  return hipGetLastError();
}

}  // namespace
}  // namespace xrmm

extern "C" int xrmm_stream_read(const void* src, uint64_t bytes, void* sink, int32_t loads_per_lane, void* stream) {
  if (!src || !sink) return xrmm::set_status(XRMM_EINVAL, "null pointer");
  if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0 || (bytes & 15u) != 0)
    return xrmm::set_status(XRMM_EINVAL, "stream read: source and byte count must be multiples of 16");
  const uint64_t n16 = bytes / 16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* s = static_cast<uint32_t*>(sink);
  hipError_t e;
  switch (loads_per_lane) {
    case 1: e = xrmm::launch_read<1>(src, n16, s, st); break;
    case 2: e = xrmm::launch_read<2>(src, n16, s, st); break;
    case 4: e = xrmm::launch_read<4>(src, n16, s, st); break;
    case 8: e = xrmm::launch_read<8>(src, n16, s, st); break;
    default: return xrmm::set_status(XRMM_EINVAL, "stream read: loads_per_lane must be 1, 2, 4 or 8");
  }
  if (e != hipSuccess) return xrmm::set_status(XRMM_EDEVICE, std::string("stream read launch: ") + hipGetErrorString(e));
  return xrmm::set_status(XRMM_OK, "");
}
