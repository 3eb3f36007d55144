// Measurement probes: the plain HBM stream that bounds the decode GEMVs and
// the sustained MFMA rate that bounds the prefill GEMM, both on the device
// and with the operand data the kernels see.
//
// k_stream_read reads a buffer once with 16-byte loads (non-temporal, the
// decode kernels' policy, or the default policy) and writes nothing but one
// word in the practically impossible case that the XOR of everything it read
// equals a fixed constant, which keeps the loads live. One-shot form: each
// lane issues its U loads back to back (stride 256 chunks, so every wave load
// instruction reads 1 KB of contiguous bytes) and then retires, like a
// one-shot decode GEMV. Persistent form: a fixed grid walks the buffer in
// strides of the whole grid, U loads per lane per step. Timing it on the
// decode workload's byte count gives the achievable read rate that a decode
// kernel's time is compared with.
//
// k_mfma_peak issues back-to-back v_mfma_f32_32x32x16_f16 on operands loaded
// from a caller buffer (random binary16 values: the switching activity of a
// real GEMM, which sets the clock the chip sustains under load). Each lane
// holds four A and four B fragments and every MFMA of an unrolled group of 16
// takes another (A, B) pair, spread over 4 or 8 independent accumulators.
// Every wave records the shader-clock counter (s_memtime) around its loop and
// the constant-rate counter (s_memrealtime) at the loop's start and end, so
// the host can tell how many waves ran at once and what clock they ran at.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/xrmm.h"
#include "xrmm_internal.h"

namespace xrmm {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f16acc_t __attribute__((ext_vector_type(16)));

template <bool NT>
__device__ __forceinline__ u32x4_t ld16(const u32x4_t* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

template <int U, bool NT>
__global__ __launch_bounds__(256) void k_stream_read(const u32x4_t* __restrict__ src, uint64_t n16, uint32_t* sink) {
  const uint64_t base = static_cast<uint64_t>(blockIdx.x) * 256u * U + threadIdx.x;
  u32x4_t v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint64_t i = base + 256u * u;
    v[u] = i < n16 ? ld16<NT>(src + i) : u32x4_t{0u, 0u, 0u, 0u};
  }
  u32x4_t acc = v[0];
#pragma unroll
  for (int u = 1; u < U; ++u) acc ^= v[u];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[0] = 1u;
}

template <int U, bool NT>
__global__ __launch_bounds__(256) void k_stream_read_persistent(const u32x4_t* __restrict__ src, uint64_t n16,
                                                                uint32_t* sink) {
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * 256u * U;
  u32x4_t acc = {0u, 0u, 0u, 0u};
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * 256u * U + threadIdx.x; base < n16; base += step) {
    u32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t i = base + 256u * u;
      v[u] = i < n16 ? ld16<NT>(src + i) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[0] = 1u;
}

template <int U, bool NT>
hipError_t launch_read(const void* src, uint64_t n16, uint32_t* sink, int32_t workgroups, hipStream_t st) {
  const uint64_t per = 256u * U;
  const auto* s = static_cast<const u32x4_t*>(src);
  if (workgroups > 0) {
    hipLaunchKernelGGL((k_stream_read_persistent<U, NT>), dim3(static_cast<uint32_t>(workgroups)), dim3(256), 0, st, s,
                       n16, sink);
  } else {
    const uint64_t grid = (n16 + per - 1) / per;
    if (grid > 0x7FFFFFFFu) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_stream_read<U, NT>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, st, s, n16, sink);
  }
  return hipGetLastError();
}

template <bool NT>
hipError_t read_dispatch(const void* src, uint64_t n16, uint32_t* sink, int32_t u, int32_t wg, hipStream_t st) {
  switch (u) {
    case 1: return launch_read<1, NT>(src, n16, sink, wg, st);
    case 2: return launch_read<2, NT>(src, n16, sink, wg, st);
    case 4: return launch_read<4, NT>(src, n16, sink, wg, st);
    default: return launch_read<8, NT>(src, n16, sink, wg, st);
  }
}

// Fragments per lane of each operand, and MFMAs per unrolled group.
constexpr int kFrag = 4;
constexpr int kGroup = 16;

// NACC independent accumulators; lane 0 of every wave writes four words:
// shader-clock cycles of its loop, constant-rate ticks at the loop's start
// and end, and the workgroup index.
// Register budgets: up to 4 (NACC 4) or 3 (NACC 8) waves per SIMD must fit, so
// that 16 waves per CU can run at once with 4 accumulators.
template <int NACC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NACC == 4 ? 4 : 3, 8))) void k_mfma_peak(const h8_t* __restrict__ ops, uint32_t iters, float* sink,
                                                    uint64_t* clocks) {
  const int tid = threadIdx.x, lane = tid & 63;
  h8_t a[kFrag], b[kFrag];
#pragma unroll
  for (int j = 0; j < kFrag; ++j) {
    // 2 * kFrag fragments of 64 lanes: 8 KB of operands, the same for every wave
    a[j] = ops[j * 64 + lane];
    b[j] = ops[(kFrag + j) * 64 + lane];
  }
  f16acc_t acc[NACC];
#pragma unroll
  for (int j = 0; j < NACC; ++j) acc[j] = f16acc_t{};
  // the operands are in registers before the clocks start
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_sched_barrier(0);
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_sched_barrier(0);
  uint32_t it = 0;  // iters >= 1 (checked on the host): no branch ahead of the loop
  do {
#pragma unroll
    for (int g = 0; g < kGroup; ++g)
      acc[g % NACC] =
          __builtin_amdgcn_mfma_f32_32x32x16_f16(a[g % kFrag], b[(g / kFrag) % kFrag], acc[g % NACC], 0, 0, 0);
  } while (++it < iters);
  __builtin_amdgcn_sched_barrier(0);
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NACC; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  if (s == 1.2345678e30f) sink[0] = s;
  if (lane == 0) {
    const uint64_t w = static_cast<uint64_t>(blockIdx.x) * (blockDim.x >> 6) + (tid >> 6);
    clocks[4 * w] = t1 - t0;
    clocks[4 * w + 1] = r0;
    clocks[4 * w + 2] = r1;
    clocks[4 * w + 3] = blockIdx.x;
  }
}

}  // namespace
}  // namespace xrmm

extern "C" int xrmm_stream_read_ex(const void* src, uint64_t bytes, void* sink, int32_t loads_per_lane,
                                   int32_t nontemporal, int32_t workgroups, void* stream) {
  if (!src || !sink) return xrmm::set_status(XRMM_EINVAL, "null pointer");
  if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0 || (bytes & 15u) != 0)
    return xrmm::set_status(XRMM_EINVAL, "stream read: source and byte count must be multiples of 16");
  if (loads_per_lane != 1 && loads_per_lane != 2 && loads_per_lane != 4 && loads_per_lane != 8)
    return xrmm::set_status(XRMM_EINVAL, "stream read: loads_per_lane must be 1, 2, 4 or 8");
  if (workgroups < 0 || workgroups > (1 << 20))
    return xrmm::set_status(XRMM_EINVAL, "stream read: workgroups must be 0 (one-shot grid) or 1..1048576");
  const uint64_t n16 = bytes / 16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* s = static_cast<uint32_t*>(sink);
  const hipError_t e = nontemporal ? xrmm::read_dispatch<true>(src, n16, s, loads_per_lane, workgroups, st)
                                   : xrmm::read_dispatch<false>(src, n16, s, loads_per_lane, workgroups, st);
  if (e != hipSuccess) return xrmm::set_status(XRMM_EDEVICE, std::string("stream read launch: ") + hipGetErrorString(e));
  return xrmm::set_status(XRMM_OK, "");
}

extern "C" int xrmm_stream_read(const void* src, uint64_t bytes, void* sink, int32_t loads_per_lane, void* stream) {
  return xrmm_stream_read_ex(src, bytes, sink, loads_per_lane, 1, 0, stream);
}

extern "C" int64_t xrmm_mfma_peak_operand_bytes(void) {
  return static_cast<int64_t>(2 * xrmm::kFrag * 64 * sizeof(xrmm::h8_t));
}

extern "C" int64_t xrmm_mfma_peak_flops(int32_t workgroups, int32_t waves, int32_t iters) {
  // kGroup MFMAs of 32 x 32 x 16 (2 * 16384 flops) per wave and iteration
  return static_cast<int64_t>(workgroups) * waves * iters * xrmm::kGroup * 2 * 32 * 32 * 16;
}

extern "C" int xrmm_mfma_peak(const void* operands, void* sink, void* clocks, int32_t workgroups, int32_t waves,
                              int32_t accumulators, int32_t iters, void* stream) {
  if (!operands || !sink || !clocks) return xrmm::set_status(XRMM_EINVAL, "null pointer");
  if ((reinterpret_cast<uintptr_t>(operands) & 15u) != 0 || (reinterpret_cast<uintptr_t>(clocks) & 7u) != 0)
    return xrmm::set_status(XRMM_EINVAL, "mfma peak: operands must be 16-byte and clocks 8-byte aligned");
  if (workgroups <= 0 || workgroups > (1 << 16) || iters <= 0 || iters > (1 << 24) || waves < 1 || waves > 4)
    return xrmm::set_status(XRMM_EINVAL, "mfma peak: workgroups must be 1..65536, waves 1..4, iters 1..16777216");
  if (accumulators != 4 && accumulators != 8)
    return xrmm::set_status(XRMM_EINVAL, "mfma peak: accumulators must be 4 or 8");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const auto* o = static_cast<const xrmm::h8_t*>(operands);
  float* sk = static_cast<float*>(sink);
  uint64_t* ck = static_cast<uint64_t*>(clocks);
  const dim3 grid(static_cast<uint32_t>(workgroups)), block(static_cast<uint32_t>(64 * waves));
  if (accumulators == 4)
    hipLaunchKernelGGL(xrmm::k_mfma_peak<4>, grid, block, 0, st, o, static_cast<uint32_t>(iters), sk, ck);
  else
    hipLaunchKernelGGL(xrmm::k_mfma_peak<8>, grid, block, 0, st, o, static_cast<uint32_t>(iters), sk, ck);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return xrmm::set_status(XRMM_EDEVICE, std::string("mfma peak launch: ") + hipGetErrorString(e));
  return xrmm::set_status(XRMM_OK, "");
}
