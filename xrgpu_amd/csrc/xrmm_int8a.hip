// Opt-in int8-activation MatMulNBits (the upstream operator's accuracy_level
// 4; xrGPU's own shader stays float32 at every level,
// kernels/_shared/extended/shaders/complex_kernel.glsl:83).
//
// 1. k_i8a_quant: one wave per (row, block of 128 activations): scale =
//    max|a| / 127, codes rint(a / scale) (float32, round half to even), the
//    codes of each group of 8 stored as k0 k2 k4 k6 k1 k3 k5 k7 so that they
//    line up with the low and high nibbles of a weight dword.
// 2. k_i8a_gemv: one wave per output column; its lanes split K into chunks of
//    32 codes, convert the column's codes once to signed bytes (code - zero:
//    (c | 0x80) - z, then ^ 0x80, per byte without borrows), and for each row
//    form exact int32 chunk sums with v_dot4_i32_i8, scaled by the weight
//    block's and the activation block's scales in float32.
#include <atomic>
#include <mutex>

#include "xrmm_device.h"
#include "xrmm_quant.h"

namespace xrmm {

namespace {

constexpr int I8T = 256;

template <typename T>
__global__ __launch_bounds__(I8T) void k_i8a_quant(Int8aArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t blk = static_cast<int64_t>(blockIdx.x) * (I8T / 64) + (threadIdx.x >> 6);
  const int64_t nb = a.K / kI8aBlock;
  if (blk >= a.M * nb) return;  // whole waves
  const int64_t m = blk / nb, b = blk % nb;
  const T* src = static_cast<const T*>(a.A) + m * a.K + b * kI8aBlock;
  const float x0 = static_cast<float>(src[2 * lane]), x1 = static_cast<float>(src[2 * lane + 1]);
  float mx = fmaxf(fabsf(x0), fabsf(x1));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  const float scale = __fdiv_rn(mx, 127.f);
  auto code = [&](float x) -> int8_t {
    if (scale == 0.f) return 0;
    const float q = rintf(__fdiv_rn(x, scale));
    return static_cast<int8_t>(fminf(fmaxf(q, -127.f), 127.f));
  };
  // element 2 lane + e sits at position p = 2 (lane % 4) + e of its group of 8
  int8_t* dst = a.qa + m * a.K + b * kI8aBlock + (lane >> 2) * 8;
  const int p = 2 * (lane & 3);
  dst[p >> 1] = code(x0);            // even position -> slots 0..3
  dst[4 + (p >> 1)] = code(x1);      // odd position  -> slots 4..7
  if (lane == 0) a.as[m * nb + b] = scale;
}

template <typename T, int CPL>
__global__ __launch_bounds__(I8T) void k_i8a_gemv(Int8aArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(xcd_slot(blockIdx.x, gridDim.x)) * (I8T / 64) + (threadIdx.x >> 6);
  if (n >= a.N) return;  // whole waves
  const uint32_t chunks = static_cast<uint32_t>(a.K / 32);
  const int64_t kb = a.K >> a.lbs;
  const T* S = static_cast<const T*>(a.S);
  // the column's codes as signed bytes, and each chunk's weight scale
  uint32_t lo[CPL][4], hi[CPL][4];
  float ws[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint32_t c = static_cast<uint32_t>(lane + 64 * j);
    const bool in = c < chunks;
    const uint32_t cc = in ? c : 0;
    const u32x4 w = ld16(a.B + n * (a.K / 2) + cc * 16);
    const int64_t blk = (static_cast<int64_t>(cc) * 32) >> a.lbs;
    uint32_t z = 8;
    if (a.Z) z = (a.Z[n * a.zrow + blk / 2] >> (4 * (blk & 1))) & 15u;
    const uint32_t zz = z * 0x01010101u;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      lo[j][d] = (((w[d] & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
      hi[j][d] = ((((w[d] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
    }
    ws[j] = in ? static_cast<float>(S[n * kb + blk]) : 0.f;
  }
  const float bias = a.bias ? static_cast<float>(static_cast<const T*>(a.bias)[n]) : 0.f;
  const int64_t nb = a.K / kI8aBlock;
  for (int64_t m = 0; m < a.M; ++m) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t c = static_cast<uint32_t>(lane + 64 * j);
      const uint32_t cc = c < chunks ? c : 0;
      const int8_t* q = a.qa + m * a.K + cc * 32;
      const u32x4 q0 = ld16(q), q1 = ld16(q + 16);
      int s = 0;
      s = __builtin_amdgcn_sdot4(static_cast<int>(lo[j][0]), static_cast<int>(q0[0]), s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(hi[j][0]), static_cast<int>(q0[1]), s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(lo[j][1]), static_cast<int>(q0[2]), s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(hi[j][1]), static_cast<int>(q0[3]), s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(lo[j][2]), static_cast<int>(q1[0]), s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(hi[j][2]), static_cast<int>(q1[1]), s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(lo[j][3]), static_cast<int>(q1[2]), s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int>(hi[j][3]), static_cast<int>(q1[3]), s, false);
      const float sa = a.as[m * nb + (cc * 32) / kI8aBlock];
      acc = __builtin_fmaf(static_cast<float>(s), ws[j] * sa, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) static_cast<T*>(a.Y)[m * a.N + n] = static_cast<T>(acc + bias);
  }
}

template <typename T>
hipError_t launch_t(const Int8aArgs& a, hipStream_t st) {
  const int64_t blocks = a.M * (a.K / kI8aBlock);
  hipLaunchKernelGGL(k_i8a_quant<T>, dim3(static_cast<uint32_t>((blocks + 3) / 4)), dim3(I8T), 0, st, a);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  const dim3 grid(static_cast<uint32_t>((a.N + 3) / 4));
  const int64_t cpl = (a.K / 32 + 63) / 64;
  if (cpl <= 1) hipLaunchKernelGGL((k_i8a_gemv<T, 1>), grid, dim3(I8T), 0, st, a);
  else if (cpl <= 2) hipLaunchKernelGGL((k_i8a_gemv<T, 2>), grid, dim3(I8T), 0, st, a);
  else if (cpl <= 4) hipLaunchKernelGGL((k_i8a_gemv<T, 4>), grid, dim3(I8T), 0, st, a);
  else hipLaunchKernelGGL((k_i8a_gemv<T, 8>), grid, dim3(I8T), 0, st, a);
  return hipGetLastError();
}

}  // namespace

// Scratch of the allocation-free entry point: activation codes and scales
// (xrmm_matmul_nbits_int8a_noalloc). Each GPU holds its own copy for the
// lifetime of the process; host code must use the address from i8a_scratch,
// never this name (in host code it is a stand-in, not a device address).
static __device__ __align__(256) uint8_t scratch[kI8aScratchBytes];

namespace {
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;
}  // namespace

hipError_t i8a_scratch(hipStream_t stream, void** ptr) {
  int dev = 0;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      int cur = 0;
      if ((e = hipGetDevice(&cur)) != hipSuccess) return e;
      if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (cur != dev) (void)hipSetDevice(cur);
      if (e != hipSuccess) return e;
      if (p == nullptr) return hipErrorInvalidSymbol;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return hipSuccess;
}

hipError_t launch_i8a(const Int8aArgs& a, hipStream_t st) {
  if (a.M == 0) return hipSuccess;
  if (a.K > kI8aMaxK) return hipErrorInvalidValue;  // the GEMV would drop the chunks past 16384 codes
  return a.f16 ? launch_t<f16>(a, st) : launch_t<float>(a, st);
}

}  // namespace xrmm
