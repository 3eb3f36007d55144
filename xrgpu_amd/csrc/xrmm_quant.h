// Internal interface of the GatherBlockQuantized and MatMulBnb4 paths
// (xrmm_quant.hip): argument blocks, launches and kernel choice.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xrmm {

constexpr uint32_t kGbqIndexError = 55;  // the shader's failure code for an out-of-range index

struct GbqArgs {
  const uint8_t* data;  // [rows, pcols] packed codes, low-first
  const void* idx;      // [n] int32 (or uint32 read as int32) / int64
  int idx64;
  const float* scales;  // [rows, blocks]
  const uint8_t* zp;    // [rows, zpcols] packed zero points, or null (midpoint)
  float* out;           // [n, width]
  uint32_t* status;     // device word receiving kGbqIndexError (max), or null
  int64_t rows, pcols, n, width, blocks, zpcols;
  int bits, bs;
};

bool gbq_fast_ok(const GbqArgs& a);
hipError_t launch_gbq(const GbqArgs& a, hipStream_t st);

struct Bnb4Args {
  const void* A;       // [M, K] float32 / float16
  const uint8_t* B;    // flat [N * K] codes, two per byte, even index in the high nibble
  const void* absmax;  // [ceil(N * K / bs)] in A's dtype
  void* Y;             // [M, N] in A's dtype
  int64_t M, K, N;
  int bs, qt, tb, f16;
};

bool bnb4_fast_ok(const Bnb4Args& a);
hipError_t launch_bnb4(const Bnb4Args& a, hipStream_t st);

}  // namespace xrmm

namespace xrmm {

// Opt-in int8-activation MatMulNBits (accuracy_level 4 of the upstream
// operator; not the reference's float32 arithmetic).
constexpr int kI8aBlock = 128;  // activations per quantization block
// A wave holds one column's codes in registers: 64 lanes x at most 8 chunks
// of 32 codes.
constexpr int64_t kI8aMaxK = 64 * 8 * 32;

struct Int8aArgs {
  const void* A;        // [M, K] float32 / float16
  const uint8_t* B;     // [N, K / bs, bs / 2] 4-bit codes, low-first
  const void* S;        // [N, K / bs] scales in A's dtype
  const uint8_t* Z;     // [N, zrow] packed 4-bit zero points, or null (8)
  const void* bias;     // [N] or null
  void* Y;              // [M, N] in A's dtype
  int8_t* qa;           // workspace: [M, K] codes, each 8-group as k0 k2 k4 k6 k1 k3 k5 k7
  float* as;            // workspace: [M, K / 128] scales
  int64_t M, K, N, zrow;
  int bs, lbs, f16;
};

inline int64_t i8a_workspace_bytes(int64_t M, int64_t K) {
  return (M * K + 255) / 256 * 256 + M * (K / kI8aBlock) * 4;
}

hipError_t launch_i8a(const Int8aArgs& a, hipStream_t st);

// Bytes of the static device scratch behind xrmm_matmul_nbits_int8a_noalloc.
constexpr int64_t kI8aScratchBytes = int64_t(2) << 20;

// Device address of that scratch on the device `stream` runs on, looked up once
// per device (hipGetSymbolAddress with the device current) and cached.
hipError_t i8a_scratch(hipStream_t stream, void** ptr);

}  // namespace xrmm
