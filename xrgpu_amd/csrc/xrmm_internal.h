// Internal interfaces shared by the kernel file and the host ABI of libxrmm.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <string>

namespace xrmm {

enum Op { OP_MATMUL = 0, OP_QKV = 1, OP_MLP = 2 };
enum ZpKind { ZP_NONE = 0, ZP_FLOAT = 1, ZP_PACKED = 2 };
enum DT { DT_F32 = 0, DT_F16 = 1 };

// One packed projection: weights, scales, optional zero points and bias, and
// where its output goes.
struct Proj {
  const uint8_t* B;    // [N, kb, blob]
  const void* scales;  // [N, kb] of dtype
  const void* zp;      // nullptr | float [N, kb] | packed u8 [N, zrow]
  const void* bias;    // nullptr | [N] of dtype
  void* Y;             // [M, N] of dtype (unused for the Mlp up projection)
  int64_t N;
};

// Everything a launch needs; passed to kernels by value.
struct Launch {
  int op;
  int dtype;     // T1: DT_F32 / DT_F16
  int zp_kind;   // ZpKind
  int zp_dtype;  // DT_F32 / DT_F16 for ZP_FLOAT
  int bits;
  int block_size;
  int act;       // Mlp activation kind
  int nproj;     // 1 (MatMul), 3 (Qkv), 2 (Mlp: gate, up)
  int bs_log2;   // log2(block_size) when it is a power of two, else -1
  int64_t M, K, kb, blob, zrow;
  const void* A;
  const void* skip;      // nullable
  const void* gamma;     // nullable
  void* residual;        // nullable
  float eps;
  Proj p[3];
  // Only kernels that never round a dequantised weight to binary16 (the dot
  // GEMV applies scales to float32 block sums, the four-row MFMA GEMV to
  // float32 chunk sums of exact integer weights, the generic kernel uses the
  // reference formula): set when a binary16 weight (code - z) * scale could
  // leave the binary16 range.
  bool exact_weights;
  // MatMulNBits split-K (k_gemm_q4 with more than one split): float32 partial
  // tiles and per-tile arrival counters (zero-filled before first use; the
  // kernel leaves them zero-filled). nullptr / 1: no split.
  void* ws;
  int32_t splits;
  // Qkv / Mlp prefill: binary16 [M, K] for the normalised activations
  // x = RMSNorm(A + skip) * gamma (or A + skip), written by the prologue
  // kernel before the GEMM reads it. nullptr: the GEMM normalises in place.
  void* xs;
};

// While alive on the calling thread, launches described on that thread set
// Launch::exact_weights (the request lifecycle turns it on at run time for
// weights whose scales it has checked on the host).
class ExactWeightsScope {
 public:
  explicit ExactWeightsScope(bool on);
  ~ExactWeightsScope();
  ExactWeightsScope(const ExactWeightsScope&) = delete;
  ExactWeightsScope& operator=(const ExactWeightsScope&) = delete;
  static bool active();

 private:
  bool prev_;
};

// Kernel families the dispatcher chooses between.
enum Kernel { K_GENERIC = 0, K_GEMV_Q4 = 1, K_GEMM_Q4 = 2, K_GEMV_DOT = 3, K_GEMM_BIG = 4, K_GEMV_SK = 5, K_GEMV_MQ = 6,
              K_GEMV_F32 = 7, K_GEMM_FUSED = 8, K_GEMM_BIG_FUSED = 9, K_GEMM_THIN = 10, K_GEMM_F32X = 11,
              K_F32_SPLIT = 12 };

// Whether a Qkv / Mlp launch has a prologue (skip or normScale) whose
// normalised activations a prefill GEMM can take from L.xs.
inline bool fused_prologue(const Launch& L) { return L.op != OP_MATMUL && (L.skip != nullptr || L.gamma != nullptr); }
// Bytes of L.xs for the geometry (binary16 [M, K], 256-byte multiple).
inline int64_t fused_xs_bytes(const Launch& L) { return (L.M * L.K * 2 + 255) / 256 * 256; }

// MatMulNBits with float32 arithmetic on the matrix cores
// (xrmm_gemm_f32x.hip): whether a geometry fits, its K splits, the workspace
// it needs (prepared float32 rows and split partials; the launch takes it
// from Launch::ws), and the launch.
bool f32x_fits(const Launch& L, int64_t min_rows = 17);
int f32x_splits(const Launch& L);
int64_t f32x_workspace_bytes(const Launch& L);
// act_out: Mlp's two projections (one N, no float zero points, split K)
// finished as act(gate) * up [M][N] float32 by the combine
hipError_t launch_gemm_f32x(const Launch& L, hipStream_t st, float* act_out = nullptr, int act = 0);

// Float32 Qkv / Mlp as a prologue and one float32 MatMulNBits per projection
// (xrmm_f32_split.hip): whether a geometry fits, the workspace it needs
// (Launch::xs: x, Mlp's gate / up rows, the projections' workspace), and the
// launch.
bool f32split_fits(const Launch& L);
int64_t f32split_xs_bytes(const Launch& L);
hipError_t launch_f32_split(const Launch& L, hipStream_t st);

// Choose a kernel family for the geometry (host only, no device calls).
Kernel select_kernel(const Launch& L);
const char* kernel_name(Kernel k);
// The family xrmm_select_kernel names, for a caller that does (with_ws) or
// does not supply the MatMulNBits / Qkv / Mlp workspace; null (and the
// status set) for an invalid geometry.
const char* select_kernel_name(int32_t op, int64_t M, int64_t K, int64_t N, int32_t bits, int32_t block_size,
                               int32_t dtype, int32_t zp_dtype, bool with_ws);

// Enqueue the operator on `stream`. Returns hipSuccess or the launch error.
hipError_t launch(const Launch& L, hipStream_t stream);

// Record the status of an ABI call for xrmm_last_error ("" when XRMM_OK).
int set_status(int code, const std::string& msg);

// MatMulNBits split-K: splits for the geometry (1: none) and the workspace
// bytes they need (0 when there is no split).
int gemm_splits(const Launch& L);
int64_t gemm_workspace_bytes(const Launch& L, int splits);

// W [N, K] in out_dtype (see xrmm_dequantize).
hipError_t launch_dequantize(const Launch& L, void* W, int out_dtype, hipStream_t stream);

// Prepacked 4-bit weights (xrmm_prepack_weights): bytes of the layout, 0 when
// the geometry has none (the layout needs 4-bit codes and whole 32-code
// chunks per column).
int64_t prepacked_bytes(int64_t N, int64_t kb, int64_t block_size, int bits);
// Write L.p[0].B (N x kb x blob) to `out` in the prepacked layout.
hipError_t launch_prepack(const Launch& L, void* out, hipStream_t stream);
// Whether the prepacked GEMM runs this geometry (float16, 4-bit, the fast
// kernels' alignment and block conditions, 32-bit index ranges).
bool prepacked_ok(const Launch& L);
// MatMulNBits with L.p[0].B prepacked (prepacked_ok must hold).
hipError_t launch_prepacked(const Launch& L, hipStream_t stream);

// Raises a kernel's dynamic-LDS cap to `bytes` once per device. `done` is a
// per-kernel array of flags the call site owns (a function-local static,
// zero-initialised at load time); the flags are atomic, so host threads may
// launch concurrently, and a repeated attribute call from a race is harmless.
// Device ordinals beyond the table are not cached (the attribute is set on
// every launch there).
constexpr int kMaxDevices = 64;
inline hipError_t raise_lds_cap(const void* kern, int bytes, std::atomic<int> (&done)[kMaxDevices]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (done[dev].load(std::memory_order_acquire) != 0) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done[dev].store(1, std::memory_order_release);
  return e;
}

}  // namespace xrmm
