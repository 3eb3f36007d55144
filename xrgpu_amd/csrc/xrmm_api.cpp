// C ABI of libxrmm: argument validation and dispatch of the zero-copy entry
// points. The error classes mirror the reference's std::invalid_argument
// (contract / geometry) and std::runtime_error (device) split.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/xrmm.h"
#include "xrmm_internal.h"
#include "xrmm_moe.h"
#include "xrmm_quant.h"

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int ok() {
  g_error.clear();
  return XRMM_OK;
}

int dev_fail(hipError_t e, const char* where) {
  return fail(XRMM_EDEVICE, std::string(where) + ": " + hipGetErrorString(e));
}

bool t1_ok(int32_t d) { return d == XRMM_F32 || d == XRMM_F16; }

// zero-point dtype -> kind; -1 if invalid
int zp_kind_of(int32_t zp_dtype) {
  if (zp_dtype == XRMM_UNSPECIFIED) return xrmm::ZP_NONE;
  if (zp_dtype == XRMM_F32 || zp_dtype == XRMM_F16) return xrmm::ZP_FLOAT;
  if (zp_dtype == XRMM_U8) return xrmm::ZP_PACKED;
  return -1;
}

// Shared geometry checks; fills the common part of the launch description.
int geometry(xrmm::Launch& L, int op, int64_t M, int64_t K, int32_t bits, int32_t block_size,
             int32_t dtype, int32_t zp_dtype) {
  if (!t1_ok(dtype)) return fail(XRMM_EINVAL, "T1 must be float32 or float16");
  if (bits != 2 && bits != 4 && bits != 8) return fail(XRMM_EINVAL, "bits must be 2, 4 or 8");
  if (block_size <= 0) return fail(XRMM_EINVAL, "Invalid packed matmul geometry: block_size must be positive");
  if (K <= 0) return fail(XRMM_EINVAL, "Invalid packed matmul geometry: K must be positive");
  if (M < 0) return fail(XRMM_EINVAL, "M must be non-negative");
  const int zk = zp_kind_of(zp_dtype);
  if (zk < 0) return fail(XRMM_EINVAL, "zero points must be float32, float16 or packed uint8");
  std::memset(&L, 0, sizeof(L));
  L.op = op;
  L.dtype = dtype == XRMM_F32 ? xrmm::DT_F32 : xrmm::DT_F16;
  L.zp_kind = zk;
  L.zp_dtype = zp_dtype == XRMM_F32 ? xrmm::DT_F32 : xrmm::DT_F16;
  L.bits = bits;
  L.block_size = block_size;
  L.M = M;
  L.K = K;
  L.kb = (K + block_size - 1) / block_size;
  L.blob = (static_cast<int64_t>(block_size) * bits + 7) / 8;
  L.zrow = (L.kb * bits + 7) / 8;
  L.bs_log2 = -1;
  for (int i = 0; i < 31; ++i)
    if (block_size == (1 << i)) L.bs_log2 = i;
  L.exact_weights = xrmm::ExactWeightsScope::active();
  return XRMM_OK;
}

int run(const xrmm::Launch& L, void* stream) {
  hipError_t e = xrmm::launch(L, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return dev_fail(e, "kernel launch");
  return ok();
}

}  // namespace

namespace xrmm {
// Status reporting shared with the request-level lifecycle (xrmm_operator.cpp).
int set_status(int code, const std::string& msg) {
  g_error = code == XRMM_OK ? std::string() : msg;
  return code;
}

namespace {
thread_local bool g_exact_weights = false;
}

ExactWeightsScope::ExactWeightsScope(bool on) : prev_(g_exact_weights) { g_exact_weights = on; }
ExactWeightsScope::~ExactWeightsScope() { g_exact_weights = prev_; }
bool ExactWeightsScope::active() { return g_exact_weights; }

const char* select_kernel_name(int32_t op, int64_t M, int64_t K, int64_t N, int32_t bits, int32_t block_size,
                               int32_t dtype, int32_t zp_dtype, bool with_ws) {
  Launch L;
  if (op < OP_MATMUL || op > OP_MLP) {
    fail(XRMM_EINVAL, "unknown operator code");
    return nullptr;
  }
  if (geometry(L, op, M, K, bits, block_size, dtype, zp_dtype)) return nullptr;
  // aligned placeholders: the selection only looks at pointer alignment
  static const uint8_t dummy[16] __attribute__((aligned(16))) = {0};
  L.nproj = op == OP_QKV ? 3 : op == OP_MLP ? 2 : 1;
  L.A = dummy;
  if (op == OP_QKV) L.gamma = dummy;  // normScaleT is required for Qkv
  for (int i = 0; i < L.nproj; ++i) L.p[i] = Proj{dummy, dummy, zp_dtype == XRMM_UNSPECIFIED ? nullptr : dummy, nullptr, nullptr, N};
  if (with_ws) {
    L.xs = const_cast<uint8_t*>(dummy);
    L.ws = const_cast<uint8_t*>(dummy);
  }
  ok();
  return kernel_name(select_kernel(L));
}
}  // namespace xrmm

extern "C" {

const char* xrmm_last_error(void) { return g_error.c_str(); }

const char* xrmm_version(void) { return "xrmm 0.1.0 gfx950"; }

int xrmm_matmul_nbits(const void* A, const void* B, const void* scales, const void* zero_points,
                      int32_t zp_dtype, const void* bias, void* Y, int64_t M, int64_t K, int64_t N,
                      int32_t bits, int32_t block_size, int32_t dtype, void* stream) {
  xrmm::Launch L;
  if (int rc = geometry(L, xrmm::OP_MATMUL, M, K, bits, block_size, dtype, zp_dtype)) return rc;
  if (N <= 0) return fail(XRMM_EINVAL, "Packed matmul N required");
  if (zp_dtype != XRMM_UNSPECIFIED && !zero_points) return fail(XRMM_EINVAL, "zero-point dtype given without zero points");
  if (M > 0 && (!A || !B || !scales || !Y)) return fail(XRMM_EINVAL, "null tensor pointer");
  L.nproj = 1;
  L.A = A;
  L.p[0] = xrmm::Proj{static_cast<const uint8_t*>(B), scales, zero_points, bias, Y, N};
  return run(L, stream);
}

int64_t xrmm_matmul_nbits_workspace_bytes(int64_t M, int64_t K, int64_t N, int32_t bits, int32_t block_size,
                                          int32_t dtype) {
  xrmm::Launch L;
  if (N <= 0 || geometry(L, xrmm::OP_MATMUL, M, K, bits, block_size, dtype, XRMM_UNSPECIFIED) != XRMM_OK) {
    g_error.clear();
    return 0;
  }
  L.nproj = 1;
  L.p[0].N = N;
  // aligned placeholders: the choice depends on the geometry (and on a
  // workspace being there)
  static const uint8_t dummy[16] __attribute__((aligned(16))) = {0};
  L.A = dummy;
  L.p[0].B = dummy;
  L.p[0].scales = dummy;
  L.ws = const_cast<uint8_t*>(dummy);
  const xrmm::Kernel k = M > 0 ? xrmm::select_kernel(L) : xrmm::K_GENERIC;
  if (k == xrmm::K_GEMM_F32X) {
    // sized for float zero points (their row sums), the kind that needs most
    xrmm::Launch Lz = L;
    Lz.zp_kind = xrmm::ZP_FLOAT;
    return xrmm::f32x_workspace_bytes(Lz);
  }
  if (k != xrmm::K_GEMM_Q4 && k != xrmm::K_GEMM_THIN) return 0;
  L.ws = nullptr;
  return xrmm::gemm_workspace_bytes(L, xrmm::gemm_splits(L));
}

int xrmm_matmul_nbits_ws(const void* A, const void* B, const void* scales, const void* zero_points, int32_t zp_dtype,
                         const void* bias, void* Y, int64_t M, int64_t K, int64_t N, int32_t bits, int32_t block_size,
                         int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  xrmm::Launch L;
  if (int rc = geometry(L, xrmm::OP_MATMUL, M, K, bits, block_size, dtype, zp_dtype)) return rc;
  if (N <= 0) return fail(XRMM_EINVAL, "Packed matmul N required");
  if (zp_dtype != XRMM_UNSPECIFIED && !zero_points) return fail(XRMM_EINVAL, "zero-point dtype given without zero points");
  if (M > 0 && (!A || !B || !scales || !Y)) return fail(XRMM_EINVAL, "null tensor pointer");
  L.nproj = 1;
  L.A = A;
  L.p[0] = xrmm::Proj{static_cast<const uint8_t*>(B), scales, zero_points, bias, Y, N};
  if (workspace && M > 0) {
    // the float32 MFMA GEMM runs only with a workspace: row exponents and
    // split partials
    xrmm::Launch Lw = L;
    Lw.ws = workspace;
    if (xrmm::select_kernel(Lw) == xrmm::K_GEMM_F32X) {
      const int64_t need = xrmm::f32x_workspace_bytes(L);
      if (workspace_bytes < need)
        return fail(XRMM_EINVAL, "workspace smaller than xrmm_matmul_nbits_workspace_bytes: " + std::to_string(need));
      if (reinterpret_cast<uintptr_t>(workspace) & 255u) return fail(XRMM_EINVAL, "workspace must be 256-byte aligned");
      L.ws = workspace;
      return run(L, stream);
    }
  }
  const xrmm::Kernel k = M > 0 ? xrmm::select_kernel(L) : xrmm::K_GENERIC;
  if (workspace && (k == xrmm::K_GEMM_Q4 || k == xrmm::K_GEMM_THIN)) {
    const int splits = xrmm::gemm_splits(L);
    const int64_t need = xrmm::gemm_workspace_bytes(L, splits);
    if (need > 0) {
      if (workspace_bytes < need)
        return fail(XRMM_EINVAL, "workspace smaller than xrmm_matmul_nbits_workspace_bytes: " + std::to_string(need));
      if (reinterpret_cast<uintptr_t>(workspace) & 255u) return fail(XRMM_EINVAL, "workspace must be 256-byte aligned");
      L.ws = workspace;
      L.splits = splits;
    }
  }
  return run(L, stream);
}

int64_t xrmm_prepacked_bytes(int64_t N, int64_t K, int32_t bits, int32_t block_size) {
  if (N <= 0 || K <= 0 || block_size <= 0) return 0;
  return xrmm::prepacked_bytes(N, (K + block_size - 1) / block_size, block_size, bits);
}

int xrmm_prepack_weights(const void* B, void* packed, int64_t N, int64_t K, int32_t bits, int32_t block_size,
                         void* stream) {
  xrmm::Launch L;
  if (int rc = geometry(L, xrmm::OP_MATMUL, 1, K, bits, block_size, XRMM_F16, XRMM_UNSPECIFIED)) return rc;
  if (N <= 0) return fail(XRMM_EINVAL, "Packed matmul N required");
  if (xrmm::prepacked_bytes(N, L.kb, block_size, bits) == 0)
    return fail(XRMM_EINVAL, "prepacked weights need 4-bit codes and whole 32-code chunks per column");
  if (!B || !packed) return fail(XRMM_EINVAL, "null tensor pointer");
  if ((reinterpret_cast<uintptr_t>(B) & 15u) || (reinterpret_cast<uintptr_t>(packed) & 15u))
    return fail(XRMM_EINVAL, "prepack: B and the packed buffer must be 16-byte aligned");
  L.nproj = 1;
  L.p[0] = xrmm::Proj{static_cast<const uint8_t*>(B), nullptr, nullptr, nullptr, nullptr, N};
  const hipError_t e = xrmm::launch_prepack(L, packed, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return dev_fail(e, "prepack launch");
  return ok();
}

int xrmm_matmul_nbits_prepacked(const void* A, const void* packed, const void* scales, const void* zero_points,
                                int32_t zp_dtype, const void* bias, void* Y, int64_t M, int64_t K, int64_t N,
                                int32_t bits, int32_t block_size, int32_t dtype, void* stream) {
  xrmm::Launch L;
  if (int rc = geometry(L, xrmm::OP_MATMUL, M, K, bits, block_size, dtype, zp_dtype)) return rc;
  if (N <= 0) return fail(XRMM_EINVAL, "Packed matmul N required");
  if (zp_dtype != XRMM_UNSPECIFIED && !zero_points) return fail(XRMM_EINVAL, "zero-point dtype given without zero points");
  if (M == 0) return ok();
  if (!A || !packed || !scales || !Y) return fail(XRMM_EINVAL, "null tensor pointer");
  L.nproj = 1;
  L.A = A;
  L.p[0] = xrmm::Proj{static_cast<const uint8_t*>(packed), scales, zero_points, bias, Y, N};
  if (!xrmm::prepacked_ok(L))
    return fail(XRMM_EINVAL, "prepacked weights run float16 activations with 4-bit codes, a power-of-two block_size "
                             ">= 16, K a multiple of 8 and 16-byte aligned tensors");
  const hipError_t e = xrmm::launch_prepacked(L, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return dev_fail(e, "kernel launch");
  return ok();
}

}  // extern "C"

namespace {

int qkv_launch(xrmm::Launch& L, const void* A, const void* skip, const void* norm_scale, const void* q_B,
               const void* q_scales, const void* q_zero_points, const void* k_B, const void* k_scales,
               const void* k_zero_points, const void* v_B, const void* v_scales, const void* v_zero_points,
               int32_t zp_dtype, void* Q, void* Kout, void* V, void* residual, int64_t M, int64_t K, int64_t Nq,
               int64_t Nkv, int32_t bits, int32_t block_size, float epsilon, int32_t dtype) {
  if (int rc = geometry(L, xrmm::OP_QKV, M, K, bits, block_size, dtype, zp_dtype)) return rc;
  if (Nq <= 0 || Nkv <= 0) return fail(XRMM_EINVAL, "Nq and Nkv must be positive");
  if (!norm_scale) return fail(XRMM_EINVAL, "Missing complex input: normScaleT");
  if (M > 0 && (!A || !q_B || !k_B || !v_B || !q_scales || !k_scales || !v_scales || !Q || !Kout || !V))
    return fail(XRMM_EINVAL, "null tensor pointer");
  if (zp_dtype == XRMM_UNSPECIFIED && (q_zero_points || k_zero_points || v_zero_points))
    return fail(XRMM_EINVAL, "zero points given without a zero-point dtype");
  L.nproj = 3;
  L.A = A;
  L.skip = skip;
  L.gamma = norm_scale;
  L.residual = residual;
  L.eps = epsilon;
  L.p[0] = xrmm::Proj{static_cast<const uint8_t*>(q_B), q_scales, q_zero_points, nullptr, Q, Nq};
  L.p[1] = xrmm::Proj{static_cast<const uint8_t*>(k_B), k_scales, k_zero_points, nullptr, Kout, Nkv};
  L.p[2] = xrmm::Proj{static_cast<const uint8_t*>(v_B), v_scales, v_zero_points, nullptr, V, Nkv};
  return XRMM_OK;
}

int mlp_launch(xrmm::Launch& L, const void* A, const void* skip, const void* norm_scale, const void* gate_B,
               const void* gate_scales, const void* gate_zero_points, const void* gate_bias, const void* up_B,
               const void* up_scales, const void* up_zero_points, const void* up_bias, int32_t zp_dtype, void* Y,
               void* residual, int64_t M, int64_t K, int64_t N, int32_t bits, int32_t block_size, float epsilon,
               int32_t activation, int32_t dtype) {
  if (int rc = geometry(L, xrmm::OP_MLP, M, K, bits, block_size, dtype, zp_dtype)) return rc;
  if (N <= 0) return fail(XRMM_EINVAL, "Packed matmul N required");
  if (activation < XRMM_ACT_NONE || activation > XRMM_ACT_SWIGLU) return fail(XRMM_EINVAL, "Unknown fused activation");
  if (M > 0 && (!A || !gate_B || !gate_scales || !up_B || !up_scales || !Y))
    return fail(XRMM_EINVAL, "null tensor pointer");
  if (zp_dtype == XRMM_UNSPECIFIED && (gate_zero_points || up_zero_points))
    return fail(XRMM_EINVAL, "zero points given without a zero-point dtype");
  L.nproj = 2;
  L.A = A;
  L.skip = skip;
  L.gamma = norm_scale;
  L.residual = residual;
  L.eps = epsilon;
  L.act = activation;
  L.p[0] = xrmm::Proj{static_cast<const uint8_t*>(gate_B), gate_scales, gate_zero_points, gate_bias, Y, N};
  L.p[1] = xrmm::Proj{static_cast<const uint8_t*>(up_B), up_scales, up_zero_points, up_bias, nullptr, N};
  return XRMM_OK;
}

// Bytes of the workspace a Qkv / Mlp launch would use (0: its kernel reads
// none): the normalised binary16 rows of the float16 prefill GEMMs, or the
// float32 path's x, gate / up rows and projection workspace. The selection
// looks at the workspace pointer, so it is asked with a placeholder one.
int64_t xs_need(xrmm::Launch L) {
  if (L.M <= 0) return 0;
  static const uint8_t dummy[16] __attribute__((aligned(16))) = {0};
  L.xs = const_cast<uint8_t*>(dummy);
  const xrmm::Kernel k = xrmm::select_kernel(L);
  if (k == xrmm::K_F32_SPLIT) return xrmm::f32split_xs_bytes(L);
  if (!xrmm::fused_prologue(L)) return 0;
  return k == xrmm::K_GEMM_FUSED || k == xrmm::K_GEMM_BIG_FUSED || k == xrmm::K_GEMM_THIN ? xrmm::fused_xs_bytes(L) : 0;
}

// Attach a caller's workspace when the launch uses one.
int attach_xs(xrmm::Launch& L, void* workspace, int64_t workspace_bytes) {
  const int64_t need = xs_need(L);
  if (need == 0 || workspace == nullptr) return XRMM_OK;
  if (workspace_bytes < need)
    return fail(XRMM_EINVAL, "workspace smaller than xrmm_matmul_nbits_fused_workspace_bytes: " + std::to_string(need));
  if (reinterpret_cast<uintptr_t>(workspace) & 255u) return fail(XRMM_EINVAL, "workspace must be 256-byte aligned");
  L.xs = workspace;
  return XRMM_OK;
}

}  // namespace

extern "C" {

int xrmm_matmul_nbits_qkv(const void* A, const void* skip, const void* norm_scale, const void* q_B,
                          const void* q_scales, const void* q_zero_points, const void* k_B,
                          const void* k_scales, const void* k_zero_points, const void* v_B,
                          const void* v_scales, const void* v_zero_points, int32_t zp_dtype, void* Q,
                          void* Kout, void* V, void* residual, int64_t M, int64_t K, int64_t Nq,
                          int64_t Nkv, int32_t bits, int32_t block_size, float epsilon, int32_t dtype,
                          void* stream) {
  return xrmm_matmul_nbits_qkv_ws(A, skip, norm_scale, q_B, q_scales, q_zero_points, k_B, k_scales, k_zero_points,
                                  v_B, v_scales, v_zero_points, zp_dtype, Q, Kout, V, residual, M, K, Nq, Nkv, bits,
                                  block_size, epsilon, dtype, nullptr, 0, stream);
}

int xrmm_matmul_nbits_qkv_ws(const void* A, const void* skip, const void* norm_scale, const void* q_B,
                             const void* q_scales, const void* q_zero_points, const void* k_B,
                             const void* k_scales, const void* k_zero_points, const void* v_B,
                             const void* v_scales, const void* v_zero_points, int32_t zp_dtype, void* Q,
                             void* Kout, void* V, void* residual, int64_t M, int64_t K, int64_t Nq,
                             int64_t Nkv, int32_t bits, int32_t block_size, float epsilon, int32_t dtype,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  xrmm::Launch L;
  if (int rc = qkv_launch(L, A, skip, norm_scale, q_B, q_scales, q_zero_points, k_B, k_scales, k_zero_points, v_B,
                          v_scales, v_zero_points, zp_dtype, Q, Kout, V, residual, M, K, Nq, Nkv, bits, block_size,
                          epsilon, dtype))
    return rc;
  if (int rc = attach_xs(L, workspace, workspace_bytes)) return rc;
  return run(L, stream);
}

int xrmm_matmul_nbits_mlp(const void* A, const void* skip, const void* norm_scale, const void* gate_B,
                          const void* gate_scales, const void* gate_zero_points, const void* gate_bias,
                          const void* up_B, const void* up_scales, const void* up_zero_points,
                          const void* up_bias, int32_t zp_dtype, void* Y, void* residual, int64_t M,
                          int64_t K, int64_t N, int32_t bits, int32_t block_size, float epsilon,
                          int32_t activation, int32_t dtype, void* stream) {
  return xrmm_matmul_nbits_mlp_ws(A, skip, norm_scale, gate_B, gate_scales, gate_zero_points, gate_bias, up_B,
                                  up_scales, up_zero_points, up_bias, zp_dtype, Y, residual, M, K, N, bits, block_size,
                                  epsilon, activation, dtype, nullptr, 0, stream);
}

int xrmm_matmul_nbits_mlp_ws(const void* A, const void* skip, const void* norm_scale, const void* gate_B,
                             const void* gate_scales, const void* gate_zero_points, const void* gate_bias,
                             const void* up_B, const void* up_scales, const void* up_zero_points,
                             const void* up_bias, int32_t zp_dtype, void* Y, void* residual, int64_t M,
                             int64_t K, int64_t N, int32_t bits, int32_t block_size, float epsilon,
                             int32_t activation, int32_t dtype, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  xrmm::Launch L;
  if (int rc = mlp_launch(L, A, skip, norm_scale, gate_B, gate_scales, gate_zero_points, gate_bias, up_B, up_scales,
                          up_zero_points, up_bias, zp_dtype, Y, residual, M, K, N, bits, block_size, epsilon,
                          activation, dtype))
    return rc;
  if (int rc = attach_xs(L, workspace, workspace_bytes)) return rc;
  return run(L, stream);
}

int64_t xrmm_matmul_nbits_fused_workspace_bytes(int32_t op, int64_t M, int64_t K, int64_t N, int64_t Nkv,
                                                int32_t bits, int32_t block_size, int32_t dtype, int32_t has_skip,
                                                int32_t has_norm_scale) {
  xrmm::Launch L;
  if ((op != xrmm::OP_QKV && op != xrmm::OP_MLP) || N <= 0 || (op == xrmm::OP_QKV && Nkv <= 0) ||
      geometry(L, op, M, K, bits, block_size, dtype, XRMM_UNSPECIFIED) != XRMM_OK) {
    g_error.clear();
    return 0;
  }
  static const uint8_t dummy[16] __attribute__((aligned(16))) = {0};
  L.nproj = op == xrmm::OP_QKV ? 3 : 2;
  L.A = dummy;
  L.skip = has_skip ? dummy : nullptr;
  L.gamma = (has_norm_scale || op == xrmm::OP_QKV) ? dummy : nullptr;
  for (int i = 0; i < L.nproj; ++i)
    L.p[i] = xrmm::Proj{dummy, dummy, nullptr, nullptr, nullptr, (op == xrmm::OP_QKV && i > 0) ? Nkv : N};
  return xs_need(L);
}

int xrmm_dequantize(const void* B, const void* scales, const void* zero_points, int32_t zp_dtype, void* W,
                    int64_t N, int64_t K, int32_t bits, int32_t block_size, int32_t scale_dtype,
                    int32_t out_dtype, void* stream) {
  xrmm::Launch L;
  if (int rc = geometry(L, xrmm::OP_MATMUL, 0, K, bits, block_size, scale_dtype, zp_dtype)) return rc;
  if (N <= 0) return fail(XRMM_EINVAL, "N must be positive");
  if (!t1_ok(out_dtype)) return fail(XRMM_EINVAL, "output dtype must be float32 or float16");
  if (!B || !scales || !W) return fail(XRMM_EINVAL, "null tensor pointer");
  if (zp_dtype != XRMM_UNSPECIFIED && !zero_points) return fail(XRMM_EINVAL, "zero-point dtype given without zero points");
  L.nproj = 1;
  L.p[0] = xrmm::Proj{static_cast<const uint8_t*>(B), scales, zero_points, nullptr, nullptr, N};
  hipError_t e = xrmm::launch_dequantize(L, W, out_dtype == XRMM_F32 ? xrmm::DT_F32 : xrmm::DT_F16,
                                         static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return dev_fail(e, "dequantize launch");
  return ok();
}

const char* xrmm_select_kernel(int32_t op, int64_t M, int64_t K, int64_t N, int32_t bits, int32_t block_size,
                               int32_t dtype, int32_t zp_dtype) {
  // the front ends (ops.py, the request lifecycle) supply the Qkv / Mlp
  // prefill workspace and the MatMulNBits one, so the selection assumes them
  return xrmm::select_kernel_name(op, M, K, N, bits, block_size, dtype, zp_dtype, true);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// com.microsoft.QMoE (opcode 1030)

namespace {

// The planner checks of complex_plan.cpp:121-127 over plain sizes (messages
// follow the reference's wording); fills the launch block.
int qmoe_geometry(xrmm::MoeArgs& a, int64_t tokens, int64_t hidden, int64_t experts, int64_t fc1_rows, int32_t k,
                  int32_t bits, int32_t block_size, int32_t activation, int32_t swiglu_fusion) {
  if (tokens < 0 || hidden <= 0 || experts < 1 || k < 1 || k > experts)
    return fail(XRMM_EINVAL, "Invalid MoE input or routing geometry");
  const bool swiglu = activation == XRMM_ACT_SWIGLU;
  const int64_t fusion = swiglu && swiglu_fusion ? 2 : 1;
  if (fc1_rows < 0 || fc1_rows % fusion != 0) return fail(XRMM_EINVAL, "Invalid MoE weight geometry");
  if (bits != 4 && bits != 8) return fail(XRMM_EINVAL, "Unsupported QMoE integer layout");
  if (!((activation == XRMM_ACT_RELU && swiglu_fusion == 0) || (swiglu && swiglu_fusion == 1)))
    return fail(XRMM_EINVAL, "Invalid quantized SwiGLU fusion");
  const int64_t inter = fc1_rows / fusion;
  if ((hidden * bits) % 8 != 0 || (inter * bits) % 8 != 0) return fail(XRMM_EINVAL, "Invalid packed expert projection");
  if (block_size != 0 && (block_size < 16 || (block_size & (block_size - 1)) != 0 || hidden % block_size != 0 ||
                          inter % block_size != 0))
    return fail(XRMM_EINVAL, "Invalid quantized expert block size");
  if (tokens * k > int64_t(1) << 31 || hidden > int64_t(1) << 24 || inter > int64_t(1) << 24)
    return fail(XRMM_EINVAL, "QMoE geometry beyond 32-bit indexing");
  std::memset(&a, 0, sizeof(a));
  a.T = tokens;
  a.H = hidden;
  a.E = experts;
  a.F1 = fc1_rows;
  a.I = inter;
  a.k = k;
  a.bits = bits;
  a.bs = block_size;
  a.act = activation;
  return XRMM_OK;
}

}  // namespace

int64_t xrmm_qmoe_workspace_bytes(int64_t tokens, int32_t k, int64_t hidden, int64_t inter) {
  if (tokens < 0 || k < 1 || hidden < 0 || inter < 0) return -1;
  return xrmm::moe_workspace_bytes(tokens, k, hidden, inter);
}

int xrmm_qmoe(const void* input, const void* router, const void* fc1, const void* fc1_scales, const void* fc2,
              const void* fc2_scales, void* output, void* workspace, int64_t workspace_bytes, int64_t tokens,
              int64_t hidden, int64_t experts, int64_t fc1_rows, int32_t k, int32_t bits, int32_t block_size,
              int32_t activation, int32_t swiglu_fusion, float alpha, float beta, float swiglu_limit,
              int32_t has_limit, void* stream) {
  xrmm::MoeArgs a;
  if (int rc = qmoe_geometry(a, tokens, hidden, experts, fc1_rows, k, bits, block_size, activation, swiglu_fusion))
    return rc;
  // empty tensors (no intermediate width) may come without storage
  if (tokens > 0 && (!input || !router || !output || (a.I > 0 && (!fc1 || !fc2 || !fc1_scales || !fc2_scales))))
    return fail(XRMM_EINVAL, "null tensor pointer");
  const int64_t need = xrmm::moe_workspace_bytes(tokens, k, hidden, a.I);
  if (tokens > 0 && (!workspace || workspace_bytes < need))
    return fail(XRMM_EINVAL, "QMoE workspace smaller than xrmm_qmoe_workspace_bytes");
  auto al = [](int64_t b) { return (b + 255) / 256 * 256; };
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  a.x = static_cast<const float*>(input);
  a.router = static_cast<const float*>(router);
  a.fc1 = static_cast<const uint8_t*>(fc1);
  a.s1 = static_cast<const float*>(fc1_scales);
  a.fc2 = static_cast<const uint8_t*>(fc2);
  a.s2 = static_cast<const float*>(fc2_scales);
  a.y = static_cast<float*>(output);
  a.sel = reinterpret_cast<int32_t*>(ws);
  a.wts = reinterpret_cast<float*>(ws + al(tokens * k * 4));
  a.h = reinterpret_cast<float*>(ws + 2 * al(tokens * k * 4));
  const int64_t ksmax = xrmm::moe_yp_segments(tokens, k, hidden, a.I);
  a.yp = reinterpret_cast<float*>(ws + 2 * al(tokens * k * 4) + al(tokens * k * a.I * 4));
  a.cnt = reinterpret_cast<uint32_t*>(ws + 2 * al(tokens * k * 4) + al(tokens * k * a.I * 4) +
                                      al(tokens * k * ksmax * hidden * 4));
  a.alpha = alpha;
  a.beta = beta;
  a.limit = swiglu_limit;
  a.has_limit = has_limit != 0;
  const hipError_t e = xrmm::launch_qmoe(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return dev_fail(e, "QMoE launch");
  return ok();
}

const char* xrmm_qmoe_kernel(int64_t tokens, int64_t hidden, int64_t experts, int64_t fc1_rows, int32_t k, int32_t bits,
                             int32_t block_size, int32_t activation, int32_t swiglu_fusion) {
  xrmm::MoeArgs a{};
  if (qmoe_geometry(a, tokens, hidden, experts, fc1_rows, k, bits, block_size, activation, swiglu_fusion)) return nullptr;
  // pointers of 16-byte aligned allocations: the choice then depends on the geometry only
  static const uint8_t probe[16] __attribute__((aligned(16))) = {};
  a.x = reinterpret_cast<const float*>(probe);
  a.fc1 = a.fc2 = probe;
  a.h = a.yp = reinterpret_cast<float*>(const_cast<uint8_t*>(probe));
  return xrmm::moe_kernel_name(a);
}

// ---------------------------------------------------------------------------
// com.microsoft.GatherBlockQuantized (opcode 1031), com.microsoft.MatMulBnb4 (1026)

int xrmm_gather_block_quantized(const void* data, const void* indices, int32_t indices_dtype, const void* scales,
                                const void* zero_points, void* output, void* status, int64_t rows,
                                int64_t packed_cols, int64_t n_indices, int32_t bits, int32_t block_size,
                                void* stream) {
  // complex_plan.cpp:129
  if ((bits != 4 && bits != 8) || block_size < 16 || (block_size & (block_size - 1)) != 0)
    return fail(XRMM_EINVAL, "Unsupported GatherBlockQuantized geometry");
  if (rows < 0 || packed_cols < 0 || n_indices < 0) return fail(XRMM_EINVAL, "Unsupported GatherBlockQuantized geometry");
  if (indices_dtype != XRMM_I32 && indices_dtype != XRMM_U32 && indices_dtype != XRMM_I64)
    return fail(XRMM_EINVAL, "Logical dtype outside frozen contract: indicesT");
  xrmm::GbqArgs a{};
  a.width = packed_cols * (8 / bits);
  a.blocks = (a.width + block_size - 1) / block_size;
  a.zpcols = (a.blocks * bits + 7) / 8;
  if (n_indices > 0 && a.width > 0 && (!data || !indices || !scales || !output))
    return fail(XRMM_EINVAL, "null tensor pointer");
  if (n_indices * a.width >= (int64_t(1) << 40)) return fail(XRMM_EINVAL, "GatherBlockQuantized output too large");
  a.data = static_cast<const uint8_t*>(data);
  a.idx = indices;
  a.idx64 = indices_dtype == XRMM_I64;
  a.scales = static_cast<const float*>(scales);
  a.zp = static_cast<const uint8_t*>(zero_points);
  a.out = static_cast<float*>(output);
  a.status = static_cast<uint32_t*>(status);
  a.rows = rows;
  a.pcols = packed_cols;
  a.n = n_indices;
  a.bits = bits;
  a.bs = block_size;
  const hipError_t e = xrmm::launch_gbq(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return dev_fail(e, "GatherBlockQuantized launch");
  return ok();
}

namespace {

int bnb4_geometry(xrmm::Bnb4Args& a, int64_t M, int64_t K, int64_t N, int32_t block_size, int32_t quant_type,
                  int32_t trans_b, int32_t dtype) {
  // complex_plan.cpp:117-120
  if (!t1_ok(dtype)) return fail(XRMM_EINVAL, "Logical dtype outside frozen contract: aT");
  if (K <= 0 || block_size <= 0) return fail(XRMM_EINVAL, "Invalid packed matmul geometry");
  if (N <= 0) return fail(XRMM_EINVAL, "Packed matmul N required");
  if (M < 0) return fail(XRMM_EINVAL, "Invalid packed matmul geometry");
  if (quant_type != 0 && quant_type != 1) return fail(XRMM_EINVAL, "MatMulBnb4 quant_type must be 0 (FP4) or 1 (NF4)");
  if (N * K >= (int64_t(1) << 40)) return fail(XRMM_EINVAL, "MatMulBnb4 weight too large");
  a = xrmm::Bnb4Args{};
  a.M = M;
  a.K = K;
  a.N = N;
  a.bs = block_size;
  a.qt = quant_type;
  a.tb = trans_b != 0;
  a.f16 = dtype == XRMM_F16;
  return XRMM_OK;
}

}  // namespace

int xrmm_matmul_bnb4(const void* A, const void* B, const void* absmax, void* Y, int64_t M, int64_t K, int64_t N,
                     int32_t block_size, int32_t quant_type, int32_t trans_b, int32_t dtype, void* stream) {
  xrmm::Bnb4Args a;
  if (int rc = bnb4_geometry(a, M, K, N, block_size, quant_type, trans_b, dtype)) return rc;
  if (M > 0 && (!A || !B || !absmax || !Y)) return fail(XRMM_EINVAL, "null tensor pointer");
  a.A = A;
  a.B = static_cast<const uint8_t*>(B);
  a.absmax = absmax;
  a.Y = Y;
  const hipError_t e = xrmm::launch_bnb4(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return dev_fail(e, "MatMulBnb4 launch");
  return ok();
}

const char* xrmm_matmul_bnb4_kernel(int64_t M, int64_t K, int64_t N, int32_t block_size, int32_t quant_type,
                                    int32_t trans_b, int32_t dtype) {
  xrmm::Bnb4Args a;
  if (bnb4_geometry(a, M, K, N, block_size, quant_type, trans_b, dtype)) return nullptr;
  static const uint8_t probe[16] __attribute__((aligned(16))) = {};
  a.A = probe;
  a.B = probe;
  ok();
  return xrmm::bnb4_fast_ok(a) ? "bnb4_gemv" : "bnb4_scalar";
}

// ---------------------------------------------------------------------------
// opt-in int8 activations (accuracy_level 4 of the upstream operator)

int64_t xrmm_matmul_nbits_int8a_workspace_bytes(int64_t M, int64_t K) {
  if (M < 0 || K <= 0 || K % xrmm::kI8aBlock != 0 || K > xrmm::kI8aMaxK) return -1;
  return xrmm::i8a_workspace_bytes(M, K);
}

int xrmm_matmul_nbits_int8a_noalloc(const void* A, const void* B, const void* scales, const void* zero_points,
                                    int32_t zp_dtype, const void* bias, void* Y, int64_t M, int64_t K, int64_t N,
                                    int32_t bits, int32_t block_size, int32_t dtype, void* stream) {
  // Same contract as xrmm_matmul_nbits_int8a; the workspace is the library's
  // static device scratch, so nothing is allocated. Inputs past the scratch
  // are rejected before any device work.
  if (M > 0 && K > 0 && K % xrmm::kI8aBlock == 0 && K <= xrmm::kI8aMaxK &&
      xrmm::i8a_workspace_bytes(M, K) > xrmm::kI8aScratchBytes)
    return fail(XRMM_EINVAL, "allocation-free int8-activation path: M*K codes and scales exceed the " +
                                 std::to_string(xrmm::kI8aScratchBytes) + "-byte device scratch");
  void* ws = nullptr;
  if (M > 0) {
    const hipError_t e = xrmm::i8a_scratch(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return dev_fail(e, "int8-activation scratch (hipGetSymbolAddress)");
  }
  return xrmm_matmul_nbits_int8a(A, B, scales, zero_points, zp_dtype, bias, Y, ws, xrmm::kI8aScratchBytes, M, K, N,
                                 bits, block_size, dtype, stream);
}

int xrmm_matmul_nbits_int8a(const void* A, const void* B, const void* scales, const void* zero_points,
                            int32_t zp_dtype, const void* bias, void* Y, void* workspace, int64_t workspace_bytes,
                            int64_t M, int64_t K, int64_t N, int32_t bits, int32_t block_size, int32_t dtype,
                            void* stream) {
  if (!t1_ok(dtype)) return fail(XRMM_EINVAL, "T1 must be float32 or float16");
  if (bits != 4 || block_size < 32 || (block_size & (block_size - 1)) != 0 || K <= 0 || K % xrmm::kI8aBlock != 0 ||
      K % block_size != 0 || N <= 0 || M < 0)
    return fail(XRMM_EINVAL, "int8-activation path: bits 4, power-of-two block_size >= 32 dividing K, K a multiple of 128");
  if (K > xrmm::kI8aMaxK) return fail(XRMM_EINVAL, "int8-activation path: K up to 16384 (one wave holds a column's codes)");
  if (zp_dtype != XRMM_UNSPECIFIED && zp_dtype != XRMM_U8)
    return fail(XRMM_EINVAL, "int8-activation path: zero points must be absent or packed uint8");
  if (M == 0) return ok();
  if (!A || !B || !scales || !Y || !workspace || (zp_dtype == XRMM_U8 && !zero_points))
    return fail(XRMM_EINVAL, "null tensor pointer");
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (!al(A) || !al(B) || !al(workspace)) return fail(XRMM_EINVAL, "int8-activation path: A, B and the workspace must be 16-byte aligned");
  if (workspace_bytes < xrmm::i8a_workspace_bytes(M, K))
    return fail(XRMM_EINVAL, "workspace smaller than xrmm_matmul_nbits_int8a_workspace_bytes");
  xrmm::Int8aArgs a{};
  a.A = A;
  a.B = static_cast<const uint8_t*>(B);
  a.S = scales;
  a.Z = zp_dtype == XRMM_U8 ? static_cast<const uint8_t*>(zero_points) : nullptr;
  a.bias = bias;
  a.Y = Y;
  a.qa = static_cast<int8_t*>(workspace);
  a.as = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + (M * K + 255) / 256 * 256);
  a.M = M;
  a.K = K;
  a.N = N;
  a.bs = block_size;
  a.lbs = __builtin_ctz(static_cast<unsigned>(block_size));
  const int64_t kb = K / block_size;
  a.zrow = (kb * 4 + 7) / 8;
  a.f16 = dtype == XRMM_F16;
  const hipError_t e = xrmm::launch_i8a(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return dev_fail(e, "int8-activation MatMulNBits launch");
  return ok();
}
