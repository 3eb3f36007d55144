// Float32 MatMulNBitsQkv / MatMulNBitsMlp (T1 = float32, the dtype of every
// upstream Qkv / Mlp bench case) as a prologue and one MatMulNBits per
// projection on the float32-arithmetic kernels.
//
// The reference forms packedInput x = (A + skip) * inversesqrt(mean(r^2) +
// eps) * gamma (or A + skip) in float32 (complex_kernel.glsl:81), then each
// projection's float32 dot products (:83; Mlp: act(gate + gate_bias) *
// (up + up_bias)). Here k_f32_prologue writes x (and the residual A + skip)
// to the workspace once per row, each projection runs as a float32
// MatMulNBits on x (up to 16 rows: the float32 GEMV with all projections on
// one grid and the prologue done on its staged rows; beyond: k_f32_prologue
// into the workspace, then the float32-arithmetic MFMA GEMM per projection;
// both meet the float32 bar), Qkv's straight into Q, K and V, Mlp's into
// float32 gate / up rows that k_mlp_act combines.
//
// Workspace (Launch::xs): x [M][K] (when there is a prologue), gate and up
// [M][N] (Mlp), then the MatMulNBits workspace of the projections (the MFMA
// GEMM's prepared rows and split partials; the projections run one after
// another on the stream and share it).
#include "xrmm_gemv.h"
#include "xrmm_gemv_f32.h"

namespace xrmm {

namespace {

int64_t al256(int64_t b) { return (b + 255) / 256 * 256; }

// One workgroup per row: r = A + skip (float32), the residual, and x = r or
// r * inversesqrt(sum(r^2) / K + eps) * gamma. Rows of up to 256 * kProHeld
// elements stay in registers: every load of the row (and of gamma) is issued
// before the first use, and x is written once.
constexpr int kProHeld = 16;

__global__ __launch_bounds__(256) void k_f32_prologue(const float* __restrict__ A, const float* __restrict__ skip,
                                                      const float* __restrict__ gamma, float* __restrict__ x,
                                                      float* __restrict__ residual, int K, float eps) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int64_t o = static_cast<int64_t>(m) * K;
  const bool held = K <= 256 * kProHeld;
  float ss = 0.f;
  float rv[kProHeld], gv[kProHeld];
  if (held) {
#pragma unroll
    for (int j = 0; j < kProHeld; ++j) {
      const int k = tid + 256 * j;
      rv[j] = k < K ? (skip ? A[o + k] + skip[o + k] : A[o + k]) : 0.f;
      gv[j] = k < K && gamma ? gamma[k] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kProHeld; ++j) {
      const int k = tid + 256 * j;
      if (k < K) {
        if (!gamma) x[o + k] = rv[j];
        if (residual) residual[o + k] = rv[j];
        ss = __builtin_fmaf(rv[j], rv[j], ss);
      }
    }
  } else {
    for (int k = tid; k < K; k += 256) {
      const float r = skip ? A[o + k] + skip[o + k] : A[o + k];
      x[o + k] = r;
      if (residual) residual[o + k] = r;
      ss = __builtin_fmaf(r, r, ss);
    }
  }
  if (!gamma) return;  // uniform
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if (lane == 0) red[tid >> 6] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.f / __builtin_sqrtf(ss / static_cast<float>(K) + eps);
  if (held) {
#pragma unroll
    for (int j = 0; j < kProHeld; ++j) {
      const int k = tid + 256 * j;
      if (k < K) x[o + k] = rv[j] * inv * gv[j];
    }
    return;
  }
  // each thread rescales the elements it wrote
  for (int k = tid; k < K; k += 256) x[o + k] = x[o + k] * inv * gamma[k];
}

// Mlp: y = act(gate) * up (the biases are in gate and up already).
__global__ __launch_bounds__(256) void k_mlp_act(const float* __restrict__ g, const float* __restrict__ u,
                                                 float* __restrict__ y, int64_t n, int act) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) y[i] = activate(g[i], act) * u[i];
}

// Projection p of a float32 Qkv / Mlp as a MatMulNBits launch on `A` into `Y`.
Launch projection(const Launch& L, int p, const void* A, void* Y, void* ws) {
  Launch L2 = L;
  L2.op = OP_MATMUL;
  L2.nproj = 1;
  L2.A = A;
  L2.skip = nullptr;
  L2.gamma = nullptr;
  L2.residual = nullptr;
  L2.p[0] = L.p[p];
  L2.p[0].Y = Y;
  L2.p[1] = Proj{};
  L2.p[2] = Proj{};
  if (!L.p[p].zp) L2.zp_kind = ZP_NONE;
  L2.ws = ws;
  L2.splits = 1;
  L2.xs = nullptr;
  return L2;
}

bool has_prologue(const Launch& L) { return L.skip || L.gamma || L.residual; }

// x is reserved whether or not the call has a prologue: the workspace size is
// asked without knowing whether the caller wants the residual
// Rows from which the projections share one MFMA GEMM grid (below: one
// float32 GEMV grid). From 5 rows the GEMV's float32 FMAs cost more than the
// GEMM's weight decode: Mlp K = 2048, N = 5632 at 16 rows 38.7 -> 26.2 us,
// Qkv K = 4096, N = 3 x 4096 at 8 rows 54.2 -> 49.6 us, at 16 rows 99.8 ->
// 51.5 us (5 rows: Mlp 23.7 -> 24.4, Qkv 53.3 -> 49.8 us).
#ifndef XRMM_F32_SPLIT_GEMM_ROWS
#define XRMM_F32_SPLIT_GEMM_ROWS 5
#endif
constexpr int64_t kGridRows = XRMM_F32_SPLIT_GEMM_ROWS;

int64_t x_bytes(const Launch& L) { return al256(L.M * L.K * 4); }
int64_t gu_bytes(const Launch& L) { return L.op == OP_MLP ? 2 * al256(L.M * L.p[0].N * 4) : 0; }

// All projections as one MatMulNBits launch on `A` (outputs `Y[p]`): one
// float32 GEMV grid, or one MFMA GEMM grid (given `ws`); the zero-point kind
// applies only when every projection carries zero points.
Launch projections(const Launch& L, const void* A, void* const* Y, void* ws, bool& uniform_zp) {
  Launch Lg = projection(L, 0, A, Y[0], ws);
  Lg.nproj = L.nproj;
  int with_zp = 0;
  for (int p = 0; p < L.nproj; ++p) {
    Lg.p[p] = L.p[p];
    Lg.p[p].Y = Y[p];
    with_zp += L.p[p].zp != nullptr;
  }
  Lg.zp_kind = with_zp ? L.zp_kind : ZP_NONE;
  uniform_zp = with_zp == 0 || with_zp == L.nproj;
  return Lg;
}

// The projections' MatMulNBits workspace: the largest MFMA GEMM need, one
// projection or all on one grid (sized for float zero points, the kind that
// needs most), from kGridRows rows on.
int64_t proj_ws_bytes(const Launch& L) {
  if (L.M < kGridRows) return 0;
  static const uint8_t dummy[16] __attribute__((aligned(16))) = {0};
  int64_t need = 0;
  for (int p = 0; p < L.nproj; ++p) {
    Launch L2 = projection(L, p, dummy, nullptr, const_cast<uint8_t*>(dummy));
    L2.p[0].B = L.p[p].B ? L.p[p].B : dummy;
    L2.p[0].scales = L.p[p].scales ? L.p[p].scales : dummy;
    if (select_kernel(L2) != K_GEMM_F32X) continue;
    L2.zp_kind = ZP_FLOAT;
    const int64_t b = f32x_workspace_bytes(L2);
    need = b > need ? b : need;
  }
  void* const ys[3] = {nullptr, nullptr, nullptr};
  bool uz = true;
  Launch Lm = projections(L, dummy, ys, const_cast<uint8_t*>(dummy), uz);
  Lm.zp_kind = ZP_FLOAT;
  const int64_t b = f32x_workspace_bytes(Lm);
  return b > need ? b : need;
}

}  // namespace

// Float32 Qkv / Mlp whose every projection runs on the float32 GEMV or the
// float32-arithmetic MFMA GEMM (given the workspace), with K and the
// projections' shapes inside their limits.
bool f32split_fits(const Launch& L) {
  if ((L.op != OP_QKV && L.op != OP_MLP) || L.dtype != DT_F32 || L.M < 1) return false;
  const int64_t lim = int64_t(1) << 31;
  if (L.M * L.K >= lim / 4 || L.M * L.p[0].N >= lim / 4) return false;
  static const uint8_t dummy[16] __attribute__((aligned(16))) = {0};
  for (int p = 0; p < L.nproj; ++p) {
    // the projections read x from the workspace (256-byte aligned) or A
    Launch L2 = projection(L, p, has_prologue(L) ? dummy : L.A, nullptr, L.M > 16 ? const_cast<uint8_t*>(dummy) : nullptr);
    const Kernel k = select_kernel(L2);
    if (k != K_GEMV_F32 && k != K_GEMM_F32X) return false;
  }
  return true;
}

int64_t f32split_xs_bytes(const Launch& L) { return x_bytes(L) + gu_bytes(L) + proj_ws_bytes(L); }

hipError_t launch_f32_split(const Launch& L, hipStream_t st) {
  uint8_t* w = static_cast<uint8_t*>(L.xs);
  float* g = reinterpret_cast<float*>(w + x_bytes(L));
  float* u = reinterpret_cast<float*>(w + x_bytes(L) + gu_bytes(L) / 2);
  auto out_of = [&](int p) { return L.op == OP_MLP ? static_cast<void*>(p == 0 ? g : u) : L.p[p].Y; };
  // below kGridRows rows: every projection on one float32 GEMV grid, when
  // they all fit it; up to 4 rows (one row chunk of the grid) the prologue runs on
  // the GEMV's staged rows, beyond that once per row in k_f32_prologue (each
  // row chunk's workgroups would otherwise all redo it)
  const bool fuse = L.M <= 4;
  bool act_done = false;
  Launch Lg = projection(L, 0, fuse || !has_prologue(L) ? L.A : w, out_of(0), nullptr);
  Lg.nproj = L.nproj;
  if (fuse) {
    Lg.skip = L.skip;
    Lg.gamma = L.gamma;
    Lg.residual = L.residual;
    Lg.eps = L.eps;
  }
  int with_zp = 0;
  for (int p = 0; p < L.nproj; ++p) {
    Lg.p[p] = L.p[p];
    Lg.p[p].Y = out_of(p);
    with_zp += L.p[p].zp != nullptr;
  }
  // one zero-point kind on the grid: all projections carry zero points or none
  Lg.zp_kind = with_zp ? L.zp_kind : ZP_NONE;
  bool one = L.M < kGridRows && L.M <= 16 && (with_zp == 0 || with_zp == L.nproj) && f32_fits(Lg) && fits_i32(Lg);
  for (int p = 0; p < L.nproj && one; ++p) one = select_kernel(projection(L, p, Lg.A, nullptr, nullptr)) == K_GEMV_F32;
  if (one) {
    if (!fuse && has_prologue(L)) {
      hipLaunchKernelGGL(k_f32_prologue, dim3(static_cast<uint32_t>(L.M)), dim3(256), 0, st,
                         static_cast<const float*>(L.A), static_cast<const float*>(L.skip),
                         static_cast<const float*>(L.gamma), static_cast<float*>(static_cast<void*>(w)),
                         static_cast<float*>(L.residual), static_cast<int>(L.K), L.eps);
      if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    hipError_t e;
    if (Lg.zp_kind == ZP_NONE) e = launch_f32_for<ZP_NONE>(Lg, st);
    else if (Lg.zp_kind == ZP_PACKED) e = launch_f32_for<ZP_PACKED>(Lg, st);
    else e = launch_f32_for<ZP_FLOAT>(Lg, st);
    if (e != hipSuccess) return e;
  } else {
    const void* x = L.A;
    if (has_prologue(L)) {
      float* xf = reinterpret_cast<float*>(w);
      hipLaunchKernelGGL(k_f32_prologue, dim3(static_cast<uint32_t>(L.M)), dim3(256), 0, st,
                         static_cast<const float*>(L.A), static_cast<const float*>(L.skip),
                         static_cast<const float*>(L.gamma), xf, static_cast<float*>(L.residual), static_cast<int>(L.K),
                         L.eps);
      if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
      x = xf;
    }
    void* pws = L.M >= kGridRows ? w + x_bytes(L) + gu_bytes(L) : nullptr;
    // all projections on one MFMA GEMM grid (one prepass of x) when each
    // takes the MFMA GEMM, else one launch per projection
    void* const ys[3] = {out_of(0), L.nproj > 1 ? out_of(1) : nullptr, L.nproj > 2 ? out_of(2) : nullptr};
    bool uz = true;
    const Launch Lm = projections(L, x, ys, pws, uz);
    const bool grid = pws != nullptr && uz && f32x_fits(Lm, kGridRows);
    // Mlp with split K and no float zero points (whose non-finite rows are
    // recomputed after the combine): the combine forms act(gate) * up
    act_done = grid && L.op == OP_MLP && Lm.zp_kind != ZP_FLOAT && f32x_splits(Lm) > 1;
    if (grid) {
      if (hipError_t e = launch_gemm_f32x(Lm, st, act_done ? static_cast<float*>(L.p[0].Y) : nullptr, L.act);
          e != hipSuccess)
        return e;
    } else {
      for (int p = 0; p < L.nproj; ++p)
        if (hipError_t e = launch(projection(L, p, x, out_of(p), pws), st); e != hipSuccess) return e;
    }
  }
  if (L.op == OP_MLP && !act_done) {
    const int64_t n = L.M * L.p[0].N;
    hipLaunchKernelGGL(k_mlp_act, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, st, g, u,
                       static_cast<float*>(L.p[0].Y), n, L.act);
  }
  return hipGetLastError();
}

}  // namespace xrmm
