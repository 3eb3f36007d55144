// MatMulNBits with float32 arithmetic on the matrix cores (the kernels are in
// xrmm_gemm_f32x.h): the geometry check, the K splits, the workspace layout
// and the launch.
#include "xrmm_gemm_f32x.h"

namespace xrmm {

namespace {

int64_t al256(int64_t b) { return (b + 255) / 256 * 256; }

// The workspace's first kFxKeep bytes are left alone: front ends share one
// workspace between this GEMM and the split-K GEMMs, whose arrival counters
// live there and must stay zero. Then, for float32 activations, the row
// exponents and the prepared binary16 terms (hi, lo); for float zero points
// the rows' block sums [kb][M] and their non-finite flags; then the split
// partials.
constexpr int64_t kFxKeep = 4096;

// K padded to whole K steps of 64 (blocks of 32 may leave half a step,
// which the kernel reads as a block past the last, of scale zero)
int64_t fx_kd(const Launch& L) { return (L.kb * L.block_size + fx::KS - 1) / fx::KS * fx::KS; }

int64_t fx_hl_bytes(const Launch& L) {
  return L.dtype == DT_F32 ? al256(L.M * 4) + 2 * al256(L.M * fx_kd(L) * 2) : 0;
}
int64_t fx_rs_bytes(const Launch& L) {
  return L.zp_kind == ZP_FLOAT ? al256(L.kb * L.M * 4) + al256(L.M * 4) : 0;
}
int64_t fx_prep_bytes(const Launch& L) { return fx_hl_bytes(L) + fx_rs_bytes(L); }

// columns and column tiles of all projections (Qkv / Mlp put theirs side by
// side on one grid)
int64_t fx_cols(const Launch& L) {
  int64_t n = 0;
  for (int p = 0; p < L.nproj; ++p) n += L.p[p].N;
  return n;
}
int64_t fx_ctiles(const Launch& L) {
  int64_t t = 0;
  for (int p = 0; p < L.nproj; ++p) t += (L.p[p].N + fx::CT - 1) / fx::CT;
  return t;
}

}  // namespace

// K splits when the tiles are fewer than 256 (one per CU), eight at most,
// each split at least 8 K steps of 64: float32 activations as many as keep
// the grid within 256 workgroups (a second round of a few workgroups costs
// a whole K pass: K = 4096, N = 14336 at 8 rows 44.0 us with 5 splits, 30.9
// with 4), float16 activations at least 256 workgroups (K = 5120,
// N = 17408 at 128 rows: 57.6 us with 2 splits, 61.9 with 1).
int f32x_splits(const Launch& L) {
  const int64_t tiles = ((L.M + fx::RT - 1) / fx::RT) * fx_ctiles(L);
  const int64_t ksteps = fx_kd(L) / fx::KS;
  int64_t s = L.dtype == DT_F32 ? (tiles < 256 ? 256 / tiles : 1) : (256 + tiles - 1) / tiles;
  if (s > 8) s = 8;
  if (s > ksteps / 8) s = ksteps / 8;
  return s < 1 ? 1 : static_cast<int>(s);
}

int64_t f32x_workspace_bytes(const Launch& L) {
  const int s = f32x_splits(L);
  return kFxKeep + fx_prep_bytes(L) + (s > 1 ? al256(int64_t(s) * L.M * fx_cols(L) * 4) : 0);
}

// MatMulNBits with at least `min_rows` rows (17 for one MatMulNBits): float32 activations with 2-, 4- or
// 8-bit codes (any K), float16 activations with 2- or 8-bit codes (4-bit with
// exact weights; K a multiple of 8, A 16-byte aligned); blocks of 32 or more
// codes (powers of two), packed, float
// (of the activations' type, blocks of 64 or more) or no zero points,
// 16-byte aligned B, 32-bit offsets; up to three projections of one A (the
// same zero-point kind, present on all or none). The caller supplies the
// workspace.
bool f32x_fits(const Launch& L, int64_t min_rows) {
  if (L.op != OP_MATMUL || L.M < min_rows || L.M < 1 || (L.bits != 2 && L.bits != 4 && L.bits != 8)) return false;
  if (L.nproj < 1 || L.nproj > 3) return false;
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (L.dtype == DT_F16) {
    if (L.bits == 4 && !L.exact_weights) return false;  // the binary16 GEMMs
    if (L.K % 8 != 0 || !al(L.A)) return false;
  } else if (L.dtype != DT_F32) {
    return false;
  }
  if (L.block_size < 32 || L.bs_log2 < 5) return false;
  if (L.zp_kind == ZP_FLOAT && (L.zp_dtype != L.dtype || L.block_size < 64)) return false;
  const int64_t lim = int64_t(1) << 31, rowb = fx_kd(L) * L.bits / 8;  // rows as read (past the last: zeros)
  for (int p = 0; p < L.nproj; ++p) {
    if (!al(L.p[p].B) || (L.zp_kind != ZP_NONE && L.p[p].zp == nullptr)) return false;
    if (L.p[p].N * rowb >= lim || L.p[p].N * L.kb >= lim) return false;
  }
  return L.M * fx_kd(L) * 4 < lim && L.M * L.K * 4 < lim && L.kb * L.M * 4 < lim &&
         int64_t(f32x_splits(L)) * L.M * fx_cols(L) < lim && L.M < lim / fx::RT;
}

hipError_t launch_gemm_f32x(const Launch& L, hipStream_t st, float* act_out, int act) {
  if (act_out && (L.nproj != 2 || L.p[0].N != L.p[1].N || L.zp_kind == ZP_FLOAT || f32x_splits(L) < 2))
    return hipErrorInvalidValue;
  fx::Args a{};
  a.Yact = act_out;
  a.act = act;
  a.A = L.A;
  a.np = L.nproj;
  int cb = 0, ct = 0;
  for (int p = 0; p < L.nproj; ++p) {
    fx::Proj1& q = a.pr[p];
    q.B = L.p[p].B;
    q.S = L.p[p].scales;
    q.Z = L.zp_kind == ZP_PACKED ? static_cast<const uint8_t*>(L.p[p].zp) : nullptr;
    q.Zf = L.zp_kind == ZP_FLOAT ? L.p[p].zp : nullptr;
    q.bias = L.p[p].bias;
    q.Y = L.p[p].Y;
    q.N = static_cast<int>(L.p[p].N);
    q.cb = cb;
    q.ct = ct;
    cb += q.N;
    ct += (q.N + fx::CT - 1) / fx::CT;
  }
  a.NT = cb;
  a.M = static_cast<int>(L.M);
  a.K = static_cast<int>(L.K);
  a.kb = static_cast<int>(L.kb);
  a.bs = static_cast<int>(L.block_size);
  a.Kd = static_cast<int>(fx_kd(L));
  a.rowb = static_cast<int>(L.kb * L.block_size * L.bits / 8);
  a.zrow = static_cast<int>(L.zrow);
  a.bits = L.bits;
  a.splits = f32x_splits(L);
  uint8_t* w = static_cast<uint8_t*>(L.ws) + kFxKeep;
  int32_t* ex = nullptr;
  f16 *hi = nullptr, *lo = nullptr;
  if (L.dtype == DT_F32) {
    ex = reinterpret_cast<int32_t*>(w);
    hi = reinterpret_cast<f16*>(w + al256(L.M * 4));
    lo = hi + al256(L.M * fx_kd(L) * 2) / 2;
  }
  float* rsum = nullptr;
  int32_t* bad = nullptr;
  if (L.zp_kind == ZP_FLOAT) {
    rsum = reinterpret_cast<float*>(w + fx_hl_bytes(L));
    bad = reinterpret_cast<int32_t*>(w + fx_hl_bytes(L) + al256(L.kb * L.M * 4));
  }
  a.ex = ex;
  a.Ahi = hi;
  a.Alo = lo;
  a.rsum = rsum;
  a.bad = bad;
  const int vecf = (L.K % 4 == 0 && (reinterpret_cast<uintptr_t>(L.A) & 15u) == 0) ? 1 : 0;
  const float* Af = static_cast<const float*>(L.A);
  const f16* Ah = static_cast<const f16*>(L.A);
  if (L.dtype == DT_F32 && rsum)
    fx::launch_prep<float, true, true>(Af, a.M, a.K, a.Kd, a.bs, a.kb, vecf, ex, hi, lo, rsum, bad, st);
  else if (L.dtype == DT_F32)
    fx::launch_prep<float, true, false>(Af, a.M, a.K, a.Kd, a.bs, a.kb, vecf, ex, hi, lo, rsum, bad, st);
  else if (rsum)  // float16: K % 8 == 0 and A 16-byte aligned
    fx::launch_prep<f16, false, true>(Ah, a.M, a.K, a.Kd, a.bs, a.kb, 1, ex, hi, lo, rsum, bad, st);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  a.part = reinterpret_cast<float*>(w + fx_prep_bytes(L));
  return L.dtype == DT_F32 ? fx::launch_gemm<float>(a, st) : fx::launch_gemm_f16(a, st);
}

}  // namespace xrmm
