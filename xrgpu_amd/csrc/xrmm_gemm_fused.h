// MatMulNBitsQkv / MatMulNBitsMlp for more than 16 rows (prefill): a 128 x 128
// LDS-tiled GEMM with the operators' prologue and epilogue fused (fp16
// activations, 4-bit weights, v_mfma_f32_32x32x16_f16, float32 accumulation).
//
// Tiles. Four waves (2 x 2) own 64 x 64 of a 128 x 128 tile, as 2 x 2 MFMA
// tiles of 32 x 32. Qkv lays the three projections' column tiles side by side
// on the grid (128 output columns each). Mlp covers 64 output columns per
// tile: the staged B tile holds gate columns 0..31, up columns 0..31, gate
// 32..63, up 32..63, so a wave's two MFMA column tiles are the gate and the up
// projection of the same 32 outputs and act(g) * u forms in registers.
//
// Prologue. packedInput (complex_kernel.glsl:81): r = A + skip, and with
// normScale x = r * inv * gamma, inv = 1 / sqrt(sum_k r^2 / K + eps) per row.
// The factor inv is common to the whole row, so it comes out of the sum: the
// tiles stage u = r * gamma (rounded once to binary16) and each thread adds
// r^2 of the pieces it stages; a workgroup streams all of K for its rows, so
// after the K loop it holds every row's sum of squares and scales the row's
// outputs by inv in the epilogue. The first column tile writes the residual
// (r rounded once). The binary16 stage limits |r * gamma| to 65504.
//
// Pipeline. K steps of 64; each thread's activations (+ skip, gamma), weight
// chunk and its raw scale / zero point are loaded into registers two steps
// ahead (two register sets alternate); weights are dequantised on the way into
// LDS (the routine and pair order of the other kernels: the staged weight is
// the reference's float32 weight rounded once to binary16).
#pragma once
#include "xrmm_device.h"

namespace xrmm {

constexpr int GF_BM = 128, GF_BN = 128, GF_BK = 64, GF_LDK = GF_BK + 8;

// Column tiles of one projection (Qkv: 128 outputs per tile; Mlp: 64).
__host__ __device__ inline int64_t gf_tiles(int op, int64_t n) { return op == OP_MLP ? (n + 63) / 64 : (n + 127) / 128; }

template <int ZPK, int SPC, int OPK>
__global__ __launch_bounds__(256) void k_gemm_fused(Launch L) {
  static_assert(OPK == OP_QKV || OPK == OP_MLP, "fused operators");
  constexpr bool MLP = OPK == OP_MLP;
  __shared__ __align__(16) f16 As[GF_BM * GF_LDK];
  __shared__ __align__(16) f16 Bs[GF_BN * GF_LDK];
  __shared__ float rowinv[GF_BM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t M = L.M, K = L.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * GF_BM;
  const bool skip = L.skip != nullptr, norm = L.gamma != nullptr;

  // this tile's projection and first output column
  int pi = 0;
  int64_t n0 = static_cast<int64_t>(blockIdx.x) * (MLP ? 64 : 128);
  if constexpr (!MLP) {
    const int64_t t0 = gf_tiles(OPK, L.p[0].N), t1 = gf_tiles(OPK, L.p[1].N);
    const int64_t t = blockIdx.x;
    pi = t < t0 ? 0 : t < t0 + t1 ? 1 : 2;
    n0 = (t - (pi == 0 ? 0 : pi == 1 ? t0 : t0 + t1)) * 128;
  }
  const Proj& P = L.p[pi];
  const int64_t N = P.N;
  const int64_t Kp = L.kb * L.block_size;
  const int64_t row_bytes = Kp / 2, nchunk = row_bytes / 16;
  const int64_t ktiles = (Kp + GF_BK - 1) / GF_BK;
  const f16* A = static_cast<const f16*>(L.A);
  const f16* S = static_cast<const f16*>(L.skip);
  const f16* G = static_cast<const f16*>(L.gamma);

  // B staging: thread t stages half t % 2 of LDS column t / 2. Qkv: column
  // n0 + t / 2 of the projection; Mlp: gate (b / 32 even) or up of output
  // n0 + 32 (b / 64) + b % 32.
  const int bcol = tid >> 1, bh = tid & 1;
  const Proj& PB = MLP ? L.p[(bcol >> 5) & 1] : P;
  const int64_t bn = MLP ? n0 + 32 * (bcol >> 6) + (bcol & 31) : n0 + bcol;
  const bool bnval = bn < N;
  const uint8_t* Bcol = PB.B + (bnval ? bn : 0) * row_bytes;

  // activation staging: thread t stages pieces t + 256 i (row (t >> 3) + 32 i,
  // k group t & 7): the same k group for all four, so one gamma load per step.
  // Registers of one step, loaded two steps ahead.
  const int grp = tid & 7;
  struct Regs {
    f16x8 a[4], s[4], g;
    u32x4 b;
    RawMeta<SPC> m;
  };
  float sq[4] = {0.f, 0.f, 0.f, 0.f};
  auto gload = [&](Regs& r, int64_t kt) {
    const int64_t k = kt * GF_BK + grp * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = m0 + (tid >> 3) + 32 * i;
      const bool ok = m < M && k < K;  // K % 8 == 0: groups are whole
      r.a[i] = ok ? __builtin_bit_cast(f16x8, ld16(A + m * K + k)) : f16x8{};
      r.s[i] = (ok && skip) ? __builtin_bit_cast(f16x8, ld16(S + m * K + k)) : f16x8{};
    }
    r.g = (norm && k < K) ? __builtin_bit_cast(f16x8, ld16(G + k)) : f16x8{};
    const int64_t ch = kt * 2 + bh;
    const bool bok = bnval && ch < nchunk;
    r.b = bok ? ld16(Bcol + ch * 16) : u32x4{0u, 0u, 0u, 0u};
    r.m = ld_meta_raw<ZPK, SPC>(L, PB, bn, ch, bok);
  };
  f16* res = static_cast<f16*>(L.residual);
  const bool write_res = res != nullptr && blockIdx.x == 0;
  auto sstore = [&](const Regs& rg, int64_t kt) {
    const int64_t k = kt * GF_BK + grp * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (tid >> 3) + 32 * i;
      f16x8 u, r16;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float r = skip ? __fadd_rn(static_cast<float>(rg.a[i][e]), static_cast<float>(rg.s[i][e]))
                             : static_cast<float>(rg.a[i][e]);
        sq[i] = __builtin_fmaf(r, r, sq[i]);
        u[e] = static_cast<f16>(norm ? r * static_cast<float>(rg.g[e]) : r);
        r16[e] = static_cast<f16>(r);
      }
      *reinterpret_cast<f16x8*>(As + row * GF_LDK + grp * 8) = pair_order(u);
      const int64_t m = m0 + row;
      if (write_res && m < M && k < K) *reinterpret_cast<f16x8*>(res + m * K + k) = r16;
    }
    const int64_t ch = kt * 2 + bh;
    f16x8 b[4];
    dq_regs<ZPK, SPC>(rg.b, meta_of<ZPK, SPC>(L, rg.m, ch, bnval && ch < nchunk), b);
#pragma unroll
    for (int d = 0; d < 4; ++d) *reinterpret_cast<f16x8*>(Bs + bcol * GF_LDK + bh * 32 + d * 8) = b[d];
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // One K step: stage the registers of step kt, refill them with step kt + 2
  // (loads past the last step return zeros), multiply.
  auto step = [&](Regs& r, int64_t kt) {
    __syncthreads();
    sstore(r, kt);
    __syncthreads();
    gload(r, kt + 2);
#pragma unroll
    for (int kk = 0; kk < GF_BK / 16; ++kk) {
      f16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const f16x8*>(As + (wm * 64 + i * 32 + (lane & 31)) * GF_LDK + kk * 16 + (lane >> 5) * 8);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const f16x8*>(Bs + (wn * 64 + j * 32 + (lane & 31)) * GF_LDK + kk * 16 + (lane >> 5) * 8);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };
  Regs r0, r1;
  gload(r0, 0);
  gload(r1, 1);
  int64_t kt = 0;
  for (; kt + 1 < ktiles; kt += 2) {
    step(r0, kt);
    step(r1, kt + 1);
  }
  if (kt < ktiles) step(r0, kt);

  // rows' sums of squares: the eight threads of a row (consecutive lanes) add
  // their partials
  if (norm) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = sq[i];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      if (grp == 0) rowinv[(tid >> 3) + 32 * i] = __builtin_amdgcn_rsqf(v / static_cast<float>(K) + L.eps);
    }
  }
  __syncthreads();

  // epilogue: lane holds D[8 (r / 4) + 4 (lane / 32) + r % 4][lane % 32] of each
  // 32 x 32 tile
  f16* Y = static_cast<f16*>(P.Y);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      const int64_t m = m0 + row;
      if (m >= M) continue;
      const float inv = norm ? rowinv[row] : 1.f;
      if constexpr (MLP) {
        const int64_t n = n0 + wn * 32 + (lane & 31);
        if (n >= N) continue;
        const float gb = L.p[0].bias ? static_cast<float>(static_cast<const f16*>(L.p[0].bias)[n]) : 0.f;
        const float ub = L.p[1].bias ? static_cast<float>(static_cast<const f16*>(L.p[1].bias)[n]) : 0.f;
        const float g = __builtin_fmaf(acc[i][0][r], inv, gb), u = __builtin_fmaf(acc[i][1][r], inv, ub);
        Y[m * N + n] = static_cast<f16>(activate(g, L.act) * u);
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
          if (n < N) Y[m * N + n] = static_cast<f16>(acc[i][j][r] * inv);
        }
      }
    }
  }
}

template <int ZPK, int SPC, int OPK>
inline hipError_t launch_gemm_fused3(const Launch& L, hipStream_t st) {
  int64_t cols = 0;
  for (int i = 0; i < (OPK == OP_MLP ? 1 : 3); ++i) cols += gf_tiles(OPK, L.p[i].N);
  const int64_t rows = (L.M + GF_BM - 1) / GF_BM;
  if (cols > 0x7FFFFFFF || rows > 65535) return hipErrorInvalidValue;  // launch limits
  hipLaunchKernelGGL((k_gemm_fused<ZPK, SPC, OPK>), dim3(static_cast<uint32_t>(cols), static_cast<uint32_t>(rows)),
                     dim3(256), 0, st, L);
  return hipGetLastError();
}

template <int ZPK>
inline hipError_t launch_gemm_fused2(const Launch& L, hipStream_t st) {
  const bool one = L.block_size >= 32;  // whole 32-code blocks per chunk half
  if (L.op == OP_MLP)
    return one ? launch_gemm_fused3<ZPK, 1, OP_MLP>(L, st) : launch_gemm_fused3<ZPK, 2, OP_MLP>(L, st);
  return one ? launch_gemm_fused3<ZPK, 1, OP_QKV>(L, st) : launch_gemm_fused3<ZPK, 2, OP_QKV>(L, st);
}

// Entry of one zero-point kind (defined in xrmm_gemm_fused_zp.hip).
template <int ZPK>
hipError_t launch_gemm_fused_for(const Launch& L, hipStream_t st);

}  // namespace xrmm
