// HIP kernels of libxrmm for gfx950 (MI355X): MatMulNBits, MatMulNBitsQkv and
// MatMulNBitsMlp.
//
// The arithmetic follows xrGPU's serial shader
// (kernels/_shared/extended/shaders/complex_kernel.glsl:80 nbitWeight,
// :81 packedInput, :83 packedMatmul, :39-47 fused/logistic); the work
// decomposition is this file's own:
//
//  * k_gemv_q4   M <= 16, fp16, 4-bit. One workgroup owns a 16-column tile;
//                its waves split K. Packed weights stream with 16-byte loads,
//                are dequantised in registers to fp16 and multiplied on
//                v_mfma_f32_16x16x32_f16 against the activations staged once
//                in LDS. Qkv/Mlp fuse the RMS prologue and the SwiGLU epilogue.
//  * k_gemv_dot / k_gemv_sk / k_gemv_mq / k_gemv_f32 (xrmm_gemv_*.h): the
//                decode GEMVs (v_dot2 on block sums, split-K MFMA, four-row
//                MFMA for Qkv, float32 activations).
//  * k_gemm_q4   MatMulNBits, 16 < M, fp16, 4-bit, while 256 x 256 tiles would
//                not fill the chip. LDS-tiled MFMA GEMM with 128 x 128 tiles:
//                activation tiles and weight tiles dequantised to fp16 are
//                staged in LDS and fed to v_mfma_f32_32x32x16_f16.
//  * k_gemm_fused  Qkv / Mlp, 16 < M (xrmm_gemm_fused.h): the same tiling with
//                the RMS prologue, residual and SwiGLU epilogue fused.
//  * k_gemm_q4_big  M >= 128, fp16, 4-bit (xrmm_gemm.h): 256 x 256 tiles on
//                eight waves, dequantisation interleaved with the MFMAs.
//  * k_generic   every other geometry (fp32, 2/8-bit, float zero points with a
//                non-fast block size, unaligned tensors): one wave per column
//                and row block, the reference's float32 weight formula.
//
// Dequantisation (4-bit, integer zero point): code - z is exact in binary16
// and (code - z) * scale is rounded once, so the staged fp16 weight equals the
// reference's float32 weight rounded once to binary16. Codes are widened with
// the exponent-bias trick: OR-ing a nibble into the mantissa of 1024.0h gives
// 1024 + code exactly (and 1024 + 16*code for the high nibble of a byte).
#include <atomic>
#include <cstdlib>

#include "xrmm_gemv.h"
#include "xrmm_gemv_dot.h"
#include "xrmm_gemv_mq.h"
#include "xrmm_gemv_f32.h"
#include "xrmm_gemv_sk.h"
#include "xrmm_gemm.h"
#include "xrmm_gemm_fused.h"
#include "xrmm_gemm_thin.h"

namespace xrmm {

// ---------------------------------------------------------------------------
// generic kernel: one wave per (column, block of MB rows)

template <int MB>
__global__ __launch_bounds__(64) void k_generic(Launch L) {
  const int lane = threadIdx.x;
  int64_t col = blockIdx.x;
  int pi = 0;
  if (L.op == OP_QKV) {
    if (col >= L.p[0].N) {
      col -= L.p[0].N;
      pi = 1;
      if (col >= L.p[1].N) {
        col -= L.p[1].N;
        pi = 2;
      }
    }
  }
  const Proj& P = L.p[pi];
  const int64_t M = L.M, K = L.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * MB;
  const bool norm = L.op != OP_MATMUL;

  auto raw = [&](int64_t m, int64_t k) -> float {
    float x = ld_t(L.A, m * K + k, L.dtype);
    if (norm && L.skip) x = __fadd_rn(x, ld_t(L.skip, m * K + k, L.dtype));
    return x;
  };

  float inv[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    inv[i] = 1.f;
    const int64_t m = m0 + i;
    if (norm && L.gamma && m < M) {
      float s = 0.f;
      for (int64_t k = lane; k < K; k += 64) {
        const float r = raw(m, k);
        s += r * r;
      }
      s = wave_sum(s);
      inv[i] = 1.f / sqrtf(s / static_cast<float>(K) + L.eps);
    }
  }
  if (norm && L.residual && blockIdx.x == 0) {
    for (int i = 0; i < MB; ++i) {
      const int64_t m = m0 + i;
      if (m >= M) break;
      for (int64_t k = lane; k < K; k += 64) st_t(L.residual, m * K + k, raw(m, k), L.dtype);
    }
  }

  float acc[MB], acc2[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = acc2[i] = 0.f;
  for (int64_t k = lane; k < K; k += 64) {
    const float w = weight_f32(L, P, col, k);
    const float wu = L.op == OP_MLP ? weight_f32(L, L.p[1], col, k) : 0.f;
    const float gk = (norm && L.gamma) ? ld_t(L.gamma, k, L.dtype) : 1.f;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int64_t m = m0 + i;
      if (m < M) {
        float x = raw(m, k);
        if (norm && L.gamma) x = x * (inv[i] * gk);
        acc[i] += x * w;
        acc2[i] += x * wu;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    acc[i] = wave_sum(acc[i]);
    if (L.op == OP_MLP) acc2[i] = wave_sum(acc2[i]);
  }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int64_t m = m0 + i;
      if (m >= M) break;
      float y = acc[i];
      if (L.op == OP_MATMUL) {
        if (P.bias) y += ld_t(P.bias, col, L.dtype);
      } else if (L.op == OP_MLP) {
        const float gb = P.bias ? ld_t(P.bias, col, L.dtype) : 0.f;
        const float ub = L.p[1].bias ? ld_t(L.p[1].bias, col, L.dtype) : 0.f;
        y = activate(y + gb, L.act) * (acc2[i] + ub);
      }
      st_t(P.Y, m * P.N + col, y, L.dtype);
    }
  }
}

// ---------------------------------------------------------------------------
// GEMM for M > 16: fp16 activations, 4-bit weights, MFMA 32x32x16

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64, GM_LDK = GM_BK + 8;
// Split-K workspace layout: a fixed block of per-tile arrival counters (the
// same place for every geometry, so workspaces can be shared between calls of
// different shapes), then the float32 partial tiles.
constexpr uint32_t kGemmCounterBytes = 4096;

// KG groups of four waves split the K steps (step kt goes to group kt % KG):
// with few output tiles (N / 128 x M / 128 workgroups against 256 CUs) one
// group's serial K loop is the critical path, and a second group halves it
// and fills a second wave per SIMD. The groups' partial tiles meet in LDS.
template <int ZPK, int SPC, int KG>
__global__ __launch_bounds__(256 * KG) void k_gemm_q4(Launch L) {
  static_assert(KG == 1 || KG == 2, "K groups");
  // one array for every group's A and B stage, so the reduction of the
  // groups' partial tiles can reuse it as one contiguous block
  __shared__ __align__(16) f16 stages[KG][(GM_BM + GM_BN) * GM_LDK];
  const int tid_all = threadIdx.x, kg = tid_all >> 8, tid = tid_all & 255;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  f16* As = stages[kg];
  f16* Bs = stages[kg] + GM_BM * GM_LDK;
  const Proj& P = L.p[0];
  const int64_t M = L.M, N = P.N, K = L.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * GM_BM, n0 = static_cast<int64_t>(blockIdx.x) * GM_BN;
  const int64_t Kp = L.kb * L.block_size;
  const int64_t row_bytes = Kp / 2, nchunk = row_bytes / 16;
  const int64_t ktiles = (Kp + GM_BK - 1) / GM_BK;
  const f16* A = static_cast<const f16*>(L.A);

  // global -> register staging, two of the group's steps ahead: each
  // thread's four 16-byte activation pieces, one weight chunk and its raw
  // scale / zero point
  struct Regs {
    f16x8 a[4];
    u32x4 b;
    RawMeta<SPC> m;
  };
  // Loads go through buffer resources with 32-bit offsets: an offset past the
  // bound reads zero, so rows past M, k past K and columns past N need no
  // branch around the load (a divergent select became one, and every later
  // wait a full drain). The fast path guarantees 32-bit index ranges.
  constexpr uint32_t OOB = 0x80000000u;
  const int bcol = tid >> 1, bh = tid & 1;
  const int64_t bn = n0 + bcol;
  const bool bnval = bn < N;
  const uint32_t K32 = static_cast<uint32_t>(K), kb = static_cast<uint32_t>(L.kb);
  const rsrc_t rA = mk_rsrc(A, static_cast<uint32_t>(M) * K32 * 2u);
  const rsrc_t rB = mk_rsrc(P.B, static_cast<uint32_t>(N) * static_cast<uint32_t>(row_bytes));
  const uint32_t zrow = ZPK == ZP_PACKED ? static_cast<uint32_t>(L.zrow) : kb * (L.zp_dtype == DT_F32 ? 4u : 2u);
  // scale / zero-point bounds rounded to 16 bytes (16-byte aligned tensors keep
  // the rounded bound inside the block holding their last byte)
  const rsrc_t rS = mk_rsrc(P.scales, (static_cast<uint32_t>(N) * kb * 2u + 15u) & ~15u);
  const rsrc_t rZ = mk_rsrc(P.zp ? P.zp : P.scales, (static_cast<uint32_t>(N) * zrow + 15u) & ~15u);
  const uint32_t bcol_off = bnval ? static_cast<uint32_t>(bn) * static_cast<uint32_t>(row_bytes) : OOB;
  const uint32_t scol = bnval ? static_cast<uint32_t>(bn) * kb * 2u : OOB;
  const uint32_t zcol = bnval ? static_cast<uint32_t>(bn) * zrow : OOB;
  uint32_t aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i, row = idx >> 3, grp = idx & 7;
    const int64_t m = m0 + row;
    aoff[i] = m < M ? (static_cast<uint32_t>(m) * K32 + static_cast<uint32_t>(grp) * 8u) * 2u : OOB;
  }

  // this workgroup's K steps: split blockIdx.z of L.splits (loads past the
  // split's last step return zeros, like those past the row's end)
  const int64_t kps = (ktiles + L.splits - 1) / L.splits;
  const int64_t kbeg = static_cast<int64_t>(blockIdx.z) * kps;
  const int64_t kend = kbeg + kps < ktiles ? kbeg + kps : ktiles;
  auto gload = [&](Regs& r, int64_t kt) {
    const uint32_t k = static_cast<uint32_t>(kt) * GM_BK + static_cast<uint32_t>(tid & 7) * 8u;
    const uint32_t kpast = (k < K32 && kt < kend) ? 0u : OOB;  // K % 8 == 0: groups are whole
#pragma unroll
    for (int i = 0; i < 4; ++i)
      r.a[i] = __builtin_bit_cast(f16x8, bld16(rA, (aoff[i] | kpast) + static_cast<uint32_t>(kt) * (GM_BK * 2), 0));
    const uint32_t ch = static_cast<uint32_t>(kt) * 2u + static_cast<uint32_t>(bh);
    const uint32_t past = (ch < static_cast<uint32_t>(nchunk) && kt < kend) ? 0u : OOB;
    r.b = bld16(rB, (bcol_off | past) + ch * 16u, 0);
#pragma unroll
    for (int q = 0; q < SPC; ++q) {
      const uint32_t b = (ch * 32u + q * 16u) >> L.bs_log2;  // block of this half-chunk
      r.m.s[q] = bld_u16(rS, (scol | past) + b * 2u, 0);
      r.m.z[q] = 0u;
      if constexpr (ZPK == ZP_PACKED) r.m.z[q] = bld_u8(rZ, (zcol | past) + (b >> 1), 0);
      else if constexpr (ZPK == ZP_FLOAT)
        r.m.z[q] = L.zp_dtype == DT_F32 ? bld_u32(rZ, (zcol | past) + b * 4u, 0) : bld_u16(rZ, (zcol | past) + b * 2u, 0);
    }
  };
  auto sstore = [&](const Regs& r, int64_t kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i, row = idx >> 3, grp = idx & 7;
      *reinterpret_cast<f16x8*>(As + row * GM_LDK + grp * 8) = pair_order(r.a[i]);
    }
    const int64_t ch = kt * 2 + bh;
    f16x8 b[4];
    dq_regs<ZPK, SPC>(r.b, meta_of<ZPK, SPC>(L, r.m, ch, bnval && ch < nchunk), b);
#pragma unroll
    for (int d = 0; d < 4; ++d) *reinterpret_cast<f16x8*>(Bs + bcol * GM_LDK + bh * 32 + d * 8) = b[d];
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // One K step of the group: stage the registers of step kt, refill them
  // with the group's step after next (loads past the last step return
  // zeros), multiply. Every group runs the same number of steps (a step past
  // the end stages zeros), so the workgroup barriers pair up.
  // fragments of K slice kk (0..3): lane (r, g) = (lane % 32, lane / 32)
  // reads row / column r, k = 16 kk + 8 g .. + 7; the next slice's are read
  // before the current slice's MFMAs, so the LDS latency hides behind them
  f16x8 fa[2][2], fb[2][2];
  auto read_frags = [&](int kk, int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      fa[buf][i] = *reinterpret_cast<const f16x8*>(As + (wm * 64 + i * 32 + (lane & 31)) * GM_LDK + kk * 16 + (lane >> 5) * 8);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      fb[buf][j] = *reinterpret_cast<const f16x8*>(Bs + (wn * 64 + j * 32 + (lane & 31)) * GM_LDK + kk * 16 + (lane >> 5) * 8);
  };
  auto step = [&](Regs& r, int64_t kt) {
    __syncthreads();
    sstore(r, kt);
    __syncthreads();
    read_frags(0, 0);
    gload(r, kt + 2 * KG);
#pragma unroll
    for (int kk = 0; kk < GM_BK / 16; ++kk) {
      if (kk + 1 < GM_BK / 16) read_frags(kk + 1, (kk + 1) & 1);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk & 1][i], fb[kk & 1][j], acc[i][j], 0, 0, 0);
    }
  };
  const int64_t gsteps = (kend - kbeg + KG - 1) / KG;  // steps per group
  Regs r0, r1;
  gload(r0, kbeg + kg);
  gload(r1, kbeg + kg + KG);
  int64_t i = 0;
  for (; i + 1 < gsteps; i += 2) {
    step(r0, kbeg + i * KG + kg);
    step(r1, kbeg + (i + 1) * KG + kg);
  }
  if (i < gsteps) step(r0, kbeg + i * KG + kg);

  if constexpr (KG == 2) {
    // group 1's partial tiles through LDS (the stages are free now) to group 0
    float* red = reinterpret_cast<float*>(&stages[0][0]);
    static_assert(sizeof(stages) >= 256 * 64 * sizeof(float), "the partial tiles fit the stages");
    __syncthreads();
    if (kg == 1) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) red[((ii * 2 + j) * 16 + r) * 256 + tid] = acc[ii][j][r];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[ii][j][r] += red[((ii * 2 + j) * 16 + r) * 256 + tid];
    }
  }
  // from here on group 0 holds the tile; group 1 stays for the barriers only

  if (L.splits > 1) {
    // Split-K: every split's partial tile goes to the workspace with 16-byte
    // system-coherent stores (sc0 sc1: written through past the per-XCD L2s);
    // each thread waits for its stores, the barrier orders them before thread
    // 0's arrival count, and the last split of the tile reads all the partials
    // back with system-coherent loads (they follow its count through s_last)
    // and adds them in split order, so the result does not depend on which
    // split arrives last. It then clears the tile's counter, leaving the
    // workspace as it found it. The count stays relaxed: an acquire-release
    // count would write back and invalidate the whole L2 around it in every
    // workgroup, for stores that are not in L2.
    constexpr int COHERENT = 1 | 16;  // sc0 | sc1
    __shared__ int s_last;
    const uint32_t tiles = gridDim.x * gridDim.y;
    const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x;
    uint32_t* cnt = static_cast<uint32_t*>(L.ws);
    const uint32_t pbase = kGemmCounterBytes;  // the partial tiles follow the counter block
    const uint32_t tile_bytes = 256u * 64u * 4u;
    const rsrc_t rW = mk_rsrc(static_cast<uint8_t*>(L.ws) + pbase, tiles * static_cast<uint32_t>(L.splits) * tile_bytes);
    // thread tid's 16 float4 of a partial: piece (i j q) at ((i 2 + j) 4 + q) 256 + tid.
    // A piece holds rows m0 + wm 64 + i 32 + 8 q + 4 (lane / 32) + 0..3 of one
    // column; pieces whose rows all lie past M are neither stored nor read
    // (their offset is past the resource: the store is dropped, the load
    // returns zero), so a tile with few rows moves only the rows it has.
    const int64_t prow = m0 + wm * 64 + 4 * (lane >> 5);
    auto poff = [&](uint32_t sp, int piece) {
      const int ii = piece >> 3, q = piece & 3;
      if (prow + ii * 32 + 8 * q >= M) return 0x80000000u;
      return (tile * static_cast<uint32_t>(L.splits) + sp) * tile_bytes + (static_cast<uint32_t>(piece) * 256u + tid) * 16u;
    };
    if (kg == 0) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 v = {acc[ii][j][4 * q], acc[ii][j][4 * q + 1], acc[ii][j][4 * q + 2], acc[ii][j][4 * q + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rW, poff(blockIdx.z, (ii * 2 + j) * 4 + q),
                                                   0, COHERENT);
          }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid_all == 0)
      s_last = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               static_cast<uint32_t>(L.splits - 1);
    __syncthreads();
    if (!s_last || kg != 0) return;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[ii][j][r] = 0.f;
    for (int sp = 0; sp < L.splits; ++sp) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 v = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rW, poff(static_cast<uint32_t>(sp), (ii * 2 + j) * 4 + q), 0,
                                                             COHERENT));
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[ii][j][4 * q + e] += v[e];
          }
    }
    if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (kg != 0) return;

  // epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each 32x32 tile
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
    if (n >= N) continue;
    const float bias = P.bias ? static_cast<float>(static_cast<const f16*>(P.bias)[n]) : 0.f;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * 64 + ii * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < M) static_cast<f16*>(P.Y)[m * N + n] = static_cast<f16>(acc[ii][j][r] + bias);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Qkv / Mlp prefill prologue: packedInput (complex_kernel.glsl:81) once per
// row, for the GEMMs that read the normalised activations from L.xs.
// r = A + skip in float32; with normScale, inv = 1 / sqrt(sum_k r^2 / K + eps)
// and x = r * (gamma * inv), without it x = r; x is rounded once to binary16
// after the normalisation, so it stays in range wherever the normalised value
// does (|r * gamma| itself may exceed 65504). The residual output receives r
// rounded once. One workgroup per row, 16-byte pieces (K % 8 == 0 and 16-byte
// aligned tensors: the fast path's conditions). P > 0: each thread holds its
// P pieces of the row (and of gamma) in registers, all loaded at once (rows
// up to 256 x 8 x P); P = 0: two passes, the second finding its pieces in
// the L1 / L2.
template <int P>
__global__ __launch_bounds__(256) void k_rms_rows(Launch L) {
  const int tid = threadIdx.x;
  const int64_t m = blockIdx.x, K = L.K;
  const f16* A = static_cast<const f16*>(L.A) + m * K;
  const f16* S = L.skip ? static_cast<const f16*>(L.skip) + m * K : nullptr;
  const f16* G = static_cast<const f16*>(L.gamma);
  f16* X = static_cast<f16*>(L.xs) + m * K;
  f16* R = L.residual ? static_cast<f16*>(L.residual) + m * K : nullptr;
  auto row = [&](const f16x8& a, const f16x8& sk, float r[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      r[e] = S ? __fadd_rn(static_cast<float>(a[e]), static_cast<float>(sk[e])) : static_cast<float>(a[e]);
  };
  auto finish = [&](int64_t k, const float r[8], const f16x8& g, float inv) {
    f16x8 x, r16;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = static_cast<f16>(G ? r[e] * __builtin_fmaf(static_cast<float>(g[e]), inv, 0.f) : r[e]);
      r16[e] = static_cast<f16>(r[e]);
    }
    *reinterpret_cast<f16x8*>(X + k) = x;
    if (R) *reinterpret_cast<f16x8*>(R + k) = r16;
  };
  __shared__ float red[4];
  auto row_inv = [&](float sq) {
    for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = sq;
    __syncthreads();
    return __builtin_amdgcn_rsqf(((red[0] + red[1]) + (red[2] + red[3])) / static_cast<float>(K) + L.eps);
  };
  if constexpr (P > 0) {
    // the row's pieces (and gamma's) held in registers: one pass over memory,
    // every load issued before the first use
    f16x8 a[P], sk[P], g[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t k = (int64_t(tid) + 256 * p) * 8;
      const bool ok = k < K;
      a[p] = ok ? __builtin_bit_cast(f16x8, ld16(A + k)) : f16x8{};
      sk[p] = ok && S ? __builtin_bit_cast(f16x8, ld16(S + k)) : f16x8{};
      g[p] = ok && G ? __builtin_bit_cast(f16x8, ld16(G + k)) : f16x8{};
    }
    float inv = 1.f;
    if (G) {
      float sq = 0.f;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        float r[8];
        row(a[p], sk[p], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) sq = __builtin_fmaf(r[e], r[e], sq);  // zero past K
      }
      inv = row_inv(sq);
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t k = (int64_t(tid) + 256 * p) * 8;
      if (k >= K) break;
      float r[8];
      row(a[p], sk[p], r);
      finish(k, r, g[p], inv);
    }
  } else {
    // long rows: two passes, the second finds its pieces in the L1 / L2
    auto load_row = [&](int64_t k, float r[8]) {
      const f16x8 a = __builtin_bit_cast(f16x8, ld16(A + k));
      const f16x8 sk = S ? __builtin_bit_cast(f16x8, ld16(S + k)) : f16x8{};
      row(a, sk, r);
    };
    float inv = 1.f;
    if (G) {
      float sq = 0.f;
      for (int64_t k = int64_t(tid) * 8; k < K; k += 256 * 8) {
        float r[8];
        load_row(k, r);
#pragma unroll
        for (int e = 0; e < 8; ++e) sq = __builtin_fmaf(r[e], r[e], sq);
      }
      inv = row_inv(sq);
    }
    for (int64_t k = int64_t(tid) * 8; k < K; k += 256 * 8) {
      float r[8];
      load_row(k, r);
      const f16x8 g = G ? __builtin_bit_cast(f16x8, ld16(G + k)) : f16x8{};
      finish(k, r, g, inv);
    }
  }
}

// The prologue, then the operator's GEMM description on its output: A is the
// normalised binary16 rows, with no skip, normScale or residual left to do.
static hipError_t run_prologue(const Launch& L, Launch& Lx, hipStream_t st) {
  if (L.M > 0x7FFFFFFF) return hipErrorInvalidValue;  // launch limit
  // pieces of 8 per thread: rows up to 16384 held in registers
  const int64_t pieces = (L.K / 8 + 255) / 256;
  auto kern = pieces <= 1 ? k_rms_rows<1> : pieces <= 2 ? k_rms_rows<2> : pieces <= 4 ? k_rms_rows<4>
            : pieces <= 8 ? k_rms_rows<8> : k_rms_rows<0>;
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(L.M)), dim3(256), 0, st, L);
  Lx = L;
  Lx.A = L.xs;
  Lx.skip = nullptr;
  Lx.gamma = nullptr;
  Lx.residual = nullptr;
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// dequantisation kernel (xrmm_dequantize)

template <int ZPK, int SPC>
__global__ __launch_bounds__(256) void k_dequant_q4_f16(Launch L, f16* W) {
  // one thread per 16-byte chunk: 32 codes of one column
  const Proj& P = L.p[0];
  const int64_t row_bytes = L.kb * L.blob, nchunk = row_bytes / 16;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= P.N * nchunk) return;
  const int64_t n = gid / nchunk, ch = gid - n * nchunk;
  const u32x4 w = ld16(P.B + n * row_bytes + ch * 16);
  f16x8 b[4];
  dq_chunk<ZPK, SPC>(L, P, n, ch, true, w, b);
  const int order[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
  for (int d = 0; d < 4; ++d)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = ch * 32 + d * 8 + order[i];
      if (k < L.K) W[n * L.K + k] = b[d][i];
    }
}

__global__ __launch_bounds__(256) void k_dequant_f32(Launch L, void* W, int out_dtype) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= L.p[0].N * L.K) return;
  const int64_t n = gid / L.K, k = gid - n * L.K;
  st_t(W, gid, weight_f32(L, L.p[0], n, k), out_dtype);
}

// ---------------------------------------------------------------------------
// dispatch

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }


// fp16, 4-bit, blocks of whole 16-code halves, rows of whole 16-byte chunks,
// K a multiple of 8 and 16-byte aligned tensors.
static bool q4_fast_ok(const Launch& L) {
  if (L.dtype != DT_F16 || L.bits != 4) return false;
  if (L.bs_log2 < 4) return false;  // power-of-two block_size >= 16
  const int64_t Kp = L.kb * L.block_size;
  if (Kp % 32 != 0 || L.K % 8 != 0) return false;
  if (!aligned16(L.A) || !aligned16(L.skip) || !aligned16(L.gamma) || !aligned16(L.residual)) return false;
  for (int i = 0; i < L.nproj; ++i) {
    if (!aligned16(L.p[i].B) || !aligned16(L.p[i].scales) || !aligned16(L.p[i].zp)) return false;
    if (L.zp_kind == ZP_FLOAT && L.p[i].zp == nullptr) return false;
  }
  return true;
}

int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// From this many rows the 256 x 256 GEMM wastes less on partial row tiles than
// the 128 x 128 one loses to its lower MFMA rate.
constexpr int64_t kGemmBigMinM = 128;

// ...and only with enough 256 x 256 tiles to occupy half of the 256 CUs (one
// workgroup per CU): with fewer, the 128 x 128 GEMM's four times as many tiles
// win (M=1024 K=14336 N=4096, 64 tiles: 245 against 321 us; M=256 K=4096
// N=14336, 56 tiles: 75 against 96 us; at 112 and 128 tiles the two tie; at
// 448 tiles the big GEMM takes 256 against 367 us). The environment variable
// XRMM_GEMM_BIG_MIN_TILES overrides the threshold (0: the big GEMM from
// kGemmBigMinM rows on). Every zero-point kind follows the same rule.
constexpr int64_t kGemmBigMinTiles = 128;

static int64_t gemm_big_min_tiles() {
  const char* e = std::getenv("XRMM_GEMM_BIG_MIN_TILES");
  if (e != nullptr && *e != 0) {
    char* end = nullptr;
    const long long v = std::strtoll(e, &end, 10);
    if (end != nullptr && *end == 0 && v >= 0) return v;
  }
  return kGemmBigMinTiles;
}

static bool gemm_big_fills(const Launch& L) {
  const int64_t tiles = (L.M + GB_M - 1) / GB_M * ((L.p[0].N + 255) / 256);
  return tiles >= gemm_big_min_tiles();
}

// The same rule for the Qkv / Mlp grid of the 256 x 256 pipeline.
static bool gemm_big_fused_fills(const Launch& L) {
  uint32_t t0, t1, nc;
  gemm_fused_tiles(L, t0, t1, nc);
  return (L.M + GB_M - 1) / GB_M * int64_t(nc) >= gemm_big_min_tiles();
}

// Rows from which the split-K MFMA GEMV takes over from the dot GEMV (up to
// 16 rows): the dot kernel's VALU work grows with every row, the MFMA's does
// not. Measured with K = 4096: MatMulNBits at two rows is a tie (10.0 vs
// 10.2 us at N = 14336), at four rows split-K wins (10.8 vs 16.2 us); Qkv at
// four rows stays on the dot kernel (10.9 vs 16.6 us: 384 tiles leave the
// split-K grid short of workgroups); Mlp has no dot kernel.
inline int64_t split_k_min_rows(int op) { return op == OP_MATMUL ? 3 : op == OP_QKV ? 5 : 1; }

// Qkv with up to four rows: the MFMA GEMV (integer zero points, whole 32-code
// blocks, K up to 4096 at 4 bits) takes the GQA decode workload in 8.6 us
// against 10.7 us on the dot GEMV, whose four activation rows cost 16
// v_dot2 per weight dword; for MatMulNBits it only ties the split-K GEMV at
// three or four rows (10.1 / 10.4 against 10.0 / 9.9 us at K = 4096,
// N = 14336) and loses to the dot GEMV below.
inline bool mq_takes(const Launch& L) { return L.op == OP_QKV && L.M <= 4 && mq_fits(L); }

// 17..64 rows: the thin GEMM (weights straight into the MFMA operands,
// activations shared through LDS). MatMulNBits where the split-K GEMV does
// not apply, or everywhere in that range with XRMM_THIN_OVER_SK; Mlp on the
// prologue's normalised rows (or rows that need no prologue), unless
// XRMM_THIN_MLP is 0.
#ifndef XRMM_THIN_OVER_SK
#define XRMM_THIN_OVER_SK 0
#endif
#ifndef XRMM_THIN_MLP
#define XRMM_THIN_MLP 1
#endif
inline bool thin_takes(const Launch& L) {
  if (L.M <= 16 || L.M > 64) return false;
  if (L.op == OP_MATMUL) return XRMM_THIN_OVER_SK || !sk_fits(L);
  if (L.op == OP_MLP)
    return XRMM_THIN_MLP && L.p[0].N == L.p[1].N && (L.xs != nullptr || !fused_prologue(L));
  return false;
}

// Rows from which MatMulNBits takes the float32-arithmetic MFMA GEMM: 17, or
// fewer for large weight matrices, where the float32 GEMV's FMAs per row
// cost more than the GEMM's fixed prepass and decode. Measured with 4-bit
// codes and float32 activations: K = N = 4096 at 12 rows 25.4 -> 20.4 us, at
// 16 rows 32.0 -> 20.8; K = 4096, N = 14336 at 5 rows 54.4 -> 29.8, at 16
// rows 110.9 -> 30.1; K = 2048, N = 5632 stays on the GEMV (16.5 against
// 20.1 us at 16 rows); float16 activations at K = N = 4096, 12 rows: 8-bit
// 22.3 -> 15.5, 2-bit 17.2 -> 13.1 us. Float16 4-bit (exact weights) keeps
// 17: its dot GEMVs stay in binary16 arithmetic.
inline int64_t f32x_min_rows(const Launch& L) {
  if (L.dtype == DT_F16 && L.bits == 4) return 17;
  const int64_t w = L.K * L.p[0].N;
  return w >= (int64_t(1) << 25) ? 5 : w >= (int64_t(1) << 24) ? 12 : 17;
}

Kernel select_kernel(const Launch& L) {
  // float32 Qkv / Mlp with the caller's workspace: prologue + float32
  // MatMulNBits per projection
  if (L.op != OP_MATMUL && L.dtype == DT_F32 && L.xs != nullptr && f32split_fits(L)) return K_F32_SPLIT;
  if (L.exact_weights) {
    // the dot and four-row MFMA GEMVs and the float32-arithmetic GEMM keep
    // weights out of binary16; every other fast kernel stages binary16 weights
    if (L.ws != nullptr && f32x_fits(L, f32x_min_rows(L))) return K_GEMM_F32X;
    if (q4_fast_ok(L) && fits_i32(L) && mq_takes(L)) return K_GEMV_MQ;
    if (q4_fast_ok(L) && fits_i32(L) && (L.op == OP_MATMUL || (L.op == OP_QKV && L.gamma)) && L.M >= 1 &&
        L.M < split_k_min_rows(L.op) && dot_fits(L))
      return K_GEMV_DOT;
    // MatMulNBits at any row count on the float32-arithmetic GEMV
    if (f32_fits(L) && fits_i32(L)) return K_GEMV_F32;
    return K_GENERIC;
  }
  // more than 16 rows (fewer for large weight matrices) of float32
  // activations, or of float16 activations with 2- or 8-bit codes, and a
  // caller workspace: the float32-arithmetic GEMM
  if (L.ws != nullptr && f32x_fits(L, f32x_min_rows(L))) return K_GEMM_F32X;
  // float32 activations (the contract's T1 = float32) and float16 with 8-bit
  // codes, any row count: the float32-arithmetic GEMV
  if (f32_fits(L) && fits_i32(L)) return K_GEMV_F32;
  if (q4_fast_ok(L) && fits_i32(L)) {
    if (mq_takes(L)) return K_GEMV_MQ;
    if (thin_takes(L)) return K_GEMM_THIN;
    if (L.M >= split_k_min_rows(L.op) && sk_fits(L)) return K_GEMV_SK;
    if ((L.op == OP_MATMUL || (L.op == OP_QKV && L.gamma)) && L.M >= 1 && dot_fits(L)) return K_GEMV_DOT;
    if (L.M >= 1 && L.M <= 16 && gemv_tiles(L) != 0) return K_GEMV_Q4;
    if (L.M >= kGemmBigMinM && L.op == OP_MATMUL && gemm_big_fills(L)) return K_GEMM_BIG;
    if (L.M > 16 && L.op == OP_MATMUL) return K_GEMM_Q4;
    // Qkv / Mlp prefill on the 256 x 256 pipeline: its K loop is the
    // MatMulNBits one, so the prologue's normalised rows (L.xs) must exist
    // unless there is nothing to normalise
    if (L.M >= kGemmBigMinM && (L.xs != nullptr || !fused_prologue(L)) && gemm_big_fused_fills(L))
      return K_GEMM_BIG_FUSED;
    if (L.M > 16) return K_GEMM_FUSED;
  }
  return K_GENERIC;
}

const char* kernel_name(Kernel k) {
  switch (k) {
    case K_GEMV_Q4: return "gemv_q4_mfma";
    case K_GEMV_DOT: return "gemv_q4_dot";
    case K_GEMV_SK: return "gemv_q4_splitk";
    case K_GEMV_MQ: return "gemv_q4_mq";
    case K_GEMV_F32: return "gemv_q4_f32";
    case K_GEMM_Q4: return "gemm_q4_mfma";
    case K_GEMM_BIG: return "gemm_q4_big";
    case K_GEMM_FUSED: return "gemm_q4_fused";
    case K_GEMM_BIG_FUSED: return "gemm_q4_big_fused";
    case K_GEMM_THIN: return "gemm_q4_thin";
    case K_GEMM_F32X: return "gemm_f32_mfma";
    case K_F32_SPLIT: return "f32_proj";
    default: return "generic";
  }
}

// Two K groups while the tiles fill less than one round of the CUs
// (XRMM_GEMM_KG overrides: 1 or 2).
static int gemm_kgroups(int64_t wgs) {
  const char* e = std::getenv("XRMM_GEMM_KG");
  if (e != nullptr && (*e == '1' || *e == '2') && e[1] == 0) return *e - '0';
  const int cus = device_cus();
  return wgs < (cus > 0 ? cus : 256) ? 2 : 1;
}

// Split-K over workgroups for MatMulNBits tiles that leave CUs idle: as many
// splits as fit one round of the CUs, each split at least eight K steps,
// eight splits at most (each adds a 64 KB float32 partial tile per tile to
// the workspace traffic). Measured, K = 14336, N = 4096, 64 rows (32 tiles,
// 8 splits): 39.5 against 153.8 us without the split.
int gemm_splits(const Launch& L) {
  if (select_kernel(L) == K_GEMM_THIN) return static_cast<int>(thin_args(L, true).S);
  const int64_t tiles = ((L.p[0].N + GM_BN - 1) / GM_BN) * ((L.M + GM_BM - 1) / GM_BM);
  if (tiles * 4 > kGemmCounterBytes) return 1;
  const int64_t ktiles = (L.kb * L.block_size + GM_BK - 1) / GM_BK;
  const int cus = device_cus() > 0 ? device_cus() : 256;
  int64_t s = cus / tiles;  // within one round, so a short grid keeps its two K groups
  s = s > 8 ? 8 : s;
  s = s > ktiles / 8 ? ktiles / 8 : s;
  return s < 2 ? 1 : static_cast<int>(s);
}

int64_t gemm_workspace_bytes(const Launch& L, int splits) {
  if (splits < 2) return 0;
  if (select_kernel(L) == K_GEMM_THIN) return thin_ws_bytes(L);
  const int64_t tiles = ((L.p[0].N + GM_BN - 1) / GM_BN) * ((L.M + GM_BM - 1) / GM_BM);
  return kGemmCounterBytes + tiles * splits * int64_t(256 * 64 * 4);
}

template <int ZPK, int SPC>
static hipError_t launch_gemm2(const Launch& L, hipStream_t st) {
  const int splits = L.ws != nullptr && L.splits > 1 ? L.splits : 1;
  Launch Ls = L;
  Ls.splits = splits;
  const dim3 grid(static_cast<uint32_t>((L.p[0].N + GM_BN - 1) / GM_BN), static_cast<uint32_t>((L.M + GM_BM - 1) / GM_BM),
                  static_cast<uint32_t>(splits));
  if (grid.y > 65535) return hipErrorInvalidValue;  // launch limit
  if (gemm_kgroups(int64_t(grid.x) * grid.y * grid.z) == 2)
    hipLaunchKernelGGL((k_gemm_q4<ZPK, SPC, 2>), grid, dim3(512), 0, st, Ls);
  else
    hipLaunchKernelGGL((k_gemm_q4<ZPK, SPC, 1>), grid, dim3(256), 0, st, Ls);
  return hipGetLastError();
}

template <int ZPK>
static hipError_t launch_gemm1(const Launch& L, hipStream_t st) {
  return spc_of(L.block_size) == 1 ? launch_gemm2<ZPK, 1>(L, st) : launch_gemm2<ZPK, 2>(L, st);
}

static int effective_zpk(const Launch& L) {
  // a zero-point kind applies only when every projection carries zero points
  if (L.zp_kind == ZP_NONE) return ZP_NONE;
  for (int i = 0; i < L.nproj; ++i)
    if (!L.p[i].zp) return -1;
  return L.zp_kind;
}

hipError_t launch(const Launch& L, hipStream_t st) {
  if (L.M == 0) return hipSuccess;
  Kernel k = select_kernel(L);
  if (k == K_F32_SPLIT) return launch_f32_split(L, st);  // per projection (each with its own zero points)
  const int zpk = effective_zpk(L);
  if (zpk < 0) k = K_GENERIC;  // mixed presence of zero points
  if (k == K_GEMM_F32X) return launch_gemm_f32x(L, st);
  if (k == K_GEMV_F32) {
    if (zpk == ZP_NONE) return launch_f32_for<ZP_NONE>(L, st);
    if (zpk == ZP_PACKED) return launch_f32_for<ZP_PACKED>(L, st);
    return launch_f32_for<ZP_FLOAT>(L, st);
  }
  if (k == K_GEMV_MQ) return zpk == ZP_PACKED ? launch_mq_for<ZP_PACKED>(L, st) : launch_mq_for<ZP_NONE>(L, st);
  if (k == K_GEMV_DOT) {
    if (zpk == ZP_NONE) return launch_dot_for<ZP_NONE>(L, st);
    if (zpk == ZP_PACKED) return launch_dot_for<ZP_PACKED>(L, st);
    return launch_dot_for<ZP_FLOAT>(L, st);
  }
  if (k == K_GEMV_SK) {
    if (zpk == ZP_NONE) return launch_sk_for<ZP_NONE>(L, st);
    if (zpk == ZP_PACKED) return launch_sk_for<ZP_PACKED>(L, st);
    return launch_sk_for<ZP_FLOAT>(L, st);
  }
  if (k == K_GEMV_Q4) {
    if (zpk == ZP_NONE) return launch_gemv_for<ZP_NONE>(L, st);
    if (zpk == ZP_PACKED) return launch_gemv_for<ZP_PACKED>(L, st);
    return launch_gemv_for<ZP_FLOAT>(L, st);
  }
  if (k == K_GEMM_BIG) {
    if (zpk == ZP_NONE) return launch_gemm_big_for<ZP_NONE>(L, st);
    if (zpk == ZP_PACKED) return launch_gemm_big_for<ZP_PACKED>(L, st);
    return launch_gemm_big_for<ZP_FLOAT>(L, st);
  }
  if (k == K_GEMM_FUSED || k == K_GEMM_BIG_FUSED) {
    // with a workspace the prologue normalises once per row and the GEMM
    // reads its binary16 output; without one only the 128 x 128 GEMM runs,
    // normalising inside its K loop
    Launch Lx = L;
    if (L.xs != nullptr && fused_prologue(L)) {
      const hipError_t e = run_prologue(L, Lx, st);
      if (e != hipSuccess) return e;
    }
    if (k == K_GEMM_BIG_FUSED) {
      if (zpk == ZP_NONE) return launch_gemm_big_fused_for<ZP_NONE>(Lx, st);
      if (zpk == ZP_FLOAT) return launch_gemm_big_fused_for<ZP_FLOAT>(Lx, st);
      return launch_gemm_big_fused_for<ZP_PACKED>(Lx, st);
    }
    if (zpk == ZP_NONE) return launch_gemm_fused_for<ZP_NONE>(Lx, st);
    if (zpk == ZP_FLOAT) return launch_gemm_fused_for<ZP_FLOAT>(Lx, st);
    return launch_gemm_fused_for<ZP_PACKED>(Lx, st);
  }
  if (k == K_GEMM_THIN) {
    // Mlp: the prologue first, the GEMM on its normalised rows
    Launch Lx = L;
    if (L.op != OP_MATMUL && L.xs != nullptr && fused_prologue(L)) {
      const hipError_t e = run_prologue(L, Lx, st);
      if (e != hipSuccess) return e;
    }
    if (zpk == ZP_NONE) return launch_gemm_thin_for<ZP_NONE>(Lx, st);
    if (zpk == ZP_FLOAT) return launch_gemm_thin_for<ZP_FLOAT>(Lx, st);
    return launch_gemm_thin_for<ZP_PACKED>(Lx, st);
  }
  if (k == K_GEMM_Q4) {
    if (zpk == ZP_NONE) return launch_gemm1<ZP_NONE>(L, st);
    if (zpk == ZP_FLOAT) return launch_gemm1<ZP_FLOAT>(L, st);
    return launch_gemm1<ZP_PACKED>(L, st);
  }
  int64_t cols = L.p[0].N;
  if (L.op == OP_QKV) cols += L.p[1].N + L.p[2].N;
  constexpr int MB = 8;
  if (cols > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;  // launch limit
  const dim3 grid(static_cast<uint32_t>(cols), static_cast<uint32_t>((L.M + MB - 1) / MB));
  hipLaunchKernelGGL(k_generic<MB>, grid, dim3(64), 0, st, L);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// offline weight prepack for the prefill GEMM (xrmm_prepack_weights)
//
// Layout: [K step s][column n][32 bytes], a K step being 64 codes, so the
// 256 columns of a GEMM tile read one K step as one contiguous 8 KB block
// (whole 1 KB pieces per wave load instead of 32-byte pieces of 32 column
// rows). Inside each dword the eight codes c0..c7 of eight consecutive k are
// reordered to nibble slots (c0 c2 c4 c6 c1 c3 c5 c7): the dequantisation's
// exponent-bias pairs (slots 0/4, 1/5, 2/6, 3/7) then come out in natural k
// order, so the GEMM stages the activations as they are, without the pair
// permutation. Codes, scales and zero points are otherwise unchanged; a
// second 16-byte half past the column's last chunk is zero.

// Reorder the nibbles of x (c_i at bits 4i) to slots (c0 c2 c4 c6 c1 c3 c5 c7).
__device__ __forceinline__ uint32_t prepack_dword(uint32_t x) {
  auto squeeze = [](uint32_t b) {  // low nibbles of the four bytes -> one 16-bit value
    const uint32_t t = (b | (b >> 4)) & 0x00FF00FFu;
    return (t & 0xFFu) | ((t >> 8) & 0xFF00u);
  };
  return squeeze(x & 0x0F0F0F0Fu) | (squeeze((x >> 4) & 0x0F0F0F0Fu) << 16);
}

// One thread per 16-byte half (s, n, h): consecutive threads write
// consecutive 16 bytes.
__global__ __launch_bounds__(256) void k_prepack_q4(const uint8_t* __restrict__ B, uint8_t* __restrict__ out,
                                                    uint32_t N, uint32_t nchunk, uint64_t pieces) {
  const uint64_t t = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
  if (t >= pieces) return;
  const uint32_t h = static_cast<uint32_t>(t & 1u);
  const uint64_t sn = t >> 1;
  const uint32_t n = static_cast<uint32_t>(sn % N), s = static_cast<uint32_t>(sn / N);
  const uint32_t ch = 2u * s + h;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (ch < nchunk) v = ld16(B + (static_cast<uint64_t>(n) * nchunk + ch) * 16u);
#pragma unroll
  for (int d = 0; d < 4; ++d) v[d] = prepack_dword(v[d]);
  *reinterpret_cast<u32x4*>(out + t * 16u) = v;
}

int64_t prepacked_bytes(int64_t N, int64_t kb, int64_t block_size, int bits) {
  const int64_t Kp = kb * block_size;
  if (bits != 4 || N <= 0 || Kp <= 0 || Kp % 32 != 0) return 0;
  return (Kp + 63) / 64 * N * 32;
}

hipError_t launch_prepack(const Launch& L, void* out, hipStream_t st) {
  const Proj& P = L.p[0];
  const int64_t bytes = prepacked_bytes(P.N, L.kb, L.block_size, L.bits);
  if (bytes == 0) return hipErrorInvalidValue;
  const uint64_t pieces = static_cast<uint64_t>(bytes / 16);
  const uint64_t grid = (pieces + 255) / 256;
  if (grid > 0x7FFFFFFFu || P.N > 0xFFFFFFFFLL) return hipErrorInvalidValue;  // launch limits
  hipLaunchKernelGGL(k_prepack_q4, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, st, P.B, static_cast<uint8_t*>(out),
                     static_cast<uint32_t>(P.N), static_cast<uint32_t>(L.kb * L.blob / 16), pieces);
  return hipGetLastError();
}

bool prepacked_ok(const Launch& L) {
  return L.op == OP_MATMUL && L.M >= 1 && q4_fast_ok(L) && fits_i32(L) &&
         prepacked_bytes(L.p[0].N, L.kb, L.block_size, L.bits) != 0;
}

hipError_t launch_prepacked(const Launch& L, hipStream_t st) {
  const int zpk = L.zp_kind == ZP_NONE || !L.p[0].zp ? ZP_NONE : L.zp_kind;
  if (zpk == ZP_NONE) return launch_gemm_big_pk_for<ZP_NONE>(L, st);
  if (zpk == ZP_PACKED) return launch_gemm_big_pk_for<ZP_PACKED>(L, st);
  return launch_gemm_big_pk_for<ZP_FLOAT>(L, st);
}

hipError_t launch_dequantize(const Launch& L, void* W, int out_dtype, hipStream_t st) {
  const Proj& P = L.p[0];
  if (P.N == 0 || L.K == 0) return hipSuccess;
  if (out_dtype == DT_F16 && L.bits == 4 && L.dtype == DT_F16 && L.bs_log2 >= 4 &&
      (L.kb * L.block_size) % 32 == 0 && aligned16(P.B)) {
    const int64_t n = P.N * (L.kb * L.blob / 16);
    if ((n + 255) / 256 > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;  // launch limit
    const dim3 grid(static_cast<uint32_t>((n + 255) / 256));
    const int spc = spc_of(L.block_size);
    const int zpk = P.zp ? L.zp_kind : ZP_NONE;
    f16* out = static_cast<f16*>(W);
#define XRMM_DQ(Z, S) hipLaunchKernelGGL((k_dequant_q4_f16<Z, S>), grid, dim3(256), 0, st, L, out)
    if (zpk == ZP_NONE) {
      if (spc == 1) XRMM_DQ(ZP_NONE, 1); else XRMM_DQ(ZP_NONE, 2);
    } else if (zpk == ZP_PACKED) {
      if (spc == 1) XRMM_DQ(ZP_PACKED, 1); else XRMM_DQ(ZP_PACKED, 2);
    } else {
      if (spc == 1) XRMM_DQ(ZP_FLOAT, 1); else XRMM_DQ(ZP_FLOAT, 2);
    }
#undef XRMM_DQ
    return hipGetLastError();
  }
  const int64_t n = P.N * L.K;
  if ((n + 255) / 256 > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;  // launch limit
  hipLaunchKernelGGL(k_dequant_f32, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, st, L, W, out_dtype);
  return hipGetLastError();
}

}  // namespace xrmm
