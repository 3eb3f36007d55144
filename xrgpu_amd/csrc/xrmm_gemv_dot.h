// Decode GEMV for M <= 4 rows (fp16 activations, 4-bit weights). After one
// barrier that publishes the staged activations, each wave runs on its own:
// no LDS traffic and no barrier on the weight stream.
//
// Work split. A wave owns C consecutive output columns (a column is one row
// of B: kb * blob bytes) and walks them in order. Its lanes split K: lane l
// takes the 16-byte chunks l, l + 64, l + 128, ... of every column, so each
// wave load instruction reads 1 KB of contiguous weights. Loads of the next P
// columns are in flight while a column is computed, so arithmetic overlaps the
// HBM stream instead of following it.
//
// Activations live in registers. Lane l needs the same 32 activations per
// chunk for every column. The workgroup stages them once in LDS, already in
// the nibble-pair order below and laid out so that a wave's 64 lanes read
// consecutive 16-byte pieces (no bank conflicts), together with the per-chunk
// activation sums; every wave then copies its lanes' pairs into registers.
// Reads past K go through a buffer resource and return zero, so padding
// contributes nothing.
//
// Arithmetic. A dword x of a chunk holds the codes c0..c7 of eight
// consecutive k (low nibble first, complex_kernel.glsl:80). OR-ing masked
// nibbles into the mantissa of 1024.0h gives exact binary16 values:
//   (x & 0x000F000F) | 0x6400  -> (1024 + c0, 1024 + c4)
//   (x & 0x00F000F0) | 0x6400  -> (1024 + 16 c1, 1024 + 16 c5)
// and the same on x >> 8 for (c2, c6), (c3, c7). v_dot2_f32_f16 multiplies
// these pairs with the matching activation pairs and accumulates in float32
// (fp16 products are exact in float32). With P_lo / P_hi the two sums of a
// chunk,
//   sum_k c_k a_k = P_lo + P_hi / 16 - (1024 sum_lo a + 64 sum_hi a),
// and the block's contribution is s * (sum_k c_k a_k - z * sum_k a_k). The
// bracketed activation sums are per-lane constants computed once, so a chunk
// costs 9 VALU per dword plus three per row. Integer-valued inputs stay exact
// (every intermediate is an integer below 2^24).
//
// Reduction. Each lane ends a column with a partial sum per row; DPP steps
// reduce within rows of 16 lanes and four readlanes finish the wave sum.
#pragma once
#include "xrmm_device.h"

namespace xrmm {

__device__ __forceinline__ f16x2 h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }

__device__ __forceinline__ float dot2(uint32_t w, f16x2 a, float acc) {
  return __builtin_amdgcn_fdot2(h2(w), a, acc, false);
}

// Row sums over 16-lane rows with DPP, then the four row sums combined through
// readlane: every lane returns the wave total.
__device__ __forceinline__ float wave_total(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)); // row_half_mirror
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)); // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

// Offset past the end of every buffer resource: such loads return zero.
constexpr uint32_t kOOB = 0x80000000u;

// 16-byte pieces per lane of a wave's scale (or zero-point) block: the block
// holds at most DOT_META_PIECES KB.
constexpr int DOT_META_PIECES = 4;

// Compact kernel arguments: every field is read in the kernel's first scalar
// batch, before any branch, so a wave issues its first weight loads after a
// single kernel-argument round trip.
struct DotProj {
  const uint8_t* B;
  const void* S;
  const void* Z;
  void* Y;
  uint32_t N;
  uint32_t wg0;  // first wave of this projection on the grid (global wave index)
};

struct DotArgs {
  const void* A;
  const void* bias;   // MatMulNBits only
  const void* skip;   // Qkv: nullable, added to A
  const void* gamma;  // Qkv: RMS scale [K]
  void* residual;     // Qkv: nullable, receives A + skip
  float eps;
  DotProj p[3];       // MatMulNBits: p[0]; Qkv: Q, K, V side by side on the grid
  uint32_t K, kb, rowb, zrow, M;
  uint32_t bsl;         // log2(block_size)
  uint32_t zesz;        // bytes per float zero point (2 or 4)
  uint32_t meta_bytes;  // per-wave LDS bytes: C*kb*2 scales (+ C*zrow zero points), 16-aligned
  uint32_t zoff;        // offset of the zero points inside a wave's LDS slice
  uint32_t act_bytes;   // LDS bytes of the staged activation pairs and sums
};

// LDS bytes of the staged activations: pairs [MR][CPL][4][64] x 16 B, then the
// sums [MR][CPL][SPC][2][64] x 4 B (negated bias, activation sum).
template <int MR, int CPL, int SPC>
__host__ __device__ constexpr uint32_t dot_act_bytes() {
  return MR * CPL * 4 * 64 * 16 + MR * CPL * SPC * 2 * 64 * 4;
}

// OPK: OP_MATMUL, or OP_QKV with SK = whether the skip input is present.
template <int ZPK, int SPC, int CPL, int C, int P, int MR, int W, int MP, int OPK, bool SK = false>
__global__ __launch_bounds__(W * 64) void k_gemv_dot(DotArgs a) {
  static_assert(MP >= 1 && MP <= DOT_META_PIECES, "scale pieces");
  static_assert(OPK == OP_MATMUL || OPK == OP_QKV, "operator");
  static_assert(OPK == OP_QKV || !SK, "skip is a Qkv input");
  constexpr bool QKV = OPK == OP_QKV;
  constexpr int DPH = 4 / SPC;  // dwords per block of a chunk
  constexpr uint32_t PAIRS = MR * CPL * 4 * 64 * 16;
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The wave's projection: Qkv lays the waves of Q, K and V side by side on
  // the grid (a workgroup may hold waves of two projections: they share the
  // activations). Every projection's fields are loaded with the other
  // arguments and picked with scalar selects, so no load depends on the choice.
#ifndef XRMM_DOT_XCD
#define XRMM_DOT_XCD 1
#endif
  const uint32_t bid = XRMM_DOT_XCD ? xcd_slot(blockIdx.x, gridDim.x) : blockIdx.x;
  const uint32_t gw = bid * W + wave;  // global wave index
  uint32_t pi = 0;
  if constexpr (QKV) pi = (gw >= a.p[1].wg0 ? 1u : 0u) + (gw >= a.p[2].wg0 ? 1u : 0u);
  auto pick = [&](auto v0, auto v1, auto v2) { return QKV ? (pi == 0 ? v0 : pi == 1 ? v1 : v2) : v0; };
  const uint8_t* Bp = pick(a.p[0].B, a.p[1].B, a.p[2].B);
  const void* Sp = pick(a.p[0].S, a.p[1].S, a.p[2].S);
  const void* Zp = pick(a.p[0].Z, a.p[1].Z, a.p[2].Z);
  void* Yp = pick(a.p[0].Y, a.p[1].Y, a.p[2].Y);
  const uint32_t N = pick(a.p[0].N, a.p[1].N, a.p[2].N);
  const uint32_t wg0 = pick(a.p[0].wg0, a.p[1].wg0, a.p[2].wg0);
  const uint32_t K = a.K, kb = a.kb, rowb = a.rowb, zrow = a.zrow;
  const uint32_t nchunk = rowb >> 4;
  const int M = static_cast<int>(a.M);
  const uint32_t col0 = (gw - wg0) * C;
  // Columns past N (the grid's last waves) are clamped for loading and never
  // stored; no early exit, so no branch separates the argument loads.
  auto clampc = [&](uint32_t c) { return c < N ? c : N - 1; };

  // Issue order matters: the vector-memory counter retires loads in issue
  // order, so the small loads the prologue consumes (scales / zero points of
  // the wave's columns, activations) go first and the weight stream follows;
  // waiting for the small loads then never waits for weights.

  // ---- scales / zero points of the wave's C columns: contiguous blocks,
  // 16 bytes per lane per load (bytes past a block read as zero)
  const uint32_t c0 = clampc(col0);
  const uint32_t sbytes = C * kb * 2u;
  const uint32_t zbytes = ZPK == ZP_NONE ? 0u : C * zrow;
  // Loads start at the dword boundary at or below the wave's block (sdel /
  // zdel bytes earlier): the range check zeroes a whole dword that straddles
  // the bound, which only stays harmless for dword-aligned starts (a packed
  // zero-point row may have any byte count, so a block may start anywhere).
  const uint32_t sdel = (c0 * kb * 2u) & 3u, zdel = (c0 * zrow) & 3u;
  u32x4 sv[MP], zv[ZPK == ZP_NONE ? 1 : MP];
  {
    // The bound is rounded up to 16 bytes so that dwords holding the last
    // bytes are not zeroed. Tensors on this path start 16-byte aligned, so the
    // rounded bound stays inside the aligned 16-byte block holding the
    // tensor's last byte; the extra bytes are never used.
    const rsrc_t rS = mk_rsrc(Sp, (N * kb * 2u + 15u) & ~15u);
#pragma unroll
    for (int q = 0; q < MP; ++q) {
      const uint32_t o = lane * 16u + 1024u * q;
      sv[q] = bld16_nt(rS, o < sbytes + sdel ? c0 * kb * 2u - sdel + o : kOOB, 0);  // predicated, no branch: a branch here costs a full wait
    }
    if constexpr (ZPK != ZP_NONE) {
      const rsrc_t rZ = mk_rsrc(Zp, (N * zrow + 15u) & ~15u);
#pragma unroll
      for (int q = 0; q < MP; ++q) {
        const uint32_t o = lane * 16u + 1024u * q;
        zv[q] = bld16_nt(rZ, o < zbytes + zdel ? c0 * zrow - zdel + o : kOOB, 0);
      }
    }
  }

  // Keep the issue order: the compiler may not move later loads ahead.
  __builtin_amdgcn_sched_barrier(0);

  // ---- activations of the workgroup's staging items: item (m, j, l) is
  // chunk l + 64 j of row m (32 activations, four 16-byte groups)
  constexpr int ITEMS = MR * CPL * 64;
  constexpr int IPT = (ITEMS + W * 64 - 1) / (W * 64);  // items per thread
  const rsrc_t rA = mk_rsrc(a.A, static_cast<uint32_t>(M) * K * 2u);
  // Qkv also loads skip (when present) and the RMS scale of the same k. When
  // every item of a thread has the same chunk index (W a multiple of CPL), the
  // thread loads the scale once.
  constexpr bool GSAME = W % CPL == 0;
  constexpr int GI = !QKV ? 1 : GSAME ? 1 : IPT;
  const rsrc_t rK = mk_rsrc(a.skip, SK ? static_cast<uint32_t>(M) * K * 2u : 0u);
  const rsrc_t rG = mk_rsrc(a.gamma, QKV ? K * 2u : 0u);
  u32x4 raw[IPT][4], rsk[SK ? IPT : 1][4], rgm[GI][4];
#pragma unroll
  for (int it = 0; it < IPT; ++it) {
    const int item = tid + it * W * 64;
    const int m = item / (CPL * 64), jl = item % (CPL * 64);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t k = static_cast<uint32_t>(jl) * 32u + 8u * g;
      const bool ok = item < ITEMS && m < M && k < K;  // K % 8 == 0 on this path: groups are whole
      const uint32_t off = ok ? (static_cast<uint32_t>(m) * K + k) * 2u : kOOB;
      raw[it][g] = bld16(rA, off, 0);
      if constexpr (SK) rsk[it][g] = bld16(rK, off, 0);
      if constexpr (QKV) {
        if (!GSAME || it == 0) rgm[GSAME ? 0 : it][g] = bld16(rG, k < K ? k * 2u : kOOB, 0);
      }
    }
  }

  __builtin_amdgcn_sched_barrier(0);

  // ---- weights of the first P columns: the HBM stream
  const rsrc_t rB = mk_rsrc(Bp, N * rowb);
  uint32_t vb[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint32_t ch = static_cast<uint32_t>(lane + 64 * j);
    vb[j] = (ch < nchunk ? ch : nchunk - 1) * 16u;  // past-the-row lanes reuse the last chunk (zero activations)
  }
  u32x4 wbuf[P + 1][CPL];
  auto issue = [&](u32x4(&w)[CPL], uint32_t col) {
    const uint32_t cb = clampc(col) * rowb;
#pragma unroll
    for (int j = 0; j < CPL; ++j) w[j] = bld16_nt(rB, vb[j], cb);
  };
#pragma unroll
  for (int i = 0; i < P; ++i) issue(wbuf[i], col0 + i);

  __builtin_amdgcn_sched_barrier(0);

  // ---- stage: this wave's scales / zero points into its own LDS slice, the
  // workgroup's activations into pair order, plus the per-chunk constants
  unsigned char* meta = smem + a.act_bytes + wave * a.meta_bytes;
#pragma unroll
  for (int q = 0; q < MP; ++q) {
    const uint32_t o = lane * 16u + 1024u * q;
    if (o < sbytes + sdel) *reinterpret_cast<u32x4*>(meta + o) = sv[q];
    if (ZPK != ZP_NONE && o < zbytes + zdel) *reinterpret_cast<u32x4*>(meta + a.zoff + o) = zv[ZPK == ZP_NONE ? 0 : q];
  }
  // Qkv: r = A + skip in float32 and x = r * inv * gamma with
  // inv = 1 / sqrt(sum_k r^2 / K + eps) per row (packedInput,
  // complex_kernel.glsl:81); x is staged in binary16, so it is normalised
  // before rounding (r * gamma alone could leave the binary16 range). The
  // workgroup holds whole rows: the row sums of squares reduce once through
  // LDS. Per element each pass is one or two mixed-precision FMAs (binary16
  // operands, float32 arithmetic).
  if constexpr (QKV) {
    __shared__ float red[W][MR];
    auto rval = [&](const f16x8& av, const f16x8& sv, int e) {
      if constexpr (SK) return __fadd_rn(static_cast<float>(av[e]), static_cast<float>(sv[e]));
      else return static_cast<float>(av[e]);
    };
    float sq[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) sq[m] = 0.f;
#pragma unroll
    for (int it = 0; it < IPT; ++it) {
      const int item = tid + it * W * 64;
      const int m = item / (CPL * 64);
      float part[2] = {0.f, 0.f};
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f16x8 av = __builtin_bit_cast(f16x8, raw[it][g]);
        const f16x8 sv = __builtin_bit_cast(f16x8, rsk[SK ? it : 0][g]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float r = rval(av, sv, e);
          part[e & 1] = __builtin_fmaf(r, r, part[e & 1]);
        }
      }
#pragma unroll
      for (int mm = 0; mm < MR; ++mm) sq[mm] += (item < ITEMS && m == mm) ? part[0] + part[1] : 0.f;
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float t = wave_total(sq[m]);
      if (lane == 0) red[wave][m] = t;
    }
    __syncthreads();
    float inv[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) t += red[w][m];
      inv[m] = __builtin_amdgcn_rsqf(t / static_cast<float>(K) + a.eps);
    }
    f16* res = static_cast<f16*>(a.residual);
    const bool write_res = res != nullptr && bid == 0;
#pragma unroll
    for (int it = 0; it < IPT; ++it) {
      const int item = tid + it * W * 64;
      const int m = item / (CPL * 64), jl = item % (CPL * 64);
      float im = inv[0];
#pragma unroll
      for (int mm = 1; mm < MR; ++mm) im = m == mm ? inv[mm] : im;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f16x8 av = __builtin_bit_cast(f16x8, raw[it][g]);
        const f16x8 sv = __builtin_bit_cast(f16x8, rsk[SK ? it : 0][g]);
        const f16x8 gv = __builtin_bit_cast(f16x8, rgm[GSAME ? 0 : it][g]);
        f16x8 x;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float t = __builtin_fmaf(static_cast<float>(gv[e]), im, 0.f);
          x[e] = static_cast<f16>(rval(av, sv, e) * t);
        }
        raw[it][g] = __builtin_bit_cast(u32x4, x);
        const uint32_t k = static_cast<uint32_t>(jl) * 32u + 8u * g;
        if (write_res && item < ITEMS && m < M && k < K) {
          f16x8 rr;
#pragma unroll
          for (int e = 0; e < 8; ++e) rr[e] = static_cast<f16>(rval(av, sv, e));
          *reinterpret_cast<f16x8*>(res + static_cast<uint32_t>(m) * K + k) = rr;
        }
      }
    }
  }
  // Whether any staged activation is +-Inf or NaN. The per-chunk sums below
  // are finite exactly when all 32 activations of the chunk are (|sum| <=
  // 32 * 65504 * 1032, far below FLT_MAX), so they double as the detector.
  bool nonfinite = false;
  {
    const f16x2 c1024 = {static_cast<f16>(1024.f), static_cast<f16>(1024.f)};
    const f16x2 c64 = {static_cast<f16>(64.f), static_cast<f16>(64.f)};
    const f16x2 c1032 = {static_cast<f16>(1032.f), static_cast<f16>(1032.f)};
    const f16x2 c72 = {static_cast<f16>(72.f), static_cast<f16>(72.f)};
    const f16x2 c1 = {static_cast<f16>(1.f), static_cast<f16>(1.f)};
#pragma unroll
    for (int it = 0; it < IPT; ++it) {
      const int item = tid + it * W * 64;
      if (item < ITEMS) {
        const int m = item / (CPL * 64), j = (item / 64) % CPL, l = item % 64;
        f16x2 pr[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const u32x4 r = raw[it][g];  // halfs a0..a7 as dwords (a0,a1) (a2,a3) (a4,a5) (a6,a7)
          pr[4 * g + 0] = h2(__builtin_amdgcn_perm(r[2], r[0], 0x05040100u));  // (a0, a4)
          pr[4 * g + 1] = h2(__builtin_amdgcn_perm(r[2], r[0], 0x07060302u));  // (a1, a5)
          pr[4 * g + 2] = h2(__builtin_amdgcn_perm(r[3], r[1], 0x05040100u));  // (a2, a6)
          pr[4 * g + 3] = h2(__builtin_amdgcn_perm(r[3], r[1], 0x07060302u));  // (a3, a7)
          *reinterpret_cast<u32x4*>(smem + (((m * CPL + j) * 4 + g) * 64 + l) * 16) =
              u32x4{__builtin_bit_cast(uint32_t, pr[4 * g]), __builtin_bit_cast(uint32_t, pr[4 * g + 1]),
                    __builtin_bit_cast(uint32_t, pr[4 * g + 2]), __builtin_bit_cast(uint32_t, pr[4 * g + 3])};
        }
        // -(1024 sum_lo a + 64 sum_hi a) [- 8 sum a when z is implicit] and sum a,
        // per block half; four partial chains keep the dependency depth short
#pragma unroll
        for (int h = 0; h < SPC; ++h) {
          float b[4] = {0.f, 0.f, 0.f, 0.f}, t[2] = {0.f, 0.f};
#pragma unroll
          for (int e = 4 * DPH * h; e < 4 * DPH * (h + 1); ++e) {
            const f16x2 w = ZPK == ZP_NONE ? ((e & 1) ? c72 : c1032) : ((e & 1) ? c64 : c1024);
            b[e & 3] = __builtin_amdgcn_fdot2(pr[e], w, b[e & 3], false);
            if constexpr (ZPK != ZP_NONE) t[e & 1] = __builtin_amdgcn_fdot2(pr[e], c1, t[e & 1], false);
          }
          float* sums = reinterpret_cast<float*>(smem + PAIRS) + (((m * CPL + j) * SPC + h) * 2) * 64 + l;
          const float nb = -((b[0] + b[1]) + (b[2] + b[3]));
          nonfinite |= !__builtin_isfinite(nb);
          sums[0] = nb;
          sums[64] = t[0] + t[1];
        }
      }
    }
  }
  __shared__ uint32_t wave_nonfinite[W];
  {
    const bool any = __builtin_amdgcn_ballot_w64(nonfinite) != 0;
    if (lane == 0) wave_nonfinite[wave] = any ? 1u : 0u;
  }
  __syncthreads();
  uint32_t special = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) special |= wave_nonfinite[w];

  if (special != 0) {
    // Some staged activation is +-Inf or NaN: the folded-bias sums above would
    // turn an infinite activation into Inf - Inf. The workgroup takes the
    // reference's per-element form instead (complex_kernel.glsl:80,83):
    // W = (code - z) * scale in float32, then sum += x * W, so +-Inf * W gives
    // +-Inf (NaN where W is 0) exactly as the serial shader does. Activations
    // come from the staged pairs (A, or the normalised Qkv input).
    const f16* S16 = static_cast<const f16*>(Sp);
    f16* Yo = static_cast<f16*>(Yp);
    const f16* bo = QKV ? nullptr : static_cast<const f16*>(a.bias);
    for (int i = 0; i < C; ++i) {
      const uint32_t col = col0 + static_cast<uint32_t>(i);
      if (col >= N) break;
      float y[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) y[m] = 0.f;
      for (uint32_t k = lane; k < K; k += 64) {
        const uint32_t b = k >> a.bsl;
        const uint32_t byte = Bp[col * rowb + (k >> 1)];  // 4-bit: byte k/2 of the row, low nibble first
        const float code = static_cast<float>((byte >> ((k & 1u) * 4u)) & 15u);
        float z = 8.f;
        if constexpr (ZPK == ZP_PACKED) {
          z = static_cast<float>((static_cast<const uint8_t*>(Zp)[col * zrow + (b >> 1)] >> ((b & 1u) * 4u)) & 15u);
        } else if constexpr (ZPK == ZP_FLOAT) {
          z = a.zesz == 4 ? static_cast<const float*>(Zp)[col * kb + b]
                          : static_cast<float>(static_cast<const f16*>(Zp)[col * kb + b]);
        }
        const float w = (code - z) * static_cast<float>(S16[col * kb + b]);
        const uint32_t ch = k >> 5, g = (k >> 3) & 3u, e = k & 7u;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const f16* xp = reinterpret_cast<const f16*>(
              smem + ((((m * CPL + (ch >> 6)) * 4 + g) * 64 + (ch & 63u)) * 16u) + (e & 3u) * 4u + (e >> 2) * 2u);
          y[m] = __builtin_fmaf(static_cast<float>(*xp), w, y[m]);
        }
      }
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float tot = wave_total(y[m]);
        if (lane == 0 && m < M) Yo[static_cast<uint32_t>(m) * N + col] = static_cast<f16>(tot + (bo ? static_cast<float>(bo[col]) : 0.f));
      }
    }
    return;
  }

  // ---- this lane's activation pairs and constants, into registers
  f16x2 ap[MR][CPL][16];
  float nbias[MR][CPL][SPC], asum[MR][CPL][SPC];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(smem + (((m * CPL + j) * 4 + g) * 64 + lane) * 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) ap[m][j][4 * g + e] = h2(v[e]);
      }
#pragma unroll
      for (int h = 0; h < SPC; ++h) {
        const float* sums = reinterpret_cast<const float*>(smem + PAIRS) + (((m * CPL + j) * SPC + h) * 2) * 64 + lane;
        nbias[m][j][h] = sums[0];
        asum[m][j][h] = sums[64];
      }
    }

  // per-lane LDS offsets of the scale / zero point of chunk round j
  uint32_t ls[CPL], lz[CPL], zsh[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint32_t ch = static_cast<uint32_t>(lane + 64 * j);
    const uint32_t chc = ch < nchunk ? ch : nchunk - 1;
    const uint32_t b = SPC == 1 ? (chc * 32u) >> a.bsl : 2u * chc;  // first block of the chunk
    ls[j] = b * 2u;
    lz[j] = ZPK == ZP_PACKED ? (b >> 1) : b * a.zesz;
    zsh[j] = (b & 1u) * 4u;
  }

  const f16* biasp = QKV ? nullptr : static_cast<const f16*>(a.bias);
  f16* Y = static_cast<f16*>(Yp);
  float out[MR];  // lane i < C keeps column col0 + i
#pragma unroll
  for (int m = 0; m < MR; ++m) out[m] = 0.f;

#pragma unroll
  for (int i = 0; i < C; ++i) {
    if (col0 + i >= N) break;  // wave-uniform, after the loads are in flight
    if (i + P < C) issue(wbuf[(i + P) % (P + 1)], col0 + i + P);
    const u32x4(&w)[CPL] = wbuf[i % (P + 1)];
    const unsigned char* ms = meta + sdel + i * kb * 2u;
    const unsigned char* mz = meta + a.zoff + zdel + i * zrow;
    float y[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) y[m] = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t magic = 0x64006400u;
      uint32_t lo[8], hi[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t x = w[j][q], x8 = x >> 8;
        lo[2 * q] = and_or(x, 0x000F000Fu, magic);
        hi[2 * q] = and_or(x, 0x00F000F0u, magic);
        lo[2 * q + 1] = and_or(x8, 0x000F000Fu, magic);
        hi[2 * q + 1] = and_or(x8, 0x00F000F0u, magic);
      }
      uint32_t zb = 0;
      if constexpr (ZPK == ZP_PACKED) zb = mz[lz[j]];
#pragma unroll
      for (int h = 0; h < SPC; ++h) {
        const float s = static_cast<float>(*reinterpret_cast<const f16*>(ms + ls[j] + 2u * h));
        float z = 0.f;
        if constexpr (ZPK == ZP_PACKED) {
          z = static_cast<float>((zb >> (SPC == 1 ? zsh[j] : 4u * h)) & 15u);
        } else if constexpr (ZPK == ZP_FLOAT) {
          z = a.zesz == 4 ? *reinterpret_cast<const float*>(mz + lz[j] + 4u * h)
                          : static_cast<float>(*reinterpret_cast<const f16*>(mz + lz[j] + 2u * h));
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          float pl = nbias[m][j][h], ph = 0.f;
#pragma unroll
          for (int q = DPH * h; q < DPH * (h + 1); ++q) {
            pl = dot2(lo[2 * q], ap[m][j][4 * q + 0], pl);
            ph = dot2(hi[2 * q], ap[m][j][4 * q + 1], ph);
            pl = dot2(lo[2 * q + 1], ap[m][j][4 * q + 2], pl);
            ph = dot2(hi[2 * q + 1], ap[m][j][4 * q + 3], ph);
          }
          float t = __builtin_fmaf(ph, 0.0625f, pl);
          if constexpr (ZPK != ZP_NONE) t = __builtin_fmaf(-z, asum[m][j][h], t);
          y[m] = __builtin_fmaf(s, t, y[m]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float tot = wave_total(y[m]);
      out[m] = lane == i ? tot : out[m];
    }
  }

  // lane i < C writes column col0 + i
  const uint32_t mycol = col0 + static_cast<uint32_t>(lane);
  if (lane < C && mycol < N) {
    const float b = biasp ? static_cast<float>(biasp[mycol]) : 0.f;
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) Y[static_cast<uint32_t>(m) * N + mycol] = static_cast<f16>(out[m] + b);
  }
}

// Host side: argument block for a geometry and C columns per wave, and the
// workgroup's LDS bytes.
inline uint32_t dot_waves(int64_t N, int C) { return static_cast<uint32_t>((N + C - 1) / C); }

inline DotArgs dot_args(const Launch& L, int C, int W, uint32_t act_bytes) {
  DotArgs a;
  a.A = L.A;
  a.bias = L.p[0].bias;
  a.skip = L.skip;
  a.gamma = L.gamma;
  a.residual = L.residual;
  a.eps = L.eps;
  uint32_t wv = 0;  // waves before this projection
  for (int i = 0; i < 3; ++i) {
    const bool used = i < L.nproj;
    const Proj& P = L.p[used ? i : 0];
    a.p[i] = DotProj{P.B, P.scales, P.zp, P.Y, static_cast<uint32_t>(P.N), used ? wv : 0xFFFFFFFFu};
    if (used) wv += dot_waves(P.N, C);
  }
  (void)W;
  a.K = static_cast<uint32_t>(L.K);
  a.kb = static_cast<uint32_t>(L.kb);
  a.rowb = static_cast<uint32_t>(L.kb * L.blob);
  a.zesz = L.zp_dtype == DT_F32 ? 4u : 2u;
  a.zrow = L.zp_kind == ZP_PACKED ? static_cast<uint32_t>(L.zrow) : a.kb * a.zesz;
  a.M = static_cast<uint32_t>(L.M);
  a.bsl = static_cast<uint32_t>(L.bs_log2);
  const uint32_t sb = static_cast<uint32_t>(C) * a.kb * 2u;
  // + up to 3 bytes before a dword-aligned load start: scale blocks start
  // dword-aligned when C is even, packed zero-point blocks anywhere
  a.zoff = (sb + ((C & 1) ? 3u : 0u) + 15u) & ~15u;
  const uint32_t zb = L.zp_kind == ZP_NONE ? 0u : static_cast<uint32_t>(C) * a.zrow;
  a.meta_bytes = (a.zoff + zb + (L.zp_kind == ZP_PACKED ? 3u : 0u) + 15u) & ~15u;
  a.act_bytes = act_bytes;
  return a;
}

inline size_t dot_lds_bytes(const DotArgs& a, int W) { return a.act_bytes + static_cast<size_t>(W) * a.meta_bytes; }

// Launch shape of the dot GEMV: columns per wave (C) and waves per workgroup
// (W); P columns' weight loads are issued before the activation staging, so
// with P = C every weight load of a wave is in flight before its barrier
// (decode workload 7.4 us against 7.8 us with P = 1; issuing later columns'
// loads as earlier ones are consumed, or staging each lane's activations in
// registers without LDS, measured slower). Measured: 2 x 4 on the one-row
// decode workload;
// 2 x 12 with four rows (wide), where the activation staging is four times
// larger and fewer, larger workgroups amortise it; each wave picks its Qkv
// projection from its global wave index, so the Qkv GQA decode workload fills
// exactly 256 workgroups (10.67 us against 10.95 us for 8 waves x 4 columns).
// The XRMM_DOT_* macros override the shape for tuning builds; every
// translation unit of one library must see the same values.
#ifndef XRMM_DOT_P
#define XRMM_DOT_P 2
#endif
#ifndef XRMM_DOT_NARROW_C
#define XRMM_DOT_NARROW_C 2
#endif
#ifndef XRMM_DOT_NARROW_W
#define XRMM_DOT_NARROW_W 4
#endif
#ifndef XRMM_DOT_WIDE_C
#define XRMM_DOT_WIDE_C 2
#endif
#ifndef XRMM_DOT_WIDE_W
#define XRMM_DOT_WIDE_W 12
#endif
constexpr bool dot_wide(int mr, int cpl) { return mr >= 4 && cpl <= 4; }
constexpr int dot_c(int mr, int cpl) { return dot_wide(mr, cpl) ? XRMM_DOT_WIDE_C : XRMM_DOT_NARROW_C; }
constexpr int dot_w(int mr, int cpl) { return dot_wide(mr, cpl) ? XRMM_DOT_WIDE_W : XRMM_DOT_NARROW_W; }
constexpr int dot_p(int mr, int cpl) { return XRMM_DOT_P < dot_c(mr, cpl) ? XRMM_DOT_P : dot_c(mr, cpl); }

// Chunk rounds per lane (a power of two >= ceil(chunks / 64)) and rows (1, 2
// or 4) the dot GEMV is instantiated for; 0 when it does not apply.
inline int dot_cpl(const Launch& L) {
  const int64_t chunks = L.kb * L.blob / 16;
  for (int c = 1; c <= 8; c *= 2)
    if (chunks <= 64 * c) return c;
  return 0;
}

inline int dot_mr(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 0; }

// 16-byte pieces per lane that a wave's scale / zero-point block needs: 1 or
// DOT_META_PIECES (0 if the block is larger).
inline int dot_meta_pieces(const Launch& L) {
  const int64_t c = dot_c(dot_mr(L.M), dot_cpl(L));
  const int64_t sb = c * L.kb * 2;
  const int64_t zb = L.zp_kind == ZP_PACKED ? c * L.zrow
                     : L.zp_kind == ZP_FLOAT ? c * L.kb * (L.zp_dtype == DT_F32 ? 4 : 2) : 0;
  const int64_t sl = sb + ((c & 1) ? 3 : 0), zl = zb + (L.zp_kind == ZP_PACKED ? 3 : 0);  // as in dot_args
  const int64_t mx = sl > zl ? sl : zl;
  return mx <= 1024 ? 1 : mx <= 1024 * DOT_META_PIECES ? DOT_META_PIECES : 0;
}

// Whether the dot GEMV applies: rows, chunk rounds and scale blocks within its
// instantiations, and the workgroup's LDS (staged activations, W waves' scale /
// zero-point slices, the Qkv row-sum scratch and the per-wave non-finite flags)
// within 160 KB.
inline bool dot_fits(const Launch& L) {
  const int mr = dot_mr(L.M), cpl = dot_cpl(L);
  if (mr == 0 || cpl == 0 || dot_meta_pieces(L) == 0) return false;
  const int c = dot_c(mr, cpl), w = dot_w(mr, cpl), spc = L.block_size >= 32 ? 1 : 2;
  const int64_t act = int64_t(mr) * cpl * 4 * 64 * 16 + int64_t(mr) * cpl * spc * 2 * 64 * 4;
  const int64_t zesz = L.zp_dtype == DT_F32 ? 4 : 2;
  const int64_t zrow = L.zp_kind == ZP_PACKED ? L.zrow : L.kb * zesz;
  const int64_t zoff = (int64_t(c) * L.kb * 2 + ((c & 1) ? 3 : 0) + 15) & ~int64_t(15);  // as in dot_args
  const int64_t meta = (zoff + (L.zp_kind == ZP_NONE ? 0 : int64_t(c) * zrow) + (L.zp_kind == ZP_PACKED ? 3 : 0) + 15) &
                       ~int64_t(15);
  const int64_t stat = int64_t(w) * mr * 4 + int64_t(w) * 4;  // Qkv row sums, per-wave non-finite flags
  return act + w * meta + stat <= 160 * 1024;
}

template <int ZPK, int SPC, int CPL, int MR, int MP, int OPK, bool SK>
inline hipError_t launch_dot6(const Launch& L, hipStream_t st) {
  constexpr int C = dot_c(MR, CPL), W = dot_w(MR, CPL);
  const DotArgs a = dot_args(L, C, W, dot_act_bytes<MR, CPL, SPC>());
  uint32_t waves = 0;
  for (int i = 0; i < L.nproj; ++i) waves += dot_waves(L.p[i].N, C);
  const uint32_t grid = (waves + W - 1) / W;
  const size_t lds = dot_lds_bytes(a, W);
  auto kern = k_gemv_dot<ZPK, SPC, CPL, C, dot_p(MR, CPL), MR, W, MP, OPK, SK>;
  if (lds > 64 * 1024) {
    static std::atomic<int> done[kMaxDevices];  // per instantiation and device
    (void)raise_lds_cap(reinterpret_cast<const void*>(kern), static_cast<int>(160 * 1024 - 1024), done);
    (void)hipGetLastError();
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(W * 64), lds, st, a);
  return hipGetLastError();
}

template <int ZPK, int SPC, int CPL, int MR, int MP, int OPK>
inline hipError_t launch_dot5(const Launch& L, hipStream_t st) {
  if constexpr (OPK == OP_QKV)
    return L.skip ? launch_dot6<ZPK, SPC, CPL, MR, MP, OPK, true>(L, st) : launch_dot6<ZPK, SPC, CPL, MR, MP, OPK, false>(L, st);
  else
    return launch_dot6<ZPK, SPC, CPL, MR, MP, OPK, false>(L, st);
}

template <int ZPK, int SPC, int CPL, int MR, int OPK>
inline hipError_t launch_dot4(const Launch& L, hipStream_t st) {
  return dot_meta_pieces(L) == 1 ? launch_dot5<ZPK, SPC, CPL, MR, 1, OPK>(L, st)
                                 : launch_dot5<ZPK, SPC, CPL, MR, DOT_META_PIECES, OPK>(L, st);
}

template <int ZPK, int SPC, int CPL, int OPK>
inline hipError_t launch_dot3(const Launch& L, hipStream_t st) {
  switch (dot_mr(L.M)) {
    case 1: return launch_dot4<ZPK, SPC, CPL, 1, OPK>(L, st);
    case 2: return launch_dot4<ZPK, SPC, CPL, 2, OPK>(L, st);
    default: return launch_dot4<ZPK, SPC, CPL, 4, OPK>(L, st);
  }
}

template <int ZPK, int SPC, int OPK>
inline hipError_t launch_dot2(const Launch& L, hipStream_t st) {
  switch (dot_cpl(L)) {
    case 1: return launch_dot3<ZPK, SPC, 1, OPK>(L, st);
    case 2: return launch_dot3<ZPK, SPC, 2, OPK>(L, st);
    case 4: return launch_dot3<ZPK, SPC, 4, OPK>(L, st);
    default: return launch_dot3<ZPK, SPC, 8, OPK>(L, st);
  }
}

// Entry of one zero-point kind (defined in xrmm_gemv_dot_zp.hip).
template <int ZPK>
hipError_t launch_dot_for(const Launch& L, hipStream_t st);

}  // namespace xrmm
