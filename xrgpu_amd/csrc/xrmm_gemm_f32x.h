// MatMulNBits on the matrix cores with float32 arithmetic: float32
// activations, and float16 activations with 2- or 8-bit codes (whose weights
// (code - z) * scale binary16 would round), for more rows than the GEMVs serve
// well. The reference forms W = (code - z) * scale in float32 and sums x * W
// in float32 (complex_kernel.glsl:80,83).
//
// Arithmetic. The codes enter v_mfma_f32_32x32x16_f16 as the exact binary16
// integers code - z (z the packed zero point or the midpoint 2^(bits - 1)),
// each block's float32 sum is multiplied by the block's float32 scale as it
// joins the row's running sum, and the bias is added once at the end. A float
// zero point z splits into zi = rint(z) (the integer the codes meet) and
// zf = z - zi: the block then also adds -scale * zf * (the block's sum of the
// row's activations), sums the prepass computes. A row holding +-Inf or NaN
// is recomputed by k_fx_fix in the reference's serial form (the split would
// turn Inf * (code - z) into Inf * 0 where code == zi).
//  * float16 activations are exact binary16 operands: every product and every
//    block sum is exact or float32-rounded, the output is rounded once.
//  * float32 activations are first prepared by k_fx_prep: each row scaled by a
//    power of two that puts its largest finite magnitude near 2^14 (exact), and
//    every scaled value v split into hi = fp16(v) and lo = fp16(v - hi) (lo = 0
//    for non-finite v, so +-Inf and NaN reach the sums as the float32 products
//    would); each weight fragment meets hi and lo, so every product keeps
//    about 22 bits of the activation and the result meets the float32 bar
//    (1e-5 max|Y|); the power of two is undone at the end.
//
// Launches: k_fx_prep (float32 activations, or float zero points: one
// workgroup per row), k_gemm_fx
// (64-row x 256-column tiles over 8 waves of 64 x 32, K steps of 64 through a
// double-buffered LDS; the codes stay raw dwords in LDS and each wave
// dequantises a fragment's eight codes as it reads them; optionally K split
// over workgroups), with split K k_fx_combine (the splits added in split
// order, then the bias), and with float zero points k_fx_fix.
#pragma once

#include <atomic>
#include <type_traits>

#include "xrmm_device.h"

namespace xrmm {
namespace fx {

// One projection of the grid (Qkv and Mlp put theirs side by side: the same
// A, K, codes and zero-point kind).
struct Proj1 {
  const uint8_t* B;
  const void* S;      // scales [N][kb], the activations' type
  const uint8_t* Z;   // packed zero points or null
  const void* Zf;     // float zero points [N][kb] (the activations' type) or null
  const void* bias;
  void* Y;
  int N;
  int cb;  // first column among all projections' (the partials' layout)
  int ct;  // first column tile on the grid
};

struct Args {
  const void* A;     // float16 activations [M][K] (read directly)
  const f16* Ahi;    // float32 activations, prepared: [M][Kd] binary16 terms (Kd: K padded to whole K steps)
  const f16* Alo;
  Proj1 pr[3];
  int np;              // projections
  int NT;              // columns of all projections
  const int32_t* ex;   // float32 activations: the row exponents
  const float* rsum;   // float zero points: block sums of the (scaled) rows, [kb][M]
  const int32_t* bad;  // float zero points: rows holding +-Inf or NaN
  float* part;         // [splits][M][NT] with split K
  float* Yact;         // Mlp (two projections of one N): act(gate) * up [M][N] from the combine, or null
  int act;             // its activation
  int M, K, kb, bs, Kd, rowb, zrow, bits, splits;
};

// projection p of the grid (wave-uniform selects, no indexing of the argument)
__device__ __forceinline__ Proj1 pick(const Args& a, int p) { return p == 0 ? a.pr[0] : p == 1 ? a.pr[1] : a.pr[2]; }

hipError_t launch_gemm_f16(const Args& a, hipStream_t st);  // xrmm_gemm_f32x_h.hip

namespace {

constexpr int RT = 64;   // rows per tile
constexpr int CT = 256;  // columns per tile
constexpr int KS = 64;   // K step
constexpr int LD = KS + 8;
constexpr int NT = 512;

// halfs per stage: A (hi, and lo for float32 activations), then the codes as
// [fragment][column][BITS / 4 dwords] (2-bit: [fragment pair][column])
template <bool LO, int BITS>
constexpr int stage_halfs() {
  return (LO ? 2 : 1) * RT * LD + (KS / 8) * CT * BITS / 4 * 2;
}
template <bool LO, int BITS>
constexpr size_t lds_bytes() {
  return 2 * static_cast<size_t>(stage_halfs<LO, BITS>()) * sizeof(_Float16);
}

// Exponent e with |v| * 2^-e near 2^14 for the row maximum v (0 for a row
// without a nonzero finite value), at least -126 so that 2^e and 2^-e are
// both normal float32 values (rows of tiny values keep fewer bits).
__device__ __forceinline__ int row_exp(float mx) {
  if (!(mx > 0.f) || !__builtin_isfinite(mx)) return 0;
  int e = 0;
  (void)__builtin_frexpf(mx, &e);  // mx = f * 2^e, f in [0.5, 1)
  return e - 15 < -126 ? -126 : e - 15;
}

__device__ __forceinline__ float fin_abs(float x) {
  const float v = __builtin_fabsf(x);
  return __builtin_isfinite(v) ? v : 0.f;
}

// One workgroup per row. HL (float32 activations): the row's exponent into
// ex[m] and its binary16 terms hi / lo into [m][Kd] in pair order (c0 c4 c1
// c5 c2 c6 c3 c7 within each group of eight, the order the weight fragments
// are dequantised in), zero from K to Kd. RS (float zero points): whether the
// row holds +-Inf or NaN into bad[m], and the float32 sums of its (scaled)
// values over each block into rsum[b][m] (zero for such a row; each block's
// sum in a fixed order, group by group). vec: K % VW == 0 and A 16-byte
// aligned (16-byte loads), else element loads. P > 0: the row's groups of
// eight stay in registers, P per thread (Kd <= 2048 P), and the row is read
// once; P == 0: any Kd, the row is read again for each pass.
constexpr int kPrepMaxGroups = 4096;  // groups of eight with P > 0 (Kd <= 32768)

template <typename TA, bool HL, bool RS, int P>
__global__ __launch_bounds__(256) void k_fx_prep(const TA* __restrict__ A, int M, int K, int Kd, int bs, int kb, int vec,
                                                 int32_t* __restrict__ ex, f16* __restrict__ hi, f16* __restrict__ lo,
                                                 float* __restrict__ rsum, int32_t* __restrict__ bad) {
  constexpr int VW = 16 / sizeof(TA);
  __shared__ float red[4];
  __shared__ int nred[4];
  __shared__ float s_gsum[RS && P > 0 ? kPrepMaxGroups : 1];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const TA* row = A + static_cast<int64_t>(m) * K;
  const int ng = Kd / 8;
  float mx = 0.f;
  int nf = 0;
  auto see = [&](float x) {
    const float v = __builtin_fabsf(x);
    if (__builtin_isfinite(v)) mx = fmaxf(mx, v);
    else nf = 1;
  };
  // group g's eight values (zero past K)
  auto group = [&](int g, float (&x8)[8]) {
    const int k0 = g * 8;
    if (vec && VW == 4) {
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      const f32x4 v0 = k0 < K ? *reinterpret_cast<const f32x4*>(row + k0) : zero;
      const f32x4 v1 = k0 + 4 < K ? *reinterpret_cast<const f32x4*>(row + k0 + 4) : zero;
      x8[0] = v0.x, x8[1] = v0.y, x8[2] = v0.z, x8[3] = v0.w;
      x8[4] = v1.x, x8[5] = v1.y, x8[6] = v1.z, x8[7] = v1.w;
    } else if (vec) {
      const u32x4 z4 = {0u, 0u, 0u, 0u};
      const f16x8 v = __builtin_bit_cast(f16x8, k0 < K ? *reinterpret_cast<const u32x4*>(row + k0) : z4);
#pragma unroll
      for (int q = 0; q < 8; ++q) x8[q] = static_cast<float>(v[q]);
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) x8[q] = k0 + q < K ? static_cast<float>(row[k0 + q]) : 0.f;
    }
  };
  float xr[P > 0 ? P : 1][8];
  if constexpr (P > 0) {
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int g = tid + 256 * i;
      if (g < ng) {
        group(g, xr[i]);
#pragma unroll
        for (int q = 0; q < 8; ++q) see(xr[i][q]);
      }
    }
  } else if (vec) {
    for (int k = tid * VW; k < K; k += 256 * VW) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(row + k);
      if constexpr (VW == 4) {
        const f32x4 v = __builtin_bit_cast(f32x4, w);
        see(v.x), see(v.y), see(v.z), see(v.w);
      } else {
        const f16x8 v = __builtin_bit_cast(f16x8, w);
#pragma unroll
        for (int q = 0; q < 8; ++q) see(static_cast<float>(v[q]));
      }
    }
  } else {
    for (int k = tid; k < K; k += 256) see(static_cast<float>(row[k]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    nf |= __shfl_xor(nf, off, 64);
  }
  if (lane == 0) {
    red[tid >> 6] = mx;
    nred[tid >> 6] = nf;
  }
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  nf = nred[0] | nred[1] | nred[2] | nred[3];
  const int e = HL ? row_exp(mx) : 0;
  const float rs = __builtin_ldexpf(1.f, -e);
  if (tid == 0) {
    if constexpr (HL) ex[m] = e;
    if constexpr (RS) bad[m] = nf;
  }
  // the binary16 terms of one group, stored in pair order 0 4 1 5 2 6 3 7
  auto terms = [&](int g, const float (&x8)[8]) {
    f16x8 vh, vl;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float x = x8[(q >> 1) + 4 * (q & 1)] * rs;
      const f16 t = static_cast<f16>(x);
      vh[q] = t;
      vl[q] = __builtin_isfinite(x) ? static_cast<f16>(x - static_cast<float>(t)) : static_cast<f16>(0.f);
    }
    *reinterpret_cast<f16x8*>(hi + static_cast<int64_t>(m) * Kd + g * 8) = vh;
    *reinterpret_cast<f16x8*>(lo + static_cast<int64_t>(m) * Kd + g * 8) = vl;
  };
  if constexpr (P > 0) {
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int g = tid + 256 * i;
      if (g < ng) {
        if constexpr (HL) terms(g, xr[i]);
        if constexpr (RS) {
          float t = 0.f;
#pragma unroll
          for (int q = 0; q < 8; ++q) t += xr[i][q] * rs;
          s_gsum[g] = t;
        }
      }
    }
    if constexpr (RS) {
      __syncthreads();
      const int gpb = bs / 8;  // groups per block
      for (int b = tid; b < kb; b += 256) {
        float acc = 0.f;
        for (int g = b * gpb; g < (b + 1) * gpb; ++g) acc += s_gsum[g];
        rsum[static_cast<int64_t>(b) * M + m] = nf ? 0.f : acc;
      }
    }
  } else {
    if constexpr (HL) {
      for (int g = tid; g < ng; g += 256) {
        float x8[8];
        group(g, x8);
        terms(g, x8);
      }
    }
    if constexpr (RS) {
      for (int b = tid; b < kb; b += 256) {
        const int k1 = (b + 1) * bs < K ? (b + 1) * bs : K;
        float acc = 0.f;
        for (int k = b * bs; k < k1; ++k) acc += static_cast<float>(row[k]) * rs;
        rsum[static_cast<int64_t>(b) * M + m] = nf ? 0.f : acc;
      }
    }
  }
}

// The prepass for a row of Kd: P = groups of eight per thread, 0 past
// kPrepMaxGroups.
template <typename TA, bool HL, bool RS>
void launch_prep(const TA* A, int M, int K, int Kd, int bs, int kb, int vec, int32_t* ex, f16* hi, f16* lo, float* rsum,
                 int32_t* bad, hipStream_t st) {
  const dim3 g(static_cast<uint32_t>(M)), b(256);
  const int ng = Kd / 8;
  if (ng <= 256) hipLaunchKernelGGL((k_fx_prep<TA, HL, RS, 1>), g, b, 0, st, A, M, K, Kd, bs, kb, vec, ex, hi, lo, rsum, bad);
  else if (ng <= 512) hipLaunchKernelGGL((k_fx_prep<TA, HL, RS, 2>), g, b, 0, st, A, M, K, Kd, bs, kb, vec, ex, hi, lo, rsum, bad);
  else if (ng <= 1024) hipLaunchKernelGGL((k_fx_prep<TA, HL, RS, 4>), g, b, 0, st, A, M, K, Kd, bs, kb, vec, ex, hi, lo, rsum, bad);
  else if (ng <= 2048) hipLaunchKernelGGL((k_fx_prep<TA, HL, RS, 8>), g, b, 0, st, A, M, K, Kd, bs, kb, vec, ex, hi, lo, rsum, bad);
  else if (ng <= kPrepMaxGroups)
    hipLaunchKernelGGL((k_fx_prep<TA, HL, RS, 16>), g, b, 0, st, A, M, K, Kd, bs, kb, vec, ex, hi, lo, rsum, bad);
  else hipLaunchKernelGGL((k_fx_prep<TA, HL, RS, 0>), g, b, 0, st, A, M, K, Kd, bs, kb, vec, ex, hi, lo, rsum, bad);
}

// Zero points ZK: 0 none (the midpoint), 1 packed, 2 float. Block modes BKM:
// 2, 4 = blocks of 32, 64 codes (a block's sum is scaled every 2, 4 MFMA K
// slices); 8 = blocks of 128 or more (scaled at the end of every
// block_size / 64 K steps).
template <typename T, int BITS, int ZK, int BKM>
__global__ __launch_bounds__(NT, 1) void k_gemm_fx(Args a, int nct) {
  constexpr bool LO = std::is_same<T, float>::value;  // float32 activations: hi and lo terms
  constexpr int STAGE = stage_halfs<LO, BITS>();
  constexpr int NQ = BITS == 2 ? 4 : BITS == 4 ? 2 : 1;  // dequantisation constants per block
  constexpr uint32_t OOB = 0x80000000u;
  extern __shared__ __align__(16) unsigned char smem[];
  f16* lds = reinterpret_cast<f16*>(smem);
  __shared__ float s_ru[RT];  // 2^e per row
  __shared__ __align__(16) float s_rsum[2][2][RT];  // float zero points: [stage][block of the step][row]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // a wave: IM x JN MFMA tiles of 32 x 32, here 64 rows x 32 columns, so each
  // dequantised weight fragment feeds IM tiles (10-20 % faster than 32 rows x
  // 64 columns, which dequantises every fragment in two waves)
  constexpr int IM = 2, JN = 1;
  constexpr int WR = 32 * IM, WC = 32 * JN, WNW = CT / WC;
  const int wm = wave / WNW, wn = wave % WNW;
  // workgroup b: split b % splits of tile b / splits (column tiles fastest)
  const int sp = static_cast<int>(blockIdx.x) % a.splits, tb = static_cast<int>(blockIdx.x) / a.splits;
  // column tile ct of all projections' tiles: this workgroup's projection
  const int ct = tb % nct;
  const int pj = a.np > 1 && ct >= a.pr[1].ct ? (a.np > 2 && ct >= a.pr[2].ct ? 2 : 1) : 0;
  const Proj1 P = pick(a, pj);
  const int m0 = (tb / nct) * RT, n0 = (ct - P.ct) * CT;
  if constexpr (LO) {
    if (tid < RT) {
      const int m = m0 + tid;
      s_ru[tid] = __builtin_ldexpf(1.f, m < a.M ? a.ex[m] : 0);
    }
  }

  // ---- thread t stages A row t / 8, K 8 (t % 8) .. + 7 of the step, and
  // half t % 2 of column t / 2's codes of the step
  const int arow = tid >> 3, agrp = tid & 7;
  const int am = m0 + arow;
  const rsrc_t rAh = LO ? mk_rsrc(a.Ahi, static_cast<uint32_t>(a.M) * static_cast<uint32_t>(a.Kd) * 2u)
                        : mk_rsrc(a.A, static_cast<uint32_t>(a.M) * static_cast<uint32_t>(a.K) * 2u);
  const rsrc_t rAl = mk_rsrc(LO ? a.Alo : a.Ahi, LO ? static_cast<uint32_t>(a.M) * static_cast<uint32_t>(a.Kd) * 2u : 0u);
  const int bcol = tid >> 1, bh = tid & 1;
  const int bn = n0 + bcol;
  const rsrc_t rB = mk_rsrc(P.B, static_cast<uint32_t>(P.N) * static_cast<uint32_t>(a.rowb));
  const uint32_t boff = bn < P.N ? static_cast<uint32_t>(bn) * static_cast<uint32_t>(a.rowb) : OOB;
  // K steps [kstep0, kstep0 + ksteps) of this split; splits hold whole blocks
  const int kall = a.Kd / KS;
  const int bsteps = BKM == 8 ? a.bs / KS : 1;
  const int kper = ((kall + a.splits - 1) / a.splits + bsteps - 1) / bsteps * bsteps;
  const int kstep0 = sp * kper;
  const int ksteps = kall - kstep0 < kper ? kall - kstep0 : kper;

  constexpr int NB = BKM == 8 ? 1 : 4 / BKM;  // blocks touched per step
  struct Regs {
    u32x4 a[LO ? 2 : 1];
    u32x4 b[BITS == 8 ? 2 : 1];
    u32x2 b2;  // 2-bit codes
    float rs;  // float zero points: a row's block sum (threads below RT * NB)
  };
  auto gload = [&](Regs& r, int ks) {
    const bool ok = ks < ksteps;
    const int k = (kstep0 + ks) * KS + agrp * 8;
    if constexpr (ZK == 2) {
      // row tid % RT's sum over block tid / RT of the step, from an address
      // clamped into range (threads past RT * NB store nothing)
      const int f = tid / RT < NB ? tid / RT : NB - 1;
      const int kst = kstep0 + (ks < ksteps ? ks : ksteps - 1);
      const int b = BKM == 8 ? (kst * KS) / a.bs : kst * NB + f;
      const int blk = b < a.kb ? b : a.kb - 1;
      const int m = m0 + (tid & (RT - 1)) < a.M ? m0 + (tid & (RT - 1)) : a.M - 1;
      r.rs = a.rsum[static_cast<int64_t>(blk) * a.M + m];
    }
    if constexpr (LO) {
      // the prepared terms are zero from K to Kd
      const uint32_t off = ok && am < a.M ? (static_cast<uint32_t>(am) * static_cast<uint32_t>(a.Kd) + static_cast<uint32_t>(k)) * 2u : OOB;
      r.a[0] = bld16(rAh, off, 0);
      r.a[1] = bld16(rAl, off, 0);
    } else {
      // K % 8 == 0: a group of eight is whole or past K
      const bool in = ok && am < a.M && k < a.K;
      r.a[0] = bld16(rAh, in ? (static_cast<uint32_t>(am) * static_cast<uint32_t>(a.K) + static_cast<uint32_t>(k)) * 2u : OOB, 0);
    }
    const uint32_t bo = (ok ? boff : OOB) + static_cast<uint32_t>((kstep0 + ks) * KS * BITS / 8);
    if constexpr (BITS == 2) {
      r.b2 = bld8(rB, bo + bh * 8, 0);
    } else {
#pragma unroll
      for (int i = 0; i < BITS / 4; ++i) r.b[i] = bld16(rB, bo + static_cast<uint32_t>((bh * (BITS / 4) + i) * 16), 0);
    }
  };
  auto sstore = [&](const Regs& r, int stage) {
    f16* Ah = lds + stage * STAGE;
    f16* Al = Ah + RT * LD;
    uint32_t* Bw = reinterpret_cast<uint32_t*>(Ah + (LO ? 2 : 1) * RT * LD);
    if constexpr (ZK == 2) {
      if (tid < RT * NB) s_rsum[stage][tid / RT][tid & (RT - 1)] = r.rs;
    }
    if constexpr (LO) {
      *reinterpret_cast<u32x4*>(Ah + arow * LD + agrp * 8) = r.a[0];
      *reinterpret_cast<u32x4*>(Al + arow * LD + agrp * 8) = r.a[1];
    } else {
      // halfs h0..h7 -> pair order h0 h4 h1 h5 h2 h6 h3 h7 (the vector's
      // elements by name: this compiler folds v[i >> 2][i & 3] over an array
      // of vectors to element 0 of each vector)
      const u32x4 w = r.a[0];
      const u32x4 p = {__builtin_amdgcn_perm(w.z, w.x, 0x05040100u), __builtin_amdgcn_perm(w.z, w.x, 0x07060302u),
                       __builtin_amdgcn_perm(w.w, w.y, 0x05040100u), __builtin_amdgcn_perm(w.w, w.y, 0x07060302u)};
      *reinterpret_cast<u32x4*>(Ah + arow * LD + agrp * 8) = p;
    }
    if constexpr (BITS == 2) {
      // dword d of this half: fragment pair 2 bh + d
      Bw[(2 * bh) * CT + bcol] = r.b2.x;
      Bw[(2 * bh + 1) * CT + bcol] = r.b2.y;
    } else if constexpr (BITS == 4) {
      const u32x4 b0 = r.b[0];
      const uint32_t w[4] = {b0.x, b0.y, b0.z, b0.w};
#pragma unroll
      for (int d = 0; d < 4; ++d) Bw[(4 * bh + d) * CT + bcol] = w[d];
    } else {
      const u32x4 b0 = r.b[0], b1 = r.b[1];
      const uint32_t w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int d = 0; d < 4; ++d)
        *reinterpret_cast<u32x2*>(Bw + ((4 * bh + d) * CT + bcol) * 2) = u32x2{w[2 * d], w[2 * d + 1]};
    }
  };

  // this lane's columns
  int col[JN];
#pragma unroll
  for (int j = 0; j < JN; ++j) {
    const int c = n0 + wn * WC + j * 32 + (lane & 31);
    col[j] = c < P.N ? c : P.N - 1;
  }
  // Per block and column: the scale, the dequantisation constants
  // -(base + z), z the (integer) zero point, exact in binary16 (the bases are
  // the values of the magic exponents the code bits are or-ed into), and for
  // float zero points -scale * (z - zi), zi = rint(z) in [-1024, 1024].
  struct Meta {
    float s[JN];
    f16x2 n[NQ][JN];
    float nz[JN];
  };
  auto mload = [&](int blk0) {
    // a block past the last (the second half of a last K step of blocks of
    // 32) has scale zero; its codes (the next column's, or zeros) meet zero
    // activations
    const bool past = blk0 >= a.kb;
    const int blk = past ? a.kb - 1 : blk0;
    Meta mt;
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      const float sv = static_cast<float>(static_cast<const T*>(P.S)[static_cast<int64_t>(col[j]) * a.kb + blk]);
      mt.s[j] = past ? 0.f : sv;
      float z = static_cast<float>(1 << (BITS - 1));
      if constexpr (ZK == 1) {
        const uint32_t zb = P.Z[static_cast<int64_t>(col[j]) * a.zrow + (blk * BITS) / 8];
        z = static_cast<float>((zb >> ((blk * BITS) % 8)) & ((1u << BITS) - 1u));
      } else if constexpr (ZK == 2) {
        const float zv = static_cast<float>(static_cast<const T*>(P.Zf)[static_cast<int64_t>(col[j]) * a.kb + blk]);
        z = fminf(fmaxf(__builtin_rintf(zv), -1024.f), 1024.f);  // NaN -> -1024, its fraction NaN
        mt.nz[j] = past ? 0.f : -(mt.s[j] * (zv - z));
      }
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const float base = BITS == 2 ? static_cast<float>(1024 >> (2 * q)) : q == 0 ? 1024.f : 64.f;
        const f16 v = static_cast<f16>(-base - z);
        mt.n[q][j] = f16x2{v, v};
      }
    }
    return mt;
  };
  const f16x2 inv16 = {static_cast<f16>(0.0625f), static_cast<f16>(0.0625f)};
  const uint32_t sel2 = (lane >> 5) ? 0x0c030c02u : 0x0c010c00u;  // 2-bit: this lane's fragment half
  // a fragment's eight codes -> code - z as exact binary16 in pair order
  auto dq = [&](const uint32_t* w, const Meta& mt, int j) {
    const uint32_t magic = 0x64006400u;
    if constexpr (BITS == 2) {
      // bytes [c0..c3, 0, c4..c7, 0]; code bits 2q..2q+1 under magic
      // exponents of 1024, 256, 64, 16 (ulp 1, 1/4, 1/16, 1/64)
      const uint32_t t = __builtin_amdgcn_perm(0u, w[0], sel2);
      const f16x2 d0 = as_h2(and_or(t, 0x00030003u, magic)) + mt.n[0][j];
      const f16x2 d1 = as_h2(and_or(t, 0x000C000Cu, 0x5C005C00u)) + mt.n[1][j];
      const f16x2 d2 = as_h2(and_or(t, 0x00300030u, 0x54005400u)) + mt.n[2][j];
      const f16x2 d3 = as_h2(and_or(t, 0x00C000C0u, 0x4C004C00u)) + mt.n[3][j];
      return f16x8{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
    } else if constexpr (BITS == 4) {
      const uint32_t x = w[0], x8 = x >> 8;
      const f16x2 d0 = as_h2(and_or(x, 0x000F000Fu, magic)) + mt.n[0][j];
      const f16x2 d1 = __builtin_elementwise_fma(as_h2(and_or(x, 0x00F000F0u, magic)), inv16, mt.n[1][j]);
      const f16x2 d2 = as_h2(and_or(x8, 0x000F000Fu, magic)) + mt.n[0][j];
      const f16x2 d3 = __builtin_elementwise_fma(as_h2(and_or(x8, 0x00F000F0u, magic)), inv16, mt.n[1][j]);
      return f16x8{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
    } else {
      const uint32_t x0 = w[0], x1 = w[1];  // c0..c3, c4..c7
      const f16x2 d0 = as_h2(__builtin_amdgcn_perm(x1, x0, 0x0c040c00u) | magic) + mt.n[0][j];
      const f16x2 d1 = as_h2(__builtin_amdgcn_perm(x1, x0, 0x0c050c01u) | magic) + mt.n[0][j];
      const f16x2 d2 = as_h2(__builtin_amdgcn_perm(x1, x0, 0x0c060c02u) | magic) + mt.n[0][j];
      const f16x2 d3 = as_h2(__builtin_amdgcn_perm(x1, x0, 0x0c070c03u) | magic) + mt.n[0][j];
      return f16x8{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
    }
  };

  const f32x16 zero16 = {};
  f32x16 acc[IM * JN], yacc[IM * JN];  // tile (i, j) at i JN + j
#pragma unroll
  for (int t = 0; t < IM * JN; ++t) {
    acc[t] = zero16;
    yacc[t] = zero16;
  }
  // a block's sums into the running sums (with float zero points, plus
  // -scale * zf * the row's block sum, block f of the step on `stage`);
  // blocks of 128 or more codes start from zeroed sums, shorter ones from a
  // zero accumulator operand
  auto flush = [&](const Meta& mt, int stage, int f) {
    float rr[IM][16];
    if constexpr (ZK == 2) {
#pragma unroll
      for (int i = 0; i < IM; ++i) {
        // row tile i's rows wm WR + 32 i + 8 (q / 4) + 4 (lane / 32) + q % 4, by name
        const float* rp = &s_rsum[stage][f][wm * WR + 32 * i + 4 * (lane >> 5)];
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(rp), v1 = *reinterpret_cast<const f32x4*>(rp + 8);
        const f32x4 v2 = *reinterpret_cast<const f32x4*>(rp + 16), v3 = *reinterpret_cast<const f32x4*>(rp + 24);
        const float t[16] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
#pragma unroll
        for (int q = 0; q < 16; ++q) rr[i][q] = t[q];
      }
    }
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
      for (int j = 0; j < JN; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          float y = yacc[i * JN + j][q];
          if constexpr (ZK == 2) y = __builtin_fmaf(mt.nz[j], rr[i][q], y);
          yacc[i * JN + j][q] = __builtin_fmaf(mt.s[j], acc[i * JN + j][q], y);
          if constexpr (BKM == 8) acc[i * JN + j][q] = 0.f;
        }
  };
  auto mfmas = [&](int stage, const Meta (&mt)[NB]) {
    const f16* Ah = lds + stage * STAGE;
    const f16* Al = Ah + RT * LD;
    const uint32_t* Bw = reinterpret_cast<const uint32_t*>(Ah + (LO ? 2 : 1) * RT * LD);
#pragma unroll
    for (int kk = 0; kk < KS / 16; ++kk) {
      const int ko = kk * 16 + (lane >> 5) * 8;
      f16x8 fh[IM], fl[IM];
#pragma unroll
      for (int i = 0; i < IM; ++i) {
        const int ar = wm * WR + 32 * i + (lane & 31);
        fh[i] = *reinterpret_cast<const f16x8*>(Ah + ar * LD + ko);
        if constexpr (LO) fl[i] = *reinterpret_cast<const f16x8*>(Al + ar * LD + ko);
      }
      const Meta& m = mt[BKM == 8 ? 0 : kk / BKM];
      const bool first = BKM != 8 && kk % BKM == 0;
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const int c = wn * WC + j * 32 + (lane & 31);
        const uint32_t* w = BITS == 2 ? Bw + kk * CT + c : Bw + ((ko >> 3) * CT + c) * (BITS / 4);
        const f16x8 fb = dq(w, m, j);
#pragma unroll
        for (int i = 0; i < IM; ++i) {
          f32x16& ac = acc[i * JN + j];
          ac = __builtin_amdgcn_mfma_f32_32x32x16_f16(fh[i], fb, first ? zero16 : ac, 0, 0, 0);
          if constexpr (LO) ac = __builtin_amdgcn_mfma_f32_32x32x16_f16(fl[i], fb, ac, 0, 0, 0);
        }
      }
      if constexpr (BKM != 8) {
        if ((kk + 1) % BKM == 0) flush(m, stage, kk / BKM);
      }
    }
  };
  // the block metadata of step ks (clamped to the split's last step, so a
  // prefetch past the end reads in bounds)
  auto mstep = [&](Meta (&mt)[NB], int ks) {
    const int kg = kstep0 + (ks < ksteps ? ks : ksteps - 1);
#pragma unroll
    for (int f = 0; f < NB; ++f) mt[f] = mload(BKM == 8 ? (kg * KS) / a.bs : kg * NB + f);
  };
  // step ks on stage ks % 2 with its metadata `mc` (loaded a step earlier):
  // `mn` receives step ks + 1's metadata and `fill` step ks + 2's operands,
  // both issued before the matrix work so their latency hides behind it;
  // `nxt` (step ks + 1) goes to the other stage
  auto step = [&](int ks, int stage, Regs& nxt, Regs& fill, const Meta (&mc)[NB], Meta (&mn)[NB]) {
    mstep(mn, ks + 1);
    gload(fill, ks + 2);
    // the loads stay ahead of the matrix work (the scheduler would sink them
    // below the stores of `nxt`, whose wait would then drain them as well)
    __builtin_amdgcn_sched_barrier(0);
    mfmas(stage, mc);
    if constexpr (BKM == 8) {
      if ((kstep0 + ks + 1) % bsteps == 0) flush(mc[0], stage, 0);
    }
    if (ks + 1 < ksteps) sstore(nxt, stage ^ 1);
    __syncthreads();
  };
  __syncthreads();  // s_ru
  if (ksteps > 0) {  // uniform: a split past the end keeps zero sums
    Regs r0, r1;
    Meta m0[NB], m1[NB];
    mstep(m0, 0);
    gload(r0, 0);
    gload(r1, 1);
    sstore(r0, 0);
    __syncthreads();
    int ks = 0;
    for (; ks + 1 < ksteps; ks += 2) {
      step(ks, 0, r1, r0, m0, m1);
      step(ks + 1, 1, r0, r1, m1, m0);
    }
    if (ks < ksteps) step(ks, 0, r1, r0, m0, m1);
  }

  // ---- epilogue: lane holds D[8 (q / 4) + 4 (lane / 32) + q % 4][lane % 32]
#pragma unroll
  for (int j = 0; j < JN; ++j) {
    const int c = n0 + wn * WC + j * 32 + (lane & 31);
    if (c >= P.N) continue;
    const float b = (a.splits == 1 && P.bias) ? static_cast<float>(static_cast<const T*>(P.bias)[c]) : 0.f;
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int r = wm * WR + 32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
        const int m = m0 + r;
        if (m >= a.M) continue;
        const float v = LO ? yacc[i * JN + j][q] * s_ru[r] : yacc[i * JN + j][q];
        if (a.splits == 1) static_cast<T*>(P.Y)[static_cast<int64_t>(m) * P.N + c] = static_cast<T>(v + b);
        else a.part[(static_cast<int64_t>(sp) * a.M + m) * a.NT + P.cb + c] = v;
      }
  }
}

// Every split's partial is loaded before the first add (a loop of dependent
// load-then-add pays the memory latency once per split).
constexpr int kMaxSplits = 8;

// Y = the splits' partials added in split order, then the bias, rounded once
// (element i of [M][NT]: the projection of its column). With Yact (Mlp: gate
// and up of one N side by side), element i of [M][N] is act(gate) * up of
// the two sums, as float32 gate / up rows would give it.
template <typename T>
__global__ __launch_bounds__(256) void k_fx_combine(Args a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t MN = static_cast<int64_t>(a.M) * a.NT;
  if (a.Yact) {
    const int N = a.pr[0].N;
    if (i >= static_cast<int64_t>(a.M) * N) return;
    const int64_t m = i / N, c = i % N, ig = m * a.NT + c, iu = ig + N;
    float gv[kMaxSplits], uv[kMaxSplits];
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) {
      gv[s] = s < a.splits ? a.part[s * MN + ig] : 0.f;
      uv[s] = s < a.splits ? a.part[s * MN + iu] : 0.f;
    }
    float g = gv[0], u = uv[0];
#pragma unroll
    for (int s = 1; s < kMaxSplits; ++s)
      if (s < a.splits) {
        g += gv[s];
        u += uv[s];
      }
    if (a.pr[0].bias) g += static_cast<float>(static_cast<const T*>(a.pr[0].bias)[c]);
    if (a.pr[1].bias) u += static_cast<float>(static_cast<const T*>(a.pr[1].bias)[c]);
    a.Yact[i] = activate(g, a.act) * u;
    return;
  }
  if (i >= MN) return;
  const int m = static_cast<int>(i / a.NT), gc = static_cast<int>(i % a.NT);
  const int pj = a.np > 1 && gc >= a.pr[1].cb ? (a.np > 2 && gc >= a.pr[2].cb ? 2 : 1) : 0;
  const Proj1 P = pick(a, pj);
  const int c = gc - P.cb;
  float v[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) v[s] = s < a.splits ? a.part[s * MN + i] : 0.f;
  float y = v[0];
#pragma unroll
  for (int s = 1; s < kMaxSplits; ++s)
    if (s < a.splits) y += v[s];
  if (P.bias) y += static_cast<float>(static_cast<const T*>(P.bias)[c]);
  static_cast<T*>(P.Y)[static_cast<int64_t>(m) * P.N + c] = static_cast<T>(y);
}

// Float zero points: rows holding +-Inf or NaN recomputed in the reference's
// serial form, W = (code - z) * scale in float32 and one float32 sum over K
// (complex_kernel.glsl:80,83); one workgroup per row, the others exit at once.
template <typename T, int BITS>
__global__ __launch_bounds__(256) void k_fx_fix(Args a) {
  const int m = blockIdx.x;
  if (!a.bad[m]) return;
  const T* row = static_cast<const T*>(a.A) + static_cast<int64_t>(m) * a.K;
  const int blob = a.bs * BITS / 8;
  for (int g = threadIdx.x; g < a.NT; g += 256) {
    const int pj = a.np > 1 && g >= a.pr[1].cb ? (a.np > 2 && g >= a.pr[2].cb ? 2 : 1) : 0;
    const Proj1 P = pick(a, pj);
    const int n = g - P.cb;
    const T* S = static_cast<const T*>(P.S);
    const T* Zf = static_cast<const T*>(P.Zf);
    const uint8_t* Bn = P.B + static_cast<int64_t>(n) * a.rowb;
    float acc = 0.f;
    for (int k = 0; k < a.K; ++k) {
      const int b = k / a.bs, e = k - b * a.bs;
      const uint32_t c = (static_cast<uint32_t>(Bn[b * blob + (e * BITS) / 8]) >> ((e * BITS) % 8)) & ((1u << BITS) - 1u);
      const int64_t i = static_cast<int64_t>(n) * a.kb + b;
      const float w = (static_cast<float>(c) - static_cast<float>(Zf[i])) * static_cast<float>(S[i]);
      acc += static_cast<float>(row[k]) * w;
    }
    if (P.bias) acc += static_cast<float>(static_cast<const T*>(P.bias)[n]);
    static_cast<T*>(P.Y)[static_cast<int64_t>(m) * P.N + n] = static_cast<T>(acc);
  }
}

template <typename T, int BITS, int ZK, int BKM>
hipError_t launch1(const Args& a, int nct, int64_t grid, hipStream_t st) {
  auto kern = k_gemm_fx<T, BITS, ZK, BKM>;
  constexpr size_t lds = lds_bytes<std::is_same<T, float>::value, BITS>();
  if constexpr (lds > 64 * 1024) {
    static std::atomic<int> done[kMaxDevices];  // per instantiation and device
    if (hipError_t e = raise_lds_cap(reinterpret_cast<const void*>(kern), static_cast<int>(lds), done); e != hipSuccess)
      return e;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(grid)), dim3(NT), lds, st, a, nct);
  return hipGetLastError();
}

// Blocks of 32 with float zero points are not instantiated (their block
// metadata and row sums would spill).
template <typename T, int BITS, int ZK>
hipError_t launch_b(const Args& a, int nct, int64_t grid, hipStream_t st) {
  if (a.bs == 32) {
    if constexpr (ZK == 2) return hipErrorInvalidValue;
    else return launch1<T, BITS, ZK, 2>(a, nct, grid, st);
  }
  if (a.bs == 64) return launch1<T, BITS, ZK, 4>(a, nct, grid, st);
  return launch1<T, BITS, ZK, 8>(a, nct, grid, st);
}

template <typename T, int BITS>
hipError_t launch_z(const Args& a, int nct, int64_t grid, hipStream_t st) {
  if (a.pr[0].Zf) {
    if (hipError_t e = launch_b<T, BITS, 2>(a, nct, grid, st); e != hipSuccess) return e;
    if (a.splits > 1) {
      const int64_t MN = static_cast<int64_t>(a.M) * a.NT;
      hipLaunchKernelGGL(k_fx_combine<T>, dim3(static_cast<uint32_t>((MN + 255) / 256)), dim3(256), 0, st, a);
    }
    hipLaunchKernelGGL((k_fx_fix<T, BITS>), dim3(static_cast<uint32_t>(a.M)), dim3(256), 0, st, a);
    return hipGetLastError();
  }
  hipError_t e = a.pr[0].Z ? launch_b<T, BITS, 1>(a, nct, grid, st) : launch_b<T, BITS, 0>(a, nct, grid, st);
  if (e != hipSuccess) return e;
  if (a.splits > 1) {
    const int64_t MN = static_cast<int64_t>(a.M) * (a.Yact ? a.pr[0].N : a.NT);
    hipLaunchKernelGGL(k_fx_combine<T>, dim3(static_cast<uint32_t>((MN + 255) / 256)), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

// The GEMM (then the combine with split K, and the recomputation of
// non-finite rows with float zero points) for activations of type T.
template <typename T>
hipError_t launch_gemm(const Args& a, hipStream_t st) {
  int nct = 0;
  for (int p = 0; p < a.np; ++p) nct += (a.pr[p].N + CT - 1) / CT;
  const int64_t grid = static_cast<int64_t>((a.M + RT - 1) / RT) * nct * a.splits;
  if (a.bits == 8) return launch_z<T, 8>(a, nct, grid, st);
  if (a.bits == 2) return launch_z<T, 2>(a, nct, grid, st);
  return launch_z<T, 4>(a, nct, grid, st);
}

}  // namespace

}  // namespace fx
}  // namespace xrmm
