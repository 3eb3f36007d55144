// MatMulNBits on the matrix cores with float32 arithmetic: float32
// activations, and float16 activations with 2- or 8-bit codes (whose weights
// (code - z) * scale binary16 would round), for more rows than the GEMVs serve
// well. The reference forms W = (code - z) * scale in float32 and sums x * W
// in float32 (complex_kernel.glsl:80,83).
//
// Arithmetic. The codes enter v_mfma_f32_32x32x16_f16 as the exact binary16
// integers code - z (z the packed zero point or the midpoint 2^(bits - 1)),
// each block's float32 sum is multiplied by the block's float32 scale as it
// joins the row's running sum, and the bias is added once at the end.
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
// Launches: k_fx_prep (float32 only: one workgroup per row), k_gemm_fx
// (64-row x 256-column tiles over 8 waves of 32 x 64, K steps of 64 through a
// double-buffered LDS; the codes stay raw dwords in LDS and each wave
// dequantises a fragment's eight codes as it reads them; optionally K split
// over workgroups), and with split K k_fx_combine (the splits added in split
// order, then the bias).
#pragma once

#include <atomic>
#include <type_traits>

#include "xrmm_device.h"

namespace xrmm {
namespace fx {

struct Args {
  const void* A;     // float16 activations [M][K] (read directly)
  const f16* Ahi;    // float32 activations, prepared: [M][Kd] binary16 terms
  const f16* Alo;
  const uint8_t* B;
  const void* S;     // scales [N][kb], the activations' type
  const uint8_t* Z;  // packed zero points or null
  const void* bias;
  void* Y;
  const int32_t* ex;  // float32 activations: the row exponents
  float* part;        // [splits][M][N] with split K
  int M, K, N, kb, bs, Kd, rowb, zrow, bits, splits;
};

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

// One workgroup per float32 row: its exponent into ex[m] and its binary16
// terms hi / lo into [m][Kd] in pair order (c0 c4 c1 c5 c2 c6 c3 c7 within
// each group of eight, the order the weight fragments are dequantised in),
// zero from K to Kd. Needs K % 4 == 0 and a 16-byte aligned A.
__global__ __launch_bounds__(256) void k_fx_prep(const float* __restrict__ A, int K, int Kd, int32_t* __restrict__ ex,
                                                 f16* __restrict__ hi, f16* __restrict__ lo) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const float* row = A + static_cast<int64_t>(m) * K;
  float mx = 0.f;
  for (int k = tid * 4; k < K; k += 1024) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(row + k);
    mx = fmaxf(fmaxf(mx, fin_abs(v.x)), fmaxf(fin_abs(v.y), fmaxf(fin_abs(v.z), fin_abs(v.w))));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const int e = row_exp(mx);
  if (tid == 0) ex[m] = e;
  const float rs = __builtin_ldexpf(1.f, -e);
  f16* h = hi + static_cast<int64_t>(m) * Kd;
  f16* l = lo + static_cast<int64_t>(m) * Kd;
  for (int g = tid; g < Kd / 8; g += 256) {
    const int k0 = g * 8;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const f32x4 v0 = k0 < K ? *reinterpret_cast<const f32x4*>(row + k0) : zero;
    const f32x4 v1 = k0 + 4 < K ? *reinterpret_cast<const f32x4*>(row + k0 + 4) : zero;
    const float xs[8] = {v0.x, v1.x, v0.y, v1.y, v0.z, v1.z, v0.w, v1.w};  // pair order
    f16x8 vh, vl;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float x = xs[q] * rs;
      const f16 t = static_cast<f16>(x);
      vh[q] = t;
      vl[q] = __builtin_isfinite(x) ? static_cast<f16>(x - static_cast<float>(t)) : static_cast<f16>(0.f);
    }
    *reinterpret_cast<f16x8*>(h + k0) = vh;
    *reinterpret_cast<f16x8*>(l + k0) = vl;
  }
}

// Block modes: 2, 4 = blocks of 32, 64 codes (a block's sum is scaled every
// 2, 4 MFMA K slices); 8 = blocks of 128 or more (scaled at the end of every
// block_size / 64 K steps).
template <typename T, int BITS, bool ZP, int BKM>
__global__ __launch_bounds__(NT, 1) void k_gemm_fx(Args a, int nct) {
  constexpr bool LO = std::is_same<T, float>::value;  // float32 activations: hi and lo terms
  constexpr int STAGE = stage_halfs<LO, BITS>();
  constexpr int NQ = BITS == 2 ? 4 : BITS == 4 ? 2 : 1;  // dequantisation constants per block
  constexpr uint32_t OOB = 0x80000000u;
  extern __shared__ __align__(16) unsigned char smem[];
  f16* lds = reinterpret_cast<f16*>(smem);
  __shared__ float s_ru[RT];  // 2^e per row
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  // workgroup b: split b % splits of tile b / splits (column tiles fastest)
  const int sp = static_cast<int>(blockIdx.x) % a.splits, tb = static_cast<int>(blockIdx.x) / a.splits;
  const int m0 = (tb / nct) * RT, n0 = (tb % nct) * CT;
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
  const rsrc_t rB = mk_rsrc(a.B, static_cast<uint32_t>(a.N) * static_cast<uint32_t>(a.rowb));
  const uint32_t boff = bn < a.N ? static_cast<uint32_t>(bn) * static_cast<uint32_t>(a.rowb) : OOB;
  // K steps [kstep0, kstep0 + ksteps) of this split; splits hold whole blocks
  const int kall = a.Kd / KS;
  const int bsteps = BKM == 8 ? a.bs / KS : 1;
  const int kper = ((kall + a.splits - 1) / a.splits + bsteps - 1) / bsteps * bsteps;
  const int kstep0 = sp * kper;
  const int ksteps = kall - kstep0 < kper ? kall - kstep0 : kper;

  struct Regs {
    u32x4 a[LO ? 2 : 1];
    u32x4 b[BITS == 8 ? 2 : 1];
    u32x2 b2;  // 2-bit codes
  };
  auto gload = [&](Regs& r, int ks) {
    const bool ok = ks < ksteps;
    const int k = (kstep0 + ks) * KS + agrp * 8;
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

  // this lane's two columns
  int col[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = n0 + wn * 64 + j * 32 + (lane & 31);
    col[j] = c < a.N ? c : a.N - 1;
  }
  // Per block and column: the scale and the dequantisation constants
  // -(base + z), z the zero point, exact in binary16; the bases are the
  // values of the magic exponents the code bits are or-ed into.
  struct Meta {
    float s[2];
    f16x2 n[NQ][2];
  };
  auto mload = [&](int blk) {
    Meta mt;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      mt.s[j] = static_cast<float>(static_cast<const T*>(a.S)[static_cast<int64_t>(col[j]) * a.kb + blk]);
      float z = static_cast<float>(1 << (BITS - 1));
      if constexpr (ZP) {
        const uint32_t zb = a.Z[static_cast<int64_t>(col[j]) * a.zrow + (blk * BITS) / 8];
        z = static_cast<float>((zb >> ((blk * BITS) % 8)) & ((1u << BITS) - 1u));
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
  f32x16 acc[2], yacc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    acc[j] = zero16;
    yacc[j] = zero16;
  }
  // a block's sums into the running sums; blocks of 128 or more codes start
  // from zeroed sums, shorter ones from a zero accumulator operand
  auto flush = [&](const Meta& mt) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        yacc[j][q] = __builtin_fmaf(mt.s[j], acc[j][q], yacc[j][q]);
        if constexpr (BKM == 8) acc[j][q] = 0.f;
      }
  };
  constexpr int NB = BKM == 8 ? 1 : 4 / BKM;  // blocks touched per step
  auto mfmas = [&](int stage, const Meta (&mt)[NB]) {
    const f16* Ah = lds + stage * STAGE;
    const f16* Al = Ah + RT * LD;
    const uint32_t* Bw = reinterpret_cast<const uint32_t*>(Ah + (LO ? 2 : 1) * RT * LD);
#pragma unroll
    for (int kk = 0; kk < KS / 16; ++kk) {
      const int ko = kk * 16 + (lane >> 5) * 8;
      const int ar = wm * 32 + (lane & 31);
      const f16x8 fh = *reinterpret_cast<const f16x8*>(Ah + ar * LD + ko);
      f16x8 fl;
      if constexpr (LO) fl = *reinterpret_cast<const f16x8*>(Al + ar * LD + ko);
      const Meta& m = mt[BKM == 8 ? 0 : kk / BKM];
      const bool first = BKM != 8 && kk % BKM == 0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = wn * 64 + j * 32 + (lane & 31);
        const uint32_t* w = BITS == 2 ? Bw + kk * CT + c : Bw + ((ko >> 3) * CT + c) * (BITS / 4);
        const f16x8 fb = dq(w, m, j);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fh, fb, first ? zero16 : acc[j], 0, 0, 0);
        if constexpr (LO) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fl, fb, acc[j], 0, 0, 0);
      }
      if constexpr (BKM != 8) {
        if ((kk + 1) % BKM == 0) flush(m);
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
      if ((kstep0 + ks + 1) % bsteps == 0) flush(mc[0]);
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
  for (int j = 0; j < 2; ++j) {
    const int c = n0 + wn * 64 + j * 32 + (lane & 31);
    if (c >= a.N) continue;
    const float b = (a.splits == 1 && a.bias) ? static_cast<float>(static_cast<const T*>(a.bias)[c]) : 0.f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int r = wm * 32 + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
      const int m = m0 + r;
      if (m >= a.M) continue;
      const float v = LO ? yacc[j][q] * s_ru[r] : yacc[j][q];
      if (a.splits == 1) static_cast<T*>(a.Y)[static_cast<int64_t>(m) * a.N + c] = static_cast<T>(v + b);
      else a.part[(static_cast<int64_t>(sp) * a.M + m) * a.N + c] = v;
    }
  }
}

// Y = the splits' partials added in split order, then the bias, rounded once.
template <typename T>
__global__ __launch_bounds__(256) void k_fx_combine(Args a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t MN = static_cast<int64_t>(a.M) * a.N;
  if (i >= MN) return;
  float y = a.part[i];
  for (int s = 1; s < a.splits; ++s) y += a.part[s * MN + i];
  if (a.bias) y += static_cast<float>(static_cast<const T*>(a.bias)[i % a.N]);
  static_cast<T*>(a.Y)[i] = static_cast<T>(y);
}

template <typename T, int BITS, bool ZP, int BKM>
hipError_t launch1(const Args& a, int nct, int64_t grid, hipStream_t st) {
  auto kern = k_gemm_fx<T, BITS, ZP, BKM>;
  constexpr size_t lds = lds_bytes<std::is_same<T, float>::value, BITS>();
  if constexpr (lds > 64 * 1024) {
    static std::atomic<int> done[kMaxDevices];  // per instantiation and device
    if (hipError_t e = raise_lds_cap(reinterpret_cast<const void*>(kern), static_cast<int>(lds), done); e != hipSuccess)
      return e;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(grid)), dim3(NT), lds, st, a, nct);
  return hipGetLastError();
}

template <typename T, int BITS, bool ZP>
hipError_t launch_b(const Args& a, int nct, int64_t grid, hipStream_t st) {
  if (a.bs == 32) return launch1<T, BITS, ZP, 2>(a, nct, grid, st);
  if (a.bs == 64) return launch1<T, BITS, ZP, 4>(a, nct, grid, st);
  return launch1<T, BITS, ZP, 8>(a, nct, grid, st);
}

// The GEMM (and the combine with split K) for activations of type T.
template <typename T>
hipError_t launch_gemm(const Args& a, hipStream_t st) {
  const int nct = (a.N + CT - 1) / CT;
  const int64_t grid = static_cast<int64_t>((a.M + RT - 1) / RT) * nct * a.splits;
  const bool zp = a.Z != nullptr;
  hipError_t e;
  if (a.bits == 8) e = zp ? launch_b<T, 8, true>(a, nct, grid, st) : launch_b<T, 8, false>(a, nct, grid, st);
  else if (a.bits == 2) e = zp ? launch_b<T, 2, true>(a, nct, grid, st) : launch_b<T, 2, false>(a, nct, grid, st);
  else e = zp ? launch_b<T, 4, true>(a, nct, grid, st) : launch_b<T, 4, false>(a, nct, grid, st);
  if (e != hipSuccess) return e;
  if (a.splits > 1) {
    const int64_t MN = static_cast<int64_t>(a.M) * a.N;
    hipLaunchKernelGGL(k_fx_combine<T>, dim3(static_cast<uint32_t>((MN + 255) / 256)), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace

}  // namespace fx
}  // namespace xrmm
