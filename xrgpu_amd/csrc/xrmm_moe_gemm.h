// Grouped-expert QMoE for many tokens (included by xrmm_moe.hip): instead of
// one pass over an expert's rows per (token, slot) pair, the pairs routed to
// each expert are gathered into the rows of one GEMM per expert, so every
// expert matrix is read once per 64 pairs.
//
// Launches (row scales, 4-bit codes):
//  1. routing (k_moe_route with the row exponents of x, below);
//  2. k_moe_group: per-expert pair counts, offsets, row-tile offsets and the
//     pair lists (one workgroup; the order of pairs inside a list does not
//     change any result, every GEMM row being independent);
//  3. k_moe_ggemm FC1: rows = an expert's pairs (their tokens' x), columns =
//     its FC1 rows, K = H; the epilogue applies the row scale, the activation
//     (SwiGLU rows 2j / 2j + 1 sit in neighbouring lanes) and writes h[pair],
//     folding each pair's largest |h| into an arrival-order-free atomic max;
//  4. k_moe_ggemm FC2: rows = the pairs' h, columns = the expert's FC2 rows,
//     K = I, split over a.ks workgroups when the tiles are few; writes each
//     split's yp[pair][split] (row scale applied);
//  5. k_moe_combine: y[t] = sum over slots (ascending expert index) of
//     w * (the slot's splits summed in split order), one fused multiply-add
//     per slot in slot order.
//
// Arithmetic. The codes enter v_mfma_f32_32x32x16_f16 as the exact binary16
// integers code - 8 (no scale), the row scale multiplies the float32 sum. The
// float32 activations are split into two binary16 terms per element: a row
// is first scaled by a power of two that puts its largest finite magnitude
// near 2^14 (exact), then hi = binary16(v) and lo = binary16(v - hi); the
// MFMA takes hi and lo against the same weights, so each product keeps about
// 22 bits of the activation, and the power of two is undone on the sum.
// Non-finite activations keep lo = 0, so +-Inf and NaN reach the sums as the
// reference's float32 products would.
#pragma once

namespace xrmm {
namespace {

constexpr int MG_RT = 64;   // pairs per row tile
constexpr int MG_CT = 256;  // columns per tile
constexpr int MG_K = 64;    // K step
constexpr int MG_LD = MG_K + 8;
constexpr int MG_T = 512;   // threads: 8 waves, 2 (rows of 32) x 4 (columns of 64)
// halfs per stage: A hi, A lo (rows of MG_LD), then the raw codes as
// [fragment of the step][column], a fragment being eight codes (one dword
// of 4-bit codes, two of 8-bit codes)
template <int BITS>
constexpr int mg_stage() {
  return 2 * MG_RT * MG_LD + (MG_K / 8) * MG_CT * (BITS / 4) * 2;
}
template <int BITS>
constexpr size_t mg_lds() {
  return 2 * mg_stage<BITS>() * sizeof(_Float16);
}

// Block-scale modes of the GEMM: 0 = one scale per row (applied to the row's
// sum in the epilogue); 1, 2, 4 = blocks of 16, 32, 64 codes (a block's sum
// is scaled and added every 1, 2, 4 MFMA K slices); 8 = blocks of 128 or
// more (scaled at the end of every block_size / 64 K steps).
inline int mg_block_mode(int bs) { return bs == 0 ? 0 : bs == 16 ? 1 : bs == 32 ? 2 : bs == 64 ? 4 : 8; }

// Lists of the grouped path, inside the workspace's counter region.
struct MgLists {
  int32_t* off;    // [E + 1] first list entry of each expert
  int32_t* toff;   // [E + 1] first row tile of each expert
  int32_t* list;   // [T k] pair indices grouped by expert
  uint32_t* hmax;  // [T k] bits of the largest finite |h| of each pair
  int32_t* ex;     // [T] row exponent of x
};

// Exponent e such that |v| * 2^-e is near 2^14 for the row maximum v
// (0 for an all-zero row).
__device__ __forceinline__ int mg_row_exp(float mx) {
  if (!(mx > 0.f) || !__builtin_isfinite(mx)) return 0;
  int e = 0;
  (void)__builtin_frexpf(mx, &e);  // mx = f * 2^e, f in [0.5, 1)
  return e - 15;
}

// Row exponents of x: one wave per token, over the row's finite |x|.
__global__ __launch_bounds__(256) void k_moe_xexp(const float* __restrict__ x, int T, int64_t H, int32_t* __restrict__ ex) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;  // whole waves
  const float* xr = x + static_cast<int64_t>(t) * H;
  float m = 0.f;
  for (int64_t i = lane; i < H; i += 64) {
    const float v = __builtin_fabsf(xr[i]);
    if (__builtin_isfinite(v)) m = fmaxf(m, v);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (lane == 0) ex[t] = mg_row_exp(m);
}

// Pair counts, offsets and lists; also clears hmax. One workgroup of
// MG_T threads; E <= kMoeGroupMaxExperts (LDS counters).
__global__ __launch_bounds__(MG_T) void k_moe_group(const int32_t* __restrict__ sel, int npairs, int E, MgLists g) {
  __shared__ int cnt[kMoeGroupMaxExperts];
  __shared__ int part[MG_T];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += MG_T) cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < npairs; p += MG_T) {
    const int e = min(max(sel[p], 0), E - 1);
    atomicAdd(&cnt[e], 1);
    g.hmax[p] = 0u;
  }
  __syncthreads();
  // exclusive scans of the counts and of the row tiles: each thread sums a
  // run of experts, the runs' totals are scanned in LDS
  const int per = (E + MG_T - 1) / MG_T, e0 = tid * per;
  int s = 0, st = 0;
  for (int e = e0; e < e0 + per && e < E; ++e) {
    s += cnt[e];
    st += (cnt[e] + MG_RT - 1) / MG_RT;
  }
  part[tid] = s;
  __syncthreads();
  for (int d = 1; d < MG_T; d <<= 1) {
    const int v = tid >= d ? part[tid - d] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  const int sbase = part[tid] - s;
  __syncthreads();
  part[tid] = st;
  __syncthreads();
  for (int d = 1; d < MG_T; d <<= 1) {
    const int v = tid >= d ? part[tid - d] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  const int tbase = part[tid] - st;
  int a = sbase, b = tbase;
  for (int e = e0; e < e0 + per && e < E; ++e) {
    g.off[e] = a;
    g.toff[e] = b;
    const int c = cnt[e];
    a += c;
    b += (c + MG_RT - 1) / MG_RT;
  }
  if (tid == MG_T - 1) {
    g.off[E] = a;  // the last thread's run ends at E
    g.toff[E] = b;
  }
  __syncthreads();
  // positions: a cursor per expert (the order inside a list is free)
  for (int e = tid; e < E; e += MG_T) cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < npairs; p += MG_T) {
    const int e = min(max(sel[p], 0), E - 1);
    const int pos = atomicAdd(&cnt[e], 1);
    g.list[g.off[e] + pos] = p;
  }
}

enum MgStage { MG_FC1_RELU = 0, MG_FC1_SWIGLU = 1, MG_FC2 = 2 };

// Largest finite |v| over the 32 lanes of a lane half (lanes l, l ^ 1, ... l ^ 16).
__device__ __forceinline__ float mg_half_max(float v) {
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// One 64-pair x 256-column tile of an expert's matrix; BITS-bit codes, block
// mode BKM (mg_block_mode).
template <int ST, int BITS, int BKM>
__global__ __launch_bounds__(MG_T, 2) void k_moe_ggemm(MoeArgs a, MgLists g, int nct) {
  constexpr bool FC2 = ST == MG_FC2;
  constexpr int MG_STAGE = mg_stage<BITS>();
  constexpr int BW = BITS / 4;  // dwords per fragment
  extern __shared__ __align__(16) unsigned char smem[];
  f16* lds = reinterpret_cast<f16*>(smem);
  __shared__ int s_pair[MG_RT];
  __shared__ float s_rs[MG_RT];  // 2^-e per row (staging)
  __shared__ float s_ru[MG_RT];  // 2^e per row (epilogue)
  constexpr uint32_t OOB = 0x80000000u;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int E = static_cast<int>(a.E);
  // FC2: workgroup b is split b % ks of tile b / ks
  const int ks2 = FC2 ? a.ks : 1;
  const int sp = static_cast<int>(blockIdx.x) % ks2, tb = static_cast<int>(blockIdx.x) / ks2;
  const int rt = tb / nct, ct = tb % nct;
  const int total = g.toff[E];
  if (rt >= total) return;  // uniform: the grid is an upper bound of the row tiles
  // expert of this row tile: the last e with toff[e] <= rt
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (g.toff[mid] <= rt) lo = mid;
    else hi = mid - 1;
  }
  const int e = lo;
  const int lb = g.off[e] + (rt - g.toff[e]) * MG_RT;  // first list entry of the tile
  const int nrow = min(MG_RT, g.off[e + 1] - lb);
  const int Kd = static_cast<int>(FC2 ? a.I : a.H);   // reduction length
  const int Nd = static_cast<int>(FC2 ? a.H : a.F1);  // rows of the expert matrix
  const int n0 = ct * MG_CT;
  if (tid < MG_RT) {
    const int p = tid < nrow ? g.list[lb + tid] : -1;
    s_pair[tid] = p;
    int ex = 0;
    if (p >= 0) {
      if constexpr (FC2) ex = mg_row_exp(__builtin_bit_cast(float, g.hmax[p]));
      else ex = g.ex[p / a.k];
    }
    s_rs[tid] = __builtin_ldexpf(1.f, -ex);
    s_ru[tid] = __builtin_ldexpf(1.f, ex);
  }
  __syncthreads();

  // ---- global loads: thread t stages A row t / 8, floats 8 (t % 8) .. + 7 of
  // the step, and 32 codes (16 bytes) of column t / 2, half t % 2. The rows
  // belong to different tokens, so A goes through per-lane addresses (a
  // buffer resource would have to be wave-uniform); rows past the tile's
  // pairs repeat its first pair and their sums are never written.
  const int arow = tid >> 3, agrp = tid & 7;
  const int apair = s_pair[arow] < 0 ? s_pair[0] : s_pair[arow];
  const float ascale = s_rs[arow];
  const float* Asrc = FC2 ? a.h : a.x;
  const float* Arow = Asrc + (FC2 ? static_cast<int64_t>(apair) * a.I : static_cast<int64_t>(apair / a.k) * a.H) + agrp * 8;
  const int bcol = tid >> 1, bh = tid & 1;
  const uint32_t rowb = static_cast<uint32_t>(Kd) * BITS / 8u;  // bytes per expert row
  const uint8_t* Wb = FC2 ? a.fc2 + static_cast<int64_t>(e) * a.H * rowb : a.fc1 + static_cast<int64_t>(e) * a.F1 * rowb;
  const rsrc_t rB = mk_rsrc(Wb, static_cast<uint32_t>(Nd) * rowb);
  const bool bval = n0 + bcol < Nd;
  const uint32_t boff = bval ? static_cast<uint32_t>(n0 + bcol) * rowb : OOB;
  // this workgroup's K steps [kstep0, kstep0 + ksteps); splits of blocks of
  // 128 codes or more hold whole blocks (a split past the end holds none and
  // writes zero partials)
  const int kall = (Kd + MG_K - 1) / MG_K;
  const int bsteps = BKM == 8 ? a.bs / MG_K : 1;  // K steps per block
  const int kper = ((kall + ks2 - 1) / ks2 + bsteps - 1) / bsteps * bsteps;
  const int kstep0 = sp * kper;
  const int ksteps = kall - kstep0 < kper ? kall - kstep0 : kper;

  struct Regs {
    u32x4 a[2];
    u32x4 b[BW];
  };
  // steps past the end reload the last one (never staged)
  auto gload = [&](Regs& r, int ks) {
    const bool ok = ks < ksteps;
    int kst = kstep0 + (ok ? ks : ksteps - 1);
    kst = kst < kall - 1 ? kst : kall - 1;
    const float* pa = Arow + kst * MG_K;
    r.a[0] = *reinterpret_cast<const u32x4*>(pa);
    r.a[1] = *reinterpret_cast<const u32x4*>(pa + 4);
#pragma unroll
    for (int i = 0; i < BW; ++i)
      r.b[i] = bld16(rB, (ok ? boff : OOB) + static_cast<uint32_t>((kstep0 + ks) * MG_K * BITS / 8 + (bh * BW + i) * 16), 0);
  };
  // A: scaled, split into binary16 hi / lo in the pair order of the codes;
  // B: the raw code dwords (dequantised when a fragment is read)
  auto sstore = [&](const Regs& r, int stage) {
    f16* Ah = lds + stage * MG_STAGE;
    f16* Al = Ah + MG_RT * MG_LD;
    uint32_t* Bw = reinterpret_cast<uint32_t*>(Al + MG_RT * MG_LD);  // [fragment][column][BW dwords]
    f16x8 vh, vl;
    // the eight floats by name first: this compiler folds v[i >> 2][i & 3]
    // over an array of vectors to element 0 of each vector
    const f32x4 lo4 = __builtin_bit_cast(f32x4, r.a[0]), hi4 = __builtin_bit_cast(f32x4, r.a[1]);
    const float xs[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float x = xs[(q >> 1) + 4 * (q & 1)] * ascale;  // pair order 0 4 1 5 2 6 3 7
      const f16 h = static_cast<f16>(x);
      vh[q] = h;
      vl[q] = __builtin_isfinite(x) ? static_cast<f16>(x - static_cast<float>(h)) : static_cast<f16>(0.f);
    }
    *reinterpret_cast<f16x8*>(Ah + arow * MG_LD + agrp * 8) = vh;
    *reinterpret_cast<f16x8*>(Al + arow * MG_LD + agrp * 8) = vl;
    // fragment 4 bh + d of the step (codes 32 bh + 8 d .. + 7) of column bcol
    if constexpr (BW == 1) {
#pragma unroll
      for (int d = 0; d < 4; ++d) Bw[(4 * bh + d) * MG_CT + bcol] = r.b[0][d];
    } else {
      // the eight dwords by name (no v[i >> 1][...] indexing, see above)
      const u32x4 b0 = r.b[0], b1 = r.b[BW - 1];
      const uint32_t w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int d = 0; d < 4; ++d)
        *reinterpret_cast<u32x2*>(Bw + ((4 * bh + d) * MG_CT + bcol) * 2) = u32x2{w[2 * d], w[2 * d + 1]};
    }
  };
  // a fragment's eight codes -> c - 2^(bits - 1) as exact binary16, pair
  // order (c0 c4 c1 c5 c2 c6 c3 c7, the activations' staging order)
  const f16x2 n1032 = {static_cast<f16>(-1032.f), static_cast<f16>(-1032.f)};
  const f16x2 inv16 = {static_cast<f16>(0.0625f), static_cast<f16>(0.0625f)};
  const f16x2 n72 = {static_cast<f16>(-72.f), static_cast<f16>(-72.f)};
  const f16x2 n1152 = {static_cast<f16>(-1152.f), static_cast<f16>(-1152.f)};
  auto dq = [&](const uint32_t* w) {
    const uint32_t magic = 0x64006400u;
    if constexpr (BW == 1) {
      const uint32_t x = w[0], x8 = x >> 8;
      const f16x2 d0 = as_h2(and_or(x, 0x000F000Fu, magic)) + n1032;
      const f16x2 d1 = __builtin_elementwise_fma(as_h2(and_or(x, 0x00F000F0u, magic)), inv16, n72);
      const f16x2 d2 = as_h2(and_or(x8, 0x000F000Fu, magic)) + n1032;
      const f16x2 d3 = __builtin_elementwise_fma(as_h2(and_or(x8, 0x00F000F0u, magic)), inv16, n72);
      return f16x8{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
    } else {
      // bytes c0..c3 in w[0], c4..c7 in w[1]: (c_i, c_i+4) into the low bytes
      // of a half pair, then 0x64 above each: 1024 + c exactly
      const uint32_t x0 = w[0], x1 = w[1];
      const f16x2 d0 = as_h2(__builtin_amdgcn_perm(x1, x0, 0x0c040c00u) | magic) + n1152;
      const f16x2 d1 = as_h2(__builtin_amdgcn_perm(x1, x0, 0x0c050c01u) | magic) + n1152;
      const f16x2 d2 = as_h2(__builtin_amdgcn_perm(x1, x0, 0x0c060c02u) | magic) + n1152;
      const f16x2 d3 = as_h2(__builtin_amdgcn_perm(x1, x0, 0x0c070c03u) | magic) + n1152;
      return f16x8{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
    }
  };

  // block sums (acc) and, with block scales, the scaled running sums (yacc)
  f32x16 acc[2], yacc[BKM ? 2 : 1];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[j][q] = 0.f;
#pragma unroll
  for (int j = 0; j < (BKM ? 2 : 1); ++j)
#pragma unroll
    for (int q = 0; q < 16; ++q) yacc[j][q] = 0.f;
  // the scales of this lane's two columns: [E, Nd] (row scales) or
  // [E, Nd, Kd / block_size]
  const int nblk = BKM ? Kd / a.bs : 1;
  const float* S = FC2 ? a.s2 + static_cast<int64_t>(e) * a.H * nblk : a.s1 + static_cast<int64_t>(e) * a.F1 * nblk;
  int scol[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = n0 + wn * 64 + j * 32 + (lane & 31);
    scol[j] = (c < Nd ? c : Nd - 1) * nblk;
  }
  // block flushes per step: 4 / BKM inside the step, or one at its end
  constexpr int NFL = BKM == 0 ? 0 : BKM == 8 ? 1 : 4 / BKM;
  constexpr int NSL = NFL ? NFL : 1;
  // (kept in place by scheduling barriers: moved among the next block's
  // MFMAs it would hold two copies of the accumulators)
  auto flush = [&](const float (&sc)[2]) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        yacc[BKM ? j : 0][q] = __builtin_fmaf(sc[j], acc[j][q], yacc[BKM ? j : 0][q]);
        acc[j][q] = 0.f;
      }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto mfmas = [&](int stage, const float (&sl)[NSL][2]) {
    const f16* Ah = lds + stage * MG_STAGE;
    const f16* Al = Ah + MG_RT * MG_LD;
    const uint32_t* Bw = reinterpret_cast<const uint32_t*>(Al + MG_RT * MG_LD);
#pragma unroll
    for (int kk = 0; kk < MG_K / 16; ++kk) {
      const int ko = kk * 16 + (lane >> 5) * 8;
      const int ar = wm * 32 + (lane & 31);
      const f16x8 fh = *reinterpret_cast<const f16x8*>(Ah + ar * MG_LD + ko);
      const f16x8 fl = *reinterpret_cast<const f16x8*>(Al + ar * MG_LD + ko);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // codes k = ko .. ko + 7 of column wn 64 + 32 j + lane % 32: fragment ko / 8
        const f16x8 fb = dq(Bw + ((ko >> 3) * MG_CT + wn * 64 + j * 32 + (lane & 31)) * BW);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fh, fb, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fl, fb, acc[j], 0, 0, 0);
      }
      if constexpr (BKM >= 1 && BKM <= 4) {
        if ((kk + 1) % BKM == 0) flush(sl[kk / BKM]);
      }
    }
  };
  // the step's block scales, loaded before its fill loads (so waiting for
  // them never waits for the fill)
  auto sload = [&](int ks, float (&sl)[NSL][2]) {
    if constexpr (NFL > 0) {
      const int kg = kstep0 + (ks < ksteps ? ks : ksteps - 1);  // in range
#pragma unroll
      for (int f = 0; f < NFL; ++f) {
        const int b = BKM == 8 ? (kg * MG_K) / a.bs : kg * NFL + f;
#pragma unroll
        for (int j = 0; j < 2; ++j) sl[f][j] = S[scol[j] + b];
      }
    }
  };

  // two register sets, loads two steps ahead; double-buffered LDS, one
  // barrier per step
  // step ks on stage ks % 2: `nxt` holds step ks + 1 (stored to the other
  // stage during the step), `fill` receives step ks + 2
  auto step = [&](int ks, int stage, Regs& nxt, Regs& fill) {
    float sl[NSL][2];
    sload(ks, sl);
    gload(fill, ks + 2);
    mfmas(stage, sl);
    if constexpr (BKM == 8) {
      if ((kstep0 + ks + 1) % bsteps == 0) flush(sl[0]);
    }
    if (ks + 1 < ksteps) sstore(nxt, stage ^ 1);
    __syncthreads();
  };
  if (ksteps > 0) {  // uniform: a split past the end keeps zero sums
    Regs r0, r1;
    gload(r0, 0);
    gload(r1, 1);
    sstore(r0, 0);
    __syncthreads();
    int ks = 0;
    for (; ks + 1 < ksteps; ks += 2) {
      step(ks, 0, r1, r0);
      step(ks + 1, 1, r0, r1);
    }
    if (ks < ksteps) step(ks, 0, r1, r0);
  }

  // ---- epilogue: lane holds D[8 (q / 4) + 4 (lane / 32) + q % 4][lane % 32]
  float rmax[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) rmax[q] = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = n0 + wn * 64 + j * 32 + (lane & 31);
    const float sc = BKM ? 1.f : (c < Nd ? S[c] : 0.f);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int r = wm * 32 + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
      const int p = s_pair[r];
      const float v = (BKM ? yacc[BKM ? j : 0][q] : acc[j][q] * sc) * s_ru[r];
      if constexpr (FC2) {
        if (p >= 0 && c < Nd) a.yp[(static_cast<int64_t>(p) * ks2 + sp) * a.H + c] = v;
      } else if constexpr (ST == MG_FC1_SWIGLU) {
        // gate = row 2m (even lane), linear = row 2m + 1 (odd lane)
        const float other = __shfl_xor(v, 1, 64);
        const float o = swiglu(v, other, a);
        if ((lane & 1) == 0 && p >= 0 && c < Nd) {
          a.h[static_cast<int64_t>(p) * a.I + c / 2] = o;
          if (__builtin_isfinite(o)) rmax[q] = fmaxf(rmax[q], __builtin_fabsf(o));
        }
      } else {
        const float o = fmaxf(v, 0.f);
        if (p >= 0 && c < Nd) {
          a.h[static_cast<int64_t>(p) * a.I + c] = o;
          if (__builtin_isfinite(o)) rmax[q] = fmaxf(rmax[q], o);
        }
      }
    }
  }
  if constexpr (!FC2) {
    // each row's largest |h| over this tile, into the pair's running maximum
    // (non-negative floats order like their bit patterns)
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const float m = mg_half_max(rmax[q]);
      const int r = wm * 32 + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
      const int p = s_pair[r];
      if ((lane & 31) == 0 && p >= 0 && m > 0.f) atomicMax(g.hmax + p, __builtin_bit_cast(uint32_t, m));
    }
  }
}

// y[t][n] = sum over slots s of w[t k + s] * yp[t k + s][n], in slot order,
// each slot's a.ks FC2 splits summed first in split order.
__global__ __launch_bounds__(256) void k_moe_combine(MoeArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= a.T * a.H) return;
  const int64_t t = i / a.H, n = i % a.H;
  float y = 0.f;
  for (int s = 0; s < a.k; ++s) {
    const int64_t pair = t * a.k + s;
    const float* part = a.yp + pair * a.ks * a.H + n;
    float v = part[0];
    for (int sp = 1; sp < a.ks; ++sp) v += part[static_cast<int64_t>(sp) * a.H];
    y = __builtin_fmaf(a.wts[pair], v, y);
  }
  a.y[i] = y;
}

}  // namespace
}  // namespace xrmm
