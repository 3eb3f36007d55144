// Split-K MFMA GEMV for up to 16 rows (fp16 activations, 4-bit weights): the
// batched-decode kernel of all three operators (MatMulNBits, Qkv, Mlp).
//
// Work split. The output columns form tiles of 16 MFMA columns: 16 columns of
// one projection (MatMulNBits, Qkv), or 8 gate and the same 8 up columns (Mlp,
// so that act(gate) * up is formed inside the tile). A workgroup owns `tpw`
// consecutive tiles; its W waves split K: wave w takes the chunks
// [w * 4 CPL, (w + 1) * 4 CPL) of every column, and lane (j, g) of the wave
// takes CPL consecutive chunks of column j (a chunk is 16 bytes, 32 codes).
// Each wave therefore needs only its own K slice of the activations, for
// all 16 rows: it loads that slice once into registers, already in the
// MFMA operand order, and reuses it for every tile. No activation staging in
// LDS and no barrier before the weight stream; the only barrier combines the
// W partial sums of each tile at the end.
//
// Weight stream. In the MFMA operand layout a column's K slice lives in four
// lanes, so loading it directly would read each 128-byte line in pieces spread
// over several instructions (measured: about five L2 requests per line).
// Instead a wave loads a tile's K slice coalesced (consecutive lanes read
// consecutive 16-byte pieces of one column, whole lines per instruction) and
// transposes it through its own LDS slice (a padded column stride keeps the
// reads conflict-free); no barrier is involved.
//
// Memory order. Loads retire in issue order, so a wave issues the activation
// slice, then every tile's scales / zero points, then the weights of the
// first TQ tiles; each consumed tile's registers are refilled with the
// weights of the tile TQ ahead.
//
// Arithmetic. v_mfma_f32_16x16x32_f16: lane (j, g) supplies, for MFMA d of
// chunk i, the eight codes of dword d dequantised to binary16 (dq8: the
// exact (code - z) * scale rounded once, in pair order [c0 c4 c1 c5 c2 c6 c3
// c7]) as B[k][j], and row j's activations of the same eight k in the same
// order as A[j][k]; the MFMA's 32 k are the four lane groups' dwords. Tile
// partials accumulate in float32.
#pragma once
#include <cstdlib>

#include "xrmm_device.h"

namespace xrmm {

struct SkProj {
  const uint8_t* B;
  const void* S;
  const void* Z;
  const void* bias;
  void* Y;
  uint32_t N;
  uint32_t t0;  // first tile of this projection (Qkv lays Q, K, V tiles in order)
};

struct SkArgs {
  const void* A;
  const void* skip;   // Qkv / Mlp: nullable, added to A
  const void* gamma;  // Qkv / Mlp: nullable RMS scale [K]
  void* residual;     // nullable: receives A + skip (workgroup 0 writes it)
  float eps;
  int act;            // Mlp activation kind
  SkProj p[3];
  uint32_t K, kb, rowb, zrow, M;
  uint32_t bsl;       // log2(block_size)
  uint32_t zesz;      // bytes per float zero point (2 or 4)
  uint32_t tiles;     // tiles of the whole launch
  uint32_t tpw;       // tiles per workgroup (<= sk_tmax(W))
  uint32_t chunks;    // row chunks of 16 (more than 16 rows: the grid repeats per chunk)
};

// Tiles per workgroup at most: the LDS holds every wave's partial sum of
// every tile (W x TMAX KB) beside the transpose slices.
constexpr int sk_tmax(int w) { return w >= 16 ? 7 : 8; }
#ifndef XRMM_SK_TQ
#define XRMM_SK_TQ 2
#endif
constexpr int SK_TQ = XRMM_SK_TQ;  // tiles whose weights a wave keeps in flight

// Scales (and zero points) of one lane's CPL chunks of one column: SPL
// consecutive blocks, SPL = max(1, 32 CPL / block_size). Raw dwords: binary16
// scales two per dword (low half first); packed zero points as loaded (the
// nibbles of blocks b0 .. b0 + SPL - 1); float zero points as binary16 pairs or
// float32 words.
template <int SPL>
struct SkMeta {
  uint32_t s[(SPL + 1) / 2];
  uint32_t z[SPL];
};

// Loads of 2, 4, 8 or 16 bytes into dwords (the low 16 bits for 2 bytes).
template <int BYTES>
__device__ __forceinline__ void ld_small(const uint8_t* p, uint32_t* out) {
  if constexpr (BYTES == 1) out[0] = *p;
  else if constexpr (BYTES == 2) out[0] = *reinterpret_cast<const uint16_t*>(p);
  else if constexpr (BYTES == 4) out[0] = *reinterpret_cast<const uint32_t*>(p);
  else if constexpr (BYTES == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    out[0] = v.x;
    out[1] = v.y;
  } else {
    static_assert(BYTES == 16, "load size");
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  }
}

template <int ZPK, int OPK, int W, int CPL, int SPL, bool NRM>
__global__ __launch_bounds__(W * 64) void k_gemv_sk(SkArgs a) {
  // The normalising prologue holds the activations and the skip input at
  // once, so it keeps fewer weight tiles in flight.
  constexpr int TQ = NRM ? 2 : SK_TQ, TMAX = sk_tmax(W);
  constexpr bool MLP = OPK == OP_MLP, QKV = OPK == OP_QKV;
  static_assert(SPL >= 1 && SPL <= CPL, "scales per lane");
  static_assert(!NRM || OPK != OP_MATMUL, "normalisation is a Qkv / Mlp prologue");
  constexpr int CPW = 4 * CPL;            // chunks of one column in a wave's K slice
  constexpr int XS = CPW * 16 + 16;       // LDS bytes per column of a transposed tile (padded)
  // LDS: one region per wave. It first stages the wave's activation slice
  // (16 rows x OPR 16-byte pieces, padded rows), then holds the wave's tile
  // partial sums (TMAX x 1 KB) and its weight transpose slice (16 x XS).
  constexpr int OPR = CPW * 4;            // 16-byte pieces of one row of the K slice
  constexpr int XA = OPR * 16 + 16;       // LDS bytes per staged activation row (padded)
  constexpr int RG = (16 * XA > TMAX * 1024 + 16 * XS ? 16 * XA : TMAX * 1024 + 16 * XS);
  __shared__ __align__(16) unsigned char lds[W][RG];
  __shared__ float rsq[W][16];

  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t j = lane & 15, g = lane >> 4;
  // Workgroup -> (tile group x, row chunk y). The row chunks of one tile group
  // are eight workgroups apart: consecutive workgroups go to consecutive XCDs,
  // so they run on one XCD, close in time, and share its L2 copy of the
  // weights (one HBM read for up to 64 rows). With one chunk x = blockIdx.x.
  const uint32_t bid = blockIdx.x, nch = a.chunks;
  const uint32_t gx = (bid & 7u) + 8u * (bid / (8u * nch)), gy = (bid >> 3) % nch;
  const uint32_t tb = gx * a.tpw;  // first tile of the workgroup
  if (tb >= a.tiles) return;       // padding of the grid to whole groups of eight (uniform)
  const uint32_t m0 = 16u * gy;    // first row of the chunk
  const uint32_t K = a.K, kb = a.kb, rowb = a.rowb, M = a.M - m0 < 16u ? a.M - m0 : 16u;
  const uint32_t ch0 = (w * 4 + g) * CPL;  // first chunk of this lane
  const uint32_t k0 = ch0 * 32;            // first k of this lane
  const uint32_t b0 = k0 >> a.bsl;         // first block of this lane
  const uint32_t tpw = a.tpw < a.tiles - tb ? a.tpw : a.tiles - tb;

  // ---- activations: the wave's K slice of all 16 rows, loaded coalesced
  // (consecutive lanes read consecutive 16-byte pieces of a row); the LDS
  // region transposes them to the MFMA operand order below. (Loaded in that
  // order directly, every load instruction touched 64 different lines.)
  constexpr int AI = 16 * OPR / 64;  // coalesced loads per lane
  static_assert(AI == 4 * CPL, "activation staging");
  const rsrc_t rA = mk_rsrc(static_cast<const f16*>(a.A) + m0 * K, M * K * 2u);
  u32x4 craw[AI];
  uint32_t coff[AI];
#pragma unroll
  for (int r = 0; r < AI; ++r) {
    const uint32_t e = static_cast<uint32_t>(r * 64 + lane), row = e / OPR, o = e % OPR;
    const uint32_t k = w * CPW * 32u + o * 8u;
    coff[r] = (row < M && k < K) ? (row * K + k) * 2u : 0x80000000u;  // K % 8 == 0: pieces are whole
    craw[r] = bld16(rA, coff[r], 0);
  }
  u32x4 csk[NRM ? AI : 1];
  if constexpr (NRM) {
    const rsrc_t rK = mk_rsrc(a.skip ? static_cast<const f16*>(a.skip) + m0 * K : nullptr, a.skip ? M * K * 2u : 0u);
#pragma unroll
    for (int r = 0; r < AI; ++r) csk[r] = bld16(rK, coff[r], 0);
  }

  // Keep the issue order (activations, metadata, weights): the vector-memory
  // counter retires loads in order, so a small load scheduled behind the
  // weights would make its first use wait for the whole stream.
  __builtin_amdgcn_sched_barrier(0);

  // ---- per tile: this lane's projection and column, and its pointers
  auto proj_of = [&](uint32_t tt) -> uint32_t {
    if constexpr (MLP) return j >> 3;
    else if constexpr (QKV) return (tt >= a.p[1].t0 ? 1u : 0u) + (tt >= a.p[2].t0 ? 1u : 0u);
    else return 0u;
  };
  auto sel = [&](uint32_t pi, auto v0, auto v1, auto v2) { return pi == 0 ? v0 : pi == 1 ? v1 : v2; };
  struct Ptrs {
    const uint8_t* s;
    const uint8_t* z;
  };
  // Scale / zero-point pointers of this lane's column in tile t.
  auto ptrs = [&](int t) -> Ptrs {
    const uint32_t tt = tb + static_cast<uint32_t>(t);
    const uint32_t pi = proj_of(tt);
    const uint32_t N = sel(pi, a.p[0].N, a.p[1].N, a.p[2].N);
    uint32_t col;
    if constexpr (MLP) col = tt * 8u + (j & 7u);
    else col = (tt - sel(pi, a.p[0].t0, a.p[1].t0, a.p[2].t0)) * 16u + j;
    col = col < N ? col : N - 1u;  // columns past N: loaded, never stored
    Ptrs p;
    p.s = static_cast<const uint8_t*>(sel(pi, a.p[0].S, a.p[1].S, a.p[2].S)) + (static_cast<size_t>(col) * kb + b0) * 2u;
    if constexpr (ZPK == ZP_PACKED)
      p.z = static_cast<const uint8_t*>(sel(pi, a.p[0].Z, a.p[1].Z, a.p[2].Z)) + (static_cast<size_t>(col) * a.zrow + (b0 >> 1));
    else if constexpr (ZPK == ZP_FLOAT)
      p.z = static_cast<const uint8_t*>(sel(pi, a.p[0].Z, a.p[1].Z, a.p[2].Z)) + (static_cast<size_t>(col) * kb + b0) * a.zesz;
    else
      p.z = nullptr;
    return p;
  };

  // ---- weights of the first TQ tiles: the HBM stream starts here
  // Weights are loaded coalesced: load q of a tile reads pieces q*64 + lane
  // of the tile's 16 x CPW chunks in column-major order, so consecutive lanes
  // read consecutive 16-byte pieces of one column (whole 128-byte lines).
  // The wave's LDS slice then transposes them to the MFMA lane order.
  u32x4 wbuf[TQ][CPL];
  SkMeta<SPL> mbuf[TQ];
  // Buffer resources bound each projection's weights: a load of a tile past
  // the workgroup's last gets an out-of-range offset and returns zeros
  // without touching memory. (A branch around those loads would make every
  // later wait a full drain; re-reading real lines would cost bandwidth.)
  // Each load instruction covers 64 / CPW <= 8 columns that lie in one
  // projection (Mlp: all gate or all up), so its resource is wave-uniform.
  static_assert(CPW >= 8, "a load must not straddle the gate / up halves");
  const rsrc_t rB0 = mk_rsrc(a.p[0].B, a.p[0].N * rowb);
  const rsrc_t rB1 = mk_rsrc(QKV || MLP ? a.p[1].B : a.p[0].B, (QKV || MLP ? a.p[1].N : a.p[0].N) * rowb);
  const rsrc_t rB2 = mk_rsrc(QKV ? a.p[2].B : a.p[0].B, (QKV ? a.p[2].N : a.p[0].N) * rowb);
  // Tile t's scales / zero points, then its weights, into slot u = t % TQ.
  auto issue = [&](int t, int u) {
    // all-ones for a live tile; opaque to the compiler, which would otherwise
    // turn the selects below into branches around the loads
    uint32_t lm = __builtin_amdgcn_readfirstlane(t < static_cast<int>(tpw) ? 0xFFFFFFFFu : 0u);
    asm volatile("s_mov_b32 %0, %0" : "+s"(lm));
    {
      const Ptrs p = ptrs(static_cast<int>(static_cast<uint32_t>(t) & lm));  // past the last: the first tile's (cached)
      ld_small<2 * SPL>(p.s, mbuf[u].s);
      if constexpr (ZPK == ZP_PACKED) {
        ld_small<SPL <= 2 ? 1 : SPL / 2>(p.z, mbuf[u].z);
      } else if constexpr (ZPK == ZP_FLOAT) {
        if (a.zesz == 4) ld_small<4 * SPL>(p.z, mbuf[u].z);
        else ld_small<2 * SPL>(p.z, mbuf[u].z);
      }
    }
    const uint32_t tt = tb + (static_cast<uint32_t>(t) & lm);
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      const uint32_t pc = static_cast<uint32_t>(q * 64 + lane);
      const uint32_t c = pc / CPW, pp = pc % CPW;  // MFMA column and piece of this load
      uint32_t pi, col;
      if constexpr (MLP) {
        pi = (q * 64 / CPW) >> 3;  // the instruction's half: gate or up
        col = tt * 8u + (c & 7u);
      } else {
        pi = proj_of(tt);
        col = (tt - sel(pi, a.p[0].t0, a.p[1].t0, a.p[2].t0)) * 16u + c;
      }
      const uint32_t N = sel(pi, a.p[0].N, a.p[1].N, a.p[2].N);
      col = col < N ? col : N - 1u;  // columns past N: loaded, never stored
      const uint32_t off = ((col * rowb + (w * CPW + pp) * 16u) & lm) | (0x80000000u & ~lm);
      wbuf[u][q] = bld16_nt(pi == 0 ? rB0 : pi == 1 ? rB1 : rB2, off, 0);
    }
  };
#pragma unroll
  for (int t = 0; t < TQ; ++t) issue(t, t);
  __builtin_amdgcn_sched_barrier(0);

  // ---- transpose the staged activations: lane (j, g) takes row j's pieces
  // of its chunks g CPL .. g CPL + CPL - 1 (piece 4 chunk + d holds k of
  // dword d of that chunk)
  unsigned char* rg = lds[w];
  auto restage = [&](const u32x4(&src)[AI], u32x4(&dst)[CPL][4]) {
#pragma unroll
    for (int r = 0; r < AI; ++r) {
      const uint32_t e = static_cast<uint32_t>(r * 64 + lane);
      *reinterpret_cast<u32x4*>(rg + (e / OPR) * XA + (e % OPR) * 16) = src[r];
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int d = 0; d < 4; ++d) dst[i][d] = *reinterpret_cast<const u32x4*>(rg + j * XA + ((g * CPL + i) * 4 + d) * 16);
  };
  u32x4 araw[CPL][4], sraw[NRM ? CPL : 1][4];
  restage(craw, araw);
  if constexpr (NRM) restage(csk, sraw);

  // ---- prologue (Qkv / Mlp with skip or RMS scale): r = A + skip in
  // float32, x = r * inv * gamma with inv = 1 / sqrt(sum_k r^2 / K + eps)
  // per row (packedInput, complex_kernel.glsl:81); x is rounded to binary16
  // for the MFMA. Each lane holds 32 CPL elements of row j; the row sums of
  // squares combine over the lane groups and the waves.
  f16x8 aop[CPL][4];
  if constexpr (NRM) {
    const bool has_skip = a.skip != nullptr, has_gamma = a.gamma != nullptr;
    // r in float32 feeds the row statistic; r rounded once to binary16 (the
    // residual output's value) replaces the activations in their registers.
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const f16x8 av = __builtin_bit_cast(f16x8, araw[i][d]);
        const f16x8 sv = __builtin_bit_cast(f16x8, sraw[i][d]);
        f16x8 rr;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float r = has_skip ? __fadd_rn(static_cast<float>(av[e]), static_cast<float>(sv[e])) : static_cast<float>(av[e]);
          sq = __builtin_fmaf(r, r, sq);
          rr[e] = static_cast<f16>(r);
        }
        araw[i][d] = __builtin_bit_cast(u32x4, rr);
      }
    float inv = 1.f;
    if (has_gamma) {
      sq += __shfl_xor(sq, 16, 64);
      sq += __shfl_xor(sq, 32, 64);
      if (lane < 16) rsq[w][lane] = sq;
      __syncthreads();
      float t = 0.f;
#pragma unroll
      for (int v = 0; v < W; ++v) t += rsq[v][j];
      inv = 1.f / sqrtf(t / static_cast<float>(K) + a.eps);
    }
    const bool write_res = a.residual != nullptr && gx == 0 && j < M;
    const rsrc_t rG = mk_rsrc(a.gamma, has_gamma ? K * 2u : 0u);
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t k = k0 + 32u * i + 8u * d;
        const f16x8 rr = __builtin_bit_cast(f16x8, araw[i][d]);
        const f16x8 gv = __builtin_bit_cast(f16x8, bld16(rG, k < K ? k * 2u : 0x80000000u, 0));
        f16x8 x;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = has_gamma ? static_cast<f16>(static_cast<float>(rr[e]) * (inv * static_cast<float>(gv[e]))) : rr[e];
        aop[i][d] = pair_order(x);
        if (write_res && k < K) *reinterpret_cast<f16x8*>(static_cast<f16*>(a.residual) + (m0 + j) * K + k) = rr;
      }
  } else {
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int d = 0; d < 4; ++d) aop[i][d] = pair_order(__builtin_bit_cast(f16x8, araw[i][d]));
  }

  // ---- tiles, in a loop over groups of TQ (the code stays small enough for
  // the instruction cache): transpose, refill the slot with the tile TQ
  // ahead, dequantise, multiply, park the partial sum in LDS
  f32x4* part = reinterpret_cast<f32x4*>(rg);  // [TMAX][64]
  unsigned char* xb = rg + TMAX * 1024;
  for (int t0 = 0; t0 < static_cast<int>(tpw); t0 += TQ) {
#pragma unroll
    for (int u = 0; u < TQ; ++u) {
      const int t = t0 + u;
      // piece (c, pp) -> lane (j = c, g = pp / CPL), slot pp % CPL
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        const uint32_t pc = static_cast<uint32_t>(q * 64 + lane);
        *reinterpret_cast<u32x4*>(xb + (pc / CPW) * XS + (pc % CPW) * 16) = wbuf[u][q];
      }
      const SkMeta<SPL> m = mbuf[u];
      // refill as soon as the registers are free, pinned there
      __builtin_amdgcn_sched_barrier(0);
      issue(t + TQ, u);
      __builtin_amdgcn_sched_barrier(0);
      u32x4 wt[CPL];
#pragma unroll
      for (int i = 0; i < CPL; ++i) wt[i] = *reinterpret_cast<const u32x4*>(xb + j * XS + (g * CPL + i) * 16);
      if (t < static_cast<int>(tpw)) {  // wave-uniform
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
          const int bi = i * SPL / CPL;  // this chunk's block among the lane's SPL
          const f16 s = __builtin_bit_cast(f16, static_cast<uint16_t>(m.s[bi >> 1] >> (16 * (bi & 1))));
          float z = 8.f;
          if constexpr (ZPK == ZP_PACKED) {
            const uint32_t sh = SPL == 1 ? (b0 & 1u) * 4u : 4u * bi;
            z = static_cast<float>((m.z[0] >> sh) & 15u);
          } else if constexpr (ZPK == ZP_FLOAT) {
            z = a.zesz == 4 ? __builtin_bit_cast(float, m.z[bi])
                            : static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(m.z[bi >> 1] >> (16 * (bi & 1)))));
          }
          const u32x4 wv = wt[i];
          if constexpr (ZPK == ZP_FLOAT) {
            const float sf = static_cast<float>(s);
#pragma unroll
            for (int d = 0; d < 4; ++d) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[i][d], dq8_f32z(wv[d], z, sf), acc, 0, 0, 0);
          } else {
            const Dq cst = dq_consts(z, s);
#pragma unroll
            for (int d = 0; d < 4; ++d) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[i][d], dq8(wv[d], cst), acc, 0, 0, 0);
          }
        }
        part[t * 64 + lane] = acc;
      }
    }
  }
  __syncthreads();

  // ---- combine the W partial sums: thread (t, l) owns lane l of tile t;
  // output rows 4 (l / 16) .. + 3, MFMA column l % 16
  const uint32_t t = static_cast<uint32_t>(tid) >> 6;
  if (t >= tpw) return;
  const uint32_t l = static_cast<uint32_t>(lane);
  const uint32_t jj = l & 15u, gg = l >> 4;
  if (MLP && jj >= 8) return;  // up columns are read by their gate lane
  auto part_of = [&](int v, uint32_t tl) { return reinterpret_cast<const f32x4*>(lds[v])[tl]; };
  f32x4 y = part_of(0, t * 64 + l);
#pragma unroll
  for (int v = 1; v < W; ++v) y += part_of(v, t * 64 + l);
  const uint32_t tt = tb + t;
  const uint32_t pi = MLP ? 0u : proj_of(tt);
  const SkProj& P = a.p[pi];
  const uint32_t N = P.N;
  const uint32_t col = MLP ? tt * 8u + jj : (tt - P.t0) * 16u + jj;
  if (col >= N) return;
  f16* Y = static_cast<f16*>(P.Y) + m0 * N;
  if constexpr (MLP) {
    f32x4 u = part_of(0, t * 64 + l + 8);
#pragma unroll
    for (int v = 1; v < W; ++v) u += part_of(v, t * 64 + l + 8);
    const float gb = a.p[0].bias ? static_cast<float>(static_cast<const f16*>(a.p[0].bias)[col]) : 0.f;
    const float ub = a.p[1].bias ? static_cast<float>(static_cast<const f16*>(a.p[1].bias)[col]) : 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t m = 4u * gg + r;
      if (m < M) Y[m * N + col] = static_cast<f16>(activate(y[r] + gb, a.act) * (u[r] + ub));
    }
  } else {
    const float b = (!QKV && P.bias) ? static_cast<float>(static_cast<const f16*>(P.bias)[col]) : 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t m = 4u * gg + r;
      if (m < M) Y[m * N + col] = static_cast<f16>(y[r] + b);
    }
  }
}

// ---------------------------------------------------------------------------
// host side

// Waves (the K split) and chunks per lane for the geometry: a column's chunks
// split exactly over 4 lane groups x 8 waves; 0 when no split applies.
// (Measured on the batched SwiGLU workload: 16 waves of 2 chunks, four waves
// per SIMD, ran 9% slower than 8 waves of 4 chunks.)
struct SkShape {
  int w, cpl;
};

#ifndef XRMM_SK_W128
#define XRMM_SK_W128 8
#endif
inline SkShape sk_shape(const Launch& L) {
  const int64_t chunks = L.kb * L.blob / 16;
  if (chunks == 64) return {8, 2};
  if (chunks == 128) return XRMM_SK_W128 == 16 ? SkShape{16, 2} : SkShape{8, 4};
  return {0, 0};
}

inline int sk_spl(const Launch& L, int cpl) {
  const int64_t s = int64_t(32) * cpl / L.block_size;
  return s >= 1 ? static_cast<int>(s) : 1;
}

inline int64_t sk_tiles(const Launch& L, int64_t& t1, int64_t& t2) {
  t1 = t2 = 0;
  if (L.op == OP_MLP) return (L.p[0].N + 7) / 8;
  const int64_t t0n = (L.p[0].N + 15) / 16;
  if (L.op != OP_QKV) return t0n;
  t1 = t0n;
  t2 = t1 + (L.p[1].N + 15) / 16;
  return t2 + (L.p[2].N + 15) / 16;
}

// Rows the split-K GEMV takes at most, in chunks of 16 that share the weight
// stream through L2. Measured against the 128 x 128 GEMMs (K = 4096,
// N = 14336 unless noted): MatMulNBits at 32 / 64 rows 19 / 37 us against
// 57 / 58 us, at 128 rows 65 against 61 us; Mlp (K = 2048, N = 5632) at
// 32 / 64 rows 21 / 39 against 59 / 64 us, at 128 rows 77 against 67 us; Qkv
// (Nq = 4096, Nkv = 1024) at 64 rows 47 against 100 us. Each chunk
// dequantises the weights again, so the cost grows with the chunks.
// XRMM_SK_MAX_ROWS overrides the limit (measurement).
#ifndef XRMM_SK_MAX_ROWS
#define XRMM_SK_MAX_ROWS 64
#endif
inline int64_t sk_max_rows() {
  static const int64_t v = [] {
    const char* e = std::getenv("XRMM_SK_MAX_ROWS");
    if (e != nullptr && *e != 0) {
      char* end = nullptr;
      const long long r = std::strtoll(e, &end, 10);
      if (end != nullptr && *end == 0 && r >= 16 && r <= 256) return static_cast<int64_t>(r);
    }
    return static_cast<int64_t>(XRMM_SK_MAX_ROWS);
  }();
  return v;
}

// Whether the split-K GEMV applies: M <= sk_max_rows(), a column splits evenly
// over the waves, block_size >= 32, Mlp gate and up of one width.
inline bool sk_fits(const Launch& L) {
  if (L.M < 1 || L.M > sk_max_rows() || sk_shape(L).w == 0 || L.block_size < 32 || L.bs_log2 < 5) return false;
  if (L.op == OP_MLP && L.p[0].N != L.p[1].N) return false;
  return true;
}

inline int sk_num_cus() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

template <int ZPK, int OPK, int W, int CPL, int SPL, bool NRM>
inline hipError_t launch_sk5(const Launch& L, hipStream_t st) {
  SkArgs a;
  a.A = L.A;
  a.skip = L.skip;
  a.gamma = L.gamma;
  a.residual = L.residual;
  a.eps = L.eps;
  a.act = L.act;
  int64_t t1 = 0, t2 = 0;
  const int64_t tiles = sk_tiles(L, t1, t2);
  const uint32_t t0s[3] = {0u, static_cast<uint32_t>(t1), static_cast<uint32_t>(t2)};
  for (int i = 0; i < 3; ++i) {
    const Proj& P = L.p[i < L.nproj ? i : 0];
    a.p[i] = SkProj{P.B, P.scales, P.zp, P.bias, P.Y, static_cast<uint32_t>(P.N),
                    OPK == OP_QKV || i == 0 ? t0s[i] : 0xFFFFFFFFu};
  }
  a.K = static_cast<uint32_t>(L.K);
  a.kb = static_cast<uint32_t>(L.kb);
  a.rowb = static_cast<uint32_t>(L.kb * L.blob);
  a.zrow = static_cast<uint32_t>(L.zrow);
  a.M = static_cast<uint32_t>(L.M);
  a.bsl = static_cast<uint32_t>(L.bs_log2);
  a.zesz = L.zp_dtype == DT_F32 ? 4u : 2u;
  a.tiles = static_cast<uint32_t>(tiles);
  const int64_t cus = sk_num_cus();
  // Tiles per workgroup: one workgroup per CU at a time (its LDS holds every
  // wave's partial tiles), so the grid of tile groups x row chunks is sized
  // to one round of the CUs; every workgroup stages its chunk's activations,
  // so fewer, larger groups also stage less (Mlp, K = 2048, N = 5632, 32
  // rows: 13.4 us with 240 workgroups against 21.7 us with 352; Qkv, 64 rows:
  // 23.2 against 37.5 us).
  int64_t tpw = ((tiles * ((L.M + 15) / 16)) + cus - 1) / cus;
  tpw = tpw < 1 ? 1 : tpw > sk_tmax(W) ? sk_tmax(W) : tpw;
  a.tpw = static_cast<uint32_t>(tpw);
  a.chunks = static_cast<uint32_t>((L.M + 15) / 16);
  int64_t groups = (tiles + tpw - 1) / tpw;
  if (a.chunks > 1) groups = (groups + 7) / 8 * 8;  // whole groups of eight workgroups per chunk
  const uint32_t grid = static_cast<uint32_t>(groups * a.chunks);
  hipLaunchKernelGGL((k_gemv_sk<ZPK, OPK, W, CPL, SPL, NRM>), dim3(grid), dim3(W * 64), 0, st, a);
  return hipGetLastError();
}

template <int ZPK, int OPK, int W, int CPL, int SPL>
inline hipError_t launch_sk4(const Launch& L, hipStream_t st) {
  if constexpr (OPK == OP_MATMUL)
    return launch_sk5<ZPK, OPK, W, CPL, SPL, false>(L, st);
  else
    return (L.skip || L.gamma || L.residual) ? launch_sk5<ZPK, OPK, W, CPL, SPL, true>(L, st)
                                             : launch_sk5<ZPK, OPK, W, CPL, SPL, false>(L, st);
}

template <int ZPK, int OPK, int W, int CPL>
inline hipError_t launch_sk3(const Launch& L, hipStream_t st) {
  const int spl = sk_spl(L, CPL);
  if constexpr (CPL >= 4)
    if (spl >= 4) return launch_sk4<ZPK, OPK, W, CPL, 4>(L, st);
  if constexpr (CPL >= 2)
    if (spl >= 2) return launch_sk4<ZPK, OPK, W, CPL, 2>(L, st);
  return launch_sk4<ZPK, OPK, W, CPL, 1>(L, st);
}

template <int ZPK, int OPK>
inline hipError_t launch_sk2(const Launch& L, hipStream_t st) {
  const SkShape sh = sk_shape(L);
  if (sh.w == 16) return launch_sk3<ZPK, OPK, 16, 2>(L, st);
  return sh.cpl == 2 ? launch_sk3<ZPK, OPK, 8, 2>(L, st) : launch_sk3<ZPK, OPK, 8, 4>(L, st);
}

// Entry of one zero-point kind (defined in xrmm_gemv_sk_zp.hip).
template <int ZPK>
hipError_t launch_sk_for(const Launch& L, hipStream_t st);

}  // namespace xrmm
