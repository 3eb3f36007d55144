// Prefill GEMM (M > 16): fp16 activations x 4-bit weights dequantised to fp16
// in LDS, v_mfma_f32_32x32x16_f16 with float32 accumulation.
//
// Tiling. A workgroup of 8 waves (two per SIMD) owns a 256 x 256 output tile;
// wave (wm, wn) owns rows 64 wm .. + 63 and columns 128 wn .. + 127 as 2 x 4
// MFMA tiles of 32 x 32 (128 accumulator registers per lane, so two waves fit
// a SIMD and the hardware interleaves one wave's dequantisation and LDS work
// with the other's MFMAs). The 32x32x16 form is used because it reaches the
// matrix cores' full fp16 rate on gfx950; the 16x16x32 form does not.
//
// Tile widths. One workgroup fills a CU, so a grid of T tiles on C CUs runs
// ceil(T / C) rounds and a partial last round leaves CUs idle (M = 2048,
// N = 14336: 448 tiles, 1.75 rounds of work in 2). The grid may therefore
// mix 256-wide tiles with 192-wide ones (waves own 2 x 3 MFMA tiles, 0.75 of
// the work): with k rounds of wide tiles followed by j rounds of narrow ones
// every CU does k + 0.75 j tile-units (1 + 0.75 for the shape above). The
// host picks the mix with the shortest makespan (gemm_tiles); wide tiles
// come first on the grid, so they are dispatched first.
//
// Pipeline. K advances in steps of 64 over a double-buffered LDS. Global loads
// run two steps ahead into two register sets (each thread: four 16-byte pieces
// of the activation tile, one 16-byte chunk of one weight column and its raw
// scale / zero-point bits), so a load has two steps of MFMAs to arrive before
// its data is written to LDS. The weights are dequantised on the way into LDS
// with the same routine and pair order as the GEMV and xrmm_dequantize;
// fragments of the next K slice are read before the current slice's MFMAs.
// One barrier per step separates the stages.
#pragma once
#include "xrmm_device.h"

namespace xrmm {

constexpr int GB_M = 256, GB_N = 256, GB_K = 64, GB_T = 512;
constexpr int GB_LD = GB_K + 8;                      // halfs per staged row (pad spreads banks)
constexpr int GB_STAGE = (GB_M + GB_N) * GB_LD;      // halfs per pipeline stage
constexpr size_t GB_LDS = 2 * GB_STAGE * sizeof(_Float16);  // two stages: 147,456 bytes
constexpr int GB_TM = 2;                             // 32x32 MFMA row tiles per wave (column tiles: TN)

// Tile plan of a launch: the grid's first `nbig` = row tiles x nb workgroups
// take 256 x 256 tiles (column tiles 0 .. nb - 1); the rest take 256 x 192
// tiles (columns 256 nb + 192 j, j < ns). tile_of orders each set.
struct GemmTiles {
  uint32_t nb, ns, nbig;
};

// Shortest-makespan mix of k rounds of wide tiles (`ww` output columns) and j
// rounds of narrow ones (`nw` columns, costing `ncost` of a wide tile) on
// `cus` CUs (one workgroup per CU); all-wide tiles when no mix is shorter.
// For j narrow rounds only the fewest wide rounds that still cover N matter,
// so the search is over j alone (a few iterations per launch). MatMulNBits:
// 256 / 192 columns (waves of 2 x 4 / 2 x 3 MFMA tiles, cost 0.75); Mlp:
// 128 / 64 outputs (gate and up interleaved, 2 x 4 / 2 x 2 MFMA tiles; the
// narrow tile stages the same activations for half the MFMAs, so it costs
// more than half).
inline GemmTiles gemm_tiles(int64_t M, int64_t N, int cus, int64_t ww = 256, int64_t nw = 192, double ncost = 0.75) {
  const int64_t mt = (M + GB_M - 1) / GB_M, full = (N + ww - 1) / ww;
  GemmTiles best{static_cast<uint32_t>(full), 0u, static_cast<uint32_t>(mt * full)};
  if (cus <= 0 || mt * full <= cus || cus % mt != 0) return best;
  const int64_t per = cus / mt;  // column tiles per row tile in one round
  double best_t = static_cast<double>((mt * full + cus - 1) / cus);
  for (int64_t j = 1; j <= 16; ++j) {
    const int64_t rest = N - nw * j * per;  // columns left for the wide tiles
    const int64_t k = rest > 0 ? (rest + ww * per - 1) / (ww * per) : 0;
    const double t = static_cast<double>(k) + ncost * static_cast<double>(j);
    if (t < best_t - 0.05) {
      best_t = t;
      best = GemmTiles{static_cast<uint32_t>(k * per), static_cast<uint32_t>(j * per), static_cast<uint32_t>(mt * k * per)};
    }
  }
  return best;
}

// Cost of a narrow (64-output) Mlp tile against a wide (128-output) one.
#ifndef XRMM_MLP_NARROW_COST
#define XRMM_MLP_NARROW_COST 0.6
#endif

// Global-load registers of one K step.
template <int SPC>
struct GbRegs {
  u32x4 a[4];        // activations: pieces tid + 512 i of the 256 x 64 tile
  u32x4 b;           // column n0 + tid / 2, chunk 2 ks + tid % 2
  uint32_t s[SPC];   // raw scale bits per block half
  uint32_t z[SPC];   // raw zero-point bits (packed: the byte)
};

// One output tile: rows m0 .. m0 + 255, staged columns 0 .. 64 TN - 1.
// MatMulNBits and Qkv: staged column c is output column n0 + c of projection
// pi. Mlp (TN = 4 or 2): staged columns 32 g .. 32 g + 31 are the gate (g
// even) or up (g odd) projection of outputs n0 + 32 (g / 2) .. + 31, so the
// tile covers 32 TN outputs and a wave's MFMA column tiles j = 0, 1 (and 2, 3)
// hold the gate and up projection of the same 32 outputs; act(g + gate bias)
// * (u + up bias) forms in registers. A staging wave's 32 columns belong to
// one projection, so each wave's buffer resources stay uniform.
template <int ZPK, int SPC, int TN, bool PK, int OPK = OP_MATMUL>
__device__ __forceinline__ void gemm_tile(const Launch& L, const int m0, const int n0, const int pi = 0) {
  static_assert(OPK != OP_MLP || TN % 2 == 0, "Mlp tiles pair gate and up MFMA column tiles");
  constexpr bool MLP = OPK == OP_MLP;
  extern __shared__ __align__(16) unsigned char smem[];
  f16* lds = reinterpret_cast<f16*>(smem);
  constexpr uint32_t OOB = 0x80000000u;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // the projection this wave stages B from (Mlp: staged column group
  // (tid / 2) / 32 = wave, gate for even waves, up for odd)
  const int bpi = MLP ? (wave & 1) : pi;
  const Proj& P = L.p[bpi];
  const int M = static_cast<int>(L.M), N = static_cast<int>(P.N), K = static_cast<int>(L.K);
  const int Kp = static_cast<int>(L.kb * L.block_size);
  const uint32_t rowb = static_cast<uint32_t>(Kp / 2);
  const int nchunk = static_cast<int>(rowb / 16);
  const int ksteps = (Kp + GB_K - 1) / GB_K;
  const uint32_t kb = static_cast<uint32_t>(L.kb);

  const rsrc_t rA = mk_rsrc(L.A, static_cast<uint32_t>(M) * static_cast<uint32_t>(K) * 2u);
  // Thread t loads half h = t % 2 of column n0 + t / 2 each step. Its offsets
  // are past every resource bound when the column does not exist, so loads
  // return zero with no per-step select (a divergent select would become a
  // branch around the load).
  const int bc = tid >> 1, bh = tid & 1;
  const int bn = MLP ? n0 + 32 * (bc >> 6) + (bc & 31) : n0 + bc;
  const bool bnval = bc < 64 * TN && bn < N;  // narrow tiles: threads past the tile load nothing
  const uint32_t zrow = ZPK == ZP_PACKED ? static_cast<uint32_t>(L.zrow) : kb * (L.zp_dtype == DT_F32 ? 4u : 2u);
  // PK: B in the prepacked layout [K step][column][32 bytes] (prepack_q4)
  const uint32_t ksteps_b = static_cast<uint32_t>(ksteps);
  const rsrc_t rB = mk_rsrc(P.B, PK ? ksteps_b * static_cast<uint32_t>(N) * 32u : static_cast<uint32_t>(N) * rowb);
  // scale / zero-point bounds rounded to 16 bytes: the range check zeroes a
  // whole dword straddling the bound, and 16-byte aligned tensors keep the
  // rounded bound inside the block holding their last byte
  const rsrc_t rS = mk_rsrc(P.scales, (static_cast<uint32_t>(N) * kb * 2u + 15u) & ~15u);
  const rsrc_t rZ = mk_rsrc(P.zp ? P.zp : P.scales, (static_cast<uint32_t>(N) * zrow + 15u) & ~15u);
  const uint32_t bcol = bnval ? static_cast<uint32_t>(bn) * rowb : OOB;
  const uint32_t scol = bnval ? static_cast<uint32_t>(bn) * kb * 2u : OOB;
  const uint32_t zcol = bnval ? static_cast<uint32_t>(bn) * zrow : OOB;

  auto gload = [&](GbRegs<SPC>& r, int ks) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = tid + GB_T * i, row = p >> 3, grp = p & 7;
      const int m = m0 + row, k = ks * GB_K + grp * 8;
      const bool ok = m < M && k < K;  // K % 8 == 0: groups are whole
      r.a[i] = bld16(rA, ok ? static_cast<uint32_t>(m * K + k) * 2u : OOB, 0);
    }
    const int ch = ks * 2 + bh;
    const uint32_t past = ch < nchunk ? 0u : OOB;
    if constexpr (PK)
      r.b = bld16(rB, (bnval && ks < ksteps) ? (static_cast<uint32_t>(ks) * static_cast<uint32_t>(N) + static_cast<uint32_t>(bn)) * 32u + static_cast<uint32_t>(bh) * 16u : OOB, 0);
    else
      r.b = bld16(rB, bcol + past + static_cast<uint32_t>(ch) * 16u, 0);
#pragma unroll
    for (int q = 0; q < SPC; ++q) {
      const uint32_t b = static_cast<uint32_t>(ch * 32 + q * 16) >> L.bs_log2;  // block of this half-chunk
      r.s[q] = bld_u16(rS, scol + past + b * 2u, 0);
      if constexpr (ZPK == ZP_PACKED) r.z[q] = bld_u8(rZ, zcol + past + (b >> 1), 0);
      else if constexpr (ZPK == ZP_FLOAT)
        r.z[q] = L.zp_dtype == DT_F32 ? bld_u32(rZ, zcol + past + b * 4u, 0) : bld_u16(rZ, zcol + past + b * 2u, 0);
    }
  };
  // Metadata of the chunk held in r (step ks): the scale and zero point of each
  // 16-code half, as the constants the dequantisation uses.
  struct StepMeta {
    Dq c[SPC];
    float z[SPC], s[SPC];
  };
  auto meta = [&](const GbRegs<SPC>& r, int ks) {
    StepMeta mt;
#pragma unroll
    for (int q = 0; q < SPC; ++q) {
      const f16 sc = __builtin_bit_cast(f16, static_cast<uint16_t>(r.s[q]));
      float z;
      if constexpr (ZPK == ZP_NONE) {
        z = 8.f;
      } else if constexpr (ZPK == ZP_PACKED) {
        const uint32_t b = static_cast<uint32_t>((ks * 2 + bh) * 32 + q * 16) >> L.bs_log2;
        z = static_cast<float>((r.z[q] >> ((b & 1u) * 4u)) & 15u);
      } else {
        z = L.zp_dtype == DT_F32 ? __builtin_bit_cast(float, r.z[q])
                                 : static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(r.z[q])));
      }
      mt.z[q] = z;
      mt.s[q] = static_cast<float>(sc);
      if constexpr (ZPK != ZP_FLOAT) mt.c[q] = dq_consts(z, sc);
    }
    return mt;
  };
  // Part d (0..3) of writing a step's registers to LDS stage `stage`:
  // activation piece d and weight dword d (codes 8 d .. 8 d + 7 of the chunk).
  auto store_part = [&](const GbRegs<SPC>& r, const StepMeta& mt, int stage, int d) {
    f16* As = lds + stage * GB_STAGE;
    f16* Bs = As + GB_M * GB_LD;
    const int p = tid + GB_T * d, row = p >> 3, grp = p & 7;
    // prepacked codes dequantise in natural k order, the others in pair order
    *reinterpret_cast<f16x8*>(As + row * GB_LD + grp * 8) =
        PK ? __builtin_bit_cast(f16x8, r.a[d]) : pair_order(__builtin_bit_cast(f16x8, r.a[d]));
    const int q = d / (4 / SPC);
    f16x8 b;
    if constexpr (ZPK == ZP_FLOAT) b = dq8_f32z(r.b[d], mt.z[q], mt.s[q]);
    else b = dq8(r.b[d], mt.c[q]);
    *reinterpret_cast<f16x8*>(Bs + bc * GB_LD + bh * 32 + d * 8) = b;
  };

  f32x16 acc[GB_TM][TN];
#pragma unroll
  for (int i = 0; i < GB_TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragments of K slice kk (0..3) of a stage: lane (r, g) = (lane % 32,
  // lane / 32) reads row / column r, k = 16 kk + 8 g .. + 7.
  f16x8 fa[2][GB_TM], fb[2][TN];
  auto read_frags = [&](int stage, int kk, int buf) {
    const int ko = kk * 16 + (lane >> 5) * 8;
    const f16* As = lds + stage * GB_STAGE + (wm * 64 + (lane & 31)) * GB_LD + ko;
    const f16* Bs = lds + stage * GB_STAGE + (GB_M + wn * 32 * TN + (lane & 31)) * GB_LD + ko;
#pragma unroll
    for (int i = 0; i < GB_TM; ++i) fa[buf][i] = *reinterpret_cast<const f16x8*>(As + i * 32 * GB_LD);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[buf][j] = *reinterpret_cast<const f16x8*>(Bs + j * 32 * GB_LD);
  };
  auto mfmas = [&](int buf) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < GB_TM; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[buf][i], fb[buf][j], acc[i][j], 0, 0, 0);
  };
  // One K step on LDS stage `stage`: `fill` receives step ks + 2 (its previous
  // contents, step ks, are already in LDS) and `nxt` (step ks + 1, loaded a step
  // earlier) is written to the other stage in four parts, one beside each K
  // slice's MFMAs, so the dequantisation overlaps the matrix cores. Steps past
  // the last one load with offsets beyond every bound (zeros) and write a stage
  // nothing reads, so the step has no branches.
  auto step = [&](int ks, int stage, GbRegs<SPC>& nxt, GbRegs<SPC>& fill) {
    gload(fill, ks + 2);
    const StepMeta mt = meta(nxt, ks + 1);
#pragma unroll
    for (int kk = 0; kk < GB_K / 16; ++kk) {
      if (kk + 1 < GB_K / 16) read_frags(stage, kk + 1, (kk + 1) & 1);
      store_part(nxt, mt, stage ^ 1, kk);
      mfmas(kk & 1);
    }
    __syncthreads();
    read_frags(stage ^ 1, 0, 0);
  };

  GbRegs<SPC> r0, r1;
  gload(r0, 0);
  gload(r1, 1);
  {
    const StepMeta mt = meta(r0, 0);
#pragma unroll
    for (int d = 0; d < 4; ++d) store_part(r0, mt, 0, d);
  }
  __syncthreads();
  read_frags(0, 0, 0);
  int ks = 0;
  for (; ks + 1 < ksteps; ks += 2) {
    step(ks, 0, r1, r0);      // r1 holds step ks + 1, r0 receives ks + 2
    step(ks + 1, 1, r0, r1);  // r0 holds step ks + 2, r1 receives ks + 3
  }
  if (ks < ksteps) step(ks, 0, r1, r0);

  // Epilogue: lane holds D[8 (e / 4) + 4 (lane / 32) + e % 4][lane % 32] of
  // each 32x32 tile. The tile (+ bias, rounded once to binary16) goes through
  // LDS row-major, so Y is written in whole 16-byte pieces of its rows (a
  // wave stores 1 KB of two rows per instruction) instead of 2-byte scatters
  // that leave partial lines.
  constexpr int OUTW = MLP ? 32 * TN : 64 * TN;  // output columns of the tile
  constexpr int YLD = OUTW + 8;  // halfs per staged output row (pad spreads banks)
  static_assert(GB_M * YLD * 2 <= static_cast<int>(GB_LDS), "the output tile fits the LDS");
  __syncthreads();  // every wave's last fragment reads are done
  if constexpr (MLP) {
    const f16* gbias = static_cast<const f16*>(L.p[0].bias);
    const f16* ubias = static_cast<const f16*>(L.p[1].bias);
#pragma unroll
    for (int jp = 0; jp < TN / 2; ++jp) {
      const int c = wn * 16 * TN + jp * 32 + (lane & 31);  // output column inside the tile
      const bool cv = n0 + c < N;
      const float gb = (gbias != nullptr && cv) ? static_cast<float>(gbias[n0 + c]) : 0.f;
      const float ub = (ubias != nullptr && cv) ? static_cast<float>(ubias[n0 + c]) : 0.f;
#pragma unroll
      for (int i = 0; i < GB_TM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          lds[r * YLD + c] = static_cast<f16>(activate(acc[i][2 * jp][e] + gb, L.act) * (acc[i][2 * jp + 1][e] + ub));
        }
    }
  } else {
    const f16* biasp = static_cast<const f16*>(P.bias);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int c = wn * 32 * TN + j * 32 + (lane & 31);
      const float bias = (biasp != nullptr && n0 + c < N) ? static_cast<float>(biasp[n0 + c]) : 0.f;
#pragma unroll
      for (int i = 0; i < GB_TM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          lds[r * YLD + c] = static_cast<f16>(acc[i][j][e] + bias);
        }
    }
  }
  __syncthreads();
  f16* Y = static_cast<f16*>(L.p[pi].Y);
  constexpr int PPR = OUTW / 8;  // 16-byte pieces per tile row
  const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15u) == 0;
  for (int idx = tid; idx < GB_M * PPR; idx += GB_T) {
    const int r = idx / PPR, p = idx % PPR;
    const int m = m0 + r, n = n0 + 8 * p;
    if (m >= M || n >= N) continue;
    const f16* src = lds + r * YLD + 8 * p;
    f16* dst = Y + static_cast<int64_t>(m) * N + n;
    if (vec) {
      *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
    } else {
      for (int e = 0; e < 8 && n + e < N; ++e) dst[e] = src[e];
    }
  }
}

// Tile of workgroup b among the T = mt * nc tiles of one width. Consecutive
// workgroups are dispatched to consecutive XCDs (eight on gfx950, each with
// its own L2), so when T % 8 == 0 workgroup b takes logical tile
// (b % 8) * (T / 8) + b / 8: every XCD walks a contiguous range of the
// logical order. That order is a raster grouped by XRMM_GEMM_GROUP row tiles
// (row fastest inside a group), so the tiles one XCD runs at once share a few
// activation row panels and weight column panels in its L2 instead of
// spanning every row panel.
#ifndef XRMM_GEMM_GROUP
#define XRMM_GEMM_GROUP 4
#endif
__device__ __forceinline__ void tile_of(uint32_t b, uint32_t mt, uint32_t nc, uint32_t& row, uint32_t& col) {
  const uint32_t T = mt * nc;
  const uint32_t l = (T & 7u) == 0 ? (b & 7u) * (T >> 3) + (b >> 3) : b;
  constexpr uint32_t G = XRMM_GEMM_GROUP;
  const uint32_t g = l / (G * nc);
  const uint32_t rows = mt - g * G < G ? mt - g * G : G;  // row tiles in this group
  const uint32_t r = l - g * G * nc;
  row = g * G + r % rows;
  col = r / rows;
}

// The grid is one dimension: workgroup bid takes a wide tile when bid < nbig
// (a scalar, uniform branch), else a narrow one.
template <int ZPK, int SPC, bool PK = false>
__global__ __launch_bounds__(GB_T, 1) void k_gemm_q4_big(Launch L, GemmTiles t) {
  const uint32_t bid = blockIdx.x;
  const uint32_t mt = static_cast<uint32_t>((L.M + GB_M - 1) / GB_M);
  uint32_t row, col;
  if (bid < t.nbig) {
    tile_of(bid, mt, t.nb, row, col);
    gemm_tile<ZPK, SPC, 4, PK>(L, static_cast<int>(row) * GB_M, static_cast<int>(col) * 256);
  } else {
    tile_of(bid - t.nbig, mt, t.ns, row, col);
    gemm_tile<ZPK, SPC, 3, PK>(L, static_cast<int>(row) * GB_M, static_cast<int>(t.nb * 256u + col * 192u));
  }
}

// MatMulNBitsQkv / MatMulNBitsMlp on the same pipeline, all tiles 256 wide.
// L.A holds the normalised activations (the operator's prologue has run, or
// there is none), so the K loop is the MatMulNBits one. Qkv: the three
// projections' column tiles (t0, t1 and nc - t0 - t1 of them) sit side by
// side on one grid, so the GQA geometry fills the CUs with one launch. Mlp:
// a tile covers 128 outputs of the gate and up projections (256 staged
// columns).
template <int ZPK, int SPC, int OPK>
__global__ __launch_bounds__(GB_T, 1) void k_gemm_q4_big_fused(Launch L, uint32_t t0, uint32_t t1, uint32_t nc,
                                                               GemmTiles t) {
  const uint32_t mt = static_cast<uint32_t>((L.M + GB_M - 1) / GB_M);
  uint32_t row, col;
  if constexpr (OPK == OP_MLP) {
    // wide tiles (128 outputs) first on the grid, then narrow ones (64)
    const uint32_t bid = blockIdx.x;
    if (bid < t.nbig) {
      tile_of(bid, mt, t.nb, row, col);
      gemm_tile<ZPK, SPC, 4, false, OP_MLP>(L, static_cast<int>(row) * GB_M, static_cast<int>(col) * 128, 0);
    } else {
      tile_of(bid - t.nbig, mt, t.ns, row, col);
      gemm_tile<ZPK, SPC, 2, false, OP_MLP>(L, static_cast<int>(row) * GB_M,
                                            static_cast<int>(t.nb * 128u + col * 64u), 0);
    }
  } else {
    tile_of(blockIdx.x, mt, nc, row, col);
    const int pi = col < t0 ? 0 : col < t0 + t1 ? 1 : 2;
    const uint32_t lc = col - (pi == 0 ? 0u : pi == 1 ? t0 : t0 + t1);
    gemm_tile<ZPK, SPC, 4, false, OP_QKV>(L, static_cast<int>(row) * GB_M, static_cast<int>(lc) * 256, pi);
  }
}

// Column tiles of the fused grid: Qkv per projection (256 outputs each),
// Mlp 128 outputs per tile.
inline void gemm_fused_tiles(const Launch& L, uint32_t& t0, uint32_t& t1, uint32_t& nc) {
  if (L.op == OP_MLP) {
    t0 = t1 = 0;
    nc = static_cast<uint32_t>((L.p[0].N + 127) / 128);
  } else {
    t0 = static_cast<uint32_t>((L.p[0].N + 255) / 256);
    t1 = static_cast<uint32_t>((L.p[1].N + 255) / 256);
    nc = t0 + t1 + static_cast<uint32_t>((L.p[2].N + 255) / 256);
  }
}

// Compute units of the current device (cached per device ordinal).
int device_cus();

template <int ZPK, int SPC, bool PK = false>
inline hipError_t launch_gemm_big(const Launch& L, hipStream_t st) {
  auto kern = k_gemm_q4_big<ZPK, SPC, PK>;
  // more than 64 KB of dynamic LDS needs the attribute; set once per
  // instantiation and device
  static std::atomic<int> done[kMaxDevices];
  const hipError_t attr = raise_lds_cap(reinterpret_cast<const void*>(kern), static_cast<int>(GB_LDS), done);
  if (attr != hipSuccess) return attr;
  const GemmTiles t = gemm_tiles(L.M, L.p[0].N, device_cus());
  const int64_t mt = (L.M + GB_M - 1) / GB_M;
  const dim3 grid(static_cast<uint32_t>(mt * (t.nb + t.ns)));
  hipLaunchKernelGGL(kern, grid, dim3(GB_T), GB_LDS, st, L, t);
  return hipGetLastError();
}

template <int ZPK, int SPC, int OPK>
inline hipError_t launch_gemm_big_fused(const Launch& L, hipStream_t st) {
  auto kern = k_gemm_q4_big_fused<ZPK, SPC, OPK>;
  static std::atomic<int> done[kMaxDevices];
  const hipError_t attr = raise_lds_cap(reinterpret_cast<const void*>(kern), static_cast<int>(GB_LDS), done);
  if (attr != hipSuccess) return attr;
  uint32_t t0, t1, nc;
  gemm_fused_tiles(L, t0, t1, nc);
  GemmTiles t{nc, 0u, 0u};
  int64_t tiles = (L.M + GB_M - 1) / GB_M * static_cast<int64_t>(nc);
  if (OPK == OP_MLP) {
    t = gemm_tiles(L.M, L.p[0].N, device_cus(), 128, 64, XRMM_MLP_NARROW_COST);
    tiles = (L.M + GB_M - 1) / GB_M * static_cast<int64_t>(t.nb + t.ns);
  }
  if (tiles > 0x7FFFFFFF) return hipErrorInvalidValue;  // launch limit
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(tiles)), dim3(GB_T), GB_LDS, st, L, t0, t1, nc, t);
  return hipGetLastError();
}

// Defined once per zero-point kind (xrmm_gemm_zp.hip).
template <int ZPK>
hipError_t launch_gemm_big_for(const Launch& L, hipStream_t st);
// Qkv / Mlp on the 256 x 256 pipeline (L.A already normalised).
template <int ZPK>
hipError_t launch_gemm_big_fused_for(const Launch& L, hipStream_t st);
// The same GEMM on prepacked weights (L.p[0].B in the prepack_q4 layout).
template <int ZPK>
hipError_t launch_gemm_big_pk_for(const Launch& L, hipStream_t st);

}  // namespace xrmm
