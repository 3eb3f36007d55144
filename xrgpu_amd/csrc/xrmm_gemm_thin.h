// Short-prefill GEMM (17..64 rows of fp16 activations x 4-bit weights): the
// weight stream dominates, so weights go from memory straight into the MFMA
// operand registers (dequantised there, no LDS round trip) and only the
// activations, shared by every wave of the workgroup, are staged in LDS.
//
// Work split. A workgroup owns NT = 32 CG output columns and one K split
// (grid = column tiles x splits). Its eight waves are CG column groups of 32
// columns times KQ = 8 / CG K groups; K advances in chunks of KC, and in
// iteration i K group q takes chunk c0 + KQ i + q of the split (the
// iterations in a rotated order per workgroup, see cfirst), so the
// workgroup stages KQ consecutive chunks of the activations per iteration
// (double-buffered) and each wave multiplies all rows (two 32-row MFMA
// tiles) by its 32 columns.
//
// Operands of v_mfma_f32_32x32x16_f16: lane (n, g) = (lane % 32, lane / 32)
// loads 16-byte pieces 2 j + g of column n's chunk (32 codes each, j < KC /
// 64); dword d of piece 2 j + g supplies the lane's eight B values of MFMA
// step (j, d), dequantised by dq8 in the pair order (c0 c4 c1 c5 c2 c6 c3 c7).
// The activations are staged in the same pair order, so lane (m, g) reads its
// eight A values of step (j, d) as one 16-byte piece of row m at k =
// 32 (2 j + g) + 8 d.
//
// Memory order. The vector-memory counter retires loads in issue order, so
// each iteration issues the next iteration's activations before the weights
// two iterations ahead: waiting for those activations at the end of the
// iteration then waits only for weights issued an iteration earlier, and
// every weight load has two iterations to arrive.
//
// End. The K groups' accumulators meet in LDS; with several splits every
// split's float32 partial tile goes to the workspace and the last split of a
// tile to arrive adds them in split order (deterministic), clears the tile's
// counter and writes Y (+ bias, rounded once to binary16).
//
// MatMulNBitsMlp (MLP): the two column groups are the gate and the up
// projection of the same 32 outputs (CG = 2), the activations are the
// prologue's normalised rows, and the up group's tile reaches the gate
// group through LDS for act(g + gate bias) * (u + up bias); one split.
#pragma once
#include "xrmm_device.h"

namespace xrmm {

constexpr int GT_T = 512;     // threads (eight waves)
constexpr int GT_IMAX = 8;    // iterations per round (the round's loop is unrolled)
constexpr uint32_t kThinCounterBytes = 4096;  // per-tile arrival counters, then the partial tiles

struct ThinArgs {
  uint32_t S;       // K splits
  uint32_t nkc;     // chunks of KC codes in the padded K
  uint32_t cps;     // chunks per split
  uint32_t ni;      // iterations per split (chunks per K group)
  uint32_t tiles;   // column tiles
};

// Block-metadata slots per column and iteration (the KQ chunks of an
// iteration span at most KQ KC / 16 blocks of 16 codes, or two blocks when
// blocks are longer than the iteration).
template <int CG, int KC>
__host__ __device__ constexpr int thin_meta_slots() {
  return (8 / CG) * KC / 16;
}

// LDS bytes: two buffers of KQ chunks x rows x (KC + 8) halfs, and with
// staged metadata (integer zero points) two buffers of NT columns x slots of
// binary16 scales and zero-point nibbles (one byte each).
template <int CG, int KC, int MT, bool STG>
__host__ __device__ constexpr int thin_lds_bytes() {
  return 2 * (8 / CG) * (32 * MT) * (KC + 8) * 2 + (STG ? 2 * 32 * CG * thin_meta_slots<CG, KC>() * 3 : 0);
}

template <int ZPK, int SPC, int CG, int KC, int MT, bool MLP = false>
__global__ __launch_bounds__(GT_T) void k_gemm_thin(Launch L, ThinArgs t) {
  static_assert(!MLP || CG == 2, "Mlp tiles pair one gate and one up column group");
  // Integer zero points (and none): the iteration's scales and zero points
  // are staged in LDS with the activations, loaded by consecutive threads
  // along each column's block row. Float zero points: each lane loads its
  // pieces' metadata itself.
  constexpr bool STG = ZPK != ZP_FLOAT;
  constexpr int KQ = 8 / CG, NT = 32 * CG, ROWS = 32 * MT;
  constexpr int MS = thin_meta_slots<CG, KC>();     // metadata slots per column and iteration
  constexpr int MPT = NT * MS / GT_T;               // metadata slots per thread
  static_assert(MPT * GT_T == NT * MS, "metadata slots divide over the threads");
  constexpr int META = NT * MS * 3;                 // bytes per metadata buffer (scales, then nibbles)
  constexpr int LD = KC + 8;                  // halfs per staged row
  constexpr int CH = ROWS * LD;               // halfs per staged chunk
  constexpr int BUF = KQ * CH;                // halfs per buffer
  constexpr int PJ = KC / 64;                 // pieces per lane per iteration
  constexpr int GPR = KC / 8;                 // 8-half groups per staged row
  constexpr int APT = KQ * ROWS * GPR / GT_T; // activation pieces per thread per iteration
  static_assert(APT * GT_T == KQ * ROWS * GPR, "activation pieces divide over the threads");
  constexpr uint32_t OOB = 0x80000000u;
  extern __shared__ __align__(16) unsigned char smem[];
  f16* lds = reinterpret_cast<f16*>(smem);
  unsigned char* mlds = smem + 2 * BUF * 2;  // metadata buffers

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = wave % CG, kq = wave / CG;
  const uint32_t bid = blockIdx.x;
  const uint32_t tile = bid / t.S, sp = bid % t.S;
  // the wave's projection: Mlp gate (group 0) or up (group 1); the index is
  // wave-uniform, so the buffer resources below stay scalar
  const Proj& P = L.p[MLP ? cg : 0];
  const uint32_t M = static_cast<uint32_t>(L.M), N = static_cast<uint32_t>(P.N), K = static_cast<uint32_t>(L.K);
  const uint32_t kb = static_cast<uint32_t>(L.kb);
  const uint32_t rowb = static_cast<uint32_t>(L.kb * L.block_size / 2);
  const uint32_t nchunk = rowb / 16;
  const uint32_t c0 = sp * t.cps;
  const uint32_t c1 = c0 + t.cps < t.nkc ? c0 + t.cps : t.nkc;
  // First chunk of loop iteration i. The workgroups of one split (about
  // one XCD's share, all wanting the same activations) walk its iterations
  // from different starting points, so each activation chunk is fetched from
  // memory by one of them and found in the L2 by the others, instead of every
  // workgroup missing on the same chunk at the same time.
  const uint32_t rot = t.ni > 1 ? tile % t.ni : 0u;
  auto cfirst = [&](uint32_t i) {
    uint32_t ii = i + rot;
    ii = ii >= t.ni ? ii - t.ni : ii;
    return c0 + KQ * ii;
  };

  // ---- this lane's weight column (Mlp: output column of both groups)
  constexpr uint32_t NO = MLP ? 32u : static_cast<uint32_t>(NT);  // output columns per tile
  const uint32_t n0 = tile * NO;
  const uint32_t n = n0 + (MLP ? 0u : 32u * cg) + static_cast<uint32_t>(lane & 31);
  const uint32_t g = static_cast<uint32_t>(lane >> 5);
  const bool nval = n < N;
  const uint32_t zrow = ZPK == ZP_PACKED ? static_cast<uint32_t>(L.zrow) : kb * (L.zp_dtype == DT_F32 ? 4u : 2u);
  const rsrc_t rB = mk_rsrc(P.B, N * rowb);
  const rsrc_t rS = mk_rsrc(P.scales, (N * kb * 2u + 15u) & ~15u);
  const rsrc_t rZ = mk_rsrc(P.zp ? P.zp : P.scales, (N * zrow + 15u) & ~15u);
  const uint32_t bcol = nval ? n * rowb : OOB;
  const uint32_t scol = nval ? n * kb * 2u : OOB;
  const uint32_t zcol = nval ? n * zrow : OOB;

  struct WRegs {
    u32x4 w[PJ];
    uint32_t s[STG ? 1 : PJ][SPC], z[STG ? 1 : PJ][SPC];
  };
  // weights of iteration i (chunk c0 + KQ i + kq of this K group); `live`
  // false turns the loads into zero reads instead of branching around them
  // (a branch around a load makes every later wait a full drain)
  auto wload = [&](WRegs& r, uint32_t i, bool live) {
    const uint32_t c = cfirst(i) + static_cast<uint32_t>(kq);
    const bool cv = live & (c < c1);
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const uint32_t pc = c * (KC / 32) + 2u * j + g;  // 16-byte piece of the column
      const uint32_t past = (cv & (pc < nchunk)) ? 0u : OOB;
      // default cache policy: a 128-byte line of the column is read by four
      // load instructions (two pieces each of two chunks), so it should stay
      // in the caches between them (non-temporal loads measured 10% slower)
      r.w[j] = bld16(rB, (bcol | past) + pc * 16u, 0);
      if constexpr (!STG) {
#pragma unroll
      for (int q = 0; q < SPC; ++q) {
        const uint32_t b = (pc * 32u + 16u * q) >> L.bs_log2;
        r.s[j][q] = bld_u16(rS, (scol | past) + b * 2u, 0);
        r.z[j][q] = 0u;
        if constexpr (ZPK == ZP_PACKED) r.z[j][q] = bld_u8(rZ, (zcol | past) + (b >> 1), 0);
        else if constexpr (ZPK == ZP_FLOAT)
          r.z[j][q] = L.zp_dtype == DT_F32 ? bld_u32(rZ, (zcol | past) + b * 4u, 0) : bld_u16(rZ, (zcol | past) + b * 2u, 0);
      }
      }
    }
  };

  // ---- activations: KQ chunks x ROWS rows of an iteration, APT 16-byte
  // pieces per thread (rows past M and k past K read zero)
  const rsrc_t rA = mk_rsrc(L.A, M * K * 2u);
  // first block of iteration i's chunks, and how many blocks they span
  auto blk0 = [&](uint32_t i) { return (cfirst(i) * KC) >> L.bs_log2; };
  auto nblk = [&](uint32_t i) { return ((((cfirst(i) + KQ) * KC) - 1u) >> L.bs_log2) - blk0(i) + 1u; };
  struct MRegs {
    uint32_t s[STG ? MPT : 1], z[STG ? MPT : 1];
  };
  // metadata of iteration i: slot e = tid + GT_T x is block blk0 + e % MS of
  // column n0 + e / MS
  // Mlp: the first half of the slots (x < MPT / 2) are the gate columns, the
  // second half the up columns, so each load's projection is known at compile time
  static_assert(!MLP || (MPT % 2 == 0 && GT_T * (MPT / 2) == 32 * MS), "gate slots, then up slots");
  const rsrc_t rS0 = mk_rsrc(L.p[0].scales, (N * kb * 2u + 15u) & ~15u);
  const rsrc_t rS1 = MLP ? mk_rsrc(L.p[1].scales, (N * kb * 2u + 15u) & ~15u) : rS0;
  const void* z0 = L.p[0].zp ? L.p[0].zp : L.p[0].scales;
  const rsrc_t rZ0 = mk_rsrc(z0, (N * zrow + 15u) & ~15u);
  const rsrc_t rZ1 = MLP ? mk_rsrc(L.p[1].zp ? L.p[1].zp : L.p[1].scales, (N * zrow + 15u) & ~15u) : rZ0;
  auto mload = [&](MRegs& mr, uint32_t i, bool live) {
    if constexpr (STG) {
      const uint32_t b0 = blk0(i), nb = nblk(i);
      const bool it = live & (cfirst(i) < c1);
#pragma unroll
      for (int x = 0; x < MPT; ++x) {
        const bool up = MLP && x >= MPT / 2;
        const uint32_t e = static_cast<uint32_t>(tid + GT_T * x), ct = e / MS, sl = e % MS, b = b0 + sl;
        const uint32_t col = n0 + (MLP ? (ct & 31u) : ct);
        const bool ok = it & (sl < nb) & (col < N) & (b < kb);
        mr.s[x] = bld_u16(up ? rS1 : rS0, ok ? col * kb * 2u + b * 2u : OOB, 0);
        mr.z[x] = 0u;
        if constexpr (ZPK == ZP_PACKED) mr.z[x] = bld_u8(up ? rZ1 : rZ0, ok ? col * zrow + (b >> 1) : OOB, 0);
      }
    }
  };
  auto mstore = [&](const MRegs& mr, int buf, uint32_t i) {
    if constexpr (STG) {
      unsigned char* ms = mlds + buf * META;
      const uint32_t b0 = blk0(i);
#pragma unroll
      for (int x = 0; x < MPT; ++x) {
        const uint32_t e = static_cast<uint32_t>(tid + GT_T * x);
        *reinterpret_cast<uint16_t*>(ms + e * 2u) = static_cast<uint16_t>(mr.s[x]);
        if constexpr (ZPK == ZP_PACKED) ms[NT * MS * 2 + e] = static_cast<unsigned char>((mr.z[x] >> (((b0 + e % MS) & 1u) * 4u)) & 15u);
      }
    }
  };
  auto aload = [&](u32x4 (&ra)[APT], uint32_t i, bool live) {
#pragma unroll
    for (int e = 0; e < APT; ++e) {
      const int p = tid + GT_T * e;
      const int q = p / (ROWS * GPR), rem = p % (ROWS * GPR), row = rem / GPR, grp = rem % GPR;
      const uint32_t c = cfirst(i) + static_cast<uint32_t>(q);
      const uint32_t k = c * KC + static_cast<uint32_t>(grp) * 8u;
      const bool ok = live & (c < c1) & (static_cast<uint32_t>(row) < M) & (k < K);  // K % 8 == 0
      ra[e] = bld16(rA, ok ? (static_cast<uint32_t>(row) * K + k) * 2u : OOB, 0);
    }
  };
  auto astore = [&](const u32x4 (&ra)[APT], int buf) {
#pragma unroll
    for (int e = 0; e < APT; ++e) {
      const int p = tid + GT_T * e;
      const int q = p / (ROWS * GPR), rem = p % (ROWS * GPR), row = rem / GPR, grp = rem % GPR;
      *reinterpret_cast<f16x8*>(lds + buf * BUF + q * CH + row * LD + grp * 8) = pair_order(__builtin_bit_cast(f16x8, ra[e]));
    }
  };

  f32x16 acc[MT];
#pragma unroll
  for (int r = 0; r < MT; ++r)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[r][e] = 0.f;

  // one iteration's MFMAs on buffer `buf` with the weights of `r`
  auto compute = [&](const WRegs& r, int buf, uint32_t i) {
    const uint32_t c = cfirst(i) + static_cast<uint32_t>(kq);
    const f16* As = lds + buf * BUF + kq * CH + (lane & 31) * LD + g * 32;
    const unsigned char* ms = mlds + buf * META + (32u * cg + static_cast<uint32_t>(lane & 31)) * MS * 2u;
    const unsigned char* mz = mlds + buf * META + NT * MS * 2 + (32u * cg + static_cast<uint32_t>(lane & 31)) * MS;
    const uint32_t b0 = blk0(i);
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      Dq dc[SPC];
      float zf[SPC], sf[SPC];
#pragma unroll
      for (int q = 0; q < SPC; ++q) {
        const uint32_t pc = c * (KC / 32) + 2u * j + g;
        const uint32_t b = (pc * 32u + 16u * q) >> L.bs_log2;
        const uint16_t sbits = STG ? *reinterpret_cast<const uint16_t*>(ms + (b - b0) * 2u) : static_cast<uint16_t>(r.s[STG ? 0 : j][q]);
        const f16 sc = __builtin_bit_cast(f16, sbits);
        float z;
        if constexpr (ZPK == ZP_NONE) {
          z = 8.f;
        } else if constexpr (ZPK == ZP_PACKED) {
          z = static_cast<float>(mz[b - b0]);
        } else {
          z = L.zp_dtype == DT_F32 ? __builtin_bit_cast(float, r.z[STG ? 0 : j][q])
                                   : static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(r.z[STG ? 0 : j][q])));
        }
        zf[q] = z;
        sf[q] = static_cast<float>(sc);
        if constexpr (ZPK != ZP_FLOAT) dc[q] = dq_consts(z, sc);
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int q = d / (4 / SPC);
        f16x8 b;
        if constexpr (ZPK == ZP_FLOAT) b = dq8_f32z(r.w[j][d], zf[q], sf[q]);
        else b = dq8(r.w[j][d], dc[q]);
#pragma unroll
        for (int rt = 0; rt < MT; ++rt) {
          const f16x8 a = *reinterpret_cast<const f16x8*>(As + rt * 32 * LD + j * 64 + d * 8);
          acc[rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[rt], 0, 0, 0);
        }
      }
    }
  };

  // ---- pipeline: weights two iterations ahead, activations one ahead, in
  // rounds of up to GT_IMAX iterations (one round unless a single split
  // covers a long K). Measured slower and not kept: every weight load of a
  // round issued at its start (activations two iterations ahead), 31.1
  // against 27.0 us on the down projection; a rolled loop of three
  // iterations per body, 35.4 us.
  for (uint32_t base = 0; base < t.ni; base += GT_IMAX) {
    const uint32_t nr = t.ni - base < GT_IMAX ? t.ni - base : GT_IMAX;
    WRegs wr[GT_IMAX];
    u32x4 ra[APT];
    MRegs mr;
    aload(ra, base, true);
    mload(mr, base, true);
    wload(wr[0], base, true);
    wload(wr[1], base + 1, nr > 1);
    astore(ra, 0);  // buffer 0 was last read before the previous round's final barrier
    mstore(mr, 0, base);
    aload(ra, base + 1, nr > 1);
    mload(mr, base + 1, nr > 1);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < GT_IMAX; ++i) {
      if (static_cast<uint32_t>(i) >= nr) break;
      if (i + 2 < GT_IMAX) wload(wr[i + 2], base + i + 2, static_cast<uint32_t>(i + 2) < nr);
      compute(wr[i], i & 1, base + i);
      // buffer (i + 1) % 2 was last read in iteration i - 1; after the
      // round's last iteration the store lands in a buffer nothing reads
      astore(ra, (i + 1) & 1);
      mstore(mr, (i + 1) & 1, base + i + 1);
      if (i + 2 < GT_IMAX) {
        aload(ra, base + i + 2, static_cast<uint32_t>(i + 2) < nr);
        mload(mr, base + i + 2, static_cast<uint32_t>(i + 2) < nr);
      }
      __syncthreads();
    }
  }

  // ---- K groups meet in LDS (the activation buffers are free now)
  float* red = reinterpret_cast<float*>(smem);
  static_assert((KQ - 1) * CG * MT * 16 * 64 * 4 <= thin_lds_bytes<CG, KC, MT, STG>(), "the K-group partials fit the LDS");
  if (kq > 0) {
#pragma unroll
    for (int r = 0; r < MT; ++r)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[((((kq - 1) * CG + cg) * MT + r) * 16 + e) * 64 + lane] = acc[r][e];
  }
  __syncthreads();
  // from here on the first CG waves (K group 0) hold the tile; the others
  // stay for the workgroup barriers only
  if (kq == 0) {
#pragma unroll
    for (int q = 1; q < KQ; ++q)
#pragma unroll
      for (int r = 0; r < MT; ++r)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[r][e] += red[((((q - 1) * CG + cg) * MT + r) * 16 + e) * 64 + lane];
  }

  // lane holds D[8 (e / 4) + 4 (lane / 32) + e % 4][lane % 32] of row tile r
  const uint32_t prow = 4u * g;
  if constexpr (MLP) {
    // the up group's tile (past the K-group partials) for the gate group
    float* upt = red + (KQ - 1) * CG * MT * 16 * 64;
    static_assert(((KQ - 1) * CG + 1) * MT * 16 * 64 * 4 <= thin_lds_bytes<CG, KC, MT, STG>(), "the up tile fits the LDS");
    if (kq == 0 && cg == 1) {
#pragma unroll
      for (int r = 0; r < MT; ++r)
#pragma unroll
        for (int e = 0; e < 16; ++e) upt[(r * 16 + e) * 64 + lane] = acc[r][e];
    }
    __syncthreads();
    if (kq != 0 || cg != 0 || !nval) return;
    const float gb = L.p[0].bias ? static_cast<float>(static_cast<const f16*>(L.p[0].bias)[n]) : 0.f;
    const float ub = L.p[1].bias ? static_cast<float>(static_cast<const f16*>(L.p[1].bias)[n]) : 0.f;
    f16* Y = static_cast<f16*>(L.p[0].Y);
#pragma unroll
    for (int r = 0; r < MT; ++r)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t m = 32u * r + 8u * (e >> 2) + prow + (e & 3);
        const float u = upt[(r * 16 + e) * 64 + lane] + ub;
        if (m < M) Y[m * N + n] = static_cast<f16>(activate(acc[r][e] + gb, L.act) * u);
      }
    return;
  }
  if (t.S > 1) {
    // Split-K: system-coherent (sc0 sc1) 16-byte stores of this split's
    // partial tile, every wave waits for its own, then one arrival count per
    // workgroup; the last split reads the partials back coherently in split
    // order. The count stays relaxed (an acquire-release count would write
    // back and invalidate the whole L2 in every workgroup for stores that
    // bypass it); the partial stores and loads are coherent themselves.
    constexpr int COHERENT = 1 | 16;
    constexpr uint32_t PIECES = MT * 4;
    constexpr uint32_t TILE_BYTES = PIECES * CG * 64 * 16;
    __shared__ int s_last;
    uint32_t* cnt = static_cast<uint32_t*>(L.ws);
    const rsrc_t rW = mk_rsrc(static_cast<uint8_t*>(L.ws) + kThinCounterBytes, t.tiles * t.S * TILE_BYTES);
    auto poff = [&](uint32_t s, uint32_t piece) {
      const uint32_t r = piece >> 2, q = piece & 3u;
      if (32u * r + 8u * q + prow >= M) return OOB;  // rows past M move nothing
      return ((tile * t.S + s) * PIECES + piece) * (CG * 64u * 16u) + (static_cast<uint32_t>(cg) * 64u + lane) * 16u;
    };
    if (kq == 0) {
#pragma unroll
      for (uint32_t piece = 0; piece < PIECES; ++piece) {
        const uint32_t r = piece >> 2, q = piece & 3u;
        const f32x4 v = {acc[r][4 * q], acc[r][4 * q + 1], acc[r][4 * q + 2], acc[r][4 * q + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rW, poff(sp, piece), 0, COHERENT);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == t.S - 1;
    __syncthreads();
    if (!s_last || kq != 0) return;
#pragma unroll
    for (int r = 0; r < MT; ++r)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[r][e] = 0.f;
    for (uint32_t s = 0; s < t.S; ++s) {
#pragma unroll
      for (uint32_t piece = 0; piece < PIECES; ++piece) {
        const uint32_t r = piece >> 2, q = piece & 3u;
        const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rW, poff(s, piece), 0, COHERENT));
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[r][4 * q + e] += v[e];
      }
    }
    if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (kq != 0 || !nval) return;
  const float bias = P.bias ? static_cast<float>(static_cast<const f16*>(P.bias)[n]) : 0.f;
  f16* Y = static_cast<f16*>(P.Y);
#pragma unroll
  for (int r = 0; r < MT; ++r)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t m = 32u * r + 8u * (e >> 2) + prow + (e & 3);
      if (m < M) Y[m * N + n] = static_cast<f16>(acc[r][e] + bias);
    }
}

// Host plan: with a workspace, splits so that tiles x splits fills about one
// round of the CUs (eight at most, and each split gives every K group at
// least one chunk); without one, a single split. S = 0: no plan (more column
// tiles than arrival counters).
template <int CG, int KC>
inline ThinArgs thin_plan(int64_t Kp, int64_t N, int cus, bool have_ws) {
  constexpr int KQ = 8 / CG, NT = 32 * CG;
  ThinArgs a{};
  a.tiles = static_cast<uint32_t>((N + NT - 1) / NT);
  a.nkc = static_cast<uint32_t>((Kp + KC - 1) / KC);
  int64_t s = have_ws ? (cus > 0 ? cus : 256) / static_cast<int64_t>(a.tiles) : 1;
  s = s > 8 ? 8 : s;
  if (s > static_cast<int64_t>(a.nkc) / KQ) s = static_cast<int64_t>(a.nkc) / KQ;
  if (s < 1) s = 1;
  if (s > 1 && a.tiles * 4 > kThinCounterBytes) s = 1;
  a.S = static_cast<uint32_t>(s);
  a.cps = static_cast<uint32_t>((a.nkc + s - 1) / s);
  a.ni = (a.cps + KQ - 1) / KQ;
  return a;
}

template <int CG, int MT>
inline int64_t thin_workspace_bytes(const ThinArgs& a) {
  if (a.S < 2) return 0;
  return kThinCounterBytes + int64_t(a.tiles) * a.S * (MT * 4) * CG * 64 * 16;
}

// Column groups per workgroup (2: 64-column tiles, 128-code chunks; 4:
// 128-column tiles, 256-code chunks). Every translation unit of one library
// must see the same value.
#ifndef XRMM_THIN_CG
#define XRMM_THIN_CG 2
#endif
constexpr int kThinCG = XRMM_THIN_CG;
constexpr int kThinKC = kThinCG == 2 ? 128 : 256;

// Compute units of the current device (cached per device ordinal).
int device_cus();

// Mlp tiles hold 32 outputs (gate and up columns of them), one split.
inline ThinArgs thin_args(const Launch& L, bool have_ws) {
  if (L.op == OP_MLP) return thin_plan<2, 128>(L.kb * L.block_size, 2 * L.p[0].N, device_cus(), false);
  return thin_plan<kThinCG, kThinKC>(L.kb * L.block_size, L.p[0].N, device_cus(), have_ws);
}

// Split-K workspace bytes of the geometry (0: no split).
inline int64_t thin_ws_bytes(const Launch& L) {
  if (L.op == OP_MLP) return 0;
  const ThinArgs a = thin_args(L, true);
  return L.M <= 32 ? thin_workspace_bytes<kThinCG, 1>(a) : thin_workspace_bytes<kThinCG, 2>(a);
}

template <int ZPK, int SPC, int MT, bool MLP>
inline hipError_t launch_thin3(const Launch& L, hipStream_t st) {
  constexpr int CG = MLP ? 2 : kThinCG, KC = MLP ? 128 : kThinKC;
  auto kern = k_gemm_thin<ZPK, SPC, CG, KC, MT, MLP>;
  constexpr int lds = thin_lds_bytes<CG, KC, MT, ZPK != ZP_FLOAT>();
  if (lds > 64 * 1024) {
    static std::atomic<int> done[kMaxDevices];
    const hipError_t e = raise_lds_cap(reinterpret_cast<const void*>(kern), lds, done);
    if (e != hipSuccess) return e;
  }
  const bool ws = !MLP && L.ws != nullptr && L.splits > 1;
  ThinArgs a = thin_args(L, ws);
  if (ws && a.S != static_cast<uint32_t>(L.splits)) a = thin_args(L, false);  // planned for another split: run unsplit
  const uint64_t grid = uint64_t(a.tiles) * a.S;
  if (grid == 0 || grid > 0x7FFFFFFFu) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(grid)), dim3(GT_T), lds, st, L, a);
  return hipGetLastError();
}

template <int ZPK, bool MLP>
inline hipError_t launch_thin2(const Launch& L, hipStream_t st) {
  if (L.block_size >= 32)
    return L.M <= 32 ? launch_thin3<ZPK, 1, 1, MLP>(L, st) : launch_thin3<ZPK, 1, 2, MLP>(L, st);
  return L.M <= 32 ? launch_thin3<ZPK, 2, 1, MLP>(L, st) : launch_thin3<ZPK, 2, 2, MLP>(L, st);
}

// MatMulNBits, or MatMulNBitsMlp on rows that need no prologue (normalised
// rows from the prologue, or no skip and no normScale).
template <int ZPK>
inline hipError_t launch_thin(const Launch& L, hipStream_t st) {
  return L.op == OP_MLP ? launch_thin2<ZPK, true>(L, st) : launch_thin2<ZPK, false>(L, st);
}

// Defined once per zero-point kind (xrmm_gemm_zp.hip).
template <int ZPK>
hipError_t launch_gemm_thin_for(const Launch& L, hipStream_t st);

}  // namespace xrmm
