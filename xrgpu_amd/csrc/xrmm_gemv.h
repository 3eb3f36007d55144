// GEMV kernel family (M <= 16) and its host-side launch helpers. Each
// zero-point kind is instantiated in its own translation unit
// (xrmm_gemv_zp.hip built once per kind) so the instantiations compile in
// parallel.
#pragma once
#include "xrmm_device.h"

namespace xrmm {

// ---------------------------------------------------------------------------
// GEMV for M <= 16: fp16 activations, 4-bit weights, MFMA 16x16x32
//
// A workgroup of GEMV_WAVES waves owns TILES consecutive 16-column tiles of one
// projection; the GEMV_WAVES / TILES waves that share a tile split its K range
// in 128-byte steps (8 chunks of 16 bytes per column). Lane (c, g) of a wave
// streams column c; in step s it takes chunks 8s + g and 8s + 4 + g, so the
// four lanes of a column read whole 128-byte lines.
//
// Per-block scales and zero points are not loaded per chunk (2-byte scattered
// loads cost as much as the weight stream itself): the workgroup loads its
// whole scale / zero-point tile with coalesced 16-byte loads into LDS, and
// lanes read their block's scale from there.
//
// Memory ordering matters because the vector-memory counter retires loads in
// issue order: the activation loads and the scale / zero-point tile loads are
// issued first, then the first batch of weight loads, so that staging waits
// only for those while the weight stream is in flight. Weights and tiles are
// read through raw buffer resources: each load address is a per-lane VGPR
// offset fixed for the whole kernel plus a wave-uniform SGPR offset, and reads
// past the end of a resource return zero, so the loads carry no address
// arithmetic and no branches. Chunks past the end of a row meet zero
// activations (the staged row is zero-padded and those lanes read a zero
// block), so whatever they read contributes nothing.

constexpr int GEMV_WAVES = 4;
constexpr int GEMV_NT = GEMV_WAVES * 64;
constexpr int GEMV_SB = 4;           // steps per load batch
constexpr int GEMV_SA_FLAT = 4;      // staged 8-element groups per thread in one flat register pass
constexpr int GEMV_SA_ROWS = 8;      // staged groups per lane when one wave stages one row
constexpr int GEMV_TILE_PIECES = 4;  // 16-byte pieces per thread of a scale or zero-point tile (16 KB)

// Activation staging modes (chosen on the host from M, K and the operator).
enum Stage {
  ST_FLAT = 0,   // no normalisation, all groups fit one register pass
  ST_ROWS = 1,   // normalisation, one row per wave, row fits one register pass
  ST_MULTI = 2,  // anything else: streamed passes after the first weight batch
};

// LDS layout of a GEMV workgroup (identical on host and device). The K-split
// reduction reuses the start of the buffer after the main loop.
struct GemvLds {
  uint32_t zero_off;   // 64-byte zero block after the staged rows
  uint32_t s_off[2];   // scale tile of each weight stream
  uint32_t z_off[2];   // zero-point tile of each weight stream
  uint32_t s_bytes, z_bytes, total;
};

__host__ __device__ inline uint32_t align16(uint32_t x) { return (x + 15u) & ~15u; }

__host__ __device__ inline GemvLds gemv_lds(const Launch& L, int tiles) {
  GemvLds y;
  const uint32_t rows = 16u * static_cast<uint32_t>(tiles);
  const uint32_t kb = static_cast<uint32_t>(L.kb);
  const uint32_t a = static_cast<uint32_t>(L.M * (L.kb * L.block_size + 8) * 2);
  const int streams = L.op == OP_MLP ? 2 : 1;
  y.zero_off = a;
  y.s_bytes = rows * kb * 2;
  y.z_bytes = L.zp_kind == ZP_PACKED ? rows * static_cast<uint32_t>(L.zrow)
              : L.zp_kind == ZP_FLOAT ? rows * kb * (L.zp_dtype == DT_F32 ? 4u : 2u)
                                      : 0u;
  uint32_t off = align16(a + 64);
  for (int i = 0; i < 2; ++i) {
    y.s_off[i] = off;
    if (i < streams) off = align16(off + y.s_bytes);
    y.z_off[i] = off;
    if (i < streams) off = align16(off + y.z_bytes);
  }
  const uint32_t red = static_cast<uint32_t>(GEMV_WAVES - tiles) * 64u * (streams == 2 ? 8u : 4u) * 4u;
  y.total = off > red ? off : red;
  return y;
}

template <int ZPK, int SPC, int OP, int TILES, bool DB, int STAGE>
__global__ __launch_bounds__(GEMV_NT) void k_gemv_q4(Launch L) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float s_inv[16];
  constexpr int KS = GEMV_WAVES / TILES;  // waves per tile (K split)
  constexpr int SB = GEMV_SB;
  constexpr bool MLP = OP == OP_MLP;
  constexpr bool NORM = OP != OP_MATMUL;
  constexpr int NS = MLP ? 2 : 1;  // weight streams
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = static_cast<int>(L.M);
  const int64_t K = L.K;
  const int64_t Kp = L.kb * L.block_size;  // padded K, a multiple of 32
  const int64_t ldA = Kp + 8;               // halfs per staged row
  const int64_t groups = Kp / 8;            // 8-element groups per staged row
  const int kb = static_cast<int>(L.kb);
  const GemvLds lay = gemv_lds(L, TILES);
  const f16* A = static_cast<const f16*>(L.A);
  const f16* SK = static_cast<const f16*>(L.skip);
  const f16* GM = static_cast<const f16*>(L.gamma);
  f16* As = reinterpret_cast<f16*>(smem);
  const f16* Azero = reinterpret_cast<const f16*>(smem + lay.zero_off);
  float* red = reinterpret_cast<float*>(smem);

  // workgroup -> projection and first tile
  int64_t wg = blockIdx.x;
  int pi = 0;
  if constexpr (OP == OP_QKV) {
    const int64_t w0 = ((L.p[0].N + 15) / 16 + TILES - 1) / TILES;
    const int64_t w1 = ((L.p[1].N + 15) / 16 + TILES - 1) / TILES;
    if (wg >= w0) {
      wg -= w0;
      pi = 1;
      if (wg >= w1) {
        wg -= w1;
        pi = 2;
      }
    }
  }
  const Proj& P = L.p[pi];
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform copy for scalar offsets
  const int tl = wv % TILES, ks = wv / TILES;
  const int c = lane & 15, g = lane >> 4;
  const uint32_t n0 = static_cast<uint32_t>(wg * TILES * 16);
  const int64_t n = n0 + tl * 16 + c;
  const bool nval = n < P.N;
  const uint32_t nrows = static_cast<uint32_t>(P.N - n0 < 16 * TILES ? P.N - n0 : 16 * TILES);
  const uint32_t rowb = static_cast<uint32_t>(L.kb * L.blob);
  const int nchunk = static_cast<int>(rowb >> 4);
  const int steps = (nchunk + 7) >> 3;
  const int nsw = steps > ks ? (steps - ks + KS - 1) / KS : 0;  // steps of this wave
  const int sh = L.bs_log2 - 5;
  const uint32_t zrow = static_cast<uint32_t>(L.zrow);
  const uint32_t zesz = L.zp_dtype == DT_F32 ? 4u : 2u;

  // weight streams: buffer resources bounded by each tensor, lane offsets
  rsrc_t rB[NS];
#pragma unroll
  for (int q = 0; q < NS; ++q) rB[q] = mk_rsrc(L.p[pi + q].B, static_cast<uint32_t>(L.p[pi + q].N) * rowb);
  const uint32_t vB = static_cast<uint32_t>(n) * rowb + g * 16;
  // block of the chunk starting at code 32 * (cu + g): bu + bl (see block_u)
  const uint32_t bl = SPC == 1 ? (g >> sh) : 2u * g;
  auto block_u = [&](uint32_t cu, int half) -> uint32_t { return SPC == 1 ? (cu >> sh) : 2u * cu + half; };
  auto cu_of = [&](int i, int h) { return static_cast<uint32_t>((ks + i * KS) * 8 + h * 4); };

  // ---- activation staging, phase 1: issue the register-resident loads
  // (MatMul stages flat; Qkv/Mlp stage one row per wave so the row statistic
  // is a wave reduction). Index arithmetic is 32-bit: the host routes
  // geometries beyond 2^30 elements to the generic kernel.
  const int Ki = static_cast<int>(K), Kpi = static_cast<int>(Kp), gi = static_cast<int>(groups);
  const int total = M * gi;
  constexpr int SA = NORM ? GEMV_SA_ROWS : GEMV_SA_FLAT;
  f16x8 sa[SA], ss[NORM ? SA : 1], sg[NORM ? SA : 1];
  if constexpr (STAGE == ST_FLAT) {
#pragma unroll
    for (int i = 0; i < SA; ++i) {
      const uint32_t idx = static_cast<uint32_t>(i * GEMV_NT + tid);
      const uint32_t m = idx / static_cast<uint32_t>(gi);
      const uint32_t k = (idx - m * gi) * 8;
      const bool ok = idx < static_cast<uint32_t>(total) && k < static_cast<uint32_t>(Ki);
      sa[i] = __builtin_bit_cast(f16x8, ld16(A + (ok ? m * Ki + k : 0u)));
    }
  } else if constexpr (STAGE == ST_ROWS) {
    // wave w stages row w; lane holds groups lane + 64 i of that row
#pragma unroll
    for (int i = 0; i < SA; ++i) {
      const int k = (i * 64 + lane) * 8;
      const bool ok = wave < M && k < Ki;
      const int off = ok ? wave * Ki + k : 0;
      sa[i] = __builtin_bit_cast(f16x8, ld16(A + off));
      ss[i] = __builtin_bit_cast(f16x8, ld16((SK ? SK : A) + off));
      sg[i] = __builtin_bit_cast(f16x8, ld16((GM ? GM : A) + (ok ? k : 0)));
    }
  }

  // ---- scale / zero-point tiles of this workgroup's columns (coalesced)
  // The range check of a buffer load zeroes a whole dword that straddles the
  // bound, so a tile bound is rounded up to 16 bytes. Tiles start 16-byte
  // aligned, so the rounded bound stays inside the aligned 16-byte block that
  // holds the tensor's last byte (never past its page); those extra elements
  // are never indexed.
  u32x4 ts[NS][GEMV_TILE_PIECES], tz[NS][GEMV_TILE_PIECES];
#pragma unroll
  for (int q = 0; q < NS; ++q) {
    const Proj& Q = L.p[pi + q];
    const rsrc_t rS = mk_rsrc(static_cast<const uint8_t*>(Q.scales) + static_cast<size_t>(n0) * kb * 2,
                              align16(nrows * kb * 2));
#pragma unroll
    for (int i = 0; i < GEMV_TILE_PIECES; ++i) ts[q][i] = bld16(rS, (i * GEMV_NT + tid) * 16, 0);
    if constexpr (ZPK != ZP_NONE) {
      const uint32_t zr = ZPK == ZP_PACKED ? zrow : kb * zesz;
      const rsrc_t rZ = mk_rsrc(static_cast<const uint8_t*>(Q.zp) + static_cast<size_t>(n0) * zr, align16(nrows * zr));
#pragma unroll
      for (int i = 0; i < GEMV_TILE_PIECES; ++i) tz[q][i] = bld16(rZ, (i * GEMV_NT + tid) * 16, 0);
    }
  }

  // ---- first batch of weights: the HBM stream starts here
  u32x4 wa[NS][2 * SB], wb[NS][2 * SB];
  auto load_batch = [&](u32x4(&w)[NS][2 * SB], int i0) {
#pragma unroll
    for (int j = 0; j < SB; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < NS; ++q) w[q][2 * j + h] = bld16(rB[q], vB, cu_of(i0 + j, h) * 16);
  };
  load_batch(wa, 0);

  // ---- tiles to LDS
#pragma unroll
  for (int q = 0; q < NS; ++q)
#pragma unroll
    for (int i = 0; i < GEMV_TILE_PIECES; ++i) {
      const uint32_t off = (i * GEMV_NT + tid) * 16;
      if (off < lay.s_bytes) *reinterpret_cast<u32x4*>(smem + lay.s_off[q] + off) = ts[q][i];
      if (ZPK != ZP_NONE && off < lay.z_bytes) *reinterpret_cast<u32x4*>(smem + lay.z_off[q] + off) = tz[q][i];
    }

  // ---- activation staging, phase 2: write LDS (pair order), normalising for Qkv/Mlp
  auto put = [&](int m, int k, f16x8 v) { *reinterpret_cast<f16x8*>(As + m * ldA + k) = pair_order(v); };
  if constexpr (STAGE == ST_FLAT) {
#pragma unroll
    for (int i = 0; i < SA; ++i) {
      const uint32_t idx = static_cast<uint32_t>(i * GEMV_NT + tid);
      if (idx < static_cast<uint32_t>(total)) {
        const uint32_t m = idx / static_cast<uint32_t>(gi);
        const uint32_t k = (idx - m * gi) * 8;
        put(m, k, k < static_cast<uint32_t>(Ki) ? sa[i] : f16x8{});
      }
    }
  } else if constexpr (STAGE == ST_ROWS) {
    if (wave < M) {
      // r = A + skip in float32 (packedInput, complex_kernel.glsl:81)
      auto rval = [&](int i, int e, bool ok) {
        const float a = ok ? static_cast<float>(sa[i][e]) : 0.f;
        return SK ? __fadd_rn(a, ok ? static_cast<float>(ss[i][e]) : 0.f) : a;
      };
      float sq = 0.f;
#pragma unroll
      for (int i = 0; i < SA; ++i) {
        const bool ok = (i * 64 + lane) * 8 < Ki;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float r = rval(i, e, ok);
          sq += r * r;
        }
      }
      const float inv = GM ? 1.f / sqrtf(wave_sum(sq) / static_cast<float>(K) + L.eps) : 1.f;
#pragma unroll
      for (int i = 0; i < SA; ++i) {
        const int k = (i * 64 + lane) * 8;
        if (k < Kpi) {
          const bool ok = k < Ki;
          f16x8 x = {}, rr;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float r = rval(i, e, ok);
            rr[e] = static_cast<f16>(r);
            if (ok) x[e] = static_cast<f16>(GM ? r * (inv * static_cast<float>(sg[i][e])) : r);
          }
          put(wave, k, x);
          if (L.residual && blockIdx.x == 0 && ok)
            *reinterpret_cast<f16x8*>(static_cast<f16*>(L.residual) + wave * Ki + k) = rr;
        }
      }
    }
  } else {
    static_assert(STAGE == ST_MULTI, "staging mode");
    // streamed passes (loads queue behind the weight batch)
    if (NORM && GM) {
      for (int m = wave; m < M; m += GEMV_WAVES) {
        float sq = 0.f;
        for (int64_t j = lane; j < K / 8; j += 64) {
          const f16x8 a = __builtin_bit_cast(f16x8, ld16(A + m * K + j * 8));
          const f16x8 sk = SK ? __builtin_bit_cast(f16x8, ld16(SK + m * K + j * 8)) : f16x8{};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float rv = __fadd_rn(static_cast<float>(a[e]), static_cast<float>(sk[e]));
            sq += rv * rv;
          }
        }
        sq = wave_sum(sq);
        if (lane == 0) s_inv[m] = 1.f / sqrtf(sq / static_cast<float>(K) + L.eps);
      }
      __syncthreads();
    }
    for (int64_t idx = tid; idx < total; idx += GEMV_NT) {
      const int m = static_cast<int>(idx / groups);
      const int64_t k = (idx - static_cast<int64_t>(m) * groups) * 8;
      f16x8 v = {};
      if (k < K) {
        v = __builtin_bit_cast(f16x8, ld16(A + m * K + k));
        if constexpr (NORM) {
          const f16x8 sk = SK ? __builtin_bit_cast(f16x8, ld16(SK + m * K + k)) : f16x8{};
          float rv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) rv[e] = __fadd_rn(static_cast<float>(v[e]), static_cast<float>(sk[e]));
          if (L.residual && blockIdx.x == 0) {
            f16x8 rr;
#pragma unroll
            for (int e = 0; e < 8; ++e) rr[e] = static_cast<f16>(rv[e]);
            *reinterpret_cast<f16x8*>(static_cast<f16*>(L.residual) + m * K + k) = rr;
          }
          if (GM) {
            const f16x8 gm = __builtin_bit_cast(f16x8, ld16(GM + k));
            const float inv = s_inv[m];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = static_cast<f16>(rv[e] * (inv * static_cast<float>(gm[e])));
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = static_cast<f16>(rv[e]);
          }
        }
      }
      put(m, static_cast<int>(k), v);
    }
  }
  if (tid < 4) *reinterpret_cast<u32x4*>(smem + lay.zero_off + tid * 16) = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();

  // ---- main loop: dequantise each chunk and multiply on MFMA
  // Lanes whose activation row does not exist (c >= M) or whose chunk is past
  // the row read the zero block instead of masking the read.
  const bool aval = c < M;
  const f16* Arow = As + c * ldA + g * 32;
  const uint32_t trow = tl * 16 + c;  // this lane's row in the tiles
  // inrow = false: the chunk is past the row; it multiplies zero activations
  // and takes block 0's metadata so that every LDS index stays in its tile.
  auto dq_chunk_lds = [&](int q, const u32x4& w, uint32_t cu, bool inrow, f16x8 out[4]) {
    const uint16_t* St = reinterpret_cast<const uint16_t*>(smem + lay.s_off[q]) + trow * kb;
#pragma unroll
    for (int half = 0; half < SPC; ++half) {
      const uint32_t b = inrow ? block_u(cu, half) + bl : 0u;
      const f16 s = __builtin_bit_cast(f16, St[b]);
      float z = 8.f;
      if constexpr (ZPK == ZP_PACKED) {
        const uint8_t zb = (smem + lay.z_off[q])[trow * zrow + (b >> 1)];
        z = static_cast<float>((zb >> ((b & 1) * 4)) & 15u);
      } else if constexpr (ZPK == ZP_FLOAT) {
        const unsigned char* Zt = smem + lay.z_off[q] + trow * kb * zesz;
        z = zesz == 4 ? reinterpret_cast<const float*>(Zt)[b]
                      : static_cast<float>(reinterpret_cast<const f16*>(Zt)[b]);
      }
      if constexpr (ZPK == ZP_FLOAT) {
        const float sf = static_cast<float>(s);
#pragma unroll
        for (int d = half * (4 / SPC); d < (half + 1) * (4 / SPC); ++d) out[d] = dq8_f32z(w[d], z, sf);
      } else {
        const Dq cst = dq_consts(z, s);
#pragma unroll
        for (int d = half * (4 / SPC); d < (half + 1) * (4 / SPC); ++d) out[d] = dq8(w[d], cst);
      }
    }
  };
  f32x4 acc[NS];
#pragma unroll
  for (int q = 0; q < NS; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](u32x4(&w)[NS][2 * SB], int i0) {
#pragma unroll
    for (int j = 0; j < SB; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t cu = cu_of(i0 + j, h);
        // lane c is activation row c for the A operand (independent of whether
        // column n0 + c exists, which only concerns its B operand)
        const bool cval = aval && (i0 + j) < nsw && static_cast<int>(cu) + g < nchunk;
        const f16* ap = cval ? Arow + cu * 32 : Azero;
        f16x8 a[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) a[d] = *reinterpret_cast<const f16x8*>(ap + d * 8);
#pragma unroll
        for (int q = 0; q < NS; ++q) {
          f16x8 b[4];
          dq_chunk_lds(q, w[q][2 * j + h], cu, static_cast<int>(cu) + g < nchunk, b);
#pragma unroll
          for (int d = 0; d < 4; ++d) acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[d], b[d], acc[q], 0, 0, 0);
        }
      }
  };
  if constexpr (DB) {
    for (int i0 = 0; i0 < nsw; i0 += 2 * SB) {
      if (i0 + SB < nsw) load_batch(wb, i0 + SB);
      compute(wa, i0);
      if (i0 + SB >= nsw) break;
      if (i0 + 2 * SB < nsw) load_batch(wa, i0 + 2 * SB);
      compute(wb, i0 + SB);
    }
  } else {
    for (int i0 = 0; i0 < nsw; i0 += SB) {
      if (i0 > 0) load_batch(wa, i0);
      compute(wa, i0);
    }
  }

  // ---- combine the K-split partial sums of a tile through LDS
  constexpr int NACC = 4 * NS;
  if constexpr (KS > 1) {
    __syncthreads();  // every wave is done reading the staged activations
    if (ks > 0) {
      float* dst = red + (((ks - 1) * TILES + tl) * 64 + lane) * NACC;
#pragma unroll
      for (int q = 0; q < NS; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[4 * q + r] = acc[q][r];
    }
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int w = 1; w < KS; ++w) {
      const float* src = red + (((w - 1) * TILES + tl) * 64 + lane) * NACC;
#pragma unroll
      for (int q = 0; q < NS; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[q][r] += src[4 * q + r];
    }
  }
  if (!nval) return;

  // ---- epilogue: lane (c, g) holds rows 4g..4g+3 of column n
  float bias = 0.f, ubias = 0.f;
  if constexpr (OP != OP_QKV) {
    if (P.bias) bias = static_cast<float>(static_cast<const f16*>(P.bias)[n]);
  }
  if constexpr (MLP) {
    if (L.p[1].bias) ubias = static_cast<float>(static_cast<const f16*>(L.p[1].bias)[n]);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * g + r;
    if (m < M) {
      float y = acc[0][r] + bias;
      if constexpr (MLP) y = activate(y, L.act) * (acc[NS - 1][r] + ubias);
      static_cast<f16*>(P.Y)[static_cast<int64_t>(m) * P.N + n] = static_cast<f16>(y);
    }
  }
}

// ---------------------------------------------------------------------------
// host-side selection and launch

inline int spc_of(int block_size) { return block_size >= 32 ? 1 : 2; }

inline constexpr int64_t kMaxLds = 160 * 1024 - 1024;

// 32-bit in-kernel index arithmetic of the fast kernels
inline bool fits_i32(const Launch& L) {
  const int64_t lim = int64_t(1) << 30;
  if (L.M * L.K >= lim || L.kb * L.block_size >= lim) return false;
  for (int i = 0; i < L.nproj; ++i) {
    // buffer-resource byte ranges are 32-bit
    if (L.p[i].N * L.kb * L.blob >= lim || L.p[i].N * L.kb * 4 >= lim || L.M * L.p[i].N >= lim) return false;
  }
  return true;
}

inline bool gemv_fits(const Launch& L, int tiles) {
  const GemvLds y = gemv_lds(L, tiles);
  const uint32_t tile_cap = GEMV_TILE_PIECES * GEMV_NT * 16;
  return y.total <= kMaxLds && y.s_bytes <= tile_cap && y.z_bytes <= tile_cap;
}

// Column tiles per GEMV workgroup: one tile split over all waves when the
// staged activations are small; for larger M the staging is shared by as many
// tiles (4, else 2) as the LDS holds. 0 if no layout fits.
inline int gemv_tiles(const Launch& L) {
  if (L.M >= 8) {
    if (gemv_fits(L, 4)) return 4;
    if (gemv_fits(L, 2)) return 2;
  }
  return gemv_fits(L, 1) ? 1 : 0;
}

inline int gemv_stage(const Launch& L) {
  const int64_t groups = L.kb * L.block_size / 8;
  if (L.op == OP_MATMUL) return L.M * groups <= static_cast<int64_t>(GEMV_SA_FLAT) * GEMV_NT ? ST_FLAT : ST_MULTI;
  return (L.M <= GEMV_WAVES && groups <= static_cast<int64_t>(GEMV_SA_ROWS) * 64) ? ST_ROWS : ST_MULTI;
}

// steps of 128 bytes per column handled by one wave
inline int64_t gemv_wave_steps(const Launch& L, int tiles) {
  const int64_t steps = (L.kb * L.blob / 16 + 7) / 8;
  const int ks = GEMV_WAVES / tiles;
  return (steps + ks - 1) / ks;
}

template <int ZPK, int SPC, int OP, int TILES, bool DB, int STAGE>
inline hipError_t launch_gemv6(const Launch& L, hipStream_t st) {
  auto wgs = [](int64_t n) { return ((n + 15) / 16 + TILES - 1) / TILES; };
  const int64_t grid = wgs(L.p[0].N) + (OP == OP_QKV ? wgs(L.p[1].N) + wgs(L.p[2].N) : 0);
  const int64_t lds = gemv_lds(L, TILES).total;
  auto kern = k_gemv_q4<ZPK, SPC, OP, TILES, DB, STAGE>;
  if (lds > 64 * 1024) {
    // Raises the dynamic-LDS cap where the runtime keeps one; an error here
    // surfaces from the launch itself if the size is really unsupported.
    static std::atomic<int> done[kMaxDevices];  // per instantiation and device
    (void)raise_lds_cap(reinterpret_cast<const void*>(kern), static_cast<int>(kMaxLds), done);
    (void)hipGetLastError();
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(grid)), dim3(GEMV_NT), static_cast<size_t>(lds), st, L);
  return hipGetLastError();
}

template <int ZPK, int SPC, int OP, int TILES, bool DB>
inline hipError_t launch_gemv5(const Launch& L, hipStream_t st) {
  constexpr int REG = OP == OP_MATMUL ? ST_FLAT : ST_ROWS;
  return gemv_stage(L) == ST_MULTI ? launch_gemv6<ZPK, SPC, OP, TILES, DB, ST_MULTI>(L, st)
                                   : launch_gemv6<ZPK, SPC, OP, TILES, DB, REG>(L, st);
}

template <int ZPK, int SPC, int OP, int TILES>
inline hipError_t launch_gemv4(const Launch& L, hipStream_t st) {
  return gemv_wave_steps(L, TILES) > GEMV_SB ? launch_gemv5<ZPK, SPC, OP, TILES, true>(L, st)
                                             : launch_gemv5<ZPK, SPC, OP, TILES, false>(L, st);
}

template <int ZPK, int SPC, int OP>
inline hipError_t launch_gemv3(const Launch& L, hipStream_t st) {
  switch (gemv_tiles(L)) {
    case 4: return launch_gemv4<ZPK, SPC, OP, 4>(L, st);
    case 2: return launch_gemv4<ZPK, SPC, OP, 2>(L, st);
    default: return launch_gemv4<ZPK, SPC, OP, 1>(L, st);
  }
}

template <int ZPK, int SPC>
inline hipError_t launch_gemv2(const Launch& L, hipStream_t st) {
  switch (L.op) {
    case OP_QKV: return launch_gemv3<ZPK, SPC, OP_QKV>(L, st);
    case OP_MLP: return launch_gemv3<ZPK, SPC, OP_MLP>(L, st);
    default: return launch_gemv3<ZPK, SPC, OP_MATMUL>(L, st);
  }
}

template <int ZPK>
inline hipError_t launch_gemv1(const Launch& L, hipStream_t st) {
  return spc_of(L.block_size) == 1 ? launch_gemv2<ZPK, 1>(L, st) : launch_gemv2<ZPK, 2>(L, st);
}

// Entry of one zero-point kind (defined in xrmm_gemv_zp.hip).
template <int ZPK>
hipError_t launch_gemv_for(const Launch& L, hipStream_t st);

}  // namespace xrmm
