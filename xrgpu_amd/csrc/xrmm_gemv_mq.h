// MFMA GEMV for up to four rows (fp16 activations, 4-bit weights, integer
// zero points): the Qkv decode shape (four rows, RMS prologue) and
// MatMulNBits with three or four rows.
//
// Work split. A workgroup owns one or two tiles of 16 output columns (TT);
// its W waves split K: wave w takes chunks [w*4J, (w+1)*4J) of every column
// (a chunk is 16 bytes = 32 codes of one column), and one staging of its K
// slice of the activations serves every tile. Lane l = 16 g + n loads chunk w*4J + 4j + g
// of column n for j = 0..J-1, so one load instruction reads 64 contiguous
// bytes of each of 16 columns. Every weight load of a wave is issued before
// its activation staging, so the whole stream is in flight from the start.
//
// Arithmetic. A dword x of a chunk holds codes c0..c7 (low nibble first,
// complex_kernel.glsl:80). OR-ing masked nibbles into the mantissa of 1024.0h
// gives exact binary16 pairs (1024 + c0, 1024 + c4), (1024 + 16 c1,
// 1024 + 16 c5) and the same on x >> 8; one packed add (low nibbles) or packed
// fma with 1/16 (high nibbles) turns each pair into (c - z) exactly, so the
// weights enter the matrix core as exact integers and the block scale is
// applied in float32 afterwards (no binary16 rounding of (c - z) * scale).
//
// v_mfma_f32_16x16x32_f16 multiplies A (16 rows x 32 k) by B (32 k x 16
// columns); lane l supplies A[l % 16][8 (l / 16) + i] and B[8 (l / 16) + i]
// [l % 16], i = 0..7, and receives D[4 (l / 16) + i][l % 16], i = 0..3. The
// activations enter block-diagonally: A row 4 g + r holds activation row r
// on k-group g and zeros elsewhere. D row 4 g + r then sums only k-group g,
// which is exactly the chunk lane (n, g) loaded: after the four MFMAs of a
// chunk (its four dwords), lane (n, g) holds the chunk's sums for rows 0..3
// of column n and scales them by its own block scale. Only the 16 lanes with
// n / 4 == g read activations (from the wave's LDS slice); the others read a
// zero word.
//
// Activations. Each wave stages only its own K slice of the (up to four)
// activation rows in LDS, in the pair order of the weight dwords
// (a0, a4, a1, a5, a2, a6, a3, a7). For Qkv the per-row RMS factor comes out
// of the sum: a wave stages u = (A + skip) * gamma and its partial sum(r^2),
// and the factor multiplies the row totals at the end. The workgroup's one
// barrier before the MFMAs publishes the tile's scales / zero points.
//
// End. Every lane's partial sums (its column, its k-group, four rows) meet in
// LDS after one barrier, and 16 x M threads add the 4 W of them, add the bias
// (or apply the RMS factor) and store.
#pragma once
#include "xrmm_gemv_dot.h"

namespace xrmm {

// Largest value over the wave (NaN lanes are ignored).
__device__ __forceinline__ float mq_wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Sum over each row of 16 lanes; every lane of the row receives it.
__device__ __forceinline__ float mq_row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));  // row_half_mirror
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));  // row_mirror
  return v;
}

// 16-byte loads per thread that stage a tile's scales (16 rows of kb fp16
// values) with eight waves: one covers kb <= 256.
constexpr int MQ_META_LOADS = 1;

struct MqProj {
  const uint8_t* B;
  const void* S;
  const uint8_t* Z;
  void* Y;
  uint32_t N;
  uint32_t t0;  // first tile of this projection on the grid
};

struct MqArgs {
  const void* A;
  const void* bias;   // MatMulNBits only
  const void* skip;   // Qkv: nullable
  const void* gamma;  // Qkv: RMS scale [K]
  void* residual;     // Qkv: nullable, receives A + skip
  float eps;
  MqProj p[3];
  uint32_t K, kb, rowb, zrow, M, bsl, nchunk;
  // log2 of a column's scale row (kb * 2 bytes) and packed zero-point row
  // (zrow bytes) when they are powers of two of at least 16 bytes: the tile's
  // rows are then staged with 16 bytes of padding each, so the 16 columns'
  // per-lane reads fall on different banks. 0: staged unpadded.
  uint32_t sshift, zshift;
};

// Padded LDS offset of byte o of the tile's contiguous rows (row bytes 2^sh).
__device__ __forceinline__ uint32_t mq_pad(uint32_t o, uint32_t sh) {
  return sh ? o + ((o >> sh) << 4) : o;
}

// LDS row stride of a wave's activation slice: 4J chunks x 32 halves plus 16
// bytes, so the 16 diagonal lanes' 16-byte reads (rows r, k-groups g: offsets
// r * stride + 64 g) fall on distinct banks.
template <int J>
__host__ __device__ constexpr uint32_t mq_row_stride() {
  return 4 * J * 32 * 2 + 16;
}

// LDS bytes of one wave's slice: four rows, then one zero 16-byte word read by
// the lanes off the block diagonal.
template <int J>
__host__ __device__ constexpr uint32_t mq_slice_bytes() {
  return 4 * mq_row_stride<J>() + 16;
}

template <int ZPK, int J, int W, int OPK, bool SK, int TT>
__global__ __launch_bounds__(W * 64) void k_gemv_mq(MqArgs a) {
  static_assert(TT == 1 || TT == 2, "one or two 16-column tiles per workgroup");
  static_assert(ZPK == ZP_NONE || ZPK == ZP_PACKED, "integer zero points");
  static_assert(OPK == OP_MATMUL || OPK == OP_QKV, "operator");
  constexpr bool QKV = OPK == OP_QKV;
  constexpr uint32_t CPW = 4 * J;              // chunks per wave
  constexpr uint32_t SLICE = mq_slice_bytes<J>();
  constexpr uint32_t ROWB = mq_row_stride<J>();  // LDS row stride of the slice
  __shared__ __align__(16) unsigned char act[W][SLICE];
  // partial sums: [row i][column n][wave w, k-group g] with a padded column
  // stride, so the 16 columns' writes spread over the banks and an output
  // thread reads its 4 W values as 16-byte pieces
  constexpr int PST = ((4 * W + 3) / 4) * 4 + 4;
  __shared__ __align__(16) float part[TT][4][16][PST];
  __shared__ float red[QKV ? W : 1][4][4];  // per wave, row and 16-lane row of the wave
  __shared__ __align__(16) unsigned char meta_s[MQ_META_LOADS * W * 64 * 16 + 16 * 16 * TT];
  __shared__ __align__(16) unsigned char meta_z[ZPK == ZP_PACKED ? MQ_META_LOADS * W * 64 * 16 + 16 * 16 * TT : 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t n = lane & 15, g = lane >> 4;
  const uint32_t tile = xcd_slot(blockIdx.x, gridDim.x);
  uint32_t pi = 0;
  if constexpr (QKV) pi = (tile >= a.p[1].t0 ? 1u : 0u) + (tile >= a.p[2].t0 ? 1u : 0u);
  auto pick = [&](auto v0, auto v1, auto v2) { return QKV ? (pi == 0 ? v0 : pi == 1 ? v1 : v2) : v0; };
  const uint8_t* Bp = pick(a.p[0].B, a.p[1].B, a.p[2].B);
  const void* Sp = pick(a.p[0].S, a.p[1].S, a.p[2].S);
  const uint8_t* Zp = pick(a.p[0].Z, a.p[1].Z, a.p[2].Z);
  void* Yp = pick(a.p[0].Y, a.p[1].Y, a.p[2].Y);
  const uint32_t N = pick(a.p[0].N, a.p[1].N, a.p[2].N);
  const uint32_t t0 = pick(a.p[0].t0, a.p[1].t0, a.p[2].t0);
  const uint32_t K = a.K, rowb = a.rowb, nchunk = a.nchunk;
  const int M = static_cast<int>(a.M);
  const uint32_t col0 = (tile - t0) * 16u * TT;
  const uint32_t ch0 = wave * CPW;              // first chunk of this wave

  // ---- this wave's activation slice first (the staging waits for it, and
  // the vector-memory counter retires in issue order): 16-byte piece
  // q*64 + lane is row r = idx / (16 J), group pc = idx % (16 J)
  // (k = slice start + 8 pc)
  const rsrc_t rA = mk_rsrc(a.A, static_cast<uint32_t>(M) * K * 2u);
  const rsrc_t rK = mk_rsrc(a.skip, SK ? static_cast<uint32_t>(M) * K * 2u : 0u);
  const rsrc_t rG = mk_rsrc(a.gamma, QKV ? K * 2u : 0u);
  const uint32_t k0 = ch0 * 32u;
  // gamma depends on the piece's k only, the same for every row: one load
  u32x4 ar[J], sk[SK ? J : 1], gm[1];
#pragma unroll
  for (int q = 0; q < J; ++q) {
    const uint32_t idx = q * 64u + lane, r = idx / (16u * J), pc = idx % (16u * J);
    const uint32_t k = k0 + 8u * pc;
    const bool ok = static_cast<int>(r) < M && k < K;  // K % 8 == 0 on this path
    const uint32_t off = ok ? (r * K + k) * 2u : kOOB;
    ar[q] = bld16(rA, off, 0);
    if constexpr (SK) sk[q] = bld16(rK, off, 0);
    if constexpr (QKV) {
      if (q == 0) gm[0] = bld16(rG, k < K ? k * 2u : kOOB, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- the tile's scales (and packed zero points): 16 consecutive rows of
  // [N, kb], i.e. 32 kb contiguous bytes (16 zrow for zero points), loaded
  // with 16-byte pieces by the workgroup and staged in LDS. Zero-point loads
  // start at the dword boundary at or below the tile's bytes: the range check
  // zeroes a whole dword that straddles the bound. (Scale blocks start
  // dword-aligned: 16 columns of whole fp16 rows.)
  const uint32_t ncols = N - col0 < 16u * TT ? N - col0 : 16u * TT;
  const uint32_t sb0 = col0 * a.kb * 2u, sbytes = ncols * a.kb * 2u;
  const uint32_t zb0 = col0 * a.zrow, zbytes = ZPK == ZP_PACKED ? ncols * a.zrow : 0u;
  const uint32_t zdel = zb0 & 3u;
  const rsrc_t rS = mk_rsrc(Sp, (N * a.kb * 2u + 15u) & ~15u);
  const rsrc_t rZ = mk_rsrc(Zp, ZPK == ZP_PACKED ? (N * a.zrow + 15u) & ~15u : 0u);
  u32x4 sv[MQ_META_LOADS], zv[ZPK == ZP_PACKED ? MQ_META_LOADS : 1];
#pragma unroll
  for (int q = 0; q < MQ_META_LOADS; ++q) {
    const uint32_t o = (q * W * 64u + static_cast<uint32_t>(tid)) * 16u;
    sv[q] = bld16_nt(rS, o < sbytes ? sb0 + o : kOOB, 0);
    if constexpr (ZPK == ZP_PACKED) zv[q] = bld16_nt(rZ, o < zbytes + zdel ? zb0 - zdel + o : kOOB, 0);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- the weights: J chunks per lane, all in flight before the staging
  // (the column offset differs per lane, so it goes into the vector offset:
  // a per-lane scalar offset would serialise the load over the columns)
  const rsrc_t rB = mk_rsrc(Bp, N * rowb);
  u32x4 wv[TT][J];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const uint32_t col = col0 + 16u * tt + n;
    const uint32_t colc = col < N ? col : N - 1;  // loads clamp, stores check
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t ch = ch0 + 4u * j + g;
      wv[tt][j] = bld16_nt(rB, ch < nchunk ? colc * rowb + ch * 16u : kOOB, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- stage the slice: pair order, binary16
  unsigned char* slice = act[wave];
  auto pair_store = [&](uint32_t r, uint32_t pc, const f16x8& x) {
    const u32x4 v = __builtin_bit_cast(u32x4, x);
    const u32x4 p = {__builtin_amdgcn_perm(v[2], v[0], 0x05040100u), __builtin_amdgcn_perm(v[2], v[0], 0x07060302u),
                     __builtin_amdgcn_perm(v[3], v[1], 0x05040100u), __builtin_amdgcn_perm(v[3], v[1], 0x07060302u)};
    *reinterpret_cast<u32x4*>(slice + r * ROWB + pc * 16u) = p;
  };
  if (lane == 0) *reinterpret_cast<u32x4*>(slice + 4 * ROWB) = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int q = 0; q < MQ_META_LOADS; ++q) {
    const uint32_t o = (q * W * 64u + static_cast<uint32_t>(tid)) * 16u;
    if (o < sbytes) *reinterpret_cast<u32x4*>(meta_s + mq_pad(o, a.sshift)) = sv[q];
    if (ZPK == ZP_PACKED && o < zbytes + zdel)
      *reinterpret_cast<u32x4*>(meta_z + mq_pad(o, a.zshift)) = zv[ZPK == ZP_PACKED ? q : 0];
  }
  // Qkv: the RMS factor of a row is common to all its k, so it comes out of
  // the sum: y_r = inv_r * sum_k (r_k gamma_k) W_k with r = A + skip and
  // inv_r = 1 / sqrt(sum_k r_k^2 / K + eps) (packedInput,
  // complex_kernel.glsl:81). Each wave stages u = r * gamma of its own slice
  // (rounded once to binary16) and its partial sum(r^2); the factor is applied
  // to the four row totals at the end, so no barrier waits for the sums here.
  // A wave whose |u| would leave the binary16 range stages u * 2^-e instead
  // and scales its partial totals back by 2^e (exact).
  float escale = 1.f;
  if constexpr (QKV) {
    float sq[4] = {0.f, 0.f, 0.f, 0.f};
    float mx = 0.f;
    f16* res = static_cast<f16*>(a.residual);
    const bool write_res = res != nullptr && tile == 0;
    // without skip r = A, and u = A * gamma is one packed binary16 multiply
    // per pair (the product of two binary16 values rounded once, as the
    // float32 product rounded to binary16 would be); the sum of squares takes
    // v_dot2_f32_f16 (exact products, float32 sums) and the range check works
    // on the binary16 bit patterns (|u| > 32768 exactly when the magnitude
    // bits exceed 0x7800)
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 big = {0, 0};
#pragma unroll
    for (int q = 0; q < J; ++q) {
      const uint32_t idx = q * 64u + lane, r = idx / (16u * J), pc = idx % (16u * J);
      const f16x8 av = __builtin_bit_cast(f16x8, ar[q]);
      const f16x8 sv = __builtin_bit_cast(f16x8, sk[SK ? q : 0]);
      const f16x8 gv = __builtin_bit_cast(f16x8, gm[0]);
      f16x8 u, rv;
      float s2 = 0.f;
      if constexpr (SK) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float rf = __fadd_rn(static_cast<float>(av[e]), static_cast<float>(sv[e]));
          const float uf = rf * static_cast<float>(gv[e]);
          s2 = __builtin_fmaf(rf, rf, s2);
          mx = __builtin_fmaxf(mx, __builtin_fabsf(uf));
          u[e] = static_cast<f16>(uf);
          rv[e] = static_cast<f16>(rf);
        }
      } else {
        float s2b = 0.f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const f16x2 a2 = h2(ar[q][d]), g2 = h2(gm[0][d]);
          const f16x2 u2 = a2 * g2;
          u[2 * d] = u2[0];
          u[2 * d + 1] = u2[1];
          if (d & 1) s2b = __builtin_amdgcn_fdot2(a2, a2, s2b, false);
          else s2 = __builtin_amdgcn_fdot2(a2, a2, s2, false);
          big = __builtin_elementwise_max(big, __builtin_bit_cast(u16x2, as_u32(u2) & 0x7FFF7FFFu));
        }
        s2 += s2b;
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) sq[rr] += r == static_cast<uint32_t>(rr) ? s2 : 0.f;
      pair_store(r, pc, u);
      const uint32_t k = k0 + 8u * pc;
      if (SK && write_res && static_cast<int>(r) < M && k < K) *reinterpret_cast<f16x8*>(res + r * K + k) = rv;
      if (!SK && write_res && static_cast<int>(r) < M && k < K) *reinterpret_cast<u32x4*>(res + r * K + k) = ar[q];
    }
    // the rows' partial sums of squares, one per 16-lane row of the wave (the
    // end adds them up with the waves')
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const float t = mq_row16_sum(sq[rr]);
      if ((lane & 15) == 0) red[wave][rr][lane >> 4] = t;
    }
    // Rescale only when some |u| exceeds 32768 (a ballot; the wave-wide
    // maximum is taken only then). NaN compares false: a NaN row stays NaN
    // through the unscaled path.
    if (!SK) mx = (big[0] > 0x7800 || big[1] > 0x7800) ? 65536.f : 0.f;  // only the comparison below uses it
    if (__builtin_amdgcn_ballot_w64(mx > 32768.f) != 0) {
      const float wmx = mq_wave_max(mx);
      int e = 0;
      (void)__builtin_frexpf(wmx / 32768.f, &e);
      escale = __builtin_ldexpf(1.f, e);
      const float down = __builtin_ldexpf(1.f, -e);
#pragma unroll
      for (int q = 0; q < J; ++q) {
        const uint32_t idx = q * 64u + lane, r = idx / (16u * J), pc = idx % (16u * J);
        const f16x8 av = __builtin_bit_cast(f16x8, ar[q]);
        const f16x8 sv = __builtin_bit_cast(f16x8, sk[SK ? q : 0]);
        const f16x8 gv = __builtin_bit_cast(f16x8, gm[0]);
        f16x8 u;
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) {
          const float rf = SK ? __fadd_rn(static_cast<float>(av[e2]), static_cast<float>(sv[e2])) : static_cast<float>(av[e2]);
          u[e2] = static_cast<f16>(rf * static_cast<float>(gv[e2]) * down);
        }
        pair_store(r, pc, u);
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < J; ++q) {
      const uint32_t idx = q * 64u + lane, r = idx / (16u * J), pc = idx % (16u * J);
      pair_store(r, pc, __builtin_bit_cast(f16x8, ar[q]));
    }
  }
  __syncthreads();  // the tile's scales / zero points
  // the slice is read back by other lanes of this wave only: LDS operations of
  // one wave complete in order, so no barrier, only no compiler reordering
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- MFMA over the lane's chunks: the slice's activation operands first
  // (one wait), then four MFMAs per chunk
  const bool diag = (n >> 2) == g;
  const uint32_t r_of = n & 3u;
  const unsigned char* zero = slice + 4 * ROWB;
  u32x4 aop[J][4];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int t = 0; t < 4; ++t)
      aop[j][t] = *reinterpret_cast<const u32x4*>(diag ? slice + r_of * ROWB + (4u * j + g) * 64u + 16u * t : zero);
  uint32_t sraw[TT][J], zraw[TT][J];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t ch = ch0 + 4u * j + g;
      const uint32_t b = ((ch < nchunk ? ch : nchunk - 1u) * 32u) >> a.bsl;
      const uint32_t nn = col0 + 16u * tt + n < N ? 16u * tt + n : 0u;
      sraw[tt][j] = *reinterpret_cast<const uint16_t*>(meta_s + mq_pad((nn * a.kb + b) * 2u, a.sshift));
      zraw[tt][j] = ZPK == ZP_PACKED ? meta_z[mq_pad(zdel + nn * a.zrow + (b >> 1), a.zshift)] >> ((b & 1u) * 4u) : 8u;
    }
  const f16x2 k1024 = {static_cast<f16>(1024.f), static_cast<f16>(1024.f)};
  const f16x2 k64 = {static_cast<f16>(64.f), static_cast<f16>(64.f)};
  const f16x2 inv16 = {static_cast<f16>(0.0625f), static_cast<f16>(0.0625f)};
  f32x4 yt[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
  f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const f16 zf = static_cast<f16>(static_cast<float>(zraw[tt][j] & 15u));
    const f16x2 zz = {zf, zf};
    const f16x2 nlo = -(k1024 + zz), nhi = -(k64 + zz);  // exact: small integers
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4 av = aop[j][t];
      const uint32_t x = wv[tt][j][t], x8 = x >> 8;
      const uint32_t magic = 0x64006400u;
      const f16x2 w0 = h2(and_or(x, 0x000F000Fu, magic)) + nlo;                                  // c0, c4
      const f16x2 w1 = __builtin_elementwise_fma(h2(and_or(x, 0x00F000F0u, magic)), inv16, nhi);  // c1, c5
      const f16x2 w2 = h2(and_or(x8, 0x000F000Fu, magic)) + nlo;                                 // c2, c6
      const f16x2 w3 = __builtin_elementwise_fma(h2(and_or(x8, 0x00F000F0u, magic)), inv16, nhi); // c3, c7
      const f16x8 b = {w0[0], w0[1], w1[0], w1[1], w2[0], w2[1], w3[0], w3[1]};
      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av), b, d, 0, 0, 0);
    }
    const float s = static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(sraw[tt][j])));
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = __builtin_fmaf(s, d[i], y[i]);
  }
  yt[tt] = y;
  }

  // ---- the four k-group lanes of a column, then the waves
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) part[tt][i][n][wave * 4 + g] = yt[tt][i] * escale;
  __syncthreads();
  if (tid < 64 * TT) {
    const uint32_t tt = static_cast<uint32_t>(tid) >> 6;
    const uint32_t i = (static_cast<uint32_t>(tid) >> 4) & 3u, nn = static_cast<uint32_t>(tid) & 15u;
    const uint32_t c = col0 + 16u * tt + nn;
    if (static_cast<int>(i) < M && c < N) {
      float t4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(&part[tt][i][nn][w * 4]);
#pragma unroll
        for (int q = 0; q < 4; ++q) t4[q] += v[q];
      }
      float t = (t4[0] + t4[1]) + (t4[2] + t4[3]);
      if constexpr (QKV) {
        float sq = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) sq += (red[w][i][0] + red[w][i][1]) + (red[w][i][2] + red[w][i][3]);
        t *= __builtin_amdgcn_rsqf(sq / static_cast<float>(K) + a.eps);
      } else {
        if (a.bias) t += static_cast<float>(static_cast<const f16*>(a.bias)[c]);
      }
      static_cast<f16*>(Yp)[i * N + c] = static_cast<f16>(t);
    }
  }
}

// Host side.
constexpr int kMqWaves = 8;

// Chunk rounds per wave (J) for a geometry: the W waves' 4J chunks must cover
// the row; 0 when the kernel does not apply.
inline int mq_j(const Launch& L) {
  const int64_t nchunk = L.kb * L.blob / 16;
  for (int j = 1; j <= 4; j *= 2)
    if (nchunk <= int64_t(kMqWaves) * 4 * j) return j;
  return 0;
}

// Whether the MFMA GEMV applies (beyond the shared fp16 4-bit conditions):
// up to four rows, whole 32-code blocks (block_size >= 32), integer zero
// points, a row of at most 8 x 16 chunks (K up to 4096 at 4 bits).
inline bool mq_fits(const Launch& L) {
  if (L.M < 1 || L.M > 4 || L.block_size < 32 || L.zp_kind == ZP_FLOAT) return false;
  if (16 * L.kb * 2 > int64_t(MQ_META_LOADS) * kMqWaves * 64 * 16) return false;  // a tile's scales in one pass
  if (L.op != OP_MATMUL && !(L.op == OP_QKV && L.gamma)) return false;
  return mq_j(L) != 0;
}

// Tiles per workgroup: two when the one-tile grid has more workgroups than
// the device has CUs and two tiles' scales still fit one staging pass. A
// workgroup stages its K slices of the activations once for all its tiles,
// so pairing halves that work and the activation reads per column, and a
// grid of at most one workgroup per CU leaves no CU with twice the work of
// another (the Qkv GQA decode geometry: 384 one-tile workgroups on 256 CUs,
// or 192 two-tile ones).
int device_cus();
inline int mq_tt(const Launch& L) {
  int64_t tiles = 0;
  for (int i = 0; i < L.nproj; ++i) tiles += (L.p[i].N + 15) / 16;
  const int cus = device_cus() > 0 ? device_cus() : 256;
  const bool fits2 = 32 * L.kb * 2 <= int64_t(MQ_META_LOADS) * kMqWaves * 64 * 16;
  return (tiles > cus && fits2) ? 2 : 1;
}

template <int ZPK, int J, int OPK, bool SK, int TT>
inline hipError_t launch_mq4(const Launch& L, hipStream_t st) {
  MqArgs a{};
  a.A = L.A;
  a.bias = L.p[0].bias;
  a.skip = L.skip;
  a.gamma = L.gamma;
  a.residual = L.residual;
  a.eps = L.eps;
  uint32_t tiles = 0;
  for (int i = 0; i < 3; ++i) {
    const bool used = i < L.nproj;
    const Proj& P = L.p[used ? i : 0];
    a.p[i] = MqProj{P.B, P.scales, static_cast<const uint8_t*>(P.zp), P.Y, static_cast<uint32_t>(P.N),
                    used ? tiles : 0xFFFFFFFFu};
    if (used) tiles += static_cast<uint32_t>((P.N + 16 * TT - 1) / (16 * TT));
  }
  a.K = static_cast<uint32_t>(L.K);
  a.kb = static_cast<uint32_t>(L.kb);
  a.rowb = static_cast<uint32_t>(L.kb * L.blob);
  a.zrow = static_cast<uint32_t>(L.zrow);
  a.M = static_cast<uint32_t>(L.M);
  a.bsl = static_cast<uint32_t>(L.bs_log2);
  a.nchunk = a.rowb / 16u;
  // padded staging when a row is a power of two of at least 16 bytes (so no
  // 16-byte piece straddles two rows) and, for zero points, every tile's
  // bytes start dword-aligned (zrow a multiple of 16 makes col0 * zrow one)
  auto pow2_shift = [](int64_t bytes) -> uint32_t {
    if (bytes < 16 || (bytes & (bytes - 1)) != 0) return 0u;
    uint32_t sh = 0;
    while ((int64_t(1) << sh) < bytes) ++sh;
    return sh;
  };
  a.sshift = pow2_shift(L.kb * 2);
  a.zshift = ZPK == ZP_PACKED ? pow2_shift(L.zrow) : 0u;
  hipLaunchKernelGGL((k_gemv_mq<ZPK, J, kMqWaves, OPK, SK, TT>), dim3(tiles), dim3(kMqWaves * 64), 0, st, a);
  return hipGetLastError();
}

template <int ZPK, int J, int OPK, int TT>
inline hipError_t launch_mq3t(const Launch& L, hipStream_t st) {
  if constexpr (OPK == OP_QKV)
    return L.skip ? launch_mq4<ZPK, J, OPK, true, TT>(L, st) : launch_mq4<ZPK, J, OPK, false, TT>(L, st);
  else
    return launch_mq4<ZPK, J, OPK, false, TT>(L, st);
}

template <int ZPK, int J, int OPK>
inline hipError_t launch_mq3(const Launch& L, hipStream_t st) {
  return mq_tt(L) == 2 ? launch_mq3t<ZPK, J, OPK, 2>(L, st) : launch_mq3t<ZPK, J, OPK, 1>(L, st);
}

template <int ZPK, int OPK>
inline hipError_t launch_mq2(const Launch& L, hipStream_t st) {
  switch (mq_j(L)) {
    case 1: return launch_mq3<ZPK, 1, OPK>(L, st);
    case 2: return launch_mq3<ZPK, 2, OPK>(L, st);
    default: return launch_mq3<ZPK, 4, OPK>(L, st);
  }
}

// Entry of one zero-point kind (defined in xrmm_gemv_mq_zp.hip).
template <int ZPK>
hipError_t launch_mq_for(const Launch& L, hipStream_t st);

}  // namespace xrmm
