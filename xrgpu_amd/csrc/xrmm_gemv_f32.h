// MatMulNBits GEMV in float32 arithmetic: float32 activations (the
// contract's T1 = float32), and float16 calls that no binary16-weight kernel
// takes (8-bit codes; weights whose dequantised value binary16 cannot hold).
// 4- or 8-bit weights, any number of rows in chunks of up to four (the grid's
// second dimension: each chunk reads the weights again, from the L2 / the
// Infinity Cache for all but the first). Float32 arithmetic throughout, as the
// reference's serial loop (complex_kernel.glsl:80,83): activations, scales and
// bias convert exactly to float32, codes convert exactly to float32 and
// multiply the activations with fused multiply-adds, so the float32 bar
// (1e-5 * max|Y|) holds with margin; float16 outputs are rounded once.
//
// Work split. A wave owns C consecutive output columns; its lanes split K:
// lane l takes the 16-byte chunks l, l + 64, ... of each column, so one load
// instruction reads 1 KB of contiguous codes. Every weight load of the wave is
// issued before the activation staging. The workgroup stages the activation
// rows once in LDS (float32, natural order) together with their sums per 16
// codes, and the wave's scale / zero-point block in its own LDS slice; one
// barrier, then no further synchronisation.
//
// Arithmetic. For a dword x of 4-bit codes c0..c7 (low nibble first),
// x & 0x0F0F0F0F holds c0, c2, c4, c6 in its bytes and (x >> 4) & 0x0F0F0F0F
// holds c1, c3, c5, c7; 8-bit codes are the dword's bytes.
// v_cvt_f32_ubyte{0..3} turns each byte into a float.
// sum_k (c_k - z) a_k = sum_k c_k a_k - z sum_k a_k per 16 codes, with the
// activation sums from the staging, then times the block scale.
#pragma once
#include "xrmm_gemv_dot.h"

namespace xrmm {

struct F32Args {
  const void* A;       // T [M, K]
  const uint8_t* B;
  const void* S;       // T [N, kb]
  const void* Z;       // packed u8 [N, zrow] or float [N, kb] (zesz bytes each)
  const void* bias;    // T [N] or null
  void* Y;             // T [M, N]
  uint32_t N, K, kb, rowb, zrow, M, bsl, zesz;
  uint32_t meta_bytes;  // per-wave LDS slice: C*kb*4 scales (+ zero points), 16-aligned
  uint32_t zoff;        // zero points' offset inside the slice
  // further projections on the same grid (Qkv's K and V, Mlp's up; the same
  // A, K, block size and zero-point kind): projection p owns the grid's
  // columns [c1 or c2, ...), each projection's count rounded up to whole waves
  uint32_t np, c1, c2;
  const uint8_t *B1, *B2;
  const void *S1, *S2, *Z1, *Z2, *bias1, *bias2;
  void *Y1, *Y2;
  uint32_t N1, N2;
  // Qkv / Mlp prologue on the staged rows (null: none): r = A + skip, the
  // residual r, x = r * inversesqrt(sum(r^2) / K + eps) * gamma
  const void* skip;
  const void* gamma;
  void* residual;
  float eps;
};

// LDS of the staged activations: [MR][nchunk] chunks of 128 / BITS floats
// (a chunk is 16 bytes of codes) at a stride of 4 more (the pad spreads the
// lanes of a 16-byte read over the banks), then the sums [MR][nchunk * H],
// one per 16 codes (H = 2 halves of a 4-bit chunk, 1 for 8-bit).
template <int BITS>
__host__ __device__ constexpr uint32_t f32_chunk_stride() {
  return 128 / BITS + 4;
}

template <int MR, int BITS = 4>
__host__ __device__ constexpr uint32_t f32_act_bytes(uint32_t nchunk) {
  return MR * nchunk * f32_chunk_stride<BITS>() * 4u + MR * nchunk * (64u / BITS) / 8u * 4u;
}

// Byte i of x as a float (the compiler emits v_cvt_f32_ubyte{i}).
__device__ __forceinline__ float ubyte(uint32_t x, int i) {
  return static_cast<float>((x >> (8 * i)) & 0xFFu);
}

// T: float (activations, scales, bias and outputs in float32) or f16.
template <typename T, int ZPK, int CPL, int C, int MR, int W, int BITS = 4>
__global__ __launch_bounds__(W * 64) void k_gemv_f32(F32Args a) {
  static_assert(BITS == 2 || BITS == 4 || BITS == 8, "2-, 4- or 8-bit codes");
  constexpr uint32_t TS = sizeof(T);
  constexpr uint32_t CODES = 128 / BITS;         // codes per 16-byte chunk
  constexpr uint32_t H = CODES / 16;             // 16-code halves per chunk
  constexpr uint32_t CS = f32_chunk_stride<BITS>();
  constexpr float ZMID = static_cast<float>(1 << (BITS - 1));  // implicit zero point 2^(bits - 1)
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // this wave's projection and its first column (wave-uniform)
  const uint32_t gcol = (xcd_slot(blockIdx.x, gridDim.x) * W + wave) * C;
  const uint32_t pj = a.np > 1 && gcol >= a.c1 ? (a.np > 2 && gcol >= a.c2 ? 2u : 1u) : 0u;
  const uint8_t* PB = pj == 0 ? a.B : pj == 1 ? a.B1 : a.B2;
  const void* PS = pj == 0 ? a.S : pj == 1 ? a.S1 : a.S2;
  const void* PZ = pj == 0 ? a.Z : pj == 1 ? a.Z1 : a.Z2;
  const void* Pbias = pj == 0 ? a.bias : pj == 1 ? a.bias1 : a.bias2;
  void* PY = pj == 0 ? a.Y : pj == 1 ? a.Y1 : a.Y2;
  const uint32_t N = pj == 0 ? a.N : pj == 1 ? a.N1 : a.N2;
  const uint32_t K = a.K, kb = a.kb, rowb = a.rowb, zrow = a.zrow;
  const uint32_t nchunk = rowb >> 4;
  // this workgroup's chunk of up to MR rows (the grid's second dimension)
  const uint32_t m0 = blockIdx.y * MR;
  const int M = static_cast<int>(a.M - m0 < MR ? a.M - m0 : MR);
  const T* A = static_cast<const T*>(a.A) + static_cast<size_t>(m0) * K;
  T* Yo = static_cast<T*>(PY) + static_cast<size_t>(m0) * N;
  const uint32_t col0 = gcol - (pj == 0 ? 0u : pj == 1 ? a.c1 : a.c2);
  auto clampc = [&](uint32_t c) { return c < N ? c : N - 1; };
  const uint32_t act_floats = MR * nchunk * CS;
  float* xs = reinterpret_cast<float*>(smem);        // [MR][nchunk][CS]
  float* sums = xs + act_floats;                     // [MR][H * nchunk]
  unsigned char* meta = smem + f32_act_bytes<MR, BITS>(nchunk) + wave * a.meta_bytes;

  // ---- the wave's scale / zero-point block (C consecutive rows), 16-byte
  // pieces; loads start at the dword boundary at or below the block
  const uint32_t c0 = clampc(col0);
  const uint32_t sbytes = C * kb * TS;
  const uint32_t zbytes = ZPK == ZP_NONE ? 0u : C * zrow;
  const uint32_t zdel = (c0 * zrow) & 3u;
  constexpr int MP = 4;  // up to 4 KB per block
  u32x4 sv[MP], zv[ZPK == ZP_NONE ? 1 : MP];
  {
    // a dword straddling the range's end reads as zero, so the range ends on
    // the dword boundary past the last float16 scale (the scales are 16-byte
    // aligned, so that dword lies in the page of the last scale)
    const rsrc_t rS = mk_rsrc(PS, (N * kb * TS + 3u) & ~3u);
#pragma unroll
    for (int q = 0; q < MP; ++q) {
      const uint32_t o = lane * 16u + 1024u * q;
      sv[q] = bld16_nt(rS, o < sbytes ? c0 * kb * TS + o : kOOB, 0);
    }
    if constexpr (ZPK != ZP_NONE) {
      const rsrc_t rZ = mk_rsrc(PZ, (N * zrow + 15u) & ~15u);
#pragma unroll
      for (int q = 0; q < MP; ++q) {
        const uint32_t o = lane * 16u + 1024u * q;
        zv[q] = bld16_nt(rZ, o < zbytes + zdel ? c0 * zrow - zdel + o : kOOB, 0);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- activations of the workgroup: pieces of 4 values (16 bytes of
  // float32, 8 of float16), thread t takes pieces t, t + 64 W, ...
  const rsrc_t rA = mk_rsrc(A, static_cast<uint32_t>(M) * K * TS);
  constexpr int PIECES_PER_ROW_MAX = 64 * CPL * CODES / 4;  // nchunk * CODES floats / 4
  constexpr int PPT = (MR * PIECES_PER_ROW_MAX + W * 64 - 1) / (W * 64);
  const uint32_t ppr = nchunk * (CODES / 4);  // pieces per staged row
  u32x4 av[PPT];
#pragma unroll
  for (int it = 0; it < PPT; ++it) {
    const uint32_t p = static_cast<uint32_t>(tid) + it * W * 64u;
    const uint32_t m = p / ppr, k = (p % ppr) * 4u;
    const bool ok = static_cast<int>(m) < M && k < K;  // K % 4 == 0 on this path
    if constexpr (TS == 4) {
      av[it] = bld16(rA, ok ? (m * K + k) * 4u : kOOB, 0);
    } else {
      // four halves, widened exactly at the staging
      const u32x2 h = bld8(rA, ok ? (m * K + k) * 2u : kOOB, 0);
      const f16x2 h0 = as_h2(h[0]), h1 = as_h2(h[1]);
      const f32x4 f = {static_cast<float>(h0[0]), static_cast<float>(h0[1]), static_cast<float>(h1[0]),
                       static_cast<float>(h1[1])};
      av[it] = __builtin_bit_cast(u32x4, f);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- weights: every chunk of the wave's C columns
  const rsrc_t rB = mk_rsrc(PB, N * rowb);
  u32x4 wv[C][CPL];
#pragma unroll
  for (int i = 0; i < C; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t ch = static_cast<uint32_t>(lane + 64 * j);
      wv[i][j] = bld16_nt(rB, ch < nchunk ? clampc(col0 + i) * rowb + ch * 16u : kOOB, 0);
    }
  __builtin_amdgcn_sched_barrier(0);

  // ---- stage: the wave's meta slice, the activations and their 16-code sums
#pragma unroll
  for (int q = 0; q < MP; ++q) {
    const uint32_t o = lane * 16u + 1024u * q;
    if (o < sbytes) *reinterpret_cast<u32x4*>(meta + o) = sv[q];
    if (ZPK != ZP_NONE && o < zbytes + zdel) *reinterpret_cast<u32x4*>(meta + a.zoff + o) = zv[ZPK == ZP_NONE ? 0 : q];
  }
#pragma unroll
  for (int it = 0; it < PPT; ++it) {
    const uint32_t p = static_cast<uint32_t>(tid) + it * W * 64u;
    if (p < MR * ppr) *reinterpret_cast<u32x4*>(xs + (p / (CODES / 4)) * CS + (p % (CODES / 4)) * 4u) = av[it];
  }
  __syncthreads();
  if (a.skip || a.gamma || a.residual) {  // uniform: the Qkv / Mlp prologue (float32 calls)
    // each thread reworks the pieces it staged: r = x + skip (the residual,
    // written by the workgroups of the grid's first column), its rows' sums
    // of r^2, then x = r * inv * gamma
    auto ld4 = [](const T* q) {
      if constexpr (TS == 4) {
        return *reinterpret_cast<const f32x4*>(q);
      } else {
        const u32x2 h = *reinterpret_cast<const u32x2*>(q);
        const f16x2 h0 = as_h2(h[0]), h1 = as_h2(h[1]);
        return f32x4{static_cast<float>(h0[0]), static_cast<float>(h0[1]), static_cast<float>(h1[0]), static_cast<float>(h1[1])};
      }
    };
    float ss[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) ss[m] = 0.f;
#pragma unroll
    for (int it = 0; it < PPT; ++it) {
      const uint32_t p = static_cast<uint32_t>(tid) + it * W * 64u;
      const uint32_t m = p / ppr, k = (p % ppr) * 4u;
      if (p >= MR * ppr || static_cast<int>(m) >= M || k >= K) continue;
      f32x4* px = reinterpret_cast<f32x4*>(xs + (p / (CODES / 4)) * CS + (p % (CODES / 4)) * 4u);
      f32x4 v = *px;
      const size_t o = static_cast<size_t>(m0 + m) * K + k;
      if (a.skip) v += ld4(static_cast<const T*>(a.skip) + o);
      if (a.residual && blockIdx.x == 0) {
        T* r = static_cast<T*>(a.residual) + o;
        r[0] = static_cast<T>(v.x), r[1] = static_cast<T>(v.y), r[2] = static_cast<T>(v.z), r[3] = static_cast<T>(v.w);
      }
      *px = v;
      const float q = __builtin_fmaf(v.x, v.x, __builtin_fmaf(v.y, v.y, __builtin_fmaf(v.z, v.z, v.w * v.w)));
#pragma unroll
      for (int mm = 0; mm < MR; ++mm) ss[mm] += static_cast<int>(m) == mm ? q : 0.f;
    }
    if (a.gamma) {
      __shared__ float s_ss[W][MR];
#pragma unroll
      for (int mm = 0; mm < MR; ++mm) {
        const float t = wave_sum(ss[mm]);
        if (lane == 0) s_ss[wave][mm] = t;
      }
      __syncthreads();
      float inv[MR];
#pragma unroll
      for (int mm = 0; mm < MR; ++mm) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) t += s_ss[w][mm];
        inv[mm] = 1.f / __builtin_sqrtf(t / static_cast<float>(K) + a.eps);
      }
#pragma unroll
      for (int it = 0; it < PPT; ++it) {
        const uint32_t p = static_cast<uint32_t>(tid) + it * W * 64u;
        const uint32_t m = p / ppr, k = (p % ppr) * 4u;
        if (p >= MR * ppr || static_cast<int>(m) >= M || k >= K) continue;
        f32x4* px = reinterpret_cast<f32x4*>(xs + (p / (CODES / 4)) * CS + (p % (CODES / 4)) * 4u);
        float im = inv[0];
#pragma unroll
        for (int mm = 1; mm < MR; ++mm) im = static_cast<int>(m) == mm ? inv[mm] : im;
        const f32x4 gv = ld4(static_cast<const T*>(a.gamma) + k);
        const f32x4 v = *px;
        *px = f32x4{v.x * im * gv.x, v.y * im * gv.y, v.z * im * gv.z, v.w * im * gv.w};
      }
    }
    __syncthreads();
  }
  // sums per 16 codes: thread t sums half h = t, t + 64 W, ...
  for (uint32_t h = static_cast<uint32_t>(tid); h < MR * nchunk * H; h += W * 64u) {
    const float* x = xs + (h / H) * CS + (h % H) * 16u;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      s0 += x[e];
      s1 += x[e + 1];
    }
    sums[h] = s0 + s1;
  }
  __syncthreads();

  // ---- columns
  float out[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) out[m] = 0.f;
  const unsigned char* zmeta = meta + a.zoff + zdel;
#pragma unroll
  for (int i = 0; i < C; ++i) {
    if (col0 + i >= N) break;  // wave-uniform
    float y[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) y[m] = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t ch = static_cast<uint32_t>(lane + 64 * j);
      const uint32_t chc = ch < nchunk ? ch : nchunk - 1;  // past-the-row lanes: in-range reads, no contribution
#pragma unroll
      for (int h = 0; h < static_cast<int>(H); ++h) {  // 16-code halves (8-bit: the chunk)
        const uint32_t b = (chc * CODES + 16u * h) >> a.bsl;
        const float s = static_cast<float>(*reinterpret_cast<const T*>(meta + (i * kb + b) * TS));
        float z = ZMID;
        if constexpr (ZPK == ZP_PACKED) {
          if constexpr (BITS == 2) z = static_cast<float>((zmeta[i * zrow + (b >> 2)] >> ((b & 3u) * 2u)) & 3u);
          else if constexpr (BITS == 4) z = static_cast<float>((zmeta[i * zrow + (b >> 1)] >> ((b & 1u) * 4u)) & 15u);
          else z = static_cast<float>(zmeta[i * zrow + b]);
        } else if constexpr (ZPK == ZP_FLOAT) {
          const unsigned char* zp = zmeta + i * zrow + b * a.zesz;
          z = a.zesz == 4 ? *reinterpret_cast<const float*>(zp) : static_cast<float>(*reinterpret_cast<const f16*>(zp));
        }
        float cv[16];
        if constexpr (BITS == 2) {
          // one dword: code 4 e + s in bits 8 e + 2 s .. + 1
          const uint32_t x = wv[i][j][h];
#pragma unroll
          for (int sh = 0; sh < 4; ++sh) {
            const uint32_t v = (x >> (2 * sh)) & 0x03030303u;
#pragma unroll
            for (int e = 0; e < 4; ++e) cv[4 * e + sh] = ubyte(v, e);
          }
        } else if constexpr (BITS == 4) {
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const uint32_t x = wv[i][j][2 * h + q];
            const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              cv[8 * q + 2 * e] = ubyte(lo, e);
              cv[8 * q + 2 * e + 1] = ubyte(hi, e);
            }
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) cv[4 * q + e] = ubyte(wv[i][j][q], e);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const float* x = xs + (m * nchunk + chc) * CS + 16u * h;
          const f32x4 x0 = *reinterpret_cast<const f32x4*>(x), x1 = *reinterpret_cast<const f32x4*>(x + 4);
          const f32x4 x2 = *reinterpret_cast<const f32x4*>(x + 8), x3 = *reinterpret_cast<const f32x4*>(x + 12);
          const float xv[16] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3],
                                x2[0], x2[1], x2[2], x2[3], x3[0], x3[1], x3[2], x3[3]};
          float p0 = 0.f, p1 = 0.f;
#pragma unroll
          for (int e = 0; e < 16; e += 2) {
            p0 = __builtin_fmaf(cv[e], xv[e], p0);
            p1 = __builtin_fmaf(cv[e + 1], xv[e + 1], p1);
          }
          const float sa = sums[(m * nchunk + chc) * H + h];
          float t = __builtin_fmaf(-z, sa, p0 + p1);
          if (!__builtin_isfinite(sa)) {
            // an infinite activation: the folded form would give Inf - Inf;
            // the reference's per-element (code - z) * a keeps +-Inf
            t = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) t = __builtin_fmaf(cv[e] - z, xv[e], t);
          }
          // lanes past the row read the last chunk (in-range addresses) and
          // add nothing: a zero scale would turn an infinite activation into NaN
          y[m] = ch < nchunk ? __builtin_fmaf(s, t, y[m]) : y[m];
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float tot = wave_total(y[m]);
      out[m] = lane == i ? tot : out[m];
    }
  }
  const uint32_t mycol = col0 + static_cast<uint32_t>(lane);
  if (lane < C && mycol < N) {
    const float b = Pbias ? static_cast<float>(static_cast<const T*>(Pbias)[mycol]) : 0.f;
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) Yo[static_cast<uint32_t>(m) * N + mycol] = static_cast<T>(out[m] + b);
  }
}

// Host side: C columns per wave, W waves per workgroup.
constexpr int kF32C = 2, kF32W = 8;

inline int f32_cpl(const Launch& L) {
  const int64_t chunks = L.kb * L.blob / 16;
  for (int c = 1; c <= 4; c *= 2)
    if (chunks <= 64 * c) return c;
  return 0;
}

// Rows per workgroup: 1, 2 or 4 (more rows: chunks on the grid's y), fewer
// where a thread would hold more than 16 activation loads (2-bit rows of more
// than 64 chunks).
inline int f32_mr(const Launch& L) {
  int mr = L.M <= 1 ? 1 : L.M <= 2 ? 2 : 4;
  const int cpl = f32_cpl(L);
  while (mr > 1 && mr * cpl * 8 / L.bits > 16) mr /= 2;
  return mr;
}

// Bytes of one activation, scale, bias or output value: float32 or float16.
inline int64_t f32_esz(const Launch& L) { return L.dtype == DT_F16 ? 2 : 4; }

inline uint32_t f32_meta_bytes(const Launch& L, uint32_t& zoff) {
  const uint32_t sb = static_cast<uint32_t>(kF32C * L.kb * f32_esz(L));
  zoff = (sb + 15u) & ~15u;
  const int64_t zrow = L.zp_kind == ZP_PACKED ? L.zrow : L.kb * (L.zp_dtype == DT_F32 ? 4 : 2);
  const uint32_t zb = L.zp_kind == ZP_NONE ? 0u : static_cast<uint32_t>(kF32C * zrow);
  return (zoff + zb + 3u + 15u) & ~15u;
}

// fp32, or fp16 with 2- or 8-bit codes or float32 weights required (`exact`:
// dequantised weights binary16 cannot hold); 2-, 4- or 8-bit, power-of-two
// block_size >= 16, K a multiple of 4, 16-byte aligned tensors, rows of at
// most 256 chunks (whole 16-byte chunks), the wave's scale / zero-point block
// within 4 KB and the staging within 160 KB of LDS; at most 65535 chunks of
// four rows (the grid's y).
inline bool f32_fits(const Launch& L) {
  const bool t_ok = L.dtype == DT_F32 || (L.dtype == DT_F16 && (L.bits != 4 || L.exact_weights));
  if (!t_ok || (L.bits != 2 && L.bits != 4 && L.bits != 8) || L.bs_log2 < 4 || L.op != OP_MATMUL || L.K % 4 != 0)
    return false;
  if ((L.kb * L.block_size) % (128 / L.bits) != 0) return false;
  const int mr = f32_mr(L), cpl = f32_cpl(L);
  if (L.M < 1 || (L.M + mr - 1) / mr > 65535) return false;
  if (cpl == 0) return false;
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (!al(L.A) || L.nproj < 1 || L.nproj > 3) return false;
  for (int i = 0; i < L.nproj; ++i) {  // further projections: Qkv / Mlp on one grid
    if (!al(L.p[i].B) || !al(L.p[i].scales) || !al(L.p[i].zp)) return false;
    if (L.zp_kind != ZP_NONE && L.p[i].zp == nullptr) return false;
  }
  if (!al(L.skip) || !al(L.gamma) || !al(L.residual)) return false;  // the staged prologue's 16-byte pieces
  uint32_t zoff = 0;
  const uint32_t meta = f32_meta_bytes(L, zoff);
  if (kF32C * L.kb * f32_esz(L) > 4096 || meta - zoff > 4096 + 16) return false;
  const uint32_t nchunk = static_cast<uint32_t>(L.kb * L.blob / 16);
  if (mr * f32_cpl(L) * 8 / L.bits > 16) return false;  // activation loads per thread (registers)
  const int64_t codes = 128 / L.bits;
  const int64_t lds = int64_t(mr) * nchunk * (codes + 4) * 4 + int64_t(mr) * nchunk * (codes / 16) * 4 + int64_t(kF32W) * meta;
  return lds <= 159 * 1024;
}

template <typename T, int ZPK, int CPL, int MR, int BITS>
inline hipError_t launch_f32_k(const Launch& L, hipStream_t st) {
  F32Args a{};
  const Proj& P = L.p[0];
  a.A = L.A;
  a.B = P.B;
  a.S = P.scales;
  a.Z = P.zp;
  a.bias = P.bias;
  a.Y = P.Y;
  a.N = static_cast<uint32_t>(P.N);
  a.K = static_cast<uint32_t>(L.K);
  a.kb = static_cast<uint32_t>(L.kb);
  a.rowb = static_cast<uint32_t>(L.kb * L.blob);
  a.zesz = L.zp_dtype == DT_F32 ? 4u : 2u;
  a.zrow = L.zp_kind == ZP_PACKED ? static_cast<uint32_t>(L.zrow) : a.kb * a.zesz;
  a.M = static_cast<uint32_t>(L.M);
  a.bsl = static_cast<uint32_t>(L.bs_log2);
  a.meta_bytes = f32_meta_bytes(L, a.zoff);
  a.skip = L.skip;
  a.gamma = L.gamma;
  a.residual = L.residual;
  a.eps = L.eps;
  // the projections' columns on the grid, each rounded up to whole waves
  auto wcols = [](int64_t n) { return static_cast<uint32_t>((n + kF32C - 1) / kF32C * kF32C); };
  uint32_t cols = wcols(P.N);
  a.np = static_cast<uint32_t>(L.nproj);
  if (L.nproj > 1) {
    a.c1 = cols;
    a.B1 = L.p[1].B, a.S1 = L.p[1].scales, a.Z1 = L.p[1].zp, a.bias1 = L.p[1].bias, a.Y1 = L.p[1].Y;
    a.N1 = static_cast<uint32_t>(L.p[1].N);
    cols += wcols(L.p[1].N);
  }
  if (L.nproj > 2) {
    a.c2 = cols;
    a.B2 = L.p[2].B, a.S2 = L.p[2].scales, a.Z2 = L.p[2].zp, a.bias2 = L.p[2].bias, a.Y2 = L.p[2].Y;
    a.N2 = static_cast<uint32_t>(L.p[2].N);
    cols += wcols(L.p[2].N);
  }
  const uint32_t nchunk = a.rowb / 16u;
  const size_t lds = f32_act_bytes<MR, BITS>(nchunk) + size_t(kF32W) * a.meta_bytes;
  auto kern = k_gemv_f32<T, ZPK, CPL, kF32C, MR, kF32W, BITS>;
  if (lds > 64 * 1024) {
    static std::atomic<int> done[kMaxDevices];  // per instantiation and device
    // 1 KB of the 160 KB stays for the kernel's static LDS (the prologue's sums)
    const hipError_t attr = raise_lds_cap(reinterpret_cast<const void*>(kern), 159 * 1024, done);
    if (attr != hipSuccess) return attr;
  }
  const uint32_t waves = cols / kF32C;
  const uint32_t chunks = static_cast<uint32_t>((L.M + MR - 1) / MR);
  hipLaunchKernelGGL(kern, dim3((waves + kF32W - 1) / kF32W, chunks), dim3(kF32W * 64), lds, st, a);
  return hipGetLastError();
}

// the activation loads per thread f32_fits admits (2-bit: MR CPL <= 4; the
// other shapes are not instantiated)
template <typename T, int ZPK, int CPL, int MR, int BITS>
inline hipError_t launch_f32_3(const Launch& L, hipStream_t st) {
  if constexpr (MR * CPL * 8 / BITS > 16) return hipErrorInvalidValue;
  else return launch_f32_k<T, ZPK, CPL, MR, BITS>(L, st);
}

template <typename T, int ZPK, int CPL, int BITS>
inline hipError_t launch_f32_2(const Launch& L, hipStream_t st) {
  switch (f32_mr(L)) {
    case 1: return launch_f32_3<T, ZPK, CPL, 1, BITS>(L, st);
    case 2: return launch_f32_3<T, ZPK, CPL, 2, BITS>(L, st);
    default: return launch_f32_3<T, ZPK, CPL, 4, BITS>(L, st);
  }
}

template <typename T, int ZPK, int BITS>
inline hipError_t launch_f32_b(const Launch& L, hipStream_t st) {
  switch (f32_cpl(L)) {
    case 1: return launch_f32_2<T, ZPK, 1, BITS>(L, st);
    case 2: return launch_f32_2<T, ZPK, 2, BITS>(L, st);
    default: return launch_f32_2<T, ZPK, 4, BITS>(L, st);
  }
}

template <typename T, int ZPK>
inline hipError_t launch_f32_t(const Launch& L, hipStream_t st) {
  if (L.bits == 8) return launch_f32_b<T, ZPK, 8>(L, st);
  if (L.bits == 2) return launch_f32_b<T, ZPK, 2>(L, st);
  return launch_f32_b<T, ZPK, 4>(L, st);
}

template <int ZPK>
inline hipError_t launch_f32_1(const Launch& L, hipStream_t st) {
  return L.dtype == DT_F16 ? launch_f32_t<f16, ZPK>(L, st) : launch_f32_t<float, ZPK>(L, st);
}

// Entry of one zero-point kind (defined in xrmm_gemv_f32_zp.hip).
template <int ZPK>
hipError_t launch_f32_for(const Launch& L, hipStream_t st);

}  // namespace xrmm
