// HIP kernels of libxrmm for gfx950 (MI355X): MatMulNBits, MatMulNBitsQkv and
// MatMulNBitsMlp.
//
// The arithmetic follows xrGPU's serial shader
// (kernels/_shared/extended/shaders/complex_kernel.glsl:80 nbitWeight,
// :81 packedInput, :83 packedMatmul, :39-47 fused/logistic); the work
// decomposition is this file's own:
//
//  * k_gemv_q4   M <= 16, fp16, 4-bit. One workgroup owns a 16-column tile;
//                its waves split K. Packed weights stream with 16-byte loads,
//                are dequantised in registers to fp16 and multiplied on
//                v_mfma_f32_16x16x32_f16 against the activations staged once
//                in LDS. Qkv/Mlp fuse the RMS prologue and the SwiGLU epilogue.
//  * k_gemm_q4   M > 16, fp16, 4-bit. LDS-tiled MFMA GEMM: activation tiles and
//                weight tiles dequantised to fp16 are staged in LDS and fed to
//                v_mfma_f32_32x32x16_f16.
//  * k_generic   every other geometry (fp32, 2/8-bit, float zero points with a
//                non-fast block size, unaligned tensors): one wave per column
//                and row block, the reference's float32 weight formula.
//
// Dequantisation (4-bit, integer zero point): code - z is exact in binary16
// and (code - z) * scale is rounded once, so the staged fp16 weight equals the
// reference's float32 weight rounded once to binary16. Codes are widened with
// the exponent-bias trick: OR-ing a nibble into the mantissa of 1024.0h gives
// 1024 + code exactly (and 1024 + 16*code for the high nibble of a byte).
#include "xrmm_internal.h"

namespace xrmm {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// scalar helpers

__device__ __forceinline__ float ld_t(const void* p, int64_t i, int dt) {
  return dt == DT_F32 ? static_cast<const float*>(p)[i]
                      : static_cast<float>(static_cast<const f16*>(p)[i]);
}

__device__ __forceinline__ void st_t(void* p, int64_t i, float v, int dt) {
  if (dt == DT_F32)
    static_cast<float*>(p)[i] = v;
  else
    static_cast<f16*>(p)[i] = static_cast<f16>(v);  // v_cvt_f16_f32: RNE
}

// z(n, b) (complex_kernel.glsl:80): midpoint when absent, the float element, or
// the ONNX Runtime packed low-first field.
__device__ __forceinline__ float zp_value(const Launch& L, const Proj& P, int64_t n, int64_t b) {
  if (!P.zp) return static_cast<float>(1u << (L.bits - 1));
  if (L.zp_kind == ZP_FLOAT) return ld_t(P.zp, n * L.kb + b, L.zp_dtype);
  const int64_t bit = b * L.bits;
  const uint32_t byte = static_cast<const uint8_t*>(P.zp)[n * L.zrow + (bit >> 3)];
  return static_cast<float>((byte >> (bit & 7)) & ((1u << L.bits) - 1u));
}

// nbitWeight (complex_kernel.glsl:80): (float(code) - z) * scale in float32.
__device__ __forceinline__ float weight_f32(const Launch& L, const Proj& P, int64_t n, int64_t k) {
  const int64_t b = k / L.block_size;
  const int64_t bit = (k - b * L.block_size) * L.bits;
  const uint32_t byte = P.B[(n * L.kb + b) * L.blob + (bit >> 3)];
  const uint32_t q = (byte >> (bit & 7)) & ((1u << L.bits) - 1u);
  const float z = zp_value(L, P, n, b);
  const float s = ld_t(P.scales, n * L.kb + b, L.dtype);
  return __fmul_rn(__fsub_rn(static_cast<float>(q), z), s);
}

// logistic / fused (complex_kernel.glsl:39-47), erf form of gelu for 1027.
__device__ __forceinline__ float logistic(float x) {
  return x >= 0.f ? 1.f / (1.f + expf(-x)) : expf(x) / (1.f + expf(x));
}

__device__ __forceinline__ float activate(float x, int kind) {
  switch (kind) {
    case 1: return x > 0.f ? x : 0.f;
    case 2: return x * logistic(x);
    case 3: return .5f * x * (1.f + erff(x * .7071067811865475f));
    case 4: return tanhf(x);
    case 5: return logistic(x);
    default: return x;
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---------------------------------------------------------------------------
// 4-bit dequantisation to binary16 (shared by GEMV, GEMM and xrmm_dequantize)

__device__ __forceinline__ f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }

// Per-block constants: -(1024 + z), -(64 + z) and the scale, each as a pair.
struct Dq {
  f16x2 nz1024, nz64, s;
};

__device__ __forceinline__ Dq dq_consts(float z, f16 s) {
  Dq c;
  const f16 a = static_cast<f16>(-(1024.f + z)), b = static_cast<f16>(-(64.f + z));
  c.nz1024 = f16x2{a, a};
  c.nz64 = f16x2{b, b};
  c.s = f16x2{s, s};
  return c;
}

// Eight low-first codes of one dword -> (code - z) * scale, in the order
// [c0, c4, c1, c5, c2, c6, c3, c7]. The activations are staged in the same
// order, so the dot product is unchanged.
__device__ __forceinline__ f16x8 dq8(uint32_t x, const Dq& c) {
  const uint32_t lo = 0x000F000Fu, hi = 0x00F000F0u, magic = 0x64006400u;
  const uint32_t x8 = x >> 8;
  const f16x2 inv16 = {static_cast<f16>(0.0625f), static_cast<f16>(0.0625f)};
  // 1024 + c - (1024 + z) and (1024 + 16c)/16 - (64 + z): both exact
  f16x2 d0 = as_h2((x & lo) | magic) + c.nz1024;
  f16x2 d1 = __builtin_elementwise_fma(as_h2((x & hi) | magic), inv16, c.nz64);
  f16x2 d2 = as_h2((x8 & lo) | magic) + c.nz1024;
  f16x2 d3 = __builtin_elementwise_fma(as_h2((x8 & hi) | magic), inv16, c.nz64);
  d0 = d0 * c.s;
  d1 = d1 * c.s;
  d2 = d2 * c.s;
  d3 = d3 * c.s;
  return f16x8{d0.x, d0.y, d1.x, d1.y, d2.x, d2.y, d3.x, d3.y};
}

// Float zero point of arbitrary value: the reference float32 weight, rounded
// once to binary16 (same pair order as dq8).
__device__ __forceinline__ f16x8 dq8_f32z(uint32_t x, float z, float s) {
  f16x8 r;
  const int order[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float q = static_cast<float>((x >> (4 * order[i])) & 15u);
    r[i] = static_cast<f16>(__fmul_rn(__fsub_rn(q, z), s));
  }
  return r;
}

// Pair order of eight consecutive activations, matching dq8.
__device__ __forceinline__ f16x8 pair_order(f16x8 v) {
  return __builtin_shufflevector(v, v, 0, 4, 1, 5, 2, 6, 3, 7);
}

template <int ZPK>
__device__ __forceinline__ float zp_fast(const Launch& L, const Proj& P, int64_t n, int64_t b) {
  if constexpr (ZPK == ZP_NONE) {
    return 8.f;
  } else if constexpr (ZPK == ZP_PACKED) {
    const uint32_t byte = static_cast<const uint8_t*>(P.zp)[n * L.zrow + (b >> 1)];
    return static_cast<float>((byte >> ((b & 1) * 4)) & 15u);
  } else {
    return ld_t(P.zp, n * L.kb + b, L.zp_dtype);
  }
}

// Dequantise one 16-byte chunk (32 codes) of column n starting at code 32*ch.
// SPC = 1 when the chunk lies in one block (block_size % 32 == 0), 2 when
// each 16-code half lies in one block (block_size % 16 == 0).
template <int ZPK, int SPC>
__device__ __forceinline__ void dq_chunk(const Launch& L, const Proj& P, int64_t n, int64_t ch,
                                         bool valid, u32x4 w, f16x8 out[4]) {
#pragma unroll
  for (int half = 0; half < SPC; ++half) {
    const int64_t b = (ch * 32 + half * 16) / L.block_size;
    f16 s = static_cast<f16>(0.f);
    float z = 8.f;
    if (valid) {
      s = static_cast<const f16*>(P.scales)[n * L.kb + b];
      z = zp_fast<ZPK>(L, P, n, b);
    }
    if constexpr (ZPK == ZP_FLOAT) {
      const float sf = static_cast<float>(s);
#pragma unroll
      for (int d = half * (4 / SPC); d < (half + 1) * (4 / SPC); ++d) out[d] = dq8_f32z(w[d], z, sf);
    } else {
      const Dq c = dq_consts(z, s);
#pragma unroll
      for (int d = half * (4 / SPC); d < (half + 1) * (4 / SPC); ++d) out[d] = dq8(w[d], c);
    }
  }
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *static_cast<const u32x4*>(p);
}

// ---------------------------------------------------------------------------
// generic kernel: one wave per (column, block of MB rows)

template <int MB>
__global__ __launch_bounds__(64) void k_generic(Launch L) {
  const int lane = threadIdx.x;
  int64_t col = blockIdx.x;
  int pi = 0;
  if (L.op == OP_QKV) {
    if (col >= L.p[0].N) {
      col -= L.p[0].N;
      pi = 1;
      if (col >= L.p[1].N) {
        col -= L.p[1].N;
        pi = 2;
      }
    }
  }
  const Proj& P = L.p[pi];
  const int64_t M = L.M, K = L.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * MB;
  const bool norm = L.op != OP_MATMUL;

  auto raw = [&](int64_t m, int64_t k) -> float {
    float x = ld_t(L.A, m * K + k, L.dtype);
    if (norm && L.skip) x = __fadd_rn(x, ld_t(L.skip, m * K + k, L.dtype));
    return x;
  };

  float inv[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    inv[i] = 1.f;
    const int64_t m = m0 + i;
    if (norm && L.gamma && m < M) {
      float s = 0.f;
      for (int64_t k = lane; k < K; k += 64) {
        const float r = raw(m, k);
        s += r * r;
      }
      s = wave_sum(s);
      inv[i] = 1.f / sqrtf(s / static_cast<float>(K) + L.eps);
    }
  }
  if (norm && L.residual && blockIdx.x == 0) {
    for (int i = 0; i < MB; ++i) {
      const int64_t m = m0 + i;
      if (m >= M) break;
      for (int64_t k = lane; k < K; k += 64) st_t(L.residual, m * K + k, raw(m, k), L.dtype);
    }
  }

  float acc[MB], acc2[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = acc2[i] = 0.f;
  for (int64_t k = lane; k < K; k += 64) {
    const float w = weight_f32(L, P, col, k);
    const float wu = L.op == OP_MLP ? weight_f32(L, L.p[1], col, k) : 0.f;
    const float gk = (norm && L.gamma) ? ld_t(L.gamma, k, L.dtype) : 1.f;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int64_t m = m0 + i;
      if (m < M) {
        float x = raw(m, k);
        if (norm && L.gamma) x = x * (inv[i] * gk);
        acc[i] += x * w;
        acc2[i] += x * wu;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    acc[i] = wave_sum(acc[i]);
    if (L.op == OP_MLP) acc2[i] = wave_sum(acc2[i]);
  }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int64_t m = m0 + i;
      if (m >= M) break;
      float y = acc[i];
      if (L.op == OP_MATMUL) {
        if (P.bias) y += ld_t(P.bias, col, L.dtype);
      } else if (L.op == OP_MLP) {
        const float gb = P.bias ? ld_t(P.bias, col, L.dtype) : 0.f;
        const float ub = L.p[1].bias ? ld_t(L.p[1].bias, col, L.dtype) : 0.f;
        y = activate(y + gb, L.act) * (acc2[i] + ub);
      }
      st_t(P.Y, m * P.N + col, y, L.dtype);
    }
  }
}

// ---------------------------------------------------------------------------
// GEMV for M <= 16: fp16 activations, 4-bit weights, MFMA 16x16x32

constexpr int GEMV_WAVES = 4;

template <int ZPK, int SPC, int OP>
__global__ __launch_bounds__(GEMV_WAVES * 64) void k_gemv_q4(Launch L) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float s_inv[16];
  constexpr int NT = GEMV_WAVES * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = static_cast<int>(L.M);
  const int64_t K = L.K;
  const int64_t Kp = L.kb * L.block_size;  // padded K, a multiple of 32
  const int64_t ldA = Kp + 8;               // halfs per staged row
  f16* As = reinterpret_cast<f16*>(smem);
  float* red = reinterpret_cast<float*>(smem);

  // tile -> projection
  int64_t tile = blockIdx.x;
  int pi = 0;
  if constexpr (OP == OP_QKV) {
    const int64_t t0 = (L.p[0].N + 15) / 16, t1 = (L.p[1].N + 15) / 16;
    if (tile >= t0) {
      tile -= t0;
      pi = 1;
      if (tile >= t1) {
        tile -= t1;
        pi = 2;
      }
    }
  }
  const Proj& P = L.p[pi];
  const int64_t n0 = tile * 16;
  const int64_t groups = Kp / 8;

  // RMS statistic of r = A + skip per row (packedInput, complex_kernel.glsl:81)
  if constexpr (OP != OP_MATMUL) {
    if (L.gamma) {
      for (int m = wave; m < M; m += GEMV_WAVES) {
        float s = 0.f;
        for (int64_t j = lane; j < K / 8; j += 64) {
          const f16x8 a = __builtin_bit_cast(f16x8, ld16(static_cast<const f16*>(L.A) + m * K + j * 8));
          f16x8 sk = {};
          if (L.skip) sk = __builtin_bit_cast(f16x8, ld16(static_cast<const f16*>(L.skip) + m * K + j * 8));
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float r = __fadd_rn(static_cast<float>(a[i]), static_cast<float>(sk[i]));
            s += r * r;
          }
        }
        s = wave_sum(s);
        if (lane == 0) s_inv[m] = 1.f / sqrtf(s / static_cast<float>(K) + L.eps);
      }
      __syncthreads();
    }
  }

  // stage the activations (normalised for Qkv/Mlp) in pair order
  for (int64_t idx = tid; idx < static_cast<int64_t>(M) * groups; idx += NT) {
    const int m = static_cast<int>(idx / groups);
    const int64_t k = (idx - static_cast<int64_t>(m) * groups) * 8;
    f16x8 v = {};
    if (k < K) {
      v = __builtin_bit_cast(f16x8, ld16(static_cast<const f16*>(L.A) + m * K + k));
      if constexpr (OP != OP_MATMUL) {
        f16x8 sk = {};
        if (L.skip) sk = __builtin_bit_cast(f16x8, ld16(static_cast<const f16*>(L.skip) + m * K + k));
        float r[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = __fadd_rn(static_cast<float>(v[i]), static_cast<float>(sk[i]));
        if (L.residual && blockIdx.x == 0) {
          f16x8 rr;
#pragma unroll
          for (int i = 0; i < 8; ++i) rr[i] = static_cast<f16>(r[i]);
          *reinterpret_cast<f16x8*>(static_cast<f16*>(L.residual) + m * K + k) = rr;
        }
        if (L.gamma) {
          const f16x8 g = __builtin_bit_cast(f16x8, ld16(static_cast<const f16*>(L.gamma) + k));
          const float inv = s_inv[m];
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = static_cast<f16>(r[i] * (inv * static_cast<float>(g[i])));
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = static_cast<f16>(r[i]);
        }
      }
    }
    *reinterpret_cast<f16x8*>(As + m * ldA + k) = pair_order(v);
  }
  __syncthreads();

  // main loop: lane (c, g) streams column n0 + c, chunk 8s + 4h + g
  const int c = lane & 15, g = lane >> 4;
  const int64_t n = n0 + c;
  const bool nval = n < P.N;
  const int64_t row_bytes = L.kb * L.blob;
  const int64_t nchunk = row_bytes >> 4;
  const uint8_t* Brow = P.B + (nval ? n : 0) * row_bytes;
  const uint8_t* Urow = nullptr;
  if constexpr (OP == OP_MLP) Urow = L.p[1].B + (nval ? n : 0) * row_bytes;
  const bool aval = c < M;
  const f16* Arow = As + c * ldA;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
  const int64_t steps = (nchunk + 7) / 8;

  u32x4 wb[2], wu[2];
  auto load_step = [&](int64_t s) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t ch = s * 8 + h * 4 + g;
      const bool ok = nval && ch < nchunk;
      wb[h] = ok ? ld16(Brow + ch * 16) : u32x4{0u, 0u, 0u, 0u};
      if constexpr (OP == OP_MLP) wu[h] = ok ? ld16(Urow + ch * 16) : u32x4{0u, 0u, 0u, 0u};
    }
  };

  int64_t s = wave;
  if (s < steps) load_step(s);
  for (; s < steps; s += GEMV_WAVES) {
    u32x4 cb[2] = {wb[0], wb[1]}, cu[2];
    if constexpr (OP == OP_MLP) {
      cu[0] = wu[0];
      cu[1] = wu[1];
    }
    if (s + GEMV_WAVES < steps) load_step(s + GEMV_WAVES);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t ch = s * 8 + h * 4 + g;
      const bool cval = ch < nchunk;
      f16x8 b[4];
      dq_chunk<ZPK, SPC>(L, P, n, ch, nval && cval, cb[h], b);
      f16x8 a[4];
#pragma unroll
      for (int d = 0; d < 4; ++d)
        a[d] = (aval && cval) ? *reinterpret_cast<const f16x8*>(Arow + ch * 32 + d * 8) : f16x8{};
#pragma unroll
      for (int d = 0; d < 4; ++d) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[d], b[d], acc, 0, 0, 0);
      if constexpr (OP == OP_MLP) {
        f16x8 u[4];
        dq_chunk<ZPK, SPC>(L, L.p[1], n, ch, nval && cval, cu[h], u);
#pragma unroll
        for (int d = 0; d < 4; ++d) acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[d], u[d], acc2, 0, 0, 0);
      }
    }
  }

  // reduce the waves' partial sums through LDS
  __syncthreads();
  constexpr int NACC = OP == OP_MLP ? 8 : 4;
  if (wave > 0) {
    float* dst = red + ((wave - 1) * 64 + lane) * NACC;
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[r] = acc[r];
    if constexpr (OP == OP_MLP) {
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[4 + r] = acc2[r];
    }
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < GEMV_WAVES; ++w) {
    const float* src = red + ((w - 1) * 64 + lane) * NACC;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] += src[r];
    if constexpr (OP == OP_MLP) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc2[r] += src[4 + r];
    }
  }
  if (!nval) return;
  // lane (c, g) holds rows 4g..4g+3 of column n
  float bias = 0.f, ubias = 0.f;
  if constexpr (OP == OP_MATMUL) {
    if (P.bias) bias = static_cast<float>(static_cast<const f16*>(P.bias)[n]);
  }
  if constexpr (OP == OP_MLP) {
    if (P.bias) bias = static_cast<float>(static_cast<const f16*>(P.bias)[n]);
    if (L.p[1].bias) ubias = static_cast<float>(static_cast<const f16*>(L.p[1].bias)[n]);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * g + r;
    if (m < M) {
      float y = acc[r] + bias;
      if constexpr (OP == OP_MLP) y = activate(y, L.act) * (acc2[r] + ubias);
      static_cast<f16*>(P.Y)[static_cast<int64_t>(m) * P.N + n] = static_cast<f16>(y);
    }
  }
}

// ---------------------------------------------------------------------------
// GEMM for M > 16: fp16 activations, 4-bit weights, MFMA 32x32x16

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64, GM_LDK = GM_BK + 8;

template <int ZPK, int SPC>
__global__ __launch_bounds__(256) void k_gemm_q4(Launch L) {
  __shared__ __align__(16) f16 As[GM_BM * GM_LDK];
  __shared__ __align__(16) f16 Bs[GM_BN * GM_LDK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const Proj& P = L.p[0];
  const int64_t M = L.M, N = P.N, K = L.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * GM_BM, n0 = static_cast<int64_t>(blockIdx.x) * GM_BN;
  const int64_t Kp = L.kb * L.block_size;
  const int64_t row_bytes = Kp / 2, nchunk = row_bytes / 16;
  const int64_t ktiles = (Kp + GM_BK - 1) / GM_BK;
  const f16* A = static_cast<const f16*>(L.A);

  // global -> register staging
  f16x8 ra[4];
  u32x4 rb;
  const int bcol = tid >> 1, bh = tid & 1;
  const int64_t bn = n0 + bcol;
  const bool bnval = bn < N;
  const uint8_t* Bcol = P.B + (bnval ? bn : 0) * row_bytes;

  auto gload = [&](int64_t kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i, row = idx >> 3, grp = idx & 7;
      const int64_t m = m0 + row, k = kt * GM_BK + grp * 8;
      ra[i] = (m < M && k < K) ? __builtin_bit_cast(f16x8, ld16(A + m * K + k)) : f16x8{};
    }
    const int64_t ch = kt * 2 + bh;
    rb = (bnval && ch < nchunk) ? ld16(Bcol + ch * 16) : u32x4{0u, 0u, 0u, 0u};
  };
  auto sstore = [&](int64_t kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i, row = idx >> 3, grp = idx & 7;
      *reinterpret_cast<f16x8*>(As + row * GM_LDK + grp * 8) = pair_order(ra[i]);
    }
    const int64_t ch = kt * 2 + bh;
    f16x8 b[4];
    dq_chunk<ZPK, SPC>(L, P, bn, ch, bnval && ch < nchunk, rb, b);
#pragma unroll
    for (int d = 0; d < 4; ++d) *reinterpret_cast<f16x8*>(Bs + bcol * GM_LDK + bh * 32 + d * 8) = b[d];
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  gload(0);
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    __syncthreads();
    sstore(kt);
    __syncthreads();
    if (kt + 1 < ktiles) gload(kt + 1);
#pragma unroll
    for (int kk = 0; kk < GM_BK / 16; ++kk) {
      f16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const f16x8*>(As + (wm * 64 + i * 32 + (lane & 31)) * GM_LDK + kk * 16 + (lane >> 5) * 8);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const f16x8*>(Bs + (wn * 64 + j * 32 + (lane & 31)) * GM_LDK + kk * 16 + (lane >> 5) * 8);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each 32x32 tile
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
    if (n >= N) continue;
    const float bias = P.bias ? static_cast<float>(static_cast<const f16*>(P.bias)[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < M) static_cast<f16*>(P.Y)[m * N + n] = static_cast<f16>(acc[i][j][r] + bias);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dequantisation kernel (xrmm_dequantize)

template <int ZPK, int SPC>
__global__ __launch_bounds__(256) void k_dequant_q4_f16(Launch L, f16* W) {
  // one thread per 16-byte chunk: 32 codes of one column
  const Proj& P = L.p[0];
  const int64_t row_bytes = L.kb * L.blob, nchunk = row_bytes / 16;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= P.N * nchunk) return;
  const int64_t n = gid / nchunk, ch = gid - n * nchunk;
  const u32x4 w = ld16(P.B + n * row_bytes + ch * 16);
  f16x8 b[4];
  dq_chunk<ZPK, SPC>(L, P, n, ch, true, w, b);
  const int order[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
  for (int d = 0; d < 4; ++d)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = ch * 32 + d * 8 + order[i];
      if (k < L.K) W[n * L.K + k] = b[d][i];
    }
}

__global__ __launch_bounds__(256) void k_dequant_f32(Launch L, void* W, int out_dtype) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= L.p[0].N * L.K) return;
  const int64_t n = gid / L.K, k = gid - n * L.K;
  st_t(W, gid, weight_f32(L, L.p[0], n, k), out_dtype);
}

// ---------------------------------------------------------------------------
// dispatch

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int spc_of(int block_size) { return block_size % 32 == 0 ? 1 : 2; }

// fp16, 4-bit, blocks of whole 16-code halves, rows of whole 16-byte chunks,
// K a multiple of 8 and 16-byte aligned tensors.
static bool q4_fast_ok(const Launch& L) {
  if (L.dtype != DT_F16 || L.bits != 4) return false;
  if (L.block_size % 16 != 0) return false;
  const int64_t Kp = L.kb * L.block_size;
  if (Kp % 32 != 0 || L.K % 8 != 0) return false;
  if (!aligned16(L.A) || !aligned16(L.skip) || !aligned16(L.gamma) || !aligned16(L.residual)) return false;
  for (int i = 0; i < L.nproj; ++i) {
    if (!aligned16(L.p[i].B)) return false;
    if (L.zp_kind == ZP_FLOAT && L.p[i].zp == nullptr) return false;
  }
  return true;
}

static int64_t gemv_lds_bytes(const Launch& L) {
  const int64_t a = L.M * (L.kb * L.block_size + 8) * 2;
  const int64_t r = (GEMV_WAVES - 1) * 64 * (L.op == OP_MLP ? 8 : 4) * 4;
  return a > r ? a : r;
}

constexpr int64_t kMaxLds = 160 * 1024 - 1024;

Kernel select_kernel(const Launch& L) {
  if (q4_fast_ok(L)) {
    if (L.M >= 1 && L.M <= 16 && gemv_lds_bytes(L) <= kMaxLds) return K_GEMV_Q4;
    if (L.M > 16 && L.op == OP_MATMUL && L.zp_kind != ZP_FLOAT) return K_GEMM_Q4;
  }
  return K_GENERIC;
}

const char* kernel_name(Kernel k) {
  switch (k) {
    case K_GEMV_Q4: return "gemv_q4_mfma";
    case K_GEMM_Q4: return "gemm_q4_mfma";
    default: return "generic";
  }
}

template <int ZPK, int SPC, int OP>
static hipError_t launch_gemv3(const Launch& L, hipStream_t st) {
  const int64_t tiles = (L.p[0].N + 15) / 16 + (OP == OP_QKV ? (L.p[1].N + 15) / 16 + (L.p[2].N + 15) / 16 : 0);
  const int64_t lds = gemv_lds_bytes(L);
  auto kern = k_gemv_q4<ZPK, SPC, OP>;
  if (lds > 64 * 1024) {
    static bool raised = false;  // per instantiation
    if (!raised) {
      // Raises the dynamic-LDS cap where the runtime keeps one; an error here
      // surfaces from the launch itself if the size is really unsupported.
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(kMaxLds));
      (void)hipGetLastError();
      raised = true;
    }
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(tiles)), dim3(GEMV_WAVES * 64), static_cast<size_t>(lds), st, L);
  return hipGetLastError();
}

template <int ZPK, int SPC>
static hipError_t launch_gemv2(const Launch& L, hipStream_t st) {
  switch (L.op) {
    case OP_QKV: return launch_gemv3<ZPK, SPC, OP_QKV>(L, st);
    case OP_MLP: return launch_gemv3<ZPK, SPC, OP_MLP>(L, st);
    default: return launch_gemv3<ZPK, SPC, OP_MATMUL>(L, st);
  }
}

template <int ZPK>
static hipError_t launch_gemv1(const Launch& L, hipStream_t st) {
  return spc_of(L.block_size) == 1 ? launch_gemv2<ZPK, 1>(L, st) : launch_gemv2<ZPK, 2>(L, st);
}

template <int ZPK, int SPC>
static hipError_t launch_gemm2(const Launch& L, hipStream_t st) {
  const dim3 grid(static_cast<uint32_t>((L.p[0].N + GM_BN - 1) / GM_BN), static_cast<uint32_t>((L.M + GM_BM - 1) / GM_BM));
  hipLaunchKernelGGL((k_gemm_q4<ZPK, SPC>), grid, dim3(256), 0, st, L);
  return hipGetLastError();
}

template <int ZPK>
static hipError_t launch_gemm1(const Launch& L, hipStream_t st) {
  return spc_of(L.block_size) == 1 ? launch_gemm2<ZPK, 1>(L, st) : launch_gemm2<ZPK, 2>(L, st);
}

static int effective_zpk(const Launch& L) {
  // a zero-point kind applies only when every projection carries zero points
  if (L.zp_kind == ZP_NONE) return ZP_NONE;
  for (int i = 0; i < L.nproj; ++i)
    if (!L.p[i].zp) return -1;
  return L.zp_kind;
}

hipError_t launch(const Launch& L, hipStream_t st) {
  if (L.M == 0) return hipSuccess;
  Kernel k = select_kernel(L);
  const int zpk = effective_zpk(L);
  if (zpk < 0) k = K_GENERIC;  // mixed presence of zero points
  if (k == K_GEMV_Q4) {
    if (zpk == ZP_NONE) return launch_gemv1<ZP_NONE>(L, st);
    if (zpk == ZP_PACKED) return launch_gemv1<ZP_PACKED>(L, st);
    return launch_gemv1<ZP_FLOAT>(L, st);
  }
  if (k == K_GEMM_Q4) {
    if (zpk == ZP_NONE) return launch_gemm1<ZP_NONE>(L, st);
    return launch_gemm1<ZP_PACKED>(L, st);
  }
  int64_t cols = L.p[0].N;
  if (L.op == OP_QKV) cols += L.p[1].N + L.p[2].N;
  constexpr int MB = 8;
  const dim3 grid(static_cast<uint32_t>(cols), static_cast<uint32_t>((L.M + MB - 1) / MB));
  hipLaunchKernelGGL(k_generic<MB>, grid, dim3(64), 0, st, L);
  return hipGetLastError();
}

hipError_t launch_dequantize(const Launch& L, void* W, int out_dtype, hipStream_t st) {
  const Proj& P = L.p[0];
  if (P.N == 0 || L.K == 0) return hipSuccess;
  if (out_dtype == DT_F16 && L.bits == 4 && L.dtype == DT_F16 && L.block_size % 16 == 0 &&
      (L.kb * L.block_size) % 32 == 0 && aligned16(P.B)) {
    const int64_t n = P.N * (L.kb * L.blob / 16);
    const dim3 grid(static_cast<uint32_t>((n + 255) / 256));
    const int spc = spc_of(L.block_size);
    const int zpk = P.zp ? L.zp_kind : ZP_NONE;
    f16* out = static_cast<f16*>(W);
#define XRMM_DQ(Z, S) hipLaunchKernelGGL((k_dequant_q4_f16<Z, S>), grid, dim3(256), 0, st, L, out)
    if (zpk == ZP_NONE) {
      if (spc == 1) XRMM_DQ(ZP_NONE, 1); else XRMM_DQ(ZP_NONE, 2);
    } else if (zpk == ZP_PACKED) {
      if (spc == 1) XRMM_DQ(ZP_PACKED, 1); else XRMM_DQ(ZP_PACKED, 2);
    } else {
      if (spc == 1) XRMM_DQ(ZP_FLOAT, 1); else XRMM_DQ(ZP_FLOAT, 2);
    }
#undef XRMM_DQ
    return hipGetLastError();
  }
  const int64_t n = P.N * L.K;
  hipLaunchKernelGGL(k_dequant_f32, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, st, L, W, out_dtype);
  return hipGetLastError();
}

}  // namespace xrmm
