// Device-side building blocks shared by the kernels of libxrmm: vector types,
// storage conversions, the reference weight formula and the 4-bit
// dequantisation to binary16.
#pragma once
#include "xrmm_internal.h"

namespace xrmm {


typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

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

// Wave sums of eight per-lane values in 10 exchanges instead of 48: each
// exchange over lane bit 5, 4 and 3 halves the values a lane keeps, then
// bits 2..0 finish the sum. Lane l returns the sum of value
// row8(l) = 4*bit3 + 2*bit4 + bit5.
__device__ __forceinline__ int row8(int lane) { return ((lane >> 3) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 5) & 1); }

__device__ __forceinline__ float reduce8(const float (&v)[8], int lane) {
  float a4[4], a2[2];
  const bool h5 = (lane & 32) != 0, h4 = (lane & 16) != 0, h3 = (lane & 8) != 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) a4[i] = (h5 ? v[2 * i + 1] : v[2 * i]) + __shfl_xor(h5 ? v[2 * i] : v[2 * i + 1], 32, 64);
#pragma unroll
  for (int i = 0; i < 2; ++i) a2[i] = (h4 ? a4[2 * i + 1] : a4[2 * i]) + __shfl_xor(h4 ? a4[2 * i] : a4[2 * i + 1], 16, 64);
  float a1 = (h3 ? a2[1] : a2[0]) + __shfl_xor(h3 ? a2[0] : a2[1], 8, 64);
  a1 += __shfl_xor(a1, 4, 64);
  a1 += __shfl_xor(a1, 2, 64);
  return a1 + __shfl_xor(a1, 1, 64);
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

// (x & mask) | bits in one VOP3 instruction. gfx9 VOP3 encodings take no
// literal and at most one scalar operand, so the mask lives in an SGPR and the
// OR-ed exponent bits in a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(bits));
  return r;
}

__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// Eight low-first codes of one dword -> (code - z) * scale, in the order
// [c0, c4, c1, c5, c2, c6, c3, c7]. The activations are staged in the same
// order, so the dot product is unchanged. 13 VALU instructions.
__device__ __forceinline__ f16x8 dq8(uint32_t x, const Dq& c) {
  const uint32_t magic = 0x64006400u;  // 1024.0h in both halves
  const uint32_t x8 = x >> 8;
  const f16x2 inv16 = {static_cast<f16>(0.0625f), static_cast<f16>(0.0625f)};
  // 1024 + c - (1024 + z) and (1024 + 16c)/16 - (64 + z): both exact
  const f16x2 d0 = (as_h2(and_or(x, 0x000F000Fu, magic)) + c.nz1024) * c.s;
  const f16x2 d1 = __builtin_elementwise_fma(as_h2(and_or(x, 0x00F000F0u, magic)), inv16, c.nz64) * c.s;
  const f16x2 d2 = (as_h2(and_or(x8, 0x000F000Fu, magic)) + c.nz1024) * c.s;
  const f16x2 d3 = __builtin_elementwise_fma(as_h2(and_or(x8, 0x00F000F0u, magic)), inv16, c.nz64) * c.s;
  return __builtin_bit_cast(f16x8, u32x4{as_u32(d0), as_u32(d1), as_u32(d2), as_u32(d3)});
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

// Per-chunk metadata of a 16-byte chunk (32 codes) of column n starting at
// code 32*ch: the scale and zero point of each block the chunk touches.
// SPC = 1 when the chunk lies in one block (block_size % 32 == 0), 2 when each
// 16-code half lies in one block (block_size == 16). Block sizes on the fast
// path are powers of two, so the block index is a shift.
template <int SPC>
struct Meta {
  f16 s[SPC];
  float z[SPC];
};

template <int ZPK, int SPC>
__device__ __forceinline__ Meta<SPC> ld_meta(const Launch& L, const Proj& P, int64_t n, int64_t ch, bool valid) {
  Meta<SPC> m;
#pragma unroll
  for (int half = 0; half < SPC; ++half) {
    const int64_t b = (ch * 32 + half * 16) >> L.bs_log2;
    m.s[half] = static_cast<f16>(0.f);
    m.z[half] = 8.f;
    if (valid) {
      m.s[half] = static_cast<const f16*>(P.scales)[n * L.kb + b];
      m.z[half] = zp_fast<ZPK>(L, P, n, b);
    }
  }
  return m;
}

// The same metadata as raw bits, loaded together with a chunk's weights so
// that the loads of a pipeline stage are all in flight at once (ld_meta's
// conversion would make the load's first use follow it immediately):
// binary16 scale bits, and the zero point's raw bits (packed: the byte;
// float: binary16 or float32 bits). Converted by meta_of when consumed.
template <int SPC>
struct RawMeta {
  uint32_t s[SPC];
  uint32_t z[SPC];
};

template <int ZPK, int SPC>
__device__ __forceinline__ RawMeta<SPC> ld_meta_raw(const Launch& L, const Proj& P, int64_t n, int64_t ch, bool valid) {
  RawMeta<SPC> r;
#pragma unroll
  for (int half = 0; half < SPC; ++half) {
    const int64_t b = (ch * 32 + half * 16) >> L.bs_log2;
    r.s[half] = 0u;
    r.z[half] = 0u;
    if (valid) {
      r.s[half] = static_cast<const uint16_t*>(P.scales)[n * L.kb + b];
      if constexpr (ZPK == ZP_PACKED)
        r.z[half] = static_cast<const uint8_t*>(P.zp)[n * L.zrow + (b >> 1)];
      else if constexpr (ZPK == ZP_FLOAT)
        r.z[half] = L.zp_dtype == DT_F32 ? static_cast<const uint32_t*>(P.zp)[n * L.kb + b]
                                         : static_cast<const uint16_t*>(P.zp)[n * L.kb + b];
    }
  }
  return r;
}

template <int ZPK, int SPC>
__device__ __forceinline__ Meta<SPC> meta_of(const Launch& L, const RawMeta<SPC>& r, int64_t ch, bool valid) {
  Meta<SPC> m;
#pragma unroll
  for (int half = 0; half < SPC; ++half) {
    const int64_t b = (ch * 32 + half * 16) >> L.bs_log2;
    m.s[half] = __builtin_bit_cast(f16, static_cast<uint16_t>(r.s[half]));
    float z = 8.f;
    if constexpr (ZPK == ZP_PACKED)
      z = static_cast<float>((r.z[half] >> ((b & 1) * 4)) & 15u);
    else if constexpr (ZPK == ZP_FLOAT)
      z = L.zp_dtype == DT_F32 ? __builtin_bit_cast(float, r.z[half])
                               : static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(r.z[half])));
    m.z[half] = valid ? z : 8.f;
  }
  return m;
}

// Dequantise the chunk's four dwords with its metadata (pair order per dword).
template <int ZPK, int SPC>
__device__ __forceinline__ void dq_regs(u32x4 w, const Meta<SPC>& m, f16x8 out[4]) {
#pragma unroll
  for (int half = 0; half < SPC; ++half) {
    if constexpr (ZPK == ZP_FLOAT) {
      const float sf = static_cast<float>(m.s[half]);
#pragma unroll
      for (int d = half * (4 / SPC); d < (half + 1) * (4 / SPC); ++d) out[d] = dq8_f32z(w[d], m.z[half], sf);
    } else {
      const Dq c = dq_consts(m.z[half], m.s[half]);
#pragma unroll
      for (int d = half * (4 / SPC); d < (half + 1) * (4 / SPC); ++d) out[d] = dq8(w[d], c);
    }
  }
}

template <int ZPK, int SPC>
__device__ __forceinline__ void dq_chunk(const Launch& L, const Proj& P, int64_t n, int64_t ch,
                                         bool valid, u32x4 w, f16x8 out[4]) {
  dq_regs<ZPK, SPC>(w, ld_meta<ZPK, SPC>(L, P, n, ch, valid), out);
}

// Raw buffer resources: loads through them are bounds-checked by the hardware
// (an offset at or beyond `bytes` reads as zero), and the per-lane offset is a
// 32-bit VGPR plus a wave-uniform SGPR, so streaming loads need no per-load
// address arithmetic. 0x00020000 is the gfx9 raw-buffer format word.
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t mk_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ u32x4 bld16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), 0));
}

// Streaming variants for data read exactly once (weights, scales): the
// non-temporal cache policy (aux = 2, "nt") keeps them from displacing
// reused lines.
#ifndef XRMM_WAUX
#define XRMM_WAUX 2
#endif
__device__ __forceinline__ u32x4 bld16_nt(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), XRMM_WAUX));
}

__device__ __forceinline__ uint32_t bld_u16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}

__device__ __forceinline__ uint32_t bld_u8(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}

__device__ __forceinline__ uint32_t bld_u32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}

__device__ __forceinline__ u32x2 bld8(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(voff), static_cast<int>(soff), 0));
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *static_cast<const u32x4*>(p);
}

// Logical index of workgroup b on a grid of n. The dispatcher hands
// consecutive workgroups to consecutive XCDs (eight on gfx950, each with its
// own L2), so the first 8 floor(n / 8) workgroups are renumbered to make XCD
// b % 8 walk the contiguous range (b % 8) * (n / 8) ... of the logical order;
// the remainder keeps its index. Output lines then fill inside one XCD's L2
// instead of collecting partial writes from all eight.
__device__ __forceinline__ uint32_t xcd_slot(uint32_t b, uint32_t n) {
  const uint32_t per = n >> 3;
  return b < (per << 3) ? (b & 7u) * per + (b >> 3) : b;
}

}  // namespace xrmm
