// com.microsoft.QMoE (opcode 1030) on gfx950: top-k routing, expert FC1 with
// its activation, expert FC2 with the routing-weighted combine.
//
// Semantics (kernels/_shared/extended/shaders/complex_kernel.glsl:158-160,
// planned by kernels/_shared/extended/complex_plan.cpp:121-128): float32
// activations, uint8-packed expert weights with codes low-first in a byte and
// the midpoint zero point 2^(bits-1), float32 scales per row (block_size 0) or
// per block of a row; an expert's rank counts the experts with a larger logit
// or an equal logit and a larger index; the softmax runs over the k selected
// experts only; FC1 rows 2j / 2j + 1 are gate / linear for SwiGLU (fusion 1),
// row j for ReLU; experts are combined in ascending index order.
//
// Geometries with 16-byte rows (every practical one) take two launches on the
// caller's stream:
//  1. k_moe_gemv FC1: one workgroup per (token, slot) pair and tile of 64
//     FC1 rows. It routes the token itself (the rank rule above, softmax over
//     the selected logits), stages x in LDS and streams the selected expert's
//     rows with 16-byte loads per lane, the next unit's weights and scales in
//     flight while the current one is computed; the activation runs in the
//     epilogue; h [T, k, I] float32 goes to the workspace.
//  2. k_moe_gemv FC2: the same loop over each pair's FC2 rows against h,
//     partial outputs per slot; the last workgroup of a (token, tile) to
//     arrive sums the k partials with the routing weights in slot order.
// Codes become (code - midpoint) exactly in binary16 (magic-number
// construction) and multiply into float32 sums with v_fma_mix_f32; a scale
// multiplies the sum of its block (or the row's total for row scales). Other
// geometries take a routing kernel and one-thread-per-output kernels.
#include <algorithm>

#include "xrmm_device.h"
#include "xrmm_moe.h"

namespace xrmm {

namespace {

constexpr int MOE_T = 256;  // threads per workgroup: 4 waves

// ---------------------------------------------------------------------------
// routing

__global__ __launch_bounds__(MOE_T) void k_moe_route(const float* __restrict__ router, int32_t* __restrict__ sel,
                                                     float* __restrict__ wts, int T, int E, int k) {
  const int t = blockIdx.x * (MOE_T / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;  // whole waves
  const float* l = router + static_cast<int64_t>(t) * E;
  auto rank_of = [&](int e, float v) {
    int r = 0;
    for (int e2 = 0; e2 < E; ++e2) {
      const float o = l[e2];
      r += (o > v || (o == v && e2 > e)) ? 1 : 0;
    }
    return r;
  };
  float mx = -__builtin_huge_valf();
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    if (e < E) {
      const float v = l[e];
      if (rank_of(e, v) < k) mx = fmaxf(mx, v);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float den = 0.f;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    if (e < E) {
      const float v = l[e];
      if (rank_of(e, v) < k) den += expf(v - mx);
    }
  }
  den = wave_sum(den);
  int base = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    bool s = false;
    float v = 0.f;
    if (e < E) {
      v = l[e];
      s = rank_of(e, v) < k;
    }
    const uint64_t m = __ballot(s);
    if (s) {
      // NaN logits rank 0 and can push the count past k: extra experts are
      // dropped rather than written past the slot array
      const int slot = base + __popcll(m & ((uint64_t(1) << lane) - 1));
      if (slot < k) sel[static_cast<int64_t>(t) * k + slot] = e;
      if (slot < k)
        wts[static_cast<int64_t>(t) * k + slot] = expf(v - mx) / den;
    }
    base += __popcll(m);
  }
}

// ---------------------------------------------------------------------------
// row-group GEMV over packed expert rows

enum Stage { ST_FC1_RELU = 0, ST_FC1_SWIGLU = 1, ST_FC2 = 2 };
enum ScaleMode { SM_ROW = 0, SM_CHUNK = 1, SM_HALF = 2 };  // scales per row / per 16-byte chunk / per 8-byte half

constexpr int MOE_RPW = 8;     // rows of one group: loaded together, reduced together
constexpr int MOE_MAX_K = 64;  // slots of one token in the fused routing

__device__ __forceinline__ float swiglu(float gate, float lin, const MoeArgs& a) {
  if (a.has_limit) {
    gate = fminf(gate, a.limit);
    lin = fminf(fmaxf(lin, -a.limit), a.limit);
  }
  const float z = a.alpha * gate;
  const float lg = z >= 0.f ? 1.f / (1.f + expf(-z)) : expf(z) / (1.f + expf(z));
  return gate * lg * (lin + a.beta);
}

// The codes of one dword minus the midpoint, as exact binary16 pairs
// (0x6400 | c is 1024 + c and 0x6400 | (c << 4) is 1024 + 16c, so one
// subtraction or one multiply-add by 1/16 leaves c - mid), each multiplied
// into the float32 sum against its activation (binary16 -> float32 is exact;
// the compiler fuses the conversion into v_fma_mix_f32). 4-bit pairs:
// (c0,c4) (c1,c5) (c2,c6) (c3,c7); 8-bit pairs: (c0,c2) (c1,c3).
template <int BITS>
__device__ __forceinline__ float dword_dot(uint32_t w, const float* x, float acc) {
  const uint32_t magic = 0x64006400u;
  if constexpr (BITS == 4) {
    const f16x2 n1032 = {static_cast<f16>(-1032.f), static_cast<f16>(-1032.f)};
    const f16x2 inv16 = {static_cast<f16>(0.0625f), static_cast<f16>(0.0625f)};
    const f16x2 n72 = {static_cast<f16>(-72.f), static_cast<f16>(-72.f)};
    const uint32_t w8 = w >> 8;
    const f16x2 d0 = as_h2(and_or(w, 0x000F000Fu, magic)) + n1032;
    const f16x2 d1 = __builtin_elementwise_fma(as_h2(and_or(w, 0x00F000F0u, magic)), inv16, n72);
    const f16x2 d2 = as_h2(and_or(w8, 0x000F000Fu, magic)) + n1032;
    const f16x2 d3 = __builtin_elementwise_fma(as_h2(and_or(w8, 0x00F000F0u, magic)), inv16, n72);
    acc = __builtin_fmaf(static_cast<float>(d0[0]), x[0], acc);
    acc = __builtin_fmaf(static_cast<float>(d1[0]), x[1], acc);
    acc = __builtin_fmaf(static_cast<float>(d2[0]), x[2], acc);
    acc = __builtin_fmaf(static_cast<float>(d3[0]), x[3], acc);
    acc = __builtin_fmaf(static_cast<float>(d0[1]), x[4], acc);
    acc = __builtin_fmaf(static_cast<float>(d1[1]), x[5], acc);
    acc = __builtin_fmaf(static_cast<float>(d2[1]), x[6], acc);
    return __builtin_fmaf(static_cast<float>(d3[1]), x[7], acc);
  } else {
    const f16x2 n1152 = {static_cast<f16>(-1152.f), static_cast<f16>(-1152.f)};
    const f16x2 d0 = as_h2(and_or(w, 0x00FF00FFu, magic)) + n1152;
    const f16x2 d1 = as_h2(and_or(w >> 8, 0x00FF00FFu, magic)) + n1152;
    acc = __builtin_fmaf(static_cast<float>(d0[0]), x[0], acc);
    acc = __builtin_fmaf(static_cast<float>(d1[0]), x[1], acc);
    acc = __builtin_fmaf(static_cast<float>(d0[1]), x[2], acc);
    return __builtin_fmaf(static_cast<float>(d1[1]), x[3], acc);
  }
}

}  // namespace
}  // namespace xrmm
#include "xrmm_moe_gemm.h"
namespace xrmm {
namespace {

__device__ __forceinline__ float bld_f32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, bld_u32(r, voff, soff));
}

// LDS layout of an activation vector: the CPC floats of 16-byte chunk c sit
// at c * (CPC + 4), so the 64 lanes of a wave reading their own chunks with
// 16-byte reads hit disjoint banks in every group of 16 lanes.
template <int CPC>
__device__ __forceinline__ int64_t lds_index(int64_t i) {
  return (i / CPC) * (CPC + 4) + (i % CPC);
}

// Copies n floats (a multiple of 4, 16-byte aligned) into LDS in the chunk
// layout above, zero-filled up to kpad (a multiple of 1024): float4 loads,
// four per thread in flight before their stores.
template <int CPC>
__device__ __forceinline__ void stage_vec(float* dst, const float* __restrict__ src, int64_t n, int64_t kpad) {
  const int tid = threadIdx.x;
  for (int64_t base = 0; base < kpad; base += 16 * MOE_T) {
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = base + (static_cast<int64_t>(j) * MOE_T + tid) * 4;
      v[j] = i < n ? *reinterpret_cast<const float4*>(src + i) : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = base + (static_cast<int64_t>(j) * MOE_T + tid) * 4;
      if (i < kpad) *reinterpret_cast<float4*>(dst + lds_index<CPC>(i)) = v[j];
    }
  }
}

// Routing of one token inside the FC1 prologue (complex_kernel.glsl:159-160):
// an expert's rank counts the experts with a larger logit, or an equal logit
// and a larger index; the experts of rank < k, in ascending index order, fill
// the slots; the weights are the softmax over the selected logits, maximum and
// denominator taken in ascending index order. Every thread of the workgroup
// calls it; `lr` holds the token's E logits in LDS, `fl` (E ints) and `sl`
// (MOE_MAX_K ints) are LDS scratch. The slot's expert and weight come back
// through `out_e` / `out_w` (LDS) after the final barrier.
__device__ void route_slot(int E, int k, int slot, const float* lr, int* fl, int* sl, int* out_e, float* out_w) {
  const int tid = threadIdx.x, lane = tid & 63;
  for (int e = tid; e < E; e += MOE_T) {
    const float v = lr[e];
    int rank = 0;
    for (int e2 = 0; e2 < E; ++e2) {
      const float o = lr[e2];
      rank += (o > v || (o == v && e2 > e)) ? 1 : 0;
    }
    fl[e] = rank < k ? 1 : 0;
  }
  __syncthreads();
  if (tid < 64) {
    // NaN logits rank 0 and can push the count past k: slots past k are dropped
    int base = 0;
    for (int e0 = 0; e0 < E && base < k; e0 += 64) {
      const int e = e0 + lane;
      const bool s = e < E && fl[e] != 0;
      const uint64_t m = __ballot(s);
      const int pos = base + __popcll(m & ((uint64_t(1) << lane) - 1));
      if (s && pos < k) sl[pos] = e;
      base += __popcll(m);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (tid == 0) {
      float mx = -__builtin_huge_valf();
      for (int s = 0; s < k; ++s) mx = fmaxf(mx, lr[sl[s]]);
      float den = 0.f;
      for (int s = 0; s < k; ++s) den += expf(lr[sl[s]] - mx);
      *out_e = sl[slot];
      *out_w = expf(lr[sl[slot]] - mx) / den;
    }
  }
  __syncthreads();
}

// One expert matrix (FC1 or FC2) against the activation vector of each
// (token, slot) pair. Workgroup b covers pair, row tile and reduction segment
// (b / (tiles * a.ks), (b / a.ks) % tiles, b % a.ks): rows
// [tile * 32 * gpw, +32 * gpw), steps [kseg * a.seg, +a.seg) of 64
// sixteen-byte chunks. Each of its 4 waves owns gpw groups of 8 consecutive
// rows; a unit of work is one group over one step (one chunk per lane), and
// the loads of unit u + 1 (weights and their scales) are in flight while unit
// u is computed. Rows and chunks past the end load through out-of-range
// buffer offsets, which read zero and touch no memory.
//
// FC1 (ST_FC1_*, one segment): routes the pair's token, stages x in LDS,
// writes the activated outputs h[pair] (SwiGLU rows 2j / 2j+1 fall in one
// group) and clears the FC2 arrival counters. FC2: stages its segment of
// h[pair] and writes a partial output per (slot, segment); the last of the
// k * a.ks workgroups of a (token, row tile) to arrive sums the partials
// (segments, then slots with their routing weights) in a fixed order, so the
// result does not depend on scheduling. With k = 1 and one segment FC2
// writes the output directly.
#ifndef XRMM_MOE_FC1_WGS
#define XRMM_MOE_FC1_WGS 1024  // FC1 workgroups to aim at: four resident per CU
#endif
#ifndef XRMM_MOE_FC2_WGS
#define XRMM_MOE_FC2_WGS 1024  // FC2 workgroups to aim at through reduction segments
#endif

template <int BITS, int SM, int ST>
__global__ __launch_bounds__(MOE_T) void k_moe_gemv(MoeArgs a, int gpw, int tiles, int tiles2) {
  extern __shared__ __align__(16) float xs[];
  __shared__ int s_e, s_last;
  __shared__ float s_w;
  constexpr int RPW = MOE_RPW;
  constexpr int CPC = 128 / BITS;  // codes per 16-byte chunk
  constexpr int CPD = 32 / BITS;   // codes per dword
  constexpr int NS = SM == SM_HALF ? 2 : 1;
  constexpr bool fc2 = ST == ST_FC2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ks = fc2 ? a.ks : 1;
  const int64_t pair = blockIdx.x / (static_cast<uint32_t>(tiles) * ks);
  const int tile = static_cast<int>((blockIdx.x / ks) % tiles);
  const int kseg = static_cast<int>(blockIdx.x % ks);
  const int64_t t = pair / a.k;
  const int slot = static_cast<int>(pair % a.k);
  const int64_t Kd = fc2 ? a.I : a.H;            // reduction length (codes per row)
  const int Nd = static_cast<int>(fc2 ? a.H : a.F1);  // rows of one expert's matrix
  const uint32_t rowb = static_cast<uint32_t>(Kd * BITS / 8);
  const uint32_t chunks = rowb / 16;
  const int steps = static_cast<int>((chunks + 63) / 64);
  const int s0 = fc2 ? kseg * a.seg : 0;
  const int nst = fc2 ? min(a.seg, steps - s0) : steps;  // steps of this segment
  const int64_t k_lo = static_cast<int64_t>(s0) * 64 * CPC;
  const int64_t kpad = static_cast<int64_t>(nst) * 64 * CPC;
  const int64_t kpad_lds = kpad / CPC * (CPC + 4);
  const uint32_t spr = SM == SM_ROW ? 1u : static_cast<uint32_t>(Kd >> a.lbs);  // scales per row
  const int row_base = (tile * 4 + wave) * (RPW * gpw);
  const int E = static_cast<int>(a.E);
  const bool combine = a.k * ks > 1;

  int e;
  float wgt = 1.f;
  if constexpr (!fc2) {
    float* lr = xs + kpad_lds;
    int* fl = reinterpret_cast<int*>(lr + E);
    int* sl = fl + E;
    const float* lsrc = a.router + t * a.E;
    for (int i = tid; i < E; i += MOE_T) lr[i] = lsrc[i];
    stage_vec<CPC>(xs, a.x + t * a.H, Kd, kpad);
    if (a.clear)
      for (int64_t i = static_cast<int64_t>(blockIdx.x) * MOE_T + tid; i < a.T * tiles2;
           i += static_cast<int64_t>(gridDim.x) * MOE_T)
        a.cnt[i] = 0u;
    __syncthreads();
    route_slot(E, a.k, slot, lr, fl, sl, &s_e, &s_w);
    e = s_e;
    if (tile == 0 && tid == 0) {
      a.sel[pair] = s_e;
      a.wts[pair] = s_w;
    }
  } else {
    e = min(max(a.sel[pair], 0), E - 1);  // an index out of range can never be read
    wgt = a.wts[pair];
  }

  const uint8_t* We = (fc2 ? a.fc2 : a.fc1) + static_cast<int64_t>(e) * Nd * rowb;
  const float* Se = (fc2 ? a.s2 : a.s1) + static_cast<int64_t>(e) * Nd * spr;
  const rsrc_t rW = mk_rsrc(We, static_cast<uint32_t>(Nd) * rowb);
  const rsrc_t rS = mk_rsrc(Se, static_cast<uint32_t>(Nd) * spr * 4u);
  const int myrow = row8(lane);

  struct Buf {
    u32x4 w[RPW];
    float s[RPW][NS];
    float rs;  // row scale of row8(lane) (block_size 0)
  };
  // Loads of unit (g, s): rows are wave-uniform, so each row's offset is a
  // scalar operand (clamped to the last row: rows past the end read real
  // memory and are never written); the lane's chunk is the vector offset,
  // out of range past the row end or past the wave's last group.
  auto issue = [&](Buf& b, int g, int s) {
    const uint32_t c = static_cast<uint32_t>(s) * 64u + static_cast<uint32_t>(lane);
    const bool in = g < gpw && c < chunks;
    const uint32_t voff = in ? c * 16u : 0x80000000u;
    const int row0 = row_base + g * RPW;
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      b.w[r] = bld16_nt(rW, voff, static_cast<uint32_t>(min(row0 + r, Nd - 1)) * rowb);
    if constexpr (SM != SM_ROW) {
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        const uint32_t so = in ? ((c * CPC + q * (CPC / NS)) >> a.lbs) * 4u : 0x80000000u;
#pragma unroll
        for (int r = 0; r < RPW; ++r)
          b.s[r][q] = bld_f32(rS, so, static_cast<uint32_t>(min(row0 + r, Nd - 1)) * spr * 4u);
      }
    } else {
      b.rs = bld_f32(rS, g < gpw ? static_cast<uint32_t>(min(row0 + myrow, Nd - 1)) * 4u : 0x80000000u, 0);
    }
  };

  Buf buf[2];
  issue(buf[0], 0, s0);
  if constexpr (fc2) {
    // this segment of h, zero-padded to whole steps, staged while unit 0 loads
    stage_vec<CPC>(xs, a.h + pair * a.I + k_lo, min(Kd - k_lo, kpad), kpad);
    __syncthreads();
  }

  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.f;

  auto consume = [&](const Buf& b, int g, int s) {
    const int sl = s - s0;  // step within the segment
    const float* xq = xs + (static_cast<int64_t>(sl) * 64 + lane) * (CPC + 4);
    float part[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) part[r] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      float xv[CPD];
#pragma unroll
      for (int q = 0; q < CPD / 4; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(xq + d * CPD + 4 * q);
        xv[4 * q] = v.x;
        xv[4 * q + 1] = v.y;
        xv[4 * q + 2] = v.z;
        xv[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        if constexpr (SM == SM_ROW) {
          acc[r] = dword_dot<BITS>(b.w[r][d], xv, acc[r]);
        } else {
          part[r] = dword_dot<BITS>(b.w[r][d], xv, part[r]);
          if (NS == 2 && d == 1) {  // first of two scale blocks complete
            acc[r] = __builtin_fmaf(b.s[r][0], part[r], acc[r]);
            part[r] = 0.f;
          }
        }
      }
    }
    if constexpr (SM != SM_ROW) {
#pragma unroll
      for (int r = 0; r < RPW; ++r) acc[r] = __builtin_fmaf(b.s[r][NS - 1], part[r], acc[r]);
    }
    if (sl == nst - 1) {  // the group is complete: reduce, scale, write
      float v = reduce8(acc, lane);
#pragma unroll
      for (int r = 0; r < RPW; ++r) acc[r] = 0.f;
      if constexpr (SM == SM_ROW) v *= b.rs;
      const int row = row_base + g * RPW + myrow;
      if constexpr (ST == ST_FC1_SWIGLU) {
        const float lin = __shfl_xor(v, 32, 64);  // row + 1
        if ((lane & 39) == 0 && row + 1 < Nd) a.h[pair * a.I + row / 2] = swiglu(v, lin, a);
      } else if constexpr (ST == ST_FC1_RELU) {
        if ((lane & 7) == 0 && row < Nd) a.h[pair * a.I + row] = fmaxf(v, 0.f);
      } else {
        if ((lane & 7) == 0 && row < Nd) {
          if (!combine)
            a.y[t * a.H + row] = wgt * v;
          else  // device-coherent store: read back by another workgroup
            __hip_atomic_store(a.yp + (pair * ks + kseg) * a.H + row, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  };

  // units in (group, step) order, two per trip so the buffers are named
  // statically; (g, s) past the wave's last group load nothing
  int g = 0, s = s0;
  auto next = [&](int& gg, int& ss) {
    if (++ss == s0 + nst) {
      ss = s0;
      ++gg;
    }
  };
  // (the scheduling barriers keep each unit's loads ahead of the previous
  // unit's arithmetic: the memory counter retires in issue order)
  while (g < gpw) {
    int g1 = g, s1 = s;
    next(g1, s1);
    issue(buf[1], g1, s1);
    __builtin_amdgcn_sched_barrier(0);
    consume(buf[0], g, s);
    int g2 = g1, s2 = s1;
    next(g2, s2);
    issue(buf[0], g2, s2);
    __builtin_amdgcn_sched_barrier(0);
    if (g1 < gpw) consume(buf[1], g1, s1);
    g = g2;
    s = s2;
  }

  if constexpr (fc2) {
    if (combine) {
      // The partials went out as device-coherent (agent-scope atomic) stores,
      // which bypass the per-XCD L2 for the memory side. Every thread waits
      // until its stores are acknowledged (s_waitcnt 0 covers stores on this
      // architecture), the barrier orders all of them before thread 0's
      // arrival count, and the last of the token's k * ks workgroups on this
      // row tile issues its device-coherent loads only after its count
      // returned (they depend on it through s_last), so it reads every
      // acknowledged partial. The count stays relaxed on purpose: an
      // acquire-release count makes the compiler write back and invalidate
      // the whole L2 around it in every workgroup, which measured 80 us
      // against 51 us per Mixtral decode step, for stores that are not in L2.
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0)
        s_last = __hip_atomic_fetch_add(a.cnt + t * tiles2 + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 static_cast<uint32_t>(a.k * ks - 1);
      __syncthreads();
      if (s_last) {
        const int rows = 4 * RPW * gpw;
        for (int i = tid; i < rows; i += MOE_T) {
          const int row = tile * rows + i;
          if (row < Nd) {
            float y = 0.f;
            for (int s = 0; s < a.k; ++s) {
              const float* p = a.yp + (t * a.k + s) * ks * a.H + row;
              float v = 0.f;
              for (int q = 0; q < ks; ++q)
                v += __hip_atomic_load(p + static_cast<int64_t>(q) * a.H, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              y = __builtin_fmaf(a.wts[t * a.k + s], v, y);
            }
            a.y[t * a.H + row] = y;
          }
        }
      }
    }
  }
}
// ---------------------------------------------------------------------------
// scalar fallback (any shape): one thread per output element

__device__ __forceinline__ float expert_weight(const uint8_t* W, const float* S, int64_t e, int64_t row, int64_t col,
                                               int64_t rows, int64_t cols, int64_t spr, const MoeArgs& a) {
  const int bits = a.bits;
  const int64_t pc = (cols * bits + 7) / 8;
  const uint32_t byte = W[(e * rows + row) * pc + (col * bits) / 8];
  const uint32_t q = (byte >> ((col * bits) % 8)) & ((1u << bits) - 1u);
  const float v = static_cast<float>(q) - static_cast<float>(1u << (bits - 1));
  return __fmul_rn(v, S[(e * rows + row) * spr + (spr > 1 ? col / (a.bs > 0 ? a.bs : 1) : 0)]);
}

__global__ __launch_bounds__(MOE_T) void k_moe_fc1_scalar(MoeArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * MOE_T + threadIdx.x;  // (pair, j)
  if (i >= a.T * a.k * a.I) return;
  const int64_t pair = i / a.I, j = i % a.I, t = pair / a.k;
  const int64_t e = min(max(a.sel[pair], 0), static_cast<int>(a.E) - 1);
  const int64_t spr = a.bs ? a.H / a.bs : 1;
  const bool sw = a.act == XRMM_ACT_SWIGLU_CODE;
  const int64_t gr = sw ? 2 * j : j, lr = 2 * j + 1;
  float g = 0.f, l = 0.f;
  for (int64_t kk = 0; kk < a.H; ++kk) {
    const float xv = a.x[t * a.H + kk];
    g = __builtin_fmaf(xv, expert_weight(a.fc1, a.s1, e, gr, kk, a.F1, a.H, spr, a), g);
    if (sw) l = __builtin_fmaf(xv, expert_weight(a.fc1, a.s1, e, lr, kk, a.F1, a.H, spr, a), l);
  }
  a.h[pair * a.I + j] = sw ? swiglu(g, l, a) : fmaxf(g, 0.f);
}

__global__ __launch_bounds__(MOE_T) void k_moe_fc2_scalar(MoeArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * MOE_T + threadIdx.x;  // (token, c)
  if (i >= a.T * a.H) return;
  const int64_t t = i / a.H, c = i % a.H;
  const int64_t spr = a.bs ? a.I / a.bs : 1;
  float y = 0.f;
  for (int s = 0; s < a.k; ++s) {
    const int64_t pair = t * a.k + s, e = min(max(a.sel[pair], 0), static_cast<int>(a.E) - 1);
    float v = 0.f;
    for (int64_t j = 0; j < a.I; ++j)
      v = __builtin_fmaf(a.h[pair * a.I + j], expert_weight(a.fc2, a.s2, e, c, j, a.H, a.I, spr, a), v);
    y = __builtin_fmaf(a.wts[pair], v, y);
  }
  a.y[i] = y;
}

__global__ __launch_bounds__(MOE_T) void k_moe_zero(float* y, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * MOE_T + threadIdx.x;
  if (i < n) y[i] = 0.f;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Floats of LDS for an activation vector of kd codes (whole steps, padded
// chunk layout).
int64_t moe_kpad(int64_t kd, int bits) {
  const int64_t cpc = 128 / bits, per_step = 64 * cpc;
  return (kd + per_step - 1) / per_step * 64 * (cpc + 4);
}

template <int BITS, int SM, int ST>
hipError_t launch_gemv(const MoeArgs& a, int gpw, hipStream_t st) {
  const bool fc2 = ST == ST_FC2;
  const int64_t Nd = fc2 ? a.H : a.F1;
  const int64_t per_step_lds = 64 * (128 / BITS + 4);
  const size_t lds = static_cast<size_t>(fc2 ? a.seg * per_step_lds : moe_kpad(a.H, BITS) + 2 * a.E + MOE_MAX_K) * 4;
  auto kern = k_moe_gemv<BITS, SM, ST>;
  if (lds > 64 * 1024) {
    static std::atomic<int> done[kMaxDevices];  // per instantiation and device
    (void)raise_lds_cap(reinterpret_cast<const void*>(kern), static_cast<int>(kMoeMaxLds), done);
    (void)hipGetLastError();
  }
  const int64_t tiles = (Nd + 32 * gpw - 1) / (32 * gpw);
  const int64_t blocks = a.T * a.k * tiles * (fc2 ? a.ks : 1);
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(blocks)), dim3(MOE_T), lds, st, a, gpw, static_cast<int>(tiles),
                     static_cast<int>(moe_tiles2(a.H)));
  return hipGetLastError();
}

template <int BITS, int SM>
hipError_t launch_fast(const MoeArgs& args, hipStream_t st) {
  MoeArgs a = args;
  const int64_t steps2 = (a.I * BITS / 8 / 16 + 63) / 64;
  const int64_t ks0 = moe_fc2_segments_max(a.T, a.k, a.H, steps2, XRMM_MOE_FC2_WGS);
  a.seg = static_cast<int>((steps2 + ks0 - 1) / ks0);
  a.ks = static_cast<int>((steps2 + a.seg - 1) / a.seg);
  a.clear = a.k * a.ks > 1;
  a.lbs = a.bs ? __builtin_ctz(static_cast<unsigned>(a.bs)) : 0;
  // FC1 row groups per wave: enough rows per workgroup that the launch stays
  // within one resident round
  const int64_t tiles32 = a.T * a.k * ((a.F1 + 31) / 32);
  const int gpw1 = static_cast<int>(std::min<int64_t>(16, std::max<int64_t>(1, (tiles32 + XRMM_MOE_FC1_WGS - 1) / XRMM_MOE_FC1_WGS)));
  hipError_t e = a.act == XRMM_ACT_SWIGLU_CODE ? launch_gemv<BITS, SM, ST_FC1_SWIGLU>(a, gpw1, st)
                                               : launch_gemv<BITS, SM, ST_FC1_RELU>(a, gpw1, st);
  if (e != hipSuccess) return e;
  return launch_gemv<BITS, SM, ST_FC2>(a, 1, st);
}

}  // namespace

bool moe_fast_ok(const MoeArgs& a) {
  // whole 16-byte chunks per row, aligned tensors, vectors within LDS
  if ((a.H * a.bits / 8) % 16 != 0 || (a.I * a.bits / 8) % 16 != 0) return false;
  if (!aligned16(a.x) || !aligned16(a.fc1) || !aligned16(a.fc2) || !aligned16(a.h)) return false;
  if ((moe_kpad(a.H, a.bits) + 2 * a.E + MOE_MAX_K) * 4 > kMoeMaxLds || moe_kpad(a.I, a.bits) * 4 > kMoeMaxLds)
    return false;
  if (a.k > MOE_MAX_K || a.E > 4096) return false;
  if (a.act == XRMM_ACT_SWIGLU_CODE && a.F1 % 2 != 0) return false;
  // each expert's code and scale matrices within a 32-bit buffer range
  const int64_t lim = int64_t(1) << 31;
  const int64_t spr1 = a.bs ? a.H / a.bs : 1, spr2 = a.bs ? a.I / a.bs : 1;
  if (a.F1 * a.H * a.bits / 8 >= lim || a.H * a.I * a.bits / 8 >= lim) return false;
  if (a.F1 * spr1 * 4 >= lim || a.H * spr2 * 4 >= lim) return false;
  // block scales: whole blocks per 16-byte chunk, or two blocks per chunk
  if (a.bs != 0 && a.bs < 64 / a.bits) return false;
  return a.T * a.k * ((a.F1 + 31) / 32) < (int64_t(1) << 31) && a.T * a.k * moe_tiles2(a.H) * 1024 < (int64_t(1) << 31);
}

// Grouped-expert path (xrmm_moe_gemm.h): 4-bit codes with row scales, K
// steps of whole 64-element runs, at least XRMM_MOE_GROUP_MIN (token, slot)
// pairs, and the lists fitting the workspace's counter region.
#ifndef XRMM_MOE_GROUP_MIN
#define XRMM_MOE_GROUP_MIN 32
#endif
bool moe_grouped_ok(const MoeArgs& a) {
  if ((a.bits != 4 && a.bits != 8) || a.H % 64 != 0 || a.I % 64 != 0 || a.E > kMoeGroupMaxExperts) return false;
  // row scales, or power-of-two blocks of at least 32 codes that divide both
  // rows (blocks of 16, one scaled sum per MFMA slice, need more registers
  // than a wave has and spill: 5.6 ms against 0.95 ms for blocks of 64 at
  // T = 256 on the Mixtral experts)
  if (a.bs != 0 && (a.bs < 32 || (a.bs & (a.bs - 1)) != 0 || a.H % a.bs != 0 || a.I % a.bs != 0)) return false;
  if (a.T * a.k < XRMM_MOE_GROUP_MIN) return false;
  if (!aligned16(a.x) || !aligned16(a.fc1) || !aligned16(a.fc2) || !aligned16(a.h) || !aligned16(a.yp)) return false;
  if (a.act == XRMM_ACT_SWIGLU_CODE && a.F1 != 2 * a.I) return false;
  const int64_t lim = int64_t(1) << 31;
  // 32-bit row-tile grid and pair indices (the workspace's last region holds
  // the lists for up to kMoeGroupMaxExperts experts)
  return a.F1 * a.H / 2 < lim && a.H * a.I / 2 < lim && a.T * a.k * a.I < lim &&
         a.T * a.k * a.H * moe_group_fc2_splits(a.T, a.k, a.H, a.I) < lim;
}

const char* moe_kernel_name(const MoeArgs& a) {
  return moe_grouped_ok(a) ? "qmoe_grouped" : moe_fast_ok(a) ? "qmoe_rows" : "qmoe_scalar";
}

namespace {
// One grouped GEMM launch of stage ST, BITS-bit codes, block mode BKM.
template <int ST, int BITS, int BKM>
hipError_t mg_launch(const MoeArgs& a, const MgLists& g, int nct, int64_t grid, hipStream_t st) {
  auto kern = k_moe_ggemm<ST, BITS, BKM>;
  constexpr size_t lds = mg_lds<BITS>();
  if constexpr (lds > 64 * 1024) {
    static std::atomic<int> done[kMaxDevices];  // per instantiation and device
    if (hipError_t e = raise_lds_cap(reinterpret_cast<const void*>(kern), static_cast<int>(lds), done); e != hipSuccess)
      return e;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(grid)), dim3(MG_T), lds, st, a, g, nct);
  return hipGetLastError();
}

template <int ST, int BITS>
hipError_t mg_launch_b(const MoeArgs& a, const MgLists& g, int nct, int64_t grid, hipStream_t st) {
  switch (mg_block_mode(a.bs)) {  // blocks of 16 (mode 1) do not take this path
    case 0: return mg_launch<ST, BITS, 0>(a, g, nct, grid, st);
    case 2: return mg_launch<ST, BITS, 2>(a, g, nct, grid, st);
    case 4: return mg_launch<ST, BITS, 4>(a, g, nct, grid, st);
    default: return mg_launch<ST, BITS, 8>(a, g, nct, grid, st);
  }
}

template <int ST>
hipError_t mg_launch_s(const MoeArgs& a, const MgLists& g, int nct, int64_t grid, hipStream_t st) {
  return a.bits == 8 ? mg_launch_b<ST, 8>(a, g, nct, grid, st) : mg_launch_b<ST, 4>(a, g, nct, grid, st);
}

hipError_t launch_grouped(const MoeArgs& a0, hipStream_t st) {
  MoeArgs a = a0;
  a.ks = static_cast<int>(moe_group_fc2_splits(a.T, a.k, a.H, a.I));  // FC2 K splits (the combine sums them)
  MgLists g;
  int32_t* base = reinterpret_cast<int32_t*>(a.cnt);
  g.off = base;
  g.toff = g.off + (a.E + 1);
  g.list = g.toff + (a.E + 1);
  g.hmax = reinterpret_cast<uint32_t*>(g.list + a.T * a.k);
  g.ex = reinterpret_cast<int32_t*>(g.hmax + a.T * a.k);
  const int T = static_cast<int>(a.T), npairs = static_cast<int>(a.T * a.k), E = static_cast<int>(a.E);
  hipLaunchKernelGGL(k_moe_route, dim3(static_cast<uint32_t>((a.T + 3) / 4)), dim3(MOE_T), 0, st, a.router, a.sel, a.wts,
                     T, E, a.k);
  hipLaunchKernelGGL(k_moe_xexp, dim3(static_cast<uint32_t>((a.T + 3) / 4)), dim3(256), 0, st, a.x, T, a.H, g.ex);
  hipLaunchKernelGGL(k_moe_group, dim3(1), dim3(MG_T), 0, st, a.sel, npairs, E, g);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  // row tiles: at most one partial tile per expert beyond the full ones
  const int64_t rtmax = (a.T * a.k + MG_RT - 1) / MG_RT + a.E;
  const int nct1 = static_cast<int>((a.F1 + MG_CT - 1) / MG_CT), nct2 = static_cast<int>((a.H + MG_CT - 1) / MG_CT);
  if (rtmax * nct1 > 0x7FFFFFFF || rtmax * nct2 * a.ks > 0x7FFFFFFF) return hipErrorInvalidValue;
  const hipError_t e1 = a.act == XRMM_ACT_SWIGLU_CODE ? mg_launch_s<MG_FC1_SWIGLU>(a, g, nct1, rtmax * nct1, st)
                                                      : mg_launch_s<MG_FC1_RELU>(a, g, nct1, rtmax * nct1, st);
  if (e1 != hipSuccess) return e1;
  if (hipError_t e = mg_launch_s<MG_FC2>(a, g, nct2, rtmax * nct2 * a.ks, st); e != hipSuccess) return e;
  hipLaunchKernelGGL(k_moe_combine, dim3(static_cast<uint32_t>((a.T * a.H + 255) / 256)), dim3(256), 0, st, a);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_qmoe(const MoeArgs& a, hipStream_t st) {
  if (a.T == 0) return hipSuccess;
  if (a.I == 0) {  // no intermediate width: every expert contributes zero
    hipLaunchKernelGGL(k_moe_zero, dim3(static_cast<uint32_t>((a.T * a.H + MOE_T - 1) / MOE_T)), dim3(MOE_T), 0, st, a.y,
                       a.T * a.H);
    return hipGetLastError();
  }
  if (moe_grouped_ok(a)) return launch_grouped(a, st);
  if (moe_fast_ok(a)) {  // routing runs inside the FC1 launch
    const int cpc = 128 / a.bits;
    const int sm = a.bs == 0 ? SM_ROW : a.bs >= cpc ? SM_CHUNK : SM_HALF;
    if (a.bits == 4) {
      if (sm == SM_ROW) return launch_fast<4, SM_ROW>(a, st);
      if (sm == SM_CHUNK) return launch_fast<4, SM_CHUNK>(a, st);
      return launch_fast<4, SM_HALF>(a, st);
    }
    if (sm == SM_ROW) return launch_fast<8, SM_ROW>(a, st);
    return launch_fast<8, SM_CHUNK>(a, st);
  }
  // one thread per (token, slot, column) and per (token, column): the grids
  // must stay within the launch limit of 2^31 - 1 workgroups
  const int64_t lim = (int64_t(1) << 31) - 1;
  if ((a.T * a.k * a.I + MOE_T - 1) / MOE_T > lim || (a.T * a.H + MOE_T - 1) / MOE_T > lim) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_moe_route, dim3(static_cast<uint32_t>((a.T + 3) / 4)), dim3(MOE_T), 0, st, a.router, a.sel, a.wts,
                     static_cast<int>(a.T), static_cast<int>(a.E), a.k);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  hipLaunchKernelGGL(k_moe_fc1_scalar, dim3(static_cast<uint32_t>((a.T * a.k * a.I + MOE_T - 1) / MOE_T)), dim3(MOE_T), 0,
                     st, a);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  hipLaunchKernelGGL(k_moe_fc2_scalar, dim3(static_cast<uint32_t>((a.T * a.H + MOE_T - 1) / MOE_T)), dim3(MOE_T), 0, st,
                     a);
  return hipGetLastError();
}

}  // namespace xrmm
