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
// Three launches on the caller's stream:
//  1. k_moe_route: one wave per token; writes the k selected experts (ascending
//     index) and their softmax weights into the workspace.
//  2. k_moe_rows (FC1): a workgroup stages the token's activation vector once
//     in LDS; each wave owns RPW consecutive rows of the selected expert's FC1
//     and walks K with 16-byte weight loads per lane (the next step's loads in
//     flight while the current step is computed); activation applied in the
//     epilogue; h [T, k, I] float32 in the workspace.
//  3. k_moe_rows (FC2): the same kernel over the hidden rows of each selected
//     expert's FC2, the activation vector being h of that (token, slot),
//     accumulated with the routing weight over the k slots.
// Arithmetic is float32 throughout: per dword the codes convert with
// v_cvt_f32_ubyte (low and high nibbles masked into separate bytes) and
// accumulate (code - midpoint, exact) with FMAs against the activations; the
// scale multiplies the group's sum (block scales) or the row's total (row
// scales).
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

__device__ __forceinline__ float swiglu(float gate, float lin, const MoeArgs& a) {
  if (a.has_limit) {
    gate = fminf(gate, a.limit);
    lin = fminf(fmaxf(lin, -a.limit), a.limit);
  }
  const float z = a.alpha * gate;
  const float lg = z >= 0.f ? 1.f / (1.f + expf(-z)) : expf(z) / (1.f + expf(z));
  return gate * lg * (lin + a.beta);
}

// sum over the codes of one dword of a chunk against their activations:
// (q - mid) is formed exactly in float32 before its product (taking mid out
// through the activation sum instead would cancel most of the bits for
// 8-bit codes, whose midpoint is 128)
template <int BITS>
__device__ __forceinline__ float dword_dot(uint32_t w, const float* x, float acc) {
  constexpr float mid = static_cast<float>(1 << (BITS - 1));
  if constexpr (BITS == 4) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    acc = __builtin_fmaf(static_cast<float>(lo & 0xFFu) - mid, x[0], acc);
    acc = __builtin_fmaf(static_cast<float>(hi & 0xFFu) - mid, x[1], acc);
    acc = __builtin_fmaf(static_cast<float>((lo >> 8) & 0xFFu) - mid, x[2], acc);
    acc = __builtin_fmaf(static_cast<float>((hi >> 8) & 0xFFu) - mid, x[3], acc);
    acc = __builtin_fmaf(static_cast<float>((lo >> 16) & 0xFFu) - mid, x[4], acc);
    acc = __builtin_fmaf(static_cast<float>((hi >> 16) & 0xFFu) - mid, x[5], acc);
    acc = __builtin_fmaf(static_cast<float>(lo >> 24) - mid, x[6], acc);
    return __builtin_fmaf(static_cast<float>(hi >> 24) - mid, x[7], acc);
  } else {
    acc = __builtin_fmaf(static_cast<float>(w & 0xFFu) - mid, x[0], acc);
    acc = __builtin_fmaf(static_cast<float>((w >> 8) & 0xFFu) - mid, x[1], acc);
    acc = __builtin_fmaf(static_cast<float>((w >> 16) & 0xFFu) - mid, x[2], acc);
    return __builtin_fmaf(static_cast<float>(w >> 24) - mid, x[3], acc);
  }
}

template <int BITS, int SM, int ST, int RPW>
__global__ __launch_bounds__(MOE_T) void k_moe_rows(MoeArgs a) {
  extern __shared__ __align__(16) float xs[];
  constexpr int CPC = 128 / BITS;  // codes per 16-byte chunk
  constexpr int CPD = 32 / BITS;   // codes per dword
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool fc2 = ST == ST_FC2;
  const int64_t Kd = fc2 ? a.I : a.H;    // reduction length (codes per row)
  const int64_t Nd = fc2 ? a.H : a.F1;   // rows of one expert's matrix
  const uint32_t rowb = static_cast<uint32_t>(Kd * BITS / 8);
  const int64_t kpad = (Kd + 64 * CPC - 1) / (64 * CPC) * (64 * CPC);
  const int steps = static_cast<int>(kpad / (64 * CPC));
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * (MOE_T / 64) + wave) * RPW;
  const int64_t spr = SM == SM_ROW ? 1 : Kd / a.bs;  // scales per row
  const uint8_t* W = fc2 ? a.fc2 : a.fc1;
  const float* S = fc2 ? a.s2 : a.s1;

  // FC1: one (token, slot) per blockIdx.y; FC2: one token, every slot
  const int64_t p = blockIdx.y;
  const int nslots = fc2 ? a.k : 1;
  float yacc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) yacc[r] = 0.f;

  for (int sl = 0; sl < nslots; ++sl) {
    const int64_t pair = fc2 ? p * a.k + sl : p;
    const int e = min(max(a.sel[pair], 0), static_cast<int>(a.E) - 1);  // an index out of range can never be read
    const float wgt = fc2 ? a.wts[pair] : 1.f;
    // stage the activation vector (zero-padded to whole steps)
    const float* src = fc2 ? a.h + pair * a.I : a.x + (pair / a.k) * a.H;
    if (sl > 0) __syncthreads();  // every wave is done with the previous vector
    for (int64_t i = tid; i < kpad; i += MOE_T) xs[i] = i < Kd ? src[i] : 0.f;
    __syncthreads();

    const uint8_t* We = W + static_cast<int64_t>(e) * Nd * rowb;
    const float* Se = S + static_cast<int64_t>(e) * Nd * spr;
    const rsrc_t rW = mk_rsrc(We, static_cast<uint32_t>(Nd) * rowb);
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.f;
    auto ld = [&](u32x4(&w)[RPW], int s) {
      const uint32_t c = static_cast<uint32_t>(s * 64 + lane);  // chunk of the row
      const bool in = static_cast<int64_t>(c) * CPC < Kd;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const int64_t row = row0 + r;
        const uint32_t off = (in && row < Nd) ? static_cast<uint32_t>(row) * rowb + c * 16u : 0x80000000u;
        w[r] = bld16_nt(rW, off, 0);
      }
    };
    u32x4 wb[2][RPW];
    ld(wb[0], 0);
    for (int s = 0; s < steps; ++s) {
      if (s + 1 < steps) ld(wb[(s + 1) & 1], s + 1);
      const int64_t k0 = (static_cast<int64_t>(s) * 64 + lane) * CPC;
      float xv[CPC];
#pragma unroll
      for (int q = 0; q < CPC / 4; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(xs + k0 + 4 * q);
        xv[4 * q] = v.x;
        xv[4 * q + 1] = v.y;
        xv[4 * q + 2] = v.z;
        xv[4 * q + 3] = v.w;
      }
      constexpr int G = SM == SM_HALF ? 2 : 1;  // scale groups per chunk
      const bool in = k0 < Kd;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const u32x4 w = wb[s & 1][r];
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
          if constexpr (SM == SM_ROW) {
#pragma unroll
            for (int d = 0; d < 4; ++d) acc[r] = dword_dot<BITS>(w[d], xv + d * CPD, acc[r]);
          } else {
            float part = 0.f;
#pragma unroll
            for (int d = gi * 4 / G; d < (gi + 1) * 4 / G; ++d) part = dword_dot<BITS>(w[d], xv + d * CPD, part);
            const int64_t row = row0 + r;
            const float sc = (in && row < Nd) ? Se[row * spr + (k0 + gi * CPC / G) / a.bs] : 0.f;
            acc[r] = __builtin_fmaf(sc, part, acc[r]);
          }
        }
      }
    }
    // wave sums; row scale for per-row scales
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      float v = wave_sum(acc[r]);
      const int64_t row = row0 + r;
      if constexpr (SM == SM_ROW) v *= row < Nd ? Se[row] : 0.f;
      acc[r] = v;
    }
    if constexpr (ST == ST_FC2) {
#pragma unroll
      for (int r = 0; r < RPW; ++r) yacc[r] = __builtin_fmaf(wgt, acc[r], yacc[r]);
    } else {
      // FC1 epilogue: activation, h[pair][j]
      float* hp = a.h + pair * a.I;
      if (lane == 0) {
        if constexpr (ST == ST_FC1_SWIGLU) {
#pragma unroll
          for (int r = 0; r + 1 < RPW; r += 2) {
            const int64_t j = (row0 + r) / 2;
            if (row0 + r + 1 < Nd) hp[j] = swiglu(acc[r], acc[r + 1], a);
          }
        } else {
#pragma unroll
          for (int r = 0; r < RPW; ++r)
            if (row0 + r < Nd) hp[row0 + r] = fmaxf(acc[r], 0.f);
        }
      }
    }
  }
  if constexpr (ST == ST_FC2) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < RPW; ++r)
        if (row0 + r < Nd) a.y[p * a.H + row0 + r] = yacc[r];
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

template <int BITS, int SM, int ST, int RPW>
hipError_t launch_rows(const MoeArgs& a, hipStream_t st) {
  const bool fc2 = ST == ST_FC2;
  const int64_t Kd = fc2 ? a.I : a.H, Nd = fc2 ? a.H : a.F1;
  const int64_t kpad = (Kd + 64 * (128 / BITS) - 1) / (64 * (128 / BITS)) * (64 * (128 / BITS));
  const size_t lds = static_cast<size_t>(kpad) * sizeof(float);
  auto kern = k_moe_rows<BITS, SM, ST, RPW>;
  if (lds > 64 * 1024) {
    static bool raised = false;  // per instantiation
    if (!raised) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(kMoeMaxLds));
      (void)hipGetLastError();
      raised = true;
    }
  }
  const int64_t rows_per_wg = (MOE_T / 64) * RPW;
  const dim3 grid(static_cast<uint32_t>((Nd + rows_per_wg - 1) / rows_per_wg),
                  static_cast<uint32_t>(fc2 ? a.T : a.T * a.k));
  hipLaunchKernelGGL(kern, grid, dim3(MOE_T), lds, st, a);
  return hipGetLastError();
}

template <int BITS, int SM>
hipError_t launch_fast(const MoeArgs& a, hipStream_t st) {
  hipError_t e = a.act == XRMM_ACT_SWIGLU_CODE ? launch_rows<BITS, SM, ST_FC1_SWIGLU, 16>(a, st)
                                               : launch_rows<BITS, SM, ST_FC1_RELU, 16>(a, st);
  if (e != hipSuccess) return e;
  return launch_rows<BITS, SM, ST_FC2, 4>(a, st);
}

}  // namespace

bool moe_fast_ok(const MoeArgs& a) {
  // whole 16-byte chunks per row, aligned tensors, activation vectors within LDS
  if ((a.H * a.bits / 8) % 16 != 0 || (a.I * a.bits / 8) % 16 != 0) return false;
  if (!aligned16(a.x) || !aligned16(a.fc1) || !aligned16(a.fc2) || !aligned16(a.h)) return false;
  const int64_t cpc = 128 / a.bits;
  for (int64_t kd : {a.H, a.I}) {
    const int64_t kpad = (kd + 64 * cpc - 1) / (64 * cpc) * (64 * cpc);
    if (kpad * 4 > kMoeMaxLds) return false;
  }
  if (a.act == XRMM_ACT_SWIGLU_CODE && a.F1 % 2 != 0) return false;
  // one expert's matrix within a 32-bit buffer range
  const int64_t lim = int64_t(1) << 31;
  if (a.F1 * a.H * a.bits / 8 >= lim || a.H * a.I * a.bits / 8 >= lim) return false;
  // block scales: a whole number of blocks per 16-byte chunk, or two per chunk
  if (a.bs != 0 && a.bs < cpc / 2) return false;
  return a.T * a.k <= 65535 && a.T <= 65535;
}

const char* moe_kernel_name(const MoeArgs& a) { return moe_fast_ok(a) ? "qmoe_rows" : "qmoe_scalar"; }

hipError_t launch_qmoe(const MoeArgs& a, hipStream_t st) {
  if (a.T == 0) return hipSuccess;
  hipLaunchKernelGGL(k_moe_route, dim3(static_cast<uint32_t>((a.T + 3) / 4)), dim3(MOE_T), 0, st, a.router, a.sel, a.wts,
                     static_cast<int>(a.T), static_cast<int>(a.E), a.k);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  if (a.I == 0) {  // no intermediate width: every expert contributes zero
    hipLaunchKernelGGL(k_moe_zero, dim3(static_cast<uint32_t>((a.T * a.H + MOE_T - 1) / MOE_T)), dim3(MOE_T), 0, st, a.y,
                       a.T * a.H);
    return hipGetLastError();
  }
  if (moe_fast_ok(a)) {
    const int cpc = 128 / a.bits;
    const int sm = a.bs == 0 ? SM_ROW : a.bs >= cpc ? SM_CHUNK : SM_HALF;
    if (a.bits == 4) {
      if (sm == SM_ROW) return launch_fast<4, SM_ROW>(a, st);
      if (sm == SM_CHUNK) return launch_fast<4, SM_CHUNK>(a, st);
      return launch_fast<4, SM_HALF>(a, st);
    }
    if (sm == SM_ROW) return launch_fast<8, SM_ROW>(a, st);
    if (sm == SM_CHUNK) return launch_fast<8, SM_CHUNK>(a, st);
    return launch_fast<8, SM_HALF>(a, st);
  }
  hipLaunchKernelGGL(k_moe_fc1_scalar, dim3(static_cast<uint32_t>((a.T * a.k * a.I + MOE_T - 1) / MOE_T)), dim3(MOE_T), 0,
                     st, a);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  hipLaunchKernelGGL(k_moe_fc2_scalar, dim3(static_cast<uint32_t>((a.T * a.H + MOE_T - 1) / MOE_T)), dim3(MOE_T), 0, st,
                     a);
  return hipGetLastError();
}

}  // namespace xrmm
