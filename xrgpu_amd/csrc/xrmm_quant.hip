// com.microsoft.GatherBlockQuantized (opcode 1031) and com.microsoft.MatMulBnb4
// (opcode 1026) on gfx950.
//
// GatherBlockQuantized (gatherQuant, kernels/_shared/extended/shaders/
// complex_kernel.glsl:85; planner complex_plan.cpp:129): output row o is row
// indices[o] of the packed table, each code (low-first in a byte) minus its
// block's zero point (packed low-first, default 2^(bits-1)) times the block's
// float32 scale. An index outside [0, rows) leaves its row zero and records
// failure code 55 (the reference fails the run with "GPU operator contract
// validation failed: code 55", vulkan.cpp:115). It is an HBM-bound gather:
// one thread per 32-bit word of a selected row (8 or 4 codes), float4 stores.
//
// MatMulBnb4 (bnbWeight complex_kernel.glsl:82, the 1026 branch of
// packedMatmul :83): W[k][n] = codebook[code] * absmax[flat / block_size]
// with flat = n*K + k (transB) or k*N + n, two codes per byte, even flat index
// in the high nibble; NF4 for quant_type 1, FP4 for 0; Y = A W in float32,
// stored in A's dtype. The fast GEMV (transB, K a multiple of 32, blocks of 16
// or a multiple of 32 dividing K) streams each output column's contiguous
// codes with one 16-byte chunk (32 codes) per lane, looks codes up in a
// 16-entry float32 table in LDS (exact reference values) and accumulates in
// float32 against A rows staged in LDS; the absmax of a chunk multiplies the
// chunk's partial sum. Everything else runs one thread per output element in
// the reference's serial order.
#include "xrmm_device.h"
#include "xrmm_quant.h"

namespace xrmm {

namespace {

constexpr int QT = 256;  // threads per workgroup

// bitsandbytes codebooks (complex_kernel.glsl:82): NF4 (quant_type 1), FP4 (0)
__constant__ float kNF4[16] = {-1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.3949174880981445f,
                               -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
                               0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
                               0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
                               0.7229568362236023f, 1.0f};
__constant__ float kFP4[16] = {0.0f, 0.0052083333333333f, 0.6666666666666666f, 1.0f, 0.3333333333333333f, 0.5f,
                               0.1666666666666666f, 0.25f, -0.0f, -0.0052083333333333f, -0.6666666666666666f,
                               -1.0f, -0.3333333333333333f, -0.5f, -0.1666666666666666f, -0.25f};

// ---------------------------------------------------------------------------
// GatherBlockQuantized

// controlIndex (complex_kernel.glsl:31): int32 as is, int64 saturated.
__device__ __forceinline__ int64_t gbq_index(const GbqArgs& a, int64_t o) {
  if (a.idx64) {
    const int64_t v = static_cast<const int64_t*>(a.idx)[o];
    return v > INT32_MAX ? INT32_MAX : v < INT32_MIN ? INT32_MIN : v;
  }
  return static_cast<const int32_t*>(a.idx)[o];
}

__device__ __forceinline__ uint32_t gbq_zero(const GbqArgs& a, int64_t r, int64_t blk, int bits) {
  if (!a.zp) return 1u << (bits - 1);
  const uint32_t byte = a.zp[r * a.zpcols + (blk * bits) / 8];
  return (byte >> ((blk * bits) % 8)) & ((1u << bits) - 1u);
}

__device__ __forceinline__ void gbq_flag(const GbqArgs& a) {
  if (a.status) atomicMax(a.status, kGbqIndexError);
}

// One thread per 32-bit word of a selected row; workgroup b covers output row
// b / bpr and words [(b % bpr) * QT, +QT).
template <int BITS>
__global__ __launch_bounds__(QT) void k_gbq_words(GbqArgs a, int64_t bpr) {
  constexpr int CPW = 32 / BITS;  // codes per word
  const int64_t o = blockIdx.x / bpr;
  const int64_t w = (blockIdx.x % bpr) * QT + threadIdx.x;
  const int64_t words = a.pcols / 4;
  const int64_t r = gbq_index(a, o);
  float* dst = a.out + o * a.width + w * CPW;
  if (r < 0 || r >= a.rows) {
    if (w == 0) gbq_flag(a);
    if (w < words)
      for (int i = 0; i < CPW; i += 4) *reinterpret_cast<float4*>(dst + i) = float4{0.f, 0.f, 0.f, 0.f};
    return;
  }
  if (w >= words) return;
  const uint32_t word = *reinterpret_cast<const uint32_t*>(a.data + r * a.pcols + w * 4);
  const int64_t blk = (w * CPW) / a.bs;  // block_size >= 16 >= CPW: one block per word
  const float scale = a.scales[r * a.blocks + blk];
  const float z = static_cast<float>(gbq_zero(a, r, blk, BITS));
  float v[CPW];
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const uint32_t q = (word >> (BITS * i)) & ((1u << BITS) - 1u);
    v[i] = __fmul_rn(__fsub_rn(static_cast<float>(q), z), scale);
  }
#pragma unroll
  for (int i = 0; i < CPW; i += 4) *reinterpret_cast<float4*>(dst + i) = float4{v[i], v[i + 1], v[i + 2], v[i + 3]};
}

// One thread per output element (any row width or alignment).
__global__ __launch_bounds__(QT) void k_gbq_scalar(GbqArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * QT + threadIdx.x;
  if (i >= a.n * a.width) return;
  const int64_t o = i / a.width, j = i % a.width;
  const int64_t r = gbq_index(a, o);
  if (r < 0 || r >= a.rows) {
    if (j == 0) gbq_flag(a);
    a.out[i] = 0.f;
    return;
  }
  const int bits = a.bits;
  const uint32_t packed = a.data[r * a.pcols + (j * bits) / 8];
  const uint32_t q = (packed >> ((j * bits) % 8)) & ((1u << bits) - 1u);
  const int64_t blk = j / a.bs;
  const float z = static_cast<float>(gbq_zero(a, r, blk, bits));
  a.out[i] = __fmul_rn(__fsub_rn(static_cast<float>(q), z), a.scales[r * a.blocks + blk]);
}

// ---------------------------------------------------------------------------
// MatMulBnb4

__device__ __forceinline__ float bnb_code(const uint8_t* B, int64_t flat) {
  const uint32_t byte = B[flat / 2];
  return static_cast<float>((flat & 1) == 0 ? byte >> 4 : byte & 15u);
}

// One thread per output element, the reference's serial float32 order:
// sum += a * (codebook[code] * absmax).
template <typename T>
__global__ __launch_bounds__(QT) void k_bnb4_scalar(Bnb4Args a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * QT + threadIdx.x;
  if (i >= a.M * a.N) return;
  const int64_t m = i / a.N, n = i % a.N;
  const float* book = a.qt == 1 ? kNF4 : kFP4;
  const T* A = static_cast<const T*>(a.A);
  const T* am = static_cast<const T*>(a.absmax);
  float sum = 0.f;
  for (int64_t k = 0; k < a.K; ++k) {
    const int64_t flat = a.tb ? n * a.K + k : k * a.N + n;
    const float w = __fmul_rn(book[static_cast<int>(bnb_code(a.B, flat))], static_cast<float>(am[flat / a.bs]));
    sum = __fadd_rn(sum, __fmul_rn(static_cast<float>(A[m * a.K + k]), w));
  }
  static_cast<T*>(a.Y)[i] = static_cast<T>(sum);
}

#ifndef XRMM_BNB_PIN
#define XRMM_BNB_PIN 2  // columns whose table lookups may be in flight together
#endif

constexpr int BNB_RPW = 8;  // output columns per wave
constexpr int BNB_CPC = 32;  // codes per 16-byte chunk

// Fast GEMV: workgroup (b % ctiles, b / ctiles) covers columns
// [ctile * 32, +32) and A rows [rgroup * MR, +MR); each wave owns 8 columns,
// its lanes split K into 16-byte chunks, one step of 64 chunks per unit with
// the next step's codes and absmax in flight. A rows live in LDS as float32 in
// a padded chunk layout (stride 36 floats per chunk: conflict-free 16-byte
// reads); the 16-entry codebook sits beside them.
template <typename T, int MR, int NS>
__global__ __launch_bounds__(QT) void k_bnb4_gemv(Bnb4Args a, int ctiles) {
  extern __shared__ __align__(16) float xs[];  // [MR][steps * 64 * 36], then the table
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t bid = xcd_slot(blockIdx.x, gridDim.x);
  const int ctile = static_cast<int>(bid % static_cast<uint32_t>(ctiles));
  const int64_t m0 = static_cast<int64_t>(bid / static_cast<uint32_t>(ctiles)) * MR;
  const int K = static_cast<int>(a.K), N = static_cast<int>(a.N);
  const uint32_t colb = static_cast<uint32_t>(K / 2);  // bytes of one column
  const uint32_t chunks = colb / 16;
  const int steps = static_cast<int>((chunks + 63) / 64);
  const int per_row = steps * 64 * (BNB_CPC + 4);
  float* tbl = xs + MR * per_row;
  const float* book = a.qt == 1 ? kNF4 : kFP4;
  const T* A = static_cast<const T*>(a.A);

  const int n0 = (ctile * 4 + wave) * BNB_RPW;
  const uint32_t apc = static_cast<uint32_t>(K / a.bs);  // absmax blocks per column
  const rsrc_t rB = mk_rsrc(a.B, static_cast<uint32_t>(N) * colb);
  const rsrc_t rS = mk_rsrc(a.absmax, static_cast<uint32_t>(N) * apc * static_cast<uint32_t>(sizeof(T)));
  struct Buf {
    u32x4 w[BNB_RPW];
    float s[BNB_RPW][NS];
  };
  auto ld_scale = [&](uint32_t voff, uint32_t soff) -> float {
    if constexpr (sizeof(T) == 4) {
      return __builtin_bit_cast(float, bld_u32(rS, voff, soff));
    } else {
      return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(bld_u16(rS, voff, soff))));
    }
  };
  auto issue = [&](Buf& b, int s) {
    const uint32_t c = static_cast<uint32_t>(s) * 64u + static_cast<uint32_t>(lane);
    const bool in = s < steps && c < chunks;
    const uint32_t voff = in ? c * 16u : 0x80000000u;
#pragma unroll
    for (int r = 0; r < BNB_RPW; ++r) b.w[r] = bld16_nt(rB, voff, static_cast<uint32_t>(min(n0 + r, N - 1)) * colb);
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const uint32_t so = in ? ((c * BNB_CPC + q * (BNB_CPC / NS)) / static_cast<uint32_t>(a.bs)) * sizeof(T) : 0x80000000u;
#pragma unroll
      for (int r = 0; r < BNB_RPW; ++r)
        b.s[r][q] = ld_scale(so, static_cast<uint32_t>(min(n0 + r, N - 1)) * apc * static_cast<uint32_t>(sizeof(T)));
    }
  };

  float acc[MR][BNB_RPW];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int r = 0; r < BNB_RPW; ++r) acc[m][r] = 0.f;

  auto consume = [&](const Buf& b, int s) {
    const float* xq = xs + (static_cast<int64_t>(s) * 64 + lane) * (BNB_CPC + 4);
    float part[MR][BNB_RPW];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int r = 0; r < BNB_RPW; ++r) part[m][r] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {  // 8 codes per dword: flat order hi(b0) lo(b0) hi(b1) lo(b1) ...
      float xv[MR][8];
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float4 u = *reinterpret_cast<const float4*>(xq + m * per_row + d * 8);
        const float4 v = *reinterpret_cast<const float4*>(xq + m * per_row + d * 8 + 4);
        xv[m][0] = u.x; xv[m][1] = u.y; xv[m][2] = u.z; xv[m][3] = u.w;
        xv[m][4] = v.x; xv[m][5] = v.y; xv[m][6] = v.z; xv[m][7] = v.w;
      }
#pragma unroll
      for (int r = 0; r < BNB_RPW; ++r) {
        const uint32_t w = b.w[r][d];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t code = (w >> (8 * (i >> 1) + ((i & 1) ? 0 : 4))) & 15u;
          const float val = tbl[code];
#pragma unroll
          for (int m = 0; m < MR; ++m) part[m][r] = __builtin_fmaf(val, xv[m][i], part[m][r]);
        }
        if (NS == 2 && d == 1) {  // first of two absmax blocks complete
#pragma unroll
          for (int m = 0; m < MR; ++m) {
            acc[m][r] = __builtin_fmaf(b.s[r][0], part[m][r], acc[m][r]);
            part[m][r] = 0.f;
          }
        }
        // XRMM_BNB_PIN columns' lookups and products at a time: the empty asm
        // makes their partial sums live here, so the products cannot sink
        // past later lookups and the table reads in flight (and their
        // registers) stay bounded
        if ((r + 1) % XRMM_BNB_PIN == 0) {
#pragma unroll
          for (int rr = r + 1 - XRMM_BNB_PIN; rr <= r; ++rr)
#pragma unroll
            for (int m = 0; m < MR; ++m) asm volatile("" : "+v"(part[m][rr]));
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int r = 0; r < BNB_RPW; ++r) acc[m][r] = __builtin_fmaf(b.s[r][NS - 1], part[m][r], acc[m][r]);
  };

  Buf buf[2];
  issue(buf[0], 0);  // the first codes are in flight while A is staged

  // table and A rows -> LDS (float32, zero past K and past M): loads of four
  // 8-element pieces per thread in flight before their stores
  if (tid < 16) tbl[tid] = book[tid];
  {
    const int per_piece = 8, pieces = steps * 64 * BNB_CPC / per_piece;
    for (int m = 0; m < MR; ++m) {
      const bool live = m0 + m < a.M;
      const T* src = A + (m0 + m) * a.K;
      for (int p0 = 0; p0 < pieces; p0 += 4 * QT) {
        float v[4][per_piece];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int piece = p0 + j * QT + tid;
          const int k0 = piece * per_piece;
          if (live && k0 < K) {  // K is a multiple of 32: whole pieces
            if constexpr (sizeof(T) == 4) {
              const float4 u = *reinterpret_cast<const float4*>(src + k0);
              const float4 w = *reinterpret_cast<const float4*>(src + k0 + 4);
              v[j][0] = u.x; v[j][1] = u.y; v[j][2] = u.z; v[j][3] = u.w;
              v[j][4] = w.x; v[j][5] = w.y; v[j][6] = w.z; v[j][7] = w.w;
            } else {
              const f16x8 h = *reinterpret_cast<const f16x8*>(src + k0);
#pragma unroll
              for (int e = 0; e < 8; ++e) v[j][e] = static_cast<float>(h[e]);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[j][e] = 0.f;
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int piece = p0 + j * QT + tid;
          if (piece < pieces) {
            const int k0 = piece * per_piece;  // 8 floats inside one 32-code chunk
            float* dst = xs + m * per_row + (k0 / BNB_CPC) * (BNB_CPC + 4) + k0 % BNB_CPC;
            *reinterpret_cast<float4*>(dst) = float4{v[j][0], v[j][1], v[j][2], v[j][3]};
            *reinterpret_cast<float4*>(dst + 4) = float4{v[j][4], v[j][5], v[j][6], v[j][7]};
          }
        }
      }
    }
  }
  __syncthreads();

  for (int s = 0; s < steps; s += 2) {
    issue(buf[1], s + 1);
    __builtin_amdgcn_sched_barrier(0);
    consume(buf[0], s);
    issue(buf[0], s + 2);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < steps) consume(buf[1], s + 1);
  }

  const int n = n0 + row8(lane);
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const float v = reduce8(acc[m], lane);
    if ((lane & 7) == 0 && n < N && m0 + m < a.M) static_cast<T*>(a.Y)[(m0 + m) * a.N + n] = static_cast<T>(v);
  }
}

template <typename T, int MR>
hipError_t launch_bnb4_fast(const Bnb4Args& a, hipStream_t st) {
  const int64_t ctiles = (a.N + 31) / 32;
  const int64_t groups = (a.M + MR - 1) / MR;
  const int64_t steps = (a.K / 32 + 63) / 64;
  const size_t lds = static_cast<size_t>(MR * steps * 64 * (BNB_CPC + 4) + 16) * sizeof(float);
  const dim3 grid(static_cast<uint32_t>(ctiles * groups));
  if (a.bs == 16) {
    auto kern = k_bnb4_gemv<T, MR, 2>;
    static std::atomic<int> done[kMaxDevices];  // per instantiation and device
    if (lds > 64 * 1024) (void)raise_lds_cap(reinterpret_cast<const void*>(kern), 160 * 1024, done);
    hipLaunchKernelGGL(kern, grid, dim3(QT), lds, st, a, static_cast<int>(ctiles));
  } else {
    auto kern = k_bnb4_gemv<T, MR, 1>;
    static std::atomic<int> done[kMaxDevices];  // per instantiation and device
    if (lds > 64 * 1024) (void)raise_lds_cap(reinterpret_cast<const void*>(kern), 160 * 1024, done);
    hipLaunchKernelGGL(kern, grid, dim3(QT), lds, st, a, static_cast<int>(ctiles));
  }
  return hipGetLastError();
}

int bnb4_rows_per_pass(int64_t M) { return M <= 1 ? 1 : M == 2 ? 2 : 4; }

}  // namespace

bool gbq_fast_ok(const GbqArgs& a) {
  const auto al = [](const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; };
  return a.pcols % 4 == 0 && al(a.data, 4) && al(a.out, 16) && a.bs >= 16;
}

hipError_t launch_gbq(const GbqArgs& a, hipStream_t st) {
  if (a.n == 0 || a.width == 0) return hipSuccess;
  if (gbq_fast_ok(a)) {
    const int64_t bpr = (a.pcols / 4 + QT - 1) / QT;
    if (a.n * bpr > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;  // launch limit
    const dim3 grid(static_cast<uint32_t>(a.n * bpr));
    if (a.bits == 4)
      hipLaunchKernelGGL(k_gbq_words<4>, grid, dim3(QT), 0, st, a, bpr);
    else
      hipLaunchKernelGGL(k_gbq_words<8>, grid, dim3(QT), 0, st, a, bpr);
    return hipGetLastError();
  }
  if ((a.n * a.width + QT - 1) / QT > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;  // launch limit
  hipLaunchKernelGGL(k_gbq_scalar, dim3(static_cast<uint32_t>((a.n * a.width + QT - 1) / QT)), dim3(QT), 0, st, a);
  return hipGetLastError();
}

bool bnb4_fast_ok(const Bnb4Args& a) {
  if (!a.tb || a.K % 32 != 0 || a.K % a.bs != 0 || !(a.bs == 16 || a.bs % 32 == 0)) return false;
  if ((reinterpret_cast<uintptr_t>(a.B) & 15) != 0 || (reinterpret_cast<uintptr_t>(a.A) & 15) != 0) return false;
  if (a.N * (a.K / 2) >= (int64_t(1) << 31) || a.K > (int64_t(1) << 20)) return false;
  const int64_t steps = (a.K / 32 + 63) / 64;
  const int64_t lds = (bnb4_rows_per_pass(a.M) * steps * 64 * (BNB_CPC + 4) + 16) * 4;
  return lds <= 160 * 1024 && (a.N + 31) / 32 * ((a.M + 3) / 4) < (int64_t(1) << 31);
}

hipError_t launch_bnb4(const Bnb4Args& a, hipStream_t st) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  if (bnb4_fast_ok(a)) {
    const int mr = bnb4_rows_per_pass(a.M);
    if (a.f16) {
      if (mr == 1) return launch_bnb4_fast<f16, 1>(a, st);
      if (mr == 2) return launch_bnb4_fast<f16, 2>(a, st);
      return launch_bnb4_fast<f16, 4>(a, st);
    }
    if (mr == 1) return launch_bnb4_fast<float, 1>(a, st);
    if (mr == 2) return launch_bnb4_fast<float, 2>(a, st);
    return launch_bnb4_fast<float, 4>(a, st);
  }
  if ((a.M * a.N + QT - 1) / QT > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;  // launch limit
  const dim3 grid(static_cast<uint32_t>((a.M * a.N + QT - 1) / QT));
  if (a.f16)
    hipLaunchKernelGGL(k_bnb4_scalar<f16>, grid, dim3(QT), 0, st, a);
  else
    hipLaunchKernelGGL(k_bnb4_scalar<float>, grid, dim3(QT), 0, st, a);
  return hipGetLastError();
}

}  // namespace xrmm
