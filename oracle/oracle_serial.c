/* Serial float32 restatement of xrGPU's packedMatmul (test infrastructure only).
 *
 * This file is part of the oracle: only the tests and the CPU-baseline leg of
 * the benchmark load it; the product library never does.
 *
 * It follows the loop order and float32 arithmetic of
 *   kernels/_shared/extended/shaders/complex_kernel.glsl:80  nbitWeight
 *   kernels/_shared/extended/shaders/complex_kernel.glsl:81  packedInput
 *   kernels/_shared/extended/shaders/complex_kernel.glsl:83  packedMatmul
 *   kernels/_shared/extended/shaders/complex_kernel.glsl:39-47 fused/logistic
 * for opcodes 1025 (MatMulNBits), 1027 (Mlp) and 1028 (Qkv): one float32
 * accumulator per output, j walking K in order, sum += a*w.
 *
 * Differences from the shader, none of which change a result bit:
 *  - the RMS statistic of packedInput is computed once per row instead of once
 *    per (row, col, j); the serial float32 sum is the same value each time;
 *  - tensors arrive widened to float32 (f16 -> f32 is exact) and outputs leave
 *    as float32; the caller applies the single RNE rounding to binary16.
 *
 * Zero points: zp_kind 0 = none (2^(bits-1)), 1 = float [N,kb], 2 = packed
 * uint8 [N, ceil(kb*bits/8)] (ONNX Runtime layout, an extension).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

static float zero_point(int zp_kind, const float* zf, const uint8_t* zq, int64_t n, int64_t b,
                        int64_t kb, int bits) {
  if (zp_kind == 1) return zf[n * kb + b];
  if (zp_kind == 2) {
    int64_t row = (kb * bits + 7) / 8;
    uint8_t byte = zq[n * row + (b * bits) / 8];
    return (float)((byte >> ((b * bits) % 8)) & ((1u << bits) - 1u));
  }
  return (float)(1u << (bits - 1));
}

/* complex_kernel.glsl:80 */
static float nbit_weight(const uint8_t* B, const float* scales, int zp_kind, const float* zf,
                         const uint8_t* zq, int64_t col, int64_t k, int64_t K, int bits,
                         int64_t block) {
  int64_t blocks = (K + block - 1) / block, block_bytes = (block * bits + 7) / 8;
  int64_t element = k % block, shift = (element * bits) % 8;
  uint32_t packed = B[(col * blocks + k / block) * block_bytes + (element * bits) / 8];
  uint32_t q = (packed >> shift) & ((1u << bits) - 1u);
  float z = zero_point(zp_kind, zf, zq, col, k / block, blocks, bits);
  return ((float)q - z) * scales[col * blocks + k / block];
}

static float logistic(float x) { return x >= 0.f ? 1.f / (1.f + expf(-x)) : expf(x) / (1.f + expf(x)); }

/* complex_kernel.glsl:41-47 (erf form of gelu for opcode 1027) */
static float fused(float x, int kind) {
  if (kind == 1) return x > 0.f ? x : 0.f;
  if (kind == 2) return x * logistic(x);
  if (kind == 3) return .5f * x * (1.f + erff(x * .7071067811865475f));
  if (kind == 4) return tanhf(x);
  if (kind == 5) return logistic(x);
  return x;
}

/* Normalised input rows x[M,K] and residual r[M,K] (complex_kernel.glsl:81). */
static void packed_input(const float* A, const float* skip, const float* gamma, float eps,
                         int64_t M, int64_t K, float* x, float* r) {
  for (int64_t m = 0; m < M; ++m) {
    float square = 0.f;
    for (int64_t j = 0; j < K; ++j) {
      float a = A[m * K + j] + (skip ? skip[m * K + j] : 0.f);
      r[m * K + j] = a;
      square += a * a;
    }
    float inv = gamma ? 1.f / sqrtf(square / (float)K + eps) : 1.f;
    for (int64_t j = 0; j < K; ++j)
      x[m * K + j] = gamma ? r[m * K + j] * (inv * gamma[j]) : r[m * K + j];
  }
}

/* Opcode 1025: Y[M,N] = A @ W^T + bias. */
void oracle_matmul_nbits(const float* A, const uint8_t* B, const float* scales, int zp_kind,
                         const float* zf, const uint8_t* zq, const float* bias, float* Y,
                         int64_t M, int64_t K, int64_t N, int bits, int64_t block) {
  for (int64_t row = 0; row < M; ++row)
    for (int64_t col = 0; col < N; ++col) {
      float sum = 0.f;
      for (int64_t j = 0; j < K; ++j)
        sum += A[row * K + j] * nbit_weight(B, scales, zp_kind, zf, zq, col, j, K, bits, block);
      if (bias) sum += bias[col];
      Y[row * N + col] = sum;
    }
}

/* Opcode 1028: Q/K/V from one normalised input; x and r are [M,K] work arrays. */
void oracle_matmul_nbits_qkv(const float* A, const float* skip, const float* gamma, float eps,
                             const uint8_t* const* Bs, const float* const* Ss, int zp_kind,
                             const float* const* zfs, const uint8_t* const* zqs, float* Q,
                             float* Kout, float* V, float* residual, float* x, int64_t M,
                             int64_t K, int64_t Nq, int64_t Nkv, int bits, int64_t block) {
  packed_input(A, skip, gamma, eps, M, K, x, residual);
  float* outs[3] = {Q, Kout, V};
  for (int64_t row = 0; row < M; ++row)
    for (int branch = 0; branch < 3; ++branch) {
      int64_t n = branch ? Nkv : Nq;
      for (int64_t col = 0; col < n; ++col) {
        float sum = 0.f;
        for (int64_t j = 0; j < K; ++j)
          sum += x[row * K + j] * nbit_weight(Bs[branch], Ss[branch], zp_kind,
                                              zfs ? zfs[branch] : NULL, zqs ? zqs[branch] : NULL,
                                              col, j, K, bits, block);
        outs[branch][row * n + col] = sum;
      }
    }
}

/* Opcode 1027: Y = fused(g + gate_bias, act) * (u + up_bias). */
void oracle_matmul_nbits_mlp(const float* A, const float* skip, const float* gamma, float eps,
                             const uint8_t* gB, const float* gS, const float* gbias,
                             const uint8_t* uB, const float* uS, const float* ubias, int act,
                             float* Y, float* residual, float* x, int64_t M, int64_t K, int64_t N,
                             int bits, int64_t block) {
  packed_input(A, skip, gamma, eps, M, K, x, residual);
  for (int64_t row = 0; row < M; ++row)
    for (int64_t col = 0; col < N; ++col) {
      float sum = 0.f, up = 0.f;
      for (int64_t j = 0; j < K; ++j) {
        float a = x[row * K + j];
        sum += a * nbit_weight(gB, gS, 0, NULL, NULL, col, j, K, bits, block);
        up += a * nbit_weight(uB, uS, 0, NULL, NULL, col, j, K, bits, block);
      }
      Y[row * N + col] = fused(sum + (gbias ? gbias[col] : 0.f), act) * (up + (ubias ? ubias[col] : 0.f));
    }
}
