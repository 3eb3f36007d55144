// Internal interface of the QMoE path (xrmm_moe.hip): argument block, launch
// and kernel choice. Shared by the zero-copy entry and the operator lifecycle.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xrmm {

constexpr int XRMM_ACT_SWIGLU_CODE = 6;   // activation_lower code of swiglu (complex_plan.cpp:55)
constexpr int XRMM_ACT_RELU_CODE = 1;
constexpr int64_t kMoeMaxLds = 160 * 1024 - 1024;

struct MoeArgs {
  const float* x;        // [T, H]
  const float* router;   // [T, E]
  const uint8_t* fc1;    // [E, F1, H * bits / 8]
  const float* s1;       // [E, F1] (block_size 0) or [E, F1, H / block_size]
  const uint8_t* fc2;    // [E, H, I * bits / 8]
  const float* s2;       // [E, H] or [E, H, I / block_size]
  float* y;              // [T, H]
  int32_t* sel;          // workspace [T, k]: selected experts, ascending index
  float* wts;            // workspace [T, k]: their softmax weights
  float* h;              // workspace [T, k, I]: activated FC1 outputs
  int64_t T, H, E, F1, I;
  int k, bits, bs, act;
  float alpha, beta, limit;
  int has_limit;
};

// Workspace bytes for T tokens, k slots, intermediate width I (three
// 256-byte-aligned regions: sel, wts, h).
inline int64_t moe_workspace_bytes(int64_t T, int64_t k, int64_t I) {
  auto al = [](int64_t b) { return (b + 255) / 256 * 256; };
  return al(T * k * 4) + al(T * k * 4) + al(T * k * I * 4);
}

bool moe_fast_ok(const MoeArgs& a);
const char* moe_kernel_name(const MoeArgs& a);
hipError_t launch_qmoe(const MoeArgs& a, hipStream_t st);

}  // namespace xrmm
