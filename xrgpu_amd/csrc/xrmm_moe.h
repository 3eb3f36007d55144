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
  float* yp;             // workspace [T, k, ks, H]: FC2 partial outputs per slot and segment
  uint32_t* cnt;         // workspace: FC2 arrival counters [T, moe_tiles2(H)] or the grouped path's lists
  int64_t T, H, E, F1, I;
  int k, bits, bs, act;
  float alpha, beta, limit;
  int has_limit;
  int ks, seg, clear;    // FC2 reduction segments, steps per segment; FC1 clears cnt
  int lbs;               // log2(block_size) (block sizes are powers of two)
};

// Row tiles of the FC2 launch (32 rows each): one arrival counter per token
// and tile.
inline int64_t moe_tiles2(int64_t H) { return (H + 31) / 32; }

// FC2 splits its reduction into up to this many segments so that a small
// batch still launches about `wgs` (at most 1024) workgroups: steps is the
// number of 64-chunk steps of an FC2 row.
inline int64_t moe_fc2_segments_max(int64_t T, int64_t k, int64_t H, int64_t steps, int64_t wgs = 1024) {
  const int64_t base = T * k * moe_tiles2(H);
  if (base <= 0) return 1;
  if (wgs > 1024) wgs = 1024;
  int64_t ks = (wgs + base - 1) / base;
  if (ks > steps) ks = steps;
  return ks < 1 ? 1 : ks;
}

// Most experts the grouped-expert path takes (its per-expert counts live in
// LDS and its offsets in the workspace).
constexpr int64_t kMoeGroupMaxExperts = 4096;

// 32-bit words of the grouped path's lists: offsets and row-tile offsets
// (E + 1 each), the pair list and the per-pair |h| maxima (T k each) and the
// row exponents of x (T).
inline int64_t moe_list_words(int64_t T, int64_t k) { return 2 * (kMoeGroupMaxExperts + 1) + 2 * T * k + T; }

// K splits of the grouped path's FC2 GEMM (64-pair x 256-column tiles over
// K = I): enough for about 512 workgroups (two per CU) when the pairs would
// make fewer, four at most, each split at least 16 steps of 64. From the
// geometry alone (one tile per 64 pairs), so the workspace bound and the
// launch agree.
inline int64_t moe_group_fc2_splits(int64_t T, int64_t k, int64_t H, int64_t I) {
  const int64_t tiles = ((T * k + 63) / 64) * ((H + 255) / 256);
  if (tiles <= 0) return 1;
  int64_t s = (512 + tiles - 1) / tiles;
  if (s > 4) s = 4;
  if (s > I / 64 / 16) s = I / 64 / 16;
  return s < 1 ? 1 : s;
}

// FC2 partials per (token, slot) the workspace holds: the per-pair path's
// segment bound (8-bit rows, which have the most steps) or the grouped
// path's K splits, whichever is larger.
inline int64_t moe_yp_segments(int64_t T, int64_t k, int64_t H, int64_t I) {
  const int64_t a = moe_fc2_segments_max(T, k, H, (I + 1023) / 1024), b = moe_group_fc2_splits(T, k, H, I);
  return a > b ? a : b;
}

// Workspace bytes for T tokens, k slots, hidden width H, intermediate width
// I: five 256-byte-aligned regions (sel, wts, h, yp, cnt); the last region
// holds either path's words.
inline int64_t moe_workspace_bytes(int64_t T, int64_t k, int64_t H, int64_t I) {
  auto al = [](int64_t b) { return (b + 255) / 256 * 256; };
  const int64_t ks = moe_yp_segments(T, k, H, I);
  const int64_t words = T * moe_tiles2(H) > moe_list_words(T, k) ? T * moe_tiles2(H) : moe_list_words(T, k);
  return al(T * k * 4) + al(T * k * 4) + al(T * k * I * 4) + al(T * k * ks * H * 4) + al(words * 4);
}

bool moe_fast_ok(const MoeArgs& a);
const char* moe_kernel_name(const MoeArgs& a);
hipError_t launch_qmoe(const MoeArgs& a, hipStream_t st);

}  // namespace xrmm
