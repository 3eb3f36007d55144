// One zero-point kind of the prefill GEMM; the build compiles this file once
// per kind with -DXRMM_ZPK=<0|1|2>.
#include "xrmm_gemm.h"
#include "xrmm_gemm_thin.h"

#ifndef XRMM_ZPK
#error "XRMM_ZPK must be defined"
#endif

namespace xrmm {

template <>
hipError_t launch_gemm_big_for<XRMM_ZPK>(const Launch& L, hipStream_t st) {
  return L.block_size >= 32 ? launch_gemm_big<XRMM_ZPK, 1>(L, st) : launch_gemm_big<XRMM_ZPK, 2>(L, st);
}

template <>
hipError_t launch_gemm_big_fused_for<XRMM_ZPK>(const Launch& L, hipStream_t st) {
  const bool one = L.block_size >= 32;
  if (L.op == OP_MLP)
    return one ? launch_gemm_big_fused<XRMM_ZPK, 1, OP_MLP>(L, st) : launch_gemm_big_fused<XRMM_ZPK, 2, OP_MLP>(L, st);
  return one ? launch_gemm_big_fused<XRMM_ZPK, 1, OP_QKV>(L, st) : launch_gemm_big_fused<XRMM_ZPK, 2, OP_QKV>(L, st);
}

template <>
hipError_t launch_gemm_big_pk_for<XRMM_ZPK>(const Launch& L, hipStream_t st) {
  return L.block_size >= 32 ? launch_gemm_big<XRMM_ZPK, 1, true>(L, st) : launch_gemm_big<XRMM_ZPK, 2, true>(L, st);
}

template <>
hipError_t launch_gemm_thin_for<XRMM_ZPK>(const Launch& L, hipStream_t st) {
  return launch_thin<XRMM_ZPK>(L, st);
}

}  // namespace xrmm
