// One zero-point kind of the fused Qkv / Mlp prefill GEMM; the build compiles
// this file once per kind with -DXRMM_ZPK=<0|1|2>.
#include "xrmm_gemm_fused.h"

#ifndef XRMM_ZPK
#error "XRMM_ZPK must be defined"
#endif

namespace xrmm {

template <>
hipError_t launch_gemm_fused_for<XRMM_ZPK>(const Launch& L, hipStream_t st) {
  return launch_gemm_fused2<XRMM_ZPK>(L, st);
}

}  // namespace xrmm
