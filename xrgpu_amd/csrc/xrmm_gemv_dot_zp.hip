// One zero-point kind of the dot GEMV family; the build compiles this file
// once per kind with -DXRMM_ZPK=<0|1|2>.
#include "xrmm_gemv_dot.h"

#ifndef XRMM_ZPK
#error "XRMM_ZPK must be defined"
#endif

namespace xrmm {

template <>
hipError_t launch_dot_for<XRMM_ZPK>(const Launch& L, hipStream_t st) {
  if (L.op == OP_QKV)
    return L.block_size >= 32 ? launch_dot2<XRMM_ZPK, 1, OP_QKV>(L, st) : launch_dot2<XRMM_ZPK, 2, OP_QKV>(L, st);
  return L.block_size >= 32 ? launch_dot2<XRMM_ZPK, 1, OP_MATMUL>(L, st) : launch_dot2<XRMM_ZPK, 2, OP_MATMUL>(L, st);
}

}  // namespace xrmm
