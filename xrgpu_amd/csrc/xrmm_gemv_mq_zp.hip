// One zero-point kind of the four-row MFMA GEMV; the build compiles this file
// once per integer kind with -DXRMM_ZPK=<0|2>.
#include "xrmm_gemv_mq.h"

#ifndef XRMM_ZPK
#error "XRMM_ZPK must be defined"
#endif

namespace xrmm {

template <>
hipError_t launch_mq_for<XRMM_ZPK>(const Launch& L, hipStream_t st) {
  return L.op == OP_QKV ? launch_mq2<XRMM_ZPK, OP_QKV>(L, st) : launch_mq2<XRMM_ZPK, OP_MATMUL>(L, st);
}

}  // namespace xrmm
