// One zero-point kind of the split-K GEMV family; the build compiles this file
// once per kind with -DXRMM_ZPK=<0|1|2>.
#include "xrmm_gemv_sk.h"

#ifndef XRMM_ZPK
#error "XRMM_ZPK must be defined"
#endif

namespace xrmm {

template <>
hipError_t launch_sk_for<XRMM_ZPK>(const Launch& L, hipStream_t st) {
  switch (L.op) {
    case OP_QKV: return launch_sk2<XRMM_ZPK, OP_QKV>(L, st);
    case OP_MLP: return launch_sk2<XRMM_ZPK, OP_MLP>(L, st);
    default: return launch_sk2<XRMM_ZPK, OP_MATMUL>(L, st);
  }
}

}  // namespace xrmm
