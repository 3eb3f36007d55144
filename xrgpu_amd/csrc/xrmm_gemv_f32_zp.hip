// One zero-point kind of the float32-activation GEMV; the build compiles this
// file once per kind with -DXRMM_ZPK=<0|1|2>.
#include "xrmm_gemv_f32.h"

#ifndef XRMM_ZPK
#error "XRMM_ZPK must be defined"
#endif

namespace xrmm {

template <>
hipError_t launch_f32_for<XRMM_ZPK>(const Launch& L, hipStream_t st) {
  return launch_f32_1<XRMM_ZPK>(L, st);
}

}  // namespace xrmm
