// The float32-arithmetic MFMA GEMM for float16 activations (2- and 8-bit
// codes, and 4-bit ones whose weights binary16 cannot hold): its kernel
// instantiations, in a unit of their own so that they compile beside the
// float32 ones.
#include "xrmm_gemm_f32x.h"

namespace xrmm {
namespace fx {

hipError_t launch_gemm_f16(const Args& a, hipStream_t st) { return launch_gemm<f16>(a, st); }

}  // namespace fx
}  // namespace xrmm
