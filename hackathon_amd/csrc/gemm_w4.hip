// W4A16 (MXFP4 weights, fp16 activations) GEMM instantiations of the
// contraction kernels (see gemm_kernels.h).
#include "gemm_kernels.h"

namespace c3h {
namespace gk {

int launch_w4a16(Problem p, hipStream_t s, int out_dtype) {
  if (out_dtype == C3H_F32) return launch_w4<float>(p, s);
  return launch_w4<f16_t>(p, s);
}

}  // namespace gk
}  // namespace c3h
