// fp8 (E4M3) GEMM instantiations of the contraction kernels (see gemm_kernels.h).
#include "gemm_kernels.h"

namespace c3h {
namespace gk {

int launch_f8(Problem p, hipStream_t s, int out_dtype) {
  if (out_dtype == C3H_F32) return launch_fp8<float>(p, s);
  if (out_dtype == C3H_BF16) return launch_fp8<bf16_t>(p, s);
  return launch_fp8<f16_t>(p, s);
}

}  // namespace gk
}  // namespace c3h
