// fp16 dense-GEMM instantiations of the contraction kernels (see gemm_kernels.h).
#include "gemm_kernels.h"

namespace c3h {
namespace gk {

int launch_f16_dense(Problem p, int64_t batch, hipStream_t s) {
  return launch_h<MmaF16, f16_t, kDenseK>(p, batch, s, C3H_F16);
}

}  // namespace gk
}  // namespace c3h
