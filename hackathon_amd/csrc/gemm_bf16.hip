// bf16 dense-GEMM instantiations of the contraction kernels (see gemm_kernels.h).
#include "gemm_kernels.h"

namespace c3h {
namespace gk {

int launch_bf16_dense(Problem p, int64_t batch, hipStream_t s) {
  return launch_h<MmaBF16, bf16_t, kDenseK>(p, batch, s, C3H_BF16);
}

}  // namespace gk
}  // namespace c3h
