// int8 GEMM instantiations of the contraction kernels (see gemm_kernels.h).
#include "gemm_kernels.h"

namespace c3h {
namespace gk {

int launch_i8(Problem p, hipStream_t s, int mode, int out_dtype) {
  if (mode == 0) return launch_mfma<MmaI8, int32_t, kDenseK>(p, 1, s, "qgemm");
  if (mode == 1 || out_dtype == C3H_I8) return launch_mfma<MmaI8, int8_t, kDenseK>(p, 1, s, "qgemm");
  if (out_dtype == C3H_F32) return launch_mfma<MmaI8, float, kDenseK>(p, 1, s, "qgemm");
  if (out_dtype == C3H_BF16) return launch_mfma<MmaI8, bf16_t, kDenseK>(p, 1, s, "qgemm");
  return launch_mfma<MmaI8, f16_t, kDenseK>(p, 1, s, "qgemm");
}

}  // namespace gk
}  // namespace c3h
