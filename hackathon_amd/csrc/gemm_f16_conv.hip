// fp16 implicit-GEMM conv instantiations of the contraction kernels (see gemm_kernels.h).
#include "gemm_kernels.h"

namespace c3h {
namespace gk {

int launch_f16_conv(Problem p, hipStream_t s, int am) {
  if (am == kConvTap) return launch_h<MmaF16, f16_t, kConvTap>(p, 1, s, C3H_F16);
  if (am == kConv) return launch_h<MmaF16, f16_t, kConv>(p, 1, s, C3H_F16);
  if (am == kConvStem) return launch_h<MmaF16, f16_t, kConvStem>(p, 1, s, C3H_F16);
  return fail(C3H_EUNSUPPORTED, "conv2d: unknown A mode %d", am);
}

}  // namespace gk
}  // namespace c3h
