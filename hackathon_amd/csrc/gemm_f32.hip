// fp32 GEMM / conv instantiations of the contraction kernels (see gemm_kernels.h).
#include "gemm_kernels.h"

namespace c3h {
namespace gk {

int launch_f32_modes(Problem p, int64_t batch, hipStream_t s, int am, bool b_kcontig) {
  if (am == kDenseM) return b_kcontig ? launch_f32<kDenseM, true>(p, batch, s) : launch_f32<kDenseM, false>(p, batch, s);
  if (am == kDenseK) return b_kcontig ? launch_f32<kDenseK, true>(p, batch, s) : launch_f32<kDenseK, false>(p, batch, s);
  if (am == kConv) return launch_f32<kConv, true>(p, batch, s);
  return fail(C3H_EUNSUPPORTED, "gemm_f32: unknown A mode %d", am);
}

}  // namespace gk
}  // namespace c3h
