// fp32 GEMM / conv instantiations of the contraction kernels (see gemm_kernels.h).
#include "gemm_kernels.h"

namespace c3h {
namespace gk {

// Direct fp32 convolution for 4-channel packed inputs (c_pack = c_stride =
// 4: the 3-channel first conv of the CIFAR ResNet).  With K = kh * kw * 4 the
// implicit-GEMM tiles do little useful work per address computation (that
// conv ran at 7 TFLOP/s, 129 us for 67 MB of output), so here each thread
// computes 16 output channels of one pixel with VALU FMAs: per filter tap one
// 16-byte load of the pixel's 4 channels, times the weights held transposed
// ([K][o]) in LDS, where a 16-channel weight row is four ds_read_b128 that
// the wave's lanes of one channel group share.  Each output sums its K
// products in K order (tap-major, channel-minor), one rounding per FMA;
// the epilogue is apply_epilogue8, the arithmetic of every other path.
// TPP threads per pixel (o = 16 TPP); NHWC output.
template <int TPP>
__global__ void __launch_bounds__(256) conv_direct_c4_kernel(Problem p) {
  extern __shared__ float wt[];  // [K][o]
  const KArg<Problem>& pk = kernel_arg<Problem>();
  constexpr int O = 16 * TPP;
  const int K = p.kh * p.kw * 4;
  const float* w = static_cast<const float*>(p.b);
  for (int i = threadIdx.x; i < O * K; i += 256) {
    const int oc = i / K, k = i - oc * K;
    wt[k * O + oc] = w[static_cast<int64_t>(oc) * p.ldb + k];
  }
  __syncthreads();
  const int cg = threadIdx.x % TPP;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * (256 / TPP) + threadIdx.x / TPP;
  if (m >= p.m) return;  // no barrier follows
  const int wo_i = static_cast<int>(m % p.wo);
  const int64_t t = m / p.wo;
  const int ho_i = static_cast<int>(t % p.ho);
  const int64_t ni = t / p.ho;
  const float* x = static_cast<const float*>(p.a);
  float acc[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
  for (int i = 0; i < p.kh; ++i) {
    const int hi = ho_i * p.sh - p.pt + i * p.dh;
    if (hi < 0 || hi >= p.ch) continue;
    for (int j = 0; j < p.kw; ++j) {
      const int wi = wo_i * p.sw - p.pl + j * p.dw;
      if (wi < 0 || wi >= p.cw) continue;
      const float4 xv = *reinterpret_cast<const float4*>(x + ((ni * p.ch + hi) * p.cw + wi) * 4);
      const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
      const float* wrow = wt + (i * p.kw + j) * 4 * O + 16 * cg;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const float4 wv = *reinterpret_cast<const float4*>(wrow + c * O + 4 * q4);
          acc[4 * q4 + 0] = fmaf(xs[c], wv.x, acc[4 * q4 + 0]);
          acc[4 * q4 + 1] = fmaf(xs[c], wv.y, acc[4 * q4 + 1]);
          acc[4 * q4 + 2] = fmaf(xs[c], wv.z, acc[4 * q4 + 2]);
          acc[4 * q4 + 3] = fmaf(xs[c], wv.w, acc[4 * q4 + 3]);
        }
      }
    }
  }
  float* out = static_cast<float*>(p.out);
  const float* resp = static_cast<const float*>(pk.epi.residual);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t n = 16 * cg + 8 * h;
    float res[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (resp) Elem<float>::load8(resp + m * O + n, res);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = acc[8 * h + e];
    apply_epilogue8(pk.epi, v, m, n, O, res, 0);
    Elem<float>::store8(out + m * O + n, v);
  }
}

// *handled = false (return 0) when the direct kernel does not apply; else
// the launch's status (0 or a negative C3H_ error).
int launch_conv_direct_c4(Problem p, hipStream_t s, bool* handled) {
  *handled = false;
  const int64_t k = static_cast<int64_t>(p.kh) * p.kw * 4;
  const size_t smem = static_cast<size_t>(p.n * k) * sizeof(float);
  const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  if (switches().disable_direct_conv || p.c_pack != 4 || p.c_stride != 4 || p.out_nchw || p.ldo != p.n ||
      p.ldb < k || smem > 64 * 1024 || !al16(p.a) || !al16(p.out) || (p.epi.residual && !al16(p.epi.residual)))
    return 0;
  const int tpp = static_cast<int>(p.n / 16);
  if (p.n % 16 != 0 || (tpp != 1 && tpp != 2 && tpp != 4 && tpp != 8 && tpp != 16)) return 0;
  const int64_t blocks = ceil_div(p.m, 256 / tpp);
  if (blocks > 2147483647LL) return 0;
  *handled = true;
  const dim3 g(static_cast<unsigned>(blocks)), b(256);
  switch (tpp) {
    case 1: hipLaunchKernelGGL(conv_direct_c4_kernel<1>, g, b, smem, s, p); break;
    case 2: hipLaunchKernelGGL(conv_direct_c4_kernel<2>, g, b, smem, s, p); break;
    case 4: hipLaunchKernelGGL(conv_direct_c4_kernel<4>, g, b, smem, s, p); break;
    case 8: hipLaunchKernelGGL(conv_direct_c4_kernel<8>, g, b, smem, s, p); break;
    default: hipLaunchKernelGGL(conv_direct_c4_kernel<16>, g, b, smem, s, p); break;
  }
  return launch_status("conv_direct_c4");
}

int launch_f32_modes(Problem p, int64_t batch, hipStream_t s, int am, bool b_kcontig) {
  if (am == kDenseM) return b_kcontig ? launch_f32<kDenseM, true>(p, batch, s) : launch_f32<kDenseM, false>(p, batch, s);
  if (am == kDenseK) return b_kcontig ? launch_f32<kDenseK, true>(p, batch, s) : launch_f32<kDenseK, false>(p, batch, s);
  if (am == kConv) return launch_f32<kConv, true>(p, batch, s);
  return fail(C3H_EUNSUPPORTED, "gemm_f32: unknown A mode %d", am);
}

}  // namespace gk
}  // namespace c3h
