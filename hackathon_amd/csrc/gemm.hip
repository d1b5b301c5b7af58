// C entry points of the contraction kernels (GEMM, implicit-GEMM Conv2d,
// split-K, int8, fp8 and W4A16 GEMM).  The kernels and launch templates
// live in gemm_kernels.h; the per-type launchers are instantiated in
// gemm_bf16.hip, gemm_bf16_conv.hip, gemm_f16.hip, gemm_f16_conv.hip,
// gemm_i8.hip, gemm_f8.hip, gemm_w4.hip and gemm_f32.hip.
#include <stdlib.h>
#include <mutex>

#include "gemm_kernels.h"

using namespace c3h;
using namespace c3h::gk;

namespace {

// =====================================================================
// SIMT fp32 GEMM for operands the MFMA path cannot vector-load (odd K,
// misaligned rows): one thread per output, same epilogue.
// =====================================================================
__global__ void __launch_bounds__(256) gemm_simple_kernel(Problem p) {
  const int64_t bz = blockIdx.z;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x & 15);
  const int64_t m = static_cast<int64_t>(blockIdx.y) * 16 + (threadIdx.x >> 4);
  if (m >= p.m || n >= p.n) return;
  const float* A = static_cast<const float*>(p.a) + bz * p.stride_a;
  const float* B = static_cast<const float*>(p.b) + bz * p.stride_b;
  float acc = 0.0f;
  for (int64_t k = 0; k < p.k; ++k) {
    const float av = p.trans_a ? A[k * p.lda + m] : A[m * p.lda + k];
    const float bv = p.trans_b ? B[n * p.ldb + k] : B[k * p.ldb + n];
    acc = fmaf(av, bv, acc);
  }
  float* outp = static_cast<float*>(p.out) + bz * p.stride_out;
  const int64_t o = m * p.ldo + n;
  const float res = p.epi.residual ? static_cast<const float*>(p.epi.residual)[bz * p.stride_res + o] : 0.0f;
  outp[o] = apply_epilogue(kernel_arg<Problem>().epi, acc, m, n, p.n, res, bz * p.stride_bias);
}

}  // namespace

extern "C" {

int c3h_gemm(const c3h_gemm_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr, "gemm: null args");
  C3H_REQUIRE(a->m >= 0 && a->n >= 0 && a->k >= 0 && a->batch >= 1, "gemm: bad sizes");
  C3H_REQUIRE(a->batch <= 65535, "gemm: batch %lld too large", static_cast<long long>(a->batch));
  int rc = check_epilogue(a->epi, a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16);
  if (rc) return rc;
  rc = check_row_max(a->epi, a->n, a->ldo, a->out, a->out_dtype, a->batch);
  if (rc) return rc;
  if (a->m == 0 || a->n == 0) return C3H_OK;
  C3H_REQUIRE(a->k >= 1, "gemm: k must be >= 1 for a non-empty output");
  C3H_REQUIRE(a->ldo >= a->n, "gemm: ldo < n");
  Problem p;
  memset(&p, 0, sizeof(p));
  p.a = a->a; p.b = a->b; p.out = a->out;
  p.m = a->m; p.n = a->n; p.k = a->k;
  p.lda = a->lda; p.ldb = a->ldb; p.ldo = a->ldo;
  p.stride_a = a->stride_a; p.stride_b = a->stride_b; p.stride_out = a->stride_out;
  p.stride_bias = a->stride_bias; p.stride_res = a->stride_res;
  p.trans_a = a->trans_a; p.trans_b = a->trans_b;
  p.out_dtype = a->out_dtype;
  p.epi = a->epi;
  p.ho = 1; p.wo = 1;
  {
    const int es = dtype_size(a->in_dtype);
    p.a_bytes = ((a->m - 1) * a->lda + a->k) * es;
    p.b_bytes = ((a->n - 1) * a->ldb + a->k) * es;
  }
  int64_t tiles = ceil_div(a->m, 64) * ceil_div(a->n, 64);
  C3H_REQUIRE(tiles < (1LL << 31), "gemm: too many tiles");
  hipStream_t s = as_stream(stream);
  if (a->in_dtype == C3H_F32) {
    C3H_REQUIRE(a->out_dtype == C3H_F32, "gemm: fp32 inputs require fp32 output");
    // float4 global loads need 16-byte aligned rows on the contiguous side.
    bool a_ok = aligned(a->a, 16) && (a->lda % 4 == 0) && (a->stride_a % 4 == 0);
    bool b_ok = aligned(a->b, 16) && (a->ldb % 4 == 0) && (a->stride_b % 4 == 0);
    if (!(a_ok && b_ok) || a->m * a->n * a->batch < 4096) {
      dim3 grid(static_cast<unsigned>(ceil_div(a->n, 16)), static_cast<unsigned>(ceil_div(a->m, 16)),
                static_cast<unsigned>(a->batch));
      C3H_REQUIRE(grid.y <= 65535, "gemm_simple: m too large");
      hipLaunchKernelGGL(gemm_simple_kernel, grid, dim3(256), 0, s, p);
      return launch_status("gemm_simple");
    }
    if (a->trans_a) {
      return launch_f32_modes(p, a->batch, s, kDenseM, a->trans_b != 0);
    }
    return launch_f32_modes(p, a->batch, s, kDenseK, a->trans_b != 0);
  }
  if (a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16) {
    C3H_REQUIRE(!a->trans_a && a->trans_b, "gemm: 16-bit path needs A [m,k] and B packed [n,k] (trans_b=1)");
    C3H_REQUIRE(a->k % 8 == 0 && a->lda % 8 == 0 && a->ldb % 8 == 0 && a->stride_a % 8 == 0 && a->stride_b % 8 == 0,
                "gemm: 16-bit path needs k, lda, ldb multiples of 8");
    C3H_REQUIRE(aligned(a->a, 16) && aligned(a->b, 16), "gemm: 16-bit operands must be 16-byte aligned");
    return a->in_dtype == C3H_BF16 ? launch_bf16_dense(p, a->batch, s) : launch_f16_dense(p, a->batch, s);
  }
  return fail(C3H_EUNSUPPORTED, "gemm: input dtype %d unsupported", a->in_dtype);
}

int c3h_conv2d(const c3h_conv_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr, "conv2d: null args");
  C3H_REQUIRE(a->n >= 0 && a->c >= 1 && a->h >= 1 && a->w_ >= 1 && a->o >= 1, "conv2d: bad sizes");
  C3H_REQUIRE(a->kh >= 1 && a->kw >= 1 && a->sh >= 1 && a->sw >= 1 && a->dh >= 1 && a->dw >= 1, "conv2d: bad kernel");
  C3H_REQUIRE(a->ho >= 1 && a->wo >= 1, "conv2d: bad output size");
  C3H_REQUIRE(a->c_stride >= a->c && a->c_pack >= a->c, "conv2d: c_stride/c_pack < c");
  int rc = check_epilogue(a->epi);
  if (rc) return rc;
  if (a->n == 0) return C3H_OK;
  Problem p;
  memset(&p, 0, sizeof(p));
  p.a = a->x; p.b = a->w; p.out = a->out;
  p.cn = a->n; p.cc = a->c; p.ch = a->h; p.cw = a->w_;
  p.c_stride = a->c_stride; p.c_pack = a->c_pack;
  p.kh = a->kh; p.kw = a->kw; p.sh = a->sh; p.sw = a->sw;
  p.pt = a->pad_top; p.pl = a->pad_left; p.dh = a->dh; p.dw = a->dw;
  p.ho = a->ho; p.wo = a->wo;
  p.out_nchw = a->out_layout == 0;
  p.out_dtype = a->out_dtype;
  p.epi = a->epi;
  p.m = static_cast<int64_t>(a->n) * a->ho * a->wo;
  p.n = a->o;
  p.ldo = a->o;
  p.a_bytes = static_cast<int64_t>(a->n) * a->h * a->w_ * a->c_stride * dtype_size(a->in_dtype);
  C3H_REQUIRE(p.m < (int64_t{1} << 31), "conv2d: n*ho*wo must be below 2^31");
  C3H_REQUIRE(static_cast<int64_t>(a->kh) * (a->kw + 8) * a->c_pack < (int64_t{1} << 31), "conv2d: K too large");
  p.fd_hw = make_fastdiv(static_cast<uint32_t>(a->ho * a->wo));
  p.fd_wo = make_fastdiv(static_cast<uint32_t>(a->wo));
  p.fd_cpack = make_fastdiv(static_cast<uint32_t>(a->c_pack));
  hipStream_t s = as_stream(stream);
  if (a->in_dtype == C3H_F32) {
    // Packed K order (kh, kw, c_pack); 4-wide vectors must stay in one pixel.
    C3H_REQUIRE(a->c_pack % 4 == 0 && a->c_stride % 4 == 0, "conv2d fp32: c_pack and c_stride must be multiples of 4");
    C3H_REQUIRE(a->out_dtype == C3H_F32, "conv2d fp32: output must be fp32");
    C3H_REQUIRE(aligned(a->x, 16) && aligned(a->w, 16), "conv2d fp32: x and w must be 16-byte aligned");
    p.kw_pack = a->kw;
    p.fd_kwpack = make_fastdiv(static_cast<uint32_t>(p.kw_pack));
    p.k = static_cast<int64_t>(a->kh) * a->kw * a->c_pack;
    p.ldb = p.k;
    bool handled = false;
    rc = launch_conv_direct_c4(p, s, &handled);  // 4-channel inputs: direct VALU conv
    if (handled) return rc;
    return launch_f32_modes(p, 1, s, kConv, true);
  }
  if (a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16) {
    C3H_REQUIRE(aligned(a->x, 16) && aligned(a->w, 16), "conv2d: x and w must be 16-byte aligned");
    if (a->c_pack % 8 == 0 && a->c_stride % 8 == 0) {
      p.kw_pack = a->kw;
      p.fd_kwpack = make_fastdiv(static_cast<uint32_t>(p.kw_pack));
      p.k = static_cast<int64_t>(a->kh) * a->kw * a->c_pack;
      p.ldb = ceil_div(p.k, 32) * 32;  // weights padded to whole 32-wide K tiles
      p.b_bytes = static_cast<int64_t>(a->o) * p.ldb * 2;
      bool handled = false;
      rc = conv3x3_c64_launch(a, s, &handled);
      if (handled || rc) return rc;
      // A 64-wide K tile stays inside one filter tap when c_pack % 64 == 0.
      const int am = a->c_pack % 64 == 0 ? kConvTap : kConv;
      return a->in_dtype == C3H_BF16 ? launch_bf16_conv(p, s, am) : launch_f16_conv(p, s, am);
    }
    // Narrow-channel stem: c_pack = c_stride = 4, kw padded to a multiple of
    // 2 so each 32-wide K tile covers whole pixels (8-byte vectors).
    C3H_REQUIRE(a->c_pack == 4 && a->c_stride == 4, "conv2d: 16-bit path needs c_pack%8==0 or c_pack==c_stride==4");
    p.kw_pack = static_cast<int>(ceil_div(a->kw, 8) * 8);
    p.fd_kwpack = make_fastdiv(static_cast<uint32_t>(p.kw_pack));
    p.k = static_cast<int64_t>(a->kh) * p.kw_pack * 4;
    p.ldb = p.k;
    return a->in_dtype == C3H_BF16 ? launch_bf16_conv(p, s, kConvStem) : launch_f16_conv(p, s, kConvStem);
  }
  return fail(C3H_EUNSUPPORTED, "conv2d: input dtype %d unsupported", a->in_dtype);
}

int c3h_gemm_splitk_reduce(const c3h_splitk_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr && a->partial != nullptr && a->out != nullptr, "splitk_reduce: null args");
  C3H_REQUIRE(a->m >= 0 && a->n >= 0 && a->splits >= 1 && a->ldo >= a->n, "splitk_reduce: bad sizes");
  C3H_REQUIRE(a->out_dtype == C3H_F32 || a->out_dtype == C3H_BF16 || a->out_dtype == C3H_F16,
              "splitk_reduce: output dtype must be fp32, bf16 or fp16");
  int rc = check_epilogue(a->epi);
  if (rc) return rc;
  const int64_t mn = a->m * a->n;
  if (mn == 0) return C3H_OK;
  C3H_REQUIRE(ceil_div(mn, 256) < (int64_t{1} << 31), "splitk_reduce: too many outputs");
  const dim3 g(static_cast<unsigned>(ceil_div(mn, 256))), b(256);
  hipStream_t s = as_stream(stream);
  if (a->out_dtype == C3H_F32) hipLaunchKernelGGL(splitk_reduce_kernel<float>, g, b, 0, s, *a);
  else if (a->out_dtype == C3H_BF16) hipLaunchKernelGGL(splitk_reduce_kernel<bf16_t>, g, b, 0, s, *a);
  else hipLaunchKernelGGL(splitk_reduce_kernel<f16_t>, g, b, 0, s, *a);
  return launch_status("splitk_reduce");
}

}  // extern "C"

namespace {

// Bytes of fp32 partials a split-K GEMM needs, or -1 if the sizes overflow.
int64_t splitk_partial_bytes(const c3h_gemm_args* a, int32_t splits) {
  if (a->m < 0 || a->n < 0 || splits < 1) return -1;
  const int64_t mn = a->m * a->n;
  if (a->n != 0 && mn / a->n != a->m) return -1;
  if (mn > (INT64_MAX / 4) / splits) return -1;
  return mn * splits * 4;
}

// The split-K GEMM over a given fp32 partial buffer (the caller has checked
// its size): `splits` batched partial GEMMs over K/splits each, plain
// epilogue, then the ordered reduce with a's epilogue.
int gemm_splitk_into(const c3h_gemm_args* a, int32_t splits, float* partial, hipStream_t s) {
  C3H_REQUIRE(a->batch == 1, "gemm_splitk: batch must be 1 (one GEMM split along K)");
  C3H_REQUIRE(splits >= 1 && splits <= 64, "gemm_splitk: splits %d outside [1, 64]", splits);
  C3H_REQUIRE(a->k >= splits && a->k % splits == 0, "gemm_splitk: k %lld is not a multiple of splits %d",
              static_cast<long long>(a->k), splits);
  C3H_REQUIRE(a->out_dtype == C3H_F32 || a->out_dtype == C3H_BF16 || a->out_dtype == C3H_F16,
              "gemm_splitk: output dtype must be fp32, bf16 or fp16");
  int rc = check_epilogue(a->epi);
  if (rc) return rc;
  if (a->m == 0 || a->n == 0) return C3H_OK;
  const int64_t ks = a->k / splits;
  c3h_gemm_args g = *a;
  g.out = partial;
  g.k = ks;
  g.ldo = a->n;
  g.batch = splits;
  g.stride_a = a->trans_a ? ks * a->lda : ks;
  g.stride_b = a->trans_b ? ks : ks * a->ldb;
  g.stride_out = a->m * a->n;
  g.stride_bias = g.stride_res = 0;
  g.out_dtype = C3H_F32;
  memset(&g.epi, 0, sizeof(g.epi));
  g.epi.alpha = 1.0f;
  g.epi.beta = 1.0f;
  rc = c3h_gemm(&g, s);
  if (rc) return rc;
  c3h_splitk_args r;
  memset(&r, 0, sizeof(r));
  r.partial = partial;
  r.out = a->out;
  r.m = a->m;
  r.n = a->n;
  r.ldo = a->ldo;
  r.splits = splits;
  r.out_dtype = a->out_dtype;
  r.epi = a->epi;
  return c3h_gemm_splitk_reduce(&r, s);
}

}  // namespace

// ---------------------------------------------------------------------
// Static split-K scratch for c3h_gemm_splitk_noalloc: fp32 partials live in
// this file-scope device array instead of a caller or library allocation.
// Each GPU the library runs on holds its own copy (kScratchBytes) until the
// process ends.  In host code `scratch` only names the symbol: its device
// address on a given GPU comes from hipGetSymbolAddress with that GPU
// current, kept per device in g_scratch_ptr, and only that address is ever
// passed to kernels.
// ---------------------------------------------------------------------
static constexpr int64_t kScratchBytes = int64_t{32} << 20;
static __device__ __align__(256) float scratch[kScratchBytes / 4];

namespace {
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The scratch address on the current device, resolved on first use.
int scratch_for_current(void** out) {
  int dev = 0;
  C3H_HIP_CHECK(hipGetDevice(&dev));
  C3H_REQUIRE(dev >= 0 && dev < kMaxDevices, "gemm scratch: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    C3H_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    C3H_REQUIRE(ptr != nullptr, "gemm scratch: hipGetSymbolAddress returned a null address on device %d", dev);
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return C3H_OK;
}
}  // namespace

namespace c3h {
int gemm_scratch_setup(int device) {
  int cur = -1;
  C3H_HIP_CHECK(hipGetDevice(&cur));
  C3H_REQUIRE(cur == device, "gemm scratch: device %d is not current (%d is)", device, cur);
  void* ptr = nullptr;
  return scratch_for_current(&ptr);
}
}  // namespace c3h

extern "C" {

int c3h_gemm_splitk_noalloc(const c3h_gemm_args* a, int32_t splits, void* stream) {
  C3H_REQUIRE(a != nullptr, "gemm_splitk_noalloc: null args");
  const int64_t need = splitk_partial_bytes(a, splits);
  C3H_REQUIRE(need >= 0, "gemm_splitk_noalloc: bad sizes or splits");
  C3H_REQUIRE(need <= kScratchBytes,
              "gemm_splitk_noalloc: the partials need %lld bytes (splits*m*n*4), above the %lld-byte static "
              "scratch; use c3h_gemm_splitk with a workspace",
              static_cast<long long>(need), static_cast<long long>(kScratchBytes));
  void* ptr = nullptr;
  int rc = scratch_for_current(&ptr);
  if (rc) return rc;
  return gemm_splitk_into(a, splits, static_cast<float*>(ptr), as_stream(stream));
}

int c3h_gemm_splitk(const c3h_gemm_args* a, int32_t splits, void* workspace, size_t workspace_bytes, void* stream) {
  C3H_REQUIRE(a != nullptr, "gemm_splitk: null args");
  const int64_t need = splitk_partial_bytes(a, splits);
  C3H_REQUIRE(need >= 0, "gemm_splitk: bad sizes or splits");
  C3H_REQUIRE(need == 0 || (workspace != nullptr && static_cast<int64_t>(workspace_bytes) >= need),
              "gemm_splitk: workspace of %zu bytes is smaller than the %lld bytes of partials (splits*m*n*4)",
              workspace_bytes, static_cast<long long>(need));
  C3H_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0, "gemm_splitk: workspace must be 16-byte aligned");
  return gemm_splitk_into(a, splits, static_cast<float*>(workspace), as_stream(stream));
}

int c3h_gemm_fp8(const c3h_fp8_gemm_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr, "gemm_fp8: null args");
  C3H_REQUIRE(a->m >= 0 && a->n >= 0 && a->k >= 1, "gemm_fp8: bad sizes");
  C3H_REQUIRE(a->k % 16 == 0 && a->lda % 16 == 0 && a->ldb % 16 == 0, "gemm_fp8: k, lda, ldb must be multiples of 16");
  C3H_REQUIRE(a->lda >= a->k && a->ldb >= a->k && a->ldo >= a->n, "gemm_fp8: leading dimension too small");
  C3H_REQUIRE(aligned(a->a, 16) && aligned(a->b, 16), "gemm_fp8: operands must be 16-byte aligned");
  C3H_REQUIRE(a->a_scale != nullptr && a->b_scale != nullptr && aligned(a->b_scale, 16),
              "gemm_fp8: a_scale and a 16-byte aligned b_scale are required");
  C3H_REQUIRE(a->out_dtype == C3H_F32 || a->out_dtype == C3H_BF16 || a->out_dtype == C3H_F16,
              "gemm_fp8: output dtype must be fp32, bf16 or fp16");
  C3H_REQUIRE(a->m < (int64_t{1} << 31) && a->n < (int64_t{1} << 31), "gemm_fp8: m and n must be below 2^31");
  int rc = check_epilogue(a->epi, true);
  if (rc) return rc;
  rc = check_row_max(a->epi, a->n, a->ldo, a->out, a->out_dtype, 1);
  if (rc) return rc;
  if (a->m == 0 || a->n == 0) return C3H_OK;
  C3H_REQUIRE(ceil_div(a->m, 64) * ceil_div(a->n, 64) < (int64_t{1} << 31), "gemm_fp8: too many tiles");
  Problem p;
  memset(&p, 0, sizeof(p));
  p.a = a->a; p.b = a->b; p.out = a->out;
  p.m = a->m; p.n = a->n; p.k = a->k; p.lda = a->lda; p.ldb = a->ldb; p.ldo = a->ldo;
  p.a_rows = a->a_scale; p.b_scale = a->b_scale;
  p.out_dtype = a->out_dtype;
  p.epi = a->epi;
  p.ho = 1; p.wo = 1;
  p.a_bytes = (a->m - 1) * a->lda + a->k;
  p.b_bytes = (a->n - 1) * a->ldb + a->k;
  hipStream_t s = as_stream(stream);
  return launch_f8(p, s, a->out_dtype);
}

int c3h_gemm_w4a16(const c3h_w4a16_gemm_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr, "gemm_w4a16: null args");
  C3H_REQUIRE(a->m >= 0 && a->n >= 0 && a->k >= 1, "gemm_w4a16: bad sizes");
  C3H_REQUIRE(a->k % 32 == 0, "gemm_w4a16: k must be a multiple of 32 (the MXFP4 block)");
  C3H_REQUIRE(a->lda % 8 == 0 && a->lda >= a->k, "gemm_w4a16: lda must be a multiple of 8 and >= k");
  C3H_REQUIRE(a->ldb % 4 == 0 && a->ldb >= a->k / 2, "gemm_w4a16: ldb (bytes) must be a multiple of 4 and >= k/2");
  C3H_REQUIRE(a->ldbs >= a->k / 32 && a->ldo >= a->n, "gemm_w4a16: ldbs >= k/32 and ldo >= n required");
  C3H_REQUIRE(aligned(a->a, 16) && aligned(a->b_codes, 4), "gemm_w4a16: A must be 16-byte and codes 4-byte aligned");
  C3H_REQUIRE(a->b_scales != nullptr, "gemm_w4a16: b_scales required");
  C3H_REQUIRE(a->out_dtype == C3H_F32 || a->out_dtype == C3H_F16, "gemm_w4a16: output dtype must be fp32 or fp16");
  int rc = check_epilogue(a->epi, true);
  if (rc) return rc;
  rc = check_row_max(a->epi, a->n, a->ldo, a->out, a->out_dtype, 1);
  if (rc) return rc;
  if (a->m == 0 || a->n == 0) return C3H_OK;
  const int64_t a_bytes = ((a->m - 1) * a->lda + a->k) * 2;
  const int64_t b_bytes = (a->n - 1) * a->ldb + a->k / 2;
  const int64_t s_bytes = (a->n - 1) * a->ldbs + a->k / 32;
  C3H_REQUIRE(a_bytes < (int64_t{1} << 31) && b_bytes < (int64_t{1} << 31) && s_bytes < (int64_t{1} << 31),
              "gemm_w4a16: A, codes and scales must each be below 2^31 bytes");
  C3H_REQUIRE(ceil_div(a->m, 64) * ceil_div(a->n, 64) < (int64_t{1} << 31), "gemm_w4a16: too many tiles");
  Problem p;
  memset(&p, 0, sizeof(p));
  p.a = a->a; p.b = a->b_codes; p.out = a->out;
  p.m = a->m; p.n = a->n; p.k = a->k; p.lda = a->lda; p.ldb = a->ldb; p.ldo = a->ldo;
  p.b_blk = a->b_scales; p.ldbs = a->ldbs; p.bs_bytes = s_bytes;
  p.trans_b = 1;
  p.out_dtype = a->out_dtype;
  p.epi = a->epi;
  p.ho = 1; p.wo = 1;
  p.a_bytes = a_bytes;
  p.b_bytes = b_bytes;
  return launch_w4a16(p, as_stream(stream), a->out_dtype);
}

int c3h_qgemm(const c3h_qgemm_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr, "qgemm: null args");
  C3H_REQUIRE(a->m >= 0 && a->n >= 0 && a->k >= 1, "qgemm: bad sizes");
  C3H_REQUIRE(a->a_zero == 0 && a->b_zero == 0, "qgemm: only symmetric (zero-point 0) operands are supported");
  C3H_REQUIRE(a->mode >= 0 && a->mode <= 3, "qgemm: bad mode %d", a->mode);
  C3H_REQUIRE(a->mode == 0 || a->b_scale != nullptr, "qgemm: b_scale required");
  C3H_REQUIRE((a->mode != 1 && a->mode != 3) || a->y_scale != 0.0f, "qgemm: y_scale must be nonzero");
  C3H_REQUIRE(a->k % 16 == 0 && a->lda % 16 == 0 && a->ldb % 16 == 0, "qgemm: k, lda, ldb must be multiples of 16");
  C3H_REQUIRE(aligned(a->a, 16) && aligned(a->b, 16), "qgemm: operands must be 16-byte aligned");
  C3H_REQUIRE(a->mode < 2 || a->out_dtype == C3H_F32 || a->out_dtype == C3H_BF16 || a->out_dtype == C3H_F16 ||
                  a->out_dtype == C3H_I8,
              "qgemm: dequantized output dtype must be float, or int8 (quantized again)");
  const bool requant_out = a->mode >= 2 && a->out_dtype == C3H_I8;
  C3H_REQUIRE(!requant_out || (quant_scale_ok(a->q_scale) && a->q_zero >= -128 && a->q_zero <= 127),
              "qgemm: an int8 output of mode %d needs a positive normal q_scale and an int8 q_zero", a->mode);
  C3H_REQUIRE(!requant_out || a->act_dtype == C3H_F32 || a->act_dtype == C3H_BF16 || a->act_dtype == C3H_F16,
              "qgemm: act_dtype must be fp32, bf16 or fp16");
  C3H_REQUIRE(!requant_out || a->epi.residual == nullptr, "qgemm: no residual into an int8 output");
  int rc = check_epilogue(a->epi, a->mode >= 2 && a->out_dtype != C3H_I8);
  if (rc) return rc;
  rc = check_row_max(a->epi, a->n, a->ldo, a->out, a->out_dtype, 1);
  if (rc) return rc;
  if (a->m == 0 || a->n == 0) return C3H_OK;
  Problem p;
  memset(&p, 0, sizeof(p));
  p.a = a->a; p.b = a->b; p.out = a->out;
  p.m = a->m; p.n = a->n; p.k = a->k; p.lda = a->lda; p.ldb = a->ldb; p.ldo = a->ldo;
  p.a_scale = a->a_scale; p.y_scale = a->y_scale; p.b_scale = a->b_scale;
  p.y_zero = a->y_zero; p.qmode = a->mode; p.out_dtype = a->out_dtype;
  p.q_scale = requant_out ? a->q_scale : 1.0f; p.q_zero = a->q_zero; p.act_dtype = a->act_dtype;
  p.q_mul = requant_out ? quant_multiplier(a->q_scale, a->q_zero, a->act_dtype) : 0.0f;
  p.epi = a->epi;
  p.ho = 1; p.wo = 1;
  p.a_bytes = (a->m - 1) * a->lda + a->k;
  p.b_bytes = (a->n - 1) * a->ldb + a->k;
  hipStream_t s = as_stream(stream);
  return launch_i8(p, s, a->mode, a->out_dtype);
}

}  // extern "C"
