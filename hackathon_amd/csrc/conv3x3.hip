// Spatially tiled 3x3 convolution for 64 -> 64 channels (gfx950), the
// 56x56 layer-1 convolutions of ResNet-18 224: Conv 3x3 / stride 1 / pad 1
// + per-channel bias (folded BatchNorm) + optional residual + optional ReLU,
// NHWC 16-bit activations, fp32 accumulation on v_mfma_f32_16x16x32_{bf16,f16}.
//
// The implicit-GEMM kernels (gemm.hip) gather each input pixel once per
// filter tap, so the 3x3 layer moves 9x its input through L2 -> LDS, and
// with N = 64 output channels every LDS byte feeds few MFMAs.  Here:
//   * a tile is a band of R full output rows of one image (R * W <= 112
//     pixels, 2 rows at W = 56); its (R + 2) x (W + 2) input patch, halo and
//     zero padding included, is brought into LDS once by buffer_load ... lds
//     (out-of-image pixels read zeros) and all nine taps read it from there;
//   * blocks are persistent, two per CU (60 KB of LDS each: two patch
//     stages; at most 256 registers per wave), and walk contiguous ranges
//     of bands: the next band's patch is in flight while the current one is
//     multiplied, one block's waits and epilogue overlap the other's MFMAs,
//     and the halo rows bands share were just fetched into this XCD's L2;
//   * each of the 4 waves keeps its 32 output channels' weights (all
//     K = 576) in registers as 36 MFMA fragments, loaded once per block;
//     waves are 2 (pixels) x 2 (channels), 64 pixels (the band padded to
//     128) x 32 channels each, so every A fragment read from LDS feeds two
//     MFMAs;
//   * the band's residual is loaded into registers before the MFMAs, and a
//     band's kTM output stores per wave stay in flight while the next band
//     is multiplied;
//   * residual loads and output stores move 16 bytes per lane, 8 channels
//     of one pixel (each wave's 64 bytes of a pixel in one access): two lane
//     swaps (permlane32 / permlane16) convert between that layout and the
//     MFMA accumulators' 4 channels per lane.
// The K order (tap-major, then channel chunks 0-31 and 32-63 with lane group
// g supplying chunk g) and the epilogue arithmetic ((acc + bias) + residual,
// then max 0) are those of the tap-uniform implicit-GEMM kernel, so the
// outputs are bit-identical to c3h_conv2d's generic path.
#include <type_traits>
#include <utility>

#include "common.h"

namespace c3h {
namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) int i32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((address_space(3))) void* lds_void_ptr;

constexpr int kC = 64;                 // input channels: one tap = one 128-byte pixel row
constexpr int kO = 64;                 // output channels
constexpr int kK = 9 * kC;             // 576
constexpr int kTilePix = 112;          // output pixels per band (7 MFMA row tiles, padded to 8)
constexpr int kWaves = 4;              // 2 (pixels) x 2 (channels)
constexpr int kWavePix = 64;           // 4 row tiles per wave (the band padded to 128 pixels)
constexpr int kTM = kWavePix / 16;     // 4
constexpr int kTN = 2;                 // 32 channels per wave
constexpr int kMaxPatch = 240;                           // patch pixels per stage
constexpr int kPitch = 144;                              // LDS bytes per patch pixel: 128 of channels + 16 of padding
constexpr int kGroups = (kMaxPatch * kPitch + 1023) / 1024;  // 34 DMA instructions of 1 KB per stage
constexpr int kSlots = (kGroups + kWaves - 1) / kWaves;  // 9 DMA slots per wave
constexpr int kStage = kGroups * 1024;                   // 34816 bytes: the last DMA stays inside its stage
static_assert(kMaxPatch * kPitch <= kStage, "patch fits a stage");
constexpr uint32_t kOob = 0x80000000u;  // buffer offset past num_records: reads zeros

struct Conv3x3Args {
  const void* x;
  const void* w;  // [64][576] packed (kh, kw, c)
  void* out;      // NHWC [n, h, w, 64]
  const float* bias;
  const void* residual;
  int n, h, wd, rows;  // wd: width; rows: output rows per band
  int bands, tiles;   // bands per image, n * bands
  int pw, npix;       // patch width w + 2, patch pixels (rows + 2) * pw
  uint32_t pw_magic;  // pix / pw == (pix * pw_magic) >> 20 for pix < kMaxPatch (checked on the host)
  int band_pix;       // rows * w
  int relu;
  int x_bytes;
};

// Calls f(integral_constant<0>) ... f(<N - 1>): indices that are constants
// before unrolling, so register arrays indexed by them stay in registers.
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <bool F16>
struct Frag {
  typedef typename std::conditional<F16, f16x8, bf16x8>::type vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    if constexpr (F16) return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// s_waitcnt vmcnt(N), lgkmcnt/expcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <bool F16>
__device__ __forceinline__ float to_f32(uint32_t bits) {
  if constexpr (F16) return f16_bits_to_f32(static_cast<uint16_t>(bits));
  else return bf16_bits_to_f32(static_cast<uint16_t>(bits));
}
template <bool F16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (F16) return f32x2_to_f16x2_bits(lo, hi);
  else return f32x2_to_bf16x2_bits(lo, hi);
}

template <typename T, bool F16>
__global__ void __launch_bounds__(kWaves * 64, 2) conv3x3_c64_kernel(Conv3x3Args p) {
  typedef typename Frag<F16>::vec vec;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, lg = lane >> 4;
  const int W = p.wd, H = p.h, pw = p.pw;

  // This wave's weights: output channel nb + 16 j + l16, K chunk 4 s + lg.
  vec bw[kTN][18];
  {
    const T* w = static_cast<const T*>(p.w);
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int s = 0; s < 18; ++s)
        bw[j][s] = *reinterpret_cast<const vec*>(w + (wn * 32 + 16 * j + l16) * kK + s * 32 + lg * 8);
  }

  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.x), 0, p.x_bytes, 0x00020000);
  // out and residual have x's extent (NHWC, 64 channels): below 2^31 bytes.
  const __amdgpu_buffer_rsrc_t rs_out = __builtin_amdgcn_make_buffer_rsrc(p.out, 0, p.x_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_res =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.residual), 0, p.x_bytes, 0x00020000);
  // LDS layout: patch pixel pix at byte pix * 144 (its 64 channels, then 16
  // bytes of padding).  Sixteen consecutive pixels then start on sixteen
  // different 16-byte bank groups, so fragment reads are conflict-free
  // without a swizzle, and a fragment's address is a per-lane base plus
  // constants.  DMA instruction g (slot j = (g - wave) / 4) fills stage
  // bytes [1024 g, 1024 g + 1024): lane l writes 16 bytes at 1024 g + 16 l,
  // which is chunk c = (byte % 144) / 16 of patch pixel byte / 144 (c = 8 is
  // the padding: read out of range, as are pixels past the patch and its
  // zero columns).  The pixel's patch row pr and its input offset relative
  // to (h0 - 1, 0) do not depend on the band; they are kept per slot as
  // pr << 16 | offset (pr = 0x7fff when the lane loads nothing, so the row
  // check fails), and a band costs an add, a mask, a compare and a select.
  int sdma[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    const int byte = (wave + kWaves * j) * 1024 + lane * 16;
    const int pix = byte / kPitch, c = (byte - pix * kPitch) >> 4;
    const int pr = static_cast<int>((static_cast<uint32_t>(pix) * p.pw_magic) >> 20);
    const int wi = pix - pr * pw - 1;
    const bool ok = wave + kWaves * j < kGroups && c < 8 && pix < p.npix &&
                    static_cast<unsigned>(wi) < static_cast<unsigned>(W);
    sdma[j] = ok ? (pr << 16) | ((pr * W + wi) * (kC * 2) + c * 16) : 0x7fff << 16;
  }
  auto issue = [&](int t, int buf) {
    const int img = t / p.bands, h0 = (t - img * p.bands) * p.rows;
    // byte offset of input pixel (h0 - 1, 0) of image img
    const int band_base = (img * H + h0 - 1) * W * (kC * 2);
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      const int g = wave + kWaves * j;
      uint8_t* dst = smem + buf * kStage + g * 1024;
      if (g < kGroups) {
        const int hi = h0 - 1 + (sdma[j] >> 16);
        const int off = band_base + (sdma[j] & 0xffff);
        const uint32_t voff = static_cast<unsigned>(hi) < static_cast<unsigned>(H) ? static_cast<uint32_t>(off) : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_ptr)dst, 16, voff, 0, 0, 0);
      }
    }
  };

  // LDS byte of output pixel q = wm * 64 + 16 i + l16's fragment chunk lg at
  // tap (0, 0) of stage 0; pixels past the band (the padding to 128, or a
  // band shorter than 112 pixels) read the band's last pixel and are never
  // stored.  A tap (kh, kw), K half ks and stage add (kh * pw + kw) * 144 +
  // 64 ks + stage * 34816: kh's part per band in a scalar register, the rest
  // as the read's immediate offset.
  uint32_t a0[kTM];
  const int band_pix = p.band_pix;
#pragma unroll
  for (int i = 0; i < kTM; ++i) {
    const int q = min(wm * kWavePix + 16 * i + l16, band_pix - 1);
    const int r = q / W;
    a0[i] = static_cast<uint32_t>((r * pw + (q - r * W)) * kPitch + lg * 16);
  }

  float bias[kTN][4];
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const int n = wn * 32 + 16 * j + 4 * lg;
#pragma unroll
    for (int r = 0; r < 4; ++r) bias[j][r] = p.bias ? p.bias[n + r] : 0.0f;
  }
  // Retire the weight and bias loads before the band loop.  Left pending,
  // the compiler's wait insertion merges them into the loop header's state
  // and emits a vmcnt wait before every weight use in every band, which
  // also waits for the next band's patch DMA and serializes it with the MFMAs.
  // The wait alone does not pin the loads: the scheduler sinks them past it
  // to the loop entry.  An empty asm that takes every weight register as an
  // operand right after the wait keeps them above it.
  wait_vm<0>();
#pragma unroll
  for (int j = 0; j < kTN; ++j)
#pragma unroll
    for (int s = 0; s < 18; ++s) asm volatile("" : "+v"(bw[j][s]));

  // Bands [t_begin, t_end) of this block: a contiguous, balanced range.
  const int t_begin = static_cast<int>(static_cast<int64_t>(blockIdx.x) * p.tiles / gridDim.x);
  const int t_end = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * p.tiles / gridDim.x);
  int t = t_begin;
  if (t < t_end) issue(t, 0);
  int buf = 0;

  for (bool first = true; t < t_end; ++t, first = false) {
    // This wave's DMAs of band t are complete (vector-memory operations
    // retire in issue order; the only later ones are the previous band's
    // kTM stores, which may stay in flight); the barrier makes every
    // wave's complete and retires all reads of the other stage.
    if (first) wait_vm<0>();
    else wait_vm<kTM>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // This band's residual, into registers now; used by the epilogue.
    const int img = t / p.bands, h0 = (t - img * p.bands) * p.rows;
    const int valid = min(p.rows, H - h0) * W;
    const uint32_t band_off = static_cast<uint32_t>((img * H + h0) * W) * (kO * 2);
    // lane's 16 bytes of a pixel: channels wn * 32 + 8 lg .. + 7
    const uint32_t col_off = static_cast<uint32_t>(wn * 32 + 8 * lg) * 2;
    uint32_t roff[kTM];
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      const int q = wm * kWavePix + 16 * i + l16;
      roff[i] = q < valid ? band_off + static_cast<uint32_t>(q) * (kO * 2) + col_off : kOob;
    }
    i32x4 rraw[kTM];
    if (p.residual) {
#pragma unroll
      for (int i = 0; i < kTM; ++i) rraw[i] = __builtin_amdgcn_raw_buffer_load_b128(rs_res, roff[i], 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < kTM; ++i) rraw[i] = i32x4{0, 0, 0, 0};
    }
    if (t + 1 < t_end) issue(t + 1, buf ^ 1);

    f32x4 acc[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int j = 0; j < kTN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    // 18 sub-steps u = (tap, ks): tap u / 2, K chunks 4 ks .. 4 ks + 3 with
    // ks = u & 1.  Each sub-step's 7 A fragments are read from LDS one
    // sub-step ahead, and a scheduling barrier between sub-steps keeps the
    // compiler from hoisting more reads (the weights hold 144 registers).
    vec av[2][kTM];
    // One address per (filter row, fragment): a0 + stage + kh * pw * 144
    // (a wave-uniform add); kw and ks are immediate offsets of the reads.
    uint32_t arow[kTM];
    auto load_a = [&](auto uc, vec (&dst)[kTM]) {
      constexpr int u = decltype(uc)::value;
      constexpr int tap = u / 2, ks = u & 1, kh = tap / 3, kw = tap % 3;
      if constexpr (kw == 0 && ks == 0) {
        const uint32_t row = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(buf * kStage + kh * pw * kPitch));
#pragma unroll
        for (int i = 0; i < kTM; ++i) arow[i] = a0[i] + row;
      }
#pragma unroll
      for (int i = 0; i < kTM; ++i) dst[i] = *reinterpret_cast<const vec*>(smem + arow[i] + (kw * kPitch + ks * 64));
    };
    load_a(std::integral_constant<int, 0>{}, av[0]);
    // MFMA section at raised wave priority (the other block on this CU's
    // SIMDs does its DMA issue and epilogue in the gaps).
    __builtin_amdgcn_s_setprio(1);
    static_for<18>([&](auto uc) {
      constexpr int u = decltype(uc)::value;
      if constexpr (u + 1 < 18) load_a(std::integral_constant<int, u + 1>{}, av[(u + 1) & 1]);
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j) acc[i][j] = Frag<F16>::mma(bw[j][u], av[u & 1][i], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    });
    __builtin_amdgcn_s_setprio(0);

    // Epilogue from the C^T accumulators: acc[i][j][r] is output pixel
    // q = wm * 64 + 16 i + l16 of the band, channel wn * 32 + 16 j + 4 lg + r.
    // The packed outputs go to the 16-byte row layout (lane row lg: the
    // wave's channels 8 lg .. 8 lg + 7 of the pixel) by ct_pair_to_rows, and
    // the residual, loaded in that layout at the top of the band (zeros past
    // it), comes back by rows_to_ct_pair.  Only lanes of one pixel trade
    // values, so a pixel's validity is uniform over them.
    // Stores are buffer stores at 32-bit byte offsets: rows past the band get
    // an offset past num_records and are dropped, so every wave issues
    // exactly kTM stores per band (the wait at the top of the loop counts
    // them).
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      uint32_t rd[kTN][2] = {{0u, 0u}, {0u, 0u}};
      if (p.residual)
        rows_to_ct_pair(uint4{static_cast<uint32_t>(rraw[i][0]), static_cast<uint32_t>(rraw[i][1]),
                              static_cast<uint32_t>(rraw[i][2]), static_cast<uint32_t>(rraw[i][3])},
                        rd[0], rd[1]);
      uint32_t pk[kTN][2];
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        const float res[4] = {to_f32<F16>(rd[j][0] & 0xffffu), to_f32<F16>(rd[j][0] >> 16),
                              to_f32<F16>(rd[j][1] & 0xffffu), to_f32<F16>(rd[j][1] >> 16)};
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float s = (acc[i][j][r] + bias[j][r]) + res[r];
          v[r] = p.relu ? fmaxf(s, 0.0f) : s;
        }
        pk[j][0] = pack2<F16>(v[0], v[1]);
        pk[j][1] = pack2<F16>(v[2], v[3]);
      }
      const uint4 z = ct_pair_to_rows(pk[0], pk[1]);
      const i32x4 packed{static_cast<int>(z.x), static_cast<int>(z.y), static_cast<int>(z.z), static_cast<int>(z.w)};
      __builtin_amdgcn_raw_buffer_store_b128(packed, rs_out, roff[i], 0, 0);
    }
    buf ^= 1;
  }
}

// Output rows per band: as many full rows as fit 112 pixels, fewer when the
// halo patch would exceed the 240 pixels of a stage (0: not covered).
int band_rows(int h, int w) {
  int r = kTilePix / w;
  if (r > h) r = h;
  while (r > 0 && (r + 2) * (w + 2) > kMaxPatch) --r;
  return r;
}

int device_cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

}  // namespace

// Launches the band kernel when the convolution is one it covers and sets
// *handled; otherwise leaves *handled false and launches nothing.
int conv3x3_c64_launch(const c3h_conv_args* a, hipStream_t s, bool* handled) {
  *handled = false;
  if (switches().disable_conv3x3) return C3H_OK;
  const c3h_epilogue& e = a->epi;
  const bool shape = (a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16) && a->out_dtype == a->in_dtype &&
                     a->kh == 3 && a->kw == 3 && a->sh == 1 && a->sw == 1 && a->dh == 1 && a->dw == 1 &&
                     a->pad_top == 1 && a->pad_left == 1 && a->ho == a->h && a->wo == a->w_ && a->c == kC &&
                     a->c_pack == kC && a->c_stride == kC && a->o == kO && a->out_layout == 1 && a->n >= 1;
  const bool epi = e.alpha == 1.0f && e.beta == 1.0f && (e.bias_mode == 0 || e.bias_mode == 2) && e.act <= 1 &&
                   e.n_inst == 0 && (e.bias_mode == 0 || (reinterpret_cast<uintptr_t>(e.bias) & 15) == 0) &&
                   (reinterpret_cast<uintptr_t>(e.residual) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(a->x) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->w) & 15) == 0;
  if (!shape || !epi) return C3H_OK;
  const int64_t x_bytes = static_cast<int64_t>(a->n) * a->h * a->w_ * kC * 2;
  if (x_bytes >= (int64_t{1} << 31) - 16 || a->h >= 0x7fff) return C3H_OK;  // the DMA row sentinel is 0x7fff
  const int rows = band_rows(a->h, a->w_);
  if (rows < 1) return C3H_OK;
  Conv3x3Args p;
  p.x = a->x;
  p.w = a->w;
  p.out = a->out;
  p.bias = e.bias_mode == 2 ? static_cast<const float*>(e.bias) : nullptr;
  p.residual = e.residual;
  p.n = a->n;
  p.h = a->h;
  p.wd = a->w_;
  p.rows = rows;
  p.bands = static_cast<int>(ceil_div(a->h, rows));
  p.tiles = a->n * p.bands;
  p.pw = a->w_ + 2;
  p.npix = (rows + 2) * p.pw;
  p.pw_magic = static_cast<uint32_t>(((1u << 20) + p.pw - 1) / p.pw);
  p.band_pix = rows * a->w_;
  for (int pix = 0; pix < kMaxPatch; ++pix)
    C3H_REQUIRE(static_cast<int>((static_cast<uint32_t>(pix) * p.pw_magic) >> 20) == pix / p.pw,
                "conv3x3: patch-width reciprocal inexact for width %d", a->w_);
  p.relu = e.act == 1;
  p.x_bytes = static_cast<int>(x_bytes);
  const int grid = p.tiles < 2 * device_cu_count() ? p.tiles : 2 * device_cu_count();
  if (a->in_dtype == C3H_BF16)
    hipLaunchKernelGGL((conv3x3_c64_kernel<bf16_t, false>), dim3(grid), dim3(kWaves * 64), 0, s, p);
  else
    hipLaunchKernelGGL((conv3x3_c64_kernel<f16_t, true>), dim3(grid), dim3(kWaves * 64), 0, s, p);
  *handled = true;
  return launch_status("conv3x3_c64");
}

}  // namespace c3h
