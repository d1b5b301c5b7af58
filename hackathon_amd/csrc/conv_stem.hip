// Fused image-network stem for gfx950: Conv 7x7 / stride 2 / pad 3 over a
// narrow (c <= 4) NCHW input, + per-channel bias, + optional ReLU, then
// MaxPool 3x3 / stride 2 / pad 1, written channels-last in 16-bit.
//
// Unfused, this is three launches and four HBM passes over the conv output
// (layout NCHW fp32 -> NHWC c4, conv -> NHWC, maxpool read, pooled write);
// fused, the conv output never leaves LDS.  Results are identical to the
// unfused sequence: inputs are rounded to 16 bits exactly as the layout
// kernel does, the conv uses the same MFMA (16x16x32, K chunk order and
// accumulation order of c3h_conv2d's narrow-channel packing), and the
// maximum of 16-bit-rounded values equals the rounding of the maximum.
//
// Work decomposition: a tile is 4 x 8 pooled pixels x 64 channels of one
// image.  It needs a 9 x 17 conv-output tile (153 pixels, 10 MFMA row
// tiles), which needs a 23 x 40 x 4 input patch.  A persistent workgroup
// (4 waves) walks a contiguous range of tiles: the next tile's patch is
// loaded into registers while the current tile's MFMAs run, so global
// latency hides behind compute, and neighbouring tiles share their input
// halo in the workgroup's L2.  Every wave keeps the whole packed weight
// (64 x 224, as 28 MFMA B fragments) in registers for the kernel's life.
#include "common.h"

using namespace c3h;

namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

constexpr int kThreads = 256;
constexpr int KH = 7, KWP = 8, CP = 4;  // filter rows, packed filter columns, packed channels
constexpr int KSTRIDE = KH * KWP * CP;  // 224: packed K per output channel
constexpr int O = 64;                   // output channels
constexpr int PH = 4, PW = 8;           // pooled tile (rows, columns)
constexpr int CTH = 2 * PH + 1;         // 9 conv tile rows
constexpr int CTW = 2 * PW + 1;         // 17 conv tile columns
constexpr int CPIX = CTH * CTW;         // 153 conv pixels per tile
constexpr int MT = (CPIX + 15) / 16;    // 10 MFMA row tiles
constexpr int PR = 2 * (CTH - 1) + KH;  // 23 patch rows
constexpr int PC = 2 * (CTW - 1) + KWP; // 40 patch columns
constexpr int PROW = PC * CP * 2;       // 320 bytes per patch row
constexpr int PATCH_BYTES = PR * PROW;  // 7360
constexpr int CS = 192;                 // conv-tile row bytes (128 used): conflict-free pool reads
constexpr int CT_BYTES = CPIX * CS;     // 29376
constexpr int SLOTS = (PR * PC + kThreads - 1) / kThreads;  // 4 patch pixels per thread
constexpr int TPW = (MT + 3) / 4;       // 3 row tiles per wave (waves 2 and 3 have 2)
static_assert(PH * PW * 8 == kThreads, "one pooled item (8 channels) per thread");

template <typename T> struct In;
template <> struct In<float> {
  static __device__ __forceinline__ uint32_t load(const float* p) { return __float_as_uint(*p); }
  static __device__ __forceinline__ float f32(uint32_t v) { return __uint_as_float(v); }
};
template <> struct In<bf16_t> {
  static __device__ __forceinline__ uint32_t load(const bf16_t* p) { return p->bits; }
  static __device__ __forceinline__ float f32(uint32_t v) { return bf16_bits_to_f32(static_cast<uint16_t>(v)); }
};
template <> struct In<f16_t> {
  static __device__ __forceinline__ uint32_t load(const f16_t* p) { return p->bits; }
  static __device__ __forceinline__ float f32(uint32_t v) { return f16_bits_to_f32(static_cast<uint16_t>(v)); }
};

template <typename MM> struct Mm;
template <> struct Mm<bf16_t> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x4 mma(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(vec, a), __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t bits(float v) { return f32_to_bf16_bits(v); }
  static __device__ __forceinline__ float f32(uint32_t b) { return bf16_bits_to_f32(static_cast<uint16_t>(b)); }
};
template <> struct Mm<f16_t> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x4 mma(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(vec, a), __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t bits(float v) { return f32_to_f16_bits(v); }
  static __device__ __forceinline__ float f32(uint32_t b) { return f16_bits_to_f32(static_cast<uint16_t>(b)); }
};

struct StemGeom {
  int64_t tiles;
  int n, c, h, w, ho, wo, po, qo, tq, tpi;
  int relu;
};

template <typename TI, typename T16>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
conv_stem_pool_kernel(const TI* __restrict__ x, const uint16_t* __restrict__ wp, const float* __restrict__ bias,
                      uint16_t* __restrict__ out, StemGeom g) {
  typedef Mm<T16> MM;
  __shared__ __attribute__((aligned(16))) uint8_t smem[PATCH_BYTES + CT_BYTES];
  uint8_t* patch = smem;
  uint8_t* ctile = smem + PATCH_BYTES;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;

  // Whole weight as B fragments: lane (n = 16 j + l16, k = 32 kh + 8 lg .. + 7).
  uint4 bw[KH][4];
#pragma unroll
  for (int kh = 0; kh < KH; ++kh)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bw[kh][j] = *reinterpret_cast<const uint4*>(wp + (16 * j + l16) * KSTRIDE + 32 * kh + 8 * lg);
  float bv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bv[j] = bias ? bias[16 * j + l16] : 0.0f;
  // Packed column kw = 7 only pads the filter: zero its half of the A operand so
  // that non-finite inputs there cannot turn 0 * x into NaN.
  const uint32_t kw7_mask = lg == 3 ? 0u : 0xffffffffu;

  // A-fragment byte offsets in the patch for this wave's row tiles (pixel m = 16 i + l16).
  int aoff[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int m = 16 * (wave + 4 * t) + l16;
    m = m < CPIX ? m : CPIX - 1;
    const int r = m / CTW, c = m - r * CTW;
    aoff[t] = 2 * r * PROW + (2 * c + 2 * lg) * (CP * 2);
  }

  const int64_t G = gridDim.x;
  const int64_t t_begin = g.tiles * blockIdx.x / G, t_end = g.tiles * (blockIdx.x + 1) / G;
  const int64_t plane = static_cast<int64_t>(g.h) * g.w;

  uint32_t pre[SLOTS][3];
  auto fetch = [&](int64_t t) {
    const int img = static_cast<int>(t / g.tpi);
    const int rem = static_cast<int>(t - static_cast<int64_t>(img) * g.tpi);
    const int pt = rem / g.tq, qt = rem - pt * g.tq;
    const int hi0 = 4 * PH * pt - 5, wi0 = 4 * PW * qt - 5;
    const TI* base = x + static_cast<int64_t>(img) * g.c * plane;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int slot = tid + s * kThreads;
      const int row = slot / PC, col = slot - row * PC;
      const int hi = hi0 + row, wi = wi0 + col;
      const bool ok = slot < PR * PC && col < PC - 1 && static_cast<unsigned>(hi) < static_cast<unsigned>(g.h) &&
                      static_cast<unsigned>(wi) < static_cast<unsigned>(g.w);
      const TI* px = base + static_cast<int64_t>(hi) * g.w + wi;
#pragma unroll
      for (int ch = 0; ch < 3; ++ch) pre[s][ch] = (ok && ch < g.c) ? In<TI>::load(px + ch * plane) : 0u;
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int slot = tid + s * kThreads;
      if (slot < PR * PC) {
        const uint32_t c0 = MM::bits(In<TI>::f32(pre[s][0])), c1 = MM::bits(In<TI>::f32(pre[s][1]));
        const uint32_t c2 = MM::bits(In<TI>::f32(pre[s][2]));
        *reinterpret_cast<uint2*>(patch + slot * (CP * 2)) = uint2{c0 | (c1 << 16), c2};
      }
    }
  };

  if (t_begin < t_end) {
    fetch(t_begin);
    stash();
  }
  __syncthreads();
  for (int64_t t = t_begin; t < t_end; ++t) {
    if (t + 1 < t_end) fetch(t + 1);

    f32x4 acc[TPW][4];
#pragma unroll
    for (int i = 0; i < TPW; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) {
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        if (wave + 4 * i < MT) {
          uint4 a = *reinterpret_cast<const uint4*>(patch + aoff[i] + kh * PROW);
          a.z &= kw7_mask;
          a.w &= kw7_mask;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = MM::mma(a, bw[kh][j], acc[i][j]);
        }
      }
    }
    // bias + ReLU, rounded to 16 bits, into the conv tile [pixel][channel].
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      if (wave + 4 * i < MT) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * (wave + 4 * i) + 4 * lg + r;
          if (m < CPIX) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              float v = acc[i][j][r] + bv[j];
              v += 0.0f;  // as c3h_conv2d's epilogue (adds the absent residual): -0 becomes +0
              if (g.relu) v = fmaxf(v, 0.0f);
              *reinterpret_cast<uint16_t*>(ctile + m * CS + (16 * j + l16) * 2) = static_cast<uint16_t>(MM::bits(v));
            }
          }
        }
      }
    }
    __syncthreads();
    if (t + 1 < t_end) stash();  // every wave is past its patch reads
    // 3x3 / stride 2 max over valid conv pixels; 8 channels per item.
    {
      const int img = static_cast<int>(t / g.tpi);
      const int rem = static_cast<int>(t - static_cast<int64_t>(img) * g.tpi);
      const int pt = rem / g.tq, qt = rem - pt * g.tq;
      {
        const int px = tid >> 3, cg = tid & 7;
        const int pr = px / PW, qc = px - pr * PW;
        const int P = PH * pt + pr, Q = PW * qt + qc;
        if (P < g.po && Q < g.qo) {
          float mx[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) mx[e] = -__builtin_huge_valf();
#pragma unroll
          for (int dr = 0; dr < 3; ++dr) {
            const int cr = 2 * P - 1 + dr;
            if (static_cast<unsigned>(cr) >= static_cast<unsigned>(g.ho)) continue;
#pragma unroll
            for (int dc = 0; dc < 3; ++dc) {
              const int cc = 2 * Q - 1 + dc;
              if (static_cast<unsigned>(cc) >= static_cast<unsigned>(g.wo)) continue;
              const int m = (2 * pr + dr) * CTW + 2 * qc + dc;
              const uint4 v = *reinterpret_cast<const uint4*>(ctile + m * CS + cg * 16);
              const uint32_t wds[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                mx[2 * e] = fmaxf(mx[2 * e], MM::f32(wds[e] & 0xffffu));
                mx[2 * e + 1] = fmaxf(mx[2 * e + 1], MM::f32(wds[e] >> 16));
              }
            }
          }
          uint32_t o4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o4[e] = MM::bits(mx[2 * e]) | (MM::bits(mx[2 * e + 1]) << 16);
          const int64_t o = ((static_cast<int64_t>(img) * g.po + P) * g.qo + Q) * O + cg * 8;
          *reinterpret_cast<uint4*>(out + o) = uint4{o4[0], o4[1], o4[2], o4[3]};
        }
      }
    }
    __syncthreads();
  }
}

int stem_grid() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                hipSuccess || cus <= 0)
      cus = 256;
  }
  return 2 * cus;  // two resident workgroups per CU
}

}  // namespace

extern "C" {

int c3h_conv_stem_pool(const c3h_conv_pool_args* a, void* stream) {
  C3H_REQUIRE(a && a->x && a->w && a->out, "conv_stem_pool: null pointer");
  C3H_REQUIRE(a->n >= 0 && a->c >= 1 && a->c <= 3 && a->h > 0 && a->w_ > 0, "conv_stem_pool: input must be [n, c<=3, h, w]");
  C3H_REQUIRE(a->o == O && a->kh == 7 && a->kw == 7 && a->sh == 2 && a->sw == 2 && a->pad_top == 3 &&
                  a->pad_left == 3 && a->k_stride == KSTRIDE,
              "conv_stem_pool: supports a 7x7 / stride 2 / pad 3 conv to 64 channels (packed K stride 224)");
  C3H_REQUIRE(a->pkh == 3 && a->pkw == 3 && a->psh == 2 && a->psw == 2 && a->ppad_top == 1 && a->ppad_left == 1,
              "conv_stem_pool: supports a 3x3 / stride 2 / pad 1 max pool");
  C3H_REQUIRE(a->ho > 0 && a->wo > 0 && a->po > 0 && a->qo > 0 && 2 * (a->po - 1) - 1 < a->ho &&
                  2 * (a->qo - 1) - 1 < a->wo,
              "conv_stem_pool: inconsistent conv/pool output sizes");
  C3H_REQUIRE(a->mm_dtype == C3H_BF16 || a->mm_dtype == C3H_F16, "conv_stem_pool: compute dtype must be BF16 or F16");
  C3H_REQUIRE(a->in_dtype == C3H_F32 || a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16,
              "conv_stem_pool: input dtype must be F32, BF16 or F16");
  C3H_REQUIRE((reinterpret_cast<uintptr_t>(a->w) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 15) == 0,
              "conv_stem_pool: weight and output must be 16-byte aligned");
  if (a->n == 0) return C3H_OK;
  StemGeom g;
  g.n = a->n; g.c = a->c; g.h = a->h; g.w = a->w_; g.ho = a->ho; g.wo = a->wo; g.po = a->po; g.qo = a->qo;
  g.tq = (a->qo + PW - 1) / PW;
  g.tpi = ((a->po + PH - 1) / PH) * g.tq;
  g.tiles = static_cast<int64_t>(a->n) * g.tpi;
  g.relu = a->relu ? 1 : 0;
  const int grid = static_cast<int>(g.tiles < stem_grid() ? g.tiles : stem_grid());
  hipStream_t s = as_stream(stream);
  const uint16_t* w = static_cast<const uint16_t*>(a->w);
  uint16_t* out = static_cast<uint16_t*>(a->out);
#define C3H_STEM(TI, MM)                                                                                         \
  hipLaunchKernelGGL((conv_stem_pool_kernel<TI, MM>), dim3(grid), dim3(kThreads), 0, s, static_cast<const TI*>(a->x), \
                     w, a->bias, out, g)
  if (a->mm_dtype == C3H_BF16) {
    if (a->in_dtype == C3H_F32) C3H_STEM(float, bf16_t);
    else if (a->in_dtype == C3H_BF16) C3H_STEM(bf16_t, bf16_t);
    else C3H_STEM(f16_t, bf16_t);
  } else {
    if (a->in_dtype == C3H_F32) C3H_STEM(float, f16_t);
    else if (a->in_dtype == C3H_BF16) C3H_STEM(bf16_t, f16_t);
    else C3H_STEM(f16_t, f16_t);
  }
#undef C3H_STEM
  return launch_status("conv_stem_pool");
}

}  // extern "C"
