// Fused image-network stem for gfx950: Conv 7x7 / stride 2 / pad 3 over a
// narrow (c <= 3) NCHW input, + per-channel bias, + optional ReLU, then
// MaxPool 3x3 / stride 2 / pad 1, written channels-last in 16-bit.
//
// Unfused, this is three launches and four HBM passes over the conv output
// (layout NCHW fp32 -> NHWC c4, conv -> NHWC, maxpool read, pooled write);
// fused, the conv output never leaves LDS.  Results are identical to the
// unfused sequence: inputs are rounded to 16 bits exactly as the layout
// kernel does, the conv uses the same MFMA (16x16x32, K chunk order and
// accumulation order of c3h_conv2d's narrow-channel packing), and the pool
// runs before the bias / ReLU / rounding, which commutes with it (below).
//
// Work decomposition: a tile is 7 x 8 pooled pixels x 64 channels of one
// image.  It needs a 15 x 17 conv-output tile (255 pixels, 16 MFMA column
// tiles, four per wave), which needs a 35 x 40 x 4 input patch.  A
// persistent workgroup (4 waves, two per CU) walks a contiguous range of
// tiles: the next tile's patch is loaded into registers while the current
// tile's MFMAs run, so global latency hides behind compute, and neighbouring
// tiles share their input halo in L2.  Every wave keeps the whole packed
// weight (64 x 224, as 28 MFMA fragments) in registers for the kernel's life.
//
// The MFMA computes C^T = W . X^T, so a lane's four accumulators are four
// consecutive channels of one conv pixel; they go to the fp32 conv tile in
// LDS as they are, one 16-byte store.  The pool takes the maximum of the raw
// accumulators and only then adds the bias, applies ReLU and rounds to 16
// bits, once per pooled value instead of once per conv value.  That is
// exact: v -> round(relu(v + b)) is monotone non-decreasing, so the maximum
// of its values is its value at the maximum.  NaN accumulators agree too:
// fmaxf skips them, and the unfused chain maps them to +0 under ReLU, which
// the maximum of the non-negative others absorbs (all-NaN windows give +0
// either way).  Without ReLU the same holds for a finite bias, with all-NaN
// windows mapped to the unfused pool's -inf.
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
constexpr int PH = 7, PW = 8;           // pooled tile (rows, columns)
constexpr int CTH = 2 * PH + 1;         // 15 conv tile rows
constexpr int CTW = 2 * PW + 1;         // 17 conv tile columns
constexpr int CPIX = CTH * CTW;         // 255 conv pixels per tile
constexpr int MT = (CPIX + 15) / 16;    // 16 MFMA pixel tiles
constexpr int PR = 2 * (CTH - 1) + KH;  // 35 patch rows
constexpr int PC = 2 * (CTW - 1) + KWP; // 40 patch columns
constexpr int PROW = PC * CP * 2;       // 320 bytes per patch row
constexpr int PATCH_BYTES = PR * PROW;  // 11200
constexpr int CS = 272;                 // fp32 conv-tile pixel stride (256 used): conflict-free 16-byte stores
constexpr int CT_BYTES = CPIX * CS;     // 69360
constexpr int SLOTS = (PR * PC + kThreads - 1) / kThreads;  // 6 patch pixels per thread
constexpr int TPW = MT / 4;             // 4 pixel tiles per wave
static_assert(MT == 4 * TPW, "the pixel tiles split evenly over the four waves");
constexpr int POOL_ITEMS = PH * PW * 8; // 448 (pooled pixel, 8-channel group) items, two rounds
constexpr uint32_t kOob = 0x80000000u;  // buffer offset past num_records: reads 0
static_assert(kThreads % 8 == 0 && POOL_ITEMS <= 2 * kThreads, "two pool rounds; a thread keeps its 8 channels");
// Two workgroups per CU must fit the 160 KiB of LDS.
static_assert(2 * (PATCH_BYTES + CT_BYTES + O * 4) <= 160 * 1024, "LDS for two workgroups per CU");

template <typename T> struct In;
template <> struct In<float> {
  static __device__ __forceinline__ uint32_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  }
  static __device__ __forceinline__ float f32(uint32_t v) { return __uint_as_float(v); }
};
template <> struct In<bf16_t> {
  static __device__ __forceinline__ uint32_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  }
  static __device__ __forceinline__ float f32(uint32_t v) { return bf16_bits_to_f32(static_cast<uint16_t>(v)); }
};
template <> struct In<f16_t> {
  static __device__ __forceinline__ uint32_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  }
  static __device__ __forceinline__ float f32(uint32_t v) { return f16_bits_to_f32(static_cast<uint16_t>(v)); }
};

template <typename MM> struct Mm;
template <> struct Mm<bf16_t> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x4 mma(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(vec, a), __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return f32x2_to_bf16x2_bits(lo, hi); }
  static __device__ __forceinline__ float f32(uint32_t b) { return bf16_bits_to_f32(static_cast<uint16_t>(b)); }
};
template <> struct Mm<f16_t> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x4 mma(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(vec, a), __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return f32x2_to_f16x2_bits(lo, hi); }
  static __device__ __forceinline__ float f32(uint32_t b) { return f16_bits_to_f32(static_cast<uint16_t>(b)); }
};

// Maximum of three accumulators as one v_max3_f32.  fmaxf on values loaded
// from LDS would first canonicalize each operand (one more VALU operation
// apiece).  The accumulators are MFMA results, which hold no signalling NaN,
// and the IEEE-mode maximum skips quiet NaN operands as fmaxf does.
__device__ __forceinline__ float max3_f32(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

struct StemGeom {
  int64_t tiles;
  int n, c, h, w, ho, wo, po, qo, tq, tpi;
  int relu;
  uint32_t image_bytes;  // c * h * w * sizeof(input element)
};

template <typename TI, typename T16>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
conv_stem_pool_kernel(const TI* __restrict__ x, const uint16_t* __restrict__ wp, const float* __restrict__ bias,
                      uint16_t* __restrict__ out, StemGeom g) {
  typedef Mm<T16> MM;
  __shared__ __attribute__((aligned(16))) uint8_t smem[PATCH_BYTES + CT_BYTES + O * 4];
  uint8_t* patch = smem;
  uint8_t* ctile = smem + PATCH_BYTES;
  // The bias lives in LDS and is read per pooled item: eight registers held
  // for the kernel's life would push the register budget into spills.
  float* bias_s = reinterpret_cast<float*>(smem + PATCH_BYTES + CT_BYTES);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;

  // Whole weight as MFMA A fragments: lane (channel 16 j + l16, k = 32 kh + 8 lg .. + 7).
  uint4 bw[KH][4];
#pragma unroll
  for (int kh = 0; kh < KH; ++kh)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bw[kh][j] = *reinterpret_cast<const uint4*>(wp + (16 * j + l16) * KSTRIDE + 32 * kh + 8 * lg);
  if (tid < O) bias_s[tid] = bias ? bias[tid] : 0.0f;  // read after the first barrier
  // Retire the weight and bias loads here (s_waitcnt vmcnt(0)).  Left
  // pending, the compiler's wait insertion carries them into the tile loop's
  // header state and waits on vmcnt before the MFMAs of every tile, which
  // also waits for the next tile's prefetch and serializes it with the MFMAs.
  __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));
  // Packed column kw = 7 only pads the filter: zero its half of the patch
  // operand so that non-finite inputs there cannot turn 0 * x into NaN.
  const uint32_t kw7_mask = lg == 3 ? 0u : 0xffffffffu;

  // Patch byte offsets of this lane's pixel (m = 16 i + l16) in each of the wave's pixel tiles.
  int aoff[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int m = 16 * (wave + 4 * t) + l16;
    m = m < CPIX ? m : CPIX - 1;
    const int r = m / CTW, c = m - r * CTW;
    aoff[t] = 2 * r * PROW + (2 * c + 2 * lg) * (CP * 2);
  }
  // This thread's patch slots: fixed (row, col) inside every tile, packed
  // as row << 8 | col; a slot past the patch gets column 255 (never loaded).
  int s_rc[SLOTS];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const int slot = tid + s * kThreads;
    s_rc[s] = slot < PR * PC ? (slot / PC) << 8 | (slot % PC) : 0xff;
  }
  const uint32_t plane_bytes = static_cast<uint32_t>(g.h) * g.w * sizeof(TI);

  const int64_t G = gridDim.x;
  const int64_t t_begin = g.tiles * blockIdx.x / G, t_end = g.tiles * (blockIdx.x + 1) / G;
  // Tile coordinates, advanced incrementally (no division in the loop).
  int img = static_cast<int>(t_begin / g.tpi);
  int rem = static_cast<int>(t_begin - static_cast<int64_t>(img) * g.tpi);
  int pt = rem / g.tq, qt = rem - pt * g.tq;

  uint32_t pre[SLOTS][3];
  auto fetch = [&](int f_img, int f_pt, int f_qt) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<TI*>(x + static_cast<int64_t>(f_img) * g.c * g.h * g.w), 0, static_cast<int>(g.image_bytes),
        0x00020000);
    const int hi0 = 4 * PH * f_pt - 5, wi0 = 4 * PW * f_qt - 5;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int col = s_rc[s] & 0xff;
      const int hi = hi0 + (s_rc[s] >> 8), wi = wi0 + col;
      const bool ok = col < PC - 1 &&
                      static_cast<unsigned>(hi) < static_cast<unsigned>(g.h) &&
                      static_cast<unsigned>(wi) < static_cast<unsigned>(g.w);
      const uint32_t off = ok ? static_cast<uint32_t>((hi * g.w + wi) * static_cast<int>(sizeof(TI))) : kOob;
#pragma unroll
      for (int ch = 0; ch < 3; ++ch)
        // Out-of-range loads get distinct offsets past the buffer (each reads
        // zero): identical ones are merged by the compiler into one load plus
        // copies that must wait for it, a vmcnt(0) stall in every fetch.
        pre[s][ch] = In<TI>::load(rs, (ok && ch < g.c) ? off + ch * plane_bytes : kOob + 4 * ch);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int slot = tid + s * kThreads;
      if (slot < PR * PC) {
        const uint32_t c01 = MM::pack(In<TI>::f32(pre[s][0]), In<TI>::f32(pre[s][1]));
        const uint32_t c2 = MM::pack(In<TI>::f32(pre[s][2]), 0.0f);
        *reinterpret_cast<uint2*>(patch + slot * (CP * 2)) = uint2{c01, c2};
      }
    }
  };

  if (t_begin < t_end) {
    fetch(img, pt, qt);
    stash();
  }
  __syncthreads();
  for (int64_t t = t_begin; t < t_end; ++t) {
    // coordinates of tile t + 1
    int n_img = img, n_pt = pt, n_qt = qt + 1;
    if (n_qt == g.tq) {
      n_qt = 0;
      if (++n_pt * g.tq == g.tpi) {
        n_pt = 0;
        ++n_img;
      }
    }
    if (t + 1 < t_end) fetch(n_img, n_pt, n_qt);

    // The kh = 0 MFMAs take a zero C operand (an inline constant), so the
    // accumulators need no zeroing moves.
    f32x4 acc[TPW][4];
    __builtin_amdgcn_s_setprio(1);  // MFMA section at raised wave priority
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) {
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        uint4 a = *reinterpret_cast<const uint4*>(patch + aoff[i] + kh * PROW);
        a.z &= kw7_mask;
        a.w &= kw7_mask;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = MM::mma(bw[kh][j], a, kh == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    // Raw accumulators into the fp32 conv tile [pixel][channel].
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int m = 16 * (wave + 4 * i) + l16;
      if (m < CPIX) {
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<f32x4*>(ctile + m * CS + (16 * j + 4 * lg) * 4) = acc[i][j];
      }
    }
    __syncthreads();
    if (t + 1 < t_end) stash();  // every wave is past its patch reads
    // 3x3 / stride 2 max over the valid conv pixels of each pooled pixel, 8
    // channels per thread, then bias (+ the absent residual's +0, as
    // c3h_conv2d), ReLU and the 16-bit rounding.
    {
      // Whether every window of the tile lies inside the conv output (uniform).
      const bool interior = pt > 0 && qt > 0 && 2 * (PH * pt + PH - 1) + 1 < g.ho && 2 * (PW * qt + PW - 1) + 1 < g.wo;
#pragma unroll
      for (int round = 0; round < 2; ++round) {
        const int item = tid + round * kThreads;
        const int px = item >> 3, cg = item & 7;
        const int pr = px / PW, qc = px - pr * PW;
        const int P = PH * pt + pr, Q = PW * qt + qc;
        if (item < POOL_ITEMS && P < g.po && Q < g.qo) {
          const uint8_t* c0 = ctile + ((2 * pr) * CTW + 2 * qc) * CS + cg * 32;
          float mx[8];
          // Row maxima first (three positions each), then the maximum of the rows.
          auto pool = [&](auto offset) {
            float rm[3][8];
#pragma unroll
            for (int dr = 0; dr < 3; ++dr) {
              f32x4 lo[3], hi[3];
#pragma unroll
              for (int dc = 0; dc < 3; ++dc) {
                lo[dc] = *reinterpret_cast<const f32x4*>(c0 + offset(dr, dc));
                hi[dc] = *reinterpret_cast<const f32x4*>(c0 + offset(dr, dc) + 16);
              }
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                rm[dr][e] = max3_f32(lo[0][e], lo[1][e], lo[2][e]);
                rm[dr][4 + e] = max3_f32(hi[0][e], hi[1][e], hi[2][e]);
              }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) mx[e] = max3_f32(rm[0][e], rm[1][e], rm[2][e]);
          };
          if (interior) {
            pool([](int dr, int dc) { return (dr * CTW + dc) * CS; });
          } else {
            // Outside the conv output a window position re-reads the window's
            // centre (2 pr + 1, 2 qc + 1), which every window holds and which
            // leaves the maximum unchanged.
            bool rok[3], cok[3];
#pragma unroll
            for (int k = 0; k < 3; ++k) {
              rok[k] = static_cast<unsigned>(2 * P - 1 + k) < static_cast<unsigned>(g.ho);
              cok[k] = static_cast<unsigned>(2 * Q - 1 + k) < static_cast<unsigned>(g.wo);
            }
            pool([&](int dr, int dc) { return (rok[dr] & cok[dc]) ? (dr * CTW + dc) * CS : (CTW + 1) * CS; });
          }
          float bv[8];
          *reinterpret_cast<f32x4*>(bv) = *reinterpret_cast<const f32x4*>(bias_s + 8 * cg);
          *reinterpret_cast<f32x4*>(bv + 4) = *reinterpret_cast<const f32x4*>(bias_s + 8 * cg + 4);
          float v[8];
          // With ReLU the zero residual's "+ 0" changes nothing (it only turns
          // -0 into +0, and the select maps both zeros and NaN to +0), so it is
          // added only without ReLU.
          if (g.relu) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float t = mx[e] + bv[e];
              v[e] = t > 0.0f ? t : 0.0f;
            }
          } else {
            // A window of NaN conv values only pools to -inf, as the unfused
            // max pool (fmaxf from -inf) gives.
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = mx[e] == mx[e] ? (mx[e] + bv[e]) + 0.0f : -__builtin_huge_valf();
          }
          const uint4 res{MM::pack(v[0], v[1]), MM::pack(v[2], v[3]), MM::pack(v[4], v[5]), MM::pack(v[6], v[7])};
          const int64_t o = ((static_cast<int64_t>(img) * g.po + P) * g.qo + Q) * O + cg * 8;
          *reinterpret_cast<uint4*>(out + o) = res;
        }
      }
    }
    __syncthreads();
    img = n_img;
    pt = n_pt;
    qt = n_qt;
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
  // Every pooled window's centre conv pixel must exist (true for pool pads 1/1).
  C3H_REQUIRE(a->ho > 0 && a->wo > 0 && a->po > 0 && a->qo > 0 && 2 * (a->po - 1) < a->ho && 2 * (a->qo - 1) < a->wo,
              "conv_stem_pool: inconsistent conv/pool output sizes");
  C3H_REQUIRE(a->mm_dtype == C3H_BF16 || a->mm_dtype == C3H_F16, "conv_stem_pool: compute dtype must be BF16 or F16");
  C3H_REQUIRE(a->in_dtype == C3H_F32 || a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16,
              "conv_stem_pool: input dtype must be F32, BF16 or F16");
  C3H_REQUIRE((reinterpret_cast<uintptr_t>(a->w) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 15) == 0,
              "conv_stem_pool: weight and output must be 16-byte aligned");
  const int64_t image_bytes = static_cast<int64_t>(a->c) * a->h * a->w_ * dtype_size(a->in_dtype);
  C3H_REQUIRE(image_bytes < (int64_t{1} << 31), "conv_stem_pool: one input image must be below 2 GiB");
  if (a->n == 0) return C3H_OK;
  StemGeom g;
  g.n = a->n; g.c = a->c; g.h = a->h; g.w = a->w_; g.ho = a->ho; g.wo = a->wo; g.po = a->po; g.qo = a->qo;
  g.tq = (a->qo + PW - 1) / PW;
  g.tpi = ((a->po + PH - 1) / PH) * g.tq;
  g.tiles = static_cast<int64_t>(a->n) * g.tpi;
  g.relu = a->relu ? 1 : 0;
  g.image_bytes = static_cast<uint32_t>(image_bytes);
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
