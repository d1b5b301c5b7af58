#pragma once
// Contraction kernels of libc3hip.so (gfx950): GEMM and implicit-GEMM Conv2d
// on MFMA, fp32 accumulation, LDS double-buffered tiles and a fused epilogue.
// Kernel templates and their host launchers; each MFMA input type is
// instantiated in its own translation unit (gemm_<type>.hip), so they build
// in parallel, and gemm.hip holds the C entry points.
//
//   fp32  : v_mfma_f32_16x16x4_f32   (configs 1-2, the reference's fp32 policy)
//   bf16  : v_mfma_f32_16x16x32_bf16 (config 3)
//   f16   : v_mfma_f32_16x16x32_f16  (config 4)
//
// A 256-thread workgroup (4 wave64s) computes a BM x BN macro tile; each wave
// owns a (BM/WM) x (BN/WN) sub-tile of 16x16 MFMA tiles.  A and B tiles are
// staged global -> registers -> LDS with two LDS buffers, so the loads of
// tile k+1 are in flight while the MFMAs of tile k run.  Tile ids are
// remapped so that consecutive tiles (sharing an A row panel) land on the
// same XCD and hit its L2.
#include <stdlib.h>
#include <mutex>
#include <type_traits>
#include <utility>

#include "common.h"

using namespace c3h;

namespace c3h {
namespace gk {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

constexpr int kThreads = 256;

// Kernel-argument view: the (single) by-value argument read in place through
// the kernarg segment pointer (constant address space, scalar loads), so a
// dynamically indexed epilogue program never makes the compiler copy the
// argument struct into scratch memory.
template <typename T>
using KArg = __attribute__((address_space(4))) T;

template <typename P>
__device__ __forceinline__ const KArg<P>& kernel_arg() {
  return *(const KArg<P>*)(__builtin_amdgcn_kernarg_segment_ptr());
}

// erf for the GELU epilogues, one branch-free formula: erf(u) =
// sign(u) (1 - erfc(|u|)) with erfc(z) = t exp(-z^2 - 1.26551223 + t P(t)),
// t = 1 / (1 + z / 2), the Chebyshev fit of Numerical Recipes (Press et al.,
// 2nd ed., section 6.2, erfcc), fractional error below 1.2e-7 for all z >= 0.
// Evaluated in fp32 it stays within 1e-6 of erfc relative for z < 4 (1e-5
// beyond, from the exponent's rounding), i.e. erf within an fp32 ulp or two.
__device__ __forceinline__ float erf_cheb(float u) {
  const float z = fabsf(u);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = fmaf(t, p, -0.82215223f);
  p = fmaf(t, p, 1.48851587f);
  p = fmaf(t, p, -1.13520398f);
  p = fmaf(t, p, 0.27886807f);
  p = fmaf(t, p, -0.18628806f);
  p = fmaf(t, p, 0.09678418f);
  p = fmaf(t, p, 0.37409196f);
  p = fmaf(t, p, 1.00002368f);
  const float ec = t * __expf(fmaf(-z, z, fmaf(t, p, -1.26551223f)));
  return u >= 0.0f ? 1.0f - ec : ec - 1.0f;
}

// GELU as the decomposed ONNX chain Div -> Erf -> Add -> Mul -> Mul computes
// it: ((x * (erf(x / c0) + c1)) * c2) with the chain's constants (c0 =
// sqrt(2), c1 = 1, c2 = 0.5 in practice).  x / c0 is x * (1 / c0) with one
// residual correction and erf is erf_cheb, each within an fp32 ulp or two of
// the chain's correctly rounded division and erf, at a fraction of their
// instructions.
__device__ __forceinline__ float gelu_erf(float x, float c0, float c1, float c2) {
  const float r0 = __builtin_amdgcn_rcpf(c0);
  float q = x * r0;
  const float rr = fmaf(-q, c0, x);
  q = rr == rr ? fmaf(rr, r0, q) : q;  // x = +-Inf: keep Inf
  return (x * (erf_cheb(q) + c1)) * c2;
}

// The chain's constants as every GELU export writes them: c0 = fp32(sqrt 2),
// c1 = 1, c2 = 0.5.  With these, act 2 evaluates gelu_std.
__device__ __forceinline__ bool gelu_std_ok(float c0, float c1, float c2) {
  return c0 == 0x1.6a09e6p+0f && c1 == 1.0f && c2 == 0.5f;
}

// GELU for the standard constants as the chain computes it, (x * (erf(q) +
// 1)) * 0.5 with q = x / sqrt 2, but with erf(q) formed from
//   E(a) = Phi(-a) = erfc(a / sqrt 2) / 2,  a = |x|:  erf(q) = sign(x) (1 - 2 E),
// E(a) = 2^P(a).  P is a degree-8 polynomial fitted to log2 Phi(-a) on
// [0, 5.75] by weighted minimax (weight E, so the error is bounded in E
// itself: 1.6e-8 absolute at most, 8e-9 past a = 2), and |x| is clamped at
// 5.75.  So erf(q) = fl(1 - 2E) lands within about one fp32 step of the
// correctly rounded erf(q) the chain adds 1 to, and the remaining steps
// round as the chain's do: x below -5.5 gives -0 (1 - 2E rounds to 1 there,
// as erf rounds to -1), +Inf gives +Inf, -Inf and NaN give NaN.  One
// v_exp_f32 and about 14 other VALU operations, against gelu_erf's ~24 and
// two transcendentals (v_rcp_f32, v_exp_f32).
__device__ __forceinline__ float gelu_std(float x) {
  const float a = fminf(fabsf(x), 5.75f);
  float p = -0x1.740f9ep-19f;
  p = fmaf(p, a, 0x1.43fa00p-15f);
  p = fmaf(p, a, -0x1.7ed53ap-13f);
  p = fmaf(p, a, -0x1.31e784p-13f);
  p = fmaf(p, a, 0x1.cfb2a2p-8f);
  p = fmaf(p, a, -0x1.ae1f04p-5f);
  p = fmaf(p, a, -0x1.d639d0p-2f);
  p = fmaf(p, a, -0x1.26aedep+0f);
  p = fmaf(p, a, -1.0f);
  const float e = __builtin_amdgcn_exp2f(p);  // p in [-27.9, -1]: no range reduction needed
  const float erf_q = __builtin_copysignf(fmaf(-2.0f, e, 1.0f), x);  // 1 - 2E >= 0
  return (x * (erf_q + 1.0f)) * 0.5f;
}

// act 2 where the constants are only known at run time (uniform `std_form`
// from gelu_std_ok, hoisted by the caller).
__device__ __forceinline__ float gelu_act(float x, float c0, float c1, float c2, bool std_form) {
  return std_form ? gelu_std(x) : gelu_erf(x, c0, c1, c2);
}

// ---------------------------------------------------------------- epilogue
// `e` is read straight from the kernel-argument segment (uniform scalar
// loads); `bias_off` selects the batch's bias slice.
__device__ __forceinline__ float apply_epilogue(const KArg<c3h_epilogue>& e, float acc, int64_t m, int64_t n,
                                                int64_t ldb_bias, float res, int64_t bias_off = 0) {
  float v = e.alpha * acc;
  const float* bias = static_cast<const float*>(e.bias) + bias_off;
  switch (e.bias_mode) {
    case 1: v += e.beta * bias[0]; break;
    case 2: v += e.beta * bias[n]; break;
    case 3: v += e.beta * bias[m]; break;
    case 4: v += e.beta * bias[m * ldb_bias + n]; break;
    default: break;
  }
  v += res;
  if (e.act == 1) v = fmaxf(v, 0.0f);
  else if (e.act == 2) v = gelu_act(v, e.imm[0], e.imm[1], e.imm[2], gelu_std_ok(e.imm[0], e.imm[1], e.imm[2]));
  if (e.n_inst > 0) {
    // Linear program: operand 0 = x (the value entering the program),
    // 1 = previous result, 2 + j = imm[j].  No register file, so the
    // program costs no scratch memory in register-heavy GEMM kernels.
    const float x = v;
    float prev = v;
    for (int i = 0; i < e.n_inst; ++i) {
      const int ca = e.inst[i].a, cb = e.inst[i].b;
      const float oa = ca == 0 ? x : (ca == 1 ? prev : e.imm[ca - 2]);
      const float ob = cb == 0 ? x : (cb == 1 ? prev : e.imm[cb - 2]);
      prev = ew_apply(e.inst[i].op, oa, ob, e.inst[i].imm);
    }
    v = prev;
  }
  return v;
}

// Epilogue of 8 consecutive columns n..n+7 of row m, in the same order and
// arithmetic as apply_epilogue.  Every decision is uniform across the wave
// and is taken once per 8 values, and bias_mode 2 reads its 8 bias values
// as two float4 loads when they are 16-byte aligned.
__device__ __forceinline__ void apply_epilogue8(const KArg<c3h_epilogue>& e, float* v, int64_t m, int64_t n,
                                                int64_t ldb_bias, const float* res, int64_t bias_off) {
  const float alpha = e.alpha, beta = e.beta;
  if (alpha != 1.0f) {
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = alpha * v[c];
  }
  const float* bias = static_cast<const float*>(e.bias) + bias_off;
  const int bm = e.bias_mode;
  if (bm == 2) {
    float b[8];
    if ((reinterpret_cast<uintptr_t>(bias + n) & 15) == 0) {
      const float4 b0 = *reinterpret_cast<const float4*>(bias + n), b1 = *reinterpret_cast<const float4*>(bias + n + 4);
      b[0] = b0.x; b[1] = b0.y; b[2] = b0.z; b[3] = b0.w; b[4] = b1.x; b[5] = b1.y; b[6] = b1.z; b[7] = b1.w;
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) b[c] = bias[n + c];
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] += beta * b[c];
  } else if (bm == 1) {
    const float b = beta * bias[0];
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] += b;
  } else if (bm == 3) {
    const float b = beta * bias[m];
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] += b;
  } else if (bm == 4) {
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] += beta * bias[m * ldb_bias + n + c];
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) v[c] += res[c];
  const int act = e.act;
  if (act == 1) {
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = fmaxf(v[c], 0.0f);
  } else if (act == 2) {
    const float c0 = e.imm[0], c1 = e.imm[1], c2 = e.imm[2];
    const bool sf = gelu_std_ok(c0, c1, c2);
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = gelu_act(v[c], c0, c1, c2, sf);
  }
  const int ni = e.n_inst;
  if (ni > 0) {
    float x[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) x[c] = v[c];
    for (int i = 0; i < ni; ++i) {
      const int op = e.inst[i].op, ca = e.inst[i].a, cb = e.inst[i].b;
      const float imm = e.inst[i].imm;
      const float ia = ca >= 2 ? e.imm[ca - 2] : 0.0f, ib = cb >= 2 ? e.imm[cb - 2] : 0.0f;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float oa = ca == 0 ? x[c] : (ca == 1 ? v[c] : ia);
        const float ob = cb == 0 ? x[c] : (cb == 1 ? v[c] : ib);
        v[c] = ew_apply(op, oa, ob, imm);
      }
    }
  }
}

// ---------------------------------------------------------------- problem
// Division by an invariant d for n < 2^31 (Granlund & Montgomery 1994, the
// round-up multiplier with a 33-bit add): l = ceil(log2 d),
// mul = floor(2^32 (2^l - d) / d) + 1, q = (mulhi(n, mul) + n) >> l.
struct FastDiv {
  uint32_t mul, shift;
};

// Buffer-load byte offset past every num_records used here: reads zeros.
constexpr uint32_t kOobOffset = 0x80000000u;

inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  const uint64_t mul = ((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1;
  return FastDiv{static_cast<uint32_t>(mul), l};
}

// Everything the kernels need, flattened from the gemm/conv args.
struct Problem {
  const void* a;
  const void* b;
  void* out;
  int64_t m, n, k;
  int64_t lda, ldb, ldo;
  int64_t stride_a, stride_b, stride_out, stride_bias, stride_res;
  int trans_a, trans_b;
  int out_dtype;
  // conv geometry (A_MODE == kConv)
  int cn, cc, ch, cw, c_stride, c_pack, kh, kw, kw_pack, sh, sw, pt, pl, dh, dw, ho, wo;
  int out_nchw;  // conv: write NCHW instead of NHWC
  int tiles_m, tiles_n;
  // conv index divisors: ho*wo, wo, c_pack, kw_pack
  FastDiv fd_hw, fd_wo, fd_cpack, fd_kwpack;
  // byte extents of A and B (buffer-resource bounds of the pipelined kernel)
  int64_t a_bytes, b_bytes;
  // int8 GEMM (c3h_qgemm): output mode and quantization parameters; with an
  // int8 output in modes 2 / 3 the epilogue's value is rounded to act_dtype
  // and quantized by (q_scale, q_zero)
  int qmode, y_zero;
  float a_scale, y_scale;
  const float* b_scale;
  float q_scale;
  int q_zero, act_dtype;
  // q_mul != 0: rne(x * q_mul) equals rne(x / q_scale) for every value x of
  // act_dtype (checked over all 65536 encodings on the host), so the
  // interior epilogue quantizes with one multiply
  float q_mul;
  const float* a_rows;  // fp8 GEMM (c3h_gemm_fp8): per-row A scale
  // W4A16 GEMM (c3h_gemm_w4a16): B holds E2M1 codes [n][ldb bytes]; b_blk the
  // E8M0 exponents [n][ldbs] of its 32-element blocks (bs_bytes in all)
  const uint8_t* b_blk;
  int64_t ldbs, bs_bytes;
  c3h_epilogue epi;
};

enum AMode { kDenseK = 0, kDenseM = 1, kConv = 2 };

// XCD-aware tile id: hardware dispatches workgroup i to XCD i % 8.  Give each
// XCD a contiguous range of tile ids (N-fastest) so neighbouring tiles that
// share an A panel share an L2.
__device__ __forceinline__ void tile_coords(const Problem& p, int& tm, int& tn) {
  const int total = p.tiles_m * p.tiles_n;
  int bid = blockIdx.x;
  int tile = bid;
  if ((total & 7) == 0) {
    const int per = total >> 3;
    tile = (bid & 7) * per + (bid >> 3);
  }
  tm = tile / p.tiles_n;
  tn = tile - tm * p.tiles_n;
}

// Decomposed conv output row m -> (input row base offset, hi0, wi0).
struct ConvRow {
  int64_t base;  // element offset of x[n][0][0][0]
  int hi0, wi0;
  bool valid;
};

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

// m < 2^31 (checked on the host): 32-bit index math with invariant divisors.
__device__ __forceinline__ ConvRow conv_row(const Problem& p, int64_t m) {
  ConvRow r;
  r.valid = m < p.m;
  const uint32_t mm = r.valid ? static_cast<uint32_t>(m) : 0u;
  const uint32_t img = fdiv(mm, p.fd_hw);
  const uint32_t rem = mm - img * static_cast<uint32_t>(p.ho * p.wo);
  const uint32_t ho = fdiv(rem, p.fd_wo);
  const uint32_t wo = rem - ho * static_cast<uint32_t>(p.wo);
  r.base = static_cast<int64_t>(img) * p.ch * p.cw * p.c_stride;
  r.hi0 = static_cast<int>(ho) * p.sh - p.pt;
  r.wi0 = static_cast<int>(wo) * p.sw - p.pl;
  return r;
}

// Element offset in x of the VEC-wide K slice starting at k, or -1 when it is
// padding.  K order is (kh, kw_pack, c_pack) with c fastest.
__device__ __forceinline__ int64_t conv_k_offset(const Problem& p, const ConvRow& r, int64_t k) {
  if (!r.valid || k >= p.k) return -1;
  const uint32_t kk = static_cast<uint32_t>(k);
  const uint32_t tap = fdiv(kk, p.fd_cpack);
  const int c0 = static_cast<int>(kk - tap * static_cast<uint32_t>(p.c_pack));
  const uint32_t khi = fdiv(tap, p.fd_kwpack);
  const int kwi = static_cast<int>(tap - khi * static_cast<uint32_t>(p.kw_pack));
  if (kwi >= p.kw || c0 >= p.cc) return -1;
  const int hi = r.hi0 + static_cast<int>(khi) * p.dh;
  const int wi = r.wi0 + kwi * p.dw;
  if (hi < 0 || hi >= p.ch || wi < 0 || wi >= p.cw) return -1;
  return r.base + (static_cast<int64_t>(hi) * p.cw + wi) * p.c_stride + c0;
}

// Epilogue through LDS: a wave stages one 16-row strip of its accumulator
// sub-tile (16 x WTN fp32, row stride WTN + 4) and then stores it with
// consecutive lanes on consecutive output addresses: row-major [m, n] output
// is written as 4 lanes per row, WTN/4 contiguous columns each; NCHW conv
// output is written one column (channel) per lane, 16 consecutive pixels.
template <typename TO, int WTN>
__device__ __forceinline__ void store_strip(const Problem& p, const float* stage, int lane, int64_t mrow0,
                                            int64_t ncol0, TO* outp, const TO* resp, int64_t bias_off) {
  constexpr int SS = WTN + 4;
  if (!p.out_nchw) {
    const int row = lane >> 2;
    const int c0 = (lane & 3) * (WTN / 4);
    const int64_t m = mrow0 + row;
    if (m >= p.m) return;
    if constexpr (std::is_same<TO, float>::value && (WTN == 64 || WTN == 32)) {
      // fp32 rows with all WTN / 4 columns inside N, 16-byte aligned: the
      // lane's residual comes in as WTN / 16 vector loads issued together
      // (one memory round trip per strip instead of one per column) and the
      // results leave as vector stores.  Same per-element arithmetic.
      constexpr int NV = WTN / 16;
      const int64_t o0 = m * p.ldo + ncol0 + c0;
      const bool vec = ncol0 + c0 + WTN / 4 <= p.n && (p.ldo & 3) == 0 && (o0 & 3) == 0 &&
                       (reinterpret_cast<uintptr_t>(outp) & 15) == 0 &&
                       (resp == nullptr || (reinterpret_cast<uintptr_t>(resp) & 15) == 0);
      if (vec) {
        const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 r0 = resp ? *reinterpret_cast<const float4*>(resp + o0) : zero;
        const float4 r1 = resp ? *reinterpret_cast<const float4*>(resp + o0 + 4) : zero;
        const float4 r2 = NV == 4 && resp ? *reinterpret_cast<const float4*>(resp + o0 + 8) : zero;
        const float4 r3 = NV == 4 && resp ? *reinterpret_cast<const float4*>(resp + o0 + 12) : zero;
        const float* srow = stage + row * SS + c0;
        const KArg<c3h_epilogue>& e = kernel_arg<Problem>().epi;
        // A rolled loop (four epilogue copies, not sixteen) keeps the
        // caller's strip loop small enough to unroll, so the accumulators
        // stay in registers.
#pragma unroll 1
        for (int v = 0; v < NV; ++v) {
          const float4 r = v == 0 ? r0 : v == 1 ? r1 : v == 2 ? r2 : r3;
          const int c = 4 * v;
          const int64_t n = ncol0 + c0 + c;
          *reinterpret_cast<float4*>(outp + o0 + c) =
              make_float4(apply_epilogue(e, srow[c], m, n, p.n, r.x, bias_off),
                          apply_epilogue(e, srow[c + 1], m, n + 1, p.n, r.y, bias_off),
                          apply_epilogue(e, srow[c + 2], m, n + 2, p.n, r.z, bias_off),
                          apply_epilogue(e, srow[c + 3], m, n + 3, p.n, r.w, bias_off));
        }
        return;
      }
    }
    for (int c = 0; c < WTN / 4; ++c) {
      const int64_t n = ncol0 + c0 + c;
      if (n >= p.n) break;
      const int64_t o = m * p.ldo + n;
      const float res = resp ? Elem<TO>::to_f32(resp[o]) : 0.0f;
      outp[o] = Elem<TO>::from_f32(apply_epilogue(kernel_arg<Problem>().epi, stage[row * SS + c0 + c], m, n, p.n, res, bias_off));
    }
  } else {
    const int64_t hw = static_cast<int64_t>(p.ho) * p.wo;
    for (int col = lane; col < WTN; col += 64) {
      const int64_t n = ncol0 + col;
      if (n >= p.n) break;
      for (int row = 0; row < 16; ++row) {
        const int64_t m = mrow0 + row;
        if (m >= p.m) break;
        const int64_t img = m / hw, pix = m - img * hw;
        const int64_t o = (img * p.n + n) * hw + pix;
        const float res = resp ? Elem<TO>::to_f32(resp[o]) : 0.0f;
        outp[o] = Elem<TO>::from_f32(apply_epilogue(kernel_arg<Problem>().epi, stage[row * SS + col], m, n, p.n, res, bias_off));
      }
    }
  }
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
}

// =====================================================================
// fp32 kernel: v_mfma_f32_16x16x4_f32.  LDS tiles are stored k-major
// (As[k][m], Bs[k][n]) so each lane's MFMA operand is one conflict-free
// ds_read_b32.
// =====================================================================
template <int BM, int BN, int WM, int WN, int AM, bool B_KCONTIG>
__global__ void __launch_bounds__(kThreads) gemm_f32_kernel(Problem p) {
  constexpr int BK = 16;
  constexpr int PADM = 16;  // row stride = BM + 16 floats -> 16-bank skew per k
  constexpr int SA = BM + PADM, SB = BN + PADM;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int WTN = BN / WN;
  constexpr int kTileFloats = 2 * BK * SA + 2 * BK * SB;
  constexpr int kStageFloats = 4 * 16 * (WTN + 4);
  __shared__ __attribute__((aligned(16))) float smem[kTileFloats > kStageFloats ? kTileFloats : kStageFloats];
  float (*As)[BK][SA] = reinterpret_cast<float (*)[BK][SA]>(smem);
  float (*Bs)[BK][SB] = reinterpret_cast<float (*)[BK][SB]>(smem + 2 * BK * SA);

  int tm, tn;
  tile_coords(p, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const int64_t bz = blockIdx.z;
  const float* A = static_cast<const float*>(p.a) + bz * p.stride_a;
  const float* B = static_cast<const float*>(p.b) + bz * p.stride_b;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;

  // A tile: BM x BK floats.  K-contiguous modes: thread loads float4 along k
  // (4 threads per row).  M-contiguous mode: float4 along m.
  constexpr int A_VECS = BM * BK / 4 / kThreads;  // float4 per thread
  constexpr int B_VECS = BN * BK / 4 / kThreads;
  static_assert(A_VECS >= 1 && B_VECS >= 1, "tile too small");
  float4 ra[A_VECS], rb[B_VECS];

  ConvRow crow[A_VECS];
  if (AM == kConv) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      int e = tid + kThreads * i;
      crow[i] = conv_row(p, m0 + e / (BK / 4));
    }
  }

  auto load_a = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      int e = tid + kThreads * i;
      if (AM == kDenseM) {
        int kr = e / (BM / 4), mc = (e % (BM / 4)) * 4;
        int64_t k = k0 + kr, m = m0 + mc;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < p.k) {
          const float* src = A + k * p.lda + m;
          if (m + 3 < p.m) v = *reinterpret_cast<const float4*>(src);
          else {
            if (m < p.m) v.x = src[0];
            if (m + 1 < p.m) v.y = src[1];
            if (m + 2 < p.m) v.z = src[2];
          }
        }
        ra[i] = v;
      } else {
        int mr = e / (BK / 4), kc = (e % (BK / 4)) * 4;
        int64_t m = m0 + mr, k = k0 + kc;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (AM == kDenseK) {
          if (m < p.m) {
            const float* src = A + m * p.lda + k;
            if (k + 3 < p.k) v = *reinterpret_cast<const float4*>(src);
            else {
              if (k < p.k) v.x = src[0];
              if (k + 1 < p.k) v.y = src[1];
              if (k + 2 < p.k) v.z = src[2];
            }
          }
        } else {
          int64_t off = conv_k_offset(p, crow[i], k);
          if (off >= 0) v = *reinterpret_cast<const float4*>(A + off);
        }
        ra[i] = v;
      }
    }
  };
  auto load_b = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      int e = tid + kThreads * i;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (B_KCONTIG) {  // B stored [n][k]
        int nr = e / (BK / 4), kc = (e % (BK / 4)) * 4;
        int64_t n = n0 + nr, k = k0 + kc;
        if (n < p.n) {
          const float* src = B + n * p.ldb + k;
          if (k + 3 < p.k) v = *reinterpret_cast<const float4*>(src);
          else {
            if (k < p.k) v.x = src[0];
            if (k + 1 < p.k) v.y = src[1];
            if (k + 2 < p.k) v.z = src[2];
          }
        }
      } else {  // B stored [k][n]
        int kr = e / (BN / 4), nc = (e % (BN / 4)) * 4;
        int64_t k = k0 + kr, n = n0 + nc;
        if (k < p.k) {
          const float* src = B + k * p.ldb + n;
          if (n + 3 < p.n) v = *reinterpret_cast<const float4*>(src);
          else {
            if (n < p.n) v.x = src[0];
            if (n + 1 < p.n) v.y = src[1];
            if (n + 2 < p.n) v.z = src[2];
          }
        }
      }
      rb[i] = v;
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      int e = tid + kThreads * i;
      if (AM == kDenseM) {
        int kr = e / (BM / 4), mc = (e % (BM / 4)) * 4;
        *reinterpret_cast<float4*>(&As[buf][kr][mc]) = ra[i];
      } else {
        int mr = e / (BK / 4), kc = (e % (BK / 4)) * 4;
        As[buf][kc + 0][mr] = ra[i].x;
        As[buf][kc + 1][mr] = ra[i].y;
        As[buf][kc + 2][mr] = ra[i].z;
        As[buf][kc + 3][mr] = ra[i].w;
      }
    }
#pragma unroll
    for (int i = 0; i < B_VECS; ++i) {
      int e = tid + kThreads * i;
      if (B_KCONTIG) {
        int nr = e / (BK / 4), kc = (e % (BK / 4)) * 4;
        Bs[buf][kc + 0][nr] = rb[i].x;
        Bs[buf][kc + 1][nr] = rb[i].y;
        Bs[buf][kc + 2][nr] = rb[i].z;
        Bs[buf][kc + 3][nr] = rb[i].w;
      } else {
        int kr = e / (BN / 4), nc = (e % (BN / 4)) * 4;
        *reinterpret_cast<float4*>(&Bs[buf][kr][nc]) = rb[i];
      }
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t ktiles = ceil_div(p.k, BK);
  load_a(0);
  load_b(0);
  store_tiles(0);
  __syncthreads();
  const int lrow = lane & 15, lk = lane >> 4;
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) {
      load_a((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }
#pragma unroll
    for (int ks = 0; ks < BK / 4; ++ks) {
      float av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) av[i] = As[cur][ks * 4 + lk][wm * (BM / WM) + i * 16 + lrow];
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[j] = Bs[cur][ks * 4 + lk][wn * (BN / WN) + j * 16 + lrow];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < ktiles) {
      store_tiles(cur ^ 1);
      __syncthreads();
    }
  }

  // Epilogue: lane holds rows 4*(lane/16)+r, col lane%16 of each 16x16 tile;
  // stage each 16-row strip through LDS and store it coalesced.
  float* outp = static_cast<float*>(p.out) + bz * p.stride_out;
  const float* resp = p.epi.residual ? static_cast<const float*>(p.epi.residual) + bz * p.stride_res : nullptr;
  const int64_t bias_off = bz * p.stride_bias;
  __syncthreads();
  float* stage = smem + wave * 16 * (WTN + 4);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) stage[(lk * 4 + r) * (WTN + 4) + j * 16 + lrow] = acc[i][j][r];
    wave_sync_lds();
    store_strip<float, WTN>(p, stage, lane, m0 + wm * (BM / WM) + i * 16, n0 + wn * WTN, outp, resp, bias_off);
    wave_sync_lds();
  }
}

// =====================================================================
// MFMA kernel for 16-bit (v_mfma_f32_16x16x32_{bf16,f16}) and int8
// (v_mfma_i32_16x16x64_i8, exact int32 accumulation) operands.  A tile row
// is 128 bytes of K (64 16-bit or 128 int8 elements); LDS rows hold eight
// 16-byte chunks XOR-swizzled by (row & 7), so a lane's MFMA operand is one
// ds_read_b128 and 8 consecutive rows reading the same K chunk hit 8
// distinct bank groups.  Every thread moves 16-byte vectors; since 256 % 8
// == 0 a thread's vectors share one K chunk and step 32 rows apart.
//
// A operand modes:
//   kDenseK    A[m][k] row-major (lda).
//   kConvTap   implicit-GEMM conv with c_pack % 64 == 0: a 64-wide K tile lies
//              inside one filter tap, so (kh, kw, c0) is uniform per tile and
//              advanced incrementally; each row keeps its pixel base.
//   kConv      generic implicit GEMM (c_pack % 8 == 0): per-vector tap math.
//   kConvStem  c_pack == c_stride == 4, kw padded to 8: a vector is two taps
//              of one input row (two 8-byte halves, each bounds-checked).
// =====================================================================
typedef __attribute__((ext_vector_type(4))) int i32x4;

// kStep: 16-byte K chunks of a tile row one MFMA consumes per lane group
// (4: two MFMA steps per 128-byte row; 8: one step).  kScaled: accumulators
// are multiplied by a_rows[m] * b_scale[n] before the epilogue.
struct MmaBF16 {
  typedef bf16x8 vec;
  typedef f32x4 acc_t;
  static constexpr int ES = 2;
  static constexpr bool kInt = false;
  static constexpr int kStep = 4;
  static constexpr bool kScaled = false;
  static __device__ __forceinline__ acc_t mma(vec a, vec b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
struct MmaF16 {
  typedef f16x8 vec;
  typedef f32x4 acc_t;
  static constexpr int ES = 2;
  static constexpr bool kInt = false;
  static constexpr int kStep = 4;
  static constexpr bool kScaled = false;
  static __device__ __forceinline__ acc_t mma(vec a, vec b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
struct MmaI8 {
  typedef i32x4 vec;
  typedef i32x4 acc_t;
  static constexpr int ES = 1;
  static constexpr bool kInt = true;
  static constexpr int kStep = 4;
  static constexpr bool kScaled = false;
  static __device__ __forceinline__ acc_t mma(vec a, vec b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
};
// OCP E4M3 x E4M3 -> fp32 (v_mfma_f32_16x16x128_f8f6f4, format code 0 on
// both operands, no block scales).  A lane supplies 32 K bytes: lane group g
// (lane >> 4) takes tile-row chunks g and g + 4.  A and B use the same
// lane/byte -> k assignment, so the dot product covers each k exactly once
// whatever order the instruction walks K in.
typedef __attribute__((ext_vector_type(8))) int i32x8;
struct MmaF8 {
  typedef i32x8 vec;
  typedef f32x4 acc_t;
  static constexpr int ES = 1;
  static constexpr bool kInt = false;
  static constexpr int kStep = 8;
  static constexpr bool kScaled = true;
  static __device__ __forceinline__ acc_t mma(vec a, vec b, acc_t c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
};

// MFMA operand of tile row `r` (row base `row`, XOR-swizzled 16-byte chunks)
// for the K step starting at chunk ks.
template <typename Mma>
__device__ __forceinline__ typename Mma::vec read_operand(const uint8_t* row, int r, int ks, int lchunk) {
  if constexpr (Mma::kStep == 8) {
    const i32x4 lo = *reinterpret_cast<const i32x4*>(row + ((lchunk ^ (r & 7)) << 4));
    const i32x4 hi = *reinterpret_cast<const i32x4*>(row + (((lchunk + 4) ^ (r & 7)) << 4));
    return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  } else {
    return *reinterpret_cast<const typename Mma::vec*>(row + (((ks + lchunk) ^ (r & 7)) << 4));
  }
}

enum AMode16 { kConvTap = 3, kConvStem = 4 };

// Grouped tile order: each XCD (blockIdx % 8) owns a contiguous range of tile
// ids, walked in column-major groups of 8 tile rows so blocks resident at
// the same time share both A and B panels in that XCD's L2.
__device__ __forceinline__ void tile_coords_of(const Problem& p, int id, int& tm, int& tn) {
  // XCD x = id % 8 receives ids x, x + 8, ...: count q + (x < r) of them for
  // total = 8 q + r; its j-th one takes tile x q + min(x, r) + j, so every
  // XCD walks a contiguous tile range (a bijection for any total).
  const int total = p.tiles_m * p.tiles_n;
  const int x = id & 7, q = total >> 3, r = total & 7;
  const int tile = x * q + min(x, r) + (id >> 3);
  constexpr int G = 8;
  const int group = tile / (G * p.tiles_n);
  const int first_m = group * G;
  const int gsize = min(p.tiles_m - first_m, G);
  const int in_group = tile - group * G * p.tiles_n;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}
__device__ __forceinline__ void tile_coords_grouped(const Problem& p, int& tm, int& tn) {
  tile_coords_of(p, blockIdx.x, tm, tn);
}

// Vectorized epilogue of one 16-row strip (row-major [m, n] output): each
// lane owns 8 consecutive columns, so a row is written as WTN/8 16-byte
// (bf16/fp16) or 32-byte (fp32) stores.  Called from a runtime loop over
// strips: the whole wave tile is staged in LDS first, so the accumulators are
// only ever indexed by unrolled (constant) indices.
template <typename TO, int WTN>
__device__ __forceinline__ void store_strip_vec(const float* stage, int lane, int64_t mrow0, int64_t ncol0,
                                                          TO* outp, const TO* resp, int64_t bias_off, bool vec_ok) {
  const KArg<Problem>& p = kernel_arg<Problem>();
  constexpr int SS = WTN + 4;
  constexpr int LPR = WTN / 8;
  constexpr int RPP = 64 / LPR;
  static_assert(LPR >= 1 && 64 % LPR == 0 && RPP <= 16, "strip shape");
  const int64_t pm = p.m, pn = p.n, ldo = p.ldo;
  for (int pass = 0; pass < 16 / RPP; ++pass) {
    const int row = pass * RPP + lane / LPR;
    const int c0 = (lane % LPR) * 8;
    const int64_t m = mrow0 + row;
    const int64_t n = ncol0 + c0;
    if (m >= pm || n >= pn) continue;
    const float4 lo = *reinterpret_cast<const float4*>(stage + row * SS + c0);
    const float4 hi = *reinterpret_cast<const float4*>(stage + row * SS + c0 + 4);
    float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    const int64_t o = m * ldo + n;
    if (vec_ok && n + 8 <= pn) {
      float res[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (resp) Elem<TO>::load8(resp + o, res);
      apply_epilogue8(p.epi, v, m, n, pn, res, bias_off);
      Elem<TO>::store8(outp + o, v);
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        if (n + c < pn) {
          const float res = resp ? Elem<TO>::to_f32(resp[o + c]) : 0.0f;
          outp[o + c] = Elem<TO>::from_f32(apply_epilogue(p.epi, v[c], m, n + c, pn, res, bias_off));
        }
      }
    }
  }
}

// int8 GEMM epilogue of one 16-row strip: the stage holds int32 accumulator
// bits.  qmode 0 writes int32, 1 requantizes to int8, 2 dequantizes, 3
// requantizes then dequantizes (QLinearMatMul -> DequantizeLinear); 2 and 3
// continue through the float epilogue into TO.
template <typename TO, int WTN>
__device__ __forceinline__ void store_strip_q(const float* stage, int lane, int64_t mrow0, int64_t ncol0, TO* outp,
                                              const TO* resp, bool vec_ok) {
  const KArg<Problem>& p = kernel_arg<Problem>();
  constexpr int SS = WTN + 4;
  constexpr int LPR = WTN / 8;
  constexpr int RPP = 64 / LPR;
  const int64_t pm = p.m, pn = p.n, ldo = p.ldo;
  const int mode = p.qmode;
  const float sa = p.a_scale, sy = p.y_scale, zy = static_cast<float>(p.y_zero);
  const bool requant = mode == 1 || mode == 3;
  const QuantDiv qd(p.q_scale);  // int8 output of modes 2 / 3
  // A lane's 8 columns are the same in every pass: their multipliers
  // ((sa * sb) / sy requantizing, sa * sb for mode 2) are computed once.
  const int c0 = (lane % LPR) * 8;
  float mult[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int64_t nc = ncol0 + c0 + c;
    const float bsc = (mode != 0 && nc < pn) ? p.b_scale[nc] : 0.0f;
    mult[c] = requant ? (sa * bsc) / sy : sa * bsc;
  }
  for (int pass = 0; pass < 16 / RPP; ++pass) {
    const int row = pass * RPP + lane / LPR;
    const int64_t m = mrow0 + row;
    const int64_t n = ncol0 + c0;
    if (m >= pm || n >= pn) continue;
    const int4 lo = *reinterpret_cast<const int4*>(stage + row * SS + c0);
    const int4 hi = *reinterpret_cast<const int4*>(stage + row * SS + c0 + 4);
    const int acc[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    const int64_t o = m * ldo + n;
    const bool full = vec_ok && n + 8 <= pn;
    if constexpr (std::is_same<TO, int32_t>::value) {
      int32_t* out = outp;
      if (full) {
        reinterpret_cast<int4*>(out + o)[0] = lo;
        reinterpret_cast<int4*>(out + o)[1] = hi;
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (n + c < pn) out[o + c] = acc[c];
      }
    } else {
      float v[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        if (requant) {
          float y = rintf(static_cast<float>(acc[c]) * mult[c]) + zy;
          y = fminf(fmaxf(y, -128.0f), 127.0f);
          v[c] = mode == 1 ? y : (y - zy) * sy;
        } else {
          v[c] = static_cast<float>(acc[c]) * mult[c];
        }
      }
      if constexpr (std::is_same<TO, int8_t>::value) {
        int8_t* out = outp;
        if (mode >= 2) {
          // the float epilogue (no residual into an int8 output), rounded to
          // the activation type, then QuantizeLinear: codes in v
          float res[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          if (full) {
            apply_epilogue8(p.epi, v, m, n, pn, res, 0);
          } else {
#pragma unroll
            for (int c = 0; c < 8; ++c)
              if (n + c < pn) v[c] = apply_epilogue(p.epi, v[c], m, n + c, pn, 0.0f, 0);
          }
#pragma unroll
          for (int c = 0; c < 8; ++c) v[c] = static_cast<float>(qd.code(round_to_dtype(v[c], p.act_dtype), p.q_zero));
        }
        if (full) {
          uint32_t w[2] = {0u, 0u};
#pragma unroll
          for (int c = 0; c < 8; ++c)
            w[c >> 2] |= (static_cast<uint32_t>(static_cast<int8_t>(v[c])) & 0xffu) << (8 * (c & 3));
          *reinterpret_cast<uint2*>(out + o) = uint2{w[0], w[1]};
        } else {
#pragma unroll
          for (int c = 0; c < 8; ++c)
            if (n + c < pn) out[o + c] = static_cast<int8_t>(v[c]);
        }
      } else if (full) {
        float res[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (resp) Elem<TO>::load8(resp + o, res);
        apply_epilogue8(p.epi, v, m, n, pn, res, 0);
        Elem<TO>::store8(outp + o, v);
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          if (n + c < pn) {
            const float res = resp ? Elem<TO>::to_f32(resp[o + c]) : 0.0f;
            outp[o + c] = Elem<TO>::from_f32(apply_epilogue(p.epi, v[c], m, n + c, pn, res, 0));
          }
        }
      }
    }
  }
}

// Epilogue straight from C^T accumulators (16-bit and fp32 MFMA kernels,
// which multiply with the operands swapped): acc[i][j][r] is output row
// m = mbase + 16 i + l16, column n = nbase + 16 j + 4 lg + r, so a lane owns
// 4 consecutive columns of a row and writes them as one 8-byte (16-bit) or
// 16-byte (fp32) store after the epilogue, with no LDS round trip.
// Calls f(std::integral_constant<int, 0>) ... f(<N - 1>): indices that are
// constants before any loop unrolling, so register arrays indexed by them
// never become addressable (scratch) memory.
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// The value a consumer reads back after the epilogue stores x as TO.
template <typename TO>
__device__ __forceinline__ float stored_value(float x) {
  if constexpr (std::is_same<TO, float>::value) return x;
  else return Elem<TO>::to_f32(Elem<TO>::from_f32(x));
}

// Per-row block maxima of the stored values (the epilogue's row_max side
// output, what an ArgMax of the output finishes from), one tracker per
// 64-column block of the wave tile (TN / 4 of them) in each lane: the
// maximum ignoring NaN (v_max_f32), and a NaN witness x * 0 summed in (NaN
// once the block held a NaN -- or an infinity, which only sends the finish
// to look at the block's values).  Two VALU operations per element.  The 4
// lanes of a row then merge the same way.
struct RowMax {
  float v, nan;
  __device__ __forceinline__ void start() { v = -INFINITY; nan = 0.0f; }
  __device__ __forceinline__ void see(float x) {
    v = fmaxf(v, x);
    nan = fmaf(x, 0.0f, nan);
  }
  __device__ __forceinline__ void merge(int xaddr) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_bpermute(xaddr, __float_as_int(v))));
    nan += __int_as_float(__builtin_amdgcn_ds_bpermute(xaddr, __float_as_int(nan)));
  }
};

// Merge each row's 4 lanes (lane, lane ^ 16, lane ^ 32, lane ^ 48) and write
// its blocks from lanes 0-15, which hold rows mrow0 + lane.  Every lane of
// the wave takes part (ds_bpermute reads the other lanes' registers).
template <int NB>
__device__ __forceinline__ void row_max_store(RowMax (&t)[NB], int lane, int64_t mrow0, int64_t nbase) {
  const KArg<Problem>& p = kernel_arg<Problem>();
  const int x16 = (lane ^ 16) << 2, x32 = (lane ^ 32) << 2;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    t[b].merge(x16);
    t[b].merge(x32);
  }
  const int64_t m = mrow0 + lane;
  if (lane < 16 && m < p.m) {
    c3h_block_max* dst = p.epi.row_max + m * p.epi.row_max_ld + nbase / 64;
#pragma unroll
    for (int b = 0; b < NB; ++b)
      if (nbase + 64 * b < p.n)
        *reinterpret_cast<uint2*>(dst + b) = uint2{__float_as_uint(t[b].v), t[b].nan != t[b].nan ? 1u : 0u};
  }
}

// The 16-bit and fp32 MFMA kernels multiply with the operands swapped, so
// acc[i][j][r] is C^T: output row m = mbase + 16 i + l16, column
// n = nbase + 16 j + 4 lg + r.  A lane owns 4 consecutive columns of a row.
//
// Common epilogue (row-major output, alpha = beta = 1, bias absent or per
// column, optional residual, optional ReLU, no program) straight from the
// accumulators: one 8-byte (16-bit) or 16-byte (fp32) store per 4 values, no
// LDS round trip.  Same arithmetic as apply_epilogue: ((acc + b) + res), max 0.
// G: the GELU form (act 2, gelu_erf with imm[0..2]), a separate
// instantiation so the plain form carries no per-element GELU code.
template <typename TO, int TM, int TN, bool G, typename Acc>
__device__ __forceinline__ void epilogue_direct_impl(const Acc (&acc)[TM][TN], int64_t mbase, int64_t nbase,
                                                     int lane, TO* outp, const TO* resp, const float* bias, int act) {
  const KArg<Problem>& p = kernel_arg<Problem>();
  const bool relu = !G && act == 1;
  constexpr bool gelu = G;
  const float g0 = G ? p.epi.imm[0] : 0.0f, g1 = G ? p.epi.imm[1] : 0.0f, g2 = G ? p.epi.imm[2] : 0.0f;
  const bool gstd = G && gelu_std_ok(g0, g1, g2);
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t pm = p.m, pn = p.n, ldo = p.ldo;
  // Bias of this lane's columns, for every column tile.
  float b[TN][4];
  static_for<TN>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    const int64_t n = nbase + 16 * j + 4 * lg;
#pragma unroll
    for (int r = 0; r < 4; ++r) b[j][r] = 0.0f;
    if (bias && n + 4 <= pn) {
      const float4 q = *reinterpret_cast<const float4*>(bias + n);
      b[j][0] = q.x; b[j][1] = q.y; b[j][2] = q.z; b[j][3] = q.w;
    }
  });
  static_assert(TN % 4 == 0, "wave tiles of whole 64-column blocks (row_max)");
  const bool rb = p.epi.row_max != nullptr;
  // Row by row: a row's column tiles share cache lines, so its residual
  // loads and its stores go out back to back (interleaving rows makes L2
  // write partial lines back more than once).
  static_for<TM>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    const int64_t m = mbase + 16 * i + l16;
    RowMax best[TN / 4];
#pragma unroll
    for (int q = 0; q < TN / 4; ++q) best[q].start();
    if (m < pm) {
      float res[TN][4];
      static_for<TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int64_t n = nbase + 16 * j + 4 * lg;
#pragma unroll
        for (int r = 0; r < 4; ++r) res[j][r] = 0.0f;
        if (resp && n + 4 <= pn) Elem<TO>::load4(resp + m * ldo + n, res[j]);
      });
      static_for<TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int64_t n = nbase + 16 * j + 4 * lg;
        float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        if (n + 4 <= pn) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float t = (v[r] + b[j][r]) + res[j][r];
            v[r] = relu ? fmaxf(t, 0.0f) : (gelu ? gelu_act(t, g0, g1, g2, gstd) : t);
            if (rb) best[j / 4].see(stored_value<TO>(v[r]));
          }
          Elem<TO>::store4(outp + m * ldo + n, v);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (n + r < pn) {
              const int64_t o = m * ldo + n + r;
              float t = (v[r] + (bias ? bias[n + r] : 0.0f)) + (resp ? Elem<TO>::to_f32(resp[o]) : 0.0f);
              const float y = relu ? fmaxf(t, 0.0f) : (gelu ? gelu_act(t, g0, g1, g2, gstd) : t);
              outp[o] = Elem<TO>::from_f32(y);
              if (rb) best[j / 4].see(stored_value<TO>(y));
            }
          }
        }
      });
    }
    if (rb) row_max_store(best, lane, mbase + 16 * i, nbase);
  });
}

// GELU: act 2 is computed in registers only by the instantiations that ask
// for it (the large-tile kernel, which has no staged epilogue).
// epilogue_direct for a wave tile wholly inside the output: no bounds tests,
// the activation fixed at compile time (ACT: 0 none, 1 ReLU, 2 GELU with
// run-time constants, 3 GELU with the standard ones, gelu_std).  Same
// arithmetic: ((acc + b) + res), then the activation.
template <typename TO, int TM, int TN, int ACT, bool RB, typename Acc>
__device__ __forceinline__ void epilogue_direct_interior(const Acc (&acc)[TM][TN], int64_t mbase, int64_t nbase,
                                                         int lane, TO* outp, const TO* resp, const float* bias) {
#pragma clang fp contract(off)
  const KArg<Problem>& p = kernel_arg<Problem>();
  const float g0 = p.epi.imm[0], g1 = p.epi.imm[1], g2 = p.epi.imm[2];
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t ldo = p.ldo;
  float b[TN][4];
  static_for<TN>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
#pragma unroll
    for (int r = 0; r < 4; ++r) b[j][r] = 0.0f;
    if (bias) {
      const float4 q = *reinterpret_cast<const float4*>(bias + nbase + 16 * j + 4 * lg);
      b[j][0] = q.x; b[j][1] = q.y; b[j][2] = q.z; b[j][3] = q.w;
    }
  });
  if constexpr (sizeof(TO) == 2 && TN % 2 == 0 && ACT <= 1) {
    // 16-bit output rows 16-byte aligned: residual loads and stores of 16
    // bytes per lane (a lane row's 8 columns of each pair of column tiles),
    // converted from / to the accumulators' 4 columns per lane by lane swaps
    // (rows_to_ct_pair, ct_pair_to_rows).  Same values, wider accesses.
    // (GELU interiors keep the 8-byte form: measured faster there, the
    // fp16 decoder's FFN1 54 against 56-57 us.)
    if ((ldo & 7) == 0 && (reinterpret_cast<uintptr_t>(outp) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(resp) & 15) == 0) {
      TO* base = outp + (mbase + l16) * ldo + nbase + 8 * lg;
      const TO* rbase = resp ? resp + (mbase + l16) * ldo + nbase + 8 * lg : nullptr;
      static_for<TM>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        RowMax best[TN / 4];
        if constexpr (RB) {
#pragma unroll
          for (int q = 0; q < TN / 4; ++q) best[q].start();
        }
        float res[TN][4];
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) res[j][r] = 0.0f;
        if (rbase) {
          static_for<TN / 2>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            uint32_t d0[2], d1[2];
            rows_to_ct_pair(*reinterpret_cast<const uint4*>(rbase + 16 * i * ldo + 32 * q), d0, d1);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              Elem<TO>::unpack2(d0[h], &res[2 * q][2 * h]);
              Elem<TO>::unpack2(d1[h], &res[2 * q + 1][2 * h]);
            }
          });
        }
        uint32_t pk[TN][2];
        static_for<TN>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float t = (acc[i][j][r] + b[j][r]) + res[j][r];
            v[r] = ACT == 1 ? fmaxf(t, 0.0f) : (ACT == 3 ? gelu_std(t) : (ACT == 2 ? gelu_erf(t, g0, g1, g2) : t));
            if constexpr (RB) best[j / 4].see(stored_value<TO>(v[r]));
          }
          pk[j][0] = Elem<TO>::pack2(v[0], v[1]);
          pk[j][1] = Elem<TO>::pack2(v[2], v[3]);
        });
        static_for<TN / 2>([&](auto qc) {
          constexpr int q = decltype(qc)::value;
          *reinterpret_cast<uint4*>(base + 16 * i * ldo + 32 * q) = ct_pair_to_rows(pk[2 * q], pk[2 * q + 1]);
        });
        if constexpr (RB) row_max_store(best, lane, mbase + 16 * i, nbase);
      });
      return;
    }
  }
  TO* base = outp + (mbase + l16) * ldo + nbase + 4 * lg;
  const TO* rbase = resp ? resp + (mbase + l16) * ldo + nbase + 4 * lg : nullptr;
  static_for<TM>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    RowMax best[TN / 4];
    if constexpr (RB) {
#pragma unroll
      for (int q = 0; q < TN / 4; ++q) best[q].start();
    }
    float res[TN][4];
    static_for<TN>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
#pragma unroll
      for (int r = 0; r < 4; ++r) res[j][r] = 0.0f;
      if (rbase) Elem<TO>::load4(rbase + 16 * i * ldo + 16 * j, res[j]);
    });
    static_for<TN>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float t = (acc[i][j][r] + b[j][r]) + res[j][r];
        v[r] = ACT == 1 ? fmaxf(t, 0.0f) : (ACT == 3 ? gelu_std(t) : (ACT == 2 ? gelu_erf(t, g0, g1, g2) : t));
        if constexpr (RB) best[j / 4].see(stored_value<TO>(v[r]));
      }
      Elem<TO>::store4(base + 16 * i * ldo + 16 * j, v);
    });
    if constexpr (RB) row_max_store(best, lane, mbase + 16 * i, nbase);
  });
}

template <typename TO, int TM, int TN, bool GELU = false, typename Acc>
__device__ __forceinline__ void epilogue_direct(const Acc (&acc)[TM][TN], int64_t mbase, int64_t nbase, int lane,
                                                TO* outp, const TO* resp, const float* bias, int act) {
  const KArg<Problem>& p = kernel_arg<Problem>();
  if (mbase + 16 * TM <= p.m && nbase + 16 * TN <= p.n) {
    const bool rb = p.epi.row_max != nullptr;  // host: only with act <= 1
    if (act == 0) {
      if (rb) epilogue_direct_interior<TO, TM, TN, 0, true>(acc, mbase, nbase, lane, outp, resp, bias);
      else epilogue_direct_interior<TO, TM, TN, 0, false>(acc, mbase, nbase, lane, outp, resp, bias);
      return;
    }
    if (act == 1) {
      if (rb) epilogue_direct_interior<TO, TM, TN, 1, true>(acc, mbase, nbase, lane, outp, resp, bias);
      else epilogue_direct_interior<TO, TM, TN, 1, false>(acc, mbase, nbase, lane, outp, resp, bias);
      return;
    }
    if constexpr (GELU) {
      // GELU interiors for the standard constants only; others take the
      // general form below
      if (!rb && gelu_std_ok(p.epi.imm[0], p.epi.imm[1], p.epi.imm[2])) {
        epilogue_direct_interior<TO, TM, TN, 3, false>(acc, mbase, nbase, lane, outp, resp, bias);
        return;
      }
    }
  }
  if (GELU && act == 2) epilogue_direct_impl<TO, TM, TN, true>(acc, mbase, nbase, lane, outp, resp, bias, act);
  else epilogue_direct_impl<TO, TM, TN, false>(acc, mbase, nbase, lane, outp, resp, bias, act);
}

// int8 GEMM (c3h_qgemm) counterpart of epilogue_direct for C^T int32
// accumulators: qmode 0 stores int32, 1 requantizes to int8 (4 bytes per
// lane), 2 dequantizes and 3 requantizes then dequantizes, both followed by
// the common float epilogue (simple_epi).  Arithmetic as store_strip_q.
template <typename TO, int TM, int TN, bool G, typename Acc>
__device__ __forceinline__ void epilogue_direct_q_impl(const Acc (&acc)[TM][TN], int64_t mbase, int64_t nbase,
                                                       int lane, TO* outp, const TO* resp, const float* bias, int act) {
  const KArg<Problem>& p = kernel_arg<Problem>();
  const bool relu = !G && act == 1;
  constexpr bool gelu = G;
  const float g0 = G ? p.epi.imm[0] : 0.0f, g1 = G ? p.epi.imm[1] : 0.0f, g2 = G ? p.epi.imm[2] : 0.0f;
  const bool gstd = G && gelu_std_ok(g0, g1, g2);
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t pm = p.m, pn = p.n, ldo = p.ldo;
  const int mode = p.qmode;
  const float sa = p.a_scale, sy = p.y_scale, zy = static_cast<float>(p.y_zero);
  const bool requant = mode == 1 || mode == 3;
  const QuantDiv qd(p.q_scale);  // int8 output of modes 2 / 3
  const int act_dt = p.act_dtype, qz = p.q_zero;
  // Per-column multiplier, once per lane: (sa * sb) / sy for requantizing
  // modes, sa * sb for mode 2 (the same roundings as per element).
  float mult[TN][4], b[TN][4];
  static_for<TN>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    const int64_t n = nbase + 16 * j + 4 * lg;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float sbv = 0.0f;
      b[j][r] = 0.0f;
      if (n + r < pn) {
        if (mode != 0) sbv = p.b_scale[n + r];
        if (bias) b[j][r] = bias[n + r];
      }
      mult[j][r] = requant ? (sa * sbv) / sy : sa * sbv;
    }
  });
  static_assert(TN % 4 == 0, "wave tiles of whole 64-column blocks (row_max)");
  constexpr bool kFloatOut = !std::is_same<TO, int32_t>::value && !std::is_same<TO, int8_t>::value;
  const bool rb = kFloatOut && p.epi.row_max != nullptr;
  // Row by row, as epilogue_direct: a row's stores go out back to back.
  static_for<TM>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    const int64_t m = mbase + 16 * i + l16;
    RowMax best[TN / 4];
#pragma unroll
    for (int q = 0; q < TN / 4; ++q) best[q].start();
    if (m < pm) {
      float res[TN][4];
      static_for<TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int64_t n = nbase + 16 * j + 4 * lg;
#pragma unroll
        for (int r = 0; r < 4; ++r) res[j][r] = 0.0f;
        if constexpr (!std::is_same<TO, int32_t>::value && !std::is_same<TO, int8_t>::value) {
          if (resp && n + 4 <= pn) Elem<TO>::load4(resp + m * ldo + n, res[j]);
        }
      });
      static_for<TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int64_t n = nbase + 16 * j + 4 * lg;
        const bool nfull = n + 4 <= pn;
        const int64_t o = m * ldo + n;
        if (n < pn) {
          if constexpr (std::is_same<TO, int32_t>::value) {
            if (nfull) {
              *reinterpret_cast<int4*>(outp + o) = int4{acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (n + r < pn) outp[o + r] = acc[i][j][r];
            }
          } else {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float a = static_cast<float>(acc[i][j][r]);
              if (requant) {
                float y = rintf(a * mult[j][r]) + zy;
                y = fminf(fmaxf(y, -128.0f), 127.0f);
                v[r] = mode == 1 ? y : (y - zy) * sy;
              } else {
                v[r] = a * mult[j][r];
              }
            }
            if constexpr (std::is_same<TO, int8_t>::value) {
              if (mode >= 2) {
                // dequantized value, bias and activation, rounded to the
                // activation type, then QuantizeLinear: codes in v
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const float t = v[r] + b[j][r];
                  const float y = relu ? fmaxf(t, 0.0f) : (gelu ? gelu_act(t, g0, g1, g2, gstd) : t);
                  v[r] = static_cast<float>(qd.code(round_to_dtype(y, act_dt), qz));
                }
              }
              if (nfull) {
                uint32_t w = 0u;
#pragma unroll
                for (int r = 0; r < 4; ++r) w |= (static_cast<uint32_t>(static_cast<int8_t>(v[r])) & 0xffu) << (8 * r);
                *reinterpret_cast<uint32_t*>(outp + o) = w;
              } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  if (n + r < pn) outp[o + r] = static_cast<int8_t>(v[r]);
              }
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                float rr = res[j][r];
                if (resp && !nfull && n + r < pn) rr = Elem<TO>::to_f32(resp[o + r]);
                const float t = (v[r] + b[j][r]) + rr;
                v[r] = relu ? fmaxf(t, 0.0f) : (gelu ? gelu_act(t, g0, g1, g2, gstd) : t);
                if (rb && n + r < pn) best[j / 4].see(stored_value<TO>(v[r]));
              }
              if (nfull) {
                Elem<TO>::store4(outp + o, v);
              } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  if (n + r < pn) outp[o + r] = Elem<TO>::from_f32(v[r]);
              }
            }
          }
        }
      });
    }
    if (rb) row_max_store(best, lane, mbase + 16 * i, nbase);
  });
}

// fp8 GEMM: C^T accumulators (row m = mbase + 16 i + l16, column
// n = nbase + 16 j + 4 lg + r) times a_rows[m] * b_scale[n], in registers,
// before either epilogue.  Rows / columns past the edge get scale 0 (never
// stored).
template <int TM, int TN>
__device__ __forceinline__ void scale_acc(f32x4 (&acc)[TM][TN], int64_t mbase, int64_t nbase, int lane) {
  const KArg<Problem>& p = kernel_arg<Problem>();
  const int l16 = lane & 15, lg = lane >> 4;
  float sb[TN][4];
  static_for<TN>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    const int64_t n = nbase + 16 * j + 4 * lg;
    if (n + 4 <= p.n) {
      const float4 q = *reinterpret_cast<const float4*>(p.b_scale + n);
      sb[j][0] = q.x; sb[j][1] = q.y; sb[j][2] = q.z; sb[j][3] = q.w;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) sb[j][r] = n + r < p.n ? p.b_scale[n + r] : 0.0f;
    }
  });
  static_for<TM>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    const int64_t m = mbase + 16 * i + l16;
    const float sa = m < p.m ? p.a_rows[m] : 0.0f;
    static_for<TN>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = (acc[i][j][r] * sa) * sb[j][r];
    });
  });
}

// epilogue_direct_q for a wave tile that lies wholly inside the output (every
// row < m, every column < n), the case of all but the edge tiles: no bounds
// tests, and the output kind, activation and (int8 output of modes 2 / 3)
// rounding type fixed at compile time, so the per-element work is the
// arithmetic alone (the general form's per-element selects and bounds
// branches made the epilogue cost more VALU issue than a K = 768 main loop).
// KIND: 0 int32 accumulators (mode 0), 1 int8 codes (mode 1), 2 / 3 float
// output of mode 2 / 3, 4 / 5 int8 output of mode 2 / 3 quantized from the
// bf16-rounded epilogue value by the verified multiplier p.q_mul.  ACT: 0
// none, 1 ReLU, 2 GELU with run-time constants, 3 GELU with the standard
// ones (gelu_std).  Same values as epilogue_direct_q_impl, in fewer
// operations:
//   requantized y = saturate(rne(a * mult) + zy); mode 3 stores (y - zy) * sy,
//     which is rne(a * mult) clamped to [-128 - zy, 127 - zy], times sy (all
//     integers exact in fp32: one v_med3_f32 instead of add, clamp, subtract;
//     a NaN rne(.) gives the lower bound, as fmaxf then fminf do: v_med3_f32
//     returns min3 of its operands when one is NaN)
//   int8 codes are rne(.) + (zero + 128) through v_cvt_pk_u8_f32 (clamp to
//     [0, 255], NaN -> 0, byte insert), XOR 0x80 per byte
//   NBR (KIND 3, no bias, no residual, sy normal with 255 |sy| finite):
//     (y - zy) * sy + 0 + 0 as one fma with a +0 addend -- the zero addend
//     turns -0 into +0 as the additions do, and with |y - zy| >= 1 or 0 the
//     product never rounds to zero -- and every value is finite (the clamp
//     maps NaN and +-Inf to its bounds), so row maxima track no NaN.
template <typename TO, int TM, int TN, int KIND, int ACT, bool RB, bool NBR = false, typename Acc>
__device__ __forceinline__ void epilogue_q_interior(const Acc (&acc)[TM][TN], int64_t mbase, int64_t nbase, int lane,
                                                    TO* outp, const TO* resp, const float* bias) {
  // Each product and sum rounds on its own, as in the general form (no
  // multiply-add contraction of the dequantization with the bias).
#pragma clang fp contract(off)
  static_assert(!NBR || (KIND == 3 && ACT == 0), "NBR: mode-3 float output without activation");
  const KArg<Problem>& p = kernel_arg<Problem>();
  constexpr bool kReq = KIND == 1 || KIND == 3 || KIND == 5;
  constexpr bool kQuantOut = KIND >= 4;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t ldo = p.ldo;
  const float sa = p.a_scale, sy = p.y_scale, zy = static_cast<float>(p.y_zero);
  const float lo = -128.0f - zy, hi = 127.0f - zy, zb = zy + 128.0f;
  const float g0 = p.epi.imm[0], g1 = p.epi.imm[1], g2 = p.epi.imm[2];
  const float qmul = p.q_mul, qb = static_cast<float>(p.q_zero + 128);
  float mult[TN][4], b[TN][4];
  if constexpr (KIND != 0) {
    // Requantizing, each of the wave tile's 16 TN columns forms its
    // multiplier (sa * sb) / sy once -- column c on lane c % 64 -- and the
    // lanes that use it read it with ds_bpermute: one IEEE division per
    // column instead of one per column and row lane (the 16 row lanes of a
    // column group each needed all of theirs).
    static_assert(TN % 4 == 0, "whole 64-column groups");
    float own[TN / 4];
    if constexpr (kReq) {
#pragma unroll
      for (int t = 0; t < TN / 4; ++t) own[t] = (sa * p.b_scale[nbase + lane + 64 * t]) / sy;
    }
    static_for<TN>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      const int64_t n = nbase + 16 * j + 4 * lg;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        b[j][r] = bias ? bias[n + r] : 0.0f;
        if constexpr (kReq) {
          const int src = (16 * (j % 4) + 4 * lg + r) << 2;  // byte address of lane (column % 64)
          mult[j][r] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(own[j / 4])));
        } else {
          mult[j][r] = sa * p.b_scale[n + r];
        }
      }
    });
  }
  TO* base = outp + (mbase + l16) * ldo + nbase + 4 * lg;
  const TO* rbase = resp ? resp + (mbase + l16) * ldo + nbase + 4 * lg : nullptr;
  // 16-byte accesses where rows are 16-byte aligned: 16-bit outputs and
  // residuals (KIND 2 / 3 without GELU) by pairs of column tiles
  // (ct_pair_to_rows, rows_to_ct_pair), int8 outputs by groups of four
  // (ct_quad_to_rows); a lane row then covers 8 / 16 consecutive columns.
  constexpr bool kW16 = sizeof(TO) == 2 && TN % 2 == 0 && ACT <= 1 && (KIND == 2 || KIND == 3);
  constexpr bool kW8 = std::is_same<TO, int8_t>::value && TN % 4 == 0;
  bool wide = false;
  if constexpr (kW16 || kW8)
    wide = (ldo & (kW8 ? 15 : 7)) == 0 && (reinterpret_cast<uintptr_t>(outp) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(resp) & 15) == 0;
  constexpr int kWideCols = kW8 ? 16 : 8;
  TO* wbase = outp + (mbase + l16) * ldo + nbase + kWideCols * lg;
  const TO* wrbase = resp ? resp + (mbase + l16) * ldo + nbase + kWideCols * lg : nullptr;
  static_for<TM>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    TO* row = base + 16 * i * ldo;
    if constexpr (KIND == 0) {
      static_for<TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        *reinterpret_cast<int4*>(row + 16 * j) = int4{acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      });
    } else {
      RowMax best[TN / 4];
      if constexpr (RB) {
#pragma unroll
        for (int q = 0; q < TN / 4; ++q) best[q].start();
      }
      // Column tile j's four values v (float outputs) and int8 codes (the
      // return value: KIND 1, 4, 5), given its residual values res.
      auto tile = [&](auto jc, const float (&res)[4], float (&v)[4]) -> uint32_t {
        constexpr int j = decltype(jc)::value;
        uint32_t w = 0u;  // biased int8 codes
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float a = static_cast<float>(acc[i][j][r]);
          if constexpr (KIND == 1) {
            w = __builtin_amdgcn_cvt_pk_u8_f32(rintf(a * mult[j][r]) + zb, r, w);
          } else if constexpr (NBR) {
            v[r] = fmaf(__builtin_amdgcn_fmed3f(rintf(a * mult[j][r]), lo, hi), sy, 0.0f);
            if constexpr (RB) best[j / 4].v = fmaxf(best[j / 4].v, v[r]);
          } else {
            if constexpr (kReq) {
              v[r] = __builtin_amdgcn_fmed3f(rintf(a * mult[j][r]), lo, hi) * sy;
            } else {
              v[r] = a * mult[j][r];
            }
            const float t = kQuantOut ? v[r] + b[j][r] : (v[r] + b[j][r]) + res[r];
            v[r] = ACT == 1 ? fmaxf(t, 0.0f) : (ACT == 3 ? gelu_std(t) : (ACT == 2 ? gelu_erf(t, g0, g1, g2) : t));
            if constexpr (kQuantOut) w = __builtin_amdgcn_cvt_pk_u8_f32(rintf(bf16_round(v[r]) * qmul) + qb, r, w);
            if constexpr (RB) best[j / 4].see(stored_value<TO>(v[r]));
          }
        }
        return w ^ 0x80808080u;
      };
      bool done = false;
      if constexpr (kW16) {
        if (wide) {
          // the row block's residual, packed (all loads first), then a pair
          // of column tiles at a time
          uint4 rq[TN / 2];
#pragma unroll
          for (int q = 0; q < TN / 2; ++q)
            rq[q] = wrbase ? *reinterpret_cast<const uint4*>(wrbase + 16 * i * ldo + 32 * q) : uint4{0u, 0u, 0u, 0u};
          static_for<TN / 2>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            uint32_t d0[2], d1[2];
            rows_to_ct_pair(rq[q], d0, d1);
            float r0[4], r1[4], v0[4], v1[4];
            Elem<TO>::unpack2(d0[0], &r0[0]);
            Elem<TO>::unpack2(d0[1], &r0[2]);
            Elem<TO>::unpack2(d1[0], &r1[0]);
            Elem<TO>::unpack2(d1[1], &r1[2]);
            tile(std::integral_constant<int, 2 * q>{}, r0, v0);
            tile(std::integral_constant<int, 2 * q + 1>{}, r1, v1);
            const uint32_t p0[2] = {Elem<TO>::pack2(v0[0], v0[1]), Elem<TO>::pack2(v0[2], v0[3])};
            const uint32_t p1[2] = {Elem<TO>::pack2(v1[0], v1[1]), Elem<TO>::pack2(v1[2], v1[3])};
            *reinterpret_cast<uint4*>(wbase + 16 * i * ldo + 32 * q) = ct_pair_to_rows(p0, p1);
          });
          done = true;
        }
      }
      if constexpr (kW8) {
        if (wide) {
          static_for<TN / 4>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            const float z[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            float v[4];
            const uint32_t w4[4] = {tile(std::integral_constant<int, 4 * g>{}, z, v),
                                    tile(std::integral_constant<int, 4 * g + 1>{}, z, v),
                                    tile(std::integral_constant<int, 4 * g + 2>{}, z, v),
                                    tile(std::integral_constant<int, 4 * g + 3>{}, z, v)};
            *reinterpret_cast<uint4*>(wbase + 16 * i * ldo + 64 * g) = ct_quad_to_rows(w4);
          });
          done = true;
        }
      }
      if (!done) {
        float res[TN][4];
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) res[j][r] = 0.0f;
        if constexpr (KIND == 2 || KIND == 3) {
          if (rbase) {
            static_for<TN>([&](auto jc) {
              constexpr int j = decltype(jc)::value;
              Elem<TO>::load4(rbase + 16 * i * ldo + 16 * j, res[j]);
            });
          }
        }
        static_for<TN>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          float v[4];
          const uint32_t w = tile(jc, res[j], v);
          if constexpr (std::is_same<TO, int8_t>::value) {
            *reinterpret_cast<uint32_t*>(row + 16 * j) = w;
          } else {
            Elem<TO>::store4(row + 16 * j, v);
          }
        });
      }
      if constexpr (RB) row_max_store(best, lane, mbase + 16 * i, nbase);
    }
  });
}

template <typename TO, int TM, int TN, bool GELU = false, typename Acc>
__device__ __forceinline__ void epilogue_direct_q(const Acc (&acc)[TM][TN], int64_t mbase, int64_t nbase, int lane,
                                                  TO* outp, const TO* resp, const float* bias, int act) {
  const KArg<Problem>& p = kernel_arg<Problem>();
  // Interior wave tile: the specialized form (int8 outputs of modes 2 / 3
  // only when rounded through bf16, the W8A8 activation type, with a
  // verified multiplier; GELU only with the standard constants).
  const bool gstd = GELU && act == 2 && gelu_std_ok(p.epi.imm[0], p.epi.imm[1], p.epi.imm[2]);
  if (mbase + 16 * TM <= p.m && nbase + 16 * TN <= p.n && (act <= 1 || gstd)) {
    const int mode = p.qmode;
    if constexpr (std::is_same<TO, int32_t>::value) {
      epilogue_q_interior<TO, TM, TN, 0, 0, false>(acc, mbase, nbase, lane, outp, resp, bias);
      return;
    } else if constexpr (std::is_same<TO, int8_t>::value) {
      if (mode == 1) {
        epilogue_q_interior<TO, TM, TN, 1, 0, false>(acc, mbase, nbase, lane, outp, resp, bias);
        return;
      }
      if (p.act_dtype == C3H_BF16 && p.q_mul != 0.0f) {
        const bool m3 = mode == 3;
        if (act == 0) {
          if (m3) epilogue_q_interior<TO, TM, TN, 5, 0, false>(acc, mbase, nbase, lane, outp, resp, bias);
          else epilogue_q_interior<TO, TM, TN, 4, 0, false>(acc, mbase, nbase, lane, outp, resp, bias);
        } else if (act == 1) {
          if (m3) epilogue_q_interior<TO, TM, TN, 5, 1, false>(acc, mbase, nbase, lane, outp, resp, bias);
          else epilogue_q_interior<TO, TM, TN, 4, 1, false>(acc, mbase, nbase, lane, outp, resp, bias);
        } else if constexpr (GELU) {
          if (m3) epilogue_q_interior<TO, TM, TN, 5, 3, false>(acc, mbase, nbase, lane, outp, resp, bias);
          else epilogue_q_interior<TO, TM, TN, 4, 3, false>(acc, mbase, nbase, lane, outp, resp, bias);
        }
        return;
      }
    } else {
      const bool m3 = mode == 3;
      if (p.epi.row_max != nullptr) {  // host: only with act <= 1
        const float asy = fabsf(p.y_scale);
        if (act == 0 && m3 && !bias && !resp && asy >= 0x1p-126f && asy <= 0x1p119f) {
          epilogue_q_interior<TO, TM, TN, 3, 0, true, true>(acc, mbase, nbase, lane, outp, resp, bias);
        } else if (act == 0) {
          if (m3) epilogue_q_interior<TO, TM, TN, 3, 0, true>(acc, mbase, nbase, lane, outp, resp, bias);
          else epilogue_q_interior<TO, TM, TN, 2, 0, true>(acc, mbase, nbase, lane, outp, resp, bias);
        } else {
          if (m3) epilogue_q_interior<TO, TM, TN, 3, 1, true>(acc, mbase, nbase, lane, outp, resp, bias);
          else epilogue_q_interior<TO, TM, TN, 2, 1, true>(acc, mbase, nbase, lane, outp, resp, bias);
        }
      } else if (act == 0) {
        if (m3) epilogue_q_interior<TO, TM, TN, 3, 0, false>(acc, mbase, nbase, lane, outp, resp, bias);
        else epilogue_q_interior<TO, TM, TN, 2, 0, false>(acc, mbase, nbase, lane, outp, resp, bias);
      } else if (act == 1) {
        if (m3) epilogue_q_interior<TO, TM, TN, 3, 1, false>(acc, mbase, nbase, lane, outp, resp, bias);
        else epilogue_q_interior<TO, TM, TN, 2, 1, false>(acc, mbase, nbase, lane, outp, resp, bias);
      } else if constexpr (GELU) {
        if (m3) epilogue_q_interior<TO, TM, TN, 3, 3, false>(acc, mbase, nbase, lane, outp, resp, bias);
        else epilogue_q_interior<TO, TM, TN, 2, 3, false>(acc, mbase, nbase, lane, outp, resp, bias);
      }
      return;
    }
  }
  if (GELU && act == 2) epilogue_direct_q_impl<TO, TM, TN, true>(acc, mbase, nbase, lane, outp, resp, bias, act);
  else epilogue_direct_q_impl<TO, TM, TN, false>(acc, mbase, nbase, lane, outp, resp, bias, act);
}

// Whether epilogue_direct_q applies: int32 / int8 outputs need only aligned
// row-major stores; dequantized ones also need the common float epilogue.
__device__ __forceinline__ bool epilogue_q_direct_ok(const KArg<Problem>& p, bool vec4);

// Whether epilogue_direct applies (uniform): see its comment.
__device__ __forceinline__ bool epilogue_is_simple(const KArg<Problem>& p, bool vec4, bool gelu_ok = false) {
  const int bm = p.epi.bias_mode;
  return vec4 && !p.out_nchw && p.epi.alpha == 1.0f && p.epi.beta == 1.0f && (bm == 0 || bm == 2) &&
         p.epi.act <= (gelu_ok ? 2 : 1) && p.epi.n_inst == 0 &&
         (bm == 0 || (reinterpret_cast<uintptr_t>(p.epi.bias) & 15) == 0);
}
__device__ __forceinline__ bool epilogue_q_direct_ok(const KArg<Problem>& p, bool vec4) {
  return p.qmode <= 1 ? (vec4 && !p.out_nchw) : epilogue_is_simple(p, vec4);
}

// BUF: operands read with buffer loads at 32-bit byte offsets (A and B below
// 2^31 bytes, no batch): row bases are precomputed once, out-of-range lanes
// use an offset past num_records and read zeros, so a K step costs a few
// VALU per load instead of 64-bit address math and branches.
// Eight fp16 weights of one MXFP4 block: `codes` holds E2M1 elements 2j
// (low nibble) and 2j+1 of byte j, `e8` the block's biased exponent.  The
// scale is 2^(e8 - 127) as an fp32 (0xFF: NaN); v_cvt_scalef32_pk_f16_fp4
// decodes two elements of one byte and multiplies by it.
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 mxfp4_to_f16x8(uint32_t codes, uint32_t e8) {
  const float sc = __uint_as_float((e8 << 23) | (e8 == 0xFFu ? 0x400000u : 0u));
  const f16x2_t h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(codes, sc, 0);
  const f16x2_t h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(codes, sc, 1);
  const f16x2_t h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(codes, sc, 2);
  const f16x2_t h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(codes, sc, 3);
  return uint4{__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1), __builtin_bit_cast(uint32_t, h2),
               __builtin_bit_cast(uint32_t, h3)};
}

// BQ: B is MXFP4 (W4A16, c3h_gemm_w4a16): each thread loads the 4 code bytes
// and the exponent byte behind its 8-element K chunk and widens them to fp16
// when it stores the tile to LDS, so the MFMA loop is the fp16 one.
template <typename Mma, typename TO, int BM, int BN, int WM, int WN, int AM, bool BUF = false, bool BQ = false>
__global__ void __launch_bounds__(kThreads) mfma_gemm_kernel(Problem p) {
  constexpr bool DIRECT_GELU = false;  // GELU epilogues take the staged path here
  constexpr int ES = Mma::ES;
  constexpr int VE = 16 / ES;        // elements per 16-byte vector
  constexpr int BK = 128 / ES;       // elements per 128-byte tile row
  constexpr int RB = 128;            // LDS row bytes
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int RSTEP = kThreads / 8;  // rows between a thread's vectors
  constexpr int A_V = BM / RSTEP, B_V = BN / RSTEP;
  static_assert(WM * WN == kThreads / 64, "wave grid");
  static_assert(A_V >= 1 && B_V >= 1 && BM % RSTEP == 0 && BN % RSTEP == 0, "tile too small");
  static_assert(AM == kDenseK || ES == 2, "conv modes are 16-bit");
  static_assert(!BQ || (std::is_same<Mma, MmaF16>::value && AM == kDenseK && BUF), "W4A16: fp16, dense, buffer loads");
  constexpr int kTileBytes = 2 * (BM + BN) * RB;
  constexpr int kStageBytes = (kThreads / 64) * WTM * (WTN + 4) * 4;  // whole wave tiles, 32-bit
  __shared__ __attribute__((aligned(16))) uint8_t smem[kTileBytes > kStageBytes ? kTileBytes : kStageBytes];
  uint8_t (*As)[BM][RB] = reinterpret_cast<uint8_t (*)[BM][RB]>(smem);
  uint8_t (*Bs)[BN][RB] = reinterpret_cast<uint8_t (*)[BN][RB]>(smem + 2 * BM * RB);
  typedef typename Mma::vec vec;
  typedef typename Mma::acc_t acc_t;

  int tm, tn;
  tile_coords_grouped(p, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const int64_t bz = blockIdx.z;
  const uint8_t* A = static_cast<const uint8_t*>(p.a) + bz * p.stride_a * ES;
  const uint8_t* B = static_cast<const uint8_t*>(p.b) + bz * p.stride_b * ES;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;
  const int trow = tid >> 3;         // first tile row of this thread
  const int kchunk = tid & 7;        // 16-byte K chunk of all of this thread's vectors
  const int kc = kchunk * VE;        // ... as an element column

  // Two register sets: the loads of tile kt + 2 are issued while tile kt is
  // multiplied and tile kt + 1 is still in flight.  (BQ: codes, exponent.)
  typedef std::conditional_t<BQ, uint2, uint4> breg;
  uint4 ra0[A_V], ra1[A_V];
  breg rb0[B_V], rb1[B_V];

  // Per-row conv state (conv modes): pixel base offset, top-left input coords.
  int64_t rbase[AM == kDenseK ? 1 : A_V];
  int rhi[AM == kDenseK ? 1 : A_V], rwi[AM == kDenseK ? 1 : A_V];
  ConvRow crow[AM == kConv ? A_V : 1];
  static_assert(!BUF || AM == kDenseK || AM == kConvTap, "buffer loads: dense or tap-uniform conv");
  __amdgpu_buffer_rsrc_t rs_a, rs_b, rs_s;
  int32_t a_off[BUF ? A_V : 1];   // dense: row byte offset (-1: out of range); tap: pixel byte offset
  int32_t b_off[BUF ? B_V : 1];
  int32_t s_off[BQ ? B_V : 1];    // BQ: exponent row byte offset
  if constexpr (BUF) {
    rs_a = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.a), 0, static_cast<int>(p.a_bytes), 0x00020000);
    rs_b = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.b), 0, static_cast<int>(p.b_bytes), 0x00020000);
    if constexpr (BQ)
      rs_s = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.b_blk), 0, static_cast<int>(p.bs_bytes),
                                               0x00020000);
#pragma unroll
    for (int i = 0; i < B_V; ++i) {
      const int64_t n = n0 + trow + RSTEP * i;
      b_off[i] = n < p.n ? static_cast<int32_t>(n * p.ldb * (BQ ? 1 : ES)) : -1;
      if constexpr (BQ) s_off[i] = n < p.n ? static_cast<int32_t>(n * p.ldbs) : -1;
    }
    if (AM == kDenseK) {
#pragma unroll
      for (int i = 0; i < A_V; ++i) {
        const int64_t m = m0 + trow + RSTEP * i;
        a_off[i] = m < p.m ? static_cast<int32_t>(m * p.lda * ES) : -1;
      }
    }
  }
  if (AM == kConvTap || AM == kConvStem) {
#pragma unroll
    for (int i = 0; i < A_V; ++i) {
      const ConvRow r = conv_row(p, m0 + trow + RSTEP * i);
      rbase[i] = r.base;
      rhi[i] = r.valid ? r.hi0 : -(1 << 28);  // invalid rows fail every bounds check
      rwi[i] = r.wi0;
      if constexpr (BUF)
        a_off[i] = static_cast<int32_t>(
            (r.base + (static_cast<int64_t>(r.hi0) * p.cw + r.wi0) * p.c_stride) * ES);
    }
  } else if (AM == kConv) {
#pragma unroll
    for (int i = 0; i < A_V; ++i) crow[i] = conv_row(p, m0 + trow + RSTEP * i);
  }
  // kConvTap: the next tile's filter tap and channel base.
  int t_kh = 0, t_kw = 0, t_c0 = 0;

  // `live` is false for the tiles past the end that the fixed-depth prefetch
  // still issues: their loads read zeros, so every issue() is the same number
  // of load instructions and the compiler's vmcnt waits stay exact.
  auto load_a = [&](int64_t k0, uint4 (&ra)[A_V], bool live) {
    if constexpr (BUF) {
      if (AM == kDenseK) {
        const bool kok = live && k0 + kc < p.k;
        const int32_t koff = static_cast<int32_t>((k0 + kc) * ES);
#pragma unroll
        for (int i = 0; i < A_V; ++i) {
          const uint32_t voff = (kok && a_off[i] >= 0) ? static_cast<uint32_t>(a_off[i] + koff) : kOobOffset;
          ra[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs_a, voff, 0, 0));
        }
      } else {
        const int dh = t_kh * p.dh, dw = t_kw * p.dw;
        const int32_t tap = static_cast<int32_t>(((dh * p.cw + dw) * p.c_stride + t_c0 + kc) * ES);
#pragma unroll
        for (int i = 0; i < A_V; ++i) {
          const bool ok = live && static_cast<unsigned>(rhi[i] + dh) < static_cast<unsigned>(p.ch) &&
                          static_cast<unsigned>(rwi[i] + dw) < static_cast<unsigned>(p.cw);
          const uint32_t voff = ok ? static_cast<uint32_t>(a_off[i] + tap) : kOobOffset;
          ra[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs_a, voff, 0, 0));
        }
      }
      return;
    }
    if (AM == kDenseK) {
      const int64_t k = k0 + kc;
#pragma unroll
      for (int i = 0; i < A_V; ++i) {
        const int64_t m = m0 + trow + RSTEP * i;
        uint4 v = {0u, 0u, 0u, 0u};
        if (m < p.m && k < p.k) v = *reinterpret_cast<const uint4*>(A + (m * p.lda + k) * ES);
        ra[i] = v;
      }
    } else if (AM == kConvTap) {
      const int dh = t_kh * p.dh, dw = t_kw * p.dw;
      const int64_t tap_off = (static_cast<int64_t>(dh) * p.cw + dw) * p.c_stride + t_c0 + kc;
#pragma unroll
      for (int i = 0; i < A_V; ++i) {
        const int hi = rhi[i] + dh, wi = rwi[i] + dw;
        uint4 v = {0u, 0u, 0u, 0u};
        if (live && static_cast<unsigned>(hi) < static_cast<unsigned>(p.ch) &&
            static_cast<unsigned>(wi) < static_cast<unsigned>(p.cw))
          v = *reinterpret_cast<const uint4*>(
              A + (rbase[i] + (static_cast<int64_t>(rhi[i]) * p.cw + rwi[i]) * p.c_stride + tap_off) * ES);
        ra[i] = v;
      }
    } else if (AM == kConvStem) {
      // K order (kh, kw_pack = 8, c = 4): vector kc covers taps kw0, kw0 + 1.
      const int64_t k = k0 + kc;
      const int tap = static_cast<int>(k >> 2);
      const int khi = tap >> 3, kw0 = tap & 7;
#pragma unroll
      for (int i = 0; i < A_V; ++i) {
        uint2 lo = {0u, 0u}, hi2 = {0u, 0u};
        if (k < p.k) {
          const int hi = rhi[i] + khi * p.dh;
          if (static_cast<unsigned>(hi) < static_cast<unsigned>(p.ch)) {
            const int wa = rwi[i] + kw0 * p.dw, wb = wa + p.dw;
            const int64_t rowoff = rbase[i] + static_cast<int64_t>(hi) * p.cw * 4;
            if (kw0 < p.kw && static_cast<unsigned>(wa) < static_cast<unsigned>(p.cw))
              lo = *reinterpret_cast<const uint2*>(A + (rowoff + static_cast<int64_t>(wa) * 4) * ES);
            if (kw0 + 1 < p.kw && static_cast<unsigned>(wb) < static_cast<unsigned>(p.cw))
              hi2 = *reinterpret_cast<const uint2*>(A + (rowoff + static_cast<int64_t>(wb) * 4) * ES);
          }
        }
        ra[i] = uint4{lo.x, lo.y, hi2.x, hi2.y};
      }
    } else {
      const int64_t k = k0 + kc;
#pragma unroll
      for (int i = 0; i < A_V; ++i) {
        const int64_t off = conv_k_offset(p, crow[i], k);
        uint4 v = {0u, 0u, 0u, 0u};
        if (off >= 0) v = *reinterpret_cast<const uint4*>(A + off * ES);
        ra[i] = v;
      }
    }
  };
  auto advance_tap = [&]() {
    if (AM == kConvTap) {
      t_c0 += BK;
      if (t_c0 >= p.c_pack) {
        t_c0 = 0;
        if (++t_kw >= p.kw) {
          t_kw = 0;
          ++t_kh;
        }
      }
    }
  };
  auto load_b = [&](int64_t k0, breg (&rb)[B_V], bool live) {
    const int64_t k = k0 + kc;
    if constexpr (BQ) {
      // Out-of-range chunks read code bytes 0 (weight 0) and exponent 0.
      const bool kok = live && k < p.k;
      const int32_t koff = static_cast<int32_t>(k >> 1), soff = static_cast<int32_t>(k >> 5);
#pragma unroll
      for (int i = 0; i < B_V; ++i) {
        const bool ok = kok && b_off[i] >= 0;
        const uint32_t voff = ok ? static_cast<uint32_t>(b_off[i] + koff) : kOobOffset;
        const uint32_t eoff = ok ? static_cast<uint32_t>(s_off[i] + soff) : kOobOffset;
        rb[i].x = __builtin_amdgcn_raw_buffer_load_b32(rs_b, voff, 0, 0);
        rb[i].y = __builtin_amdgcn_raw_buffer_load_b8(rs_s, eoff, 0, 0);
      }
    } else if constexpr (BUF) {
      const bool kok = live && k < p.k;
      const int32_t koff = static_cast<int32_t>(k * ES);
#pragma unroll
      for (int i = 0; i < B_V; ++i) {
        const uint32_t voff = (kok && b_off[i] >= 0) ? static_cast<uint32_t>(b_off[i] + koff) : kOobOffset;
        rb[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs_b, voff, 0, 0));
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_V; ++i) {
        const int64_t n = n0 + trow + RSTEP * i;
        uint4 v = {0u, 0u, 0u, 0u};
        if (n < p.n && k < p.k) v = *reinterpret_cast<const uint4*>(B + (n * p.ldb + k) * ES);
        rb[i] = v;
      }
    }
  };
  // Byte offset of 16-byte chunk c of row r (XOR swizzle).
  auto swz = [](int r, int c) { return (c ^ (r & 7)) << 4; };
  auto store_tiles = [&](int buf, const uint4 (&ra)[A_V], const breg (&rb)[B_V]) {
#pragma unroll
    for (int i = 0; i < A_V; ++i) {
      const int r = trow + RSTEP * i;
      *reinterpret_cast<uint4*>(&As[buf][r][swz(r, kchunk)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_V; ++i) {
      const int r = trow + RSTEP * i;
      if constexpr (BQ) *reinterpret_cast<uint4*>(&Bs[buf][r][swz(r, kchunk)]) = mxfp4_to_f16x8(rb[i].x, rb[i].y);
      else *reinterpret_cast<uint4*>(&Bs[buf][r][swz(r, kchunk)]) = rb[i];
    }
  };

  acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{0, 0, 0, 0};

  const int64_t ktiles = ceil_div(p.k, BK);
  const int lrow = lane & 15, lchunk = lane >> 4;
  auto compute = [&](int cur) {
#pragma unroll
    for (int ks = 0; ks < 8; ks += Mma::kStep) {  // MFMA K steps of 16 * kStep bytes
      vec av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WTM + i * 16 + lrow;
        av[i] = read_operand<Mma>(&As[cur][r][0], r, ks, lchunk);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * WTN + j * 16 + lrow;
        bv[j] = read_operand<Mma>(&Bs[cur][r][0], r, ks, lchunk);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          acc[i][j] = Mma::mma(bv[j], av[i], acc[i][j]);  // C^T: see epilogue_direct
        }
    }
  };
  // LDS barrier that leaves global loads in flight: this wave's LDS stores
  // are complete (lgkmcnt 0); __syncthreads would also wait for vmcnt(0).
  auto lds_barrier = [&]() {
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  auto issue = [&](int64_t kt, uint4 (&ra)[A_V], breg (&rb)[B_V]) {
    const bool live = kt < ktiles;
    load_a(kt * BK, ra, live);
    load_b(kt * BK, rb, live);
    advance_tap();
  };

  issue(0, ra0, rb0);
  issue(1, ra1, rb1);
  store_tiles(0, ra0, rb0);
  lds_barrier();
  int64_t kt = 0;
  for (; kt + 2 <= ktiles; kt += 2) {
    // LDS buffer 0 holds tile kt; ra1/rb1 carry tile kt + 1.
    issue(kt + 2, ra0, rb0);
    compute(0);
    store_tiles(1, ra1, rb1);
    lds_barrier();
    // LDS buffer 1 holds tile kt + 1; ra0/rb0 carry tile kt + 2.
    issue(kt + 3, ra1, rb1);
    compute(1);
    if (kt + 2 < ktiles) {
      store_tiles(0, ra0, rb0);
      lds_barrier();
    }
  }
  if (kt < ktiles) compute(0);  // odd tile count: the last tile sits in buffer 0
  if constexpr (Mma::kScaled) scale_acc<TM, TN>(acc, m0 + wm * WTM, n0 + wn * WTN, lane);

  // Epilogue: a lane holds (m = 4*(lane/16)+r, n = lane%16) of each 16x16
  // tile.  The whole wave tile is staged in LDS (accumulators only ever
  // indexed by unrolled constants), then stored 16 rows at a time with 8
  // columns per lane.
  TO* outp = static_cast<TO*>(p.out) + bz * p.stride_out;
  const TO* resp = p.epi.residual ? static_cast<const TO*>(p.epi.residual) + bz * p.stride_res : nullptr;
  const int64_t bias_off = bz * p.stride_bias;
  {
    constexpr uintptr_t kA = 4 * sizeof(TO) - 1;
    const bool vec4 = (p.ldo % 4 == 0) && (p.stride_out % 4 == 0) && (p.stride_res % 4 == 0) &&
                      (p.stride_bias % 4 == 0) && ((reinterpret_cast<uintptr_t>(outp) & kA) == 0) &&
                      ((reinterpret_cast<uintptr_t>(resp) & kA) == 0);
    if constexpr (Mma::kInt) {
      if (bz == 0 && epilogue_q_direct_ok(kernel_arg<Problem>(), vec4)) {
        const float* bias = p.epi.bias_mode == 2 ? static_cast<const float*>(p.epi.bias) : nullptr;
        epilogue_direct_q<TO, TM, TN, DIRECT_GELU>(acc, m0 + wm * WTM, n0 + wn * WTN, lane, outp, resp, bias, p.epi.act);
        return;
      }
    } else if (epilogue_is_simple(kernel_arg<Problem>(), vec4)) {
      const float* bias = p.epi.bias_mode == 2 ? static_cast<const float*>(p.epi.bias) + bias_off : nullptr;
      epilogue_direct<TO, TM, TN, DIRECT_GELU>(acc, m0 + wm * WTM, n0 + wn * WTN, lane, outp, resp, bias, p.epi.act);
      return;
    }
  }
  const bool vec_ok = !p.out_nchw && (p.ldo % 8 == 0) && (p.stride_out % 8 == 0) && (p.stride_res % 8 == 0) &&
                      ((reinterpret_cast<uintptr_t>(p.out) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(p.epi.residual) & 15) == 0);
  __syncthreads();
  float* stage = reinterpret_cast<float*>(smem) + wave * WTM * (WTN + 4);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float* dst = &stage[(i * 16 + lrow) * (WTN + 4) + j * 16 + (lane >> 4) * 4 + r];  // C^T accumulators
        if constexpr (Mma::kInt) *reinterpret_cast<int*>(dst) = acc[i][j][r];
        else *dst = acc[i][j][r];
      }
  wave_sync_lds();
#pragma nounroll
  for (int i = 0; i < TM; ++i) {
    const int64_t mrow0 = m0 + wm * WTM + i * 16, ncol0 = n0 + wn * WTN;
    const float* strip = stage + i * 16 * (WTN + 4);
    if constexpr (Mma::kInt) {
      store_strip_q<TO, WTN>(strip, lane, mrow0, ncol0, outp, resp, vec_ok);
    } else {
      if (p.out_nchw) store_strip<TO, WTN>(p, strip, lane, mrow0, ncol0, outp, resp, bias_off);
      else store_strip_vec<TO, WTN>(strip, lane, mrow0, ncol0, outp, resp, bias_off, vec_ok);
    }
  }
}

// =====================================================================
// Pipelined variant: operand tiles go straight from global memory to LDS
// (buffer_load_dwordx4 ... lds) through S stages, so S-1 tiles are in flight
// while one is multiplied, without staging registers.  Lane i of a DMA load
// writes LDS bytes [16 i, 16 i + 16) from the wave's base (M0); a wave load
// covers 8 tile rows, and each lane fetches the logical K chunk that the XOR
// swizzle places at its slot.  Out-of-range lanes (M/N/K tails, conv
// padding) get a byte offset beyond the buffer's num_records and so write
// zeros.  One barrier per K tile: after it, every wave has finished the
// previous tile, whose buffer then receives tile kt + S - 1.
//
// Requirements (checked on the host): A and B each below 2^31 bytes; A mode
// kDenseK or kConvTap.
// =====================================================================
typedef __attribute__((address_space(3))) void* lds_void_ptr;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// NW waves per block.  NW = 8 is the large-tile form (256 x 256, wave tiles
// 64 x 128, one block per CU): half the operand bytes per flop of 128 x 128,
// direct epilogues only (its LDS cannot also hold a staged epilogue).
// Raised wave priority around the MFMA sections of the DMA kernel.
#ifndef C3H_MFMA_PRIO
#define C3H_MFMA_PRIO 1
#endif
constexpr bool kPrio = C3H_MFMA_PRIO != 0;

// s_waitcnt with only the LDS/scalar-memory counter constrained to 0.
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x3 << 14)); }

// vmcnt(n * per) for a runtime n in [0, 3] (the wait needs an immediate).
template <int PER>
__device__ __forceinline__ void wait_vmcnt_groups(int64_t n) {
  if (n >= 3) wait_vmcnt<3 * PER>();
  else if (n == 2) wait_vmcnt<2 * PER>();
  else if (n == 1) wait_vmcnt<PER>();
  else wait_vmcnt<0>();
}

// RP (register pipelining): the operand fragments of K tile kt + 1 are read
// from LDS into a second register set while the MFMAs of tile kt run from
// the first, and all S stages hold tiles in flight (DMA lead S - 1 tiles).
// The K order and every accumulation are those of the RP = false kernel, so
// the two are bit-identical.
//
// PP (ping-pong, eight waves, two stages): waves 0-3 (group A, one per SIMD)
// and 4-7 (group B, one per SIMD) alternate between a memory phase (issue
// this wave's DMA share of the next K tile, read its operand fragments of the
// current one) and an MFMA phase, offset by one workgroup barrier, so on
// every SIMD one wave multiplies while the other loads.  Same K order and
// accumulation as the other forms: bit-identical results.
template <typename Mma, typename TO, int BM, int BN, int WM, int WN, int AM, int S, int NW = 4, bool RP = false,
          bool PP = false>
__global__ void __launch_bounds__(NW * 64) mfma_gemm_dma_kernel(Problem p) {
  constexpr bool DIRECT = NW > 4;
  // The 160-row tile has no staged epilogue: its LDS stage would not fit two
  // blocks per CU, and the host takes it only for epilogues epilogue_direct
  // computes (tile160_wins).
  constexpr bool STAGED = !DIRECT && BM != 160;
  // GELU in registers (epilogue_direct) for 16-bit outputs as well: with the
  // branch-free erf it beats the staged epilogue.
  constexpr bool DIRECT_GELU = DIRECT || !Mma::kInt;
  constexpr int ES = Mma::ES;
  constexpr int VE = 16 / ES;
  constexpr int BK = 128 / ES;
  constexpr int RB = 128;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int GROUPS = (BM + BN) / 8;   // 8-row wave loads per stage
  constexpr int LPW = GROUPS / NW;        // wave loads per wave per stage
  constexpr int STAGE = (BM + BN) * RB;
  static_assert(WM * WN == NW && GROUPS % NW == 0 && BM % 8 == 0, "shape");
  static_assert(AM == kDenseK || AM == kConvTap, "dma kernel: dense or tap-uniform conv only");
  static_assert(S >= 2 && S <= 4 && LPW * (S - 2) < 64, "stages");
  constexpr int kStageBytes = STAGED ? NW * WTM * (WTN + 4) * 4 : 0;
  constexpr int kSmem = S * STAGE > kStageBytes ? S * STAGE : kStageBytes;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmem];
  typedef typename Mma::vec vec;
  typedef typename Mma::acc_t acc_t;

  int tm, tn;
  tile_coords_grouped(p, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  // wave index via readfirstlane: provably uniform, so each DMA's LDS base
  // (M0) is a scalar and needs no per-lane waterfall loop
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;

  const __amdgpu_buffer_rsrc_t rs_a = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rs_b = make_rsrc(p.b, p.b_bytes);
  const int lchunk_ld = (lane & 7) ^ (lane >> 3);  // logical K chunk this lane fetches
  const int kc = lchunk_ld * VE;

  // Per load slot j (group g = wave + NW j): the byte offset of this lane's
  // chunk at K tile 0 (conv: at tap (0, 0), which may lie in the padding, so
  // it can be negative), or -1 for a row past M / N; conv rows also keep
  // their top-left input coordinates (rows past M get hi0 far out of range,
  // so every tap's bounds check fails).  A and B byte extents are below 2^31
  // (dma_eligible), so 32-bit offsets cover them.  Slots j < A_SLOTS hold A
  // rows for every wave (BM / 8 is a multiple of NW), a compile-time split.
  constexpr int A_SLOTS = BM / 8 / NW;
  static_assert((BM / 8) % NW == 0, "A/B slot split");
  int32_t slot_off[LPW];
  int slot_hi[LPW], slot_wi[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int g = wave + NW * j;
    const int r = g * 8 + (lane >> 3);
    slot_hi[j] = 0;
    slot_wi[j] = 0;
    if (j < A_SLOTS) {
      const int64_t m = m0 + r;
      if (AM == kConvTap) {
        const ConvRow cr = conv_row(p, m);
        slot_off[j] = static_cast<int32_t>(
            (cr.base + (static_cast<int64_t>(cr.hi0) * p.cw + cr.wi0) * p.c_stride + kc) * ES);
        slot_hi[j] = cr.valid ? cr.hi0 : -0x40000000;
        slot_wi[j] = cr.wi0;
      } else {
        slot_off[j] = m < p.m ? static_cast<int32_t>((m * p.lda + kc) * ES) : -1;
      }
    } else {
      const int64_t n = n0 + (r - BM);
      slot_off[j] = n < p.n ? static_cast<int32_t>((n * p.ldb + kc) * ES) : -1;
    }
  }
  int t_kh = 0, t_kw = 0, t_c0 = 0;  // kConvTap: tap of the next tile to issue

  auto issue = [&](int64_t kt, int buf) {
    const bool k_ok = kt * BK + kc < p.k;
    const int32_t k_bytes = static_cast<int32_t>(kt * BK * ES);  // dense operands: uniform
    const int dh = t_kh * p.dh, dw = t_kw * p.dw;
    // conv: the tap's uniform byte offset from tap (0, 0)
    const int32_t tap_bytes = ((dh * p.cw + dw) * p.c_stride + t_c0) * ES;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int g = wave + NW * j;
      uint32_t voff = kOobOffset;
      if (j < A_SLOTS) {
        if (AM == kConvTap) {
          const int hi = slot_hi[j] + dh, wi = slot_wi[j] + dw;
          if (static_cast<unsigned>(hi) < static_cast<unsigned>(p.ch) &&
              static_cast<unsigned>(wi) < static_cast<unsigned>(p.cw))
            voff = static_cast<uint32_t>(slot_off[j] + tap_bytes);
        } else if (slot_off[j] >= 0 && k_ok) {
          voff = static_cast<uint32_t>(slot_off[j] + k_bytes);
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_a, (lds_void_ptr)(smem + buf * STAGE + g * 1024), 16, voff, 0,
                                                 0, 0);
      } else {
        if (slot_off[j] >= 0 && k_ok) voff = static_cast<uint32_t>(slot_off[j] + k_bytes);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_b, (lds_void_ptr)(smem + buf * STAGE + g * 1024), 16, voff, 0,
                                                 0, 0);
      }
    }
    if (AM == kConvTap) {
      t_c0 += BK;
      if (t_c0 >= p.c_pack) {
        t_c0 = 0;
        if (++t_kw >= p.kw) {
          t_kw = 0;
          ++t_kh;
        }
      }
    }
  };

  acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{0, 0, 0, 0};

  const int64_t ktiles = ceil_div(p.k, BK);
  const int lrow = lane & 15, lchunk = lane >> 4;
  if constexpr (PP) {
    static_assert(NW == 8 && S == 2 && !RP, "ping-pong: eight waves, two stages");
    // Barrier pairing.  A executes P, then (X_t, Y_t) per K tile t; B executes
    // P, E, then (X_t, Y_t) without the last Y.  So A's MFMA phase t (between
    // X_t and Y_t) runs beside B's memory phase t, and A's memory phase t + 1
    // beside B's MFMA phase t.  Tile t + 1 is issued in both groups' memory
    // phase t and complete before A's Y_t / B's X_t (the same barrier), after
    // which A reads it; its stage last held tile t - 1, whose reads ended
    // before the barrier that opens each group's memory phase t.
    const bool grp_b = wave >= 4;  // wave-uniform (readfirstlane): scalar branches
    auto barrier = [] {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    issue(0, 0);
    wait_vmcnt<0>();
    barrier();          // P: tile 0 in LDS
    if (grp_b) barrier();  // E: B runs one phase behind A
    constexpr int KS = 8 / Mma::kStep;
    for (int64_t kt = 0; kt < ktiles; ++kt) {
      // memory phase: this wave's share of tile kt + 1, then tile kt's fragments
      if (kt + 1 < ktiles) issue(kt + 1, static_cast<int>((kt + 1) & 1));
      const uint8_t* As = smem + (kt & 1) * STAGE;
      const uint8_t* Bs = As + BM * RB;
      vec av[KS][TM], bv[KS][TN];
#pragma unroll
      for (int q = 0; q < KS; ++q) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int r = wm * WTM + i * 16 + lrow;
          av[q][i] = read_operand<Mma>(As + r * RB, r, q * Mma::kStep, lchunk);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int r = wn * WTN + j * 16 + lrow;
          bv[q][j] = read_operand<Mma>(Bs + r * RB, r, q * Mma::kStep, lchunk);
        }
      }
      // fragments in registers (no read of this stage outlives the barrier);
      // B's share of tile kt + 1 landed before the barrier A reads it after
      wait_lgkmcnt0();
      if (grp_b) wait_vmcnt<0>();
      __builtin_amdgcn_sched_barrier(0);
      barrier();  // X_kt
      if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int q = 0; q < KS; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = Mma::mma(bv[q][j], av[q][i], acc[i][j]);
      if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      if (!grp_b) wait_vmcnt<0>();  // A's share of tile kt + 1 (issued a phase earlier)
      if (!grp_b || kt + 1 < ktiles) barrier();  // Y_kt
    }
  } else if constexpr (RP) {
    static_assert(LPW * (S - 1) < 64, "vmcnt range");
    constexpr int KS = 8 / Mma::kStep;
    constexpr int N_MFMA = KS * TM * TN;
    constexpr int N_DSR = KS * (TM + TN) * (Mma::kStep == 8 ? 2 : 1);
    constexpr int PER = N_MFMA / N_DSR;
    vec av[2][KS][TM], bv[2][KS][TN];
    auto read_frags = [&](auto set_c, int stage) {
      constexpr int SET = decltype(set_c)::value;
      const uint8_t* As = smem + stage * STAGE;
      const uint8_t* Bs = As + BM * RB;
#pragma unroll
      for (int q = 0; q < KS; ++q) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int r = wm * WTM + i * 16 + lrow;
          av[SET][q][i] = read_operand<Mma>(As + r * RB, r, q * Mma::kStep, lchunk);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int r = wn * WTN + j * 16 + lrow;
          bv[SET][q][j] = read_operand<Mma>(Bs + r * RB, r, q * Mma::kStep, lchunk);
        }
      }
    };
    // Prologue: every stage receives a tile; tile 0's fragments go to set 0.
#pragma unroll
    for (int st = 0; st < S; ++st)
      if (st < ktiles) issue(st, st);
    wait_vmcnt_groups<LPW>(min(static_cast<int64_t>(S - 1), ktiles - 1));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_frags(std::integral_constant<int, 0>{}, 0);
    auto body = [&](auto set_c, int64_t kt) {
      constexpr int SET = decltype(set_c)::value;
      // This wave's reads of tile kt are done and its part of tile kt + 1
      // has landed; after the barrier every wave is there, so tile kt's
      // stage may be refilled and tile kt + 1 read.
      wait_lgkmcnt0();
      wait_vmcnt_groups<LPW>(max(static_cast<int64_t>(0), min(static_cast<int64_t>(S - 2), ktiles - 2 - kt)));
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (kt + S < ktiles) issue(kt + S, static_cast<int>(kt % S));
      __builtin_amdgcn_sched_barrier(0);
      // Tile kt + 1's fragments into the other set (past the last tile this
      // reads a stale, in-bounds stage into the unused set), one LDS read
      // between every PER MFMAs of tile kt.
      read_frags(std::integral_constant<int, SET ^ 1>{}, static_cast<int>((kt + 1) % S));
#pragma unroll
      for (int q = 0; q < KS; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = Mma::mma(bv[SET][q][j], av[SET][q][i], acc[i][j]);
#pragma unroll
      for (int g = 0; g < N_DSR; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // one LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, PER, 0);  // PER MFMAs
      }
      if constexpr (N_MFMA > PER * N_DSR) __builtin_amdgcn_sched_group_barrier(0x008, N_MFMA - PER * N_DSR, 0);
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int64_t kt = 0; kt < ktiles; kt += 2) {
      body(std::integral_constant<int, 0>{}, kt);
      if (kt + 1 < ktiles) body(std::integral_constant<int, 1>{}, kt + 1);
    }
  } else {
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < ktiles) issue(st, st);
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    // Tiles issued after kt (at most S - 2 of them) may stay in flight.
    const int64_t later = min(static_cast<int64_t>(S - 2), ktiles - 1 - kt);
    if (later >= 2) wait_vmcnt<2 * LPW>();
    else if (later == 1) wait_vmcnt<LPW>();
    else wait_vmcnt<0>();
    // Barrier without __syncthreads' release fence: that fence would wait for
    // every outstanding DMA (vmcnt(0)) and drain the pipeline.  This wave's
    // tile-kt DMA is complete (the wait above) and its earlier LDS reads were
    // consumed by MFMAs; the empty asm statements keep the compiler from
    // moving memory operations across the barrier.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + S - 1 < ktiles) issue(kt + S - 1, static_cast<int>((kt + S - 1) % S));
    const uint8_t* As = smem + (kt % S) * STAGE;
    const uint8_t* Bs = As + BM * RB;
    // Every K step's operand fragments are read from LDS before the first
    // MFMA (a scheduling barrier keeps them there), so the later steps'
    // reads complete under the earlier steps' MFMAs.  Left to itself the
    // scheduler issues each step's reads just before its MFMAs and waits on
    // them (lgkmcnt(0) several times per K tile).
    constexpr int KS = 8 / Mma::kStep;
    vec av[KS][TM], bv[KS][TN];
#pragma unroll
    for (int q = 0; q < KS; ++q) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WTM + i * 16 + lrow;
        av[q][i] = read_operand<Mma>(As + r * RB, r, q * Mma::kStep, lchunk);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * WTN + j * 16 + lrow;
        bv[q][j] = read_operand<Mma>(Bs + r * RB, r, q * Mma::kStep, lchunk);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // The MFMA section runs at raised wave priority: of the two blocks
    // sharing a CU, the one multiplying keeps the matrix pipe fed while the
    // other waits on its DMA, barrier and LDS reads.
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int q = 0; q < KS; ++q)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          acc[i][j] = Mma::mma(bv[q][j], av[q][i], acc[i][j]);  // C^T: see epilogue_direct
        }
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
  }
  }

  if constexpr (Mma::kScaled) scale_acc<TM, TN>(acc, m0 + wm * WTM, n0 + wn * WTN, lane);
  TO* outp = static_cast<TO*>(p.out);
  const TO* resp = p.epi.residual ? static_cast<const TO*>(p.epi.residual) : nullptr;
  {
    constexpr uintptr_t kA = 4 * sizeof(TO) - 1;
    const bool vec4 = (p.ldo % 4 == 0) && ((reinterpret_cast<uintptr_t>(outp) & kA) == 0) &&
                      ((reinterpret_cast<uintptr_t>(resp) & kA) == 0);
    const float* bias = p.epi.bias_mode == 2 ? static_cast<const float*>(p.epi.bias) : nullptr;
    if constexpr (Mma::kInt) {
      // DIRECT: the host admitted only epilogues epilogue_direct_q computes
      // (big_tile_wins), GELU included; there is no staged path to fall to.
      if (DIRECT || epilogue_q_direct_ok(kernel_arg<Problem>(), vec4)) {
        epilogue_direct_q<TO, TM, TN, DIRECT_GELU>(acc, m0 + wm * WTM, n0 + wn * WTN, lane, outp, resp, bias, p.epi.act);
        return;
      }
    } else if (!STAGED || epilogue_is_simple(kernel_arg<Problem>(), vec4, DIRECT_GELU)) {
      epilogue_direct<TO, TM, TN, DIRECT_GELU>(acc, m0 + wm * WTM, n0 + wn * WTN, lane, outp, resp, bias, p.epi.act);
      return;
    }
  }
  if constexpr (STAGED) {
  const bool vec_ok = !p.out_nchw && (p.ldo % 8 == 0) && ((reinterpret_cast<uintptr_t>(p.out) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(p.epi.residual) & 15) == 0);
  __syncthreads();
  float* stage = reinterpret_cast<float*>(smem) + wave * WTM * (WTN + 4);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float* dst = &stage[(i * 16 + lrow) * (WTN + 4) + j * 16 + (lane >> 4) * 4 + r];  // C^T accumulators
        if constexpr (Mma::kInt) *reinterpret_cast<int*>(dst) = acc[i][j][r];
        else *dst = acc[i][j][r];
      }
  wave_sync_lds();
#pragma nounroll
  for (int i = 0; i < TM; ++i) {
    const int64_t mrow0 = m0 + wm * WTM + i * 16, ncol0 = n0 + wn * WTN;
    const float* strip = stage + i * 16 * (WTN + 4);
    if constexpr (Mma::kInt) {
      store_strip_q<TO, WTN>(strip, lane, mrow0, ncol0, outp, resp, vec_ok);
    } else {
      if (p.out_nchw) store_strip<TO, WTN>(p, strip, lane, mrow0, ncol0, outp, resp, 0);
      else store_strip_vec<TO, WTN>(strip, lane, mrow0, ncol0, outp, resp, 0, vec_ok);
    }
  }
  }
}

// =====================================================================
// Split-K finish (c3h_gemm_splitk_reduce): one thread per output, the
// partial products summed in split order, then the common epilogue.
// =====================================================================
template <typename TO>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(c3h_splitk_args a) {
  const KArg<c3h_splitk_args>& p = kernel_arg<c3h_splitk_args>();
  const int64_t mn = p.m * p.n;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= mn) return;
  const int64_t row = i / p.n, col = i - row * p.n;
  float v = p.partial[i];
  for (int s = 1; s < p.splits; ++s) v += p.partial[s * mn + i];
  const int64_t o = row * p.ldo + col;
  const float res = p.epi.residual ? Elem<TO>::to_f32(static_cast<const TO*>(p.epi.residual)[o]) : 0.0f;
  static_cast<TO*>(a.out)[o] = Elem<TO>::from_f32(apply_epilogue(p.epi, v, row, col, p.n, res, 0));
}


// ---------------------------------------------------------------- dispatch
template <int BM, int BN>
void grid_of(Problem& p, int64_t batch, dim3& grid) {
  p.tiles_m = static_cast<int>(ceil_div(p.m, BM));
  p.tiles_n = static_cast<int>(ceil_div(p.n, BN));
  grid = dim3(static_cast<unsigned>(p.tiles_m) * static_cast<unsigned>(p.tiles_n), 1, static_cast<unsigned>(batch));
}

template <int AM, bool BK_>
int launch_f32(Problem p, int64_t batch, hipStream_t s) {
  dim3 grid;
  if (p.n <= 64 && p.m >= 4096) {
    grid_of<256, 64>(p, batch, grid);
    hipLaunchKernelGGL((gemm_f32_kernel<256, 64, 4, 1, AM, BK_>), grid, dim3(kThreads), 0, s, p);
  } else if (p.m <= 64 || p.n <= 64 || ceil_div(p.m, 128) * ceil_div(p.n, 128) * batch < 256) {
    // narrow operands, or too few 128x128 tiles to fill the chip
    grid_of<64, 64>(p, batch, grid);
    hipLaunchKernelGGL((gemm_f32_kernel<64, 64, 2, 2, AM, BK_>), grid, dim3(kThreads), 0, s, p);
  } else {
    grid_of<128, 128>(p, batch, grid);
    hipLaunchKernelGGL((gemm_f32_kernel<128, 128, 2, 2, AM, BK_>), grid, dim3(kThreads), 0, s, p);
  }
  return launch_status("gemm_f32");
}

// The pipelined kernel needs byte offsets that fit the 32-bit buffer offset
// with room for the out-of-range sentinel, and no batch strides.
inline bool dma_eligible(const Problem& p, int64_t batch, int am) {
  if (switches().disable_dma) return false;
  // Narrow implicit-GEMM convs (N <= 64) stay on the register-prefetch
  // kernel, which measured faster there; wider ones use the DMA kernel.
  if (am == kConvTap && p.n <= 64) return false;
  return batch == 1 && (am == kDenseK || am == kConvTap) && p.a_bytes > 0 && p.b_bytes > 0 &&
         p.a_bytes < (int64_t{1} << 31) && p.b_bytes < (int64_t{1} << 31);
}

// Whether an eight-wave (one block per CU) DMA tile can take this GEMM: an
// epilogue that epilogue_direct(_q) handles (host-side restatement of
// epilogue_is_simple; plus GELU for int8, which the large-tile instantiation
// computes in registers).  int8 GEMMs writing int32 / int8 (qmode 0 / 1)
// need only aligned row-major stores (epilogue_q_direct_ok).
inline bool big_tile_ok(const Problem& p, size_t out_size, bool int_mma) {
  if (switches().disable_bigtile || p.n <= 128) return false;
  const c3h_epilogue& e = p.epi;
  const uintptr_t al = 4 * out_size - 1;
  const bool stores = !p.out_nchw && p.ldo % 4 == 0 && (reinterpret_cast<uintptr_t>(p.out) & al) == 0;
  // GELU is computed in registers by both tile sizes.
  const int max_act = 2;
  const bool simple = stores && e.alpha == 1.0f && e.beta == 1.0f && (e.bias_mode == 0 || e.bias_mode == 2) &&
                      e.act <= max_act && e.n_inst == 0 &&
                      (e.bias_mode == 0 || (reinterpret_cast<uintptr_t>(e.bias) & 15) == 0) &&
                      (reinterpret_cast<uintptr_t>(e.residual) & al) == 0;
  return int_mma && p.qmode <= 1 ? stores : simple;
}

// Tile cost in rounds of resident tiles, in units of a round of 128 x 128
// tiles at two blocks per CU: a 256 x 256 round costs 1.66 (measured: 8192^3
// GEMM, 1195 vs 994 us) and a 256 x 192 round 1.48 (0.89 of a 256 x 256
// round: int8 16384x768x3072, 45.6 vs 51.2 us).
inline double rounds_128(const Problem& p, int cus) {
  return static_cast<double>(ceil_div(ceil_div(p.m, 128) * ceil_div(p.n, 128), 2 * cus));
}
inline double rounds_256(const Problem& p, int cus) {
  return static_cast<double>(ceil_div(ceil_div(p.m, 256) * ceil_div(p.n, 256), cus)) * 1.66;
}

// Whether the 256 x 256 eight-wave DMA kernel beats 128 x 128 at two blocks
// per CU by a clear margin (near-ties measured slower: 16384x2304x768 int8).
inline bool big_tile_wins(const Problem& p, int cus, size_t out_size, bool int_mma) {
  if (!big_tile_ok(p, out_size, int_mma)) return false;
  return rounds_256(p, cus) < 0.9 * rounds_128(p, cus);
}

// Whether the 256 x 192 eight-wave kernel (N a multiple of 192) beats both:
// the W8A8 QKV (N = 2304: 3 full rounds instead of 2.25 rounds of 256 x 256
// or 4.5 of 128 x 128) and the N = 768 GEMMs (256 tiles fill the 256 CUs; 192
// tiles of 256 x 256 leave a quarter idle).
inline bool tile192_wins(const Problem& p, int cus, size_t out_size, bool int_mma) {
  if (p.n % 192 != 0 || !big_tile_ok(p, out_size, int_mma)) return false;
  const double r192 = static_cast<double>(ceil_div(ceil_div(p.m, 256) * (p.n / 192), cus)) * 1.48;
  return r192 < rounds_256(p, cus) && r192 < rounds_128(p, cus);
}

// Whether the 160 x 128 four-wave tile (wave tiles 80 x 64, two blocks per
// CU) beats 128 x 128 on a 16-bit implicit-GEMM conv: its rounds cost 1.25
// rounds of 128 x 128 tiles (the rows per tile), so it wins where it removes
// a mostly empty last round (ResNet-18 224 layer 2: 1255 tiles are 3 rounds
// of 512 slots, against 4 for the 1568 tiles of 128 x 128).  Its epilogue
// must be one epilogue_direct computes (it has no staged form): row-major
// aligned stores, alpha = beta = 1, no or per-column bias, ReLU or none.
inline bool tile160_wins(const Problem& p, int cus, size_t out_size) {
  if (switches().disable_tile160 || p.n <= 64 || p.n % 128 != 0) return false;
  const c3h_epilogue& e = p.epi;
  const uintptr_t al = 4 * out_size - 1;
  const bool simple = !p.out_nchw && p.ldo % 4 == 0 && (reinterpret_cast<uintptr_t>(p.out) & al) == 0 &&
                      e.alpha == 1.0f && e.beta == 1.0f && (e.bias_mode == 0 || e.bias_mode == 2) && e.act <= 1 &&
                      e.n_inst == 0 && e.row_max == nullptr &&
                      (e.bias_mode == 0 || (reinterpret_cast<uintptr_t>(e.bias) & 15) == 0) &&
                      (reinterpret_cast<uintptr_t>(e.residual) & al) == 0;
  if (!simple) return false;
  const double r160 = static_cast<double>(ceil_div(ceil_div(p.m, 160) * (p.n / 128), 2 * cus)) * 1.25;
  return r160 < 0.97 * rounds_128(p, cus);
}

// Register-pipelined form of the 4-wave DMA kernel: C3H_DMA_RP = 2, 3 or 4
// LDS stages (0: the two-stage kernel without register pipelining).
inline int dma_rp_stages() { return switches().dma_rp; }

inline int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

template <typename Mma, typename TO, int AM>
int launch_mfma(Problem p, int64_t batch, hipStream_t s, const char* what) {
  dim3 grid;
  if constexpr (AM == kDenseK || AM == kConvTap) {
    // 256 x 192: int8 GEMMs with bf16 output (the W8A8 decoder's QKV, out
    // projection and FFN2) and fp16 GEMMs with fp16 output (the fp16
    // decoder's QKV); the same K order as the other tiles.
    if constexpr (AM == kDenseK && ((Mma::kInt && std::is_same<TO, bf16_t>::value) ||
                                    (std::is_same<Mma, MmaF16>::value && std::is_same<TO, f16_t>::value))) {
      if (dma_eligible(p, batch, AM) && tile192_wins(p, device_cus(), sizeof(TO), Mma::kInt)) {
        grid_of<256, 192>(p, 1, grid);
        hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 256, 192, 8, 1, AM, 2, 8>), grid, dim3(512), 0, s, p);
        return launch_status(what);
      }
    }
    if (dma_eligible(p, batch, AM) && big_tile_wins(p, device_cus(), sizeof(TO), Mma::kInt)) {
      grid_of<256, 256>(p, 1, grid);
      // Convolutions take the ping-pong schedule (layer-3 3x3 convs of
      // ResNet-18 224: 75 -> 71 us); dense GEMMs measured equal or slower
      // with it (their K loops are 6-32 tiles; the LM head 246 -> 260 us).
      if constexpr (AM == kConvTap) {
        if (!switches().disable_pp) {
          hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 256, 256, 4, 2, AM, 2, 8, false, true>), grid, dim3(512),
                             0, s, p);
          return launch_status(what);
        }
      }
      hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 256, 256, 4, 2, AM, 2, 8>), grid, dim3(512), 0, s, p);
      return launch_status(what);
    }
    if (dma_eligible(p, batch, AM)) {
      const int rp = dma_rp_stages();
      if (p.n <= 64) {
        grid_of<256, 64>(p, 1, grid);
        if (rp == 2)
          hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 256, 64, 4, 1, AM, 2, 4, true>), grid, dim3(kThreads), 0, s, p);
        else if (rp == 3)
          hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 256, 64, 4, 1, AM, 3, 4, true>), grid, dim3(kThreads), 0, s, p);
        else
          hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 256, 64, 4, 1, AM, 2>), grid, dim3(kThreads), 0, s, p);
      } else {
        if constexpr (AM == kConvTap && !Mma::kInt) {
          if (rp == 0 && tile160_wins(p, device_cus(), sizeof(TO))) {
            grid_of<160, 128>(p, 1, grid);
            hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 160, 128, 2, 2, AM, 2>), grid, dim3(kThreads), 0, s, p);
            return launch_status(what);
          }
        }
        grid_of<128, 128>(p, 1, grid);
        if (rp == 2)
          hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 128, 128, 2, 2, AM, 2, 4, true>), grid, dim3(kThreads), 0, s,
                             p);
        else if (rp == 3)
          hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 128, 128, 2, 2, AM, 3, 4, true>), grid, dim3(kThreads), 0, s,
                             p);
        else if (rp == 4)
          hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 128, 128, 2, 2, AM, 4, 4, true>), grid, dim3(kThreads), 0, s,
                             p);
        else
          hipLaunchKernelGGL((mfma_gemm_dma_kernel<Mma, TO, 128, 128, 2, 2, AM, 2>), grid, dim3(kThreads), 0, s, p);
      }
      return launch_status(what);
    }
  }
  if constexpr (AM == kDenseK || AM == kConvTap) {
    if (batch == 1 && p.a_bytes > 0 && p.b_bytes > 0 && p.a_bytes < (int64_t{1} << 31) &&
        p.b_bytes < (int64_t{1} << 31) && !switches().disable_buf) {
      if (p.n <= 64) {
        grid_of<256, 64>(p, 1, grid);
        hipLaunchKernelGGL((mfma_gemm_kernel<Mma, TO, 256, 64, 4, 1, AM, true>), grid, dim3(kThreads), 0, s, p);
      } else {
        grid_of<128, 128>(p, 1, grid);
        hipLaunchKernelGGL((mfma_gemm_kernel<Mma, TO, 128, 128, 2, 2, AM, true>), grid, dim3(kThreads), 0, s, p);
      }
      return launch_status(what);
    }
  }
  if (p.n <= 64) {
    grid_of<256, 64>(p, batch, grid);
    hipLaunchKernelGGL((mfma_gemm_kernel<Mma, TO, 256, 64, 4, 1, AM>), grid, dim3(kThreads), 0, s, p);
  } else {
    grid_of<128, 128>(p, batch, grid);
    hipLaunchKernelGGL((mfma_gemm_kernel<Mma, TO, 128, 128, 2, 2, AM>), grid, dim3(kThreads), 0, s, p);
  }
  return launch_status(what);
}

// 16-bit inputs write either the same 16-bit type or fp32.
template <typename Mma, typename T, int AM>
int launch_h(Problem p, int64_t batch, hipStream_t s, int in_dtype) {
  if (p.out_dtype == C3H_F32) return launch_mfma<Mma, float, AM>(p, batch, s, "gemm_h");
  if (p.out_dtype == in_dtype) return launch_mfma<Mma, T, AM>(p, batch, s, "gemm_h");
  return fail(C3H_EUNSUPPORTED, "gemm: 16-bit inputs write fp32 or the input dtype, not %d", p.out_dtype);
}

template <int AM>
int launch_h_any(Problem p, int64_t batch, hipStream_t s, int in_dtype) {
  return in_dtype == C3H_BF16 ? launch_h<MmaBF16, bf16_t, AM>(p, batch, s, in_dtype)
                              : launch_h<MmaF16, f16_t, AM>(p, batch, s, in_dtype);
}

// fp8 GEMM: the two-stage DMA kernel where its 32-bit buffer offsets reach,
// else the register-prefetch kernel.
template <typename TO>
int launch_fp8(Problem p, hipStream_t s) {
  dim3 grid;
  if (dma_eligible(p, 1, kDenseK) && big_tile_wins(p, device_cus(), sizeof(TO), false)) {
    grid_of<256, 256>(p, 1, grid);
    hipLaunchKernelGGL((mfma_gemm_dma_kernel<MmaF8, TO, 256, 256, 4, 2, kDenseK, 2, 8>), grid, dim3(512), 0, s, p);
  } else if (dma_eligible(p, 1, kDenseK)) {
    if (p.n <= 64) {
      grid_of<256, 64>(p, 1, grid);
      hipLaunchKernelGGL((mfma_gemm_dma_kernel<MmaF8, TO, 256, 64, 4, 1, kDenseK, 2>), grid, dim3(kThreads), 0, s, p);
    } else {
      grid_of<128, 128>(p, 1, grid);
      hipLaunchKernelGGL((mfma_gemm_dma_kernel<MmaF8, TO, 128, 128, 2, 2, kDenseK, 2>), grid, dim3(kThreads), 0, s, p);
    }
  } else if (p.n <= 64) {
    grid_of<256, 64>(p, 1, grid);
    hipLaunchKernelGGL((mfma_gemm_kernel<MmaF8, TO, 256, 64, 4, 1, kDenseK>), grid, dim3(kThreads), 0, s, p);
  } else {
    grid_of<128, 128>(p, 1, grid);
    hipLaunchKernelGGL((mfma_gemm_kernel<MmaF8, TO, 128, 128, 2, 2, kDenseK>), grid, dim3(kThreads), 0, s, p);
  }
  return launch_status("gemm_fp8");
}

// W4A16 GEMM: the register-prefetch kernel with MXFP4 B and buffer loads.
template <typename TO>
int launch_w4(Problem p, hipStream_t s) {
  dim3 grid;
  if (p.n <= 64) {
    grid_of<256, 64>(p, 1, grid);
    hipLaunchKernelGGL((mfma_gemm_kernel<MmaF16, TO, 256, 64, 4, 1, kDenseK, true, true>), grid, dim3(kThreads), 0, s, p);
  } else {
    grid_of<128, 128>(p, 1, grid);
    hipLaunchKernelGGL((mfma_gemm_kernel<MmaF16, TO, 128, 128, 2, 2, kDenseK, true, true>), grid, dim3(kThreads), 0, s,
                       p);
  }
  return launch_status("gemm_w4a16");
}

// row_max_ok: the entry point can compute the row_max side output (it is
// refused everywhere else).
inline int check_epilogue(const c3h_epilogue& e, bool row_max_ok = false) {
  C3H_REQUIRE(row_max_ok || e.row_max == nullptr,
              "epilogue: row_max is taken only by c3h_gemm (16-bit inputs), c3h_qgemm (modes 2 / 3), "
              "c3h_gemm_fp8 and c3h_gemm_w4a16");
  C3H_REQUIRE(e.bias_mode >= 0 && e.bias_mode <= 4, "epilogue: bad bias_mode %d", e.bias_mode);
  C3H_REQUIRE(e.bias_mode == 0 || e.bias != nullptr, "epilogue: bias_mode %d needs a bias pointer", e.bias_mode);
  C3H_REQUIRE(e.act >= 0 && e.act <= 2, "epilogue: bad act %d", e.act);
  C3H_REQUIRE(e.act != 2 || e.n_imm >= 3, "epilogue: act 2 (gelu) reads imm[0..2]");
  C3H_REQUIRE(e.n_imm >= 0 && e.n_imm <= 8, "epilogue: n_imm %d out of range", e.n_imm);
  C3H_REQUIRE(e.n_inst >= 0 && e.n_inst <= C3H_EW_MAX_INST, "epilogue: n_inst %d out of range", e.n_inst);
  for (int i = 0; i < e.n_inst; ++i) {
    int limit = 2 + e.n_imm;
    C3H_REQUIRE(e.inst[i].a >= 0 && e.inst[i].a < limit && e.inst[i].b >= 0 && e.inst[i].b < limit,
                "epilogue: instruction %d operand outside [0,%d)", i, limit);
    C3H_REQUIRE(e.inst[i].op >= 0 && e.inst[i].op <= C3H_EW_COPY, "epilogue: bad opcode %d", e.inst[i].op);
  }
  return C3H_OK;
}

inline bool aligned(const void* ptr, int bytes) { return (reinterpret_cast<uintptr_t>(ptr) & (bytes - 1)) == 0; }

// The row_max side output is computed by the direct (register) epilogues
// only; these are the conditions under which every kernel the GEMM entry
// points select takes one (epilogue_is_simple / epilogue_q_direct_ok, and
// row-major aligned stores).
inline int check_row_max(const c3h_epilogue& e, int64_t n, int64_t ldo, const void* out, int out_dtype,
                         int64_t batch) {
  if (e.row_max == nullptr) return C3H_OK;
  C3H_REQUIRE(batch == 1, "row_max: batch 1 only");
  C3H_REQUIRE(out_dtype == C3H_F32 || out_dtype == C3H_BF16 || out_dtype == C3H_F16,
              "row_max: float outputs (fp32, bf16, fp16) only");
  const int es = dtype_size(out_dtype);
  C3H_REQUIRE(ldo % 4 == 0 && aligned(out, 4 * es) && (e.residual == nullptr || aligned(e.residual, 4 * es)),
              "row_max: needs ldo %% 4 == 0 and 4-element aligned out / residual");
  C3H_REQUIRE(e.alpha == 1.0f && e.beta == 1.0f && (e.bias_mode == 0 || (e.bias_mode == 2 && aligned(e.bias, 16))) &&
                  e.act <= 1 && e.n_inst == 0,
              "row_max: needs alpha = beta = 1, no bias or a 16-byte aligned per-column bias, act <= 1, no program");
  C3H_REQUIRE(e.row_max_ld >= ceil_div(n, 64) && aligned(e.row_max, 8),
              "row_max: row_max_ld must be >= ceil(n / 64) = %lld and the buffer 8-byte aligned",
              static_cast<long long>(ceil_div(n, 64)));
  return C3H_OK;
}


// ---------------------------------------------------------------- per-type launchers
// Defined one MFMA input type per translation unit (gemm_<type>.hip) so the
// kernel instantiations compile in parallel.
int launch_bf16_dense(Problem p, int64_t batch, hipStream_t s);   // gemm_bf16.hip
int launch_bf16_conv(Problem p, hipStream_t s, int am);            // gemm_bf16_conv.hip
int launch_f16_dense(Problem p, int64_t batch, hipStream_t s);    // gemm_f16.hip
int launch_f16_conv(Problem p, hipStream_t s, int am);             // gemm_f16_conv.hip
int launch_i8(Problem p, hipStream_t s, int mode, int out_dtype);  // gemm_i8.hip
int launch_f8(Problem p, hipStream_t s, int out_dtype);            // gemm_f8.hip
int launch_w4a16(Problem p, hipStream_t s, int out_dtype);         // gemm_w4.hip
int launch_f32_modes(Problem p, int64_t batch, hipStream_t s, int am, bool b_kcontig);  // gemm_f32.hip
int launch_conv_direct_c4(Problem p, hipStream_t s, bool* handled);  // gemm_f32.hip

}  // namespace gk
}  // namespace c3h
