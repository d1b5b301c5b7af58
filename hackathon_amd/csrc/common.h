// Internal helpers shared by the libc3hip.so translation units (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include "../../include/c3hip.h"

namespace c3h {

// Thread-local last-error message (returned by c3h_last_error()).
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
// Resolves the device address of gemm.hip's static split-K scratch array on
// `device` (which must be current); called by c3h_init.  Returns a status.
int gemm_scratch_setup(int device);

// Kernel-selection switches from the environment, read at the first launch
// and again by c3h_reload_switches() (launch paths read these, not getenv).
struct Switches {
  bool disable_dma = false;      // C3H_DISABLE_DMA: no direct-to-LDS GEMM kernel
  bool disable_bigtile = false;  // C3H_DISABLE_BIGTILE: no 256 x 256 tile
  bool disable_buf = false;      // C3H_DISABLE_BUF: no buffer-load GEMM kernel
  bool disable_conv3x3 = false;  // C3H_DISABLE_CONV3X3: no 64-channel band conv
  bool disable_direct_conv = false;  // C3H_DISABLE_DIRECT_CONV: no direct narrow-input fp32 conv
  int dma_rp = 0;                // C3H_DMA_RP: register-pipelined DMA stages (0 = off)
  bool disable_pp = false;       // C3H_DISABLE_PP: no ping-pong schedule for 256 x 256 conv tiles
  bool disable_qmul = false;     // C3H_DISABLE_QMUL: quantize by the division form only
  bool disable_tile160 = false;  // C3H_DISABLE_TILE160: no 160 x 128 conv tile
};
const Switches& switches();

#define C3H_HIP_CHECK(expr)                                                   \
  do {                                                                        \
    hipError_t err__ = (expr);                                                \
    if (err__ != hipSuccess)                                                  \
      return ::c3h::fail(C3H_EHIP, "%s failed: %s", #expr,                    \
                         hipGetErrorString(err__));                           \
  } while (0)

#define C3H_REQUIRE(cond, ...)                                                \
  do {                                                                        \
    if (!(cond)) return ::c3h::fail(C3H_EINVAL, __VA_ARGS__);                 \
  } while (0)

// Check the launch that was just enqueued.
inline int launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(C3H_EHIP, "%s launch failed: %s", what, hipGetErrorString(err));
  return C3H_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int dtype_size(int dt) {
  switch (dt) {
    case C3H_F32: case C3H_I32: return 4;
    case C3H_F16: case C3H_BF16: return 2;
    case C3H_I8: case C3H_U8: case C3H_BOOL: return 1;
    case C3H_I64: case C3H_F64: return 8;
    default: return 0;
  }
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Device-side element conversions.  bf16 and f16 narrowing round to nearest
// even; NaN stays NaN.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// gfx950 converts in hardware (v_cvt_pk_bf16_f32): round to nearest even,
// NaN quieted as (bits >> 16) | 0x40, denormals kept.  Checked equal to the
// integer formulation (u + 0x7fff + lsb) >> 16 for all 2^32 inputs.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
// Two values -> one packed pair (lo in bits 0-15): a single v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f2;
  typedef __attribute__((ext_vector_type(2))) __bf16 b2;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
}
// x rounded to bf16 and widened back, bit for bit f32_to_bf16_bits then
// bf16_bits_to_f32: one v_cvt_pk_bf16_f32 with x in the high half and +0
// (bf16 0x0000) in the low one.
__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float(f32x2_to_bf16x2_bits(0.0f, x)); }
__device__ __forceinline__ uint32_t f32x2_to_f16x2_bits(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f2;
  typedef __attribute__((ext_vector_type(2))) _Float16 h2;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, h2));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return static_cast<float>(v);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 v = static_cast<_Float16>(f);
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// Load element `i` of a buffer of runtime dtype as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
  switch (dt) {
    case C3H_F32: return static_cast<const float*>(p)[i];
    case C3H_F16: return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    case C3H_BF16: return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    case C3H_I8: return static_cast<float>(static_cast<const int8_t*>(p)[i]);
    case C3H_I32: return static_cast<float>(static_cast<const int32_t*>(p)[i]);
    case C3H_I64: return static_cast<float>(static_cast<const int64_t*>(p)[i]);
    case C3H_U8: case C3H_BOOL: return static_cast<float>(static_cast<const uint8_t*>(p)[i]);
    case C3H_F64: return static_cast<float>(static_cast<const double*>(p)[i]);
    default: return 0.0f;
  }
}

__device__ __forceinline__ void store_from_f32(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case C3H_F32: static_cast<float*>(p)[i] = v; break;
    case C3H_F16: static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v); break;
    case C3H_BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v); break;
    case C3H_F64: static_cast<double*>(p)[i] = static_cast<double>(v); break;
    default: break;
  }
}

// Typed element storage used by templated kernels.
template <typename T> struct Elem;
// load8 / store8 move 8 consecutive elements (16-byte aligned for 16-bit
// types, 32-byte for fp32) as whole vectors.
template <> struct Elem<float> {
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static __device__ __forceinline__ float from_f32(float v) { return v; }
  static __device__ __forceinline__ void load8(const float* p, float* v) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store8(float* p, const float* v) {
    reinterpret_cast<float4*>(p)[0] = float4{v[0], v[1], v[2], v[3]};
    reinterpret_cast<float4*>(p)[1] = float4{v[4], v[5], v[6], v[7]};
  }
  static __device__ __forceinline__ void load4(const float* p, float* v) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  }
  static __device__ __forceinline__ void store4(float* p, const float* v) {
    *reinterpret_cast<float4*>(p) = float4{v[0], v[1], v[2], v[3]};
  }
};

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

template <typename T, float (*ToF)(uint16_t), uint16_t (*FromF)(float), uint32_t (*Pack2)(float, float)>
struct Elem16 {
  static __device__ __forceinline__ float to_f32(T v) { return ToF(v.bits); }
  static __device__ __forceinline__ T from_f32(float v) { return T{FromF(v)}; }
  static __device__ __forceinline__ void load8(const T* p, float* v) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = ToF(static_cast<uint16_t>(w[i] & 0xffffu));
      v[2 * i + 1] = ToF(static_cast<uint16_t>(w[i] >> 16));
    }
  }
  static __device__ __forceinline__ void store8(T* p, const float* v) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = Pack2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<uint4*>(p) = uint4{w[0], w[1], w[2], w[3]};
  }
  // 4 consecutive elements, 8-byte aligned.
  static __device__ __forceinline__ void load4(const T* p, float* v) {
    const uint2 q = *reinterpret_cast<const uint2*>(p);
    v[0] = ToF(static_cast<uint16_t>(q.x & 0xffffu));
    v[1] = ToF(static_cast<uint16_t>(q.x >> 16));
    v[2] = ToF(static_cast<uint16_t>(q.y & 0xffffu));
    v[3] = ToF(static_cast<uint16_t>(q.y >> 16));
  }
  static __device__ __forceinline__ void store4(T* p, const float* v) {
    *reinterpret_cast<uint2*>(p) = uint2{Pack2(v[0], v[1]), Pack2(v[2], v[3])};
  }
  // Two elements as one dword (the first in the low half), and back.
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return Pack2(lo, hi); }
  static __device__ __forceinline__ void unpack2(uint32_t w, float* v) {
    v[0] = ToF(static_cast<uint16_t>(w & 0xffffu));
    v[1] = ToF(static_cast<uint16_t>(w >> 16));
  }
};
template <> struct Elem<bf16_t> : Elem16<bf16_t, bf16_bits_to_f32, f32_to_bf16_bits, f32x2_to_bf16x2_bits> {};
template <> struct Elem<f16_t> : Elem16<f16_t, f16_bits_to_f32, f32_to_f16_bits, f32x2_to_f16x2_bits> {};

// 16-bit outputs of the MFMA C^T accumulator layout, 16 bytes per lane.  A
// 16 x 16 output tile j of a 16x16 MFMA leaves lane (l16, lg = lane / 16)
// with row l16's columns 16 j + 4 lg .. + 3, as dwords d[j][h] (columns
// 4 lg + 2 h, + 1).  For a pair of adjacent tiles (j = 0, 1: 32 columns),
// the row layout gives lane row lg columns 8 lg .. 8 lg + 7 instead, as one
// 16-byte vector whose dword k = 2 k1 + h holds columns 8 lg + 4 k1 + 2 h,
// + 1 -- the pair that d[lg >> 1][h] holds in lane row 2 (lg & 1) + k1.  So
// the index bits (tile j, lane row bit 1, lane row bit 0) of a pair become
// (lane row bit 1, lane row bit 0, k1): a permlane32 swap exchanges the
// register index with lane row bit 1 (the upper 32 lanes of its first
// operand with the lower 32 of its second), a permlane16 swap then
// exchanges it with lane row bit 0 (odd lane rows of the first operand with
// even rows of the second).  Only lanes with the same l16 (the same output
// row) trade values.
__device__ __forceinline__ uint4 ct_pair_to_rows(const uint32_t (&d0)[2], const uint32_t (&d1)[2]) {
  uint32_t z[2][2];  // [k1][h]
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const auto e = __builtin_amdgcn_permlane32_swap(d0[h], d1[h], false, false);
    const auto f = __builtin_amdgcn_permlane16_swap(e[0], e[1], false, false);
    z[0][h] = f[0];
    z[1][h] = f[1];
  }
  return uint4{z[0][0], z[0][1], z[1][0], z[1][1]};
}
// int8 outputs: tile j of a group of four (64 columns) leaves lane (l16, lg)
// with row l16's columns 16 j + 4 lg .. + 3 as the dword w[j]; the row
// layout gives lane row lg the group's columns 16 lg .. 16 lg + 15, whose
// dword k is w[lg] of lane row k -- a transpose of (tile, lane row): tile
// bit 1 <-> lane row bit 1 (permlane32 swaps of tiles 0, 2 and 1, 3), then
// tile bit 0 <-> lane row bit 0 (permlane16 swaps of 0, 1 and 2, 3).
__device__ __forceinline__ uint4 ct_quad_to_rows(const uint32_t (&w)[4]) {
  const auto a = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  return uint4{c[0], c[1], d[0], d[1]};
}
// The inverse of ct_pair_to_rows: a row-layout vector back to the dwords d0
// (tile j = 0) and d1.
__device__ __forceinline__ void rows_to_ct_pair(const uint4 q, uint32_t (&d0)[2], uint32_t (&d1)[2]) {
  const uint32_t z[2][2] = {{q.x, q.y}, {q.z, q.w}};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const auto e = __builtin_amdgcn_permlane16_swap(z[0][h], z[1][h], false, false);
    const auto f = __builtin_amdgcn_permlane32_swap(e[0], e[1], false, false);
    d0[h] = f[0];
    d1[h] = f[1];
  }
}

// 16 bytes of T <-> fp32 values (8 for 16-bit types, 4 for fp32).
template <typename T>
__device__ __forceinline__ void load_vec16(const T* p, float* v) {
  if constexpr (sizeof(T) == 4) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
    Elem<T>::load8(p, v);
  }
}
template <typename T>
__device__ __forceinline__ void store_vec16(T* p, const float* v) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4*>(p) = float4{v[0], v[1], v[2], v[3]};
  } else {
    Elem<T>::store8(p, v);
  }
}

// x rounded to the storage type dt (bf16 / fp16; fp32 unchanged) and back:
// the value a consumer reads after the producer stores x as dt.
__device__ __forceinline__ float round_to_dtype(float x, int dt) {
  if (dt == C3H_BF16) return bf16_round(x);
  if (dt == C3H_F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  return x;
}

// x / scale rounded to nearest, for the int8 QuantizeLinear codes, without an
// IEEE division per element (about ten VALU operations, which made the
// quantizing kernels issue-bound rather than HBM-bound).  With
// scale = m 2^e (1 <= m < 2) and inv = RN(1/m), once: y = x 2^-e (exact
// wherever the quotient matters), then Markstein's correction
// q0 = RN(y inv), r = fma(-q0, m, y) (exact), q = RN(q0 + r inv) -- the
// correctly rounded y / m = x / scale whenever y and r are normal
// (P. Markstein, IBM J. Res. Dev. 34(1), 1990; Muller et al., Handbook of
// Floating-Point Arithmetic, the division-by-FMA theorems).  q0 is first
// clamped to +-2^20: a quotient that large saturates every int8 code whatever
// its rounding, and the clamp keeps an infinite q0 (x = +-Inf, or y
// overflowing) from turning r into NaN; a NaN x stays NaN.  Whenever
// |x / scale| >= 1/4 (the only quotients whose rounding can move a code) the
// result equals x / scale bit for bit, for every positive finite scale;
// smaller ones round to code zero_point either way.  One branch-free form.
// Scales QuantDiv serves (and the quantizing entry points accept): positive,
// normal, finite.
inline bool quant_scale_ok(float s) { return s >= 0x1p-126f && s <= 3.4028235e38f; }

// Host: a multiplier c such that the int8 code saturate(rne(x * c) +
// zero) equals saturate(rne(x / scale) + zero) -- the correctly rounded
// quotient's code, NaN -> -128 on both sides -- for every value x of the
// 16-bit type `dtype` (C3H_BF16 or C3H_F16: all 65536 encodings are tried).
// Candidates are fp32(1 / scale) and its neighbours up to 4 ulp away; 0 when
// none qualifies (or for another dtype, or under C3H_DISABLE_QMUL).  A 16-bit
// value has at most 11 significant bits, so x / scale lands within an ulp of
// a rounding boundary (k + 1/2) for few x, and 1 / scale itself qualifies
// for nearly every scale.  Cached per (scale, zero, dtype).
float quant_multiplier(float scale, int zero, int dtype);

struct QuantDiv {
  float m, inv;
  int e;
  // quant_multiplier(scale, zero, dtype) when the values codes4 / codes8 see
  // are all of that 16-bit dtype: their codes are then rne(x * mul), one
  // multiply, with the same result; 0 = the division form
  float mul = 0.0f;
  __device__ __forceinline__ explicit QuantDiv(float scale) {
    int ex = 0;
    m = 2.0f * frexpf(scale, &ex);
    e = ex - 1;
    inv = 1.0f / m;
  }
  // The same split made on the host (frexpf and an IEEE fp32 division give
  // the same m, e and inv there), passed to kernels that would otherwise
  // form it once per wave.
  __host__ __device__ QuantDiv(float m_, float inv_, int e_, float mul_ = 0.0f) : m(m_), inv(inv_), e(e_), mul(mul_) {}
  // dtype: the 16-bit type of every value to be quantized (C3H_BF16 /
  // C3H_F16) for the one-multiply form, or -1
  static QuantDiv on_host(float scale, int zero = 0, int dtype = -1) {
    int ex = 0;
    const float mm = 2.0f * frexpf(scale, &ex);
    return QuantDiv(mm, 1.0f / mm, ex - 1, dtype >= 0 ? quant_multiplier(scale, zero, dtype) : 0.0f);
  }
  __device__ __forceinline__ float quotient(float x) const {
    const float y = ldexpf(x, -e);
    const float q0 = fminf(fmaxf(y * inv, -0x1p20f), 0x1p20f);
    return fmaf(fmaf(-q0, m, y), inv, q0);
  }
  // Byte k of `acc` set to saturate(rne(x / scale) + zero_point) + 128: the
  // integer rne(x / scale) + (zero_point + 128) goes through
  // v_cvt_pk_u8_f32, which clamps to [0, 255] (a NaN quotient gives 0) and
  // inserts the byte, so rounding, offset, saturation and packing cost three
  // instructions.  XOR 0x80 per byte turns the biased byte into the int8 code.
  __device__ __forceinline__ uint32_t biased_byte(float x, float zp128, uint32_t k, uint32_t acc) const {
    return __builtin_amdgcn_cvt_pk_u8_f32(rintf(quotient(x)) + zp128, k, acc);
  }
  // saturate(rne(x / scale) + zero_point) as an int8 code (NaN -> -128)
  __device__ __forceinline__ int8_t code(float x, int zero_point) const {
    return static_cast<int8_t>(biased_byte(x, static_cast<float>(zero_point + 128), 0u, 0u) ^ 0x80u);
  }
  // 4 codes packed little-endian into one word (x of the dtype `mul` was
  // checked for, when it is nonzero).
  __device__ __forceinline__ uint32_t codes4(const float* x, int zero_point) const {
    const float zp128 = static_cast<float>(zero_point + 128);
    uint32_t w = 0u;
    if (mul != 0.0f) {
#pragma unroll
      for (int k = 0; k < 4; ++k) w = __builtin_amdgcn_cvt_pk_u8_f32(rintf(x[k] * mul) + zp128, k, w);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) w = biased_byte(x[k], zp128, static_cast<uint32_t>(k), w);
    }
    return w ^ 0x80808080u;
  }
  // 8 codes packed little-endian into two words.
  __device__ __forceinline__ uint2 codes8(const float* x, int zero_point) const {
    const float zp128 = static_cast<float>(zero_point + 128);
    uint32_t w[2] = {0u, 0u};
    if (mul != 0.0f) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        w[k >> 2] = __builtin_amdgcn_cvt_pk_u8_f32(rintf(x[k] * mul) + zp128, k & 3, w[k >> 2]);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k >> 2] = biased_byte(x[k], zp128, static_cast<uint32_t>(k & 3), w[k >> 2]);
    }
    return uint2{w[0] ^ 0x80808080u, w[1] ^ 0x80808080u};
  }
};

// Abramowitz & Stegun 7.1.26 rational approximation of erf (max abs error
// about 1.5e-7), the formula the reference's unfused Erf uses.
__device__ __forceinline__ float erf_as(float x) {
  float s = x < 0.0f ? -1.0f : (x > 0.0f ? 1.0f : 0.0f);
  float ax = fabsf(x);
  float t = 1.0f / (1.0f + 0.3275911f * ax);
  float t2 = t * t, t3 = t2 * t, t4 = t3 * t, t5 = t4 * t;
  float poly = 0.254829592f * t + -0.284496736f * t2 + 1.421413741f * t3 +
               -1.453152027f * t4 + 1.061405429f * t5;
  return s * (1.0f - poly * expf(-ax * ax));
}

// One elementwise instruction on fp32 values.
__device__ __forceinline__ float ew_apply(int op, float a, float b, float imm) {
  switch (op) {
    case C3H_EW_ADD: return a + b;
    case C3H_EW_SUB: return a - b;
    case C3H_EW_MUL: return a * b;
    case C3H_EW_DIV: return a / b;
    case C3H_EW_RELU: return fmaxf(a, 0.0f);
    case C3H_EW_ERF: return erff(a);
    case C3H_EW_ERF_AS: return erf_as(a);
    case C3H_EW_SQRT: return sqrtf(a);
    case C3H_EW_EXP: return expf(a);
    case C3H_EW_RECIP: return 1.0f / a;
    case C3H_EW_MAX: return fmaxf(a, b);
    case C3H_EW_MIN: return fminf(a, b);
    case C3H_EW_NEG: return -a;
    case C3H_EW_ADD_IMM: return a + imm;
    case C3H_EW_MUL_IMM: return a * imm;
    case C3H_EW_COPY: return a;
    default: return a;
  }
}

// Register file of an elementwise program: up to 24 fp32 registers addressed
// by uniform (kernel-argument) indices, so the switch compiles to scalar
// branches rather than scratch memory.
struct EwRegs {
  float r[24];
};

// conv3x3.hip: the banded 3x3 / 64-channel convolution.  Sets *handled when
// it launched (the return value is then the launch status).
int conv3x3_c64_launch(const c3h_conv_args* a, hipStream_t s, bool* handled);

}  // namespace c3h
