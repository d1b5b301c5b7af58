// Memory-bound kernel families of libc3hip.so (gfx950).  Each kernel reads
// its inputs once and writes its outputs once; launches are sized for 256 CUs
// (grid >= 4 x 256 workgroups where the problem allows) with coalesced,
// 64-lane-wide access along the fastest-varying dimension.
#include "common.h"

using namespace c3h;

namespace {

constexpr int kBlock = 256;

inline int grid_for(int64_t work, int per_thread = 1) {
  int64_t blocks = ceil_div(ceil_div(work, per_thread), kBlock);
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;  // grid-stride beyond this
  return static_cast<int>(blocks);
}

// ------------------------------------------------------------------ fill
__global__ void fill_kernel(void* out, int64_t count, int dt, double value) {
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
    switch (dt) {
      case C3H_I64: static_cast<int64_t*>(out)[i] = static_cast<int64_t>(value); break;
      case C3H_I32: static_cast<int32_t*>(out)[i] = static_cast<int32_t>(value); break;
      case C3H_I8: static_cast<int8_t*>(out)[i] = static_cast<int8_t>(value); break;
      case C3H_U8: case C3H_BOOL: static_cast<uint8_t*>(out)[i] = static_cast<uint8_t>(value); break;
      default: store_from_f32(out, dt, i, static_cast<float>(value)); break;
    }
  }
}

// ------------------------------------------------------------------ cast
__global__ void cast_kernel(const void* in, void* out, int64_t count, int idt, int odt) {
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
    if (odt == C3H_I64) {
      static_cast<int64_t*>(out)[i] = idt == C3H_I64 ? static_cast<const int64_t*>(in)[i]
                                                     : static_cast<int64_t>(load_as_f32(in, idt, i));
    } else if (odt == C3H_I32) {
      static_cast<int32_t*>(out)[i] = idt == C3H_I64 ? static_cast<int32_t>(static_cast<const int64_t*>(in)[i])
                                                     : static_cast<int32_t>(load_as_f32(in, idt, i));
    } else {
      store_from_f32(out, odt, i, load_as_f32(in, idt, i));
    }
  }
}

// ------------------------------------------------------------------ elementwise program
// Flat mode: every input is either dense with the output's shape (stride
// flag 1) or a single element (stride flag 0); general mode decomposes the
// linear index over the output shape.
template <bool kFlat>
__global__ void __launch_bounds__(kBlock) ew_kernel(c3h_ew_args a, int64_t numel) {
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < numel; idx += stride) {
    float r[C3H_EW_MAX_IN + C3H_EW_MAX_INST];
    if (kFlat) {
#pragma unroll
      for (int j = 0; j < C3H_EW_MAX_IN; ++j)
        if (j < a.n_in) r[j] = load_as_f32(a.in[j], a.in_dtype[j], a.stride[j][0] ? idx : 0);
    } else {
      int64_t off[C3H_EW_MAX_IN];
#pragma unroll
      for (int j = 0; j < C3H_EW_MAX_IN; ++j) off[j] = 0;
      int64_t rem = idx;
      for (int d = a.rank - 1; d >= 0; --d) {
        int64_t extent = a.shape[d];
        int64_t c = rem % extent;
        rem /= extent;
#pragma unroll
        for (int j = 0; j < C3H_EW_MAX_IN; ++j) off[j] += c * a.stride[j][d];
      }
#pragma unroll
      for (int j = 0; j < C3H_EW_MAX_IN; ++j)
        if (j < a.n_in) r[j] = load_as_f32(a.in[j], a.in_dtype[j], off[j]);
    }
    float v = r[0];
    for (int i = 0; i < a.n_inst; ++i) {
      const c3h_ew_inst ins = a.inst[i];
      v = ew_apply(ins.op, r[ins.a], r[ins.b], ins.imm);
      r[a.n_in + i] = v;
    }
    store_from_f32(a.out, a.out_dtype, idx, v);
  }
}

// Vectorized fast path: fp32 inputs (dense or scalar), fp32 output, 4
// elements per thread per step.
__global__ void __launch_bounds__(kBlock) ew_flat_f32x4_kernel(c3h_ew_args a, int64_t nvec) {
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t vi = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; vi < nvec; vi += stride) {
    constexpr int R = C3H_EW_MAX_IN + C3H_EW_MAX_INST;
    float rx[R], ry[R], rz[R], rw[R];
#pragma unroll
    for (int j = 0; j < C3H_EW_MAX_IN; ++j) {
      if (j < a.n_in) {
        const float* p = static_cast<const float*>(a.in[j]);
        float4 t;
        if (a.stride[j][0]) t = reinterpret_cast<const float4*>(p)[vi];
        else { float s = p[0]; t = make_float4(s, s, s, s); }
        rx[j] = t.x; ry[j] = t.y; rz[j] = t.z; rw[j] = t.w;
      }
    }
    float4 v = make_float4(rx[0], ry[0], rz[0], rw[0]);
    for (int i = 0; i < a.n_inst; ++i) {
      const c3h_ew_inst ins = a.inst[i];
      v.x = ew_apply(ins.op, rx[ins.a], rx[ins.b], ins.imm);
      v.y = ew_apply(ins.op, ry[ins.a], ry[ins.b], ins.imm);
      v.z = ew_apply(ins.op, rz[ins.a], rz[ins.b], ins.imm);
      v.w = ew_apply(ins.op, rw[ins.a], rw[ins.b], ins.imm);
      rx[a.n_in + i] = v.x; ry[a.n_in + i] = v.y; rz[a.n_in + i] = v.z; rw[a.n_in + i] = v.w;
    }
    reinterpret_cast<float4*>(a.out)[vi] = v;
  }
}

// ------------------------------------------------------------------ strided copy
template <typename T>
__global__ void __launch_bounds__(kBlock) strided_copy_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                               c3h_copy_args a, int64_t total) {
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    int64_t rem = idx, off = a.in_offset;
    for (int d = a.rank - 1; d >= 0; --d) {
      int64_t extent = a.shape[d];
      int64_t c = rem % extent;
      rem /= extent;
      off += c * a.in_stride[d];
    }
    out[idx] = in[off];
  }
}

// Tiled 2-D transpose for the case "innermost output dim is strided on the
// input while another dim is unit-stride": out[b][r][c] = in[b][c][r].
template <typename T>
__global__ void __launch_bounds__(256) transpose_tile_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                             int64_t batch, int64_t rows, int64_t cols,
                                                             int64_t in_b, int64_t out_b) {
  __shared__ T tile[32][33];
  int64_t b = blockIdx.z;
  int64_t r0 = static_cast<int64_t>(blockIdx.y) * 32, c0 = static_cast<int64_t>(blockIdx.x) * 32;
  int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  const T* src = in + b * in_b;
  T* dst = out + b * out_b;
  // in is [cols][rows] (row-major): read coalesced along rows.
  for (int k = ty; k < 32; k += 8) {
    int64_t c = c0 + k, r = r0 + tx;
    if (c < cols && r < rows) tile[k][tx] = src[c * rows + r];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    int64_t r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) dst[r * cols + c] = tile[tx][k];
  }
}

// ------------------------------------------------------------------ reductions
// Cross-lane steps of a wave reduction within each row of 16 lanes, as DPP
// moves (VALU, no LDS round trip): quad_perm [1,0,3,2] and [2,3,0,1] pair
// lanes 1 and 2 apart; row_half_mirror (lane i <-> 7 - i of each 8) and
// row_mirror (i <-> 15 - i of each 16) then pair whole quads and half-rows,
// whose lanes already hold equal partial results.  Every lane ends with its
// row's total; the last two steps (16, 32 lanes apart) cross rows.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
template <typename Op>
__device__ __forceinline__ float row16_reduce(float v, Op op) {
  v = op(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_mov<0x141>(v));  // row_half_mirror
  v = op(v, dpp_mov<0x140>(v));  // row_mirror
  return v;
}
// Cross-row steps by v_permlane16_swap / v_permlane32_swap (gfx950): with
// one register as both operands, the pair holds each lane's value and that
// of lane ^ 16 (^ 32), so each step is one VALU swap and an add -- no LDS
// round trip as with ds_bpermute -- and the same two addends as before.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_reduce(v, [](float a, float b) { return a + b; });
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// inner == 1: one wave per row.
__global__ void __launch_bounds__(kBlock) reduce_rows_kernel(c3h_reduce_args a) {
  int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + wave;
  if (row >= a.outer) return;
  const int64_t base = row * a.reduce;
  float acc = a.kind == 0 ? -INFINITY : 0.0f;
  for (int64_t i = lane; i < a.reduce; i += 64) {
    float v = load_as_f32(a.in, a.in_dtype, base + i);
    acc = a.kind == 0 ? fmaxf(acc, v) : acc + v;
  }
  acc = a.kind == 0 ? wave_max(acc) : wave_sum(acc);
  if (a.kind == 2) acc = acc / static_cast<float>(a.reduce);
  if (lane == 0) store_from_f32(a.out, a.out_dtype, row, acc);
}

// inner > 1: one thread per (outer, inner) column, coalesced across inner.
__global__ void __launch_bounds__(kBlock) reduce_cols_kernel(c3h_reduce_args a) {
  int64_t total = a.outer * a.inner;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    int64_t o = t / a.inner, in = t - o * a.inner;
    int64_t base = o * a.reduce * a.inner + in;
    float acc = a.kind == 0 ? -INFINITY : 0.0f;
    for (int64_t i = 0; i < a.reduce; ++i) {
      float v = load_as_f32(a.in, a.in_dtype, base + i * a.inner);
      acc = a.kind == 0 ? fmaxf(acc, v) : acc + v;
    }
    if (a.kind == 2) acc = acc / static_cast<float>(a.reduce);
    store_from_f32(a.out, a.out_dtype, t, acc);
  }
}

// Short reduce axis (GlobalAveragePool's 16 or 49 positions), inner % 8 ==
// 0, 16-byte aligned: a block covers one outer index and 16 vectors of 8
// inner elements (128 channels); its 256 threads are 16 position groups x 16
// vectors (thread t: group p = t / 16, vector t % 16), group p summing
// positions p, p + 16, ... two loads in flight, and the 16 partials of each
// vector are combined through LDS in group order.  Per 512 channels that is
// four blocks where reduce_cols_vec_kernel has one: its one block per outer
// index left the ResNet pools (256 images) with one wave per SIMD, too few
// loads in flight to cover HBM latency.
template <typename T>
__global__ void __launch_bounds__(kBlock) reduce_cols_vec16_kernel(c3h_reduce_args a) {
  __shared__ float part[16][16][9];
  const int t = threadIdx.x, p = t >> 4, v = t & 15;
  const int64_t o = blockIdx.x;
  const int64_t c8 = static_cast<int64_t>(blockIdx.y) * 16 + v;
  const bool live = c8 * 8 < a.inner;
  const T* in = static_cast<const T*>(a.in) + o * a.reduce * a.inner + c8 * 8;
  const bool mx = a.kind == 0;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = mx ? -INFINITY : 0.0f;
  if (live) {
    int64_t i = p;
    for (; i + 16 < a.reduce; i += 32) {
      float x0[8], x1[8];
      load_vec16(in + i * a.inner, x0);
      load_vec16(in + (i + 16) * a.inner, x1);
      if constexpr (sizeof(T) == 4) {
        load_vec16(in + i * a.inner + 4, x0 + 4);
        load_vec16(in + (i + 16) * a.inner + 4, x1 + 4);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = mx ? fmaxf(acc[e], x0[e]) : acc[e] + x0[e];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = mx ? fmaxf(acc[e], x1[e]) : acc[e] + x1[e];
    }
    if (i < a.reduce) {
      float x0[8];
      load_vec16(in + i * a.inner, x0);
      if constexpr (sizeof(T) == 4) load_vec16(in + i * a.inner + 4, x0 + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = mx ? fmaxf(acc[e], x0[e]) : acc[e] + x0[e];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) part[p][v][e] = acc[e];
  __syncthreads();
  // 128 threads, one output each (vector t / 8, element t % 8: consecutive
  // threads store consecutive channels), sum the 16 groups in group order.
  if (t < 128) {
    const int ov = t >> 3, oe = t & 7;
    const int64_t oc8 = static_cast<int64_t>(blockIdx.y) * 16 + ov;
    if (oc8 * 8 < a.inner) {
      float r = part[0][ov][oe];
#pragma unroll
      for (int q = 1; q < 16; ++q) r = mx ? fmaxf(r, part[q][ov][oe]) : r + part[q][ov][oe];
      if (a.kind == 2) r = r / static_cast<float>(a.reduce);
      store_from_f32(a.out, a.out_dtype, o * a.inner + oc8 * 8 + oe, r);
    }
  }
}

// inner % 8 == 0, 16-byte aligned (channels-last GlobalAveragePool): a block
// covers one outer index and 64 vectors of 8 inner elements; its four waves
// split the reduce axis (positions w, w + 4, ...), each thread keeping 8
// running values with four positions in flight, and the four partials are
// combined through LDS in wave order.
template <typename T>
__global__ void __launch_bounds__(kBlock) reduce_cols_vec_kernel(c3h_reduce_args a) {
  __shared__ float part[kBlock / 64][64][9];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t o = blockIdx.x;
  const int64_t c8 = static_cast<int64_t>(blockIdx.y) * 64 + lane;
  const bool live = c8 * 8 < a.inner;
  const T* in = static_cast<const T*>(a.in) + o * a.reduce * a.inner + c8 * 8;
  const float init = a.kind == 0 ? -INFINITY : 0.0f;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = init;
  if (live) {
    int64_t i = wave;
    for (; i + 12 < a.reduce; i += 16) {
      float v[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u) load_vec16(in + (i + 4 * u) * a.inner, v[u]);
      if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) load_vec16(in + (i + 4 * u) * a.inner + 4, v[u] + 4);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = a.kind == 0 ? fmaxf(acc[e], v[u][e]) : acc[e] + v[u][e];
    }
    for (; i < a.reduce; i += 4) {
      float v[8];
      load_vec16(in + i * a.inner, v);
      if constexpr (sizeof(T) == 4) load_vec16(in + i * a.inner + 4, v + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = a.kind == 0 ? fmaxf(acc[e], v[e]) : acc[e] + v[e];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) part[wave][lane][e] = acc[e];
  __syncthreads();
  if (wave == 0 && live) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float r = part[0][lane][e];
#pragma unroll
      for (int w = 1; w < kBlock / 64; ++w) r = a.kind == 0 ? fmaxf(r, part[w][lane][e]) : r + part[w][lane][e];
      if (a.kind == 2) r = r / static_cast<float>(a.reduce);
      store_from_f32(a.out, a.out_dtype, o * a.inner + c8 * 8 + e, r);
    }
  }
}

// ------------------------------------------------------------------ softmax
__global__ void __launch_bounds__(kBlock) softmax_rows_kernel(c3h_softmax_args a) {
  // one block per row (inner == 1)
  __shared__ float red[kBlock / 64];
  int64_t row = blockIdx.x;
  int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t base = row * a.axis;
  float m = -INFINITY;
  for (int64_t i = threadIdx.x; i < a.axis; i += kBlock) m = fmaxf(m, load_as_f32(a.in, a.in_dtype, base + i));
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < a.axis; i += kBlock) s += expf(load_as_f32(a.in, a.in_dtype, base + i) - m);
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  s = red[0] + red[1] + red[2] + red[3];
  for (int64_t i = threadIdx.x; i < a.axis; i += kBlock)
    store_from_f32(a.out, a.out_dtype, base + i, expf(load_as_f32(a.in, a.in_dtype, base + i) - m) / s);
}

__global__ void __launch_bounds__(kBlock) softmax_cols_kernel(c3h_softmax_args a) {
  int64_t total = a.outer * a.inner;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    int64_t o = t / a.inner, in = t - o * a.inner;
    int64_t base = o * a.axis * a.inner + in;
    float m = -INFINITY;
    for (int64_t i = 0; i < a.axis; ++i) m = fmaxf(m, load_as_f32(a.in, a.in_dtype, base + i * a.inner));
    float s = 0.0f;
    for (int64_t i = 0; i < a.axis; ++i) s += expf(load_as_f32(a.in, a.in_dtype, base + i * a.inner) - m);
    for (int64_t i = 0; i < a.axis; ++i)
      store_from_f32(a.out, a.out_dtype, base + i * a.inner,
                     expf(load_as_f32(a.in, a.in_dtype, base + i * a.inner) - m) / s);
  }
}

// ------------------------------------------------------------------ layernorm
// One wave per row; up to kCache values per lane stay in registers.
constexpr int kLnCache = 32;

__global__ void __launch_bounds__(kBlock) layernorm_kernel(c3h_layernorm_args a) {
  int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + wave;
  if (row >= a.rows) return;
  const int64_t base = row * a.cols;
  const float* scale = static_cast<const float*>(a.scale);
  const float* bias = static_cast<const float*>(a.bias);
  const bool cached = a.cols <= 64 * kLnCache;
  float vals[kLnCache];
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < kLnCache; ++j) {
    int64_t c = lane + 64 * j;
    float v = 0.0f;
    if (cached && c < a.cols) {
      v = load_as_f32(a.x, a.x_dtype, base + c);
      if (a.residual) v += load_as_f32(a.residual, a.x_dtype, base + c);
    }
    vals[j] = v;
    sum += v;
  }
  if (!cached) {
    for (int64_t c = lane; c < a.cols; c += 64) {
      float v = load_as_f32(a.x, a.x_dtype, base + c);
      if (a.residual) v += load_as_f32(a.residual, a.x_dtype, base + c);
      sum += v;
    }
  }
  const float mean = wave_sum(sum) / static_cast<float>(a.cols);
  float sq = 0.0f;
  if (cached) {
#pragma unroll
    for (int j = 0; j < kLnCache; ++j) {
      int64_t c = lane + 64 * j;
      if (c < a.cols) { float d = vals[j] - mean; sq += d * d; }
    }
  } else {
    for (int64_t c = lane; c < a.cols; c += 64) {
      float v = load_as_f32(a.x, a.x_dtype, base + c);
      if (a.residual) v += load_as_f32(a.residual, a.x_dtype, base + c);
      float d = v - mean;
      sq += d * d;
    }
  }
  const float var = wave_sum(sq) / static_cast<float>(a.cols);
  const float inv_std = 1.0f / sqrtf(var + a.epsilon);
  if (cached) {
#pragma unroll
    for (int j = 0; j < kLnCache; ++j) {
      int64_t c = lane + 64 * j;
      if (c < a.cols) {
        float y = (vals[j] - mean) * inv_std * scale[c];
        if (bias) y += bias[c];
        store_from_f32(a.out, a.out_dtype, base + c, y);
      }
    }
  } else {
    for (int64_t c = lane; c < a.cols; c += 64) {
      float v = load_as_f32(a.x, a.x_dtype, base + c);
      if (a.residual) v += load_as_f32(a.residual, a.x_dtype, base + c);
      float y = (v - mean) * inv_std * scale[c];
      if (bias) y += bias[c];
      store_from_f32(a.out, a.out_dtype, base + c, y);
    }
  }
  if (lane == 0) {
    if (a.mean_out) static_cast<float*>(a.mean_out)[row] = mean;
    if (a.invstd_out) static_cast<float*>(a.invstd_out)[row] = inv_std;
  }
}

// Vectorized LayerNorm: each wave normalizes ROWS consecutive rows, VW (8
// or 4) consecutive columns per lane per vector (16- or 8-byte loads of
// 16-bit data), NV vectors per lane per row kept in registers.  Every row's
// loads are issued before the first reduction, so a wave has ROWS * NV loads
// in flight.  Statistics in fp32: mean, then the biased variance of the
// centred values, as layernorm_kernel.  cols % VW == 0, cols <= 64 * VW * NV.
//
// TO = int8_t: the QuantizeLinear that is the LayerNorm's only consumer, in
// the same pass.  Each output is first rounded to the activation type TX
// (what the unfused LayerNorm stores), then q = saturate(rne(y / out_scale)
// + out_zero) by the same QuantDiv as quantize_kernel: bit-identical codes.
constexpr int kLnVec = 8;

// VW consecutive elements of TX as raw 32-bit words (8, 16 or 32 bytes).
template <typename TX, int VW>
struct LnRaw {
  static constexpr int W = VW * static_cast<int>(sizeof(TX)) / 4;
  uint32_t w[W];
  __device__ __forceinline__ void load(const TX* p) {
    if constexpr (W == 2) {
      const uint2 q = *reinterpret_cast<const uint2*>(p);
      w[0] = q.x; w[1] = q.y;
    } else {
#pragma unroll
      for (int i = 0; i < W / 4; ++i) {
        const uint4 q = reinterpret_cast<const uint4*>(p)[i];
        w[4 * i] = q.x; w[4 * i + 1] = q.y; w[4 * i + 2] = q.z; w[4 * i + 3] = q.w;
      }
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = 0u;
  }
  __device__ __forceinline__ void to_f32(float* v) const {
    if constexpr (sizeof(TX) == 4) {
#pragma unroll
      for (int i = 0; i < W; ++i) v[i] = __uint_as_float(w[i]);
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) {
        v[2 * i] = Elem<TX>::to_f32(TX{static_cast<uint16_t>(w[i] & 0xffffu)});
        v[2 * i + 1] = Elem<TX>::to_f32(TX{static_cast<uint16_t>(w[i] >> 16)});
      }
    }
  }
};

template <typename TX, typename TO>
struct LnStore {
  static __device__ __forceinline__ void store8(TO* p, const float* y, const QuantDiv&, int) {
    Elem<TO>::store8(p, y);
  }
  static __device__ __forceinline__ void store4(TO* p, const float* y, const QuantDiv&, int) {
    Elem<TO>::store4(p, y);
  }
};
template <typename TX>
struct LnStore<TX, int8_t> {
  // y rounded to TX, the value c3h_quantize would read back
  static __device__ __forceinline__ float stored(float y) {
    if constexpr (std::is_same<TX, bf16_t>::value) return bf16_round(y);
    else return Elem<TX>::to_f32(Elem<TX>::from_f32(y));
  }
  static __device__ __forceinline__ void store8(int8_t* p, const float* y, const QuantDiv& qd, int qz) {
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = stored(y[e]);
    *reinterpret_cast<uint2*>(p) = qd.codes8(r, qz);
  }
  static __device__ __forceinline__ void store4(int8_t* p, const float* y, const QuantDiv& qd, int qz) {
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = stored(y[e]);
    *reinterpret_cast<uint32_t*>(p) = qd.codes4(r, qz);
  }
};

// FULL: cols == 64 * VW * NV (512 columns at VW = 8, 768 at three 4-wide
// vectors): every lane's every vector is in range, so the kernel has no
// per-vector bounds branches and no zero-filled registers.
template <typename TX, typename TO, int NV, int ROWS, int VW = kLnVec, bool FULL = false>
__global__ void __launch_bounds__(kBlock) layernorm_vec_kernel(c3h_layernorm_args a, QuantDiv qd) {
  static_assert(VW == 8 || VW == 4, "vector width");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + wave) * ROWS;
  if (row0 >= a.rows) return;
  const int nvec = FULL ? 64 * NV : static_cast<int>(a.cols / VW);
  // The affine parameters are the same for every row: loaded first, so their
  // latency overlaps the row loads and reductions instead of following them.
  const float* scale = static_cast<const float*>(a.scale);
  const float* bias = static_cast<const float*>(a.bias);
  float g[NV][VW], b[NV][VW];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lane + 64 * j;
    // no bias: -0, the identity of fmaf(t, g, b) (so that t * g is rounded once either way)
#pragma unroll
    for (int e = 0; e < VW; ++e) b[j][e] = -0.0f;
    if constexpr (!FULL) {
#pragma unroll
      for (int e = 0; e < VW; ++e) g[j][e] = 0.0f;
    }
    if (FULL || vi < nvec) {
      if constexpr (VW == 8) {
        Elem<float>::load8(scale + vi * 8, g[j]);
        if (bias) Elem<float>::load8(bias + vi * 8, b[j]);
      } else {
        Elem<float>::load4(scale + vi * 4, g[j]);
        if (bias) Elem<float>::load4(bias + vi * 4, b[j]);
      }
    }
  }
  // Every vector of the wave's rows (and of the residual) is loaded as raw
  // words before any is converted, so all the loads are in flight together
  // (converting each as it lands put a wait between consecutive loads).
  typedef LnRaw<TX, VW> Raw;
  Raw xr[ROWS][NV], rr[ROWS][NV];
  const bool has_res = a.residual != nullptr;
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const int64_t row = row0 + r;
    const TX* x = static_cast<const TX*>(a.x) + row * a.cols;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vi = lane + 64 * j;
      if (row < a.rows && (FULL || vi < nvec)) xr[r][j].load(x + vi * VW);
      else xr[r][j].zero();
    }
  }
  if (has_res) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const int64_t row = row0 + r;
      const TX* res = static_cast<const TX*>(a.residual) + row * a.cols;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int vi = lane + 64 * j;
        if (row < a.rows && (FULL || vi < nvec)) rr[r][j].load(res + vi * VW);
        else rr[r][j].zero();
      }
    }
  }
  float v[ROWS][NV][VW];
#pragma unroll
  for (int r = 0; r < ROWS; ++r)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      xr[r][j].to_f32(v[r][j]);
      if (has_res) {
        float q[VW];
        rr[r][j].to_f32(q);
#pragma unroll
        for (int e = 0; e < VW; ++e) v[r][j][e] += q[e];
      }
    }
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const int64_t row = row0 + r;
    if (row >= a.rows) break;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < VW; ++e) sum += v[r][j][e];  // out-of-range vectors hold zeros
    const float mean = wave_sum(sum) / static_cast<float>(a.cols);
    // The centred values replace the inputs: the affine pass reuses them.
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (FULL || lane + 64 * j < nvec) {
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          const float d = v[r][j][e] - mean;
          v[r][j][e] = d;
          sq += d * d;
        }
      }
    }
    const float var = wave_sum(sq) / static_cast<float>(a.cols);
    const float inv_std = 1.0f / sqrtf(var + a.epsilon);
    TO* out = static_cast<TO*>(a.out) + row * a.cols;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vi = lane + 64 * j;
      if (FULL || vi < nvec) {
        float y[VW];
#pragma unroll
        for (int e = 0; e < VW; ++e) y[e] = fmaf(v[r][j][e] * inv_std, g[j][e], b[j][e]);  // (x - mean) * inv_std * scale + bias
        if constexpr (VW == 8) LnStore<TX, TO>::store8(out + vi * 8, y, qd, a.out_zero);
        else LnStore<TX, TO>::store4(out + vi * 4, y, qd, a.out_zero);
      }
    }
    if (lane == 0) {
      if (a.mean_out) static_cast<float*>(a.mean_out)[row] = mean;
      if (a.invstd_out) static_cast<float*>(a.invstd_out)[row] = inv_std;
    }
  }
}

// ------------------------------------------------------------------ batchnorm / fold
__global__ void batchnorm_kernel(c3h_batchnorm_args a) {
  int64_t total = a.n * a.c * a.hw;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const float* x = static_cast<const float*>(a.x);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t ch = (i / a.hw) % a.c;
    float sc = static_cast<const float*>(a.scale)[ch];
    float bi = static_cast<const float*>(a.bias)[ch];
    float mu = static_cast<const float*>(a.mean)[ch];
    float va = static_cast<const float*>(a.var)[ch];
    static_cast<float*>(a.out)[i] = (x[i] - mu) / sqrtf(va + a.epsilon) * sc + bi;
  }
}

__global__ void bn_fold_kernel(c3h_bnfold_args a) {
  int64_t total = a.out_channels * a.per_channel;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t o = i / a.per_channel;
    float f = a.scale[o] / sqrtf(a.var[o] + a.epsilon);
    a.w_out[i] = a.w[i] * f;
    if (i - o * a.per_channel == 0) {
      float cb = a.conv_bias ? a.conv_bias[o] : 0.0f;
      a.b_out[o] = (cb - a.mean[o]) * f + a.bias[o];
    }
  }
}

// ------------------------------------------------------------------ gather
// One thread per 16-byte chunk (or element when rows are not 16B multiples).
template <typename V>
__global__ void __launch_bounds__(kBlock) gather_kernel(c3h_gather_args a, int64_t row_vecs) {
  int64_t total = a.outer * a.n_indices * row_vecs;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const V* data = static_cast<const V*>(a.data);
  V* out = static_cast<V*>(a.out);
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    int64_t v = t % row_vecs;
    int64_t r = t / row_vecs;
    int64_t i = r % a.n_indices;
    int64_t o = r / a.n_indices;
    int64_t idx = a.indices[i];
    if (idx < 0) idx += a.axis_dim;
    if (idx < 0 || idx >= a.axis_dim) {
      if (a.error_flag) *a.error_flag = 1;
      out[t] = V{};
      continue;
    }
    out[t] = data[(o * a.axis_dim + idx) * row_vecs + v];
  }
}

// Gather with a fused per-row addend (token + positional embedding): one
// thread per 8 elements of a row, 16-byte (16-bit) or 32-byte (fp32) loads
// of the gathered row and the addend row (TA: fp32, or the data type), fp32
// add, one rounding, one vector store.  Consecutive threads take consecutive
// chunks of a row, so loads and stores are coalesced; the index is read once
// per chunk from L1.
// Each thread takes kGatherU chunks per iteration (t0, t0 + stride, ...),
// issued together: all index loads, then all row and addend loads, then the
// stores, so a thread has kGatherU independent index -> row chains in flight.
constexpr int kGatherU = 4;
template <typename T, typename TA>
__global__ void __launch_bounds__(kBlock) gather_add_kernel(c3h_gather_args a, int64_t row_vecs) {
  const int64_t total = a.n_indices * row_vecs;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const T* data = static_cast<const T*>(a.data);
  const TA* add = static_cast<const TA*>(a.addend);
  T* out = static_cast<T*>(a.out);
  for (int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t0 < total;
       t0 += stride * kGatherU) {
    int64_t r[kGatherU], c[kGatherU], idx[kGatherU];
#pragma unroll
    for (int u = 0; u < kGatherU; ++u) {
      const int64_t t = t0 + u * stride;
      r[u] = t < total ? t / row_vecs : 0;
      c[u] = (t - r[u] * row_vecs) * 8;
      idx[u] = t < total ? a.indices[r[u]] : 0;
    }
    float v[kGatherU][8], w[kGatherU][8];
#pragma unroll
    for (int u = 0; u < kGatherU; ++u) {
      if (idx[u] < 0) idx[u] += a.axis_dim;
      const bool ok = idx[u] >= 0 && idx[u] < a.axis_dim;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[u][e] = w[u][e] = 0.0f;
      if (t0 + u * stride < total && ok) {
        Elem<T>::load8(data + idx[u] * a.inner + c[u], v[u]);
        Elem<TA>::load8(add + (r[u] % a.addend_rows) * a.inner + c[u], w[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kGatherU; ++u) {
      if (t0 + u * stride >= total) break;
      if (idx[u] < 0 || idx[u] >= a.axis_dim) {
        // out-of-range index: a zero row and the error flag
        if (a.error_flag) *a.error_flag = 1;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[u][e] += w[u][e];
      }
      Elem<T>::store8(out + r[u] * a.inner + c[u], v[u]);
    }
  }
}

// ------------------------------------------------------------------ finiteness
// Any NaN / Inf among `count` values: 16-byte loads, an exponent-all-ones
// test per element, and one plain store of 1 per wave that found one (every
// writer stores the same value, so no atomic is needed).
template <typename T>
__global__ void __launch_bounds__(kBlock) nonfinite_kernel(const T* __restrict__ x, int64_t count,
                                                           int32_t* __restrict__ flag) {
  constexpr int PER = 16 / static_cast<int>(sizeof(T));
  const int64_t nvec = count / PER;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  bool bad = false;
  for (int64_t i = t0; i < nvec; i += stride) {
    const uint4 q = reinterpret_cast<const uint4*>(x)[i];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (sizeof(T) == 4) bad |= (w[k] & 0x7f800000u) == 0x7f800000u;
      else if constexpr (std::is_same<T, bf16_t>::value)
        bad |= ((w[k] & 0x7f80u) == 0x7f80u) | ((w[k] & 0x7f800000u) == 0x7f800000u);
      else bad |= ((w[k] & 0x7c00u) == 0x7c00u) | ((w[k] & 0x7c000000u) == 0x7c000000u);
    }
  }
  for (int64_t i = nvec * PER + t0; i < count; i += stride) {  // the last < PER elements
    float v;
    if constexpr (sizeof(T) == 4) v = x[i];
    else v = Elem<T>::to_f32(x[i]);
    bad |= !isfinite(v);
  }
  if (__ballot(bad) != 0 && (threadIdx.x & 63) == 0) *flag = 1;
}

// ------------------------------------------------------------------ argmax
// One 256-thread block per row; NaN counts as the maximum (NumPy rule) and
// ties resolve to the lowest index.
__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  bool vn = v != v, bn = bv != bv;
  if (vn || bn) {
    if (vn && bn) return i < bi;
    return vn;
  }
  return v > bv || (v == bv && i < bi);
}

template <bool kVec>
__global__ void __launch_bounds__(kBlock) argmax_kernel(c3h_argmax_args a) {
  __shared__ float sv[kBlock];
  __shared__ int64_t si[kBlock];
  int64_t row = blockIdx.x;
  const int64_t base = row * a.cols;
  float bv = -INFINITY;
  int64_t bi = a.cols;  // sentinel above every real index
  if (kVec) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.in) + base);
    for (int64_t c4 = threadIdx.x; c4 < a.cols / 4; c4 += kBlock) {
      float4 v = p[c4];
      int64_t c = c4 * 4;
      if (better(v.x, c, bv, bi)) { bv = v.x; bi = c; }
      if (better(v.y, c + 1, bv, bi)) { bv = v.y; bi = c + 1; }
      if (better(v.z, c + 2, bv, bi)) { bv = v.z; bi = c + 2; }
      if (better(v.w, c + 3, bv, bi)) { bv = v.w; bi = c + 3; }
    }
  } else {
    for (int64_t c = threadIdx.x; c < a.cols; c += kBlock) {
      float v = load_as_f32(a.in, a.in_dtype, base + c);
      if (better(v, c, bv, bi)) { bv = v; bi = c; }
    }
  }
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int s = kBlock / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      float ov = sv[threadIdx.x + s];
      int64_t oi = si[threadIdx.x + s];
      if (better(ov, oi, sv[threadIdx.x], si[threadIdx.x])) { sv[threadIdx.x] = ov; si[threadIdx.x] = oi; }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) a.out[row] = si[0] < a.cols ? si[0] : 0;
}

// ArgMax finish from a GEMM epilogue's row_max side output (the maximum of
// each 64-column block, NaN ignored, and a may-hold-NaN flag): one wave per
// row.  The largest block maximum mx is the row's largest non-NaN value, and
// the answer is the first column equal to mx -- in the first block whose
// maximum equals mx, read once (one column per lane) -- unless the row holds
// a NaN: then the NaN-flagged blocks are read first, in order (a flag can
// also come from an infinity; such a block holds no NaN and the search moves
// on).  c3h_argmax's rule: NaN is the maximum, the first column on ties.
// Every branch and loop below depends only on wave-wide values (ballots).
// NP > 0: n_parts <= 64 * NP, and lane l keeps blocks l, l + 64, ... in
// registers: its NP loads are issued together and the parts are read once
// (a loop with one load per iteration left the load latency exposed per
// iteration, twice).  NP == 0: any width, the parts are re-read.
template <int NP>
__global__ void __launch_bounds__(kBlock) argmax_finish_kernel(c3h_argmax_finish_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // per wave
  const c3h_block_max* p = a.parts + row * a.ld;
  float mx = -INFINITY;
  int flag = 0;
  float pmax[NP > 0 ? NP : 1];
  uint32_t pnan = 0u;  // bit t: block lane + 64 t may hold a NaN
  if constexpr (NP > 0) {
#pragma unroll
    for (int t = 0; t < NP; ++t) {
      const int64_t j = lane + 64 * t;
      c3h_block_max q = {-INFINITY, 0};
      if (j < a.n_parts) q = p[j];
      pmax[t] = q.max;
      pnan |= (q.nan != 0 ? 1u : 0u) << t;
    }
#pragma unroll
    for (int t = 0; t < NP; ++t) mx = fmaxf(mx, pmax[t]);
    flag = pnan != 0u;
  } else {
    for (int64_t j = lane; j < a.n_parts; j += 64) {
      const c3h_block_max q = p[j];
      mx = fmaxf(mx, q.max);
      flag |= q.nan;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    flag |= __shfl_xor(flag, o, 64);
  }
  const int64_t base = row * a.in_ld;
  int64_t ans = -1;
  // NP > 0: register t holds block 64 t + lane, so candidate round t is j0 = 64 t.
  auto nan_cand = [&](int64_t j0) -> bool {
    if constexpr (NP > 0) return j0 + lane < a.n_parts && ((pnan >> (j0 / 64)) & 1u) != 0u;
    else return j0 + lane < a.n_parts && p[j0 + lane].nan != 0;
  };
  auto max_cand = [&](int64_t j0) -> bool {
    if constexpr (NP > 0) {
      float v = -INFINITY;
#pragma unroll
      for (int t = 0; t < NP; ++t) v = (j0 == 64 * t) ? pmax[t] : v;
      return j0 + lane < a.n_parts && v == mx;
    } else {
      return j0 + lane < a.n_parts && p[j0 + lane].max == mx;
    }
  };
  if (flag) {
    for (int64_t j0 = 0; j0 < a.n_parts && ans < 0; j0 += 64) {
      uint64_t cand = __ballot(nan_cand(j0));
      while (cand != 0 && ans < 0) {
        const int64_t blk = j0 + __builtin_ctzll(cand);
        cand &= cand - 1;
        const int64_t col = blk * 64 + lane;
        const float x = col < a.cols ? load_as_f32(a.in, a.in_dtype, base + col) : 0.0f;
        const uint64_t hit = __ballot(x != x);
        if (hit != 0) ans = blk * 64 + __builtin_ctzll(hit);
      }
    }
  }
  for (int64_t j0 = 0; j0 < a.n_parts && ans < 0; j0 += 64) {
    uint64_t cand = __ballot(max_cand(j0));
    while (cand != 0 && ans < 0) {
      const int64_t blk = j0 + __builtin_ctzll(cand);
      cand &= cand - 1;
      const int64_t col = blk * 64 + lane;
      const float x = col < a.cols ? load_as_f32(a.in, a.in_dtype, base + col) : NAN;
      const uint64_t hit = __ballot(x == mx);
      if (hit != 0) ans = blk * 64 + __builtin_ctzll(hit);
    }
  }
  if (lane == 0) a.out[row] = ans < 0 ? 0 : ans;
}

// ------------------------------------------------------------------ im2col
__global__ void __launch_bounds__(kBlock) im2col_kernel(c3h_im2col_args a) {
  const int64_t cols = static_cast<int64_t>(a.c) * a.kh * a.kw;
  const int64_t total = static_cast<int64_t>(a.n) * a.ho * a.wo * cols;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    int64_t col = t % cols, row = t / cols;
    int kw_i = static_cast<int>(col % a.kw);
    int kh_i = static_cast<int>((col / a.kw) % a.kh);
    int ci = static_cast<int>(col / (static_cast<int64_t>(a.kw) * a.kh));
    int wo_i = static_cast<int>(row % a.wo);
    int ho_i = static_cast<int>((row / a.wo) % a.ho);
    int ni = static_cast<int>(row / (static_cast<int64_t>(a.wo) * a.ho));
    int hi = ho_i * a.sh - a.pad_top + kh_i * a.dh;
    int wi = wo_i * a.sw - a.pad_left + kw_i * a.dw;
    float v = 0.0f;
    if (hi >= 0 && hi < a.h && wi >= 0 && wi < a.w)
      v = load_as_f32(a.x, a.dtype, ((static_cast<int64_t>(ni) * a.c + ci) * a.h + hi) * a.w + wi);
    store_from_f32(a.out, a.dtype, t, v);
  }
}

// ------------------------------------------------------------------ layout NCHW <-> NHWC
// Small-channel path: one thread per pixel, channels (padded) in order.
__global__ void __launch_bounds__(kBlock) nchw_to_nhwc_small_kernel(c3h_layout_args a) {
  const int64_t hw = static_cast<int64_t>(a.h) * a.w;
  const int64_t total = static_cast<int64_t>(a.n) * hw;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < total; p += stride) {
    int64_t ni = p / hw, s = p - ni * hw;
    for (int c = 0; c < a.c_pad; ++c) {
      float v = c < a.c ? load_as_f32(a.in, a.in_dtype, (ni * a.c + c) * hw + s) : 0.0f;
      store_from_f32(a.out, a.out_dtype, p * a.c_pad + c, v);
    }
  }
}

// NCHW fp32 -> NHWC with c_pad == 4 (network inputs: 3 channels padded to 4),
// four consecutive pixels per thread: one float4 load per channel plane and
// 4 pixels x 4 channels of output written as whole 16-byte vectors.
template <typename TO>
__global__ void __launch_bounds__(kBlock) nchw_to_nhwc_c4_kernel(c3h_layout_args a) {
  const int64_t hw = static_cast<int64_t>(a.h) * a.w;
  const int64_t quads = static_cast<int64_t>(a.n) * (hw / 4);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const float* in = static_cast<const float*>(a.in);
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < quads; q += stride) {
    const int64_t ni = q / (hw / 4), s = (q - ni * (hw / 4)) * 4;
    float px[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float4 v = float4{0.f, 0.f, 0.f, 0.f};
      if (c < a.c) v = *reinterpret_cast<const float4*>(in + (ni * a.c + c) * hw + s);
      px[0][c] = v.x; px[1][c] = v.y; px[2][c] = v.z; px[3][c] = v.w;
    }
    TO* out = static_cast<TO*>(a.out) + (ni * hw + s) * 4;
#pragma unroll
    for (int p = 0; p < 4; p += 16 / (4 * static_cast<int>(sizeof(TO)))) {
      float v[16 / sizeof(TO)];
#pragma unroll
      for (int e = 0; e < static_cast<int>(16 / sizeof(TO)); ++e) v[e] = px[p + e / 4][e % 4];
      store_vec16(out + p * 4, v);
    }
  }
}

// Tiled path: per image, [C][HW] <-> [HW][Cpad] through a 32x33 LDS tile.
__global__ void __launch_bounds__(256) layout_tile_kernel(c3h_layout_args a) {
  __shared__ float tile[32][33];
  const int64_t hw = static_cast<int64_t>(a.h) * a.w;
  int64_t ni = blockIdx.z;
  int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  if (a.direction == 0) {  // NCHW -> NHWC: tile over (c, s)
    int64_t s0 = static_cast<int64_t>(blockIdx.x) * 32, c0 = static_cast<int64_t>(blockIdx.y) * 32;
    for (int k = ty; k < 32; k += 8) {
      int64_t c = c0 + k, s = s0 + tx;
      tile[k][tx] = (c < a.c && s < hw) ? load_as_f32(a.in, a.in_dtype, (ni * a.c + c) * hw + s) : 0.0f;
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
      int64_t s = s0 + k, c = c0 + tx;
      if (s < hw && c < a.c_pad) store_from_f32(a.out, a.out_dtype, (ni * hw + s) * a.c_pad + c, tile[tx][k]);
    }
  } else {  // NHWC(c_pad) -> NCHW
    int64_t s0 = static_cast<int64_t>(blockIdx.x) * 32, c0 = static_cast<int64_t>(blockIdx.y) * 32;
    for (int k = ty; k < 32; k += 8) {
      int64_t s = s0 + k, c = c0 + tx;
      tile[k][tx] = (s < hw && c < a.c) ? load_as_f32(a.in, a.in_dtype, (ni * hw + s) * a.c_pad + c) : 0.0f;
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
      int64_t c = c0 + k, s = s0 + tx;
      if (c < a.c && s < hw) store_from_f32(a.out, a.out_dtype, (ni * a.c + c) * hw + s, tile[tx][k]);
    }
  }
}

// ------------------------------------------------------------------ weight packing
__global__ void __launch_bounds__(kBlock) pack_conv_weight_kernel(c3h_pack_args a) {
  const int64_t total = static_cast<int64_t>(a.o) * a.k_stride;
  const int64_t k_real = static_cast<int64_t>(a.kh) * a.kw_pack * a.c_pack;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    int64_t o = t / a.k_stride, k = t - o * a.k_stride;
    float v = 0.0f;
    if (k < k_real) {
      int c = static_cast<int>(k % a.c_pack);
      int tap = static_cast<int>(k / a.c_pack);
      int kwi = tap % a.kw_pack, khi = tap / a.kw_pack;
      if (c < a.c && kwi < a.kw)
        v = load_as_f32(a.w, a.in_dtype, ((o * a.c + c) * a.kh + khi) * a.kw + kwi);
    }
    store_from_f32(a.out, a.out_dtype, t, v);
  }
}

// ------------------------------------------------------------------ maxpool
__global__ void __launch_bounds__(kBlock) maxpool_kernel(c3h_pool_args a) {
  const int64_t total = static_cast<int64_t>(a.n) * a.c * a.ho * a.wo;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    int ci, wo_i, ho_i, ni;
    if (a.layout == 1) {  // NHWC: channel fastest
      ci = static_cast<int>(t % a.c);
      int64_t p = t / a.c;
      wo_i = static_cast<int>(p % a.wo);
      ho_i = static_cast<int>((p / a.wo) % a.ho);
      ni = static_cast<int>(p / (static_cast<int64_t>(a.wo) * a.ho));
    } else {
      wo_i = static_cast<int>(t % a.wo);
      ho_i = static_cast<int>((t / a.wo) % a.ho);
      ci = static_cast<int>((t / (static_cast<int64_t>(a.wo) * a.ho)) % a.c);
      ni = static_cast<int>(t / (static_cast<int64_t>(a.wo) * a.ho * a.c));
    }
    float m = -INFINITY;
    for (int i = 0; i < a.kh; ++i) {
      int hi = ho_i * a.sh - a.pad_top + i * a.dh;
      if (hi < 0 || hi >= a.h) continue;
      for (int j = 0; j < a.kw; ++j) {
        int wi = wo_i * a.sw - a.pad_left + j * a.dw;
        if (wi < 0 || wi >= a.w) continue;
        int64_t off = a.layout == 1
                          ? ((static_cast<int64_t>(ni) * a.h + hi) * a.w + wi) * a.c_stride + ci
                          : ((static_cast<int64_t>(ni) * a.c + ci) * a.h + hi) * a.w + wi;
        m = fmaxf(m, load_as_f32(a.x, a.dtype, off));
      }
    }
    int64_t o = a.layout == 1
                    ? ((static_cast<int64_t>(ni) * a.ho + ho_i) * a.wo + wo_i) * a.c_stride + ci
                    : t;
    store_from_f32(a.out, a.dtype, o, m);
  }
}

// ------------------------------------------------------------------ quantize / dequantize
__global__ void quantize_kernel(c3h_quantize_args a) {
  const QuantDiv qd(a.scale);
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < a.count; i += stride) {
    a.out[i] = qd.code(load_as_f32(a.x, a.x_dtype, i), a.zero_point);
  }
}

// 8 elements per thread: one 16-byte (16-bit input) or 32-byte (fp32) load,
// one 8-byte int8 store; the same QuantDiv codes as quantize_kernel.
template <typename TX>
__global__ void __launch_bounds__(kBlock) quantize_vec_kernel(c3h_quantize_args a, QuantDiv qd) {
  const int64_t nvec = a.count / 8;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const TX* x = static_cast<const TX*>(a.x);
  // two vectors per iteration, both loads issued before either is quantized
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nvec; i += 2 * stride) {
    const int64_t i2 = i + stride;
    float v[8], v2[8];
    Elem<TX>::load8(x + i * 8, v);
    if (i2 < nvec) Elem<TX>::load8(x + i2 * 8, v2);
    *reinterpret_cast<uint2*>(a.out + i * 8) = qd.codes8(v, a.zero_point);
    if (i2 < nvec) *reinterpret_cast<uint2*>(a.out + i2 * 8) = qd.codes8(v2, a.zero_point);
  }
}

// Row-wise E4M3 quantization (c3h_quantize_fp8_rows): one wave per row.
// NV > 0: the row (cols <= 512 NV) stays in registers between the amax pass
// and the encode pass; NV == 0: any width, the encode pass re-reads the row
// (from L2).  Encoding: v_cvt_pk_fp8_f32 (round to nearest even) of values
// clamped to +-448 first, four codes packed little-endian per 32-bit word.
__device__ __forceinline__ uint2 fp8_encode8(const float* v, float inv) {
  float q[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) q[e] = fminf(fmaxf(v[e] * inv, -448.0f), 448.0f);
  int w0 = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  w0 = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], w0, true);
  int w1 = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
  w1 = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], w1, true);
  return uint2{static_cast<uint32_t>(w0), static_cast<uint32_t>(w1)};
}

template <typename TX, int NV>
__global__ void __launch_bounds__(kBlock) quantize_fp8_rows_kernel(c3h_fp8_quant_args a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + wave;
  if (row >= a.rows) return;
  const int64_t nvec = a.cols / 8;
  const TX* x = static_cast<const TX*>(a.x) + row * a.ldx;
  uint8_t* out = a.out + row * a.ldo;
  constexpr int R = NV > 0 ? NV : 1;
  float v[R][8];
  float amax = 0.0f;
  bool bad = false;
  auto scan = [&](const float* t) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float m = fabsf(t[e]);
      bad |= !(m <= 3.402823466e38f);  // Inf or NaN
      amax = fmaxf(amax, m);
    }
  };
  if constexpr (NV > 0) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t vi = lane + 64 * j;
      if (vi < nvec) {
        load_vec16(x + vi * 8, v[j]);
        if constexpr (sizeof(TX) == 4) load_vec16(x + vi * 8 + 4, v[j] + 4);
        scan(v[j]);
      }
    }
  } else {
    for (int64_t vi = lane; vi < nvec; vi += 64) {
      load_vec16(x + vi * 8, v[0]);
      if constexpr (sizeof(TX) == 4) load_vec16(x + vi * 8 + 4, v[0] + 4);
      scan(v[0]);
    }
  }
  amax = wave_max(amax);
  bad = __any(bad);
  const float inv = amax > 0.0f ? fminf(448.0f / amax, 3.402823466e38f) : 0.0f;
  const uint2 nan8 = uint2{0x7f7f7f7fu, 0x7f7f7f7fu};
  if constexpr (NV > 0) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t vi = lane + 64 * j;
      if (vi < nvec) *reinterpret_cast<uint2*>(out + vi * 8) = bad ? nan8 : fp8_encode8(v[j], inv);
    }
  } else {
    for (int64_t vi = lane; vi < nvec; vi += 64) {
      load_vec16(x + vi * 8, v[0]);
      if constexpr (sizeof(TX) == 4) load_vec16(x + vi * 8 + 4, v[0] + 4);
      *reinterpret_cast<uint2*>(out + vi * 8) = bad ? nan8 : fp8_encode8(v[0], inv);
    }
  }
  if (lane == 0) a.scale[row] = bad ? __builtin_nanf("") : amax / 448.0f;
}

// MXFP4 block quantization (c3h_quantize_mxfp4): one thread per block of 32
// columns of one row.  Weights are quantized once per compiled plan, so the
// kernel favours plain arithmetic over bandwidth: the exponent comes from
// ilogbf (floor(log2 amax), subnormals included) and the element code from
// comparisons against the round-to-nearest-even boundaries of the E2M1
// magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6 (ties 0.25, 1.25, 2.5 and 5 go down
// to the even code, ties 0.75, 1.75 and 3.5 up), saturating above 5.
__device__ __forceinline__ uint32_t e2m1_code(float x, float inv) {
  const float m = fabsf(x) * inv;
  const uint32_t c = m <= 0.25f ? 0u : m < 0.75f ? 1u : m <= 1.25f ? 2u : m < 1.75f ? 3u
                   : m <= 2.5f ? 4u : m < 3.5f ? 5u : m <= 5.0f ? 6u : 7u;
  return (c != 0u && x < 0.0f) ? (c | 8u) : c;
}

__global__ void __launch_bounds__(kBlock) quantize_mxfp4_kernel(c3h_mxfp4_quant_args a) {
  const int64_t nblk = a.cols / 32;
  const int64_t id = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (id >= a.rows * nblk) return;
  const int64_t row = id / nblk, blk = id - row * nblk;
  const int64_t x0 = row * a.ldx + blk * 32;
  float v[32];
  float amax = 0.0f;
  bool bad = false;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    v[e] = load_as_f32(a.x, a.x_dtype, x0 + e);
    const float m = fabsf(v[e]);
    bad |= !(m <= 3.402823466e38f);  // Inf or NaN
    amax = fmaxf(amax, m);
  }
  int ex = -13;
  if (amax > 0.0f) ex = min(max(ilogbf(amax) - 2, -13), 13);
  const float inv = __uint_as_float(static_cast<uint32_t>(127 - ex) << 23);  // 2^-ex
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t word = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) word |= (bad ? 0u : e2m1_code(v[8 * j + e], inv)) << (4 * e);
    w[j] = word;
  }
  *reinterpret_cast<uint4*>(a.codes + row * a.ldc + blk * 16) = uint4{w[0], w[1], w[2], w[3]};
  a.scales[row * a.lds + blk] = bad ? uint8_t{0xFF} : static_cast<uint8_t>(ex + 127);
}

template <typename TX>
int launch_fp8_rows(const c3h_fp8_quant_args& a, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(ceil_div(a.rows, kBlock / 64))), b(kBlock);
  const int64_t nvec = a.cols / 8;
  if (nvec <= 64) hipLaunchKernelGGL((quantize_fp8_rows_kernel<TX, 1>), g, b, 0, s, a);
  else if (nvec <= 128) hipLaunchKernelGGL((quantize_fp8_rows_kernel<TX, 2>), g, b, 0, s, a);
  else if (nvec <= 256) hipLaunchKernelGGL((quantize_fp8_rows_kernel<TX, 4>), g, b, 0, s, a);
  else if (nvec <= 512) hipLaunchKernelGGL((quantize_fp8_rows_kernel<TX, 8>), g, b, 0, s, a);
  else hipLaunchKernelGGL((quantize_fp8_rows_kernel<TX, 0>), g, b, 0, s, a);
  return launch_status("quantize_fp8_rows");
}

__global__ void dequantize_kernel(c3h_dequantize_args a) {
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < a.count; i += stride)
    store_from_f32(a.out, a.out_dtype, i, static_cast<float>(static_cast<int32_t>(a.q[i]) - a.zero_point) * a.scale);
}

bool ew_is_flat(const c3h_ew_args& a) {
  // Flat iff every input is either dense in output order or a single element.
  for (int j = 0; j < a.n_in; ++j) {
    bool all_zero = true, dense = true;
    int64_t expect = 1;
    for (int d = a.rank - 1; d >= 0; --d) {
      int64_t s = a.stride[j][d];
      if (s != 0) all_zero = false;
      if (a.shape[d] != 1 && s != expect) dense = false;
      expect *= a.shape[d];
    }
    if (!(all_zero || dense)) return false;
  }
  return true;
}

// Channels-last max pool, 16 bytes of channels per thread: each of the kh*kw
// taps is one 16-byte load, the window max is taken in fp32 with the same
// fmaxf / -inf semantics as maxpool_kernel (exact for 16-bit inputs).
template <typename T>
__global__ void __launch_bounds__(kBlock) maxpool_nhwc_vec_kernel(c3h_pool_args a) {
  constexpr int V = 16 / sizeof(T);
  const int groups = a.c / V;
  const int64_t total = static_cast<int64_t>(a.n) * a.ho * a.wo * groups;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    const int g = static_cast<int>(t % groups);
    const int64_t pix = t / groups;
    const int wo_i = static_cast<int>(pix % a.wo);
    const int ho_i = static_cast<int>((pix / a.wo) % a.ho);
    const int64_t ni = pix / (static_cast<int64_t>(a.wo) * a.ho);
    float m[V];
#pragma unroll
    for (int v = 0; v < V; ++v) m[v] = -INFINITY;
    for (int i = 0; i < a.kh; ++i) {
      const int hi = ho_i * a.sh - a.pad_top + i * a.dh;
      if (hi < 0 || hi >= a.h) continue;
      for (int j = 0; j < a.kw; ++j) {
        const int wi = wo_i * a.sw - a.pad_left + j * a.dw;
        if (wi < 0 || wi >= a.w) continue;
        const T* src = static_cast<const T*>(a.x) + ((ni * a.h + hi) * a.w + wi) * a.c_stride + g * V;
        float x[V];
        load_vec16(src, x);
#pragma unroll
        for (int v = 0; v < V; ++v) m[v] = fmaxf(m[v], x[v]);
      }
    }
    T* dst = static_cast<T*>(a.out) + ((ni * a.ho + ho_i) * a.wo + wo_i) * a.c_stride + g * V;
    store_vec16(dst, m);
  }
}

// Rows per wave: 1, except 2 for the 8-wide form of 513-1024 columns (case
// 2).  One row per wave measured fastest: 16384 x 512 fp16 9.3 (4 rows) ->
// 8.1 us, 16384 x 768 bf16 -> int8 14.2 (2 rows) -> 13.0 us; more waves
// in flight hide the load latency better than more rows per wave.  Case 3
// is 768 columns as three 4-wide vectors per lane.
template <typename TX, typename TO>
void launch_ln(const c3h_layernorm_args& a, int nv, void* stream) {
  const dim3 b(kBlock);
  hipStream_t st = as_stream(stream);
  auto grid = [&](int rows_per_wave) { return dim3(static_cast<unsigned>(ceil_div(a.rows, 4 * rows_per_wave))); };
  // the values quantized are the LayerNorm outputs rounded to TX
  const QuantDiv qd = std::is_same<TO, int8_t>::value
                          ? QuantDiv::on_host(a.out_scale, a.out_zero, std::is_same<TX, float>::value ? -1 : a.x_dtype)
                          : QuantDiv::on_host(1.0f);
  switch (nv) {
    case 1:
      if (a.cols == 512) hipLaunchKernelGGL((layernorm_vec_kernel<TX, TO, 1, 1, 8, true>), grid(1), b, 0, st, a, qd);
      else hipLaunchKernelGGL((layernorm_vec_kernel<TX, TO, 1, 1>), grid(1), b, 0, st, a, qd);
      break;
    case 2: hipLaunchKernelGGL((layernorm_vec_kernel<TX, TO, 2, 2>), grid(2), b, 0, st, a, qd); break;
    case 3: hipLaunchKernelGGL((layernorm_vec_kernel<TX, TO, 3, 1, 4, true>), grid(1), b, 0, st, a, qd); break;
    case 4: hipLaunchKernelGGL((layernorm_vec_kernel<TX, TO, 4, 1>), grid(1), b, 0, st, a, qd); break;
    default: hipLaunchKernelGGL((layernorm_vec_kernel<TX, TO, 8, 1>), grid(1), b, 0, st, a, qd); break;
  }
}

}  // namespace

extern "C" {

int c3h_fill(const c3h_fill_args* a, void* stream) {
  C3H_REQUIRE(a && (a->out || a->count == 0), "fill: bad args");
  if (a->count == 0) return C3H_OK;
  C3H_REQUIRE(dtype_size(a->dtype) > 0, "fill: bad dtype %d", a->dtype);
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(a->count)), dim3(kBlock), 0, as_stream(stream), a->out, a->count,
                     a->dtype, a->value);
  return launch_status("fill");
}

int c3h_cast(const c3h_cast_args* a, void* stream) {
  C3H_REQUIRE(a && a->count >= 0, "cast: bad args");
  if (a->count == 0) return C3H_OK;
  C3H_REQUIRE(dtype_size(a->in_dtype) > 0 && dtype_size(a->out_dtype) > 0, "cast: bad dtype");
  hipLaunchKernelGGL(cast_kernel, dim3(grid_for(a->count)), dim3(kBlock), 0, as_stream(stream), a->in, a->out,
                     a->count, a->in_dtype, a->out_dtype);
  return launch_status("cast");
}

int c3h_ew(const c3h_ew_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr, "ew: null args");
  C3H_REQUIRE(a->n_in >= 1 && a->n_in <= C3H_EW_MAX_IN, "ew: n_in %d out of range", a->n_in);
  C3H_REQUIRE(a->n_inst >= 1 && a->n_inst <= C3H_EW_MAX_INST, "ew: n_inst %d out of range", a->n_inst);
  C3H_REQUIRE(a->rank >= 0 && a->rank <= C3H_MAX_RANK, "ew: rank %d out of range", a->rank);
  for (int i = 0; i < a->n_inst; ++i) {
    const c3h_ew_inst& ins = a->inst[i];
    int limit = a->n_in + i;
    C3H_REQUIRE(ins.a >= 0 && ins.a < limit && ins.b >= 0 && ins.b < limit,
                "ew: instruction %d reads register outside [0,%d)", i, limit);
    C3H_REQUIRE(ins.op >= 0 && ins.op <= C3H_EW_COPY, "ew: bad opcode %d", ins.op);
  }
  int64_t numel = 1;
  for (int d = 0; d < a->rank; ++d) {
    C3H_REQUIRE(a->shape[d] >= 0, "ew: negative extent");
    numel *= a->shape[d];
  }
  if (numel == 0) return C3H_OK;
  bool flat = ew_is_flat(*a);
  bool all_f32 = a->out_dtype == C3H_F32;
  for (int j = 0; j < a->n_in; ++j) {
    all_f32 = all_f32 && a->in_dtype[j] == C3H_F32;
    if (a->stride[j][a->rank ? a->rank - 1 : 0] && (reinterpret_cast<uintptr_t>(a->in[j]) & 15)) all_f32 = false;
  }
  if (reinterpret_cast<uintptr_t>(a->out) & 15) all_f32 = false;
  c3h_ew_args k = *a;
  if (flat) {
    // Normalize flat strides to a 0/1 flag in slot 0.
    for (int j = 0; j < k.n_in; ++j) {
      bool any = false;
      for (int d = 0; d < k.rank; ++d) any = any || k.stride[j][d] != 0;
      k.stride[j][0] = any ? 1 : 0;
    }
    if (all_f32 && (numel & 3) == 0) {
      hipLaunchKernelGGL(ew_flat_f32x4_kernel, dim3(grid_for(numel / 4)), dim3(kBlock), 0, as_stream(stream), k,
                         numel / 4);
      return launch_status("ew_flat_f32x4");
    }
    hipLaunchKernelGGL(ew_kernel<true>, dim3(grid_for(numel)), dim3(kBlock), 0, as_stream(stream), k, numel);
    return launch_status("ew_flat");
  }
  hipLaunchKernelGGL(ew_kernel<false>, dim3(grid_for(numel)), dim3(kBlock), 0, as_stream(stream), k, numel);
  return launch_status("ew");
}

int c3h_strided_copy(const c3h_copy_args* a, void* stream) {
  C3H_REQUIRE(a && a->rank >= 0 && a->rank <= C3H_MAX_RANK, "strided_copy: bad rank");
  int64_t total = 1;
  for (int d = 0; d < a->rank; ++d) total *= a->shape[d];
  if (total == 0) return C3H_OK;
  hipStream_t s = as_stream(stream);
  // Tiled transpose when the output's innermost dim is strided on the input
  // and the second-innermost dim is unit-stride on the input.
  if (a->rank >= 2 && a->in_stride[a->rank - 1] != 1 && a->in_stride[a->rank - 2] == 1 &&
      a->in_stride[a->rank - 1] == a->shape[a->rank - 2] && a->in_offset == 0) {
    int64_t rows = a->shape[a->rank - 2], cols = a->shape[a->rank - 1];
    int64_t batch = total / (rows * cols);
    bool batch_dense = true;
    int64_t expect = rows * cols;
    for (int d = a->rank - 3; d >= 0; --d) {
      if (a->shape[d] != 1 && a->in_stride[d] != expect) batch_dense = false;
      expect *= a->shape[d];
    }
    if (batch_dense && batch <= 65535) {
      dim3 grid(static_cast<unsigned>(ceil_div(cols, 32)), static_cast<unsigned>(ceil_div(rows, 32)),
                static_cast<unsigned>(batch));
      switch (a->elem_bytes) {
        case 4: hipLaunchKernelGGL(transpose_tile_kernel<uint32_t>, grid, dim3(256), 0, s,
                                   static_cast<const uint32_t*>(a->in), static_cast<uint32_t*>(a->out), batch, rows, cols,
                                   rows * cols, rows * cols); return launch_status("transpose_tile");
        case 2: hipLaunchKernelGGL(transpose_tile_kernel<uint16_t>, grid, dim3(256), 0, s,
                                   static_cast<const uint16_t*>(a->in), static_cast<uint16_t*>(a->out), batch, rows, cols,
                                   rows * cols, rows * cols); return launch_status("transpose_tile");
        default: break;
      }
    }
  }
  switch (a->elem_bytes) {
    case 1: hipLaunchKernelGGL(strided_copy_kernel<uint8_t>, dim3(grid_for(total)), dim3(kBlock), 0, s,
                               static_cast<const uint8_t*>(a->in), static_cast<uint8_t*>(a->out), *a, total); break;
    case 2: hipLaunchKernelGGL(strided_copy_kernel<uint16_t>, dim3(grid_for(total)), dim3(kBlock), 0, s,
                               static_cast<const uint16_t*>(a->in), static_cast<uint16_t*>(a->out), *a, total); break;
    case 4: hipLaunchKernelGGL(strided_copy_kernel<uint32_t>, dim3(grid_for(total)), dim3(kBlock), 0, s,
                               static_cast<const uint32_t*>(a->in), static_cast<uint32_t*>(a->out), *a, total); break;
    case 8: hipLaunchKernelGGL(strided_copy_kernel<uint64_t>, dim3(grid_for(total)), dim3(kBlock), 0, s,
                               static_cast<const uint64_t*>(a->in), static_cast<uint64_t*>(a->out), *a, total); break;
    default: return fail(C3H_EINVAL, "strided_copy: elem_bytes %d unsupported", a->elem_bytes);
  }
  return launch_status("strided_copy");
}

int c3h_reduce(const c3h_reduce_args* a, void* stream) {
  C3H_REQUIRE(a && a->outer >= 0 && a->reduce >= 1 && a->inner >= 1, "reduce: bad shape");
  C3H_REQUIRE(a->kind >= 0 && a->kind <= 2, "reduce: bad kind %d", a->kind);
  if (a->outer == 0) return C3H_OK;
  if (a->inner == 1) {
    int blocks = static_cast<int>(ceil_div(a->outer, kBlock / 64));
    hipLaunchKernelGGL(reduce_rows_kernel, dim3(blocks), dim3(kBlock), 0, as_stream(stream), *a);
  } else if (a->inner % 8 == 0 && (reinterpret_cast<uintptr_t>(a->in) & 15) == 0 && a->outer < (int64_t{1} << 31) &&
             (a->in_dtype == C3H_F32 || a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16)) {
    hipStream_t st = as_stream(stream);
    if (a->reduce <= 64) {
      const dim3 g(static_cast<unsigned>(a->outer), static_cast<unsigned>(ceil_div(a->inner / 8, 16)));
      C3H_REQUIRE(g.y <= 65535, "reduce: inner too large");
      if (a->in_dtype == C3H_F32) hipLaunchKernelGGL(reduce_cols_vec16_kernel<float>, g, dim3(kBlock), 0, st, *a);
      else if (a->in_dtype == C3H_BF16)
        hipLaunchKernelGGL(reduce_cols_vec16_kernel<bf16_t>, g, dim3(kBlock), 0, st, *a);
      else hipLaunchKernelGGL(reduce_cols_vec16_kernel<f16_t>, g, dim3(kBlock), 0, st, *a);
      return launch_status("reduce");
    }
    const dim3 g(static_cast<unsigned>(a->outer), static_cast<unsigned>(ceil_div(a->inner / 8, 64)));
    C3H_REQUIRE(g.y <= 65535, "reduce: inner too large");
    if (a->in_dtype == C3H_F32) hipLaunchKernelGGL(reduce_cols_vec_kernel<float>, g, dim3(kBlock), 0, st, *a);
    else if (a->in_dtype == C3H_BF16) hipLaunchKernelGGL(reduce_cols_vec_kernel<bf16_t>, g, dim3(kBlock), 0, st, *a);
    else hipLaunchKernelGGL(reduce_cols_vec_kernel<f16_t>, g, dim3(kBlock), 0, st, *a);
  } else {
    hipLaunchKernelGGL(reduce_cols_kernel, dim3(grid_for(a->outer * a->inner)), dim3(kBlock), 0, as_stream(stream), *a);
  }
  return launch_status("reduce");
}

int c3h_softmax(const c3h_softmax_args* a, void* stream) {
  C3H_REQUIRE(a && a->outer >= 0 && a->axis >= 1 && a->inner >= 1, "softmax: bad shape");
  if (a->outer == 0) return C3H_OK;
  if (a->inner == 1) {
    C3H_REQUIRE(a->outer <= 2147483647LL, "softmax: too many rows");
    hipLaunchKernelGGL(softmax_rows_kernel, dim3(static_cast<unsigned>(a->outer)), dim3(kBlock), 0, as_stream(stream), *a);
  } else {
    hipLaunchKernelGGL(softmax_cols_kernel, dim3(grid_for(a->outer * a->inner)), dim3(kBlock), 0, as_stream(stream), *a);
  }
  return launch_status("softmax");
}

int c3h_layernorm(const c3h_layernorm_args* a, void* stream) {
  C3H_REQUIRE(a && a->rows >= 0 && a->cols >= 1 && a->x && a->scale && a->out, "layernorm: bad args");
  if (a->rows == 0) return C3H_OK;
  int blocks = static_cast<int>(ceil_div(a->rows, kBlock / 64));
  auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool quant = a->out_dtype == C3H_I8;
  const bool vec = a->cols % 8 == 0 && a->cols <= 512 * kLnVec && al16(a->x) && al16(a->scale) &&
                   (quant ? (reinterpret_cast<uintptr_t>(a->out) & 7) == 0 : al16(a->out)) &&
                   (!a->bias || al16(a->bias)) && (!a->residual || al16(a->residual)) &&
                   (a->x_dtype == C3H_F32 || a->x_dtype == C3H_BF16 || a->x_dtype == C3H_F16) &&
                   (a->out_dtype == C3H_F32 || a->out_dtype == a->x_dtype || quant);
  C3H_REQUIRE(!quant || vec, "layernorm: an int8 (quantized) output needs cols %% 8 == 0, cols <= %d, "
              "16-byte aligned inputs and an 8-byte aligned output", 512 * kLnVec);
  C3H_REQUIRE(!quant || (quant_scale_ok(a->out_scale) && a->out_zero >= -128 && a->out_zero <= 127),
              "layernorm: quantized output needs a positive normal out_scale and an int8 zero point");
  if (vec) {
    const int nv = static_cast<int>(ceil_div(a->cols / 8, 64));
    // 768 columns: 96 8-wide vectors would leave lanes 32-63 idle for the
    // second one, so 4-wide vectors, three per lane (launch_ln case 3).
    const int NVsel = a->cols == 768 ? 3 : nv <= 1 ? 1 : nv <= 2 ? 2 : nv <= 4 ? 4 : 8;
    if (quant) {
      if (a->x_dtype == C3H_F32) launch_ln<float, int8_t>(*a, NVsel, stream);
      else if (a->x_dtype == C3H_BF16) launch_ln<bf16_t, int8_t>(*a, NVsel, stream);
      else launch_ln<f16_t, int8_t>(*a, NVsel, stream);
    } else if (a->x_dtype == C3H_F32) launch_ln<float, float>(*a, NVsel, stream);
    else if (a->x_dtype == C3H_BF16 && a->out_dtype == C3H_F32) launch_ln<bf16_t, float>(*a, NVsel, stream);
    else if (a->x_dtype == C3H_BF16) launch_ln<bf16_t, bf16_t>(*a, NVsel, stream);
    else if (a->out_dtype == C3H_F32) launch_ln<f16_t, float>(*a, NVsel, stream);
    else launch_ln<f16_t, f16_t>(*a, NVsel, stream);
    return launch_status("layernorm_vec");
  }
  hipLaunchKernelGGL(layernorm_kernel, dim3(blocks), dim3(kBlock), 0, as_stream(stream), *a);
  return launch_status("layernorm");
}

int c3h_batchnorm(const c3h_batchnorm_args* a, void* stream) {
  C3H_REQUIRE(a && a->n >= 0 && a->c >= 1 && a->hw >= 1, "batchnorm: bad shape");
  int64_t total = a->n * a->c * a->hw;
  if (total == 0) return C3H_OK;
  hipLaunchKernelGGL(batchnorm_kernel, dim3(grid_for(total)), dim3(kBlock), 0, as_stream(stream), *a);
  return launch_status("batchnorm");
}

int c3h_bn_fold(const c3h_bnfold_args* a, void* stream) {
  C3H_REQUIRE(a && a->out_channels >= 1 && a->per_channel >= 1, "bn_fold: bad shape");
  hipLaunchKernelGGL(bn_fold_kernel, dim3(grid_for(a->out_channels * a->per_channel)), dim3(kBlock), 0,
                     as_stream(stream), *a);
  return launch_status("bn_fold");
}

int c3h_gather(const c3h_gather_args* a, void* stream) {
  C3H_REQUIRE(a && a->outer >= 0 && a->axis_dim >= 1 && a->inner >= 0 && a->n_indices >= 0, "gather: bad shape");
  int64_t row_bytes = a->inner * a->elem_bytes;
  int64_t total_rows = a->outer * a->n_indices;
  if (total_rows == 0 || row_bytes == 0) return C3H_OK;
  hipStream_t s = as_stream(stream);
  if (a->addend) {
    C3H_REQUIRE(a->outer == 1 && a->addend_rows >= 1, "gather: a fused addend needs outer == 1 and addend_rows >= 1");
    C3H_REQUIRE(a->inner % 8 == 0, "gather: a fused addend needs rows of a multiple of 8 elements");
    const int vec_bytes = a->dtype == C3H_F32 ? 32 : 16;
    C3H_REQUIRE((a->dtype == C3H_F32 && a->elem_bytes == 4) ||
                    ((a->dtype == C3H_BF16 || a->dtype == C3H_F16) && a->elem_bytes == 2),
                "gather: a fused addend needs dtype F32, BF16 or F16 matching elem_bytes");
    C3H_REQUIRE(a->addend_dtype == C3H_F32 || a->addend_dtype == a->dtype,
                "gather: the addend must be F32 or of the data dtype");
    const bool add32 = a->addend_dtype == C3H_F32;
    C3H_REQUIRE((reinterpret_cast<uintptr_t>(a->data) | reinterpret_cast<uintptr_t>(a->out)) % vec_bytes == 0 &&
                    reinterpret_cast<uintptr_t>(a->addend) % (add32 ? 32 : vec_bytes) == 0,
                "gather: a fused addend needs vector-aligned data, addend and out");
    const int64_t rv = a->inner / 8;
    const dim3 grid(grid_for(total_rows * rv, kGatherU));
    if (a->dtype == C3H_F32)
      hipLaunchKernelGGL((gather_add_kernel<float, float>), grid, dim3(kBlock), 0, s, *a, rv);
    else if (a->dtype == C3H_BF16 && add32)
      hipLaunchKernelGGL((gather_add_kernel<bf16_t, float>), grid, dim3(kBlock), 0, s, *a, rv);
    else if (a->dtype == C3H_BF16)
      hipLaunchKernelGGL((gather_add_kernel<bf16_t, bf16_t>), grid, dim3(kBlock), 0, s, *a, rv);
    else if (add32)
      hipLaunchKernelGGL((gather_add_kernel<f16_t, float>), grid, dim3(kBlock), 0, s, *a, rv);
    else
      hipLaunchKernelGGL((gather_add_kernel<f16_t, f16_t>), grid, dim3(kBlock), 0, s, *a, rv);
    return launch_status("gather");
  }
  bool aligned16 = (reinterpret_cast<uintptr_t>(a->data) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 15) == 0;
  if (row_bytes % 16 == 0 && aligned16) {
    int64_t rv = row_bytes / 16;
    hipLaunchKernelGGL(gather_kernel<uint4>, dim3(grid_for(total_rows * rv)), dim3(kBlock), 0, s, *a, rv);
  } else if (row_bytes % 4 == 0) {
    int64_t rv = row_bytes / 4;
    hipLaunchKernelGGL(gather_kernel<uint32_t>, dim3(grid_for(total_rows * rv)), dim3(kBlock), 0, s, *a, rv);
  } else {
    hipLaunchKernelGGL(gather_kernel<uint8_t>, dim3(grid_for(total_rows * row_bytes)), dim3(kBlock), 0, s, *a,
                       row_bytes);
  }
  return launch_status("gather");
}

int c3h_argmax(const c3h_argmax_args* a, void* stream) {
  C3H_REQUIRE(a && a->rows >= 0 && a->cols >= 1 && a->out, "argmax: bad args");
  if (a->rows == 0) return C3H_OK;
  C3H_REQUIRE(a->rows <= 2147483647LL, "argmax: too many rows");
  bool vec = a->in_dtype == C3H_F32 && (a->cols & 3) == 0 && (reinterpret_cast<uintptr_t>(a->in) & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(argmax_kernel<true>, dim3(static_cast<unsigned>(a->rows)), dim3(kBlock), 0, as_stream(stream), *a);
  else
    hipLaunchKernelGGL(argmax_kernel<false>, dim3(static_cast<unsigned>(a->rows)), dim3(kBlock), 0, as_stream(stream), *a);
  return launch_status("argmax");
}

int c3h_argmax_finish(const c3h_argmax_finish_args* a, void* stream) {
  C3H_REQUIRE(a && a->rows >= 0 && a->cols >= 1 && a->out, "argmax_finish: bad args");
  if (a->rows == 0) return C3H_OK;
  C3H_REQUIRE(a->n_parts == ceil_div(a->cols, 64) && a->ld >= a->n_parts && a->in_ld >= a->cols,
              "argmax_finish: n_parts must be ceil(cols / 64), ld >= n_parts and in_ld >= cols");
  C3H_REQUIRE(a->parts != nullptr && (reinterpret_cast<uintptr_t>(a->parts) & 7) == 0 && a->in != nullptr,
              "argmax_finish: parts (8-byte aligned) and in are required");
  C3H_REQUIRE(a->in_dtype == C3H_F32 || a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16,
              "argmax_finish: in must be fp32, bf16 or fp16");
  const int64_t blocks = ceil_div(a->rows, kBlock / 64);
  C3H_REQUIRE(blocks <= 2147483647LL, "argmax_finish: too many rows");
  const dim3 g(static_cast<unsigned>(blocks)), b(kBlock);
  hipStream_t st = as_stream(stream);
  const int64_t np = ceil_div(a->n_parts, 64);  // block maxima per lane
  if (np <= 2) hipLaunchKernelGGL(argmax_finish_kernel<2>, g, b, 0, st, *a);
  else if (np <= 4) hipLaunchKernelGGL(argmax_finish_kernel<4>, g, b, 0, st, *a);
  else if (np <= 8) hipLaunchKernelGGL(argmax_finish_kernel<8>, g, b, 0, st, *a);
  else if (np <= 16) hipLaunchKernelGGL(argmax_finish_kernel<16>, g, b, 0, st, *a);
  else hipLaunchKernelGGL(argmax_finish_kernel<0>, g, b, 0, st, *a);
  return launch_status("argmax_finish");
}

int c3h_im2col(const c3h_im2col_args* a, void* stream) {
  C3H_REQUIRE(a && a->n >= 0 && a->c >= 1 && a->ho >= 1 && a->wo >= 1 && a->kh >= 1 && a->kw >= 1, "im2col: bad shape");
  int64_t total = static_cast<int64_t>(a->n) * a->ho * a->wo * a->c * a->kh * a->kw;
  if (total == 0) return C3H_OK;
  hipLaunchKernelGGL(im2col_kernel, dim3(grid_for(total)), dim3(kBlock), 0, as_stream(stream), *a);
  return launch_status("im2col");
}

int c3h_layout(const c3h_layout_args* a, void* stream) {
  C3H_REQUIRE(a && a->n >= 0 && a->c >= 1 && a->h >= 1 && a->w >= 1 && a->c_pad >= a->c, "layout: bad shape");
  C3H_REQUIRE(a->direction == 0 || a->direction == 1, "layout: bad direction");
  if (a->n == 0) return C3H_OK;
  int64_t hw = static_cast<int64_t>(a->h) * a->w;
  if (a->direction == 0 && a->c_pad == 4 && a->in_dtype == C3H_F32 && hw % 4 == 0 &&
      (reinterpret_cast<uintptr_t>(a->in) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 15) == 0 &&
      (a->out_dtype == C3H_F32 || a->out_dtype == C3H_BF16 || a->out_dtype == C3H_F16)) {
    const dim3 grid(grid_for(a->n * hw / 4));
    if (a->out_dtype == C3H_F32)
      hipLaunchKernelGGL(nchw_to_nhwc_c4_kernel<float>, grid, dim3(kBlock), 0, as_stream(stream), *a);
    else if (a->out_dtype == C3H_BF16)
      hipLaunchKernelGGL(nchw_to_nhwc_c4_kernel<bf16_t>, grid, dim3(kBlock), 0, as_stream(stream), *a);
    else
      hipLaunchKernelGGL(nchw_to_nhwc_c4_kernel<f16_t>, grid, dim3(kBlock), 0, as_stream(stream), *a);
    return launch_status("layout_c4");
  }
  if (a->direction == 0 && a->c_pad <= 16) {
    hipLaunchKernelGGL(nchw_to_nhwc_small_kernel, dim3(grid_for(a->n * hw)), dim3(kBlock), 0, as_stream(stream), *a);
    return launch_status("layout_small");
  }
  C3H_REQUIRE(a->n <= 65535, "layout: batch too large for tiled path");
  int64_t cdim = a->direction == 0 ? a->c_pad : a->c;
  dim3 grid(static_cast<unsigned>(ceil_div(hw, 32)), static_cast<unsigned>(ceil_div(cdim, 32)),
            static_cast<unsigned>(a->n));
  hipLaunchKernelGGL(layout_tile_kernel, grid, dim3(256), 0, as_stream(stream), *a);
  return launch_status("layout_tile");
}

int c3h_maxpool2d(const c3h_pool_args* a, void* stream) {
  C3H_REQUIRE(a && a->n >= 0 && a->c >= 1 && a->ho >= 1 && a->wo >= 1, "maxpool: bad shape");
  C3H_REQUIRE(a->layout == 0 || (a->layout == 1 && a->c_stride >= a->c), "maxpool: bad layout");
  int64_t total = static_cast<int64_t>(a->n) * a->c * a->ho * a->wo;
  if (total == 0) return C3H_OK;
  const int es = dtype_size(a->dtype);
  const bool vec = a->layout == 1 && (a->dtype == C3H_F32 || a->dtype == C3H_BF16 || a->dtype == C3H_F16) &&
                   es > 0 && (a->c * es) % 16 == 0 && (a->c_stride * es) % 16 == 0 &&
                   (reinterpret_cast<uintptr_t>(a->x) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 15) == 0;
  if (vec) {
    const int64_t work = total * es / 16;
    if (a->dtype == C3H_F32)
      hipLaunchKernelGGL(maxpool_nhwc_vec_kernel<float>, dim3(grid_for(work)), dim3(kBlock), 0, as_stream(stream), *a);
    else if (a->dtype == C3H_BF16)
      hipLaunchKernelGGL(maxpool_nhwc_vec_kernel<bf16_t>, dim3(grid_for(work)), dim3(kBlock), 0, as_stream(stream), *a);
    else
      hipLaunchKernelGGL(maxpool_nhwc_vec_kernel<f16_t>, dim3(grid_for(work)), dim3(kBlock), 0, as_stream(stream), *a);
    return launch_status("maxpool_nhwc_vec");
  }
  hipLaunchKernelGGL(maxpool_kernel, dim3(grid_for(total)), dim3(kBlock), 0, as_stream(stream), *a);
  return launch_status("maxpool");
}

int c3h_pack_conv_weight(const c3h_pack_args* a, void* stream) {
  C3H_REQUIRE(a && a->o >= 1 && a->c >= 1 && a->kh >= 1 && a->kw >= 1, "pack: bad sizes");
  C3H_REQUIRE(a->c_pack >= a->c && a->kw_pack >= a->kw, "pack: c_pack/kw_pack too small");
  C3H_REQUIRE(a->k_stride >= static_cast<int64_t>(a->kh) * a->kw_pack * a->c_pack, "pack: k_stride too small");
  hipLaunchKernelGGL(pack_conv_weight_kernel, dim3(grid_for(static_cast<int64_t>(a->o) * a->k_stride)), dim3(kBlock),
                     0, as_stream(stream), *a);
  return launch_status("pack_conv_weight");
}

int c3h_nonfinite(const c3h_nonfinite_args* a, void* stream) {
  C3H_REQUIRE(a && a->flag && a->count >= 0 && (a->x || a->count == 0), "nonfinite: bad args");
  C3H_REQUIRE(a->dtype == C3H_F32 || a->dtype == C3H_BF16 || a->dtype == C3H_F16,
              "nonfinite: dtype must be F32, BF16 or F16");
  C3H_REQUIRE((reinterpret_cast<uintptr_t>(a->x) & 15) == 0, "nonfinite: x must be 16-byte aligned");
  if (a->count == 0) return C3H_OK;
  const int per = a->dtype == C3H_F32 ? 4 : 8;
  const dim3 g(grid_for(ceil_div(a->count, per), 4)), b(kBlock);
  hipStream_t st = as_stream(stream);
  if (a->dtype == C3H_F32)
    hipLaunchKernelGGL(nonfinite_kernel<float>, g, b, 0, st, static_cast<const float*>(a->x), a->count, a->flag);
  else if (a->dtype == C3H_BF16)
    hipLaunchKernelGGL(nonfinite_kernel<bf16_t>, g, b, 0, st, static_cast<const bf16_t*>(a->x), a->count, a->flag);
  else
    hipLaunchKernelGGL(nonfinite_kernel<f16_t>, g, b, 0, st, static_cast<const f16_t*>(a->x), a->count, a->flag);
  return launch_status("nonfinite");
}

int c3h_quantize(const c3h_quantize_args* a, void* stream) {
  C3H_REQUIRE(a && a->count >= 0, "quantize: bad args");
  C3H_REQUIRE(quant_scale_ok(a->scale), "quantize: scale must be a positive normal float, got %g",
              static_cast<double>(a->scale));
  if (a->count == 0) return C3H_OK;
  if (a->count % 8 == 0 && (reinterpret_cast<uintptr_t>(a->x) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(a->out) & 7) == 0 &&
      (a->x_dtype == C3H_F32 || a->x_dtype == C3H_BF16 || a->x_dtype == C3H_F16)) {
    const dim3 g(grid_for(a->count / 8, 2)), b(kBlock);
    hipStream_t st = as_stream(stream);
    const QuantDiv qd = QuantDiv::on_host(a->scale, a->zero_point, a->x_dtype == C3H_F32 ? -1 : a->x_dtype);
    if (a->x_dtype == C3H_F32) hipLaunchKernelGGL(quantize_vec_kernel<float>, g, b, 0, st, *a, qd);
    else if (a->x_dtype == C3H_BF16) hipLaunchKernelGGL(quantize_vec_kernel<bf16_t>, g, b, 0, st, *a, qd);
    else hipLaunchKernelGGL(quantize_vec_kernel<f16_t>, g, b, 0, st, *a, qd);
    return launch_status("quantize_vec");
  }
  hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(a->count)), dim3(kBlock), 0, as_stream(stream), *a);
  return launch_status("quantize");
}

int c3h_quantize_fp8_rows(const c3h_fp8_quant_args* a, void* stream) {
  C3H_REQUIRE(a && a->rows >= 0 && a->cols >= 0, "quantize_fp8_rows: bad args");
  C3H_REQUIRE(a->cols % 8 == 0 && a->ldx % 8 == 0 && a->ldo % 8 == 0 && a->ldx >= a->cols && a->ldo >= a->cols,
              "quantize_fp8_rows: cols, ldx, ldo must be multiples of 8 with ldx, ldo >= cols");
  C3H_REQUIRE((reinterpret_cast<uintptr_t>(a->x) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 7) == 0,
              "quantize_fp8_rows: x must be 16-byte and out 8-byte aligned");
  C3H_REQUIRE(a->x_dtype == C3H_F32 || a->x_dtype == C3H_BF16 || a->x_dtype == C3H_F16,
              "quantize_fp8_rows: x dtype must be fp32, bf16 or fp16");
  C3H_REQUIRE(a->scale != nullptr, "quantize_fp8_rows: scale output required");
  C3H_REQUIRE(ceil_div(a->rows, kBlock / 64) < (int64_t{1} << 31), "quantize_fp8_rows: too many rows");
  if (a->rows == 0) return C3H_OK;
  hipStream_t st = as_stream(stream);
  if (a->x_dtype == C3H_F32) return launch_fp8_rows<float>(*a, st);
  if (a->x_dtype == C3H_BF16) return launch_fp8_rows<bf16_t>(*a, st);
  return launch_fp8_rows<f16_t>(*a, st);
}

int c3h_quantize_mxfp4(const c3h_mxfp4_quant_args* a, void* stream) {
  C3H_REQUIRE(a && a->rows >= 0 && a->cols >= 0, "quantize_mxfp4: bad args");
  C3H_REQUIRE(a->cols % 32 == 0, "quantize_mxfp4: cols must be a multiple of 32");
  C3H_REQUIRE(a->ldx >= a->cols && a->ldc >= a->cols / 2 && a->lds >= a->cols / 32,
              "quantize_mxfp4: ldx >= cols, ldc >= cols/2 and lds >= cols/32 required");
  C3H_REQUIRE(a->ldc % 16 == 0 && (reinterpret_cast<uintptr_t>(a->codes) & 15) == 0,
              "quantize_mxfp4: ldc must be a multiple of 16 and codes 16-byte aligned");
  C3H_REQUIRE(a->x_dtype == C3H_F32 || a->x_dtype == C3H_BF16 || a->x_dtype == C3H_F16,
              "quantize_mxfp4: x dtype must be fp32, bf16 or fp16");
  C3H_REQUIRE(a->x != nullptr && a->codes != nullptr && a->scales != nullptr, "quantize_mxfp4: null pointer");
  const int64_t blocks = a->rows * (a->cols / 32);
  if (blocks == 0) return C3H_OK;
  C3H_REQUIRE(ceil_div(blocks, kBlock) < (int64_t{1} << 31), "quantize_mxfp4: too many blocks");
  hipLaunchKernelGGL(quantize_mxfp4_kernel, dim3(static_cast<unsigned>(ceil_div(blocks, kBlock))), dim3(kBlock), 0,
                     as_stream(stream), *a);
  return launch_status("quantize_mxfp4");
}

int c3h_dequantize(const c3h_dequantize_args* a, void* stream) {
  C3H_REQUIRE(a && a->count >= 0, "dequantize: bad args");
  if (a->count == 0) return C3H_OK;
  hipLaunchKernelGGL(dequantize_kernel, dim3(grid_for(a->count)), dim3(kBlock), 0, as_stream(stream), *a);
  return launch_status("dequantize");
}

}  // extern "C"
