// Contraction kernels of libc3hip.so (gfx950): GEMM and implicit-GEMM Conv2d
// on MFMA, fp32 accumulation, LDS double-buffered tiles and a fused epilogue.
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
#include "common.h"

using namespace c3h;

namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

constexpr int kThreads = 256;

// ---------------------------------------------------------------- epilogue
// `e` is read straight from the kernel-argument segment (uniform scalar
// loads); `bias_off` selects the batch's bias slice.
__device__ __forceinline__ float apply_epilogue(const c3h_epilogue& e, float acc, int64_t m, int64_t n,
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

// ---------------------------------------------------------------- problem
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

__device__ __forceinline__ ConvRow conv_row(const Problem& p, int64_t m) {
  ConvRow r;
  r.valid = m < p.m;
  int64_t mm = r.valid ? m : 0;
  const int64_t hw = static_cast<int64_t>(p.ho) * p.wo;
  int64_t img = mm / hw;
  int64_t rem = mm - img * hw;
  int ho = static_cast<int>(rem / p.wo);
  int wo = static_cast<int>(rem - static_cast<int64_t>(ho) * p.wo);
  r.base = img * static_cast<int64_t>(p.ch) * p.cw * p.c_stride;
  r.hi0 = ho * p.sh - p.pt;
  r.wi0 = wo * p.sw - p.pl;
  return r;
}

// Element offset in x of the VEC-wide K slice starting at k, or -1 when it is
// padding.  K order is (kh, kw_pack, c_pack) with c fastest.
__device__ __forceinline__ int64_t conv_k_offset(const Problem& p, const ConvRow& r, int64_t k) {
  if (!r.valid || k >= p.k) return -1;
  int kk = static_cast<int>(k);
  int c0 = kk % p.c_pack;
  int tap = kk / p.c_pack;
  int kwi = tap % p.kw_pack;
  int khi = tap / p.kw_pack;
  if (kwi >= p.kw || c0 >= p.cc) return -1;
  int hi = r.hi0 + khi * p.dh;
  int wi = r.wi0 + kwi * p.dw;
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
    for (int c = 0; c < WTN / 4; ++c) {
      const int64_t n = ncol0 + c0 + c;
      if (n >= p.n) break;
      const int64_t o = m * p.ldo + n;
      const float res = resp ? Elem<TO>::to_f32(resp[o]) : 0.0f;
      outp[o] = Elem<TO>::from_f32(apply_epilogue(p.epi, stage[row * SS + c0 + c], m, n, p.n, res, bias_off));
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
        outp[o] = Elem<TO>::from_f32(apply_epilogue(p.epi, stage[row * SS + col], m, n, p.n, res, bias_off));
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
// 16-bit kernel: v_mfma_f32_16x16x32_{bf16,f16}.  LDS tiles are stored
// row-major with K contiguous (As[m][k], Bs[n][k]) plus a 16-byte skew, so a
// lane's 8-element operand is one ds_read_b128.
// =====================================================================
template <typename T> struct Mfma16;
template <> struct Mfma16<bf16_t> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma16<f16_t> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <typename T, typename TO, int BM, int BN, int WM, int WN, int AM, int VEC, bool SWAP>
__global__ void __launch_bounds__(kThreads) gemm_h_kernel(Problem p) {
  constexpr int BK = 32;
  constexpr int SK = BK + 8;  // 80-byte row stride
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int WTN = BN / WN;
  constexpr int kTileBytes = 2 * BM * SK * 2 + 2 * BN * SK * 2;
  constexpr int kStageBytes = 4 * 16 * (WTN + 4) * 4;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kTileBytes > kStageBytes ? kTileBytes : kStageBytes];
  uint16_t (*As)[BM][SK] = reinterpret_cast<uint16_t (*)[BM][SK]>(smem);
  uint16_t (*Bs)[BN][SK] = reinterpret_cast<uint16_t (*)[BN][SK]>(smem + 2 * BM * SK * 2);
  typedef typename Mfma16<T>::vec vec8;

  int tm, tn;
  tile_coords(p, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const int64_t bz = blockIdx.z;
  const uint16_t* A = static_cast<const uint16_t*>(p.a) + bz * p.stride_a;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + bz * p.stride_b;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;

  // Each thread moves VEC-element vectors (VEC = 8 -> 16 B, VEC = 4 -> 8 B).
  constexpr int VPR = BK / VEC;                     // vectors per tile row
  constexpr int A_VECS = BM * VPR / kThreads;
  constexpr int B_VECS8 = BN * (BK / 8) / kThreads;  // B always 16-byte vectors
  static_assert(A_VECS >= 1 && B_VECS8 >= 1, "tile too small");
  typedef typename std::conditional<VEC == 8, uint4, uint2>::type AV;
  AV ra[A_VECS];
  uint4 rb[B_VECS8];

  ConvRow crow[A_VECS];
  if (AM == kConv) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) crow[i] = conv_row(p, m0 + (tid + kThreads * i) / VPR);
  }

  auto load_a = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      int e = tid + kThreads * i;
      int mr = e / VPR, kc = (e % VPR) * VEC;
      int64_t m = m0 + mr, k = k0 + kc;
      AV v = {};
      if (AM == kDenseK) {
        if (m < p.m && k < p.k) v = *reinterpret_cast<const AV*>(A + m * p.lda + k);
      } else {
        int64_t off = conv_k_offset(p, crow[i], k);
        if (off >= 0) v = *reinterpret_cast<const AV*>(A + off);
      }
      ra[i] = v;
    }
  };
  auto load_b = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < B_VECS8; ++i) {
      int e = tid + kThreads * i;
      int nr = e / (BK / 8), kc = (e % (BK / 8)) * 8;
      int64_t n = n0 + nr, k = k0 + kc;
      uint4 v = {0u, 0u, 0u, 0u};
      if (n < p.n && k < p.k) v = *reinterpret_cast<const uint4*>(B + n * p.ldb + k);
      rb[i] = v;
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_VECS; ++i) {
      int e = tid + kThreads * i;
      int mr = e / VPR, kc = (e % VPR) * VEC;
      *reinterpret_cast<AV*>(&As[buf][mr][kc]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_VECS8; ++i) {
      int e = tid + kThreads * i;
      int nr = e / (BK / 8), kc = (e % (BK / 8)) * 8;
      *reinterpret_cast<uint4*>(&Bs[buf][nr][kc]) = rb[i];
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
  const int lrow = lane & 15, lk = (lane >> 4) * 8;
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) {
      load_a((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }
    vec8 av[TM], bv[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
      av[i] = *reinterpret_cast<const vec8*>(&As[cur][wm * (BM / WM) + i * 16 + lrow][lk]);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      bv[j] = *reinterpret_cast<const vec8*>(&Bs[cur][wn * (BN / WN) + j * 16 + lrow][lk]);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = SWAP ? Mfma16<T>::mma(bv[j], av[i], acc[i][j]) : Mfma16<T>::mma(av[i], bv[j], acc[i][j]);
    if (kt + 1 < ktiles) {
      store_tiles(cur ^ 1);
      __syncthreads();
    }
  }

  // Epilogue: a lane holds (m = 4*(lane/16)+r, n = lane%16) of each tile
  // (with SWAP the tile is transposed); stage 16-row strips through LDS.
  TO* outp = static_cast<TO*>(p.out) + bz * p.stride_out;
  const TO* resp = p.epi.residual ? static_cast<const TO*>(p.epi.residual) + bz * p.stride_res : nullptr;
  const int64_t bias_off = bz * p.stride_bias;
  __syncthreads();
  float* stage = reinterpret_cast<float*>(smem) + wave * 16 * (WTN + 4);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (SWAP) stage[lrow * (WTN + 4) + j * 16 + (lane >> 4) * 4 + r] = acc[i][j][r];
        else stage[((lane >> 4) * 4 + r) * (WTN + 4) + j * 16 + lrow] = acc[i][j][r];
      }
    wave_sync_lds();
    store_strip<TO, WTN>(p, stage, lane, m0 + wm * (BM / WM) + i * 16, n0 + wn * WTN, outp, resp, bias_off);
    wave_sync_lds();
  }
}

// =====================================================================
// int8 kernel: v_mfma_i32_16x16x64_i8 with exact int32 accumulation
// (QLinearMatMul core).  A [m][k] and B packed [n][k], both K-contiguous;
// LDS rows of 64 bytes + 16-byte skew so a lane's 16-byte operand is one
// ds_read_b128.
// =====================================================================
typedef __attribute__((ext_vector_type(4))) int i32x4;

struct QProblem {
  const int8_t* a;
  const int8_t* b;
  void* out;
  int64_t m, n, k, lda, ldb, ldo;
  float a_scale, y_scale;
  const float* b_scale;
  int y_zero, mode, out_dtype;
  int tiles_m, tiles_n;
  c3h_epilogue epi;
};

template <int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(kThreads) qgemm_kernel(QProblem p) {
  constexpr int BK = 64;
  constexpr int SK = BK + 16;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  __shared__ __attribute__((aligned(16))) int8_t As[2][BM][SK];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN][SK];

  const int total = p.tiles_m * p.tiles_n;
  int tile = blockIdx.x;
  if ((total & 7) == 0) tile = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int tm = tile / p.tiles_n, tn = tile - (tile / p.tiles_n) * p.tiles_n;
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;
  constexpr int A_V = BM * (BK / 16) / kThreads, B_V = BN * (BK / 16) / kThreads;
  uint4 ra[A_V], rb[B_V];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_V; ++i) {
      int e = tid + kThreads * i, r = e / (BK / 16), c = (e % (BK / 16)) * 16;
      int64_t m = m0 + r, k = k0 + c;
      uint4 v = {0u, 0u, 0u, 0u};
      if (m < p.m && k < p.k) v = *reinterpret_cast<const uint4*>(p.a + m * p.lda + k);
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_V; ++i) {
      int e = tid + kThreads * i, r = e / (BK / 16), c = (e % (BK / 16)) * 16;
      int64_t n = n0 + r, k = k0 + c;
      uint4 v = {0u, 0u, 0u, 0u};
      if (n < p.n && k < p.k) v = *reinterpret_cast<const uint4*>(p.b + n * p.ldb + k);
      rb[i] = v;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_V; ++i) {
      int e = tid + kThreads * i, r = e / (BK / 16), c = (e % (BK / 16)) * 16;
      *reinterpret_cast<uint4*>(&As[buf][r][c]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_V; ++i) {
      int e = tid + kThreads * i, r = e / (BK / 16), c = (e % (BK / 16)) * 16;
      *reinterpret_cast<uint4*>(&Bs[buf][r][c]) = rb[i];
    }
  };
  i32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};
  const int64_t ktiles = ceil_div(p.k, BK);
  load(0);
  store(0);
  __syncthreads();
  const int lrow = lane & 15, lk = (lane >> 4) * 16;
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) load((kt + 1) * BK);
    i32x4 av[TM], bv[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) av[i] = *reinterpret_cast<const i32x4*>(&As[cur][wm * (BM / WM) + i * 16 + lrow][lk]);
#pragma unroll
    for (int j = 0; j < TN; ++j) bv[j] = *reinterpret_cast<const i32x4*>(&Bs[cur][wn * (BN / WN) + j * 16 + lrow][lk]);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i], bv[j], acc[i][j], 0, 0, 0);
    if (kt + 1 < ktiles) {
      store(cur ^ 1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t n = n0 + wn * (BN / WN) + j * 16 + lrow;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * (BM / WM) + i * 16 + (lane >> 4) * 4 + r;
        if (m >= p.m || n >= p.n) continue;
        const int64_t o = m * p.ldo + n;
        const int32_t iacc = acc[i][j][r];
        if (p.mode == 0) {
          static_cast<int32_t*>(p.out)[o] = iacc;
        } else if (p.mode == 1) {
          const float mult = (p.a_scale * p.b_scale[n]) / p.y_scale;
          float y = rintf(static_cast<float>(iacc) * mult) + static_cast<float>(p.y_zero);
          y = fminf(fmaxf(y, -128.0f), 127.0f);
          static_cast<int8_t*>(p.out)[o] = static_cast<int8_t>(y);
        } else {
          float deq;
          if (p.mode == 3) {
            // QLinearMatMul -> DequantizeLinear: the int8 y of mode 1, then (y - zy) * y_scale.
            const float mult = (p.a_scale * p.b_scale[n]) / p.y_scale;
            float y = rintf(static_cast<float>(iacc) * mult) + static_cast<float>(p.y_zero);
            y = fminf(fmaxf(y, -128.0f), 127.0f);
            deq = (y - static_cast<float>(p.y_zero)) * p.y_scale;
          } else {
            deq = static_cast<float>(iacc) * (p.a_scale * p.b_scale[n]);
          }
          float res = 0.0f;
          if (p.epi.residual) res = load_as_f32(p.epi.residual, p.out_dtype, o);
          store_from_f32(p.out, p.out_dtype, o, apply_epilogue(p.epi, deq, m, n, p.n, res));
        }
      }
    }
  }
}

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
  outp[o] = apply_epilogue(p.epi, acc, m, n, p.n, res, bz * p.stride_bias);
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
  } else if (p.m <= 64 || p.n <= 64) {
    grid_of<64, 64>(p, batch, grid);
    hipLaunchKernelGGL((gemm_f32_kernel<64, 64, 2, 2, AM, BK_>), grid, dim3(kThreads), 0, s, p);
  } else {
    grid_of<128, 128>(p, batch, grid);
    hipLaunchKernelGGL((gemm_f32_kernel<128, 128, 2, 2, AM, BK_>), grid, dim3(kThreads), 0, s, p);
  }
  return launch_status("gemm_f32");
}

template <typename T, typename TO, int AM, int VEC>
int launch_h_shape(Problem p, int64_t batch, hipStream_t s) {
  dim3 grid;
  if (p.n <= 64) {
    grid_of<256, 64>(p, batch, grid);
    hipLaunchKernelGGL((gemm_h_kernel<T, TO, 256, 64, 4, 1, AM, VEC, false>), grid, dim3(kThreads), 0, s, p);
  } else if (p.m <= 4096 || p.n <= 128) {
    grid_of<128, 128>(p, batch, grid);
    hipLaunchKernelGGL((gemm_h_kernel<T, TO, 128, 128, 2, 2, AM, VEC, false>), grid, dim3(kThreads), 0, s, p);
  } else {
    grid_of<128, 256>(p, batch, grid);
    hipLaunchKernelGGL((gemm_h_kernel<T, TO, 128, 256, 2, 2, AM, VEC, false>), grid, dim3(kThreads), 0, s, p);
  }
  return launch_status("gemm_h");
}

// 16-bit inputs write either the same 16-bit type or fp32.
template <typename T, int AM, int VEC>
int launch_h(Problem p, int64_t batch, hipStream_t s, int in_dtype) {
  if (p.out_dtype == C3H_F32) return launch_h_shape<T, float, AM, VEC>(p, batch, s);
  if (p.out_dtype == in_dtype) return launch_h_shape<T, T, AM, VEC>(p, batch, s);
  return fail(C3H_EUNSUPPORTED, "gemm: 16-bit inputs write fp32 or the input dtype, not %d", p.out_dtype);
}

int check_epilogue(const c3h_epilogue& e) {
  C3H_REQUIRE(e.bias_mode >= 0 && e.bias_mode <= 4, "epilogue: bad bias_mode %d", e.bias_mode);
  C3H_REQUIRE(e.bias_mode == 0 || e.bias != nullptr, "epilogue: bias_mode %d needs a bias pointer", e.bias_mode);
  C3H_REQUIRE(e.act == 0 || e.act == 1, "epilogue: bad act %d", e.act);
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

}  // namespace

extern "C" {

int c3h_gemm(const c3h_gemm_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr, "gemm: null args");
  C3H_REQUIRE(a->m >= 0 && a->n >= 0 && a->k >= 0 && a->batch >= 1, "gemm: bad sizes");
  C3H_REQUIRE(a->batch <= 65535, "gemm: batch %lld too large", static_cast<long long>(a->batch));
  int rc = check_epilogue(a->epi);
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
      return a->trans_b ? launch_f32<kDenseM, true>(p, a->batch, s) : launch_f32<kDenseM, false>(p, a->batch, s);
    }
    return a->trans_b ? launch_f32<kDenseK, true>(p, a->batch, s) : launch_f32<kDenseK, false>(p, a->batch, s);
  }
  if (a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16) {
    C3H_REQUIRE(!a->trans_a && a->trans_b, "gemm: 16-bit path needs A [m,k] and B packed [n,k] (trans_b=1)");
    C3H_REQUIRE(a->k % 8 == 0 && a->lda % 8 == 0 && a->ldb % 8 == 0 && a->stride_a % 8 == 0 && a->stride_b % 8 == 0,
                "gemm: 16-bit path needs k, lda, ldb multiples of 8");
    C3H_REQUIRE(aligned(a->a, 16) && aligned(a->b, 16), "gemm: 16-bit operands must be 16-byte aligned");
    return a->in_dtype == C3H_BF16 ? launch_h<bf16_t, kDenseK, 8>(p, a->batch, s, a->in_dtype)
                                   : launch_h<f16_t, kDenseK, 8>(p, a->batch, s, a->in_dtype);
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
  hipStream_t s = as_stream(stream);
  if (a->in_dtype == C3H_F32) {
    // Packed K order (kh, kw, c_pack); 4-wide vectors must stay in one pixel.
    C3H_REQUIRE(a->c_pack % 4 == 0 && a->c_stride % 4 == 0, "conv2d fp32: c_pack and c_stride must be multiples of 4");
    C3H_REQUIRE(a->out_dtype == C3H_F32, "conv2d fp32: output must be fp32");
    C3H_REQUIRE(aligned(a->x, 16) && aligned(a->w, 16), "conv2d fp32: x and w must be 16-byte aligned");
    p.kw_pack = a->kw;
    p.k = static_cast<int64_t>(a->kh) * a->kw * a->c_pack;
    p.ldb = p.k;
    return launch_f32<kConv, true>(p, 1, s);
  }
  if (a->in_dtype == C3H_BF16 || a->in_dtype == C3H_F16) {
    C3H_REQUIRE(aligned(a->x, 16) && aligned(a->w, 16), "conv2d: x and w must be 16-byte aligned");
    if (a->c_pack % 8 == 0 && a->c_stride % 8 == 0) {
      p.kw_pack = a->kw;
      p.k = static_cast<int64_t>(a->kh) * a->kw * a->c_pack;
      p.ldb = ceil_div(p.k, 32) * 32;  // weights padded to whole 32-wide K tiles
      return a->in_dtype == C3H_BF16 ? launch_h<bf16_t, kConv, 8>(p, 1, s, a->in_dtype)
                                     : launch_h<f16_t, kConv, 8>(p, 1, s, a->in_dtype);
    }
    // Narrow-channel stem: c_pack = c_stride = 4, kw padded to a multiple of
    // 2 so each 32-wide K tile covers whole pixels (8-byte vectors).
    C3H_REQUIRE(a->c_pack == 4 && a->c_stride == 4, "conv2d: 16-bit path needs c_pack%8==0 or c_pack==c_stride==4");
    p.kw_pack = static_cast<int>(ceil_div(a->kw, 8) * 8);
    p.k = static_cast<int64_t>(a->kh) * p.kw_pack * 4;
    p.ldb = p.k;
    return a->in_dtype == C3H_BF16 ? launch_h<bf16_t, kConv, 4>(p, 1, s, a->in_dtype)
                                   : launch_h<f16_t, kConv, 4>(p, 1, s, a->in_dtype);
  }
  return fail(C3H_EUNSUPPORTED, "conv2d: input dtype %d unsupported", a->in_dtype);
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
  C3H_REQUIRE(a->mode < 2 || a->out_dtype == C3H_F32 || a->out_dtype == C3H_BF16 || a->out_dtype == C3H_F16,
              "qgemm: dequantized output dtype must be float");
  int rc = check_epilogue(a->epi);
  if (rc) return rc;
  if (a->m == 0 || a->n == 0) return C3H_OK;
  QProblem p;
  memset(&p, 0, sizeof(p));
  p.a = a->a; p.b = a->b; p.out = a->out;
  p.m = a->m; p.n = a->n; p.k = a->k; p.lda = a->lda; p.ldb = a->ldb; p.ldo = a->ldo;
  p.a_scale = a->a_scale; p.y_scale = a->y_scale; p.b_scale = a->b_scale;
  p.y_zero = a->y_zero; p.mode = a->mode; p.out_dtype = a->out_dtype;
  p.epi = a->epi;
  hipStream_t s = as_stream(stream);
  if (p.n <= 64 || p.m <= 4096) {
    p.tiles_m = static_cast<int>(ceil_div(p.m, 128));
    p.tiles_n = static_cast<int>(ceil_div(p.n, 64));
    hipLaunchKernelGGL((qgemm_kernel<128, 64, 2, 2>), dim3(p.tiles_m * p.tiles_n), dim3(kThreads), 0, s, p);
  } else {
    p.tiles_m = static_cast<int>(ceil_div(p.m, 128));
    p.tiles_n = static_cast<int>(ceil_div(p.n, 128));
    hipLaunchKernelGGL((qgemm_kernel<128, 128, 2, 2>), dim3(p.tiles_m * p.tiles_n), dim3(kThreads), 0, s, p);
  }
  return launch_status("qgemm");
}

}  // extern "C"
