// Attention kernels of libc3hip.so (gfx950).
//
// attention_scores: the reference's FusedAttentionScores contract
//   (c35/engine.py:1250-1380): softmax(Q K^T / divisor + mask) written as a
//   full [B,H,S,S] fp32 tensor.  One workgroup per score row; the Q row is
//   staged in LDS and every dot product is computed once (the reference
//   recomputes each three times).
//
// flash_attention: the launch-grouped FusedAttentionScores + P.V MatMul.  A
//   workgroup owns 128 queries of one (batch, head) (two groups of 16 per
//   wave); K and V tiles of 64 keys are staged in LDS, the next tile's loads
//   in flight while the current one is multiplied.  Each wave computes S^T = K Q^T with
//   v_mfma_f32_16x16x32_{f16,bf16} so that a lane holds one query's scores;
//   the online-softmax state is then per lane and P^T feeds the O^T = V^T P^T
//   MFMA straight from registers (both operands use the same key order, so
//   the product is unchanged).
#include "common.h"

using namespace c3h;

namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

// ------------------------------------------------------------ scores (fp32)
constexpr int kScoreThreads = 256;
constexpr int kMaxCachedCols = 8192;

__global__ void __launch_bounds__(kScoreThreads) attention_scores_kernel(c3h_attn_scores_args a, int out_heads) {
  extern __shared__ float smem[];
  float* qrow = smem;               // [inner]
  float* srow = smem + a.inner;     // [cols] when cached
  __shared__ float red[kScoreThreads / 64];
  const int64_t segment = blockIdx.x;
  int64_t value = segment;
  const int row = static_cast<int>(value % a.rows); value /= a.rows;
  const int head = static_cast<int>(value % out_heads); value /= out_heads;
  const int batch = static_cast<int>(value);
  const int qb = a.q0 == 1 ? 0 : batch, qh = a.q1 == 1 ? 0 : head;
  const int kb = a.k0 == 1 ? 0 : batch, kh = a.k1 == 1 ? 0 : head;
  const int mb = a.m0 == 1 ? 0 : batch, mh = a.m1 == 1 ? 0 : head, mr = a.m2 == 1 ? 0 : row;
  const int64_t qbase = ((static_cast<int64_t>(qb) * a.q1 + qh) * a.rows + row) * a.inner;
  const int64_t kbase = (static_cast<int64_t>(kb) * a.k1 + kh) * static_cast<int64_t>(a.inner) * a.cols;
  const int64_t mbase = ((static_cast<int64_t>(mb) * a.m1 + mh) * a.m2 + mr) * a.m3;
  const float* mask = static_cast<const float*>(a.mask);
  const float divisor = static_cast<const float*>(a.divisor)[0];
  for (int i = threadIdx.x; i < a.inner; i += kScoreThreads) qrow[i] = load_as_f32(a.q, a.in_dtype, qbase + i);
  __syncthreads();
  const bool cached = a.cols <= kMaxCachedCols;
  auto score = [&](int col) {
    float s = 0.0f;
    for (int i = 0; i < a.inner; ++i) s = fmaf(qrow[i], load_as_f32(a.kt, a.in_dtype, kbase + static_cast<int64_t>(i) * a.cols + col), s);
    return s / divisor + mask[mbase + (a.m3 == 1 ? 0 : col)];
  };
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float m = -INFINITY;
  for (int col = threadIdx.x; col < a.cols; col += kScoreThreads) {
    float s = score(col);
    if (cached) srow[col] = s;
    m = fmaxf(m, s);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.0f;
  for (int col = threadIdx.x; col < a.cols; col += kScoreThreads) sum += expf((cached ? srow[col] : score(col)) - m);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  sum = red[0] + red[1] + red[2] + red[3];
  float* out = static_cast<float*>(a.out) + segment * a.cols;
  for (int col = threadIdx.x; col < a.cols; col += kScoreThreads)
    out[col] = expf((cached ? srow[col] : score(col)) - m) / sum;
}

// ------------------------------------------------------------ flash attention
constexpr int kD = 64;        // head dim
constexpr int QG = 2;         // 16-query groups per wave
constexpr int kBQ = 64 * QG;  // queries per workgroup
constexpr int kBK = 64;       // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
// Lazy rescaling: the exponent base of a query moves to its running maximum
// only when some query of the wave has exceeded its base by more than this
// (in exp2 units), so p = exp2(s c - base) <= 2^8, exact in range for the
// 16-bit P operand, and O, l stay consistent with the base they were summed at.
constexpr float kLazy = 8.0f;

template <typename T> struct FlashMma;
template <> struct FlashMma<bf16_t> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct FlashMma<f16_t> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// LDS tiles (128-byte rows, 16-byte chunks XOR-swizzled so every MFMA
// operand is one conflict-free ds_read_b128, as in the GEMM kernels):
//   Ks[key][dim]:  chunk c of row `key` at slot c ^ (key & 7);
//   Vt[dim][pos]:  V transposed, keys permuted by vt_pos so that the eight
//                  keys a lane holds in a P^T fragment (32 ks + 16 (i / 4) +
//                  4 g + i % 4, the S^T accumulator layout) are one chunk
//                  (4 ks + g); chunk slot c ^ vt_swz(dim).
__device__ __forceinline__ int vt_pos(int key) {
  const int r = key & 31;
  return (key & 32) + 8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3);
}
__device__ __forceinline__ int vt_swz(int dim) { return (dim ^ (dim >> 1)) & 7; }

template <typename T> __device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <> __device__ __forceinline__ uint32_t pack2<bf16_t>(float lo, float hi) { return f32x2_to_bf16x2_bits(lo, hi); }
template <> __device__ __forceinline__ uint32_t pack2<f16_t>(float lo, float hi) { return f32x2_to_f16x2_bits(lo, hi); }

// Each wave owns QG groups of 16 queries (kBQ = 64 * QG per workgroup): every
// K / V^T fragment read from LDS feeds QG MFMAs, and the tile staging is
// shared by 4 * 16 * QG queries.
template <typename T, int MASK>
__global__ void __launch_bounds__(256) flash_kernel(c3h_flash_args a) {
  typedef typename FlashMma<T>::vec vec8;
  __shared__ __attribute__((aligned(16))) uint8_t Ks[kBK * 128];
  __shared__ __attribute__((aligned(16))) uint8_t Vt[kD * 128];

  const int qtiles = (a.seq_q + kBQ - 1) / kBQ;
  // Longest first: under the causal mask query tile qt walks qt + 1 key
  // tiles' worth of work per 64 queries, so the last query tiles of every
  // (batch, head) are dispatched first and the short ones fill the gaps they
  // leave (W8A8 decoder layer: 87 -> 55 us against (bh, qt) order).  With
  // n_bh a multiple of 8 all query tiles of one (batch, head) also land on
  // one XCD, whose L2 then holds that head's K and V.
  const int nbh = a.batch * a.heads;
  const int qt = qtiles - 1 - static_cast<int>(blockIdx.x / nbh);
  const int bh = blockIdx.x % nbh;
  const int head = bh % a.heads, batch = bh / a.heads;
  // (`wave` is left as a per-lane value: declaring it uniform made the
  // causal checks scalar branches and the kernel measured 17 % slower.)
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, g = lane >> 4;
  // ds_bpermute byte addresses of lanes lane ^ 16 and lane ^ 32.
  const int xor16 = (lane ^ 16) << 2, xor32 = (lane ^ 32) << 2;

  const uint16_t* Q = static_cast<const uint16_t*>(a.q) + batch * a.q_sb + head * a.q_sh;
  const uint16_t* K = static_cast<const uint16_t*>(a.k) + batch * a.k_sb + head * a.k_sh;
  const uint16_t* V = static_cast<const uint16_t*>(a.v) + batch * a.v_sb + head * a.v_sh;
  uint16_t* O = static_cast<uint16_t*>(a.out) + batch * a.o_sb + head * a.o_sh;

  // This lane's queries (B operand column of S^T = K Q^T), one per group,
  // and their Q fragments: dims 32*ks + 8*g + [0..7].
  const int wave_q0 = qt * kBQ + wave * 16 * QG;  // this wave's first query
  const int wave_q1 = wave_q0 + 16 * QG - 1;      // ... and last
  int q[QG];
  bool q_valid[QG];
  vec8 qf[QG][2];
#pragma unroll
  for (int u = 0; u < QG; ++u) {
    q[u] = wave_q0 + 16 * u + l16;
    q_valid[u] = q[u] < a.seq_q;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint4 raw = {0u, 0u, 0u, 0u};
      if (q_valid[u]) raw = *reinterpret_cast<const uint4*>(Q + q[u] * a.q_ss + 32 * ks + 8 * g);
      qf[u][ks] = __builtin_bit_cast(vec8, raw);
    }
  }

  f32x4 o_acc[QG][4];  // O^T tiles: dims 16*d + 4*g + j, query q[u]
  // Row sums of P by the MFMA: a ones A operand makes every element of
  // l_acc[u] the sum over the tile's keys of query q[u]'s 16-bit P values,
  // the same P values O is summed from.
  f32x4 l_acc[QG];
#pragma unroll
  for (int u = 0; u < QG; ++u) {
    l_acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 4; ++d) o_acc[u][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t one2 = pack2<T>(1.0f, 1.0f);
  const vec8 ones = __builtin_bit_cast(vec8, uint4{one2, one2, one2, one2});
  // Softmax state in raw score units: p = exp2(s * c - base), c = scale * log2 e.
  const float c = a.scale * kLog2e;
  const float inv_scale = 1.0f / a.scale;
  // running max (raw), the max the exponent base was taken at, and the base
  float m_run[QG], m_base[QG], base[QG];
#pragma unroll
  for (int u = 0; u < QG; ++u) {
    m_run[u] = -INFINITY;
    m_base[u] = -INFINITY;
    base[u] = 0.0f;
  }

  const float* mask = static_cast<const float*>(a.mask);
  int kend = a.seq_k;
  if (MASK == 1) {
    int last_q = qt * kBQ + kBQ - 1;
    if (last_q + 1 < kend) kend = last_q + 1;
  }
  const int ntiles = (kend + kBK - 1) / kBK;

  // Staging: K rows (tid >> 3) and (tid >> 3) + 32, chunk tid & 7; V keys
  // kq .. kq + 3 x dims d0 .. d0 + 3, transposed in registers.  The loads are
  // buffer loads at 32-bit byte offsets from this (batch, head)'s K / V
  // (extents below 2^31, checked on the host): keys past seq_k get an
  // offset beyond the buffer and read zeros, so a load costs an add and a
  // select instead of 64-bit address arithmetic and a branch (W8A8 flash
  // family 613 -> 606 us per step, fp16 decoder 139 -> 132 us).  Issuing
  // each tile's loads two tiles ahead from a second register set measured
  // slower (613 -> 711 us): 172 VGPRs leave two waves per SIMD instead of
  // three.
  const int k_row = tid >> 3, k_chunk = tid & 7;
  // (lanes along dims: one V load instruction reads four whole 128-byte key
  // rows, 16 lanes x 8 bytes each)
  const int d0 = 4 * (tid & 15), kq = 4 * (tid >> 4);
  constexpr uint32_t kOob = 0x80000000u;
  const int k_bytes = static_cast<int>(((a.seq_k - 1) * a.k_ss + kD) * 2);
  const int v_bytes = static_cast<int>(((a.seq_k - 1) * a.v_ss + kD) * 2);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(K), 0, k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(V), 0, v_bytes, 0x00020000);
  const uint32_t k_lane = static_cast<uint32_t>(k_row * a.k_ss + 8 * k_chunk) * 2u;
  const uint32_t v_lane = static_cast<uint32_t>(kq * a.v_ss + d0) * 2u;
  uint4 kreg[2];
  uint2 vreg[4];
  auto load_tile = [&](int t) {
    const int k0 = t * kBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = k0 + k_row + 32 * i;
      const uint32_t off = key < a.seq_k ? static_cast<uint32_t>((k0 + 32 * i) * a.k_ss) * 2u + k_lane : kOob;
      kreg[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = k0 + kq + i;
      const uint32_t off = key < a.seq_k ? static_cast<uint32_t>((k0 + i) * a.v_ss) * 2u + v_lane : kOob;
      vreg[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0));
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = k_row + 32 * i;
      *reinterpret_cast<uint4*>(Ks + key * 128 + ((k_chunk ^ (key & 7)) << 4)) = kreg[i];
    }
    const int p = vt_pos(kq);  // multiple of 4: keys kq .. kq + 3 land at p .. p + 3
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int dim = d0 + jj;
      uint32_t e[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = (jj < 2) ? vreg[i].x : vreg[i].y;
        e[i] = (jj & 1) ? (w >> 16) : (w & 0xffffu);
      }
      const uint2 word = uint2{e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
      *reinterpret_cast<uint2*>(Vt + dim * 128 + (((p >> 3) ^ vt_swz(dim)) << 4) + (p & 7) * 2) = word;
    }
  };

  if (ntiles > 0) load_tile(0);
  for (int t = 0; t < ntiles; ++t) {
    const int k0 = t * kBK;
    store_tile();
    __syncthreads();
    if (t + 1 < ntiles) load_tile(t + 1);  // in flight while this tile is multiplied

    // Causal: a tile wholly after this wave's last query contributes nothing.
    if (MASK != 1 || k0 <= wave_q1) {
      // S^T tiles: keys 16*kt4 + 4*g + j (j = 0..3), query q[u].
      f32x4 s_acc[QG][4];
#pragma unroll
      for (int kt4 = 0; kt4 < 4; ++kt4) {
#pragma unroll
        for (int u = 0; u < QG; ++u) s_acc[u][kt4] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int key = 16 * kt4 + l16;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const vec8 kf = *reinterpret_cast<const vec8*>(Ks + key * 128 + (((4 * ks + g) ^ (key & 7)) << 4));
#pragma unroll
          for (int u = 0; u < QG; ++u) s_acc[u][kt4] = FlashMma<T>::mma(kf, qf[u][ks], s_acc[u][kt4]);
        }
      }
      // Key-range and causal checks run only on tiles that reach past seq_k
      // or the wave's first query (a uniform branch).
      const bool edge = (k0 + kBK > a.seq_k) || (MASK == 1 && k0 + kBK - 1 > wave_q0) || MASK == 2;
      vec8 pf[QG][2];
#pragma unroll
      for (int u = 0; u < QG; ++u) {
        float tmax = -INFINITY;
        if (edge && MASK != 2) {
          // key >= seq_k or (causal) key > q[u]  <=>  key >= lim, taken
          // relative to this lane's first key so each score costs one
          // compare against a constant offset.
          int lim = a.seq_k;
          if (MASK == 1 && q[u] + 1 < lim) lim = q[u] + 1;
          lim -= k0 + 4 * g;
#pragma unroll
          for (int kt4 = 0; kt4 < 4; ++kt4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              float sv = s_acc[u][kt4][j];
              if (16 * kt4 + j >= lim) sv = -INFINITY;
              s_acc[u][kt4][j] = sv;
              tmax = fmaxf(tmax, sv);
            }
          }
        } else if (edge) {  // additive mask: every tile
#pragma unroll
          for (int kt4 = 0; kt4 < 4; ++kt4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int key = k0 + 16 * kt4 + 4 * g + j;
              float sv = s_acc[u][kt4][j];
              if (key >= a.seq_k) sv = -INFINITY;
              if (q_valid[u] && key < a.seq_k)
                sv += mask[static_cast<int64_t>(q[u]) * a.mask_ld + key] * inv_scale;
              s_acc[u][kt4][j] = sv;
              tmax = fmaxf(tmax, sv);
            }
          }
        } else {
#pragma unroll
          for (int kt4 = 0; kt4 < 4; ++kt4)
#pragma unroll
            for (int j = 0; j < 4; ++j) tmax = fmaxf(tmax, s_acc[u][kt4][j]);
        }
        tmax = fmaxf(tmax, __int_as_float(__builtin_amdgcn_ds_bpermute(xor16, __float_as_int(tmax))));
        tmax = fmaxf(tmax, __int_as_float(__builtin_amdgcn_ds_bpermute(xor32, __float_as_int(tmax))));
        const float m_new = fmaxf(m_run[u], tmax);
        m_run[u] = m_new;
        // A finite maximum past the base by more than kLazy (any base is
        // exceeded by a finite maximum while the base is still -inf).
        const bool grow = m_new > m_base[u] && (m_base[u] == -INFINITY || (m_new - m_base[u]) * c > kLazy);
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // uniform: the whole wave moves its bases
          const float nb = m_new == -INFINITY ? 0.0f : m_new * c;
          const float corr = m_base[u] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(base[u] - nb);
          m_base[u] = m_new;
          base[u] = nb;
          l_acc[u] *= corr;
#pragma unroll
          for (int d = 0; d < 4; ++d) o_acc[u][d] *= corr;
        }
        // P^T fragments for the two 32-key halves: element i of half ks is
        // key 32*ks + 16*(i/4) + 4*g + (i%4), i.e. s_acc[2*ks + i/4][i%4].
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          float pv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i)
            pv[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_acc[u][2 * ks + i / 4][i % 4], c, -base[u]));
          const uint4 packed = {pack2<T>(pv[0], pv[1]), pack2<T>(pv[2], pv[3]), pack2<T>(pv[4], pv[5]),
                                pack2<T>(pv[6], pv[7])};
          pf[u][ks] = __builtin_bit_cast(vec8, packed);
        }
      }
      // O^T += V^T P^T: A operand = V^T row (dim 16*d + l16), chunk 4*ks + g
      // holds the same eight keys as the lane's P^T fragment.
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int dim = 16 * d + l16;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const vec8 vf = *reinterpret_cast<const vec8*>(Vt + dim * 128 + (((4 * ks + g) ^ vt_swz(dim)) << 4));
#pragma unroll
          for (int u = 0; u < QG; ++u) o_acc[u][d] = FlashMma<T>::mma(vf, pf[u][ks], o_acc[u][d]);
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int u = 0; u < QG; ++u) l_acc[u] = FlashMma<T>::mma(ones, pf[u][ks], l_acc[u]);
    }
    __syncthreads();
  }

  // O rows 16-byte aligned: each pair of dim tiles leaves as one 16-byte
  // store per lane (lane row g: dims 32 pair + 8 g .. + 7 of its query, by
  // the lane swaps of ct_pair_to_rows, which trade values only between
  // lanes of one query); otherwise 8 bytes per lane and tile.
  const bool wide = ((a.o_ss | a.o_sh | a.o_sb) & 7) == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0;
#pragma unroll
  for (int u = 0; u < QG; ++u) {
    const float l_tot = l_acc[u][0];
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    uint32_t pk[4][2];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      pk[d][0] = pack2<T>(o_acc[u][d][0] * inv, o_acc[u][d][1] * inv);
      pk[d][1] = pack2<T>(o_acc[u][d][2] * inv, o_acc[u][d][3] * inv);
    }
    if (wide) {
      const uint4 w0 = ct_pair_to_rows(pk[0], pk[1]), w1 = ct_pair_to_rows(pk[2], pk[3]);
      if (q_valid[u]) {
        *reinterpret_cast<uint4*>(O + q[u] * a.o_ss + 8 * g) = w0;
        *reinterpret_cast<uint4*>(O + q[u] * a.o_ss + 32 + 8 * g) = w1;
      }
    } else if (q_valid[u]) {
#pragma unroll
      for (int d = 0; d < 4; ++d)
        *reinterpret_cast<uint2*>(O + q[u] * a.o_ss + 16 * d + 4 * g) = uint2{pk[d][0], pk[d][1]};
    }
  }
}

}  // namespace

extern "C" {

int c3h_attention_scores(const c3h_attn_scores_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr, "attention_scores: null args");
  C3H_REQUIRE(a->rows >= 0 && a->cols >= 1 && a->inner >= 1, "attention_scores: bad sizes");
  C3H_REQUIRE((a->q0 == 1 || a->k0 == 1 || a->q0 == a->k0) && (a->q1 == 1 || a->k1 == 1 || a->q1 == a->k1),
              "attention_scores: batch/head dims do not broadcast");
  const int out0 = a->q0 > a->k0 ? a->q0 : a->k0;
  const int out1 = a->q1 > a->k1 ? a->q1 : a->k1;
  const int dims[4] = {out0, out1, a->rows, a->cols};
  const int md[4] = {a->m0, a->m1, a->m2, a->m3};
  for (int i = 0; i < 4; ++i)
    C3H_REQUIRE(md[i] == 1 || md[i] == dims[i], "attention_scores: mask dim %d (%d) does not broadcast to %d", i,
                md[i], dims[i]);
  int64_t segments = static_cast<int64_t>(out0) * out1 * a->rows;
  if (segments == 0) return C3H_OK;
  C3H_REQUIRE(segments <= 2147483647LL, "attention_scores: too many rows");
  size_t smem = (static_cast<size_t>(a->inner) + (a->cols <= kMaxCachedCols ? a->cols : 0)) * sizeof(float);
  C3H_REQUIRE(smem <= 64 * 1024, "attention_scores: inner dim too large");
  hipLaunchKernelGGL(attention_scores_kernel, dim3(static_cast<unsigned>(segments)), dim3(kScoreThreads), smem,
                     as_stream(stream), *a, out1);
  return launch_status("attention_scores");
}

int c3h_flash_attention(const c3h_flash_args* a, void* stream) {
  C3H_REQUIRE(a != nullptr, "flash: null args");
  C3H_REQUIRE(a->head_dim == kD, "flash: head_dim %d unsupported (needs 64)", a->head_dim);
  C3H_REQUIRE(a->batch >= 0 && a->heads >= 1 && a->seq_q >= 0 && a->seq_k >= 1, "flash: bad sizes");
  C3H_REQUIRE(a->mask_kind >= 0 && a->mask_kind <= 2, "flash: bad mask_kind");
  C3H_REQUIRE(a->mask_kind != 2 || a->mask != nullptr, "flash: additive mask pointer missing");
  C3H_REQUIRE(a->scale > 0.0f, "flash: scale must be positive");
  C3H_REQUIRE(a->q_ss % 8 == 0 && a->k_ss % 8 == 0 && a->v_ss % 8 == 0 && a->q_sh % 8 == 0 && a->k_sh % 8 == 0 &&
                  a->v_sh % 8 == 0 && a->q_sb % 8 == 0 && a->k_sb % 8 == 0 && a->v_sb % 8 == 0,
              "flash: Q/K/V strides must be multiples of 8 elements");
  C3H_REQUIRE(a->o_ss % 4 == 0 && a->o_sh % 4 == 0 && a->o_sb % 4 == 0, "flash: out strides must be multiples of 4");
  C3H_REQUIRE((reinterpret_cast<uintptr_t>(a->q) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->k) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(a->v) & 15) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 7) == 0,
              "flash: misaligned operands");
  // K and V rows of one (batch, head) are read with 32-bit buffer offsets
  C3H_REQUIRE((static_cast<int64_t>(a->seq_k - 1) * a->k_ss + kD) * 2 < (int64_t{1} << 31) &&
                  (static_cast<int64_t>(a->seq_k - 1) * a->v_ss + kD) * 2 < (int64_t{1} << 31),
              "flash: one head's K or V spans 2 GiB or more");
  if (a->batch == 0 || a->seq_q == 0) return C3H_OK;
  int64_t blocks = static_cast<int64_t>(a->batch) * a->heads * ((a->seq_q + kBQ - 1) / kBQ);
  C3H_REQUIRE(blocks <= 2147483647LL, "flash: too many workgroups");
  hipStream_t s = as_stream(stream);
  dim3 grid(static_cast<unsigned>(blocks));
#define C3H_FLASH_LAUNCH(T)                                                                            \
  switch (a->mask_kind) {                                                                              \
    case 0: hipLaunchKernelGGL((flash_kernel<T, 0>), grid, dim3(256), 0, s, *a); break;                \
    case 1: hipLaunchKernelGGL((flash_kernel<T, 1>), grid, dim3(256), 0, s, *a); break;                \
    default: hipLaunchKernelGGL((flash_kernel<T, 2>), grid, dim3(256), 0, s, *a); break;               \
  }
  if (a->dtype == C3H_BF16) {
    C3H_FLASH_LAUNCH(bf16_t)
  } else if (a->dtype == C3H_F16) {
    C3H_FLASH_LAUNCH(f16_t)
  } else {
    return fail(C3H_EUNSUPPORTED, "flash: dtype %d unsupported", a->dtype);
  }
#undef C3H_FLASH_LAUNCH
  return launch_status("flash_attention");
}

}  // extern "C"
