/*
 * c3hip.h -- C ABI of libc3hip.so, the MI355X (gfx950) execution backend for
 * the C3 ONNX inference compiler's numerical path.
 *
 * Boundary.  The reference executes every planned kernel step through
 *     kernel_registry.lookup(name)(inputs, outputs, params, tuning)
 * (c32/kernel_registry.py:6-17, called from c35/executor.py:576-581) and owns
 * one byte arena, persistent streams and per-plan events
 * (c35/executor.py:673-709, 757-765).  This library replaces everything below
 * that call: the arena becomes one hipMalloc slab, logical streams become
 * hipStream_t, plan events become hipEvent_t, and every registry body becomes a
 * hand-written gfx950 kernel family below.  Python binds it with ctypes
 * (hackathon_amd/_lib.py); no torch or CUDA types appear in any signature.
 *
 * Conventions.
 *   - Every entry point returns int: 0 = OK, C3H_EINVAL (-1) = invalid
 *     argument, C3H_EUNSUPPORTED (-2) = a shape/dtype combination this build
 *     does not implement, C3H_EHIP (-3) = a HIP runtime error.  The message of
 *     the last failure on the calling thread is returned by c3h_last_error().
 *   - Kernel entry points are asynchronous on the given stream (NULL = the
 *     null stream).  The library never frees caller memory.
 *   - Tensors are dense.  Shapes/strides are in elements, row-major, unless a
 *     field says otherwise.  All pointers are device pointers except where a
 *     name says "host".
 */
#ifndef C3HIP_H
#define C3HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define C3H_OK 0
#define C3H_EINVAL (-1)
#define C3H_EUNSUPPORTED (-2)
#define C3H_EHIP (-3)

#define C3H_MAX_RANK 8
#define C3H_EW_MAX_IN 8
#define C3H_EW_MAX_INST 16

/* Element types (storage). */
enum c3h_dtype {
  C3H_F32 = 0,
  C3H_F16 = 1,
  C3H_BF16 = 2,
  C3H_I8 = 3,
  C3H_I32 = 4,
  C3H_I64 = 5,
  C3H_U8 = 6,
  C3H_BOOL = 7,
  C3H_F64 = 8
};

/* Elementwise opcodes of the fused elementwise program.  The set mirrors the
 * ops a FusedEWChain may hold (c33/fusion.py:20-22, c35/engine.py:959-968)
 * plus the unfused registry unaries (c32/kernel_registry.py:200-265). */
enum c3h_ew_opcode {
  C3H_EW_ADD = 0,
  C3H_EW_SUB = 1,
  C3H_EW_MUL = 2,
  C3H_EW_DIV = 3,
  C3H_EW_RELU = 4,
  C3H_EW_ERF = 5,      /* ROCm device-library erff (fused chains, engine.py:965) */
  C3H_EW_ERF_AS = 6,   /* Abramowitz & Stegun 7.1.26 (kernel_registry.py:180-193) */
  C3H_EW_SQRT = 7,
  C3H_EW_EXP = 8,
  C3H_EW_RECIP = 9,
  C3H_EW_MAX = 10,
  C3H_EW_MIN = 11,
  C3H_EW_NEG = 12,
  C3H_EW_ADD_IMM = 13, /* a + imm   (LayerNorm's "add epsilon" step, decompositions.py:207) */
  C3H_EW_MUL_IMM = 14, /* a * imm */
  C3H_EW_COPY = 15
};

/* ------------------------------------------------------------------ */
/* Device, memory, streams, events                                      */
/* ------------------------------------------------------------------ */

typedef struct {
  char name[256];
  char arch[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;
  int32_t warp_size;
  int32_t max_threads_per_block;
  int32_t max_block_dim_x;
  int32_t max_grid_dim_x;
  int32_t lds_bytes_per_block;
  int32_t clock_khz;
  int32_t memory_clock_khz;
  int32_t memory_bus_width;
  int32_t l2_bytes;
  int64_t total_memory_bytes;
  int32_t major;
  int32_t minor;
} c3h_props;

/* Replaces c32/hardware.py:97-163 (from_cuda_properties) as the device query. */
int c3h_init(int device);
int c3h_device_count(int* count);
int c3h_device_props(int device, c3h_props* out);
const char* c3h_last_error(void);
int c3h_device_synchronize(void);
/* Re-reads the kernel-selection switches (C3H_DISABLE_DMA, C3H_DISABLE_BIGTILE,
 * C3H_DISABLE_BUF, C3H_DISABLE_CONV3X3, C3H_DISABLE_DIRECT_CONV, C3H_DMA_RP)
 * from the environment.
 * They are read once, at the first launch, otherwise; call this between
 * launches after changing them, never while another thread launches.  No
 * counterpart in the reference (its kernel choice has no switches). */
int c3h_reload_switches(void);

/* One slab per plan arena (replaces cp.empty(peak_reserved_bytes), c35/executor.py:761-765). */
int c3h_malloc(void** ptr, size_t bytes);
int c3h_free(void* ptr);
/* Pinned host staging (replaces cp.cuda.alloc_pinned_memory, c35/executor.py:496, 854). */
int c3h_host_alloc(void** ptr, size_t bytes);
int c3h_host_free(void* ptr);
int c3h_memcpy_h2d_async(void* dst, const void* host_src, size_t bytes, void* stream);
int c3h_memcpy_d2h_async(void* host_dst, const void* src, size_t bytes, void* stream);
int c3h_memcpy_d2d_async(void* dst, const void* src, size_t bytes, void* stream);
/* Synchronous helpers (host buffers may be pageable). */
int c3h_memcpy_h2d(void* dst, const void* host_src, size_t bytes);
int c3h_memcpy_d2h(void* host_dst, const void* src, size_t bytes);

/* Persistent logical streams (c35/executor.py:685-692).  All streams are
 * created at the default priority. */
int c3h_stream_create(void** stream);
int c3h_stream_destroy(void* stream);
int c3h_stream_synchronize(void* stream);
/* Plan events (c35/executor.py:694-702, 798-801). */
int c3h_event_create(void** event, int timing);
int c3h_event_destroy(void* event);
int c3h_event_record(void* event, void* stream);
int c3h_stream_wait_event(void* stream, void* event);
int c3h_event_synchronize(void* event);
int c3h_event_elapsed_ms(float* ms, void* start, void* stop);

/* ------------------------------------------------------------------ */
/* Memory-bound kernel families                                         */
/* ------------------------------------------------------------------ */

/* Fill `count` elements of `dtype` with `value` (a graph-capture-safe memset). */
typedef struct {
  void* out;
  int64_t count;
  int32_t dtype;
  int32_t pad_;
  double value;
} c3h_fill_args;
int c3h_fill(const c3h_fill_args* a, void* stream);

/* Dtype conversion of `count` elements, round-to-nearest-even for narrowing
 * float conversions. */
typedef struct {
  const void* in;
  void* out;
  int64_t count;
  int32_t in_dtype;
  int32_t out_dtype;
} c3h_cast_args;
int c3h_cast(const c3h_cast_args* a, void* stream);

/* Broadcast elementwise program.  Registers 0..n_in-1 hold the inputs
 * (converted to fp32); instruction i writes register n_in+i.  `stride[j][d]`
 * is input j's element stride for output dim d (0 = broadcast).  Replaces
 * kernel_add/sub/mul/div/relu/erf/exp/sqrt/reciprocal (kernel_registry.py:
 * 200-265), kernel_fused_residual_relu (:654-662) and op_fused_ew_chain
 * (c35/engine.py:948-1013). */
typedef struct {
  int32_t op;
  int32_t a;
  int32_t b;
  int32_t pad_;
  float imm;
  float pad2_;
} c3h_ew_inst;

typedef struct {
  const void* in[C3H_EW_MAX_IN];
  int32_t in_dtype[C3H_EW_MAX_IN];
  int64_t stride[C3H_EW_MAX_IN][C3H_MAX_RANK];
  void* out;
  int32_t out_dtype;
  int32_t rank;
  int64_t shape[C3H_MAX_RANK];
  int32_t n_in;
  int32_t n_inst;
  c3h_ew_inst inst[C3H_EW_MAX_INST];
} c3h_ew_args;
int c3h_ew(const c3h_ew_args* a, void* stream);

/* Strided copy: out (dense, `shape`) <- in at `in_stride` (elements), any
 * element size.  Implements transpose / fused transpose-reshape / split /
 * NHWO->NCHW conv reshape (kernel_registry.py:105-175, 365-372, 697-741;
 * c35/engine.py:1383-1445). */
typedef struct {
  const void* in;
  void* out;
  int32_t elem_bytes;
  int32_t rank;
  int64_t shape[C3H_MAX_RANK];
  int64_t in_stride[C3H_MAX_RANK];
  int64_t in_offset;
} c3h_copy_args;
int c3h_strided_copy(const c3h_copy_args* a, void* stream);

/* Reduction of a tensor viewed as [outer, reduce, inner] (contiguous
 * reduce-axis block).  kind: 0 max, 1 sum, 2 mean (kernel_registry.py:
 * 272-311; GlobalAveragePool decompositions.py:381-391). */
typedef struct {
  const void* in;
  void* out;
  int64_t outer;
  int64_t reduce;
  int64_t inner;
  int32_t kind;
  int32_t in_dtype;
  int32_t out_dtype;
  int32_t pad_;
} c3h_reduce_args;
int c3h_reduce(const c3h_reduce_args* a, void* stream);

/* Stable softmax along an axis of a tensor viewed as [outer, axis, inner]
 * (c35/engine.py:1016-1075, 634-650). */
typedef struct {
  const void* in;
  void* out;
  int64_t outer;
  int64_t axis;
  int64_t inner;
  int32_t in_dtype;
  int32_t out_dtype;
} c3h_softmax_args;
int c3h_softmax(const c3h_softmax_args* a, void* stream);

/* LayerNorm over the trailing `cols` of each of `rows` rows, with optional
 * residual added first (FusedResidualNorm), optional bias, optional mean and
 * inverse-std outputs (c35/engine.py:484-532, 1078-1247).
 * out_dtype C3H_I8: the QuantizeLinear that consumes the LayerNorm, fused
 * (W8A8 pre-LN inputs): each output is rounded to x_dtype -- the value the
 * unfused LayerNorm would store -- then q = saturate(rne(y / out_scale) +
 * out_zero), the codes c3h_quantize would produce from that stored value.
 * Needs cols % 8 == 0 and cols <= 4096. */
typedef struct {
  const void* x;
  const void* residual; /* may be NULL */
  const void* scale;    /* fp32 [cols] */
  const void* bias;     /* fp32 [cols] or NULL */
  void* out;
  void* mean_out;       /* fp32 [rows] or NULL */
  void* invstd_out;     /* fp32 [rows] or NULL */
  int64_t rows;
  int64_t cols;
  float epsilon;
  int32_t x_dtype;
  int32_t out_dtype;
  float out_scale;      /* out_dtype C3H_I8 only */
  int32_t out_zero;     /* out_dtype C3H_I8 only */
  int32_t pad_;
} c3h_layernorm_args;
int c3h_layernorm(const c3h_layernorm_args* a, void* stream);

/* Inference BatchNorm on NCHW (kernel_registry.py:573-584). */
typedef struct {
  const void* x;
  const void* scale;
  const void* bias;
  const void* mean;
  const void* var;
  void* out;
  int64_t n;
  int64_t c;
  int64_t hw;
  float epsilon;
  int32_t pad_;
} c3h_batchnorm_args;
int c3h_batchnorm(const c3h_batchnorm_args* a, void* stream);

/* Conv+BN parameter fold on device (c35/executor.py:400-411):
 * f = scale/sqrt(var+eps); w' = w*f[o]; b' = (b_conv - mean)*f + bias. */
typedef struct {
  const float* w;
  const float* conv_bias; /* may be NULL (zeros) */
  const float* scale;
  const float* bias;
  const float* mean;
  const float* var;
  float* w_out;
  float* b_out;
  int64_t out_channels;
  int64_t per_channel; /* C/group * kh * kw */
  float epsilon;
  int32_t pad_;
} c3h_bnfold_args;
int c3h_bn_fold(const c3h_bnfold_args* a, void* stream);

/* Gather along an axis: data viewed as [outer, axis_dim, inner] elements of
 * `elem_bytes`; int64 indices (negative wrap, out-of-range -> error flag).
 * Bit-exact row copy (kernel_registry.py:744-752, c35/engine.py:462-481).
 * If `error_flag` is non-NULL the kernel writes 1 there on a bad index (the
 * flag is never cleared by the library; out-of-range rows are written as 0).
 *
 * Optional fused addend (the decoder's token + positional embedding, the
 * Gather -> Add pair of c35/engine.py:462-481 and :226-244, in one pass):
 * when `addend` is non-NULL, outer must be 1 and `dtype` (F32, BF16 or F16)
 * names the element type of data and out; `addend_dtype` that of the addend,
 * either F32 or `dtype`.  Output row r is data[idx[r]] + addend[r %
 * addend_rows], added in fp32 and rounded once to `dtype` -- with an F32
 * addend, exactly what a 16-bit Gather followed by an Add of the fp32 table
 * stores.  `addend` is [addend_rows, inner]. */
typedef struct {
  const void* data;
  const int64_t* indices;
  void* out;
  int32_t* error_flag;
  int64_t outer;
  int64_t axis_dim;
  int64_t inner;
  int64_t n_indices;
  int32_t elem_bytes;
  int32_t dtype;
  const void* addend;
  int64_t addend_rows;
  int32_t addend_dtype;
  int32_t pad_;
} c3h_gather_args;
int c3h_gather(const c3h_gather_args* a, void* stream);

/* Argmax along the last axis of [rows, cols], first index of the maximum
 * (NumPy tie rule; harness argmax, c35/standard_runner.py:409). */
typedef struct {
  const void* in;
  int64_t* out;
  int64_t rows;
  int64_t cols;
  int32_t in_dtype;
  int32_t pad_;
} c3h_argmax_args;
int c3h_argmax(const c3h_argmax_args* a, void* stream);

/* One 64-column block of a GEMM output row (the epilogue's row_max side
 * output): the block's largest stored value ignoring NaN, and whether it may
 * hold a NaN. */
typedef struct c3h_block_max {
  float max;
  int32_t nan;
} c3h_block_max;

/* ArgMax of the rows of a GEMM output from its row_max side output: out[m] =
 * c3h_argmax's result for row m of `in` ([rows, cols], row stride in_ld,
 * in_dtype fp32 / bf16 / fp16, as stored), found from the n_parts =
 * ceil(cols / 64) block maxima of the row (row stride ld) and a read of
 * only the blocks that can hold the answer: those equal to the row's
 * maximum, or, when a block may hold a NaN, the NaN-flagged ones in order
 * (NaN is the maximum; first index on ties).  No counterpart in the
 * reference, whose ArgMax reads the logits (c35/standard_runner.py:409). */
typedef struct {
  const c3h_block_max* parts;
  const void* in;
  int64_t* out;
  int64_t rows;
  int64_t cols;
  int64_t n_parts;
  int64_t ld;
  int64_t in_ld;
  int32_t in_dtype;
  int32_t pad_;
} c3h_argmax_finish_args;
int c3h_argmax_finish(const c3h_argmax_finish_args* a, void* stream);

/* Output check of load_and_infer: writes 1 to *flag when any of the `count`
 * values at `x` (dtype F32, BF16 or F16) is NaN or +-Inf, and leaves it
 * untouched otherwise (clear it first).  The device counterpart of
 * cp.isfinite(final).all() (c35/executor.py:1177); it lets the host drain the
 * logits without scanning them. */
typedef struct {
  const void* x;
  int32_t* flag;
  int64_t count;
  int32_t dtype;
  int32_t pad_;
} c3h_nonfinite_args;
int c3h_nonfinite(const c3h_nonfinite_args* a, void* stream);

/* im2col with the reference's ordering: rows (n, ho, wo), columns (c, kh, kw),
 * zero padding (kernel_registry.py:399-453).  Input NCHW. */
typedef struct {
  const void* x;
  void* out;
  int32_t n, c, h, w;
  int32_t kh, kw, sh, sw, pad_top, pad_left, dh, dw;
  int32_t ho, wo;
  int32_t dtype;
  int32_t pad_;
} c3h_im2col_args;
int c3h_im2col(const c3h_im2col_args* a, void* stream);

/* Layout conversion between NCHW and NHWC (with channel zero-padding to
 * c_pad on the NHWC side) and optional dtype change.  direction 0: NCHW->NHWC,
 * 1: NHWC->NCHW. */
typedef struct {
  const void* in;
  void* out;
  int32_t n, c, h, w;
  int32_t c_pad;
  int32_t direction;
  int32_t in_dtype;
  int32_t out_dtype;
} c3h_layout_args;
int c3h_layout(const c3h_layout_args* a, void* stream);

/* Pack Conv weights [o][c][kh][kw] into the implicit-GEMM B layout
 * out[o][k_stride] with K ordered (kh, kw_pack, c_pack), zero where
 * c >= c, kw >= kw or k >= kh*kw_pack*c_pack; optional dtype change. */
typedef struct {
  const void* w;
  void* out;
  int32_t o, c, kh, kw;
  int32_t c_pack, kw_pack;
  int64_t k_stride;
  int32_t in_dtype;
  int32_t out_dtype;
} c3h_pack_args;
int c3h_pack_conv_weight(const c3h_pack_args* a, void* stream);

/* Max pooling 2-D (ONNX MaxPool; padding acts as -inf).  layout 0 NCHW, 1 NHWC
 * (channels padded to c_stride). */
typedef struct {
  const void* x;
  void* out;
  int32_t n, c, h, w;
  int32_t kh, kw, sh, sw, pad_top, pad_left, dh, dw;
  int32_t ho, wo;
  int32_t layout;
  int32_t c_stride;
  int32_t dtype;
  int32_t pad_;
} c3h_pool_args;
int c3h_maxpool2d(const c3h_pool_args* a, void* stream);

/* ------------------------------------------------------------------ */
/* Contractions                                                          */
/* ------------------------------------------------------------------ */

/* Epilogue applied to every GEMM / conv output element, in this order
 * (matching c35/engine.py:818-825 and the fused-node attribute ABI):
 *   v = alpha * acc
 *   v += beta * bias[...]          (bias_mode: 0 none, 1 scalar, 2 per-column
 *                                   [n], 3 per-row [m], 4 full [m, n])
 *   v += residual[...]             (if residual != NULL; same layout as out)
 *   v = act(v)                     (act: 0 none, 1 relu, 2 gelu as the ONNX
 *                                   chain Div->Erf->Add->Mul->Mul computes it:
 *                                   (v * (erf(v / imm[0]) + imm[1])) * imm[2])
 *   v = program(v)                 (n_inst > 0: a linear elementwise program;
 *                                   each instruction's operands a/b select
 *                                   0 = x (the value entering the program),
 *                                   1 = the previous instruction's result
 *                                   (x before the first), 2 + j = imm[j];
 *                                   the last result is the output)
 * Side output (row_max != NULL): for every output row m and every 64-column
 * block b, row_max[m * row_max_ld + b] = {the largest of the block's values
 * as stored, ignoring NaN (-inf if there is none); nan != 0 if the block may
 * hold a NaN (it does, or it holds an infinity)} -- what c3h_argmax_finish
 * completes an ArgMax of the rows from, reading only the few blocks that
 * can hold the answer.  It lets a GEMM that produces logits skip re-reading
 * them for the ArgMax that follows (the harness argmax,
 * c35/standard_runner.py:409).  Taken by c3h_gemm (16-bit inputs),
 * c3h_qgemm (modes 2 / 3), c3h_gemm_fp8 and c3h_gemm_w4a16 with batch 1,
 * a float output (fp32 / bf16 / fp16, row stride a multiple of 4, 4-element
 * aligned), alpha = beta = 1, bias none or per column, act <= 1 and no
 * program; refused elsewhere.  row_max_ld >= ceil(n / 64).
 */
typedef struct {
  const void* bias;      /* fp32 */
  const void* residual;  /* out_dtype, strided like out */
  float alpha;
  float beta;
  int32_t bias_mode;
  int32_t act;
  int32_t n_imm;
  int32_t n_inst;
  float imm[8];
  c3h_ew_inst inst[C3H_EW_MAX_INST];
  struct c3h_block_max* row_max; /* optional side output, see above */
  int64_t row_max_ld;            /* entries between rows of row_max */
} c3h_epilogue;

/* General (batched) GEMM: out[b] = epi(op(A[b]) op(B[b])).
 * A is [m, k] (trans_a=0, row stride lda) or [k, m] (trans_a=1); B is [k, n]
 * (trans_b=0, row stride ldb) or [n, k] (trans_b=1).  Batch strides may be 0
 * (broadcast).  Replaces kernel_matmul (kernel_registry.py:318-358) and the
 * gemm epilogue kernel (c35/engine.py:722-844).  in_dtype applies to A and B
 * (F32 -> fp32 MFMA 16x16x4; F16/BF16 -> MFMA 16x16x32 with fp32
 * accumulation); out_dtype F32/F16/BF16. */
typedef struct {
  const void* a;
  const void* b;
  void* out;
  int64_t m, n, k;
  int64_t lda, ldb, ldo;
  int64_t batch;
  int64_t stride_a, stride_b, stride_out, stride_bias, stride_res;
  int32_t trans_a;
  int32_t trans_b;
  int32_t in_dtype;
  int32_t out_dtype;
  c3h_epilogue epi;
} c3h_gemm_args;
int c3h_gemm(const c3h_gemm_args* a, void* stream);

/* Implicit-GEMM Conv2d: activations channels-last (NHWC, channel stride
 * c_stride >= c, padded channels must be zero), weights pre-packed as
 * [o][kh][kw][c_pack] (c_pack >= c, zero padded), output NHWC [n,ho,wo,o]
 * (out_layout 1) or NCHW (out_layout 0).  GEMM view: M = n*ho*wo, N = o,
 * K = kh*kw*c_pack.  Group must be 1.  Replaces im2col + conv_contract +
 * conv_reshape + add_bias (+relu / +residual relu) of one Conv node
 * (c32/decompositions.py:300-375, kernel_registry.py:318-453).
 * 16-bit 3x3 / stride 1 / pad 1 convs with c = c_pack = c_stride = o = 64,
 * NHWC output, width <= 78 and a bias / residual / ReLU epilogue run on a
 * spatially tiled kernel whose results are bit-identical to the
 * implicit-GEMM path (the environment variable C3H_DISABLE_CONV3X3 selects
 * the latter).  fp32 convs with c_pack = c_stride = 4, NHWC output and
 * o = 16, 32, 64, 128 or 256 run on a direct kernel (VALU FMAs in K order;
 * C3H_DISABLE_DIRECT_CONV selects the implicit GEMM). */
typedef struct {
  const void* x;
  const void* w;
  void* out;
  int32_t n, c, h, w_;
  int32_t c_stride;  /* NHWC channel stride of x */
  int32_t c_pack;    /* channel count of packed weights */
  int32_t o;
  int32_t kh, kw, sh, sw, pad_top, pad_left, dh, dw;
  int32_t ho, wo;
  int32_t out_layout;
  int32_t in_dtype;  /* F32 or BF16 / F16 (x and w) */
  int32_t out_dtype;
  int32_t pad_;
  c3h_epilogue epi;  /* bias_mode 2 = per output channel */
} c3h_conv_args;
int c3h_conv2d(const c3h_conv_args* a, void* stream);

/* Fused network stem: Conv 7x7 / stride 2 / pad 3 (c <= 3 input channels,
 * 64 output channels) + per-channel bias (folded BatchNorm) + optional ReLU
 * + MaxPool 3x3 / stride 2 / pad 1.  x is NCHW (F32, BF16 or F16, rounded to
 * mm_dtype on load); w is the narrow-channel packing of c3h_conv2d
 * ([64][kh][kw_pack = 8][c_pack = 4], k_stride 224); out is NHWC
 * [n, po, qo, 64] in mm_dtype (each pooled window's centre conv pixel must
 * lie inside [ho, wo]).  Bit-identical to layout -> c3h_conv2d
 * (bias, relu) -> c3h_maxpool2d (without ReLU: for a finite bias; the
 * kernel pools before the bias, which commutes with the pool for every
 * finite bias); replaces that chain for the Conv
 * (+BatchNormalization) + Relu + MaxPool nodes of c32/decompositions.py
 * :300-375 and the MaxPool that the reference registry lacks. */
typedef struct {
  const void* x;
  const void* w;
  const float* bias; /* [64] or NULL */
  void* out;
  int32_t n, c, h, w_;
  int32_t o, k_stride;
  int32_t kh, kw, sh, sw, pad_top, pad_left;
  int32_t ho, wo;    /* conv output size */
  int32_t pkh, pkw, psh, psw, ppad_top, ppad_left;
  int32_t po, qo;    /* pooled output size */
  int32_t relu;
  int32_t in_dtype;
  int32_t mm_dtype;  /* BF16 or F16: MFMA operands and output */
  int32_t pad_;
} c3h_conv_pool_args;
int c3h_conv_stem_pool(const c3h_conv_pool_args* a, void* stream);

/* Fused attention scores: softmax(Q K^T / divisor + mask) materialized, with
 * NumPy broadcast of batch/head dims and a rank<=4 mask
 * (c35/engine.py:1250-1380).  Q [q0,q1,rows,inner], Kt [k0,k1,inner,cols]. */
typedef struct {
  const void* q;
  const void* kt;
  const void* divisor;  /* fp32 scalar (device) */
  const void* mask;     /* fp32 */
  void* out;            /* fp32 [max(q0,k0), max(q1,k1), rows, cols] */
  int32_t q0, q1, k0, k1, rows, cols, inner;
  int32_t m0, m1, m2, m3;
  int32_t in_dtype;
} c3h_attn_scores_args;
int c3h_attention_scores(const c3h_attn_scores_args* a, void* stream);

/* Flash attention: out = softmax(Q K^T * scale + mask) V computed with an
 * online softmax, never materializing the scores.  Launch-grouped form of
 * FusedAttentionScores followed by its P.V MatMul (c33/fusion.py:1223-1314,
 * c35/engine.py:1250-1380, kernel_registry.py:345-353).  Q, K, V and out are
 * [B,H,S,D] tensors given by (batch, head, seq) element strides with unit
 * stride along D, so head-split views of a packed QKV buffer and a
 * [B,S,H*D] output need no copies.  mask_kind: 0 none, 1 causal (key > query
 * masked), 2 additive fp32 mask [Sq,Sk] (row stride mask_ld).  D must be 64;
 * dtype F16 or BF16 (fp32 scores and softmax state).  One head's K rows
 * ((seq_k - 1) * k_ss + 64 elements) and V rows must each span under 2 GiB. */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  const void* mask;
  void* out;
  int32_t batch, heads, seq_q, seq_k, head_dim;
  int32_t dtype;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t mask_ld;
  float scale;          /* multiplies Q.K (1/divisor) */
  int32_t mask_kind;
} c3h_flash_args;
int c3h_flash_attention(const c3h_flash_args* a, void* stream);

/* ------------------------------------------------------------------ */
/* W8A8 (QuantizeLinear / QLinearMatMul / DequantizeLinear)             */
/* ------------------------------------------------------------------ */

/* q = saturate(round_half_even(x / scale) + zero_point) into int8
 * (ONNX QuantizeLinear, per-tensor scale). */
typedef struct {
  const void* x;
  int8_t* out;
  int64_t count;
  float scale;
  int32_t zero_point;
  int32_t x_dtype;
  int32_t pad_;
} c3h_quantize_args;
int c3h_quantize(const c3h_quantize_args* a, void* stream);

/* int8 GEMM with exact int32 accumulation: acc[m,n] = sum_k (A[m,k]-za) *
 * (B[n,k]-zb); B packed [n][k] (transB).  mode 0: write int32 acc; mode 1:
 * requantize y = saturate(rne(acc * a_scale * b_scale[n] / y_scale) + zy)
 * to int8 (QLinearMatMul); mode 2: dequantize to float out_dtype
 * v = acc * (a_scale * b_scale[n]) then the epilogue (bias, act/program);
 * mode 3: QLinearMatMul followed by DequantizeLinear(y_scale, y_zero) --
 * the mode-1 int8 y, then v = (y - zy) * y_scale, then the epilogue.
 * Modes 2 and 3 with out_dtype C3H_I8 also apply the QuantizeLinear that
 * consumes the epilogue's output: each value is rounded to act_dtype (F32,
 * BF16 or F16: the type the unfused epilogue would store), then
 * out = saturate(rne(v / q_scale) + q_zero) -- the codes the separate
 * c3h_quantize of that stored tensor gives.  No residual with this form.
 * (The QuantizeLinear after W8A8's FFN1 GELU, ahead of FFN2's QLinearMatMul.) */
typedef struct {
  const int8_t* a;
  const int8_t* b;
  void* out;
  int64_t m, n, k;
  int64_t lda, ldb, ldo;
  int32_t a_zero;
  int32_t b_zero;
  float a_scale;
  float y_scale;
  const float* b_scale; /* [n] */
  int32_t y_zero;
  int32_t mode;
  int32_t out_dtype;
  int32_t act_dtype;  /* modes 2 / 3 with an int8 out: see above */
  float q_scale;
  int32_t q_zero;
  c3h_epilogue epi;
} c3h_qgemm_args;
int c3h_qgemm(const c3h_qgemm_args* a, void* stream);

/* y = (q - zero_point) * scale (ONNX DequantizeLinear, per-tensor). */
typedef struct {
  const int8_t* q;
  void* out;
  int64_t count;
  float scale;
  int32_t zero_point;
  int32_t out_dtype;
  int32_t pad_;
} c3h_dequantize_args;
int c3h_dequantize(const c3h_dequantize_args* a, void* stream);

/* Split-K finish of a GEMM whose K range was cut into `splits` batched
 * partial products (c3h_gemm with batch = splits, K/splits per batch, fp32
 * output [splits][m][n]): out = epilogue(sum_s partial[s]) summed in s
 * order, then the common epilogue into fp32 / bf16 / fp16 (residual in the
 * output dtype, row stride ldo).  Lets the compiled engine spread a GEMM
 * with few output tiles (the MLP's 256-row layers, fused_gemm_epilogue_f32,
 * R:606-633) over every CU; deterministic for a given split. */
typedef struct {
  const float* partial; /* [splits][m][n] */
  void* out;
  int64_t m, n, ldo;
  int32_t splits;
  int32_t out_dtype;
  c3h_epilogue epi;
} c3h_splitk_args;
int c3h_gemm_splitk_reduce(const c3h_splitk_args* a, void* stream);

/* Split-K GEMM in one call, over a caller workspace: the GEMM of `a`
 * (batch 1) cut along K into `splits` partial GEMMs of K/splits each, fp32
 * partials written to `workspace` ([splits][m][n], splits*m*n*4 bytes,
 * 16-byte aligned), then the ordered reduce of c3h_gemm_splitk_reduce with
 * a's epilogue into a->out.  The same two launches the compiled engine
 * issues for a GEMM with too few output tiles to fill the chip (the MLP,
 * the ResNet-18 224 classifier; fused_gemm_epilogue_f32, R:606-633), for
 * callers outside the compiled engine.  k must be a multiple of splits
 * (1 <= splits <= 64; 16-bit inputs: K/splits a multiple of 8); the
 * workspace is written before it is read.  Deterministic for a given split. */
int c3h_gemm_splitk(const c3h_gemm_args* a, int32_t splits, void* workspace, size_t workspace_bytes,
                    void* stream);

/* c3h_gemm_splitk with no workspace and no allocation: the fp32 partials go
 * to a static 32 MiB device array of the library (one per GPU, held until
 * the process ends; its address is resolved per device by c3h_init or the
 * first call on that device).  No counterpart in the reference: it is for
 * callers that cannot allocate -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Same kernels and result
 * as c3h_gemm_splitk.  Fails with C3H_EINVAL, launching nothing, when the
 * partials (splits*m*n*4 bytes) exceed 32 MiB.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (e.g. on two streams)
 * race.  The partials are fully written before they are read, so the
 * array's previous contents never matter. */
int c3h_gemm_splitk_noalloc(const c3h_gemm_args* a, int32_t splits, void* stream);

/* ------------------------------------------------------------------ */
/* fp8 (OCP E4M3) GEMM: the executable form of the reference's         */
/* structural `matmul_f8` (c32/hardware.py:80-81), chosen by the mixed  */
/* policy for aligned GEMMs (c32/strategy.py:150-157) with fp32         */
/* accumulation (c32/strategy.py:103-108).                              */
/* ------------------------------------------------------------------ */

/* Row-wise dynamic quantization to E4M3: per row r, amax = max |x[r,:]|,
 * scale[r] = amax / 448, out[r,k] = E4M3(x[r,k] * min(448 / amax, FLT_MAX))
 * (round to nearest even, saturating at +-448).  A zero row gives scale 0
 * and zero codes; a row holding Inf/NaN gives scale NaN and NaN codes
 * (0x7F).  Used for activations (rows = tokens) and for weights packed as
 * B^T [n][k] (rows = output channels).  cols % 8 == 0, ldx % 8 == 0,
 * ldo % 8 == 0, x 16-byte and out 8-byte aligned. */
typedef struct {
  const void* x;    /* [rows][ldx] fp32 / fp16 / bf16 */
  uint8_t* out;     /* [rows][ldo] E4M3 codes */
  float* scale;     /* [rows] */
  int64_t rows, cols, ldx, ldo;
  int32_t x_dtype;
  int32_t pad_;
} c3h_fp8_quant_args;
int c3h_quantize_fp8_rows(const c3h_fp8_quant_args* a, void* stream);

/* out[m,n] = epilogue((sum_k A[m,k] * B[n,k]) * a_scale[m] * b_scale[n])
 * with E4M3 operands (B packed [n][k]), fp32 accumulation on the MFMA, and
 * the common epilogue (bias, residual, activation/program) into fp32, bf16
 * or fp16.  k, lda, ldb multiples of 16; b_scale 16-byte aligned. */
typedef struct {
  const uint8_t* a;
  const uint8_t* b;
  const float* a_scale; /* [m] */
  const float* b_scale; /* [n] */
  void* out;
  int64_t m, n, k;
  int64_t lda, ldb, ldo;
  int32_t out_dtype;
  int32_t pad_;
  c3h_epilogue epi;
} c3h_fp8_gemm_args;
int c3h_gemm_fp8(const c3h_fp8_gemm_args* a, void* stream);

/* ------------------------------------------------------------------ */
/* W4A16: the executable form of the reference's structural fp4 choice */
/* for large aligned constant-weight GEMMs (c32/strategy.py:150-154),  */
/* with fp16 activations and fp32 accumulation (c32/strategy.py:       */
/* 101-108).  Weights are OCP MX FP4: E2M1 elements, one E8M0 exponent */
/* per 32 consecutive k.                                                */
/* ------------------------------------------------------------------ */

/* Block quantization of rows (weights packed B^T [n][k], rows = output
 * channels) to MXFP4.  Per row r and block b of 32 columns: amax = max |x|;
 * e = clamp(floor(log2 amax) - 2, -13, 13) (e = -13 for an all-zero block),
 * so every dequantized element is zero or a normal fp16 exactly;
 * scales[r][b] = e + 127; the element code is E2M1(|x| * 2^-e) rounded to
 * nearest even and saturated at 6 (magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6),
 * with the sign in bit 3 unless the magnitude code is 0.  A block holding
 * Inf/NaN gets scale 0xFF (NaN) and zero codes.  codes[r][j] packs columns
 * 2j (low nibble) and 2j+1 (high nibble).  cols % 32 == 0; ldc >= cols/2,
 * ldc % 16 == 0 and codes 16-byte aligned; lds >= cols/32. */
typedef struct {
  const void* x;    /* [rows][ldx] fp32 / fp16 / bf16 */
  uint8_t* codes;   /* [rows][ldc] */
  uint8_t* scales;  /* [rows][lds] */
  int64_t rows, cols, ldx, ldc, lds;
  int32_t x_dtype;
  int32_t pad_;
} c3h_mxfp4_quant_args;
int c3h_quantize_mxfp4(const c3h_mxfp4_quant_args* a, void* stream);

/* out[m,n] = epilogue(sum_k A[m,k] * W[n,k]) with A fp16 [m][lda] and
 * W[n,k] = E2M1(codes) * 2^(scales[n][k/32] - 127) widened to fp16 in
 * registers (exact under c3h_quantize_mxfp4's exponent range), fp16 MFMA
 * with fp32 accumulation, and the common epilogue into fp32 or fp16.
 * Equals c3h_gemm on the dequantized fp16 weights bit for bit.  k % 32 == 0,
 * lda % 8 == 0, ldb (bytes) % 4 == 0 and >= k/2, ldbs >= k/32; A 16-byte
 * aligned; A, codes and scales each below 2^31 bytes. */
typedef struct {
  const void* a;           /* [m][lda] fp16 */
  const uint8_t* b_codes;  /* [n][ldb] */
  const uint8_t* b_scales; /* [n][ldbs] */
  void* out;
  int64_t m, n, k;
  int64_t lda, ldb, ldbs, ldo;
  int32_t out_dtype;
  int32_t pad_;
  c3h_epilogue epi;
} c3h_w4a16_gemm_args;
int c3h_gemm_w4a16(const c3h_w4a16_gemm_args* a, void* stream);

/* ------------------------------------------------------------------ */
/* Native timeline interpreter and graph capture                        */
/* ------------------------------------------------------------------ */

/* One action of a compiled plan timeline (c35/executor.py:780-865 realized
 * natively): a kernel launch (kind = C3H_OP_*, args -> the family's args
 * struct), a copy, or an event record/wait on logical stream `stream`. */
enum c3h_op_kind {
  C3H_OP_NOP = 0,
  C3H_OP_EVENT_RECORD = 1,
  C3H_OP_EVENT_WAIT = 2,
  C3H_OP_COPY = 3,
  C3H_OP_FILL = 10,
  C3H_OP_CAST = 11,
  C3H_OP_EW = 12,
  C3H_OP_STRIDED_COPY = 13,
  C3H_OP_REDUCE = 14,
  C3H_OP_SOFTMAX = 15,
  C3H_OP_LAYERNORM = 16,
  C3H_OP_BATCHNORM = 17,
  C3H_OP_GATHER = 18,
  C3H_OP_ARGMAX = 19,
  C3H_OP_IM2COL = 20,
  C3H_OP_LAYOUT = 21,
  C3H_OP_MAXPOOL = 22,
  C3H_OP_GEMM = 23,
  C3H_OP_CONV = 24,
  C3H_OP_ATTN_SCORES = 25,
  C3H_OP_FLASH = 26,
  C3H_OP_QUANTIZE = 27,
  C3H_OP_QGEMM = 28,
  C3H_OP_DEQUANTIZE = 29,
  C3H_OP_BNFOLD = 30,
  C3H_OP_PACK = 31,
  C3H_OP_CONV_POOL = 32,
  C3H_OP_QUANT_FP8 = 33,
  C3H_OP_GEMM_FP8 = 34,
  C3H_OP_SPLITK = 35,
  C3H_OP_QUANT_MXFP4 = 36,
  C3H_OP_GEMM_W4A16 = 37,
  C3H_OP_ARGMAX_FINISH = 38,
  C3H_OP_NONFINITE = 39
};

typedef struct {
  int32_t kind;
  int32_t stream;   /* index into the streams array */
  int32_t event;    /* index into the events array (record/wait) */
  int32_t pad_;
  const void* args; /* family args struct (host memory) */
  void* dst;        /* COPY */
  const void* src;  /* COPY */
  uint64_t bytes;   /* COPY (device-to-device) */
} c3h_op;

/* Execute ops in order; streams[i] / events[i] map logical ids to handles. */
int c3h_program_run(const c3h_op* ops, int32_t n_ops, void* const* streams,
                    int32_t n_streams, void* const* events, int32_t n_events);
/* Capture the same sequence into a hipGraph (streams[0] is the capture origin;
 * the other streams are forked from and joined back to it).  The returned
 * executable graph is launched with c3h_graph_launch. */
int c3h_program_capture(const c3h_op* ops, int32_t n_ops, void* const* streams,
                        int32_t n_streams, void* const* events,
                        int32_t n_events, void** graph_exec);
int c3h_graph_launch(void* graph_exec, void* stream);
int c3h_graph_destroy(void* graph_exec);

/* ABI self-check for bindings: writes sizeof() of the argument structs in
 * this order: c3h_props, c3h_fill_args, c3h_cast_args, c3h_ew_args,
 * c3h_copy_args, c3h_reduce_args, c3h_softmax_args, c3h_layernorm_args,
 * c3h_batchnorm_args, c3h_bnfold_args, c3h_gather_args, c3h_argmax_args,
 * c3h_im2col_args, c3h_layout_args, c3h_pool_args, c3h_epilogue,
 * c3h_gemm_args, c3h_conv_args, c3h_attn_scores_args, c3h_flash_args,
 * c3h_quantize_args, c3h_qgemm_args, c3h_dequantize_args, c3h_op,
 * c3h_pack_args, c3h_conv_pool_args, c3h_fp8_quant_args, c3h_fp8_gemm_args,
 * c3h_splitk_args, c3h_mxfp4_quant_args, c3h_w4a16_gemm_args,
 * c3h_argmax_finish_args, c3h_nonfinite_args.
 * Returns the number of sizes available (host-only; needs no GPU). */
int32_t c3h_abi_sizes(int64_t* out, int32_t capacity);

#ifdef __cplusplus
}
#endif
#endif /* C3HIP_H */
