// Runtime half of libc3hip.so: device query, the plan slab, pinned staging,
// logical streams/events, and the native timeline interpreter with hipGraph
// capture.  Realizes the resource model of c35/executor.py:673-709 and
// :757-868 in C++ so a compiled plan replays without Python in the loop.
#include <math.h>
#include <stdarg.h>
#include <stdlib.h>
#include <mutex>
#include <unordered_map>
#include <vector>
#include "common.h"

namespace c3h {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

static Switches read_switches() {
  Switches w;
  w.disable_dma = getenv("C3H_DISABLE_DMA") != nullptr;
  w.disable_bigtile = getenv("C3H_DISABLE_BIGTILE") != nullptr;
  w.disable_buf = getenv("C3H_DISABLE_BUF") != nullptr;
  w.disable_conv3x3 = getenv("C3H_DISABLE_CONV3X3") != nullptr;
  w.disable_direct_conv = getenv("C3H_DISABLE_DIRECT_CONV") != nullptr;
  const char* rp = getenv("C3H_DMA_RP");
  w.dma_rp = rp ? atoi(rp) : 0;
  w.disable_pp = getenv("C3H_DISABLE_PP") != nullptr;
  w.disable_qmul = getenv("C3H_DISABLE_QMUL") != nullptr;
  w.disable_tile160 = getenv("C3H_DISABLE_TILE160") != nullptr;
  return w;
}

static Switches g_switches = read_switches();

const Switches& switches() { return g_switches; }

float quant_multiplier(float scale, int zero, int dtype) {
  if (switches().disable_qmul || !quant_scale_ok(scale) || zero < -128 || zero > 127 ||
      (dtype != C3H_BF16 && dtype != C3H_F16))
    return 0.0f;
  static std::mutex mu;
  static std::unordered_map<uint64_t, float> cache;
  uint32_t sbits;
  memcpy(&sbits, &scale, 4);
  const uint64_t key = (static_cast<uint64_t>(sbits) << 32) | (static_cast<uint64_t>(zero & 0xff) << 8) |
                       static_cast<uint64_t>(dtype & 0xff);
  {
    std::lock_guard<std::mutex> g(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  // The code as the kernels form it: rne, + zero_point + 128, v_cvt_pk_u8_f32
  // (clamp to [0, 255], NaN -> 0), - 128.
  const float zp128 = static_cast<float>(zero + 128);
  auto code = [zp128](float q) -> int {
    const float v = nearbyintf(q) + zp128;
    if (v != v) return -128;
    return static_cast<int>(fminf(fmaxf(v, 0.0f), 255.0f)) - 128;
  };
  std::vector<float> xs(65536);
  std::vector<int8_t> want(65536);
  for (uint32_t u = 0; u < 65536; ++u) {
    if (dtype == C3H_BF16) {
      const uint32_t w = u << 16;
      memcpy(&xs[u], &w, 4);
    } else {
      const uint16_t h = static_cast<uint16_t>(u);
      _Float16 f;
      memcpy(&f, &h, 2);
      xs[u] = static_cast<float>(f);
    }
    want[u] = static_cast<int8_t>(code(xs[u] / scale));  // IEEE division: the QuantizeLinear code
  }
  const float c0 = 1.0f / scale;
  uint32_t cbits;
  memcpy(&cbits, &c0, 4);
  float found = 0.0f;
  for (int d : {0, 1, -1, 2, -2, 3, -3, 4, -4}) {
    const uint32_t tb = cbits + static_cast<uint32_t>(d);
    float c;
    memcpy(&c, &tb, 4);
    if (!(c > 0.0f) || c > 3.4028235e38f) continue;
    bool ok = true;
    for (uint32_t u = 0; u < 65536 && ok; ++u) ok = code(xs[u] * c) == want[u];
    if (ok) {
      found = c;
      break;
    }
  }
  std::lock_guard<std::mutex> g(mu);
  cache[key] = found;
  return found;
}

}  // namespace c3h

using namespace c3h;

extern "C" {

const char* c3h_last_error(void) { return g_last_error; }

int c3h_reload_switches(void) {
  g_switches = read_switches();
  return C3H_OK;
}

int c3h_init(int device) {
  int count = 0;
  C3H_HIP_CHECK(hipGetDeviceCount(&count));
  C3H_REQUIRE(device >= 0 && device < count, "device %d out of range (count %d)", device, count);
  C3H_HIP_CHECK(hipSetDevice(device));
  C3H_HIP_CHECK(hipFree(nullptr));  // force context creation
  return gemm_scratch_setup(device);
}

int c3h_device_count(int* count) {
  C3H_REQUIRE(count != nullptr, "null count");
  hipError_t err = hipGetDeviceCount(count);
  if (err != hipSuccess) {
    *count = 0;
    return fail(C3H_EHIP, "hipGetDeviceCount: %s", hipGetErrorString(err));
  }
  return C3H_OK;
}

int c3h_device_props(int device, c3h_props* out) {
  C3H_REQUIRE(out != nullptr, "null props");
  hipDeviceProp_t p;
  C3H_HIP_CHECK(hipGetDeviceProperties(&p, device));
  memset(out, 0, sizeof(*out));
  snprintf(out->name, sizeof(out->name), "%s", p.name);
  snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
  out->compute_units = p.multiProcessorCount;
  out->warp_size = p.warpSize;
  out->max_threads_per_block = p.maxThreadsPerBlock;
  out->max_block_dim_x = p.maxThreadsDim[0];
  out->max_grid_dim_x = p.maxGridSize[0];
  out->lds_bytes_per_block = static_cast<int32_t>(p.sharedMemPerBlock);
  out->clock_khz = p.clockRate;
  out->memory_clock_khz = p.memoryClockRate;
  out->memory_bus_width = p.memoryBusWidth;
  out->l2_bytes = p.l2CacheSize;
  out->total_memory_bytes = static_cast<int64_t>(p.totalGlobalMem);
  out->major = p.major;
  out->minor = p.minor;
  return C3H_OK;
}

int c3h_device_synchronize(void) {
  C3H_HIP_CHECK(hipDeviceSynchronize());
  return C3H_OK;
}

int c3h_malloc(void** ptr, size_t bytes) {
  C3H_REQUIRE(ptr != nullptr, "null ptr");
  *ptr = nullptr;
  if (bytes == 0) bytes = 256;
  C3H_HIP_CHECK(hipMalloc(ptr, bytes));
  return C3H_OK;
}

int c3h_free(void* ptr) {
  if (ptr) C3H_HIP_CHECK(hipFree(ptr));
  return C3H_OK;
}

int c3h_host_alloc(void** ptr, size_t bytes) {
  C3H_REQUIRE(ptr != nullptr, "null ptr");
  if (bytes == 0) bytes = 64;
  C3H_HIP_CHECK(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
  return C3H_OK;
}

int c3h_host_free(void* ptr) {
  if (ptr) C3H_HIP_CHECK(hipHostFree(ptr));
  return C3H_OK;
}

int c3h_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return C3H_OK;
  C3H_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
  return C3H_OK;
}

int c3h_memcpy_d2h_async(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return C3H_OK;
  C3H_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
  return C3H_OK;
}

int c3h_memcpy_d2d_async(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0 || dst == src) return C3H_OK;
  C3H_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
  return C3H_OK;
}

int c3h_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return C3H_OK;
  C3H_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return C3H_OK;
}

int c3h_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return C3H_OK;
  C3H_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return C3H_OK;
}

int c3h_stream_create(void** stream) {
  C3H_REQUIRE(stream != nullptr, "null stream");
  hipStream_t s;
  C3H_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return C3H_OK;
}

int c3h_stream_destroy(void* stream) {
  if (stream) C3H_HIP_CHECK(hipStreamDestroy(as_stream(stream)));
  return C3H_OK;
}

int c3h_stream_synchronize(void* stream) {
  C3H_HIP_CHECK(hipStreamSynchronize(as_stream(stream)));
  return C3H_OK;
}

int c3h_event_create(void** event, int timing) {
  C3H_REQUIRE(event != nullptr, "null event");
  hipEvent_t e;
  C3H_HIP_CHECK(hipEventCreateWithFlags(&e, timing ? hipEventDefault : hipEventDisableTiming));
  *event = e;
  return C3H_OK;
}

int c3h_event_destroy(void* event) {
  if (event) C3H_HIP_CHECK(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
  return C3H_OK;
}

int c3h_event_record(void* event, void* stream) {
  C3H_HIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
  return C3H_OK;
}

int c3h_stream_wait_event(void* stream, void* event) {
  C3H_HIP_CHECK(hipStreamWaitEvent(as_stream(stream), reinterpret_cast<hipEvent_t>(event), 0));
  return C3H_OK;
}

int c3h_event_synchronize(void* event) {
  C3H_HIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)));
  return C3H_OK;
}

int c3h_event_elapsed_ms(float* ms, void* start, void* stop) {
  C3H_REQUIRE(ms != nullptr, "null ms");
  C3H_HIP_CHECK(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
  return C3H_OK;
}

// ---------------------------------------------------------------------------
// Timeline interpreter.
// ---------------------------------------------------------------------------
static int dispatch_op(const c3h_op& op, hipStream_t s, void* const* events, int32_t n_events) {
  switch (op.kind) {
    case C3H_OP_NOP: return C3H_OK;
    case C3H_OP_EVENT_RECORD:
      C3H_REQUIRE(op.event >= 0 && op.event < n_events, "event index %d out of range", op.event);
      C3H_HIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(events[op.event]), s));
      return C3H_OK;
    case C3H_OP_EVENT_WAIT:
      C3H_REQUIRE(op.event >= 0 && op.event < n_events, "event index %d out of range", op.event);
      C3H_HIP_CHECK(hipStreamWaitEvent(s, reinterpret_cast<hipEvent_t>(events[op.event]), 0));
      return C3H_OK;
    case C3H_OP_COPY:
      if (op.bytes && op.dst != op.src)
        C3H_HIP_CHECK(hipMemcpyAsync(op.dst, op.src, op.bytes, hipMemcpyDeviceToDevice, s));
      return C3H_OK;
    case C3H_OP_FILL: return c3h_fill(static_cast<const c3h_fill_args*>(op.args), s);
    case C3H_OP_CAST: return c3h_cast(static_cast<const c3h_cast_args*>(op.args), s);
    case C3H_OP_EW: return c3h_ew(static_cast<const c3h_ew_args*>(op.args), s);
    case C3H_OP_STRIDED_COPY: return c3h_strided_copy(static_cast<const c3h_copy_args*>(op.args), s);
    case C3H_OP_REDUCE: return c3h_reduce(static_cast<const c3h_reduce_args*>(op.args), s);
    case C3H_OP_SOFTMAX: return c3h_softmax(static_cast<const c3h_softmax_args*>(op.args), s);
    case C3H_OP_LAYERNORM: return c3h_layernorm(static_cast<const c3h_layernorm_args*>(op.args), s);
    case C3H_OP_BATCHNORM: return c3h_batchnorm(static_cast<const c3h_batchnorm_args*>(op.args), s);
    case C3H_OP_GATHER: return c3h_gather(static_cast<const c3h_gather_args*>(op.args), s);
    case C3H_OP_ARGMAX: return c3h_argmax(static_cast<const c3h_argmax_args*>(op.args), s);
    case C3H_OP_IM2COL: return c3h_im2col(static_cast<const c3h_im2col_args*>(op.args), s);
    case C3H_OP_LAYOUT: return c3h_layout(static_cast<const c3h_layout_args*>(op.args), s);
    case C3H_OP_MAXPOOL: return c3h_maxpool2d(static_cast<const c3h_pool_args*>(op.args), s);
    case C3H_OP_GEMM: return c3h_gemm(static_cast<const c3h_gemm_args*>(op.args), s);
    case C3H_OP_CONV: return c3h_conv2d(static_cast<const c3h_conv_args*>(op.args), s);
    case C3H_OP_ATTN_SCORES: return c3h_attention_scores(static_cast<const c3h_attn_scores_args*>(op.args), s);
    case C3H_OP_FLASH: return c3h_flash_attention(static_cast<const c3h_flash_args*>(op.args), s);
    case C3H_OP_QUANTIZE: return c3h_quantize(static_cast<const c3h_quantize_args*>(op.args), s);
    case C3H_OP_QGEMM: return c3h_qgemm(static_cast<const c3h_qgemm_args*>(op.args), s);
    case C3H_OP_DEQUANTIZE: return c3h_dequantize(static_cast<const c3h_dequantize_args*>(op.args), s);
    case C3H_OP_BNFOLD: return c3h_bn_fold(static_cast<const c3h_bnfold_args*>(op.args), s);
    case C3H_OP_PACK: return c3h_pack_conv_weight(static_cast<const c3h_pack_args*>(op.args), s);
    case C3H_OP_CONV_POOL: return c3h_conv_stem_pool(static_cast<const c3h_conv_pool_args*>(op.args), s);
    case C3H_OP_QUANT_FP8: return c3h_quantize_fp8_rows(static_cast<const c3h_fp8_quant_args*>(op.args), s);
    case C3H_OP_GEMM_FP8: return c3h_gemm_fp8(static_cast<const c3h_fp8_gemm_args*>(op.args), s);
    case C3H_OP_QUANT_MXFP4:
      return c3h_quantize_mxfp4(static_cast<const c3h_mxfp4_quant_args*>(op.args), s);
    case C3H_OP_GEMM_W4A16: return c3h_gemm_w4a16(static_cast<const c3h_w4a16_gemm_args*>(op.args), s);
    case C3H_OP_ARGMAX_FINISH: return c3h_argmax_finish(static_cast<const c3h_argmax_finish_args*>(op.args), s);
    case C3H_OP_NONFINITE: return c3h_nonfinite(static_cast<const c3h_nonfinite_args*>(op.args), s);
    case C3H_OP_SPLITK: return c3h_gemm_splitk_reduce(static_cast<const c3h_splitk_args*>(op.args), s);
    default: return fail(C3H_EINVAL, "unknown op kind %d", op.kind);
  }
}

static int run_ops(const c3h_op* ops, int32_t n_ops, void* const* streams, int32_t n_streams,
                   void* const* events, int32_t n_events) {
  for (int32_t i = 0; i < n_ops; ++i) {
    const c3h_op& op = ops[i];
    C3H_REQUIRE(op.stream >= 0 && op.stream < n_streams, "op %d: stream index %d out of range", i, op.stream);
    int rc = dispatch_op(op, as_stream(streams[op.stream]), events, n_events);
    if (rc != C3H_OK) {
      char buf[1024];
      snprintf(buf, sizeof(buf), "%s", g_last_error);
      return fail(rc, "op %d (kind %d): %s", i, op.kind, buf);
    }
  }
  return C3H_OK;
}

int c3h_program_run(const c3h_op* ops, int32_t n_ops, void* const* streams, int32_t n_streams,
                    void* const* events, int32_t n_events) {
  C3H_REQUIRE(ops != nullptr || n_ops == 0, "null ops");
  C3H_REQUIRE(n_streams > 0 && streams != nullptr, "no streams");
  return run_ops(ops, n_ops, streams, n_streams, events, n_events);
}

int c3h_program_capture(const c3h_op* ops, int32_t n_ops, void* const* streams, int32_t n_streams,
                        void* const* events, int32_t n_events, void** graph_exec) {
  C3H_REQUIRE(graph_exec != nullptr, "null graph_exec");
  C3H_REQUIRE(n_streams > 0 && streams != nullptr, "no streams");
  *graph_exec = nullptr;
  hipStream_t origin = as_stream(streams[0]);
  std::vector<hipEvent_t> joins;
  hipEvent_t fork;
  C3H_HIP_CHECK(hipEventCreateWithFlags(&fork, hipEventDisableTiming));
  hipError_t err = hipStreamBeginCapture(origin, hipStreamCaptureModeThreadLocal);
  if (err != hipSuccess) {
    (void)hipEventDestroy(fork);
    return fail(C3H_EHIP, "hipStreamBeginCapture: %s", hipGetErrorString(err));
  }
  int rc = C3H_OK;
  if (hipEventRecord(fork, origin) != hipSuccess) rc = fail(C3H_EHIP, "fork record failed");
  for (int32_t i = 1; rc == C3H_OK && i < n_streams; ++i)
    if (hipStreamWaitEvent(as_stream(streams[i]), fork, 0) != hipSuccess) rc = fail(C3H_EHIP, "fork wait failed");
  if (rc == C3H_OK) rc = run_ops(ops, n_ops, streams, n_streams, events, n_events);
  for (int32_t i = 1; i < n_streams; ++i) {
    hipEvent_t j;
    if (hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) { rc = fail(C3H_EHIP, "join create failed"); continue; }
    joins.push_back(j);
    if (hipEventRecord(j, as_stream(streams[i])) != hipSuccess || hipStreamWaitEvent(origin, j, 0) != hipSuccess)
      if (rc == C3H_OK) rc = fail(C3H_EHIP, "join failed");
  }
  hipGraph_t graph = nullptr;
  hipError_t end = hipStreamEndCapture(origin, &graph);
  (void)hipEventDestroy(fork);
  for (hipEvent_t j : joins) (void)hipEventDestroy(j);
  if (rc != C3H_OK) {
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
  }
  if (end != hipSuccess) return fail(C3H_EHIP, "hipStreamEndCapture: %s", hipGetErrorString(end));
  hipGraphExec_t exec = nullptr;
  err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (err != hipSuccess) return fail(C3H_EHIP, "hipGraphInstantiate: %s", hipGetErrorString(err));
  *graph_exec = exec;
  return C3H_OK;
}

int c3h_graph_launch(void* graph_exec, void* stream) {
  C3H_REQUIRE(graph_exec != nullptr, "null graph");
  C3H_HIP_CHECK(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph_exec), as_stream(stream)));
  return C3H_OK;
}

int32_t c3h_abi_sizes(int64_t* out, int32_t capacity) {
  const int64_t sizes[] = {
      sizeof(c3h_props),          sizeof(c3h_fill_args),      sizeof(c3h_cast_args),
      sizeof(c3h_ew_args),        sizeof(c3h_copy_args),      sizeof(c3h_reduce_args),
      sizeof(c3h_softmax_args),   sizeof(c3h_layernorm_args), sizeof(c3h_batchnorm_args),
      sizeof(c3h_bnfold_args),    sizeof(c3h_gather_args),    sizeof(c3h_argmax_args),
      sizeof(c3h_im2col_args),    sizeof(c3h_layout_args),    sizeof(c3h_pool_args),
      sizeof(c3h_epilogue),       sizeof(c3h_gemm_args),      sizeof(c3h_conv_args),
      sizeof(c3h_attn_scores_args), sizeof(c3h_flash_args),   sizeof(c3h_quantize_args),
      sizeof(c3h_qgemm_args),     sizeof(c3h_dequantize_args), sizeof(c3h_op),
      sizeof(c3h_pack_args),      sizeof(c3h_conv_pool_args), sizeof(c3h_fp8_quant_args),
      sizeof(c3h_fp8_gemm_args), sizeof(c3h_splitk_args), sizeof(c3h_mxfp4_quant_args),
      sizeof(c3h_w4a16_gemm_args), sizeof(c3h_argmax_finish_args), sizeof(c3h_nonfinite_args)};
  const int32_t n = static_cast<int32_t>(sizeof(sizes) / sizeof(sizes[0]));
  for (int32_t i = 0; i < n && i < capacity && out; ++i) out[i] = sizes[i];
  return n;
}

int c3h_graph_destroy(void* graph_exec) {
  if (graph_exec) C3H_HIP_CHECK(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph_exec)));
  return C3H_OK;
}

}  // extern "C"
