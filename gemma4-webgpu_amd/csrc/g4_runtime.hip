// g4_runtime.hip — context, memory, events, graphs and error reporting.
//
// Replaces the WebGPU device plumbing of src/engine.ts: initWebGPU (:354-389),
// buffer creation (:553-567), writeBuffer (:313-316), the mapAsync readback
// (:1772-1787) and the sticky device-lost flag (:105, :385-388).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "g4_internal.hpp"

namespace {
thread_local char g_err[512] = "";
constexpr size_t kScratchBytes = 16u << 20;  // reduction partials; operand blocks of batched matmuls

bool is_fatal(hipError_t e) {
  switch (e) {
    case hipErrorIllegalAddress:
    case hipErrorLaunchFailure:
    case hipErrorAssert:
    case hipErrorECCNotCorrectable:
    case hipErrorIllegalState:
    case hipErrorLaunchTimeOut:
      return true;
    default:
      return false;
  }
}
}  // namespace

namespace g4 {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(g4_ctx* ctx, hipError_t e, const char* what) {
  if (ctx && is_fatal(e)) {
    ctx->lost = true;
    return set_error(G4_ERR_DEVICE_LOST, "device lost: %s failed with %s", what,
                     hipGetErrorString(e));
  }
  if (e == hipErrorOutOfMemory)
    return set_error(G4_ERR_OOM, "%s: out of device memory", what);
  return set_error(G4_ERR_HIP, "%s failed: %s", what, hipGetErrorString(e));
}

int check_status(const volatile uint32_t* status, const char* fn) {
  if (status && *status != 0u)
    return set_error(G4_ERR_STALLED,
                     "%s: a bounded wait inside a kernel expired (status 0x%x): the q/k/v hand-off of a "
                     "g4_qkvAttnDecodeFusedWarm launch never completed and that launch wrote NaN; "
                     "g4_clear_stall, then zero its attention workspace",
                     fn, (unsigned)*status);
  return G4_OK;
}

int enter(g4_ctx* ctx, const char* fn) {
  if (!ctx) return set_error(G4_ERR_INVALID, "%s: null context", fn);
  if (ctx->lost) return set_error(G4_ERR_DEVICE_LOST, "%s: device was lost earlier", fn);
  int rc = check_status(ctx->status, fn);
  if (rc) return rc;
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  return G4_OK;
}

int check_launch(g4_ctx* ctx, const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(ctx, e, kernel);
  return G4_OK;
}

}  // namespace g4

int g4_internal_scratch(g4_ctx* ctx, size_t bytes, void** out) {
  if (bytes > ctx->scratch_bytes)
    return g4::set_error(G4_ERR_UNSUPPORTED, "internal scratch of %zu bytes requested, %zu available", bytes,
                         ctx->scratch_bytes);
  *out = ctx->scratch;
  return G4_OK;
}

extern "C" {

const char* g4_last_error(void) { return g_err; }
int g4_version(void) { return 1; }

int g4_init(int device, g4_ctx** out) {
  if (!out) return g4::set_error(G4_ERR_INVALID, "g4_init: null out");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return g4::set_error(G4_ERR_NO_DEVICE, "g4_init: no HIP device (%s)",
                         e == hipSuccess ? "count 0" : hipGetErrorString(e));
  if (device < 0 || device >= n)
    return g4::set_error(G4_ERR_INVALID, "g4_init: device %d out of range [0,%d)", device, n);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return g4::hip_fail(nullptr, e, "hipGetDeviceProperties");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return g4::set_error(G4_ERR_NO_DEVICE, "g4_init: device %d is %s; this library is built for gfx950",
                         device, prop.gcnArchName);
  e = hipSetDevice(device);
  if (e != hipSuccess) return g4::hip_fail(nullptr, e, "hipSetDevice");
  g4_ctx* ctx = new g4_ctx();
  ctx->device = device;
  ctx->num_cus = prop.multiProcessorCount;
  ctx->hbm_bytes = prop.totalGlobalMem;
  ctx->lds_max = prop.sharedMemPerBlock;
  snprintf(ctx->name, sizeof(ctx->name), "%s (%s)", prop.name, prop.gcnArchName);
  e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return g4::hip_fail(nullptr, e, "hipStreamCreate");
  }
  ctx->stream = ctx->own_stream;
  ctx->scratch_bytes = kScratchBytes;
  e = hipMalloc(&ctx->scratch, ctx->scratch_bytes);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return g4::hip_fail(nullptr, e, "hipMalloc(scratch)");
  }
  // the kernel status word: pinned, coherent host memory that kernels
  // write through its device address
  void* st = nullptr;
  e = hipHostMalloc(&st, 256, hipHostMallocMapped | hipHostMallocCoherent);
  if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&ctx->status_dev, st, 0);
  if (e != hipSuccess) {
    if (st) (void)hipHostFree(st);
    (void)hipFree(ctx->scratch);
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return g4::hip_fail(nullptr, e, "hipHostMalloc(status)");
  }
  memset(st, 0, 256);
  ctx->status = (volatile uint32_t*)st;
  g4_internal_noalloc_init(ctx);  // a failed lookup only disables g4_attnDecode_noalloc
  *out = ctx;
  return G4_OK;
}

int g4_destroy(g4_ctx* ctx) {
  if (!ctx) return G4_OK;
  (void)hipSetDevice(ctx->device);
  if (!ctx->lost) (void)hipStreamSynchronize(ctx->own_stream);
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->status) (void)hipHostFree((void*)ctx->status);
  (void)hipStreamDestroy(ctx->own_stream);
  delete ctx;
  return G4_OK;
}

int g4_set_stream(g4_ctx* ctx, void* hip_stream) {
  G4_ENTER(ctx);
  ctx->stream = hip_stream ? (hipStream_t)hip_stream : ctx->own_stream;
  return G4_OK;
}

void* g4_get_stream(g4_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int g4_device_info(g4_ctx* ctx, char* name, size_t name_len, int* num_cus, size_t* hbm_bytes) {
  G4_ENTER(ctx);
  if (name && name_len) snprintf(name, name_len, "%s", ctx->name);
  if (num_cus) *num_cus = ctx->num_cus;
  if (hbm_bytes) *hbm_bytes = ctx->hbm_bytes;
  return G4_OK;
}

int g4_alloc(g4_ctx* ctx, size_t bytes, void** dptr) {
  G4_ENTER(ctx);
  G4_REQUIRE(dptr, "g4_alloc: null out");
  *dptr = nullptr;
  G4_REQUIRE(bytes > 0, "g4_alloc: zero bytes");
  G4_HIP(ctx, hipMalloc(dptr, bytes));
  return G4_OK;
}

int g4_free(g4_ctx* ctx, void* dptr) {
  if (!ctx) return g4::set_error(G4_ERR_INVALID, "g4_free: null context");
  if (!dptr) return G4_OK;
  (void)hipSetDevice(ctx->device);
  G4_HIP(ctx, hipFree(dptr));
  return G4_OK;
}

// Calls that would put a memset node into a captured graph (such nodes have
// given wrong results on replays after the first) or synchronise inside a
// capture are refused while g4_graph_begin/end capture the stream.
#define G4_NOT_CAPTURING(ctx, fn) \
  G4_REQUIRE(!(ctx)->capturing, fn ": not allowed while a graph is being captured")

int g4_memset(g4_ctx* ctx, void* dptr, int value, size_t bytes) {
  G4_ENTER(ctx);
  G4_NOT_CAPTURING(ctx, "g4_memset");
  G4_REQUIRE(dptr || bytes == 0, "g4_memset: null pointer");
  if (bytes) G4_HIP(ctx, hipMemsetAsync(dptr, value, bytes, ctx->stream));
  return G4_OK;
}

int g4_upload(g4_ctx* ctx, void* dst, const void* src, size_t bytes, size_t dst_offset) {
  G4_ENTER(ctx);
  G4_NOT_CAPTURING(ctx, "g4_upload");
  G4_REQUIRE((dst && src) || bytes == 0, "g4_upload: null pointer");
  if (!bytes) return G4_OK;
  G4_HIP(ctx, hipMemcpyAsync((char*)dst + dst_offset, src, bytes, hipMemcpyHostToDevice,
                             ctx->stream));
  G4_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return g4::check_status(ctx->status, __func__);
}

int g4_download(g4_ctx* ctx, void* dst, const void* src, size_t bytes, size_t src_offset) {
  G4_ENTER(ctx);
  G4_NOT_CAPTURING(ctx, "g4_download");
  G4_REQUIRE((dst && src) || bytes == 0, "g4_download: null pointer");
  if (!bytes) return G4_OK;
  G4_HIP(ctx, hipMemcpyAsync(dst, (const char*)src + src_offset, bytes, hipMemcpyDeviceToHost,
                             ctx->stream));
  G4_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return g4::check_status(ctx->status, __func__);
}

int g4_download_async(g4_ctx* ctx, void* dst, const void* src, size_t bytes, size_t src_offset,
                      g4_event** ev) {
  G4_ENTER(ctx);
  G4_NOT_CAPTURING(ctx, "g4_download_async");
  G4_REQUIRE(dst && src && ev, "g4_download_async: null pointer");
  *ev = nullptr;
  if (bytes)
    G4_HIP(ctx, hipMemcpyAsync(dst, (const char*)src + src_offset, bytes, hipMemcpyDeviceToHost,
                               ctx->stream));
  return g4_event_record(ctx, ev);
}

int g4_host_alloc(g4_ctx* ctx, size_t bytes, void** host) {
  G4_ENTER(ctx);
  G4_REQUIRE(host, "g4_host_alloc: null out");
  *host = nullptr;
  G4_REQUIRE(bytes > 0, "g4_host_alloc: zero bytes");
  G4_HIP(ctx, hipHostMalloc(host, bytes, hipHostMallocDefault));
  return G4_OK;
}

int g4_host_free(void* host) {
  if (!host) return G4_OK;
  const hipError_t e = hipHostFree(host);
  if (e != hipSuccess) return g4::hip_fail(nullptr, e, "hipHostFree");
  return G4_OK;
}

int g4_copy_d2d(g4_ctx* ctx, void* dst, const void* src, size_t bytes) {
  G4_ENTER(ctx);
  G4_REQUIRE((dst && src) || bytes == 0, "g4_copy_d2d: null pointer");
  if (bytes) G4_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return G4_OK;
}

int g4_stream_sync(g4_ctx* ctx) {
  G4_ENTER(ctx);
  G4_NOT_CAPTURING(ctx, "g4_stream_sync");
  G4_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return g4::check_status(ctx->status, __func__);
}

int g4_clear_stall(g4_ctx* ctx) {
  if (!ctx) return g4::set_error(G4_ERR_INVALID, "g4_clear_stall: null context");
  if (ctx->status) *ctx->status = 0u;
  return G4_OK;
}

int g4_test_stage_wait(g4_ctx* ctx, uint32_t spin_limit, int skip_matvec) {
  G4_ENTER(ctx);
  ctx->test_spin = spin_limit;
  ctx->test_skip_matvec = skip_matvec != 0;
  return G4_OK;
}

int g4_event_record(g4_ctx* ctx, g4_event** ev) {
  G4_ENTER(ctx);
  G4_REQUIRE(ev, "g4_event_record: null out");
  g4_event* e = new g4_event();
  e->device = ctx->device;
  e->status = ctx->status;
  hipError_t he = hipEventCreate(&e->ev);
  if (he != hipSuccess) {
    delete e;
    return g4::hip_fail(ctx, he, "hipEventCreate");
  }
  he = hipEventRecord(e->ev, ctx->stream);
  if (he != hipSuccess) {
    (void)hipEventDestroy(e->ev);
    delete e;
    return g4::hip_fail(ctx, he, "hipEventRecord");
  }
  *ev = e;
  return G4_OK;
}

int g4_event_query(g4_event* ev) {
  if (!ev) return g4::set_error(G4_ERR_INVALID, "g4_event_query: null event");
  (void)hipSetDevice(ev->device);
  hipError_t e = hipEventQuery(ev->ev);
  if (e == hipSuccess) {
    const int rc = g4::check_status(ev->status, "g4_event_query");
    return rc ? rc : 1;
  }
  if (e == hipErrorNotReady) return 0;
  return g4::hip_fail(nullptr, e, "hipEventQuery");
}

int g4_event_wait(g4_event* ev) {
  if (!ev) return g4::set_error(G4_ERR_INVALID, "g4_event_wait: null event");
  (void)hipSetDevice(ev->device);
  hipError_t e = hipEventSynchronize(ev->ev);
  if (e != hipSuccess) return g4::hip_fail(nullptr, e, "hipEventSynchronize");
  return g4::check_status(ev->status, "g4_event_wait");
}

int g4_event_elapsed_ms(g4_event* a, g4_event* b, float* ms) {
  if (!a || !b || !ms) return g4::set_error(G4_ERR_INVALID, "g4_event_elapsed_ms: null");
  hipError_t e = hipEventElapsedTime(ms, a->ev, b->ev);
  if (e != hipSuccess) return g4::hip_fail(nullptr, e, "hipEventElapsedTime");
  return G4_OK;
}

int g4_event_destroy(g4_event* ev) {
  if (!ev) return G4_OK;
  (void)hipEventDestroy(ev->ev);
  delete ev;
  return G4_OK;
}

int g4_graph_begin(g4_ctx* ctx) {
  G4_ENTER(ctx);
  G4_REQUIRE(!ctx->capturing, "g4_graph_begin: already capturing");
  G4_REQUIRE(ctx->stream != nullptr, "g4_graph_begin: the legacy null stream cannot be captured");
  G4_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  ctx->capturing = true;
  return G4_OK;
}

int g4_graph_end(g4_ctx* ctx, g4_graph** graph) {
  G4_ENTER(ctx);
  G4_REQUIRE(graph, "g4_graph_end: null out");
  G4_REQUIRE(ctx->capturing, "g4_graph_end: not capturing");
  *graph = nullptr;
  ctx->capturing = false;
  hipGraph_t g = nullptr;
  G4_HIP(ctx, hipStreamEndCapture(ctx->stream, &g));
  hipGraphExec_t ex = nullptr;
  hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return g4::hip_fail(ctx, e, "hipGraphInstantiate");
  }
  g4_graph* out = new g4_graph();
  out->graph = g;
  out->exec = ex;
  *graph = out;
  return G4_OK;
}

int g4_graph_launch(g4_ctx* ctx, g4_graph* graph) {
  G4_ENTER(ctx);
  G4_REQUIRE(graph && graph->exec, "g4_graph_launch: null graph");
  G4_HIP(ctx, hipGraphLaunch(graph->exec, ctx->stream));
  return G4_OK;
}

int g4_graph_kernel_nodes(g4_graph* graph, size_t* count) {
  if (!graph || !graph->graph || !count) return g4::set_error(G4_ERR_INVALID, "g4_graph_kernel_nodes: null");
  *count = 0;
  size_t n = 0;
  hipError_t e = hipGraphGetNodes(graph->graph, nullptr, &n);
  if (e != hipSuccess) return g4::hip_fail(nullptr, e, "hipGraphGetNodes");
  std::vector<hipGraphNode_t> nodes(n);
  if (n) {
    e = hipGraphGetNodes(graph->graph, nodes.data(), &n);
    if (e != hipSuccess) return g4::hip_fail(nullptr, e, "hipGraphGetNodes");
  }
  for (size_t i = 0; i < n; ++i) {
    hipGraphNodeType t;
    e = hipGraphNodeGetType(nodes[i], &t);
    if (e != hipSuccess) return g4::hip_fail(nullptr, e, "hipGraphNodeGetType");
    if (t == hipGraphNodeTypeKernel) ++*count;
  }
  return G4_OK;
}

int g4_graph_destroy(g4_graph* graph) {
  if (!graph) return G4_OK;
  if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
  if (graph->graph) (void)hipGraphDestroy(graph->graph);
  delete graph;
  return G4_OK;
}

uint64_t g4_splitmix64(uint64_t seed, uint64_t idx) { return g4d::splitmix64(seed, idx); }

}  // extern "C"
