// N-API addon over libg4hip.so: the per-key dispatch contract of the
// reference's WebGPU backend (src/engine.ts:1466-1651 encodeTransformerPass,
// :1670-1846 sampleNextTokenSubmit) for a Node host.
//
// Device pointers, contexts, graphs and events travel to JavaScript as
// BigInt handles; null/undefined stands for NULL. Each key takes the buffers
// in the WGSL binding order of its shader and then a plain object whose
// properties are the fields of the shader's Params struct, by name
// (e.g. matmulQuant(ctx, input, weight, output, {M, N}, 'q4k')). A failing
// call throws an Error whose `code` is the G4_ERR_* name of the status and
// whose message is g4_last_error().
#define NAPI_VERSION 6
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <string>

#include "g4hip.h"

namespace {

const char* status_name(int rc) {
  switch (rc) {
    case G4_ERR_INVALID: return "G4_ERR_INVALID";
    case G4_ERR_HIP: return "G4_ERR_HIP";
    case G4_ERR_DEVICE_LOST: return "G4_ERR_DEVICE_LOST";
    case G4_ERR_OOM: return "G4_ERR_OOM";
    case G4_ERR_UNSUPPORTED: return "G4_ERR_UNSUPPORTED";
    case G4_ERR_NO_DEVICE: return "G4_ERR_NO_DEVICE";
    case G4_ERR_STALLED: return "G4_ERR_STALLED";
    default: return "G4_ERR_UNKNOWN";
  }
}

// Argument errors found here (a wrong JS type) are thrown as TypeErrors and
// the wrapper returns nullptr; `ok` turns false so no library call is made.
struct Args {
  napi_env env;
  size_t argc = 0;
  napi_value v[12];
  bool ok = true;
  Args(napi_env e, napi_callback_info info) : env(e) {
    argc = 12;
    if (napi_get_cb_info(env, info, &argc, v, nullptr, nullptr) != napi_ok) fail("bad call");
  }
  void fail(const char* msg) {
    if (ok) napi_throw_type_error(env, "G4_ERR_ARG", msg);
    ok = false;
  }
  bool present(size_t i) const {
    if (i >= argc) return false;
    napi_valuetype t;
    napi_typeof(env, v[i], &t);
    return t != napi_undefined && t != napi_null;
  }
  void* ptr(size_t i) {
    if (!present(i)) return nullptr;
    uint64_t p = 0;
    bool lossless = false;
    if (napi_get_value_bigint_uint64(env, v[i], &p, &lossless) != napi_ok || !lossless) {
      fail("expected a BigInt device handle (or null)");
      return nullptr;
    }
    return (void*)(uintptr_t)p;
  }
  uint32_t u32(size_t i) {
    uint32_t u = 0;
    if (i >= argc || napi_get_value_uint32(env, v[i], &u) != napi_ok) fail("expected a number");
    return u;
  }
  uint64_t u64(size_t i) {
    if (i >= argc) {
      fail("missing argument");
      return 0;
    }
    napi_valuetype t;
    napi_typeof(env, v[i], &t);
    if (t == napi_bigint) {
      uint64_t u = 0;
      bool lossless = false;
      napi_get_value_bigint_uint64(env, v[i], &u, &lossless);
      return u;
    }
    double d = 0;
    if (napi_get_value_double(env, v[i], &d) != napi_ok || d < 0) fail("expected a non-negative number");
    return (uint64_t)d;
  }
  float f32(size_t i) {
    double d = 0;
    if (i >= argc || napi_get_value_double(env, v[i], &d) != napi_ok) fail("expected a number");
    return (float)d;
  }
  std::string str(size_t i) {
    size_t n = 0;
    if (i >= argc || napi_get_value_string_utf8(env, v[i], nullptr, 0, &n) != napi_ok) {
      fail("expected a string");
      return std::string();
    }
    std::string out(n + 1, '\0');
    napi_get_value_string_utf8(env, v[i], &out[0], n + 1, &n);
    out.resize(n);
    return out;
  }
  // a named field of the Params object at argument i
  napi_value field(size_t i, const char* name) {
    napi_value out = nullptr;
    bool has = false;
    if (i >= argc || napi_has_named_property(env, v[i], name, &has) != napi_ok || !has) {
      std::string m = std::string("params object lacks field '") + name + "'";
      fail(m.c_str());
      return nullptr;
    }
    napi_get_named_property(env, v[i], name, &out);
    return out;
  }
  uint32_t fu32(size_t i, const char* name) {
    napi_value f = field(i, name);
    uint32_t u = 0;
    if (f && napi_get_value_uint32(env, f, &u) != napi_ok) fail(name);
    return u;
  }
  float ff32(size_t i, const char* name) {
    napi_value f = field(i, name);
    double d = 0;
    if (f && napi_get_value_double(env, f, &d) != napi_ok) fail(name);
    return (float)d;
  }
};

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

napi_value done(napi_env env, int rc) {
  if (rc != G4_OK) {
    const char* msg = g4_last_error();
    napi_throw_error(env, status_name(rc), msg && *msg ? msg : status_name(rc));
    return nullptr;
  }
  return undefined(env);
}

napi_value bigint(napi_env env, const void* p) {
  napi_value out;
  napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &out);
  return out;
}

napi_value number(napi_env env, double d) {
  napi_value out;
  napi_create_double(env, d, &out);
  return out;
}

#define CTX(a, i) ((g4_ctx*)(a).ptr(i))
#define F32P(a, i) ((float*)(a).ptr(i))
#define U16P(a, i) ((uint16_t*)(a).ptr(i))
#define U32P(a, i) ((uint32_t*)(a).ptr(i))
#define CHECKED(a) \
  if (!(a).ok) return nullptr

// ---- lifecycle, memory, synchronisation --------------------------------

napi_value Version(napi_env env, napi_callback_info) { return number(env, g4_version()); }

napi_value LastError(napi_env env, napi_callback_info) {
  napi_value s;
  const char* m = g4_last_error();
  napi_create_string_utf8(env, m ? m : "", NAPI_AUTO_LENGTH, &s);
  return s;
}

// init(device) -> ctx
napi_value Init(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const uint32_t dev = a.present(0) ? a.u32(0) : 0;
  CHECKED(a);
  g4_ctx* ctx = nullptr;
  const int rc = g4_init((int)dev, &ctx);
  if (rc != G4_OK) return done(env, rc);
  return bigint(env, ctx);
}

napi_value Destroy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  CHECKED(a);
  return done(env, g4_destroy(c));
}

// deviceInfo(ctx) -> {name, numCus, hbmBytes}
napi_value DeviceInfo(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  CHECKED(a);
  char name[256] = {0};
  int cus = 0;
  size_t hbm = 0;
  const int rc = g4_device_info(c, name, sizeof name, &cus, &hbm);
  if (rc != G4_OK) return done(env, rc);
  napi_value o, s;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &s);
  napi_set_named_property(env, o, "name", s);
  napi_set_named_property(env, o, "numCus", number(env, cus));
  napi_set_named_property(env, o, "hbmBytes", number(env, (double)hbm));
  return o;
}

// alloc(ctx, bytes) -> ptr
napi_value Alloc(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const uint64_t n = a.u64(1);
  CHECKED(a);
  void* p = nullptr;
  const int rc = g4_alloc(c, (size_t)n, &p);
  if (rc != G4_OK) return done(env, rc);
  return bigint(env, p);
}

napi_value Free(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  void* p = a.ptr(1);
  CHECKED(a);
  return done(env, g4_free(c, p));
}

// memset(ctx, ptr, value, bytes)
napi_value Memset(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  void* p = a.ptr(1);
  const uint32_t v = a.u32(2);
  const uint64_t n = a.u64(3);
  CHECKED(a);
  return done(env, g4_memset(c, p, (int)v, (size_t)n));
}

// upload(ctx, dst, typedArrayOrBuffer, dstOffset = 0): writeBuffer
napi_value Upload(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  void* dst = a.ptr(1);
  const uint64_t off = a.present(3) ? a.u64(3) : 0;
  CHECKED(a);
  bool is_ta = false, is_buf = false;
  void* data = nullptr;
  size_t bytes = 0;
  if (a.argc > 2) napi_is_typedarray(env, a.v[2], &is_ta);
  if (is_ta) {
    napi_typedarray_type t;
    size_t len, boff;
    napi_value ab;
    napi_get_typedarray_info(env, a.v[2], &t, &len, &data, &ab, &boff);
    napi_value bl;
    uint32_t bpe = 1;
    if (napi_get_named_property(env, a.v[2], "BYTES_PER_ELEMENT", &bl) == napi_ok) napi_get_value_uint32(env, bl, &bpe);
    bytes = len * bpe;
  } else {
    if (a.argc > 2) napi_is_buffer(env, a.v[2], &is_buf);
    if (!is_buf) {
      a.fail("upload: expected a typed array or Buffer");
      return nullptr;
    }
    napi_get_buffer_info(env, a.v[2], &data, &bytes);
  }
  return done(env, g4_upload(c, dst, data, bytes, (size_t)off));
}

// download(ctx, src, bytes, srcOffset = 0) -> Buffer (blocking readback)
napi_value Download(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  void* src = a.ptr(1);
  const uint64_t n = a.u64(2);
  const uint64_t off = a.present(3) ? a.u64(3) : 0;
  CHECKED(a);
  void* data = nullptr;
  napi_value buf;
  if (napi_create_buffer(env, (size_t)n, &data, &buf) != napi_ok) {
    a.fail("download: cannot allocate the host buffer");
    return nullptr;
  }
  const int rc = g4_download(c, data, src, (size_t)n, (size_t)off);
  if (rc != G4_OK) return done(env, rc);
  return buf;
}

// downloadAsync(ctx, src, bytes, srcOffset = 0) -> Promise<Buffer>: the
// readback of src/engine.ts:1772-1787 (mapAsync) without blocking the event
// loop. The copy lands in pinned host memory (g4_host_alloc) behind the work
// already enqueued; a worker thread of the libuv pool waits on its event,
// and the promise resolves on the event loop with a Buffer over that memory
// (freed with the Buffer) or rejects with the library's error (code =
// G4_ERR_* name). Depth-2 pipelining submits the next step before awaiting.
struct Readback {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  g4_event* ev = nullptr;
  void* host = nullptr;
  size_t bytes = 0;
  int rc = G4_OK;
  std::string err;
};

void readback_wait(napi_env, void* data) {  // worker thread: no N-API calls here
  Readback* r = (Readback*)data;
  r->rc = g4_event_wait(r->ev);
  if (r->rc != G4_OK) r->err = g4_last_error();
}

void free_pinned(napi_env, void* data, void*) { g4_host_free(data); }

void readback_done(napi_env env, napi_status status, void* data) {
  Readback* r = (Readback*)data;
  g4_event_destroy(r->ev);
  if (status == napi_ok && r->rc == G4_OK) {
    napi_value buf;
    if (napi_create_external_buffer(env, r->bytes, r->host, free_pinned, nullptr, &buf) == napi_ok) {
      napi_resolve_deferred(env, r->deferred, buf);
    } else {
      g4_host_free(r->host);
      napi_value msg, e;
      napi_create_string_utf8(env, "downloadAsync: cannot wrap the host buffer", NAPI_AUTO_LENGTH, &msg);
      napi_create_error(env, nullptr, msg, &e);
      napi_reject_deferred(env, r->deferred, e);
    }
  } else {
    g4_host_free(r->host);
    const int rc = r->rc != G4_OK ? r->rc : G4_ERR_INVALID;
    napi_value code, msg, e;
    napi_create_string_utf8(env, status_name(rc), NAPI_AUTO_LENGTH, &code);
    napi_create_string_utf8(env, r->err.empty() ? status_name(rc) : r->err.c_str(), NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, code, msg, &e);
    napi_reject_deferred(env, r->deferred, e);
  }
  napi_delete_async_work(env, r->work);
  delete r;
}

napi_value DownloadAsync(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  void* src = a.ptr(1);
  const uint64_t n = a.u64(2);
  const uint64_t off = a.present(3) ? a.u64(3) : 0;
  CHECKED(a);
  if (n == 0) {
    a.fail("downloadAsync: zero bytes");
    return nullptr;
  }
  Readback* r = new Readback();
  r->bytes = (size_t)n;
  int rc = g4_host_alloc(c, r->bytes, &r->host);
  if (rc == G4_OK) rc = g4_download_async(c, r->host, src, r->bytes, (size_t)off, &r->ev);
  if (rc != G4_OK) {
    g4_host_free(r->host);
    delete r;
    return done(env, rc);
  }
  napi_value promise, name;
  napi_create_promise(env, &r->deferred, &promise);
  napi_create_string_utf8(env, "g4hip.downloadAsync", NAPI_AUTO_LENGTH, &name);
  napi_create_async_work(env, nullptr, name, readback_wait, readback_done, r, &r->work);
  napi_queue_async_work(env, r->work);
  return promise;
}

// eventRecord(ctx) -> handle; eventQuery(ev) -> true once complete (throws on
// a failure, G4_ERR_STALLED included); eventWait(ev); eventDestroy(ev): for
// hosts that poll instead of awaiting a promise.
napi_value EventRecord(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  CHECKED(a);
  g4_event* ev = nullptr;
  const int rc = g4_event_record(c, &ev);
  if (rc != G4_OK) return done(env, rc);
  return bigint(env, ev);
}

napi_value EventQuery(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_event* ev = (g4_event*)a.ptr(0);
  CHECKED(a);
  const int rc = g4_event_query(ev);
  if (rc < 0) return done(env, rc);
  napi_value out;
  napi_get_boolean(env, rc == 1, &out);
  return out;
}

napi_value EventWait(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_event* ev = (g4_event*)a.ptr(0);
  CHECKED(a);
  return done(env, g4_event_wait(ev));
}

napi_value EventDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_event* ev = (g4_event*)a.ptr(0);
  CHECKED(a);
  return done(env, g4_event_destroy(ev));
}

napi_value Sync(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  CHECKED(a);
  return done(env, g4_stream_sync(c));
}

napi_value GraphBegin(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  CHECKED(a);
  return done(env, g4_graph_begin(c));
}

napi_value GraphEnd(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  CHECKED(a);
  g4_graph* g = nullptr;
  const int rc = g4_graph_end(c, &g);
  if (rc != G4_OK) return done(env, rc);
  return bigint(env, g);
}

napi_value GraphLaunch(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  g4_graph* g = (g4_graph*)a.ptr(1);
  CHECKED(a);
  return done(env, g4_graph_launch(c, g));
}

napi_value GraphDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_graph* g = (g4_graph*)a.ptr(0);
  CHECKED(a);
  return done(env, g4_graph_destroy(g));
}

// fill(ctx, kind, dst, count, seed[, mean, std]): the library's seeded
// synthetic generators ('q4k' / 'q6k': count blocks; 'f16' / 'f32': values)
napi_value Fill(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const std::string kind = a.str(1);
  void* dst = a.ptr(2);
  const uint64_t n = a.u64(3), seed = a.u64(4);
  const float mean = a.present(5) ? a.f32(5) : 0.f, sd = a.present(6) ? a.f32(6) : 1.f;
  CHECKED(a);
  if (kind == "q4k") return done(env, g4_fill_q4k(c, dst, n, seed));
  if (kind == "q6k") return done(env, g4_fill_q6k(c, dst, n, seed));
  if (kind == "f16") return done(env, g4_fill_normal_f16(c, (uint16_t*)dst, n, seed, mean, sd));
  if (kind == "f32") return done(env, g4_fill_normal_f32(c, (float*)dst, n, seed, mean, sd));
  a.fail("fill: kind must be 'q4k', 'q6k', 'f16' or 'f32'");
  return nullptr;
}

// ---- kernel keys (src/shaders.ts:34-56) --------------------------------

// matmulQuant(ctx, input, weight, output, {M, N}, wtype = 'q4k')
napi_value MatmulQuant(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = F32P(a, 1);
  const void* w = a.ptr(2);
  float* y = F32P(a, 3);
  const g4_matmul_params p{a.fu32(4, "M"), a.fu32(4, "N")};
  const std::string t = a.present(5) ? a.str(5) : "q4k";
  CHECKED(a);
  if (t == "q4k") return done(env, g4_matmulQuant_q4k(c, x, w, y, p));
  if (t == "q6k") return done(env, g4_matmulQuant_q6k(c, x, w, y, p));
  if (t == "f16") return done(env, g4_matmulQuant_f16(c, x, (const uint16_t*)w, y, p));
  a.fail("matmulQuant: wtype must be 'q4k', 'q6k' or 'f16'");
  return nullptr;
}

// matmulQuantMR4(ctx, input, weight, output, {M, N})
napi_value MatmulQuantMR4(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = F32P(a, 1);
  const void* w = a.ptr(2);
  float* y = F32P(a, 3);
  const g4_matmul_params p{a.fu32(4, "M"), a.fu32(4, "N")};
  CHECKED(a);
  return done(env, g4_matmulQuantMR4_q4k(c, x, w, y, p));
}

// kvCacheStore(ctx, k_in, v_in, k_cache, v_cache, {num_kv_heads, head_dim, position, max_seq_len}[, positionDev])
napi_value KvCacheStore(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* k = F32P(a, 1);
  const float* v = F32P(a, 2);
  uint16_t* kc = U16P(a, 3);
  uint16_t* vc = U16P(a, 4);
  const g4_kv_store_params p{a.fu32(5, "num_kv_heads"), a.fu32(5, "head_dim"), a.fu32(5, "position"),
                             a.fu32(5, "max_seq_len")};
  const uint32_t* pd = U32P(a, 6);
  CHECKED(a);
  return done(env, pd ? g4_kvCacheStore_dev(c, k, v, kc, vc, p, pd) : g4_kvCacheStore(c, k, v, kc, vc, p));
}

g4_attn_score_params score_params(Args& a, size_t i) {
  return g4_attn_score_params{a.fu32(i, "num_q_heads"), a.fu32(i, "num_kv_heads"), a.fu32(i, "head_dim"),
                              a.fu32(i, "seq_len"), a.ff32(i, "scale"), a.fu32(i, "sliding_window")};
}

// attnScore(ctx, q, k_cache, scores, {num_q_heads, num_kv_heads, head_dim, seq_len, scale, sliding_window}[, positionDev])
napi_value AttnScore(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* q = F32P(a, 1);
  const uint16_t* kc = U16P(a, 2);
  float* sc = F32P(a, 3);
  const g4_attn_score_params p = score_params(a, 4);
  const uint32_t* pd = U32P(a, 5);
  CHECKED(a);
  return done(env, pd ? g4_attnScore_dev(c, q, kc, sc, p, pd) : g4_attnScore(c, q, kc, sc, p));
}

// softmax(ctx, scores, {num_heads, seq_len}[, positionDev])
napi_value Softmax(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  float* sc = F32P(a, 1);
  const g4_softmax_params p{a.fu32(2, "num_heads"), a.fu32(2, "seq_len")};
  const uint32_t* pd = U32P(a, 3);
  CHECKED(a);
  return done(env, pd ? g4_softmax_dev(c, sc, p, pd) : g4_softmax(c, sc, p));
}

// attnOutput(ctx, probs, v_cache, output, {num_q_heads, num_kv_heads, head_dim, seq_len}[, positionDev])
napi_value AttnOutput(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* pr = F32P(a, 1);
  const uint16_t* vc = U16P(a, 2);
  float* out = F32P(a, 3);
  const g4_attn_output_params p{a.fu32(4, "num_q_heads"), a.fu32(4, "num_kv_heads"), a.fu32(4, "head_dim"),
                                a.fu32(4, "seq_len")};
  const uint32_t* pd = U32P(a, 5);
  CHECKED(a);
  return done(env, pd ? g4_attnOutput_dev(c, pr, vc, out, p, pd) : g4_attnOutput(c, pr, vc, out, p));
}

// attnDecodeWorkspaceSize({num_q_heads, ...attnScore params}) -> bytes
napi_value AttnDecodeWorkspaceSize(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const g4_attn_score_params p = score_params(a, 0);
  CHECKED(a);
  size_t n = 0;
  const int rc = g4_attnDecode_workspace_size(p, &n);
  if (rc != G4_OK) return done(env, rc);
  return number(env, (double)n);
}

// attnDecode(ctx, q, k_cache, v_cache, output, {attnScore params}, workspace, workspaceBytes[, positionDev]):
// the attnScore -> softmax -> attnOutput trio in one split-K pass
napi_value AttnDecode(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* q = F32P(a, 1);
  const uint16_t* kc = U16P(a, 2);
  const uint16_t* vc = U16P(a, 3);
  float* out = F32P(a, 4);
  const g4_attn_score_params p = score_params(a, 5);
  void* ws = a.ptr(6);
  const uint64_t wsb = a.u64(7);
  const uint32_t* pd = U32P(a, 8);
  CHECKED(a);
  return done(env, pd ? g4_attnDecode_dev(c, q, kc, vc, out, p, ws, (size_t)wsb, pd)
                      : g4_attnDecode(c, q, kc, vc, out, p, ws, (size_t)wsb));
}

// perHeadRmsNormNoWeight(ctx, data, {num_heads, head_dim, eps})
napi_value PerHeadRmsNormNoWeight(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  float* d = F32P(a, 1);
  const g4_per_head_norm_params p{a.fu32(2, "num_heads"), a.fu32(2, "head_dim"), a.ff32(2, "eps"), 0u};
  CHECKED(a);
  return done(env, g4_perHeadRmsNormNoWeight(c, d, p));
}

// fusedPerHeadNormRope(ctx, data, weight, {num_heads, head_dim, eps, position, theta, apply_divisor},
//                      rope_freqs[, positionDev])
napi_value FusedPerHeadNormRope(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  float* d = F32P(a, 1);
  const uint16_t* w = U16P(a, 2);
  const g4_norm_rope_params p{a.fu32(3, "num_heads"), a.fu32(3, "head_dim"), a.ff32(3, "eps"),
                              a.fu32(3, "position"),  a.ff32(3, "theta"),    a.fu32(3, "apply_divisor")};
  const uint16_t* rf = U16P(a, 4);
  const uint32_t* pd = U32P(a, 5);
  CHECKED(a);
  return done(env, pd ? g4_fusedPerHeadNormRope_dev(c, d, w, p, rf, pd) : g4_fusedPerHeadNormRope(c, d, w, p, rf));
}

// rmsNorm(ctx, input, weight, output, {hidden_size, eps})
napi_value RmsNorm(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = F32P(a, 1);
  const uint16_t* w = U16P(a, 2);
  float* out = F32P(a, 3);
  const g4_rms_norm_params p{a.fu32(4, "hidden_size"), a.ff32(4, "eps")};
  CHECKED(a);
  return done(env, g4_rmsNorm(c, x, w, out, p));
}

// fusedNormAdd(ctx, input, weight, residual, output, {size, eps})
napi_value FusedNormAdd(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = F32P(a, 1);
  const uint16_t* w = U16P(a, 2);
  const float* r = F32P(a, 3);
  float* out = F32P(a, 4);
  const g4_norm_add_params p{a.fu32(5, "size"), a.ff32(5, "eps")};
  CHECKED(a);
  return done(env, g4_fusedNormAdd(c, x, w, r, out, p));
}

// geluMul(ctx, gate, up, output, size)
napi_value GeluMul(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* g = F32P(a, 1);
  const float* u = F32P(a, 2);
  float* out = F32P(a, 3);
  const uint32_t n = a.u32(4);
  CHECKED(a);
  return done(env, g4_geluMul(c, g, u, out, n));
}

// logitSoftcap(ctx, logits, {size, cap})
napi_value LogitSoftcap(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  float* lg = F32P(a, 1);
  const g4_softcap_params p{a.fu32(2, "size"), a.ff32(2, "cap")};
  CHECKED(a);
  return done(env, g4_logitSoftcap(c, lg, p));
}

// embeddingLookup(ctx, embedding, num_rows, output, {hidden_size, token_id}[, tokenDev])
napi_value EmbeddingLookup(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const uint16_t* e = U16P(a, 1);
  const uint32_t rows = a.u32(2);
  float* out = F32P(a, 3);
  const g4_embedding_params p{a.fu32(4, "hidden_size"), a.fu32(4, "token_id")};
  const uint32_t* td = U32P(a, 5);
  CHECKED(a);
  return done(env, td ? g4_embeddingLookup_dev(c, e, rows, out, p, td) : g4_embeddingLookup(c, e, rows, out, p));
}

// ---- per-layer embeddings (shaders/ple_*.wgsl) --------------------------

// pleStage1Fuse(ctx, projected, norm_weight, table_q5k, table_rows, ple_inputs,
//               {num_layers, per_layer_dim, eps, token_id}[, tokenDev[, count]]):
// every layer in one dispatch (the reference dispatches one workgroup per
// layer); with tokenDev and count, the rows of count tokens at once.
napi_value PleStage1Fuse(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* proj = F32P(a, 1);
  const uint16_t* w = U16P(a, 2);
  const void* table = a.ptr(3);
  const uint32_t rows = a.u32(4);
  float* out = F32P(a, 5);
  const uint32_t nl = a.fu32(6, "num_layers"), dim = a.fu32(6, "per_layer_dim"), tok = a.fu32(6, "token_id");
  const float eps = a.ff32(6, "eps");
  const uint32_t* td = U32P(a, 7);
  const uint32_t count = a.present(8) ? a.u32(8) : 1;
  CHECKED(a);
  return done(env, g4_pleStage1Fuse(c, proj, w, table, rows, tok, td, out, nl, dim, eps, count));
}

// pleGeluMul(ctx, gate, ple_inputs, output, {layer_offset, size})
napi_value PleGeluMul(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* g = F32P(a, 1);
  const float* ple = F32P(a, 2);
  float* out = F32P(a, 3);
  const uint32_t off = a.fu32(4, "layer_offset"), n = a.fu32(4, "size");
  CHECKED(a);
  return done(env, g4_pleGeluMul(c, g, ple, out, off, n));
}

// pleSkipScaleAdd(ctx, hidden, post_normed, scale, {size})
napi_value PleSkipScaleAdd(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  float* h = F32P(a, 1);
  const float* pn = F32P(a, 2);
  const uint16_t* sc = U16P(a, 3);
  const uint32_t n = a.fu32(4, "size");
  CHECKED(a);
  return done(env, g4_pleSkipScaleAdd(c, h, pn, sc, n));
}

// argmax(ctx, logits, result, size)
napi_value Argmax(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* lg = F32P(a, 1);
  uint32_t* r = U32P(a, 2);
  const uint32_t n = a.u32(3);
  CHECKED(a);
  return done(env, g4_argmax(c, lg, r, n));
}

// topk256(ctx, logits, result, size)
napi_value Topk256(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* lg = F32P(a, 1);
  float* r = F32P(a, 2);
  const uint32_t n = a.u32(3);
  CHECKED(a);
  return done(env, g4_topk256(c, lg, r, n));
}

// advancePosition(ctx, positionDev, delta = 1)
napi_value AdvancePosition(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  uint32_t* pd = U32P(a, 1);
  const uint32_t d = a.present(2) ? a.u32(2) : 1u;
  CHECKED(a);
  return done(env, g4_advancePosition(c, pd, d));
}

// ---- GGUF files (GGUFParser, src/gguf.ts:75-101) ------------------------

// ggufOpen(path) -> handle (the file stays mapped until ggufClose)
napi_value GgufOpen(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const std::string path = a.str(0);
  CHECKED(a);
  g4_gguf* g = nullptr;
  const int rc = g4_gguf_open(path.c_str(), &g);
  if (rc != G4_OK) return done(env, rc);
  return bigint(env, g);
}

napi_value GgufClose(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_gguf* g = (g4_gguf*)a.ptr(0);
  CHECKED(a);
  return done(env, g4_gguf_close(g));
}

void set_num(napi_env env, napi_value o, const char* k, double d) {
  napi_set_named_property(env, o, k, number(env, d));
}

// ggufInfo(handle) -> {version, tensorCount, kvCount, dataOffset, alignment}
napi_value GgufInfo(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const g4_gguf* g = (const g4_gguf*)a.ptr(0);
  CHECKED(a);
  uint32_t v = 0, al = 0;
  uint64_t nt = 0, nkv = 0, off = 0;
  const int rc = g4_gguf_info(g, &v, &nt, &nkv, &off, &al);
  if (rc != G4_OK) return done(env, rc);
  napi_value o;
  napi_create_object(env, &o);
  set_num(env, o, "version", v);
  set_num(env, o, "tensorCount", (double)nt);
  set_num(env, o, "kvCount", (double)nkv);
  set_num(env, o, "dataOffset", (double)off);
  set_num(env, o, "alignment", al);
  return o;
}

// the reference's GGUFValue type names (src/gguf.ts:50-72)
const char* value_type_name(uint32_t t) {
  static const char* names[] = {"uint8", "int8", "uint16", "int16", "uint32", "int32", "float32",
                                "bool", "string", "array", "uint64", "int64", "float64"};
  return t < 13 ? names[t] : "unknown";
}

// one element as {type, value}: 64-bit integers as BigInt, the rest as Number /
// Boolean / String
napi_value gguf_value(napi_env env, const g4_gguf* g, uint64_t i, uint64_t e, uint32_t t, int* rc) {
  napi_value o, val;
  napi_create_object(env, &o);
  napi_value tn;
  napi_create_string_utf8(env, value_type_name(t), NAPI_AUTO_LENGTH, &tn);
  napi_set_named_property(env, o, "type", tn);
  if (t == 8) {
    const char* s = nullptr;
    uint64_t n = 0;
    *rc = g4_gguf_kv_string(g, i, e, &s, &n);
    if (*rc) return nullptr;
    napi_create_string_utf8(env, s, (size_t)n, &val);
  } else {
    double f = 0;
    int64_t iv = 0;
    uint64_t u = 0;
    *rc = g4_gguf_kv_number(g, i, e, &f, &iv, &u);
    if (*rc) return nullptr;
    if (t == 10) napi_create_bigint_uint64(env, u, &val);
    else if (t == 11) napi_create_bigint_int64(env, iv, &val);
    else if (t == 7) napi_get_boolean(env, u != 0, &val);
    else napi_create_double(env, f, &val);
  }
  napi_set_named_property(env, o, "value", val);
  return o;
}

// ggufMetadata(handle) -> {key: {type, value}} as GGUFParser's kv map
// (arrays: value is an array of {type, value}; nested arrays: value null)
napi_value GgufMetadata(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const g4_gguf* g = (const g4_gguf*)a.ptr(0);
  CHECKED(a);
  uint64_t nkv = 0;
  int rc = g4_gguf_info(g, nullptr, nullptr, &nkv, nullptr, nullptr);
  if (rc != G4_OK) return done(env, rc);
  napi_value out;
  napi_create_object(env, &out);
  for (uint64_t i = 0; i < nkv; ++i) {
    const char* key = nullptr;
    uint32_t t = 0, at = 0;
    uint64_t n = 0;
    rc = g4_gguf_kv(g, i, &key, &t, &at, &n);
    if (rc != G4_OK) return done(env, rc);
    napi_value entry;
    if (t == 9) {
      napi_create_object(env, &entry);
      napi_value tn, arr;
      napi_create_string_utf8(env, "array", NAPI_AUTO_LENGTH, &tn);
      napi_set_named_property(env, entry, "type", tn);
      if (at == 9) {
        napi_get_null(env, &arr);
      } else {
        napi_create_array_with_length(env, (size_t)n, &arr);
        for (uint64_t e = 0; e < n; ++e) {
          napi_value el = gguf_value(env, g, i, e, at, &rc);
          if (rc != G4_OK) return done(env, rc);
          napi_set_element(env, arr, (uint32_t)e, el);
        }
      }
      napi_set_named_property(env, entry, "value", arr);
    } else {
      entry = gguf_value(env, g, i, 0, t, &rc);
      if (rc != G4_OK) return done(env, rc);
    }
    napi_set_named_property(env, out, key, entry);
  }
  return out;
}

// ggufTensors(handle) -> [{name, dims, type, offset, nbytes, index}] (GGUFTensor)
napi_value GgufTensors(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const g4_gguf* g = (const g4_gguf*)a.ptr(0);
  CHECKED(a);
  uint64_t nt = 0;
  int rc = g4_gguf_info(g, nullptr, &nt, nullptr, nullptr, nullptr);
  if (rc != G4_OK) return done(env, rc);
  napi_value out;
  napi_create_array_with_length(env, (size_t)nt, &out);
  for (uint64_t i = 0; i < nt; ++i) {
    const char* name = nullptr;
    uint32_t nd = 0, t = 0;
    uint64_t dims[4], off = 0, nb = 0;
    rc = g4_gguf_tensor(g, i, &name, &nd, dims, &t, &off, &nb);
    if (rc != G4_OK) return done(env, rc);
    napi_value o, nm, dv;
    napi_create_object(env, &o);
    napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &nm);
    napi_set_named_property(env, o, "name", nm);
    napi_create_array_with_length(env, nd, &dv);
    for (uint32_t d = 0; d < nd; ++d) napi_set_element(env, dv, d, number(env, (double)dims[d]));
    napi_set_named_property(env, o, "dims", dv);
    set_num(env, o, "type", t);
    set_num(env, o, "offset", (double)off);
    set_num(env, o, "nbytes", (double)nb);
    set_num(env, o, "index", (double)i);
    napi_set_element(env, out, (uint32_t)i, o);
  }
  return out;
}

// ggufUpload(ctx, handle, index, dst, dstBytes): the tensor's bytes as they are
napi_value GgufUpload(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const g4_gguf* g = (const g4_gguf*)a.ptr(1);
  const uint64_t idx = a.u64(2);
  void* dst = a.ptr(3);
  const uint64_t n = a.u64(4);
  CHECKED(a);
  return done(env, g4_gguf_upload(c, g, idx, dst, (size_t)n));
}

// ggufUploadF16(ctx, handle, index, dst, dstElems): F32 / F16 / BF16 as f16
napi_value GgufUploadF16(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const g4_gguf* g = (const g4_gguf*)a.ptr(1);
  const uint64_t idx = a.u64(2);
  uint16_t* dst = U16P(a, 3);
  const uint64_t n = a.u64(4);
  CHECKED(a);
  return done(env, g4_gguf_upload_f16(c, g, idx, dst, (size_t)n));
}

// dequantF16(ctx, 'q4k' | 'q6k' | 'q5k' | 'q8_0', blocks, nblocks, out):
// blocks (256 values; Q8_0: 32) to f16 rows
napi_value DequantF16(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const std::string t = a.str(1);
  const void* b = a.ptr(2);
  const uint64_t n = a.u64(3);
  uint16_t* out = U16P(a, 4);
  CHECKED(a);
  const int w = t == "q4k" ? 0 : t == "q6k" ? 1 : t == "q5k" ? 2 : t == "q8_0" ? 3 : -1;
  if (w < 0) {
    a.fail("dequantF16: wtype must be 'q4k', 'q6k', 'q5k' or 'q8_0'");
    return nullptr;
  }
  return done(env, g4_dequantF16(c, w, b, n, out));
}

// ---- the MI355X decode step (Decoder.step_fused in g4hip/decoder.py) -----
// Keys with no counterpart among the reference's kernel keys: a host that
// captures the whole step as a graph issues these instead of the per-key
// sequence. Buffers travel in a plain object by name (BigInt or null).

void* fptr(Args& a, size_t i, const char* name) {
  napi_value f = nullptr;
  bool has = false;
  if (i >= a.argc || napi_has_named_property(a.env, a.v[i], name, &has) != napi_ok || !has) return nullptr;
  napi_get_named_property(a.env, a.v[i], name, &f);
  napi_valuetype t;
  napi_typeof(a.env, f, &t);
  if (t == napi_undefined || t == napi_null) return nullptr;
  uint64_t p = 0;
  bool lossless = false;
  if (napi_get_value_bigint_uint64(a.env, f, &p, &lossless) != napi_ok || !lossless) {
    std::string m = std::string("field '") + name + "' must be a BigInt device handle (or null)";
    a.fail(m.c_str());
    return nullptr;
  }
  return (void*)(uintptr_t)p;
}

// an array of up to `maxn` BigInt handles (kind 0) or numbers (kind 1) at argument i
int array_at(Args& a, size_t i, void** ptrs, uint32_t* nums, int maxn, int kind) {
  bool is = false;
  if (i >= a.argc || napi_is_array(a.env, a.v[i], &is) != napi_ok || !is) {
    a.fail("expected an array");
    return 0;
  }
  uint32_t n = 0;
  napi_get_array_length(a.env, a.v[i], &n);
  if (n < 1 || (int)n > maxn) {
    a.fail("array length out of range");
    return 0;
  }
  for (uint32_t k = 0; k < n; ++k) {
    napi_value e;
    napi_get_element(a.env, a.v[i], k, &e);
    if (kind == 0) {
      uint64_t p = 0;
      bool lossless = false;
      if (napi_get_value_bigint_uint64(a.env, e, &p, &lossless) != napi_ok || !lossless) {
        a.fail("expected BigInt device handles");
        return 0;
      }
      ptrs[k] = (void*)(uintptr_t)p;
    } else if (napi_get_value_uint32(a.env, e, &nums[k]) != napi_ok) {
      a.fail("expected numbers");
      return 0;
    }
  }
  return (int)n;
}

g4_attn_fused_params fused_params(Args& a, size_t i) {
  g4_attn_fused_params p{};
  p.num_q_heads = a.fu32(i, "num_q_heads");
  p.num_kv_heads = a.fu32(i, "num_kv_heads");
  p.head_dim = a.fu32(i, "head_dim");
  p.max_seq_len = a.fu32(i, "max_seq_len");
  p.scale = a.ff32(i, "scale");
  p.sliding_window = a.fu32(i, "sliding_window");
  p.eps = a.ff32(i, "eps");
  p.theta = a.ff32(i, "theta");
  p.apply_divisor = a.fu32(i, "apply_divisor");
  return p;
}

int wtype_of(Args& a, size_t i) {
  const std::string t = a.str(i);
  if (t == "q4k") return 0;
  if (t == "q6k") return 1;
  a.fail("wtype must be 'q4k' or 'q6k'");
  return -1;
}

// digitsBytes(K) -> bytes of a digit block over K activations
napi_value DigitsBytes(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const uint32_t K = a.u32(0);
  CHECKED(a);
  size_t n = 0;
  const int rc = g4_digitsBytes(K, &n);
  if (rc != G4_OK) return done(env, rc);
  return number(env, (double)n);
}

// attnFusedWorkspaceSize(params) -> bytes (zero them once; the kernels keep their counters zero)
napi_value AttnFusedWorkspaceSize(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const g4_attn_fused_params p = fused_params(a, 0);
  CHECKED(a);
  size_t n = 0;
  const int rc = g4_attnDecodeFused_workspace_size(p, &n);
  if (rc != G4_OK) return done(env, rc);
  return number(env, (double)n);
}

// ropeTable(ctx, theta, applyDivisor, ropeFreqs, headDim, rows, table)
napi_value RopeTable(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float theta = a.f32(1);
  const uint32_t ad = a.u32(2);
  const uint16_t* rf = U16P(a, 3);
  const uint32_t hd = a.u32(4), rows = a.u32(5);
  float* t = F32P(a, 6);
  CHECKED(a);
  return done(env, g4_ropeTable(c, theta, ad, rf, hd, rows, t));
}

// matmulWarmRegion(ctx, wtype, M, N, weight) -> {base, totalBytes, wgBytes, nwgs}:
// the bytes each workgroup of the one-vector matvec over W [M x N] reads
napi_value MatmulWarmRegion(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const int wt = wtype_of(a, 1);
  const uint32_t M = a.u32(2), N = a.u32(3);
  const void* w = a.ptr(4);
  CHECKED(a);
  g4_warm_region r{};
  const int rc = g4_matmulWarmRegion(c, wt, M, N, w, &r);
  if (rc != G4_OK) return done(env, rc);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "base", bigint(env, r.base));
  napi_set_named_property(env, o, "totalBytes", number(env, (double)r.total_bytes));
  napi_set_named_property(env, o, "wgBytes", number(env, (double)r.wg_bytes));
  napi_set_named_property(env, o, "nwgs", number(env, r.nwgs));
  return o;
}

// up to 4 regions from an array of matmulWarmRegion objects at argument i
int regions_at(Args& a, size_t i, g4_warm_region* out) {
  if (!a.present(i)) return 0;
  bool is = false;
  uint32_t n = 0;
  if (napi_is_array(a.env, a.v[i], &is) != napi_ok || !is || napi_get_array_length(a.env, a.v[i], &n) != napi_ok ||
      n > 4) {
    a.fail("regions: an array of at most 4 matmulWarmRegion objects");
    return 0;
  }
  for (uint32_t k = 0; k < n; ++k) {
    napi_value e, f;
    napi_get_element(a.env, a.v[i], k, &e);
    uint64_t p = 0;
    bool lossless = false;
    double d = 0;
    if (napi_get_named_property(a.env, e, "base", &f) != napi_ok ||
        napi_get_value_bigint_uint64(a.env, f, &p, &lossless) != napi_ok || !lossless) {
      a.fail("region base must be a BigInt");
      return 0;
    }
    out[k].base = (const void*)(uintptr_t)p;
    napi_get_named_property(a.env, e, "totalBytes", &f);
    napi_get_value_double(a.env, f, &d);
    out[k].total_bytes = (uint64_t)d;
    napi_get_named_property(a.env, e, "wgBytes", &f);
    napi_get_value_double(a.env, f, &d);
    out[k].wg_bytes = (uint64_t)d;
    napi_get_named_property(a.env, e, "nwgs", &f);
    napi_get_value_double(a.env, f, &d);
    out[k].nwgs = (uint32_t)d;
    out[k].reserved = 0;
  }
  return (int)n;
}

// attnDecodeFused(ctx, {q, k, v, qNorm, kNorm, ropeFreqs, kCache, vCache, out,
//   workspace, position, ropeCs}, params, workspaceBytes, ropeRows[, regions]):
// the fused attention block at the device position; its idle workgroups read
// `regions` (matmulWarmRegion of the launches that follow) into the L2 caches
napi_value AttnDecodeFused(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* q = (const float*)fptr(a, 1, "q");
  const float* k = (const float*)fptr(a, 1, "k");
  const float* v = (const float*)fptr(a, 1, "v");
  const uint16_t* qn = (const uint16_t*)fptr(a, 1, "qNorm");
  const uint16_t* kn = (const uint16_t*)fptr(a, 1, "kNorm");
  const uint16_t* rf = (const uint16_t*)fptr(a, 1, "ropeFreqs");
  uint16_t* kc = (uint16_t*)fptr(a, 1, "kCache");
  uint16_t* vc = (uint16_t*)fptr(a, 1, "vCache");
  float* out = (float*)fptr(a, 1, "out");
  void* ws = fptr(a, 1, "workspace");
  const uint32_t* pos = (const uint32_t*)fptr(a, 1, "position");
  const float* cs = (const float*)fptr(a, 1, "ropeCs");
  const g4_attn_fused_params p = fused_params(a, 2);
  const uint64_t wsb = a.u64(3);
  const uint32_t rows = a.present(4) ? a.u32(4) : 0;
  g4_warm_region reg[4] = {};
  const int nreg = regions_at(a, 5, reg);
  CHECKED(a);
  return done(env, g4_attnDecodeFusedWarm(c, q, k, v, qn, kn, rf, kc, vc, out, p, ws, (size_t)wsb, pos,
                                          nreg ? reg : nullptr, nreg, cs, rows));
}

// normAddScaleMatmulSegments(ctx, wtype, {x, w1, residual, scale, w2, hOut},
//   weights[], outputs[], rows[], N, eps)
napi_value NormAddScaleMatmulSegments(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const int wt = wtype_of(a, 1);
  const float* x = (const float*)fptr(a, 2, "x");
  const uint16_t* w1 = (const uint16_t*)fptr(a, 2, "w1");
  const float* res = (const float*)fptr(a, 2, "residual");
  const uint16_t* sc = (const uint16_t*)fptr(a, 2, "scale");
  const uint16_t* w2 = (const uint16_t*)fptr(a, 2, "w2");
  float* h = (float*)fptr(a, 2, "hOut");
  void* W[4] = {};
  void* Y[4] = {};
  uint32_t R[4] = {};
  const int n = array_at(a, 3, W, nullptr, 4, 0);
  const int ny = array_at(a, 4, Y, nullptr, 4, 0);
  const int nr = array_at(a, 5, nullptr, R, 4, 1);
  const uint32_t N = a.u32(6);
  const float eps = a.f32(7);
  CHECKED(a);
  if (n != ny || n != nr) {
    a.fail("weights, outputs and rows differ in length");
    return nullptr;
  }
  return done(env, g4_normAddScaleMatmulSegments(c, wt, x, w1, res, sc, w2, h, W, (float* const*)Y, R, n, N, eps,
                                                 0.f));
}

// qkvAttnDecodeFused(ctx, {x, w1, residual, scale, w2, hOut}, weights[], outputs[], N, eps,
//   {qNorm, kNorm, ropeFreqs, kCache, vCache, out, workspace, position, ropeCs}, params, workspaceBytes,
//   ropeRows[, regions]): the Q4_K q (or q/k/v) matvecs and the attention
// block over them, in one launch where the shape allows
napi_value QkvAttnDecodeFused(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = (const float*)fptr(a, 1, "x");
  const uint16_t* w1 = (const uint16_t*)fptr(a, 1, "w1");
  const float* res = (const float*)fptr(a, 1, "residual");
  const uint16_t* sc = (const uint16_t*)fptr(a, 1, "scale");
  const uint16_t* w2 = (const uint16_t*)fptr(a, 1, "w2");
  float* h = (float*)fptr(a, 1, "hOut");
  void* W[4] = {};
  void* Y[4] = {};
  const int n = array_at(a, 2, W, nullptr, 3, 0);
  const int ny = array_at(a, 3, Y, nullptr, 3, 0);
  const uint32_t N = a.u32(4);
  const float eps = a.f32(5);
  const uint16_t* qn = (const uint16_t*)fptr(a, 6, "qNorm");
  const uint16_t* kn = (const uint16_t*)fptr(a, 6, "kNorm");
  const uint16_t* rf = (const uint16_t*)fptr(a, 6, "ropeFreqs");
  uint16_t* kc = (uint16_t*)fptr(a, 6, "kCache");
  uint16_t* vc = (uint16_t*)fptr(a, 6, "vCache");
  float* out = (float*)fptr(a, 6, "out");
  void* ws = fptr(a, 6, "workspace");
  const uint32_t* pos = (const uint32_t*)fptr(a, 6, "position");
  const float* cs = (const float*)fptr(a, 6, "ropeCs");
  const g4_attn_fused_params p = fused_params(a, 7);
  const uint64_t wsb = a.u64(8);
  const uint32_t rows = a.u32(9);
  g4_warm_region reg[4] = {};
  const int nreg = regions_at(a, 10, reg);
  CHECKED(a);
  if (n != ny) {
    a.fail("weights and outputs differ in length");
    return nullptr;
  }
  return done(env, g4_qkvAttnDecodeFusedWarm(c, x, w1, res, sc, w2, h, W, (float* const*)Y, n, N, eps, qn, kn, rf,
                                             kc, vc, out, p, ws, (size_t)wsb, pos, nreg ? reg : nullptr, nreg, cs,
                                             rows));
}

// normAddGateUpGeluDigits(ctx, {o, wPost, residual, wPre, wGate, wUp, hOut, out, digits}, {M, N}, eps)
napi_value NormAddGateUpGeluDigits(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* o = (const float*)fptr(a, 1, "o");
  const uint16_t* wpo = (const uint16_t*)fptr(a, 1, "wPost");
  const float* res = (const float*)fptr(a, 1, "residual");
  const uint16_t* wpr = (const uint16_t*)fptr(a, 1, "wPre");
  const void* wg = fptr(a, 1, "wGate");
  const void* wu = fptr(a, 1, "wUp");
  float* h = (float*)fptr(a, 1, "hOut");
  float* out = (float*)fptr(a, 1, "out");
  void* dg = fptr(a, 1, "digits");
  g4_matmul_params p{a.fu32(2, "M"), a.fu32(2, "N")};
  const float eps = a.f32(3);
  CHECKED(a);
  return done(env, g4_normAddGateUpGeluDigits_q4k(c, o, wpo, res, wpr, wg, wu, h, out, dg, p, eps));
}

// matmulQuantDigits(ctx, digits, weight, output, {M, N}): Q6_K over a digit block
napi_value MatmulQuantDigits(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const void* dg = a.ptr(1);
  const void* w = a.ptr(2);
  float* y = F32P(a, 3);
  g4_matmul_params p{a.fu32(4, "M"), a.fu32(4, "N")};
  CHECKED(a);
  return done(env, g4_matmulQuantDigits_q6k(c, dg, w, y, p));
}

// normAddMatmulArgmax(ctx, wtype, {x, w1, residual, w2, hOut, weight, logits, result, positions},
//   rows, N, eps, softcap, delta): the LM head with its argmax candidates
napi_value NormAddMatmulArgmax(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const int wt = wtype_of(a, 1);
  const float* x = (const float*)fptr(a, 2, "x");
  const uint16_t* w1 = (const uint16_t*)fptr(a, 2, "w1");
  const float* res = (const float*)fptr(a, 2, "residual");
  const uint16_t* w2 = (const uint16_t*)fptr(a, 2, "w2");
  float* h = (float*)fptr(a, 2, "hOut");
  const void* w = fptr(a, 2, "weight");
  float* lg = (float*)fptr(a, 2, "logits");
  uint32_t* r = (uint32_t*)fptr(a, 2, "result");
  uint32_t* pos = (uint32_t*)fptr(a, 2, "positions");
  const uint32_t rows = a.u32(3), N = a.u32(4);
  const float eps = a.f32(5), cap = a.f32(6);
  const uint32_t delta = a.u32(7);
  CHECKED(a);
  return done(env, g4_normAddMatmulArgmax(c, wt, x, w1, res, w2, h, w, lg, rows, N, eps, cap, r, pos, delta));
}

// pleGate(ctx, {x, w1, residual, hOut, wGate, pleInputs, out}, {M, N, ple_stride, layer_offset, batch}, eps)
napi_value PleGate(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = (const float*)fptr(a, 1, "x");
  const uint16_t* w1 = (const uint16_t*)fptr(a, 1, "w1");
  const float* res = (const float*)fptr(a, 1, "residual");
  float* h = (float*)fptr(a, 1, "hOut");
  const uint16_t* wg = (const uint16_t*)fptr(a, 1, "wGate");
  const float* pin = (const float*)fptr(a, 1, "pleInputs");
  float* out = (float*)fptr(a, 1, "out");
  const uint32_t M = a.fu32(2, "M"), N = a.fu32(2, "N"), st = a.fu32(2, "ple_stride");
  const uint32_t off = a.fu32(2, "layer_offset"), b = a.fu32(2, "batch");
  const float eps = a.f32(3);
  CHECKED(a);
  return done(env, g4_pleGate(c, x, w1, res, h, wg, pin, st, off, out, M, N, eps, b));
}

// matmulF16(ctx, x, weight, y, {M, N, batch}): f16 rows times f32 vectors
napi_value MatmulF16(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = F32P(a, 1);
  const uint16_t* w = U16P(a, 2);
  float* y = F32P(a, 3);
  const uint32_t M = a.fu32(4, "M"), N = a.fu32(4, "N"), b = a.fu32(4, "batch");
  CHECKED(a);
  return done(env, g4_matmulF16(c, x, w, y, M, N, b));
}

// batchPrepScale(ctx, {x, w1, residual, scale, w2, hOut, out}, {nparts, N, batch}, eps)
napi_value BatchPrepScale(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = (const float*)fptr(a, 1, "x");
  const uint16_t* w1 = (const uint16_t*)fptr(a, 1, "w1");
  const float* res = (const float*)fptr(a, 1, "residual");
  const uint16_t* sc = (const uint16_t*)fptr(a, 1, "scale");
  const uint16_t* w2 = (const uint16_t*)fptr(a, 1, "w2");
  float* h = (float*)fptr(a, 1, "hOut");
  float* out = (float*)fptr(a, 1, "out");
  void* ops = fptr(a, 1, "ops");
  const uint32_t np = a.fu32(2, "nparts"), N = a.fu32(2, "N"), b = a.fu32(2, "batch");
  const float eps = a.f32(3);
  CHECKED(a);
  return done(env, g4_batchPrepScale(c, x, np, w1, res, sc, w2, h, out, ops, N, b, eps));
}

// argmaxAdvance(ctx, logits, result, size, positions, delta): argmax, then *positions += delta
napi_value ArgmaxAdvance(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* lg = F32P(a, 1);
  uint32_t* r = U32P(a, 2);
  const uint32_t n = a.u32(3);
  uint32_t* pos = U32P(a, 4);
  const uint32_t d = a.u32(5);
  CHECKED(a);
  return done(env, g4_argmaxAdvance(c, lg, r, n, 1, pos, d));
}

// ---- the ragged multi-sequence step and the batched prefill --------------
// (BatchDecoder.step / prefill in g4hip/decoder.py.) The reference runs one
// forward per sequence and per prompt token (src/engine.ts:1923-1938); these
// keys take `batch` rows at once over paged K/V pools (pages of page_size
// rows [num_kv_heads][head_dim], a page table per row, the row lengths on the
// device). Paged params travel as plain objects with the C structs' fields.

g4_paged_attn_params paged_params(Args& a, size_t i) {
  g4_paged_attn_params p{};
  p.num_seqs = a.fu32(i, "num_seqs");
  p.num_q_heads = a.fu32(i, "num_q_heads");
  p.num_kv_heads = a.fu32(i, "num_kv_heads");
  p.head_dim = a.fu32(i, "head_dim");
  p.page_size = a.fu32(i, "page_size");
  p.max_pages = a.fu32(i, "max_pages");
  p.max_seq_len = a.fu32(i, "max_seq_len");
  p.num_pages = a.fu32(i, "num_pages");
  p.scale = a.ff32(i, "scale");
  p.sliding_window = a.fu32(i, "sliding_window");
  return p;
}

g4_paged_attn_fused_params paged_fused_params(Args& a, size_t i) {
  const g4_paged_attn_params b = paged_params(a, i);
  g4_paged_attn_fused_params p{};
  p.num_seqs = b.num_seqs;
  p.num_q_heads = b.num_q_heads;
  p.num_kv_heads = b.num_kv_heads;
  p.head_dim = b.head_dim;
  p.page_size = b.page_size;
  p.max_pages = b.max_pages;
  p.max_seq_len = b.max_seq_len;
  p.num_pages = b.num_pages;
  p.scale = b.scale;
  p.sliding_window = b.sliding_window;
  p.eps = a.ff32(i, "eps");
  p.theta = a.ff32(i, "theta");
  p.apply_divisor = a.fu32(i, "apply_divisor");
  return p;
}

napi_value size_result(napi_env env, int rc, size_t n) {
  if (rc != G4_OK) return done(env, rc);
  return number(env, (double)n);
}

// batchOperandBytes(N, batch) / batchSubOperandBytes(K, batch) -> bytes of the
// matrix-core operand blocks of `batch` vectors of N (K) values
napi_value BatchOperandBytes(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const uint32_t N = a.u32(0), b = a.u32(1);
  CHECKED(a);
  size_t n = 0;
  const int rc = g4_batchOperandBytes(N, b, &n);
  return size_result(env, rc, n);
}
napi_value BatchSubOperandBytes(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const uint32_t K = a.u32(0), b = a.u32(1);
  CHECKED(a);
  size_t n = 0;
  const int rc = g4_batchSubOperandBytes(K, b, &n);
  return size_result(env, rc, n);
}

// pagedAttnWorkspaceSize(params) -> bytes of pagedAttnDecode's split-K workspace
napi_value PagedAttnWorkspaceSize(napi_env env, napi_callback_info info) {
  Args a(env, info);
  const g4_paged_attn_params p = paged_params(a, 0);
  CHECKED(a);
  size_t n = 0;
  const int rc = g4_pagedAttnDecode_workspace_size(p, &n);
  return size_result(env, rc, n);
}

// copy(ctx, dst, src, bytes): a device-to-device copy on the stream
napi_value Copy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  void* d = a.ptr(1);
  const void* s = a.ptr(2);
  const uint64_t n = a.u64(3);
  CHECKED(a);
  return done(env, g4_copy_d2d(c, d, s, n));
}

// embeddingLookupBatch(ctx, embedding, num_rows, output, {hidden_size}, tokensDev, count)
napi_value EmbeddingLookupBatch(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const uint16_t* e = U16P(a, 1);
  const uint32_t rows = a.u32(2);
  float* out = F32P(a, 3);
  const uint32_t H = a.fu32(4, "hidden_size");
  const uint32_t* td = U32P(a, 5);
  const uint32_t n = a.u32(6);
  CHECKED(a);
  return done(env, g4_embeddingLookupBatch(c, e, rows, out, H, td, n));
}

// advanceSeqLens(ctx, seqLens, numSeqs, delta)
napi_value AdvanceSeqLens(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  uint32_t* sl = U32P(a, 1);
  const uint32_t n = a.u32(2), d = a.u32(3);
  CHECKED(a);
  return done(env, g4_advanceSeqLens(c, sl, n, d));
}

// batchPrep(ctx, {x, w1, residual, w2, hOut, out, ops}, {nparts, N, batch}, eps)
napi_value BatchPrep(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = (const float*)fptr(a, 1, "x");
  const uint16_t* w1 = (const uint16_t*)fptr(a, 1, "w1");
  const float* res = (const float*)fptr(a, 1, "residual");
  const uint16_t* w2 = (const uint16_t*)fptr(a, 1, "w2");
  float* h = (float*)fptr(a, 1, "hOut");
  float* out = (float*)fptr(a, 1, "out");
  void* ops = fptr(a, 1, "ops");
  const uint32_t np = a.fu32(2, "nparts"), N = a.fu32(2, "N"), b = a.fu32(2, "batch");
  const float eps = a.f32(3);
  CHECKED(a);
  return done(env, g4_batchPrep(c, x, np, w1, res, w2, h, out, ops, N, b, eps));
}

// matmulSegmentsBatchPartial(ctx, wtype, {x, ops}, weights, outputs, rows,
//   {N, batch, max_ksplit}[, softcap]) -> the chunk count K was split into
napi_value MatmulSegmentsBatchPartial(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const int wt = wtype_of(a, 1);
  const float* x = (const float*)fptr(a, 2, "x");
  const void* ops = fptr(a, 2, "ops");
  void* W[4] = {};
  void* Y[4] = {};
  uint32_t R[4] = {};
  const int n = array_at(a, 3, W, nullptr, 4, 0);
  const int ny = array_at(a, 4, Y, nullptr, 4, 0);
  const int nr = array_at(a, 5, nullptr, R, 4, 1);
  const uint32_t N = a.fu32(6, "N"), b = a.fu32(6, "batch"), mk = a.fu32(6, "max_ksplit");
  const float cap = a.present(7) ? a.f32(7) : 0.f;
  CHECKED(a);
  if (n != ny || n != nr) {
    a.fail("weights, outputs and rows differ in length");
    return nullptr;
  }
  uint32_t ks = 0;
  const int rc = g4_matmulSegmentsBatchPartial(c, wt, x, ops, W, (float* const*)Y, R, n, N, b, mk, cap, &ks);
  return size_result(env, rc, ks);
}

// pagedAttnPrologue(ctx, {qParts, kParts, vParts, qNorm, kNorm, ropeFreqs, qOut,
//   kPool, vPool, pageTable, seqLens, ropeCs}, nparts, pagedFusedParams, ropeRows)
napi_value PagedAttnPrologue(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* qp = (const float*)fptr(a, 1, "qParts");
  const float* kp = (const float*)fptr(a, 1, "kParts");
  const float* vp = (const float*)fptr(a, 1, "vParts");
  const uint16_t* qn = (const uint16_t*)fptr(a, 1, "qNorm");
  const uint16_t* kn = (const uint16_t*)fptr(a, 1, "kNorm");
  const uint16_t* rf = (const uint16_t*)fptr(a, 1, "ropeFreqs");
  float* qo = (float*)fptr(a, 1, "qOut");
  uint16_t* kc = (uint16_t*)fptr(a, 1, "kPool");
  uint16_t* vc = (uint16_t*)fptr(a, 1, "vPool");
  const int32_t* pt = (const int32_t*)fptr(a, 1, "pageTable");
  const uint32_t* sl = (const uint32_t*)fptr(a, 1, "seqLens");
  const float* cs = (const float*)fptr(a, 1, "ropeCs");
  const uint32_t np = a.u32(2);
  const g4_paged_attn_fused_params p = paged_fused_params(a, 3);
  const uint32_t rows = a.u32(4);
  CHECKED(a);
  return done(env, g4_pagedAttnPrologue(c, qp, kp, vp, np, qn, kn, rf, qo, kc, vc, pt, sl, p, cs, rows));
}

// pagedAttnDecode(ctx, {q, kPool, vPool, pageTable, seqLens, out, workspace, ops},
//   pagedParams, workspaceBytes): ops also receives the output as the o
//   projection's operand blocks (null: the attention alone)
napi_value PagedAttnDecode(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* q = (const float*)fptr(a, 1, "q");
  const uint16_t* kc = (const uint16_t*)fptr(a, 1, "kPool");
  const uint16_t* vc = (const uint16_t*)fptr(a, 1, "vPool");
  const int32_t* pt = (const int32_t*)fptr(a, 1, "pageTable");
  const uint32_t* sl = (const uint32_t*)fptr(a, 1, "seqLens");
  float* out = (float*)fptr(a, 1, "out");
  void* ws = fptr(a, 1, "workspace");
  void* ops = fptr(a, 1, "ops");
  const g4_paged_attn_params p = paged_params(a, 2);
  const uint64_t wsb = a.u64(3);
  CHECKED(a);
  return done(env, ops ? g4_pagedAttnDecodeOps(c, q, kc, vc, pt, sl, out, p, ws, wsb, ops)
                       : g4_pagedAttnDecode(c, q, kc, vc, pt, sl, out, p, ws, wsb));
}

// gateUpGeluBatch(ctx, {x, ops, wGate, wUp, out, downOps}, {M, N}, batch): the
// Q4_K gate/up pair and the GELU product over `batch` rows; with downOps the
// product is also written as the down projection's sub-block-scaled operand
// blocks (out may then be null)
napi_value GateUpGeluBatch(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* x = (const float*)fptr(a, 1, "x");
  const void* ops = fptr(a, 1, "ops");
  const void* wg = fptr(a, 1, "wGate");
  const void* wu = fptr(a, 1, "wUp");
  float* out = (float*)fptr(a, 1, "out");
  void* dops = fptr(a, 1, "downOps");
  const g4_matmul_params p{a.fu32(2, "M"), a.fu32(2, "N")};
  const uint32_t b = a.u32(3);
  CHECKED(a);
  return done(env, dops ? g4_gateUpGeluBatchOps(c, x, ops, wg, wu, out, dops, p, b)
                        : g4_gateUpGeluBatch(c, x, ops, wg, wu, out, p, b));
}

// matmulSubBatchPartial(ctx, downOps, weight, out, {M, K, batch, max_ksplit})
//   -> the chunk count (the Q6_K down projection over gateUpGeluBatch's blocks)
napi_value MatmulSubBatchPartial(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const void* ops = a.ptr(1);
  const void* w = a.ptr(2);
  float* out = F32P(a, 3);
  const uint32_t M = a.fu32(4, "M"), K = a.fu32(4, "K"), b = a.fu32(4, "batch"), mk = a.fu32(4, "max_ksplit");
  CHECKED(a);
  uint32_t ks = 0;
  const int rc = g4_matmulSubBatchPartial(c, ops, w, out, M, K, b, mk, &ks);
  return size_result(env, rc, ks);
}

// argmaxBatch(ctx, logits, result, size, batch) / topk256Batch(...): per row
napi_value ArgmaxBatch(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* lg = F32P(a, 1);
  uint32_t* r = U32P(a, 2);
  const uint32_t n = a.u32(3), b = a.u32(4);
  CHECKED(a);
  return done(env, g4_argmaxBatch(c, lg, r, n, b));
}
napi_value Topk256Batch(napi_env env, napi_callback_info info) {
  Args a(env, info);
  g4_ctx* c = CTX(a, 0);
  const float* lg = F32P(a, 1);
  float* r = F32P(a, 2);
  const uint32_t n = a.u32(3), b = a.u32(4);
  CHECKED(a);
  return done(env, g4_topk256Batch(c, lg, r, n, b));
}

struct Entry {
  const char* name;
  napi_callback fn;
};

const Entry kEntries[] = {
    {"version", Version},
    {"lastError", LastError},
    {"init", Init},
    {"destroy", Destroy},
    {"deviceInfo", DeviceInfo},
    {"alloc", Alloc},
    {"free", Free},
    {"memset", Memset},
    {"upload", Upload},
    {"download", Download},
    {"downloadAsync", DownloadAsync},
    {"eventRecord", EventRecord},
    {"eventQuery", EventQuery},
    {"eventWait", EventWait},
    {"eventDestroy", EventDestroy},
    {"sync", Sync},
    {"graphBegin", GraphBegin},
    {"graphEnd", GraphEnd},
    {"graphLaunch", GraphLaunch},
    {"graphDestroy", GraphDestroy},
    {"fill", Fill},
    {"matmulQuant", MatmulQuant},
    {"matmulQuantMR4", MatmulQuantMR4},
    {"kvCacheStore", KvCacheStore},
    {"attnScore", AttnScore},
    {"softmax", Softmax},
    {"attnOutput", AttnOutput},
    {"attnDecodeWorkspaceSize", AttnDecodeWorkspaceSize},
    {"attnDecode", AttnDecode},
    {"perHeadRmsNormNoWeight", PerHeadRmsNormNoWeight},
    {"fusedPerHeadNormRope", FusedPerHeadNormRope},
    {"rmsNorm", RmsNorm},
    {"fusedNormAdd", FusedNormAdd},
    {"geluMul", GeluMul},
    {"logitSoftcap", LogitSoftcap},
    {"embeddingLookup", EmbeddingLookup},
    {"argmax", Argmax},
    {"topk256", Topk256},
    {"advancePosition", AdvancePosition},
    {"pleStage1Fuse", PleStage1Fuse},
    {"pleGeluMul", PleGeluMul},
    {"pleSkipScaleAdd", PleSkipScaleAdd},
    {"ggufOpen", GgufOpen},
    {"ggufClose", GgufClose},
    {"ggufInfo", GgufInfo},
    {"ggufMetadata", GgufMetadata},
    {"ggufTensors", GgufTensors},
    {"ggufUpload", GgufUpload},
    {"ggufUploadF16", GgufUploadF16},
    {"dequantF16", DequantF16},
    {"digitsBytes", DigitsBytes},
    {"attnFusedWorkspaceSize", AttnFusedWorkspaceSize},
    {"ropeTable", RopeTable},
    {"matmulWarmRegion", MatmulWarmRegion},
    {"attnDecodeFused", AttnDecodeFused},
    {"normAddScaleMatmulSegments", NormAddScaleMatmulSegments},
    {"qkvAttnDecodeFused", QkvAttnDecodeFused},
    {"normAddGateUpGeluDigits", NormAddGateUpGeluDigits},
    {"matmulQuantDigits", MatmulQuantDigits},
    {"normAddMatmulArgmax", NormAddMatmulArgmax},
    {"pleGate", PleGate},
    {"matmulF16", MatmulF16},
    {"batchPrepScale", BatchPrepScale},
    {"argmaxAdvance", ArgmaxAdvance},
    {"batchOperandBytes", BatchOperandBytes},
    {"batchSubOperandBytes", BatchSubOperandBytes},
    {"pagedAttnWorkspaceSize", PagedAttnWorkspaceSize},
    {"copy", Copy},
    {"embeddingLookupBatch", EmbeddingLookupBatch},
    {"advanceSeqLens", AdvanceSeqLens},
    {"batchPrep", BatchPrep},
    {"matmulSegmentsBatchPartial", MatmulSegmentsBatchPartial},
    {"pagedAttnPrologue", PagedAttnPrologue},
    {"pagedAttnDecode", PagedAttnDecode},
    {"gateUpGeluBatch", GateUpGeluBatch},
    {"matmulSubBatchPartial", MatmulSubBatchPartial},
    {"argmaxBatch", ArgmaxBatch},
    {"topk256Batch", Topk256Batch},
};

}  // namespace

NAPI_MODULE_INIT() {
  for (const Entry& e : kEntries) {
    napi_value fn;
    napi_create_function(env, e.name, NAPI_AUTO_LENGTH, e.fn, nullptr, &fn);
    napi_set_named_property(env, exports, e.name, fn);
  }
  return exports;
}
