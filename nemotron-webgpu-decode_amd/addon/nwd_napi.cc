// nwd_napi.cc — Node.js N-API addon over the C ABI of libnwd_attn.
//
// This is the binding a JavaScript host (the reference's engine/runtime.js,
// or js/attention_layer.js here) uses in place of WebGPU buffers, bind
// groups and dispatches for the attention slice:
//   createEmptyStorage (kernels/gpu.js:91-96)      -> malloc / free
//   queue.writeBuffer / mapAsync readback
//     (engine/runtime.js:451-452, kernels/gpu.js:141-169) -> upload / download
//   dispatchWorkgroups of kv_append / sparse_attn
//     (engine/runtime.js:389-391)                  -> kvAppend / decode /
//                                                      appendDecode / prefill
// All library calls run on one stream the addon owns (a blocking stream, so
// the synchronous upload / download / zero, which use the null stream, are
// ordered with it). captureBegin / captureEnd record the calls in between
// into a HIP graph that graphLaunch replays with one call: the counterpart of
// the reference's cached op list, built once and submitted every token
// (engine/runtime.js:385-429).
// Device addresses cross into JavaScript as BigInt so the host can offset
// into a buffer (one position entry per step) the way the reference offsets
// uniform writes. Every failing call throws an Error naming the operation
// and carrying the library's message, as the reference names the failing
// bind group (engine/runtime.js:431-445).
#include <hip/hip_runtime_api.h>
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <map>
#include <string>

#include "nwd_attn.h"

namespace {

constexpr int kMaxDevices = 64;
hipStream_t g_streams[kMaxDevices] = {};

// Device buffers made by malloc (base address -> bytes). Every copy and
// write through the addon must stay inside one of them: a wrongly sized
// typed array is refused instead of writing past a buffer. (Node calls the
// addon from its one JavaScript thread.)
std::map<uintptr_t, size_t> g_allocs;

// True when [p, p + bytes) lies inside one allocation made by malloc.
bool in_allocation(const void* p, size_t bytes) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  auto it = g_allocs.upper_bound(a);
  if (it == g_allocs.begin()) return false;
  --it;
  const size_t off = a - it->first;
  return off <= it->second && bytes <= it->second - off;
}

std::string range_error(const char* op, const void* p, size_t bytes) {
  return std::string(op) + ": " + std::to_string(bytes) + " bytes at device address " +
         std::to_string(reinterpret_cast<uintptr_t>(p)) +
         " do not fit inside one buffer allocated by malloc";
}

// The addon's stream on the current device, created on first use.
hipStream_t stream() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  if (!g_streams[dev] && hipStreamCreate(&g_streams[dev]) != hipSuccess) g_streams[dev] = nullptr;
  return g_streams[dev];
}

napi_value throw_error(napi_env env, const std::string& msg) {
  napi_throw_error(env, nullptr, msg.c_str());
  return nullptr;
}

bool get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok) return false;
  for (size_t i = argc; i < want; ++i) napi_get_undefined(env, &argv[i]);
  return true;
}

bool get_ptr(napi_env env, napi_value v, void** out) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_null || t == napi_undefined) {
    *out = nullptr;
    return true;
  }
  uint64_t u = 0;
  bool lossless = false;
  if (t == napi_bigint) {
    if (napi_get_value_bigint_uint64(env, v, &u, &lossless) != napi_ok || !lossless) return false;
  } else if (t == napi_number) {
    double d = 0;
    napi_get_value_double(env, v, &d);
    if (d < 0) return false;
    u = (uint64_t)d;
  } else {
    return false;
  }
  *out = reinterpret_cast<void*>(static_cast<uintptr_t>(u));
  return true;
}

bool get_i32(napi_env env, napi_value v, int32_t* out, int32_t dflt) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_undefined) {
    *out = dflt;
    return true;
  }
  return napi_get_value_int32(env, v, out) == napi_ok;
}

napi_value make_ptr(napi_env env, const void* p) {
  napi_value r;
  napi_create_bigint_uint64(env, static_cast<uint64_t>(reinterpret_cast<uintptr_t>(p)), &r);
  return r;
}

napi_value make_i32(napi_env env, int32_t v) {
  napi_value r;
  napi_create_int32(env, v, &r);
  return r;
}

nwd_ctx* get_ctx(napi_env env, napi_value v) {
  void* p = nullptr;
  if (!get_ptr(env, v, &p) || !p) return nullptr;
  return static_cast<nwd_ctx*>(p);
}

napi_value check(napi_env env, nwd_ctx* ctx, const char* op, int rc) {
  if (rc == NWD_OK) return make_i32(env, 0);
  return throw_error(env, std::string(op) + ": " + nwd_last_error(ctx) + " (status " +
                              std::to_string(rc) + ")");
}

// Typed array -> (data, bytes)
bool get_bytes(napi_env env, napi_value v, void** data, size_t* bytes) {
  bool is_ta = false;
  napi_is_typedarray(env, v, &is_ta);
  if (!is_ta) return false;
  napi_typedarray_type type;
  size_t length = 0, offset = 0;
  napi_value ab;
  if (napi_get_typedarray_info(env, v, &type, &length, data, &ab, &offset) != napi_ok) return false;
  size_t elem = 1;
  switch (type) {
    case napi_int16_array: case napi_uint16_array: elem = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
    default: elem = 1;
  }
  *bytes = length * elem;
  return true;
}

int32_t field(napi_env env, napi_value obj, const char* name, int32_t dflt) {
  bool has = false;
  napi_has_named_property(env, obj, name, &has);
  if (!has) return dflt;
  napi_value v;
  napi_get_named_property(env, obj, name, &v);
  int32_t r = dflt;
  napi_get_value_int32(env, v, &r);
  return r;
}

// create({nHeads, nKvHeads, headDim, maxSeq, maxBatch, qF16, oF16, kvF16, scale}) -> ctx
napi_value Create(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return throw_error(env, "create: bad arguments");
  nwd_desc d;
  d.n_heads = field(env, argv[0], "nHeads", 0);
  d.n_kv_heads = field(env, argv[0], "nKvHeads", 0);
  d.head_dim = field(env, argv[0], "headDim", 128);
  d.max_seq = field(env, argv[0], "maxSeq", 0);
  d.max_batch = field(env, argv[0], "maxBatch", 1);
  d.q_dtype = field(env, argv[0], "qF16", 0) ? NWD_F16 : NWD_F32;
  d.o_dtype = field(env, argv[0], "oF16", 0) ? NWD_F16 : NWD_F32;
  d.kv_dtype = field(env, argv[0], "kvF16", 0) ? NWD_F16 : NWD_F32;
  d.scale = 0.f;
  bool has = false;
  napi_has_named_property(env, argv[0], "scale", &has);
  if (has) {
    napi_value v;
    double s = 0;
    napi_get_named_property(env, argv[0], "scale", &v);
    napi_get_value_double(env, v, &s);
    d.scale = (float)s;
  }
  nwd_ctx* ctx = nullptr;
  int rc = nwd_create(&d, &ctx);
  if (rc != NWD_OK)
    return throw_error(env, std::string("create: ") + nwd_last_error(nullptr));
  return make_ptr(env, ctx);
}

napi_value Destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  nwd_destroy(get_ctx(env, argv[0]));
  return make_i32(env, 0);
}

napi_value CacheBytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  nwd_ctx* ctx = get_ctx(env, argv[0]);
  if (!ctx) return throw_error(env, "cacheBytes: ctx is null");
  napi_value r;
  napi_create_bigint_uint64(env, nwd_cache_bytes(ctx), &r);
  return r;
}

napi_value Malloc(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  int64_t bytes = 0;
  bool lossless = true;
  napi_valuetype t;
  napi_typeof(env, argv[0], &t);
  if (t == napi_bigint) napi_get_value_bigint_int64(env, argv[0], &bytes, &lossless);
  else napi_get_value_int64(env, argv[0], &bytes);
  if (bytes <= 0 || !lossless) return throw_error(env, "malloc: size must be positive");
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, (size_t)bytes);
  if (e != hipSuccess) return throw_error(env, std::string("malloc: ") + hipGetErrorString(e));
  g_allocs[reinterpret_cast<uintptr_t>(p)] = (size_t)bytes;
  return make_ptr(env, p);
}

napi_value Free(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  void* p = nullptr;
  if (!get_ptr(env, argv[0], &p)) return throw_error(env, "free: bad pointer");
  if (p) {
    auto it = g_allocs.find(reinterpret_cast<uintptr_t>(p));
    if (it == g_allocs.end()) return throw_error(env, "free: not a buffer allocated by malloc");
    g_allocs.erase(it);
    (void)hipFree(p);
  }
  return make_i32(env, 0);
}

// upload(devPtr, typedArray): synchronous host -> device copy
napi_value Upload(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  void* dst = nullptr;
  void* src = nullptr;
  size_t bytes = 0;
  if (!get_ptr(env, argv[0], &dst) || !dst || !get_bytes(env, argv[1], &src, &bytes))
    return throw_error(env, "upload: expected (devicePtr, TypedArray)");
  if (!in_allocation(dst, bytes)) return throw_error(env, range_error("upload", dst, bytes));
  hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) return throw_error(env, std::string("upload: ") + hipGetErrorString(e));
  return make_i32(env, 0);
}

// setI32(devPtr, value): stream-ordered write of one int32 (the position
// before a step, as the reference's queue.writeBuffer of its uniforms,
// engine/runtime.js:451-452); does not wait for the device.
napi_value SetI32(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  void* dst = nullptr;
  int32_t v = 0;
  if (!get_ptr(env, argv[0], &dst) || !dst || napi_get_value_int32(env, argv[1], &v) != napi_ok)
    return throw_error(env, "setI32: expected (devicePtr, int32)");
  if (!in_allocation(dst, 4)) return throw_error(env, range_error("setI32", dst, 4));
  hipError_t e = hipMemsetD32Async(dst, v, 1, stream());
  if (e != hipSuccess) return throw_error(env, std::string("setI32: ") + hipGetErrorString(e));
  return make_i32(env, 0);
}

// download(typedArray, devPtr): synchronous device -> host copy
napi_value Download(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  void* dst = nullptr;
  void* src = nullptr;
  size_t bytes = 0;
  if (!get_bytes(env, argv[0], &dst, &bytes) || !get_ptr(env, argv[1], &src) || !src)
    return throw_error(env, "download: expected (TypedArray, devicePtr)");
  if (!in_allocation(src, bytes)) return throw_error(env, range_error("download", src, bytes));
  hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return throw_error(env, std::string("download: ") + hipGetErrorString(e));
  return make_i32(env, 0);
}

// zero(devPtr, bytes): the engine's reset() wipe (engine/runtime.js:615-633)
napi_value Zero(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  get_args(env, info, 2, argv);
  void* dst = nullptr;
  int64_t bytes = 0;
  bool lossless = true;
  napi_valuetype t;
  napi_typeof(env, argv[1], &t);
  if (t == napi_bigint) napi_get_value_bigint_int64(env, argv[1], &bytes, &lossless);
  else napi_get_value_int64(env, argv[1], &bytes);
  if (!get_ptr(env, argv[0], &dst) || !dst || bytes < 0 || !lossless)
    return throw_error(env, "zero: expected (devicePtr, bytes)");
  if (!in_allocation(dst, (size_t)bytes)) return throw_error(env, range_error("zero", dst, (size_t)bytes));
  hipError_t e = hipMemset(dst, 0, (size_t)bytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) return throw_error(env, std::string("zero: ") + hipGetErrorString(e));
  return make_i32(env, 0);
}

napi_value Sync(napi_env env, napi_callback_info info) {
  (void)info;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return throw_error(env, std::string("sync: ") + hipGetErrorString(e));
  return make_i32(env, 0);
}

// kvAppend(ctx, kNew, vNew, kCache, vCache, pos, batch, nTokens)
napi_value KvAppend(napi_env env, napi_callback_info info) {
  napi_value a[8];
  get_args(env, info, 8, a);
  nwd_ctx* ctx = get_ctx(env, a[0]);
  void *kn, *vn, *kc, *vc, *pos;
  int32_t batch, n;
  if (!ctx || !get_ptr(env, a[1], &kn) || !get_ptr(env, a[2], &vn) || !get_ptr(env, a[3], &kc) ||
      !get_ptr(env, a[4], &vc) || !get_ptr(env, a[5], &pos) || !get_i32(env, a[6], &batch, 1) ||
      !get_i32(env, a[7], &n, 1))
    return throw_error(env, "kvAppend: bad arguments");
  return check(env, ctx, "kvAppend",
               nwd_kv_append(ctx, kn, vn, kc, vc, static_cast<const int32_t*>(pos), batch, n, stream()));
}

// decode(ctx, q, kCache, vCache, pos, out, batch, maxLen)
napi_value Decode(napi_env env, napi_callback_info info) {
  napi_value a[8];
  get_args(env, info, 8, a);
  nwd_ctx* ctx = get_ctx(env, a[0]);
  void *q, *kc, *vc, *pos, *out;
  int32_t batch, max_len;
  if (!ctx || !get_ptr(env, a[1], &q) || !get_ptr(env, a[2], &kc) || !get_ptr(env, a[3], &vc) ||
      !get_ptr(env, a[4], &pos) || !get_ptr(env, a[5], &out) || !get_i32(env, a[6], &batch, 1) ||
      !get_i32(env, a[7], &max_len, 0))
    return throw_error(env, "decode: bad arguments");
  return check(env, ctx, "decode",
               nwd_decode_attn(ctx, q, kc, vc, static_cast<const int32_t*>(pos), out, batch,
                               max_len, stream()));
}

// appendDecode(ctx, q, kNew, vNew, kCache, vCache, pos, out, batch, maxLen)
napi_value AppendDecode(napi_env env, napi_callback_info info) {
  napi_value a[10];
  get_args(env, info, 10, a);
  nwd_ctx* ctx = get_ctx(env, a[0]);
  void *q, *kn, *vn, *kc, *vc, *pos, *out;
  int32_t batch, max_len;
  if (!ctx || !get_ptr(env, a[1], &q) || !get_ptr(env, a[2], &kn) || !get_ptr(env, a[3], &vn) ||
      !get_ptr(env, a[4], &kc) || !get_ptr(env, a[5], &vc) || !get_ptr(env, a[6], &pos) ||
      !get_ptr(env, a[7], &out) || !get_i32(env, a[8], &batch, 1) || !get_i32(env, a[9], &max_len, 0))
    return throw_error(env, "appendDecode: bad arguments");
  return check(env, ctx, "appendDecode",
               nwd_append_decode(ctx, q, kn, vn, kc, vc, static_cast<const int32_t*>(pos), out,
                                 batch, max_len, stream()));
}

// prefill(ctx, q, kCache, vCache, pos0, out, batch, nNew, maxLen)
napi_value Prefill(napi_env env, napi_callback_info info) {
  napi_value a[9];
  get_args(env, info, 9, a);
  nwd_ctx* ctx = get_ctx(env, a[0]);
  void *q, *kc, *vc, *pos, *out;
  int32_t batch, n_new, max_len;
  if (!ctx || !get_ptr(env, a[1], &q) || !get_ptr(env, a[2], &kc) || !get_ptr(env, a[3], &vc) ||
      !get_ptr(env, a[4], &pos) || !get_ptr(env, a[5], &out) || !get_i32(env, a[6], &batch, 1) ||
      !get_i32(env, a[7], &n_new, 1) || !get_i32(env, a[8], &max_len, 0))
    return throw_error(env, "prefill: bad arguments");
  return check(env, ctx, "prefill",
               nwd_prefill_attn(ctx, q, kc, vc, static_cast<const int32_t*>(pos), out, batch,
                                n_new, max_len, stream()));
}

// {quant, scales, zp: BigInt device addresses, n, nBlocks} -> nwd_q4_weight
bool get_q4(napi_env env, napi_value obj, nwd_q4_weight* w) {
  napi_valuetype t;
  if (napi_typeof(env, obj, &t) != napi_ok || t != napi_object) return false;
  const char* names[3] = {"quant", "scales", "zp"};
  void* p[3];
  for (int i = 0; i < 3; ++i) {
    napi_value v;
    bool has = false;
    if (napi_has_named_property(env, obj, names[i], &has) != napi_ok || !has) return false;
    napi_get_named_property(env, obj, names[i], &v);
    if (!get_ptr(env, v, &p[i])) return false;
  }
  w->quant = p[0];
  w->scales = static_cast<const float*>(p[1]);
  w->zp = p[2];
  w->n = field(env, obj, "n", 0);
  w->n_blocks = field(env, obj, "nBlocks", 0);
  return true;
}

// q4Gemv(ctx, a, w, y, batch, epilogue): matmul_nbits_sg.wgsl, epilogue
// 0 plain, 1 relu2, 2 accumulate into y (o_proj + residual add)
napi_value Q4Gemv(napi_env env, napi_callback_info info) {
  napi_value a[6];
  get_args(env, info, 6, a);
  nwd_ctx* ctx = get_ctx(env, a[0]);
  void *x, *y;
  nwd_q4_weight w;
  int32_t batch, epi;
  if (!ctx || !get_ptr(env, a[1], &x) || !get_q4(env, a[2], &w) || !get_ptr(env, a[3], &y) ||
      !get_i32(env, a[4], &batch, 1) || !get_i32(env, a[5], &epi, 0))
    return throw_error(env, "q4Gemv: bad arguments");
  return check(env, ctx, "q4Gemv",
               nwd_q4_gemv(ctx, static_cast<const float*>(x), &w, static_cast<float*>(y), batch,
                           epi, stream()));
}

// qkvAppend(ctx, x, wq, wk, wv, qOut, kCache, vCache, pos, batch): the q/k/v
// projections and kv_append in one launch
napi_value QkvAppend(napi_env env, napi_callback_info info) {
  napi_value a[10];
  get_args(env, info, 10, a);
  nwd_ctx* ctx = get_ctx(env, a[0]);
  void *x, *q, *kc, *vc, *pos;
  nwd_q4_weight wq, wk, wv;
  int32_t batch;
  if (!ctx || !get_ptr(env, a[1], &x) || !get_q4(env, a[2], &wq) || !get_q4(env, a[3], &wk) ||
      !get_q4(env, a[4], &wv) || !get_ptr(env, a[5], &q) || !get_ptr(env, a[6], &kc) ||
      !get_ptr(env, a[7], &vc) || !get_ptr(env, a[8], &pos) || !get_i32(env, a[9], &batch, 1))
    return throw_error(env, "qkvAppend: bad arguments");
  return check(env, ctx, "qkvAppend",
               nwd_qkv_append(ctx, static_cast<const float*>(x), &wq, &wk, &wv, q, kc, vc,
                              static_cast<const int32_t*>(pos), batch, stream()));
}

// argmax(ctx, x, n, out, batch): argmax_partial + argmax_merge
napi_value Argmax(napi_env env, napi_callback_info info) {
  napi_value a[5];
  get_args(env, info, 5, a);
  nwd_ctx* ctx = get_ctx(env, a[0]);
  void *x, *out;
  int32_t n, batch;
  if (!ctx || !get_ptr(env, a[1], &x) || !get_i32(env, a[2], &n, 0) || !get_ptr(env, a[3], &out) ||
      !get_i32(env, a[4], &batch, 1))
    return throw_error(env, "argmax: bad arguments");
  return check(env, ctx, "argmax",
               nwd_argmax(ctx, static_cast<const float*>(x), n, static_cast<uint32_t*>(out), batch,
                          stream()));
}

// lmHeadArgmax(ctx, h, w, logits (null for none), out, batch): lm-head, argmax0, argmax1
napi_value LmHeadArgmax(napi_env env, napi_callback_info info) {
  napi_value a[6];
  get_args(env, info, 6, a);
  nwd_ctx* ctx = get_ctx(env, a[0]);
  void *h, *logits, *out;
  nwd_q4_weight w;
  int32_t batch;
  if (!ctx || !get_ptr(env, a[1], &h) || !get_q4(env, a[2], &w) || !get_ptr(env, a[3], &logits) ||
      !get_ptr(env, a[4], &out) || !get_i32(env, a[5], &batch, 1))
    return throw_error(env, "lmHeadArgmax: bad arguments");
  return check(env, ctx, "lmHeadArgmax",
               nwd_lm_head_argmax(ctx, static_cast<const float*>(h), &w, static_cast<float*>(logits),
                                  static_cast<uint32_t*>(out), batch, stream()));
}

// deviceStatus(ctx) -> 0, or throws with the position error
napi_value DeviceStatus(napi_env env, napi_callback_info info) {
  napi_value a[1];
  get_args(env, info, 1, a);
  nwd_ctx* ctx = get_ctx(env, a[0]);
  if (!ctx) return throw_error(env, "deviceStatus: ctx is null");
  return check(env, ctx, "deviceStatus", nwd_device_status(ctx, stream()));
}

// captureBegin(): the library calls that follow are recorded, not run.
napi_value CaptureBegin(napi_env env, napi_callback_info) {
  hipStream_t s = stream();
  hipError_t e = s ? hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) : hipErrorInvalidValue;
  if (e != hipSuccess) return throw_error(env, std::string("captureBegin: ") + hipGetErrorString(e));
  return make_i32(env, 0);
}

// captureEnd() -> graph handle (BigInt) of the calls recorded since captureBegin
napi_value CaptureEnd(napi_env env, napi_callback_info) {
  hipGraph_t g = nullptr;
  hipGraphExec_t x = nullptr;
  hipError_t e = hipStreamEndCapture(stream(), &g);
  if (e == hipSuccess) e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  if (g) (void)hipGraphDestroy(g);
  if (e != hipSuccess) return throw_error(env, std::string("captureEnd: ") + hipGetErrorString(e));
  napi_value r;
  napi_create_bigint_uint64(env, static_cast<uint64_t>(reinterpret_cast<uintptr_t>(x)), &r);
  return r;
}

// graphLaunch(handle): replays a captured graph on the addon's stream
napi_value GraphLaunch(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  void* h = nullptr;
  if (!get_ptr(env, argv[0], &h) || !h) return throw_error(env, "graphLaunch: expected (graph)");
  hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(h), stream());
  if (e != hipSuccess) return throw_error(env, std::string("graphLaunch: ") + hipGetErrorString(e));
  return make_i32(env, 0);
}

// graphDestroy(handle)
napi_value GraphDestroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  void* h = nullptr;
  if (!get_ptr(env, argv[0], &h)) return throw_error(env, "graphDestroy: expected (graph)");
  if (h) (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(h));
  return make_i32(env, 0);
}

napi_value Init(napi_env env, napi_value exports) {
  const napi_property_descriptor props[] = {
      {"create", nullptr, Create, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"destroy", nullptr, Destroy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"cacheBytes", nullptr, CacheBytes, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"malloc", nullptr, Malloc, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"free", nullptr, Free, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"upload", nullptr, Upload, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"download", nullptr, Download, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"zero", nullptr, Zero, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"setI32", nullptr, SetI32, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"captureBegin", nullptr, CaptureBegin, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"captureEnd", nullptr, CaptureEnd, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"graphLaunch", nullptr, GraphLaunch, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"graphDestroy", nullptr, GraphDestroy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sync", nullptr, Sync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"kvAppend", nullptr, KvAppend, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decode", nullptr, Decode, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"appendDecode", nullptr, AppendDecode, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"prefill", nullptr, Prefill, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"deviceStatus", nullptr, DeviceStatus, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"q4Gemv", nullptr, Q4Gemv, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"qkvAppend", nullptr, QkvAppend, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"argmax", nullptr, Argmax, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"lmHeadArgmax", nullptr, LmHeadArgmax, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
  };
  napi_define_properties(env, exports, sizeof(props) / sizeof(props[0]), props);
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
