/* Thin N-API addon over the C ABI (include/bitgpu_attn.h) for the TypeScript engine host.
 *
 * Handles: a cache is a napi External wrapping bg_kv_cache*; device pointers and streams are
 * BigInt (uint64) values; host buffers are ArrayBuffer / TypedArray views. Every function
 * returns undefined or a value and throws a JS Error('bitgpu: ...') on a BG_E_* status, with
 * err.code = the status and err.name = 'GpuOutOfMemoryError' for BG_E_OOM (src/errors.ts:14-19).
 * No copies on the hot path: attention/prologue/write take device pointers only.
 * The small device helpers (devAlloc/devFree/h2d/d2h/sync) exist so a JS host without its own
 * HIP allocator can own buffers; the engine would use its own.
 */
#define NAPI_VERSION 6
#include <node_api.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/bitgpu_attn.h"

/* HIP runtime entry points used by the helpers (declared here to avoid the HIP headers). */
extern int hipMalloc(void** ptr, size_t size);
extern int hipFree(void* ptr);
extern int hipMemcpy(void* dst, const void* src, size_t size, int kind);
extern int hipDeviceSynchronize(void);
enum { HIP_H2D = 1, HIP_D2H = 2 };

#define CHECK_NAPI(call)                                     \
  do {                                                       \
    if ((call) != napi_ok) {                                 \
      napi_throw_error(env, NULL, "bitgpu: N-API failure"); \
      return NULL;                                           \
    }                                                        \
  } while (0)

static napi_value throw_status(napi_env env, int32_t rc) {
  napi_value msg, err, code, name;
  napi_create_string_utf8(env, bg_last_error_message(), NAPI_AUTO_LENGTH, &msg);
  napi_create_error(env, NULL, msg, &err);
  napi_create_int32(env, rc, &code);
  napi_set_named_property(env, err, "code", code);
  napi_create_string_utf8(env, rc == BG_E_OOM ? "GpuOutOfMemoryError" : "Error", NAPI_AUTO_LENGTH, &name);
  napi_set_named_property(env, err, "name", name);
  napi_throw(env, err);
  return NULL;
}

#define RC(call)                                  \
  do {                                            \
    int32_t rc_ = (call);                         \
    if (rc_ != BG_OK) return throw_status(env, rc_); \
  } while (0)

static int32_t arg_i32(napi_env env, napi_value v) {
  int32_t x = 0;
  napi_get_value_int32(env, v, &x);
  return x;
}
static double arg_f64(napi_env env, napi_value v) {
  double x = 0;
  napi_get_value_double(env, v, &x);
  return x;
}
/* BigInt (or null/undefined -> NULL) to a pointer */
static void* arg_ptr(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_bigint) return NULL;
  uint64_t x = 0;
  bool lossless = false;
  napi_get_value_bigint_uint64(env, v, &x, &lossless);
  return (void*)(uintptr_t)x;
}
static bg_kv_cache* arg_cache(napi_env env, napi_value v) {
  void* p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok) return NULL;
  return (bg_kv_cache*)p;
}
static void* arg_host(napi_env env, napi_value v, size_t* len) {
  bool is_ab = false, is_ta = false;
  void* data = NULL;
  *len = 0;
  napi_is_arraybuffer(env, v, &is_ab);
  if (is_ab) {
    napi_get_arraybuffer_info(env, v, &data, len);
    return data;
  }
  napi_is_typedarray(env, v, &is_ta);
  if (is_ta) {
    napi_typedarray_type type;
    size_t n, off;
    napi_value ab;
    napi_get_typedarray_info(env, v, &type, &n, &data, &ab, &off);
    size_t es = (type == napi_float64_array || type == napi_bigint64_array || type == napi_biguint64_array) ? 8
                : (type == napi_float32_array || type == napi_int32_array || type == napi_uint32_array) ? 4
                : (type == napi_int16_array || type == napi_uint16_array) ? 2 : 1;
    *len = n * es;
    return data;
  }
  return NULL;
}
static napi_value i32(napi_env env, int32_t x) {
  napi_value r;
  napi_create_int32(env, x, &r);
  return r;
}
static napi_value ptr_value(napi_env env, void* p) {
  napi_value r;
  napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &r);
  return r;
}

#define ARGS(n)                 \
  size_t argc = n;              \
  napi_value a[n];              \
  CHECK_NAPI(napi_get_cb_info(env, info, &argc, a, NULL, NULL));

static napi_value js_version(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value r;
  napi_create_string_utf8(env, bg_version(), NAPI_AUTO_LENGTH, &r);
  return r;
}

/* ropeTables(theta, rotDim, positions, yarnFactor, yarnOrig, cosF32, sinF32) */
static napi_value js_rope_tables(napi_env env, napi_callback_info info) {
  ARGS(7);
  size_t lc, ls;
  float* c = (float*)arg_host(env, a[5], &lc);
  float* s = (float*)arg_host(env, a[6], &ls);
  const int32_t rot = arg_i32(env, a[1]), pos = arg_i32(env, a[2]);
  if (!c || !s || lc < (size_t)pos * (rot / 2) * 4 || ls < lc) {
    napi_throw_range_error(env, NULL, "bitgpu: rope table arrays are too small");
    return NULL;
  }
  RC(bg_rope_tables(arg_f64(env, a[0]), rot, pos, arg_f64(env, a[3]), arg_i32(env, a[4]), c, s));
  return NULL;
}

/* evictPlan(fill, need, sinks, maxSeq) -> [newFill, batch, keep] */
static napi_value js_evict_plan(napi_env env, napi_callback_info info) {
  ARGS(4);
  int32_t nf, b, k;
  RC(bg_evict_plan(arg_i32(env, a[0]), arg_i32(env, a[1]), arg_i32(env, a[2]), arg_i32(env, a[3]), &nf, &b, &k));
  napi_value arr;
  napi_create_array_with_length(env, 3, &arr);
  napi_set_element(env, arr, 0, i32(env, nf));
  napi_set_element(env, arr, 1, i32(env, b));
  napi_set_element(env, arr, 2, i32(env, k));
  return arr;
}

static napi_value js_ring_map(napi_env env, napi_callback_info info) {
  ARGS(4);
  int32_t p;
  RC(bg_ring_map(arg_i32(env, a[0]), arg_i32(env, a[1]), arg_i32(env, a[2]), arg_i32(env, a[3]), &p));
  return i32(env, p);
}

static void cache_finalize(napi_env env, void* data, void* hint) {
  (void)env;
  (void)data;
  (void)hint; /* explicit kvDestroy owns the lifetime; GC never frees device memory behind JS */
}

/* kvCreate(nLayers, kvHeads, headDim, dtype, capacity, maxSeq, roll, sinks, ropeMode) -> External */
static napi_value js_kv_create(napi_env env, napi_callback_info info) {
  ARGS(9);
  bg_kv_cache* c = NULL;
  RC(bg_kv_create(arg_i32(env, a[0]), arg_i32(env, a[1]), arg_i32(env, a[2]), arg_i32(env, a[3]), arg_i32(env, a[4]),
                  arg_i32(env, a[5]), arg_i32(env, a[6]), arg_i32(env, a[7]), arg_i32(env, a[8]), &c));
  napi_value ext;
  CHECK_NAPI(napi_create_external(env, c, cache_finalize, NULL, &ext));
  return ext;
}

static napi_value js_kv_destroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  RC(bg_kv_destroy(arg_cache(env, a[0])));
  return NULL;
}

static napi_value js_kv_capacity(napi_env env, napi_callback_info info) {
  ARGS(1);
  int32_t cap;
  RC(bg_kv_capacity(arg_cache(env, a[0]), &cap));
  return i32(env, cap);
}

static napi_value js_kv_grow(napi_env env, napi_callback_info info) {
  ARGS(3);
  RC(bg_kv_grow(arg_cache(env, a[0]), arg_i32(env, a[1]), arg_ptr(env, a[2])));
  return NULL;
}

static napi_value js_kv_set_rope(napi_env env, napi_callback_info info) {
  ARGS(5);
  RC(bg_kv_set_rope(arg_cache(env, a[0]), arg_ptr(env, a[1]), arg_ptr(env, a[2]), arg_i32(env, a[3]), arg_i32(env, a[4])));
  return NULL;
}

/* kvWrite(cache, layer, which, srcDev, rows, dstRow0, stream) -- appendKV */
static napi_value js_kv_write(napi_env env, napi_callback_info info) {
  ARGS(7);
  RC(bg_kv_write(arg_cache(env, a[0]), arg_i32(env, a[1]), arg_i32(env, a[2]), arg_ptr(env, a[3]), arg_i32(env, a[4]),
                 arg_i32(env, a[5]), arg_ptr(env, a[6])));
  return NULL;
}

/* qkvPrologue(cache, layer, q, qStride, k, v, S, H, qGamma, kGamma, eps, cos, sin, ropePositions,
 *             rotDim, pos0, slot0, qOut, stream) */
static napi_value js_qkv_prologue(napi_env env, napi_callback_info info) {
  ARGS(19);
  RC(bg_qkv_prologue(arg_cache(env, a[0]), arg_i32(env, a[1]), arg_ptr(env, a[2]), arg_i32(env, a[3]),
                     arg_ptr(env, a[4]), arg_ptr(env, a[5]), arg_i32(env, a[6]), arg_i32(env, a[7]), arg_ptr(env, a[8]),
                     arg_ptr(env, a[9]), (float)arg_f64(env, a[10]), arg_ptr(env, a[11]), arg_ptr(env, a[12]),
                     arg_i32(env, a[13]), arg_i32(env, a[14]), arg_i32(env, a[15]), arg_i32(env, a[16]),
                     arg_ptr(env, a[17]), arg_ptr(env, a[18])));
  return NULL;
}

/* attention(cache, layer, q, S, H, posBase, scale, gate, gateStride, out, stream) -- ATT */
static napi_value js_attention(napi_env env, napi_callback_info info) {
  ARGS(11);
  RC(bg_attention(arg_cache(env, a[0]), arg_i32(env, a[1]), arg_ptr(env, a[2]), arg_i32(env, a[3]), arg_i32(env, a[4]),
                  arg_i32(env, a[5]), (float)arg_f64(env, a[6]), arg_ptr(env, a[7]), arg_i32(env, a[8]),
                  arg_ptr(env, a[9]), arg_ptr(env, a[10])));
  return NULL;
}

/* gemvSplit(x, K, sign, scales, N0, N1, N2, out0, out1, out2, stream);
   gemvResid(x, K, sign, scales, N, resid, y, stream);
   qkvProjPrologue(cache, li, x, K, sign, scales, H, qGamma, kGamma, eps, cos, sin, ropePositions,
                   rotDim, pos, slot, qOut, stream) -- device buffers as BigInt pointers */
static napi_value js_gemv_split(napi_env env, napi_callback_info info) {
  ARGS(11);
  RC(bg_gemv_split(arg_ptr(env, a[0]), arg_i32(env, a[1]), arg_ptr(env, a[2]), arg_ptr(env, a[3]), arg_i32(env, a[4]),
                   arg_i32(env, a[5]), arg_i32(env, a[6]), arg_ptr(env, a[7]), arg_ptr(env, a[8]), arg_ptr(env, a[9]),
                   arg_ptr(env, a[10])));
  return NULL;
}
static napi_value js_gemv_resid(napi_env env, napi_callback_info info) {
  ARGS(8);
  RC(bg_gemv_resid(arg_ptr(env, a[0]), arg_i32(env, a[1]), arg_ptr(env, a[2]), arg_ptr(env, a[3]), arg_i32(env, a[4]),
                   arg_ptr(env, a[5]), arg_ptr(env, a[6]), arg_ptr(env, a[7])));
  return NULL;
}
static napi_value js_qkv_proj_prologue(napi_env env, napi_callback_info info) {
  ARGS(18);
  RC(bg_qkv_proj_prologue(arg_cache(env, a[0]), arg_i32(env, a[1]), arg_ptr(env, a[2]), arg_i32(env, a[3]),
                          arg_ptr(env, a[4]), arg_ptr(env, a[5]), arg_i32(env, a[6]), arg_ptr(env, a[7]),
                          arg_ptr(env, a[8]), (float)arg_f64(env, a[9]), arg_ptr(env, a[10]), arg_ptr(env, a[11]),
                          arg_i32(env, a[12]), arg_i32(env, a[13]), arg_i32(env, a[14]), arg_i32(env, a[15]),
                          arg_ptr(env, a[16]), arg_ptr(env, a[17])));
  return NULL;
}

static napi_value js_kv_evict(napi_env env, napi_callback_info info) {
  ARGS(3);
  int32_t nf;
  RC(bg_kv_evict(arg_cache(env, a[0]), arg_i32(env, a[1]), arg_i32(env, a[2]), &nf));
  return i32(env, nf);
}

static napi_value js_kv_evict_for(napi_env env, napi_callback_info info) {
  ARGS(3);
  int32_t nf;
  RC(bg_kv_evict_for(arg_cache(env, a[0]), arg_i32(env, a[1]), arg_i32(env, a[2]), &nf));
  return i32(env, nf);
}

/* kvRingState(cache) -> [head, evicted]; kvRingReset(cache, evicted) */
static napi_value js_kv_ring_state(napi_env env, napi_callback_info info) {
  ARGS(1);
  int32_t head;
  int64_t ev;
  RC(bg_kv_ring_state(arg_cache(env, a[0]), &head, &ev));
  napi_value r, x;
  napi_create_array_with_length(env, 2, &r);
  napi_set_element(env, r, 0, i32(env, head));
  napi_create_double(env, (double)ev, &x);
  napi_set_element(env, r, 1, x);
  return r;
}
static napi_value js_kv_ring_reset(napi_env env, napi_callback_info info) {
  ARGS(2);
  RC(bg_kv_ring_reset(arg_cache(env, a[0]), (int64_t)arg_f64(env, a[1])));
  return NULL;
}

/* kvSetQ8Block(cache, block): q8 scale block, 32 or head_dim */
static napi_value js_kv_set_q8_block(napi_env env, napi_callback_info info) {
  ARGS(2);
  RC(bg_kv_set_q8_block(arg_cache(env, a[0]), arg_i32(env, a[1])));
  return NULL;
}

static napi_value js_kv_region_bytes(napi_env env, napi_callback_info info) {
  ARGS(3);
  size_t b;
  RC(bg_kv_region_bytes(arg_cache(env, a[0]), arg_i32(env, a[1]), arg_i32(env, a[2]), &b));
  napi_value r;
  napi_create_double(env, (double)b, &r);
  return r;
}

/* kvExportRows(cache, layer, region, base, count, hostView, stream) / kvImportRows(...) */
static napi_value transfer(napi_env env, napi_callback_info info, int import_) {
  ARGS(7);
  bg_kv_cache* c = arg_cache(env, a[0]);
  size_t need = 0, have = 0;
  RC(bg_kv_region_bytes(c, arg_i32(env, a[2]), arg_i32(env, a[4]), &need));
  void* host = arg_host(env, a[5], &have);
  if (!host || have < need) {
    napi_throw_range_error(env, NULL, "bitgpu: host buffer is smaller than the region");
    return NULL;
  }
  if (import_)
    RC(bg_kv_import_rows(c, arg_i32(env, a[1]), arg_i32(env, a[2]), arg_i32(env, a[3]), arg_i32(env, a[4]), host,
                         arg_ptr(env, a[6])));
  else
    RC(bg_kv_export_rows(c, arg_i32(env, a[1]), arg_i32(env, a[2]), arg_i32(env, a[3]), arg_i32(env, a[4]), host,
                         arg_ptr(env, a[6])));
  return NULL;
}
static napi_value js_kv_export(napi_env env, napi_callback_info info) { return transfer(env, info, 0); }
static napi_value js_kv_import(napi_env env, napi_callback_info info) { return transfer(env, info, 1); }

/* ---- device helpers ---- */
static napi_value js_dev_alloc(napi_env env, napi_callback_info info) {
  ARGS(1);
  void* p = NULL;
  if (hipMalloc(&p, (size_t)arg_f64(env, a[0])) != 0) return throw_status(env, BG_E_OOM);
  return ptr_value(env, p);
}
static napi_value js_dev_free(napi_env env, napi_callback_info info) {
  ARGS(1);
  hipFree(arg_ptr(env, a[0]));
  return NULL;
}
static napi_value js_h2d(napi_env env, napi_callback_info info) {
  ARGS(2);
  size_t n;
  void* h = arg_host(env, a[1], &n);
  if (hipMemcpy(arg_ptr(env, a[0]), h, n, HIP_H2D) != 0) return throw_status(env, BG_E_DEVICE);
  return NULL;
}
static napi_value js_d2h(napi_env env, napi_callback_info info) {
  ARGS(2);
  size_t n;
  void* h = arg_host(env, a[0], &n);
  if (hipMemcpy(h, arg_ptr(env, a[1]), n, HIP_D2H) != 0) return throw_status(env, BG_E_DEVICE);
  return NULL;
}
static napi_value js_sync(napi_env env, napi_callback_info info) {
  (void)info;
  if (hipDeviceSynchronize() != 0) return throw_status(env, BG_E_DEVICE);
  return NULL;
}

/* streamCreate() -> bigint; streamDestroy(stream); eventCreate() -> bigint;
   eventRecord(event, stream); eventElapsedUs(start, end) -> number; eventDestroy(event) */
static napi_value js_stream_create(napi_env env, napi_callback_info info) {
  (void)info;
  void* st = NULL;
  RC(bg_stream_create(&st));
  return ptr_value(env, st);
}
static napi_value js_stream_destroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  RC(bg_stream_destroy(arg_ptr(env, a[0])));
  return NULL;
}
static napi_value js_event_create(napi_env env, napi_callback_info info) {
  (void)info;
  void* ev = NULL;
  RC(bg_event_create(&ev));
  return ptr_value(env, ev);
}
static napi_value js_event_record(napi_env env, napi_callback_info info) {
  ARGS(2);
  RC(bg_event_record(arg_ptr(env, a[0]), arg_ptr(env, a[1])));
  return NULL;
}
static napi_value js_event_elapsed_us(napi_env env, napi_callback_info info) {
  ARGS(2);
  float us = 0.0f;
  RC(bg_event_elapsed_us(arg_ptr(env, a[0]), arg_ptr(env, a[1]), &us));
  napi_value r;
  napi_create_double(env, (double)us, &r);
  return r;
}
static napi_value js_event_destroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  RC(bg_event_destroy(arg_ptr(env, a[0])));
  return NULL;
}

static napi_value init(napi_env env, napi_value exports) {
  napi_property_descriptor p[] = {
      {"version", 0, js_version, 0, 0, 0, napi_default, 0},
      {"ropeTables", 0, js_rope_tables, 0, 0, 0, napi_default, 0},
      {"evictPlan", 0, js_evict_plan, 0, 0, 0, napi_default, 0},
      {"ringMap", 0, js_ring_map, 0, 0, 0, napi_default, 0},
      {"kvCreate", 0, js_kv_create, 0, 0, 0, napi_default, 0},
      {"kvDestroy", 0, js_kv_destroy, 0, 0, 0, napi_default, 0},
      {"kvCapacity", 0, js_kv_capacity, 0, 0, 0, napi_default, 0},
      {"kvGrow", 0, js_kv_grow, 0, 0, 0, napi_default, 0},
      {"kvSetRope", 0, js_kv_set_rope, 0, 0, 0, napi_default, 0},
      {"kvWrite", 0, js_kv_write, 0, 0, 0, napi_default, 0},
      {"qkvPrologue", 0, js_qkv_prologue, 0, 0, 0, napi_default, 0},
      {"attention", 0, js_attention, 0, 0, 0, napi_default, 0},
      {"gemvSplit", 0, js_gemv_split, 0, 0, 0, napi_default, 0},
      {"gemvResid", 0, js_gemv_resid, 0, 0, 0, napi_default, 0},
      {"qkvProjPrologue", 0, js_qkv_proj_prologue, 0, 0, 0, napi_default, 0},
      {"kvEvict", 0, js_kv_evict, 0, 0, 0, napi_default, 0},
      {"kvEvictFor", 0, js_kv_evict_for, 0, 0, 0, napi_default, 0},
      {"kvRingState", 0, js_kv_ring_state, 0, 0, 0, napi_default, 0},
      {"kvRingReset", 0, js_kv_ring_reset, 0, 0, 0, napi_default, 0},
      {"kvSetQ8Block", 0, js_kv_set_q8_block, 0, 0, 0, napi_default, 0},
      {"kvRegionBytes", 0, js_kv_region_bytes, 0, 0, 0, napi_default, 0},
      {"kvExportRows", 0, js_kv_export, 0, 0, 0, napi_default, 0},
      {"kvImportRows", 0, js_kv_import, 0, 0, 0, napi_default, 0},
      {"devAlloc", 0, js_dev_alloc, 0, 0, 0, napi_default, 0},
      {"devFree", 0, js_dev_free, 0, 0, 0, napi_default, 0},
      {"h2d", 0, js_h2d, 0, 0, 0, napi_default, 0},
      {"d2h", 0, js_d2h, 0, 0, 0, napi_default, 0},
      {"sync", 0, js_sync, 0, 0, 0, napi_default, 0},
      {"streamCreate", 0, js_stream_create, 0, 0, 0, napi_default, 0},
      {"streamDestroy", 0, js_stream_destroy, 0, 0, 0, napi_default, 0},
      {"eventCreate", 0, js_event_create, 0, 0, 0, napi_default, 0},
      {"eventRecord", 0, js_event_record, 0, 0, 0, napi_default, 0},
      {"eventElapsedUs", 0, js_event_elapsed_us, 0, 0, 0, napi_default, 0},
      {"eventDestroy", 0, js_event_destroy, 0, 0, 0, napi_default, 0},
  };
  napi_define_properties(env, exports, sizeof(p) / sizeof(p[0]), p);
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
