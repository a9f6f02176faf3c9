// C ABI of the attention hot path (include/bitgpu_attn.h): the KV-cache object, argument
// validation, workspace management and kernel dispatch. Host code only; the kernels live in
// kv_pack.hip, norm_rope.hip, decode.hip, prefill.hip and attn_f32.hip.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "../../include/bitgpu_attn.h"
#include "bg_kernels.h"

using bg::LayerView;

struct bg_kv_cache {
  int n_layers = 0, kv_heads = 0, D = 0, dtype = 0;
  int capacity = 0;   // logical capacity (reference kvCapacity)
  int cap = 0;        // physical slots (capacity rounded up to 32)
  int max_seq = 0;
  int roll = 0, sinks = 0, rope_abs = 0;
  int head = 0;       // ring origin
  int64_t evicted = 0;
  std::vector<void*> k, v;
  std::vector<float*> ks, vs;
  const float* cos_tab = nullptr;
  const float* sin_tab = nullptr;
  int rope_positions = 0;
  float* ws = nullptr;
  size_t ws_floats = 0;
  unsigned* ws_count = nullptr;
  size_t ws_counters = 0;
  // f16 copy of one q8 layer's attended slots for long prefills (K then V, cap_copy slots each)
  void* pf16 = nullptr;
  float* pf_ml = nullptr;  // split-K prefill (m, l), bg::prefill_split_ml_bytes() once allocated
  // workspaces replaced by a larger one, kept until destroy: launches captured in a graph before
  // the growth still use them (and find their slots holding the empty marker)
  std::vector<std::pair<float*, size_t>> retired_ws;
  std::vector<unsigned*> retired_count;
  int pf16_cap = 0;
  int num_cus = 256;
  int device = 0;
  int q8_row = 0;     // q8: one scale per row (bg_kv_set_q8_block with head_dim)
  // decode merge error word: pinned, coherent host memory the kernel writes when a merger's
  // bounded wait gives up (err_dev is its device address)
  unsigned* err_host = nullptr;
  unsigned* err_dev = nullptr;
  // snapshot staging buffer (grown on demand, kept until destroy)
  void* stage = nullptr;
  size_t stage_bytes = 0;
  // fused decode projection: the gather buffer of raw rows [kProjMaxHeads][D], the empty marker
  // in every value between launches
  float* proj_raw = nullptr;
};

namespace {

thread_local std::string g_err;

int32_t fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = std::string("bitgpu: ") + buf;
  return code;
}

int32_t hip_fail(hipError_t e, const char* what) {
  if (e == hipErrorOutOfMemory) return fail(BG_E_OOM, "GPU out of memory during %s: %s", what, hipGetErrorString(e));
  return fail(BG_E_DEVICE, "HIP error during %s: %s", what, hipGetErrorString(e));
}

int round32(int x) { return (x + 31) & ~31; }

size_t elem_bytes(int dtype) { return (size_t)bg::kv_elem_bytes(dtype); }

// Test hook: BG_FAULT_GROW_ALLOC=n makes the n-th device allocation inside bg_kv_grow fail,
// so the rollback path can be exercised from the host without exhausting memory.
hipError_t grow_malloc(void** p, size_t bytes, int* counter) {
  const char* f = getenv("BG_FAULT_GROW_ALLOC");
  (*counter)++;
  if (f && atoi(f) == *counter) {
    *p = nullptr;
    return hipErrorOutOfMemory;
  }
  return hipMalloc(p, bytes);
}

LayerView view(const bg_kv_cache* c, int layer) {
  LayerView L;
  L.k = c->k[layer];
  L.v = c->v[layer];
  L.ks = c->dtype == BG_KV_Q8 ? c->ks[layer] : nullptr;
  L.vs = c->dtype == BG_KV_Q8 ? c->vs[layer] : nullptr;
  L.cap = c->cap;
  L.kv_heads = c->kv_heads;
  L.D = c->D;
  L.dtype = c->dtype;
  L.ring.roll = c->roll;
  L.ring.sinks = c->sinks;
  L.ring.W = c->max_seq - c->sinks;
  L.ring.head = c->head;
  L.max_seq = c->max_seq;
  L.cos_tab = c->cos_tab;
  L.sin_tab = c->sin_tab;
  L.rope_positions = c->rope_positions;
  L.rope_abs = c->rope_abs;
  L.evicted = c->evicted;
  L.q8_row = c->q8_row;
  return L;
}

void free_layers(std::vector<void*>& k, std::vector<void*>& v, std::vector<float*>& ks, std::vector<float*>& vs) {
  for (auto p : k) if (p) (void)hipFree(p);
  for (auto p : v) if (p) (void)hipFree(p);
  for (auto p : ks) if (p) (void)hipFree(p);
  for (auto p : vs) if (p) (void)hipFree(p);
  k.clear(); v.clear(); ks.clear(); vs.clear();
}

// heads (query + key + value) the fused decode projection's arrival counters cover
constexpr int kProjMaxHeads = 1024;

// slots the caller may address: the window in sink mode, the grown capacity otherwise
int addressable(const bg_kv_cache* c) { return c->roll ? c->max_seq : c->capacity; }

// ---- the allocation-free entry point's scratch ------------------------------------------------
// bg_attention_noalloc keeps the decode kernel's split partials here instead of in a workspace
// the library allocates: one array per GPU, held until the process ends. Host code never passes
// the array's name to a kernel (on the host it is a stand-in, not a device address): the device
// address comes from hipGetSymbolAddress, once per device, and only that pointer is used.
// Between launches every slot holds the decode kernel's empty marker; the set-up fills it once.
// Layout: the first kScratchBytes hold split partials (decode, split-K prefill) and the empty
// marker between launches; the kScratchMlBytes after them hold a split-K prefill's (m, l) values.
constexpr size_t kScratchBytes = (size_t)8 << 20;     // 8 MiB per GPU
constexpr size_t kScratchMlBytes = (size_t)256 << 10;  // 256 KiB
__device__ __align__(256) unsigned char scratch[kScratchBytes + kScratchMlBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

__global__ void fill_u32_kernel(uint32_t* p, uint32_t value, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = value;
}

// live caches, for bg_stream_sync's check of their merge error words
std::mutex g_caches_mu;
std::set<bg_kv_cache*> g_caches;

// test hooks of the decode merge (bg_debug_merge_hooks): a poll bound and a split that stores
// no partial; 0 and -1 in normal use
std::atomic<int> g_merge_spin{0};
std::atomic<int> g_withhold_split{-1};

// Workgroup placement per device: > 0 the XCD count when workgroups go to XCDs round robin
// (the decode kernel's L2 partial exchange is on), -1 probed and off (no round robin, or a
// merger later found itself on another XCD than its splits), 0 not probed yet.
std::mutex g_xcd_mu;
int g_xcd_state[kMaxDevices] = {};

int xcd_state(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return -1;
  std::lock_guard<std::mutex> lock(g_xcd_mu);
  if (g_xcd_state[dev] == 0) {
    int nx = 0;
    if (bg::probe_xcd_round_robin(&nx) != hipSuccess) {
      (void)hipGetLastError();
      nx = 0;
    }
    g_xcd_state[dev] = nx > 0 ? nx : -1;
  }
  return g_xcd_state[dev];
}

void xcd_disable(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_xcd_mu);
  g_xcd_state[dev] = -1;
}

bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return cs != hipStreamCaptureStatusNone;
}

// An earlier decode launch on this cache gave up waiting for a split partial (its output was
// stored as NaN): wait for every launch to finish, refill the split workspace with the empty
// marker (a late partial may have landed after its merger gave up) and report it once.
int32_t take_merge_error(bg_kv_cache* c, hipStream_t st) {
  const unsigned code = c->err_host ? __atomic_load_n(c->err_host, __ATOMIC_ACQUIRE) : 0u;
  if (code == 0) return BG_OK;
  // 2: a merger ran on another XCD than the splits whose partials it waited for (the L2
  // exchange relies on round-robin placement): use written-through partials from now on
  if (code == 2) xcd_disable(c->device);
  if (capturing(st))
    return fail(BG_E_DEVICE, "an earlier decode split merge gave up waiting for a split; call bg_stream_sync "
                             "outside graph capture to reset the workspace");
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess && c->ws)
    e = hipMemsetD32((hipDeviceptr_t)c->ws, (int)bg::decode_workspace_empty(), c->ws_floats);
  for (const auto& r : c->retired_ws)
    if (e == hipSuccess) e = hipMemsetD32((hipDeviceptr_t)r.first, (int)bg::decode_workspace_empty(), r.second);
  if (e == hipSuccess && c->proj_raw)
    e = hipMemsetD32((hipDeviceptr_t)c->proj_raw, (int)bg::kWorkspaceEmpty, bg::qkv_proj_raw_floats(kProjMaxHeads, c->D));
  int dev = 0;
  if (e == hipSuccess) e = hipGetDevice(&dev);
  if (e == hipSuccess && dev >= 0 && dev < kMaxDevices) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev])
      e = hipMemsetD32((hipDeviceptr_t)g_scratch_ptr[dev], (int)bg::decode_workspace_empty(), kScratchBytes / 4);
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(e, "workspace reset after a merge timeout");
  __atomic_store_n(c->err_host, 0u, __ATOMIC_RELEASE);
  if (code == 2)
    return fail(BG_E_DEVICE, "decode split merge gave up waiting for a split: a merging workgroup ran on another "
                             "XCD than its splits, so their partials stayed in that XCD's L2; partials are written "
                             "through to memory from now on. Outputs of bg_attention calls on this cache since the last "
                             "check may be wrong (the merge that gave up stored NaN); the split workspace has been reset");
  return fail(BG_E_DEVICE, "decode split merge gave up waiting for a split (GPU shared or oversubscribed): outputs "
                           "of bg_attention calls on this cache since the last check may be wrong (the merge that gave "
                           "up stored NaN; a partial that landed after it can have been taken by a later launch); the "
                           "split workspace has been reset");
}

}  // namespace

extern "C" {

const char* bg_last_error_message(void) { return g_err.c_str(); }

int32_t bg_debug_merge_hooks(int32_t spin_limit, int32_t withhold_split) {
  if (spin_limit < 0) return fail(BG_E_INVALID, "bg_debug_merge_hooks: spin_limit %d < 0", spin_limit);
  g_merge_spin.store(spin_limit, std::memory_order_relaxed);
  g_withhold_split.store(withhold_split < 0 ? -1 : withhold_split, std::memory_order_relaxed);
  return BG_OK;
}

const char* bg_version(void) { return "bitgpu-mi355x-attn 0.1.0 (gfx950)"; }

int32_t bg_rope_tables(double theta, int32_t rot_dim, int32_t positions, double yarn_factor,
                       int32_t yarn_original_max_positions, float* cos_out, float* sin_out) {
  // synthRope, src/engine.ts:117-147: f64 inverse frequencies and angles, one f32 rounding
  if (rot_dim <= 0 || (rot_dim & 1) || positions < 0 || !cos_out || !sin_out || !(theta > 0))
    return fail(BG_E_INVALID, "bg_rope_tables: bad arguments (rot_dim %d, positions %d)", rot_dim, positions);
  const int half = rot_dim / 2;
  const double factor = yarn_factor > 1.0 ? yarn_factor : 1.0;
  std::vector<double> inv(half);
  double lo = 0, hi = 0;
  if (factor != 1.0) {
    const double orig = (double)yarn_original_max_positions;
    lo = std::max(0.0, std::floor((rot_dim * std::log(orig / (32 * 2 * M_PI))) / (2 * std::log(theta))));
    hi = std::min((double)(half - 1), std::ceil((rot_dim * std::log(orig / (2 * M_PI))) / (2 * std::log(theta))));
  }
  for (int j = 0; j < half; j++) {
    const double pf = std::pow(theta, (2.0 * j) / rot_dim);
    if (factor == 1.0) {
      inv[j] = 1.0 / pf;
    } else {
      const double ramp = std::min(1.0, std::max(0.0, (j - lo) / (hi - lo)));
      inv[j] = (1.0 / (factor * pf)) * ramp + (1.0 / pf) * (1 - ramp);
    }
  }
  const double mscale = factor == 1.0 ? 1.0 : (double)(float)(0.1 * std::log(factor) + 1);
  for (int p = 0; p < positions; p++)
    for (int j = 0; j < half; j++) {
      const double a = p * inv[j];
      cos_out[(size_t)p * half + j] = (float)(std::cos(a) * mscale);
      sin_out[(size_t)p * half + j] = (float)(std::sin(a) * mscale);
    }
  return BG_OK;
}

int32_t bg_evict_plan(int32_t fill, int32_t need, int32_t sinks, int32_t max_seq_len, int32_t* new_fill,
                      int32_t* batch, int32_t* keep) {
  // evict(), src/engine.ts:1188-1212
  if (!new_fill || sinks < 0 || fill < sinks || max_seq_len <= sinks)
    return fail(BG_E_INVALID, "bg_evict_plan: bad arguments (fill %d, sinks %d, max_seq %d)", fill, sinks, max_seq_len);
  const int recent = fill - sinks;
  const int quarter = (max_seq_len - sinks + 3) / 4;
  const int b = std::min(recent, std::max(need, quarter));
  const int k = recent - b;
  *new_fill = k <= 0 ? sinks : sinks + k;
  if (batch) *batch = b;
  if (keep) *keep = k;
  return BG_OK;
}

int32_t bg_ring_map(int32_t sinks, int32_t max_seq_len, int32_t head, int32_t logical, int32_t* physical) {
  if (!physical || sinks < 0 || max_seq_len <= sinks || head < 0 || head >= max_seq_len - sinks || logical < 0 ||
      logical >= max_seq_len)
    return fail(BG_E_INVALID, "bg_ring_map: bad arguments (sinks %d, max_seq %d, head %d, logical %d)", sinks,
                max_seq_len, head, logical);
  bg::Ring r;
  r.roll = 1;
  r.sinks = sinks;
  r.W = max_seq_len - sinks;
  r.head = head;
  *physical = r.phys(logical);
  return BG_OK;
}

int32_t bg_stream_sync(void* stream) {
  hipError_t e = stream ? hipStreamSynchronize((hipStream_t)stream) : hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(e, "stream sync");
  std::lock_guard<std::mutex> lock(g_caches_mu);
  for (bg_kv_cache* c : g_caches) {
    int32_t rc = take_merge_error(c, (hipStream_t)stream);
    if (rc != BG_OK) return rc;
  }
  return BG_OK;
}

int32_t bg_stream_create(void** stream) {
  if (!stream) return fail(BG_E_INVALID, "bg_stream_create: out is NULL");
  *stream = nullptr;
  hipStream_t s;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);  // default priority
  if (e != hipSuccess) return hip_fail(e, "stream create");
  *stream = (void*)s;
  return BG_OK;
}

int32_t bg_stream_destroy(void* stream) {
  if (!stream) return BG_OK;
  hipError_t e = hipStreamDestroy((hipStream_t)stream);
  return e == hipSuccess ? BG_OK : hip_fail(e, "stream destroy");
}

int32_t bg_event_create(void** event) {
  if (!event) return fail(BG_E_INVALID, "bg_event_create: out is NULL");
  *event = nullptr;
  hipEvent_t ev;
  hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) return hip_fail(e, "event create");
  *event = (void*)ev;
  return BG_OK;
}

int32_t bg_event_record(void* event, void* stream) {
  if (!event) return fail(BG_E_INVALID, "bg_event_record: event is NULL");
  hipError_t e = hipEventRecord((hipEvent_t)event, (hipStream_t)stream);
  return e == hipSuccess ? BG_OK : hip_fail(e, "event record");
}

int32_t bg_event_elapsed_us(void* start, void* end, float* us) {
  if (!start || !end || !us) return fail(BG_E_INVALID, "bg_event_elapsed_us: NULL argument");
  hipError_t e = hipEventSynchronize((hipEvent_t)end);
  if (e != hipSuccess) return hip_fail(e, "event synchronize");
  float ms = 0.0f;
  e = hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)end);
  if (e != hipSuccess) return hip_fail(e, "event elapsed time");
  *us = ms * 1000.0f;
  return BG_OK;
}

int32_t bg_event_destroy(void* event) {
  if (!event) return BG_OK;
  hipError_t e = hipEventDestroy((hipEvent_t)event);
  return e == hipSuccess ? BG_OK : hip_fail(e, "event destroy");
}

int32_t bg_kv_create(int32_t n_layers, int32_t kv_heads, int32_t head_dim, int32_t dtype, int32_t capacity,
                     int32_t max_seq_len, int32_t roll, int32_t sinks, int32_t rope_pos_mode, bg_kv_cache** out) {
  if (!out) return fail(BG_E_INVALID, "bg_kv_create: out is NULL");
  *out = nullptr;
  if (n_layers < 1 || kv_heads < 1 || max_seq_len < 1)
    return fail(BG_E_INVALID, "bg_kv_create: n_layers %d, kv_heads %d, max_seq_len %d must be >= 1", n_layers, kv_heads, max_seq_len);
  if (head_dim != 128 && head_dim != 256)
    return fail(BG_E_UNSUPPORTED, "bg_kv_create: head_dim %d unsupported (128 or 256)", head_dim);
  if (dtype != BG_KV_F32 && dtype != BG_KV_F16 && dtype != BG_KV_Q8)
    return fail(BG_E_INVALID, "bg_kv_create: unknown kv dtype %d", dtype);
  if (dtype == BG_KV_Q8 && head_dim % 32 != 0)  // src/engine.ts:372-373
    return fail(BG_E_INVALID, "kvCache 'q8' needs head_dim divisible by 32 (got %d)", head_dim);
  {
    // one kv head's K (or V) region, and the f16 prefill copy of a q8 layer, are addressed with
    // 32-bit byte offsets by the buffer loads of the prefill kernel
    const long long eb = dtype == BG_KV_F32 ? 4 : 2;
    const long long per_head = (((long long)max_seq_len + 31) & ~31LL) * head_dim * eb;
    if (per_head > 0x7fffffffLL)
      return fail(BG_E_UNSUPPORTED, "bg_kv_create: max_seq_len %d x head_dim %d needs %lld bytes per kv head and layer, "
                                    "beyond the 2^31 - 1 a kernel addresses", max_seq_len, head_dim, per_head);
  }
  if (roll) {
    if (sinks < 1) return fail(BG_E_INVALID, "bg_kv_create: sink mode needs sinks >= 1 (got %d)", sinks);
    if (max_seq_len < sinks + 64)  // src/engine.ts:311-312
      return fail(BG_E_INVALID, "overflow 'sinks' needs maxSeqLen >= sinkTokens + 64 (got %d with %d sinks)", max_seq_len, sinks);
    if (rope_pos_mode != BG_ROPE_SLOT && rope_pos_mode != BG_ROPE_ABSOLUTE)
      return fail(BG_E_INVALID, "bg_kv_create: unknown rope position mode %d", rope_pos_mode);
  }
  bg_kv_cache* c = new bg_kv_cache();
  c->n_layers = n_layers;
  c->kv_heads = kv_heads;
  c->D = head_dim;
  c->dtype = dtype;
  c->max_seq = max_seq_len;
  c->roll = roll ? 1 : 0;
  c->sinks = roll ? sinks : 0;
  c->rope_abs = roll && rope_pos_mode == BG_ROPE_ABSOLUTE;
  // The ring needs the whole window resident; otherwise start at min(maxSeqLen, capacity)
  // (KV_INITIAL = 512 when capacity <= 0, src/engine.ts:1044-1046) and grow by doubling.
  int initial = capacity > 0 ? capacity : 512;
  c->capacity = roll ? max_seq_len : std::min(max_seq_len, initial);
  c->cap = round32(c->capacity);
  int dev = 0;
  (void)hipGetDevice(&dev);
  c->device = dev;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) c->num_cus = cus;
  (void)xcd_state(dev);  // probe the workgroup placement once per device
  const size_t row = (size_t)c->cap * kv_heads * head_dim * elem_bytes(dtype);
  const size_t srow = (size_t)c->cap * kv_heads * (head_dim / 32) * sizeof(float);
  for (int l = 0; l < n_layers; l++) {
    void *kp = nullptr, *vp = nullptr;
    float *ksp = nullptr, *vsp = nullptr;
    hipError_t e = hipMalloc(&kp, row);
    if (e == hipSuccess) e = hipMalloc(&vp, row);
    if (e == hipSuccess && dtype == BG_KV_Q8) e = hipMalloc((void**)&ksp, srow);
    if (e == hipSuccess && dtype == BG_KV_Q8) e = hipMalloc((void**)&vsp, srow);
    c->k.push_back(kp);
    c->v.push_back(vp);
    c->ks.push_back(ksp);
    c->vs.push_back(vsp);
    if (e == hipSuccess) e = hipMemset(kp, 0, row);
    if (e == hipSuccess) e = hipMemset(vp, 0, row);
    if (e == hipSuccess && ksp) e = hipMemset(ksp, 0, srow);
    if (e == hipSuccess && vsp) e = hipMemset(vsp, 0, srow);
    if (e != hipSuccess) {
      free_layers(c->k, c->v, c->ks, c->vs);
      delete c;
      return hip_fail(e, "KV cache allocation");
    }
  }
  hipError_t e = hipHostMalloc((void**)&c->err_host, 64, hipHostMallocMapped | hipHostMallocCoherent);
  if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&c->err_dev, c->err_host, 0);
  const size_t praw = bg::qkv_proj_raw_floats(kProjMaxHeads, head_dim);
  if (e == hipSuccess) e = hipMalloc((void**)&c->proj_raw, praw * sizeof(float));
  if (e == hipSuccess) e = hipMemsetD32((hipDeviceptr_t)c->proj_raw, (int)bg::kWorkspaceEmpty, praw);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    if (c->err_host) (void)hipHostFree(c->err_host);
    if (c->proj_raw) (void)hipFree(c->proj_raw);
    free_layers(c->k, c->v, c->ks, c->vs);
    delete c;
    return hip_fail(e, "KV cache side buffers allocation");
  }
  *c->err_host = 0;
  {
    std::lock_guard<std::mutex> lock(g_caches_mu);
    g_caches.insert(c);
  }
  *out = c;
  return BG_OK;
}

int32_t bg_kv_destroy(bg_kv_cache* c) {
  if (!c) return BG_OK;
  {
    std::lock_guard<std::mutex> lock(g_caches_mu);
    g_caches.erase(c);
  }
  (void)hipDeviceSynchronize();
  if (c->err_host) (void)hipHostFree(c->err_host);
  if (c->stage) (void)hipFree(c->stage);
  if (c->proj_raw) (void)hipFree(c->proj_raw);
  free_layers(c->k, c->v, c->ks, c->vs);
  if (c->ws) (void)hipFree(c->ws);
  if (c->ws_count) (void)hipFree(c->ws_count);
  if (c->pf16) (void)hipFree(c->pf16);
  if (c->pf_ml) (void)hipFree(c->pf_ml);
  for (const auto& r : c->retired_ws) (void)hipFree(r.first);
  for (unsigned* r : c->retired_count) (void)hipFree(r);
  delete c;
  return BG_OK;
}

int32_t bg_kv_capacity(const bg_kv_cache* c, int32_t* capacity) {
  if (!c || !capacity) return fail(BG_E_INVALID, "bg_kv_capacity: NULL argument");
  *capacity = c->capacity;
  return BG_OK;
}

int32_t bg_kv_grow(bg_kv_cache* c, int32_t needed, void* stream) {
  if (!c) return fail(BG_E_INVALID, "bg_kv_grow: NULL cache");
  // ensureKvCapacity, src/engine.ts:1120-1178
  needed = std::min(needed, c->max_seq);
  if (needed <= c->capacity) return BG_OK;
  const int newCap = std::min(c->max_seq, std::max(needed, c->capacity * 2));
  const int ncap = round32(newCap);
  hipStream_t st = (hipStream_t)stream;
  const size_t eb = elem_bytes(c->dtype);
  const size_t nrow = (size_t)ncap * c->kv_heads * c->D * eb;
  const size_t nsrow = (size_t)ncap * c->kv_heads * (c->D / 32) * sizeof(float);
  std::vector<void*> nk, nv;
  std::vector<float*> nks, nvs;
  int counter = 0;
  hipError_t e = hipSuccess;
  for (int l = 0; l < c->n_layers && e == hipSuccess; l++) {
    void *kp = nullptr, *vp = nullptr;
    float *ksp = nullptr, *vsp = nullptr;
    e = grow_malloc(&kp, nrow, &counter);
    if (e == hipSuccess) e = grow_malloc(&vp, nrow, &counter);
    if (e == hipSuccess && c->dtype == BG_KV_Q8) e = grow_malloc((void**)&ksp, nsrow, &counter);
    if (e == hipSuccess && c->dtype == BG_KV_Q8) e = grow_malloc((void**)&vsp, nsrow, &counter);
    nk.push_back(kp);
    nv.push_back(vp);
    nks.push_back(ksp);
    nvs.push_back(vsp);
  }
  if (e != hipSuccess) {
    // roll back: keep the old buffers (src/engine.ts:1157-1173)
    free_layers(nk, nv, nks, nvs);
    (void)hipGetLastError();
    return fail(BG_E_OOM, "KV cache growth to %d positions failed: %s", newCap, hipGetErrorString(e));
  }
  // copy every head's rows: [kvh][cap][...] regions keep their head stride = cap
  for (int l = 0; l < c->n_layers && e == hipSuccess; l++) {
    e = hipMemsetAsync(nk[l], 0, nrow, st);
    if (e == hipSuccess) e = hipMemsetAsync(nv[l], 0, nrow, st);
    if (e == hipSuccess && nks[l]) e = hipMemsetAsync(nks[l], 0, nsrow, st);
    if (e == hipSuccess && nvs[l]) e = hipMemsetAsync(nvs[l], 0, nsrow, st);
    for (int h = 0; h < c->kv_heads && e == hipSuccess; h++) {
      const size_t ob = (size_t)c->cap * c->D * eb, nb = (size_t)ncap * c->D * eb;
      e = hipMemcpyAsync((char*)nk[l] + h * nb, (char*)c->k[l] + h * ob, ob, hipMemcpyDeviceToDevice, st);
      if (e == hipSuccess) e = hipMemcpyAsync((char*)nv[l] + h * nb, (char*)c->v[l] + h * ob, ob, hipMemcpyDeviceToDevice, st);
      if (e == hipSuccess && nks[l]) {
        const size_t os = (size_t)c->cap * (c->D / 32) * sizeof(float), ns = (size_t)ncap * (c->D / 32) * sizeof(float);
        e = hipMemcpyAsync((char*)nks[l] + h * ns, (char*)c->ks[l] + h * os, os, hipMemcpyDeviceToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync((char*)nvs[l] + h * ns, (char*)c->vs[l] + h * os, os, hipMemcpyDeviceToDevice, st);
      }
    }
  }
  if (e == hipSuccess) e = st ? hipStreamSynchronize(st) : hipDeviceSynchronize();
  if (e != hipSuccess) {
    free_layers(nk, nv, nks, nvs);
    return hip_fail(e, "KV cache growth copy");
  }
  free_layers(c->k, c->v, c->ks, c->vs);
  c->k = nk;
  c->v = nv;
  c->ks = nks;
  c->vs = nvs;
  c->capacity = newCap;
  c->cap = ncap;
  return BG_OK;
}

int32_t bg_kv_set_q8_block(bg_kv_cache* c, int32_t block) {
  if (!c) return fail(BG_E_INVALID, "bg_kv_set_q8_block: NULL cache");
  if (c->dtype != BG_KV_Q8) return fail(BG_E_STATE, "bg_kv_set_q8_block: the cache is not q8");
  if (block != 32 && block != c->D)
    return fail(BG_E_UNSUPPORTED, "bg_kv_set_q8_block: block %d (32 or head_dim %d)", block, c->D);
  c->q8_row = block == c->D && block != 32;
  return BG_OK;
}

int32_t bg_kv_set_rope(bg_kv_cache* c, const float* cos_tab, const float* sin_tab, int32_t positions, int32_t rot_dim) {
  if (!c || !cos_tab || !sin_tab || positions < 1) return fail(BG_E_INVALID, "bg_kv_set_rope: bad arguments");
  if (rot_dim != c->D) return fail(BG_E_UNSUPPORTED, "read-time rotation needs rot_dim == head_dim (%d vs %d)", rot_dim, c->D);
  c->cos_tab = cos_tab;
  c->sin_tab = sin_tab;
  c->rope_positions = positions;
  return BG_OK;
}

int32_t bg_kv_write(bg_kv_cache* c, int32_t layer, int32_t which, const float* src, int32_t rows, int32_t dst_row0,
                    void* stream) {
  if (!c || !src) return fail(BG_E_INVALID, "bg_kv_write: NULL argument");
  if (layer < 0 || layer >= c->n_layers) return fail(BG_E_INVALID, "bg_kv_write: layer %d out of range", layer);
  if (which != BG_K && which != BG_V) return fail(BG_E_INVALID, "bg_kv_write: which must be BG_K or BG_V");
  if (rows < 0 || dst_row0 < 0) return fail(BG_E_INVALID, "bg_kv_write: negative rows/dst_row0");
  const long last = (long)dst_row0 + rows;  // exclusive reference row
  if (rows > 0 && (last + c->kv_heads - 1) / c->kv_heads > addressable(c))
    return fail(BG_E_INVALID, "bg_kv_write: rows reach position %ld beyond capacity %d", (last - 1) / c->kv_heads, addressable(c));
  hipError_t e = bg::launch_kv_write(view(c, layer), which, src, rows, dst_row0, (hipStream_t)stream);
  return e == hipSuccess ? BG_OK : hip_fail(e, "kv write launch");
}

int32_t bg_qkv_prologue(bg_kv_cache* c, int32_t layer, const float* q, int32_t q_stride, const float* k, const float* v,
                        int32_t S, int32_t H, const float* q_gamma, const float* k_gamma, float eps,
                        const float* cos_tab, const float* sin_tab, int32_t rope_positions, int32_t rot_dim,
                        int32_t pos0, int32_t slot0, float* q_out, void* stream) {
  if (!c) return fail(BG_E_INVALID, "bg_qkv_prologue: NULL cache");
  if (layer < 0 || layer >= c->n_layers) return fail(BG_E_INVALID, "bg_qkv_prologue: layer %d out of range", layer);
  if (S < 1) return fail(BG_E_INVALID, "bg_qkv_prologue: S must be >= 1");
  if (q) {
    if (H < c->kv_heads || H % c->kv_heads) return fail(BG_E_INVALID, "heads %d must be a multiple of kv_heads %d", H, c->kv_heads);
    if (!q_out || !q_gamma) return fail(BG_E_INVALID, "bg_qkv_prologue: q needs q_out and q_gamma");
    if (q_stride < c->D) return fail(BG_E_INVALID, "bg_qkv_prologue: q_stride %d < head_dim %d", q_stride, c->D);
  }
  if (k && !k_gamma) return fail(BG_E_INVALID, "bg_qkv_prologue: k needs k_gamma");
  const bool ropes = q || (k && !c->roll);
  if (ropes) {
    if (!cos_tab || !sin_tab) return fail(BG_E_INVALID, "bg_qkv_prologue: rope tables are NULL");
    if (rot_dim < 2 || (rot_dim & 1) || rot_dim > c->D) return fail(BG_E_INVALID, "bg_qkv_prologue: bad rot_dim %d", rot_dim);
    if (pos0 < 0 || (long)pos0 + S > rope_positions)
      return fail(BG_E_INVALID, "bg_qkv_prologue: positions %d..%d outside the %d-row rope table", pos0, pos0 + S - 1, rope_positions);
  }
  // rows are read and written 16 bytes a lane
  const uintptr_t mis = ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)q_out | (uintptr_t)q_gamma |
                         (uintptr_t)k_gamma | (uintptr_t)cos_tab | (uintptr_t)sin_tab) & 15;
  if (mis || (q && (q_stride & 3)))
    return fail(BG_E_INVALID, "bg_qkv_prologue: buffers must be 16-byte aligned and q_stride a multiple of 4");
  if ((k || v) && (slot0 < 0 || (long)slot0 + S > addressable(c)))
    return fail(BG_E_INVALID, "bg_qkv_prologue: slots %d..%d beyond capacity %d", slot0, slot0 + S - 1, addressable(c));
  bg::PrologueArgs a;
  a.q = q;
  a.q_stride = q_stride;
  a.k = k;
  a.v = v;
  a.S = S;
  a.H = H;
  a.q_gamma = q_gamma;
  a.k_gamma = k_gamma;
  a.eps = eps;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.rot_dim = rot_dim;
  a.pos0 = pos0;
  a.slot0 = slot0;
  a.q_out = q_out;
  hipError_t e = bg::launch_qkv_prologue(view(c, layer), a, (hipStream_t)stream);
  return e == hipSuccess ? BG_OK : hip_fail(e, "prologue launch");
}

// The attention workspace: decode split partials, f32 split partials or split-K prefill partials
// (each launch uses one kind; every slot holds the empty marker between launches). Grows to at
// least `need` floats and `counters` counters, keeping the larger of old and new.
static int32_t ensure_workspace_floats(bg_kv_cache* c, size_t need, size_t counters) {
  if (need < c->ws_floats) need = c->ws_floats;
  if (counters < c->ws_counters) counters = c->ws_counters;
  if (need <= c->ws_floats && counters <= c->ws_counters) return BG_OK;
  // grow at least twofold, so that few workspaces are ever retired
  if (need < 2 * c->ws_floats) need = 2 * c->ws_floats;
  float* ws = nullptr;
  unsigned* cnt = nullptr;
  hipError_t e = hipMalloc((void**)&ws, need * sizeof(float));
  if (e == hipSuccess && counters) e = hipMalloc((void**)&cnt, counters * sizeof(unsigned));
  if (e == hipSuccess && counters) e = hipMemset(cnt, 0, counters * sizeof(unsigned));
  // split slots start out "empty"; every launch leaves them that way
  if (e == hipSuccess) e = hipMemsetD32((hipDeviceptr_t)ws, (int)bg::decode_workspace_empty(), need);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    // the old workspace stays in use
    if (ws) (void)hipFree(ws);
    if (cnt) (void)hipFree(cnt);
    (void)hipGetLastError();
    return fail(e == hipErrorOutOfMemory ? BG_E_OOM : BG_E_DEVICE, "attention workspace allocation: %s",
                hipGetErrorString(e));
  }
  // launches captured before keep using the old buffers: retire them instead of freeing
  if (c->ws) c->retired_ws.emplace_back(c->ws, c->ws_floats);
  if (c->ws_count && cnt) c->retired_count.push_back(c->ws_count);
  c->ws = ws;
  c->ws_floats = need;
  if (cnt) {
    c->ws_count = cnt;
    c->ws_counters = counters;
  }
  return BG_OK;
}

// split-K prefill: partials in the workspace, (m, l) in a buffer of their own
static int32_t ensure_prefill_split(bg_kv_cache* c, size_t floats) {
  int32_t rc = ensure_workspace_floats(c, floats, 0);
  if (rc != BG_OK || c->pf_ml) return rc;
  hipError_t e = hipMalloc((void**)&c->pf_ml, bg::prefill_split_ml_bytes());
  if (e != hipSuccess) {
    c->pf_ml = nullptr;
    return hip_fail(e, "split prefill (m, l) allocation");
  }
  return BG_OK;
}

static int32_t ensure_workspace(bg_kv_cache* c, int S, int H) {
  size_t counters = 0;
  size_t need = bg::decode_workspace_floats(view(c, 0), S, H, c->num_cus, &counters);
  if (c->dtype == BG_KV_F32) {
    const size_t f = bg::f32_workspace_floats(view(c, 0), S, H);
    need = f > need ? f : need;
  }
  return ensure_workspace_floats(c, need, counters);
}

// the f16 prefill copy holds one layer at the cache's physical capacity (zero-filled, so slots
// past the dequantized range read as finite zeros)
static int32_t ensure_prefill_copy(bg_kv_cache* c) {
  if (c->pf16 && c->pf16_cap == c->cap) return BG_OK;
  if (c->pf16) (void)hipFree(c->pf16);
  c->pf16 = nullptr;
  c->pf16_cap = 0;
  const size_t bytes = (size_t)2 * c->kv_heads * c->cap * c->D * sizeof(uint16_t);
  hipError_t e = hipMalloc(&c->pf16, bytes);
  if (e == hipSuccess) e = hipMemset(c->pf16, 0, bytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    if (c->pf16) (void)hipFree(c->pf16);
    c->pf16 = nullptr;
    return hip_fail(e, "prefill f16 copy allocation");
  }
  c->pf16_cap = c->cap;
  return BG_OK;
}

int32_t bg_attention_reserve(bg_kv_cache* c, int32_t S, int32_t H) {
  if (!c || S < 1 || H < 1 || H % c->kv_heads) return fail(BG_E_INVALID, "bg_attention_reserve: bad arguments");
  if (c->dtype != BG_KV_F32 && !bg::decode_preferred(view(c, 0), S, H)) {
    if (bg::prefill_wants_f16_copy(view(c, 0), S, H)) {
      int32_t rc = ensure_prefill_copy(c);
      if (rc != BG_OK) return rc;
    }
    const size_t pf = bg::prefill_workspace_floats_max(view(c, 0), S, H, c->num_cus);
    return pf > 0 ? ensure_prefill_split(c, pf) : BG_OK;
  }
  if (!bg::decode_supported(view(c, 0), S, H) && !bg::f32_split_supported(view(c, 0), S, H)) return BG_OK;
  return ensure_workspace(c, S, H);
}

// Argument checks shared by bg_attention and bg_attention_noalloc.
static int32_t check_attention_args(bg_kv_cache* c, int32_t layer, const float* q, int32_t S, int32_t H,
                                    int32_t pos_base, float scale, const float* gate, int32_t gate_stride, float* out) {
  if (!c || !q || !out) return fail(BG_E_INVALID, "bg_attention: NULL argument");
  if (layer < 0 || layer >= c->n_layers) return fail(BG_E_INVALID, "bg_attention: layer %d out of range", layer);
  if (S < 1 || H < 1 || H % c->kv_heads) return fail(BG_E_INVALID, "bg_attention: S %d, heads %d (kv_heads %d)", S, H, c->kv_heads);
  if (pos_base < 0 || (long)pos_base + S > addressable(c))
    return fail(BG_E_INVALID, "bg_attention: positions %d..%d exceed the cache (%d slots)", pos_base, pos_base + S - 1, addressable(c));
  if (gate && gate_stride < c->D) return fail(BG_E_INVALID, "bg_attention: gate_stride %d < head_dim", gate_stride);
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(BG_E_INVALID, "bg_attention: scale must be positive");
  if (c->roll) {
    if (!c->cos_tab) return fail(BG_E_STATE, "bg_attention: sink mode needs bg_kv_set_rope first");
    // valid slots are logical < pos_base + S; their rotation index is the slot, or slot +
    // evicted (absolute mode); masked slots clamp their index inside the table
    const long need = (long)pos_base + S + (c->rope_abs ? c->evicted : 0);
    if (c->rope_positions < need)
      return fail(BG_E_INVALID, "bg_attention: rope table has %d rows, read-time rotation needs %ld", c->rope_positions, need);
  }
  return BG_OK;
}

static bg::AttnArgs attention_args(bg_kv_cache* c, const float* q, int32_t S, int32_t H, int32_t pos_base, float scale,
                                   const float* gate, int32_t gate_stride, float* out) {
  bg::AttnArgs a;
  a.q = q;
  a.S = S;
  a.H = H;
  a.pos_base = pos_base;
  a.scale = scale;
  a.gate = gate;
  a.gate_stride = gate_stride;
  a.out = out;
  a.ws_o = nullptr;
  a.ws_ml = nullptr;
  a.pf_ml = nullptr;
  a.ws_count = nullptr;
  a.ws_floats = 0;
  a.num_cus = c->num_cus;
  a.err = c->err_dev;
  a.spin_limit = g_merge_spin.load(std::memory_order_relaxed);
  a.withhold_split = g_withhold_split.load(std::memory_order_relaxed);
  const int xs = xcd_state(c->device);
  a.n_xcd = xs > 0 ? xs : 0;
  return a;
}

int32_t bg_attention(bg_kv_cache* c, int32_t layer, const float* q, int32_t S, int32_t H, int32_t pos_base, float scale,
                     const float* gate, int32_t gate_stride, float* out, void* stream) {
  int32_t rc0 = check_attention_args(c, layer, q, S, H, pos_base, scale, gate, gate_stride, out);
  if (rc0 != BG_OK) return rc0;
  hipStream_t st = (hipStream_t)stream;
  rc0 = take_merge_error(c, st);
  if (rc0 != BG_OK) return rc0;
  LayerView L = view(c, layer);
  bg::AttnArgs a = attention_args(c, q, S, H, pos_base, scale, gate, gate_stride, out);
  hipError_t e;
  if (c->dtype == BG_KV_F32 && bg::f32_split_supported(L, S, H)) {
    int32_t rc = ensure_workspace(c, S, H);
    if (rc != BG_OK) return rc;
    a.ws_o = c->ws;
    a.ws_count = c->ws_count;
    a.ws_floats = c->ws_floats;
    e = bg::launch_attention_f32_split(L, a, st);
  } else if (c->dtype == BG_KV_F32) {
    e = bg::launch_attention_f32(L, a, st);
  } else if (bg::decode_preferred(L, S, H)) {
    int32_t rc = ensure_workspace(c, S, H);
    if (rc != BG_OK) return rc;
    a.ws_o = c->ws;
    a.ws_count = c->ws_count;
    a.ws_floats = c->ws_floats;
    e = bg::launch_attention_decode(L, a, st);
  } else if (bg::prefill_supported(L, S, H)) {
    const size_t pf = bg::prefill_workspace_floats(L, S, H, pos_base, c->num_cus);
    if (pf > 0) {
      int32_t rc = ensure_prefill_split(c, pf);
      if (rc != BG_OK) return rc;
      a.ws_o = c->ws;
      a.ws_floats = c->ws_floats;
      a.pf_ml = c->pf_ml;
    }
    if (bg::prefill_wants_f16_copy(L, S, H)) {
      // dequantize the attended slots once, then run the f16 path on the copy
      int32_t rc = ensure_prefill_copy(c);
      if (rc != BG_OK) return rc;
      int n = (pos_base + S + 63) & ~63;
      n = n < c->cap ? n : c->cap;
      LayerView F = L;
      F.k = c->pf16;
      F.v = (uint16_t*)c->pf16 + (size_t)c->kv_heads * c->cap * c->D;
      F.ks = nullptr;
      F.vs = nullptr;
      F.dtype = bg::KV_F16;
      e = bg::launch_kv_dequant_f16(L, n, F.k, F.v, st);
      if (e == hipSuccess) e = bg::launch_attention_prefill(F, a, st);
    } else {
      e = bg::launch_attention_prefill(L, a, st);
    }
  } else {
    return fail(BG_E_UNSUPPORTED, "bg_attention: no kernel for S %d, heads %d", S, H);
  }
  return e == hipSuccess ? BG_OK : hip_fail(e, "attention launch");
}

int32_t bg_attention_noalloc(bg_kv_cache* c, int32_t layer, const float* q, int32_t S, int32_t H, int32_t pos_base,
                             float scale, const float* gate, int32_t gate_stride, float* out, void* stream) {
  int32_t rc = check_attention_args(c, layer, q, S, H, pos_base, scale, gate, gate_stride, out);
  if (rc != BG_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "bg_attention_noalloc: current device");
  if (dev < 0 || dev >= kMaxDevices) return fail(BG_E_UNSUPPORTED, "bg_attention_noalloc: device %d beyond %d", dev, kMaxDevices);
  void* ptr = nullptr;
  {
    // set-up, once per device with that device current: the array's device address, then
    // every slot set to the empty marker (a fill kernel, completed before first use)
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
      if (capturing(st))
        return fail(BG_E_STATE, "bg_attention_noalloc: the first call on a device sets up its scratch and "
                                "cannot be captured; call it once outside graph capture");
      void* p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "scratch symbol address");
      hipLaunchKernelGGL(fill_u32_kernel, dim3(256), dim3(256), 0, st, (uint32_t*)p, bg::decode_workspace_empty(),
                         kScratchBytes / 4);
      e = hipGetLastError();
      if (e == hipSuccess) e = st ? hipStreamSynchronize(st) : hipDeviceSynchronize();
      if (e != hipSuccess) return hip_fail(e, "scratch set-up");
      g_scratch_ptr[dev] = p;
    }
    ptr = g_scratch_ptr[dev];
  }
  rc = take_merge_error(c, st);
  if (rc != BG_OK) return rc;
  LayerView L = view(c, layer);
  bg::AttnArgs a = attention_args(c, q, S, H, pos_base, scale, gate, gate_stride, out);
  if (c->dtype == BG_KV_F32) {
    // the f32 kernels run without partials here (the matrix-core kernel for every shape)
    e = bg::launch_attention_f32(L, a, st);
  } else if (bg::decode_preferred(L, S, H)) {
    bg::DecodePlan pl;
    // the most splits any occupancy gives (a lower residency only merges splits)
    if (!bg::decode_plan(L, S, H, pos_base, c->num_cus, 1 << 20, &pl)) return fail(BG_E_UNSUPPORTED, "decode plan");
    const size_t need = bg::decode_partial_floats(L, S, H, pl.n_splits) * sizeof(float);
    if (pl.n_splits > 1 && need > kScratchBytes)
      return fail(BG_E_INVALID, "bg_attention_noalloc: the split partials of S %d, heads %d over %d positions need %zu "
                                "bytes, beyond the %zu-byte scratch (use bg_attention)", S, H, pos_base + S, need, kScratchBytes);
    a.ws_o = (float*)ptr;
    a.ws_floats = kScratchBytes / sizeof(float);
    e = bg::launch_attention_decode(L, a, st);
  } else if (bg::prefill_supported(L, S, H)) {
    // a q8 cache is staged in-kernel (no f16 copy): the same values, so the same results; a
    // split-K prefill keeps its partials in the scratch (the split plan caps them below it)
    if (bg::prefill_split_ml_bytes() > kScratchMlBytes)
      return fail(BG_E_UNSUPPORTED, "bg_attention_noalloc: the scratch's (m, l) area is smaller than a split prefill needs");
    a.ws_o = (float*)ptr;
    a.ws_floats = kScratchBytes / sizeof(float);
    a.pf_ml = (float*)((char*)ptr + kScratchBytes);
    e = bg::launch_attention_prefill(L, a, st);
  } else {
    return fail(BG_E_UNSUPPORTED, "bg_attention_noalloc: no kernel for S %d, heads %d", S, H);
  }
  return e == hipSuccess ? BG_OK : hip_fail(e, "attention launch");
}

static int32_t check_gemv(const char* who, const float* x, int32_t K, const uint32_t* sign, const float* scales) {
  if (!x || !sign || !scales) return fail(BG_E_INVALID, "%s: NULL argument", who);
  if (K < 128 || K % 128) return fail(BG_E_INVALID, "%s: K %d must be a positive multiple of 128", who, K);
  if (((uintptr_t)x | (uintptr_t)sign | (uintptr_t)scales) & 15)
    return fail(BG_E_INVALID, "%s: x, sign and scales must be 16-byte aligned", who);
  return BG_OK;
}

int32_t bg_gemv_split(const float* x, int32_t K, const uint32_t* sign, const float* scales, int32_t N0, int32_t N1,
                      int32_t N2, float* out0, float* out1, float* out2, void* stream) {
  int32_t rc = check_gemv("bg_gemv_split", x, K, sign, scales);
  if (rc != BG_OK) return rc;
  if (N0 < 0 || N1 < 0 || N2 < 0 || (N0 && !out0) || (N1 && !out1) || (N2 && !out2))
    return fail(BG_E_INVALID, "bg_gemv_split: output ranges %d/%d/%d need their buffers", N0, N1, N2);
  bg::GemvArgs a{x, K, sign, scales, N0, N1, N2, out0, out1, out2, nullptr};
  hipError_t e = bg::launch_gemv(a, (hipStream_t)stream);
  return e == hipSuccess ? BG_OK : hip_fail(e, "gemv launch");
}

int32_t bg_gemv_resid(const float* x, int32_t K, const uint32_t* sign, const float* scales, int32_t N,
                      const float* resid, float* y, void* stream) {
  int32_t rc = check_gemv("bg_gemv_resid", x, K, sign, scales);
  if (rc != BG_OK) return rc;
  if (N < 0 || !resid || !y) return fail(BG_E_INVALID, "bg_gemv_resid: N %d needs resid and y", N);
  bg::GemvArgs a{x, K, sign, scales, N, 0, 0, y, nullptr, nullptr, resid};
  hipError_t e = bg::launch_gemv(a, (hipStream_t)stream);
  return e == hipSuccess ? BG_OK : hip_fail(e, "gemv launch");
}

int32_t bg_qkv_proj_prologue(bg_kv_cache* c, int32_t layer, const float* x, int32_t K, const uint32_t* sign,
                             const float* scales, int32_t H, const float* q_gamma, const float* k_gamma, float eps,
                             const float* cos_tab, const float* sin_tab, int32_t rope_positions, int32_t rot_dim,
                             int32_t pos, int32_t slot, float* q_out, void* stream) {
  if (!c) return fail(BG_E_INVALID, "bg_qkv_proj_prologue: NULL cache");
  int32_t rc = check_gemv("bg_qkv_proj_prologue", x, K, sign, scales);
  if (rc != BG_OK) return rc;
  if (layer < 0 || layer >= c->n_layers) return fail(BG_E_INVALID, "bg_qkv_proj_prologue: layer %d out of range", layer);
  if (H < c->kv_heads || H % c->kv_heads || H + 2 * c->kv_heads > kProjMaxHeads)
    return fail(BG_E_INVALID, "bg_qkv_proj_prologue: heads %d (kv_heads %d, at most %d heads in all)", H, c->kv_heads,
                kProjMaxHeads);
  if (!q_out || !q_gamma || !k_gamma || !cos_tab || !sin_tab)
    return fail(BG_E_INVALID, "bg_qkv_proj_prologue: NULL q_out, gamma or rope table");
  if (((uintptr_t)q_out | (uintptr_t)q_gamma | (uintptr_t)k_gamma | (uintptr_t)cos_tab | (uintptr_t)sin_tab) & 15)
    return fail(BG_E_INVALID, "bg_qkv_proj_prologue: buffers must be 16-byte aligned");
  if (rot_dim < 2 || (rot_dim & 1) || rot_dim > c->D) return fail(BG_E_INVALID, "bg_qkv_proj_prologue: bad rot_dim %d", rot_dim);
  if (pos < 0 || pos >= rope_positions)
    return fail(BG_E_INVALID, "bg_qkv_proj_prologue: position %d outside the %d-row rope table", pos, rope_positions);
  if (slot < 0 || slot >= addressable(c))
    return fail(BG_E_INVALID, "bg_qkv_proj_prologue: slot %d beyond capacity %d", slot, addressable(c));
  bg::QkvProjArgs a;
  a.x = x;
  a.K = K;
  a.sign = sign;
  a.scales = scales;
  a.H = H;
  a.q_gamma = q_gamma;
  a.k_gamma = k_gamma;
  a.eps = eps;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.rot_dim = rot_dim;
  a.pos = pos;
  a.slot = slot;
  a.q_out = q_out;
  a.raw = c->proj_raw;
  a.err = c->err_dev;
  a.spin_limit = g_merge_spin.load(std::memory_order_relaxed);
  const int xs = xcd_state(c->device);
  a.n_xcd = xs > 0 ? xs : 0;
  a.num_cus = c->num_cus;
  hipError_t e = bg::launch_qkv_proj(view(c, layer), a, (hipStream_t)stream);
  return e == hipSuccess ? BG_OK : hip_fail(e, "qkv projection launch");
}

int32_t bg_kv_evict(bg_kv_cache* c, int32_t fill, int32_t need, int32_t* new_fill) {
  if (!c || !new_fill) return fail(BG_E_INVALID, "bg_kv_evict: NULL argument");
  if (!c->roll) return fail(BG_E_STATE, "bg_kv_evict: cache is not in sink mode");
  if (fill < c->sinks || fill > c->max_seq) return fail(BG_E_INVALID, "bg_kv_evict: fill %d outside [%d, %d]", fill, c->sinks, c->max_seq);
  int32_t nf, batch, keep;
  int32_t rc = bg_evict_plan(fill, need, c->sinks, c->max_seq, &nf, &batch, &keep);
  if (rc != BG_OK) return rc;
  // rows [sinks+batch, sinks+batch+keep) become [sinks, sinks+keep): the ring origin moves by batch
  const int W = c->max_seq - c->sinks;
  c->head = (int)(((long)c->head + batch) % W);
  c->evicted += batch;
  *new_fill = nf;
  return BG_OK;
}

int32_t bg_kv_evict_for(bg_kv_cache* c, int32_t fill, int32_t n, int32_t* new_fill) {
  // evictFor, src/engine.ts:1214
  if (!c || !new_fill) return fail(BG_E_INVALID, "bg_kv_evict_for: NULL argument");
  if (c->roll && fill + n > c->max_seq) return bg_kv_evict(c, fill, fill + n - c->max_seq, new_fill);
  *new_fill = fill;
  return BG_OK;
}

int32_t bg_kv_ring_state(const bg_kv_cache* c, int32_t* head, int64_t* evicted) {
  if (!c || !head || !evicted) return fail(BG_E_INVALID, "bg_kv_ring_state: NULL argument");
  *head = c->head;
  *evicted = c->evicted;
  return BG_OK;
}

int32_t bg_decode_plan(int32_t kv_heads, int32_t head_dim, int32_t dtype, int32_t S, int32_t H, int32_t pos_base,
                       int32_t num_cus, int32_t resident_per_cu, int32_t* out) {
  if (!out || kv_heads < 1 || S < 1 || H < kv_heads || H % kv_heads || pos_base < 0 || num_cus < 1 ||
      resident_per_cu < 1 || (head_dim != 128 && head_dim != 256))
    return fail(BG_E_INVALID, "bg_decode_plan: bad arguments");
  LayerView L{};
  L.kv_heads = kv_heads;
  L.D = head_dim;
  L.dtype = dtype;
  L.cap = round32(pos_base + S);
  L.max_seq = L.cap;
  bg::DecodePlan p;
  if (!bg::decode_plan(L, S, H, pos_base, num_cus, resident_per_cu, &p))
    return fail(BG_E_UNSUPPORTED, "bg_decode_plan: the decode kernel does not take S %d, heads %d", S, H);
  out[0] = p.waves;
  out[1] = p.n_splits;
  out[2] = p.tiles_per_split;
  out[3] = p.n_mergers;
  out[4] = p.grid;
  out[5] = p.n_tiles;
  return BG_OK;
}

int32_t bg_diag_stream_read(const void* buf, size_t bytes, int32_t workgroups, int32_t nontemporal, uint32_t* sink,
                            void* stream) {
  if (!buf || !sink || bytes == 0 || bytes % 16 || workgroups < 1 || workgroups > 65535)
    return fail(BG_E_INVALID, "bg_diag_stream_read: bad arguments (bytes %zu, workgroups %d)", bytes, workgroups);
  const hipError_t e = bg::launch_stream_read(buf, bytes, workgroups, nontemporal != 0, sink, (hipStream_t)stream);
  return e == hipSuccess ? BG_OK : hip_fail(e, "bg_diag_stream_read");
}

int32_t bg_kv_ring_reset(bg_kv_cache* c, int64_t evicted) {
  if (!c) return fail(BG_E_INVALID, "bg_kv_ring_reset: NULL cache");
  if (!c->roll) return fail(BG_E_STATE, "bg_kv_ring_reset: cache is not in sink mode");
  if (evicted < 0) return fail(BG_E_INVALID, "bg_kv_ring_reset: evicted %lld < 0", (long long)evicted);
  c->head = 0;
  c->evicted = evicted;
  return BG_OK;
}

int32_t bg_kv_region_bytes(const bg_kv_cache* c, int32_t region, int32_t count, size_t* bytes) {
  if (!c || !bytes || count < 0) return fail(BG_E_INVALID, "bg_kv_region_bytes: bad arguments");
  if (region == BG_K || region == BG_V) {
    *bytes = (size_t)count * c->kv_heads * c->D * elem_bytes(c->dtype);
  } else if ((region == BG_KSCALE || region == BG_VSCALE) && c->dtype == BG_KV_Q8) {
    *bytes = (size_t)count * c->kv_heads * (c->D / 32) * sizeof(float);
  } else {
    return fail(BG_E_INVALID, "bg_kv_region_bytes: region %d not present in this storage mode", region);
  }
  return BG_OK;
}

static int32_t transfer(bg_kv_cache* c, int32_t layer, int32_t region, int32_t base, int32_t count, void* host,
                        bool import_, void* stream) {
  size_t bytes = 0;
  int32_t rc = bg_kv_region_bytes(c, region, count, &bytes);
  if (rc != BG_OK) return rc;
  if (!host && count > 0) return fail(BG_E_INVALID, "snapshot transfer: NULL host buffer");
  if (layer < 0 || layer >= c->n_layers) return fail(BG_E_INVALID, "snapshot transfer: layer %d out of range", layer);
  if (base < 0 || (long)base + count > addressable(c))
    return fail(BG_E_INVALID, "snapshot transfer: positions %d..%d beyond capacity %d", base, base + count - 1, addressable(c));
  if (count == 0) return BG_OK;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipSuccess;
  if (bytes > c->stage_bytes) {
    // wait for earlier transfers that use the old buffer, then grow it
    e = hipDeviceSynchronize();
    if (e == hipSuccess && c->stage) e = hipFree(c->stage);
    c->stage = nullptr;
    c->stage_bytes = 0;
    if (e == hipSuccess) e = hipMalloc(&c->stage, bytes);
    if (e != hipSuccess) return hip_fail(e, "snapshot staging allocation");
    c->stage_bytes = bytes;
  }
  void* dev = c->stage;
  LayerView L = view(c, layer);
  if (import_) {
    e = hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = bg::launch_kv_import(L, region, base, count, dev, st);
  } else {
    e = bg::launch_kv_export(L, region, base, count, dev, st);
    if (e == hipSuccess) e = hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, st);
  }
  if (e == hipSuccess) e = st ? hipStreamSynchronize(st) : hipDeviceSynchronize();
  return e == hipSuccess ? BG_OK : hip_fail(e, import_ ? "snapshot import" : "snapshot export");
}

int32_t bg_kv_export_rows(bg_kv_cache* c, int32_t layer, int32_t region, int32_t base, int32_t count, void* host,
                          void* stream) {
  if (!c) return fail(BG_E_INVALID, "bg_kv_export_rows: NULL cache");
  return transfer(c, layer, region, base, count, host, false, stream);
}

int32_t bg_kv_import_rows(bg_kv_cache* c, int32_t layer, int32_t region, int32_t base, int32_t count, const void* host,
                          void* stream) {
  if (!c) return fail(BG_E_INVALID, "bg_kv_import_rows: NULL cache");
  return transfer(c, layer, region, base, count, const_cast<void*>(host), true, stream);
}

}  // extern "C"
