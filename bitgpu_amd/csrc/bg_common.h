// Shared device/host definitions of the MI355X attention library: storage layout of the KV
// cache, the sink-mode ring map and small wave64 helpers. Included by every .hip file.
//
// KV cache layout (per layer; "slot" = physical position row):
//   K   : [kv_head][cap][D]                 row-major, element type of the storage mode
//   V   : [kv_head][cap/32][4 panels][D][8]  32-slot tiles stored transposed: panel p of a
//                                             tile holds, for every dim, 8 slots contiguously
//   Ks,Vs (q8): [kv_head][cap][D/32] f32     one scale per 32-value block
// The V tile order puts the 8 slots one MFMA lane group reduces over next to each other, so
// both the decode and the prefill P.V products load their operand with one contiguous 16/32 B
// read per lane instead of a gather. Slot j of a tile lives in panel (2*(j/16) + (j%8)/4) at
// index (4*((j%16)/8) + j%4). cap is a multiple of 32.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace bg {

enum KvType : int { KV_F32 = 0, KV_F16 = 1, KV_Q8 = 2 };

constexpr int kTile = 32;   // slots per V tile
constexpr int kBlock = 32;  // q8 values per scale

__host__ __device__ inline int kv_elem_bytes(int dtype) { return dtype == KV_F32 ? 4 : dtype == KV_F16 ? 2 : 1; }

// slot-in-tile -> (panel, index within the 8-slot panel row) and back
__host__ __device__ inline int tile_panel(int j) { return 2 * (j >> 4) + ((j & 7) >> 2); }
__host__ __device__ inline int tile_index(int j) { return 4 * ((j & 15) >> 3) + (j & 3); }
__host__ __device__ inline int tile_slot(int p, int i) { return 16 * (p >> 1) + 8 * (i >> 2) + 4 * (p & 1) + (i & 3); }

// element offset of V[kvh][slot][d] inside one layer's V buffer
__host__ __device__ inline size_t v_offset(int kvh, int slot, int d, int cap, int D) {
  int t = slot >> 5, j = slot & 31;
  return ((size_t)kvh * cap + (size_t)t * kTile) * D + (size_t)tile_panel(j) * (8 * D) + (size_t)d * 8 + tile_index(j);
}
__host__ __device__ inline size_t k_offset(int kvh, int slot, int d, int cap, int D) {
  return ((size_t)kvh * cap + slot) * D + d;
}
__host__ __device__ inline size_t scale_offset(int kvh, int slot, int b, int cap, int D) {
  return ((size_t)kvh * cap + slot) * (D / kBlock) + b;
}

// Sink-mode ring: logical slots [0, sinks) are fixed; logical slots >= sinks live in a ring of
// W = max_seq - sinks physical slots whose origin advances by each eviction batch.
struct Ring {
  int roll;     // 0: logical == physical
  int sinks;
  int W;        // ring size
  int head;     // ring origin, in [0, W)
  __host__ __device__ inline int phys(int L) const {
    if (!roll || L < sinks) return L;
    int r = L - sinks + head;
    r = r >= W ? r - W : r;
    return sinks + r;
  }
  __host__ __device__ inline int logical(int P) const {
    if (!roll || P < sinks) return P;
    int r = P - sinks - head;
    r = r < 0 ? r + W : r;
    return sinks + r;
  }
};

// ---- q8 pack: WGSL pack4x8snorm on a block-scaled value (shaders/copy_kv8.wgsl:24-40) ----
// code = floor(0.5 + 127 * clamp(v / s, -1, 1)); explicit _rn intrinsics keep every step one
// IEEE rounding (no contraction into an FMA, correctly rounded division).
__device__ inline int q8_code(float v, float s) {
  float e = __fdiv_rn(v, s);
  e = fminf(fmaxf(e, -1.0f), 1.0f);
  float t = __fadd_rn(__fmul_rn(127.0f, e), 0.5f);
  return (int)floorf(t);
}
__device__ inline float q8_scale_of(float absmax) { return fmaxf(absmax, 1e-30f); }

// ---- wave64 reductions (DPP/permute via the compiler's cross-lane builtins) ----
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// reduce over the 16 lanes of a lane group (lanes 16g .. 16g+15)
__device__ inline float group16_max(float v) {
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ inline float group16_sum(float v) {
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Split partials travel between workgroups (possibly on different XCDs, whose L2s are not
// coherent) as relaxed agent-scope atomics: the stores write through (sc1) and the loads read
// coherently, so no L2 writeback fence is needed; the writer waits for its stores
// (vmcnt(0)) before taking the ticket.
__device__ inline void st_coherent(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline float ld_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_coherent2(float* p, float a, float b) {
  union { float f[2]; uint64_t u; } x;
  x.f[0] = a;
  x.f[1] = b;
  __hip_atomic_store((uint64_t*)p, x.u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float2 ld_coherent2(const float* p) {
  union { float f[2]; uint64_t u; } x;
  x.u = __hip_atomic_load((uint64_t*)const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(x.f[0], x.f[1]);
}
__device__ inline void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace bg
