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

// One IEEE-rounded product / sum that is never fused into an fma with its neighbour. The library
// is compiled with contraction on (hipcc's default), and __fmul_rn / __fadd_rn are plain
// operators in this toolchain, so a * b + c through them still becomes one fma; contraction is
// off inside these two.
__device__ inline float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ inline float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// ---- q8 pack: WGSL pack4x8snorm on a block-scaled value (shaders/copy_kv8.wgsl:24-40) ----
// code = floor(0.5 + 127 * clamp(v / s, -1, 1)), every step one IEEE rounding (a correctly
// rounded division; the product and the sum not fused).
__device__ inline int q8_code(float v, float s) {
  float e = __fdiv_rn(v, s);
  e = fminf(fmaxf(e, -1.0f), 1.0f);
  float t = add_rn(mul_rn(127.0f, e), 0.5f);
  return (int)floorf(t);
}
__device__ inline float q8_scale_of(float absmax) { return fmaxf(absmax, 1e-30f); }

// q8 -> f16 MFMA operand, the one definition shared by the prefill staging and the prefill's f16
// copy: u = code + 128 (the biased byte), s = scale * (1/127) in f32, the f32 fma u*s - 128*s
// (one rounding of code * s), then RNE to f16. The f32 value is pinned so the compiler cannot
// fuse the fma and the conversion into a mixed-precision fma (one rounding instead of two),
// which it does for some call sites and not others.
__device__ inline float q8_stage_f32(uint32_t u, float s) {
  float a = fmaf((float)u, s, -128.0f * s);
  asm("" : "+v"(a));
  return a;
}
__device__ inline _Float16 q8_stage_f16(uint32_t u, float s) { return (_Float16)q8_stage_f32(u, s); }

// ---- cross-lane exchange and reductions, all in the VALU (no LDS round trip) ----
// Inside a 16-lane row: DPP quad_perm [1,0,3,2] and [2,3,0,1] pair lanes i^1 and i^2; once a
// quad holds one value, row_half_mirror (lane 7-i of each 8) and then row_mirror (lane 15-i)
// pair it with the other quad and the other half. Across rows: v_permlane16_swap swaps the odd
// rows of its first operand with the even rows of its second, v_permlane32_swap the upper half
// of the first with the lower half of the second; swapping a value with itself leaves the two
// results holding x[l] and x[l ^ 16] (or x[l ^ 32]) in some order.
template <int CTRL>
__device__ inline float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
// {x[l], x[l^16]} and {x[l], x[l^32]} as an unordered pair
__device__ inline float2 pair16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float2 pair32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// x[l ^ 32] (the other half of the wave)
__device__ inline float xor32(float v) {
  const float2 r = pair32(v);
  return (__lane_id() < 32) ? r.y : r.x;
}
// reduce over aligned groups of N lanes (N = 2, 4, 8, 16, 32, 64); every lane of a group gets
// the same bits
template <int N>
__device__ inline float group_max(float v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "group size");
  v = fmaxf(v, dpp_mov<kDppXor1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp_mov<kDppXor2>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp_mov<kDppMirror>(v));
  if constexpr (N >= 32) { const float2 r = pair16(v); v = fmaxf(r.x, r.y); }
  if constexpr (N >= 64) { const float2 r = pair32(v); v = fmaxf(r.x, r.y); }
  return v;
}
template <int N>
__device__ inline float group_sum(float v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "group size");
  v += dpp_mov<kDppXor1>(v);
  if constexpr (N >= 4) v += dpp_mov<kDppXor2>(v);
  if constexpr (N >= 8) v += dpp_mov<kDppHalfMirror>(v);
  if constexpr (N >= 16) v += dpp_mov<kDppMirror>(v);
  if constexpr (N >= 32) { const float2 r = pair16(v); v = r.x + r.y; }
  if constexpr (N >= 64) { const float2 r = pair32(v); v = r.x + r.y; }
  return v;
}
__device__ inline float wave_sum(float v) { return group_sum<64>(v); }
__device__ inline float wave_max(float v) { return group_max<64>(v); }
// reduce over the 16 lanes of a lane group (lanes 16g .. 16g+15)
__device__ inline float group16_max(float v) { return group_max<16>(v); }
__device__ inline float group16_sum(float v) { return group_sum<16>(v); }

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

// the XCD (accelerator complex die) this wave runs on: hardware register XCC_ID, bits 3:0
__device__ inline int xcc_id() {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return (int)(x & 0xf);
}

// Streaming (nontemporal) vector stores of data no kernel re-reads soon from the cache hierarchy:
// a device copy moves 6.2 TB/s read + write with them against 5.4 TB/s with plain stores.
__device__ inline void st_stream16(void* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(u4{a, b, c, d}, (u4*)p);
}
__device__ inline void st_stream16f(void* p, float a, float b, float c, float d) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(f4{a, b, c, d}, (f4*)p);
}
__device__ inline void st_stream8(void* p, uint32_t a, uint32_t b) {
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store(u2{a, b}, (u2*)p);
}
__device__ inline void st_stream4(void* p, uint32_t a) { __builtin_nontemporal_store(a, (uint32_t*)p); }

}  // namespace bg
