// KV-cache append (the copy / copy_kv16 / copy_kv8 equivalents) and the snapshot-layout
// export/import gathers.
//
// kv_write: one wave per cache row of D values. Lane l owns D/64 consecutive values, so a q8
// block of 32 values is held by 32/(D/64) adjacent lanes and its absolute maximum is a
// shuffle reduction inside that lane group (shaders/copy_kv8.wgsl:25-36 does the same with a
// shared-memory pass). Rows follow the reference's cache-row numbering (src/engine.ts:1385-1393):
// reference row R = position * KV + kv_head.
#include "bg_kernels.h"
#include "bg_store.h"

namespace bg {

template <int D, int DT>
__global__ __launch_bounds__(64) void kv_write_kernel(LayerView L, int which, const float* __restrict__ src,
                                                      int rows, int dst_row0) {
  constexpr int EPL = D / 64;               // values per lane
  const int r = blockIdx.x;
  if (r >= rows) return;
  const int lane = threadIdx.x;
  const int R = dst_row0 + r;
  const int pos = R / L.kv_heads, kvh = R % L.kv_heads;
  const float* x = src + (size_t)r * D + lane * EPL;
  float v[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) v[e] = x[e];
  store_row<D, DT>(L, which, L.ring.phys(pos), kvh, v, lane);
}

template <int D>
static hipError_t kv_write_d(const LayerView& L, int which, const float* src, int rows, int dst_row0, hipStream_t st) {
  dim3 g(rows), b(64);
  switch (L.dtype) {
    case KV_F32: hipLaunchKernelGGL((kv_write_kernel<D, KV_F32>), g, b, 0, st, L, which, src, rows, dst_row0); break;
    case KV_F16: hipLaunchKernelGGL((kv_write_kernel<D, KV_F16>), g, b, 0, st, L, which, src, rows, dst_row0); break;
    default: hipLaunchKernelGGL((kv_write_kernel<D, KV_Q8>), g, b, 0, st, L, which, src, rows, dst_row0); break;
  }
  return hipGetLastError();
}

hipError_t launch_kv_write(const LayerView& L, int which, const float* src, int rows, int dst_row0, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  // head_dim is 128 or 256 (bg_kv_create rejects the rest)
  switch (L.D) {
    case 128: return kv_write_d<128>(L, which, src, rows, dst_row0, st);
    default: return kv_write_d<256>(L, which, src, rows, dst_row0, st);
  }
}

// ---- snapshot layout gathers: region element e of [count, KV, n] in reference order ----------
// region 0/1: K/V elements (f32 / f16 bits / int8 codes); 2/3: K/V block scales.
__global__ void kv_export_kernel(LayerView L, int region, int base, int count, void* __restrict__ dst, int import_) {
  const int D = L.D;
  const int n = region < 2 ? D : D / kBlock;
  const size_t total = (size_t)count * L.kv_heads * n;
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
    const int i = (int)(e % n);
    const size_t rowi = e / n;
    const int kvh = (int)(rowi % L.kv_heads);
    const int pos = base + (int)(rowi / L.kv_heads);
    const int slot = L.ring.phys(pos);
    if (region >= 2) {
      float* sc = region == 2 ? L.ks : L.vs;
      size_t off = scale_offset(kvh, slot, i, L.cap, D);
      if (import_) sc[off] = ((const float*)dst)[e];
      else ((float*)dst)[e] = sc[off];
      continue;
    }
    size_t off = region == 0 ? k_offset(kvh, slot, i, L.cap, D) : v_offset(kvh, slot, i, L.cap, D);
    void* buf = region == 0 ? L.k : L.v;
    if (L.dtype == KV_F32) {
      if (import_) ((float*)buf)[off] = ((const float*)dst)[e];
      else ((float*)dst)[e] = ((const float*)buf)[off];
    } else if (L.dtype == KV_F16) {
      if (import_) ((uint16_t*)buf)[off] = ((const uint16_t*)dst)[e];
      else ((uint16_t*)dst)[e] = ((const uint16_t*)buf)[off];
    } else {
      if (import_) ((int8_t*)buf)[off] = ((const int8_t*)dst)[e];
      else ((int8_t*)dst)[e] = ((const int8_t*)buf)[off];
    }
  }
}

hipError_t launch_kv_export(const LayerView& L, int region, int base, int count, void* dst, hipStream_t st) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(kv_export_kernel, dim3(1024), dim3(256), 0, st, L, region, base, count, dst, 0);
  return hipGetLastError();
}
hipError_t launch_kv_import(const LayerView& L, int region, int base, int count, const void* src, hipStream_t st) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(kv_export_kernel, dim3(1024), dim3(256), 0, st, L, region, base, count, const_cast<void*>(src), 1);
  return hipGetLastError();
}

// ---- q8 -> f16 copy of the attended slots, for a long prefill ---------------------------------
// A q8 prefill stages (dequantizes) every K/V tile once per query block that attends it. For a
// long prompt the attended slots are dequantized once here into an f16 copy laid out like an f16
// cache (K row-major, V in 32-slot transposed tiles), and the prefill runs its direct-to-LDS f16
// path on that copy. The values are exactly the ones the q8 staging produces: the code, biased
// to u = code + 128, times s = scale * (1/127) in one f32 fma (u * s - 128 * s), then RNE to f16
// (q8_stage_f16).

template <int D>
__global__ __launch_bounds__(256) void kv_dequant_kernel(LayerView L, int n_slots, __half* __restrict__ kdst,
                                                         __half* __restrict__ vdst) {
  constexpr int NB = D / kBlock;
  const size_t per_head = (size_t)n_slots * D / 16;  // 16-value chunks of K (and of V) per kv head
  const size_t total = per_head * L.kv_heads;
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < 2 * total; c += (size_t)gridDim.x * blockDim.x) {
    const bool isv = c >= total;
    const size_t cc = isv ? c - total : c;
    const int kvh = (int)(cc / per_head);
    const size_t e0 = (cc % per_head) * 16;  // element offset inside the kv head's region
    const size_t base = (size_t)kvh * L.cap * D;
    const uint4 w = *(const uint4*)((const int8_t*)(isv ? L.v : L.k) + base + e0);
    const uint32_t ww[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u, w.w ^ 0x80808080u};
    _Float16 o[16];
    if (!isv) {
      const int slot = (int)(e0 / D), d0 = (int)(e0 % D);
      const float s = L.ks[((size_t)kvh * L.cap + slot) * NB + d0 / kBlock] * (1.0f / 127.0f);
#pragma unroll
      for (int i = 0; i < 16; i++) o[i] = q8_stage_f16((ww[i >> 2] >> (8 * (i & 3))) & 0xffu, s);
      uint4* dst = (uint4*)(kdst + base + e0);
      dst[0] = *(const uint4*)&o[0];
      dst[1] = *(const uint4*)&o[8];
    } else {
      // 16 bytes of a V tile = 2 dims x the 8 slots of one panel
      const int t = (int)(e0 / ((size_t)kTile * D));
      const int wi = (int)(e0 % ((size_t)kTile * D));
      const int panel = wi / (8 * D), d0 = (wi % (8 * D)) / 8;
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int d = d0 + h;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int slot = t * kTile + tile_slot(panel, e);
          const float s = L.vs[((size_t)kvh * L.cap + slot) * NB + d / kBlock] * (1.0f / 127.0f);
          const int i = 8 * h + e;
          o[i] = q8_stage_f16((ww[i >> 2] >> (8 * (i & 3))) & 0xffu, s);
        }
      }
      uint4* dst = (uint4*)(vdst + base + e0);
      dst[0] = *(const uint4*)&o[0];
      dst[1] = *(const uint4*)&o[8];
    }
  }
}

hipError_t launch_kv_dequant_f16(const LayerView& L, int n_slots, void* kdst, void* vdst, hipStream_t st) {
  if (L.dtype != KV_Q8 || n_slots <= 0 || n_slots % kTile || n_slots > L.cap) return hipErrorInvalidValue;
  const size_t chunks = 2 * (size_t)n_slots * L.D / 16 * L.kv_heads;
  const int grid = (int)((chunks + 255) / 256 < 4096 ? (chunks + 255) / 256 : 4096);
  switch (L.D) {
    case 128: hipLaunchKernelGGL((kv_dequant_kernel<128>), dim3(grid), dim3(256), 0, st, L, n_slots, (__half*)kdst, (__half*)vdst); break;
    default: hipLaunchKernelGGL((kv_dequant_kernel<256>), dim3(grid), dim3(256), 0, st, L, n_slots, (__half*)kdst, (__half*)vdst); break;
  }
  return hipGetLastError();
}

}  // namespace bg
