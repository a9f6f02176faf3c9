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
  switch (L.D) {
    case 64: return kv_write_d<64>(L, which, src, rows, dst_row0, st);
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

}  // namespace bg
