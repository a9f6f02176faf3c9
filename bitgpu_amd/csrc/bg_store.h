// Storing one cache row (D values spread D/64 per lane over a wave) in the storage mode's
// format: f32 copy (shaders/copy.wgsl), f16 RNE (shaders/copy_kv16.wgsl:13) or q8 codes with
// one f32 scale per 32 values (shaders/copy_kv8.wgsl:24-40).
#pragma once

#include "bg_kernels.h"

namespace bg {

template <int D, int DT>
__device__ inline void store_row(const LayerView& L, int which, int slot, int kvh, const float (&v)[D / 64], int lane) {
  constexpr int EPL = D / 64;
  const int d0 = lane * EPL;
  if constexpr (DT == KV_Q8) {
    constexpr int LPB = kBlock / EPL;  // lanes per q8 block
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) m = fmaxf(m, fabsf(v[e]));
    m = group_max<LPB>(m);
    if (L.q8_row) m = wave_max(m);  // per-row scale: the row's 64 lanes
    const float s = q8_scale_of(m);
    float* sc = which == 0 ? L.ks : L.vs;
    if ((lane % LPB) == 0) sc[scale_offset(kvh, slot, d0 / kBlock, L.cap, D)] = s;
    int8_t* base = (int8_t*)(which == 0 ? L.k : L.v);
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const int8_t c = (int8_t)q8_code(v[e], s);
      const size_t off = which == 0 ? k_offset(kvh, slot, d0 + e, L.cap, D) : v_offset(kvh, slot, d0 + e, L.cap, D);
      base[off] = c;
    }
  } else if constexpr (DT == KV_F16) {
    __half* base = (__half*)(which == 0 ? L.k : L.v);
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const size_t off = which == 0 ? k_offset(kvh, slot, d0 + e, L.cap, D) : v_offset(kvh, slot, d0 + e, L.cap, D);
      base[off] = __float2half_rn(v[e]);
    }
  } else {
    float* base = (float*)(which == 0 ? L.k : L.v);
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const size_t off = which == 0 ? k_offset(kvh, slot, d0 + e, L.cap, D) : v_offset(kvh, slot, d0 + e, L.cap, D);
      base[off] = v[e];
    }
  }
}

}  // namespace bg
