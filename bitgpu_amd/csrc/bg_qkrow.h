// A Q/K head row spread over D/4 lanes, 4 consecutive dims (16 bytes) a lane: the RMSNorm, the
// rotate_half RoPE and the K-cache store, shared by the fused prologue and the fused decode
// projection so both produce the same bits for the same row.
//
// Arithmetic follows the reference kernels: y = x * inverseSqrt(sum(x^2) / D + eps) * gamma as
// two rounded products (shaders/rmsnorm_rope_sg.wgsl:24,28) and y*cos + rot*sin as two rounded
// products and a rounded sum (tools/reference.py:149-152; shaders/rmsnorm_rope_sg.wgsl:32), none
// of them fused into an fma (mul_rn / add_rn).
// The rotate_half partner of a lane's dims is lane l ^ (rot / 8) of the row (a lane exchange)
// when that is 8, 16 or 32 lanes, else it is read back from the row staged in LDS.
#pragma once

#include "bg_kernels.h"

namespace bg {

// 1 / sqrt(mean(x^2) + eps) of a row whose D values sit 4 a lane over LPR adjacent lanes
template <int D, int LPR>
__device__ inline float row_inv_rms(const float (&x)[4], float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; e++) ss = add_rn(ss, mul_rn(x[e], x[e]));
  ss = group_sum<LPR>(ss);
  // ss / D is exact as a product: D is a power of two
  return rsqrtf(add_rn(ss * (1.0f / D), eps));
}

__device__ inline void row_scale(float (&x)[4], float inv, const float (&g)[4]) {
#pragma unroll
  for (int e = 0; e < 4; e++) x[e] = mul_rn(mul_rn(x[e], inv), g[e]);
}

// The rotate_half partners of this lane's dims (x[d + half] below half, x[d - half] above) by a
// lane exchange: lane l ^ half/4 holds them when half is a multiple of 4 and half/4 is
// 8 (DPP row_ror:8 inside a 16-lane row), 16 (v_permlane16_swap) or 32 lanes (v_permlane32_swap);
// false for other widths. Every lane of the wave must take part (rot is wave-uniform); rows are
// aligned to their D/4 lanes, so the partner lies in the same row.
constexpr int kDppRor8 = 0x128;
__device__ inline bool rope_partner_lanes(const float (&x)[4], int rot, float (&p)[4]) {
  const int half = rot >> 1;
  if ((half & 3) != 0) return false;
  const int h4 = half >> 2;
  if (h4 == 16) {
    const bool odd = (__lane_id() & 16) != 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float2 r = pair16(x[e]);
      p[e] = odd ? r.x : r.y;
    }
    return true;
  }
  if (h4 == 32) {
#pragma unroll
    for (int e = 0; e < 4; e++) p[e] = xor32(x[e]);
    return true;
  }
  if (h4 == 8) {
#pragma unroll
    for (int e = 0; e < 4; e++) p[e] = dpp_mov<kDppRor8>(x[e]);
    return true;
  }
  return false;
}

// Rotate this lane's dims 4c..4c+3 (< rot) with the partners p from rope_partner_lanes: the
// rotate_half value is -p (d < half) or p
__device__ inline void row_rope_lanes(float (&x)[4], const float (&p)[4], int c, int rot, const float (&cs)[4],
                                      const float (&sn)[4]) {
  const int half = rot >> 1;
  if (4 * c >= rot) return;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float rv = 4 * c < half ? -p[e] : p[e];
    x[e] = add_rn(mul_rn(x[e], cs[e]), mul_rn(rv, sn[e]));
  }
}

// Rotate this lane's dims 4c..4c+3 (< rot); `row` is the normed row in LDS, which supplies the
// rotate_half partner -x[d + half] (d < half) or x[d - half]
__device__ inline void row_rope(float (&x)[4], const float* row, int c, int rot, const float (&cs)[4],
                                const float (&sn)[4]) {
  const int half = rot >> 1;
  if (4 * c >= rot) return;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int d = 4 * c + e;
    if (d < rot) {
      const float rv = d < half ? -row[d + half] : row[d - half];
      x[e] = add_rn(mul_rn(x[e], cs[e]), mul_rn(rv, sn[e]));
    }
  }
}

// cos / sin entries of dims 4c..4c+3 at table row p (zeros past rot)
__device__ inline void row_tables(const float* cos_tab, const float* sin_tab, int p, int rot, int c, float (&cs)[4],
                                  float (&sn)[4]) {
  const int half = rot >> 1;
  const size_t prow = (size_t)p * half;
  if ((half & 3) == 0 && 4 * c < rot) {
    const int ti = 4 * c < half ? 4 * c : 4 * c - half;
    const float4 c4 = *(const float4*)(cos_tab + prow + ti), s4 = *(const float4*)(sin_tab + prow + ti);
    cs[0] = c4.x; cs[1] = c4.y; cs[2] = c4.z; cs[3] = c4.w;
    sn[0] = s4.x; sn[1] = s4.y; sn[2] = s4.z; sn[3] = s4.w;
    return;
  }
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int d = 4 * c + e;
    const int ti = d < half ? d : d - half;
    cs[e] = d < rot ? cos_tab[prow + ti] : 0.0f;
    sn[e] = d < rot ? sin_tab[prow + ti] : 0.0f;
  }
}

__device__ inline void load4(const float* p, float (&v)[4]) {
  const float4 f = *(const float4*)p;
  v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
}

// Store one K row (4 dims a lane, lanes c = 0 .. D/4-1) in the storage format: f32 / f16 as one
// vector store a lane, q8 as the lane's four codes in one word plus the block scale (32 dims =
// 8 lanes; in per-row mode the row maximum, in every block's slot) from the block's first lane.
template <int D, int DT>
__device__ inline void store_k4(const LayerView& L, int slot, int kvh, const float (&y)[4], int c) {
  const size_t off = k_offset(kvh, slot, 4 * c, L.cap, D);
  if constexpr (DT == KV_Q8) {
    float m = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
    m = group_max<kBlock / 4>(m);
    if (L.q8_row) m = group_max<D / 4>(m);
    const float sc = q8_scale_of(m);
    if ((c % (kBlock / 4)) == 0) L.ks[scale_offset(kvh, slot, (4 * c) / kBlock, L.cap, D)] = sc;
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) w |= (uint32_t)(uint8_t)(int8_t)q8_code(y[e], sc) << (8 * e);
    st_stream4((int8_t*)L.k + off, w);
  } else if constexpr (DT == KV_F16) {
    union { __half h[4]; uint2 u; } o;
#pragma unroll
    for (int e = 0; e < 4; e++) o.h[e] = __float2half_rn(y[e]);
    st_stream8((__half*)L.k + off, o.u.x, o.u.y);
  } else {
    st_stream16f((float*)L.k + off, y[0], y[1], y[2], y[3]);
  }
}

// Store one V row (4 dims a lane) into its slot of the transposed V tile: one element store per
// dim (the row's dims are 8 values apart), q8 scale per 32 dims as for K.
template <int D, int DT>
__device__ inline void store_v4(const LayerView& L, int slot, int kvh, const float (&y)[4], int c) {
  if constexpr (DT == KV_Q8) {
    float m = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
    m = group_max<kBlock / 4>(m);
    if (L.q8_row) m = group_max<D / 4>(m);
    const float sc = q8_scale_of(m);
    if ((c % (kBlock / 4)) == 0) L.vs[scale_offset(kvh, slot, (4 * c) / kBlock, L.cap, D)] = sc;
#pragma unroll
    for (int e = 0; e < 4; e++) ((int8_t*)L.v)[v_offset(kvh, slot, 4 * c + e, L.cap, D)] = (int8_t)q8_code(y[e], sc);
  } else if constexpr (DT == KV_F16) {
#pragma unroll
    for (int e = 0; e < 4; e++) ((__half*)L.v)[v_offset(kvh, slot, 4 * c + e, L.cap, D)] = __float2half_rn(y[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++) ((float*)L.v)[v_offset(kvh, slot, 4 * c + e, L.cap, D)] = y[e];
  }
}

}  // namespace bg
