// One head row held by one wave (D/64 consecutive values per lane): RMSNorm times gamma and
// rotate_half RoPE, in the reference's numpy forms -- y = (x / sqrt(mean(x^2) + eps)) * gamma
// (tools/reference.py:107) and y*cos + rot*sin as two rounded products and a rounded sum
// (tools/reference.py:149-152; shaders/rmsnorm_rope_sg.wgsl:32), no FMA contraction. Shared by
// the fused prologue and the fused decode step so both produce the same bits.
#pragma once

#include "bg_kernels.h"

namespace bg {

// cos / sin table entries of this lane's dims at table row p (dims >= rot: 0, unused)
template <int D>
__device__ inline void rope_entries(const float* cos_tab, const float* sin_tab, int p, int rot, bool on,
                                    float (&cs)[D / 64], float (&sn)[D / 64], int lane) {
  constexpr int EPL = D / 64;
  const int half = rot >> 1;
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    const int d = lane * EPL + e;
    const int ti = d < rot ? (d < half ? d : d - half) : 0;
    cs[e] = on ? cos_tab[(size_t)p * half + ti] : 0.0f;
    sn[e] = on ? sin_tab[(size_t)p * half + ti] : 0.0f;
  }
}

// v <- RMSNorm(v) * gamma, then (rope) rotate dims < rot; the rotate_half partner (d +- rot/2)
// is read back through `row`, this wave's own D floats of LDS (no workgroup barrier)
template <int D>
__device__ inline void rmsnorm_rope_wave(float (&v)[D / 64], const float* gamma, float eps, bool rope, int rot,
                                         const float (&cs)[D / 64], const float (&sn)[D / 64], float* row, int lane) {
  constexpr int EPL = D / 64;
  const int d0 = lane * EPL;
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < EPL; e++) ss = __fadd_rn(ss, __fmul_rn(v[e], v[e]));
  ss = wave_sum(ss);
  const float rms = __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps));
#pragma unroll
  for (int e = 0; e < EPL; e++) v[e] = __fmul_rn(__fdiv_rn(v[e], rms), gamma[d0 + e]);
  if (rope) {
    const int half = rot >> 1;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // earlier partner reads of `row` are done
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int e = 0; e < EPL; e++) row[d0 + e] = v[e];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const int d = d0 + e;
      if (d < rot) {
        const float rv = d < half ? -row[d + half] : row[d - half];
        v[e] = __fadd_rn(__fmul_rn(v[e], cs[e]), __fmul_rn(rv, sn[e]));
      }
    }
  }
}

}  // namespace bg
