// Exact-f32 causal GQA attention over an f32 KV cache (kvCache 'f32', the reference default).
//
// Replaces attention_sg.wgsl / attention_wg.wgsl / attention_sg_roll.wgsl and the f32
// attention_online_cache.wgsl. All arithmetic is f32 (no f16 operands), so it meets the
// reference's max-abs 1e-4 bar for f32 storage. One wave per (query row, head); per 64-slot
// tile each lane scores one slot with a full f32 dot product (Q broadcast from LDS), the wave
// does one online-softmax update, then each lane accumulates D/64 output dims from the
// transposed V tile. Sink mode rotates each key at read by its logical (or absolute) position
// exactly as attention_sg_roll.wgsl:40-51 (k*cos + rot*sin).
#include "bg_kernels.h"

namespace bg {

template <int D, bool ROLL>
__global__ __launch_bounds__(64) void attn_f32_kernel(LayerView L, AttnArgs a, int n_scan, int phys_limit) {
  constexpr int EPL = D / 64;
  __shared__ float qsh[D];
  __shared__ float psh[64];
  const int lane = threadIdx.x;
  const int row = blockIdx.x;  // s * H + h
  const int s = row / a.H, h = row % a.H;
  const int G = a.H / L.kv_heads;
  const int kvh = h / G;
  const float* qr = a.q + (size_t)row * D;
#pragma unroll
  for (int e = 0; e < EPL; e++) qsh[lane + 64 * e] = qr[lane + 64 * e];
  __syncthreads();
  const float* K = (const float*)L.k;
  const float* V = (const float*)L.v;
  const int limit = a.pos_base + s;
  float m = -1e30f, l = 0.0f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) acc[e] = 0.0f;

  for (int j0 = 0; j0 < n_scan; j0 += 64) {
    const int P = j0 + lane;
    const int Lg = L.ring.logical(P);
    const bool ok = P < n_scan && P < phys_limit && Lg <= limit;
    float sc = -INFINITY;
    if (ok) {
      const float* kr = K + k_offset(kvh, P, 0, L.cap, D);
      float dot = 0.0f;
      if constexpr (ROLL) {
        long ri = (L.rope_abs && Lg >= L.ring.sinks) ? (long)Lg + L.evicted : (long)Lg;
        ri = ri < L.rope_positions ? ri : 0;
        const float* ct = L.cos_tab + (size_t)ri * (D / 2);
        const float* st = L.sin_tab + (size_t)ri * (D / 2);
        for (int d = 0; d < D; d++) {
          const int i = d < D / 2 ? d : d - D / 2;
          const float rv = d < D / 2 ? -kr[d + D / 2] : kr[d - D / 2];
          const float kd = __fadd_rn(__fmul_rn(kr[d], ct[i]), __fmul_rn(rv, st[i]));
          dot = fmaf(qsh[d], kd, dot);
        }
      } else {
        for (int d = 0; d < D; d++) dot = fmaf(qsh[d], kr[d], dot);
      }
      sc = dot * a.scale;
    }
    const float mt = wave_max(sc);
    const float mn = fmaxf(m, mt);
    const float corr = expf(m - mn);
    const float pj = ok ? expf(sc - mn) : 0.0f;
    l = l * corr + wave_sum(pj);
    m = mn;
    psh[lane] = pj;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[e] *= corr;
    const int jn = min(64, n_scan - j0);
    for (int j = 0; j < jn; j++) {
      const float pv = psh[j];
      if (pv != 0.0f) {
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[e] = fmaf(pv, V[v_offset(kvh, j0 + j, lane + 64 * e, L.cap, D)], acc[e]);
      }
    }
    __syncthreads();
  }
  float* o = a.out + (size_t)row * D;
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    const int d = lane + 64 * e;
    float r = acc[e] / l;
    if (a.gate) r = r / (1.0f + expf(-a.gate[(size_t)row * a.gate_stride + d]));
    o[d] = r;
  }
}

hipError_t launch_attention_f32(const LayerView& L, const AttnArgs& a, hipStream_t st) {
  const int n_scan = (L.ring.roll && L.ring.head != 0) ? L.max_seq : a.pos_base + a.S;
  const int phys_limit = L.ring.roll ? L.max_seq : L.cap;
  dim3 g(a.S * a.H), b(64);
  const bool roll = L.ring.roll != 0;
  if (L.D == 128) {
    if (roll) hipLaunchKernelGGL((attn_f32_kernel<128, true>), g, b, 0, st, L, a, n_scan, phys_limit);
    else hipLaunchKernelGGL((attn_f32_kernel<128, false>), g, b, 0, st, L, a, n_scan, phys_limit);
  } else {
    if (roll) hipLaunchKernelGGL((attn_f32_kernel<256, true>), g, b, 0, st, L, a, n_scan, phys_limit);
    else hipLaunchKernelGGL((attn_f32_kernel<256, false>), g, b, 0, st, L, a, n_scan, phys_limit);
  }
  return hipGetLastError();
}

}  // namespace bg
