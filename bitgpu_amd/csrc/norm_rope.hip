// Fused attention prologue: per-head RMSNorm + RoPE for Q (to an f32 buffer) and K (straight
// into the KV cache in its storage format), plus the V append, for S positions in one launch.
//
// Replaces rmsnorm_rope_sg{,_kv16,_kv8}.wgsl (decode), rmsnorm_sg + rope + copy* (prefill) and
// split_head + rmsnorm + rope_partial + copy* (hybrid) of the reference (src/engine.ts:1527-1540,
// 1569-1576, 1470-1485). One wave per head row; lane l owns D/64 consecutive values; the
// sum of squares is a wave reduction and the rotate_half partner (d +- rot/2) is read back
// through LDS, so any rot_dim (full or partial) works with one code path.
//
// Arithmetic follows the reference's numpy forms: y = (x / sqrt(mean(x^2) + eps)) * gamma
// (tools/reference.py:107) and y*cos + rot*sin as two rounded products and a rounded sum
// (tools/reference.py:149-152; shaders/rmsnorm_rope_sg.wgsl:32), no FMA contraction.
#include "bg_kernels.h"
#include "bg_store.h"

namespace bg {

template <int D, int DT>
__global__ __launch_bounds__(64) void qkv_prologue_kernel(LayerView L, PrologueArgs a, int rope_k) {
  constexpr int EPL = D / 64;
  __shared__ float row[D];
  const int lane = threadIdx.x;
  const int nq = a.q ? a.S * a.H : 0;
  const int nk = a.k ? a.S * L.kv_heads : 0;
  const int nv = a.v ? a.S * L.kv_heads : 0;
  int r = blockIdx.x;
  int kind;  // 0 q, 1 k, 2 v
  const float* x;
  int s, head;
  if (r < nq) {
    kind = 0;
    s = r / a.H;
    head = r % a.H;
    x = a.q + ((size_t)s * a.H + head) * a.q_stride;
  } else if ((r -= nq) < nk) {
    kind = 1;
    s = r / L.kv_heads;
    head = r % L.kv_heads;
    x = a.k + (size_t)r * D;
  } else if ((r -= nk) < nv) {
    kind = 2;
    s = r / L.kv_heads;
    head = r % L.kv_heads;
    x = a.v + (size_t)r * D;
  } else {
    return;
  }
  const int d0 = lane * EPL;
  float v[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) v[e] = x[d0 + e];

  if (kind != 2) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) ss = __fadd_rn(ss, __fmul_rn(v[e], v[e]));
    ss = wave_sum(ss);
    const float rms = __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), a.eps));
    const float* g = kind == 0 ? a.q_gamma : a.k_gamma;
#pragma unroll
    for (int e = 0; e < EPL; e++) v[e] = __fmul_rn(__fdiv_rn(v[e], rms), g[d0 + e]);
    const bool rope = kind == 0 || rope_k;
    if (rope) {
#pragma unroll
      for (int e = 0; e < EPL; e++) row[d0 + e] = v[e];
      __syncthreads();
      const int rot = a.rot_dim, half = rot >> 1;
      const int p = a.pos0 + s;
      const float* ct = a.cos_tab + (size_t)p * half;
      const float* st = a.sin_tab + (size_t)p * half;
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        const int d = d0 + e;
        if (d < rot) {
          const float rv = d < half ? -row[d + half] : row[d - half];
          const int ti = d < half ? d : d - half;
          v[e] = __fadd_rn(__fmul_rn(v[e], ct[ti]), __fmul_rn(rv, st[ti]));
        }
      }
    }
  }
  if (kind == 0) {
    float* o = a.q_out + ((size_t)s * a.H + head) * D;
#pragma unroll
    for (int e = 0; e < EPL; e++) o[d0 + e] = v[e];
  } else {
    store_row<D, DT>(L, kind == 1 ? 0 : 1, L.ring.phys(a.slot0 + s), head, v, lane);
  }
}

template <int D>
static hipError_t prologue_d(const LayerView& L, const PrologueArgs& a, hipStream_t st) {
  const int rows = (a.q ? a.S * a.H : 0) + (a.k ? a.S * L.kv_heads : 0) + (a.v ? a.S * L.kv_heads : 0);
  if (rows == 0) return hipSuccess;
  const int rope_k = L.ring.roll ? 0 : 1;  // sink mode caches K unroped (src/engine.ts:1530-1533)
  dim3 g(rows), b(64);
  switch (L.dtype) {
    case KV_F32: hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_F32>), g, b, 0, st, L, a, rope_k); break;
    case KV_F16: hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_F16>), g, b, 0, st, L, a, rope_k); break;
    default: hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_Q8>), g, b, 0, st, L, a, rope_k); break;
  }
  return hipGetLastError();
}

hipError_t launch_qkv_prologue(const LayerView& L, const PrologueArgs& a, hipStream_t st) {
  switch (L.D) {
    case 64: return prologue_d<64>(L, a, st);
    case 128: return prologue_d<128>(L, a, st);
    default: return prologue_d<256>(L, a, st);
  }
}

}  // namespace bg
