// Exact-f32 causal GQA attention over an f32 KV cache (kvCache 'f32', the reference default).
//
// Replaces attention_sg.wgsl / attention_wg.wgsl / attention_sg_roll.wgsl and the f32
// attention_online_cache.wgsl. All arithmetic is f32 (no f16 operands), so it meets the
// reference's max-abs 1e-4 bar for f32 storage. Sink mode rotates each key at read by its
// logical (or absolute) position exactly as attention_sg_roll.wgsl:40-51 (k*cos + rot*sin).
//
// Decode / verify (R = G*S <= 16 rows per kv head): split-K over all CUs. A workgroup of 4
// waves owns one kv head and a range of 64-slot tiles, every K/V byte read once for all R rows;
// a wave scores 16 slots per tile with its 4 lane groups each taking a quarter of the dims
// (float4 loads, exact f32 dot products completed by two shuffles), runs the online softmax
// per row and accumulates P.V from the transposed V panels (each lane 8 contiguous slots of
// its dims). Waves merge through LDS; splits through the workspace, last workgroup merging.
// Larger row counts (f32 prefill) run on the f32 matrix cores (prefill_f32.hip).
#include "bg_kernels.h"

namespace bg {

// ------------------------------------------------------------------------------------------
// split-K decode / verify

struct F32Split {
  int G, R;
  int n_scan, phys_limit;
  int n_tiles, tps, n_splits;
  float qscale;  // scale * log2(e)
};

// splits a merge reads in one batch (same order and arithmetic as the loop past it)
constexpr int kF32MergeBatch = 16;

// MB: more than kF32MergeBatch splits (a separate instantiation, so the short merge keeps its code)
template <int D, bool ROLL, int RM, bool MB>
__global__ __launch_bounds__(256) void attn_f32_split_kernel(LayerView L, AttnArgs a, F32Split sp) {
  constexpr int EPL = D / 64;   // output dims per lane
  constexpr int DQ = D / 4;     // K dims per lane group
  // q rows during the tile loop, the 4 waves' partial O after it
  __shared__ __align__(16) float big[4 * RM * D];
  __shared__ float psh[4][RM][16];
  __shared__ float mw[4][RM], lw[4][RM];
  __shared__ unsigned s_last;
  float* qsh = big;  // [RM][D]

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int KV = L.kv_heads;
  const int kvh = blockIdx.x % KV;
  const int split = blockIdx.x / KV;
  const int cap = L.cap;
  const int R = sp.R;

  for (int i = tid; i < RM * D; i += 256) {
    const int r = i / D, d = i % D;
    float v = 0.0f;
    if (r < R) {
      const int s = r / sp.G, h = kvh * sp.G + r % sp.G;
      v = a.q[((size_t)s * a.H + h) * D + d] * sp.qscale;
    }
    qsh[i] = v;
  }
  __syncthreads();

  const float* K = (const float*)L.k;
  const float* V = (const float*)L.v;
  float m[RM], l[RM], acc[RM][EPL];
#pragma unroll
  for (int r = 0; r < RM; r++) {
    m[r] = -1e30f;
    l[r] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[r][e] = 0.0f;
  }
  const int t0 = split * sp.tps;
  const int t1 = min(t0 + sp.tps, sp.n_tiles);
  for (int t = t0; t < t1; t++) {
    const int jw = t * 64 + wave * 16;  // this wave's 16 slots
    const int P = jw + n;
    // K quarter of slot P, dims g*DQ ..
    float k[DQ];
    {
      const float* kr = K + k_offset(kvh, min(P, cap - 1), g * DQ, cap, D);
#pragma unroll
      for (int i = 0; i < DQ; i += 4) {
        const float4 f = *(const float4*)(kr + i);
        k[i] = f.x;
        k[i + 1] = f.y;
        k[i + 2] = f.z;
        k[i + 3] = f.w;
      }
    }
    // the tile's V panels, loaded with K so both are in flight together
    const int t32 = min(jw >> 5, cap / 32 - 1);
    const int half = (jw >> 4) & 1;
    float4 vq[EPL][2][2];
#pragma unroll
    for (int e = 0; e < EPL; e++)
#pragma unroll
      for (int pp = 0; pp < 2; pp++) {
        const float* vt = V + ((size_t)kvh * cap + (size_t)t32 * 32) * D + (size_t)(2 * half + pp) * 8 * D +
                          (size_t)(lane + 64 * e) * 8;
        vq[e][pp][0] = *(const float4*)vt;
        vq[e][pp][1] = *(const float4*)(vt + 4);
      }
    const int Lg = ROLL ? L.ring.logical(P) : P;
    if constexpr (ROLL) {
      // partner dims (i, i + D/2) sit in lane groups g and g ^ 2
      int Lr = P < sp.phys_limit ? Lg : 0;
      long ri = (L.rope_abs && Lr >= L.ring.sinks) ? (long)Lr + L.evicted : (long)Lr;
      ri = ri < L.rope_positions ? ri : 0;
      const int i0 = (g & 1) * DQ;  // table index of this group's first dim
      const float* ct = L.cos_tab + (size_t)ri * (D / 2) + i0;
      const float* st = L.sin_tab + (size_t)ri * (D / 2) + i0;
#pragma unroll
      for (int i = 0; i < DQ; i++) {
        const float other = xor32(k[i]);
        const float rv = g < 2 ? -other : other;
        k[i] = add_rn(mul_rn(k[i], ct[i]), mul_rn(rv, st[i]));
      }
    }
    float x[RM];
#pragma unroll
    for (int r = 0; r < RM; r++) {
      const float* qr = qsh + r * D + g * DQ;
      float dot = 0.0f;
#pragma unroll
      for (int i = 0; i < DQ; i++) dot = fmaf(qr[i], k[i], dot);
      { const float2 r = pair16(dot); dot = r.x + r.y; }
      { const float2 r = pair32(dot); dot = r.x + r.y; }
      const int s = r / sp.G;
      const bool ok = r < R && P < sp.n_scan && P < sp.phys_limit && Lg <= a.pos_base + s;
      x[r] = ok ? dot : -INFINITY;
    }
#pragma unroll
    for (int r = 0; r < RM; r++) {
      const float mt = group16_max(x[r]);
      const float mn = fmaxf(m[r], mt);
      const float corr = exp2f(m[r] - mn);
      const float pr = exp2f(x[r] - mn);
      l[r] = l[r] * corr + group16_sum(pr);
      m[r] = mn;
#pragma unroll
      for (int e = 0; e < EPL; e++) acc[r][e] *= corr;
      if (g == 0) psh[wave][r][n] = pr;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // P.V: the wave's 16 slots are panels 2*half, 2*half+1 of one 32-slot tile
#pragma unroll
    for (int e = 0; e < EPL; e++) {
#pragma unroll
      for (int pp = 0; pp < 2; pp++) {
        const int panel = 2 * half + pp;
        const float4 va = vq[e][pp][0], vb = vq[e][pp][1];
        const float vv[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const int j = tile_slot(panel, i) - 16 * half;  // slot within the wave's 16
#pragma unroll
          for (int r = 0; r < RM; r++) acc[r][e] = fmaf(psh[wave][r][j], vv[i], acc[r][e]);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---------------- merge the 4 waves ----------------
  __syncthreads();  // q rows no longer needed
  float* ow = big;  // [4][RM][D]
#pragma unroll
  for (int r = 0; r < RM; r++) {
    if (lane == 0) {
      mw[wave][r] = m[r];
      lw[wave][r] = l[r];
    }
#pragma unroll
    for (int e = 0; e < EPL; e++) ow[((size_t)wave * RM + r) * D + lane + 64 * e] = acc[r][e];
  }
  __syncthreads();
  const bool single = sp.n_splits == 1;
  float* wso = a.ws_o + ((size_t)kvh * sp.n_splits + split) * R * D;
  float* wsml = a.ws_ml + ((size_t)kvh * sp.n_splits + split) * R * 2;
  for (int i = tid; i < R * D; i += 256) {
    const int r = i / D, d = i % D;
    float M = -1e30f;
#pragma unroll
    for (int w = 0; w < 4; w++) M = fmaxf(M, mw[w][r]);
    float o = 0.0f, lt = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float f = exp2f(mw[w][r] - M);
      o += ow[((size_t)w * RM + r) * D + d] * f;
      lt += lw[w][r] * f;
    }
    if (single) {
      const int s = r / sp.G, h = kvh * sp.G + r % sp.G;
      float res = o / lt;
      if (a.gate) res = res / (1.0f + expf(-a.gate[((size_t)s * a.H + h) * a.gate_stride + d]));
      a.out[((size_t)s * a.H + h) * D + d] = res;
    } else {
      st_coherent(&wso[i], o);
      if (d == 0) st_coherent2(&wsml[2 * r], M, lt);
    }
  }
  if (single) return;

  // ---------------- the last workgroup of this kv head merges the splits ----------------
  wait_stores();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&a.ws_count[kvh * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (unsigned)(sp.n_splits - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  const int NS = sp.n_splits;
  const float* wo = a.ws_o + (size_t)kvh * NS * R * D;
  const float* wml = a.ws_ml + (size_t)kvh * NS * R * 2;
  for (int i = tid; i < R * D; i += 256) {
    const int r = i / D, d = i % D;
    float M = -1e30f;
    float o = 0.0f, lt = 0.0f;
    if constexpr (!MB) {
      // every split's (m, l) and o issued before any is used: one memory round trip instead of
      // one per split (a loop that waits for each load: C1 9.2 against 7.3 us per layer)
      float2 mlv[kF32MergeBatch];
      float ov[kF32MergeBatch];
#pragma unroll
      for (int q = 0; q < kF32MergeBatch; q++) {
        const int qc = q < NS ? q : NS - 1;
        mlv[q] = ld_coherent2(&wml[((size_t)qc * R + r) * 2]);
        ov[q] = ld_coherent(&wo[(size_t)qc * R * D + i]);
      }
#pragma unroll
      for (int q = 0; q < kF32MergeBatch; q++) M = q < NS ? fmaxf(M, mlv[q].x) : M;
#pragma unroll
      for (int q = 0; q < kF32MergeBatch; q++) {
        if (q < NS) {
          const float f = exp2f(mlv[q].x - M);
          o += ov[q] * f;
          lt += mlv[q].y * f;
        }
      }
    } else {
      // more splits: the same in batches of kF32MergeBatch, a pass for the maximum, then one for
      // the sums (split order kept)
      for (int q0 = 0; q0 < NS; q0 += kF32MergeBatch) {
        float mv[kF32MergeBatch];
#pragma unroll
        for (int j = 0; j < kF32MergeBatch; j++) {
          const int qc = q0 + j < NS ? q0 + j : NS - 1;
          mv[j] = ld_coherent2(&wml[((size_t)qc * R + r) * 2]).x;
        }
#pragma unroll
        for (int j = 0; j < kF32MergeBatch; j++) M = q0 + j < NS ? fmaxf(M, mv[j]) : M;
      }
      for (int q0 = 0; q0 < NS; q0 += kF32MergeBatch) {
        float2 mlv[kF32MergeBatch];
        float ov[kF32MergeBatch];
#pragma unroll
        for (int j = 0; j < kF32MergeBatch; j++) {
          const int qc = q0 + j < NS ? q0 + j : NS - 1;
          mlv[j] = ld_coherent2(&wml[((size_t)qc * R + r) * 2]);
          ov[j] = ld_coherent(&wo[(size_t)qc * R * D + i]);
        }
#pragma unroll
        for (int j = 0; j < kF32MergeBatch; j++) {
          if (q0 + j < NS) {
            const float f = exp2f(mlv[j].x - M);
            o += ov[j] * f;
            lt += mlv[j].y * f;
          }
        }
      }
    }
    const int s = r / sp.G, h = kvh * sp.G + r % sp.G;
    float res = o / lt;
    if (a.gate) res = res / (1.0f + expf(-a.gate[((size_t)s * a.H + h) * a.gate_stride + d]));
    a.out[((size_t)s * a.H + h) * D + d] = res;
  }
  __syncthreads();
  if (tid == 0) __hip_atomic_store(&a.ws_count[kvh * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

bool f32_split_supported(const LayerView& L, int S, int H) {
  if (L.dtype != KV_F32 || (L.D != 128 && L.D != 256)) return false;
  const int R = (H / L.kv_heads) * S;
  return R >= 1 && R <= 16;
}

// workspace floats for any launch on this cache: at most one split per 64-slot tile
size_t f32_workspace_floats(const LayerView& L, int S, int H) {
  const int R = (H / L.kv_heads) * S;
  const int ns_max = (L.cap + 63) / 64;
  return (size_t)L.kv_heads * ns_max * R * ((size_t)L.D + 2);
}

template <int D, bool ROLL, int RM>
static void launch_split_rm(const LayerView& L, const AttnArgs& a, const F32Split& sp, hipStream_t st) {
  // splits beyond one merge batch (long f32 contexts): 1500 / 4096 / 16384 slots 24.7 / 33.2 / 47.9
  // -> 12.3 / 15.7 / 31.3 us with the batched passes
  if (sp.n_splits > kF32MergeBatch)
    hipLaunchKernelGGL((attn_f32_split_kernel<D, ROLL, RM, true>), dim3(sp.n_splits * L.kv_heads), dim3(256), 0, st, L, a, sp);
  else
    hipLaunchKernelGGL((attn_f32_split_kernel<D, ROLL, RM, false>), dim3(sp.n_splits * L.kv_heads), dim3(256), 0, st, L, a, sp);
}

template <int D, bool ROLL>
static void launch_split_d(const LayerView& L, const AttnArgs& a, const F32Split& sp, hipStream_t st) {
  if (sp.R <= 2) launch_split_rm<D, ROLL, 2>(L, a, sp, st);
  else if (sp.R <= 4) launch_split_rm<D, ROLL, 4>(L, a, sp, st);
  else if (sp.R <= 8) launch_split_rm<D, ROLL, 8>(L, a, sp, st);
  else launch_split_rm<D, ROLL, 16>(L, a, sp, st);
}

hipError_t launch_attention_f32_split(const LayerView& L, const AttnArgs& a, hipStream_t st) {
  F32Split sp;
  sp.G = a.H / L.kv_heads;
  sp.R = sp.G * a.S;
  sp.n_scan = (L.ring.roll && L.ring.head != 0) ? L.max_seq : a.pos_base + a.S;
  sp.phys_limit = L.ring.roll ? L.max_seq : L.cap;
  sp.n_tiles = (sp.n_scan + 63) / 64;
  const int cus = a.num_cus > 0 ? a.num_cus : 256;
  // one workgroup per CU, at least one tile each
  sp.tps = (sp.n_tiles * L.kv_heads + cus - 1) / cus;
  sp.tps = sp.tps < 1 ? 1 : sp.tps;
  sp.n_splits = (sp.n_tiles + sp.tps - 1) / sp.tps;
  sp.qscale = a.scale * 1.4426950408889634f;
  const size_t need = (size_t)L.kv_heads * sp.n_splits * sp.R * ((size_t)L.D + 2);
  if (sp.n_splits > 1 && (a.ws_o == nullptr || a.ws_count == nullptr || need > a.ws_floats)) return hipErrorInvalidValue;
  AttnArgs b = a;
  b.ws_ml = a.ws_o ? a.ws_o + (size_t)L.kv_heads * sp.n_splits * sp.R * L.D : nullptr;
  const bool roll = L.ring.roll != 0;
  if (L.D == 128) {
    if (roll) launch_split_d<128, true>(L, b, sp, st);
    else launch_split_d<128, false>(L, b, sp, st);
  } else {
    if (roll) launch_split_d<256, true>(L, b, sp, st);
    else launch_split_d<256, false>(L, b, sp, st);
  }
  return hipGetLastError();
}

}  // namespace bg
