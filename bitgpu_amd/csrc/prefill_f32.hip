// Causal GQA prefill over an f32 KV cache (kvCache 'f32', the reference default) on the f32
// matrix cores of gfx950.
//
// Replaces attention_sg.wgsl / attention_wg.wgsl (and their _roll and f32
// attention_online_cache forms) for more than 16 rows per kv head: those run one subgroup per
// (query, head) scanning every position serially (attention_sg.wgsl:21-44), each GQA head
// re-reading its group's K/V. Here:
//
//   items  = (query block, kv head): QB = 128 / G queries x the G heads of one kv head, 128 rows,
//            4 waves of 32 rows; every K/V byte a block attends is read once for all its rows.
//            Heaviest (latest queries) first; when a CU holds two workgroups and the grid fits at
//            once, each heavy item is paired with its mirror light item on one CU (workgroups b
//            and b + n/2 share a CU when the grid is dispatched in one wave).
//   tiles  = 32 keys a step, K rows and the cache's transposed 32-slot V tile staged into LDS
//            (double-buffered, one barrier a step); sink mode rotates K at staging by the slot's
//            logical (or absolute) position, in f32 with the reference's operand order
//            (attention_sg_roll.wgsl:40-51).
//   QK     = S^T = K . Q^T on v_mfma_f32_32x32x2_f32 (f32 products, f32 accumulation): K as A
//            (lane = key, one b128 LDS read feeds 4 MFMAs), the row's query (times scale * log2 e)
//            in registers as B; two independent accumulator chains.
//   softmax= online, base 2, per 32-key step; each row's 32 scores sit in lanes l and l ^ 32.
//   PV     = O^T += V^T . P^T on the same instruction: the 32x32 result layout puts key
//            8 (r / 4) + 4 (l / 32) + r % 4 of the row in register r of lane l, and the cache's V
//            tile stores exactly those keys of a dim in panel l / 32 (r < 8) and 2 + l / 32 -- so
//            register r of S^T is the B operand of PV MFMA r and the V operand is two contiguous
//            b128 reads a panel: no transpose of P or V.
// All arithmetic is f32, so the output meets the reference's max-abs 1e-4 bar for f32 storage.
#include <mutex>

#include "bg_kernels.h"

namespace bg {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kF32KT = 32;   // keys per step
constexpr int kF32Rows = 128;  // rows per workgroup (4 waves x 32)

template <int D>
struct F32Smem {
  static constexpr int KS = D + 4;                         // padded K row (floats)
  static constexpr size_t k_floats = (size_t)kF32KT * KS;  // one K buffer
  static constexpr size_t v_floats = (size_t)kF32KT * D;   // one V tile (4 panels x D x 8)
  static constexpr size_t bytes = 2 * (k_floats + v_floats) * 4;
};

struct F32PrefillParams {
  LayerView L;
  const float* q;
  int S, H, G, QB;
  int pos_base;
  float qscale;  // scale * log2(e)
  const float* gate;
  int gate_stride;
  float* out;
  int n_scan_fixed;  // sink mode: physical slots scanned by every block; 0: causal bound
  int phys_limit;
  int n_qblocks;
  int mirror;
};

template <int D, bool ROLL>
__global__ __launch_bounds__(256) void prefill_f32_kernel(F32PrefillParams p) {
  using SM = F32Smem<D>;
  constexpr int KS = SM::KS;
  constexpr int NQ = D / 8;   // 8-dim blocks: one float4 of Q per lane each
  constexpr int NO = D / 32;  // 32-dim output blocks
  extern __shared__ __align__(16) float smf[];
  // double buffers: K [2][32][KS], then V [2][32 * D]
  auto kb = [&](int buf) { return smf + buf * SM::k_floats; };
  auto vb = [&](int buf) { return smf + 2 * SM::k_floats + buf * SM::v_floats; };

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 31, hk = lane >> 5;
  const LayerView& L = p.L;
  const int KV = L.kv_heads;

  const int bid = blockIdx.x;
  const int n_items = p.n_qblocks * KV;
  const int half = (n_items + 1) / 2;
  const int item = !p.mirror || bid < half ? bid : n_items - 1 - (bid - half);
  const int kvh = item % KV;
  const int qb = p.n_qblocks - 1 - item / KV;
  const int s0 = qb * p.QB;
  const int G = p.G;

  // this lane's row (column n of the wave's 32 x 32 blocks)
  const int r = wave * 32 + n;
  const int qi = s0 + r / G;
  const int h = kvh * G + r % G;
  const bool row_ok = r < p.QB * G && qi < p.S;
  const int limit = row_ok ? p.pos_base + qi : -1;
  const int last_q = min(s0 + p.QB, p.S) - 1;
  // the last query row of this wave (wave-uniform): steps past it are masked for every row
  const int wave_last_q = min(s0 + min((wave * 32 + 31) / G, p.QB - 1), p.S - 1);
  const int wave_limit = (wave * 32 < p.QB * G) ? p.pos_base + wave_last_q : -1;
  const int n_keys = p.n_scan_fixed > 0 ? p.n_scan_fixed : p.pos_base + last_q + 1;
  const int kmax = min(n_keys, p.phys_limit);
  const int steps = (n_keys + kF32KT - 1) / kF32KT;

  // Q as the B operand: lane (n, hk) holds dims 8 t + 4 hk .. + 3 of its row, times qscale
  float4 qv[NQ];
  {
    const float* qr = p.q + ((size_t)(row_ok ? qi : 0) * p.H + (row_ok ? h : 0)) * D + 4 * hk;
#pragma unroll
    for (int t = 0; t < NQ; t++) {
      float4 x = *(const float4*)(qr + 8 * t);
      const float f = row_ok ? p.qscale : 0.0f;
      qv[t] = make_float4(x.x * f, x.y * f, x.z * f, x.w * f);
    }
  }

  const float* Kg = (const float*)L.k + (size_t)kvh * L.cap * D;
  const float* Vg = (const float*)L.v + (size_t)kvh * L.cap * D;
  // staging: thread tid copies K pair items (key, dims c..c+3 and c+D/2..) and V float4s
  constexpr int KPI = kF32KT * (D / 8) / 256;  // K pair items a thread
  constexpr int VPI = kF32KT * D / 4 / 256;    // V float4 a thread
  float4 kr[KPI][2], vr[VPI];
  auto fetch = [&](int step) {
    const int j0 = step * kF32KT;
#pragma unroll
    for (int i = 0; i < KPI; i++) {
      const int it = tid + 256 * i;
      const int key = it / (D / 8), c = 4 * (it % (D / 8));
      const float* row = Kg + (size_t)(j0 + key) * D;
      kr[i][0] = *(const float4*)(row + c);
      kr[i][1] = *(const float4*)(row + c + D / 2);
    }
#pragma unroll
    for (int i = 0; i < VPI; i++) vr[i] = *(const float4*)(Vg + (size_t)j0 * D + 4 * (tid + 256 * i));
  };
  auto stage = [&](int step, int buf) {
    const int j0 = step * kF32KT;
#pragma unroll
    for (int i = 0; i < KPI; i++) {
      const int it = tid + 256 * i;
      const int key = it / (D / 8), c = 4 * (it % (D / 8));
      float4 lo = kr[i][0], hi = kr[i][1];
      if constexpr (ROLL) {
        // k_d cos + rot_d sin, rot = -k_{d+D/2} (d < D/2) or k_{d-D/2}, at the slot's position
        const int P = j0 + key;
        int Lg = L.ring.logical(P);
        Lg = P < p.phys_limit ? Lg : 0;
        long ri = (L.rope_abs && Lg >= L.ring.sinks) ? (long)Lg + L.evicted : (long)Lg;
        ri = ri < L.rope_positions ? ri : 0;
        const float4 cs = *(const float4*)(L.cos_tab + (size_t)ri * (D / 2) + c);
        const float4 sn = *(const float4*)(L.sin_tab + (size_t)ri * (D / 2) + c);
        // two rounded products and a rounded sum, not fused
        auto rot = [](float a, float b, float co, float si) { return add_rn(mul_rn(a, co), mul_rn(-b, si)); };
        auto rot2 = [](float b, float a, float co, float si) { return add_rn(mul_rn(b, co), mul_rn(a, si)); };
        lo = make_float4(rot(kr[i][0].x, kr[i][1].x, cs.x, sn.x), rot(kr[i][0].y, kr[i][1].y, cs.y, sn.y),
                         rot(kr[i][0].z, kr[i][1].z, cs.z, sn.z), rot(kr[i][0].w, kr[i][1].w, cs.w, sn.w));
        hi = make_float4(rot2(kr[i][1].x, kr[i][0].x, cs.x, sn.x), rot2(kr[i][1].y, kr[i][0].y, cs.y, sn.y),
                         rot2(kr[i][1].z, kr[i][0].z, cs.z, sn.z), rot2(kr[i][1].w, kr[i][0].w, cs.w, sn.w));
      }
      *(float4*)(kb(buf) + key * KS + c) = lo;
      *(float4*)(kb(buf) + key * KS + c + D / 2) = hi;
    }
#pragma unroll
    for (int i = 0; i < VPI; i++) {
      // slots past the last valid one read as 0 (their probabilities are 0; 0 * garbage could
      // be NaN)
      const int f = 4 * (tid + 256 * i);  // float offset in the tile: panel (D*8), dim 8, index
      float4 x = vr[i];
      if (j0 + kF32KT > kmax) {
        const int panel = f / (D * 8), idx = f % 8;
        float* e = &x.x;
#pragma unroll
        for (int u = 0; u < 4; u++)
          if (j0 + tile_slot(panel, idx + u) >= kmax) e[u] = 0.0f;
      }
      *(float4*)(vb(buf) + f) = x;
    }
  };

  floatx16 o[NO];
#pragma unroll
  for (int b = 0; b < NO; b++)
#pragma unroll
    for (int i = 0; i < 16; i++) o[b][i] = 0.0f;
  float m = -1e30f, lsum = 0.0f;

  if (steps > 0) {
    fetch(0);
    stage(0, 0);
  }
  __syncthreads();
  for (int step = 0; step < steps; step++) {
    const int buf = step & 1;
    if (step + 1 < steps) fetch(step + 1);
    const int j0 = step * kF32KT;
    // a step past every row of this wave (plain cache) is all masked: nothing to add
    const bool active = p.n_scan_fixed > 0 || j0 <= wave_limit;
    if (active) {
      const float* kt = kb(buf);
      floatx16 s0v, s1v;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        s0v[i] = 0.0f;
        s1v[i] = 0.0f;
      }
#pragma unroll
      for (int t = 0; t < NQ; t++) {
        const float4 kk = *(const float4*)(kt + n * KS + 8 * t + 4 * hk);
        floatx16& acc = (t & 1) ? s1v : s0v;
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.x, qv[t].x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.y, qv[t].y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.z, qv[t].z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.w, qv[t].w, acc, 0, 0, 0);
      }
      // register e holds key 8 (e / 4) + 4 hk + e % 4 of this lane's row
      float sv[16];
      float mt = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int P = j0 + 8 * (e >> 2) + 4 * hk + (e & 3);
        const int Lg = ROLL ? L.ring.logical(P) : P;
        const bool ok = P < kmax && Lg <= limit;
        sv[e] = ok ? s0v[e] + s1v[e] : -INFINITY;
        mt = fmaxf(mt, sv[e]);
      }
      {
        const float2 pr = pair32(mt);
        mt = fmaxf(pr.x, pr.y);
      }
      // the reference maximum is raised only when a step's maximum exceeds it by more than 8
      // (log2 units: probabilities stay below 2^8), so most steps leave O and l unscaled
      if (__any(mt > m + 8.0f)) {
        const float mn = fmaxf(m, mt);
        const float corr = __builtin_amdgcn_exp2f(m - mn);
        m = mn;
        lsum *= corr;
#pragma unroll
        for (int b = 0; b < NO; b++)
#pragma unroll
          for (int i = 0; i < 16; i++) o[b][i] *= corr;
      }
      float ps = 0.0f;
      floatx16 pv;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        pv[e] = __builtin_amdgcn_exp2f(sv[e] - m);
        ps += pv[e];
      }
      {
        const float2 pr = pair32(ps);
        ps = pr.x + pr.y;
      }
      lsum += ps;
      // PV: dim block b, MFMA e takes key slot e of this lane's panel pair
      const float* vt = vb(buf);
#pragma unroll
      for (int b = 0; b < NO; b++) {
        const int d = 32 * b + n;
        const float4 v0 = *(const float4*)(vt + (size_t)hk * (D * 8) + d * 8);
        const float4 v1 = *(const float4*)(vt + (size_t)hk * (D * 8) + d * 8 + 4);
        const float4 v2 = *(const float4*)(vt + (size_t)(2 + hk) * (D * 8) + d * 8);
        const float4 v3 = *(const float4*)(vt + (size_t)(2 + hk) * (D * 8) + d * 8 + 4);
        const float va[16] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w,
                              v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
#pragma unroll
        for (int e = 0; e < 16; e++) o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[e], pv[e], o[b], 0, 0, 0);
      }
    }
    if (step + 1 < steps) stage(step + 1, buf ^ 1);
    __syncthreads();
  }

  // O^T block b: register e of lane (n, hk) holds dim 32 b + 8 (e / 4) + 4 hk + e % 4 of row n
  if (row_ok) {
    const float inv_l = 1.0f / lsum;
    float* orow = p.out + ((size_t)qi * p.H + h) * D;
    const float* grow = p.gate ? p.gate + ((size_t)qi * p.H + h) * p.gate_stride : nullptr;
#pragma unroll
    for (int b = 0; b < NO; b++)
#pragma unroll
      for (int e4 = 0; e4 < 4; e4++) {
        const int d = 32 * b + 8 * e4 + 4 * hk;
        float x[4];
#pragma unroll
        for (int u = 0; u < 4; u++) x[u] = o[b][4 * e4 + u] * inv_l;
        if (grow) {
#pragma unroll
          for (int u = 0; u < 4; u++) x[u] = x[u] / (1.0f + expf(-grow[d + u]));
        }
        *(float4*)(orow + d) = make_float4(x[0], x[1], x[2], x[3]);
      }
  }
}

// workgroups of an instantiation a CU holds at once (its LDS allowance set first), per kernel
template <int D, bool ROLL>
static hipError_t pf32_resident(int* out) {
  static std::mutex mu;
  static int resident = 0;
  std::lock_guard<std::mutex> lock(mu);
  if (resident == 0) {
    const void* fn = (const void*)prefill_f32_kernel<D, ROLL>;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)F32Smem<D>::bytes);
    if (e != hipSuccess) return e;
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, 256, F32Smem<D>::bytes) != hipSuccess || nb < 1) {
      (void)hipGetLastError();
      nb = 1;
    }
    resident = nb;
  }
  *out = resident;
  return hipSuccess;
}

template <int D, bool ROLL>
static hipError_t launch_pf32(F32PrefillParams p, int grid, int cus, hipStream_t st) {
  int resident = 1;
  const hipError_t e = pf32_resident<D, ROLL>(&resident);
  if (e != hipSuccess) return e;
  // two or more workgroups a CU and a grid held at once: pair heavy and light items on a CU;
  // otherwise heaviest first (the dispatcher hands each freed CU the next, lighter item)
  p.mirror = (resident >= 2 && grid <= resident * cus) ? 1 : 0;
  hipLaunchKernelGGL((prefill_f32_kernel<D, ROLL>), dim3(grid), dim3(256), F32Smem<D>::bytes, st, p);
  return hipGetLastError();
}

hipError_t launch_attention_f32(const LayerView& L, const AttnArgs& a, hipStream_t st) {
  F32PrefillParams p;
  p.L = L;
  p.q = a.q;
  p.S = a.S;
  p.H = a.H;
  p.G = a.H / L.kv_heads;
  p.QB = kF32Rows / p.G;
  if (p.QB < 1) return hipErrorInvalidValue;  // more than 128 heads per kv head
  p.pos_base = a.pos_base;
  p.qscale = a.scale * 1.4426950408889634f;
  p.gate = a.gate;
  p.gate_stride = a.gate_stride;
  p.out = a.out;
  p.n_scan_fixed = L.ring.roll ? ((L.ring.head != 0) ? L.max_seq : a.pos_base + a.S) : 0;
  p.phys_limit = L.ring.roll ? L.max_seq : L.cap;
  p.n_qblocks = (a.S + p.QB - 1) / p.QB;
  const int grid = p.n_qblocks * L.kv_heads;
  const int cus = a.num_cus > 0 ? a.num_cus : 256;
  p.mirror = 0;
  const bool roll = L.ring.roll != 0;
  if (L.D == 128) return roll ? launch_pf32<128, true>(p, grid, cus, st) : launch_pf32<128, false>(p, grid, cus, st);
  if (L.D == 256) return roll ? launch_pf32<256, true>(p, grid, cus, st) : launch_pf32<256, false>(p, grid, cus, st);
  return hipErrorInvalidValue;
}

}  // namespace bg
