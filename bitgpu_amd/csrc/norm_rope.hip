// Fused attention prologue: per-head RMSNorm + RoPE for Q (to an f32 buffer) and K (straight
// into the KV cache in its storage format), plus the V append, for S positions in one launch.
//
// Replaces rmsnorm_rope_sg{,_kv16,_kv8}.wgsl (decode), rmsnorm_sg + rope + copy* (prefill) and
// split_head + rmsnorm + rope_partial + copy* (hybrid) of the reference (src/engine.ts:1527-1540,
// 1569-1576, 1470-1485). Workgroups of 4 waves, one work item per wave:
//   Q / K rows four rows per wave, all loads (rows and the lanes' cos/sin entries) issued before
//              any compute; lane l owns D/64 consecutive values of a row, the sum of squares is
//              a wave reduction and the rotate_half partner (d +- rot/2) is read back through
//              the wave's own LDS row (any rot_dim, full or partial, one code path; no
//              workgroup barrier).
//   V row      one position, stored into the transposed V tile (single rows: a partial group at
//              either end of the range, every row in sink mode).
//   V group    16 consecutive, 16-aligned slots of one kv head: each lane holds its dims for all
//              16 slots, so every (dim, 8-slot panel) of the transposed tile is one contiguous
//              16-byte (f16) / 8-byte (q8) / 32-byte (f32) store instead of eight scattered ones.
//
// Arithmetic follows the reference's numpy forms: y = (x / sqrt(mean(x^2) + eps)) * gamma
// (tools/reference.py:107) and y*cos + rot*sin as two rounded products and a rounded sum
// (tools/reference.py:149-152; shaders/rmsnorm_rope_sg.wgsl:32), no FMA contraction.
#include "bg_kernels.h"
#include "bg_row.h"
#include "bg_store.h"

namespace bg {

struct PrologueGrid {
  int nq, nk;       // Q rows, K rows
  int nvs, ng;      // single V rows and 16-slot V groups per kv head
  int vs_lo;        // single V rows are s in [0, vs_lo) and [vs_lo + 16*ng, S)
  int rope_k;       // K is rotated at write (0 in sink mode: rotation happens at read)
};

template <int D, int DT>
__device__ inline void store_vgroup(const LayerView& L, int kvh, int slot_base, const float (&v)[16][D / 64], int lane) {
  constexpr int EPL = D / 64;
  const int d0 = lane * EPL;
  const int t_base = slot_base & ~31;   // first slot of the 32-slot tile
  const int a = (slot_base >> 4) & 1;   // which half of the tile: panels 2a, 2a+1
  if constexpr (DT == KV_Q8) {
    constexpr int LPB = kBlock / EPL;   // lanes per q8 block
    float sc[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
      float m = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; e++) m = fmaxf(m, fabsf(v[j][e]));
      m = group_max<LPB>(m);
      sc[j] = q8_scale_of(m);
      if ((lane % LPB) == 0) L.vs[scale_offset(kvh, slot_base + j, d0 / kBlock, L.cap, D)] = sc[j];
    }
    int8_t* base = (int8_t*)L.v;
#pragma unroll
    for (int e = 0; e < EPL; e++)
#pragma unroll
      for (int b = 0; b < 2; b++) {
        uint32_t w[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const int j = tile_slot(2 * a + b, i) - 16 * a;
          const uint32_t c = (uint32_t)(uint8_t)(int8_t)q8_code(v[j][e], sc[j]);
          w[i >> 2] |= c << (8 * (i & 3));
        }
        *(uint2*)(base + v_offset(kvh, t_base + tile_slot(2 * a + b, 0), d0 + e, L.cap, D)) = make_uint2(w[0], w[1]);
      }
  } else if constexpr (DT == KV_F16) {
    __half* base = (__half*)L.v;
#pragma unroll
    for (int e = 0; e < EPL; e++)
#pragma unroll
      for (int b = 0; b < 2; b++) {
        union { __half h[8]; uint4 u; } o;
#pragma unroll
        for (int i = 0; i < 8; i++) o.h[i] = __float2half_rn(v[tile_slot(2 * a + b, i) - 16 * a][e]);
        *(uint4*)(base + v_offset(kvh, t_base + tile_slot(2 * a + b, 0), d0 + e, L.cap, D)) = o.u;
      }
  } else {
    float* base = (float*)L.v;
#pragma unroll
    for (int e = 0; e < EPL; e++)
#pragma unroll
      for (int b = 0; b < 2; b++) {
        float* dst = base + v_offset(kvh, t_base + tile_slot(2 * a + b, 0), d0 + e, L.cap, D);
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = v[tile_slot(2 * a + b, i) - 16 * a][e];
        *(float4*)dst = make_float4(o[0], o[1], o[2], o[3]);
        *(float4*)(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
      }
  }
}

template <int D, int DT>
__global__ __launch_bounds__(256) void qkv_prologue_kernel(LayerView L, PrologueArgs a, PrologueGrid gr) {
  constexpr int EPL = D / 64;
  constexpr int NR = 4;  // Q/K rows per wave
  __shared__ float rowbuf[4][D];  // one row per wave for the rotate_half partner
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int KV = L.kv_heads;
  int item = blockIdx.x * 4 + wave;
  const int d0 = lane * EPL;

  const int nqk = gr.nq + gr.nk;
  const int nqk_items = (nqk + NR - 1) / NR;
  if (item < nqk_items) {
    // ---------------- NR Q/K rows: RMSNorm (+ RoPE); every load issued before any compute ----------------
    const int rot = a.rot_dim;
    float v[NR][EPL], cs[NR][EPL], sn[NR][EPL];
#pragma unroll
    for (int j = 0; j < NR; j++) {
      const int r = min(item * NR + j, nqk - 1);  // past the end: recompute the last row, not stored
      const bool isq = r < gr.nq;
      int s;
      const float* x;
      if (isq) {
        s = r / a.H;
        x = a.q + ((size_t)s * a.H + r % a.H) * a.q_stride;
      } else {
        s = (r - gr.nq) / KV;
        x = a.k + (size_t)(r - gr.nq) * D;
      }
#pragma unroll
      for (int e = 0; e < EPL; e++) v[j][e] = x[d0 + e];
      // table rows only for rows that rotate (the range is validated only for those)
      rope_entries<D>(a.cos_tab, a.sin_tab, a.pos0 + s, rot, isq || gr.rope_k, cs[j], sn[j], lane);
    }
#pragma unroll
    for (int j = 0; j < NR; j++) {
      const int r = item * NR + j;
      const bool isq = r < gr.nq;
      const bool rope = isq || gr.rope_k;
      float y[EPL];
#pragma unroll
      for (int e = 0; e < EPL; e++) y[e] = v[j][e];
      rmsnorm_rope_wave<D>(y, isq ? a.q_gamma : a.k_gamma, a.eps, rope, rot, cs[j], sn[j], rowbuf[wave], lane);
      if (r < nqk) {
        if (isq) {
          float* o = a.q_out + (size_t)r * D;  // r = s * H + head
#pragma unroll
          for (int e = 0; e < EPL; e++) o[d0 + e] = y[e];
        } else {
          const int rk = r - gr.nq;
          store_row<D, DT>(L, 0, L.ring.phys(a.slot0 + rk / KV), rk % KV, y, lane);
        }
      }
    }
    return;
  }
  item -= nqk_items;
  if (item < gr.nvs * KV) {
    // ---------------- single V row ----------------
    const int head = item % KV, i = item / KV;
    const int s = i < gr.vs_lo ? i : i + 16 * gr.ng;
    const float* x = a.v + ((size_t)s * KV + head) * D;
    float v[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) v[e] = x[d0 + e];
    store_row<D, DT>(L, 1, L.ring.phys(a.slot0 + s), head, v, lane);
    return;
  }
  item -= gr.nvs * KV;
  if (item < gr.ng * KV) {
    // ---------------- V group: 16 aligned slots of one kv head ----------------
    const int head = item % KV, gi = item / KV;
    const int s_first = gr.vs_lo + 16 * gi;
    float v[16][EPL];
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const float* x = a.v + ((size_t)(s_first + j) * KV + head) * D;
#pragma unroll
      for (int e = 0; e < EPL; e++) v[j][e] = x[d0 + e];
    }
    store_vgroup<D, DT>(L, head, a.slot0 + s_first, v, lane);
  }
}

template <int D>
static hipError_t prologue_d(const LayerView& L, const PrologueArgs& a, hipStream_t st) {
  PrologueGrid gr;
  gr.nq = a.q ? a.S * a.H : 0;
  gr.nk = a.k ? a.S * L.kv_heads : 0;
  gr.rope_k = L.ring.roll ? 0 : 1;  // sink mode caches K unroped (src/engine.ts:1530-1533)
  gr.ng = 0;
  gr.nvs = 0;
  gr.vs_lo = 0;
  if (a.v) {
    gr.vs_lo = a.S;
    if (!L.ring.roll) {  // plain cache: slots are positions, groups of 16 aligned slots
      const int lo = (16 - (a.slot0 & 15)) & 15;
      if (a.S > lo) {
        const int ng = (a.S - lo) / 16;
        if (ng > 0) {
          gr.ng = ng;
          gr.vs_lo = lo;
        }
      }
    }
    gr.nvs = a.S - 16 * gr.ng;
  }
  const long items = ((long)gr.nq + gr.nk + 3) / 4 + (long)(gr.nvs + gr.ng) * L.kv_heads;
  if (items == 0) return hipSuccess;
  dim3 g((unsigned)((items + 3) / 4)), b(256);
  switch (L.dtype) {
    case KV_F32: hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_F32>), g, b, 0, st, L, a, gr); break;
    case KV_F16: hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_F16>), g, b, 0, st, L, a, gr); break;
    default: hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_Q8>), g, b, 0, st, L, a, gr); break;
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
