// Fused attention prologue: per-head RMSNorm + RoPE for Q (to an f32 buffer) and K (straight
// into the KV cache in its storage format), plus the V append, for S positions in one launch.
//
// Replaces rmsnorm_rope_sg{,_kv16,_kv8}.wgsl (decode), rmsnorm_sg + rope + copy* (prefill) and
// split_head + rmsnorm + rope_partial + copy* (hybrid) of the reference (src/engine.ts:1527-1540,
// 1569-1576, 1470-1485). Workgroups of 4 waves, one work item per wave:
//   Q / K rows 8 (D=128) or 4 (D=256) rows per wave: a lane owns 4 consecutive dims (one
//              16-byte load), a row spans D/4 lanes; every load (rows and the lanes' cos/sin
//              entries) is issued before any compute; the sum of squares is a reduction over
//              the row's lanes (DPP / permlane), and the rotate_half partner (d +- rot/2) comes
//              from lane l ^ rot/8 by a lane exchange when that is 8, 16 or 32 lanes (rot_dim
//              64, 128, 256), else it is read back through the wave's own LDS rows (any even
//              rot_dim, full or partial; no workgroup barrier). Q leaves as one 16-byte store a lane, K as 16 / 8 /
//              4 bytes (f32 / f16 / q8 codes, plus one scale per 32 dims).
//   V row      one position, stored into the transposed V tile (single rows: a partial group at
//              either end of the range, every row in sink mode).
//   V group    16 consecutive, 16-aligned slots of one kv head: each lane holds its dims for all
//              16 slots, so every (dim, 8-slot panel) of the transposed tile is one contiguous
//              16-byte (f16) / 8-byte (q8) / 32-byte (f32) store instead of eight scattered ones.
//
// Arithmetic follows the reference kernels: y = x * inverseSqrt(mean(x^2) + eps) * gamma as two
// rounded products (shaders/rmsnorm_rope_sg.wgsl:24,28; the numpy oracle's x / sqrt(..) agrees to
// a few ulp) and y*cos + rot*sin as two rounded products and a rounded sum
// (tools/reference.py:149-152; shaders/rmsnorm_rope_sg.wgsl:32), no FMA contraction. Inputs are
// read once: nontemporal loads keep them from displacing lines the next kernel reuses.
#include "bg_kernels.h"
#include "bg_qkrow.h"
#include "bg_store.h"

namespace bg {

struct PrologueGrid {
  int nq, nk;       // Q rows, K rows
  int nvs, ng;      // single V rows and 16-slot V groups per kv head
  int vs_lo;        // single V rows are s in [0, vs_lo) and [vs_lo + 16*ng, S)
  int rope_k;       // K is rotated at write (0 in sink mode: rotation happens at read)
};

// Slot (within a 16-slot group) of entry i of the group's panel b: tile_slot(2a + b, i) - 16a,
// which does not depend on the half a of the tile. A compile-time index keeps the group's values
// in fixed registers (an index through a, known only at run time, makes the compiler select
// among all 16 rows for every entry).
__host__ __device__ constexpr int vgroup_slot(int b, int i) { return 8 * (i >> 2) + 4 * b + (i & 3); }

// Store panel b of a 16-slot group (its 8 slots, v[i] = slot vgroup_slot(b, i) of the group, D/64
// consecutive dims a lane) into the transposed V tile: every (dim, panel) is one contiguous
// 16-byte (f16) / 8-byte (q8) / 32-byte (f32) store; q8 scales are per (slot, 32 dims).
template <int D, int DT, int B>
__device__ inline void store_vpanel(const LayerView& L, int kvh, int slot_base, const float (&v)[8][D / 64], int lane) {
  constexpr int EPL = D / 64;
  const int d0 = lane * EPL;
  const int t_base = slot_base & ~31;   // first slot of the 32-slot tile
  const int a = (slot_base >> 4) & 1;   // which half of the tile: panels 2a, 2a+1
  const size_t off0 = v_offset(kvh, t_base + tile_slot(2 * a + B, 0), d0, L.cap, D);  // entry 0 of dim d0
  if constexpr (DT == KV_Q8) {
    constexpr int LPB = kBlock / EPL;   // lanes per q8 block
    float sc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      float m = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; e++) m = fmaxf(m, fabsf(v[i][e]));
      m = group_max<LPB>(m);
      if (L.q8_row) m = wave_max(m);  // per-row scale: the row's 64 lanes
      sc[i] = q8_scale_of(m);
      if ((lane % LPB) == 0) L.vs[scale_offset(kvh, slot_base + vgroup_slot(B, i), d0 / kBlock, L.cap, D)] = sc[i];
    }
    int8_t* base = (int8_t*)L.v + off0;
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      uint32_t w[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; i++) w[i >> 2] |= (uint32_t)(uint8_t)(int8_t)q8_code(v[i][e], sc[i]) << (8 * (i & 3));
      st_stream8(base + 8 * e, w[0], w[1]);
    }
  } else if constexpr (DT == KV_F16) {
    __half* base = (__half*)L.v + off0;
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      union { __half h[8]; uint4 u; } o;
#pragma unroll
      for (int i = 0; i < 8; i++) o.h[i] = __float2half_rn(v[i][e]);
      st_stream16(base + 8 * e, o.u.x, o.u.y, o.u.z, o.u.w);
    }
  } else {
    float* base = (float*)L.v + off0;
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      st_stream16f(base + 8 * e, v[0][e], v[1][e], v[2][e], v[3][e]);
      st_stream16f(base + 8 * e + 4, v[4][e], v[5][e], v[6][e], v[7][e]);
    }
  }
}

// A Q/K row spread over D/4 lanes, 4 consecutive dims (16 bytes) a lane: 64 / (D/4) rows per
// wave instruction, RB rows per wave item, every load issued before any compute.
typedef float floatx4_t __attribute__((ext_vector_type(4)));
__device__ inline float4 ld_stream4(const float* p) {
  const floatx4_t v = __builtin_nontemporal_load((const floatx4_t*)p);
  return make_float4(v[0], v[1], v[2], v[3]);
}

// EPL consecutive floats (EPL = 2 or 4), nontemporal
template <int EPL>
__device__ inline void ld_stream(const float* p, float (&v)[EPL]) {
  if constexpr (EPL == 4) {
    const float4 f = ld_stream4(p);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else {
    typedef float floatx2_t __attribute__((ext_vector_type(2)));
    const floatx2_t f = __builtin_nontemporal_load((const floatx2_t*)p);
    v[0] = f[0]; v[1] = f[1];
  }
}

template <int D>
struct RowLayout {
  static constexpr int LPR = D / 4;         // lanes per row
  static constexpr int RPI = 64 / LPR;      // rows per wave instruction
  static constexpr int NI = 4;              // load instructions per item
  static constexpr int RB = RPI * NI;       // rows per wave item
};

// SP: every batch of RB rows shares one position (H and KV multiples of RB), so a wave loads one
// cos/sin row and holds it once (fewer registers: 8 waves a SIMD instead of 6)
template <int D, int DT, bool SP>
__global__ __launch_bounds__(256) void qkv_prologue_kernel(LayerView L, PrologueArgs a, PrologueGrid gr) {
  using RL = RowLayout<D>;
  constexpr int EPL = D / 64;
  constexpr int LPR = RL::LPR, RPI = RL::RPI, NI = RL::NI, RB = RL::RB;
  // each wave's rows for the rotate_half partner (any rot_dim: the partner d +- rot/2 may sit in
  // another lane or straddle lanes)
  __shared__ __align__(16) float rowbuf[4][RB][D];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int KV = L.kv_heads;
  const int d0 = lane * EPL;

  // Work items: Q/K row batches (Q rows first, then K rows) and V items. The kinds are
  // interleaved evenly over the grid (the V items among all, then the K batches among the Q
  // batches), so the memory-bound Q batches overlap the divide-heavy q8 K rows and the V stores
  // instead of running one after the other.
  const int nqk = gr.nq + gr.nk;
  const int nqk_items = (nqk + RB - 1) / RB;
  const int nv_items = (gr.nvs + gr.ng) * KV;
  const long n_items = (long)nqk_items + nv_items;
  const long pos = (long)blockIdx.x * 4 + wave;
  if (pos >= n_items) return;
  int item;
  {
    const long v0 = pos * nv_items / n_items, v1 = (pos + 1) * nv_items / n_items;
    if (v1 > v0) {
      item = nqk_items + (int)v0;
    } else {
      const long p = pos - v0;                       // position among the Q/K batches
      const int bq = gr.nq / RB;                     // batches of Q rows only
      const long nkb = nqk_items - bq;               // batches holding K rows
      const long k0 = p * nkb / nqk_items, k1 = (p + 1) * nkb / nqk_items;
      item = k1 > k0 ? bq + (int)k0 : (int)(p - k0);
    }
  }
  if (item < nqk_items) {
    // ---------------- RB Q/K rows: RMSNorm (+ RoPE) ----------------
    const int h = lane / LPR, c = lane % LPR;  // row within an instruction, lane within the row
    const int rot = a.rot_dim, half = rot >> 1;
    const bool vec_tab = (half & 3) == 0;     // a lane's 4 dims are 4 consecutive table entries
    // one table row serves the whole batch when its rows share a position (every batch of a
    // Q or K range whose head count is a multiple of the batch)
    const int rf = item * RB, rl = min(item * RB + RB - 1, nqk - 1);
    const bool same_pos = SP || (rl < gr.nq ? rf / a.H == rl / a.H : (rf >= gr.nq && (rf - gr.nq) / KV == (rl - gr.nq) / KV));
    constexpr int NT = SP ? 1 : NI;  // table rows held
    float x[NI][4], cs[NT][4], sn[NT][4];
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const int r = min(item * RB + RPI * i + h, nqk - 1);  // past the end: recompute the last row, not stored
      const bool isq = r < gr.nq;
      int s;
      const float* src;
      if (isq) {
        s = r / a.H;
        src = a.q + ((size_t)s * a.H + r % a.H) * a.q_stride;
      } else {
        s = (r - gr.nq) / KV;
        src = a.k + (size_t)(r - gr.nq) * D;
      }
      const float4 v4 = ld_stream4(src + 4 * c);
      x[i][0] = v4.x; x[i][1] = v4.y; x[i][2] = v4.z; x[i][3] = v4.w;
      if (i > 0 && same_pos) {
        if constexpr (!SP) {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            cs[i < NT ? i : 0][e] = cs[0][e];
            sn[i < NT ? i : 0][e] = sn[0][e];
          }
        }
        continue;
      }
      // table entries only for rows that rotate (the range is validated only for those)
      const bool on = (isq || gr.rope_k) && 4 * c < rot;
      const size_t prow = (size_t)(a.pos0 + s) * half;
      if (on && vec_tab) {
        const int ti = 4 * c < half ? 4 * c : 4 * c - half;
        const float4 c4 = *(const float4*)(a.cos_tab + prow + ti), s4 = *(const float4*)(a.sin_tab + prow + ti);
        const int ti2 = i < NT ? i : 0;
        cs[ti2][0] = c4.x; cs[ti2][1] = c4.y; cs[ti2][2] = c4.z; cs[ti2][3] = c4.w;
        sn[ti2][0] = s4.x; sn[ti2][1] = s4.y; sn[ti2][2] = s4.z; sn[ti2][3] = s4.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int d = 4 * c + e;
          const int ti = d < half ? d : d - half;
          const bool one = on && d < rot;
          cs[i < NT ? i : 0][e] = one ? a.cos_tab[prow + ti] : 0.0f;
          sn[i < NT ? i : 0][e] = one ? a.sin_tab[prow + ti] : 0.0f;
        }
      }
    }
    // RMSNorm as the reference kernel: y = x * inverseSqrt(sum(x^2) / D + eps) * gamma
    // (shaders/rmsnorm_rope_sg.wgsl:24,28), no FMA contraction (bg_qkrow.h)
    float gq[4], gk[4];
    {
      const float4 g4 = a.q_gamma ? *(const float4*)(a.q_gamma + 4 * c) : make_float4(0, 0, 0, 0);
      const float4 k4 = a.k_gamma ? *(const float4*)(a.k_gamma + 4 * c) : make_float4(0, 0, 0, 0);
      gq[0] = g4.x; gq[1] = g4.y; gq[2] = g4.z; gq[3] = g4.w;
      gk[0] = k4.x; gk[1] = k4.y; gk[2] = k4.z; gk[3] = k4.w;
    }
    float* rb = &rowbuf[wave][0][0];
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const int r = item * RB + RPI * i + h;
      const bool isq = r < gr.nq;
      row_scale(x[i], row_inv_rms<D, LPR>(x[i], a.eps), isq ? gq : gk);
    }
    // the rotate_half partners by a lane exchange (every lane, before the per-row branches) where
    // the rotary width allows it, else through the wave's LDS rows
    float pr[NI][4];
    bool lanes = true;
#pragma unroll
    for (int i = 0; i < NI; i++) lanes = rope_partner_lanes(x[i], rot, pr[i]);
    if (!lanes) {
#pragma unroll
      for (int i = 0; i < NI; i++)
        *(float4*)(rb + (RPI * i + h) * D + 4 * c) = make_float4(x[i][0], x[i][1], x[i][2], x[i][3]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const int r = item * RB + RPI * i + h;
      const bool isq = r < gr.nq;
      // y*cos + rot*sin as two rounded products and a rounded sum (tools/reference.py:149-152;
      // shaders/rmsnorm_rope_sg.wgsl:32); rot = -x[d + half] below half, x[d - half] above
      if (isq || gr.rope_k) {
        if (lanes) row_rope_lanes(x[i], pr[i], c, rot, cs[i < NT ? i : 0], sn[i < NT ? i : 0]);
        else row_rope(x[i], rb + (RPI * i + h) * D, c, rot, cs[i < NT ? i : 0], sn[i < NT ? i : 0]);
      }
      if (r < nqk) {
        if (isq) {
          st_stream16f(a.q_out + (size_t)r * D + 4 * c, x[i][0], x[i][1], x[i][2], x[i][3]);
        } else {
          const int rk = r - gr.nq;
          store_k4<D, DT>(L, L.ring.phys(a.slot0 + rk / KV), rk % KV, x[i], c);
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
    ld_stream<EPL>(x + d0, v);
    store_row<D, DT>(L, 1, L.ring.phys(a.slot0 + s), head, v, lane);
    return;
  }
  item -= gr.nvs * KV;
  if (item < gr.ng * KV) {
    // ---------------- V group: 16 aligned slots of one kv head, one panel at a time ----------------
    const int head = item % KV, gi = item / KV;
    const int s_first = gr.vs_lo + 16 * gi;
    float v[8][EPL];
#pragma unroll
    for (int i = 0; i < 8; i++) ld_stream<EPL>(a.v + ((size_t)(s_first + vgroup_slot(0, i)) * KV + head) * D + d0, v[i]);
    store_vpanel<D, DT, 0>(L, head, a.slot0 + s_first, v, lane);
#pragma unroll
    for (int i = 0; i < 8; i++) ld_stream<EPL>(a.v + ((size_t)(s_first + vgroup_slot(1, i)) * KV + head) * D + d0, v[i]);
    store_vpanel<D, DT, 1>(L, head, a.slot0 + s_first, v, lane);
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
  const long items = ((long)gr.nq + gr.nk + RowLayout<D>::RB - 1) / RowLayout<D>::RB + (long)(gr.nvs + gr.ng) * L.kv_heads;
  if (items == 0) return hipSuccess;
  dim3 g((unsigned)((items + 3) / 4)), b(256);  // one item per wave
  constexpr int RB = RowLayout<D>::RB;
  const bool sp = (gr.nq == 0 || a.H % RB == 0) && (gr.nk == 0 || L.kv_heads % RB == 0);
  switch (L.dtype) {
    case KV_F32:
      if (sp) hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_F32, true>), g, b, 0, st, L, a, gr);
      else hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_F32, false>), g, b, 0, st, L, a, gr);
      break;
    case KV_F16:
      if (sp) hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_F16, true>), g, b, 0, st, L, a, gr);
      else hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_F16, false>), g, b, 0, st, L, a, gr);
      break;
    default:
      if (sp) hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_Q8, true>), g, b, 0, st, L, a, gr);
      else hipLaunchKernelGGL((qkv_prologue_kernel<D, KV_Q8, false>), g, b, 0, st, L, a, gr);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_qkv_prologue(const LayerView& L, const PrologueArgs& a, hipStream_t st) {
  switch (L.D) {
    case 128: return prologue_d<128>(L, a, st);
    default: return prologue_d<256>(L, a, st);
  }
}

}  // namespace bg
