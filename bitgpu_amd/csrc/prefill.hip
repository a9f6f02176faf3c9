// Causal GQA prefill attention over an f16 or q8 KV cache on gfx950 MFMA (f16 in, f32 acc).
//
// Replaces the prefill/verify dispatch of attention_sg_kv16.wgsl / attention_sg_kv8.wgsl and the
// hybrid attention_online_cache_kv8.wgsl (src/engine.ts:1579-1580, 1486-1489), which run one
// subgroup or workgroup per (query, head) with a serial key loop. Here prefill is a dense
// contraction:
//   workgroup = 4 waves x 32 rows; a row is a (query, head) pair, GQA heads of one kv head are
//               packed into the rows so every K/V byte staged in LDS serves G heads.
//   per 32-key tile: K (row-major) and V^T (the cache's transposed tile) are staged into LDS as
//               f16 -- q8 codes are dequantized (code/127 * block scale) on the way in, sink-mode
//               keys are rotated at their slot position on the way in;
//   S^T = K Q^T with v_mfma_f32_32x32x16_f16 (A = K from LDS, B = Q^T held in registers), so each
//               lane holds 16 keys of ONE row and the online-softmax rescale is lane-local;
//   O^T += V^T P^T with v_mfma_f32_32x32x16_f16: the S^T accumulator registers are already in
//               the B-operand layout of P^T for the cache's V tile panel order, no transpose.
// The output gate (gate_sigmoid.wgsl:13) is applied at the store.
#include "bg_kernels.h"

namespace bg {

typedef _Float16 half8p __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

union PH8 {
  half8p h;
  uint4 u;
};

constexpr float kLog2eP = 1.4426950408889634f;

struct PrefillParams {
  LayerView L;
  const float* q;
  int S, H, G;
  int QB;            // queries per workgroup (QB * G <= 128)
  int pos_base;
  float qscale;      // scale * log2(e)
  const float* gate;
  int gate_stride;
  float* out;
  int n_qblocks;
  int n_scan_fixed;  // >0: scan this many physical slots for every block (sink mode after a wrap)
  int phys_limit;
};

template <int D>
struct PrefillSmem {
  static constexpr int KSTRIDE = D + 8;                          // f16 per staged K row (padded)
  static constexpr size_t k_bytes = (size_t)32 * KSTRIDE * 2;
  static constexpr size_t v_bytes = (size_t)32 * D * 2;
  static constexpr size_t total = k_bytes + v_bytes;
};

template <int D, int DT, bool ROLL>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillParams p) {
  using SM = PrefillSmem<D>;
  constexpr int NC = D / 16;   // QK k-chunks
  constexpr int ND = D / 32;   // output dim chunks
  __shared__ __align__(16) _Float16 ks[32 * SM::KSTRIDE];
  __shared__ __align__(16) _Float16 vs[32 * D];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g2 = lane >> 5, n = lane & 31;
  const int KV = p.L.kv_heads;
  const int kvh = blockIdx.x % KV;
  const int qb = p.n_qblocks - 1 - (int)(blockIdx.x / KV);  // heaviest (latest) blocks first
  const int s0 = qb * p.QB;

  // this lane's row
  const int r = wave * 32 + n;
  const int qi = s0 + r / p.G;
  const int h = kvh * p.G + r % p.G;
  const bool row_ok = r < p.QB * p.G && qi < p.S;
  const int limit = p.pos_base + qi;

  // Q^T operand: dims 16c + 8*g2 + [0..8)
  half8p qf[NC];
  {
    const float* qr = p.q + ((size_t)(row_ok ? qi : 0) * p.H + (row_ok ? h : 0)) * D;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      PH8 t;
      if (row_ok) {
        const float4 a = *(const float4*)(qr + 16 * c + 8 * g2);
        const float4 b = *(const float4*)(qr + 16 * c + 8 * g2 + 4);
        t.h = half8p{(_Float16)(a.x * p.qscale), (_Float16)(a.y * p.qscale), (_Float16)(a.z * p.qscale),
                     (_Float16)(a.w * p.qscale), (_Float16)(b.x * p.qscale), (_Float16)(b.y * p.qscale),
                     (_Float16)(b.z * p.qscale), (_Float16)(b.w * p.qscale)};
      } else {
        t.u = make_uint4(0, 0, 0, 0);
      }
      qf[c] = t.h;
    }
  }

  floatx16 o[ND];
#pragma unroll
  for (int i = 0; i < ND; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[i][e] = 0.0f;
  float m = -1e30f, lsum = 0.0f;

  const int last_q = min(s0 + p.QB, p.S) - 1;
  const int n_scan = p.n_scan_fixed > 0 ? p.n_scan_fixed : p.pos_base + last_q + 1;
  const int n_tiles = (n_scan + 31) / 32;
  const Ring ring = p.L.ring;
  const int cap = p.L.cap;
  constexpr int NB = D / 32;

  for (int tile = 0; tile < n_tiles; tile++) {
    const int j0 = tile * 32;
    // ---------------- stage K and V^T into LDS as f16 ----------------
    __syncthreads();
    if constexpr (DT == KV_F16) {
      const __half* kg = (const __half*)p.L.k + ((size_t)kvh * cap + j0) * D;
      const __half* vg = (const __half*)p.L.v + ((size_t)kvh * cap + j0) * D;
      constexpr int CH = 32 * D / 8;  // 16-byte chunks per tile
      for (int c = tid; c < CH; c += 256) {
        const int key = c / (D / 8), col = (c % (D / 8)) * 8;
        uint4 kv = *(const uint4*)(kg + (size_t)key * D + col);
        if constexpr (ROLL) {
          // rotation needs the partner half: handled below
        }
        *(uint4*)(ks + key * SM::KSTRIDE + col) = kv;
        *(uint4*)(vs + (size_t)c * 8) = *(const uint4*)(vg + (size_t)c * 8);
      }
    } else {
      const int8_t* kg = (const int8_t*)p.L.k + ((size_t)kvh * cap + j0) * D;
      const int8_t* vg = (const int8_t*)p.L.v + ((size_t)kvh * cap + j0) * D;
      const float* ksg = p.L.ks + ((size_t)kvh * cap + j0) * NB;
      const float* vsg = p.L.vs + ((size_t)kvh * cap + j0) * NB;
      constexpr int CH = 32 * D / 8;  // 8-code chunks per tile
      for (int c = tid; c < CH; c += 256) {
        const int key = c / (D / 8), col = (c % (D / 8)) * 8;
        const uint2 w = *(const uint2*)(kg + (size_t)key * D + col);
        const float sk = ksg[key * NB + col / 32] * (1.0f / 127.0f);
        PH8 t;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          t.h[e] = (_Float16)((float)(int8_t)(w.x >> (8 * e)) * sk);
          t.h[4 + e] = (_Float16)((float)(int8_t)(w.y >> (8 * e)) * sk);
        }
        *(uint4*)(ks + key * SM::KSTRIDE + col) = t.u;
        // V^T chunk c = (panel, dim, 8 slots)
        const int pnl = c / D, dim = c % D;
        const uint2 wv = *(const uint2*)(vg + (size_t)c * 8);
        PH8 tv;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int slot = tile_slot(pnl, e);
          const float sv = vsg[slot * NB + dim / 32] * (1.0f / 127.0f);
          const uint32_t ww = e < 4 ? wv.x : wv.y;
          tv.h[e] = (_Float16)((float)(int8_t)(ww >> (8 * (e & 3))) * sv);
        }
        *(uint4*)(vs + (size_t)c * 8) = tv.u;
      }
    }
    if constexpr (ROLL) {
      __syncthreads();
      // rotate the staged keys at their rope position: pairs (i, i + D/2)
      constexpr int PAIRS = 32 * D / 2;
      for (int c = tid; c < PAIRS; c += 256) {
        const int key = c / (D / 2), i = c % (D / 2);
        const int P = j0 + key;
        int Lg = ring.logical(P);
        Lg = P < p.phys_limit ? Lg : 0;
        long ri = (p.L.rope_abs && Lg >= ring.sinks) ? (long)Lg + p.L.evicted : (long)Lg;
        ri = ri < p.L.rope_positions ? ri : 0;
        const float cs = p.L.cos_tab[(size_t)ri * (D / 2) + i], sn = p.L.sin_tab[(size_t)ri * (D / 2) + i];
        const float a = (float)ks[key * SM::KSTRIDE + i], b = (float)ks[key * SM::KSTRIDE + i + D / 2];
        ks[key * SM::KSTRIDE + i] = (_Float16)__fadd_rn(__fmul_rn(a, cs), __fmul_rn(-b, sn));
        ks[key * SM::KSTRIDE + i + D / 2] = (_Float16)__fadd_rn(__fmul_rn(b, cs), __fmul_rn(a, sn));
      }
    }
    __syncthreads();

    // ---------------- S^T = K Q^T ----------------
    floatx16 sacc;
#pragma unroll
    for (int e = 0; e < 16; e++) sacc[e] = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      PH8 a;
      a.u = *(const uint4*)(ks + n * SM::KSTRIDE + 16 * c + 8 * g2);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.h, qf[c], sacc, 0, 0, 0);
    }
    // ---------------- mask + online softmax (row = this lane's n) ----------------
    float x[16];
    float mt = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int P = j0 + 8 * k + 4 * g2 + e;
        const int Lg = ring.logical(P);
        const bool ok = row_ok && P < n_scan && P < p.phys_limit && Lg <= limit;
        const float v = ok ? sacc[4 * k + e] : -INFINITY;
        x[4 * k + e] = v;
        mt = fmaxf(mt, v);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m, mt);
    const float corr = exp2f(m - mn);
    m = mn;
    float ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      x[i] = exp2f(x[i] - mn);
      ps += x[i];
    }
    lsum = lsum * corr + ps;
#pragma unroll
    for (int i = 0; i < ND; i++) o[i] *= corr;
    // ---------------- O^T += V^T P^T ----------------
#pragma unroll
    for (int t = 0; t < 2; t++) {
      half8p pb;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        pb[e] = (_Float16)x[8 * t + e];
        pb[4 + e] = (_Float16)x[8 * t + 4 + e];
      }
      const int pnl = 2 * t + g2;
#pragma unroll
      for (int dc = 0; dc < ND; dc++) {
        PH8 a;
        a.u = *(const uint4*)(vs + ((size_t)pnl * D + 32 * dc + n) * 8);
        o[dc] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.h, pb, o[dc], 0, 0, 0);
      }
    }
  }
  // ---------------- store ----------------
  lsum += __shfl_xor(lsum, 32, 64);
  if (!row_ok) return;
  const float inv = 1.0f / lsum;
  float* orow = p.out + ((size_t)qi * p.H + h) * D;
  const float* grow = p.gate ? p.gate + ((size_t)qi * p.H + h) * p.gate_stride : nullptr;
#pragma unroll
  for (int dc = 0; dc < ND; dc++)
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int d = 32 * dc + 8 * k + 4 * g2;
      float4 v;
      v.x = o[dc][4 * k + 0] * inv;
      v.y = o[dc][4 * k + 1] * inv;
      v.z = o[dc][4 * k + 2] * inv;
      v.w = o[dc][4 * k + 3] * inv;
      if (grow) {
        // gate_sigmoid.wgsl:13 form: x / (1 + exp(-g)); the division by l stays a multiply by
        // its reciprocal, within the f16-operand tolerance of this path
        v.x = (o[dc][4 * k + 0] / lsum) / (1.0f + expf(-grow[d + 0]));
        v.y = (o[dc][4 * k + 1] / lsum) / (1.0f + expf(-grow[d + 1]));
        v.z = (o[dc][4 * k + 2] / lsum) / (1.0f + expf(-grow[d + 2]));
        v.w = (o[dc][4 * k + 3] / lsum) / (1.0f + expf(-grow[d + 3]));
      }
      *(float4*)(orow + d) = v;
    }
}

bool prefill_supported(const LayerView& L, int S, int H) {
  if (L.dtype == KV_F32) return false;
  if (L.D != 128 && L.D != 256) return false;
  const int G = H / L.kv_heads;
  return G >= 1 && G <= 128 && S >= 1;
}

template <int D, int DT, bool ROLL>
static hipError_t launch_pf(const PrefillParams& p, hipStream_t st) {
  hipLaunchKernelGGL((prefill_kernel<D, DT, ROLL>), dim3(p.n_qblocks * p.L.kv_heads), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_attention_prefill(const LayerView& L, const AttnArgs& a, hipStream_t st) {
  PrefillParams p;
  p.L = L;
  p.q = a.q;
  p.S = a.S;
  p.H = a.H;
  p.G = a.H / L.kv_heads;
  p.QB = 128 / p.G;
  p.pos_base = a.pos_base;
  p.qscale = a.scale * kLog2eP;
  p.gate = a.gate;
  p.gate_stride = a.gate_stride;
  p.out = a.out;
  p.n_qblocks = (a.S + p.QB - 1) / p.QB;
  p.n_scan_fixed = (L.ring.roll && L.ring.head != 0) ? L.max_seq : 0;
  p.phys_limit = L.ring.roll ? L.max_seq : L.cap;
  const bool roll = L.ring.roll != 0;
  if (L.D == 128) {
    if (L.dtype == KV_Q8) return roll ? launch_pf<128, KV_Q8, true>(p, st) : launch_pf<128, KV_Q8, false>(p, st);
    return roll ? launch_pf<128, KV_F16, true>(p, st) : launch_pf<128, KV_F16, false>(p, st);
  }
  if (L.dtype == KV_Q8) return roll ? launch_pf<256, KV_Q8, true>(p, st) : launch_pf<256, KV_Q8, false>(p, st);
  return roll ? launch_pf<256, KV_F16, true>(p, st) : launch_pf<256, KV_F16, false>(p, st);
}

}  // namespace bg
