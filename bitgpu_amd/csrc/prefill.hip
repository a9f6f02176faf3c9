// Causal GQA prefill attention over an f16 or q8 KV cache on gfx950 MFMA (f16 in, f32 acc).
//
// Replaces the prefill/verify dispatch of attention_sg_kv16.wgsl / attention_sg_kv8.wgsl and the
// hybrid attention_online_cache_kv8.wgsl (src/engine.ts:1579-1580, 1486-1489), which run one
// subgroup or workgroup per (query, head) with a serial key loop. Here prefill is a dense
// contraction:
//   rows      a row is a (query, head) pair; the G heads of one kv head are packed into the rows
//             so every staged K/V byte serves G heads. A wave owns 32 rows, a workgroup 128.
//   teams     a workgroup is 8 waves = two teams of 4. Both teams hold the same 128 rows; team 0
//             scans the first half of the block's key range, team 1 the second half, and the two
//             online-softmax states are merged through LDS at the end. Two waves per SIMD (one
//             of each team) let one wave's softmax overlap the other's MFMAs, and the halves are
//             equal so neither team idles. Blocks are launched heaviest (latest queries) first.
//   staging   per step a team stages KT keys (64 for D=128, 32 for D=256): K row-major and V^T
//             (the cache's transposed 32-slot tiles) into LDS as f16, double-buffered with one
//             barrier per step; the next step's global loads are in flight while this step
//             computes. q8 codes are dequantized (code * block scale / 127) once per workgroup
//             on the way in; sink-mode keys are rotated at their slot position on the way in.
//   S^T = K Q^T  v_mfma_f32_32x32x16_f16, A = K from LDS, B = Q^T held in registers: a lane
//             holds 16 keys of ONE row, so the softmax is lane-local plus one cross-half shuffle.
//   softmax   base 2; masks only on steps that reach past the block's first query (causal
//             diagonal) or the scanned range; the running max is raised only when a step's max
//             exceeds it by more than 8 (so P <= 2^8, exact-range f16) -- most steps skip the
//             O rescale.
//   O^T += V^T P^T  v_mfma_f32_32x32x16_f16: the S^T accumulator registers are already in the
//             B-operand layout of P^T for the V tile's panel order, no transpose.
// The output gate (gate_sigmoid.wgsl:13) is applied at the store.
#include "bg_kernels.h"

namespace bg {

typedef _Float16 half8p __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

union PH8 {
  half8p h;
  uint4 u;
  _Float16 e[8];
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
struct PfCfg {
  static constexpr int KT = D == 128 ? 64 : 32;   // keys per step
  static constexpr int NSUB = KT / 32;            // 32-key MFMA sub-tiles per step
  static constexpr int KS = D + 8;                // staged K row stride in f16 (bank spread)
  static constexpr int K_HALFS = KT * KS;
  static constexpr int V_HALFS = KT * D;
  static constexpr int BUF_HALFS = K_HALFS + V_HALFS;   // one team's buffer
  static constexpr int NC = D / 16;               // QK k-chunks
  static constexpr int ND = D / 32;               // output dim chunks
  static constexpr int NB = D / 32;               // q8 scale blocks per row
  static constexpr size_t stage_bytes = (size_t)4 * BUF_HALFS * 2;          // 2 teams x 2 buffers
  static constexpr size_t merge_bytes = (size_t)4 * 64 * (ND * 16 + 2) * 4;  // team 1's states
  static constexpr size_t smem = stage_bytes > merge_bytes ? stage_bytes : merge_bytes;
};

// One thread's share of a step's staging: 16 dims of one key in each half of the row (the rope
// partners i and i + D/2 sit in the same thread) and 4 V^T chunks of 8 slots (f16: 4 chunks
// spread over the step; q8: the chunks of 4 neighbouring dims of one panel, which share the
// 8 slot scales of one block).
template <int D, int DT>
struct StageRegs {
  static constexpr bool Q8 = DT == KV_Q8;
  uint4 k[Q8 ? 2 : 4];        // q8: 16 codes per half; f16: 2 x 8 values per half
  float ksc[Q8 ? 2 : 1];
  uint4 v[Q8 ? 2 : 4];        // q8: 4 dims x 8 slots of codes; f16: 4 x 8 values
  float vsc[Q8 ? 8 : 1];      // q8: block scale of each of the 8 slots
};

template <int D, int DT, bool ROLL>
struct Stager {
  using C = PfCfg<D>;
  static constexpr int PH = D / 32;   // threads per key (16 dims per half each)
  // K piece of this thread
  int tt, key, cb;
  // q8 V chunk group of this thread: dims 4*vdg .. 4*vdg+3 of panel vpanel of 32-slot tile vu
  int vu, vpanel, vdg;

  __device__ explicit Stager(int t) {
    tt = t;
    key = t / PH;
    cb = 16 * (t % PH);
    vdg = t % (D / 4);
    vpanel = (t / (D / 4)) & 3;
    vu = t / D;
  }

  // issue the global loads of the step whose first key is slot j0
  __device__ __forceinline__ void load(StageRegs<D, DT>& R, const PrefillParams& p, int kvh, int j0) const {
    const LayerView& L = p.L;
    const int cap = L.cap;
    const int slot = min(j0 + key, cap - 1);  // past the end: a valid row whose keys are masked
    if constexpr (DT == KV_Q8) {
      const int8_t* kr = (const int8_t*)L.k + ((size_t)kvh * cap + slot) * D;
      R.k[0] = *(const uint4*)(kr + cb);
      R.k[1] = *(const uint4*)(kr + cb + D / 2);
      const float* ks = L.ks + ((size_t)kvh * cap + slot) * C::NB;
      R.ksc[0] = ks[cb / 32];
      R.ksc[1] = ks[(cb + D / 2) / 32];
      const int t32 = min((j0 >> 5) + vu, cap / 32 - 1);
      const int8_t* vt = (const int8_t*)L.v + ((size_t)kvh * cap + (size_t)t32 * 32) * D +
                         ((size_t)vpanel * D + 4 * vdg) * 8;
      R.v[0] = *(const uint4*)vt;
      R.v[1] = *(const uint4*)(vt + 16);
      const float* vs = L.vs + ((size_t)kvh * cap + (size_t)t32 * 32) * C::NB + (4 * vdg) / 32;
#pragma unroll
      for (int e = 0; e < 8; e++) R.vsc[e] = vs[(size_t)tile_slot(vpanel, e) * C::NB];
    } else {
      const __half* kr = (const __half*)L.k + ((size_t)kvh * cap + slot) * D;
      R.k[0] = *(const uint4*)(kr + cb);
      R.k[1] = *(const uint4*)(kr + cb + 8);
      R.k[2] = *(const uint4*)(kr + cb + D / 2);
      R.k[3] = *(const uint4*)(kr + cb + D / 2 + 8);
      // V^T: the step's KT slots are KT * D contiguous values; chunk = tt + 256 i
      const int t32 = j0 >> 5;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int c = tt + 256 * i;                 // 16-byte chunk within the step
        const int u = c / (4 * D);                  // 32-slot tile of the chunk
        const int tu = min(t32 + u, cap / 32 - 1);
        const __half* vt = (const __half*)L.v + ((size_t)kvh * cap + (size_t)tu * 32) * D;
        R.v[i] = *(const uint4*)(vt + (size_t)(c % (4 * D)) * 8);
      }
    }
  }

  // convert (dequantize / rotate) and write into one team buffer; j0 = the staged step's first key
  __device__ __forceinline__ void store(const StageRegs<D, DT>& R, const PrefillParams& p, int j0, _Float16* kb,
                                        _Float16* vb) const {
    float a[16], b[16];  // the two halves of this thread's 16-dim K piece
    if constexpr (DT == KV_Q8) {
      const float sa = R.ksc[0] * (1.0f / 127.0f), sb = R.ksc[1] * (1.0f / 127.0f);
      const uint32_t wa[4] = {R.k[0].x, R.k[0].y, R.k[0].z, R.k[0].w};
      const uint32_t wb[4] = {R.k[1].x, R.k[1].y, R.k[1].z, R.k[1].w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t ua = wa[i] ^ 0x80808080u, ub = wb[i] ^ 0x80808080u;  // biased: u = c + 128
#pragma unroll
        for (int e = 0; e < 4; e++) {
          a[4 * i + e] = fmaf((float)((ua >> (8 * e)) & 0xffu), sa, -128.0f * sa);  // = c * sa, one rounding
          b[4 * i + e] = fmaf((float)((ub >> (8 * e)) & 0xffu), sb, -128.0f * sb);
        }
      }
    } else {
      PH8 h;
#pragma unroll
      for (int i = 0; i < 2; i++) {
        h.u = R.k[i];
#pragma unroll
        for (int e = 0; e < 8; e++) a[8 * i + e] = (float)h.e[e];
        h.u = R.k[2 + i];
#pragma unroll
        for (int e = 0; e < 8; e++) b[8 * i + e] = (float)h.e[e];
      }
    }
    if constexpr (ROLL) {
      // pairs (i, i + D/2) at the key's rope position, f32 with one rounding per step (the
      // table rows are loaded here, not with the step's data, to keep registers for the MFMAs)
      const LayerView& L = p.L;
      const int P = j0 + key;
      int Lg = L.ring.logical(P);
      Lg = P < p.phys_limit ? Lg : 0;
      long ri = (L.rope_abs && Lg >= L.ring.sinks) ? (long)Lg + L.evicted : (long)Lg;
      ri = ri < L.rope_positions ? ri : 0;
      const float* ct = L.cos_tab + (size_t)ri * (D / 2) + cb;
      const float* st = L.sin_tab + (size_t)ri * (D / 2) + cb;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float4 cv = *(const float4*)(ct + 4 * i), sv = *(const float4*)(st + 4 * i);
        const float c4[4] = {cv.x, cv.y, cv.z, cv.w};
        const float s4[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float x = a[4 * i + e], y = b[4 * i + e];
          a[4 * i + e] = __fadd_rn(__fmul_rn(x, c4[e]), __fmul_rn(-y, s4[e]));
          b[4 * i + e] = __fadd_rn(__fmul_rn(y, c4[e]), __fmul_rn(x, s4[e]));
        }
      }
    }
    if constexpr (DT == KV_Q8 || ROLL) {
      PH8 o;
#pragma unroll
      for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int e = 0; e < 8; e++) o.e[e] = (_Float16)a[8 * i + e];
        *(uint4*)(kb + key * C::KS + cb + 8 * i) = o.u;
#pragma unroll
        for (int e = 0; e < 8; e++) o.e[e] = (_Float16)b[8 * i + e];
        *(uint4*)(kb + key * C::KS + cb + D / 2 + 8 * i) = o.u;
      }
    } else {
      *(uint4*)(kb + key * C::KS + cb) = R.k[0];
      *(uint4*)(kb + key * C::KS + cb + 8) = R.k[1];
      *(uint4*)(kb + key * C::KS + cb + D / 2) = R.k[2];
      *(uint4*)(kb + key * C::KS + cb + D / 2 + 8) = R.k[3];
    }
    if constexpr (DT == KV_Q8) {
      const uint32_t w[8] = {R.v[0].x, R.v[0].y, R.v[0].z, R.v[0].w, R.v[1].x, R.v[1].y, R.v[1].z, R.v[1].w};
      float sv[8], nb[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        sv[e] = R.vsc[e] * (1.0f / 127.0f);
        nb[e] = -128.0f * sv[e];
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {  // chunk i: dim 4*vdg + i, 8 slots
        PH8 o;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const uint32_t u = w[2 * i + (e >> 2)] ^ 0x80808080u;
          o.e[e] = (_Float16)fmaf((float)((u >> (8 * (e & 3))) & 0xffu), sv[e], nb[e]);
        }
        *(uint4*)(vb + ((size_t)(vu * 4 + vpanel) * D + 4 * vdg + i) * 8) = o.u;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) *(uint4*)(vb + (size_t)(tt + 256 * i) * 8) = R.v[i];
    }
  }
};

template <int D, int DT, bool ROLL, int TEAMS>
__global__ __launch_bounds__(256 * TEAMS) void prefill_kernel(PrefillParams p) {
  using C = PfCfg<D>;
  constexpr int KT = C::KT, NSUB = C::NSUB, NC = C::NC, ND = C::ND, KS = C::KS;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  _Float16* smem = (_Float16*)smem_raw;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int team = TEAMS == 2 ? wave >> 2 : 0, wt = wave & 3;
  const int tt = tid & 255;  // thread index within the team
  const int g2 = lane >> 5, n = lane & 31;
  const int KV = p.L.kv_heads;
  const int kvh = blockIdx.x % KV;
  const int qb = p.n_qblocks - 1 - (int)(blockIdx.x / KV);  // heaviest (latest) blocks first
  const int s0 = qb * p.QB;

  // this lane's row
  const int r = wt * 32 + n;
  const int qi = s0 + r / p.G;
  const int h = kvh * p.G + r % p.G;
  const bool row_ok = r < p.QB * p.G && qi < p.S;
  const int limit = p.pos_base + qi;

  // key range of the block, split into two equal halves with two teams (team 1 takes the
  // larger one)
  const int last_q = min(s0 + p.QB, p.S) - 1;
  const int n_scan = p.n_scan_fixed > 0 ? p.n_scan_fixed : p.pos_base + last_q + 1;
  const int T = (n_scan + KT - 1) / KT;
  const int T0 = TEAMS == 2 ? T / 2 : 0;
  const int my_first = team ? T0 : 0;
  const int my_count = team || TEAMS == 1 ? T - T0 : T0;
  const int steps = T - T0;
  // the earliest key index any row of the block masks (causal diagonal or scan end)
  const int mask_from = min(min(p.pos_base + s0 + 1, n_scan), p.phys_limit);

  _Float16* const tbuf = smem + (size_t)(team * 2) * C::BUF_HALFS;  // this team's 2 buffers

  const Stager<D, DT, ROLL> stg(tt);
  // The staging is branch-free: a team past its last step re-stages a valid (clamped) tile into
  // the buffer nobody reads this step, so the registers stay registers and loads stay counted.
  const int t_last = T - 1;
  {
    StageRegs<D, DT> R;
    const int j0 = min(my_first, t_last) * KT;
    stg.load(R, p, kvh, j0);
    stg.store(R, p, j0, tbuf, tbuf + C::K_HALFS);
  }

  // Q^T operand: dims 16c + 8*g2 + [0..8), pre-scaled by scale*log2(e)
  half8p qf[NC];
  {
    const float* qr = p.q + ((size_t)(row_ok ? qi : 0) * p.H + (row_ok ? h : 0)) * D;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const float4 a = *(const float4*)(qr + 16 * c + 8 * g2);
      const float4 b = *(const float4*)(qr + 16 * c + 8 * g2 + 4);
      const float sc = row_ok ? p.qscale : 0.0f;
      qf[c] = half8p{(_Float16)(a.x * sc), (_Float16)(a.y * sc), (_Float16)(a.z * sc), (_Float16)(a.w * sc),
                     (_Float16)(b.x * sc), (_Float16)(b.y * sc), (_Float16)(b.z * sc), (_Float16)(b.w * sc)};
    }
  }

  floatx16 o[ND];
#pragma unroll
  for (int i = 0; i < ND; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[i][e] = 0.0f;
  float m = -1e30f, lsum = 0.0f;
  const Ring ring = p.L.ring;
  __syncthreads();

  for (int s = 0; s < steps; s++) {
    StageRegs<D, DT> R;
    const int jn = min(my_first + s + 1, t_last) * KT;
    stg.load(R, p, kvh, jn);

    if (s < my_count) {
      const int j0 = (my_first + s) * KT;
      const _Float16* kb = tbuf + (size_t)(s & 1) * C::BUF_HALFS;
      const _Float16* vb = kb + C::K_HALFS;
      // ---------------- S^T = K Q^T ----------------
      floatx16 sacc[NSUB];
#pragma unroll
      for (int u = 0; u < NSUB; u++)
#pragma unroll
        for (int e = 0; e < 16; e++) sacc[u][e] = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; c++)
#pragma unroll
        for (int u = 0; u < NSUB; u++) {
          PH8 a;
          a.u = *(const uint4*)(kb + (u * 32 + n) * KS + 16 * c + 8 * g2);
          sacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.h, qf[c], sacc[u], 0, 0, 0);
        }
      // ---------------- mask + online softmax (row = this lane's n) ----------------
      float x[NSUB][16];
      float mt = -INFINITY;
      if (ROLL || j0 + KT > mask_from) {
#pragma unroll
        for (int u = 0; u < NSUB; u++)
#pragma unroll
          for (int k = 0; k < 4; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const int P = j0 + 32 * u + 8 * k + 4 * g2 + e;
              const int Lg = ring.logical(P);
              const bool ok = P < n_scan && P < p.phys_limit && Lg <= limit;
              const float v = ok ? sacc[u][4 * k + e] : -INFINITY;
              x[u][4 * k + e] = v;
              mt = fmaxf(mt, v);
            }
      } else {
#pragma unroll
        for (int u = 0; u < NSUB; u++)
#pragma unroll
          for (int e = 0; e < 16; e++) {
            x[u][e] = sacc[u][e];
            mt = fmaxf(mt, x[u][e]);
          }
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      // raise the reference max only when this step's max exceeds it by more than 2^8
      const bool grow = mt > m + 8.0f;
      if (__any(grow)) {
        const float mn = grow ? mt : m;
        const float corr = exp2f(m - mn);
        m = mn;
        lsum *= corr;
#pragma unroll
        for (int i = 0; i < ND; i++) o[i] *= corr;
      }
      float ps = 0.0f;
#pragma unroll
      for (int u = 0; u < NSUB; u++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          x[u][e] = exp2f(x[u][e] - m);
          ps += x[u][e];
        }
      lsum += ps;
      // ---------------- O^T += V^T P^T ----------------
#pragma unroll
      for (int u = 0; u < NSUB; u++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
          half8p pb;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            pb[e] = (_Float16)x[u][8 * t + e];
            pb[4 + e] = (_Float16)x[u][8 * t + 4 + e];
          }
          const int pnl = 2 * t + g2;
#pragma unroll
          for (int dc = 0; dc < ND; dc++) {
            PH8 a;
            a.u = *(const uint4*)(vb + ((size_t)(u * 4 + pnl) * D + 32 * dc + n) * 8);
            o[dc] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.h, pb, o[dc], 0, 0, 0);
          }
        }
    }

    {
      _Float16* kb = tbuf + (size_t)((s + 1) & 1) * C::BUF_HALFS;
      stg.store(R, p, jn, kb, kb + C::K_HALFS);
    }
    __syncthreads();
  }

  // ---------------- merge the two teams' states ----------------
  float* ms = (float*)smem_raw;  // [wt][ND*16 + 2][lane]
  constexpr int SL = ND * 16 + 2;
  if (TEAMS == 2 && team == 1) {
    float* w = ms + (size_t)wt * SL * 64 + lane;
#pragma unroll
    for (int dc = 0; dc < ND; dc++)
#pragma unroll
      for (int e = 0; e < 16; e++) w[(dc * 16 + e) * 64] = o[dc][e];
    w[(ND * 16) * 64] = m;
    w[(ND * 16 + 1) * 64] = lsum;
  }
  if constexpr (TEAMS == 2) {
    __syncthreads();
    if (team == 1) return;
    const float* w = ms + (size_t)wt * SL * 64 + lane;
    const float m1 = w[(ND * 16) * 64], l1 = w[(ND * 16 + 1) * 64];
    const float M = fmaxf(m, m1);
    const float a0 = exp2f(m - M), a1 = exp2f(m1 - M);
#pragma unroll
    for (int dc = 0; dc < ND; dc++)
#pragma unroll
      for (int e = 0; e < 16; e++) o[dc][e] = o[dc][e] * a0 + w[(dc * 16 + e) * 64] * a1;
    lsum = lsum * a0 + l1 * a1;
  }
  // ---------------- store ----------------
  lsum += __shfl_xor(lsum, 32, 64);
  if (!row_ok) return;
  const float inv = 1.0f / lsum;
  float* orow = p.out + ((size_t)qi * p.H + h) * D;
  const float* grow_ = p.gate ? p.gate + ((size_t)qi * p.H + h) * p.gate_stride : nullptr;
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
      if (grow_) {
        // gate_sigmoid.wgsl:13 form: x / (1 + exp(-g))
        v.x = (o[dc][4 * k + 0] / lsum) / (1.0f + expf(-grow_[d + 0]));
        v.y = (o[dc][4 * k + 1] / lsum) / (1.0f + expf(-grow_[d + 1]));
        v.z = (o[dc][4 * k + 2] / lsum) / (1.0f + expf(-grow_[d + 2]));
        v.w = (o[dc][4 * k + 3] / lsum) / (1.0f + expf(-grow_[d + 3]));
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

// two teams where the registers allow two waves per SIMD (D=128); D=256 keeps its O and Q^T in
// one wave per SIMD's 512 registers
template <int D, int DT, bool ROLL>
static hipError_t launch_pf(const PrefillParams& p, hipStream_t st) {
  constexpr int TEAMS = D == 128 ? 2 : 1;
  constexpr size_t smem = TEAMS == 2 ? PfCfg<D>::smem : PfCfg<D>::stage_bytes / 2;
  static bool attr_set = false;  // per instantiation
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)prefill_kernel<D, DT, ROLL, TEAMS>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((prefill_kernel<D, DT, ROLL, TEAMS>), dim3(p.n_qblocks * p.L.kv_heads), dim3(256 * TEAMS),
                     smem, st, p);
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
