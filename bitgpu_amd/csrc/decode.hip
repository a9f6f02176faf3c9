// Split-K GQA decode / verify attention over an f16 or q8 KV cache on gfx950 MFMA.
//
// Replaces attention_sg{,_kv16,_kv8}{,_roll}.wgsl for small S (decode S=1, speculative verify
// S<=12): those run one subgroup per (query, head) scanning every position serially
// (attention_sg.wgsl:31-42). Here the context is split across all CUs:
//
//   grid  = n_splits x KV workgroups, 4 waves each; a workgroup owns one kv head and a range of
//           32-slot tiles; its waves take every 4th tile. All R = (H/KV)*S query rows of the
//           GQA group are served by one read of each K/V byte.
//   QK    = v_mfma_f32_16x16x32_f16 with K as the B operand (lane = slot, 8 dims per lane
//           group) and a block-diagonal Q as A: row group g of the 16 output rows only sees the
//           dims lane group g loaded, so the MFMA returns 4 partial dot products per slot that
//           three permlane swaps reduce-scatter into one full score per lane -- no padding rows.
//           q8 codes enter the MFMA as exact f16 integers (xor/perm/pk_add, no float convert);
//           the per-32 block scale multiplies the MFMA result. Q is split hi+lo f16 so the
//           product keeps ~f32 accuracy.
//   softmax = online, base 2, per 32-slot tile; probabilities (times the q8 V block scale) go
//           through a 2 KB-per-block LDS transpose into the B operand of
//   PV    = v_mfma_f32_16x16x32_f16 with V^T (the cache's transposed V tile, 16 B per lane)
//           as A and P^T as B.
//   merge = the 4 waves combine through LDS; splits write (m, l, o) partials and the last
//           workgroup of each kv head (atomic ticket) does the log-sum-exp merge, the output
//           gate (gate_sigmoid.wgsl:13) and the store -- one launch per layer.
// Sink mode reads unroped K and rotates it at read by the slot's logical (or absolute) position
// (attention_sg_roll.wgsl:40-51), in f32 before the f16 conversion.
#include "bg_kernels.h"

namespace bg {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4v __attribute__((ext_vector_type(4)));

constexpr int NW = 4;  // waves per workgroup
constexpr float kLog2e = 1.4426950408889634f;

union H8 {
  half8 h;
  uint4 u;
  uint32_t w[4];
  half2v p[4];
};

// 8 int8 codes (two little-endian words) -> 8 exact f16 values.
__device__ inline half8 q8_to_half8(uint32_t w0, uint32_t w1) {
  H8 r;
  const uint32_t a0 = w0 ^ 0x80808080u, a1 = w1 ^ 0x80808080u;  // biased: u = c + 128
  r.w[0] = __builtin_amdgcn_perm(0x64646464u, a0, 0x04010400u);   // f16 1024+u0 | 1024+u1
  r.w[1] = __builtin_amdgcn_perm(0x64646464u, a0, 0x04030402u);
  r.w[2] = __builtin_amdgcn_perm(0x64646464u, a1, 0x04010400u);
  r.w[3] = __builtin_amdgcn_perm(0x64646464u, a1, 0x04030402u);
  const half2v bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
  for (int i = 0; i < 4; i++) r.p[i] = r.p[i] + bias;             // exact: u - 128 = c
  return r.h;
}

__device__ inline float code_of(uint32_t w, int byte) { return (float)(int8_t)(w >> (8 * byte)); }

__device__ inline uint4 ld16(const void* p) { return *(const uint4*)p; }


// which dims lane group g feeds into QK MFMA #t (element e = 0..7 of the lane's half8)
template <int D, bool QUARTER>
__device__ inline int qk_dim(int g, int t, int e) {
  if constexpr (QUARTER) {
    return g * (D / 4) + 8 * t + e;
  } else {
    constexpr int TH = D / 64;
    return t < TH ? g * (D / 8) + 8 * t + e : D / 2 + g * (D / 8) + 8 * (t - TH) + e;
  }
}

struct DecodeParams {
  LayerView L;
  const float* q;
  int S, H, G, R;
  int pos_base;
  float qscale;      // scale * log2(e) (/127 for q8 without rotation)
  const float* gate;
  int gate_stride;
  float* out;
  int n_scan;        // physical slots to scan
  int phys_limit;    // physical slots that can hold data
  int n_tiles, tiles_per_split, n_splits;
  float* ws_o;       // [KV][n_splits][R][D]
  float* ws_ml;      // [KV][n_splits][R][2]
  unsigned* ws_count;  // [KV]
  int merge_ext;     // 1: the splits only publish; decode_merge_kernel merges after this launch
};

// Shared memory plan (bytes): Q operands, per-wave P^T tiles, per-wave corr; after the tile
// loop the same space holds the per-wave partials, then the split merge's weights and sums.
template <int D, int DT, bool ROLL, int NSET, int NW>
struct DecodeSmem {
  static constexpr bool QUARTER = (DT == KV_Q8) && !ROLL;
  static constexpr int NT = D / 32;                       // QK MFMAs per 16-slot tile
  static constexpr int NBV = (DT == KV_Q8) ? D / 32 : 1;  // P copies (one per V scale block)
  static constexpr int RS = 16 * NSET;                    // padded rows
  static constexpr int NPMAX = RS / 4;                    // QK passes
  // + one 32-byte sink for the stores of operand slots past the last pass
  __host__ __device__ static size_t q_bytes(int np) { return (size_t)np * NT * 2 * 64 * 16 + 32; }
  static constexpr size_t p_bytes_wave = (size_t)NBV * RS * 32 * 2;
  static constexpr size_t c_bytes_wave = (size_t)RS * 4;
  static constexpr int DP = D + 4;                        // padded row of a wave partial
  __host__ __device__ static size_t merge_bytes(int R) { return (size_t)NW * R * (DP + 1) * 4; }
  __host__ __device__ static size_t total(int np, int R) {
    size_t a = q_bytes(np) + NW * (p_bytes_wave + c_bytes_wave);
    size_t b = merge_bytes(R);
    return a > b ? a : b;
  }
};

// One wave's raw loads for a 32-slot tile (kept in flight while the previous tile computes).
template <int D, int DT, bool QUARTER>
struct TileRegs {
  static constexpr int NB = D / 32;
  static constexpr int KU = (DT == KV_Q8) ? D / 64 : D / 32;  // uint4 of K per lane per slot
  static constexpr int VU = (DT == KV_Q8) ? NB : 2 * NB;     // uint4 of V per lane per tile
  uint4 kr[2][KU];
  float ksc[2][2];
  uint4 vr[VU];
  float vsc[2][DT == KV_Q8 ? NB : 1];
};

template <int D, int DT, bool QUARTER>
__device__ __forceinline__ void load_tile(TileRegs<D, DT, QUARTER>& T, int j0, int g, int n,
                                          const unsigned char* kbase, const unsigned char* vbase,
                                          const float* ksb, const float* vsb) {
  constexpr int NB = D / 32;
  constexpr int KU = TileRegs<D, DT, QUARTER>::KU;
  constexpr int NSUB = QUARTER ? (D / 128) : 1;
  constexpr size_t eb = (DT == KV_Q8) ? 1 : 2;
#pragma unroll
  for (int t2 = 0; t2 < 2; t2++) {
    const int P = j0 + 16 * t2 + n;
    const unsigned char* row = kbase + (size_t)P * D * eb;
    if constexpr (QUARTER) {
#pragma unroll
      for (int i = 0; i < KU; i++) T.kr[t2][i] = ld16(row + g * (D / 4) + 16 * i);
#pragma unroll
      for (int i = 0; i < NSUB; i++) T.ksc[t2][i] = ksb[(size_t)P * NB + g * NSUB + i];
    } else {
      constexpr int HU = KU / 2;  // uint4 per half piece
#pragma unroll
      for (int i = 0; i < HU; i++) {
        T.kr[t2][i] = ld16(row + (g * (D / 8)) * eb + 16 * i);
        T.kr[t2][HU + i] = ld16(row + (D / 2 + g * (D / 8)) * eb + 16 * i);
      }
      if constexpr (DT == KV_Q8) {
        T.ksc[t2][0] = ksb[(size_t)P * NB + (g * (D / 8)) / 32];
        T.ksc[t2][1] = ksb[(size_t)P * NB + (D / 2 + g * (D / 8)) / 32];
      }
    }
    if constexpr (DT == KV_Q8) {
#pragma unroll
      for (int b = 0; b < NB; b += 4) {
        const float4 f = *(const float4*)(vsb + (size_t)P * NB + b);
        T.vsc[t2][b] = f.x;
        T.vsc[t2][b + 1] = f.y;
        T.vsc[t2][b + 2] = f.z;
        T.vsc[t2][b + 3] = f.w;
      }
    }
  }
  const unsigned char* vt = vbase + ((size_t)j0 * D + (size_t)g * 8 * D) * eb;
#pragma unroll
  for (int b = 0; b < NB; b++) {
    if constexpr (DT == KV_Q8) {
      T.vr[b] = ld16(vt + (size_t)(32 * b + 2 * n) * 8);
    } else {
      T.vr[2 * b] = ld16(vt + (size_t)(32 * b + 2 * n) * 16);
      T.vr[2 * b + 1] = ld16(vt + (size_t)(32 * b + 2 * n) * 16 + 16);
    }
  }
}

template <int D, int DT, bool ROLL, int NSET, int NW>
__global__ __launch_bounds__(64 * NW) void decode_kernel(DecodeParams p) {
  using SM = DecodeSmem<D, DT, ROLL, NSET, NW>;
  constexpr bool QUARTER = SM::QUARTER;
  constexpr int NT = SM::NT;
  constexpr int NBV = SM::NBV;
  constexpr int RS = SM::RS;
  constexpr int NB = D / 32;         // q8 scale blocks per row
  constexpr int NSUB = QUARTER ? (D / 128) : 1;  // scale blocks inside one lane group's quarter
  constexpr int KU = TileRegs<D, DT, QUARTER>::KU;
  constexpr int NTHR = 64 * NW;

  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;      // lane group
  const int n = lane & 15;
  const int kvh = blockIdx.x % p.L.kv_heads;
  const int split = blockIdx.x / p.L.kv_heads;
  const int NP = (p.R + 3) >> 2;

  uint4* qs = (uint4*)smem;                                           // [NP][NT][2][64]
  unsigned char* pbase = smem + SM::q_bytes(NP);
  _Float16* pl = (_Float16*)(pbase + wave * (SM::p_bytes_wave + SM::c_bytes_wave));  // [NBV][RS][32]
  float* cl = (float*)((unsigned char*)pl + SM::p_bytes_wave);                         // [RS]

  const Ring ring = p.L.ring;
  const int cap = p.L.cap;
  const size_t eb = (DT == KV_Q8) ? 1 : 2;
  const unsigned char* kbase = (const unsigned char*)p.L.k + (size_t)kvh * cap * D * eb;
  const unsigned char* vbase = (const unsigned char*)p.L.v + (size_t)kvh * cap * D * eb;
  const float* ksb = p.L.ks + (size_t)kvh * cap * NB;
  const float* vsb = p.L.vs + (size_t)kvh * cap * NB;

  const int t_begin = split * p.tiles_per_split;
  const int t_end = min(t_begin + p.tiles_per_split, p.n_tiles);

  // Q operands (block diagonal, hi/lo f16). The setup is straight-line code -- every load is
  // unconditional (spare slots read query 0, a wave without tiles re-reads the split's last
  // tile) and spare slots store to a sink -- so the q gather, issued first, can be waited for
  // on its own while the first tile's loads stay in flight.
  TileRegs<D, DT, QUARTER> A, B;
  const int tile0 = t_begin + wave;
  {
    constexpr int QMAX = (SM::NPMAX * NT * 64 + NTHR - 1) / NTHR;  // operand slots per thread
    const int NQ = NP * NT * 64;
    float qv[QMAX][8];
    bool use[QMAX];
#pragma unroll
    for (int i = 0; i < QMAX; i++) {
      const int idx = i * NTHR + tid;
      const int l = idx & 63, t = (idx >> 6) % NT, pass = (idx >> 6) / NT;
      const int gg = l >> 4, ii = l & 15;
      const int rho = 4 * pass + (ii & 3);
      use[i] = idx < NQ && (ii >> 2) == gg && rho < p.R;
      const int s = use[i] ? rho / p.G : 0, h = use[i] ? kvh * p.G + rho % p.G : 0;
      const float* qr = p.q + ((size_t)s * p.H + h) * D + (use[i] ? qk_dim<D, QUARTER>(gg, t, 0) : 0);
      const float4 a = *(const float4*)qr, b = *(const float4*)(qr + 4);
      qv[i][0] = a.x; qv[i][1] = a.y; qv[i][2] = a.z; qv[i][3] = a.w;
      qv[i][4] = b.x; qv[i][5] = b.y; qv[i][6] = b.z; qv[i][7] = b.w;
    }
    const int ta = tile0 < t_end ? tile0 : t_end - 1;
    load_tile<D, DT, QUARTER>(A, ta * 32, g, n, kbase, vbase, ksb, vsb);
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first wait
#pragma unroll
    for (int i = 0; i < QMAX; i++) {
      const int idx = i * NTHR + tid;
      H8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float x = use[i] ? qv[i][e] * p.qscale : 0.0f;
        const _Float16 h16 = (_Float16)x;
        hi.h[e] = h16;
        lo.h[e] = (_Float16)(x - (float)h16);
      }
      const int l = idx & 63, pt = idx >> 6;   // pt = pass * NT + t
      const int o0 = idx < NQ ? (pt * 2 + 0) * 64 + l : 2 * NQ;
      const int o1 = idx < NQ ? (pt * 2 + 1) * 64 + l : 2 * NQ + 1;
      qs[o0] = hi.u;
      qs[o1] = lo.u;
    }
  }
  // zero this wave's P tiles (rows never written stay zero) and set corr = 1
  {
    uint4* pz = (uint4*)pl;
    for (int i = lane; i < (int)(SM::p_bytes_wave / 16); i += 64) pz[i] = make_uint4(0, 0, 0, 0);
    for (int i = lane; i < RS; i += 64) cl[i] = 1.0f;
  }
  __syncthreads();

  float m[SM::NPMAX], lsum[SM::NPMAX];
#pragma unroll
  for (int i = 0; i < SM::NPMAX; i++) { m[i] = -1e30f; lsum[i] = 0.0f; }
  floatx4 o[NSET][D / 16];
#pragma unroll
  for (int s = 0; s < NSET; s++)
#pragma unroll
    for (int i = 0; i < D / 16; i++) o[s][i] = floatx4{0, 0, 0, 0};

  auto process = [&](const TileRegs<D, DT, QUARTER>& T, int tile) {
    const int j0 = tile * 32;
    // ---------------- K operands ----------------
    // K operand for QK MFMA t of 16-slot group t2: converted just in time (plain cache) or
    // materialized once after the read-time rotation (sink mode)
    half8 kb[2][ROLL ? NT : 1];
    auto kop = [&](int t2, int t) -> half8 {
      if constexpr (ROLL) {
        return kb[t2][t];
      } else if constexpr (DT == KV_Q8) {
        const uint4 u = T.kr[t2][t >> 1];
        return (t & 1) ? q8_to_half8(u.z, u.w) : q8_to_half8(u.x, u.y);
      } else {
        H8 h;  // piece 0 holds MFMAs t < NT/2, piece 1 the rest, stored back to back
        h.u = T.kr[t2][t];
        return h.h;
      }
    };
#pragma unroll
    for (int t2 = 0; t2 < 2; t2++) {
      if constexpr (!ROLL) {
        (void)t2;
      } else {
        // read-time rotation: dims (i, i + D/2) of this lane group, at the slot's rope position
        const int P = j0 + 16 * t2 + n;
        int Lg = ring.logical(P);
        Lg = P < p.phys_limit ? Lg : 0;
        long ri = (p.L.rope_abs && Lg >= ring.sinks) ? (long)Lg + p.L.evicted : (long)Lg;
        ri = ri < p.L.rope_positions ? ri : 0;
        const float* ct = p.L.cos_tab + (size_t)ri * (D / 2) + g * (D / 8);
        const float* st = p.L.sin_tab + (size_t)ri * (D / 2) + g * (D / 8);
        constexpr int HT = NT / 2;  // MFMAs per half
#pragma unroll
        for (int t = 0; t < HT; t++) {
          float a[8], b2[8];
          if constexpr (DT == KV_Q8) {
            const uint4 u0 = T.kr[t2][t >> 1], u1 = T.kr[t2][KU / 2 + (t >> 1)];
            const uint32_t wa0 = (t & 1) ? u0.z : u0.x, wa1 = (t & 1) ? u0.w : u0.y;
            const uint32_t wb0 = (t & 1) ? u1.z : u1.x, wb1 = (t & 1) ? u1.w : u1.y;
            const float sa = T.ksc[t2][0] * (1.0f / 127.0f), sb = T.ksc[t2][1] * (1.0f / 127.0f);
#pragma unroll
            for (int e = 0; e < 4; e++) {
              a[e] = code_of(wa0, e) * sa;
              a[4 + e] = code_of(wa1, e) * sa;
              b2[e] = code_of(wb0, e) * sb;
              b2[4 + e] = code_of(wb1, e) * sb;
            }
          } else {
            H8 h0, h1;
            h0.u = T.kr[t2][t];
            h1.u = T.kr[t2][HT + t];
#pragma unroll
            for (int e = 0; e < 8; e++) { a[e] = (float)h0.h[e]; b2[e] = (float)h1.h[e]; }
          }
          H8 r0, r1;
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const float c = ct[8 * t + e], s = st[8 * t + e];
            r0.h[e] = (_Float16)__fadd_rn(__fmul_rn(a[e], c), __fmul_rn(-b2[e], s));
            r1.h[e] = (_Float16)__fadd_rn(__fmul_rn(b2[e], c), __fmul_rn(a[e], s));
          }
          kb[t2][t] = r0.h;
          kb[t2][HT + t] = r1.h;
        }
      }
    }

    // ---------------- QK + online softmax, one pass per 4 query rows ----------------
#pragma unroll
    for (int pass = 0; pass < SM::NPMAX; pass++) {
      if (pass >= NP) break;
      float sc[2];
#pragma unroll
      for (int t2 = 0; t2 < 2; t2++) {
        floatx4 c[NSUB];
#pragma unroll
        for (int i = 0; i < NSUB; i++) c[i] = floatx4{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < NT; t++) {
          H8 ahi, alo;
          ahi.u = qs[((pass * NT + t) * 2 + 0) * 64 + lane];
          alo.u = qs[((pass * NT + t) * 2 + 1) * 64 + lane];
          const int sub = QUARTER ? (t >> 2) : 0;
          const half8 kt = kop(t2, t);
          c[sub] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi.h, kt, c[sub], 0, 0, 0);
          c[sub] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo.h, kt, c[sub], 0, 0, 0);
        }
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          if constexpr (QUARTER) {
            float acc = c[0][e] * T.ksc[t2][0];
#pragma unroll
            for (int i = 1; i < NSUB; i++) acc = fmaf(c[i][e], T.ksc[t2][i], acc);
            v[e] = acc;
          } else {
            v[e] = c[0][e];
          }
        }
        // reduce-scatter over the 4 lane groups: lane group g ends with query row g of the pass.
        // permlane32_swap(a, b) leaves lanes l < 32 with {a[l], a[l+32]} and lanes l >= 32 with
        // {b[l-32], b[l]}; permlane16_swap does the same for odd/even row pairs.
        const auto u0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[0]), __float_as_uint(v[2]), false, false);
        const auto u1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[1]), __float_as_uint(v[3]), false, false);
        const float k0 = __uint_as_float(u0[0]) + __uint_as_float(u0[1]);  // rows 0,1: dims of v[0]; rows 2,3: v[2]
        const float k1 = __uint_as_float(u1[0]) + __uint_as_float(u1[1]);
        const auto u2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(k0), __float_as_uint(k1), false, false);
        sc[t2] = __uint_as_float(u2[0]) + __uint_as_float(u2[1]);
      }
      // mask + online softmax for row rho = 4*pass + g
      const int rho = 4 * pass + g;
      const int qi = rho / p.G;
      const bool row_ok = rho < p.R;
      const int limit = p.pos_base + qi;
      float x[2];
#pragma unroll
      for (int t2 = 0; t2 < 2; t2++) {
        const int P = j0 + 16 * t2 + n;
        const int Lg = ring.logical(P);
        const bool ok = row_ok && P < p.n_scan && P < p.phys_limit && Lg <= limit;
        x[t2] = ok ? sc[t2] : -INFINITY;
      }
      const float mt = group16_max(fmaxf(x[0], x[1]));
      const float mn = fmaxf(m[pass], mt);
      const float corr = exp2f(m[pass] - mn);
      const float p0 = exp2f(x[0] - mn), p1 = exp2f(x[1] - mn);
      lsum[pass] = lsum[pass] * corr + p0 + p1;
      m[pass] = mn;
      if (n == 0 && rho < RS) cl[rho] = corr;
      if (rho < RS) {
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
          const int j = 16 * t2 + n;
          const float pv = t2 ? p1 : p0;
          const int col = tile_panel(j) * 8 + tile_index(j);
#pragma unroll
          for (int b = 0; b < NBV; b++) {
            const float w = (DT == KV_Q8) ? pv * (T.vsc[t2][b] * (1.0f / 127.0f)) : pv;
            pl[((size_t)b * RS + rho) * 32 + col] = (_Float16)w;
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---------------- PV ----------------
    auto vop = [&](int b, int par) -> half8 {
      if constexpr (DT == KV_Q8) {
        return par ? q8_to_half8(T.vr[b].z, T.vr[b].w) : q8_to_half8(T.vr[b].x, T.vr[b].y);
      } else {
        H8 e;
        e.u = T.vr[2 * b + par];
        return e.h;
      }
    };
#pragma unroll
    for (int st = 0; st < NSET; st++) {
      const float cr = cl[16 * st + n];
#pragma unroll
      for (int i = 0; i < D / 16; i++) o[st][i] *= cr;
#pragma unroll
      for (int b = 0; b < NB; b++) {
        H8 pb;
        pb.u = *(const uint4*)(pl + ((size_t)(NBV > 1 ? b : 0) * RS + 16 * st + n) * 32 + 8 * g);
        o[st][2 * b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop(b, 0), pb.h, o[st][2 * b], 0, 0, 0);
        o[st][2 * b + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop(b, 1), pb.h, o[st][2 * b + 1], 0, 0, 0);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // software pipeline: the next tile's loads are in flight while this one computes. The
  // prefetch is unconditional (past the end it re-reads the current, cached tile) so the
  // compiler can count outstanding loads instead of draining them every tile.
  for (int tile = tile0; tile < t_end; tile += 2 * NW) {
    const int t1 = tile + NW < t_end ? tile + NW : tile;
    load_tile<D, DT, QUARTER>(B, t1 * 32, g, n, kbase, vbase, ksb, vsb);
    process(A, tile);
    if (tile + NW >= t_end) break;
    const int t2n = tile + 2 * NW < t_end ? tile + 2 * NW : tile + NW;
    load_tile<D, DT, QUARTER>(A, t2n * 32, g, n, kbase, vbase, ksb, vsb);
    process(B, tile + NW);
  }

  // ---------------- combine the waves of the workgroup ----------------
  // The row maxima go through an LDS array of their own (the tile loop never touches it), so
  // one barrier publishes them and ends every wave's use of the tile-loop space. Each wave then
  // rescales its own o and l to the workgroup maximum of the row and stores them as float4
  // (rows padded by 4 floats to spread the banks); the sum over the waves is plain adds.
  __shared__ float s_mw[NW][RS];
#pragma unroll
  for (int pass = 0; pass < SM::NPMAX; pass++) {
    if (pass >= NP) break;
    const int rho = 4 * pass + g;
    if (n == 0 && rho < p.R) s_mw[wave][rho] = m[pass];
  }
  __syncthreads();
  constexpr int DP = SM::DP;
  float* lw = (float*)smem;               // [NW][R]
  float* ow = lw + NW * p.R;              // [NW][R][DP]
  auto row_max = [&](int rho) {
    float M = s_mw[0][rho];
#pragma unroll
    for (int w = 1; w < NW; w++) M = fmaxf(M, s_mw[w][rho]);
    return M;
  };
#pragma unroll
  for (int pass = 0; pass < SM::NPMAX; pass++) {
    if (pass >= NP) break;
    const float lt = group16_sum(lsum[pass]);
    const int rho = 4 * pass + g;
    if (n == 0 && rho < p.R) lw[wave * p.R + rho] = lt * __builtin_amdgcn_exp2f(m[pass] - row_max(rho));
  }
#pragma unroll
  for (int st = 0; st < NSET; st++) {
    const int rho = 16 * st + n;
    if (rho < p.R) {
      const float f = __builtin_amdgcn_exp2f(s_mw[wave][rho] - row_max(rho));
      float* orow = ow + ((size_t)wave * p.R + rho) * DP + 8 * g;
      // o[st][2b + par][e] holds dim 32b + 8g + 2e + par: dims 32b + 8g + 4h .. +3 are
      // (e, par) = (2h, 0), (2h, 1), (2h + 1, 0), (2h + 1, 1)
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int h = 0; h < 2; h++)
          *(float4*)(orow + 32 * b + 4 * h) = make_float4(o[st][2 * b][2 * h] * f, o[st][2 * b + 1][2 * h] * f,
                                                          o[st][2 * b][2 * h + 1] * f, o[st][2 * b + 1][2 * h + 1] * f);
    }
  }
  __syncthreads();

  const bool single = p.n_splits == 1;
  constexpr int kSC1 = 16;  // cache policy sc1: agent-coherent (written through / read from memory)
  const int C4 = p.R * (D / 4);
  float* wso = single ? p.out : p.ws_o + ((size_t)kvh * p.n_splits + split) * p.R * D;
  float* wsml = single ? p.out : p.ws_ml + ((size_t)kvh * p.n_splits + split) * p.R * 2;
  const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc((void*)wso, (short)0, 0x7fffffff, 0x00020000);
  for (int c = tid; c < C4; c += NTHR) {
    const int rho = c / (D / 4), d = 4 * (c % (D / 4));
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float lt = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float4 v = *(const float4*)(ow + ((size_t)w * p.R + rho) * DP + d);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
      lt += lw[w * p.R + rho];
    }
    if (single) {
      const int s = rho / p.G, h = kvh * p.G + rho % p.G;
      float r[4] = {acc.x / lt, acc.y / lt, acc.z / lt, acc.w / lt};
      if (p.gate) {
        const float* gr = p.gate + ((size_t)s * p.H + h) * p.gate_stride + d;
#pragma unroll
        for (int e = 0; e < 4; e++) r[e] = r[e] / (1.0f + expf(-gr[e]));
      }
      *(float4*)(p.out + ((size_t)s * p.H + h) * D + d) = make_float4(r[0], r[1], r[2], r[3]);
    } else if (p.merge_ext) {  // read by the next launch: plain stores
      *(float4*)(wso + rho * D + d) = acc;
      if (d == 0) *(float2*)&wsml[2 * rho] = make_float2(row_max(rho), lt);
    } else {
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, acc), ors, (rho * D + d) * 4, 0, kSC1);
      if (d == 0) st_coherent2(&wsml[2 * rho], row_max(rho), lt);
    }
  }
  if (single || p.merge_ext) return;

  // ---------------- last workgroup of this kv head merges the splits ----------------
  __shared__ unsigned s_last;
  wait_stores();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&p.ws_count[kvh], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == (unsigned)(p.n_splits - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  // Coherent reads of the other workgroups' partials: buffer loads with the sc1 cache policy --
  // ordinary loads to the compiler, so a batch stays in flight.
  const int NS = p.n_splits;
  const int R = p.R;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.ws_o + (size_t)kvh * NS * R * D), (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.ws_ml + (size_t)kvh * NS * R * 2), (short)0, 0x7fffffff, 0x00020000);
  // partial float4 loads in flight per thread (D=256 partials are twice as long and its four
  // waves have a full SIMD's registers after the tile loop)
  constexpr int MAXL = D == 128 ? 8 : 16;
  const int TPC = NTHR >= C4 ? NTHR / C4 : 1;  // threads per float4 column
  const int CPT = NTHR / TPC;                  // columns per pass
  float* wts = (float*)smem;                   // [NS][R] merge weights
  float* mls = wts + NS * R;                   // [NS][R][2] (split lists longer than a wave)
  float4* red = (float4*)(mls + 2 * NS * R);   // [TPC][CPT] partial sums
  // (1) (m, l) of the splits. Up to 64 splits: a wave takes a row, one split per lane, in
  // registers. Issued first and unconditionally (indices clamped), so waiting for them does not
  // wait for the partials behind them.
  constexpr int RPW = (RS + NW - 1) / NW;      // rows per wave
  const bool lane_split = NS <= 64;
  uint2 mlv[RPW];
#pragma unroll
  for (int k = 0; k < RPW; k++) {
    const int rho = min(wave + k * NW, R - 1);
    const int sp = min(lane, NS - 1);
    mlv[k] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(mrs, (sp * R + rho) * 8, 0, kSC1));
  }
  floatx4 pre[MAXL];
  {
    const int c = tid % CPT, k = tid / CPT;
    const bool act = c < C4 && k < TPC;
    // branch-free (an out-of-range split re-reads the last one and gets weight 0), so all loads
    // of a batch stay in flight together
#pragma unroll
    for (int i = 0; i < MAXL; i++) {
      const int sp = min(k + TPC * i, NS - 1);
      const int cc = act ? c : 0;
      pre[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (sp * R * D + 4 * cc) * 4, 0, kSC1));
    }
  }
  // (2) weights w[sp][rho] = 2^(m_sp - M) / sum_sp l_sp 2^(m_sp - M)
  if (lane_split) {
#pragma unroll
    for (int k = 0; k < RPW; k++) {
      const int rho = wave + k * NW;
      if (rho < R) {
        const bool ok = lane < NS;
        const float mi = ok ? __uint_as_float(mlv[k].x) : -INFINITY;
        const float li = ok ? __uint_as_float(mlv[k].y) : 0.0f;
        const float M = wave_max(mi);
        const float e = __builtin_amdgcn_exp2f(mi - M);
        const float lt = wave_sum(li * e);
        if (ok) wts[lane * R + rho] = e / lt;
      }
    }
  } else {
    for (int i = tid; i < NS * R; i += NTHR) {
      const uint2 u = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(mrs, i * 8, 0, kSC1));
      mls[2 * i] = __uint_as_float(u.x);
      mls[2 * i + 1] = __uint_as_float(u.y);
    }
    __syncthreads();
    for (int rho = wave; rho < R; rho += NW) {
      float mx = -INFINITY;
      for (int sp = lane; sp < NS; sp += 64) mx = fmaxf(mx, mls[2 * (sp * R + rho)]);
      mx = wave_max(mx);
      float lt = 0.0f;
      for (int sp = lane; sp < NS; sp += 64) lt += mls[2 * (sp * R + rho) + 1] * __builtin_amdgcn_exp2f(mls[2 * (sp * R + rho)] - mx);
      lt = wave_sum(lt);
      for (int sp = lane; sp < NS; sp += 64) wts[sp * R + rho] = __builtin_amdgcn_exp2f(mls[2 * (sp * R + rho)] - mx) / lt;
    }
  }
  __syncthreads();
  // (3) weighted sum of the partials, TPC threads per column, MAXL loads in flight per thread;
  // with more than one batch the next is issued before the current one is consumed (loads past
  // the last split re-read it and get weight 0)
  const int BS = TPC * MAXL;  // splits per batch
  for (int c0 = 0; c0 < C4; c0 += CPT) {
    const int c = c0 + tid % CPT;
    const int k = tid / CPT;
    const bool act = c < C4 && k < TPC;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (act) {
      const int rho = (4 * c) / D;
      auto issue = [&](floatx4 (&v)[MAXL], int b0) {
#pragma unroll
        for (int i = 0; i < MAXL; i++) {
          const int sp = min(b0 + k + TPC * i, NS - 1);
          v[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (sp * R * D + 4 * c) * 4, 0, kSC1));
        }
      };
      auto consume = [&](const floatx4 (&v)[MAXL], int b0) {
#pragma unroll
        for (int i = 0; i < MAXL; i++) {
          const int sp = b0 + k + TPC * i;
          const float w = sp < NS ? wts[sp * R + rho] : 0.0f;
          acc.x += v[i][0] * w;
          acc.y += v[i][1] * w;
          acc.z += v[i][2] * w;
          acc.w += v[i][3] * w;
        }
      };
      floatx4 va[MAXL], vb[MAXL];
      if (c0 == 0) {
#pragma unroll
        for (int i = 0; i < MAXL; i++) va[i] = pre[i];
      } else {
        issue(va, 0);
      }
      if (NS <= BS) {
        consume(va, 0);
      } else {
        for (int b0 = 0; b0 < NS; b0 += 2 * BS) {
          issue(vb, b0 + BS);
          consume(va, b0);
          if (b0 + BS >= NS) break;
          issue(va, b0 + 2 * BS);
          consume(vb, b0 + BS);
        }
      }
      red[(size_t)k * CPT + (c - c0)] = acc;
    }
    __syncthreads();
    if (act && k == 0) {
      for (int kk = 1; kk < TPC; kk++) {
        const float4 v = red[(size_t)kk * CPT + (c - c0)];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
      const int rho = (4 * c) / D, d = (4 * c) % D;
      const int s = rho / p.G, h = kvh * p.G + rho % p.G;
      float r[4] = {acc.x, acc.y, acc.z, acc.w};
      if (p.gate) {
        const float* gr = p.gate + ((size_t)s * p.H + h) * p.gate_stride + d;
#pragma unroll
        for (int e = 0; e < 4; e++) r[e] = r[e] / (1.0f + expf(-gr[e]));
      }
      *(float4*)(p.out + ((size_t)s * p.H + h) * D + d) = make_float4(r[0], r[1], r[2], r[3]);
    }
    __syncthreads();
  }
  if (tid == 0) __hip_atomic_store(&p.ws_count[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // ready for the next launch
}

// ------------------------------------------------------------------------------------------
// Split merge as a launch of its own, for split lists whose partials are too many for one
// workgroup to read quickly (n_splits * R * D * 4 bytes per kv head): one wave per (64-dim
// chunk, row, kv head). Per chunk of up to 64 splits, lane s holds split s's (m, l) and every
// lane loads its dim of all the chunk's partials at once; the chunk folds into a running
// log-sum-exp (M, L, acc).
struct MergeParams {
  const float* ws_o;   // [KV][n_splits][R][D]
  const float* ws_ml;  // [KV][n_splits][R][2]
  int n_splits, R, G, H;
  const float* gate;
  int gate_stride;
  float* out;
};

template <int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(MergeParams p) {
  const int lane = threadIdx.x;
  const int d = blockIdx.x * 64 + lane, rho = blockIdx.y, kvh = blockIdx.z;
  const int NS = p.n_splits, R = p.R;
  const float* o = p.ws_o + (size_t)kvh * NS * R * D + (size_t)rho * D + d;  // + sp * R * D
  const float* ml = p.ws_ml + (size_t)kvh * NS * R * 2 + (size_t)rho * 2;    // + sp * R * 2
  float M = -INFINITY, L = 0.0f, acc = 0.0f;
  for (int s0 = 0; s0 < NS; s0 += 64) {
    const int nc = min(64, NS - s0);
    // unconditional loads (indices past the chunk re-read its last split, weight 0)
    const float2 v = *(const float2*)(ml + (size_t)(s0 + min(lane, nc - 1)) * R * 2);
    float ov[64];
#pragma unroll
    for (int j = 0; j < 64; j++) ov[j] = o[(size_t)(s0 + min(j, nc - 1)) * R * D];
    const bool ok = lane < nc;
    const float mi = ok ? v.x : -INFINITY;
    const float Mn = fmaxf(M, wave_max(mi));
    const float e = ok ? __builtin_amdgcn_exp2f(mi - Mn) : 0.0f;
    const float sc = __builtin_amdgcn_exp2f(M - Mn);  // 0 on the first chunk
    L = L * sc + wave_sum(ok ? v.y * e : 0.0f);
    acc *= sc;
#pragma unroll
    for (int j = 0; j < 64; j++) acc = fmaf(ov[j], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j)), acc);
    M = Mn;
  }
  const int s = rho / p.G, h = kvh * p.G + rho % p.G;
  float r = acc / L;
  if (p.gate) r = r / (1.0f + expf(-p.gate[((size_t)s * p.H + h) * p.gate_stride + d]));
  p.out[((size_t)s * p.H + h) * D + d] = r;
}

// partials per kv head above which the merge runs as its own launch (one workgroup reads
// them at roughly 40-70 GB/s; the extra launch costs about 2 us)
constexpr size_t kExtMergeBytes = 96 * 1024;

static int nset_for(int R) { return (R + 15) / 16; }

// dynamic LDS of the tile loop and wave combine (DecodeSmem::total for the launch's template
// arguments); the in-launch split merge needs less (at most 96 KB of partials per kv head)
static size_t decode_lds_bytes(int D, int dtype, int R) {
  const int nset = nset_for(R);
  const int NW = (D == 128 && nset == 1) ? 8 : 4;
  const int RS = 16 * nset, NT = D / 32, NBV = dtype == KV_Q8 ? D / 32 : 1;
  const size_t a = (size_t)((R + 3) / 4) * NT * 2 * 64 * 16 + 32 + (size_t)NW * ((size_t)NBV * RS * 32 * 2 + (size_t)RS * 4);
  const size_t b = (size_t)NW * R * (D + 5) * 4;
  return a > b ? a : b;
}
constexpr size_t kDecodeLdsMax = 159 * 1024;  // + the static wave maxima and ticket flag

bool decode_supported(const LayerView& L, int S, int H) {
  if (L.dtype == KV_F32) return false;
  if (L.D != 128 && L.D != 256) return false;
  const int G = H / L.kv_heads;
  const int R = G * S;
  // more rows than the operand and P^T tiles fit in LDS (D=256: about 20) go to the prefill kernel
  return R >= 1 && nset_for(R) <= 3 && decode_lds_bytes(L.D, L.dtype, R) <= kDecodeLdsMax;
}

// waves per workgroup: 8 where the registers allow two workgroups' worth per CU, else 4
static int waves_for(int D, int nset) { return (D == 128 && nset == 1) ? 8 : 4; }

struct Split { int n_tiles, tps, n_splits, n_scan, phys_limit; };

static Split plan_split(const LayerView& L, int S, int pos_base, int num_cus, int nw) {
  Split s;
  s.n_scan = (L.ring.roll && L.ring.head != 0) ? L.max_seq : pos_base + S;
  s.phys_limit = L.ring.roll ? L.max_seq : L.cap;
  s.n_tiles = (s.n_scan + 31) / 32;
  const int cus = num_cus > 0 ? num_cus : 256;
  // one workgroup per CU: tiles_per_split = ceil(tiles * KV / CUs), at least one tile per wave
  int tps = (s.n_tiles * L.kv_heads + cus - 1) / cus;
  tps = tps < nw ? nw : tps;
  s.tps = tps;
  s.n_splits = (s.n_tiles + tps - 1) / tps;
  return s;
}

size_t decode_workspace_floats(const LayerView& L, int S, int H, int num_cus, size_t* counters) {
  // upper bound over every pos_base: tiles_per_split >= 4 waves, so at most cap/32/4 splits
  (void)num_cus;
  const int R = (H / L.kv_heads) * S;
  const int ns_max = (L.cap / 32 + 3) / 4;
  *counters = (size_t)L.kv_heads;
  return (size_t)L.kv_heads * ns_max * R * ((size_t)L.D + 2);
}

template <int D, int DT, bool ROLL, int NSET>
static hipError_t launch_cfg(const LayerView& L, const AttnArgs& a, hipStream_t st) {
  constexpr int NW = (D == 128 && NSET == 1) ? 8 : 4;
  using SM = DecodeSmem<D, DT, ROLL, NSET, NW>;
  const Split sp = plan_split(L, a.S, a.pos_base, a.num_cus, NW);
  DecodeParams p;
  p.L = L;
  p.q = a.q;
  p.S = a.S;
  p.H = a.H;
  p.G = a.H / L.kv_heads;
  p.R = p.G * a.S;
  p.pos_base = a.pos_base;
  p.qscale = a.scale * kLog2e * (SM::QUARTER ? (1.0f / 127.0f) : 1.0f);
  p.gate = a.gate;
  p.gate_stride = a.gate_stride;
  p.out = a.out;
  p.n_scan = sp.n_scan;
  p.phys_limit = sp.phys_limit;
  p.n_tiles = sp.n_tiles;
  p.tiles_per_split = sp.tps;
  p.n_splits = sp.n_splits;
  const size_t need = (size_t)L.kv_heads * sp.n_splits * p.R * ((size_t)D + 2);
  if (sp.n_splits > 1 && (a.ws_o == nullptr || need > a.ws_floats)) return hipErrorInvalidValue;
  p.ws_o = a.ws_o;
  p.ws_ml = a.ws_o ? a.ws_o + (size_t)L.kv_heads * sp.n_splits * p.R * D : nullptr;
  p.ws_count = a.ws_count;
  p.merge_ext = sp.n_splits > 1 && (size_t)sp.n_splits * p.R * D * 4 > kExtMergeBytes;
  const int NP = (p.R + 3) / 4;
  size_t smem = SM::total(NP, p.R);
  if (smem != decode_lds_bytes(D, DT, p.R)) return hipErrorInvalidValue;  // the two plans agree
  if (sp.n_splits > 1 && !p.merge_ext) {
    // the in-launch merge reuses the space: weights + l [NS][R] and float4 partial sums
    const size_t C4 = (size_t)p.R * D / 4;
    const size_t tpc = (size_t)64 * NW >= C4 ? (size_t)64 * NW / C4 : 1;
    const size_t cpt = (size_t)64 * NW / tpc;
    const size_t merge = (size_t)3 * sp.n_splits * p.R * 4 + tpc * cpt * 16;
    smem = smem > merge ? smem : merge;
  }
  if (smem > kDecodeLdsMax) return hipErrorInvalidValue;
  if (smem > 64 * 1024) {
    static size_t attr_bytes = 0;
    if (smem > attr_bytes) {
      hipError_t e = hipFuncSetAttribute((const void*)decode_kernel<D, DT, ROLL, NSET, NW>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      if (e != hipSuccess) return e;
      attr_bytes = smem;
    }
  }
  hipLaunchKernelGGL((decode_kernel<D, DT, ROLL, NSET, NW>), dim3(sp.n_splits * L.kv_heads), dim3(64 * NW), smem, st, p);
  if (p.merge_ext) {
    MergeParams m;
    m.ws_o = p.ws_o;
    m.ws_ml = p.ws_ml;
    m.n_splits = p.n_splits;
    m.R = p.R;
    m.G = p.G;
    m.H = p.H;
    m.gate = p.gate;
    m.gate_stride = p.gate_stride;
    m.out = p.out;
    hipLaunchKernelGGL((decode_merge_kernel<D>), dim3(D / 64, p.R, L.kv_heads), dim3(64), 0, st, m);
  }
  return hipGetLastError();
}

template <int D, int DT, bool ROLL>
static hipError_t launch_nset(const LayerView& L, const AttnArgs& a, int nset, hipStream_t st) {
  switch (nset) {
    case 1: return launch_cfg<D, DT, ROLL, 1>(L, a, st);
    case 2: return launch_cfg<D, DT, ROLL, 2>(L, a, st);
    default: return launch_cfg<D, DT, ROLL, 3>(L, a, st);
  }
}

template <int D>
static hipError_t launch_d(const LayerView& L, const AttnArgs& a, int nset, hipStream_t st) {
  const bool roll = L.ring.roll != 0;
  if (L.dtype == KV_Q8) {
    return roll ? launch_nset<D, KV_Q8, true>(L, a, nset, st) : launch_nset<D, KV_Q8, false>(L, a, nset, st);
  }
  return roll ? launch_nset<D, KV_F16, true>(L, a, nset, st) : launch_nset<D, KV_F16, false>(L, a, nset, st);
}

hipError_t launch_attention_decode(const LayerView& L, const AttnArgs& a, hipStream_t st) {
  const int R = (a.H / L.kv_heads) * a.S;
  const int nset = nset_for(R);
  return L.D == 128 ? launch_d<128>(L, a, nset, st) : launch_d<256>(L, a, nset, st);
}

}  // namespace bg
