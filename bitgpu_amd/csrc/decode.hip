// Split-K GQA decode / verify attention over an f16 or q8 KV cache on gfx950 MFMA.
//
// Replaces attention_sg{,_kv16,_kv8}{,_roll}.wgsl for small S (decode S=1, speculative verify
// S<=12): those run one subgroup per (query, head) scanning every position serially
// (attention_sg.wgsl:31-42). Here the context is split across all CUs:
//
//   grid  = n_splits x KV workgroups, NW = 4 or 8 waves each; a workgroup owns one kv head and
//           a range of 32-slot tiles; its waves take every NW-th tile. All R = (H/KV)*S query rows of the
//           GQA group are served by one read of each K/V byte.
//   QK    = v_mfma_f32_16x16x32_f16 with K as the B operand (lane = slot, 8 dims per lane
//           group) and a block-diagonal Q as A, in passes of 4 or 8 query rows: with 4, row
//           group g of the 16 output rows only sees the dims lane group g loaded, so the MFMA
//           returns 4 partial dot products per slot that three permlane swaps reduce-scatter
//           into one full score per lane; with 8 (more than 4 rows per kv head), each half of
//           the output rows sees two lane groups and one swap per pair of rows leaves two full
//           scores per lane. q8 codes enter the MFMA as exact f16 integers (xor/perm/pk_add,
//           no float convert); the per-32 block scale multiplies the MFMA result. Q is split
//           hi+lo f16 so the product keeps ~f32 accuracy.
//   tiles = each wave keeps two 32-slot tiles in flight in registers; q8 launches whose plan
//           gives every wave one tile run a one-tile variant (half the registers: two
//           workgroups a CU).
//   softmax = online, base 2, per 32-slot tile; probabilities (times the q8 V block scale) go
//           through a 2 KB-per-block LDS transpose into the B operand of
//   PV    = v_mfma_f32_16x16x32_f16 with V^T (the cache's transposed V tile, 16 B per lane)
//           as A and P^T as B.
//   merge = the waves combine through LDS; splits write (m, l, o) partials into slots that
//           hold an "empty" marker between launches (into their XCD's L2 when all splits of a
//           kv head share an XCD, else written through); the last splits of each kv head poll
//           their units' slots and each does the log-sum-exp merge, the output gate
//           (gate_sigmoid.wgsl:13) and the store for its (row, 64-dim) units -- one launch per
//           layer. A merger waits only on splits dispatched before it, the grid never exceeds
//           what the GPU holds at once, and the wait is bounded: a merger that gives up stores
//           NaN and raises the cache's host-visible error word (bg_attention then returns
//           BG_E_DEVICE and resets the workspace).
// Sink mode reads unroped K and rotates it at read by the slot's logical (or absolute) position
// (attention_sg_roll.wgsl:40-51), in f32 (x*c - y*s with the c product fused into the sum) before
// the f16 conversion.
#include <algorithm>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "bg_kernels.h"

namespace bg {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef unsigned u32x2v __attribute__((ext_vector_type(2)));

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

// K/V tile bytes are read once per launch: nontemporal loads (streaming cache policy) keep them
// from displacing reusable lines and sustain a higher HBM rate than plain loads.
__device__ inline uint4 ld16(const void* p) {
  const u32x4v v = __builtin_nontemporal_load((const u32x4v*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ inline float ldnt(const float* p) { return __builtin_nontemporal_load(p); }
__device__ inline float4 ldnt4(const float* p) {
  const floatx4 v = __builtin_nontemporal_load((const floatx4*)p);
  return make_float4(v[0], v[1], v[2], v[3]);
}


// which dims lane group g feeds into QK MFMA #t (element e = 0..7 of the lane's half8). A pass
// of PR = 4 query rows gives each lane group's rows a block-diagonal quarter of the MFMA's k
// range; a pass of PR = 8 rows gives each half of the 16 rows two lane groups. With q8 codes
// (QUARTER) the k range a row sees in one MFMA must lie in one 32-dim scale block: PR = 4 walks
// a contiguous quarter of D per lane group; PR = 8 pairs lane groups 2h and 2h+1 on block t/2 of
// half h (16 contiguous bytes per lane and block: MFMA t even takes bytes 0-7, odd 8-15).
template <int D, bool QUARTER, int PR>
__device__ inline int qk_dim(int g, int t, int e) {
  if constexpr (QUARTER && PR == 4) {
    return g * (D / 4) + 8 * t + e;
  } else if constexpr (QUARTER) {
    return (g >> 1) * (D / 2) + 32 * (t >> 1) + 16 * (g & 1) + 8 * (t & 1) + e;
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
  // tiles skip_t0 .. skip_t0 + skip_n - 1 hold only slots that every row masks (empty ring slots
  // in sink mode) and are not scanned: tile index t covers slots from 32 (t < skip_t0 ? t : t + skip_n)
  int skip_t0, skip_n;
  // split partials, [KV][units][n_splits][17] float4 with unit = (row, 64-dim chunk): 16 float4
  // of o, then (m, l, -, -). Every slot holds kPartialEmpty except between a split's store and
  // the merger's read of it in the same launch.
  float4* ws;
  int n_mergers;       // the last n_mergers splits also merge: merger i takes units i, i + n_mergers, ..
  unsigned* err;       // host-visible error word: a merger's bounded wait gave up
  int spin_limit;      // poll rounds before a merger gives up
  int withhold_split;  // test hook: this split stores no partial (-1: none)
  // > 0: workgroups numbered in groups of xcd_group consecutive splits per kv head, so the kv
  // heads of one split share blockIdx mod 8 (one XCD when workgroups go to XCDs round robin):
  // sink mode's cos/sin rows of a slot are then fetched into one L2 for all kv heads. The last
  // group is padded; its padding workgroups exit at once.
  int xcd_group;
  // > 0: the splits of a kv head share blockIdx mod xcd_local (the number of XCDs). The GPU
  // dispatches a grid's workgroups to its XCDs round robin (from a starting XCD that changes
  // from launch to launch, the same for the whole grid), so they share one L2, and every split
  // stores its partial into that L2 (a plain store, no write-through): the mergers' agent-scope
  // loads see lines written on their own XCD, from any CU, an L2 round trip after the store
  // instead of a memory round trip (C3 16k 13.6 -> 13.2 us, 4k 8.0 -> 7.8). 0: partials are
  // written through to memory.
  int xcd_local;
};

// "not written yet" marker of a partial slot: a quiet NaN with a payload that arithmetic on
// finite inputs never produces
constexpr uint32_t kPartialEmpty = kWorkspaceEmpty;
constexpr int kUnitF4 = 17;  // float4 per (unit, split) slot
// splits per kv head at most (the merge holds a column of every split in registers)
constexpr int kMaxSplits = 256;

// Shared memory plan (bytes): Q operands, then one part per wave: its P^T tiles and corr in the
// tile loop, its raw partial o rows after it.
template <int D, int DT, bool ROLL, int NSET, int NW, int PR>
struct DecodeSmem {
  static constexpr bool QUARTER = (DT == KV_Q8) && !ROLL;
  static constexpr int NT = D / 32;                       // QK MFMAs per 16-slot tile
  static constexpr int NBV = (DT == KV_Q8) ? D / 32 : 1;  // P copies (one per V scale block)
  static constexpr int RS = 16 * NSET;                    // padded rows
  static constexpr int NPMAX = RS / PR;                   // QK passes
  // + one 32-byte sink for the stores of operand slots past the last pass
  __host__ __device__ static size_t q_bytes(int np) { return (size_t)np * NT * 2 * 64 * 16 + 32; }
  static constexpr size_t p_bytes_wave = (size_t)NBV * RS * 32 * 2;
  static constexpr size_t c_bytes_wave = (size_t)RS * 4;
  static constexpr int DP = D + 4;                        // padded row of a wave partial
  // a wave's part: its P tiles and corrections in the tile loop, then its raw o rows
  __host__ __device__ static size_t wave_bytes(int R) {
    const size_t t = p_bytes_wave + c_bytes_wave, o = (size_t)R * DP * 4;
    return t > o ? t : o;
  }
  __host__ __device__ static size_t total(int np, int R) { return q_bytes(np) + NW * wave_bytes(R); }
};

// One wave's raw loads for a 32-slot tile (kept in flight while the previous tile computes).
template <int D, int DT, bool QUARTER, int PR>
struct TileRegs {
  static constexpr int NB = D / 32;
  static constexpr int KU = (DT == KV_Q8) ? D / 64 : D / 32;  // uint4 of K per lane per slot
  static constexpr int VU = (DT == KV_Q8) ? NB : 2 * NB;     // uint4 of V per lane per tile
  // K scale blocks a lane's output rows see per slot: its quarter (PR = 4) or half (PR = 8) of
  // D with q8 codes in the MFMA; the two rope halves' blocks when rotating in f32
  static constexpr int KSN = QUARTER ? (PR == 4 ? D / 128 : D / 64) : 2;
  uint4 kr[2][KU];
  float ksc[2][KSN];
  uint4 vr[VU];
  float vsc[2][DT == KV_Q8 ? NB : 1];
};

// The K part of a tile's loads (K codes and both scale rows: the V scales are folded into the
// probabilities) and the V part are issued separately, so each can be re-issued for a later tile
// as soon as its phase of the current tile has consumed it.
template <int D, int DT, bool QUARTER, int PR>
__device__ __forceinline__ void load_tile_k(TileRegs<D, DT, QUARTER, PR>& T, int j0, int g, int n,
                                            const unsigned char* kbase, const float* ksb, const float* vsb) {
  constexpr int NB = D / 32;
  constexpr int KU = TileRegs<D, DT, QUARTER, PR>::KU;
  constexpr int KSN = TileRegs<D, DT, QUARTER, PR>::KSN;
  constexpr size_t eb = (DT == KV_Q8) ? 1 : 2;
#pragma unroll
  for (int t2 = 0; t2 < 2; t2++) {
    const int P = j0 + 16 * t2 + n;
    const unsigned char* row = kbase + (size_t)P * D * eb;
    if constexpr (QUARTER) {
      // uint4 i holds the codes of MFMAs 2i and 2i+1 (qk_dim)
      const int kb0 = PR == 4 ? g * (D / 4) : (g >> 1) * (D / 2) + 16 * (g & 1);
      const int kstep = PR == 4 ? 16 : 32;
#pragma unroll
      for (int i = 0; i < KU; i++) T.kr[t2][i] = ld16(row + kb0 + kstep * i);
      const int sb0 = PR == 4 ? g * KSN : (g >> 1) * KSN;
#pragma unroll
      for (int i = 0; i < KSN; i++) T.ksc[t2][i] = ldnt(ksb + (size_t)P * NB + sb0 + i);
    } else {
      constexpr int HU = KU / 2;  // uint4 per half piece
#pragma unroll
      for (int i = 0; i < HU; i++) {
        T.kr[t2][i] = ld16(row + (g * (D / 8)) * eb + 16 * i);
        T.kr[t2][HU + i] = ld16(row + (D / 2 + g * (D / 8)) * eb + 16 * i);
      }
      if constexpr (DT == KV_Q8) {
        T.ksc[t2][0] = ldnt(ksb + (size_t)P * NB + (g * (D / 8)) / 32);
        T.ksc[t2][1] = ldnt(ksb + (size_t)P * NB + (D / 2 + g * (D / 8)) / 32);
      }
    }
    if constexpr (DT == KV_Q8) {
#pragma unroll
      for (int b = 0; b < NB; b += 4) {
        const float4 f = ldnt4(vsb + (size_t)P * NB + b);
        T.vsc[t2][b] = f.x;
        T.vsc[t2][b + 1] = f.y;
        T.vsc[t2][b + 2] = f.z;
        T.vsc[t2][b + 3] = f.w;
      }
    }
  }
}

template <int D, int DT, bool QUARTER, int PR>
__device__ __forceinline__ void load_tile_v(TileRegs<D, DT, QUARTER, PR>& T, int j0, int g, int n,
                                            const unsigned char* vbase) {
  constexpr int NB = D / 32;
  constexpr size_t eb = (DT == KV_Q8) ? 1 : 2;
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

// Sink mode: the rope rows of a tile's two slots a lane rotates (cos and sin of its lane group's
// D/8 dims of the first half, at each slot's rope position), loaded with the tile's K part so
// that the rotation does not wait a memory round trip after the tile has arrived. ON = false (no
// rotation, or a kernel without the registers for it): empty, and the rotation reads the table
// itself.
template <int D, bool ON>
struct RopeRegs {
  float4 c[2][D / 32], s[2][D / 32];
};
template <int D>
struct RopeRegs<D, false> {};

// the table row of physical slot P (sink-mode positions: logical slot, plus the evicted count past
// the sinks in absolute mode; slots past the ring and rows past the table read row 0, unused)
__device__ __forceinline__ long rope_row(const LayerView& L, int phys_limit, int P) {
  int Lg = L.ring.logical(P);
  Lg = P < phys_limit ? Lg : 0;
  long ri = (L.rope_abs && Lg >= L.ring.sinks) ? (long)Lg + L.evicted : (long)Lg;
  return ri < L.rope_positions ? ri : 0;
}

template <int D, bool ON>
__device__ __forceinline__ void load_rope(RopeRegs<D, ON>& R, const LayerView& L, int phys_limit, int j0, int g,
                                          int n) {
  if constexpr (ON) {
#pragma unroll
    for (int t2 = 0; t2 < 2; t2++) {
      const long ri = rope_row(L, phys_limit, j0 + 16 * t2 + n);
      const float* ct = L.cos_tab + (size_t)ri * (D / 2) + g * (D / 8);
      const float* st = L.sin_tab + (size_t)ri * (D / 2) + g * (D / 8);
#pragma unroll
      for (int i = 0; i < D / 32; i++) {
        R.c[t2][i] = *(const float4*)(ct + 4 * i);
        R.s[t2][i] = *(const float4*)(st + 4 * i);
      }
    }
  }
}

// PR: query rows per QK pass (4, or 8 for more than 4 rows: half the MFMAs, operand reads and
// reductions per row). NPT > 0: the launch has exactly NPT passes (compiled straight-line); 0:
// up to the set's RS / PR passes, counted at run time. ONE: every wave has at most one tile (the
// plan gives a split one tile a wave): no second tile in registers, so two workgroups fit a CU.
template <int D, int DT, bool ROLL, int NSET, int NW, int NPT, int PR, bool ONE>
__global__ __launch_bounds__(64 * NW) void decode_kernel(DecodeParams p) {
  using SM = DecodeSmem<D, DT, ROLL, NSET, NW, PR>;
  using TR = TileRegs<D, DT, SM::QUARTER, PR>;
  constexpr int NPK = NPT > 0 ? NPT : SM::NPMAX;  // passes compiled
  constexpr bool QUARTER = SM::QUARTER;
  constexpr int NT = SM::NT;
  constexpr int NBV = SM::NBV;
  constexpr int RS = SM::RS;
  constexpr int NB = D / 32;         // q8 scale blocks per row
  constexpr int KU = TR::KU;
  constexpr int RL = PR / 4;         // query rows per lane and pass after the reduction
  constexpr int NTHR = 64 * NW;
  // q8 without rotation: QK on the int8 matrix cores (the K codes as they are)
  constexpr bool I8 = QUARTER;
  constexpr int NT8 = D / 64;        // int8 QK MFMAs per 16-slot group (16 dims a lane group each)
  constexpr int NSB = TR::KSN;       // scale blocks a lane's output rows see

  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  // wave-uniform (scalar) so the tile loop's trip count is uniform control flow: with a
  // divergent one the loop becomes exec-masked flow and the tile prefetch is waited for at the
  // loop head instead of staying in flight
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4;      // lane group
  const int n = lane & 15;
  int kvh, split;
  if (p.xcd_group > 0) {
    const int span = p.xcd_group * p.L.kv_heads, r = blockIdx.x % span;
    kvh = r / p.xcd_group;
    split = (blockIdx.x / span) * p.xcd_group + r % p.xcd_group;
  } else {
    kvh = blockIdx.x % p.L.kv_heads;
    split = blockIdx.x / p.L.kv_heads;
  }
  if (split >= p.n_splits) return;  // padding of the last split group (the whole workgroup)
  const int NP = NPT > 0 ? NPT : (p.R + PR - 1) / PR;
  // query row of pass `pass` that lane group g holds in slot i (i < RL) after the reduction
  auto row_of = [&](int pass, int i) { return PR == 4 ? 4 * pass + g : 8 * pass + 2 * i + (g >> 1) + 4 * (g & 1); };

  uint4* qs = (uint4*)smem;                                           // [NP][NT][2][64]
  unsigned char* pbase = smem + SM::q_bytes(NP);
  _Float16* pl = (_Float16*)(pbase + wave * SM::wave_bytes(p.R));  // [NBV][RS][32]
  float* cl = (float*)((unsigned char*)pl + SM::p_bytes_wave);                         // [RS]

  const Ring ring = p.L.ring;
  const int cap = p.L.cap;
  const size_t eb = (DT == KV_Q8) ? 1 : 2;
  const unsigned char* kbase = (const unsigned char*)p.L.k + (size_t)kvh * cap * D * eb;
  const unsigned char* vbase = (const unsigned char*)p.L.v + (size_t)kvh * cap * D * eb;
  const float* ksb = p.L.ks + (size_t)kvh * cap * NB;
  const float* vsb = p.L.vs + (size_t)kvh * cap * NB;

  // splits take the tiles in reverse order: the last, shorter range goes to split 0 (dispatched
  // first), the mergers (the highest splits) take the first tiles (C4 verify5 16.89 -> 16.44 us,
  // C4 decode 11.31 -> 11.13, C5 decode 14.75 -> 14.52; the plain order measured 0.7-0.85 us
  // slower for the one-tile kernel at 2049-8192 slots and C3 4k)
  const int t_begin = (p.n_splits - 1 - split) * p.tiles_per_split;
  const int t_end = min(t_begin + p.tiles_per_split, p.n_tiles);
  auto sl = [&](int t) { return 32 * (t < p.skip_t0 ? t : t + p.skip_n); };  // first slot of tile t

  // Q operands (block diagonal, hi/lo f16). The setup is straight-line code -- every load is
  // unconditional (spare slots read query 0, a wave without tiles re-reads the split's last
  // tile) and spare slots store to a sink.
  TR A, B;
  // sink mode at D = 128 on 4-wave workgroups of up to two row sets: each tile's rope rows travel
  // with its K part (the 64 registers a tile more would spill the 8-wave kernels, whose waves have
  // half the register file, and the three-set one)
  constexpr bool RPRE = ROLL && D == 128 && NW == 4 && NSET <= 2;
  using RP = RopeRegs<D, RPRE>;
  RP RA, RB;
  const int tile0 = t_begin + wave;
  // The first tile is issued once q has arrived (q issued alone returns in ~0.3 us, while
  // behind every CU's first tile, ~19 MB queued at once, it returns only after them), and the
  // query's conversion below runs while the tile streams in. The scheduling barriers keep the
  // compiler from moving the tile loads above the wait or below the conversion.
  auto issue_first = [&]() {
    __builtin_amdgcn_s_waitcnt(0xf70);  // vmcnt(0): q has arrived
    __builtin_amdgcn_sched_barrier(0);
    const int ta = tile0 < t_end ? tile0 : t_end - 1;
    // a wave without a tile (the short last range) still issues its loads, but every lane at
    // the same address, so that they fetch next to nothing (C5 decode at 8193 slots: 65 splits,
    // 260 workgroups, four CUs hold two; 14.42 -> 12.92 us); the same for every load of a tile
    // the wave does not own below
    const bool own = tile0 < t_end;
    load_tile_k<D, DT, QUARTER, PR>(A, sl(ta), own ? g : 0, own ? n : 0, kbase, ksb, vsb);
    load_rope<D, RPRE>(RA, p.L, p.phys_limit, sl(ta), own ? g : 0, own ? n : 0);
    load_tile_v<D, DT, QUARTER, PR>(A, sl(ta), own ? g : 0, own ? n : 0, vbase);
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (I8) {
    // int8 operands: lane (gg, ii) of pass `pass` holds, for each int8 MFMA t8, the 16 dims
    // qk_dim(gg, 2 t8, 0..15) of A row ii's query (zero off the block diagonal) as hi and lo
    // bytes, value ~ scale * (hi + lo / 256) with the scale = max |value| of the row's 32-dim
    // scale block / 127. A thread takes one float4 of one (pass, A row, block): the 8 threads
    // of a block are neighbouring lanes, which share its max by three swaps, and each writes its
    // 4 dims' bytes into the lane and MFMA that hold them (PR = 4: lane group ii / 4, MFMA
    // 2 b + c / 4; PR = 8: lane group 2 (ii / 8) + c / 4, MFMA b).
    constexpr int QI = (NPK * 16 * NSB * 8 + NTHR - 1) / NTHR;  // float4 chunks per thread
    const int NQC = NP * 16 * NSB * 8;
    float4 qv[QI];
#pragma unroll
    for (int i = 0; i < QI; i++) {
      const int u = i * NTHR + tid;
      const int c = u & 7, unit = u >> 3;
      const int b = unit % NSB, ii = (unit / NSB) & 15, pass = unit / (16 * NSB);
      const int rho = PR * pass + (ii & (PR - 1));
      const bool use = u < NQC && rho < p.R;
      const int s = use ? rho / p.G : 0, h = use ? kvh * p.G + rho % p.G : 0;
      const int d = PR == 4 ? (ii >> 2) * (D / 4) + 32 * b + 4 * c : (ii >> 3) * (D / 2) + 32 * b + 4 * c;
      qv[i] = *(const float4*)(p.q + ((size_t)s * p.H + h) * D + (use ? d : 0));
      if (!use) qv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    issue_first();
    unsigned char* q8b = (unsigned char*)smem;                      // [NP][NT8][hi, lo][64] x 16 bytes
    float* qsc = (float*)(q8b + (size_t)NP * NT8 * 2 * 64 * 16);  // [NP][NSB][16 A rows]
#pragma unroll
    for (int i = 0; i < QI; i++) {
      const int u = i * NTHR + tid;
      const int c = u & 7, unit = u >> 3;
      const int b = unit % NSB, ii = (unit / NSB) & 15, pass = unit / (16 * NSB);
      float4 f = qv[i];
      f.x *= p.qscale;
      f.y *= p.qscale;
      f.z *= p.qscale;
      f.w *= p.qscale;
      float mx = fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w)));
      mx = fmaxf(mx, __shfl_xor(mx, 1));
      mx = fmaxf(mx, __shfl_xor(mx, 2));
      mx = fmaxf(mx, __shfl_xor(mx, 4));
      if (u < NQC) {
        const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
        const float y[4] = {f.x * inv, f.y * inv, f.z * inv, f.w * inv};
        uint32_t hv = 0, lv = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float hf = rintf(y[e]);
          const float lf = fminf(fmaxf(rintf((y[e] - hf) * 256.0f), -127.0f), 127.0f);
          hv |= ((uint32_t)(int)hf & 255u) << (8 * e);
          lv |= ((uint32_t)(int)lf & 255u) << (8 * e);
        }
        const int gg = PR == 4 ? ii >> 2 : 2 * (ii >> 3) + (c >> 2);
        const int t8 = PR == 4 ? 2 * b + (c >> 2) : b;
        const int l = 16 * gg + ii;
        uint32_t* o = (uint32_t*)(q8b + ((size_t)((pass * NT8 + t8) * 2) * 64 + l) * 16) + (c & 3);
        o[0] = hv;        // hi
        o[64 * 4] = lv;   // lo: the next 64 lanes' slots
        if (c == 0) qsc[(pass * NSB + b) * 16 + ii] = mx * (1.0f / (127.0f * 256.0f));
      }
    }
    // the off-diagonal operand slots are zero
    for (int i = tid; i < NP * NT8 * 2 * 64; i += NTHR) {
      const int l = i & 63, gg = l >> 4, ii = l & 15;
      const bool diag = PR == 4 ? (ii >> 2) == gg : (ii >> 3) == (gg >> 1);
      if (!diag) *(uint4*)(q8b + (size_t)i * 16) = make_uint4(0, 0, 0, 0);
    }
  } else {
    constexpr int QMAX = (NPK * NT * 64 + NTHR - 1) / NTHR;  // operand slots per thread
    const int NQ = NP * NT * 64;
    float qv[QMAX][8];
    bool use[QMAX];
#pragma unroll
    for (int i = 0; i < QMAX; i++) {
      const int idx = i * NTHR + tid;
      const int l = idx & 63, t = (idx >> 6) % NT, pass = (idx >> 6) / NT;
      const int gg = l >> 4, ii = l & 15;
      // A row ii: query row rho of the pass, nonzero on the k chunks of its row group's lane groups
      const int rho = PR * pass + (ii & (PR - 1));
      const bool diag = PR == 4 ? (ii >> 2) == gg : (ii >> 3) == (gg >> 1);
      use[i] = idx < NQ && diag && rho < p.R;
      const int s = use[i] ? rho / p.G : 0, h = use[i] ? kvh * p.G + rho % p.G : 0;
      const float* qr = p.q + ((size_t)s * p.H + h) * D + (use[i] ? qk_dim<D, QUARTER, PR>(gg, t, 0) : 0);
      const float4 a = *(const float4*)qr, b = *(const float4*)(qr + 4);
      qv[i][0] = a.x; qv[i][1] = a.y; qv[i][2] = a.z; qv[i][3] = a.w;
      qv[i][4] = b.x; qv[i][5] = b.y; qv[i][6] = b.z; qv[i][7] = b.w;
    }
    issue_first();
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

  float m[NPK][RL], lsum[NPK][RL];
#pragma unroll
  for (int i = 0; i < NPK; i++)
#pragma unroll
    for (int j = 0; j < RL; j++) { m[i][j] = -1e30f; lsum[i][j] = 0.0f; }
  floatx4 o[NSET][D / 16];
#pragma unroll
  for (int s = 0; s < NSET; s++)
#pragma unroll
    for (int i = 0; i < D / 16; i++) o[s][i] = floatx4{0, 0, 0, 0};

  bool rescale = false;  // the last qk_softmax raised a reference max: pv rescales O first
  auto qk_softmax = [&](const TR& T, const RP& Rr, int tile) {
    const int j0 = sl(tile);
    // ---------------- K operands ----------------
    // f16 K operand for QK MFMA t of 16-slot group t2: as loaded (f16 cache) or materialized
    // once after the read-time rotation (sink mode); q8 codes without rotation enter the int8
    // MFMAs as they are
    half8 kb[2][ROLL ? NT : 1];
    auto kop = [&](int t2, int t) -> half8 {
      if constexpr (ROLL) {
        return kb[t2][t];
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
        // (the rows in Rr, or read here without the prefetch)
        const long ri = RPRE ? 0 : rope_row(p.L, p.phys_limit, j0 + 16 * t2 + n);
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
            float c, s;
            if constexpr (RPRE) {
              const float4 cv = Rr.c[t2][2 * t + e / 4], sv = Rr.s[t2][2 * t + e / 4];
              c = (e & 3) == 0 ? cv.x : (e & 3) == 1 ? cv.y : (e & 3) == 2 ? cv.z : cv.w;
              s = (e & 3) == 0 ? sv.x : (e & 3) == 1 ? sv.y : (e & 3) == 2 ? sv.z : sv.w;
            } else {
              c = ct[8 * t + e];
              s = st[8 * t + e];
            }
            // the products with s as fma(x, s, +0) (the same value as x * s but for the sign of
            // a zero, which the sum below cannot see): the f16 x then enters a mixed-precision
            // fma directly instead of being converted first. The product with c and the sum are
            // contracted into that fma (one f32 rounding where the reference's rope has two;
            // the result is rounded to f16 at once, so the keys match to the f16 rounding)
            const float bs = __builtin_fmaf(b2[e], s, 0.0f), as = __builtin_fmaf(a[e], s, 0.0f);
            r0.h[e] = (_Float16)__fadd_rn(__fmul_rn(a[e], c), -bs);
            r1.h[e] = (_Float16)__fadd_rn(__fmul_rn(b2[e], c), as);
          }
          kb[t2][t] = r0.h;
          kb[t2][HT + t] = r1.h;
        }
      }
    }

    // ---------------- QK + online softmax, one pass per PR query rows ----------------
    // The reference max of a row is raised only when a tile's max exceeds it by more than 8 (in
    // log2 units, so P <= 2^8 stays well inside f16); most tiles then leave O and l unscaled.
    float xs[NPK][RL][2], mts[NPK][RL];
#pragma unroll
    for (int pass = 0; pass < NPK; pass++) {
      if (pass >= NP) break;
      float sc[2][RL];
      // int8: the query scales of the lane's C rows 4g .. 4g+3, one float4 a block
      float4 qsv[I8 ? NSB : 1];
      if constexpr (I8) {
        const float* qsc = (const float*)((const unsigned char*)smem + (size_t)NP * NT8 * 2 * 64 * 16);
#pragma unroll
        for (int b = 0; b < NSB; b++) qsv[b] = *(const float4*)(qsc + (pass * NSB + b) * 16 + 4 * g);
      }
#pragma unroll
      for (int t2 = 0; t2 < 2; t2++) {
        float v[4];
        if constexpr (I8) {
          // C row 4g+e of block b: the integer sum of hi x code plus that of lo x code / 256,
          // exact in int32 (|sum| <= 32 * 127 * 127 a block), times the query and key scales
          const u32x4v* q8o = (const u32x4v*)smem;
          i32x4v ch[NSB], cl[NSB];
#pragma unroll
          for (int b = 0; b < NSB; b++) ch[b] = cl[b] = i32x4v{0, 0, 0, 0};
#pragma unroll
          for (int t8 = 0; t8 < NT8; t8++) {
            const int b = PR == 4 ? t8 >> 1 : t8;
            const i32x4v ahi = __builtin_bit_cast(i32x4v, q8o[((pass * NT8 + t8) * 2 + 0) * 64 + lane]);
            const i32x4v alo = __builtin_bit_cast(i32x4v, q8o[((pass * NT8 + t8) * 2 + 1) * 64 + lane]);
            const i32x4v kt = __builtin_bit_cast(i32x4v, T.kr[t2][t8]);
            ch[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, kt, ch[b], 0, 0, 0);
            cl[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, kt, cl[b], 0, 0, 0);
          }
#pragma unroll
          for (int e = 0; e < 4; e++) {
            float acc = 0.0f;
#pragma unroll
            for (int b = 0; b < NSB; b++) {
              const float qk = (e == 0 ? qsv[b].x : e == 1 ? qsv[b].y : e == 2 ? qsv[b].z : qsv[b].w) * T.ksc[t2][b];
              acc = fmaf((float)(ch[b][e] * 256 + cl[b][e]), qk, acc);
            }
            v[e] = acc;
          }
        } else {
          floatx4 c = floatx4{0, 0, 0, 0};
#pragma unroll
          for (int t = 0; t < NT; t++) {
            H8 ahi, alo;
            ahi.u = qs[((pass * NT + t) * 2 + 0) * 64 + lane];
            alo.u = qs[((pass * NT + t) * 2 + 1) * 64 + lane];
            const half8 kt = kop(t2, t);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi.h, kt, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo.h, kt, c, 0, 0, 0);
          }
#pragma unroll
          for (int e = 0; e < 4; e++) v[e] = c[e];
        }
        // Lane group g' holds output rows 4g'..4g'+3 (v[0..3]) of the slot. permlane32_swap(a, b)
        // leaves lanes l < 32 with {a[l], a[l+32]} and lanes l >= 32 with {b[l-32], b[l]};
        // permlane16_swap does the same between lane groups 0/1 and 2/3.
        if constexpr (PR == 4) {
          // output row 4g'+e = query row e of the pass over quarter g': reduce-scatter over the
          // 4 lane groups, lane group g ends with query row g
          const auto u0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[0]), __float_as_uint(v[2]), false, false);
          const auto u1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[1]), __float_as_uint(v[3]), false, false);
          const float k0 = __uint_as_float(u0[0]) + __uint_as_float(u0[1]);  // rows 0,1: dims of v[0]; rows 2,3: v[2]
          const float k1 = __uint_as_float(u1[0]) + __uint_as_float(u1[1]);
          const auto u2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(k0), __float_as_uint(k1), false, false);
          sc[t2][0] = __uint_as_float(u2[0]) + __uint_as_float(u2[1]);
        } else {
          // output row 4g'+e = query row 4(g' & 1) + e of the pass over half g' >> 1: one swap
          // adds the halves (lane groups g' and g'+2), lane group g ends with rows row_of(pass, 0)
          // (from v[0] / v[1]) and row_of(pass, 1) (from v[2] / v[3])
          const auto u0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[0]), __float_as_uint(v[1]), false, false);
          const auto u1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[2]), __float_as_uint(v[3]), false, false);
          sc[t2][0] = __uint_as_float(u0[0]) + __uint_as_float(u0[1]);
          sc[t2][RL - 1] = __uint_as_float(u1[0]) + __uint_as_float(u1[1]);
        }
      }
      // mask + online softmax for the lane's rows
#pragma unroll
      for (int i = 0; i < RL; i++) {
        const int rho = row_of(pass, i);
        const int qi = rho / p.G;
        const bool row_ok = rho < p.R;
        const int limit = p.pos_base + qi;
        float x[2];
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
          const int P = j0 + 16 * t2 + n;
          const int Lg = ROLL ? ring.logical(P) : P;  // a plain cache is never a ring
          const bool ok = row_ok && P < p.n_scan && P < p.phys_limit && Lg <= limit;
          x[t2] = ok ? sc[t2][i] : -INFINITY;
        }
        xs[pass][i][0] = x[0];
        xs[pass][i][1] = x[1];
        mts[pass][i] = group16_max(fmaxf(x[0], x[1]));
      }
    }
    bool grow = false;
#pragma unroll
    for (int pass = 0; pass < NPK; pass++) {
      if (pass >= NP) break;
#pragma unroll
      for (int i = 0; i < RL; i++) grow = grow || mts[pass][i] > m[pass][i] + 8.0f;
    }
    rescale = __any(grow);
#pragma unroll
    for (int pass = 0; pass < NPK; pass++) {
      if (pass >= NP) break;
#pragma unroll
      for (int i = 0; i < RL; i++) {
        const int rho = row_of(pass, i);
        if (rescale) {
          const float mn = fmaxf(m[pass][i], mts[pass][i]);
          // the hardware exp2 (no denormal results: a factor below 2^-126 becomes 0, which
          // changes no f32 sum that also holds the tile's own terms >= 2^-8, nor an f16 P)
          const float corr = __builtin_amdgcn_exp2f(m[pass][i] - mn);
          lsum[pass][i] *= corr;
          m[pass][i] = mn;
          if (n == 0 && rho < RS) cl[rho] = corr;
        }
        const float p0 = __builtin_amdgcn_exp2f(xs[pass][i][0] - m[pass][i]);
        const float p1 = __builtin_amdgcn_exp2f(xs[pass][i][1] - m[pass][i]);
        lsum[pass][i] += p0 + p1;
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
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // ---------------- PV ----------------
  auto pv = [&](const TR& T) {
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
      if (rescale) {
        const float cr = cl[16 * st + n];
#pragma unroll
        for (int i = 0; i < D / 16; i++) o[st][i] *= cr;
      }
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

  // software pipeline over this wave's tiles (every NW-th tile from tile0): two tiles are in
  // flight. For q8 each phase's registers are re-issued for the tile two ahead as soon as that
  // phase of the current tile is done (K part after QK + softmax, V part after PV), so the memory
  // queue refills while the rest of the tile computes. The loop bodies' loads are unconditional
  // and there is no early exit, so every path into a loop head has the same loads outstanding
  // and the compiler counts them instead of draining them.
  const int nmy = tile0 < t_end ? (t_end - tile0 + NW - 1) / NW : 0;  // this wave's tiles
  // a tile's K part (with its rope rows) and its V part
  auto issue_k = [&](TR& T, RP& Rr, int tile, int gg, int nn) {
    load_tile_k<D, DT, QUARTER, PR>(T, sl(tile), gg, nn, kbase, ksb, vsb);
    load_rope<D, RPRE>(Rr, p.L, p.phys_limit, sl(tile), gg, nn);
  };
  auto issue_v = [&](TR& T, int tile, int gg, int nn) {
    load_tile_v<D, DT, QUARTER, PR>(T, sl(tile), gg, nn, vbase);
  };
  int it = 0;
  if constexpr (ONE) {
    (void)it;
    if (nmy >= 1) {
      qk_softmax(A, RA, tile0);
      pv(A);
    }
  } else if constexpr (DT == KV_Q8) {
    {
      const int tb = nmy > 1 ? tile0 + NW : (tile0 < t_end ? tile0 : t_end - 1);
      issue_k(B, RB, tb, nmy > 1 ? g : 0, nmy > 1 ? n : 0);
      issue_v(B, tb, nmy > 1 ? g : 0, nmy > 1 ? n : 0);
    }
    for (; it + 4 <= nmy; it += 2) {
      const int ta = tile0 + it * NW;
      qk_softmax(A, RA, ta);
      issue_k(A, RA, ta + 2 * NW, g, n);
      pv(A);
      issue_v(A, ta + 2 * NW, g, n);
      qk_softmax(B, RB, ta + NW);
      issue_k(B, RB, ta + 3 * NW, g, n);
      pv(B);
      issue_v(B, ta + 3 * NW, g, n);
    }
    // the last one to three tiles: A and B hold tiles it and it + 1
    const int r = nmy - it;
    const int ta = tile0 + it * NW;
    if (r >= 1) {
      qk_softmax(A, RA, ta);
      pv(A);
    }
    if (r == 3) {
      issue_k(A, RA, ta + 2 * NW, g, n);
      issue_v(A, ta + 2 * NW, g, n);
    }
    if (r >= 2) {
      qk_softmax(B, RB, ta + NW);
      pv(B);
    }
    if (r == 3) {
      qk_softmax(A, RA, ta + 2 * NW);
      pv(A);
    }
  } else {
    // f16 tiles are twice as large: the registers hold two whole tiles, so the next tile is
    // issued before a tile is processed and re-issued only after both of its phases (past the
    // end the prefetch is issued at one address)
    for (; it + 2 <= nmy; it += 2) {
      const int ta = tile0 + it * NW;
      issue_k(B, RB, ta + NW, g, n);
      issue_v(B, ta + NW, g, n);
      qk_softmax(A, RA, ta);
      pv(A);
      const bool next = it + 2 < nmy;
      const int tn = next ? ta + 2 * NW : ta + NW;
      issue_k(A, RA, tn, next ? g : 0, next ? n : 0);
      issue_v(A, tn, next ? g : 0, next ? n : 0);
      qk_softmax(B, RB, ta + NW);
      pv(B);
    }
    if (it < nmy) {
      qk_softmax(A, RA, tile0 + it * NW);
      pv(A);
    }
  }

  // ---------------- combine the waves of the workgroup ----------------
  // Each wave leaves its raw partial (no rescaling, so nothing to wait for) in its own part of
  // LDS: the row maxima and sums in two small arrays the tile loop never touches, the o rows
  // (padded by 4 floats to spread the banks) over its own P tiles, which no other wave reads;
  // one barrier publishes them. The sum over the waves (below) rescales to the workgroup maximum.
  __shared__ __align__(16) float s_mw[RS][NW];
  __shared__ __align__(16) float s_lw[RS][NW];
  constexpr int DP = SM::DP;
  const size_t wbytes = SM::wave_bytes(p.R);
#pragma unroll
  for (int pass = 0; pass < NPK; pass++) {
    if (pass >= NP) break;
#pragma unroll
    for (int i = 0; i < RL; i++) {
      const float lt = group16_sum(lsum[pass][i]);
      const int rho = row_of(pass, i);
      if (n == 0 && rho < p.R) {
        s_mw[rho][wave] = m[pass][i];
        s_lw[rho][wave] = lt;
      }
    }
  }
#pragma unroll
  for (int st = 0; st < NSET; st++) {
    const int rho = 16 * st + n;
    if (rho < p.R) {
      float* orow = (float*)(pbase + wave * wbytes) + rho * DP + 8 * g;
      // o[st][2b + par][e] holds dim 32b + 8g + 2e + par: dims 32b + 8g + 4h .. +3 are
      // (e, par) = (2h, 0), (2h, 1), (2h + 1, 0), (2h + 1, 1)
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int h = 0; h < 2; h++)
          *(float4*)(orow + 32 * b + 4 * h) = make_float4(o[st][2 * b][2 * h], o[st][2 * b + 1][2 * h],
                                                          o[st][2 * b][2 * h + 1], o[st][2 * b + 1][2 * h + 1]);
    }
  }
  __syncthreads();

  const bool single = p.n_splits == 1;
  constexpr int kSC1 = 16;  // cache policy sc1: agent-coherent (written through / read from memory)
  constexpr int UPR = D / 64;  // merge units per row
  const int NS = p.n_splits;
  const int units = p.R * UPR;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.ws + (size_t)kvh * units * NS * kUnitF4), (short)0, 0x7fffffff, 0x00020000);
  // Each column (CW floats) of the R x D partial is summed over the waves by one thread, every
  // LDS read of the column independent of the others (a row's maxima and sums are two vector
  // reads a 4 waves); the column loop has a compile-time trip bound and is unrolled, so a
  // thread's columns are read together. The 8-wave kernels (D=128, up to 16 rows) take float2
  // columns, so that twice the threads share the pass (C3 32k 17.58 -> 17.41 us)
  constexpr int CW = NW == 8 ? 2 : 4;
  constexpr int CPR = D / CW;  // columns per row
  constexpr int CMAX = (RS * CPR + NTHR - 1) / NTHR;
  const int NC = p.R * CPR;
#pragma unroll
  for (int j = 0; j < CMAX; j++) {
    const int c = tid + j * NTHR;
    if (c < NC) {
      const int rho = c / CPR, d = CW * (c % CPR);
      float v[NW][CW], mw[NW], lw[NW];
#pragma unroll
      for (int w = 0; w < NW; w += 4) {
        *(float4*)&mw[w] = *(const float4*)&s_mw[rho][w];
        *(float4*)&lw[w] = *(const float4*)&s_lw[rho][w];
      }
#pragma unroll
      for (int w = 0; w < NW; w++) {
        const float* src = (const float*)(pbase + w * wbytes) + rho * DP + d;
        if constexpr (CW == 4) {
          *(float4*)v[w] = *(const float4*)src;
        } else {
          *(float2*)v[w] = *(const float2*)src;
        }
      }
      float mx = mw[0];
#pragma unroll
      for (int w = 1; w < NW; w++) mx = fmaxf(mx, mw[w]);
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      float lt = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; w++) {
        const float f = __builtin_amdgcn_exp2f(mw[w] - mx);
#pragma unroll
        for (int e = 0; e < CW; e++) acc[e] += v[w][e] * f;
        lt += lw[w] * f;
      }
      if (single) {
        const int s = rho / p.G, h = kvh * p.G + rho % p.G;
        float r[CW];
#pragma unroll
        for (int e = 0; e < CW; e++) r[e] = acc[e] / lt;
        if (p.gate) {
          const float* gr = p.gate + ((size_t)s * p.H + h) * p.gate_stride + d;
#pragma unroll
          for (int e = 0; e < CW; e++) r[e] = r[e] / (1.0f + expf(-gr[e]));
        }
        float* orow = p.out + ((size_t)s * p.H + h) * D + d;
        if constexpr (CW == 4) {
          *(float4*)orow = make_float4(r[0], r[1], r[2], r[3]);
        } else {
          *(float2*)orow = make_float2(r[0], r[1]);
        }
      } else if (split != p.withhold_split) {
        const int slot = ((rho * UPR + d / 64) * NS + split) * kUnitF4;
        const int off = slot * 16 + (d % 64) * 4;
        const float4 ml = make_float4(mx, lt, 0.0f, 0.0f);
        // plain stores into the XCD's L2 (see xcd_local), else written through
        if (p.xcd_local > 0) {
          if constexpr (CW == 4)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, make_float4(acc[0], acc[1], acc[2], acc[3])), wrs, off, 0, 0);
          else
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2v, make_float2(acc[0], acc[1])), wrs, off, 0, 0);
          if (d % 64 == 0) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, ml), wrs, (slot + 16) * 16, 0, 0);
        } else {
          if constexpr (CW == 4)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, make_float4(acc[0], acc[1], acc[2], acc[3])), wrs, off, 0, kSC1);
          else
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2v, make_float2(acc[0], acc[1])), wrs, off, 0, kSC1);
          if (d % 64 == 0) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, ml), wrs, (slot + 16) * 16, 0, kSC1);
        }
      }
    }
  }
  const int first_merger = NS - p.n_mergers;
  if (single || split < first_merger) return;

  // ---------------- merge (the last n_mergers splits) ----------------
  // Merger j (split first_merger + j) takes units j, j + n_mergers, .. (unit = one row x 64
  // dims). The unit's slots of every split are polled until none holds kPartialEmpty (the data
  // itself is the completion signal: no flag, ticket or store acknowledgement to wait for),
  // merged by log-sum-exp, the output stored and kPartialEmpty written back for the next launch.
  // Mergers are the highest split indices, so workgroups are dispatched before the mergers that
  // wait on them; the host also sizes the grid to fit the GPU at once. The wait is bounded
  // (p.spin_limit rounds): a merger that gives up stores NaN and raises p.err.
  // Up to 32 splits one wave merges a unit alone: no barrier and no LDS, so a unit is done as
  // soon as its own slots have arrived (C3 32k 18.65 -> 17.8 us, C4 verify5 18.4 -> 17.0); when
  // units outnumber the mergers, wave w of merger j takes units j + w * n_mergers, ... More
  // splits (C5 decode: 65) are shared by the workgroup's waves (one wave polling 17 slots a lane
  // a round measured 1.2 us slower), which meet once, at the sum of their parts.
  // Lane (k, c) of split group kg holds float4 column c of splits kg, kg + KG, .. (OB at a time)
  // and every lane l the (m, l) of splits l, l + 64, ..; the lane reductions give every wave the
  // log-sum-exp maximum and sum (the same in every wave, bit for bit), and a lane takes its
  // splits' weights from their lanes by ds_bpermute. The empty markers go back as each batch is
  // consumed, with the split in the scalar offset so that consecutive stores share their address
  // registers (a register rewritten under a pending store makes the compiler wait for that
  // store's acknowledgement).
  constexpr int MLC = (kMaxSplits + 63) / 64;  // (m, l) slots per lane
  const int c = lane & 15, k = lane >> 4;
  const u32x4v empty4 = {kPartialEmpty, kPartialEmpty, kPartialEmpty, kPartialEmpty};
  bool gave_up = false;  // wave-uniform
  auto merge = [&](auto wg_tag) {
    constexpr bool WG = decltype(wg_tag)::value;
    constexpr int KG = WG ? 4 * NW : 4;  // split groups
    // o slots per lane and batch: 8 for one wave (32 splits); across the workgroup 4, or 5 for
    // the D=256 one-tile kernel (80 a batch: its 8193-8448-slot contexts take 65-66 splits)
    constexpr int OB = WG ? ((ONE && D == 256) ? 5 : 4) : 8;
    const int kg = WG ? 4 * wave + k : k;
    // (m, l) registers per lane: one covers the 32 splits a wave merges alone
    constexpr int MLU = WG ? MLC : 1;
    const int j0 = split - first_merger;
    for (int u = WG ? j0 : j0 + wave * p.n_mergers; u < units; u += WG ? p.n_mergers : p.n_mergers * NW) {
      const int rho = u / UPR, d0 = (u % UPR) * 64;
      const int ubase = u * NS * kUnitF4;
      // the gate's sigmoid denominators (gate_sigmoid.wgsl: x / (1 + exp(-g))) before the wait,
      // so that its load is not a memory round trip after the merge
      float gden[4] = {1.0f, 1.0f, 1.0f, 1.0f};
      if (p.gate) {
        const float* gr = p.gate + ((size_t)(rho / p.G) * p.H + kvh * p.G + rho % p.G) * p.gate_stride + d0 + 4 * c;
#pragma unroll
        for (int e = 0; e < 4; e++) gden[e] = 1.0f + expf(-gr[e]);
      }
      floatx4 v[OB];
      float2 ml[MLU];
      // poll batch b0 of the o slots (and the (m, l) slots) until nothing is missing; bounded:
      // every split of the grid runs to completion on its own, so the data arrives, and the
      // bound only guarantees an exit. Returns false when the bound ran out.
      auto poll = [&](int b0, bool with_ml) -> bool {
        for (int it = 0; it < p.spin_limit; it++) {
          // a compiler memory barrier: every round's loads are issued again (other workgroups
          // write the slots; without it the compiler may reuse the last round's values)
          __asm__ volatile("" ::: "memory");
          bool missing = false;
#pragma unroll
          for (int i = 0; i < OB; i++) {
            const int sp = b0 + kg + KG * i;
            v[i] = sp < NS ? __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (ubase + sp * kUnitF4 + c) * 16, 0, kSC1))
                           : floatx4{0.f, 0.f, 0.f, 0.f};
          }
          if (with_ml) {
#pragma unroll
            for (int j = 0; j < MLU; j++) {
              const int sp = 64 * j + lane;
              ml[j] = make_float2(-INFINITY, 0.0f);
              if (64 * j < NS && sp < NS)
                ml[j] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(wrs, (ubase + sp * kUnitF4 + 16) * 16, 0, kSC1));
            }
#pragma unroll
            for (int j = 0; j < MLU; j++)
              missing = missing || __float_as_uint(ml[j].x) == kPartialEmpty || __float_as_uint(ml[j].y) == kPartialEmpty;
          }
#pragma unroll
          for (int i = 0; i < OB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) missing = missing || __float_as_uint(v[i][e]) == kPartialEmpty;
          if (!__any(missing)) return true;
          __builtin_amdgcn_s_sleep(1);
        }
        return false;
      };
      // the weights of every split: w[j] at lane l is split 64 j + l (0 past the last split)
      float w[MLU];
      // consume a batch: weighted sum, then mark its slots empty again. Every weight is fetched
      // before any is used (one LDS wait), and slots past the last split hold zeros.
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      const int vo = (ubase + kg * kUnitF4 + c) * 16;
      auto consume = [&](int b0) {
        float wi[OB];
#pragma unroll
        for (int i = 0; i < OB; i++) {
          const int sp = b0 + kg + KG * i;
          // the weight of split sp from lane sp % 64 of w[sp / 64]
          wi[i] = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (sp & 63), __float_as_int(w[0])));
#pragma unroll
          for (int j = 1; j < MLU; j++) {
            const float t = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (sp & 63), __float_as_int(w[j])));
            wi[i] = (sp >> 6) == j ? t : wi[i];
          }
        }
#pragma unroll
        for (int i = 0; i < OB; i++) {
          acc.x += v[i][0] * wi[i];
          acc.y += v[i][1] * wi[i];
          acc.z += v[i][2] * wi[i];
          acc.w += v[i][3] * wi[i];
        }
#pragma unroll
        for (int i = 0; i < OB; i++)
          if (b0 + kg + KG * i < NS) __builtin_amdgcn_raw_buffer_store_b128(empty4, wrs, vo, (b0 + KG * i) * kUnitF4 * 16, kSC1);
      };
      if constexpr (WG) {
        gave_up = !poll(0, true) || gave_up;
      } else {
        // one wave, every split in one batch: two poll rounds in flight, each check waits only
        // for the older round, so a slot that lands is seen about half a round trip sooner.
        // The loads are unconditional (slots past the last split re-read the last split's, and
        // are zeroed once complete), so the wait can count the younger round's loads.
        auto issue = [&](floatx4 (&vv)[OB], float2 (&mm)[MLU]) {
          __asm__ volatile("" ::: "memory");  // issued again every round (see poll)
#pragma unroll
          for (int i = 0; i < OB; i++) {
            const int sp = min(kg + KG * i, NS - 1);
            vv[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (ubase + sp * kUnitF4 + c) * 16, 0, kSC1));
          }
          mm[0] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(wrs, (ubase + min(lane, NS - 1) * kUnitF4 + 16) * 16, 0, kSC1));
          __builtin_amdgcn_sched_barrier(0);  // the round is issued before the older one is checked
        };
        auto complete = [&](const floatx4 (&vv)[OB], const float2 (&mm)[MLU]) {
          bool missing = __float_as_uint(mm[0].x) == kPartialEmpty || __float_as_uint(mm[0].y) == kPartialEmpty;
#pragma unroll
          for (int i = 0; i < OB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) missing = missing || __float_as_uint(vv[i][e]) == kPartialEmpty;
          return !__any(missing);
        };
        floatx4 v2[OB];
        float2 ml2[MLU];
        bool ok = false;
        issue(v, ml);
        for (int it = 0; it < p.spin_limit; it++) {
          issue(v2, ml2);
          if (complete(v, ml)) {
            ok = true;
            break;
          }
          issue(v, ml);
          if (complete(v2, ml2)) {
#pragma unroll
            for (int i = 0; i < OB; i++) v[i] = v2[i];
            ml[0] = ml2[0];
            ok = true;
            break;
          }
        }
        gave_up = !ok || gave_up;
#pragma unroll
        for (int i = 0; i < OB; i++)
          if (kg + KG * i >= NS) v[i] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (lane >= NS) ml[0] = make_float2(-INFINITY, 0.0f);
      }
      {
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < MLU; j++) M = fmaxf(M, ml[j].x);
        M = wave_max(M);
        float e[MLU], lt = 0.0f;
#pragma unroll
        for (int j = 0; j < MLU; j++) {
          e[j] = __builtin_amdgcn_exp2f(ml[j].x - M);
          lt += ml[j].y * e[j];
        }
        const float rl = 1.0f / wave_sum(lt);
#pragma unroll
        for (int j = 0; j < MLU; j++) w[j] = e[j] * rl;
      }
      // the (m, l) slots back to empty once every wave that reads them has (one wave: now;
      // the workgroup: wave 0 after the waves meet below)
      auto reset_ml = [&]() {
        const int vm = (ubase + lane * kUnitF4 + 16) * 16;
#pragma unroll
        for (int j = 0; j < MLU; j++)
          if (64 * j + lane < NS) __builtin_amdgcn_raw_buffer_store_b128(empty4, wrs, vm, 64 * j * kUnitF4 * 16, kSC1);
      };
      if constexpr (!WG) reset_ml();
      consume(0);
      for (int b0 = KG * OB; b0 < NS; b0 += KG * OB) {
        gave_up = !poll(b0, false) || gave_up;
        consume(b0);
      }
      // the four split groups of a wave hold the same column in lanes c, c + 16, c + 32, c + 48:
      // two permlane swaps sum them
      {
        float* a4 = &acc.x;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float2 t = pair16(a4[e]);
          a4[e] = t.x + t.y;
          t = pair32(a4[e]);
          a4[e] = t.x + t.y;
        }
      }
      if constexpr (WG) {
        // the waves' parts meet in LDS (the operand space: the wave combine above no longer
        // reads it), one barrier; wave 0 sums them
        float4* red = (float4*)smem;  // [NW][16]
        int* gu = (int*)(red + NW * 16);
        if (lane < 16) red[wave * 16 + c] = acc;
        if (lane == 0) gu[wave] = gave_up;
        __syncthreads();
        if (wave == 0) {
          reset_ml();
          float4 part[NW];
          int g2 = 0;
#pragma unroll
          for (int w2 = 0; w2 < NW; w2++) {
            part[w2] = red[w2 * 16 + c];
            g2 |= gu[w2];
          }
          acc = part[0];
#pragma unroll
          for (int w2 = 1; w2 < NW; w2++) {
            acc.x += part[w2].x;
            acc.y += part[w2].y;
            acc.z += part[w2].z;
            acc.w += part[w2].w;
          }
          gave_up = g2 != 0;
        }
      }
      if ((!WG || wave == 0) && lane < 16) {
        const int s = rho / p.G, h = kvh * p.G + rho % p.G, d = d0 + 4 * c;
        float r[4] = {acc.x, acc.y, acc.z, acc.w};
        if (p.gate) {
#pragma unroll
          for (int e = 0; e < 4; e++) r[e] = r[e] / gden[e];
        }
        if (gave_up) r[0] = r[1] = r[2] = r[3] = __builtin_nanf("");
        *(float4*)(p.out + ((size_t)s * p.H + h) * D + d) = make_float4(r[0], r[1], r[2], r[3]);
      }
      // the next unit's parts reuse the LDS space
      if constexpr (WG) {
        if (u + p.n_mergers < units) __syncthreads();
      }
    }
  };
  if (NS > 32)
    merge(std::true_type{});
  else
    merge(std::false_type{});
  // one vector store from one lane, system scope: the host reads the word without a copy. 2:
  // the L2 exchange was on, so a split may have stored on another XCD (the library then writes
  // partials through); a split withheld by the test hook is no placement question (1)
  if (gave_up && lane == 0)
    __hip_atomic_store(p.err, (p.xcd_local > 0 && p.withhold_split < 0) ? 2u : 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

static int nset_for(int R) { return (R + 15) / 16; }
// query rows per QK pass: 8 once there are more than 4
static int rows_per_pass(int R) { return R > 4 ? 8 : 4; }

// dynamic LDS of the tile loop and wave combine (DecodeSmem::total for the launch's template
// arguments); the split merge uses none
// NW: waves per workgroup (the most a shape launches with, 8 for D=128 single-set, bounds the rest);
// PR: query rows per pass
static size_t decode_lds_bytes(int D, int dtype, int R, int NW, int PR) {
  const int nset = nset_for(R);
  const int RS = 16 * nset, NT = D / 32, NBV = dtype == KV_Q8 ? D / 32 : 1;
  const size_t t = (size_t)NBV * RS * 32 * 2 + (size_t)RS * 4, o = (size_t)R * (D + 4) * 4;
  return (size_t)((R + PR - 1) / PR) * NT * 2 * 64 * 16 + 32 + (size_t)NW * (t > o ? t : o);
}
constexpr size_t kDecodeLdsMax = 158 * 1024;  // + the static wave maxima and sums (at most 1.5 KB)

bool decode_supported(const LayerView& L, int S, int H) {
  if (L.dtype == KV_F32) return false;
  if (L.D != 128 && L.D != 256) return false;
  const int G = H / L.kv_heads;
  const int R = G * S;
  // up to 48 rows at D=128 and 20 at D=256 (past that the D=256 row sets no longer fit the
  // register file), within LDS; more go to the prefill kernel
  const int nw_max = (L.D == 128 && nset_for(R) == 1) ? 8 : 4;
  return R >= 1 && nset_for(R) <= 3 && (L.D == 128 || R <= 20) &&
         decode_lds_bytes(L.D, L.dtype, R, nw_max, rows_per_pass(R)) <= kDecodeLdsMax;
}

bool decode_preferred(const LayerView& L, int S, int H) {
  if (!decode_supported(L, S, H)) return false;
  const int R = (H / L.kv_heads) * S;
  if (R <= 16 || L.ring.roll) return true;  // one row set, or read-time rotation
  if (L.D == 256) return false;             // more row sets at D=256 spill
  return L.dtype == KV_Q8 && R <= 24;
}

// Split-K plan of one decode launch. Waves: D=128 single-set shapes run 8-wave workgroups (every
// wave takes at least one tile) when each CU gets 8 tiles or more, otherwise 4-wave workgroups,
// which split a short range over twice as many CUs. Splits: one workgroup per CU,
// tiles_per_split = ceil(tiles * KV / CUs), at least one tile per wave, at most kMaxSplits
// splits. Residency: the merge needs every split to run, so the grid is capped at the
// workgroups the GPU holds at once (resident_per_cu x CUs, from the kernel's occupancy); below
// two splits per kv head there is a single split and no merge.
bool decode_plan(const LayerView& L, int S, int H, int pos_base, int num_cus, int resident_per_cu, DecodePlan* out) {
  if (!decode_supported(L, S, H)) return false;
  DecodePlan s;
  const int R = (H / L.kv_heads) * S;
  s.nset = nset_for(R);
  s.passes = (R + rows_per_pass(R) - 1) / rows_per_pass(R);
  s.n_scan = (L.ring.roll && L.ring.head != 0) ? L.max_seq : pos_base + S;
  s.phys_limit = L.ring.roll ? L.max_seq : L.cap;
  s.n_tiles = (s.n_scan + 31) / 32;
  // sink mode after the wrap scans every physical slot; the ring slots whose logical index lies
  // past the last row's position (the room eviction left) are masked for every row, and the
  // longest run of whole tiles of them is skipped (C4 at position 100000: 11 of 129 tiles)
  s.skip_t0 = 0;
  s.skip_n = 0;
  if (L.ring.roll && L.ring.head != 0) {
    const int sk = L.ring.sinks, W = L.ring.W;
    const int first = pos_base + S;  // the first logical slot no row sees
    if (first >= sk && first < sk + W) {
      const int a = sk + (first - sk + L.ring.head) % W;  // its physical slot
      const int len = sk + W - first;                       // masked ring slots
      auto take = [&](int x, int y) {                       // physical slots [x, y)
        const int t0 = (x + 31) / 32, t1 = y / 32;
        if (t1 - t0 > s.skip_n) {
          s.skip_t0 = t0;
          s.skip_n = t1 - t0;
        }
      };
      if (a + len <= sk + W) {
        take(a, a + len);
      } else {
        take(a, sk + W);
        take(sk, sk + (a + len - (sk + W)));
      }
      // the last tile may be partial: only whole tiles below n_scan are skipped
      if (s.skip_t0 + s.skip_n > s.n_scan / 32) s.skip_n = s.n_scan / 32 - s.skip_t0;
      if (s.skip_n < 0) s.skip_n = 0;
      s.n_tiles -= s.skip_n;
    }
  }
  const int cus = num_cus > 0 ? num_cus : 256;
  s.waves = (L.D == 128 && s.nset == 1 && (long)s.n_tiles * L.kv_heads >= 8L * cus) ? 8 : 4;
  int tps = (s.n_tiles * L.kv_heads + cus - 1) / cus;
  tps = tps < s.waves ? s.waves : tps;
  const int tps_min = (s.n_tiles + kMaxSplits - 1) / kMaxSplits;
  tps = tps < tps_min ? tps_min : tps;
  const long resident = (long)(resident_per_cu > 0 ? resident_per_cu : 1) * cus;
  // a q8 or sink-mode 4-wave single-set plan whose waves would take two tiles at one workgroup a
  // CU takes one tile a wave instead when a CU holds two workgroups and the GPU holds the larger
  // grid (q8 and rotated tiles cost more compute per byte, so two tiles in series on one wave
  // cost more than a CU running two workgroups: C4 decode 10.67 -> 10.23 us; measured slower for
  // plain f16)
  if ((L.dtype == KV_Q8 || L.ring.roll) && s.waves == 4 && s.nset == 1 && resident_per_cu >= 2 && tps > s.waves && tps <= 2 * s.waves) {
    const int ns1 = (s.n_tiles + s.waves - 1) / s.waves;
    if (ns1 <= kMaxSplits && (long)ns1 * L.kv_heads <= resident) tps = s.waves;
  }
  int ns = (s.n_tiles + tps - 1) / tps;
  const int max_splits = (int)(resident / L.kv_heads);
  if (max_splits < 2) {
    tps = s.n_tiles;
    ns = 1;
  } else if (ns > max_splits) {
    tps = (s.n_tiles + max_splits - 1) / max_splits;
    ns = (s.n_tiles + tps - 1) / tps;
  }
  s.tiles_per_split = tps;
  s.n_splits = ns;
  // merge units (one row x 64 dims), one a merging split
  const int units = R * (L.D / 64);
  s.n_mergers = ns > 1 ? (units < ns ? units : ns) : 0;
  s.grid = ns * L.kv_heads;
  s.xcd_group = 0;
  // sink mode: number the splits in groups of 8 so that the kv heads of a split share an XCD's
  // L2 for the slots' cos/sin rows (per kv head split k keeps a higher index than split j < k, so
  // the mergers are still dispatched after every split they wait on)
  if (L.ring.roll && ns > 1 && L.kv_heads > 1) {
    const long padded = (long)((ns + 7) / 8) * 8 * L.kv_heads;
    if (padded <= resident) {
      s.xcd_group = 8;
      s.grid = (int)padded;
    }
  }
  *out = s;
  return true;
}

static std::mutex g_decode_fn_mu;

// dynamic LDS past 64 KB must be allowed per kernel before a launch (and before an occupancy
// query counts it); the allowance only ever grows. Caller holds g_decode_fn_mu.
static hipError_t allow_lds_locked(const void* fn, size_t smem) {
  static std::map<const void*, size_t> allowed;
  if (smem <= 64 * 1024) return hipSuccess;
  size_t& a = allowed[fn];
  if (smem <= a) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e == hipSuccess) a = smem;
  return e;
}

// workgroups of one decode instantiation that fit a CU at once with `smem` bytes of dynamic
// LDS (cached per kernel and size)
static int resident_blocks(const void* fn, int threads, size_t smem) {
  static std::map<std::pair<const void*, size_t>, int> memo;
  std::lock_guard<std::mutex> lock(g_decode_fn_mu);
  auto it = memo.find({fn, smem});
  if (it != memo.end()) return it->second;
  int nb = 0;
  if (allow_lds_locked(fn, smem) != hipSuccess) (void)hipGetLastError();
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, threads, smem) != hipSuccess || nb < 1) {
    (void)hipGetLastError();
    nb = 1;
  }
  memo[{fn, smem}] = nb;
  return nb;
}

uint32_t decode_workspace_empty() { return kPartialEmpty; }

__global__ void xcd_probe_kernel(int* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

hipError_t probe_xcd_round_robin(int* n_xcd) {
  *n_xcd = 0;
  constexpr int kProbe = 4096;
  int* d = nullptr;
  hipError_t e = hipMalloc((void**)&d, kProbe * sizeof(int));
  if (e != hipSuccess) return e;
  std::vector<int> h(kProbe, -1);
  hipLaunchKernelGGL(xcd_probe_kernel, dim3(kProbe), dim3(64), 0, 0, d);
  e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpy(h.data(), d, kProbe * sizeof(int), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return e;
  // round robin from a starting XCD r (the same for every workgroup of the grid): workgroup b on
  // XCD (b + r) mod nx, so workgroups with equal b mod nx share an XCD
  int nx = 0;
  for (int x : h) nx = std::max(nx, x + 1);
  bool rr = nx >= 2 && h[0] >= 0;
  for (int b = 0; b < kProbe && rr; b++) rr = h[b] == (b + h[0]) % nx;
  *n_xcd = rr ? nx : 0;
  return hipSuccess;
}

size_t decode_partial_floats(const LayerView& L, int S, int H, int n_splits) {
  const int R = (H / L.kv_heads) * S;
  return (size_t)L.kv_heads * R * (L.D / 64) * n_splits * kUnitF4 * 4;
}

size_t decode_workspace_floats(const LayerView& L, int S, int H, int num_cus, size_t* counters) {
  // upper bound over every pos_base: tiles_per_split >= 4 waves, so at most cap/32/4 splits
  // (and kMaxSplits); one 17-float4 slot per (kv head, unit, split). The caller fills it with
  // kPartialEmpty once (decode_workspace_fill) and every launch leaves it that way.
  (void)num_cus;
  const int R = (H / L.kv_heads) * S;
  int ns_max = (L.cap / 32 + 3) / 4;
  ns_max = ns_max < kMaxSplits ? ns_max : kMaxSplits;
  *counters = (size_t)L.kv_heads * kCounterStride;
  return (size_t)L.kv_heads * R * (L.D / 64) * ns_max * kUnitF4 * 4;
}

template <int D, int DT, bool ROLL, int NSET, int NPT, int NW, int PR, bool ONE = false>
static hipError_t launch_cfg(const LayerView& L, const AttnArgs& a, hipStream_t st) {
  using SM = DecodeSmem<D, DT, ROLL, NSET, NW, PR>;
  const void* fn = (const void*)decode_kernel<D, DT, ROLL, NSET, NW, NPT, PR, ONE>;
  const int R = (a.H / L.kv_heads) * a.S;
  if (rows_per_pass(R) != PR) return hipErrorInvalidValue;
  const int NP = (R + PR - 1) / PR;
  const size_t smem = SM::total(NP, R);
  if (smem != decode_lds_bytes(D, DT, R, NW, PR)) return hipErrorInvalidValue;  // the two plans agree
  if (smem > kDecodeLdsMax) return hipErrorInvalidValue;
  {
    std::lock_guard<std::mutex> lock(g_decode_fn_mu);
    const hipError_t e = allow_lds_locked(fn, smem);
    if (e != hipSuccess) return e;
  }
  DecodePlan sp;
  if (!decode_plan(L, a.S, a.H, a.pos_base, a.num_cus, resident_blocks(fn, 64 * NW, smem), &sp)) return hipErrorInvalidValue;
  if (sp.waves != NW || sp.nset != NSET || (NPT > 0 && sp.passes != NPT)) return hipErrorInvalidValue;
  if (ONE && sp.n_splits > 1 && sp.tiles_per_split > NW) return hipErrorInvalidValue;  // a wave with two tiles
  if (ONE && sp.n_splits == 1 && sp.n_tiles > NW) return hipErrorInvalidValue;
  DecodeParams p;
  p.L = L;
  p.q = a.q;
  p.S = a.S;
  p.H = a.H;
  p.G = a.H / L.kv_heads;
  p.R = R;
  p.pos_base = a.pos_base;
  p.qscale = a.scale * kLog2e * (SM::QUARTER ? (1.0f / 127.0f) : 1.0f);
  p.gate = a.gate;
  p.gate_stride = a.gate_stride;
  p.out = a.out;
  p.n_scan = sp.n_scan;
  p.phys_limit = sp.phys_limit;
  p.n_tiles = sp.n_tiles;
  p.skip_t0 = sp.skip_t0;
  p.skip_n = sp.skip_n;
  p.tiles_per_split = sp.tiles_per_split;
  p.n_splits = sp.n_splits;
  const int units = R * (D / 64);
  const size_t need = (size_t)L.kv_heads * units * sp.n_splits * kUnitF4 * 4;
  if (sp.n_splits > 1 && (a.ws_o == nullptr || a.err == nullptr || need > a.ws_floats || sp.n_splits > kMaxSplits))
    return hipErrorInvalidValue;
  p.ws = (float4*)a.ws_o;
  p.n_mergers = sp.n_mergers;
  p.err = a.err;
  p.spin_limit = a.spin_limit > 0 ? a.spin_limit : (1 << 20);
  p.withhold_split = a.withhold_split;
  p.xcd_group = sp.xcd_group;
  // L2 exchange: every split of a kv head shares blockIdx mod n_xcd when the kv heads are a
  // multiple of the XCD count and the plain numbering is used
  p.xcd_local = (a.n_xcd > 0 && sp.n_splits > 1 && sp.xcd_group == 0 && L.kv_heads % a.n_xcd == 0) ? a.n_xcd : 0;
  hipLaunchKernelGGL((decode_kernel<D, DT, ROLL, NSET, NW, NPT, PR, ONE>), dim3(sp.grid), dim3(64 * NW), smem, st, p);
  return hipGetLastError();
}

template <int D, int DT, bool ROLL>
static hipError_t launch_nset(const LayerView& L, const AttnArgs& a, int nset, hipStream_t st) {
  DecodePlan pl;
  if (!decode_plan(L, a.S, a.H, a.pos_base, a.num_cus, 1, &pl)) return hipErrorInvalidValue;
  const int np = pl.passes;
  const int R = (a.H / L.kv_heads) * a.S;
  switch (nset) {
    case 1: {
      // straight-line passes: one pass of 4 rows (G = 4 decode), one of 8 (5-8 rows: G = 6
      // decode, short verifies), two of 8 (9-16 rows)
      if constexpr (D == 128) {
        if (pl.waves == 8) {
          if (R <= 4) return launch_cfg<D, DT, ROLL, 1, 1, 8, 4>(L, a, st);
          if (np == 1) return launch_cfg<D, DT, ROLL, 1, 1, 8, 8>(L, a, st);
          return launch_cfg<D, DT, ROLL, 1, 2, 8, 8>(L, a, st);
        }
      }
      // q8 and sink mode: one tile a wave when the plan for the one-tile kernel's residency gives
      // it (the two-tile kernel's prefetch would re-read the wave's only tile)
      if constexpr (DT == KV_Q8 || ROLL) {
        auto one_tile = [&](const void* fn, int pr) {
          const size_t smem = decode_lds_bytes(D, DT, R, 4, pr);
          DecodePlan p1;
          return decode_plan(L, a.S, a.H, a.pos_base, a.num_cus, resident_blocks(fn, 256, smem), &p1) &&
                 p1.waves == 4 && (p1.n_splits > 1 ? p1.tiles_per_split == 4 : p1.n_tiles <= 4);
        };
        if (R <= 4 && one_tile((const void*)decode_kernel<D, DT, ROLL, 1, 4, 1, 4, true>, 4))
          return launch_cfg<D, DT, ROLL, 1, 1, 4, 4, true>(L, a, st);
        if (R > 4 && np == 1 && one_tile((const void*)decode_kernel<D, DT, ROLL, 1, 4, 1, 8, true>, 8))
          return launch_cfg<D, DT, ROLL, 1, 1, 4, 8, true>(L, a, st);
        if (R > 4 && np == 2 && one_tile((const void*)decode_kernel<D, DT, ROLL, 1, 4, 2, 8, true>, 8))
          return launch_cfg<D, DT, ROLL, 1, 2, 4, 8, true>(L, a, st);
      }
      if (R <= 4) return launch_cfg<D, DT, ROLL, 1, 1, 4, 4>(L, a, st);
      if (np == 1) return launch_cfg<D, DT, ROLL, 1, 1, 4, 8>(L, a, st);
      return launch_cfg<D, DT, ROLL, 1, 2, 4, 8>(L, a, st);
    }
    case 2:
      // 17-24 rows (the 5-row verify of G = 4 heads: 20) take three passes of 8
      if (np == 3) return launch_cfg<D, DT, ROLL, 2, 3, 4, 8>(L, a, st);
      return launch_cfg<D, DT, ROLL, 2, 0, 4, 8>(L, a, st);
    default: return launch_cfg<D, DT, ROLL, 3, 0, 4, 8>(L, a, st);
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
