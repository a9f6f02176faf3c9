// Causal GQA prefill attention over an f16 or q8 KV cache on gfx950 MFMA (f16 in, f32 acc).
//
// Replaces the prefill/verify dispatch of attention_sg_kv16.wgsl / attention_sg_kv8.wgsl and the
// hybrid attention_online_cache_kv8.wgsl (src/engine.ts:1579-1580, 1486-1489), which run one
// subgroup or workgroup per (query, head) with a serial key loop. Here prefill is a dense
// contraction:
//   rows      a row is a (query, head) pair; the G heads of one kv head are packed into the rows
//             so every staged K/V byte serves G heads. A wave owns 32 rows, a workgroup of 4
//             waves one query block of 128 rows, over the block's whole key range.
//   occupancy D=128: 64 KB of LDS and at most 256 registers a wave, so two workgroups share a
//             CU; their waves meet no common barrier, so one's softmax overlaps the other's
//             MFMAs. D=256: one workgroup a CU, each wave with a full SIMD's 512 registers.
//   items     (query block, kv head) pairs, heaviest (latest queries) first. A D=128 grid that
//             fits at once pairs each heavy item with its mirror light item on one CU, so all
//             CUs scan about the same number of keys; other grids are balanced by the
//             dispatcher.
//   staging   per step a workgroup stages KT keys (64 for D=128, 32 for D=256) of K (row-major, 16-byte
//             chunks XOR-swizzled by row so the MFMA operand reads hit distinct banks) and V^T
//             (the cache's transposed 32-slot tiles, copied as they are) into LDS as f16,
//             double-buffered with one barrier per step. An f16 cache is copied by the gfx950
//             direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds: no registers, no VALU); q8
//             codes are dequantized (code * block scale / 127) and sink-mode keys rotated at
//             their slot position through registers, once per workgroup. Either way the next
//             step's loads are in flight while this step computes.
//   pipeline  D=256 with f16 tiles (one wave per SIMD): K is staged one step ahead of V and
//             iteration s runs the QK MFMAs of step s+1 with the exp2 / f16 / row-sum work of step
//             s between them, then the PV MFMAs of step s -- the VALU work hides under MFMAs
//             instead of sitting between them.
//   S^T = K Q^T  v_mfma_f32_32x32x16_f16, A = K from LDS, B = Q^T held in registers: a lane
//             holds 16 keys of ONE row, so the softmax is lane-local plus one cross-half shuffle.
//   softmax   base 2 with the hardware exp2 (results below 2^-126 flush to 0, as the f16 P
//             operand would); masks only on steps that reach past the block's first query (causal
//             diagonal) or the scanned range; the running max is raised only when a step's max
//             exceeds it by more than 8 (so P <= 2^8, exact-range f16) -- most steps skip the
//             O rescale. The row sum accumulates the f16 P the PV product uses (v_dot2).
//   O^T += V^T P^T  v_mfma_f32_32x32x16_f16: the S^T accumulator registers are already in the
//             B-operand layout of P^T for the V tile's panel order, no transpose.
// The output gate (gate_sigmoid.wgsl:13) is applied at the store.
#include <algorithm>
#include <type_traits>

#include "bg_kernels.h"

namespace bg {

typedef _Float16 half8p __attribute__((ext_vector_type(8)));
typedef _Float16 half2p __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
// native 16-byte vector (HIP's uint4 is a struct whose copies become memcpys the optimizer
// cannot always keep in registers)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ inline u32x4 ldv(const void* p) { return *(const u32x4*)p; }
__device__ inline void stv(void* p, u32x4 v) { *(u32x4*)p = v; }

typedef __attribute__((address_space(3))) void* lds_vptr;

union PH8 {
  half8p h;
  u32x4 u;
  half2p p[4];
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
  int mirror;        // pair items heavy / light over the one wave of the grid (see the kernel)
  // split-K: n_parts > 1 splits every item's key range into parts of part_steps steps, each
  // scanned by its own workgroup, which leaves its partial in pws for prefill_merge_kernel
  int n_parts, part_steps;
  int split_waves;   // waves whose rows can be valid (fewer when the grid has fewer rows than 128)
  float4* pws;       // [item][part][split_waves][4 * D/32][64] float4: o slots (empty marker between launches)
  float2* pml;       // [item][part][split_waves][64] (m, l) of each lane's row
};

template <int D>
struct PfCfg {
  static constexpr int KT = D == 128 ? 64 : 32;   // keys per step
  static constexpr int NSUB = KT / 32;            // 32-key MFMA sub-tiles per step
  static constexpr int CPR = D / 8;               // 16-byte chunks per K row
  static constexpr int TILE = KT * D;             // f16 values of one staged K (or V) tile
  static constexpr int NC = D / 16;               // QK k-chunks
  static constexpr int ND = D / 32;               // output dim chunks
  static constexpr int NB = D / 32;               // q8 scale blocks per row
};

// staged K: chunk c of row r lives at chunk position r * CPR + (c ^ (r & 15))
template <int D>
__device__ inline int k_chunk_pos(int r, int c) { return r * PfCfg<D>::CPR + (c ^ (r & 15)); }

// One thread's share of a register-staged step (q8 or sink mode): 16 dims of one key in each
// half of the row (the rope partners i and i + D/2 sit in the same thread) and 4 V^T chunks of
// 8 slots (f16: 4 chunks spread over the step; q8: the chunks of 4 neighbouring dims of one
// panel, which share the 8 slot scales of one block).
template <int D, int DT>
struct StageRegs {
  static constexpr bool Q8 = DT == KV_Q8;
  u32x4 k[Q8 ? 2 : 4];        // q8: 16 codes per half; f16: 2 x 8 values per half
  float ksc[Q8 ? 2 : 1];
  u32x4 v[Q8 ? 2 : 4];        // q8: 4 dims x 8 slots of codes; f16: 4 x 8 values
  float vsc[Q8 ? 8 : 1];      // q8: block scale of each of the 8 slots
};

template <int D, int DT, bool ROLL>
struct Stager {
  using C = PfCfg<D>;
  static constexpr int PH = D / 32;   // threads per key (16 dims per half each)
  int tt, wt, lane;
  // K piece of this thread
  int key, cb;
  // q8 V chunk group of this thread: dims 4*vdg .. 4*vdg+3 of panel vpanel of 32-slot tile vu
  int vu, vpanel, vdg;

  __device__ explicit Stager(int t) {
    tt = t;
    wt = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: the copies' LDS bases are scalars
    lane = t & 63;
    key = t / PH;
    cb = 16 * (t % PH);
    vdg = t % (D / 4);
    vpanel = (t / (D / 4)) & 3;
    vu = t / D;
  }

  // f16 cache without rotation: this wave's 4 K and 4 V chunks of 64 lanes copied straight
  // into LDS (the step's tiles are 4 waves x 4 x 64 chunks of 16 bytes each). The copies use the
  // buffer form (a descriptor over the kv head's K or V region, a 32-bit lane offset): the
  // compiler tracks those as vector-memory writes into one LDS array, whereas the global form
  // counts as an access that may touch any LDS, after which every LDS read wait in the step
  // becomes a wait for all outstanding reads.
  __device__ __forceinline__ static __amdgpu_buffer_rsrc_t region(const void* base, int kvh, int cap) {
    constexpr int kRawDwordFormat = 0x00020000;  // descriptor word 3: 32-bit data, raw access
    return __builtin_amdgcn_make_buffer_rsrc((void*)((const char*)base + (size_t)kvh * cap * D * 2), (short)0,
                                             cap * D * 2, kRawDwordFormat);
  }
  __device__ __forceinline__ void dma_k(const PrefillParams& p, int kvh, int j0, _Float16* kdst) const {
    const int cap = p.L.cap;
    const __amdgpu_buffer_rsrc_t rs = region(p.L.k, kvh, cap);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int pb = (4 * i + wt) * 64;   // first chunk position of this wave instruction
      const int P = pb + lane;
      const int r = P / C::CPR;
      const int c = (P % C::CPR) ^ (r & 15);
      const uint32_t off = (uint32_t)min(j0 + r, cap - 1) * (D * 2) + c * 16;  // past the end: masked keys
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_vptr)(kdst + pb * 8), 16, off, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void dma_v(const PrefillParams& p, int kvh, int j0, _Float16* vdst) const {
    const int cap = p.L.cap;
    const __amdgpu_buffer_rsrc_t rs = region(p.L.v, kvh, cap);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int pb = (4 * i + wt) * 64;
      const int P = pb + lane;
      const int u = P / (4 * D);        // 32-slot tile of the chunk (4*D chunks per tile)
      const int tu = min((j0 >> 5) + u, cap / 32 - 1);
      const uint32_t off = (uint32_t)tu * (32 * D * 2) + (uint32_t)(P % (4 * D)) * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_vptr)(vdst + pb * 8), 16, off, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void dma(const PrefillParams& p, int kvh, int j0, _Float16* kdst, _Float16* vdst) const {
    dma_k(p, kvh, j0, kdst);
    dma_v(p, kvh, j0, vdst);
  }

  // register staging: issue the global loads of the step whose first key is slot j0
  __device__ __forceinline__ void load(StageRegs<D, DT>& R, const PrefillParams& p, int kvh, int j0) const {
    const LayerView& L = p.L;
    const int cap = L.cap;
    const int slot = min(j0 + key, cap - 1);  // past the end: a valid row whose keys are masked
    if constexpr (DT == KV_Q8) {
      const int8_t* kr = (const int8_t*)L.k + ((size_t)kvh * cap + slot) * D;
      R.k[0] = ldv(kr + cb);
      R.k[1] = ldv(kr + cb + D / 2);
      const float* ks = L.ks + ((size_t)kvh * cap + slot) * C::NB;
      R.ksc[0] = ks[cb / 32];
      R.ksc[1] = ks[(cb + D / 2) / 32];
      const int t32 = min((j0 >> 5) + vu, cap / 32 - 1);
      const int8_t* vt = (const int8_t*)L.v + ((size_t)kvh * cap + (size_t)t32 * 32) * D +
                         ((size_t)vpanel * D + 4 * vdg) * 8;
      R.v[0] = ldv(vt);
      R.v[1] = ldv(vt + 16);
      const float* vs = L.vs + ((size_t)kvh * cap + (size_t)t32 * 32) * C::NB + (4 * vdg) / 32;
#pragma unroll
      for (int e = 0; e < 8; e++) R.vsc[e] = vs[(size_t)tile_slot(vpanel, e) * C::NB];
    } else {
      const __half* kr = (const __half*)L.k + ((size_t)kvh * cap + slot) * D;
      R.k[0] = ldv(kr + cb);
      R.k[1] = ldv(kr + cb + 8);
      R.k[2] = ldv(kr + cb + D / 2);
      R.k[3] = ldv(kr + cb + D / 2 + 8);
      // V^T: the step's KT slots are KT * D contiguous values; chunk = tt + 256 i
      const int t32 = j0 >> 5;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int c = tt + 256 * i;                 // 16-byte chunk within the step
        const int u = c / (4 * D);                  // 32-slot tile of the chunk
        const int tu = min(t32 + u, cap / 32 - 1);
        const __half* vt = (const __half*)L.v + ((size_t)kvh * cap + (size_t)tu * 32) * D;
        R.v[i] = ldv(vt + (size_t)(c % (4 * D)) * 8);
      }
    }
  }

  // register staging: convert (dequantize / rotate) and write into one buffer; j0 = the staged
  // step's first key
  __device__ __forceinline__ void store(const StageRegs<D, DT>& R, const PrefillParams& p, int j0, _Float16* kb,
                                        _Float16* vb) const {
    float a[16], b[16];  // the two halves of this thread's 16-dim K piece
    if constexpr (DT == KV_Q8) {
      const float sa = R.ksc[0] * (1.0f / 127.0f), sb = R.ksc[1] * (1.0f / 127.0f);
      const uint32_t wa[4] = {R.k[0][0], R.k[0][1], R.k[0][2], R.k[0][3]};
      const uint32_t wb[4] = {R.k[1][0], R.k[1][1], R.k[1][2], R.k[1][3]};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t ua = wa[i] ^ 0x80808080u, ub = wb[i] ^ 0x80808080u;  // biased: u = c + 128
#pragma unroll
        for (int e = 0; e < 4; e++) {
          a[4 * i + e] = q8_stage_f32((ua >> (8 * e)) & 0xffu, sa);  // = c * sa, one f32 rounding
          b[4 * i + e] = q8_stage_f32((ub >> (8 * e)) & 0xffu, sb);
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
          a[4 * i + e] = add_rn(mul_rn(x, c4[e]), mul_rn(-y, s4[e]));
          b[4 * i + e] = add_rn(mul_rn(y, c4[e]), mul_rn(x, s4[e]));
        }
      }
    }
    const int ca = cb / 8, cbb = (cb + D / 2) / 8;  // first chunk of each half
    if constexpr (DT == KV_Q8 || ROLL) {
      PH8 o;
#pragma unroll
      for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int e = 0; e < 8; e++) o.e[e] = (_Float16)a[8 * i + e];
        stv(kb + k_chunk_pos<D>(key, ca + i) * 8, o.u);
#pragma unroll
        for (int e = 0; e < 8; e++) o.e[e] = (_Float16)b[8 * i + e];
        stv(kb + k_chunk_pos<D>(key, cbb + i) * 8, o.u);
      }
    } else {
      stv(kb + k_chunk_pos<D>(key, ca) * 8, R.k[0]);
      stv(kb + k_chunk_pos<D>(key, ca + 1) * 8, R.k[1]);
      stv(kb + k_chunk_pos<D>(key, cbb) * 8, R.k[2]);
      stv(kb + k_chunk_pos<D>(key, cbb + 1) * 8, R.k[3]);
    }
    if constexpr (DT == KV_Q8) {
      const uint32_t w[8] = {R.v[0][0], R.v[0][1], R.v[0][2], R.v[0][3], R.v[1][0], R.v[1][1], R.v[1][2], R.v[1][3]};
      float sv[8];
#pragma unroll
      for (int e = 0; e < 8; e++) sv[e] = R.vsc[e] * (1.0f / 127.0f);
#pragma unroll
      for (int i = 0; i < 4; i++) {  // chunk i: dim 4*vdg + i, 8 slots
        PH8 o;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const uint32_t u = w[2 * i + (e >> 2)] ^ 0x80808080u;
          o.e[e] = q8_stage_f16((u >> (8 * (e & 3))) & 0xffu, sv[e]);
        }
        stv(vb + ((size_t)(vu * 4 + vpanel) * D + 4 * vdg + i) * 8, o.u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) stv(vb + (size_t)(tt + 256 * i) * 8, R.v[i]);
    }
  }
};

template <int D, int DT, bool ROLL>
__global__ __launch_bounds__(256, D == 128 ? 2 : 1) void prefill_kernel(PrefillParams p) {
  using C = PfCfg<D>;
  constexpr int KT = C::KT, NSUB = C::NSUB, NC = C::NC, ND = C::ND, TILE = C::TILE;
  constexpr bool DMA = DT == KV_F16 && !ROLL;
  // software-pipelined steps where a wave has its SIMD to itself (D=256: 512 registers a wave);
  // D=128 runs two workgroups per CU, whose waves overlap one's softmax with the other's MFMAs
  constexpr bool PIPE = DMA && D == 256;
  // Double buffers as four distinct arrays: the compiler then knows a copy into one buffer cannot
  // alias the reads of the other, and adds no waits between them. 64 KB: two workgroups a CU.
  __shared__ __align__(16) _Float16 lk0[TILE];
  __shared__ __align__(16) _Float16 lk1[TILE];
  __shared__ __align__(16) _Float16 lv0[TILE];
  __shared__ __align__(16) _Float16 lv1[TILE];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int g2 = lane >> 5, n = lane & 31;
  const int KV = p.L.kv_heads;
  const Ring ring = p.L.ring;
  _Float16* const k0 = lk0;
  _Float16* const k1 = lk1;
  _Float16* const v0 = lv0;
  _Float16* const v1 = lv1;
  const Stager<D, DT, ROLL> stg(tid);
  const int r = wave * 32 + n;  // this lane's row within the block

  // Work items are (query block, kv head) pairs ordered heaviest (latest queries) first. A grid
  // the CUs hold at once (mirror) pairs them: workgroup b < n/2 takes item b, the rest the mirrors
  // n-1-(b-n/2), so that each CU holds one heavy and one light item and every CU scans about the
  // same number of keys. A larger grid runs heaviest first, balanced by the dispatcher.
  // Split-K (a grid far smaller than the GPU): workgroup b scans part b % n_parts of item
  // b / n_parts.
  const int bid = blockIdx.x;
  const int n_items = p.n_qblocks * KV;
  const int half = (n_items + 1) / 2;
  const bool split = p.n_parts > 1;
  const int part = split ? bid % p.n_parts : 0;
  const int item = split ? bid / p.n_parts : !p.mirror || bid < half ? bid : n_items - 1 - (bid - half);
  const int kvh = item % KV;
  const int qb = p.n_qblocks - 1 - item / KV;
  const int s0 = qb * p.QB;
  const int G = p.G;

  const int qi = s0 + r / G;
  const int h = kvh * G + r % G;
  const bool row_ok = r < p.QB * p.G && qi < p.S;
  const int limit = p.pos_base + qi;

  // key range of the block in KT-key steps
  const int last_q = min(s0 + p.QB, p.S) - 1;
  const int n_scan = p.n_scan_fixed > 0 ? p.n_scan_fixed : p.pos_base + last_q + 1;
  const int steps_item = (n_scan + KT - 1) / KT;
  // this workgroup's steps [t0, steps) of the block's key range
  const int t0 = part * p.part_steps;
  const int steps = split ? min(t0 + p.part_steps, steps_item) : steps_item;
  if (t0 >= steps) return;  // a part past the block's range (the whole workgroup)
  const int t_last = steps - 1;
  // the earliest key index any row of the block masks (causal diagonal or scan end)
  const int mask_from = min(min(p.pos_base + s0 + 1, n_scan), p.phys_limit);

  // ---------------- prologue: Q and the first tile, loads issued together ----------------
  // each lane gathers its own Q^T operand (16 dims of one row per dim chunk)
  float4 qraw[2 * NC];
  {
    const float* qr = p.q + ((size_t)(row_ok ? qi : 0) * p.H + (row_ok ? h : 0)) * D;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      qraw[2 * c] = *(const float4*)(qr + 16 * c + 8 * g2);
      qraw[2 * c + 1] = *(const float4*)(qr + 16 * c + 8 * g2 + 4);
    }
  }
  const int j00 = t0 * KT;
  StageRegs<D, DT> R0;
  if constexpr (PIPE) {
    // K and V of the first step and K of the second (K is staged one step ahead of V)
    stg.dma(p, kvh, j00, k0, v0);
    stg.dma_k(p, kvh, min(t0 + 1, t_last) * KT, k1);
  } else if constexpr (DMA) {
    stg.dma(p, kvh, j00, k0, v0);
  } else {
    stg.load(R0, p, kvh, j00);
  }
  // Q^T operand: dims 16c + 8*g2 + [0..8), pre-scaled by scale*log2(e)
  half8p qf[NC];
  auto to_h8 = [](const float4& a, const float4& b, float sc) {
    return half8p{(_Float16)(a.x * sc), (_Float16)(a.y * sc), (_Float16)(a.z * sc), (_Float16)(a.w * sc),
                  (_Float16)(b.x * sc), (_Float16)(b.y * sc), (_Float16)(b.z * sc), (_Float16)(b.w * sc)};
  };
  {
    const float sc = row_ok ? p.qscale : 0.0f;
#pragma unroll
    for (int c = 0; c < NC; c++) qf[c] = to_h8(qraw[2 * c], qraw[2 * c + 1], sc);
  }
  if constexpr (!DMA) stg.store(R0, p, j00, k0, v0);

  floatx16 o[ND];
#pragma unroll
  for (int i = 0; i < ND; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[i][e] = 0.0f;
  float m = -1e30f, lsum = 0.0f;
  if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0xf70);  // vmcnt(0): this wave's copies landed
  __syncthreads();

  if constexpr (PIPE) {
    // ---------------- software-pipelined steps (f16 tiles copied straight into LDS) ----------------
    // Iteration s: copy K of step s+2 and V of step s+1; S of step s+1 = K Q^T on the MFMAs while
    // the VALU turns S of step s into P (exp2, f16, row sum); O += V P of step s; mask and max of
    // S of step s+1. The MFMA pipe runs QK and PV back to back and the softmax VALU work runs
    // under the QK MFMAs instead of between them. K buffers alternate s+1 (read) / s+2 (filled),
    // V buffers s (read) / s+1 (filled).
    constexpr int NA = NSUB == 1 ? 2 : NSUB;
    float x[NSUB][16];  // S of the step whose P is computed next (masked, log2 units)
    // S^T = K Q^T into sacc from the K tile at kc; with WITH_P, P of x is computed under it
    auto qk = [&](auto with_p, const _Float16* kc, floatx16 (&sacc)[NA], PH8 (&pb)[NSUB][2]) {
      constexpr bool WP = decltype(with_p)::value;
#pragma unroll
      for (int u = 0; u < NA; u++)
#pragma unroll
        for (int e = 0; e < 16; e++) sacc[u][e] = 0.0f;
      PH8 ka[NC][NSUB];
      auto rd = [&](int c) {
#pragma unroll
        for (int u = 0; u < NSUB; u++) ka[c][u].u = ldv(kc + k_chunk_pos<D>(u * 32 + n, 2 * c + g2) * 8);
      };
      const half2p ones = {(_Float16)1.0f, (_Float16)1.0f};
      // in program order, each piece fenced: the reads of chunk c+2 ahead of chunk c's MFMAs,
      // then a share of the P work (the scheduler left alone runs one accumulator chain first
      // and waits for every read)
      rd(0);
      if (NC > 1) rd(1);
#pragma unroll
      for (int c = 0; c < NC; c++) {
        if (c + 2 < NC) rd(c + 2);
#pragma unroll
        for (int u = 0; u < NSUB; u++) {
          const int acc = NSUB == 1 ? (c & 1) : u;
          sacc[acc] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[c][u].h, qf[c], sacc[acc], 0, 0, 0);
        }
        if constexpr (WP) {
          // the 16*NSUB values of P spread evenly over the NC chunks, in order (so the row sum
          // adds the same pairs in the same order as a whole group at a time would)
          constexpr int NPI = 16 * NSUB, PER = (NPI + NC - 1) / NC;
#pragma unroll
          for (int k = 0; k < PER; k++) {
            const int i = c * PER + k;
            if (i < NPI) {
              const int u = i >> 4, e = i & 15;
              pb[u][e >> 3].e[e & 7] = (_Float16)__builtin_amdgcn_exp2f(x[u][e] - m);
              if (e & 1) lsum = __builtin_amdgcn_fdot2(pb[u][e >> 3].p[(e & 7) >> 1], ones, lsum, false);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // the accumulators are taken here, so no QK MFMA is sunk past this phase to its use
#pragma unroll
      for (int u = 0; u < NA; u++) asm volatile("" : "+v"(sacc[u]));
      if constexpr (NSUB == 1) sacc[0] += sacc[1];
    };
    // mask S of step s1 into x and return its row max
    auto mask_max = [&](int s1, const floatx16 (&sacc)[NA]) {
      const bool live = s1 < steps;  // the look-ahead past the last step is all masked
      const int j0 = (live ? s1 : 0) * KT;
      float mt = -INFINITY;
      if (!live || j0 + KT > mask_from) {
#pragma unroll
        for (int u = 0; u < NSUB; u++)
#pragma unroll
          for (int k = 0; k < 4; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const int P = j0 + 32 * u + 8 * k + 4 * g2 + e;
              const bool ok = live && P < n_scan && P < p.phys_limit && P <= limit;
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
      const float2 r = pair32(mt);
      return fmaxf(r.x, r.y);
    };
    // raise the reference max only when a step's max exceeds it by more than 2^8
    auto raise = [&](float mt) {
      const bool grow = mt > m + 8.0f;
      if (__any(grow)) {
        const float mn = grow ? mt : m;
        const float corr = __builtin_amdgcn_exp2f(m - mn);
        m = mn;
        lsum *= corr;
#pragma unroll
        for (int i = 0; i < ND; i++) o[i] *= corr;
      }
    };
    {
      floatx16 sacc[NA];
      PH8 pb[NSUB][2];
      qk(std::false_type{}, k0, sacc, pb);
      raise(mask_max(t0, sacc));
    }
    __syncthreads();  // the first K buffer and the Q operand area are free

    auto pstep = [&](int s, const _Float16* kn, const _Float16* vc, _Float16* kd, _Float16* vd) {
      stg.dma_k(p, kvh, min(s + 2, t_last) * KT, kd);
      stg.dma_v(p, kvh, min(s + 1, t_last) * KT, vd);
      floatx16 sacc[NA];
      PH8 pb[NSUB][2];
      qk(std::true_type{}, kn, sacc, pb);
      // (each phase's MFMAs stay in their phase: the schedule groups below would otherwise take
      // the QK MFMAs of one 32-key half, and the reads feeding them, out of order)
      __builtin_amdgcn_sched_barrier(0);
      // O^T += V^T P^T of step s
      PH8 va[2 * NSUB][ND];
#pragma unroll
      for (int ut = 0; ut < 2 * NSUB; ut++)
#pragma unroll
        for (int dc = 0; dc < ND; dc++)
          va[ut][dc].u = ldv(vc + ((size_t)((ut >> 1) * 4 + 2 * (ut & 1) + g2) * D + 32 * dc + n) * 8);
#pragma unroll
      for (int u = 0; u < NSUB; u++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int dc = 0; dc < ND; dc++)
            o[dc] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[2 * u + t][dc].h, pb[u][t].h, o[dc], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, ND, 0);
#pragma unroll
      for (int ut = 0; ut < 2 * NSUB - 1; ut++) {
        __builtin_amdgcn_sched_group_barrier(0x100, ND, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, ND, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, ND, 0);
      raise(mask_max(s + 1, sacc));
      __builtin_amdgcn_s_waitcnt(0xf70);  // vmcnt(0): this wave's copies landed
      __syncthreads();
    };
    for (int s = t0; s < steps; s += 2) {
      pstep(s, k1, v0, k0, v1);
      if (s + 1 < steps) pstep(s + 1, k0, v1, k1, v0);
    }
  } else {
    // ---------------- one step: stage step s+1 into (kn, vn), compute step s from (kc, vc) ----------------
    auto step = [&](int s, const _Float16* kc, const _Float16* vc, _Float16* kn, _Float16* vn) {
      const int jn = min(s + 1, t_last) * KT;
      StageRegs<D, DT> R;
      if constexpr (DMA) {
        stg.dma(p, kvh, jn, kn, vn);
      } else {
        stg.load(R, p, kvh, jn);
        // the loads above stay ahead of the compute (left alone, the compiler sinks them to
        // their use after it and every step waits for global memory)
        __builtin_amdgcn_sched_barrier(0);
      }

      const int j0 = s * KT;
      // S^T = K Q^T
      // one 32-key sub-tile (D=256): two accumulators over even / odd dim chunks, so the QK
      // MFMAs form two independent chains
      constexpr int NA = NSUB == 1 ? 2 : NSUB;
      floatx16 sacc[NA];
#pragma unroll
      for (int u = 0; u < NA; u++)
#pragma unroll
        for (int e = 0; e < 16; e++) sacc[u][e] = 0.0f;
      // K operands read two dim chunks ahead of the MFMAs that use them, so each chunk's MFMAs
      // cover later chunks' LDS latency
      {
        PH8 ka[NC][NSUB];
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
          for (int u = 0; u < NSUB; u++) ka[c][u].u = ldv(kc + k_chunk_pos<D>(u * 32 + n, 2 * c + g2) * 8);
#pragma unroll
        for (int c = 0; c < NC; c++) {
#pragma unroll
          for (int u = 0; u < NSUB; u++) {
            const int acc = NSUB == 1 ? (c & 1) : u;
            sacc[acc] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[c][u].h, qf[c], sacc[acc], 0, 0, 0);
          }
        }
        // schedule: the reads of two dim chunks first, then each chunk's MFMAs followed by the
        // reads two chunks ahead (left alone, the scheduler waits for every read pair in turn)
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * NSUB, 0);
#pragma unroll
        for (int c = 0; c < NC - 1; c++) {
          __builtin_amdgcn_sched_group_barrier(0x008, NSUB, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, NSUB, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NSUB, 0);
      }
      if constexpr (NSUB == 1) sacc[0] += sacc[1];
      // mask + online softmax (row = this lane's n)
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
              const int Lg = ROLL ? ring.logical(P) : P;
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
      { const float2 r = pair32(mt); mt = fmaxf(r.x, r.y); }
      // raise the reference max only when this step's max exceeds it by more than 2^8
      const bool grow = mt > m + 8.0f;
      if (__any(grow)) {
        const float mn = grow ? mt : m;
        const float corr = __builtin_amdgcn_exp2f(m - mn);
        m = mn;
        lsum *= corr;
#pragma unroll
        for (int i = 0; i < ND; i++) o[i] *= corr;
      }
      // P = exp2(S - m) as the f16 B operand of P^T; O^T += V^T P^T
      const half2p ones = {(_Float16)1.0f, (_Float16)1.0f};
      // V^T operands of 32-key group (u, t) for every output dim chunk; read ahead of the MFMAs
      // that use them (see the schedule below)
      PH8 va[2 * NSUB][ND];
#pragma unroll
      for (int ut = 0; ut < 2 * NSUB; ut++)
#pragma unroll
        for (int dc = 0; dc < ND; dc++)
          va[ut][dc].u = ldv(vc + ((size_t)((ut >> 1) * 4 + 2 * (ut & 1) + g2) * D + 32 * dc + n) * 8);
#pragma unroll
      for (int u = 0; u < NSUB; u++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
          PH8 pb;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            pb.e[e] = (_Float16)__builtin_amdgcn_exp2f(x[u][8 * t + e] - m);
            pb.e[4 + e] = (_Float16)__builtin_amdgcn_exp2f(x[u][8 * t + 4 + e] - m);
          }
#pragma unroll
          for (int i = 0; i < 4; i++) lsum = __builtin_amdgcn_fdot2(pb.p[i], ones, lsum, false);
#pragma unroll
          for (int dc = 0; dc < ND; dc++)
            o[dc] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[2 * u + t][dc].h, pb.h, o[dc], 0, 0, 0);
        }
      // schedule: the V^T reads of the first key group, then each group's MFMAs followed by the
      // next group's reads
      __builtin_amdgcn_sched_group_barrier(0x100, ND, 1);
#pragma unroll
      for (int ut = 0; ut < 2 * NSUB - 1; ut++) {
        __builtin_amdgcn_sched_group_barrier(0x100, ND, 1);
        __builtin_amdgcn_sched_group_barrier(0x008, ND, 1);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, ND, 1);

      if constexpr (DMA) {
        __builtin_amdgcn_s_waitcnt(0xf70);  // vmcnt(0): this wave's copies of step s+1 landed
      } else {
        stg.store(R, p, jn, kn, vn);
      }
      __syncthreads();
    };

    // ---------------- main loop, two steps per turn so the buffers are fixed arrays ----------------
    for (int s = t0; s < steps; s += 2) {
      step(s, k0, v0, k1, v1);
      if (s + 1 < steps) step(s + 1, k1, v1, k0, v0);
    }
  }

  // ---------------- store ----------------
  {
    { const float2 r = pair32(lsum); lsum = r.x + r.y; }
    if (split) {
      // the part's partial: lane l of wave w keeps its own layout (rows and dims as in o), so
      // each slot is one contiguous 1 KB store; the merge runs as the next kernel on the stream
      if (wave >= p.split_waves) return;  // no valid rows (and no barrier follows)
      const size_t pi = ((size_t)item * p.n_parts + part) * p.split_waves + wave;
      float4* pw = p.pws + pi * 4 * ND * 64 + lane;
#pragma unroll
      for (int dc = 0; dc < ND; dc++)
#pragma unroll
        for (int k = 0; k < 4; k++)
          pw[(4 * dc + k) * 64] = make_float4(o[dc][4 * k], o[dc][4 * k + 1], o[dc][4 * k + 2], o[dc][4 * k + 3]);
      p.pml[pi * 64 + lane] = make_float2(m, lsum);
      return;
    }
    if constexpr (D == 128) {
      // through one LDS array per wave (16 KB, the tiles are no longer read): rows written
      // swizzled, read back and stored as contiguous 512-byte rows (the register layout
      // scatters 16 bytes per row)
      float4* rows = (float4*)(wave == 0 ? lk0 : wave == 1 ? lk1 : wave == 2 ? lv0 : lv1);
      // lane and G laundered: the swizzled addresses below are computed here, not at the
      // kernel start (where they would be held, or spilled, through the step loop)
      int ln = lane, Ge = G;
      asm volatile("" : "+v"(ln), "+s"(Ge));
      const int en = ln & 31, eg = ln >> 5;
      const float inv = 1.0f / lsum;
      if (p.gate) {  // the gate divides o / l first (gate_sigmoid.wgsl:13 on the normalized row)
#pragma unroll
        for (int dc = 0; dc < ND; dc++)
#pragma unroll
          for (int k = 0; k < 4; k++)
            rows[en * 32 + ((8 * dc + 2 * k + eg) ^ en)] =
                make_float4(o[dc][4 * k] / lsum, o[dc][4 * k + 1] / lsum, o[dc][4 * k + 2] / lsum, o[dc][4 * k + 3] / lsum);
      } else {
#pragma unroll
        for (int dc = 0; dc < ND; dc++)
#pragma unroll
          for (int k = 0; k < 4; k++)
            rows[en * 32 + ((8 * dc + 2 * k + eg) ^ en)] =
                make_float4(o[dc][4 * k] * inv, o[dc][4 * k + 1] * inv, o[dc][4 * k + 2] * inv, o[dc][4 * k + 3] * inv);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int cl = en;
      auto emit = [&](auto gated) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const int rl = 2 * i + eg;                 // row within the wave
          const int rb = wave * 32 + rl;               // row within the block
          const int qq = s0 + rb / Ge, hh = kvh * Ge + rb % Ge;
          float4 v = rows[rl * 32 + (cl ^ (rl & 31))];
          if (rb < p.QB * Ge && qq < p.S) {
            if constexpr (decltype(gated)::value) {
              // gate_sigmoid.wgsl:13 form: x / (1 + exp(-g))
              const float4 gv = *(const float4*)(p.gate + ((size_t)qq * p.H + hh) * p.gate_stride + 4 * cl);
              v.x = v.x / (1.0f + expf(-gv.x));
              v.y = v.y / (1.0f + expf(-gv.y));
              v.z = v.z / (1.0f + expf(-gv.z));
              v.w = v.w / (1.0f + expf(-gv.w));
            }
            *(float4*)(p.out + ((size_t)qq * p.H + hh) * D + 4 * cl) = v;
          }
        }
      };
      if (p.gate) emit(std::true_type{});
      else emit(std::false_type{});
    } else if (row_ok) {
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
  }
}

// Split-K merge: workgroup (item, wave, o slot) combines that slot of the wave's 32 rows over the
// parts by log-sum-exp, applies the gate (gate_sigmoid.wgsl:13 form) and stores the output
// float4s; the four 64-lane groups take every fourth part and meet through LDS. Every o slot it
// read gets the empty marker back, so the workspace the decode kernel shares keeps its invariant
// (the (m, l) values live outside that workspace and are only read).
template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams p) {
  constexpr int KT = PfCfg<D>::KT, ND = D / 32, NSL = 4 * ND;
  const int KV = p.L.kv_heads;
  const int sl = blockIdx.x % NSL;
  const int iw = blockIdx.x / NSL;
  const int item = iw / p.split_waves, wave = iw % p.split_waves;
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int kvh = item % KV;
  const int qb = p.n_qblocks - 1 - item / KV;
  const int s0 = qb * p.QB;
  const int n = lane & 31, g2 = lane >> 5, r = wave * 32 + n;
  const int qi = s0 + r / p.G, h = kvh * p.G + r % p.G;
  const bool row_ok = r < p.QB * p.G && qi < p.S;
  const int last_q = min(s0 + p.QB, p.S) - 1;
  const int n_scan = p.n_scan_fixed > 0 ? p.n_scan_fixed : p.pos_base + last_q + 1;
  const int steps_item = (n_scan + KT - 1) / KT;
  const int np = (steps_item + p.part_steps - 1) / p.part_steps;  // parts that scanned keys
  const size_t pstride = (size_t)p.split_waves;                   // per part, in (wave) units
  const size_t pi0 = (size_t)item * p.n_parts * p.split_waves + wave;
  __shared__ float red_m[4][64];
  __shared__ float4 red_o[4][64];
  __shared__ float red_l[4][64];
  // up to 4 * PB parts: every part's (m, l) and partial column loaded before any is used (one
  // memory round trip instead of one per part and group; D=128 f16 verify S=5-12 12.6-13.9 ->
  // 11.6-13.0 us); same order and arithmetic as the loops past it
  constexpr int PB = 8;
  float mx = -INFINITY;
  float2 mlb[PB];
  float4 vb[PB];
  const bool batch = np <= 4 * PB;
  if (batch) {
#pragma unroll
    for (int j = 0; j < PB; j++) {
      const int q = grp + 4 * j, qc = q < np ? q : np - 1;
      const size_t pi = pi0 + qc * pstride;
      mlb[j] = p.pml[pi * 64 + lane];
      vb[j] = p.pws[(pi * NSL + sl) * 64 + lane];
    }
#pragma unroll
    for (int j = 0; j < PB; j++) mx = grp + 4 * j < np ? fmaxf(mx, mlb[j].x) : mx;
  } else {
    for (int q = grp; q < np; q += 4) mx = fmaxf(mx, p.pml[(pi0 + q * pstride) * 64 + lane].x);
  }
  red_m[grp][lane] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red_m[0][lane], red_m[1][lane]), fmaxf(red_m[2][lane], red_m[3][lane]));
  const float em = __uint_as_float(kWorkspaceEmpty);
  const float4 empty = make_float4(em, em, em, em);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float lt = 0.0f;
  if (batch) {
#pragma unroll
    for (int j = 0; j < PB; j++) {
      const int q = grp + 4 * j;
      if (q < np) {
        const size_t pi = pi0 + q * pstride;
        const float w = __builtin_amdgcn_exp2f(mlb[j].x - M);
        acc.x += vb[j].x * w;
        acc.y += vb[j].y * w;
        acc.z += vb[j].z * w;
        acc.w += vb[j].w * w;
        lt += mlb[j].y * w;
        p.pws[(pi * NSL + sl) * 64 + lane] = empty;
      }
    }
  }
  for (int q = batch ? np : grp; q < np; q += 4) {
    const size_t pi = pi0 + q * pstride;
    const float2 ml = p.pml[pi * 64 + lane];
    const float w = __builtin_amdgcn_exp2f(ml.x - M);
    float4* slot = p.pws + (pi * NSL + sl) * 64 + lane;
    const float4 v = *slot;
    acc.x += v.x * w;
    acc.y += v.y * w;
    acc.z += v.z * w;
    acc.w += v.w * w;
    lt += ml.y * w;
    *slot = empty;
  }
  red_o[grp][lane] = acc;
  red_l[grp][lane] = lt;
  __syncthreads();
  if (grp == 0 && row_ok) {
    float4 o = red_o[0][lane];
    float L = red_l[0][lane];
#pragma unroll
    for (int g = 1; g < 4; g++) {
      const float4 b = red_o[g][lane];
      o.x += b.x;
      o.y += b.y;
      o.z += b.z;
      o.w += b.w;
      L += red_l[g][lane];
    }
    const int d = 32 * (sl >> 2) + 8 * (sl & 3) + 4 * g2;
    float rr[4] = {o.x / L, o.y / L, o.z / L, o.w / L};
    if (p.gate) {
      const float* gr = p.gate + ((size_t)qi * p.H + h) * p.gate_stride + d;
#pragma unroll
      for (int e = 0; e < 4; e++) rr[e] = rr[e] / (1.0f + expf(-gr[e]));
    }
    *(float4*)(p.out + ((size_t)qi * p.H + h) * D + d) = make_float4(rr[0], rr[1], rr[2], rr[3]);
  }
}

bool prefill_supported(const LayerView& L, int S, int H) {
  if (L.dtype == KV_F32) return false;
  if (L.D != 128 && L.D != 256) return false;
  const int G = H / L.kv_heads;
  return G >= 1 && G <= 128 && S >= 1;
}

bool prefill_wants_f16_copy(const LayerView& L, int S, int H) {
  // each K/V tile is staged once per query block (128 rows of (query, head) pairs); from four
  // blocks on, one dequantizing pass plus the f16 direct-to-LDS staging costs less
  if (L.dtype != KV_Q8 || L.ring.roll) return false;
  const int G = H / L.kv_heads;
  const int QB = 128 / G;
  return (S + QB - 1) / QB >= 4;
}

// D=128 runs two workgroups a CU (64 KB of LDS and 256 registers a wave each). A D=128 grid that
// fits at once is dispatched as one wave, the first half of the workgroups one a CU and the second
// half beside them, so pairing item b with its mirror (see the kernel) pairs heavy and light items
// on each CU. Other grids (D=256: one workgroup a CU) run heaviest first, balanced by the
// dispatcher.
static bool pf_mirror(const LayerView& L, int n_items, int num_cus) { return L.D == 128 && n_items <= 2 * num_cus; }

// Split-K plan of a prefill launch. A grid of (query block, kv head) items far smaller than the
// GPU (short prompts after a long context, speculative verify with many heads per kv head) leaves
// most CUs idle while each workgroup scans the whole key range; such a grid is split into parts
// of at least kPfMinPartSteps steps, up to a full GPU's worth of workgroups, with all partials
// within kPfSplitMaxBytes (the allocation-free entry point's scratch holds them too, so both
// entry points make the same split and return the same results).
constexpr size_t kPfSplitMaxBytes = (size_t)8 << 20;
constexpr int kPfMinPartSteps = 4;
constexpr size_t kPfSplitMlBytes = (size_t)256 << 10;  // (m, l) of the split partials
struct PfSplitPlan {
  int n_parts, part_steps, waves;
  size_t floats;
};
static PfSplitPlan pf_split_plan(const LayerView& L, int S, int H, int pos_base, int num_cus) {
  PfSplitPlan r{1, 0, 4, 0};
  const int G = H / L.kv_heads, QB = 128 / G;
  const int n_items = (S + QB - 1) / QB * L.kv_heads;
  const int KT = L.D == 128 ? PfCfg<128>::KT : PfCfg<256>::KT;
  const int per_cu = L.D == 128 ? 2 : 1;  // workgroups a CU holds
  const long slots = (L.ring.roll && L.ring.head != 0) ? (long)L.max_seq : (long)pos_base + S;
  const int steps_max = (int)((slots + KT - 1) / KT);
  if (2 * n_items > per_cu * num_cus) return r;
  // partials only for the waves holding rows: (query, head) rows of a block, 32 a wave
  const int waves = std::min(4, (std::min(QB, S) * G + 31) / 32);
  const size_t part_bytes = (size_t)waves * 4 * (L.D / 32) * 64 * sizeof(float4);
  const size_t ml_bytes = (size_t)waves * 64 * sizeof(float2);
  int P = per_cu * num_cus / n_items;
  P = std::min(P, steps_max / kPfMinPartSteps);
  P = std::min(P, (int)(kPfSplitMaxBytes / (part_bytes * n_items)));
  P = std::min(P, (int)(kPfSplitMlBytes / (ml_bytes * n_items)));
  if (P < 2) return r;
  const int ps = (steps_max + P - 1) / P;
  const int np = (steps_max + ps - 1) / ps;
  if (np < 2) return r;
  r.n_parts = np;
  r.part_steps = ps;
  r.waves = waves;
  r.floats = (size_t)n_items * np * part_bytes / sizeof(float);
  return r;
}

size_t prefill_workspace_floats(const LayerView& L, int S, int H, int pos_base, int num_cus) {
  if (!prefill_supported(L, S, H)) return 0;
  return pf_split_plan(L, S, H, pos_base, num_cus).floats;
}

size_t prefill_split_ml_bytes() { return kPfSplitMlBytes; }

size_t prefill_workspace_floats_max(const LayerView& L, int S, int H, int num_cus) {
  if (!prefill_supported(L, S, H)) return 0;
  const int G = H / L.kv_heads, QB = 128 / G;
  const int n_items = (S + QB - 1) / QB * L.kv_heads;
  const int per_cu = L.D == 128 ? 2 : 1;
  if (2 * n_items > per_cu * num_cus) return 0;
  return kPfSplitMaxBytes / sizeof(float);
}

template <int D, int DT, bool ROLL>
static hipError_t launch_pf(const PrefillParams& p, hipStream_t st) {
  const int n_items = p.n_qblocks * p.L.kv_heads;
  hipLaunchKernelGGL((prefill_kernel<D, DT, ROLL>), dim3(n_items * p.n_parts), dim3(256), 0, st, p);
  if (p.n_parts > 1)
    hipLaunchKernelGGL((prefill_merge_kernel<D>), dim3(n_items * p.split_waves * 4 * (D / 32)), dim3(256), 0, st, p);
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
  p.mirror = pf_mirror(L, p.n_qblocks * L.kv_heads, a.num_cus);
  p.n_parts = 1;
  p.part_steps = 0;
  p.split_waves = 4;
  p.pws = nullptr;
  p.pml = nullptr;
  const PfSplitPlan sp = pf_split_plan(L, a.S, a.H, a.pos_base, a.num_cus);
  if (sp.n_parts > 1) {
    if (!a.ws_o || !a.pf_ml || sp.floats > a.ws_floats) return hipErrorInvalidValue;  // the caller sizes them
    p.n_parts = sp.n_parts;
    p.part_steps = sp.part_steps;
    p.split_waves = sp.waves;
    p.pws = (float4*)a.ws_o;
    p.pml = (float2*)a.pf_ml;
    p.mirror = 0;
  }
  const bool roll = L.ring.roll != 0;
  if (L.D == 128) {
    if (L.dtype == KV_Q8) return roll ? launch_pf<128, KV_Q8, true>(p, st) : launch_pf<128, KV_Q8, false>(p, st);
    return roll ? launch_pf<128, KV_F16, true>(p, st) : launch_pf<128, KV_F16, false>(p, st);
  }
  if (L.dtype == KV_Q8) return roll ? launch_pf<256, KV_Q8, true>(p, st) : launch_pf<256, KV_Q8, false>(p, st);
  return roll ? launch_pf<256, KV_F16, true>(p, st) : launch_pf<256, KV_F16, false>(p, st);
}

}  // namespace bg
