// 1-bit decode projections on either side of attention (M = 1 GEMVs over sign-bit weights).
//
// Replaces matmul_split_sg.wgsl (fusedMM: the qkv and gate/up projections, outputs routed to up
// to three buffers by row range) and matmul_resid_mr_sg.wgsl (residMM: o_proj / down_proj with
// the residual added), src/engine.ts:1344-1380, and fuses the decode attention prologue into
// the qkv projection (src/engine.ts:1526-1540: matmul_split_sg, appendKV(V), rmsnorm_rope_sg(Q),
// ROPE_K / rmsnorm_rope_sg_kv8(K)).
//
// Weights: row n, weight k is bit k % 32 of sign word [n][k / 32] (set = +1, clear = -1) times the
// f32 scale [n][k / 128] (shaders/matmul_split_sg.wgsl:24-35).
//
//   rows    a wave computes kGemvRW output rows; a lane owns one 32-weight word of each row per
//           2048-weight tile of K. Rows up to kLutMaxK long (the Qwen3-8B qkv and o_proj): the
//           workgroup first tabulates, for every word of x and each of its 8 nibbles, the 16
//           signed sums of the nibble's 4 x values (64 KB of LDS at K = 4096); a word's signed sum
//           is then 8 table reads (indexed by the word's nibbles) and 7 adds instead of 32
//           sign flips and adds. Longer rows: the lane holds the 32 x values under its word
//           (eight 16-byte loads from LDS or memory, reused by the wave's rows) and the word's
//           signs flip their sign bits (one xor each), four partial sums per word. Either way
//           times the word's block scale; a DPP / permlane wave sum finishes the row. With the
//           table (at most two tiles) x is loaded first and both tiles' weights are issued
//           before the table is built, so it is built under their latency; longer
//           rows keep two tiles' loads (the rows' words and scales, x) in flight, the next tile
//           issued before the current one's arithmetic. The residual is loaded at the start.
//   fused   the qkv kernel's workgroups own 32 rows of one head; all but the head's last one
//           store their raw rows into the cache's gather buffer (the XCD's L2 when the head's
//           workgroups share an XCD) and are done; the last one polls them in (no arrival
//           ticket, no store acknowledgement: 6.66 -> 5.9 us at the 8B shape), writes the
//           empty markers back at once, normalizes and ropes the head (Q -> q_out; K -> the
//           cache row, unroped in sink mode) or stores it (V), with the fused prologue's row
//           arithmetic (bg_qkrow.h; the rope partner by a lane exchange). Markers first, the
//           lane exchange and x before the weights: 5.65 -> 5.30 us; 24-row workgroups over
//           every CU (a workgroup may hold the end of one head and the start of the next): 5.19;
//           the poll before the finisher's barrier: 4.85.
#include <map>
#include <mutex>

#include "bg_kernels.h"
#include "bg_qkrow.h"

namespace bg {

// 2 rows a wave, 8 waves a workgroup (16 rows): o_proj at the 8B shape 3.8 us against 4.4 with 4
// rows on 4 waves (the same rows a workgroup, twice the waves to cover the loads' latency), 4.3
// with 4 rows on 8 waves
constexpr int kGemvRW = 2;
constexpr int kGemvWaves = 8;
constexpr int kGemvThreads = 64 * kGemvWaves;

// One 2048-weight tile of a wave's rows: the lane's sign word (word 64t + l) and block scale of
// each row and the 32 x values under the word.
template <int RW>
struct GemvTile {
  uint32_t word[RW];
  float sc[RW];
  float xv[32];
};

// x staged in LDS by the workgroup: word w's 32 values at float offset 36 w (4 floats of pad
// per word keep the lanes' 16-byte reads of consecutive words on different banks)
constexpr int kXPad = 36;
constexpr int kGemvLdsMaxK = 12288;  // 54 KB of LDS; longer rows read x from global memory

// Where a lane finds the x values under its words: kXGlobal (memory), kXLds (x staged in LDS),
// kXLut (the nibble table below; K <= kLutMaxK)
constexpr int kXGlobal = 0, kXLds = 1, kXLut = 2;
constexpr int kLutMaxK = 4096;  // 16 K bytes of LDS: 64 KB at the limit

__host__ __device__ constexpr size_t gemv_lut_bytes(int K) { return (size_t)K * 16; }

// The nibble table: lut[(16 g + e) W + w] = sum over k < 4 of (bit k of e set ? +x : -x) of
// x[32 w + 4 g + k], summed as (k0, k1) + (k2, k3): every signed combination of a nibble's four
// x values (bit set = weight +1, as in the word loop). W-fastest, so the lanes' reads (one word
// each) fall on distinct banks. The NT threads of the workgroup build it (ceil(8 K / 32 / NT)
// (word, nibble) pairs each at most) in two parts: the x loads are issued before the weight loads
// (vector-memory waits retire in issue order, so the build then waits for x alone and runs under
// the weights' latency), the table is written after them, then a barrier.
template <int NT>
struct LutX {
  static constexpr int kPairs = (8 * (kLutMaxK / 32) + NT - 1) / NT;
  float4 v[kPairs];
};
// pair i = g W + w (i < 8 W <= 1024): g = floor(i * ceil(2^20 / W) / 2^20), exact for W < 1000
__device__ __forceinline__ int lut_pair_g(int i, unsigned inv_w) { return (int)(__umul24((unsigned)i, inv_w) >> 20); }
template <int NT>
__device__ __forceinline__ void gemv_lut_load(const float* __restrict__ x, int K, LutX<NT>& X) {
  const int W = K >> 5;
  const unsigned inv_w = ((1u << 20) + W - 1) / W;
#pragma unroll
  for (int j = 0; j < LutX<NT>::kPairs; j++) {
    const int i = threadIdx.x + NT * j;
    const int ic = i < 8 * W ? i : 8 * W - 1;  // unconditional load, as for the weights
    const int g = lut_pair_g(ic, inv_w), w = ic - g * W;
    X.v[j] = *(const float4*)(x + 32 * w + 4 * g);
  }
}
template <int NT>
__device__ __forceinline__ void gemv_lut_write(const LutX<NT>& X, float* lut, int K) {
  const int W = K >> 5;
  const unsigned inv_w = ((1u << 20) + W - 1) / W;
#pragma unroll
  for (int j = 0; j < LutX<NT>::kPairs; j++) {
    const int i = threadIdx.x + NT * j;
    if (i < 8 * W) {
      const int g = lut_pair_g(i, inv_w), w = i - g * W;
      const float4 v = X.v[j];
      const float a[4] = {-v.x - v.y, v.x - v.y, v.y - v.x, v.x + v.y};
      const float b[4] = {-v.z - v.w, v.z - v.w, v.w - v.z, v.z + v.w};
      float* d = lut + (size_t)(16 * g) * W + w;
#pragma unroll
      for (int e = 0; e < 16; e++) d[(size_t)e * W] = a[e & 3] + b[e >> 2];
    }
  }
  __syncthreads();
}
// BF: every load unconditional (clamped address, the value zeroed after), so no branch: the wait
// counts stay exact and a later wait for loads issued before these does not drain them (the
// table build then waits for its x loads alone); otherwise rows past the end are not loaded
template <int RW, bool BF = false>
__device__ __forceinline__ void gemv_load_w(GemvTile<RW>& T, int W, int NB, const uint32_t* __restrict__ sign,
                                            const float* __restrict__ scales, int n0, int n_rows, int t, int lane) {
  const int w = 64 * t + lane;
  const bool ok = w < W;
  const int wc = ok ? w : W - 1;
#pragma unroll
  for (int r = 0; r < RW; r++) {
    const int n = n0 + r;
    const bool v = ok && n < n_rows;
    if constexpr (BF) {
      const int nc = n < n_rows ? n : n_rows - 1;
      const uint32_t wd = sign[(size_t)nc * W + wc];
      const float sc = scales[(size_t)nc * NB + (wc >> 2)];
      T.word[r] = v ? wd : 0u;
      T.sc[r] = v ? sc : 0.0f;
    } else {
      T.word[r] = v ? sign[(size_t)n * W + w] : 0u;
      T.sc[r] = v ? scales[(size_t)n * NB + (w >> 2)] : 0.0f;
    }
  }
}

template <int RW, int XM>
__device__ __forceinline__ void gemv_load_x(GemvTile<RW>& T, const float* __restrict__ x, const float* xs, int W, int t,
                                            int lane) {
  if constexpr (XM == kXLut) return;  // the table holds x
  const int w = 64 * t + lane;
  const bool ok = w < W;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    float4 f;
    if constexpr (XM == kXLds) f = ok ? *(const float4*)(xs + kXPad * w + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
    else f = ok ? *(const float4*)(x + 32 * w + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
    T.xv[4 * j] = f.x;
    T.xv[4 * j + 1] = f.y;
    T.xv[4 * j + 2] = f.z;
    T.xv[4 * j + 3] = f.w;
  }
}

template <int RW, int XM, bool BF>
__device__ __forceinline__ void gemv_load(GemvTile<RW>& T, const float* __restrict__ x, const float* xs, int W, int NB,
                                          const uint32_t* __restrict__ sign, const float* __restrict__ scales,
                                          int n0, int n_rows, int t, int lane) {
  gemv_load_w<RW, BF>(T, W, NB, sign, scales, n0, n_rows, t, lane);
  gemv_load_x<RW, XM>(T, x, xs, W, t, lane);
}

// stage x[K] into xs (the whole workgroup, coalesced 16-byte loads), then a barrier
__device__ __forceinline__ void gemv_stage_x(const float* __restrict__ x, float* xs, int K) {
  for (int i = threadIdx.x; i < K / 4; i += blockDim.x) {
    const float4 f = *(const float4*)(x + 4 * i);
    *(float4*)(xs + kXPad * (i >> 3) + 4 * (i & 7)) = f;
  }
  __syncthreads();
}

template <int RW, int XM>
__device__ __forceinline__ void gemv_accumulate(const GemvTile<RW>& T, float (&acc)[RW], const float* lut, int W, int t,
                                                int lane) {
  if constexpr (XM == kXLut) {
    // a lane past the last word reads word W-1's entries, weighted by its zero scale; entry
    // (g, e) of the lane's word at byte (16 g + e) 4W + 4w (24-bit products: the table is 64 KB)
    const int w = min(64 * t + lane, W - 1);
    const unsigned W4 = 4u * (unsigned)W;
    const char* rowg[8];
#pragma unroll
    for (int g = 0; g < 8; g++) rowg[g] = (const char*)lut + 4 * w + __umul24(16u * g, W4);
#pragma unroll
    for (int r = 0; r < RW; r++) {
      const uint32_t wd = T.word[r];
      float l[8];
#pragma unroll
      for (int g = 0; g < 8; g++) l[g] = *(const float*)(rowg[g] + __umul24(__builtin_amdgcn_ubfe(wd, 4 * g, 4), W4));
      acc[r] = fmaf(((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7])), T.sc[r], acc[r]);
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < RW; r++) {
    // clear bit i -> weight -1: flip the sign bit of x_i
    const uint32_t nw = ~T.word[r];
    float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 32; i++) p[i & 3] += __uint_as_float(__float_as_uint(T.xv[i]) ^ ((nw << (31 - i)) & 0x80000000u));
    acc[r] = fmaf((p[0] + p[1]) + (p[2] + p[3]), T.sc[r], acc[r]);
  }
}

// totals of rows n0 .. n0 + RW - 1 (rows >= n_rows give 0); every lane holds every total. Two
// tiles are in flight: the next tile's loads are issued before the current tile's arithmetic
// (a uniform trip count, so the compiler keeps them outstanding across the loop head).
// (the caller issues tile 0's weight loads into A, then stages x or builds the table, then calls
// this; xs is the staged x or the table)
template <int RW, int XM, bool BF>
__device__ inline void gemv_rows(GemvTile<RW>& A, const float* __restrict__ x, const float* xs, int K,
                                 const uint32_t* __restrict__ sign, const float* __restrict__ scales, int n0, int n_rows,
                                 int lane, float (&tot)[RW]) {
  const int W = K >> 5, NB = K >> 7;
  const int n_tiles = (W + 63) >> 6;
  float acc[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) acc[r] = 0.0f;
  GemvTile<RW> B;
  gemv_load_x<RW, XM>(A, x, xs, W, 0, lane);
  int t = 0;
  for (; t + 2 <= n_tiles; t += 2) {
    gemv_load<RW, XM, BF>(B, x, xs, W, NB, sign, scales, n0, n_rows, t + 1, lane);
    gemv_accumulate<RW, XM>(A, acc, xs, W, t, lane);
    if (t + 2 < n_tiles) gemv_load<RW, XM, BF>(A, x, xs, W, NB, sign, scales, n0, n_rows, t + 2, lane);
    gemv_accumulate<RW, XM>(B, acc, xs, W, t + 1, lane);
  }
  if (t < n_tiles) gemv_accumulate<RW, XM>(A, acc, xs, W, t, lane);
#pragma unroll
  for (int r = 0; r < RW; r++) tot[r] = wave_sum(acc[r]);
}

// rows at most kLutMaxK long: the totals of the (at most) two tiles A (tile 0) and B (tile 1),
// both loaded before the table was written
template <int RW>
__device__ __forceinline__ void gemv_lut_rows(const GemvTile<RW>& A, const GemvTile<RW>& B, const float* lut, int W,
                                              int lane, float (&tot)[RW]) {
  float acc[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) acc[r] = 0.0f;
  gemv_accumulate<RW, kXLut>(A, acc, lut, W, 0, lane);
  if (W > 64) gemv_accumulate<RW, kXLut>(B, acc, lut, W, 1, lane);
#pragma unroll
  for (int r = 0; r < RW; r++) tot[r] = wave_sum(acc[r]);
}

template <int XM>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) float xs[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int N = a.N0 + a.N1 + a.N2;
  const int n0 = (blockIdx.x * kGemvWaves + wave) * kGemvRW;
  // lane r < kGemvRW stores row n0 + r: its residual and the first tile's weights are loaded
  // before x is staged
  LutX<kGemvThreads> X;
  if constexpr (XM == kXLut) gemv_lut_load<kGemvThreads>(a.x, a.K, X);
  const float res = (a.resid && lane < kGemvRW && n0 + lane < N) ? a.resid[n0 + lane] : 0.0f;
  GemvTile<kGemvRW> A;
  gemv_load_w<kGemvRW, XM == kXLut>(A, a.K >> 5, a.K >> 7, a.sign, a.scales, n0, N, 0, lane);
  float tot[kGemvRW];
  if constexpr (XM == kXLut) {
    // K <= kLutMaxK: at most two tiles, both issued before the table is written, so the second
    // tile's latency runs under the build too (o_proj at the 8B shape: 3.77 -> 3.60 us)
    const int W = a.K >> 5;
    GemvTile<kGemvRW> B;
    gemv_load_w<kGemvRW, true>(B, W, a.K >> 7, a.sign, a.scales, n0, N, 1, lane);
    gemv_lut_write<kGemvThreads>(X, xs, a.K);
    if (n0 >= N) return;  // wave-uniform
    gemv_lut_rows<kGemvRW>(A, B, xs, W, lane, tot);
  } else {
    if constexpr (XM == kXLds) gemv_stage_x(a.x, xs, a.K);
    if (n0 >= N) return;  // wave-uniform
    gemv_rows<kGemvRW, XM, false>(A, a.x, xs, a.K, a.sign, a.scales, n0, N, lane, tot);
  }
#pragma unroll
  for (int r = 0; r < kGemvRW; r++) {
    const int n = n0 + r;
    if (lane == r && n < N) {
      const float y = a.resid ? tot[r] + res : tot[r];
      if (n < a.N0) a.out0[n] = y;
      else if (n < a.N0 + a.N1) a.out1[n - a.N0] = y;
      else a.out2[n - a.N0 - a.N1] = y;
    }
  }
}

// the LDS a kernel may take beyond the default (at most 64 KB of table plus a few static arrays),
// set once per kernel
static hipError_t gemv_allow_lds(const void* fn, size_t bytes) {
  static std::mutex mu;
  static std::map<const void*, size_t> allowed;
  std::lock_guard<std::mutex> lock(mu);
  size_t& a = allowed[fn];
  if (bytes <= a) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess) a = bytes;
  return e;
}

hipError_t launch_gemv(const GemvArgs& a, hipStream_t st) {
  const int N = a.N0 + a.N1 + a.N2;
  if (N <= 0) return hipSuccess;
  const int waves = (N + kGemvRW - 1) / kGemvRW;
  const dim3 g((waves + kGemvWaves - 1) / kGemvWaves);
  if (a.K <= kLutMaxK) {
    const size_t lds = gemv_lut_bytes(a.K);
    const hipError_t e = gemv_allow_lds((const void*)gemv_kernel<kXLut>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gemv_kernel<kXLut>, g, dim3(kGemvThreads), lds, st, a);
  } else if (a.K <= kGemvLdsMaxK) {
    const size_t lds = (size_t)(a.K / 32) * kXPad * sizeof(float);
    hipLaunchKernelGGL(gemv_kernel<kXLds>, g, dim3(kGemvThreads), lds, st, a);
  } else {
    hipLaunchKernelGGL(gemv_kernel<kXGlobal>, g, dim3(kGemvThreads), 0, st, a);
  }
  return hipGetLastError();
}

// ---- fused decode qkv projection + prologue ---------------------------------------------------
// RPW rows a workgroup (RPW / kGemvRW waves): 32 (16 waves), or 24 (12 waves) when 32-row
// workgroups would leave CUs idle (the 8B shape: 256 workgroups of 24 rows instead of 192 of 32,
// 5.27 -> 5.19 us; the table reads are VALU-bound, so the rows a CU holds set that phase). 192 of
// 32 rows measured 6.7 us against 384 of 16 rows, two on half the CUs (7.3 us), or 96 of 64 (7.5).
// s_waitcnt vmcnt(0) with expcnt and lgkmcnt left alone (gfx9 encoding: vmcnt bits 3:0 and 15:14,
// expcnt 6:4, lgkmcnt 11:8)
constexpr int kWaitVm0 = 0x0F70;
template <int RPW>
constexpr int qkv_threads() { return 64 * RPW / kGemvRW; }
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

size_t qkv_proj_raw_floats(int heads, int D) { return (size_t)heads * D; }

// Workgroup v owns rows [v RPW, v RPW + RPW) of the [Q heads | K heads | V heads] x D output.
// The workgroup holding a head's last row finishes that head: its rows of the head stay in LDS,
// its rows of the next head (RPW < D: a workgroup can straddle two heads) and every other
// workgroup's rows go into the gather buffer. The finisher's first wave polls the head's earlier
// rows until none holds the empty marker (the data is the completion signal: no ticket, no store
// acknowledgement to wait for) while its sibling waves finish their rows, and meets them at the
// barrier only after the poll (5.05 -> 4.85 us at the 8B shape); it then writes the marker back
// (written through: the next launch's workgroups may run on another XCD), normalizes, ropes and
// stores the row with the prologue's arithmetic (bg_qkrow.h: bit-identical to bg_gemv_split
// followed by bg_qkv_prologue). The rows a finisher waits on belong to lower workgroup indices,
// dispatched before it, which finish on their own; the wait is still bounded (a finisher that
// gives up stores NaN and raises the cache's error word). When the grid is a multiple of 8 and
// every eighth of the rows is whole heads, blockIdx 8m + x is workgroup v = x (grid / 8) + m, so
// with round-robin placement each XCD holds a run of whole heads and the raw rows stay in its L2.
template <int D, int DT, int XM, int RPW>
__global__ __launch_bounds__(qkv_threads<RPW>()) void qkv_proj_kernel(LayerView L, QkvProjArgs a) {
  constexpr int NT = qkv_threads<RPW>();
  constexpr int LPR = D / 4;  // lanes per row in the epilogue
  constexpr int kSC1 = 16;    // cache policy sc1: agent scope
  extern __shared__ __align__(16) float xs[];
  __shared__ __align__(16) float rrow[D];
  __shared__ __align__(16) float own[RPW];
  // wave-uniform (scalar): the finisher's waves take different branches around one barrier
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int KV = L.kv_heads;
  const int nq = a.H * D;
  const int N = nq + 2 * KV * D;  // gridDim.x * RPW
  const int nwg = gridDim.x;
  const bool grouped = (nwg & 7) == 0 && ((nwg >> 3) * RPW) % D == 0;
  const int v = grouped ? (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int r0 = v * RPW;
  const int head = r0 / D;  // of the first row; 0 .. H-1: Q heads, then K heads, then V heads
  const int hend = (head + 1) * D;
  const bool finisher = r0 + RPW >= hend;  // holds the head's last row
  const int own0 = r0 - head * D;          // the finisher's first dim of the head
  // raw rows stay in the XCD's L2 when every workgroup of the head shares it
  const bool local = grouped && a.n_xcd == 8;
  {
    const int n0 = r0 + wave * kGemvRW;
    GemvTile<kGemvRW> A;
    float tot[kGemvRW];
    if constexpr (XM == kXLut) {
      // x first, then both tiles' weights (branch-free), so the table is built under their latency
      LutX<NT> X;
      gemv_lut_load<NT>(a.x, a.K, X);
      GemvTile<kGemvRW> B;
      gemv_load_w<kGemvRW, true>(A, a.K >> 5, a.K >> 7, a.sign, a.scales, n0, N, 0, lane);
      gemv_load_w<kGemvRW, true>(B, a.K >> 5, a.K >> 7, a.sign, a.scales, n0, N, 1, lane);
      gemv_lut_write<NT>(X, xs, a.K);
      gemv_lut_rows<kGemvRW>(A, B, xs, a.K >> 5, lane, tot);
    } else {
      gemv_load_w<kGemvRW>(A, a.K >> 5, a.K >> 7, a.sign, a.scales, n0, N, 0, lane);
      if constexpr (XM == kXLds) gemv_stage_x(a.x, xs, a.K);
      gemv_rows<kGemvRW, XM, false>(A, a.x, xs, a.K, a.sign, a.scales, n0, N, lane, tot);
    }
#pragma unroll
    for (int r = 0; r < kGemvRW; r++) {
      const int n = n0 + r;
      if (lane != r) continue;
      if (finisher && n < hend) {
        own[n - r0] = tot[r];
      } else if (local) {
        a.raw[n] = tot[r];  // into the XCD's L2
      } else {
        st_coherent(a.raw + n, tot[r]);
      }
    }
  }
  if (!finisher) return;
  if (wave != 0) {
    __syncthreads();  // publishes this wave's rows in own[]; wave 0 polls before it meets them
    return;
  }

  // ---- the finishing part of the head: one wave, 4 dims a lane (D=128: both halves of the
  // wave hold the row; the lower one stores) ----
  const int c = lane % LPR;
  const bool writer = lane < LPR;
  const bool isq = head < a.H, isk = !isq && head < a.H + KV;
  const bool mine = 4 * c >= own0;  // own0 is a multiple of 8
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(a.raw + (size_t)head * D, (short)0,
                                                                      D * 4, 0x00020000);
  // the row's gamma and rope tables are loaded before the wait, so the epilogue starts on arrival
  const bool rope = isq || (isk && !L.ring.roll);  // sink mode caches K unroped (src/engine.ts:1530-1533)
  float g[4] = {1.0f, 1.0f, 1.0f, 1.0f}, cs[4], sn[4];
  if (isq || isk) load4((isq ? a.q_gamma : a.k_gamma) + 4 * c, g);
  if (rope) row_tables(a.cos_tab, a.sin_tab, a.pos, a.rot_dim, c, cs, sn);
  // the other workgroups' rows are polled before the barrier, under the sibling waves' rows
  float x[4];
  bool gave_up = false;
  if (!mine) {
    const int spins = a.spin_limit > 0 ? a.spin_limit : (1 << 20);
    bool missing = true;
    for (int it = 0; it < spins && missing; it++) {
      // a compiler memory barrier: the load is issued again every round (other workgroups
      // write the rows; without it the compiler may reuse the last round's value)
      __asm__ volatile("" ::: "memory");
      const floatx4_t v = __builtin_bit_cast(floatx4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * c, 0, kSC1));
#pragma unroll
      for (int e = 0; e < 4; e++) x[e] = v[e];
      missing = false;
#pragma unroll
      for (int e = 0; e < 4; e++) missing = missing || __float_as_uint(x[e]) == kWorkspaceEmpty;
      if (missing) __builtin_amdgcn_s_sleep(1);
    }
    gave_up = missing;
  }
  __syncthreads();  // the sibling waves' rows in own[]
  if (mine) {
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = own[4 * c + e - own0];
  }
  gave_up = __any(gave_up);
  // the empty marker back into the slots read, as soon as they are in registers (before the
  // row's stores: a marker store issued after them would wait for their acknowledgement, since
  // it reuses their data registers). Every load has arrived here (the poll waited for its own,
  // issued after gamma and the tables); the explicit vmcnt(0) says so to the compiler, which
  // would otherwise wait for the marker store's acknowledgement before using gamma.
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  if (writer && !mine) {
    const u32x4_t empty4 = {kWorkspaceEmpty, kWorkspaceEmpty, kWorkspaceEmpty, kWorkspaceEmpty};
    __builtin_amdgcn_raw_buffer_store_b128(empty4, rs, 16 * c, 0, kSC1);
  }
  if (gave_up) {
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = __builtin_nanf("");
  }
  if (isq || isk) {
    row_scale(x, row_inv_rms<D, LPR>(x, a.eps), g);
    if (rope) {
      // the rotate_half partners by a lane exchange where the width allows it, else through LDS
      float pr[4];
      if (rope_partner_lanes(x, a.rot_dim, pr)) {
        row_rope_lanes(x, pr, c, a.rot_dim, cs, sn);
      } else {
        if (writer) *(float4*)(rrow + 4 * c) = make_float4(x[0], x[1], x[2], x[3]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        row_rope(x, rrow, c, a.rot_dim, cs, sn);
      }
    }
    if (isq) {
      if (writer) *(float4*)(a.q_out + head * D + 4 * c) = make_float4(x[0], x[1], x[2], x[3]);
    } else {
      // every lane joins the q8 block maxima; the lower half stores
      if (D == 256 || writer) store_k4<D, DT>(L, L.ring.phys(a.slot), head - a.H, x, c);
    }
  } else {
    if (D == 256 || writer) store_v4<D, DT>(L, L.ring.phys(a.slot), head - a.H - KV, x, c);
  }
  if (gave_up && lane == 0) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

template <int D, int DT, int XM, int RPW>
static hipError_t launch_qkv_proj_k(const LayerView& L, const QkvProjArgs& a, dim3 g, size_t lds, hipStream_t st) {
  if constexpr (XM == kXLut) {
    const hipError_t e = gemv_allow_lds((const void*)qkv_proj_kernel<D, DT, XM, RPW>, lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((qkv_proj_kernel<D, DT, XM, RPW>), g, dim3(qkv_threads<RPW>()), lds, st, L, a);
  return hipGetLastError();
}

template <int D, int XM, int RPW>
static hipError_t launch_qkv_proj_d(const LayerView& L, const QkvProjArgs& a, dim3 g, size_t lds, hipStream_t st) {
  switch (L.dtype) {
    case KV_F32: return launch_qkv_proj_k<D, KV_F32, XM, RPW>(L, a, g, lds, st);
    case KV_F16: return launch_qkv_proj_k<D, KV_F16, XM, RPW>(L, a, g, lds, st);
    default: return launch_qkv_proj_k<D, KV_Q8, XM, RPW>(L, a, g, lds, st);
  }
}

template <int D, int RPW>
static hipError_t launch_qkv_proj_x(const LayerView& L, const QkvProjArgs& a, dim3 g, hipStream_t st) {
  if (a.K <= kLutMaxK) return launch_qkv_proj_d<D, kXLut, RPW>(L, a, g, gemv_lut_bytes(a.K), st);
  if (a.K <= kGemvLdsMaxK)
    return launch_qkv_proj_d<D, kXLds, RPW>(L, a, g, (size_t)(a.K / 32) * kXPad * sizeof(float), st);
  return launch_qkv_proj_d<D, kXGlobal, RPW>(L, a, g, 0, st);
}

hipError_t launch_qkv_proj(const LayerView& L, const QkvProjArgs& a, hipStream_t st) {
  const int N = (a.H + 2 * L.kv_heads) * L.D;
  // 24-row workgroups (D = 128) when 32-row ones would leave CUs idle and the rows fall into 8
  // runs of whole heads (one an XCD)
  if (L.D == 128 && N / 32 < a.num_cus && N % (24 * 8) == 0 && (N / 8) % 128 == 0)
    return launch_qkv_proj_x<128, 24>(L, a, dim3(N / 24), st);
  const dim3 g(N / 32);
  return L.D == 128 ? launch_qkv_proj_x<128, 32>(L, a, g, st) : launch_qkv_proj_x<256, 32>(L, a, g, st);
}

}  // namespace bg
