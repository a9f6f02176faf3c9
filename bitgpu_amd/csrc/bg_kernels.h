// Host-side launchers of the gfx950 kernels (defined in the .hip files, called by bg_api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bg_common.h"

namespace bg {

// One layer's device buffers plus the geometry the kernels need.
struct LayerView {
  void* k;            // K data
  void* v;            // V data (transposed 32-slot tiles)
  float* ks;          // q8 K scales (nullptr otherwise)
  float* vs;          // q8 V scales
  int cap;            // physical slots (multiple of 32)
  int kv_heads;
  int D;
  int dtype;          // KvType
  Ring ring;
  int max_seq;
  // read-time rotation (sink mode)
  const float* cos_tab;
  const float* sin_tab;
  int rope_positions;
  int rope_abs;       // 1: rotate by absolute position (slot + evicted for slots >= sinks)
  int64_t evicted;    // rows dropped by eviction so far
  int q8_row;         // q8 writes: 1 = one scale per row (its maximum, stored in every 32-value
                      // scale slot), 0 = one scale per 32 values
};

// kv_pack.hip
hipError_t launch_kv_write(const LayerView& L, int which, const float* src, int rows, int dst_row0,
                           hipStream_t st);
hipError_t launch_kv_export(const LayerView& L, int region, int base, int count, void* dst, hipStream_t st);
hipError_t launch_kv_import(const LayerView& L, int region, int base, int count, const void* src, hipStream_t st);
// q8 layer -> f16 copy of slots [0, n_slots) (n_slots a multiple of 32) laid out like an f16
// cache of the same capacity, with the q8 prefill staging's exact values
hipError_t launch_kv_dequant_f16(const LayerView& L, int n_slots, void* kdst, void* vdst, hipStream_t st);

// norm_rope.hip
struct PrologueArgs {
  const float* q; int q_stride;
  const float* k; const float* v;
  int S, H;
  const float* q_gamma; const float* k_gamma; float eps;
  const float* cos_tab; const float* sin_tab; int rot_dim;
  int pos0, slot0;
  float* q_out;
};
hipError_t launch_qkv_prologue(const LayerView& L, const PrologueArgs& a, hipStream_t st);

// gemv.hip: 1-bit decode projections. Row n, weight k = bit k % 32 of sign[n][k / 32] (set =
// +1) times scales[n][k / 128]; K a multiple of 128.
struct GemvArgs {
  const float* x; int K;
  const uint32_t* sign; const float* scales;
  int N0, N1, N2;                  // rows [0, N0) -> out0, [N0, N0+N1) -> out1, the rest -> out2
  float* out0; float* out1; float* out2;
  const float* resid;              // nullable: added to every output (the residual form)
};
hipError_t launch_gemv(const GemvArgs& a, hipStream_t st);
// fused decode qkv projection + prologue over the rows of H query heads, then KV key and KV
// value heads of the cache's head_dim
struct QkvProjArgs {
  const float* x; int K;
  const uint32_t* sign; const float* scales;
  int H;
  const float* q_gamma; const float* k_gamma; float eps;
  const float* cos_tab; const float* sin_tab; int rot_dim;
  int pos, slot;
  float* q_out;                    // [H, D] normed, roped rows
  float* raw;                      // [H + 2 KV][D] raw rows a head's finishing workgroup gathers;
                                   // every value the empty marker (kWorkspaceEmpty) between launches
  unsigned* err;                   // host-visible error word: a finisher's bounded wait gave up
  int spin_limit;                  // poll rounds before a finisher gives up (0: 2^20)
  int n_xcd;                       // > 0: workgroups go to XCDs round robin (see AttnArgs)
  int num_cus;                     // compute units: 24-row workgroups when 32-row ones leave some idle
};
// raw-row floats the fused projection's gather buffer holds (heads of every kind x head_dim)
size_t qkv_proj_raw_floats(int heads, int D);
// Arrival counters (the fused projection's per head, the f32 decode's per kv head) sit 256 bytes
// apart: 384 workgroups' atomics on counters packed into two lines serialize (the 8B-shape qkv
// projection took 8.6 us with them packed, 7.5 us apart).
constexpr int kCounterStride = 64;
hipError_t launch_qkv_proj(const LayerView& L, const QkvProjArgs& a, hipStream_t st);

// attention (decode.hip, attn_f32.hip, prefill.hip)
struct AttnArgs {
  const float* q;
  int S, H;
  int pos_base;
  float scale;
  const float* gate; int gate_stride;
  float* out;
  // split-K workspace
  float* ws_o; float* ws_ml; unsigned* ws_count; size_t ws_floats;
  // split-K prefill: (m, l) of the partials, prefill_split_ml_bytes() long (outside ws_o, whose
  // slots hold the empty marker between launches)
  float* pf_ml;
  int num_cus;
  // decode merge: host-visible error word, poll bound (0: default) and a test hook that makes
  // one split store no partial (-1: none)
  unsigned* err; int spin_limit; int withhold_split;
  // XCDs the GPU dispatches workgroups to round robin (workgroup b on XCD (b + r) mod n_xcd, r
  // the same for the whole grid; checked on the device once): the decode kernel then exchanges
  // split partials through one XCD's L2. 0: partials are written through to memory.
  int n_xcd;
};
// workgroup placement check of the current device: n_xcd > 0 when a probe grid's workgroups all
// ran on XCD (blockIdx + r) mod n_xcd for one r (decode.hip)
hipError_t probe_xcd_round_robin(int* n_xcd);
hipError_t launch_attention_f32(const LayerView& L, const AttnArgs& a, hipStream_t st);
// split-K f32 decode / verify (G*S <= 16 rows per kv head), workspace as for the decode kernel
hipError_t launch_attention_f32_split(const LayerView& L, const AttnArgs& a, hipStream_t st);
bool f32_split_supported(const LayerView& L, int S, int H);
size_t f32_workspace_floats(const LayerView& L, int S, int H);
hipError_t launch_attention_decode(const LayerView& L, const AttnArgs& a, hipStream_t st);
hipError_t launch_attention_prefill(const LayerView& L, const AttnArgs& a, hipStream_t st);
// workspace floats needed by the decode kernel for S rows of H heads; a new workspace is filled
// with the 32-bit pattern decode_workspace_empty() before its first use
size_t decode_workspace_floats(const LayerView& L, int S, int H, int num_cus, size_t* counters);
uint32_t decode_workspace_empty();
// floats of the split partials one decode launch with n_splits splits per kv head writes
size_t decode_partial_floats(const LayerView& L, int S, int H, int n_splits);
bool decode_supported(const LayerView& L, int S, int H);
// the dispatch: decode kernel (true) or prefill kernel for S rows of H heads. Decode takes every
// shape whose rows per kv head fit one 16-row set, and every sink-mode shape it supports; more
// rows go to the (split-K) prefill, except q8 at head_dim 128 up to 24 rows (measured faster).
bool decode_preferred(const LayerView& L, int S, int H);
// the split-K plan of a decode launch (host-only arithmetic; false when the kernel does not take
// the shape). resident_per_cu: workgroups of the launch's instantiation a CU holds at once.
struct DecodePlan {
  int waves, nset, passes;
  int n_scan, phys_limit, n_tiles;
  int tiles_per_split, n_splits, n_mergers, grid;
  int xcd_group;  // > 0: splits numbered in groups of this many per kv head (sink mode), grid padded
  int skip_t0, skip_n;  // a run of whole tiles every row masks (sink mode), not scanned
};
bool decode_plan(const LayerView& L, int S, int H, int pos_base, int num_cus, int resident_per_cu, DecodePlan* out);
// streaming-read floor (diag.hip): `workgroups` contiguous slices of `bytes` read with 16-byte
// loads, one XOR word per workgroup into sink
hipError_t launch_stream_read(const void* buf, size_t bytes, int workgroups, bool nontemporal, unsigned* sink,
                              hipStream_t st);
bool prefill_supported(const LayerView& L, int S, int H);
// a q8 prefill of S rows that stages each K/V tile for enough query blocks to run faster on an
// f16 copy of the attended slots
bool prefill_wants_f16_copy(const LayerView& L, int S, int H);
// "not written yet" marker of a split partial slot: a quiet NaN with a payload arithmetic on
// finite inputs never produces. The decode and split-K prefill kernels share the workspace and
// both leave every slot they use holding it.
constexpr uint32_t kWorkspaceEmpty = 0x7FF1DE5Au;
// workspace floats a prefill launch's split-K partials use at pos_base (0: the launch does not
// split); the most any pos_base can use for S rows of H heads is prefill_workspace_floats_max
size_t prefill_workspace_floats(const LayerView& L, int S, int H, int pos_base, int num_cus);
size_t prefill_workspace_floats_max(const LayerView& L, int S, int H, int num_cus);
size_t prefill_split_ml_bytes();

}  // namespace bg
