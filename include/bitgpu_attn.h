/* bitgpu_attn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Drop-in replacement for the per-layer attention dispatch of bitgpu v0.19.1's WebGPU engine
 * (src/engine.ts). Every entry point names the reference interface it replaces (file:line,
 * relative to the reference repository root).
 *
 * Conventions
 *   - All functions return int32_t status: BG_OK (0) or a negative BG_E_* code; the message of
 *     the last failure on the calling thread is in bg_last_error_message(). Nothing throws.
 *   - Device buffers are plain device pointers (hipMalloc'd or torch-owned); host buffers are
 *     plain host pointers. No framework types cross this boundary.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream). Work is enqueued
 *     in order on that stream; calls return before the GPU finishes unless stated otherwise.
 *   - A cache object is not re-entrant: calls on one cache must be serialized by the caller
 *     (the reference serializes every engine op through one promise chain, src/engine.ts:2877-2887),
 *     and all GPU work on one cache must be ordered on ONE stream: the layers of a cache share
 *     one split workspace and one f16 prefill copy, so two bg_attention calls on different
 *     streams could overlap on the GPU and corrupt each other's partials.
 *   - Kernels never allocate. Host-side allocations happen only in bg_kv_create, bg_kv_grow,
 *     bg_attention_reserve, lazily on the first bg_attention that needs more workspace (split
 *     partials; a split-K prefill also a 256 KiB buffer of their (m, l) values) or, for a q8
 *     cache, the f16 copy a long prefill runs on, and in the snapshot transfers (a staging
 *     buffer kept by the cache, grown when a larger region is transferred).
 *   - The decode kernel's split merge waits a bounded time for the partials of its own grid.
 *     If a wait gives up (the GPU shared with work that keeps the grid from running at once),
 *     that launch stores NaN and raises the cache's error word; the next bg_attention on the
 *     cache, or bg_stream_sync, returns BG_E_DEVICE once and resets the workspace. Until then,
 *     outputs of later launches on the cache may be wrong (a partial that lands after its
 *     merger gave up can be taken by a later launch), not only NaN.
 *   - When the device dispatches workgroups to its XCDs round robin (probed once per device at
 *     bg_kv_create), the decode kernel exchanges the split partials of a kv head through one
 *     XCD's L2. A merger that finds itself on another XCD raises the error word as above and
 *     the library writes partials through to memory from then on.
 *
 * Storage modes mirror EngineOptions.kvCache (src/types.ts:143-154): f32, f16 (one RNE rounding
 * at write, shaders/copy_kv16.wgsl:13) and q8 (int8 codes + one f32 scale per 32 values,
 * shaders/copy_kv8.wgsl:24-40). The device layout is private (head-major, V stored in
 * 32-position transposed tiles); bg_kv_export_rows / bg_kv_import_rows convert to and from the
 * reference's snapshot byte layout (src/engine.ts:2724-2734).
 */
#ifndef BITGPU_ATTN_H
#define BITGPU_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BG_OK 0
#define BG_E_INVALID (-1)     /* bad argument */
#define BG_E_OOM (-2)         /* device allocation failed (the reference's GpuOutOfMemoryError) */
#define BG_E_DEVICE (-3)      /* HIP runtime error */
#define BG_E_UNSUPPORTED (-4) /* shape or mode this build does not implement */
#define BG_E_STATE (-5)       /* not valid in the cache's current state */

enum { BG_KV_F32 = 0, BG_KV_F16 = 1, BG_KV_Q8 = 2 };
enum { BG_K = 0, BG_V = 1, BG_KSCALE = 2, BG_VSCALE = 3 };
enum { BG_ROPE_SLOT = 0, BG_ROPE_ABSOLUTE = 1 };

typedef struct bg_kv_cache bg_kv_cache;

/* ---- utilities ------------------------------------------------------------------------- */

/* Last failure message on this thread ("" if none). Replaces the Error('bitgpu: ...') text of
 * src/errors.ts:14-19. */
const char* bg_last_error_message(void);

/* Library version string. */
const char* bg_version(void);

/* RoPE tables f32 [positions, rot_dim/2]: f64 angles p * theta^(-2j/rot_dim), each entry
 * rounded once to f32; YaRN when yarn_factor > 1 (beta_fast 32, beta_slow 1, mscale
 * 0.1 ln(factor) + 1). Host-only. Replaces synthRope, src/engine.ts:117-147. */
int32_t bg_rope_tables(double theta, int32_t rot_dim, int32_t positions, double yarn_factor,
                       int32_t yarn_original_max_positions, float* cos_out, float* sin_out);

/* Sink-mode eviction arithmetic (host-only, no cache): evict(fill, need) of
 * src/engine.ts:1188-1212. Outputs the new fill, the dropped batch and the kept count. */
int32_t bg_evict_plan(int32_t fill, int32_t need, int32_t sinks, int32_t max_seq_len,
                      int32_t* new_fill, int32_t* batch, int32_t* keep);

/* Sink-mode ring map (host-only): the physical slot holding logical slot `logical` when the
 * ring origin is `head` (logical slots < sinks are fixed; the rest rotate through
 * max_seq_len - sinks slots). With bg_evict_plan it reproduces the reference's compaction
 * (src/engine.ts:1206-1209) as pure index arithmetic. */
int32_t bg_ring_map(int32_t sinks, int32_t max_seq_len, int32_t head, int32_t logical, int32_t* physical);

/* Synchronize a stream (NULL = device). Also reports (BG_E_DEVICE, once) a decode split merge
 * on any live cache that gave up waiting, after resetting that cache's workspace. */
int32_t bg_stream_sync(void* stream);

/* Host-only diagnostic with no counterpart in the reference (the WebGPU kernels have no
 * split-K): the plan bg_attention's split-K decode kernel uses for S query rows of H heads at
 * positions pos_base.. over a plain cache of kv_heads x head_dim (dtype BG_KV_F16 or
 * BG_KV_Q8), on num_cus CUs holding resident_per_cu of its workgroups at once. out[0..5] =
 * waves per workgroup, splits per kv head, 32-slot tiles per split, merging splits per kv
 * head (the last ones), grid size, tiles. The grid never exceeds resident_per_cu * num_cus.
 * A q8 launch of 4-wave workgroups whose waves would take two tiles at one workgroup a CU takes
 * one tile a wave when resident_per_cu >= 2 and the GPU holds that grid (bg_attention runs a
 * one-tile kernel that fits two workgroups a CU there).
 * BG_E_UNSUPPORTED when the shape goes to another kernel. */
int32_t bg_decode_plan(int32_t kv_heads, int32_t head_dim, int32_t dtype, int32_t S, int32_t H,
                       int32_t pos_base, int32_t num_cus, int32_t resident_per_cu, int32_t* out);

/* Test hook with no counterpart in the reference: the decode split merge's poll bound
 * (spin_limit polls before a merger gives up; 0 = the default, 2^20) and one split index that
 * stores no partial (-1 = none), for every later bg_attention / bg_attention_noalloc call in
 * the process. With a small bound and a withheld split the merge gives up while every kernel
 * exits normally (the error path of the bounded wait, forced from the host). Host-only. */
int32_t bg_debug_merge_hooks(int32_t spin_limit, int32_t withhold_split);

/* Measurement aid with no counterpart in the reference: the streaming-read floor the decode
 * kernels are held against. `workgroups` workgroups of 512 threads each read one contiguous
 * slice of the device buffer `buf` (`bytes`, a multiple of 16) with 16-byte loads, eight in
 * flight a lane, nontemporal (the decode tiles' policy) or plain, and fold them by XOR into
 * sink[workgroup] (device memory, `workgroups` words). The XOR of the sink words equals the XOR
 * of the buffer's 32-bit words. Asynchronous on `stream`; allocates nothing. */
int32_t bg_diag_stream_read(const void* buf, size_t bytes, int32_t workgroups, int32_t nontemporal,
                            uint32_t* sink, void* stream);

/* ---- streams and event timing -------------------------------------------------------------
 * For hosts without a GPU runtime of their own (the N-API addon): the reference runs every
 * dispatch on its one WebGPU queue and times with timestamp queries (src/engine.ts:503-506);
 * here a stream is that queue (default priority; NULL = the null stream in every call) and
 * two recorded events give the elapsed time between them (bg_event_elapsed_us waits for
 * `end`). */
int32_t bg_stream_create(void** stream);
int32_t bg_stream_destroy(void* stream);
int32_t bg_event_create(void** event);
int32_t bg_event_record(void* event, void* stream);
int32_t bg_event_elapsed_us(void* start, void* end, float* us);
int32_t bg_event_destroy(void* event);

/* ---- KV cache lifecycle ------------------------------------------------------------------
 * Replaces the Kc/Vc/Ksc/Vsc allocation of src/engine.ts:1044-1079, the kvCache/overflow/
 * sinkTokens/maxSeqLen options (src/types.ts:138-177) and the roll statics (1094-1111).
 * One kv head's K (or V) region of one layer must stay below 2^31 bytes (f32: 4 bytes a value,
 * f16 and q8 2, counting a q8 layer's f16 prefill copy): max_seq_len x head_dim x that at most
 * 2^31 - 1 after rounding up to 32 positions, e.g. at most 4,194,272 positions of f16 at head_dim
 * 256; a larger one is BG_E_UNSUPPORTED. */
int32_t bg_kv_create(int32_t n_layers, int32_t kv_heads, int32_t head_dim, int32_t dtype,
                     int32_t capacity, int32_t max_seq_len, int32_t roll, int32_t sinks,
                     int32_t rope_pos_mode, bg_kv_cache** out);
int32_t bg_kv_destroy(bg_kv_cache* cache);

/* Current capacity in positions. */
int32_t bg_kv_capacity(const bg_kv_cache* cache, int32_t* capacity);

/* ensureKvCapacity, src/engine.ts:1120-1178: grow every layer to >= min(needed, max_seq_len)
 * positions (doubling), preserving content. On allocation failure the cache keeps its old
 * buffers and BG_E_OOM is returned (the reference's rollback, 1157-1173). Synchronous. */
int32_t bg_kv_grow(bg_kv_cache* cache, int32_t needed, void* stream);

/* q8 scale block (src/types.ts:145-147: the reference quantizes per 32 values,
 * shaders/copy_kv8.wgsl:30-36): 32 (the default) or head_dim, one scale per (position, kv head)
 * row -- the row's maximum |value|, stored in each of the row's head_dim/32 scale slots, so the
 * cache layout, the attention kernels and the snapshot format are the same in both modes.
 * Applies to the writes that follow. BG_E_STATE for a cache that is not q8. */
int32_t bg_kv_set_q8_block(bg_kv_cache* cache, int32_t block);

/* Device rope tables [positions, rot_dim/2] used for the sink-mode read-time K rotation
 * (the rollCosT/rollSinT bindings of attIns, src/engine.ts:1097-1104,1395-1399). The caller
 * owns the buffers; they must cover max_seq_len positions (slot mode) or every absolute
 * position attended (absolute mode). */
int32_t bg_kv_set_rope(bg_kv_cache* cache, const float* cos_tab, const float* sin_tab,
                       int32_t positions, int32_t rot_dim);

/* ---- KV writes ---------------------------------------------------------------------------- */

/* appendKV, src/engine.ts:1385-1393 (copy.wgsl / copy_kv16.wgsl / copy_kv8.wgsl): `rows` f32
 * rows of head_dim values, row r landing at reference cache row dst_row0 + r, i.e. logical
 * position (dst_row0 + r) / kv_heads and kv head (dst_row0 + r) % kv_heads. which = BG_K|BG_V. */
int32_t bg_kv_write(bg_kv_cache* cache, int32_t layer, int32_t which, const float* src,
                    int32_t rows, int32_t dst_row0, void* stream);

/* Fused attention prologue for S positions in one launch, replacing (src/engine.ts)
 *   decode : rmsnorm_rope_sg(Q) + ROPE_K / rmsnorm_rope_sg_kv8(K into the cache) + appendKV(V)
 *            (1527-1540; shaders/rmsnorm_rope_sg*.wgsl)
 *   prefill: rms(q), rms(k), rope(q), rope(k), appendKV(K), appendKV(V) (1569-1576)
 *   hybrid : split_head(query) + rms + rope_partial (q and k) + appendKV(K, V) (1470-1485)
 * q: [S, H, q_stride] (first head_dim values of each row are the query; q_stride = 2*head_dim
 * reads the hybrid's interleaved query|gate projection), k, v: [S, KV, head_dim]. Any of q, k,
 * v may be NULL to skip that part. Q rows are RMSNormed with q_gamma, roped at pos0 + s and
 * written to q_out [S, H, head_dim]; K rows are normed with k_gamma, roped at pos0 + s (left
 * unroped in a sink-mode cache, which rotates at read) and stored at logical slot slot0 + s;
 * V rows are stored unchanged at slot0 + s. Tables cos_tab/sin_tab: [rope_positions,
 * rot_dim/2] (the engine's cos/sin caches, indexed by position instead of the per-call [S, D]
 * expansion of ropeBufs, src/engine.ts:994-1009); rot_dim <= head_dim (dims >= rot_dim pass
 * through). Every buffer is 16-byte aligned and q_stride a multiple of 4 (rows move 16 bytes a
 * lane); otherwise BG_E_INVALID. */
int32_t bg_qkv_prologue(bg_kv_cache* cache, int32_t layer, const float* q, int32_t q_stride,
                        const float* k, const float* v, int32_t S, int32_t H,
                        const float* q_gamma, const float* k_gamma, float eps,
                        const float* cos_tab, const float* sin_tab, int32_t rope_positions,
                        int32_t rot_dim, int32_t pos0, int32_t slot0, float* q_out, void* stream);

/* ---- 1-bit projections on either side of attention (decode, M = 1) -------------------------
 * Weights as the engine uploads them (src/engine.ts:814-830): row n, weight k is bit k % 32 of
 * sign[n][k / 32] (u32; set = +1, clear = -1) times scales[n][k / 128] (f32); K a multiple of
 * 128; x, sign and scales 16-byte aligned. */

/* fusedMM, matmul_split_sg.wgsl (src/engine.ts:1344-1360, e.g. the qkv and gate/up weights):
 * the N0 + N1 + N2 rows of W x, rows [0, N0) to out0, [N0, N0+N1) to out1, the rest to out2. */
int32_t bg_gemv_split(const float* x, int32_t K, const uint32_t* sign, const float* scales,
                      int32_t N0, int32_t N1, int32_t N2, float* out0, float* out1, float* out2,
                      void* stream);

/* residMM, matmul_resid_mr_sg.wgsl (src/engine.ts:1364-1380, o_proj at 1547 and down_proj):
 * y = W x + resid over N rows. */
int32_t bg_gemv_resid(const float* x, int32_t K, const uint32_t* sign, const float* scales,
                      int32_t N, const float* resid, float* y, void* stream);

/* The decode qkv projection fused with the attention prologue, replacing src/engine.ts:1526-1540
 * (matmul_split_sg into q, k, v; appendKV(V); rmsnorm_rope_sg(Q); ROPE_K / rmsnorm_rope_sg_kv8
 * writing K into the cache): one token, x = the normed hidden state [K]. The weight's rows are
 * the H query heads, then the cache's kv_heads key heads, then its value heads, head_dim rows
 * each (the fused qkv weight of src/engine.ts:850). Q heads are RMSNormed with q_gamma and roped
 * at `pos` into q_out [H, head_dim]; K heads normed with k_gamma, roped at `pos` (unroped in a
 * sink-mode cache) and stored at logical slot `slot`; V heads stored at `slot`. Tables as in
 * bg_qkv_prologue (16-byte aligned). H + 2 * kv_heads <= 1024. The arithmetic of the norm and
 * the rotation is bg_qkv_prologue's: the result equals bg_gemv_split followed by
 * bg_qkv_prologue bit for bit. */
int32_t bg_qkv_proj_prologue(bg_kv_cache* cache, int32_t layer, const float* x, int32_t K,
                             const uint32_t* sign, const float* scales, int32_t H,
                             const float* q_gamma, const float* k_gamma, float eps,
                             const float* cos_tab, const float* sin_tab, int32_t rope_positions,
                             int32_t rot_dim, int32_t pos, int32_t slot, float* q_out, void* stream);

/* ---- attention ---------------------------------------------------------------------------
 * runN(ATT, [S,H,KV,D,posBase,Ltot], attIns(qr, li), att, S*H), src/engine.ts:1543,1579-1580
 * (attention_{sg,wg}{,_kv16,_kv8}{,_roll}.wgsl) and the hybrid
 * attention_online_cache{,_kv8} + gate_sigmoid, src/engine.ts:1486-1491.
 * q: [S, H, head_dim] f32 (already normed/roped); query s sits at logical slot pos_base + s and
 * attends every resident slot <= pos_base + s. scale: the softmax scale (the dense kernels use
 * 1/sqrt(head_dim), attention_sg.wgsl:24; the hybrid passes 1/sqrt(head_dim) as a param).
 * gate (nullable): [S, H, gate_stride], out = attn / (1 + exp(-gate)) (gate_sigmoid.wgsl:13).
 * out: [S, H, head_dim] f32. Rows per kv head (S x H / KV) that fit one 16-row set run the
 * split-K decode kernel (and so does sink mode up to 48 rows at head_dim 128 and 20 at 256, and
 * q8 at head_dim 128 up to 24);
 * more run the MFMA prefill kernel, whose grid is split along the key range (a second kernel
 * merging the parts) when it holds far fewer query blocks than the GPU has CUs; f32 storage runs
 * an exact-f32 kernel. */
int32_t bg_attention(bg_kv_cache* cache, int32_t layer, const float* q, int32_t S, int32_t H,
                     int32_t pos_base, float scale, const float* gate, int32_t gate_stride,
                     float* out, void* stream);

/* Allocation-free variant of bg_attention. No counterpart in the reference (WebGPU dispatches
 * never allocate per call); it is for callers that cannot call hipMalloc: code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation. Same arguments and results as
 * bg_attention, but it allocates nothing: the split partials of the decode kernel and of a
 * split-K prefill live in a file-scope device array of 8 MiB per GPU (plus 256 KiB for a split
 * prefill's (m, l) values; held until the process ends) instead of the cache's workspace (the
 * prefill splits only as far as 8 MiB of partials, for either entry point); a q8 prefill stages its tiles in-kernel instead of through the f16 copy
 * (the same values: identical output); an f32 cache runs the exact-f32 kernel of one wave per
 * (query, head), which keeps no partials (agrees with bg_attention to f32 rounding). A launch
 * whose partials would exceed the array is rejected with BG_E_INVALID before anything runs.
 * The first call on a device sets the array up (a fill kernel, synchronized) and must not be
 * under graph capture (BG_E_STATE). Every call on one GPU shares that GPU's array: calls that
 * overlap on the GPU (different streams, or different host threads) race and corrupt each
 * other's outputs -- order them on one stream. */
int32_t bg_attention_noalloc(bg_kv_cache* cache, int32_t layer, const float* q, int32_t S, int32_t H,
                             int32_t pos_base, float scale, const float* gate, int32_t gate_stride,
                             float* out, void* stream);

/* Pre-size the split-K workspace for up to S query rows of H heads (otherwise sized on first
 * use), and for a q8 cache whose prefill of S rows runs on an f16 copy of the attended slots,
 * allocate that copy; for a prefill of S rows that can split along the key range, its partials
 * and (m, l) buffer. Call before capturing bg_attention into a HIP graph (a launch under capture
 * cannot allocate). A later call that needs a larger workspace allocates a new one and keeps the
 * old one until bg_kv_destroy, so launches captured before stay valid. */
int32_t bg_attention_reserve(bg_kv_cache* cache, int32_t S, int32_t H);

/* ---- sink-mode eviction (overflow 'sinks') ------------------------------------------------
 * evict / evictFor, src/engine.ts:1187-1214. The cache is a ring behind the sinks: eviction
 * advances the ring head by the reference's batch, so the resident set and its slot order match
 * the reference's memmove compaction without moving any bytes. */
int32_t bg_kv_evict(bg_kv_cache* cache, int32_t fill, int32_t need, int32_t* new_fill);
int32_t bg_kv_evict_for(bg_kv_cache* cache, int32_t fill, int32_t n, int32_t* new_fill);

/* Ring origin and the number of rows evicted so far (absolute position of logical slot
 * L >= sinks is L + evicted). */
int32_t bg_kv_ring_state(const bg_kv_cache* cache, int32_t* head, int64_t* evicted);

/* Put the sink-mode ring into its compacted state: origin 0, `evicted` rows evicted before
 * logical slot `sinks` (0 for a new conversation). The reference's cache is always compacted
 * (evict() moves the kept rows to slot `sinks`, src/engine.ts:1206-1209), so a v2 snapshot
 * restore (restoreCache, src/engine.ts:2807-2872) writes logical slots 0..cacheLen-1 into this
 * state, and a fresh conversation (cacheLen = 0) starts from it. Contents are not touched. */
int32_t bg_kv_ring_reset(bg_kv_cache* cache, int64_t evicted);

/* ---- snapshot wire format -----------------------------------------------------------------
 * Per-region export/import in the reference snapshot layout (src/engine.ts:2724-2734,
 * 2757-2771, 2847-2860): region BG_K / BG_V is [count, KV, head_dim] elements of the storage
 * type (f32, f16, or int8 codes = the little-endian bytes of the reference's packed u32 words),
 * BG_KSCALE / BG_VSCALE is [count, KV, head_dim/32] f32 (q8 only). Positions are logical
 * slots base .. base+count-1. host: host pointer. Synchronous. */
int32_t bg_kv_region_bytes(const bg_kv_cache* cache, int32_t region, int32_t count, size_t* bytes);
int32_t bg_kv_export_rows(bg_kv_cache* cache, int32_t layer, int32_t region, int32_t base,
                          int32_t count, void* host, void* stream);
int32_t bg_kv_import_rows(bg_kv_cache* cache, int32_t layer, int32_t region, int32_t base,
                          int32_t count, const void* host, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BITGPU_ATTN_H */
