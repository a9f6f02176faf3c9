"""Host-side mirror of the reference engine's per-layer attention dispatch, over the C ABI.

The reference (stfurkan/bitgpu v0.19.1, src/engine.ts) records, per layer:

* ``appendKV(pass, src, which, li, rows, dstRow0)``            -> :meth:`KvCache.append_kv`
* ``attIns(qr, li)`` + ``runN(ATT, [S,H,KV,D,posBase,Ltot])``  -> :func:`attention`
* the fused decode branch of ``layer()`` (1519-1547) and its prefill branch (1562-1581)
                                                               -> :func:`layer_attention`
* the full-attention branch of ``hybridLayer()`` (1465-1493)   -> :func:`hybrid_full_attention`
* ``ensureKvCapacity`` / ``evict`` / ``evictFor`` / ``saveCache`` / ``restoreCache``
                                                               -> :class:`KvCache` methods
  (restoreCache's checks, 2808-2845                           -> :func:`validate_snapshot`)
* ``synthRope`` (117-147)                                      -> :func:`rope_tables`
* ``fusedMM`` / ``residMM`` at S = 1 (1344-1380)                -> :func:`fused_mm` / :func:`resid_mm`
* the fused decode block's qkv projection + prologue (1526-1540) -> :func:`qkv_proj_prologue`,
  and the block through o_proj + residual (1519-1547)          -> :func:`decode_attention_block`

Device memory is owned by torch tensors (``cuda`` device, float32, contiguous); only raw
pointers cross the boundary. Every call is enqueued on torch's current stream. There is no CPU
fallback: without the built HIP library these functions raise.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np

from ._lib import (BG_E_INVALID, BG_E_STATE, BG_K, BG_KSCALE, BG_ROPE_ABSOLUTE, BG_ROPE_SLOT, BG_V, BG_VSCALE,
                   KV_DTYPES, BitgpuError, check, lib)

__all__ = ["KvCache", "attention", "qkv_prologue", "layer_attention", "hybrid_full_attention",
           "rope_tables", "evict_plan", "ring_map", "validate_snapshot", "OneBitWeight", "fused_mm", "resid_mm",
           "qkv_proj_prologue", "decode_attention_block"]


def _stream():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("bitgpu_amd: expected a device (cuda) tensor")
    if not t.is_contiguous():
        raise ValueError("bitgpu_amd: expected a contiguous tensor")
    return C.c_void_p(t.data_ptr())


def _f32(t, name):
    import torch
    if t.dtype != torch.float32:
        raise TypeError(f"bitgpu_amd: {name} must be float32, got {t.dtype}")
    return t


def rope_tables(theta: float, rot_dim: int, positions: int, yarn: dict | None = None):
    """synthRope (src/engine.ts:117-147): f32 ``[positions, rot_dim/2]`` cos/sin host arrays."""
    half = rot_dim // 2
    cos = np.empty((positions, half), np.float32)
    sin = np.empty((positions, half), np.float32)
    factor = float(yarn["factor"]) if yarn else 1.0
    orig = int(yarn["original_max_position_embeddings"]) if yarn else 0
    check(lib().bg_rope_tables(float(theta), int(rot_dim), int(positions), factor, orig,
                               cos.ctypes.data_as(C.c_void_p), sin.ctypes.data_as(C.c_void_p)))
    return cos, sin


def evict_plan(fill: int, need: int, sinks: int, max_seq_len: int):
    """evict() arithmetic of src/engine.ts:1188-1212 -> (new_fill, batch, keep)."""
    nf, b, k = C.c_int32(), C.c_int32(), C.c_int32()
    check(lib().bg_evict_plan(fill, need, sinks, max_seq_len, C.byref(nf), C.byref(b), C.byref(k)))
    return nf.value, b.value, k.value


def ring_map(sinks: int, max_seq_len: int, head: int, logical: int) -> int:
    """Physical slot of a logical slot in the sink-mode ring (bg_ring_map)."""
    out = C.c_int32()
    check(lib().bg_ring_map(sinks, max_seq_len, head, logical, C.byref(out)))
    return out.value


class KvCache:
    """The engine's per-layer KV cache (Kc/Vc/Ksc/Vsc, src/engine.ts:1044-1079).

    ``kv_cache`` is EngineOptions.kvCache ('f32' | 'f16' | 'q8'), ``overflow`` 'error' | 'sinks'
    and ``sink_tokens`` EngineOptions.sinkTokens (src/types.ts:138-177). ``rope_positions``
    selects the sink-mode key rotation: 'slot' (the reference's cache-relative positions) or
    'absolute' (true token positions). ``q8_block`` is 32 (the reference's per-32 scales) or
    head_dim (one scale per row, stored in every 32-value slot).
    """

    def __init__(self, n_layers: int, kv_heads: int, head_dim: int, kv_cache: str = "f32",
                 max_seq_len: int = 2048, capacity: int | None = None, overflow: str = "error",
                 sink_tokens: int = 4, rope_positions: str = "slot", q8_block: int = 32):
        if kv_cache not in KV_DTYPES:
            raise ValueError(f"bitgpu_amd: kvCache must be one of {sorted(KV_DTYPES)}")
        if overflow not in ("error", "sinks"):
            raise ValueError("bitgpu_amd: overflow must be 'error' or 'sinks'")
        self.n_layers, self.kv_heads, self.head_dim = n_layers, kv_heads, head_dim
        self.kv_cache, self.max_seq_len = kv_cache, max_seq_len
        self.roll = overflow == "sinks"
        self.sinks = max(1, int(sink_tokens)) if self.roll else 0
        self._h = C.c_void_p()
        mode = BG_ROPE_ABSOLUTE if rope_positions == "absolute" else BG_ROPE_SLOT
        check(lib().bg_kv_create(n_layers, kv_heads, head_dim, KV_DTYPES[kv_cache],
                                 0 if capacity is None else int(capacity), max_seq_len,
                                 1 if self.roll else 0, self.sinks, mode, C.byref(self._h)))
        self._rope_keepalive = None
        self.q8_block = q8_block
        if kv_cache == "q8" and q8_block != 32:
            check(lib().bg_kv_set_q8_block(self._h, int(q8_block)))

    # -- lifecycle ---------------------------------------------------------------------------
    def close(self):
        if self._h:
            lib().bg_kv_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    @property
    def capacity(self) -> int:
        c = C.c_int32()
        check(lib().bg_kv_capacity(self._h, C.byref(c)))
        return c.value

    def ensure_capacity(self, needed: int):
        """ensureKvCapacity (src/engine.ts:1120-1178); raises GpuOutOfMemoryError on failure
        with the old buffers kept."""
        check(lib().bg_kv_grow(self._h, int(needed), _stream()))

    def set_rope(self, cos_dev, sin_dev):
        """Bind the sink-mode rotation tables (rollCosT/rollSinT, src/engine.ts:1097-1104)."""
        _f32(cos_dev, "cos")
        _f32(sin_dev, "sin")
        check(lib().bg_kv_set_rope(self._h, _ptr(cos_dev), _ptr(sin_dev), cos_dev.shape[0], 2 * cos_dev.shape[1]))
        self._rope_keepalive = (cos_dev, sin_dev)

    # -- writes ------------------------------------------------------------------------------
    def append_kv(self, src, which: int, li: int, rows: int, dst_row0: int):
        """appendKV (src/engine.ts:1385-1393): ``rows`` f32 rows at reference row ``dst_row0``."""
        _f32(src, "src")
        if src.numel() < rows * self.head_dim:
            raise ValueError("bitgpu_amd: append_kv source is smaller than rows * head_dim")
        check(lib().bg_kv_write(self._h, li, which, _ptr(src), int(rows), int(dst_row0), _stream()))

    # -- sink-mode eviction ------------------------------------------------------------------
    def evict(self, fill: int, need: int) -> int:
        nf = C.c_int32()
        check(lib().bg_kv_evict(self._h, int(fill), int(need), C.byref(nf)))
        return nf.value

    def evict_for(self, fill: int, n: int) -> int:
        nf = C.c_int32()
        check(lib().bg_kv_evict_for(self._h, int(fill), int(n), C.byref(nf)))
        return nf.value

    def ring_state(self):
        """(ring head, rows evicted so far)."""
        h, e = C.c_int32(), C.c_int64()
        check(lib().bg_kv_ring_state(self._h, C.byref(h), C.byref(e)))
        return h.value, e.value

    # -- snapshot byte format ----------------------------------------------------------------
    def region_bytes(self, region: int, count: int) -> int:
        b = C.c_size_t()
        check(lib().bg_kv_region_bytes(self._h, region, count, C.byref(b)))
        return b.value

    def export_rows(self, li: int, region: int, base: int, count: int) -> bytes:
        buf = C.create_string_buffer(max(1, self.region_bytes(region, count)))
        check(lib().bg_kv_export_rows(self._h, li, region, base, count, C.cast(buf, C.c_void_p), _stream()))
        return buf.raw[: self.region_bytes(region, count)]

    def import_rows(self, li: int, region: int, base: int, count: int, data: bytes):
        if len(data) != self.region_bytes(region, count):
            raise ValueError("bitgpu_amd: import size does not match the region")
        buf = C.create_string_buffer(bytes(data), max(1, len(data)))
        check(lib().bg_kv_import_rows(self._h, li, region, base, count, C.cast(buf, C.c_void_p), _stream()))

    def _regions(self):
        return [BG_K, BG_V, BG_KSCALE, BG_VSCALE] if self.kv_cache == "q8" else [BG_K, BG_V]

    def save_snapshot(self, length: int, base: int = 0) -> bytes:
        """KV part of saveCache (src/engine.ts:2736-2805): per layer K, V (then Ksc, Vsc under
        q8) for positions [base, length), in the reference byte layout."""
        count = length - base
        return b"".join(self.export_rows(li, r, base, count) for li in range(self.n_layers) for r in self._regions())

    def ring_reset(self, evicted: int = 0):
        """Compacted ring state (origin 0): a new conversation, or the target of a v2 restore."""
        check(lib().bg_kv_ring_reset(self._h, int(evicted)))

    def model_stamp(self, hidden: int = 0, vocab: int = 0) -> dict:
        """The KvSnapshot.model stamp (src/types.ts:377-378); hidden/vocab are the engine's."""
        return {"layers": self.n_layers, "kvHeads": self.kv_heads, "headDim": self.head_dim, "hidden": hidden,
                "vocab": vocab}

    def save_cache(self, ids, cache_len: int | None = None, model: dict | None = None, base: int = 0):
        """saveCache (src/engine.ts:2736-2805) over this cache: a KvSnapshot dict (src/types.ts:369-390).

        ``ids`` is the conversation's fullHistory; the stored length is ``cache_len`` in sink
        mode (slots, not history) and ``len(ids) - 1`` otherwise. Returns None for no history.
        A sink-mode snapshot also records the rows evicted so far (``roll.evicted``, an extra
        field the reference does not read) so an absolute-position cache restores exactly."""
        if not ids:
            return None
        if self.roll:
            if cache_len is None:
                raise ValueError("saveCache: a sink-mode cache needs cache_len (its filled slots)")
            length = int(cache_len)
        else:
            length = len(ids) - 1
        base = max(0, min(int(base), length))
        if base > 0 and self.roll:
            raise BitgpuError(BG_E_STATE, "saveCache: delta snapshots ({ from }) are not supported under overflow 'sinks'")
        snap = {"version": 2 if self.roll else 1, "kvCache": self.kv_cache,
                "model": dict(model) if model else self.model_stamp(), "ids": list(ids),
                "data": self.save_snapshot(length, base)}
        if base > 0:
            snap["base"] = base
        if self.roll:
            snap["roll"] = {"sinkTokens": self.sinks, "cacheLen": length, "evicted": self.ring_state()[1]}
        return snap

    def restore_cache(self, snap: dict, model: dict | None = None, cache_len: int = 0, history=(),
                      hybrid: bool = False) -> int:
        """restoreCache (src/engine.ts:2807-2872): validate ``snap`` against this cache (same
        rejections and messages as the reference), then write its positions. ``cache_len`` and
        ``history`` are the engine's current cacheLen / fullHistory (a delta restore must sit
        exactly on its prefix); ``hybrid`` marks the qwen3_5 hybrid backbone, which takes full
        snapshots only. Returns the restored cacheLen. A v2 snapshot restores into the
        compacted ring (origin 0), the reference's layout after any eviction.

        As in the reference, nothing is written before every check has passed and the capacity
        has grown (ensureKvCapacity, 2846): a failed growth leaves the ring state and contents
        as they were."""
        length, base, count = validate_snapshot(
            snap, roll=self.roll, sinks=self.sinks, kv_cache=self.kv_cache,
            model=dict(model) if model else self.model_stamp(), max_seq_len=self.max_seq_len,
            data_bytes=self.n_layers * sum(self.region_bytes(r, 1) for r in self._regions()),
            cache_len=cache_len, history=history, hybrid=hybrid)
        self.ensure_capacity(length)
        if self.roll:
            self.ring_reset(int(snap["roll"].get("evicted", 0)))
        self.restore_snapshot(snap["data"], length, base)
        return length

    def restore_snapshot(self, data: bytes, length: int, base: int = 0):
        """KV part of restoreCache (src/engine.ts:2807-2872)."""
        count = length - base
        expect = self.n_layers * sum(self.region_bytes(r, count) for r in self._regions())
        if len(data) != expect:
            raise ValueError(f"restoreCache: snapshot data is {len(data)} bytes, expected {expect}")
        self.ensure_capacity(length)
        off = 0
        for li in range(self.n_layers):
            for r in self._regions():
                n = self.region_bytes(r, count)
                self.import_rows(li, r, base, count, data[off: off + n])
                off += n


def validate_snapshot(snap, *, roll: bool, sinks: int, kv_cache: str, model: dict, max_seq_len: int,
                      data_bytes: int, cache_len: int = 0, history=(), hybrid: bool = False):
    """The checks of restoreCache (src/engine.ts:2808-2845), host-only, in the reference's order
    and wording. ``data_bytes`` is snapshotBytes(1) (per-position bytes over every layer);
    ``hybrid`` is the engine's A.hybrid (the qwen3_5 backbone rejects delta snapshots, 2828).
    Raises BitgpuError; returns (len, base, count)."""
    def bad(msg):
        raise BitgpuError(BG_E_INVALID, msg)
    if not snap or snap.get("version") not in (1, 2):
        bad(f"restoreCache: unsupported snapshot version {snap.get('version') if snap else None}")
    v2 = snap["version"] == 2
    if v2 != bool(roll):
        bad("restoreCache: snapshot was saved under overflow 'sinks' (unroped keys); this engine runs overflow 'error'"
            if v2 else
            "restoreCache: snapshot was saved under overflow 'error' (roped keys); this engine runs overflow 'sinks'")
    rollinfo = snap.get("roll") or {}
    if v2 and rollinfo.get("sinkTokens") != sinks:
        bad(f"restoreCache: snapshot uses {rollinfo.get('sinkTokens')} sink tokens but this engine uses {sinks}")
    if snap.get("kvCache") != kv_cache:
        bad(f"restoreCache: snapshot was saved under kvCache '{snap.get('kvCache')}' but this engine runs "
            f"'{kv_cache}' - snapshots do not convert across modes")
    m = snap.get("model")
    keys = ("layers", "kvHeads", "headDim", "hidden", "vocab")
    if not m or any(m.get(k) != model.get(k) for k in keys):
        bad("restoreCache: snapshot is from a different model (architecture mismatch)")
    ids = snap.get("ids")
    if not isinstance(ids, (list, tuple)) or len(ids) == 0:
        bad("restoreCache: snapshot holds no tokens")
    length = int(rollinfo["cacheLen"]) if v2 else len(ids) - 1
    base = max(0, int(math.floor(snap.get("base") or 0)))
    if base > 0 and hybrid:
        bad("restoreCache: delta snapshots are not supported for the qwen3_5 hybrid backbone")
    count = length - base
    need = length + (0 if v2 else 1)
    if need > max_seq_len:
        bad(f"restoreCache: snapshot needs {need} cache slots but maxSeqLen is {max_seq_len}")
    if len(snap["data"]) != data_bytes * count:
        bad(f"restoreCache: snapshot data is {len(snap['data'])} bytes, expected {data_bytes * count}")
    if base > 0:
        if cache_len != base:
            bad(f"restoreCache: delta snapshot expects the cache at position {base} (prewarm the shared prefix "
                f"first); it is at {cache_len}")
        for i in range(base):
            if i >= len(history) or history[i] != ids[i]:
                bad(f"restoreCache: delta snapshot prefix does not match the current prewarm (token {i})")
    return length, base, count


def attention(cache: KvCache, li: int, qr, S: int, H: int, pos_base: int, scale: float | None = None,
              gate=None, gate_stride: int | None = None, out=None):
    """runN(ATT, [S,H,KV,D,posBase,Ltot], attIns(qr, li), att, S*H) (src/engine.ts:1543,1579-1580);
    with ``gate`` the hybrid's attention_online_cache + gate_sigmoid (1486-1491)."""
    import torch
    D = cache.head_dim
    _f32(qr, "q")
    if qr.numel() != S * H * D:
        raise ValueError("bitgpu_amd: q must hold S*H*head_dim values")
    if out is None:
        out = torch.empty((S, H, D), dtype=torch.float32, device=qr.device)
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))  # attention_sg.wgsl:24
    gs = 0
    if gate is not None:
        _f32(gate, "gate")
        gs = int(gate_stride if gate_stride is not None else D)
    check(lib().bg_attention(cache.handle, li, _ptr(qr), S, H, int(pos_base), float(scale), _ptr(gate), gs,
                             _ptr(out), _stream()))
    return out


def qkv_prologue(cache: KvCache, li: int, q, k, v, S: int, H: int, q_gamma, k_gamma, eps: float,
                 cos_tab, sin_tab, rot_dim: int, pos0: int, slot0: int, q_stride: int | None = None,
                 q_out=None):
    """Fused q/k RMSNorm + RoPE + K/V cache write (see include/bitgpu_attn.h bg_qkv_prologue)."""
    import torch
    D = cache.head_dim
    if q is not None and q_out is None:
        q_out = torch.empty((S, H, D), dtype=torch.float32, device=q.device)
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (q_gamma, "q_gamma"), (k_gamma, "k_gamma")):
        if t is not None:
            _f32(t, nm)
    check(lib().bg_qkv_prologue(cache.handle, li, _ptr(q), int(q_stride or D), _ptr(k), _ptr(v), S, H,
                                _ptr(q_gamma), _ptr(k_gamma), float(eps), _ptr(cos_tab), _ptr(sin_tab),
                                int(cos_tab.shape[0]) if cos_tab is not None else 0, int(rot_dim), int(pos0),
                                int(slot0), _ptr(q_out), _stream()))
    return q_out


def layer_attention(cache: KvCache, li: int, q, k, v, S: int, H: int, pos_base: int, q_norm, k_norm,
                    eps: float, cos_tab, sin_tab, slot: int | None = None):
    """The attention block of the dense ``layer()`` (src/engine.ts:1519-1547 decode, 1562-1581
    prefill/verify): q/k norm + rope, K/V append at ``posBase`` (the cache slot), attention.

    q: [S, H, D], k/v: [S, KV, D] projections (f32, device). RoPE uses position ``pos_base + s``
    for the query and the key (the engine's posBase is the slot, src/engine.ts:994-1009,
    1782-1798); in sink mode keys are stored unroped. Returns att [S, H, D].
    """
    slot = pos_base if slot is None else slot
    qr = qkv_prologue(cache, li, q, k, v, S, H, q_norm, k_norm, eps, cos_tab, sin_tab,
                      cache.head_dim, pos_base, slot)
    return attention(cache, li, qr, S, H, slot)


def hybrid_full_attention(cache: KvCache, li: int, qg, k, v, S: int, H: int, pos_base: int, q_norm, k_norm,
                          eps: float, cos_tab, sin_tab, rot_dim: int):
    """Full-attention branch of ``hybridLayer()`` (src/engine.ts:1465-1493) after the
    projections: split_head (query | gate interleave of the doubled q_proj), q/k RMSNorm with
    the baked (1 + weight) scale, partial RoPE, K/V append, attention_online_cache{,_kv8} with
    scale 1/sqrt(head_dim), then gate_sigmoid. qg: [S, H, 2D]; returns gated [S, H, D]."""
    D = cache.head_dim
    qr = qkv_prologue(cache, li, qg, k, v, S, H, q_norm, k_norm, eps, cos_tab, sin_tab, rot_dim, pos_base,
                      pos_base, q_stride=2 * D)
    import torch
    scale = float(np.float32(1.0 / math.sqrt(D)))  # the hybrid's ['f', 1/Math.sqrt(Dh)] param
    out = torch.empty((S, H, D), dtype=torch.float32, device=qg.device)
    # the gate half of each [2D] row starts D floats in; its row stride is 2D
    check(lib().bg_attention(cache.handle, li, _ptr(qr), S, H, int(pos_base), scale,
                             C.c_void_p(qg.data_ptr() + D * 4), 2 * D, _ptr(out), _stream()))
    return out


# --------------------------------------------------------------------------------------------
# 1-bit projections on either side of attention (decode, M = 1)
# --------------------------------------------------------------------------------------------
class OneBitWeight:
    """A 1-bit weight as the engine uploads it (GpuWeight, src/engine.ts:814-830): ``sign`` u32
    [N, K/32] (bit k % 32 of word k // 32 set = +1), ``scales`` f32 [N, K/128], rows split into
    ranges N0 | N1 | N2 for the fused qkv / gate-up weights (src/engine.ts:850-853)."""

    def __init__(self, sign, scales, K: int, N0: int, N1: int = 0, N2: int = 0):
        import torch
        if sign.dtype != torch.int32 or scales.dtype != torch.float32:
            raise TypeError("bitgpu_amd: sign must be int32 (raw u32 words) and scales float32")
        if K % 128 or sign.numel() != (N0 + N1 + N2) * K // 32 or scales.numel() != (N0 + N1 + N2) * K // 128:
            raise ValueError("bitgpu_amd: sign / scales do not match K and the row counts")
        self.sign, self.scales, self.K, self.N0, self.N1, self.N2 = sign, scales, K, N0, N1, N2

    @property
    def N(self) -> int:
        return self.N0 + self.N1 + self.N2


def fused_mm(w: OneBitWeight, x, outs):
    """fusedMM at S = 1 (src/engine.ts:1344-1350, matmul_split_sg.wgsl): rows of W x into up to
    three outputs by range."""
    _f32(x, "x")
    o = list(outs) + [None] * (3 - len(outs))
    check(lib().bg_gemv_split(_ptr(x), w.K, _ptr(w.sign), _ptr(w.scales), w.N0, w.N1, w.N2, _ptr(o[0]), _ptr(o[1]),
                              _ptr(o[2]), _stream()))


def resid_mm(w: OneBitWeight, x, resid, out=None):
    """residMM at S = 1 (src/engine.ts:1364-1369, matmul_resid_mr_sg.wgsl): W x + resid."""
    import torch
    _f32(x, "x")
    _f32(resid, "resid")
    if out is None:
        out = torch.empty(w.N, dtype=torch.float32, device=x.device)
    check(lib().bg_gemv_resid(_ptr(x), w.K, _ptr(w.sign), _ptr(w.scales), w.N, _ptr(resid), _ptr(out), _stream()))
    return out


def qkv_proj_prologue(cache: KvCache, li: int, x, w_qkv: OneBitWeight, H: int, q_norm, k_norm, eps: float, cos_tab,
                      sin_tab, rot_dim: int, pos: int, slot: int, q_out=None):
    """The fused decode branch of ``layer()`` up to the attention (src/engine.ts:1526-1540): the
    qkv projection of the normed hidden state x with Q norm + rope into q_out, K norm + rope into
    the cache and V appended, in one launch. Returns q_out [1, H, D]."""
    import torch
    D = cache.head_dim
    if w_qkv.N0 != H * D or w_qkv.N1 != cache.kv_heads * D or w_qkv.N2 != cache.kv_heads * D:
        raise ValueError("bitgpu_amd: the qkv weight's row ranges must be H*D | KV*D | KV*D")
    _f32(x, "x")
    if q_out is None:
        q_out = torch.empty((1, H, D), dtype=torch.float32, device=x.device)
    check(lib().bg_qkv_proj_prologue(cache.handle, li, _ptr(x), w_qkv.K, _ptr(w_qkv.sign), _ptr(w_qkv.scales), H,
                                     _ptr(q_norm), _ptr(k_norm), float(eps), _ptr(cos_tab), _ptr(sin_tab),
                                     int(cos_tab.shape[0]), int(rot_dim), int(pos), int(slot), _ptr(q_out),
                                     _stream()))
    return q_out


def decode_attention_block(cache: KvCache, li: int, n1, h, w_qkv: OneBitWeight, w_o: OneBitWeight, H: int, q_norm,
                           k_norm, eps: float, cos_tab, sin_tab, pos: int, slot: int | None = None):
    """The fused decode attention block of ``layer()`` (src/engine.ts:1519-1547): qkv projection
    + prologue, attention at the slot, o_proj with the residual h. n1: the input-layernormed
    hidden state [K]; returns h2 [hidden]."""
    slot = pos if slot is None else slot
    qr = qkv_proj_prologue(cache, li, n1, w_qkv, H, q_norm, k_norm, eps, cos_tab, sin_tab, cache.head_dim, pos, slot)
    att = attention(cache, li, qr, 1, H, slot)
    return resid_mm(w_o, att.reshape(-1), h)
