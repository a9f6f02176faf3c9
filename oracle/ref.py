"""numpy restatement of the reference attention path -- TEST INFRASTRUCTURE ONLY.

Not part of the product: only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it, as the checker or the timed CPU baseline.

Reference: stfurkan/bitgpu v0.19.1 (citations relative to its repository root).

dtype policy (mirrors the reference under numpy >= 2 / NEP 50): rmsnorm, rope and the q8/f16
quantizers run in float32; attention scores are promoted to float64 by the ``/ np.sqrt(D)``
(a numpy float64 scalar), so softmax and P.V run in float64 and the output is stored as float32
(tools/reference.py:169-175, tools/qwen35_numpy.py:105-113).

Pinning (what fixes each function independently of its own formula; tests/test_oracle.py):

* ``rope_tables`` -- Python ``math.cos/sin`` of the f64 angle, position-0 identity,
  frequency closed form, the reference's own rope_partial case tables.
* ``rmsnorm`` / ``rmsnorm_gemma`` -- constant-row closed form, float64 recomputation,
  scale invariance.
* ``rope_apply`` -- the rotation direction by the unit-vector closed form (e_j -> (cos, +sin),
  e_{j+h} -> (-sin, cos)) and by Python complex multiplication, position 0 is the identity,
  pair norms are preserved, relative-position property, passthrough of dims >= rot.
* ``attention`` -- explicit float64 loop with ``math.exp`` on tiny shapes, rows of P sum to 1,
  uniform V, one dominant key, single key, GQA grouping by explicit per-head loop.
* ``sigmoid`` / ``gated_attention`` -- sigma(0) = 1/2, sigma(x) + sigma(-x) = 1, Python
  ``1/(1+math.exp(-x))``, saturation; the gated composite against an f64 ``math.exp`` loop.
* ``q8_pack`` / ``q8_dequant`` -- zero block, block maximum -> +-127, negative zero, exact
  tie (WGSL ``floor(0.5 + 127 e)``, not round-to-even), exhaustive small grid against exact
  rational arithmetic, and the independent C restatement ``oracle/pack_ref.c``.
* ``f16_pack`` -- Python ``struct.pack('e')`` (IEEE round-to-nearest-even) on every tested value.
* ``evict`` / ``evict_for`` / ``simulate_sink_schedule`` -- a literal row-by-row simulation of
  the reference's scratch-buffer memmove (src/engine.ts:1194-1210) on token ids.
* ``unpack_signs`` / ``gemv_1bit`` -- one set bit at a time (the bit order), all-set / all-clear
  rows (closed forms +-sum(x) * scale), and an explicit per-element loop that restates the WGSL
  kernel's vec4 groups literally on small shapes.
"""
from __future__ import annotations

import math

import numpy as np

f32 = np.float32


# --------------------------------------------------------------------------------------------
# RoPE tables (src/engine.ts:117-147 synthRope; tools/reference.py:128-145;
# tools/qwen35_numpy.py:77-81 for a partial rotary dim)
# --------------------------------------------------------------------------------------------
def rope_tables(theta: float, rot_dim: int, positions: int, yarn: dict | None = None):
    """f32 cos/sin tables ``[positions, rot_dim/2]``: f64 angles ``p * inv[j]``, one rounding.

    ``yarn`` = {"factor", "original_max_position_embeddings"} follows src/engine.ts:124-141.
    """
    half = rot_dim // 2
    j = np.arange(half, dtype=np.float64)
    factor = float(yarn["factor"]) if yarn else 1.0
    pf = theta ** ((2.0 * j) / rot_dim)
    if factor == 1.0:
        inv = 1.0 / pf
        mscale = 1.0
    else:
        orig = yarn["original_max_position_embeddings"]
        lo = max(0, math.floor(rot_dim * math.log(orig / (32 * 2 * math.pi)) / (2 * math.log(theta))))
        hi = min(half - 1, math.ceil(rot_dim * math.log(orig / (2 * math.pi)) / (2 * math.log(theta))))
        ramp = np.clip((j - lo) / (hi - lo), 0, 1)
        inv = (1.0 / (factor * pf)) * ramp + (1.0 / pf) * (1 - ramp)
        mscale = float(np.float32(0.1 * math.log(factor) + 1))
    ang = np.outer(np.arange(positions, dtype=np.float64), inv)
    return (np.cos(ang) * mscale).astype(f32), (np.sin(ang) * mscale).astype(f32)


# --------------------------------------------------------------------------------------------
# RMSNorm
# --------------------------------------------------------------------------------------------
def rmsnorm(x: np.ndarray, g: np.ndarray, eps: float) -> np.ndarray:
    """Dense Qwen3 per-head RMSNorm, tools/reference.py:106-107 (weight used as-is)."""
    x = np.asarray(x, f32)
    return ((x / np.sqrt(np.mean(x.astype(f32) ** 2, -1, keepdims=True) + eps)) * np.asarray(g, f32)).astype(f32)


def rmsnorm_gemma(x: np.ndarray, g: np.ndarray, eps: float) -> np.ndarray:
    """Qwen3.5 RMSNorm with zero-centred weight, tools/qwen35_numpy.py:71-74 (scale 1 + g).

    The engine bakes ``1 + g`` into the weight at load (src/engine.ts:1403-1404), so the
    kernels receive ``gamma = 1 + g`` and compute the plain form.
    """
    x = np.asarray(x, f32)
    return (x * (1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)) * (1.0 + np.asarray(g, f32))).astype(f32)


# --------------------------------------------------------------------------------------------
# RoPE apply (tools/reference.py:146-152 full; tools/qwen35_numpy.py:84-89 partial)
# --------------------------------------------------------------------------------------------
def rope_apply(x: np.ndarray, cos_half: np.ndarray, sin_half: np.ndarray, positions, rot: int | None = None):
    """Rotate_half RoPE on the first ``rot`` dims of ``x[S, heads, D]`` at ``positions[S]``.

    ``cos_half/sin_half`` are ``[P, rot/2]`` tables; the full vector is concat(half, half)
    (src/engine.ts:997-1003). Dims >= rot pass through.
    """
    x = np.asarray(x, f32)
    D = x.shape[-1]
    rot = D if rot is None else rot
    positions = np.asarray(positions, np.int64)
    c = np.concatenate([cos_half[positions], cos_half[positions]], -1).astype(f32)  # [S, rot]
    s = np.concatenate([sin_half[positions], sin_half[positions]], -1).astype(f32)
    xr, xp = x[..., :rot], x[..., rot:]
    half = rot // 2
    rotated = np.concatenate([-xr[..., half:], xr[..., :half]], -1)
    y = xr * c[:, None, :] + rotated * s[:, None, :]
    return np.concatenate([y, xp], -1).astype(f32)


# --------------------------------------------------------------------------------------------
# Causal GQA attention over a cache (tools/reference.py:158-175; tools/qwen35_numpy.py:102-115)
# --------------------------------------------------------------------------------------------
def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, pos_base: int, scale=None,
              valid: np.ndarray | None = None) -> np.ndarray:
    """``out[s, h] = softmax_j(q[s,h].k[j,kvh] * scale + mask) . v[j,kvh]``.

    q: f32[S, H, D]; k, v: f32[L, KV, D] (cache rows in attention order); query s sits at
    position ``pos_base + s`` and attends keys ``j <= pos_base + s`` (the reference's causal
    triangle, generalised to a cache exactly as attention_sg.wgsl:31 loops ``j <= pos``).
    ``valid`` (bool[L]) drops non-resident rows (unused ring slots). ``scale`` None means the
    dense ``/ np.sqrt(D)`` of tools/reference.py:171; a number means the hybrid
    ``* scale`` with scale = 1/np.sqrt(HD) of tools/qwen35_numpy.py:105,109.
    kvh = h // (H / KV) via np.repeat (tools/reference.py:167-168).
    """
    q = np.asarray(q, f32)
    S, H, D = q.shape
    L, KV, _ = k.shape
    rep = H // KV
    kk = np.repeat(np.asarray(k, f32), rep, axis=1)
    vv = np.repeat(np.asarray(v, f32), rep, axis=1)
    j = np.arange(L)
    qpos = pos_base + np.arange(S)
    mask = np.where(j[None, :] > qpos[:, None], f32(-1e30), f32(0)).astype(f32)
    if valid is not None:
        mask = np.where(np.asarray(valid, bool)[None, :], mask, f32(-1e30)).astype(f32)
    out = np.empty((S, H, D), f32)
    for hh in range(H):
        if scale is None:
            sc = (q[:, hh] @ kk[:, hh].T) / np.sqrt(D) + mask
        else:
            sc = (q[:, hh] @ kk[:, hh].T) * np.float64(scale) + mask
        sc -= sc.max(-1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(-1, keepdims=True)
        out[:, hh] = p @ vv[:, hh]
    return out


def sigmoid(x: np.ndarray) -> np.ndarray:
    """tools/qwen35_numpy.py:58-59 (float32)."""
    return (1.0 / (1.0 + np.exp(-np.asarray(x, f32)))).astype(f32)


def gated_attention(q, k, v, gate, pos_base: int) -> np.ndarray:
    """Qwen3.5 gated full attention core, tools/qwen35_numpy.py:102-114 (no projections):
    ``o * sigmoid(gate)`` with scale ``1/np.sqrt(HD)``. gate: f32[S, H, D]."""
    D = q.shape[-1]
    o = attention(q, k, v, pos_base, scale=1.0 / np.sqrt(D))
    return (o * sigmoid(gate)).astype(f32)


# --------------------------------------------------------------------------------------------
# KV storage quantizers
# --------------------------------------------------------------------------------------------
Q8_BLOCK = 32
Q8_TINY = f32(1e-30)


def q8_pack(x: np.ndarray, block: int = Q8_BLOCK):
    """q8 cache append, shaders/copy_kv8.wgsl:24-40 with WGSL pack4x8snorm.

    Per ``block`` values: s = max(max|v|, 1e-30) (copy_kv8.wgsl:31-33); code =
    floor(0.5 + 127 * clamp(v / s, -1, 1)) (the WGSL pack4x8snorm definition), every
    operation one IEEE f32 rounding and no fused multiply-add. Returns (int8[..., D],
    f32[..., D/block]).
    """
    x = np.asarray(x, f32)
    shp = x.shape
    D = shp[-1]
    xb = x.reshape(-1, D // block, block)
    m = np.abs(xb).max(-1)
    s = np.maximum(m, Q8_TINY).astype(f32)
    e = np.clip(xb / s[..., None], f32(-1), f32(1)).astype(f32)
    t = (f32(127) * e).astype(f32)
    t = (t + f32(0.5)).astype(f32)
    c = np.floor(t).astype(np.int8)
    return c.reshape(shp), s.reshape(shp[:-1] + (D // block,))


def q8_dequant(codes: np.ndarray, scales: np.ndarray, block: int = Q8_BLOCK) -> np.ndarray:
    """``max(c / 127, -1) * s`` -- unpack4x8snorm then the block-scale multiply,
    shaders/attention_sg_kv8.wgsl:40,51 (two f32 roundings)."""
    c = np.asarray(codes, np.int8)
    shp = c.shape
    D = shp[-1]
    u = np.maximum((c.astype(f32) / f32(127)).astype(f32), f32(-1)).reshape(-1, D // block, block)
    s = np.asarray(scales, f32).reshape(-1, D // block)
    return (u * s[..., None]).astype(f32).reshape(shp)


def f16_pack(x: np.ndarray) -> np.ndarray:
    """f16 cache append, shaders/copy_kv16.wgsl:13 (IEEE round-to-nearest-even; values beyond
    the f16 range become +-inf)."""
    with np.errstate(over="ignore"):
        return np.asarray(x, f32).astype(np.float16)


def kv_roundtrip(x: np.ndarray, dtype: str) -> np.ndarray:
    """What the attention kernels read back for a value written in storage mode ``dtype``."""
    if dtype == "f32":
        return np.asarray(x, f32)
    if dtype == "f16":
        return f16_pack(x).astype(f32)
    if dtype == "q8":
        c, s = q8_pack(x)
        return q8_dequant(c, s)
    raise ValueError(dtype)


# --------------------------------------------------------------------------------------------
# Fused norm + rope (shaders/rmsnorm_rope_sg.wgsl:22-33, used for Q and for the K cache write)
# --------------------------------------------------------------------------------------------
def norm_rope(x: np.ndarray, gamma: np.ndarray, eps: float, cos_half, sin_half, positions,
              rot: int | None = None, rope: bool = True) -> np.ndarray:
    """RMSNorm per head row then rotate_half RoPE at ``positions`` (x: f32[S, R, D]).

    ``rope=False`` is the sink-mode K write, where the engine binds cos=1 / sin=0 so the
    cache stores the un-roped norm (src/engine.ts:1530-1533, 1574-1575).
    """
    y = rmsnorm(x, gamma, eps)
    if not rope:
        return y
    return rope_apply(y, cos_half, sin_half, positions, rot)


# --------------------------------------------------------------------------------------------
# Sink-mode eviction (src/engine.ts:1187-1214) and the decode schedule that drives it
# --------------------------------------------------------------------------------------------
def evict(fill: int, need: int, sinks: int, max_seq: int):
    """Returns (new_fill, batch, keep); rows [sinks+batch, sinks+batch+keep) move to
    [sinks, sinks+keep) (src/engine.ts:1188-1212)."""
    recent = fill - sinks
    batch = min(recent, max(need, -(-(max_seq - sinks) // 4)))
    keep = recent - batch
    if keep <= 0:
        return sinks, batch, keep
    return sinks + keep, batch, keep


def evict_for(fill: int, n: int, sinks: int, max_seq: int, roll: bool = True):
    """src/engine.ts:1214: evict only when the next ``n`` rows do not fit."""
    if roll and fill + n > max_seq:
        return evict(fill, fill + n - max_seq, sinks, max_seq)
    return fill, 0, 0


def simulate_sink_schedule(prompt_len: int, target_abs: int, sinks: int, max_seq: int,
                           sync_n: int = 4, final_rows: int = 1):
    """Literal simulation of a fresh greedy ``generate`` in sink mode.

    Follows src/engine.ts:2556-2570 (entry), 1705-1735 (prefill at slots 0..P-1) and
    1783-1799 (decode: ``slot = evictFor(slot, batch)`` with batch <= syncN, then one row per
    fed token at ``slot + j``). Decoding continues until the token at absolute position
    ``target_abs`` is about to be fed; then ``evictFor(slot, final_rows)`` is applied (1 for a
    decode step, the verify width for a speculative step) and the state is returned.

    The cache is an explicit list of absolute token positions per slot and eviction is the
    reference's literal row copy through a scratch buffer (src/engine.ts:1206-1209).
    Returns (slots, fill, evictions): slots[i] = absolute position held by slot i.
    """
    if sinks + prompt_len + 1 > max_seq:
        raise ValueError("prompt does not fit the rolling window")
    cache = list(range(prompt_len))       # runPrefill writes tokens 0..P-1 at slots 0..P-1
    slot = prompt_len
    fed = prompt_len                      # absolute position of the next token to feed
    events = []

    def do_evict(fill, n):
        new_fill, batch, keep = evict_for(fill, n, sinks, max_seq)
        if new_fill != fill or batch:
            scratch = cache[sinks + batch: sinks + batch + max(keep, 0)]
            for i, a in enumerate(scratch):
                cache[sinks + i] = a
            del cache[new_fill:]
            events.append((fill, batch, keep))
        return new_fill

    total = 1                             # the prefill produced the first token already
    while fed < target_abs:
        batch = min(sync_n, target_abs - fed)
        slot = do_evict(slot, batch)
        for j in range(batch):
            if slot + j < len(cache):
                cache[slot + j] = fed
            else:
                cache.append(fed)
            fed += 1
        slot += batch
        total += batch
    slot = do_evict(slot, final_rows)
    return cache[:slot], slot, events


# --------------------------------------------------------------------------------------------
# 1-bit projections (the GEMVs on either side of attention in decode)
# --------------------------------------------------------------------------------------------
def unpack_signs(sign: np.ndarray, K: int) -> np.ndarray:
    """Sign bits ``u32[N, K/32]`` -> ``float64[N, K]`` of +-1: weight k of row n is bit k % 32 of
    word k // 32, set = +1, clear = -1 (shaders/matmul_split_sg.wgsl:29-32)."""
    s = np.asarray(sign, np.uint32)
    N = s.shape[0]
    bits = (s[:, :, None] >> np.arange(32, dtype=np.uint32)[None, None, :]) & np.uint32(1)
    return np.where(bits.reshape(N, K) != 0, 1.0, -1.0)


def gemv_1bit(x: np.ndarray, sign: np.ndarray, scales: np.ndarray, resid: np.ndarray | None = None) -> np.ndarray:
    """``y[n] = sum_k x[k] * (+-1)[n, k] * scales[n, k // 128] (+ resid[n])`` in float64, returned
    as float32: matmul_split_sg.wgsl:24-35 (qkv / gate-up, outputs split by range) and
    matmul_resid_mr_sg.wgsl:24-46 (o_proj / down_proj with the residual added)."""
    x = np.asarray(x, np.float64)
    K = x.shape[-1]
    w = unpack_signs(sign, K) * np.repeat(np.asarray(scales, np.float64), 128, axis=1)
    y = w @ x
    if resid is not None:
        y = y + np.asarray(resid, np.float64)
    return y.astype(f32)


def gemv_abs_bound(x: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """``sum_k |x[k]| * scales[n, k // 128]``: the magnitude an f32 sum of the products of row n
    is measured against (its rounding error is a small multiple of this times 2^-24)."""
    xa = np.abs(np.asarray(x, np.float64))
    K = xa.shape[-1]
    return np.abs(np.asarray(scales, np.float64)) @ xa.reshape(K // 128, 128).sum(-1)
