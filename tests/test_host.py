"""CPU tests of the C ABI's host side: the library loads, exports every symbol declared in
include/*.h, and its host-only functions (rope tables, eviction arithmetic, the sink-mode ring
map, argument validation) agree with the oracle. No kernel is launched."""
import ctypes as C
import glob
import os
import re

import numpy as np
import pytest

from bitgpu_amd import _lib
from bitgpu_amd import engine as E
from oracle import ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(bg_\w+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"
    assert {n for n, _, _ in _lib.SIGNATURES} == set(names)


def test_version_and_error_message():
    lib = _lib.lib()
    assert b"gfx950" in lib.bg_version()
    h = C.c_void_p()
    rc = lib.bg_kv_create(1, 8, 96, _lib.BG_KV_F16, 0, 1024, 0, 0, 0, C.byref(h))
    assert rc == _lib.BG_E_UNSUPPORTED and not h
    assert b"head_dim 96" in lib.bg_last_error_message()


@pytest.mark.parametrize("args,code", [
    ((0, 8, 128, 0, 0, 1024, 0, 0, 0), _lib.BG_E_INVALID),          # no layers
    ((1, 8, 128, 7, 0, 1024, 0, 0, 0), _lib.BG_E_INVALID),          # unknown dtype
    ((1, 8, 128, 1, 0, 100, 1, 40, 0), _lib.BG_E_INVALID),          # sinks + 64 > maxSeqLen
    ((1, 8, 128, 1, 0, 1024, 1, 0, 0), _lib.BG_E_INVALID),          # sink mode without sinks
    ((1, 1, 256, 1, 0, 4194305, 0, 0, 0), _lib.BG_E_UNSUPPORTED),   # f16 kv head region >= 2^31 bytes
    ((1, 1, 256, 0, 0, 2097153, 0, 0, 0), _lib.BG_E_UNSUPPORTED),   # f32 kv head region >= 2^31 bytes
    ((1, 1, 128, 2, 0, 2**31 - 1, 0, 0, 0), _lib.BG_E_UNSUPPORTED), # q8 (its f16 prefill copy), no int overflow
])
def test_create_validation(args, code):
    h = C.c_void_p()
    assert _lib.lib().bg_kv_create(*args, C.byref(h)) == code
    assert _lib.lib().bg_last_error_message().startswith(b"bitgpu: ")


def test_python_wrapper_raises_bitgpu_error():
    with pytest.raises(_lib.BitgpuError, match="maxSeqLen >= sinkTokens \\+ 64"):
        E.KvCache(1, 8, 128, "f16", max_seq_len=60, overflow="sinks", sink_tokens=4)


@pytest.mark.parametrize("theta,rot,P,yarn", [(1e6, 128, 600, None), (1e7, 64, 9000, None),
                                              (1e6, 128, 300, {"factor": 4.0, "original_max_position_embeddings": 8192})])
def test_rope_tables_match_oracle(theta, rot, P, yarn):
    c, s = E.rope_tables(theta, rot, P, yarn)
    rc, rs = ref.rope_tables(theta, rot, P, yarn)
    # both round one f64 value to f32; the f64 cos/sin of two libms may differ in the last bit,
    # which can move the f32 rounding by one ulp in rare entries
    dc = np.abs(c.view(np.int32).astype(np.int64) - rc.view(np.int32).astype(np.int64))
    ds = np.abs(s.view(np.int32).astype(np.int64) - rs.view(np.int32).astype(np.int64))
    assert dc.max() <= 1 and ds.max() <= 1
    assert (dc > 0).mean() < 1e-3 and (ds > 0).mean() < 1e-3


def test_evict_plan_matches_oracle_exhaustive():
    for max_seq in (68, 130, 4100):
        for sinks in (1, 4):
            for fill in range(sinks, max_seq + 1, max(1, max_seq // 50)):
                for need in (0, 1, 4, 9, 33, max_seq):
                    assert E.evict_plan(fill, need, sinks, max_seq) == ref.evict(fill, need, sinks, max_seq)


def test_ring_reproduces_reference_compaction():
    """Drive the reference's decode schedule through bg_evict_plan + ring-head advances and
    check that the ring's logical->physical map holds exactly the tokens the reference's
    memmove compaction keeps, slot for slot."""
    sinks, max_seq = 4, 4100
    W = max_seq - sinks
    slots, fill, events = ref.simulate_sink_schedule(1000, 100_000, sinks, max_seq)
    # replay: physical ring holding token ids
    phys = np.full(max_seq, -1, np.int64)
    head, fill_r, fed = 0, 0, 0
    for t in range(1000):                        # prefill at slots 0..999
        phys[E.ring_map(sinks, max_seq, head, t)] = t
    fill_r, fed = 1000, 1000
    ev = iter(events)
    while fed < 100_000:
        batch = min(4, 100_000 - fed)
        if fill_r + batch > max_seq:
            nf, b, k = E.evict_plan(fill_r, fill_r + batch - max_seq, sinks, max_seq)
            assert (fill_r, b, k) == next(ev)
            head = (head + b) % W
            fill_r = nf
        for j in range(batch):
            phys[E.ring_map(sinks, max_seq, head, fill_r + j)] = fed
            fed += 1
        fill_r += batch
    if fill_r + 1 > max_seq:
        nf, b, k = E.evict_plan(fill_r, fill_r + 1 - max_seq, sinks, max_seq)
        head = (head + b) % W
        fill_r = nf
    assert fill_r == fill
    held = [int(phys[E.ring_map(sinks, max_seq, head, L)]) for L in range(fill_r)]
    assert held == slots
    assert head != 0                              # the window really wrapped


def test_ring_map_is_a_permutation():
    for head in (0, 1, 17, 4095):
        p = [E.ring_map(4, 4100, head, L) for L in range(4100)]
        assert sorted(p) == list(range(4100)) and p[:4] == [0, 1, 2, 3]


# ---------------------------------------------------------------- restoreCache checks
def _snap(**kw):
    s = {"version": 2, "kvCache": "f16", "model": {"layers": 2, "kvHeads": 8, "headDim": 128, "hidden": 0, "vocab": 0},
         "ids": list(range(50)), "roll": {"sinkTokens": 4, "cacheLen": 40}, "data": b"\0" * (40 * 100)}
    s.update(kw)
    return s


_MODEL = {"layers": 2, "kvHeads": 8, "headDim": 128, "hidden": 0, "vocab": 0}


def _validate(snap, roll=True, sinks=4, kv="f16", model=_MODEL, max_seq=4100, cache_len=0, history=(), hybrid=False):
    return E.validate_snapshot(snap, roll=roll, sinks=sinks, kv_cache=kv, model=model, max_seq_len=max_seq,
                               data_bytes=100, cache_len=cache_len, history=history, hybrid=hybrid)


@pytest.mark.parametrize("snap,kw,msg", [
    (_snap(version=3), {}, "unsupported snapshot version 3"),
    (_snap(), {"roll": False}, "saved under overflow 'sinks'"),
    (_snap(version=1, roll=None, data=b"\0" * 4900), {}, "saved under overflow 'error'"),
    (_snap(roll={"sinkTokens": 2, "cacheLen": 40}), {}, "uses 2 sink tokens but this engine uses 4"),
    (_snap(kvCache="q8"), {}, "kvCache 'q8' but this engine runs 'f16'"),
    (_snap(), {"model": dict(_MODEL, headDim=256)}, "different model"),
    (_snap(ids=[]), {}, "holds no tokens"),
    (_snap(roll={"sinkTokens": 4, "cacheLen": 5000}, data=b"\0" * 500000), {}, "needs 5000 cache slots"),
    (_snap(data=b"\0" * 3999), {}, "expected 4000"),
])
def test_restore_rejections(snap, kw, msg):
    """Every rejection of restoreCache (src/engine.ts:2808-2845), host-only."""
    with pytest.raises(_lib.BitgpuError, match=msg):
        _validate(snap, **kw)


def test_restore_lengths_and_delta_prefix():
    assert _validate(_snap()) == (40, 0, 40)                                  # v2: roll.cacheLen
    v1 = _snap(version=1, roll=None, data=b"\0" * 4900)
    assert _validate(v1, roll=False) == (49, 0, 49)                           # v1: ids.length - 1
    # v2 may restore exactly full (cacheLen == maxSeqLen); v1 needs one spare slot
    assert _validate(_snap(roll={"sinkTokens": 4, "cacheLen": 100}, data=b"\0" * 10000), max_seq=100)[0] == 100
    with pytest.raises(_lib.BitgpuError, match="needs 50 cache slots but maxSeqLen is 49"):
        _validate(v1, roll=False, max_seq=49)
    d = _snap(version=1, roll=None, base=10, data=b"\0" * 3900)
    assert _validate(d, roll=False, cache_len=10, history=list(range(10))) == (49, 10, 39)
    with pytest.raises(_lib.BitgpuError, match="expects the cache at position 10"):
        _validate(d, roll=False, cache_len=12, history=list(range(12)))
    with pytest.raises(_lib.BitgpuError, match=r"prefix does not match the current prewarm \(token 3\)"):
        _validate(d, roll=False, cache_len=10, history=[0, 1, 2, 7, 4, 5, 6, 7, 8, 9])


def test_restore_rejects_delta_on_the_hybrid_backbone():
    """restoreCache rejects a delta snapshot (base > 0) on the qwen3_5 hybrid backbone
    (src/engine.ts:2828), after the length and before the slot and size checks; a full
    snapshot (base 0) restores there as on a dense model."""
    d = _snap(version=1, roll=None, base=10, data=b"\0" * 3900)
    with pytest.raises(_lib.BitgpuError, match="delta snapshots are not supported for the qwen3_5 hybrid backbone"):
        _validate(d, roll=False, cache_len=10, history=list(range(10)), hybrid=True)
    # the reference's order: this check precedes the slot check (a delta that also overflows
    # maxSeqLen reports the hybrid rejection) and follows the empty-ids check
    with pytest.raises(_lib.BitgpuError, match="qwen3_5 hybrid backbone"):
        _validate(d, roll=False, cache_len=10, history=list(range(10)), hybrid=True, max_seq=20)
    with pytest.raises(_lib.BitgpuError, match="holds no tokens"):
        _validate(_snap(version=1, roll=None, base=10, ids=[]), roll=False, hybrid=True)
    full = _snap(version=1, roll=None, data=b"\0" * 4900)
    assert _validate(full, roll=False, hybrid=True) == (49, 0, 49)
    assert _validate(d, roll=False, cache_len=10, history=list(range(10)), hybrid=False) == (49, 10, 39)


# ---------------------------------------------------------------- decode split plan
def _plan(KV, D, S, H, pos_base, cus=256, resident=1, dtype=_lib.BG_KV_Q8):
    out = (C.c_int32 * 6)()
    rc = _lib.lib().bg_decode_plan(KV, D, dtype, S, H, pos_base, cus, resident, out)
    return rc, list(out)


# every decode shape the GPU tests run (kv heads, head_dim, rows S, heads H, attended positions)
_DECODE_SHAPES = [(8, 128, 1, 32, L) for L in (1, 31, 32, 33, 517, 4096, 4097, 16384, 32768)] + [
    (16, 128, 1, 16, 777), (8, 128, 1, 64, 777), (4, 256, 1, 24, 777), (8, 256, 1, 8, 777), (2, 128, 1, 16, 777),
    (4, 256, 1, 24, 4097), (2, 128, 1, 16, 32768), (2, 128, 1, 2, 32768), (1, 256, 1, 4, 32768),
    (8, 128, 12, 32, 4108), (8, 128, 5, 32, 4000), (8, 128, 5, 32, 3749), (4, 256, 2, 24, 902), (4, 256, 3, 24, 903),
    (4, 256, 1, 24, 8193), (3, 128, 1, 12, 32768), (5, 128, 1, 20, 20000), (8, 128, 1, 32, 3745),
    (1, 256, 1, 16, 5120), (1, 128, 1, 24, 1024)]


@pytest.mark.parametrize("KV,D,S,H,L", _DECODE_SHAPES)
@pytest.mark.parametrize("resident", [1, 2])
def test_decode_plan_covers_tiles_and_fits_the_gpu(KV, D, S, H, L, resident):
    """The split-K plan: the splits cover every tile exactly once, the grid never exceeds what
    the GPU holds at once (the merge waits on splits of its own grid), the merging splits are
    min(units, splits) and the wave count follows the tiles-per-CU rule."""
    cus = 256
    rc, (waves, ns, tps, nm, grid, tiles) = _plan(KV, D, S, H, L - S, cus, resident)
    assert rc == 0
    assert tiles == (L + 31) // 32
    assert ns * tps >= tiles and (ns - 1) * tps < tiles           # every tile, no empty split
    assert grid == ns * KV <= resident * cus
    R = (H // KV) * S
    units = R * (D // 64)
    assert nm == (min(units, ns) if ns > 1 else 0)
    assert ns <= 256
    if ns > 1:
        assert tps >= waves                                        # every wave has a tile
    nset = (R + 15) // 16
    assert waves == (8 if D == 128 and nset == 1 and tiles * KV >= 8 * cus else 4)


def test_decode_plan_residency_cap():
    # 3 kv heads on 256 CUs at one workgroup a CU: ceil-splitting alone would give 86 x 3 = 258
    rc, (waves, ns, tps, nm, grid, tiles) = _plan(3, 128, 1, 12, 32767, 256, 1)
    assert rc == 0 and grid <= 256 and tps == 13 and ns == 79    # tiles per split raised 12 -> 13
    # a GPU that holds fewer workgroups than two splits per kv head runs one split, no merge
    rc, (waves, ns, tps, nm, grid, tiles) = _plan(8, 128, 1, 32, 32767, 8, 1)
    assert rc == 0 and ns == 1 and nm == 0 and tps == tiles
    # shapes the decode kernel does not take
    assert _plan(8, 128, 64, 32, 1000)[0] == _lib.BG_E_UNSUPPORTED


def test_diag_stream_read_argument_validation():
    lib = _lib.lib()
    buf = (C.c_uint32 * 64)()
    p = C.cast(buf, C.c_void_p)
    assert lib.bg_diag_stream_read(p, 100, 4, 1, p, None) == _lib.BG_E_INVALID       # not a multiple of 16
    assert b"bg_diag_stream_read" in lib.bg_last_error_message()
    assert lib.bg_diag_stream_read(None, 256, 4, 1, p, None) == _lib.BG_E_INVALID
    assert lib.bg_diag_stream_read(p, 256, 4, 1, None, None) == _lib.BG_E_INVALID
    assert lib.bg_diag_stream_read(p, 256, 0, 1, p, None) == _lib.BG_E_INVALID
    assert lib.bg_diag_stream_read(p, 0, 4, 1, p, None) == _lib.BG_E_INVALID


def test_decode_plan_one_tile_rule():
    """q8, 4-wave single-set launches: when one workgroup a CU would leave waves with two tiles
    and a CU holds two workgroups, the plan gives every wave one tile on a larger grid."""
    # C5 decode: 257 tiles x 4 kv heads (8193 positions) on 256 CUs
    rc, (waves, ns, tps, nm, grid, tiles) = _plan(4, 256, 1, 24, 8192, 256, 1)
    assert rc == 0 and (waves, tps, ns, grid) == (4, 5, 52, 208)      # one a CU: one wave has two tiles
    rc, (waves, ns, tps, nm, grid, tiles) = _plan(4, 256, 1, 24, 8192, 256, 2)
    assert rc == 0 and (waves, tps, ns, grid) == (4, 4, 65, 260)      # two a CU: one tile a wave
    assert nm == min(6 * 4, 65)
    # f16 keeps one workgroup a CU (measured faster), and so does a GPU that cannot hold the grid
    assert _plan(4, 256, 1, 24, 8192, 256, 2, dtype=_lib.BG_KV_F16)[1][2] == 5
    assert _plan(4, 256, 1, 24, 8192, 128, 2)[1][2] == 9
    # more than two tiles a wave at one workgroup a CU: unchanged
    assert _plan(4, 256, 1, 24, 3 * 8192, 256, 2)[1][2] == 13


# ---------------------------------------------------------------- 1-bit projections: host checks
def test_gemv_argument_validation():
    lib = _lib.lib()
    buf = (C.c_float * 64)()
    p = C.cast(buf, C.c_void_p)
    assert lib.bg_gemv_split(p, 100, p, p, 1, 0, 0, p, None, None, None) == _lib.BG_E_INVALID    # K % 128
    assert b"multiple of 128" in lib.bg_last_error_message()
    assert lib.bg_gemv_split(None, 128, p, p, 1, 0, 0, p, None, None, None) == _lib.BG_E_INVALID
    assert lib.bg_gemv_split(p, 128, p, p, 1, 2, 0, p, None, None, None) == _lib.BG_E_INVALID    # out1 missing
    assert lib.bg_gemv_resid(p, 128, p, p, 4, None, p, None) == _lib.BG_E_INVALID
    assert lib.bg_qkv_proj_prologue(None, 0, p, 128, p, p, 8, p, p, 1e-6, p, p, 8, 128, 0, 0, p, None) == _lib.BG_E_INVALID
