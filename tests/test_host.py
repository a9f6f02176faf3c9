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


def _validate(snap, roll=True, sinks=4, kv="f16", model=_MODEL, max_seq=4100, cache_len=0, history=()):
    return E.validate_snapshot(snap, roll=roll, sinks=sinks, kv_cache=kv, model=model, max_seq_len=max_seq,
                               data_bytes=100, cache_len=cache_len, history=history)


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
