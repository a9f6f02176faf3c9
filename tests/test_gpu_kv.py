"""GPU: KV-cache writes are bit-exact with the reference quantizers, and the cache lifecycle
(growth with rollback, snapshot export/import, sink-mode ring writes) preserves every byte.

Bars: f32 rows bit-identical, f16 rows = IEEE RNE bits (shaders/copy_kv16.wgsl:13), q8 codes
and scales bit-identical to the WGSL pack4x8snorm quantizer (shaders/copy_kv8.wgsl:24-40)."""
import os

import numpy as np
import pytest
import torch

from bitgpu_amd import GpuOutOfMemoryError
from bitgpu_amd import engine as E
from bitgpu_amd._lib import BG_K, BG_V, BitgpuError
from oracle import ref
from tests.gpu_helpers import export_k_v, fill_cache_raw, run_attention, t

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _rows(L, KV, D, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((L, KV, D)) * np.exp(rng.uniform(-6, 6, (L, KV, 1)))).astype(np.float32)
    x[0] = 0.0                                    # all-zero rows: scale 1e-30, codes 0
    x[1, 0] = -0.0
    g = np.load(os.path.join(ROOT, "tests", "golden", "q8_cases.npz"))["x"]   # golden special rows
    if D == 128:
        n = min(len(g), L - 2)
        x[2:2 + n, 0] = g[:n]
    return x


@pytest.mark.parametrize("dtype", ["f32", "f16", "q8"])
@pytest.mark.parametrize("D", [128, 256])
def test_kv_write_bit_exact(dev, dtype, D):
    L, KV = 70, 4
    k, v = _rows(L, KV, D, 1), _rows(L, KV, D, 2)
    c = E.KvCache(2, KV, D, dtype, max_seq_len=256, capacity=L)
    # two appends: rows of positions [0, 37) then [37, 70) at dstRow0 = 37 * KV
    c.append_kv(t(k[:37]), BG_K, 1, 37 * KV, 0)
    c.append_kv(t(k[37:]), BG_K, 1, (L - 37) * KV, 37 * KV)
    c.append_kv(t(v), BG_V, 1, L * KV, 0)
    torch.cuda.synchronize()
    ek, ev, eks, evs = export_k_v(c, 1, 0, L)
    if dtype == "f32":
        assert np.array_equal(ek.view(np.uint32), k.view(np.uint32))
        assert np.array_equal(ev.view(np.uint32), v.view(np.uint32))
    elif dtype == "f16":
        assert np.array_equal(ek.view(np.uint16), ref.f16_pack(k).view(np.uint16))
        assert np.array_equal(ev.view(np.uint16), ref.f16_pack(v).view(np.uint16))
    else:
        ck, sk = ref.q8_pack(k)
        cv, sv = ref.q8_pack(v)
        assert np.array_equal(ek, ck) and np.array_equal(eks.view(np.uint32), sk.view(np.uint32))
        assert np.array_equal(ev, cv) and np.array_equal(evs.view(np.uint32), sv.view(np.uint32))
    c.close()


def test_grow_preserves_content_and_doubles(dev):
    KV, D = 4, 128
    c = E.KvCache(2, KV, D, "q8", max_seq_len=1000, capacity=64)
    k, v = _rows(64, KV, D, 3), _rows(64, KV, D, 4)
    fill_cache_raw(c, 0, k, v)
    before = export_k_v(c, 0, 0, 64)
    c.ensure_capacity(70)                          # doubling: max(70, 128) = 128
    assert c.capacity == 128
    after = export_k_v(c, 0, 0, 64)
    for a, b in zip(before, after):
        assert np.array_equal(a, b)
    c.ensure_capacity(5000)                        # clamped to maxSeqLen
    assert c.capacity == 1000
    c.close()


def test_grow_oom_rolls_back(dev, monkeypatch):
    KV, D = 4, 128
    c = E.KvCache(2, KV, D, "f16", max_seq_len=1000, capacity=64)
    k, v = _rows(64, KV, D, 5), _rows(64, KV, D, 6)
    fill_cache_raw(c, 1, k, v)
    monkeypatch.setenv("BG_FAULT_GROW_ALLOC", "3")     # third allocation of the growth fails
    with pytest.raises(GpuOutOfMemoryError, match="KV cache growth"):
        c.ensure_capacity(200)
    monkeypatch.delenv("BG_FAULT_GROW_ALLOC")
    assert c.capacity == 64
    ek, ev, _, _ = export_k_v(c, 1, 0, 64)
    assert np.array_equal(ek.view(np.uint16), ref.f16_pack(k).view(np.uint16))
    # the cache stays usable
    q = np.random.default_rng(0).standard_normal((1, 8, D)).astype(np.float32)
    out = run_attention(c, 1, q, 63)
    assert np.isfinite(out).all()
    c.ensure_capacity(200)
    assert c.capacity == 200
    c.close()


@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_snapshot_roundtrip_into_fresh_cache(dev, dtype):
    KV, D, L = 8, 128, 300
    a = E.KvCache(3, KV, D, dtype, max_seq_len=512, capacity=512)
    for li in range(3):
        fill_cache_raw(a, li, _rows(L, KV, D, 10 + li), _rows(L, KV, D, 20 + li))
    snap = a.save_snapshot(L)
    per_row = KV * D * (4 if dtype == "f32" else 1) + (KV * D // 32 * 4 if dtype == "q8" else 0)
    assert len(snap) == 3 * 2 * L * per_row            # src/engine.ts:2732-2733 snapshotBytes
    b = E.KvCache(3, KV, D, dtype, max_seq_len=512)    # fresh, smaller initial capacity
    b.restore_snapshot(snap, L)
    q = np.random.default_rng(1).standard_normal((1, 32, D)).astype(np.float32)
    for li in range(3):
        for x, y in zip(export_k_v(a, li, 0, L), export_k_v(b, li, 0, L)):
            if x is not None:
                assert np.array_equal(x, y)
        assert np.array_equal(run_attention(a, li, q, L - 1), run_attention(b, li, q, L - 1))
    # delta snapshot: positions [base, L)
    d = a.save_snapshot(L, base=100)
    cpart = E.KvCache(3, KV, D, dtype, max_seq_len=512, capacity=512)
    for li in range(3):
        fill_cache_raw(cpart, li, _rows(L, KV, D, 10 + li)[:100], _rows(L, KV, D, 20 + li)[:100])
    cpart.restore_snapshot(d, L, base=100)
    for li in range(3):
        assert np.array_equal(run_attention(a, li, q, L - 1), run_attention(cpart, li, q, L - 1))
    with pytest.raises(ValueError, match="expected"):
        b.restore_snapshot(snap[:-4], L)
    for x in (a, b, cpart):
        x.close()


def test_sink_ring_writes_land_at_logical_slots(dev):
    KV, D, sinks, max_seq = 2, 128, 4, 100
    c = E.KvCache(1, KV, D, "q8", max_seq_len=max_seq, overflow="sinks", sink_tokens=sinks)
    rows = _rows(max_seq, KV, D, 7)
    fill_cache_raw(c, 0, rows, rows)
    fill = c.evict_for(max_seq, 10)                    # evicts a quarter-window batch
    nf, batch, keep = ref.evict(max_seq, 10, sinks, max_seq)
    assert fill == nf and c.ring_state() == (batch, batch)
    kept = np.concatenate([rows[:sinks], rows[sinks + batch: sinks + batch + keep]])
    ck, sk = ref.q8_pack(kept)
    ek, _, eks, _ = export_k_v(c, 0, 0, fill)
    assert np.array_equal(ek, ck) and np.array_equal(eks, sk)
    new = _rows(max_seq - fill, KV, D, 8)               # these wrap around the physical ring
    fill_cache_raw(c, 0, new, new, row0=fill)
    ek, _, _, _ = export_k_v(c, 0, fill, max_seq - fill)
    assert np.array_equal(ek, ref.q8_pack(new)[0])
    c.close()


def test_argument_errors_are_raised_not_faulted(dev):
    c = E.KvCache(1, 8, 128, "f16", max_seq_len=256, capacity=64)
    q = t(np.zeros((1, 32, 128), np.float32))
    with pytest.raises(BitgpuError, match="exceed the cache"):
        E.attention(c, 0, q, 1, 32, 64)                # position 64 is beyond capacity 64
    with pytest.raises(BitgpuError, match="out of range"):
        E.attention(c, 3, q, 1, 32, 0)
    with pytest.raises(BitgpuError, match="multiple of kv_heads|heads"):
        E.attention(c, 0, t(np.zeros((1, 12, 128), np.float32)), 1, 12, 0)
    with pytest.raises(BitgpuError, match="beyond capacity"):
        c.append_kv(t(np.zeros((8, 128), np.float32)), BG_K, 0, 8, 64 * 8)
    c.close()


def test_stream_and_event_utilities(dev):
    """bg_stream_create / bg_event_*: the same attention launched on a library-created stream
    (timed by two events recorded on it) and on torch's stream gives identical bytes."""
    import ctypes as C
    from bitgpu_amd import _lib
    lib = _lib.lib()
    st, e0, e1 = C.c_void_p(), C.c_void_p(), C.c_void_p()
    _lib.check(lib.bg_stream_create(C.byref(st)))
    _lib.check(lib.bg_event_create(C.byref(e0)))
    _lib.check(lib.bg_event_create(C.byref(e1)))
    rng = np.random.default_rng(11)
    L, H, KV, D = 2000, 32, 8, 128
    k = rng.standard_normal((L, KV, D)).astype(np.float32)
    v = rng.standard_normal((L, KV, D)).astype(np.float32)
    q = t(rng.standard_normal((1, H, D)).astype(np.float32))
    c = E.KvCache(1, KV, D, "q8", max_seq_len=L, capacity=L)
    fill_cache_raw(c, 0, k, v)
    ref_out = E.attention(c, 0, q, 1, H, L - 1)
    torch.cuda.synchronize()
    with torch.cuda.stream(torch.cuda.ExternalStream(st.value)):
        _lib.check(lib.bg_event_record(e0, st))
        out = E.attention(c, 0, q, 1, H, L - 1)
        _lib.check(lib.bg_event_record(e1, st))
    us = C.c_float()
    _lib.check(lib.bg_event_elapsed_us(e0, e1, C.byref(us)))
    _lib.check(lib.bg_stream_sync(st))
    assert 0.0 < us.value < 1e6
    assert torch.equal(out, ref_out)
    for ev in (e0, e1):
        _lib.check(lib.bg_event_destroy(ev))
    _lib.check(lib.bg_stream_destroy(st))
    c.close()


@pytest.mark.parametrize("dtype", ["f16", "q8", "f32"])
def test_v2_snapshot_restores_into_a_wrapped_ring(dev, dtype):
    """saveCache / restoreCache under overflow 'sinks' (src/engine.ts:2736-2872): a v2 snapshot
    of a cache whose ring has wrapped restores into another sink-mode cache whose ring origin is
    elsewhere; the restored logical slots hold the same bytes and attention over them matches
    the oracle (keys rotated at read by their slot). Restoring it into an overflow 'error'
    cache is rejected with the reference's message."""
    rng = np.random.default_rng(61)
    H, KV, D, sinks, max_seq = 32, 8, 128, 4, 260
    from tests.gpu_helpers import rope_dev
    cos_d, sin_d, cos, sin = rope_dev(1e6, D, max_seq)

    def sink_cache():
        c = E.KvCache(1, KV, D, dtype, max_seq_len=max_seq, overflow="sinks", sink_tokens=sinks)
        c.set_rope(cos_d, sin_d)
        return c

    a = sink_cache()
    k0 = rng.standard_normal((200, KV, D)).astype(np.float32)
    fill_cache_raw(a, 0, k0, k0[::-1].copy())
    fill = a.evict_for(200, 100)                       # evict(200, 40): drops a 64-row batch
    assert fill == ref.evict(200, 40, sinks, max_seq)[0] == 136
    k1 = rng.standard_normal((100, KV, D)).astype(np.float32)
    v1 = rng.standard_normal((100, KV, D)).astype(np.float32)
    fill_cache_raw(a, 0, k1, v1, row0=fill)
    n = fill + 100
    assert a.ring_state()[0] != 0
    snap = a.save_cache(ids=list(range(1000)), cache_len=n)
    assert snap["version"] == 2 and snap["roll"]["cacheLen"] == n and snap["roll"]["sinkTokens"] == sinks

    b = sink_cache()
    junk = rng.standard_normal((max_seq, KV, D)).astype(np.float32)
    fill_cache_raw(b, 0, junk, junk)
    assert b.evict_for(max_seq, 10) == 196             # origin 64
    assert b.evict_for(196, 70) == 132                 # a second batch of 64: origin 128
    assert b.ring_state()[0] not in (0, a.ring_state()[0])
    assert b.restore_cache(snap) == n
    assert b.ring_state() == (0, a.ring_state()[1])
    for x, y in zip(export_k_v(a, 0, 0, n), export_k_v(b, 0, 0, n)):
        if x is not None:
            assert np.array_equal(x, y)
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    kst, vst, ks, vs = export_k_v(b, 0, 0, n)
    if dtype == "q8":
        kst, vst = ref.q8_dequant(kst, ks), ref.q8_dequant(vst, vs)
    kk = ref.rope_apply(kst.astype(np.float32), cos, sin, np.arange(n))
    exp = ref.attention(q, kk, vst.astype(np.float32), n - 1)
    for c in (a, b):
        out = run_attention(c, 0, q, n - 1)
        if dtype == "f32":
            assert np.abs(out - exp).max() <= 1e-4
        else:
            assert np.abs(out - exp).max() / np.abs(exp).max() <= 2e-3
    plain = E.KvCache(1, KV, D, dtype, max_seq_len=max_seq)
    with pytest.raises(BitgpuError, match="saved under overflow 'sinks'"):
        plain.restore_cache(snap)
    for c in (a, b, plain):
        c.close()


def test_restore_that_cannot_grow_writes_nothing(dev, monkeypatch):
    """restoreCache grows the cache before it writes anything (src/engine.ts:2846-2848): when the
    growth fails (host fault injector) it raises GpuOutOfMemoryError with the capacity and the
    resident rows unchanged, and the same restore then succeeds. (A sink-mode cache holds its
    whole window from creation, so only a plain cache grows here.)"""
    rng = np.random.default_rng(67)
    KV, D, n = 8, 128, 300
    a = E.KvCache(1, KV, D, "q8", max_seq_len=1024, capacity=512)
    k0 = rng.standard_normal((n, KV, D)).astype(np.float32)
    fill_cache_raw(a, 0, k0, k0[::-1].copy())
    snap = a.save_cache(ids=list(range(n + 1)))
    b = E.KvCache(1, KV, D, "q8", max_seq_len=1024, capacity=64)
    k1 = rng.standard_normal((40, KV, D)).astype(np.float32)
    fill_cache_raw(b, 0, k1, k1)
    before = export_k_v(b, 0, 0, 40)
    monkeypatch.setenv("BG_FAULT_GROW_ALLOC", "1")
    with pytest.raises(GpuOutOfMemoryError):
        b.restore_cache(snap)
    monkeypatch.delenv("BG_FAULT_GROW_ALLOC")
    assert b.capacity == 64
    for x, y in zip(before, export_k_v(b, 0, 0, 40)):
        assert np.array_equal(x, y)
    assert b.restore_cache(snap) == n
    for x, y in zip(export_k_v(a, 0, 0, n), export_k_v(b, 0, 0, n)):
        assert np.array_equal(x, y)
    a.close()
    b.close()


@pytest.mark.parametrize("D", [128, 256])
def test_q8_per_row_scale_mode(dev, D):
    """q8 with one scale per (position, kv head) row (bg_kv_set_q8_block(head_dim)): appendKV and
    the fused prologue store the codes of ref.q8_pack(x, block=D) bit for bit, the row scale in
    each 32-value slot; decode and prefill attention over such a cache match the oracle."""
    KV, H, L = 4, 16, 700
    rng = np.random.default_rng(D + 1)
    k = _rows(L, KV, D, 31)
    v = _rows(L, KV, D, 32)
    c = E.KvCache(1, KV, D, "q8", max_seq_len=1024, capacity=1024, q8_block=D)
    fill_cache_raw(c, 0, k, v)
    ek, ev, eks, evs = export_k_v(c, 0, 0, L)
    for got, gs, x in ((ek, eks, k), (ev, evs, v)):
        want, ws = ref.q8_pack(x, block=D)
        assert np.array_equal(got, want)
        assert np.array_equal(gs.view(np.uint32), np.repeat(ws, D // 32, -1).view(np.uint32))
    # the fused prologue's K write (normed, roped) in per-row mode equals the quantizer on its f32
    from tests.gpu_helpers import rope_dev
    cos_d, sin_d, _, _ = rope_dev(1e6, D, 1024)
    ones = t(np.ones(D, np.float32))
    c32 = E.KvCache(1, KV, D, "f32", max_seq_len=1024, capacity=1024)
    for cc in (c, c32):
        E.qkv_prologue(cc, 0, None, t(k[:40]), t(v[:40]), 40, H, None, ones, 1e-6, cos_d, sin_d, D, 800, 800)
    torch.cuda.synchronize()
    k32, v32, _, _ = export_k_v(c32, 0, 800, 40)
    kq, vq, ks, vs = export_k_v(c, 0, 800, 40)
    for got, gs, x in ((kq, ks, k32), (vq, vs, v32)):
        want, ws = ref.q8_pack(x, block=D)
        assert np.array_equal(got, want) and np.array_equal(gs, np.repeat(ws, D // 32, -1))
    c.close()
    c32.close()
    # attention reads it like any q8 cache (N(0,1) rows: the rows above span e^+-6 per row, whose
    # scores are beyond the f16 query operand's resolution in any storage mode)
    c = E.KvCache(1, KV, D, "q8", max_seq_len=1024, capacity=1024, q8_block=D)
    k = rng.standard_normal((L, KV, D)).astype(np.float32)
    v = rng.standard_normal((L, KV, D)).astype(np.float32)
    fill_cache_raw(c, 0, k, v)
    ek, ev, eks, evs = export_k_v(c, 0, 0, L)
    assert np.array_equal(ek, ref.q8_pack(k, block=D)[0]) and np.array_equal(ev, ref.q8_pack(v, block=D)[0])
    kk, vv = ref.q8_dequant(ek, eks), ref.q8_dequant(ev, evs)
    for S in (1, 2, 3, 300):   # decode passes of 4 and 8 rows (one and two), prefill
        q = rng.standard_normal((S, H, D)).astype(np.float32)
        out = run_attention(c, 0, q, L - S)
        exp = ref.attention(q, kk, vv, L - S)
        assert np.abs(out - exp).max() / np.abs(exp).max() <= 2e-3
    c.close()
