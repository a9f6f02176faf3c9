"""The N-API addon + JS shim (bitgpu_amd/node) that a TypeScript engine host would bind:
host-only entry points on the CPU, and one decode + prefill through the addon on the GPU,
checked against the oracle."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from bitgpu_amd import engine as E
from bitgpu_amd import _lib
from bitgpu_amd._lib import BG_E_UNSUPPORTED
from oracle import ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE_DIR = os.path.join(ROOT, "bitgpu_amd", "node")
NODE = shutil.which("node")


def run_node(script, tmp_path, timeout=120, env=None):
    p = tmp_path / "t.js"
    p.write_text(f"const b = require({json.dumps(os.path.join(NODE_DIR, 'index.js'))});\n" + script)
    r = subprocess.run([NODE, str(p)], capture_output=True, text=True, timeout=timeout,
                       env=None if env is None else {**os.environ, **env})
    assert r.returncode == 0, r.stderr
    return r.stdout


pytestmark_node = pytest.mark.skipif(NODE is None or not os.path.exists(os.path.join(NODE_DIR, "bitgpu_attn.node")),
                                     reason="node or the built addon is not available")


@pytestmark_node
def test_addon_host_functions(tmp_path):
    out = run_node("""
const res = {}
res.plans = [[4100, 4], [4100, 1], [3000, 9], [200, 500]].map(([f, n]) => b.addon.evictPlan(f, n, 4, 4100))
res.ring = [0, 3, 4, 100, 4099].map(L => b.addon.ringMap(4, 4100, 1234, L))
const [c, s] = b.synthRope(1e7, 64, 300)
res.cos = Array.from(c); res.sin = Array.from(s)
try { new b.KvCache({layers: 1, kvHeads: 8, headDim: 128, maxSeqLen: 60, overflow: 'sinks'}) } catch (e) { res.err = [e.code, e.message] }
console.log(JSON.stringify(res))
""", tmp_path)
    res = json.loads(out)
    for (f, n), got in zip([[4100, 4], [4100, 1], [3000, 9], [200, 500]], res["plans"]):
        assert tuple(got) == ref.evict(f, n, 4, 4100)
    assert res["ring"] == [E.ring_map(4, 4100, 1234, L) for L in [0, 3, 4, 100, 4099]]
    c, s = E.rope_tables(1e7, 64, 300)
    assert np.array_equal(np.array(res["cos"], np.float32), c.ravel())
    assert np.array_equal(np.array(res["sin"], np.float32), s.ravel())
    assert res["err"][0] == -1 and "maxSeqLen >= sinkTokens + 64" in res["err"][1]


@pytest.mark.gpu
@pytestmark_node
@pytest.mark.parametrize("dtype,S", [("q8", 1), ("f16", 70)])
def test_addon_attention_on_gpu(tmp_path, dtype, S):
    rng = np.random.default_rng(S)
    L, H, KV, D = 300, 32, 8, 128
    k = rng.standard_normal((L, KV, D)).astype(np.float32)
    v = rng.standard_normal((L, KV, D)).astype(np.float32)
    q = rng.standard_normal((S, H, D)).astype(np.float32)
    for name, arr in (("k", k), ("v", v), ("q", q)):
        arr.tofile(tmp_path / f"{name}.bin")
    _ = run_node(f"""
const fs = require('fs')
const rd = n => {{ const b = fs.readFileSync({json.dumps(str(tmp_path))} + '/' + n + '.bin'); return new Float32Array(b.buffer, b.byteOffset, b.length / 4) }}
const a = b.addon
const k = rd('k'), v = rd('v'), q = rd('q')
const dk = a.devAlloc(k.byteLength), dv = a.devAlloc(v.byteLength), dq = a.devAlloc(q.byteLength), dout = a.devAlloc(q.byteLength)
a.h2d(dk, k); a.h2d(dv, v); a.h2d(dq, q)
const c = new b.KvCache({{layers: 2, kvHeads: {KV}, headDim: {D}, kvCache: '{dtype}', maxSeqLen: 512, capacity: {L}}})
c.appendKV(dk, b.K, 1, {L * KV}, 0)
c.appendKV(dv, b.V, 1, {L * KV}, 0)
const st = a.streamCreate(), e0 = a.eventCreate(), e1 = a.eventCreate()
a.eventRecord(e0, st)
c.att(dq, 1, {S}, {H}, {L - S}, dout, {{stream: st}})
a.eventRecord(e1, st)
const us = a.eventElapsedUs(e0, e1)
a.sync()
const out = new Float32Array(q.length)
a.d2h(out, dout)
fs.writeFileSync({json.dumps(str(tmp_path))} + '/out.bin', Buffer.from(out.buffer))
a.eventDestroy(e0); a.eventDestroy(e1); a.streamDestroy(st)
c.dispose()
console.log(JSON.stringify({{us}}))
""", tmp_path)
    us = json.loads(_.strip().splitlines()[-1])["us"]
    assert 0.0 < us < 1e6  # the attention ran on the addon's own stream, timed by its events
    out = np.fromfile(tmp_path / "out.bin", np.float32).reshape(S, H, D)
    exp = ref.attention(q, ref.kv_roundtrip(k, dtype), ref.kv_roundtrip(v, dtype), L - S)
    assert np.abs(out - exp).max() / np.abs(exp).max() <= 2e-3


@pytest.mark.gpu
@pytestmark_node
def test_addon_ring_state_and_q8_block(tmp_path):
    """The shim's sink-mode ring state / reset (the compacted ring a v2 snapshot restores into)
    and the q8 scale block option (32 or headDim; anything else is refused)."""
    out = run_node("""
const res = {}
const c = new b.KvCache({layers: 1, kvHeads: 8, headDim: 128, kvCache: 'f16', maxSeqLen: 4100, overflow: 'sinks', sinkTokens: 4})
res.s0 = c.ringState
const fill = c.evictFor(4100, 4)
res.fill = fill
res.s1 = c.ringState
c.ringReset(12345)
res.s2 = c.ringState
c.dispose()
const q = new b.KvCache({layers: 1, kvHeads: 8, headDim: 128, kvCache: 'q8', maxSeqLen: 256, q8Block: 128})
q.dispose()
try { new b.KvCache({layers: 1, kvHeads: 8, headDim: 128, kvCache: 'q8', maxSeqLen: 256, q8Block: 64}) } catch (e) { res.err = [e.code, e.message] }
console.log(JSON.stringify(res))
""", tmp_path)
    res = json.loads(out.strip().splitlines()[-1])
    assert res["s0"] == [0, 0]
    new_fill, dropped, _ = ref.evict_for(4100, 4, 4, 4100)
    assert res["fill"] == new_fill and res["s1"][1] == dropped and res["s1"][0] == dropped % (4100 - 4)
    assert res["s2"] == [0, 12345]
    assert res["err"][0] == BG_E_UNSUPPORTED
    assert "32 or head_dim 128" in res["err"][1]


@pytest.mark.gpu
@pytestmark_node
def test_addon_oom_is_the_reference_error_class(tmp_path):
    """A failed KV growth (the host fault injector makes its first device allocation fail)
    reaches JS as the reference's GpuOutOfMemoryError (src/errors.ts:14-19): name
    'GpuOutOfMemoryError', instanceof the shim's class, and instanceof the host's own class once
    the host has passed it to setErrorClasses. The cache keeps its capacity."""
    out = run_node("""
const res = {}
const c = new b.KvCache({layers: 1, kvHeads: 8, headDim: 128, kvCache: 'f16', maxSeqLen: 4096, capacity: 64})
try { c.ensureKvCapacity(1000) } catch (e) {
  res.shim = [e instanceof b.GpuOutOfMemoryError, e instanceof Error, e.name, e.code, e.message]
}
class HostOom extends Error { constructor(m) { super(m); this.name = 'GpuOutOfMemoryError' } }
b.setErrorClasses({GpuOutOfMemoryError: HostOom})
try { c.ensureKvCapacity(1000) } catch (e) {
  res.host = [e instanceof HostOom, e.name, e.code]
}
res.cap = c.capacity
c.dispose()
try { new b.KvCache({layers: 1, kvHeads: 8, headDim: 128, maxSeqLen: 60, overflow: 'sinks'}) } catch (e) {
  res.other = [e instanceof HostOom, e.name]
}
console.log(JSON.stringify(res))
""", tmp_path, env={"BG_FAULT_GROW_ALLOC": "1"})
    res = json.loads(out.strip().splitlines()[-1])
    assert res["shim"][:4] == [True, True, "GpuOutOfMemoryError", _lib.BG_E_OOM]
    assert "KV cache growth" in res["shim"][4]
    assert res["host"] == [True, "GpuOutOfMemoryError", _lib.BG_E_OOM]
    assert res["cap"] == 64
    assert res["other"] == [False, "Error"]        # only OOM maps to the class
