'use strict'
// JS/TypeScript host shim over the N-API addon: the reference engine's attention call shapes
// (src/engine.ts) on the MI355X C ABI. ES2019, no dependencies (the reference host is TypeScript;
// index.d.ts carries the types).
//
//   reference                                          this shim
//   appendKV(pass, src, which, li, rows, dstRow0)  ->  cache.appendKV(src, which, li, rows, dstRow0)
//   runN(pass, ATT, [S,H,KV,D,posBase,Ltot],
//        attIns(qr, li), att, S*H)                 ->  cache.att(qr, li, S, H, posBase, att)
//   hybrid attention_online_cache + gate_sigmoid   ->  cache.att(qr, li, S, H, posBase, att, {scale, gate, gateStride})
//   rmsnorm_rope_sg + ROPE_K + appendKV(v)          ->  cache.prologue({...})
//   ensureKvCapacity / evict / evictFor             ->  cache.ensureKvCapacity / evict / evictFor
//   synthRope                                       ->  synthRope(theta, rotDim, positions, yarn)
//   fusedMM / residMM at S = 1 (1344-1380)          ->  fusedMM(w, x, outs) / residMM(w, x, resid, out)
//   matmul_split_sg + rmsnorm_rope_sg + ROPE_K
//     + appendKV(v), decode (1526-1540)             ->  cache.qkvProjPrologue({...})
const path = require('path')
const addon = require(path.join(__dirname, 'bitgpu_attn.node'))

const KV_DTYPE = { f32: 0, f16: 1, q8: 2 }
const K = 0
const V = 1
const KSCALE = 2
const VSCALE = 3

// The reference's error class (src/errors.ts:14-19: name 'GpuOutOfMemoryError'). A host that has
// its own class (the engine's import of src/errors.ts) hands it to setErrorClasses, so its
// `instanceof` checks match what this shim throws; this class stands in until then.
class GpuOutOfMemoryError extends Error {
  constructor(message) {
    super(message)
    this.name = 'GpuOutOfMemoryError'
  }
}
let OomClass = GpuOutOfMemoryError

function setErrorClasses(classes) {
  if (classes && typeof classes.GpuOutOfMemoryError === 'function') OomClass = classes.GpuOutOfMemoryError
}

// addon errors carry .code (BG_E_*) and .name; OOM is re-thrown as the host's error class
function call(fn) {
  try {
    return fn()
  } catch (e) {
    if (e && e.name === 'GpuOutOfMemoryError') {
      const oom = new OomClass(e.message)
      if (oom.name !== 'GpuOutOfMemoryError') oom.name = 'GpuOutOfMemoryError'
      oom.code = e.code
      throw oom
    }
    throw e
  }
}

function synthRope(theta, rotDim, positions, yarn) {
  const half = rotDim / 2
  const cos = new Float32Array(positions * half)
  const sin = new Float32Array(positions * half)
  const factor = yarn ? yarn.factor : 1
  const orig = yarn ? yarn.original_max_position_embeddings : 0
  call(() => addon.ropeTables(theta, rotDim, positions, factor, orig, cos, sin))
  return [cos, sin]
}

class KvCache {
  // opts mirror EngineOptions (src/types.ts:138-177)
  constructor({ layers, kvHeads, headDim, kvCache = 'f32', maxSeqLen = 2048, capacity = 0, overflow = 'error', sinkTokens = 4, ropePositions = 'slot', q8Block = 32 }) {
    const roll = overflow === 'sinks'
    this.kvHeads = kvHeads
    this.headDim = headDim
    this.kvCache = kvCache
    this.roll = roll
    this.h = call(() => addon.kvCreate(layers, kvHeads, headDim, KV_DTYPE[kvCache], capacity, maxSeqLen, roll ? 1 : 0, roll ? Math.max(1, Math.floor(sinkTokens)) : 0, ropePositions === 'absolute' ? 1 : 0))
    // q8 scale block: 32 (copy_kv8.wgsl) or headDim (one scale per position and kv head)
    if (kvCache === 'q8' && q8Block !== 32) call(() => addon.kvSetQ8Block(this.h, q8Block))
  }
  // sink mode: [ring origin, rows evicted so far]; ringReset(evicted) compacts the ring (the
  // state a v2 snapshot is restored into, restoreCache src/engine.ts:2807-2872)
  get ringState() { return call(() => addon.kvRingState(this.h)) }
  ringReset(evicted = 0) { call(() => addon.kvRingReset(this.h, evicted)) }
  dispose() { if (this.h) { addon.kvDestroy(this.h); this.h = null } }
  get capacity() { return addon.kvCapacity(this.h) }
  ensureKvCapacity(needed, stream = null) { call(() => addon.kvGrow(this.h, needed, stream)) }
  setRollTables(cosDev, sinDev, positions) { call(() => addon.kvSetRope(this.h, cosDev, sinDev, positions, this.headDim)) }
  appendKV(srcDev, which, li, rows, dstRow0, stream = null) { call(() => addon.kvWrite(this.h, li, which, srcDev, rows, dstRow0, stream)) }
  prologue({ li, q = null, qStride = 0, k = null, v = null, S, H, qGamma = null, kGamma = null, eps, cos, sin, ropePositions, rotDim, pos0, slot0, qOut = null, stream = null }) {
    call(() => addon.qkvPrologue(this.h, li, q, qStride || this.headDim, k, v, S, H, qGamma, kGamma, eps, cos, sin, ropePositions, rotDim, pos0, slot0, qOut, stream))
  }
  att(qr, li, S, H, posBase, out, { scale = Math.fround(1 / Math.sqrt(this.headDim)), gate = null, gateStride = 0, stream = null } = {}) {
    call(() => addon.attention(this.h, li, qr, S, H, posBase, scale, gate, gate ? (gateStride || this.headDim) : 0, out, stream))
  }
  evict(fill, need) { return call(() => addon.kvEvict(this.h, fill, need)) }
  evictFor(fill, n) { return call(() => addon.kvEvictFor(this.h, fill, n)) }
  exportRows(li, region, base, count) {
    const buf = new ArrayBuffer(addon.kvRegionBytes(this.h, region, count))
    call(() => addon.kvExportRows(this.h, li, region, base, count, buf, null))
    return buf
  }
  importRows(li, region, base, count, buf) { call(() => addon.kvImportRows(this.h, li, region, base, count, buf, null)) }
  // w = { sign, scales, K, N0, N1, N2 } (device pointers as BigInt, GpuWeight of src/engine.ts:814-830)
  qkvProjPrologue({ li, x, w, H, qGamma, kGamma, eps, cos, sin, ropePositions, rotDim, pos, slot, qOut, stream = null }) {
    call(() => addon.qkvProjPrologue(this.h, li, x, w.K, w.sign, w.scales, H, qGamma, kGamma, eps, cos, sin, ropePositions, rotDim, pos, slot === undefined ? pos : slot, qOut, stream))
  }
}

function fusedMM(w, x, outs, stream = null) {
  call(() => addon.gemvSplit(x, w.K, w.sign, w.scales, w.N0, w.N1 || 0, w.N2 || 0, outs[0] || null, outs[1] || null, outs[2] || null, stream))
}

function residMM(w, x, resid, out, stream = null) {
  call(() => addon.gemvResid(x, w.K, w.sign, w.scales, w.N || w.N0, resid, out, stream))
}

module.exports = { addon, KvCache, synthRope, fusedMM, residMM, GpuOutOfMemoryError, setErrorClasses, K, V, KSCALE, VSCALE,
  KV_DTYPE }
