// Types of the JS shim (index.js) for a TypeScript host. Device pointers and streams are bigint.
export type DevPtr = bigint
export declare const K: 0, V: 1, KSCALE: 2, VSCALE: 3
// the reference's class (src/errors.ts:14-19): name 'GpuOutOfMemoryError'; a host passes its own
// class to setErrorClasses so that its instanceof checks match what the shim throws
export declare class GpuOutOfMemoryError extends Error { readonly name: 'GpuOutOfMemoryError'; code?: number }
export declare function setErrorClasses(classes: { GpuOutOfMemoryError?: new (message: string) => Error }): void
export declare function synthRope(theta: number, rotDim: number, positions: number,
  yarn?: { factor: number; original_max_position_embeddings: number }): [Float32Array, Float32Array]
export interface KvCacheOptions {
  layers: number; kvHeads: number; headDim: number
  kvCache?: 'f32' | 'f16' | 'q8'; maxSeqLen?: number; capacity?: number
  overflow?: 'error' | 'sinks'; sinkTokens?: number; ropePositions?: 'slot' | 'absolute'
  q8Block?: number   // q8 scale block: 32 (default, copy_kv8.wgsl) or headDim (one scale per row)
}
export declare class KvCache {
  constructor(opts: KvCacheOptions)
  readonly capacity: number
  dispose(): void
  ensureKvCapacity(needed: number, stream?: DevPtr | null): void
  setRollTables(cosDev: DevPtr, sinDev: DevPtr, positions: number): void
  appendKV(srcDev: DevPtr, which: 0 | 1, li: number, rows: number, dstRow0: number, stream?: DevPtr | null): void
  prologue(a: { li: number; q?: DevPtr | null; qStride?: number; k?: DevPtr | null; v?: DevPtr | null; S: number; H: number
    qGamma?: DevPtr | null; kGamma?: DevPtr | null; eps: number; cos: DevPtr; sin: DevPtr; ropePositions: number
    rotDim: number; pos0: number; slot0: number; qOut?: DevPtr | null; stream?: DevPtr | null }): void
  att(qr: DevPtr, li: number, S: number, H: number, posBase: number, out: DevPtr,
    o?: { scale?: number; gate?: DevPtr | null; gateStride?: number; stream?: DevPtr | null }): void
  evict(fill: number, need: number): number
  evictFor(fill: number, n: number): number
  readonly ringState: [number, number]   // sink mode: [ring origin, rows evicted so far]
  ringReset(evicted?: number): void      // compacted ring, the state a v2 snapshot restores into
  exportRows(li: number, region: 0 | 1 | 2 | 3, base: number, count: number): ArrayBuffer
  importRows(li: number, region: 0 | 1 | 2 | 3, base: number, count: number, buf: ArrayBuffer): void
  qkvProjPrologue(o: { li: number; x: DevPtr; w: OneBitWeight; H: number; qGamma: DevPtr; kGamma: DevPtr; eps: number;
    cos: DevPtr; sin: DevPtr; ropePositions: number; rotDim: number; pos: number; slot?: number; qOut: DevPtr;
    stream?: DevPtr | null }): void
}
// a 1-bit weight as the engine uploads it (GpuWeight, src/engine.ts:814-830)
export interface OneBitWeight { sign: DevPtr; scales: DevPtr; K: number; N0: number; N1?: number; N2?: number; N?: number }
export declare function fusedMM(w: OneBitWeight, x: DevPtr, outs: (DevPtr | null)[], stream?: DevPtr | null): void
export declare function residMM(w: OneBitWeight, x: DevPtr, resid: DevPtr, out: DevPtr, stream?: DevPtr | null): void
// raw addon: streams (default priority) and event timing, for hosts without a GPU runtime
export declare const addon: {
  streamCreate(): DevPtr; streamDestroy(stream: DevPtr): void
  eventCreate(): DevPtr; eventRecord(event: DevPtr, stream: DevPtr | null): void
  eventElapsedUs(start: DevPtr, end: DevPtr): number; eventDestroy(event: DevPtr): void
  [name: string]: any
}
