#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (BASELINE.json metric).

Headline (`value`): decode attention over a q8 KV cache at 32k context in the Qwen3-8B/4B
attention shape (32 query heads, 8 KV heads, head_dim 128), swept over 36 distinct layers
(config C3), as HBM GB/s of algorithmic bytes; `us_per_layer` is the same measurement as time.
One "step" = one decode token's attention over all 36 layers (36 kernel launches, replayed as a
HIP graph; the cache is resident in HBM before the timed region). Also reported: the 4k/16k
sweeps, C2 causal prefill TFLOP/s, C1 f32 decode, C4 sink-mode decode/verify, C5 hybrid
prefill + decode, and the oracle numpy path timed on this host's cores.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--quick]

Only one GPU is used: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2516.6  # MI355X dense fp16/bf16 MFMA
F32_PEAK_TFLOPS = 157.3        # MI355X fp32 (matrix and vector)


def c3_bytes(L, KV=8, D=128, H=32):
    """Algorithmic bytes of one decode-attention layer over a q8 cache: K and V codes plus one
    f32 scale per 32 values, and the f32 query and output."""
    return L * KV * 2 * (D + 4 * D // 32) + 2 * H * D * 4


def causal_flops(S, H, D, past=0):
    """QK^T and PV FLOPs of a causal prefill: 2 * 2 * D * H * sum_s (past + s + 1)."""
    return 2 * 2 * D * H * (S * past + S * (S + 1) // 2)


def graph_replay_us(torch, fn, steps, warmup, per_graph=1):
    """Capture fn() `per_graph` times back to back into one HIP graph; replay warmup times
    untimed, then time `steps` replays bracketed by synchronize. Returns microseconds per fn()
    (a graph that holds a single short launch would also time the graph launch itself)."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for _ in range(per_graph):
                fn()
    torch.cuda.synchronize()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (steps * per_graph)


class DecodeSweep:
    """36 distinct q8 layer caches at context L, filled through the fused prologue."""

    def __init__(self, torch, E, W, L, layers=36, seed=3):
        cfg = W.C3
        self.L, self.layers, self.cfg = L, layers, cfg
        q, k, v = W.draw(seed, (1, cfg.H, cfg.D), (L, cfg.KV, cfg.D), (L, cfg.KV, cfg.D))
        self.q_host, self.k_host, self.v_host = q, k, v
        dev = "cuda"
        self.cos, self.sin = (torch.from_numpy(x).to(dev) for x in E.rope_tables(cfg.theta, cfg.rot, L))
        self.ones = torch.ones(cfg.D, device=dev)
        self.cache = E.KvCache(layers, cfg.KV, cfg.D, cfg.kv, max_seq_len=L, capacity=L)
        kt = torch.from_numpy(k).to(dev)
        vt = torch.from_numpy(v).to(dev)
        qt = torch.from_numpy(q).to(dev)
        for li in range(layers):
            E.qkv_prologue(self.cache, li, None, kt[: L - 1], vt[: L - 1], L - 1, cfg.H, None, self.ones, cfg.eps,
                           self.cos, self.sin, cfg.rot, 0, 0)
        self.qt, self.kt, self.vt = qt, kt[L - 1:].contiguous(), vt[L - 1:].contiguous()
        self.qr = torch.empty(1, cfg.H, cfg.D, device=dev)
        self.out = torch.empty(1, cfg.H, cfg.D, device=dev)
        self.E = E
        for li in range(layers):
            self.prologue(li)
        self.cache_attn_reserve()

    def cache_attn_reserve(self):
        from bitgpu_amd._lib import check, lib
        check(lib().bg_attention_reserve(self.cache.handle, 1, self.cfg.H))

    def prologue(self, li):
        cfg = self.cfg
        self.E.qkv_prologue(self.cache, li, self.qt, self.kt, self.vt, 1, cfg.H, self.ones, self.ones, cfg.eps,
                            self.cos, self.sin, cfg.rot, self.L - 1, self.L - 1, q_out=self.qr)

    def attention(self, li):
        self.E.attention(self.cache, li, self.qr, 1, self.cfg.H, self.L - 1, out=self.out)

    def sweep(self):
        for li in range(self.layers):
            self.attention(li)

    def full_step(self):
        for li in range(self.layers):
            self.prologue(li)
            self.attention(li)

    def close(self):
        self.cache.close()


def blas_info():
    """numpy's BLAS (numpy.show_config) and the thread settings it runs with."""
    info = {}
    try:
        cfgd = np.show_config(mode="dicts")
        b = cfgd.get("Build Dependencies", {}).get("blas", {})
        info = {"name": b.get("name"), "version": b.get("version"), "config": b.get("openblas configuration")}
    except Exception as e:  # noqa: BLE001 - a report, not a requirement
        info = {"error": str(e)}
    try:
        import threadpoolctl
        info["threadpools"] = [{"api": t.get("user_api"), "lib": t.get("internal_api"), "threads": t.get("num_threads")}
                               for t in threadpoolctl.threadpool_info()]
    except Exception:  # noqa: BLE001
        pass
    info["env"] = {k: os.environ[k] for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")
                   if k in os.environ}
    return info


def _best(fn, budget_s, reps=5):
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= reps:
            break
    return min(times), len(times)


def cpu_prefill_samples(W, budget_s=4.0):
    """The oracle's causal prefill attention for C2 (f16) and C5 (q8, gated) on a bounded sample
    of query rows (64-row blocks at four depths, tools/reference.py:158-175 and
    tools/qwen35_numpy.py:102-114 restated); the rate in FLOP/s over the sample's causal pairs
    gives the full prefill's time."""
    from oracle import ref
    out = {}
    for name, cfg, S in (("c2_prefill_f16", W.C2, W.C2_S), ("c5_prefill_q8", W.C5, W.C5_PREFILL)):
        q, k, v, g = W.prefill_inputs(cfg, S, 2)
        kk = ref.kv_roundtrip(k, cfg.kv)
        vv = ref.kv_roundtrip(v, cfg.kv)
        blocks = [int(f * S) - 64 if f == 1.0 else int(f * S) for f in (0.25, 0.5, 0.75, 1.0)]
        scale = 1.0 / np.sqrt(cfg.D) if cfg.gate else None

        def run():
            for r0 in blocks:
                rows = slice(r0, r0 + 64)
                if cfg.gate:
                    ref.gated_attention(q[rows], kk[:r0 + 64], vv[:r0 + 64], g[rows], r0)
                else:
                    ref.attention(q[rows], kk[:r0 + 64], vv[:r0 + 64], r0, scale=scale)
        best, n = _best(run, budget_s, reps=3)
        fl = sum(causal_flops(64, cfg.H, cfg.D, past=r0) for r0 in blocks)
        rate = fl / best
        out[name] = {"tflops": round(rate / 1e12, 4), "us_full_estimate": round(causal_flops(S, cfg.H, cfg.D) / rate * 1e6, 1),
                     "sample": f"4 blocks of 64 query rows at depths {blocks} of the S={S} prefill, best of {n}"}
    return out


def cpu_baseline(sweep, W, budget_s=12.0):
    """The oracle numpy path (tools/reference.py:158-175 restated, q8 dequant first) on this
    host's cores, one layer of the headline workload per repetition; best of the repetitions
    that fit the time budget."""
    from oracle import ref
    cfg = W.C3
    L = sweep.L
    cos, sin = ref.rope_tables(cfg.theta, cfg.rot, L)
    ones = np.ones(cfg.D, np.float32)
    kr = ref.norm_rope(sweep.k_host, ones, cfg.eps, cos, sin, np.arange(L))
    kc, ks = ref.q8_pack(kr)
    vc, vs = ref.q8_pack(sweep.v_host)
    qr = ref.norm_rope(sweep.q_host, ones, cfg.eps, cos, sin, [L - 1])
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        kk = ref.q8_dequant(kc, ks)
        vv = ref.q8_dequant(vc, vs)
        ref.attention(qr, kk, vv, L - 1)
        times.append(time.perf_counter() - t0)
        if len(times) >= 5:
            break
    best = min(times)
    cores = os.cpu_count()
    blas = blas_info()
    threads = max([t.get("threads") or 0 for t in blas.get("threadpools", [])] or [cores])
    return {
        "value": round(c3_bytes(L) / best / 1e9, 3),
        "unit": "GB/s",
        "us_per_layer": round(best * 1e6, 1),
        "cores": threads,
        "kind": "port",
        "sample": f"one layer of the C3 32k q8 decode (numpy oracle: q8 dequant + GQA softmax attention in "
                  f"float64), best of {len(times)}; {threads} BLAS threads on {cores} host cores",
        "blas": blas,
        "prefill": cpu_prefill_samples(W),
    }


def prologue_bytes(cfg, S):
    """HBM bytes of the fused prologue for S positions: Q read (the query half of each row) and
    written as f32, K and V read as f32 and written in the storage format (+ q8 scales)."""
    eb = {"f32": 4, "f16": 2, "q8": 1}[cfg.kv]
    sc = 2 * S * cfg.KV * (cfg.D // 32) * 4 if cfg.kv == "q8" else 0
    return 2 * S * cfg.H * cfg.D * 4 + 2 * S * cfg.KV * cfg.D * 4 + 2 * S * cfg.KV * cfg.D * eb + sc


def bench_prefill(torch, E, W, cfg, S, steps, warmup, seed):
    q, k, v, g = W.prefill_inputs(cfg, S, seed)
    dev = "cuda"
    c = E.KvCache(1, cfg.KV, cfg.D, cfg.kv, max_seq_len=S, capacity=S)
    cos, sin = (torch.from_numpy(x).to(dev) for x in E.rope_tables(cfg.theta, cfg.rot, S))
    ones = torch.ones(cfg.D, device=dev)
    qt, kt, vt = (torch.from_numpy(x).to(dev) for x in (q, k, v))
    gt = torch.from_numpy(g).to(dev) if g is not None else None
    qr = torch.empty(S, cfg.H, cfg.D, device=dev)
    out = torch.empty(S, cfg.H, cfg.D, device=dev)
    scale = float(1.0 / np.sqrt(cfg.D))

    def prologue():
        E.qkv_prologue(c, 0, qt, kt, vt, S, cfg.H, ones, ones, cfg.eps, cos, sin, cfg.rot, 0, 0, q_out=qr)

    def attn():
        E.attention(c, 0, qr, S, cfg.H, 0, scale=scale, gate=gt, gate_stride=cfg.D if gt is not None else None,
                    out=out)

    prologue()
    # several launches per graph, as in a multi-layer prefill (one launch per layer)
    per_graph = 8 if S <= 4096 else 2
    us_attn = graph_replay_us(torch, attn, steps, warmup, per_graph)
    us_pro = graph_replay_us(torch, prologue, steps, warmup, per_graph)
    fl = causal_flops(S, cfg.H, cfg.D)
    c.close()
    pb = prologue_bytes(cfg, S)
    return {"S": S, "attn_us": round(us_attn, 1), "prologue_us": round(us_pro, 1),
            "tflops": round(fl / us_attn / 1e6, 1), "mfma_frac": round(fl / us_attn / 1e6 / MFMA_F16_PEAK_TFLOPS, 4),
            "prologue_bytes": pb, "prologue_GBs": round(pb / us_pro / 1e3, 1),
            "prologue_hbm_frac": round(pb / us_pro / 1e3 / HBM_PEAK_GBS, 4)}


def make_prologue(torch, E, W, cfg, S, seed=2):
    """The fused prologue of an S-token prefill (Q, K, V) into a fresh cache; (launch, close)."""
    q, k, v, _ = W.prefill_inputs(cfg, S, seed)
    dev = "cuda"
    c = E.KvCache(1, cfg.KV, cfg.D, cfg.kv, max_seq_len=S, capacity=S)
    cos, sin = (torch.from_numpy(x).to(dev) for x in E.rope_tables(cfg.theta, cfg.rot, S))
    ones = torch.ones(cfg.D, device=dev)
    qt, kt, vt = (torch.from_numpy(x).to(dev) for x in (q, k, v))
    qr = torch.empty(S, cfg.H, cfg.D, device=dev)
    return (lambda: E.qkv_prologue(c, 0, qt, kt, vt, S, cfg.H, ones, ones, cfg.eps, cos, sin, cfg.rot, 0, 0,
                                   q_out=qr)), c.close


def profile_set(torch, E, W, names, n):
    """Launch the named kernels n times each with nothing else on the GPU (rocprofv3 --pmc passes)."""
    for name in names:
        if name == "decode_c5":
            fn, _, _, close = make_c5_decode(torch, E, W)
        elif name in ("decode_c4", "verify_c4"):
            fn, _, _, close = make_c4(torch, E, W, 1 if name == "decode_c4" else W.C4_VERIFY)
        elif name == "prologue_c2":
            fn, close = make_prologue(torch, E, W, W.C2, W.C2_S)
        elif name == "prologue_c5":
            fn, close = make_prologue(torch, E, W, W.C5, W.C5_PREFILL)
        elif name == "proj":
            run_q, run_o, close, _, _ = make_projections(torch, E)
            fn = lambda: (run_q(), run_o())
        else:
            raise SystemExit(f"bench.py: unknown --profile-set entry {name}")
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        close()


def profile_prefill(torch, E, W, n):
    """C2 (f16, S=2048) and C5 (q8, S=8192) prefill attention, n plain launches each, for
    rocprofv3 --pmc counter passes (MFMA busy cycles, MFMA ops, LDS activity)."""
    dev = "cuda"
    for cfg, S in ((W.C2, W.C2_S), (W.C5, W.C5_PREFILL)):
        q, k, v, g = W.prefill_inputs(cfg, S, 2)
        c = E.KvCache(1, cfg.KV, cfg.D, cfg.kv, max_seq_len=S, capacity=S)
        cos, sin = (torch.from_numpy(x).to(dev) for x in E.rope_tables(cfg.theta, cfg.rot, S))
        ones = torch.ones(cfg.D, device=dev)
        qt, kt, vt = (torch.from_numpy(x).to(dev) for x in (q, k, v))
        gt = torch.from_numpy(g).to(dev) if g is not None else None
        qr = torch.empty(S, cfg.H, cfg.D, device=dev)
        out = torch.empty(S, cfg.H, cfg.D, device=dev)
        E.qkv_prologue(c, 0, qt, kt, vt, S, cfg.H, ones, ones, cfg.eps, cos, sin, cfg.rot, 0, 0, q_out=qr)
        for _ in range(n):
            E.attention(c, 0, qr, S, cfg.H, 0, scale=float(1.0 / np.sqrt(cfg.D)), gate=gt,
                        gate_stride=cfg.D if gt is not None else None, out=out)
        torch.cuda.synchronize()
        c.close()


def bench_c1(torch, E, W, steps, warmup):
    cfg = W.C1
    q, k, v, _ = W.decode_inputs(cfg, W.C1_PAST, seed=1)
    dev = "cuda"
    L = W.C1_PAST + 1
    c = E.KvCache(28, cfg.KV, cfg.D, cfg.kv, max_seq_len=2048)
    c.ensure_capacity(L)
    cos, sin = (torch.from_numpy(x).to(dev) for x in E.rope_tables(cfg.theta, cfg.rot, 2048))
    ones = torch.ones(cfg.D, device=dev)
    kt, vt, qt = (torch.from_numpy(x).to(dev) for x in (k, v, q))
    for li in range(28):
        E.qkv_prologue(c, li, None, kt[:L], vt[:L], L, cfg.H, None, ones, cfg.eps, cos, sin, cfg.rot, 0, 0)
    qr = E.qkv_prologue(c, 0, qt, None, None, 1, cfg.H, ones, None, cfg.eps, cos, sin, cfg.rot, W.C1_PAST, W.C1_PAST)
    out = torch.empty(1, cfg.H, cfg.D, device=dev)
    us = graph_replay_us(torch, lambda: [E.attention(c, li, qr, 1, cfg.H, W.C1_PAST, out=out) for li in range(28)],
                         steps, warmup) / 28
    c.close()
    B = L * cfg.KV * 2 * cfg.D * 4 + 2 * cfg.H * cfg.D * 4
    return {"us_per_layer": round(us, 2), "GBs": round(B / us / 1e3, 1), "layers": 28}


def make_c4(torch, E, W, verify):
    """Sink mode at position 100000: the ring state after the reference's greedy eviction
    schedule (index arithmetic only), f16 cache, 4 sinks + 4096 window; `verify` query rows.
    Returns (launch, algorithmic bytes, resident slots, close)."""
    cfg = W.C4
    sinks, max_seq = cfg.sinks, cfg.sinks + cfg.window
    dev = "cuda"
    c = E.KvCache(1, cfg.KV, cfg.D, cfg.kv, max_seq_len=max_seq, overflow="sinks", sink_tokens=sinks)
    fill, fed = 1000, 1000
    while fed < W.C4_POSITION:
        batch = min(4, W.C4_POSITION - fed)
        fill = c.evict_for(fill, batch) + batch
        fed += batch
    fill = c.evict_for(fill, verify)
    cos, sin = (torch.from_numpy(x).to(dev) for x in E.rope_tables(cfg.theta, cfg.rot, max_seq))
    c.set_rope(cos, sin)
    rng = np.random.default_rng(4)
    k = torch.from_numpy(rng.standard_normal((fill + verify, cfg.KV, cfg.D)).astype(np.float32)).to(dev)
    v = torch.from_numpy(rng.standard_normal((fill + verify, cfg.KV, cfg.D)).astype(np.float32)).to(dev)
    q = torch.from_numpy(rng.standard_normal((verify, cfg.H, cfg.D)).astype(np.float32)).to(dev)
    ones = torch.ones(cfg.D, device=dev)
    E.qkv_prologue(c, 0, None, k, v, fill + verify, cfg.H, None, ones, cfg.eps, cos, sin, cfg.rot, 0, 0)
    qr = E.qkv_prologue(c, 0, q, None, None, verify, cfg.H, ones, None, cfg.eps, cos, sin, cfg.rot, fill, fill)
    out = torch.empty(verify, cfg.H, cfg.D, device=dev)
    B = (fill + verify) * cfg.KV * 2 * cfg.D * 2 + 2 * verify * cfg.H * cfg.D * 4
    return (lambda: E.attention(c, 0, qr, verify, cfg.H, fill, out=out)), B, fill + verify, c.close


def bench_c4(torch, E, W, steps, warmup):
    res = {}
    for verify in (1, W.C4_VERIFY):
        fn, B, slots, close = make_c4(torch, E, W, verify)
        us = graph_replay_us(torch, fn, steps, warmup, per_graph=16)
        res["decode" if verify == 1 else f"verify{verify}"] = {"us": round(us, 2), "GBs": round(B / us / 1e3, 1),
                                                               "hbm_frac": round(B / us / 1e3 / HBM_PEAK_GBS, 4),
                                                               "resident_slots": slots}
        close()
    return res


def make_c5_decode(torch, E, W, layers=16):
    """C5 decode step at 8193 cached positions over `layers` distinct q8 layers (D=256, gated).
    Returns (launch of every layer, algorithmic bytes per layer, context, close)."""
    cfg = W.C5
    L = W.C5_PREFILL + 1
    dev = "cuda"
    c = E.KvCache(layers, cfg.KV, cfg.D, cfg.kv, max_seq_len=W.C5_PREFILL + W.C5_DECODE_STEPS,
                  capacity=W.C5_PREFILL + W.C5_DECODE_STEPS)
    rng = np.random.default_rng(5)
    k = torch.from_numpy(rng.standard_normal((L, cfg.KV, cfg.D)).astype(np.float32)).to(dev)
    from bitgpu_amd._lib import BG_K, BG_V
    for li in range(layers):
        c.append_kv(k, BG_K, li, L * cfg.KV, 0)
        c.append_kv(k, BG_V, li, L * cfg.KV, 0)
    q = torch.from_numpy(rng.standard_normal((1, cfg.H, cfg.D)).astype(np.float32)).to(dev)
    g = torch.from_numpy(rng.standard_normal((1, cfg.H, cfg.D)).astype(np.float32)).to(dev)
    out = torch.empty(1, cfg.H, cfg.D, device=dev)
    scale = float(1.0 / np.sqrt(cfg.D))
    B = L * cfg.KV * 2 * (cfg.D + 4 * cfg.D // 32) + 3 * cfg.H * cfg.D * 4

    def run():
        for li in range(layers):
            E.attention(c, li, q, 1, cfg.H, L - 1, scale=scale, gate=g, gate_stride=cfg.D, out=out)
    return run, B, L, c.close


def bench_c5_decode(torch, E, W, steps, warmup):
    run, B, L, close = make_c5_decode(torch, E, W)
    us = graph_replay_us(torch, run, steps, warmup) / 16
    close()
    return {"context": L, "us_per_layer": round(us, 2), "GBs": round(B / us / 1e3, 1),
            "hbm_frac": round(B / us / 1e3 / HBM_PEAK_GBS, 4)}


def onebit_bytes(N, K):
    """HBM bytes of one 1-bit GEMV: sign bits, one f32 scale per 128 weights, x and the outputs."""
    return N * K // 8 + N * (K // 128) * 4 + K * 4 + N * 4


def make_projections(torch, E, layers=36, HD=4096, H=32, KV=8, D=128):
    """The decode projections on either side of attention in the Qwen3-8B shape (hidden 4096,
    32 heads on 8 kv heads, head_dim 128), `layers` distinct layers' weights (no cache reuse
    across launches): the fused qkv projection + prologue into a q8 cache, and o_proj +
    residual. Returns (run_qkv, run_o, close, qkv_bytes, o_bytes); each run launches every layer."""
    rng = np.random.default_rng(7)
    dev = "cuda"
    Nq = (H + 2 * KV) * D

    def weight(N, K, N0, N1=0, N2=0):
        sign = torch.from_numpy(rng.integers(0, 2 ** 32, (N, K // 32), dtype=np.uint64).astype(np.uint32).view(np.int32)).to(dev)
        sc = torch.from_numpy((np.abs(rng.standard_normal((N, K // 128))) * 0.02).astype(np.float32)).to(dev)
        return E.OneBitWeight(sign, sc, K, N0, N1, N2)
    wq = [weight(Nq, HD, H * D, KV * D, KV * D) for _ in range(layers)]
    wo = [weight(HD, H * D, HD) for _ in range(layers)]
    c = E.KvCache(layers, KV, D, "q8", max_seq_len=4096, capacity=4096)
    cos, sin = (torch.from_numpy(x).to(dev) for x in E.rope_tables(1e6, D, 4096))
    ones = torch.ones(D, device=dev)
    x = torch.randn(HD, device=dev)
    h = torch.randn(HD, device=dev)
    att = torch.randn(H * D, device=dev)
    q = torch.empty(1, H, D, device=dev)
    y = torch.empty(HD, device=dev)
    run_q = lambda: [E.qkv_proj_prologue(c, li, x, wq[li], H, ones, ones, 1e-6, cos, sin, D, 1000, 1000, q_out=q)
                     for li in range(layers)]
    run_o = lambda: [E.resid_mm(wo[li], att, h, y) for li in range(layers)]
    return run_q, run_o, c.close, onebit_bytes(Nq, HD), onebit_bytes(HD, H * D)


def bench_projections(torch, E, steps, warmup, layers=36):
    """The 1-bit decode projections (make_projections), graph-replayed, per launch."""
    run_q, run_o, close, bq, bo = make_projections(torch, E, layers)
    us_q = graph_replay_us(torch, run_q, steps, warmup) / layers
    us_o = graph_replay_us(torch, run_o, steps, warmup) / layers
    close()
    return {"qkv_proj_prologue": {"us": round(us_q, 2), "GBs": round(bq / us_q / 1e3, 1),
                                  "hbm_frac": round(bq / us_q / 1e3 / HBM_PEAK_GBS, 4), "bytes": bq},
            "o_proj_resid": {"us": round(us_o, 2), "GBs": round(bo / us_o / 1e3, 1),
                             "hbm_frac": round(bo / us_o / 1e3 / HBM_PEAK_GBS, 4), "bytes": bo},
            "shape": f"hidden 4096, 32 heads / 8 kv heads x 128, {layers} distinct layers"}


def bench_read_floor(torch, steps, warmup, layers=36, nbytes=None, grids=(256, 512, 1024, 2048)):
    """The streaming-read floor of the headline's traffic: `layers` distinct buffers of the C3
    32k layer's algorithmic bytes, each read by one bg_diag_stream_read launch (512-thread
    workgroups, one contiguous slice each, 16-byte loads), graph-replayed like the headline
    sweep. Nontemporal loads (the decode tiles' policy) at each grid size; the best grid is
    also timed with plain loads."""
    import ctypes as C
    from bitgpu_amd._lib import check, lib
    nbytes = nbytes or c3_bytes(32768)
    bufs = [torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device="cuda")
            for _ in range(layers)]
    sink = torch.empty(max(grids), dtype=torch.int32, device="cuda")

    def timed(wg, nt):
        def sweep():
            st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
            for b in bufs:
                check(lib().bg_diag_stream_read(C.c_void_p(b.data_ptr()), nbytes, wg, nt, C.c_void_p(sink.data_ptr()),
                                                st))
        return graph_replay_us(torch, sweep, steps, warmup) / layers

    def entry(us):
        return {"us_per_launch": round(us, 2), "GBs": round(nbytes / us / 1e3, 1),
                "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}

    per_grid = {wg: timed(wg, 1) for wg in grids}
    best = min(per_grid, key=per_grid.get)
    out = {"bytes_per_launch": nbytes, "buffers": layers,
           "nontemporal_by_grid": {str(wg): round(us, 2) for wg, us in per_grid.items()},
           "best_grid": best, "nontemporal": entry(per_grid[best]), "plain": entry(timed(best, 0))}
    del bufs
    torch.cuda.empty_cache()
    return out


def load_traffic(name):
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    try:
        with open(p) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--quick", action="store_true", help="headline only (no extras, no CPU baseline)")
    ap.add_argument("--profile-loop", type=int, default=0,
                    help="run only the headline sweep this many times (for rocprofv3 --pmc), print nothing else")
    ap.add_argument("--profile-prefill", type=int, default=0,
                    help="run only the C2 and C5 prefill attention this many times each (for rocprofv3 --pmc)")
    ap.add_argument("--profile-set", default="", metavar="NAMES",
                    help="comma list of decode_c5, decode_c4, verify_c4, prologue_c2, prologue_c5, proj (the 1-bit "
                         "projections, every layer): run only these "
                         "kernels --profile-n times each (for rocprofv3 --pmc), print nothing else")
    ap.add_argument("--profile-n", type=int, default=20)
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--read-floor", action="store_true",
                    help="run only the streaming-read floor of the headline's bytes and print it as JSON")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run only a device-to-device copy of MIB MiB (3 times) to calibrate the "
                         "FETCH_SIZE / WRITE_SIZE counters against known bytes")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py: this build measures one GPU only (asked for {max(args.gpus, world)}); "
              "multi-GPU sharding is a design note, not a benchmark here", file=sys.stderr)
        sys.exit(2)

    import torch
    from bitgpu_amd import engine as E
    from bitgpu_amd import workloads as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)

    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        a = torch.randn(n, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        return

    if args.profile_prefill:
        profile_prefill(torch, E, W, args.profile_prefill)
        return

    if args.read_floor:
        print(json.dumps({"read_floor_c3_32k": bench_read_floor(torch, args.steps, args.warmup)}), flush=True)
        return

    if args.profile_set:
        profile_set(torch, E, W, [x for x in args.profile_set.split(",") if x], args.profile_n)
        return

    L = 32768
    sweep = DecodeSweep(torch, E, W, L)
    if args.profile_loop:
        for _ in range(args.profile_loop):
            sweep.sweep()
        torch.cuda.synchronize()
        sweep.close()
        return

    us_sweep = graph_replay_us(torch, sweep.sweep, args.steps, args.warmup)
    us_layer = us_sweep / sweep.layers
    B = c3_bytes(L)
    gbs = B / us_layer / 1e3
    us_full = graph_replay_us(torch, sweep.full_step, max(3, args.steps // 2), args.warmup)

    extra = {}
    cpu = None
    if not args.quick:
        extra["c3_contexts"] = {}
        for Lx in (4096, 16384):
            sw = DecodeSweep(torch, E, W, Lx)
            u = graph_replay_us(torch, sw.sweep, args.steps, args.warmup) / sw.layers
            extra["c3_contexts"][str(Lx)] = {"us_per_layer": round(u, 2), "GBs": round(c3_bytes(Lx) / u / 1e3, 1),
                                             "hbm_frac": round(c3_bytes(Lx) / u / 1e3 / HBM_PEAK_GBS, 4)}
            sw.close()
        extra["c3_contexts"]["32768"] = {"us_per_layer": round(us_layer, 2), "GBs": round(gbs, 1),
                                         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        extra["c2_prefill_f16"] = bench_prefill(torch, E, W, W.C2, W.C2_S, max(3, args.steps // 2), args.warmup, 2)
        extra["c5_prefill_q8"] = bench_prefill(torch, E, W, W.C5, W.C5_PREFILL, 3, 1, 5)
        # the C2 shape with the reference's default f32 storage, on the f32 matrix cores
        pf32 = bench_prefill(torch, E, W, dataclasses.replace(W.C2, kv="f32"), W.C2_S, max(3, args.steps // 4),
                             args.warmup, 2)
        pf32["fp32_frac"] = round(pf32["tflops"] / F32_PEAK_TFLOPS, 4)
        del pf32["mfma_frac"]
        extra["c2_prefill_f32"] = pf32
        extra["c5_decode_q8"] = bench_c5_decode(torch, E, W, args.steps, args.warmup)
        extra["c1_decode_f32"] = bench_c1(torch, E, W, args.steps, args.warmup)
        extra["c4_sinks_f16"] = bench_c4(torch, E, W, args.steps, args.warmup)
        extra["projections_1bit"] = bench_projections(torch, E, args.steps, args.warmup)
        extra["read_floor_c3_32k"] = bench_read_floor(torch, args.steps, args.warmup)
        cpu = cpu_baseline(sweep, W, args.cpu_budget)
    sweep.close()

    traffic = load_traffic("decode_q8_32k_traffic.json")
    line = {
        "metric": "decode-attn HBM GB/s (Qwen3-8B attention shape, 32k ctx, q8 KV, 36 layers)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_sweep / 1e3, 4),
        "us_per_layer": round(us_layer, 2),
        "tokens_per_s": round(1e6 / us_sweep, 1),
        "step_with_prologue_ms": round(us_full / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8 KV (int8 codes + f32 scales); QK on int8 MFMA (codes x hi/lo int8 query, int32 accumulate), PV on f16 MFMA (f32 accumulate)",
        "data": "synthetic (seeded N(0,1) K/V, RMSNorm+RoPE through the fused prologue)",
        "config": {"workload": "C3 decode attention, 36 distinct layers x 32768 cached positions, batch 1",
                   "heads": 32, "kv_heads": 8, "head_dim": 128, "kv_cache": "q8", "context": L, "layers": 36},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("bytes_per_launch") if traffic else None,
                     "bytes_per_launch_algorithmic": B},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
