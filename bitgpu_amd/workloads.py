"""Synthetic workloads of the benchmark configurations (C1..C5) with seeded inputs.

Inputs follow one recipe: ``numpy.random.default_rng(seed)``, one stream per tensor in the
fixed order Q, K, V, gate, ``standard_normal`` drawn in float64 and cast to float32. Q and K
are the *pre-norm, pre-RoPE* projections (the attention prologue norms and ropes them); V is
used raw (the reference never norms or ropes V, tools/reference.py:162-168). Norm weights are
unit (gamma = 1; for the Qwen3.5 hybrid the baked ``1 + g`` with g = 0).

Only shapes and random numbers live here; no attention arithmetic.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Config:
    name: str
    H: int
    KV: int
    D: int
    kv: str             # storage mode
    theta: float
    rot: int            # rotary dims
    eps: float = 1e-6
    gate: bool = False
    layers: int = 1
    sinks: int = 0
    window: int = 0     # sink mode: max_seq_len = sinks + window


C1 = Config("C1 Qwen3-1.7B decode f32", H=16, KV=8, D=128, kv="f32", theta=1e6, rot=128)
C2 = Config("C2 Qwen3-8B prefill f16", H=32, KV=8, D=128, kv="f16", theta=1e6, rot=128)
C3 = Config("C3 Qwen3-4B decode q8 x36", H=32, KV=8, D=128, kv="q8", theta=1e6, rot=128, layers=36)
C4 = Config("C4 Qwen3-8B sinks f16", H=32, KV=8, D=128, kv="f16", theta=1e6, rot=128, sinks=4, window=4096)
C5 = Config("C5 Qwen3.5 gated hybrid q8", H=24, KV=4, D=256, kv="q8", theta=1e7, rot=64, gate=True)

CONFIGS = {"C1": C1, "C2": C2, "C3": C3, "C4": C4, "C5": C5}

# headline sizes (the benchmark configurations of BASELINE.json)
C1_PAST = 512          # cached positions before the decode step at position 512
C2_S = 2048            # prefill tokens
C3_CONTEXTS = (4096, 16384, 32768)
C4_POSITION = 100_000  # absolute position of the decoded token
C4_VERIFY = 5          # speculative-verify width
C5_PREFILL = 8192
C5_DECODE_STEPS = 256


def draw(seed: int, *shapes):
    """One independent stream per tensor, in the given order (f64 normal -> f32)."""
    out = []
    for i, shp in enumerate(shapes):
        rng = np.random.default_rng([seed, i])
        out.append(rng.standard_normal(shp).astype(np.float32))
    return out


def rows_for_positions(seed: int, positions, heads: int, D: int, tensor: int):
    """Per-position rows drawn from a stream keyed by (seed, tensor, absolute position), so a
    sparse resident set (sink mode) can be filled without drawing every evicted token."""
    out = np.empty((len(positions), heads, D), np.float32)
    for i, p in enumerate(positions):
        out[i] = np.random.default_rng([seed, tensor, int(p)]).standard_normal((heads, D)).astype(np.float32)
    return out


def decode_inputs(cfg: Config, past: int, seed: int = 0, S: int = 1):
    """K/V for positions 0..past+S-1 and Q for the S rows at positions past..past+S-1."""
    L = past + S
    q, k, v = draw(seed, (S, cfg.H, cfg.D), (L, cfg.KV, cfg.D), (L, cfg.KV, cfg.D))
    g = draw(seed + 1, (S, cfg.H, cfg.D))[0] if cfg.gate else None
    return q, k, v, g


def prefill_inputs(cfg: Config, S: int, seed: int = 0):
    q, k, v = draw(seed, (S, cfg.H, cfg.D), (S, cfg.KV, cfg.D), (S, cfg.KV, cfg.D))
    g = draw(seed + 1, (S, cfg.H, cfg.D))[0] if cfg.gate else None
    return q, k, v, g
