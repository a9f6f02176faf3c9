"""Write the committed golden fixtures under tests/golden/ (small .npz files, no pickles).

    python tests/golden/make_golden.py

Fixtures:
* ref_kernel_cases.npz -- the reference's own per-kernel cases (tools/gen-kernel-cases.py):
  its `rope_partial` (S=5, H=3, D=256, ROT=64, theta 1e7) and `attention` (S=6, H=4, KV=2,
  D=256, causal) cases. Their inputs come from `np.random.seed(0)` and the exact sequence of
  `np.random.randn` draws that script makes (lines 21, 43-45, 52-56, 70-72, 79-83, 94, 103-105,
  restated here as shapes only -- the reference script is not imported or run). Expected
  outputs follow the script's own numpy lines (rope: tools/qwen35_numpy.py:84-89; attention:
  tools/gen-kernel-cases.py:106-113), restated below. The reference's pass bar for them is
  max|delta| < 2e-3 and cosine > 0.99999 (scripts/verify-kernels.mjs:104).
* c1_decode.npz -- config C1: Q, digests of the seeded K/V, and the oracle output.
* q8_cases.npz / f16_cases.npz -- quantizer special cases with expected codes/scales/bits.
* sink_schedule.npz -- the resident set (absolute positions per slot) of a 4+4096 window after
  a greedy decode to position 100000, from the literal eviction simulation.
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from bitgpu_amd import workloads as W  # noqa: E402
from oracle import ref  # noqa: E402


def reference_kernel_case_inputs():
    """The draw sequence of tools/gen-kernel-cases.py under np.random.seed(0)."""
    np.random.seed(0)
    r = np.random.randn
    r(16, 512); r(512, 1, 4)                        # conv1d x, wc (lines 43-44)
    r(8, 2, 128); r(8, 2, 128); r(8, 4, 128)        # deltanet qa, ka, va (52-54)
    r(8, 4); r(8, 4)                                # ga, ba (55-56)
    r(32, 128); r(32, 128); r(128)                  # norm_gate core, zg, gam (70-72)
    r(8, 4); r(8, 4); r(4); r(4)                    # gbeta ag, bg, alog, dtb (79-82)
    xr = r(5, 3, 256).astype(np.float32)            # rope_partial x (94)
    qa2 = r(6, 4, 256).astype(np.float32)           # attention q, k, v (103-105)
    ka2 = r(6, 2, 256).astype(np.float32)
    va2 = r(6, 2, 256).astype(np.float32)
    return xr, qa2, ka2, va2


def ref_kernel_cases():
    xr, qa2, ka2, va2 = reference_kernel_case_inputs()
    # rope_partial: tables of gen-kernel-cases.py:95-97 (positions 0..4, rot 64, theta 1e7)
    inv = 1.0 / (1e7 ** (np.arange(0, 64, 2, dtype=np.float64) / 64))
    emb = np.concatenate([np.outer(np.arange(5), inv)] * 2, -1)
    cosr, sinr = np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)
    rope_exp = ref.rope_apply(xr, cosr[:, :32], sinr[:, :32], np.arange(5), rot=64)
    # attention: f32 scores @ scale(f64) + causal, softmax, @ v (gen-kernel-cases.py:106-113)
    att_exp = ref.attention(qa2, ka2, va2, 0, scale=1.0 / np.sqrt(256))
    return dict(rope_x=xr, rope_cos=cosr, rope_sin=sinr, rope_expected=rope_exp,
                att_q=qa2, att_k=ka2, att_v=va2, att_expected=att_exp)


def c1_decode():
    cfg = W.C1
    q, k, v, _ = W.decode_inputs(cfg, W.C1_PAST, seed=1)
    L = W.C1_PAST + 1
    cos, sin = ref.rope_tables(cfg.theta, cfg.rot, L)
    ones = np.ones(cfg.D, np.float32)
    qr = ref.norm_rope(q, ones, cfg.eps, cos, sin, [W.C1_PAST])
    kr = ref.norm_rope(k, ones, cfg.eps, cos, sin, np.arange(L))
    out = ref.attention(qr, kr, v, W.C1_PAST)
    # K/V are regenerated from the seed by the tests; the fixture pins them by digest
    return dict(q=q, k_sha256=np.frombuffer(hashlib.sha256(k.tobytes()).digest(), np.uint8),
                v_sha256=np.frombuffer(hashlib.sha256(v.tobytes()).digest(), np.uint8), expected=out)


def q8_cases():
    rng = np.random.default_rng(7)
    rows = [np.zeros(128, np.float32),                                   # all-zero block -> codes 0, scale 1e-30
            -np.zeros(128, np.float32),                                  # negative zero
            rng.standard_normal(128).astype(np.float32),
            (rng.standard_normal(128) * 1e-3).astype(np.float32),
            (rng.standard_normal(128) * 1e4).astype(np.float32),
            np.linspace(-1, 1, 128).astype(np.float32),
            # a block whose max is 127 and whose other values are exact half-steps x.5:
            # 127 * (v / 127) + 0.5 lands exactly on an integer + 0.5 + 0.5 -> floor rounds up
            np.concatenate([np.full(1, 127.0), np.arange(-15.5, 15.5, 1.0), np.full(96, 3.0)]).astype(np.float32)]
    x = np.stack(rows)
    codes, scales = ref.q8_pack(x)
    return dict(x=x, codes=codes, scales=scales, dequant=ref.q8_dequant(codes, scales))


def f16_cases():
    rng = np.random.default_rng(8)
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 1e-8, 6.1e-5, 5.96e-8, 2.98e-8,
                        1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 3.14159265], np.float32)
    x = np.concatenate([special, rng.standard_normal(243).astype(np.float32)])
    return dict(x=x, bits=ref.f16_pack(x).view(np.uint16))


def sink_schedule():
    cfg = W.C4
    slots, fill, events = ref.simulate_sink_schedule(prompt_len=1000, target_abs=W.C4_POSITION,
                                                     sinks=cfg.sinks, max_seq=cfg.sinks + cfg.window)
    ev = np.array(events, np.int64).reshape(-1, 3)
    return dict(slots=np.array(slots, np.int64), fill=np.int64(fill), events=ev)


def main():
    out = {
        "ref_kernel_cases.npz": ref_kernel_cases(),
        "c1_decode.npz": c1_decode(),
        "q8_cases.npz": q8_cases(),
        "f16_cases.npz": f16_cases(),
        "sink_schedule.npz": sink_schedule(),
    }
    for name, arrs in out.items():
        np.savez_compressed(os.path.join(HERE, name), **arrs)
        print("wrote", name, {k: v.shape for k, v in arrs.items()})


if __name__ == "__main__":
    main()
