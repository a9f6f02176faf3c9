"""GPU: end-to-end parity from the seeded raw inputs at every configuration's full size.

Each test feeds the raw (pre-norm, pre-RoPE) Q/K/V draws of bitgpu_amd.workloads through the
product path exactly as the engine does (fused prologue -> cache -> attention) and checks three
things against the oracle run on the same raw draws:

* the prologue's normed/roped queries, every row (f32, rtol/atol 4e-6: the kernel reduces the
  sum of squares in another order than numpy);
* the stored keys and values, every row: f32 to 4e-6; f16 within one f16 rounding of the oracle's
  f32 value plus 4e-6 (at most 1e-3 of the values may land on the other side of a rounding
  boundary); q8 codes within one step of ``ref.q8_pack`` of the oracle's keys (again at most
  1e-3 of them) and scales to 4e-6; V (never transformed) bit-exact;
* the attention output against ``ref.attention`` / ``ref.gated_attention`` over the oracle's own
  stored values (``kv_roundtrip``): max-abs 1e-4 for f32, relative 2e-3 and cosine > 0.99999 for
  f16 / q8 (the benchmark's stated tolerances).

Configurations: C2 (S=2048 prefill, positions to 2047), C3 (32k decode, positions to 32767),
C4 (sinks at absolute position 100000, slot and absolute RoPE, decode, 5-row verify and a
256-row prefill segment after the ring wrapped, f16 / q8 / f32), C5 (the hybrid layer as the
engine binds it: query and gate interleaved in q_proj at stride 2*head_dim, 8192-row prefill,
then 256 decode steps through the S=1 prologue), and the sink-mode prompt before any wrap.
"""
import os

import numpy as np
import pytest
import torch

from bitgpu_amd import engine as E
from bitgpu_amd import workloads as W
from oracle import ref
from tests.conftest import cosine, rel_err
from tests.gpu_helpers import export_k_v, rope_dev, t

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
F32_RTOL = F32_ATOL = 4e-6
MISMATCH_FRAC = 1e-3


def _check_q(qr_dev, qn):
    got = qr_dev.cpu().numpy() if torch.is_tensor(qr_dev) else qr_dev
    assert got.shape == qn.shape
    assert np.allclose(got, qn, rtol=F32_RTOL, atol=F32_ATOL), float(np.abs(got - qn).max())


def _check_stored(cache, li, base, kn, v_raw):
    """Stored K/V of logical slots [base, base + len(kn)) against the oracle's f32 keys kn and
    the raw values v_raw. Returns what the kernels read back (f32) for the oracle attention."""
    n = kn.shape[0]
    kq, vq, ks, vs = export_k_v(cache, li, base, n)
    dt = cache.kv_cache
    if dt == "f32":
        assert np.allclose(kq, kn, rtol=F32_RTOL, atol=F32_ATOL)
        assert np.array_equal(vq, v_raw)
        return ref.kv_roundtrip(kn, "f32"), ref.kv_roundtrip(v_raw, "f32")
    if dt == "f16":
        want = ref.f16_pack(kn)
        diff = kq.view(np.uint16) != want.view(np.uint16)
        assert diff.mean() <= MISMATCH_FRAC, diff.mean()
        # a mismatch is the other side of a rounding boundary: the stored value is within one
        # f16 rounding (half an ulp, 2^-11 relative) of the oracle's f32 key plus the f32 noise
        # of the norm/rope (absolute, where the rotation cancels to a tiny value)
        assert np.all(np.abs(kq.astype(np.float32) - kn) <= np.abs(kn) * 2.0 ** -11 + F32_ATOL)
        assert np.array_equal(vq.view(np.uint16), ref.f16_pack(v_raw).view(np.uint16))
    else:
        ck, sk = ref.q8_pack(kn)
        d = np.abs(kq.astype(np.int32) - ck.astype(np.int32))
        assert d.max() <= 1 and (d != 0).mean() <= MISMATCH_FRAC, ((d != 0).mean(), d.max())
        assert np.allclose(ks, sk, rtol=F32_RTOL, atol=0)
        cv, sv = ref.q8_pack(v_raw)
        assert np.array_equal(vq, cv) and np.array_equal(vs.view(np.uint32), sv.view(np.uint32))
    return ref.kv_roundtrip(kn, dt), ref.kv_roundtrip(v_raw, dt)


def _check_out(dtype, out, exp):
    assert np.isfinite(out).all()
    if dtype == "f32":
        assert np.abs(out - exp).max() <= 1e-4
    else:
        assert rel_err(out, exp) <= 2e-3 and cosine(out, exp) > 0.99999, (rel_err(out, exp), cosine(out, exp))


def _oracle_tables(cfg, n):
    return ref.rope_tables(cfg.theta, cfg.rot, n)


# ------------------------------------------------------------------ C2: f16 prefill, S = 2048
def test_e2e_c2_prefill(dev):
    cfg, S = W.C2, W.C2_S
    q, k, v, _ = W.prefill_inputs(cfg, S, seed=2)
    cos_d, sin_d, _, _ = rope_dev(cfg.theta, cfg.rot, S)
    ones = t(np.ones(cfg.D, np.float32))
    c = E.KvCache(1, cfg.KV, cfg.D, cfg.kv, max_seq_len=S, capacity=S)
    qr = E.qkv_prologue(c, 0, t(q), t(k), t(v), S, cfg.H, ones, ones, cfg.eps, cos_d, sin_d, cfg.rot, 0, 0)
    out = E.attention(c, 0, qr, S, cfg.H, 0)
    torch.cuda.synchronize()
    cos, sin = _oracle_tables(cfg, S)
    onesh = np.ones(cfg.D, np.float32)
    qn = ref.norm_rope(q, onesh, cfg.eps, cos, sin, np.arange(S))
    kn = ref.norm_rope(k, onesh, cfg.eps, cos, sin, np.arange(S))
    _check_q(qr, qn)
    kk, vv = _check_stored(c, 0, 0, kn, v)
    _check_out("f16", out.cpu().numpy(), ref.attention(qn, kk, vv, 0))
    c.close()


# ------------------------------------------------------------------ C2 shape with f32 storage
def test_e2e_c2_prefill_f32(dev):
    """The C2 prefill (S=2048, H32/KV8/D128) with the reference's default f32 storage: the f32
    matrix-core prefill against the oracle at max-abs 1e-4."""
    cfg, S = W.C2, W.C2_S
    q, k, v, _ = W.prefill_inputs(cfg, S, seed=12)
    cos_d, sin_d, _, _ = rope_dev(cfg.theta, cfg.rot, S)
    ones = t(np.ones(cfg.D, np.float32))
    c = E.KvCache(1, cfg.KV, cfg.D, "f32", max_seq_len=S, capacity=S)
    qr = E.qkv_prologue(c, 0, t(q), t(k), t(v), S, cfg.H, ones, ones, cfg.eps, cos_d, sin_d, cfg.rot, 0, 0)
    out = E.attention(c, 0, qr, S, cfg.H, 0)
    torch.cuda.synchronize()
    cos, sin = _oracle_tables(cfg, S)
    onesh = np.ones(cfg.D, np.float32)
    qn = ref.norm_rope(q, onesh, cfg.eps, cos, sin, np.arange(S))
    kn = ref.norm_rope(k, onesh, cfg.eps, cos, sin, np.arange(S))
    _check_q(qr, qn)
    kk, vv = _check_stored(c, 0, 0, kn, v)
    _check_out("f32", out.cpu().numpy(), ref.attention(qn, kk, vv, 0))
    c.close()


# ------------------------------------------------------------------ C3: q8 decode at 4k/16k/32k
@pytest.mark.parametrize("L", W.C3_CONTEXTS)
def test_e2e_c3_decode(dev, L):
    cfg = W.C3
    q, k, v, _ = W.decode_inputs(cfg, L - 1, seed=3)
    cos_d, sin_d, _, _ = rope_dev(cfg.theta, cfg.rot, L)
    ones = t(np.ones(cfg.D, np.float32))
    c = E.KvCache(2, cfg.KV, cfg.D, cfg.kv, max_seq_len=L, capacity=L)
    li = 1
    E.qkv_prologue(c, li, None, t(k[:L - 1]), t(v[:L - 1]), L - 1, cfg.H, None, ones, cfg.eps, cos_d, sin_d, cfg.rot,
                   0, 0)
    qr = E.qkv_prologue(c, li, t(q), t(k[L - 1:]), t(v[L - 1:]), 1, cfg.H, ones, ones, cfg.eps, cos_d, sin_d,
                        cfg.rot, L - 1, L - 1)
    out = E.attention(c, li, qr, 1, cfg.H, L - 1)
    torch.cuda.synchronize()
    cos, sin = _oracle_tables(cfg, L)
    onesh = np.ones(cfg.D, np.float32)
    qn = ref.norm_rope(q, onesh, cfg.eps, cos, sin, [L - 1])
    kn = ref.norm_rope(k, onesh, cfg.eps, cos, sin, np.arange(L))
    _check_q(qr, qn)
    kk, vv = _check_stored(c, li, 0, kn, v)
    _check_out("q8", out.cpu().numpy(), ref.attention(qn, kk, vv, L - 1))
    c.close()


# ------------------------------------------------------------------ C5: the hybrid layer as bound
def test_e2e_c5_hybrid_prefill_then_256_decode_steps(dev):
    """hybrid_full_attention (src/engine.ts:1465-1493): q_proj rows [H, 2D] hold query | gate
    per head (split_head.wgsl:12-15), partial RoPE on 64 dims with theta 1e7, scale
    1/sqrt(256), gate 1/(1+exp(-g)). 8192-row prefill, then 256 decode steps, each through the
    S=1 prologue at position 8192 + t, continuing the same q8 cache."""
    cfg, S, T = W.C5, W.C5_PREFILL, W.C5_DECODE_STEPS
    N = S + T
    # one seeded stream per tensor (Q, K, V, gate) over all N positions
    q, k, v = W.draw(5, (N, cfg.H, cfg.D), (N, cfg.KV, cfg.D), (N, cfg.KV, cfg.D))
    g = W.draw(6, (N, cfg.H, cfg.D))[0]
    qg = np.concatenate([q, g], -1)                                  # [N, H, 2D] interleaved
    cos_d, sin_d, _, _ = rope_dev(cfg.theta, cfg.rot, N)
    ones = t(np.ones(cfg.D, np.float32))
    c = E.KvCache(1, cfg.KV, cfg.D, cfg.kv, max_seq_len=N, capacity=N)
    qg_d, k_d, v_d = t(qg), t(k), t(v)
    out_p = E.hybrid_full_attention(c, 0, qg_d[:S], k_d[:S], v_d[:S], S, cfg.H, 0, ones, ones, cfg.eps, cos_d, sin_d,
                                    cfg.rot)
    torch.cuda.synchronize()
    out_p = out_p.cpu().numpy()
    checked = (0, 1, 97, 128, 200, T - 1)
    outs = {}
    for step in range(T):
        p = S + step
        o = E.hybrid_full_attention(c, 0, qg_d[p:p + 1].contiguous(), k_d[p:p + 1].contiguous(),
                                    v_d[p:p + 1].contiguous(), 1, cfg.H, p, ones, ones, cfg.eps, cos_d, sin_d, cfg.rot)
        if step in checked:
            outs[step] = o
    torch.cuda.synchronize()
    cos, sin = _oracle_tables(cfg, N)
    onesh = np.ones(cfg.D, np.float32)
    kn = ref.norm_rope(k, onesh, cfg.eps, cos, sin, np.arange(N), rot=cfg.rot)
    kk, vv = _check_stored(c, 0, 0, kn, v)
    qn = ref.norm_rope(q, onesh, cfg.eps, cos, sin, np.arange(N), rot=cfg.rot)
    # prefill rows (independent): a spread sample, including the first and the last block
    for r0 in (0, 1000, 4090, S - 64):
        rows = slice(r0, r0 + 64)
        exp = ref.gated_attention(qn[rows], kk[:r0 + 64], vv[:r0 + 64], g[rows], r0)
        _check_out("q8", out_p[rows], exp)
    for step, o in outs.items():
        p = S + step
        exp = ref.gated_attention(qn[p:p + 1], kk[:p + 1], vv[:p + 1], g[p:p + 1], p)
        _check_out("q8", o.cpu().numpy(), exp)
    c.close()


def test_e2e_c5_prologue_queries_every_row(dev):
    """The hybrid prologue's queries (read in place from the interleaved q_proj) at all 8192
    prefill rows against the oracle's norm + partial RoPE."""
    cfg, S = W.C5, W.C5_PREFILL
    q, k, v, g = W.prefill_inputs(cfg, S, seed=7)
    qg = np.concatenate([q, g], -1)
    cos_d, sin_d, _, _ = rope_dev(cfg.theta, cfg.rot, S)
    ones = t(np.ones(cfg.D, np.float32))
    c = E.KvCache(1, cfg.KV, cfg.D, cfg.kv, max_seq_len=S, capacity=S)
    qr = E.qkv_prologue(c, 0, t(qg), t(k), t(v), S, cfg.H, ones, ones, cfg.eps, cos_d, sin_d, cfg.rot, 0, 0,
                        q_stride=2 * cfg.D)
    torch.cuda.synchronize()
    cos, sin = _oracle_tables(cfg, S)
    onesh = np.ones(cfg.D, np.float32)
    _check_q(qr, ref.norm_rope(q, onesh, cfg.eps, cos, sin, np.arange(S), rot=cfg.rot))
    _check_stored(c, 0, 0, ref.norm_rope(k, onesh, cfg.eps, cos, sin, np.arange(S), rot=cfg.rot), v)
    c.close()


# ------------------------------------------------------------------ C4: sinks at position 100000
def _sink_case(dtype, rows, rope_positions="slot", seed=4):
    """Drive a sink-mode cache through the reference's greedy schedule (src/engine.ts:1783-1799)
    to absolute position 100000, reserve ``rows`` slots (evictFor), write the resident tokens'
    K/V from their seeded raw rows through the prologue, then attend ``rows`` queries.
    Returns the product outputs and the oracle's expectation from the raw rows."""
    cfg = W.C4
    sinks, max_seq = cfg.sinks, cfg.sinks + cfg.window
    c = E.KvCache(1, cfg.KV, cfg.D, dtype, max_seq_len=max_seq, overflow="sinks", sink_tokens=sinks,
                  rope_positions=rope_positions)
    fill, fed = 1000, 1000
    while fed < W.C4_POSITION:
        batch = min(4, W.C4_POSITION - fed)
        fill = c.evict_for(fill, batch) + batch
        fed += batch
    fill = c.evict_for(fill, rows)
    head, evicted = c.ring_state()
    resident, fill2, _ = ref.simulate_sink_schedule(1000, W.C4_POSITION, sinks, max_seq, final_rows=rows)
    assert fill2 == fill and head != 0 and evicted > 0
    positions = np.array(list(resident) + list(range(W.C4_POSITION, W.C4_POSITION + rows)))
    assert positions[sinks] == sinks + evicted        # logical slot L >= sinks holds token L + evicted
    k = W.rows_for_positions(seed, positions, cfg.KV, cfg.D, tensor=1)
    v = W.rows_for_positions(seed, positions, cfg.KV, cfg.D, tensor=2)
    q = W.rows_for_positions(seed, positions[-rows:], cfg.H, cfg.D, tensor=0)
    n_tab = W.C4_POSITION + rows + 8 if rope_positions == "absolute" else max_seq
    cos_d, sin_d, _, _ = rope_dev(cfg.theta, cfg.rot, n_tab)
    c.set_rope(cos_d, sin_d)
    ones = t(np.ones(cfg.D, np.float32))
    E.qkv_prologue(c, 0, None, t(k[:fill]), t(v[:fill]), fill, cfg.H, None, ones, cfg.eps, cos_d, sin_d, cfg.rot,
                   0, 0)
    qpos = W.C4_POSITION if rope_positions == "absolute" else fill
    qr = E.qkv_prologue(c, 0, t(q), t(k[fill:]), t(v[fill:]), rows, cfg.H, ones, ones, cfg.eps, cos_d, sin_d,
                        cfg.rot, qpos, fill)
    out = E.attention(c, 0, qr, rows, cfg.H, fill)
    torch.cuda.synchronize()
    # oracle: keys stored normed and unroped (src/engine.ts:1530-1533), rotated at read by the
    # slot (attention_sg_roll.wgsl:40-51) or, in absolute mode, by the true token position
    cos, sin = _oracle_tables(cfg, n_tab)
    onesh = np.ones(cfg.D, np.float32)
    qn = ref.norm_rope(q, onesh, cfg.eps, cos, sin, qpos + np.arange(rows))
    kn = ref.norm_rope(k, onesh, cfg.eps, cos, sin, None, rope=False)
    _check_q(qr, qn)
    kst, vst = _check_stored(c, 0, 0, kn, v)
    kpos = positions if rope_positions == "absolute" else np.arange(fill + rows)
    kk = ref.rope_apply(kst, cos, sin, kpos)
    exp = ref.attention(qn, kk, vst, fill)
    out = out.cpu().numpy()
    c.close()
    return out, exp


@pytest.mark.parametrize("dtype", ["f16", "q8", "f32"])
@pytest.mark.parametrize("rows", [1, W.C4_VERIFY])
def test_e2e_c4_sinks_slot_rope(dev, dtype, rows):
    out, exp = _sink_case(dtype, rows)
    _check_out(dtype, out, exp)


@pytest.mark.parametrize("dtype", ["f16", "q8", "f32"])
def test_e2e_c4_sinks_absolute_rope(dev, dtype):
    out, exp = _sink_case(dtype, 1, rope_positions="absolute")
    _check_out(dtype, out, exp)


@pytest.mark.parametrize("dtype", ["f16", "q8", "f32"])
def test_e2e_sink_prefill_segment_after_wrap(dev, dtype):
    """A 256-row prefill segment into the wrapped ring (runPrefill in sink mode,
    src/engine.ts:1705-1735): the prefill kernel with read-time rotation over a ring whose
    origin is not 0 (f16 / q8 MFMA prefill, f32 exact kernel)."""
    out, exp = _sink_case(dtype, 256)
    _check_out(dtype, out, exp)


@pytest.mark.parametrize("dtype", ["f16", "q8", "f32"])
def test_e2e_sink_prompt_before_wrap(dev, dtype):
    """The C4 prompt (1000 tokens) prefilled into an empty sink-mode cache: keys stored unroped
    and rotated at read by the slot, queries roped at their slot (src/engine.ts:1573-1580)."""
    cfg, P = W.C4, 1000
    sinks, max_seq = cfg.sinks, cfg.sinks + cfg.window
    q, k, v, _ = W.prefill_inputs(cfg, P, seed=41)
    c = E.KvCache(1, cfg.KV, cfg.D, dtype, max_seq_len=max_seq, overflow="sinks", sink_tokens=sinks)
    cos_d, sin_d, _, _ = rope_dev(cfg.theta, cfg.rot, max_seq)
    c.set_rope(cos_d, sin_d)
    ones = t(np.ones(cfg.D, np.float32))
    assert c.evict_for(0, P) == 0
    qr = E.qkv_prologue(c, 0, t(q), t(k), t(v), P, cfg.H, ones, ones, cfg.eps, cos_d, sin_d, cfg.rot, 0, 0)
    out = E.attention(c, 0, qr, P, cfg.H, 0)
    torch.cuda.synchronize()
    cos, sin = _oracle_tables(cfg, max_seq)
    onesh = np.ones(cfg.D, np.float32)
    qn = ref.norm_rope(q, onesh, cfg.eps, cos, sin, np.arange(P))
    _check_q(qr, qn)
    kst, vst = _check_stored(c, 0, 0, ref.norm_rope(k, onesh, cfg.eps, cos, sin, None, rope=False), v)
    exp = ref.attention(qn, ref.rope_apply(kst, cos, sin, np.arange(P)), vst, 0)
    _check_out(dtype, out.cpu().numpy(), exp)
    c.close()
