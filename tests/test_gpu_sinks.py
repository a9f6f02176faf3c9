"""GPU: rolling window with attention sinks (config C4) -- the ring reproduces the reference's
resident set after decoding to absolute position 100000 (bit-exact index selection), decode and
a 5-token speculative verify match the oracle with keys rotated at read by their slot
(attention_sg_roll.wgsl:40-51), and before any eviction sink mode equals the plain cache
bit-for-bit in f32 (the reference's own gate, examples/verify.html:801-805)."""
import os

import numpy as np
import pytest
import torch

from bitgpu_amd import engine as E
from bitgpu_amd import workloads as W
from oracle import ref
from tests.conftest import cosine, rel_err
from tests.gpu_helpers import export_k_v, fill_cache_raw, rope_dev, run_attention, t

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _build_c4(rope_positions="slot", dtype="f16", verify=1, seed=4):
    cfg = W.C4
    sinks, max_seq = cfg.sinks, cfg.sinks + cfg.window
    g = np.load(os.path.join(ROOT, "tests", "golden", "sink_schedule.npz"))
    slots = g["slots"]
    c = E.KvCache(1, cfg.KV, cfg.D, dtype, max_seq_len=max_seq, overflow="sinks", sink_tokens=sinks,
                  rope_positions=rope_positions)
    # replay the reference schedule's evictions on the ring (index arithmetic only)
    fill = 1000
    fed = 1000
    ev = iter(g["events"])
    while fed < W.C4_POSITION:
        batch = min(4, W.C4_POSITION - fed)
        nf = c.evict_for(fill, batch)
        if nf != fill:
            f0, b, k = next(ev)
            assert f0 == fill and nf == ref.evict(fill, fill + batch - max_seq, sinks, max_seq)[0]
        fill = nf + batch
        fed += batch
    fill = c.evict_for(fill, verify)
    assert fill == len(slots) or verify > 1
    head, evicted = c.ring_state()
    # resident rows: token ids slots[] at logical 0..fill-1 (for verify>1 recompute the set)
    if verify > 1:
        resident, fill2, _ = ref.simulate_sink_schedule(1000, W.C4_POSITION, sinks, max_seq, final_rows=verify)
        assert fill2 == fill
    else:
        resident = list(slots)
    positions = list(resident) + list(range(W.C4_POSITION, W.C4_POSITION + verify))
    k = W.rows_for_positions(seed, positions, cfg.KV, cfg.D, tensor=1)
    v = W.rows_for_positions(seed, positions, cfg.KV, cfg.D, tensor=2)
    q = W.rows_for_positions(seed, positions[-verify:], cfg.H, cfg.D, tensor=0)
    n_tab = W.C4_POSITION + verify + 8 if rope_positions == "absolute" else max_seq
    cos_d, sin_d, cos, sin = rope_dev(cfg.theta, cfg.rot, n_tab)
    c.set_rope(cos_d, sin_d)
    ones = t(np.ones(cfg.D, np.float32))
    # resident K (normed, unroped) and V at logical slots 0..fill-1
    E.qkv_prologue(c, 0, None, t(k[:fill]), t(v[:fill]), fill, cfg.H, None, ones, cfg.eps, cos_d, sin_d, cfg.rot,
                   0, 0)
    qpos = (W.C4_POSITION if rope_positions == "absolute" else fill)
    qr = E.qkv_prologue(c, 0, t(q), t(k[fill:]), t(v[fill:]), verify, cfg.H, ones, ones, cfg.eps, cos_d, sin_d,
                        cfg.rot, qpos, fill)
    out = E.attention(c, 0, qr, verify, cfg.H, fill)
    torch.cuda.synchronize()
    return c, out.cpu().numpy(), qr.cpu().numpy(), positions, fill, cos, sin, head, evicted


@pytest.mark.parametrize("verify", [1, W.C4_VERIFY])
def test_c4_sinks_slot_rope(dev, verify):
    c, out, qn, positions, fill, cos, sin, head, evicted = _build_c4(verify=verify)
    assert head != 0 and evicted > 0
    kq, vq, _, _ = export_k_v(c, 0, 0, fill + verify)
    kk = ref.rope_apply(kq.astype(np.float32), cos, sin, np.arange(fill + verify))   # rotate at read by slot
    exp = ref.attention(qn, kk, vq.astype(np.float32), fill)
    assert rel_err(out, exp) <= 2e-3 and cosine(out, exp) > 0.99999
    c.close()


def test_c4_sinks_absolute_rope(dev):
    c, out, qn, positions, fill, cos, sin, head, evicted = _build_c4(rope_positions="absolute")
    kq, vq, _, _ = export_k_v(c, 0, 0, fill + 1)
    kk = ref.rope_apply(kq.astype(np.float32), cos, sin, np.array(positions))        # true positions
    exp = ref.attention(qn, kk, vq.astype(np.float32), fill)
    assert rel_err(out, exp) <= 2e-3
    # the kernel's key position for slot L >= sinks is L + evicted
    assert positions[W.C4.sinks] == W.C4.sinks + evicted
    c.close()


def test_c4_sinks_q8(dev):
    c, out, qn, positions, fill, cos, sin, head, evicted = _build_c4(dtype="q8")
    kq, vq, ks, vs = export_k_v(c, 0, 0, fill + 1)
    kk = ref.rope_apply(ref.q8_dequant(kq, ks), cos, sin, np.arange(fill + 1))
    exp = ref.attention(qn, kk, ref.q8_dequant(vq, vs), fill)
    assert rel_err(out, exp) <= 2e-3
    c.close()


@pytest.mark.parametrize("steps,batch,verify", [(40, 7, 1), (90, 13, 5), (23, 31, 3), (7, 97, 2), (2, 500, 1),
                                                 (3, 700, 3)])
def test_sinks_masked_room_not_scanned(dev, steps, batch, verify):
    """Sink mode after the ring wrapped, at several ring origins and amounts of room: the ring
    slots past the last row's position are masked for every row, and the decode kernel does not
    scan their longest run of whole tiles (in one piece, or wrapping across the ring's end: the
    large batches leave room on both sides of it, the longer run before it (2, 500) or after it
    (3, 700)); the output matches the oracle over the logical slots."""
    KV, H, D, sinks, window = 8, 32, 128, 4, 1024
    max_seq = sinks + window
    c = E.KvCache(1, KV, D, "f16", max_seq_len=max_seq, overflow="sinks", sink_tokens=sinks)
    fill = 900
    for _ in range(steps):
        fill = c.evict_for(fill, batch) + batch
    fill = c.evict_for(fill, verify)
    head, evicted = c.ring_state()
    assert head != 0 and evicted > 0
    rng = np.random.default_rng(steps * 1000 + batch)
    k = rng.standard_normal((fill + verify, KV, D)).astype(np.float32)
    v = rng.standard_normal((fill + verify, KV, D)).astype(np.float32)
    q = rng.standard_normal((verify, H, D)).astype(np.float32)
    cos_d, sin_d, cos, sin = rope_dev(1e4, D, max_seq)
    c.set_rope(cos_d, sin_d)
    ones = t(np.ones(D, np.float32))
    E.qkv_prologue(c, 0, None, t(k[:fill]), t(v[:fill]), fill, H, None, ones, 1e-6, cos_d, sin_d, D, 0, 0)
    qr = E.qkv_prologue(c, 0, t(q), t(k[fill:]), t(v[fill:]), verify, H, ones, ones, 1e-6, cos_d, sin_d, D,
                        fill, fill)
    out = E.attention(c, 0, qr, verify, H, fill)
    torch.cuda.synchronize()
    kq, vq, _, _ = export_k_v(c, 0, 0, fill + verify)
    kk = ref.rope_apply(kq.astype(np.float32), cos, sin, np.arange(fill + verify))
    exp = ref.attention(qr.cpu().numpy(), kk, vq.astype(np.float32), fill)
    room = max_seq - (fill + verify)
    assert room >= 64  # at least one whole tile of room
    assert rel_err(out.cpu().numpy(), exp) <= 2e-3 and cosine(out.cpu().numpy(), exp) > 0.99999
    c.close()


@pytest.mark.parametrize("S", [1, 4, 40])
def test_sinks_before_eviction_equal_plain_cache_f32(dev, S):
    """Before the first eviction the sink-mode cache (unroped keys, rotated at read) gives
    bit-identical f32 outputs to the plain cache (keys roped at write)."""
    rng = np.random.default_rng(S)
    H, KV, D, L = 16, 4, 128, 200
    q = rng.standard_normal((S, H, D)).astype(np.float32)
    k = rng.standard_normal((L, KV, D)).astype(np.float32)
    v = rng.standard_normal((L, KV, D)).astype(np.float32)
    cos_d, sin_d, _, _ = rope_dev(1e6, D, 512)
    ones = t(np.ones(D, np.float32))
    outs = []
    for overflow in ("error", "sinks"):
        c = E.KvCache(1, KV, D, "f32", max_seq_len=512, capacity=512, overflow=overflow, sink_tokens=4)
        if overflow == "sinks":
            c.set_rope(cos_d, sin_d)
        past = L - S
        E.qkv_prologue(c, 0, None, t(k[:past]), t(v[:past]), past, H, None, ones, 1e-6, cos_d, sin_d, D, 0, 0)
        att = E.layer_attention(c, 0, t(q), t(k[past:]), t(v[past:]), S, H, past, ones, ones, 1e-6, cos_d, sin_d)
        torch.cuda.synchronize()
        outs.append(att.cpu().numpy())
        c.close()
    assert np.array_equal(outs[0], outs[1])
