"""GPU: the decode kernel at every query-pass configuration it compiles, against the oracle.

The decode kernel reads Q in passes of 4 rows (block-diagonal quarters of each MFMA) or, once a
kv head has more than 4 query rows, of 8 (block-diagonal halves; with q8 codes the two lane
groups of a half share one 32-dim scale block), in one, two or three 16-row sets. Plain caches
reach it up to 16 rows per kv head (q8 at head_dim 128 up to 24); sink mode (keys rotated at
read by their slot, attention_sg_roll.wgsl:40-51) takes every shape the kernel supports. Each
case compares with ``ref.attention`` over what the cache holds, at the f16 / q8 tolerance
(relative 2e-3, cosine > 0.99999)."""
import numpy as np
import pytest
import torch

from bitgpu_amd import engine as E
from bitgpu_amd import workloads as W
from oracle import ref
from tests.conftest import cosine, rel_err
from tests.gpu_helpers import cached_values, export_k_v, fill_cache_raw, rope_dev, run_attention, t

pytestmark = pytest.mark.gpu

EPS = 1e-6
THETA = 1e6


def _check(out, exp):
    assert np.isfinite(out).all()
    assert rel_err(out, exp) <= 2e-3, rel_err(out, exp)
    assert cosine(out, exp) > 0.99999


# (dtype, D, KV, G, S): rows per kv head R = G * S
PLAIN = [
    (dt, D, KV, G, S)
    for dt in ("f16", "q8")
    for D in (128, 256)
    for (KV, G, S) in ((4, 5, 1), (4, 6, 1), (2, 4, 2), (2, 3, 3), (4, 6, 2), (1, 8, 2))
] + [("q8", 128, 8, 4, 5), ("q8", 128, 8, 6, 4)]


@pytest.mark.parametrize("L", [70, 2600])
@pytest.mark.parametrize("dtype,D,KV,G,S", PLAIN)
def test_plain_cache_passes(dev, dtype, D, KV, G, S, L):
    """5-24 rows per kv head on a plain cache: a single split (70 positions) and split-K with a
    merge (2600 positions)."""
    H = G * KV
    rng = np.random.default_rng(D + 7 * G + 13 * S + L)
    k = rng.standard_normal((L, KV, D)).astype(np.float32)
    v = rng.standard_normal((L, KV, D)).astype(np.float32)
    q = (2.0 * rng.standard_normal((S, H, D))).astype(np.float32)
    c = E.KvCache(1, KV, D, dtype, max_seq_len=L, capacity=L)
    fill_cache_raw(c, 0, k, v)
    scale = 1.0 / np.sqrt(D)
    out = run_attention(c, 0, q, L - S, scale=scale)
    kk, vv = cached_values(c, 0, 0, L)
    c.close()
    _check(out, ref.attention(q, kk, vv, L - S, scale=scale))


def _sink_ring(dtype, D, KV, G, rows, sinks=4, window=700, prompt=500, position=3000, seed=9):
    """A sink-mode cache driven through the reference's greedy schedule to `position` (ring
    wrapped, origin not 0), `rows` slots reserved, the resident tokens' K/V written through the
    prologue (normed, unroped), then `rows` queries attended at their slots. Returns the product
    output and the oracle's."""
    max_seq = sinks + window
    H = G * KV
    c = E.KvCache(1, KV, D, dtype, max_seq_len=max_seq, overflow="sinks", sink_tokens=sinks)
    fill, fed = prompt, prompt
    while fed < position:
        batch = min(4, position - fed)
        fill = c.evict_for(fill, batch) + batch
        fed += batch
    fill = c.evict_for(fill, rows)
    head, evicted = c.ring_state()
    resident, fill2, _ = ref.simulate_sink_schedule(prompt, position, sinks, max_seq, final_rows=rows)
    assert fill2 == fill and head != 0 and evicted > 0
    positions = np.array(list(resident) + list(range(position, position + rows)))
    k = W.rows_for_positions(seed, positions, KV, D, tensor=1)
    v = W.rows_for_positions(seed, positions, KV, D, tensor=2)
    q = W.rows_for_positions(seed, positions[-rows:], H, D, tensor=0)
    cos_d, sin_d, _, _ = rope_dev(THETA, D, max_seq)
    c.set_rope(cos_d, sin_d)
    ones = t(np.ones(D, np.float32))
    E.qkv_prologue(c, 0, None, t(k[:fill]), t(v[:fill]), fill, H, None, ones, EPS, cos_d, sin_d, D, 0, 0)
    qr = E.qkv_prologue(c, 0, t(q), t(k[fill:]), t(v[fill:]), rows, H, ones, ones, EPS, cos_d, sin_d, D, fill, fill)
    out = E.attention(c, 0, qr, rows, H, fill)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    # oracle over the stored (normed, unroped) keys rotated by their slot and the stored values
    cos, sin = ref.rope_tables(THETA, D, max_seq)
    qn = ref.norm_rope(q, np.ones(D, np.float32), EPS, cos, sin, fill + np.arange(rows))
    kq, vq, ks, vs = export_k_v(c, 0, 0, fill + rows)
    if dtype == "q8":
        kst, vst = ref.q8_dequant(kq, ks), ref.q8_dequant(vq, vs)
    else:
        kst, vst = kq.astype(np.float32), vq.astype(np.float32)
    c.close()
    kk = ref.rope_apply(kst, cos, sin, np.arange(fill + rows))
    return out, ref.attention(qn, kk, vst, fill)


SINK = [(dt, 128, 8, 4, S) for dt in ("f16", "q8") for S in (2, 3, 5, 6, 8, 10, 12)] + \
       [(dt, 256, 4, 6, S) for dt in ("f16", "q8") for S in (1, 2, 3)] + \
       [(dt, 256, 2, 4, S) for dt in ("f16", "q8") for S in (2, 4, 5)]


@pytest.mark.parametrize("dtype,D,KV,G,S", SINK)
def test_sink_ring_passes(dev, dtype, D, KV, G, S):
    """Sink mode, ring wrapped: decode kernel with read-time rotation at 4-48 rows per kv head
    (head_dim 128) and 4-20 (head_dim 256), one to three 16-row sets."""
    out, exp = _sink_ring(dtype, D, KV, G, S)
    _check(out, exp)
