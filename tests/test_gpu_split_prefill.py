"""GPU: split-K prefill (a grid of query blocks far smaller than the GPU: speculative verify with
many heads per kv head, a short prompt chunk after a long context) against the oracle.

Each (query block, kv head) item's key range is scanned in parts by separate workgroups, whose
partials a second kernel merges by log-sum-exp (the gate applied after the merge). Tolerances as
for every f16 / q8 attention: relative 2e-3 and cosine > 0.99999 against ``ref.attention`` /
``ref.gated_attention`` over the stored values. The partials share the decode kernel's
workspace, whose slots must hold the empty marker after every launch: a decode on the same
cache right after a split prefill checks that."""
import numpy as np
import pytest

from bitgpu_amd import engine as E
from oracle import ref
from tests.conftest import cosine, rel_err
from tests.gpu_helpers import cached_values, fill_cache_raw, run_attention
from tests.test_gpu_end_to_end import _check_out, _sink_case

pytestmark = pytest.mark.gpu


def _check(out, exp):
    assert np.isfinite(out).all()
    assert rel_err(out, exp) <= 2e-3, rel_err(out, exp)
    assert cosine(out, exp) > 0.99999


def _case(dtype, H, KV, D, L, S, seed, gate):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((L, KV, D)).astype(np.float32)
    v = rng.standard_normal((L, KV, D)).astype(np.float32)
    q = rng.standard_normal((S, H, D)).astype(np.float32)
    g = rng.standard_normal((S, H, D)).astype(np.float32) if gate else None
    c = E.KvCache(1, KV, D, dtype, max_seq_len=L, capacity=L)
    fill_cache_raw(c, 0, k, v)
    return c, rng, q, g


@pytest.mark.parametrize("dtype", ["q8", "f16"])
@pytest.mark.parametrize("S", [4, 8])
def test_hybrid_verify_split(dev, dtype, S):
    """Qwen3.5 hybrid shape (24 heads on 4 kv heads, D=256, gated): an S-row verify at 8193 +
    cached positions -- 6*S rows per kv head, more than the decode kernel's LDS plan holds, four
    query-block items split over many parts."""
    H, KV, D, L = 24, 4, 256, 8193 + S
    c, _, q, g = _case(dtype, H, KV, D, L, S, seed=40 + S, gate=True)
    out = run_attention(c, 0, q, L - S, scale=1.0 / 16, gate=g)
    kk, vv = cached_values(c, 0, 0, L)
    _check(out, ref.gated_attention(q, kk, vv, g, L - S))
    c.close()


@pytest.mark.parametrize("dtype", ["q8", "f16"])
def test_chunk_after_long_context_split(dev, dtype):
    """A 64-row prompt chunk after 8000 cached positions (runPrefill segments,
    src/engine.ts:1705-1735) in the Qwen3-8B shape: 16 items split over many parts; then a decode
    step on the same cache (the workspace must be back to empty slots)."""
    H, KV, D, P, S = 32, 8, 128, 8000, 64
    L = P + S + 1
    c, rng, q, _ = _case(dtype, H, KV, D, L, S, seed=77, gate=False)
    out = run_attention(c, 0, q, P)
    kk, vv = cached_values(c, 0, 0, L)
    _check(out, ref.attention(q, kk[:P + S], vv[:P + S], P))
    q1 = rng.standard_normal((1, H, D)).astype(np.float32)
    out1 = run_attention(c, 0, q1, L - 1)
    _check(out1, ref.attention(q1, kk, vv, L - 1))
    c.close()


@pytest.mark.parametrize("dtype", ["f16", "q8"])
def test_sink_segment_after_wrap_split(dev, dtype):
    """A 32-row segment into the wrapped sink ring (read-time rotation, the scan over every
    physical slot): one query block per kv head, split into parts."""
    out, exp = _sink_case(dtype, 32)
    _check_out(dtype, out, exp)


def test_split_prefill_repeated_launches(dev):
    """Consecutive split launches with different part counts on one cache reuse the workspace:
    each launch's merge leaves every slot it read empty for the next."""
    H, KV, D = 24, 4, 256
    L = 6000
    c, rng, _, _ = _case("q8", H, KV, D, L, 1, seed=5, gate=False)
    kk, vv = cached_values(c, 0, 0, L)
    for S, upto in ((8, 6000), (5, 2500), (8, 6000), (4, 900)):
        q = rng.standard_normal((S, H, D)).astype(np.float32)
        out = run_attention(c, 0, q, upto - S, scale=1.0 / 16)
        _check(out, ref.attention(q, kk[:upto], vv[:upto], upto - S, scale=1.0 / 16))
    c.close()


@pytest.mark.parametrize("dtype,H,KV,D,L,S,gate", [
    ("q8", 128, 1, 128, 20000, 1, False),    # one kv head, 128 rows: one item split 128 ways
    ("f16", 64, 2, 256, 5000, 3, True),      # 96 rows per kv head at D=256, gated
    ("q8", 64, 1, 128, 3000, 2, True),       # 128 rows, one query block of 2 queries
])
def test_split_prefill_extreme_shapes(dev, dtype, H, KV, D, L, S, gate):
    c, _, q, g = _case(dtype, H, KV, D, L, S, seed=H + L, gate=gate)
    scale = 1.0 / np.sqrt(D)
    out = run_attention(c, 0, q, L - S, scale=scale, gate=g)
    kk, vv = cached_values(c, 0, 0, L)
    _check(out, ref.gated_attention(q, kk, vv, g, L - S) if gate else ref.attention(q, kk, vv, L - S, scale=scale))
    c.close()
