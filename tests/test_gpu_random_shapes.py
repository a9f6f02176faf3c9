"""GPU: seeded random shapes through the product path against the oracle.

The fixed-shape tests cover the benchmark configurations and the edge lengths; these draw the
rest of the space the C ABI accepts: GQA ratios 1-16 (including the odd 3, 5, 7 whose row blocks
do not fill a 32-row MFMA tile), 1-8 kv heads, head_dim 128 / 256, cached lengths that are not
tile multiples, decode (1 row), verify (2-5 rows) and prefill (up to 300 rows) of every storage
mode, with and without the output gate. Attention is compared with ``ref.attention`` /
``ref.gated_attention`` over the values the cache holds (the benchmark's stated tolerances: f32 max-abs
1e-4, f16 / q8 relative 2e-3 and cosine > 0.99999); the fused prologue with ``ref.norm_rope`` at a
random position and rotary width (rtol / atol 4e-6)."""
import numpy as np
import pytest

from bitgpu_amd import engine as E
from oracle import ref
from tests.conftest import cosine, rel_err
from tests.gpu_helpers import cached_values, export_k_v, fill_cache_raw, rope_dev, run_attention, t

pytestmark = pytest.mark.gpu


def _attention_cases(n=48, seed=2026):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        dtype = ["f32", "f16", "q8"][i % 3]
        D = int(rng.choice([128, 256]))
        KV = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 12, 16]))
        L = int(rng.integers(1, 3000))
        kind = ["decode", "verify", "prefill"][int(rng.integers(0, 3))]
        S = 1 if kind == "decode" else int(rng.integers(2, 6)) if kind == "verify" else int(rng.integers(6, 301))
        S = min(S, L)
        gate = bool(rng.integers(0, 4) == 0)
        cases.append((i, dtype, D, KV, G, L, S, gate))
    return cases


@pytest.mark.parametrize("i,dtype,D,KV,G,L,S,gate", _attention_cases())
def test_random_attention_shape(dev, i, dtype, D, KV, G, L, S, gate):
    rng = np.random.default_rng(1000 + i)
    H = G * KV
    k = rng.standard_normal((L, KV, D)).astype(np.float32)
    v = rng.standard_normal((L, KV, D)).astype(np.float32)
    q = rng.standard_normal((S, H, D)).astype(np.float32)
    g = rng.standard_normal((S, H, D)).astype(np.float32) if gate else None
    scale = 1.0 / np.sqrt(D)
    c = E.KvCache(1, KV, D, dtype, max_seq_len=max(L, 64), capacity=L)
    fill_cache_raw(c, 0, k, v)
    out = run_attention(c, 0, q, L - S, scale=scale, gate=g)
    kk, vv = cached_values(c, 0, 0, L)
    exp = ref.gated_attention(q, kk, vv, g, L - S) if gate else ref.attention(q, kk, vv, L - S, scale=scale)
    c.close()
    assert np.isfinite(out).all()
    if dtype == "f32":
        assert np.abs(out - exp).max() <= 1e-4
    else:
        assert rel_err(out, exp) <= 2e-3, rel_err(out, exp)
        assert cosine(out, exp) > 0.99999


def _prologue_cases(n=16, seed=77):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([128, 256]))
        KV = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.choice([1, 2, 3, 4, 6, 8]))
        S = int(rng.integers(1, 70))
        pos0 = int(rng.integers(0, 5000))
        rot = int(rng.choice([D, D // 2, 64]))
        out.append((i, ["f32", "f16", "q8"][i % 3], D, KV, G, S, pos0, rot))
    return out


@pytest.mark.parametrize("i,dtype,D,KV,G,S,pos0,rot", _prologue_cases())
def test_random_prologue_shape(dev, i, dtype, D, KV, G, S, pos0, rot):
    rng = np.random.default_rng(500 + i)
    H = G * KV
    q = rng.standard_normal((S, H, D)).astype(np.float32)
    k = rng.standard_normal((S, KV, D)).astype(np.float32)
    v = rng.standard_normal((S, KV, D)).astype(np.float32)
    gq = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    cos_d, sin_d, cos, sin = rope_dev(1e6, rot, pos0 + S)
    c = E.KvCache(1, KV, D, "f32", max_seq_len=pos0 + S + 64, capacity=pos0 + S)
    cq = E.KvCache(1, KV, D, dtype, max_seq_len=pos0 + S + 64, capacity=pos0 + S)
    qo = E.qkv_prologue(c, 0, t(q), t(k), t(v), S, H, t(gq), t(gk), 1e-6, cos_d, sin_d, rot, pos0, pos0)
    E.qkv_prologue(cq, 0, None, t(k), t(v), S, H, None, t(gk), 1e-6, cos_d, sin_d, rot, pos0, pos0)
    exp_q = ref.norm_rope(q, gq, 1e-6, cos, sin, pos0 + np.arange(S), rot=rot)
    exp_k = ref.norm_rope(k, gk, 1e-6, cos, sin, pos0 + np.arange(S), rot=rot)
    assert np.allclose(qo.cpu().numpy(), exp_q, rtol=4e-6, atol=4e-6)
    k32, v32, _, _ = export_k_v(c, 0, pos0, S)
    assert np.allclose(k32, exp_k, rtol=4e-6, atol=4e-6)
    assert np.array_equal(v32, v)
    # the storage-format write is the pack of the f32 one (bit-exact)
    kq, vq, ks, vs = export_k_v(cq, 0, pos0, S)
    if dtype == "f16":
        assert np.array_equal(kq.view(np.uint16), ref.f16_pack(k32).view(np.uint16))
        assert np.array_equal(vq.view(np.uint16), ref.f16_pack(v).view(np.uint16))
    elif dtype == "q8":
        ck, sk = ref.q8_pack(k32)
        cv, sv = ref.q8_pack(v)
        assert np.array_equal(kq, ck) and np.array_equal(ks.view(np.uint32), sk.view(np.uint32))
        assert np.array_equal(vq, cv) and np.array_equal(vs.view(np.uint32), sv.view(np.uint32))
    c.close()
    cq.close()
