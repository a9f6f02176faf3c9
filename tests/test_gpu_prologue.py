"""GPU: the fused attention prologue (per-head RMSNorm + RoPE for Q, K straight into the cache,
V append) against the oracle's norm/rope (tools/reference.py:106-107,146-152;
tools/qwen35_numpy.py:71-89), and the fused-write invariant: the q8 / f16 bytes the fused
kernel stores equal the reference quantizer applied to the f32 values the same kernel computes
(fused_q8 == pack(fused_f32), bit-exact)."""
import numpy as np
import pytest
import torch

from bitgpu_amd import engine as E
from oracle import ref
from tests.gpu_helpers import export_k_v, rope_dev, t

pytestmark = pytest.mark.gpu

# f32 norm/rope: the kernel reduces the sum of squares in another order than numpy's pairwise
# mean, so values agree to a few ulp, not bit for bit
RTOL, ATOL = 4e-6, 4e-6


def _prologue(dtype, S, H, KV, D, rot, theta, pos0, seed=0, q_stride=None, roll=False, gamma_seed=None):
    rng = np.random.default_rng(seed)
    qs = q_stride or D
    q = rng.standard_normal((S, H, qs)).astype(np.float32)
    k = rng.standard_normal((S, KV, D)).astype(np.float32)
    v = rng.standard_normal((S, KV, D)).astype(np.float32)
    if gamma_seed is None:
        gq = np.ones(D, np.float32)
        gk = np.ones(D, np.float32)
    else:
        g = np.random.default_rng(gamma_seed)
        gq = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
        gk = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
    cos_d, sin_d, cos, sin = rope_dev(theta, rot, pos0 + S + 3)
    kw = dict(overflow="sinks", sink_tokens=4) if roll else {}
    c = E.KvCache(1, KV, D, dtype, max_seq_len=max(pos0 + S + 64, 128), capacity=pos0 + S, **kw)
    qo = E.qkv_prologue(c, 0, t(q), t(k), t(v), S, H, t(gq), t(gk), 1e-6, cos_d, sin_d, rot, pos0, pos0,
                        q_stride=qs)
    torch.cuda.synchronize()
    exp_q = ref.norm_rope(q[..., :D], gq, 1e-6, cos, sin, pos0 + np.arange(S), rot=rot)
    exp_k = ref.norm_rope(k, gk, 1e-6, cos, sin, pos0 + np.arange(S), rot=rot, rope=not roll)
    return c, qo.cpu().numpy(), exp_q, exp_k, k, v


@pytest.mark.parametrize("D,rot,theta,H,KV", [(128, 128, 1e6, 32, 8), (256, 64, 1e7, 24, 4), (256, 256, 1e6, 8, 2)])
def test_prologue_f32_matches_oracle(dev, D, rot, theta, H, KV):
    S, pos0 = 9, 1234
    c, qo, eq, ek, k, v = _prologue("f32", S, H, KV, D, rot, theta, pos0, seed=D + rot, gamma_seed=3)
    assert np.allclose(qo, eq, rtol=RTOL, atol=ATOL)
    gk, gv, _, _ = export_k_v(c, 0, pos0, S)
    assert np.allclose(gk, ek, rtol=RTOL, atol=ATOL)
    assert np.array_equal(gv, v)                       # V is stored unchanged
    c.close()


def test_prologue_hybrid_interleaved_query(dev):
    """q_proj of the gated layer is [S, H, 2D] (query | gate per head); the prologue reads the
    query half in place (split_head.wgsl:12-15 folded away)."""
    S, H, KV, D = 5, 24, 4, 256
    c, qo, eq, ek, _, _ = _prologue("f32", S, H, KV, D, 64, 1e7, 40, seed=9, q_stride=2 * D)
    assert np.allclose(qo, eq, rtol=RTOL, atol=ATOL)
    c.close()


@pytest.mark.parametrize("dtype", ["f16", "q8"])
@pytest.mark.parametrize("D", [128, 256])
def test_fused_write_equals_pack_of_fused_f32(dev, dtype, D):
    S, H, KV, pos0 = 33, 16, 4, 700
    c32, _, _, _, _, _ = _prologue("f32", S, H, KV, D, D, 1e6, pos0, seed=11, gamma_seed=5)
    cq, _, _, _, _, v = _prologue(dtype, S, H, KV, D, D, 1e6, pos0, seed=11, gamma_seed=5)
    k32, _, _, _ = export_k_v(c32, 0, pos0, S)
    kq, vq, ks, vs = export_k_v(cq, 0, pos0, S)
    if dtype == "f16":
        assert np.array_equal(kq.view(np.uint16), ref.f16_pack(k32).view(np.uint16))
        assert np.array_equal(vq.view(np.uint16), ref.f16_pack(v).view(np.uint16))
    else:
        ck, sk = ref.q8_pack(k32)
        assert np.array_equal(kq, ck) and np.array_equal(ks.view(np.uint32), sk.view(np.uint32))
        cv, sv = ref.q8_pack(v)
        assert np.array_equal(vq, cv) and np.array_equal(vs.view(np.uint32), sv.view(np.uint32))
    c32.close()
    cq.close()


def test_sink_mode_stores_unroped_keys(dev):
    S, H, KV, D = 6, 8, 2, 128
    c, qo, eq, ek, _, _ = _prologue("f32", S, H, KV, D, D, 1e6, 20, seed=13, roll=True)
    gk, _, _, _ = export_k_v(c, 0, 20, S)
    assert np.allclose(gk, ek, rtol=RTOL, atol=ATOL)    # rmsnorm only
    assert np.allclose(qo, eq, rtol=RTOL, atol=ATOL)    # Q still roped at its slot
    c.close()
