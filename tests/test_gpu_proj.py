"""GPU: the 1-bit decode projections on either side of attention against the oracle
(oracle/ref.py gemv_1bit, restating matmul_split_sg.wgsl / matmul_resid_mr_sg.wgsl), and the
fused decode qkv projection + prologue against the unfused path (bit for bit) and the oracle.

Tolerance of a GEMV row: |y - y64| <= 4e-6 * sum_k |x_k| * scale (the f32 sum's rounding, measured
against the magnitude of its terms). The fused kernel shares the GEMV's row arithmetic and the
prologue's norm / rotation, so it must equal bg_gemv_split followed by bg_qkv_prologue exactly."""
import numpy as np
import pytest
import torch

from bitgpu_amd import engine as E
from oracle import ref
from tests.conftest import rel_err
from tests.gpu_helpers import export_k_v, rope_dev, t

pytestmark = pytest.mark.gpu
GEMV_RTOL = 4e-6


def _weight(rng, N, K, scale=0.02):
    sign = rng.integers(0, 2 ** 32, (N, K // 32), dtype=np.uint64).astype(np.uint32)
    sc = (np.abs(rng.standard_normal((N, K // 128))) * scale).astype(np.float32)
    return sign, sc


def _dev_weight(sign, sc, K, N0, N1=0, N2=0):
    return E.OneBitWeight(t(sign.view(np.int32)), t(sc), K, N0, N1, N2)


def _check_gemv(got, x, sign, sc, resid=None):
    want = ref.gemv_1bit(x, sign, sc, resid).astype(np.float64)
    bound = ref.gemv_abs_bound(x, sc) + (np.abs(resid) if resid is not None else 0)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= GEMV_RTOL * bound + 1e-30), float((err / bound).max())


@pytest.mark.parametrize("K,N0,N1,N2", [(4096, 4096, 1024, 1024),    # Qwen3-8B qkv
                                        (2560, 4096, 1024, 1024),    # Qwen3-4B qkv (K not a tile multiple)
                                        (4096, 12288, 12288, 0),     # gate | up
                                        (5120, 1000, 0, 0)])         # partial tile, rows not a wave multiple
def test_gemv_split_matches_oracle(dev, K, N0, N1, N2):
    rng = np.random.default_rng(K + N0)
    sign, sc = _weight(rng, N0 + N1 + N2, K)
    x = rng.standard_normal(K).astype(np.float32)
    w = _dev_weight(sign, sc, K, N0, N1, N2)
    outs = [torch.full((n,), float("nan"), device="cuda") for n in (N0, N1, N2) if n]
    E.fused_mm(w, t(x), outs)
    torch.cuda.synchronize()
    got = np.concatenate([o.cpu().numpy() for o in outs])
    _check_gemv(got, x, sign, sc)


@pytest.mark.parametrize("K,N", [(4096, 4096), (12288, 4096), (4096, 2560), (384, 77), (128, 64), (4224, 300), (12416, 200)])
def test_gemv_resid_matches_oracle(dev, K, N):
    """o_proj / down_proj with the residual (src/engine.ts:1547, matmul_resid_mr_sg.wgsl): rows
    read through the nibble table (K <= 4096, down to a single scale block), through x staged in
    LDS (4224 just past the table, 12288) and from memory (12416, past the staging)."""
    rng = np.random.default_rng(K * 3 + N)
    sign, sc = _weight(rng, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    h = rng.standard_normal(N).astype(np.float32)
    y = E.resid_mm(_dev_weight(sign, sc, K, N), t(x), t(h))
    torch.cuda.synchronize()
    _check_gemv(y.cpu().numpy(), x, sign, sc, h)


def _qkv_case(dtype, H, KV, D, K, pos, seed, roll=False):
    rng = np.random.default_rng(seed)
    N = (H + 2 * KV) * D
    sign, sc = _weight(rng, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    gq = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    return rng, sign, sc, x, gq, gk


@pytest.mark.parametrize("dtype", ["f16", "q8", "f32"])
@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (16, 8, 128), (8, 2, 256), (20, 2, 128), (24, 12, 128)])
def test_qkv_proj_prologue_equals_unfused(dev, dtype, H, KV, D):
    """One launch (projection, Q norm+rope, K norm+rope into the cache, V append) equals the
    projection followed by the prologue, bit for bit: q_out and every stored K / V byte.
    (32, 8), (20, 2) and (24, 12) at D=128 run 24-row workgroups (heads across workgroup
    boundaries; 256 / 128 / 256 workgroups, the Q/K/V boundaries at different places), the
    others 32-row ones."""
    _fused_equals_unfused(dtype, H, KV, D, 4096)


@pytest.mark.parametrize("K", [5120, 13312])
@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (8, 2, 256)])
def test_qkv_proj_prologue_equals_unfused_long_rows(dev, H, KV, D, K):
    """The same beyond the nibble table's 4096-weight rows: x staged in LDS (K = 5120, three
    2048-weight tiles, the last one partial) and x read from memory (K = 13312), on 24-row and
    32-row workgroups."""
    _fused_equals_unfused("q8", H, KV, D, K)


def _fused_equals_unfused(dtype, H, KV, D, K):
    pos = 777
    rng, sign, sc, x, gq, gk = _qkv_case(dtype, H, KV, D, K, pos, seed=H + KV + D)
    w = _dev_weight(sign, sc, K, H * D, KV * D, KV * D)
    cos_d, sin_d, cos, sin = rope_dev(1e6, D, 1024)
    caches, qs = [], []
    for fused in (True, False):
        c = E.KvCache(1, KV, D, dtype, max_seq_len=1024, capacity=1024)
        if fused:
            q = E.qkv_proj_prologue(c, 0, t(x), w, H, t(gq), t(gk), 1e-6, cos_d, sin_d, D, pos, pos)
        else:
            qr, kr, vr = (torch.empty(n, device="cuda") for n in (H * D, KV * D, KV * D))
            E.fused_mm(w, t(x), [qr, kr, vr])
            q = E.qkv_prologue(c, 0, qr.view(1, H, D), kr.view(1, KV, D), vr.view(1, KV, D), 1, H, t(gq), t(gk), 1e-6,
                               cos_d, sin_d, D, pos, pos)
        torch.cuda.synchronize()
        caches.append(c)
        qs.append(q.cpu().numpy())
    assert np.array_equal(qs[0].view(np.uint32), qs[1].view(np.uint32))
    for a_, b_ in zip(export_k_v(caches[0], 0, pos, 1), export_k_v(caches[1], 0, pos, 1)):
        if a_ is not None:
            assert np.array_equal(a_.view(np.uint8), b_.view(np.uint8))
    # and against the oracle: the projection in float64, then norm + rope of each head row
    y = ref.gemv_1bit(x, sign, sc)
    qn = ref.norm_rope(y[:H * D].reshape(1, H, D), gq, 1e-6, cos, sin, [pos])
    kn = ref.norm_rope(y[H * D:(H + KV) * D].reshape(1, KV, D), gk, 1e-6, cos, sin, [pos])
    assert np.allclose(qs[0], qn, rtol=1e-4, atol=1e-4)
    kq, vq, ks, vs = export_k_v(caches[0], 0, pos, 1)
    v_raw = y[(H + KV) * D:].reshape(1, KV, D)
    if dtype == "q8":
        kq, vq = ref.q8_dequant(kq, ks), ref.q8_dequant(vq, vs)
        tol = 1.5 / 127 * np.abs(kn).max()
        assert np.abs(kq - kn).max() <= tol and np.abs(vq - v_raw).max() <= 1.5 / 127 * np.abs(v_raw).max()
    else:
        assert np.allclose(kq.astype(np.float32), kn, rtol=2e-3, atol=1e-4)
        assert np.allclose(vq.astype(np.float32), v_raw, rtol=2e-3, atol=1e-4)
    for c in caches:
        c.close()


def test_qkv_proj_sink_mode_keys_unroped(dev):
    """In a sink-mode cache the fused projection stores K normed but unroped (rotated at read),
    the query still roped at its slot (src/engine.ts:1530-1533)."""
    H, KV, D, K, pos = 16, 4, 128, 2048, 90
    rng, sign, sc, x, gq, gk = _qkv_case("f32", H, KV, D, K, pos, seed=5)
    w = _dev_weight(sign, sc, K, H * D, KV * D, KV * D)
    cos_d, sin_d, cos, sin = rope_dev(1e6, D, 256)
    c = E.KvCache(1, KV, D, "f32", max_seq_len=256, overflow="sinks", sink_tokens=4)
    c.set_rope(cos_d, sin_d)
    q = E.qkv_proj_prologue(c, 0, t(x), w, H, t(gq), t(gk), 1e-6, cos_d, sin_d, D, pos, pos)
    torch.cuda.synchronize()
    y = ref.gemv_1bit(x, sign, sc)
    kn = ref.norm_rope(y[H * D:(H + KV) * D].reshape(1, KV, D), gk, 1e-6, cos, sin, None, rope=False)
    kq, vq, _, _ = export_k_v(c, 0, pos, 1)
    assert np.allclose(kq, kn, rtol=1e-4, atol=1e-4)
    assert np.allclose(q.cpu().numpy(), ref.norm_rope(y[:H * D].reshape(1, H, D), gq, 1e-6, cos, sin, [pos]),
                       rtol=1e-4, atol=1e-4)
    c.close()


def test_decode_attention_block_steps(dev):
    """The fused decode attention block (src/engine.ts:1519-1547) over several consecutive tokens
    of a q8 cache in the Qwen3-4B shape (hidden 2560, 32 heads on 8 kv heads): qkv projection +
    prologue, attention, o_proj + residual, against the oracle composite (the arrival counters
    reset after every launch, so repeated launches stay correct)."""
    H, KV, D, HD, past, steps = 32, 8, 128, 2560, 300, 4
    rng = np.random.default_rng(9)
    sign, sc = _weight(rng, (H + 2 * KV) * D, HD)
    osign, osc = _weight(rng, HD, H * D)
    w_qkv = _dev_weight(sign, sc, HD, H * D, KV * D, KV * D)
    w_o = _dev_weight(osign, osc, H * D, HD)
    gq = np.ones(D, np.float32)
    gk = np.ones(D, np.float32)
    cos_d, sin_d, cos, sin = rope_dev(1e6, D, 1024)
    c = E.KvCache(1, KV, D, "q8", max_seq_len=1024, capacity=1024)
    # cached past: raw K (normed + roped through the prologue) and V
    kp = rng.standard_normal((past, KV, D)).astype(np.float32)
    vp = rng.standard_normal((past, KV, D)).astype(np.float32)
    E.qkv_prologue(c, 0, None, t(kp), t(vp), past, H, None, t(gk), 1e-6, cos_d, sin_d, D, 0, 0)
    kall = list(ref.norm_rope(kp, gk, 1e-6, cos, sin, np.arange(past)))
    vall = list(vp)
    for s in range(steps):
        pos = past + s
        n1 = rng.standard_normal(HD).astype(np.float32)
        h = rng.standard_normal(HD).astype(np.float32)
        h2 = E.decode_attention_block(c, 0, t(n1), t(h), w_qkv, w_o, H, t(gq), t(gk), 1e-6, cos_d, sin_d, pos)
        torch.cuda.synchronize()
        y = ref.gemv_1bit(n1, sign, sc)
        qn = ref.norm_rope(y[:H * D].reshape(1, H, D), gq, 1e-6, cos, sin, [pos])
        kall.append(ref.norm_rope(y[H * D:(H + KV) * D].reshape(1, KV, D), gk, 1e-6, cos, sin, [pos])[0])
        vall.append(y[(H + KV) * D:].reshape(KV, D))
        kk = ref.kv_roundtrip(np.array(kall), "q8")
        vv = ref.kv_roundtrip(np.array(vall), "q8")
        att = ref.attention(qn, kk, vv, pos)
        want = ref.gemv_1bit(att.reshape(-1), osign, osc, h)
        got = h2.cpu().numpy()
        # the attention part of the output (the residual added on top is exact either way)
        assert rel_err(got - h, want - h) <= 2e-3, rel_err(got - h, want - h)
    c.close()
