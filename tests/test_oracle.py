"""Pins for the oracle (oracle/ref.py, oracle/pack_ref.c) -- every function is checked against
something its own formula does not restate: closed forms, invariants, independent libraries
(Python math/struct, exact fractions), brute force on tiny inputs, and the reference's own
kernel-case vectors."""
import ctypes as C
import math
import os
import struct
import subprocess
from fractions import Fraction

import numpy as np
import pytest

from oracle import ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def cref():
    so = os.path.join(ROOT, "oracle", "liboracle_ref.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib = C.CDLL(so)
    lib.oracle_q8_pack.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    lib.oracle_q8_dequant.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]
    lib.oracle_f16_pack.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p]
    lib.oracle_attention_f64.argtypes = [C.c_void_p] * 4 + [C.c_int] * 6 + [C.c_double, C.c_void_p]
    return lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- rope tables
def test_rope_tables_match_python_math():
    theta, rot, P = 1e6, 128, 300
    cos, sin = ref.rope_tables(theta, rot, P)
    for p in (0, 1, 7, 299):
        for j in (0, 1, 31, 63):
            inv = 1.0 / math.pow(theta, 2 * j / rot)
            assert cos[p, j] == np.float32(math.cos(p * inv))
            assert sin[p, j] == np.float32(math.sin(p * inv))


def test_rope_tables_closed_forms():
    cos, sin = ref.rope_tables(1e7, 64, 50)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)           # position 0 is the identity
    assert np.allclose(cos[:, 0], np.cos(np.arange(50)), atol=1e-7)  # j = 0: angle = p exactly
    assert np.allclose(cos ** 2 + sin ** 2, 1, atol=2e-7)


def test_rope_tables_yarn_ramp_limits():
    # YaRN: dims below the ramp keep the base frequency, dims above interpolate by 1/factor
    base_c, _ = ref.rope_tables(1e6, 128, 40)
    y = {"factor": 4.0, "original_max_position_embeddings": 8192}
    c, _ = ref.rope_tables(1e6, 128, 40, y)
    msc = np.float32(0.1 * math.log(4.0) + 1)
    assert np.allclose(c[:, 0], np.float32(np.float64(base_c[:, 0]) * msc), atol=1e-6)
    inv_last = 1.0 / (4.0 * 1e6 ** (126 / 128))
    assert np.allclose(c[:, 63], (np.cos(np.arange(40) * inv_last) * float(msc)).astype(np.float32), atol=1e-6)


# ---------------------------------------------------------------- rmsnorm
def test_rmsnorm_constant_row_closed_form():
    x = np.full((3, 128), 2.0, np.float32)
    y = ref.rmsnorm(x, np.ones(128, np.float32), 1e-6)
    assert np.allclose(y, 2.0 / math.sqrt(4.0 + 1e-6), rtol=1e-7)


def test_rmsnorm_matches_float64_and_scale_invariance():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    g = rng.standard_normal(256).astype(np.float32)
    y = ref.rmsnorm(x, g, 1e-6)
    x64 = x.astype(np.float64)
    y64 = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * g
    assert np.allclose(y, y64, rtol=2e-6, atol=1e-6)
    assert np.allclose(ref.rmsnorm(x * 1000, g, 0.0), ref.rmsnorm(x, g, 0.0), rtol=1e-5)
    assert np.allclose(ref.rmsnorm_gemma(x, g - 1, 1e-6), y, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- rope apply
def test_rope_identity_norms_and_relative_position():
    rng = np.random.default_rng(1)
    cos, sin = ref.rope_tables(1e4, 64, 200)
    x = rng.standard_normal((3, 2, 64)).astype(np.float32)
    assert np.array_equal(ref.rope_apply(x, cos, sin, [0, 0, 0]), x)
    y = ref.rope_apply(x, cos, sin, [5, 50, 150])
    n_in = x[..., :32] ** 2 + x[..., 32:] ** 2
    n_out = y[..., :32] ** 2 + y[..., 32:] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)
    q, k = x[0:1], x[1:2]
    d1 = (ref.rope_apply(q, cos, sin, [30]) * ref.rope_apply(k, cos, sin, [10])).sum()
    d2 = (ref.rope_apply(q, cos, sin, [120]) * ref.rope_apply(k, cos, sin, [100])).sum()
    assert abs(d1 - d2) < 1e-4


def test_rope_direction_is_complex_multiplication():
    """Unit-vector closed form: with z = x_j + i*x_{j+h}, RoPE is z * exp(i*p*inv_j), so e_j
    goes to (cos, +sin) at dims (j, j+h) and e_{j+h} to (-sin, cos). A sign flip of the
    rotate_half term (tools/reference.py:151-152) exchanges the two sines and fails here."""
    theta, rot, D = 1e6, 128, 128
    h = rot // 2
    cos, sin = ref.rope_tables(theta, rot, 4000)
    for p in (1, 17, 3999):
        for j in (0, 5, h - 1):
            a = p * (1.0 / math.pow(theta, 2 * j / rot))
            c32, s32 = np.float32(math.cos(a)), np.float32(math.sin(a))
            ej = np.zeros((1, 1, D), np.float32)
            ej[0, 0, j] = 1
            y = ref.rope_apply(ej, cos, sin, [p])[0, 0]
            assert y[j] == c32 and y[j + h] == s32
            assert np.count_nonzero(y) == 2
            ejh = np.zeros((1, 1, D), np.float32)
            ejh[0, 0, j + h] = 1
            y = ref.rope_apply(ejh, cos, sin, [p])[0, 0]
            assert y[j] == -s32 and y[j + h] == c32
    # a general vector against Python complex arithmetic in f64 (partial rotation, rot = 64)
    rng = np.random.default_rng(11)
    cos, sin = ref.rope_tables(1e7, 64, 300)
    x = rng.standard_normal((1, 1, 256)).astype(np.float32)
    y = ref.rope_apply(x, cos, sin, [257], rot=64)[0, 0]
    for j in range(32):
        a = 257 * (1.0 / math.pow(1e7, 2 * j / 64))
        z = complex(float(x[0, 0, j]), float(x[0, 0, j + 32])) * complex(math.cos(a), math.sin(a))
        assert abs(y[j] - z.real) < 1e-6 and abs(y[j + 32] - z.imag) < 1e-6
    assert np.array_equal(y[64:], x[0, 0, 64:])


def test_rope_partial_passthrough_and_reference_case():
    from tests.golden.make_golden import reference_kernel_case_inputs
    g = np.load(os.path.join(ROOT, "tests", "golden", "ref_kernel_cases.npz"))
    xr = reference_kernel_case_inputs()[0]
    assert np.array_equal(xr, g["rope_x"])            # the reference's seed-0 draw sequence
    y = ref.rope_apply(xr, g["rope_cos"][:, :32], g["rope_sin"][:, :32], np.arange(5), rot=64)
    assert np.array_equal(y[..., 64:], xr[..., 64:])  # dims >= ROT pass through
    assert np.array_equal(y, g["rope_expected"])
    # the reference tables (gen-kernel-cases.py:95-97) equal the synthRope recipe
    c, s = ref.rope_tables(1e7, 64, 5)
    assert np.array_equal(np.concatenate([c, c], -1), g["rope_cos"])
    assert np.array_equal(np.concatenate([s, s], -1), g["rope_sin"])


# ---------------------------------------------------------------- attention
def _brute_attention(q, k, v, pos_base, scale):
    S, H, D = q.shape
    KV = k.shape[1]
    out = np.zeros((S, H, D))
    for s in range(S):
        for h in range(H):
            kvh = h // (H // KV)
            sc = [float(np.dot(q[s, h].astype(np.float64), k[j, kvh].astype(np.float64))) * scale
                  for j in range(pos_base + s + 1)]
            m = max(sc)
            w = [math.exp(x - m) for x in sc]
            z = sum(w)
            for j, wj in enumerate(w):
                out[s, h] += wj / z * v[j, kvh].astype(np.float64)
    return out


def test_attention_bruteforce_gqa():
    rng = np.random.default_rng(2)
    S, H, KV, D, pb = 3, 6, 2, 16, 4
    q = rng.standard_normal((S, H, D)).astype(np.float32)
    k = rng.standard_normal((pb + S, KV, D)).astype(np.float32)
    v = rng.standard_normal((pb + S, KV, D)).astype(np.float32)
    got = ref.attention(q, k, v, pb)
    want = _brute_attention(q, k, v, pb, 1 / math.sqrt(D))
    assert np.allclose(got, want, atol=1e-6)


def test_attention_invariants():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 4, 32)).astype(np.float32)
    k = rng.standard_normal((10, 2, 32)).astype(np.float32)
    vu = np.broadcast_to(rng.standard_normal((1, 2, 32)), (10, 2, 32)).astype(np.float32)
    assert np.allclose(ref.attention(q, k, vu, 9), np.repeat(vu[:1], 2, 1), atol=1e-6)  # uniform V
    k1 = k[:1]
    v1 = rng.standard_normal((1, 2, 32)).astype(np.float32)
    assert np.allclose(ref.attention(q, k1, v1, 0), np.repeat(v1, 2, 1), atol=1e-7)   # single key
    kd = np.zeros_like(k)
    kd[6] = q[0, :2] * 100                                                             # one dominant key
    v = rng.standard_normal((10, 2, 32)).astype(np.float32)
    o = ref.attention(q, kd, v, 9)
    assert np.allclose(o[0, 0], v[6, 0], atol=1e-5)


def test_attention_reference_kernel_case(cref):
    from tests.golden.make_golden import reference_kernel_case_inputs
    g = np.load(os.path.join(ROOT, "tests", "golden", "ref_kernel_cases.npz"))
    _, q, k, v = reference_kernel_case_inputs()
    got = ref.attention(q, k, v, 0, scale=1.0 / np.sqrt(256))
    assert np.array_equal(got, g["att_expected"])
    want = np.zeros_like(got)
    cref.oracle_attention_f64(_p(q), _p(k), _p(v), None, 6, 4, 2, 256, 6, 0, 1.0 / math.sqrt(256), _p(want))
    assert np.abs(got - want).max() < 1e-6


def test_sigmoid_closed_forms():
    """tools/qwen35_numpy.py:58-59 and gate_sigmoid.wgsl:13: sigma(0) = 1/2, sigma(x) +
    sigma(-x) = 1, saturation, and agreement with Python's 1/(1+math.exp(-x))."""
    x = np.array([0.0, 1.0, -1.0, 3.5, -7.25, 20.0, -20.0, 1e-4, 88.0, -88.0], np.float32)
    s = ref.sigmoid(x)
    assert s[0] == np.float32(0.5)
    for xi, si in zip(x, s):
        want = 1.0 / (1.0 + math.exp(-float(xi)))
        assert abs(float(si) - want) <= 2 * float(np.spacing(np.float32(want)))
    rng = np.random.default_rng(12)
    r = (rng.standard_normal(1000) * 4).astype(np.float32)
    assert np.allclose(ref.sigmoid(r) + ref.sigmoid(-r), 1.0, atol=1.2e-7)
    assert ref.sigmoid(np.float32(-200)) == 0 and ref.sigmoid(np.float32(200)) == 1
    assert np.all(np.diff(ref.sigmoid(np.sort(r))) >= 0)                     # monotone


def test_gated_attention_bruteforce():
    """Gated full attention (tools/qwen35_numpy.py:102-114) against an f64 loop with math.exp
    for the softmax and for the gate 1/(1+exp(-g)); scale 1/sqrt(D) (qwen35_numpy.py:105)."""
    rng = np.random.default_rng(13)
    S, H, KV, D, pb = 3, 6, 2, 16, 5
    q = rng.standard_normal((S, H, D)).astype(np.float32)
    k = rng.standard_normal((pb + S, KV, D)).astype(np.float32)
    v = rng.standard_normal((pb + S, KV, D)).astype(np.float32)
    g = rng.standard_normal((S, H, D)).astype(np.float32) * 3
    got = ref.gated_attention(q, k, v, g, pb)
    att = _brute_attention(q, k, v, pb, 1 / math.sqrt(D))
    gate = np.vectorize(lambda t: 1.0 / (1.0 + math.exp(-t)))(g.astype(np.float64))
    assert np.allclose(got, att * gate, atol=2e-6)
    # a gate of +inf-like size passes the attention through, a very negative one zeroes it
    big = np.full_like(g, 100)
    assert np.allclose(ref.gated_attention(q, k, v, big, pb), att, atol=2e-6)
    assert np.all(ref.gated_attention(q, k, v, -big, pb) == 0)


# ---------------------------------------------------------------- q8 quantizer
def _exact_code(v, s):
    """WGSL pack4x8snorm on v/s with every f32 step rounded exactly (Fractions)."""
    f = lambda x: Fraction(float(np.float32(x)))  # noqa: E731
    e = Fraction(float(np.float32(np.float32(v) / np.float32(s))))
    e = max(Fraction(-1), min(Fraction(1), e))
    t = f(float(np.float32(127) * np.float32(float(e))))
    u = f(float(np.float32(float(t)) + np.float32(0.5)))
    return math.floor(u)


def test_q8_special_cases():
    z = np.zeros((1, 64), np.float32)
    c, s = ref.q8_pack(z)
    assert np.all(c == 0) and np.all(s == np.float32(1e-30))
    c, s = ref.q8_pack(-z)
    assert np.all(c == 0)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    c, s = ref.q8_pack(x)
    xb = x.reshape(8, 4, 32)
    cb = c.reshape(8, 4, 32)
    am = np.abs(xb).argmax(-1)
    for r in range(8):
        for b in range(4):
            i = am[r, b]
            assert cb[r, b, i] == (127 if xb[r, b, i] > 0 else -127)   # block max -> +-127
            assert s[r, b] == np.abs(xb[r, b]).max()
    assert np.abs(c.astype(np.int32)).max() <= 127


def test_q8_tie_rounds_up_not_to_even():
    # search half-integer values v with block scale 127 whose f32 steps land exactly on a tie
    ties = []
    for k2 in range(-253, 254, 2):
        v = np.float32(k2 / 2)
        e = np.float32(v / np.float32(127))
        t = np.float32(np.float32(127) * e)
        if t == v:  # 127 * fl(v/127) returned v exactly: a genuine .5 tie
            ties.append(float(v))
    assert any(int(math.floor(t)) % 2 == 0 for t in ties if t > 0)   # RNE would round these down
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127
    for t in ties[:31]:
        x[0, 1] = t
        c, _ = ref.q8_pack(x)
        assert c[0, 1] == math.floor(t + 0.5)


def test_q8_matches_exact_arithmetic_grid():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((16, 32)) * np.exp(rng.uniform(-8, 8, (16, 1)))).astype(np.float32)
    c, s = ref.q8_pack(x)
    for r in range(16):
        for i in range(32):
            assert c[r, i] == _exact_code(x[r, i], s[r, 0])


def test_q8_c_restatement_and_golden(cref):
    g = np.load(os.path.join(ROOT, "tests", "golden", "q8_cases.npz"))
    x = g["x"]
    codes = np.zeros(x.shape, np.int8)
    scales = np.zeros((x.shape[0], x.shape[1] // 32), np.float32)
    cref.oracle_q8_pack(_p(x), x.shape[0], x.shape[1], 32, _p(codes), _p(scales))
    c2, s2 = ref.q8_pack(x)
    assert np.array_equal(codes, c2) and np.array_equal(scales.view(np.uint32), s2.view(np.uint32))
    assert np.array_equal(codes, g["codes"]) and np.array_equal(scales, g["scales"])
    deq = np.zeros_like(x)
    cref.oracle_q8_dequant(_p(codes), _p(scales), x.shape[0], x.shape[1], 32, _p(deq))
    assert np.array_equal(deq, ref.q8_dequant(codes, scales))
    assert np.array_equal(deq, g["dequant"])


# ---------------------------------------------------------------- f16 quantizer
def test_f16_matches_struct_rne(cref):
    g = np.load(os.path.join(ROOT, "tests", "golden", "f16_cases.npz"))
    x = g["x"]
    bits = ref.f16_pack(x).view(np.uint16)
    for xi, b in zip(x, bits):
        try:
            want = struct.unpack("<H", struct.pack("<e", float(xi)))[0]
        except OverflowError:
            want = 0x7C00 if xi > 0 else 0xFC00
        assert b == want
    out = np.zeros(x.shape, np.uint16)
    cref.oracle_f16_pack(_p(x), x.size, _p(out))
    assert np.array_equal(out, bits) and np.array_equal(bits, g["bits"])


# ---------------------------------------------------------------- eviction
def _literal_evict(cache, fill, need, sinks, max_seq):
    recent = fill - sinks
    batch = min(recent, max(need, -(-(max_seq - sinks) // 4)))
    keep = recent - batch
    if keep <= 0:
        return cache[:sinks], sinks
    scratch = cache[sinks + batch: sinks + batch + keep]
    new = cache[:sinks] + scratch
    return new, sinks + keep


def test_evict_closed_form_exhaustive():
    for max_seq in (68, 100, 4100):
        sinks = 4
        for fill in range(sinks, max_seq + 1, max(1, max_seq // 37)):
            for need in (0, 1, 4, 9, 50, max_seq):
                nf, b, k = ref.evict(fill, need, sinks, max_seq)
                cache = list(range(fill))
                new, nf2 = _literal_evict(cache, fill, need, sinks, max_seq)
                assert nf == nf2 and len(new) == nf


def test_sink_schedule_golden():
    g = np.load(os.path.join(ROOT, "tests", "golden", "sink_schedule.npz"))
    slots, fill, events = ref.simulate_sink_schedule(1000, 100_000, 4, 4100)
    assert fill == int(g["fill"]) and np.array_equal(np.array(slots), g["slots"])
    assert np.array_equal(np.array(events).reshape(-1, 3), g["events"])
    s = np.array(slots)
    assert list(s[:4]) == [0, 1, 2, 3]                        # sinks never move
    assert np.all(np.diff(s[4:]) == 1) and s[-1] == 99_999    # the recent window is contiguous


# ---------------------------------------------------------------- 1-bit projections
def test_sign_bit_order_one_bit_at_a_time():
    """Bit k % 32 of word k // 32 is weight k (shaders/matmul_split_sg.wgsl:29-32), set = +1."""
    K = 256
    for k in (0, 1, 31, 32, 77, 255):
        sign = np.zeros((1, K // 32), np.uint32)
        sign[0, k // 32] = np.uint32(1) << np.uint32(k % 32)
        w = ref.unpack_signs(sign, K)[0]
        assert w[k] == 1.0 and np.sum(w == 1.0) == 1 and np.sum(w == -1.0) == K - 1


def test_gemv_closed_forms():
    rng = np.random.default_rng(21)
    K = 512
    x = rng.standard_normal(K).astype(np.float32)
    sc = np.abs(rng.standard_normal((2, K // 128))).astype(np.float32)
    sign = np.zeros((2, K // 32), np.uint32)
    sign[0] = 0xFFFFFFFF                                   # all +1
    y = ref.gemv_1bit(x, sign, sc)
    xb = x.astype(np.float64).reshape(K // 128, 128).sum(-1)
    assert np.allclose(y[0], sc[0] @ xb, rtol=1e-6) and np.allclose(y[1], -(sc[1] @ xb), rtol=1e-6)
    r = rng.standard_normal(2).astype(np.float32)
    assert np.allclose(ref.gemv_1bit(x, sign, sc, r), y.astype(np.float64) + r, rtol=1e-6)


def test_gemv_matches_wgsl_loop():
    """Literal restatement of matmul_resid_mr_sg.wgsl's per-lane loop: vec4 groups, the 4 bits
    at (word >> (k & 31)) & 0xf, dot times the block scale, then the cross-lane sum."""
    rng = np.random.default_rng(22)
    N, K, SG = 3, 384, 32
    x = rng.standard_normal(K).astype(np.float32)
    sign = rng.integers(0, 2 ** 32, (N, K // 32), dtype=np.uint64).astype(np.uint32)
    sc = np.abs(rng.standard_normal((N, K // 128))).astype(np.float32)
    resid = rng.standard_normal(N).astype(np.float32)
    want = np.zeros(N)
    for n in range(N):
        lanes = []
        for lane in range(SG):
            acc = 0.0
            for gi in range(lane, K // 4, SG):
                k = gi * 4
                bits4 = (int(sign[n, k >> 5]) >> (k & 31)) & 0xF
                sv = [1.0 if (bits4 >> i) & 1 else -1.0 for i in range(4)]
                acc += sum(float(x[k + i]) * sv[i] for i in range(4)) * float(sc[n, k // 128])
            lanes.append(acc)
        want[n] = sum(lanes) + float(resid[n])
    assert np.allclose(ref.gemv_1bit(x, sign, sc, resid), want, rtol=1e-6, atol=1e-6)
