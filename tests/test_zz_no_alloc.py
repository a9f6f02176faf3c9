"""GPU: bg_attention_noalloc (the allocation-free variant of bg_attention, whose decode split
partials live in the library's static per-GPU scratch array) gives bg_attention's results:
bit-identical for f16 / q8 (same kernels and split plan; a q8 prefill staged in-kernel holds the
f16 copy's exact values), within max-abs 1e-4 for f32 (exact-f32 kernel without partials). Each
case makes two calls in a row, the second with a smaller input; a launch whose partials would
not fit the scratch is rejected before anything runs."""
import ctypes as C

import numpy as np
import pytest
import torch

from bitgpu_amd import _lib
from bitgpu_amd import engine as E
from bitgpu_amd._lib import BitgpuError
from tests.gpu_helpers import fill_cache_raw, rope_dev, t

pytestmark = pytest.mark.gpu


def _noalloc(cache, li, q, S, H, pos_base, scale=None, gate=None, gate_stride=0):
    D = cache.head_dim
    out = torch.full((S, H, D), float("nan"), dtype=torch.float32, device=q.device)
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().bg_attention_noalloc(cache.handle, li, C.c_void_p(q.data_ptr()), S, H, pos_base,
                                               float(scale), None if gate is None else C.c_void_p(gate.data_ptr()),
                                               gate_stride, C.c_void_p(out.data_ptr()), st))
    return out


def _cache(dtype, H, KV, D, L, seed, layers=1):
    rng = np.random.default_rng(seed)
    c = E.KvCache(layers, KV, D, dtype, max_seq_len=L, capacity=L)
    for li in range(layers):
        fill_cache_raw(c, li, rng.standard_normal((L, KV, D)).astype(np.float32),
                       rng.standard_normal((L, KV, D)).astype(np.float32))
    return c, rng


# (dtype, H, KV, D, cache positions, [(S, attended positions), (smaller S, fewer positions)], gated)
CASES = [
    ("q8", 32, 8, 128, 32768, [(1, 32768), (1, 4096)], False),       # C3 decode, 32k then 4k
    ("f16", 32, 8, 128, 4100, [(5, 4100), (1, 1000)], False),        # verify 5 then decode
    ("q8", 24, 4, 256, 8448, [(1, 8448), (1, 2000)], True),          # hybrid decode, gated
    ("q8", 32, 8, 128, 2048, [(600, 2048), (130, 700)], False),      # prefill: copy path vs in-kernel
    ("f16", 32, 8, 128, 2048, [(512, 2048), (64, 300)], False),      # f16 prefill
    ("f32", 16, 8, 128, 2048, [(1, 513), (1, 100)], False),          # f32 decode (C1 shape)
    ("q8", 24, 4, 256, 8448, [(8, 8448), (4, 3000)], True),          # split-K prefill (hybrid verify)
    ("f16", 32, 8, 128, 8192, [(64, 8128), (32, 2000)], False),      # split-K prefill chunk
]


@pytest.mark.parametrize("dtype,H,KV,D,L,calls,gated", CASES)
def test_noalloc_matches_bg_attention(dev, dtype, H, KV, D, L, calls, gated):
    c, rng = _cache(dtype, H, KV, D, L, seed=L + H)
    for S, upto in calls:
        q = t(rng.standard_normal((S, H, D)).astype(np.float32))
        g = t(rng.standard_normal((S, H, D)).astype(np.float32)) if gated else None
        scale = 1.0 / np.sqrt(D) if gated else None
        want = E.attention(c, 0, q, S, H, upto - S, scale=scale, gate=g, gate_stride=D if gated else None)
        got = _noalloc(c, 0, q, S, H, upto - S, scale=scale, gate=g, gate_stride=D if gated else 0)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        if dtype == "f32":
            assert float((got - want).abs().max()) <= 1e-4
        else:
            assert torch.equal(got, want)
    c.close()


@pytest.mark.parametrize("dtype", ["f16", "q8"])
def test_noalloc_matches_bg_attention_sink_ring(dev, dtype):
    """Sink mode with the ring wrapped (read-time rotation, splits numbered in groups per kv head):
    decode and a 5-row verify, bit-identical to bg_attention, twice each."""
    KV, H, D, sinks, window = 8, 32, 128, 4, 700
    max_seq = sinks + window
    c = E.KvCache(1, KV, D, dtype, max_seq_len=max_seq, overflow="sinks", sink_tokens=sinks)
    cos_d, sin_d, _, _ = rope_dev(1e6, D, max_seq)
    c.set_rope(cos_d, sin_d)
    rng = np.random.default_rng(91)
    fill_cache_raw(c, 0, rng.standard_normal((max_seq, KV, D)).astype(np.float32),
                   rng.standard_normal((max_seq, KV, D)).astype(np.float32))
    fill, fed = 500, 500
    while fed < 3000:
        fill = c.evict_for(fill, 4) + 4
        fed += 4
    for S in (1, 5, 1):
        fill = c.evict_for(fill, S)
        assert c.ring_state()[0] != 0
        q = t(rng.standard_normal((S, H, D)).astype(np.float32))
        want = E.attention(c, 0, q, S, H, fill)
        got = _noalloc(c, 0, q, S, H, fill)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all() and torch.equal(got, want)
    c.close()


def test_noalloc_rejects_partials_beyond_the_scratch(dev):
    # 200 kv heads x 48 rows x 2 splits of decode partials = 10.4 MB > the 8 MiB scratch (a
    # sink-mode cache: its 48-row verify stays on the decode kernel)
    H = KV = 200
    c = E.KvCache(1, KV, 128, "q8", max_seq_len=4096, overflow="sinks", sink_tokens=4)
    cos_d, sin_d, _, _ = rope_dev(1e6, 128, 4096)
    c.set_rope(cos_d, sin_d)
    q = t(np.zeros((48, H, 128), np.float32))
    with pytest.raises(BitgpuError, match="beyond the 8388608-byte scratch") as ei:
        _noalloc(c, 0, q, 48, H, 4096 - 48)
    assert ei.value.code == _lib.BG_E_INVALID
    c.close()
