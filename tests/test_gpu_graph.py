"""GPU: attention launches captured in a HIP graph and replayed.

bg_attention_reserve sizes everything a shape needs (split-K workspace, the split prefill's (m, l)
buffer, a q8 cache's f16 copy), so the launch can be captured; the captured kernels keep no state
between launches except the workspace slots, which every launch leaves holding the empty marker
(no memset is recorded: the kernels write the marker back themselves). Each graph is replayed
several times with eager launches of other shapes on the same cache in between, and every replay
must give the eager result bit for bit. The allocation-free entry point is captured the same way
after its first (set-up) call ran eagerly."""
import numpy as np
import pytest
import torch

from bitgpu_amd import _lib
from bitgpu_amd import engine as E
from tests.gpu_helpers import fill_cache_raw, run_attention_noalloc, t

pytestmark = pytest.mark.gpu

# (dtype, H, KV, D, cached positions, S, gated): split-K decode, decode of two row sets (q8
# D=128, 24 rows), split-K prefill (hybrid verify, D=128 chunk), plain prefill
SHAPES = [
    ("q8", 32, 8, 128, 8192, 1, False),
    ("q8", 32, 8, 128, 4096, 6, False),
    ("q8", 24, 4, 256, 8200, 8, True),
    ("f16", 32, 8, 128, 8000, 64, False),
    ("f16", 32, 8, 128, 2048, 2048, False),
]


def _inputs(dtype, H, KV, D, L, S, gated, seed):
    rng = np.random.default_rng(seed)
    c = E.KvCache(1, KV, D, dtype, max_seq_len=L, capacity=L)
    fill_cache_raw(c, 0, rng.standard_normal((L, KV, D)).astype(np.float32),
                   rng.standard_normal((L, KV, D)).astype(np.float32))
    q = t(rng.standard_normal((S, H, D)).astype(np.float32))
    g = t(rng.standard_normal((S, H, D)).astype(np.float32)) if gated else None
    return c, q, g


def _replay_and_check(g, out, want, between):
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        between()
        torch.cuda.synchronize()


@pytest.mark.parametrize("dtype,H,KV,D,L,S,gated", SHAPES)
def test_graph_replay_matches_eager(dev, dtype, H, KV, D, L, S, gated):
    c, q, gate = _inputs(dtype, H, KV, D, L, S, gated, seed=L + S)
    scale = 1.0 / np.sqrt(D)
    gs = D if gated else None
    # every shape this cache runs is reserved before the capture: a workspace grown later would
    # be reallocated under the captured launch
    for rows in (1, 3, S):
        _lib.check(_lib.lib().bg_attention_reserve(c.handle, rows, H))
    want = E.attention(c, 0, q, S, H, L - S, scale=scale, gate=gate, gate_stride=gs)
    torch.cuda.synchronize()
    # eager launches of other shapes on the same cache between the replays (decode, verify)
    q1 = t(np.random.default_rng(1).standard_normal((3, H, D)).astype(np.float32))
    between = lambda: (E.attention(c, 0, q1[:1], 1, H, L - 1, scale=scale),
                       E.attention(c, 0, q1, 3, H, L - 3, scale=scale))
    out = torch.empty_like(want)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            E.attention(c, 0, q, S, H, L - S, scale=scale, gate=gate, gate_stride=gs, out=out)
    torch.cuda.synchronize()
    _replay_and_check(graph, out, want, between)
    c.close()


def test_graph_survives_workspace_growth(dev):
    """A decode captured with only its own shape reserved; then an eager split-K prefill grows the
    cache's workspace (a new, larger buffer): the captured decode keeps the buffer it was captured
    with (the cache retires it instead of freeing it) and still replays to the eager result."""
    H, KV, D, L = 24, 4, 256, 8200
    c, q, gate = _inputs("q8", H, KV, D, L, 1, True, seed=11)
    scale = 1.0 / 16
    _lib.check(_lib.lib().bg_attention_reserve(c.handle, 1, H))
    want = E.attention(c, 0, q, 1, H, L - 1, scale=scale, gate=gate, gate_stride=D)
    out = torch.empty_like(want)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            E.attention(c, 0, q, 1, H, L - 1, scale=scale, gate=gate, gate_stride=D, out=out)
    torch.cuda.synchronize()
    q8 = t(np.random.default_rng(3).standard_normal((8, H, D)).astype(np.float32))
    between = lambda: E.attention(c, 0, q8, 8, H, L - 8, scale=scale)   # split-K prefill: grows the workspace
    _replay_and_check(graph, out, want, between)
    c.close()


@pytest.mark.parametrize("dtype,H,KV,D,L,S,gated", [SHAPES[0], SHAPES[2]])
def test_graph_replay_noalloc(dev, dtype, H, KV, D, L, S, gated):
    """bg_attention_noalloc captured after an eager call: decode split partials and split-K
    prefill partials in the static scratch, every replay equal to that eager call's result."""
    import ctypes as C
    c, q, gate = _inputs(dtype, H, KV, D, L, S, gated, seed=7 + S)
    scale = 1.0 / np.sqrt(D)
    qn, gn = q.cpu().numpy(), None if gate is None else gate.cpu().numpy()
    want_np = run_attention_noalloc(c, 0, qn, L - S, scale=scale, gate=gn)   # the eager set-up call
    want = torch.from_numpy(want_np).cuda()
    out = torch.empty_like(want)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
            _lib.check(_lib.lib().bg_attention_noalloc(
                c.handle, 0, C.c_void_p(q.data_ptr()), S, H, L - S, float(scale),
                None if gate is None else C.c_void_p(gate.data_ptr()), D if gate is not None else 0,
                C.c_void_p(out.data_ptr()), st))
    torch.cuda.synchronize()
    q1 = t(np.random.default_rng(2).standard_normal((1, H, D)).astype(np.float32))
    _replay_and_check(graph, out, want, lambda: run_attention_noalloc(c, 0, q1.cpu().numpy(), L - 1, scale=scale))
    c.close()
