"""CPU: the algorithmic work every roofline fraction of bench.py rests on, against the figures
the benchmark configurations state (bytes of one q8 decode layer, causal prefill FLOPs, prologue
bytes), and the one-GPU contract (``--gpus`` above 1 exits with a message before touching a GPU)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from bitgpu_amd import workloads as W  # noqa: E402


@pytest.mark.parametrize("L,want", [(4096, 9_469_952), (16384, 37_781_504), (32768, 75_530_240)])
def test_c3_layer_bytes(L, want):
    # K and V: L rows x 8 kv heads x (128 code bytes + 4 f32 scales of 32 values); f32 q and out
    assert bench.c3_bytes(L) == want
    assert want == L * 8 * 2 * 128 + L * 8 * 2 * 4 * 4 + 2 * 32 * 128 * 4


def test_causal_prefill_flops():
    # 2 (QK and PV) x 2 (multiply-add) x D x H x sum over queries of the keys each attends
    # 2*D*H*S*(S+1): C2 34.38 GFLOP, C5 824.7 GFLOP
    assert bench.causal_flops(2048, 32, 128) == 2 * 128 * 32 * 2048 * 2049 == 34_376_515_584
    assert bench.causal_flops(8192, 24, 256) == 2 * 256 * 24 * 8192 * 8193 == 824_734_384_128
    brute = sum(4 * 128 * 32 * (100 + s + 1) for s in range(50))
    assert bench.causal_flops(50, 32, 128, past=100) == brute


def test_prologue_bytes():
    # Q read and written as f32; K and V read as f32 and written in the storage format
    c2 = 2 * 2048 * 32 * 128 * 4 + 2 * 2048 * 8 * 128 * 4 + 2 * 2048 * 8 * 128 * 2
    assert bench.prologue_bytes(W.C2, 2048) == c2 == 92_274_688
    c5 = 2 * 8192 * 24 * 256 * 4 + 2 * 8192 * 4 * 256 * 4 + 2 * 8192 * 4 * 256 * 1 + 2 * 8192 * 4 * 8 * 4
    assert bench.prologue_bytes(W.C5, 8192) == c5 == 488_636_416


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
