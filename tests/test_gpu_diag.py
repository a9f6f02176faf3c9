"""GPU: the streaming-read floor kernel (bg_diag_stream_read) reads every 16 bytes of its buffer
exactly once for any workgroup count: the XOR of its per-workgroup words equals the XOR of the
buffer's 32-bit words (a byte read twice or skipped changes it)."""
import ctypes as C

import numpy as np
import pytest
import torch

from bitgpu_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_words", [4, 4 * 1000 + 4, 1 << 20, 3 * (1 << 20) + 12])
@pytest.mark.parametrize("workgroups", [1, 7, 256, 1000])
@pytest.mark.parametrize("nontemporal", [1, 0])
def test_stream_read_covers_buffer_once(dev, n_words, workgroups, nontemporal):
    rng = np.random.default_rng(n_words + workgroups)
    host = rng.integers(0, 2 ** 32, size=n_words, dtype=np.uint64).astype(np.uint32)
    buf = torch.from_numpy(host.view(np.int32)).cuda()
    sink = torch.full((workgroups,), -1, dtype=torch.int32, device="cuda")
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().bg_diag_stream_read(C.c_void_p(buf.data_ptr()), n_words * 4, workgroups, nontemporal,
                                               C.c_void_p(sink.data_ptr()), st))
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host)
