"""GPU: the decode kernel's split merge fails loudly. A host-set test hook makes one split store
no partial and bounds the mergers' wait to a few rounds (bg_debug_merge_hooks), so the merge gives up while every
kernel still exits normally; the launch stores NaN, and the next bg_attention on the cache (or
bg_stream_sync) returns BG_E_DEVICE once, after resetting the split workspace. Later launches
match the oracle again."""
import numpy as np
import pytest
import torch

from bitgpu_amd import _lib
from bitgpu_amd import engine as E
from bitgpu_amd._lib import BitgpuError
from oracle import ref
from tests.conftest import rel_err
from tests.gpu_helpers import cached_values, fill_cache_raw, t

pytestmark = pytest.mark.gpu


def _case(dtype, L=8192, seed=71):
    rng = np.random.default_rng(seed)
    H, KV, D = 32, 8, 128
    k = rng.standard_normal((L, KV, D)).astype(np.float32)
    v = rng.standard_normal((L, KV, D)).astype(np.float32)
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    c = E.KvCache(1, KV, D, dtype, max_seq_len=L, capacity=L)
    fill_cache_raw(c, 0, k, v)
    kk, vv = cached_values(c, 0, 0, L)
    return c, t(q), ref.attention(q, kk, vv, L - 1), H


@pytest.mark.parametrize("dtype,report", [("q8", "attention"), ("f16", "stream_sync")])
def test_merge_timeout_is_reported(dev, dtype, report):
    c, q, exp, H = _case(dtype)
    L = 8192
    good = E.attention(c, 0, q, 1, H, L - 1)
    torch.cuda.synchronize()
    assert rel_err(good.cpu().numpy(), exp) <= 2e-3
    _lib.check(_lib.lib().bg_debug_merge_hooks(32, 1))  # a poll bound of 32 rounds, split 1 withheld
    try:
        bad = E.attention(c, 0, q, 1, H, L - 1)      # enqueued fine: the failure is on the GPU
        torch.cuda.synchronize()
    finally:
        _lib.check(_lib.lib().bg_debug_merge_hooks(0, -1))
    assert np.isnan(bad.cpu().numpy()).all()          # every unit waits on the withheld split
    with pytest.raises(BitgpuError, match="gave up waiting") as ei:
        if report == "attention":
            E.attention(c, 0, q, 1, H, L - 1)
        else:
            _lib.check(_lib.lib().bg_stream_sync(None))
    assert ei.value.code == _lib.BG_E_DEVICE
    _lib.check(_lib.lib().bg_stream_sync(None))        # reported once
    again = E.attention(c, 0, q, 1, H, L - 1)
    torch.cuda.synchronize()
    assert rel_err(again.cpu().numpy(), exp) <= 2e-3
    assert torch.equal(again, good)
    c.close()
