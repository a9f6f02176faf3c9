"""Helpers shared by the GPU parity tests: run the product path (C ABI through bitgpu_amd.engine)
and build the matching oracle inputs."""
import numpy as np
import torch

from bitgpu_amd import engine as E
from bitgpu_amd._lib import BG_K, BG_KSCALE, BG_V, BG_VSCALE
from oracle import ref

DEV = "cuda"


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def export_k_v(cache, li, base, count):
    """Exported K/V (+ scales) of logical positions [base, base+count) as numpy arrays."""
    KV, D = cache.kv_heads, cache.head_dim
    if cache.kv_cache == "f32":
        dt = np.float32
    elif cache.kv_cache == "f16":
        dt = np.float16
    else:
        dt = np.int8
    k = np.frombuffer(cache.export_rows(li, BG_K, base, count), dt).reshape(count, KV, D)
    v = np.frombuffer(cache.export_rows(li, BG_V, base, count), dt).reshape(count, KV, D)
    if cache.kv_cache == "q8":
        ks = np.frombuffer(cache.export_rows(li, BG_KSCALE, base, count), np.float32).reshape(count, KV, D // 32)
        vs = np.frombuffer(cache.export_rows(li, BG_VSCALE, base, count), np.float32).reshape(count, KV, D // 32)
        return k, v, ks, vs
    return k, v, None, None


def cached_values(cache, li, base, count):
    """What the kernels read back for the exported rows, as f32."""
    k, v, ks, vs = export_k_v(cache, li, base, count)
    if cache.kv_cache == "q8":
        return ref.q8_dequant(k, ks), ref.q8_dequant(v, vs)
    return k.astype(np.float32), v.astype(np.float32)


def rope_dev(theta, rot, positions):
    c, s = E.rope_tables(theta, rot, positions)
    return t(c), t(s), c, s


def fill_cache_raw(cache, li, k, v, row0=0):
    """appendKV of raw K and V rows (no norm/rope) at positions row0.."""
    L, KV, D = k.shape
    cache.append_kv(t(k), BG_K, li, L * KV, row0 * KV)
    cache.append_kv(t(v), BG_V, li, L * KV, row0 * KV)


def run_attention_noalloc(cache, li, q, pos_base, scale=None, gate=None):
    """bg_attention_noalloc through the C ABI (torch tensors in, numpy out after a sync)."""
    import ctypes as C
    from bitgpu_amd import _lib
    S, H, D = q.shape
    qt = t(q)
    gt = t(gate) if gate is not None else None
    out = torch.full((S, H, D), float("nan"), dtype=torch.float32, device=DEV)
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().bg_attention_noalloc(cache.handle, li, C.c_void_p(qt.data_ptr()), S, H, pos_base,
                                               float(scale), None if gt is None else C.c_void_p(gt.data_ptr()),
                                               D if gt is not None else 0, C.c_void_p(out.data_ptr()), st))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def run_attention(cache, li, q, pos_base, scale=None, gate=None):
    S, H, D = q.shape
    g = t(gate) if gate is not None else None
    out = E.attention(cache, li, t(q), S, H, pos_base, scale=scale, gate=g, gate_stride=D if gate is not None else None)
    torch.cuda.synchronize()
    return out.cpu().numpy()
