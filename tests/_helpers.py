"""Helpers shared by the GPU tests: seeded inputs, paged layouts, device round trips."""
from __future__ import annotations

import sys

import numpy as np

from kvcache_amd import KVC_F16, KVC_F32
from kvcache_amd.device import DeviceBuffer, np_dtype


def say(msg: str) -> None:
    """Names the case on stdout before a GPU step (flushed, so it survives a crash)."""
    print(msg, flush=True)
    sys.stdout.flush()


def normal(shape, seed, dtype=np.float32):
    return np.random.default_rng(seed).standard_normal(shape).astype(dtype)


def dev(a: np.ndarray) -> DeviceBuffer:
    return DeviceBuffer.from_numpy(a)


def host(buf: DeviceBuffer, dtype, shape) -> np.ndarray:
    return buf.to_numpy(dtype, shape)


def paged_layout(K, V, lens, block, perm=None):
    """Scatter contiguous K/V [N, Hkv, S, D] into a pool [NB, Hkv, block, D].

    Logical block b of sequence s goes to physical block perm[global b] (identity
    when perm is None), the layout of bench_throughput.cu:62-102.
    Returns (k_pool, v_pool, table_all, tab_off)."""
    N, Hkv, S, D = K.shape
    nb = [(int(L) + block - 1) // block for L in lens]
    total = int(sum(nb))
    tab_off = np.concatenate([[0], np.cumsum(nb)]).astype(np.int32)
    table = np.arange(total, dtype=np.int32) if perm is None else np.asarray(perm, np.int32)[:total]
    NB = max(total, int(table.max()) + 1 if total else 1)  # a permutation may point past `total`
    kp = np.zeros((NB, Hkv, block, D), K.dtype)
    vp = np.zeros_like(kp)
    for s in range(N):
        L = int(lens[s])
        for b in range(nb[s]):
            t0, t1 = b * block, min((b + 1) * block, L)
            phys = table[tab_off[s] + b]
            kp[phys, :, : t1 - t0] = K[s, :, t0:t1]
            vp[phys, :, : t1 - t0] = V[s, :, t0:t1]
    return kp, vp, table, tab_off


def tol(dtype: int) -> float:
    """Parity bars from the path's spec: fp32 KV 1e-5, fp16 KV 2e-3 (max abs)."""
    return 2e-3 if dtype == KVC_F16 else 1e-5


def as_np(dtype: int):
    return np_dtype(dtype)


__all__ = ["say", "normal", "dev", "host", "paged_layout", "tol", "as_np", "KVC_F16", "KVC_F32"]


class tuning:
    """Sets a library tuning knob for the duration of a with-block."""

    def __init__(self, key: str, value: int):
        self.key, self.value = key.encode(), value

    def __enter__(self):
        import ctypes as C

        from kvcache_amd._native import check, lib
        old = C.c_int(0)
        check(lib().kvc_get_tuning(self.key, C.byref(old)))
        self.old = old.value
        check(lib().kvc_set_tuning(self.key, self.value))
        return self

    def __exit__(self, *exc):
        from kvcache_amd._native import check, lib
        check(lib().kvc_set_tuning(self.key, self.old))
        return False
