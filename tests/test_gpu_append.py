"""K/V writes on the GPU: pure data movement, checked bit-exact against numpy
scatters of the reference's addressing (kv_cache.cu:5-13, qwen_kernels.cu:111-122,
270-285), including untouched bytes elsewhere in the pool."""
import numpy as np
import pytest

from kvcache_amd import KVC_F16, KVC_F32, ops
from kvcache_amd.device import DeviceBuffer

from _helpers import as_np, dev, host, normal, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [KVC_F32, KVC_F16])
@pytest.mark.parametrize("D", [64, 4])
def test_append_contiguous(dtype, D):
    say(f"append dtype={dtype} D={D}")
    H, S = 8, 10
    nt = as_np(dtype)
    kc0 = normal((H, S, D), 1, nt)
    kn, vn = normal((H, D), 2, nt), normal((H, D), 3, nt)
    kc, vc = dev(kc0), dev(kc0)
    ops.launch_append(dev(kn), dev(vn), kc, vc, 7, H, D, S, dtype=dtype)
    ek, ev = kc0.copy(), kc0.copy()
    ek[:, 7], ev[:, 7] = kn, vn
    np.testing.assert_array_equal(host(kc, nt, kc0.shape), ek)
    np.testing.assert_array_equal(host(vc, nt, kc0.shape), ev)


@pytest.mark.parametrize("dtype", [KVC_F16, KVC_F32])
def test_write_kv_paged_prefill_rows(dtype):
    say(f"write_kv paged dtype={dtype}")
    NB, Hkv, B, D, L, start = 12, 2, 16, 64, 37, 5
    nt = as_np(dtype)
    table = np.array([9, 3, 0, 11], np.int32)
    pool0 = normal((NB, Hkv, B, D), 4, nt)
    k, v = normal((L, Hkv, D), 5, nt), normal((L, Hkv, D), 6, nt)
    kp, vp = dev(pool0), dev(pool0)
    ops.qk_write_kv(dev(k), dev(v), kp, vp, dev(table), start, L, Hkv, D, B, dtype=dtype)
    ek, ev = pool0.copy(), pool0.copy()
    for r in range(L):
        pos = start + r
        ek[table[pos // B], :, pos % B] = k[r]
        ev[table[pos // B], :, pos % B] = v[r]
    np.testing.assert_array_equal(host(kp, nt, pool0.shape), ek)
    np.testing.assert_array_equal(host(vp, nt, pool0.shape), ev)


def test_batched_write_kv_and_slots():
    say("batched write_kv + slot map fp16")
    NB, Hkv, B, D = 20, 2, 16, 64
    pool0 = normal((NB, Hkv, B, D), 7, np.float16)
    tables = [[4, 7], [1], [19, 2, 3], [8]]
    wpos = np.array([17, 3, 40, -1], np.int32)   # -1: idle slot, nothing written
    tab_off = np.concatenate([[0], np.cumsum([len(t) for t in tables])]).astype(np.int32)
    table_all = np.concatenate(tables).astype(np.int32)
    k, v = normal((4, Hkv, D), 8, np.float16), normal((4, Hkv, D), 9, np.float16)
    kp, vp = dev(pool0), dev(pool0)
    ops.qk_batched_write_kv(dev(k), dev(v), kp, vp, dev(table_all), dev(tab_off), dev(wpos), 4, Hkv, D, B)
    ek, ev = pool0.copy(), pool0.copy()
    slots = []
    for r, t in enumerate(tables):
        if wpos[r] < 0:
            slots.append(-1)
            continue
        phys, inb = t[wpos[r] // B], wpos[r] % B
        ek[phys, :, inb], ev[phys, :, inb] = k[r], v[r]
        slots.append(phys * B + inb)
    np.testing.assert_array_equal(host(kp, np.float16, pool0.shape), ek)
    np.testing.assert_array_equal(host(vp, np.float16, pool0.shape), ev)
    kp2, vp2 = dev(pool0), dev(pool0)
    ops.write_kv_slots(dev(k), dev(v), kp2, vp2, dev(np.array(slots, np.int32)), 4, Hkv, D, B)
    np.testing.assert_array_equal(host(kp2, np.float16, pool0.shape), ek)
    np.testing.assert_array_equal(host(vp2, np.float16, pool0.shape), ev)


def test_fill_normal_is_deterministic_and_normal():
    say("fill_normal")
    from kvcache_amd.device import fill_normal
    n = 1 << 20
    a, b = DeviceBuffer(n * 2), DeviceBuffer(n * 2)
    fill_normal(a, n, KVC_F16, 123)
    fill_normal(b, n, KVC_F16, 123)
    x = host(a, np.float16, (n,)).astype(np.float64)
    np.testing.assert_array_equal(x, host(b, np.float16, (n,)).astype(np.float64))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01 and np.all(np.isfinite(x))
