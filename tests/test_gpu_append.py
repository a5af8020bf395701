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


# ---- fused append + decode (planned launch) ------------------------------------------
@pytest.mark.parametrize("dtype,Hq,Hkv,block", [(KVC_F16, 14, 2, 16), (KVC_F16, 8, 8, 16), (KVC_F32, 14, 2, 16),
                                                (KVC_F16, 8, 4, 4), (KVC_F16, 16, 2, 32)])
def test_fused_append_decode_equals_write_then_decode(orc, dtype, Hq, Hkv, block):
    """The step's write (qk_batched_write_kv) followed by the decode equals the fused
    launch bit for bit: the same outputs and the same pools afterwards; rows with
    wpos = -1 or outside the attended length are not written.  Write positions at the
    end of the context, inside it and at a tile's first row."""
    say(f"fused append+decode dtype={dtype} Hq={Hq} Hkv={Hkv} block={block}")
    D = 64
    nt = as_np(dtype)
    lens = np.array([1, 17, 300, 1200, 33, 0, 640, 2000], np.int32)
    wpos = lens - 1
    wpos[4] = -1                      # an idle slot: nothing written
    wpos[3] = 517                     # inside the context: row 5 of a full 32-token tile
    wpos[6] = 64                      # first row of a tile
    N = len(lens)
    nb = [(int(L) + block - 1) // block for L in lens]
    tab_off = np.concatenate([[0], np.cumsum(nb)]).astype(np.int32)
    table = np.random.default_rng(21).permutation(int(tab_off[-1]) + 7)[: tab_off[-1]].astype(np.int32)
    NB = int(table.max()) + 1
    kp0, vp0 = normal((NB, Hkv, block, D), 22, nt), normal((NB, Hkv, block, D), 23, nt)
    q, kn, vn = normal((N, Hq, D), 24, nt), normal((N, Hkv, D), 25, nt), normal((N, Hkv, D), 26, nt)
    work, nu, nr = ops.decode_plan(lens, Hq, Hkv, D, block, tab_off=tab_off, table=table, dtype=dtype)
    scale = float(1.0 / np.sqrt(D))
    dq, dkn, dvn, dtab, dwp, dw = dev(q), dev(kn), dev(vn), dev(table), dev(wpos), dev(work)

    # reference order: write the rows, then the planned decode
    kr, vr, outr = dev(kp0), dev(vp0), DeviceBuffer(q.nbytes)
    ops.qk_batched_write_kv(dkn, dvn, kr, vr, dtab, dev(tab_off), dwp, N, Hkv, D, block, dtype=dtype)
    ops.launch_batched_paged_planned(dq, kr, vr, dtab, len(table), outr, N, Hq, Hkv, D, block, scale, dw, nu, nr,
                                     dtype=dtype)
    # fused
    kf, vf, outf = dev(kp0), dev(vp0), DeviceBuffer(q.nbytes)
    ops.launch_batched_paged_append_planned(dq, dkn, dvn, dwp, kf, vf, dtab, len(table), outf, N, Hq, Hkv, D, block,
                                            scale, dw, nu, nr, dtype=dtype)
    got, ref = host(outf, nt, q.shape), host(outr, nt, q.shape)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(host(kf, nt, kp0.shape), host(kr, nt, kp0.shape))
    np.testing.assert_array_equal(host(vf, nt, kp0.shape), host(vr, nt, kp0.shape))
    # and against the CPU restatement on the written pools
    kw, vw = host(kr, nt, kp0.shape), host(vr, nt, kp0.shape)
    want = orc.batched_paged(q, kw, vw, table, tab_off, lens, Hkv, block, scale)
    bar = 2e-3 if dtype == KVC_F16 else 1e-5
    assert np.abs(got.astype(np.float64) - want).max() <= bar
