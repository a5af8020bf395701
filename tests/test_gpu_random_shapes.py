"""Seeded random shapes through the decode, prompt-attention and K/V-write entry
points, against the CPU oracle (attention) and numpy scatters (writes).

Decode: each case draws a batch of 1-24 sequences (lengths log-uniform up to 1500, with 0,
1 and the block edges B-1, B, B+1, 2B mixed in), a head layout (Hkv in 1..8, query
group 1..8), a head dimension (32, 64, 128), a block size (8, 16, 32, 48), a dtype
and a split, then runs the device-lengths paged launch, the contiguous launch and
the host-planned paged launch (reference entry points: launch_batched_paged,
batched.cu:140-147, and launch_batched_paged_flash, batched.cu:199-208;
launch_batched_decode, batched.cu:132-138).

Bars: every path within the oracle tolerance (1e-5 fp32, 2e-3 fp16, max abs);
paged == contiguous bit for bit when the block size is 16 or 32 (both launches
then take the same kernel and the same chunks; at 8 or 48 the paged launch takes
the VALU kernel, since the matrix-core kernel needs a power-of-two block of at
least 16 tokens, or other chunks, and agrees with the contiguous one within
tolerance only); a paged split that is not a multiple of the block size is refused
with KVC_ERR_ARG.
"""
import numpy as np
import pytest

from kvcache_amd import KVC_F16, KVC_F32, ops
from kvcache_amd._native import KVC_ERR_ARG, KVC_ERR_UNSUPPORTED, KvcError
from kvcache_amd.device import DeviceBuffer

from _helpers import dev, host, normal, say, tol
from test_gpu_decode import oracle_out, run_batched, run_planned

pytestmark = pytest.mark.gpu


def draw(seed):
    r = np.random.default_rng(1000 + seed)
    N = int(r.integers(1, 25))
    Hkv = int(r.choice([1, 2, 4, 8]))
    group = int(r.choice([1, 2, 3, 4, 7, 8]))
    D = int(r.choice([32, 64, 128]))
    B = int(r.choice([8, 16, 32, 48]))
    dtype = KVC_F16 if r.random() < 0.6 else KVC_F32
    edges = [0, 1, B - 1, B, B + 1, 2 * B]
    lens = np.where(r.random(N) < 0.25, r.choice(edges, N), np.exp(r.uniform(0, np.log(1500), N)).astype(int))
    split = int(r.choice([0, 0, B, 3 * B, 200, 512]))
    return N, Hkv * group, Hkv, D, B, dtype, lens.astype(np.int32), split


@pytest.mark.parametrize("seed", range(48))
def test_random_shape_parity(orc, seed):
    N, Hq, Hkv, D, B, dtype, lens, split = draw(seed)
    nt = np.float16 if dtype == KVC_F16 else np.float32
    say(f"random shape seed {seed}: N={N} Hq={Hq} Hkv={Hkv} D={D} B={B} "
        f"{'f16' if dtype == KVC_F16 else 'f32'} split={split} max_len={int(lens.max())}")
    S = max(int(lens.max()), 1)
    q = normal((N, Hq, D), 3 * seed, nt)
    K, V = normal((N, Hkv, S, D), 3 * seed + 1, nt), normal((N, Hkv, S, D), 3 * seed + 2, nt)
    ref = oracle_out(orc, q, K, V, lens)
    nb = sum((int(x) + B - 1) // B for x in lens)
    perm = np.random.default_rng(seed).permutation(nb)

    contig = run_batched(q, K, V, lens, Hkv, B, dtype, split=split, contiguous=True)
    assert np.abs(contig - ref).max() <= tol(dtype)
    planned = run_planned(q, K, V, lens, Hkv, B, dtype, perm=perm)
    assert np.abs(planned - ref).max() <= tol(dtype)
    if split % B:
        with pytest.raises(KvcError) as ei:
            run_batched(q, K, V, lens, Hkv, B, dtype, split=split, perm=perm)
        assert ei.value.status == KVC_ERR_ARG
        return
    paged = run_batched(q, K, V, lens, Hkv, B, dtype, split=split, perm=perm)
    assert np.abs(paged - ref).max() <= tol(dtype)
    if B in (16, 32):
        np.testing.assert_array_equal(paged, contig)


def draw_causal(seed):
    r = np.random.default_rng(2000 + seed)
    Hkv = int(r.choice([1, 2, 4]))
    group = int(r.choice([1, 2, 4, 7]))
    D = int(r.choice([32, 64, 128]))
    B = int(r.choice([8, 16, 32, 64]))
    dtype = KVC_F16 if r.random() < 0.6 else KVC_F32
    base = 0 if r.random() < 0.4 else int(r.integers(1, 2000))
    n = int(np.exp(r.uniform(0, np.log(500))))
    return Hkv * group, Hkv, D, B, dtype, base, n


@pytest.mark.parametrize("seed", range(24))
def test_random_causal_parity(orc, seed):
    """Prompt attention (qk_paged_causal_attn, qwen_kernels.h:19-21; the device-base
    form qkcuda_paged_causal_attn, qwen_kernels.h:45-47) over seeded random shapes:
    both forms within the oracle tolerance.  They need not agree bit for bit: the
    host form chunks the prefix from the host position, the device form plans its
    own chunks in the kernel."""
    Hq, Hkv, D, B, dtype, base, n = draw_causal(seed)
    nt = np.float16 if dtype == KVC_F16 else np.float32
    say(f"random causal seed {seed}: Hq={Hq} Hkv={Hkv} D={D} B={B} {'f16' if dtype == KVC_F16 else 'f32'} "
        f"base={base} n={n}")
    nb = (base + n + B - 1) // B
    table = np.random.default_rng(seed).permutation(nb + 5)[:nb].astype(np.int32)
    NB = int(table.max()) + 1
    kp, vp = normal((NB, Hkv, B, D), 5 * seed, nt), normal((NB, Hkv, B, D), 5 * seed + 1, nt)
    q = normal((n, Hq, D), 5 * seed + 2, nt)
    scale = float(1.0 / np.sqrt(D))
    dq, dk, dv, dt = dev(q), dev(kp), dev(vp), dev(table)
    out, out_dev = DeviceBuffer(q.nbytes), DeviceBuffer(q.nbytes)
    ops.qk_paged_causal_attn(dq, out, dk, dv, dt, base, n, Hq, Hkv, D, B, scale, dtype=dtype)
    got = host(out, nt, q.shape).astype(np.float64)
    want = orc.paged_causal(q, kp, vp, table, base, Hkv, B, scale, nthreads=8)
    assert np.abs(got - want).max() <= tol(dtype)
    pos = dev(np.array([base], np.int32))
    # the device-position form pages uniformly only: a power-of-two block of at least
    # 1 KiB per KV head; other shapes are refused, never run partially
    if B & (B - 1) or B * D * nt().itemsize < 1024:
        with pytest.raises(KvcError) as ei:
            ops.qkcuda_paged_causal_attn(dq, out_dev, dk, dv, dt, pos, n, Hq, Hkv, D, B, scale, dtype=dtype)
        assert ei.value.status == KVC_ERR_UNSUPPORTED
        return
    ops.qkcuda_paged_causal_attn(dq, out_dev, dk, dv, dt, pos, n, Hq, Hkv, D, B, scale, dtype=dtype)
    assert np.abs(host(out_dev, nt, q.shape).astype(np.float64) - want).max() <= tol(dtype)


@pytest.mark.parametrize("seed", range(24))
def test_random_kv_writes(seed):
    """K/V writes over seeded random shapes, bit-exact against numpy scatters of the
    reference's addressing: a prompt's rows through its table (qk_write_kv,
    qwen_kernels.cu:111-122), one row per sequence at its write position
    (qk_batched_write_kv, qwen_kernels.cu:270-285; position -1 writes nothing) and
    the same rows through a slot map; every other byte of the pools unchanged."""
    r = np.random.default_rng(3000 + seed)
    Hkv, D = int(r.choice([1, 2, 4, 8])), int(r.choice([32, 64, 128]))
    B = int(r.choice([1, 8, 16, 32, 48]))
    dtype = KVC_F16 if r.random() < 0.6 else KVC_F32
    nt = np.float16 if dtype == KVC_F16 else np.float32
    NB = int(r.integers(4, 80))
    say(f"random writes seed {seed}: Hkv={Hkv} D={D} B={B} {'f16' if dtype == KVC_F16 else 'f32'} NB={NB}")
    pool0 = normal((NB, Hkv, B, D), 7 * seed, nt)

    # a prompt: L rows from start through a table of distinct blocks
    cap = NB * B
    start = int(r.integers(0, cap // 2 + 1))
    L = int(r.integers(0, cap - start + 1))
    table = r.permutation(NB).astype(np.int32)
    k, v = normal((max(L, 1), Hkv, D), 7 * seed + 1, nt)[:L], normal((max(L, 1), Hkv, D), 7 * seed + 2, nt)[:L]
    kp, vp = dev(pool0), dev(pool0)
    ops.qk_write_kv(dev(k) if L else dev(np.zeros(1, nt)), dev(v) if L else dev(np.zeros(1, nt)), kp, vp,
                    dev(table), start, L, Hkv, D, B, dtype=dtype)
    ek, ev = pool0.copy(), pool0.copy()
    for i in range(L):
        pos = start + i
        ek[table[pos // B], :, pos % B], ev[table[pos // B], :, pos % B] = k[i], v[i]
    np.testing.assert_array_equal(host(kp, nt, pool0.shape), ek)
    np.testing.assert_array_equal(host(vp, nt, pool0.shape), ev)

    # one row per sequence: disjoint tables, a write position per row (or -1)
    N = int(r.integers(1, min(NB, 32) + 1))
    cuts = np.sort(r.choice(np.arange(1, NB), size=N - 1, replace=False)) if N > 1 else np.array([], int)
    blocks = r.permutation(NB).astype(np.int32)
    tables = np.split(blocks, cuts)
    tab_off = np.concatenate([[0], np.cumsum([len(t) for t in tables])]).astype(np.int32)
    wpos = np.array([int(r.integers(0, len(t) * B)) if r.random() < 0.85 else -1 for t in tables], np.int32)
    k1, v1 = normal((N, Hkv, D), 7 * seed + 3, nt), normal((N, Hkv, D), 7 * seed + 4, nt)
    kp, vp = dev(pool0), dev(pool0)
    ops.qk_batched_write_kv(dev(k1), dev(v1), kp, vp, dev(blocks), dev(tab_off), dev(wpos), N, Hkv, D, B, dtype=dtype)
    ek, ev = pool0.copy(), pool0.copy()
    slots = np.full(N, -1, np.int32)
    for i, t in enumerate(tables):
        if wpos[i] >= 0:
            phys, inb = t[wpos[i] // B], wpos[i] % B
            ek[phys, :, inb], ev[phys, :, inb] = k1[i], v1[i]
            slots[i] = phys * B + inb
    np.testing.assert_array_equal(host(kp, nt, pool0.shape), ek)
    np.testing.assert_array_equal(host(vp, nt, pool0.shape), ev)
    kp, vp = dev(pool0), dev(pool0)
    ops.write_kv_slots(dev(k1), dev(v1), kp, vp, dev(slots), N, Hkv, D, B, dtype=dtype)
    np.testing.assert_array_equal(host(kp, nt, pool0.shape), ek)
    np.testing.assert_array_equal(host(vp, nt, pool0.shape), ev)
