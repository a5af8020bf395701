"""Decode attention on the GPU (through the C ABI) against the CPU oracle.

Bars (stated by the path's spec): max abs error <= 1e-5 for fp32 KV, <= 2e-3 for
fp16 KV (fp32 accumulation, fp16 output); bit-exact for paged vs contiguous and
for every pair of code paths that must agree (identity vs shuffled tables,
uniform vs per-lane table lookups).  The reference's two-pass and flash batched
launchers are one entry point here, so they are held to the oracle, not to each
other.
"""
import numpy as np
import pytest

from kvcache_amd import KVC_F16, KVC_F32, ops
from kvcache_amd._native import KVC_ERR_WORKSPACE, KvcError, check, lib
from kvcache_amd import workloads as W
from kvcache_amd.device import DeviceBuffer

from _helpers import as_np, dev, host, normal, paged_layout, say, tol, tuning

pytestmark = pytest.mark.gpu


def run_batched(q, K, V, lens, Hkv, block, dtype, split=0, perm=None, contiguous=False, workspace=None):
    """q [N,Hq,D], K/V [N,Hkv,S,D] (numpy, already in dtype). Returns device output as float64."""
    N, Hq, D = q.shape
    S = K.shape[2]
    cap = int(max(lens)) if len(lens) else 0
    scale = float(1.0 / np.sqrt(D))
    dq, dl = dev(q), dev(np.asarray(lens, np.int32))
    out = DeviceBuffer(q.nbytes)
    if contiguous:
        dk, dv = dev(K), dev(V)
        ops.launch_batched_decode(dq, dk, dv, dl, out, N, Hq, D, S, cap, scale, Hkv=Hkv, dtype=dtype, split=split,
                                  workspace=workspace)
    else:
        kp, vp, table, tab_off = paged_layout(K, V, lens, block, perm)
        dk, dv, dt, do = dev(kp), dev(vp), dev(table), dev(tab_off)
        ops.launch_batched_paged(dq, dk, dv, dt, do, dl, out, N, Hq, D, block, cap, scale, Hkv=Hkv, dtype=dtype,
                                 split=split, workspace=workspace)
    return host(out, q.dtype, q.shape).astype(np.float64)


def oracle_out(orc, q, K, V, lens):
    return orc.batched_contig(q, K, V, np.asarray(lens, np.int32), float(1.0 / np.sqrt(q.shape[2])))


# ---- config 1: single sequence, fp32, H=8, D=64, S=1024 -------------------------------
@pytest.mark.parametrize("dtype", [KVC_F32, KVC_F16])
def test_c1_single_sequence_contiguous_vs_paged(orc, dtype):
    say(f"c1 single sequence dtype={dtype}")
    H, S, D, B = 8, 1024, 64, 16
    nt = as_np(dtype)
    q, K, V = normal((H, D), 1, nt), normal((H, S, D), 2, nt), normal((H, S, D), 3, nt)
    scale = 1.0 / np.sqrt(D)
    out_c = DeviceBuffer(q.nbytes)
    ops.launch_decode(dev(q), dev(K), dev(V), out_c, S, H, D, S, scale, dtype=dtype)
    oc = host(out_c, nt, q.shape)
    ref = orc.batched_contig(q[None], K[None], V[None], np.array([S], np.int32), scale)[0]
    assert np.abs(oc - ref).max() <= tol(dtype)
    for perm in (None, W.shuffle_perm(S // B, 42)):     # identity and main_paged.cu's shuffled table
        kp, vp, table, _ = paged_layout(K[None], V[None], [S], B, perm)
        out_p = DeviceBuffer(q.nbytes)
        ops.launch_paged(dev(q), dev(kp), dev(vp), dev(table), out_p, S, H, D, B, scale, dtype=dtype)
        np.testing.assert_array_equal(host(out_p, nt, q.shape), oc)  # README.md:68: max abs diff = 0


def test_append_then_decode_reference_flow(orc):
    # main.cu:15-66: 128 launch_append calls fill [H,S,D], then launch_decode
    say("append-then-decode H=8 S=128 D=64 fp32")
    H, S, D = 8, 128, 64
    q, K, V = normal((H, D), 4), normal((H, S, D), 5), normal((H, S, D), 6)
    kc, vc = DeviceBuffer(K.nbytes), DeviceBuffer(V.nbytes)
    kc.zero(); vc.zero()
    for pos in range(S):
        ops.launch_append(dev(np.ascontiguousarray(K[:, pos])), dev(np.ascontiguousarray(V[:, pos])), kc, vc, pos, H,
                          D, S)
    np.testing.assert_array_equal(host(kc, np.float32, K.shape), K)
    out = DeviceBuffer(q.nbytes)
    ops.launch_decode(dev(q), kc, vc, out, S, H, D, S, 1.0 / np.sqrt(D))
    ref = orc.batched_contig(q[None], K[None], V[None], np.array([S], np.int32), 1.0 / np.sqrt(D))[0]
    assert np.abs(host(out, np.float32, q.shape) - ref).max() <= 1e-5


@pytest.mark.parametrize("ns", [1, 4, 7, 16, 128])
def test_flash_decode_splits(orc, ns):
    # main_flash.cu:36: 1 = pure online, 7 does not divide 128, 128 = one token per split
    say(f"flash_decode ns={ns}")
    H, S, D = 8, 128, 64
    q, K, V = normal((H, D), 7), normal((H, S, D), 8), normal((H, S, D), 9)
    out = DeviceBuffer(q.nbytes)
    ops.launch_flash_decode(dev(q), dev(K), dev(V), out, S, H, D, S, 1.0 / np.sqrt(D), ns)
    ref = orc.flash_decode(q, K, V, S, 1.0 / np.sqrt(D), ns)
    assert np.abs(host(out, np.float32, q.shape) - ref).max() <= 1e-5


@pytest.mark.parametrize("L,ns", [(10, 6), (10, 50), (1, 4), (0, 3), (33, 33)])
def test_flash_decode_edge_splits(orc, L, ns):
    # L=10, ns=6: last split empty; ns > L is clamped (flash_decode.cu:106-107); L = 0 gives 0
    say(f"flash_decode edge L={L} ns={ns}")
    H, S, D = 4, 40, 64
    q, K, V = normal((H, D), 10), normal((H, S, D), 11), normal((H, S, D), 12)
    out = DeviceBuffer(q.nbytes)
    ws = DeviceBuffer(max(ops.flash_decode_workspace_size(H, D, max(1, min(ns, max(L, 1)))), 16))
    ws.upload(np.random.default_rng(0).integers(0, 256, ws.nbytes, dtype=np.uint8))  # never cleared: must not matter
    ops.launch_flash_decode(dev(q), dev(K), dev(V), out, L, H, D, S, 0.125, ns, workspace=ws)
    got = host(out, np.float32, q.shape)
    if L == 0:
        assert np.all(got == 0)
    else:
        assert np.abs(got - orc.flash_decode(q, K, V, L, 0.125, ns)).max() <= 1e-5


# ---- config 2: N=128 ragged, MHA H=8, fp16 ---------------------------------------------
@pytest.mark.parametrize("lengths", ["reference", "loguniform"])
def test_c2_ragged_batch(orc, lengths):
    lens = W.ref_lengths() if lengths == "reference" else W.loguniform_lengths(128, 16, 2048, 7)
    say(f"c2 ragged N=128 lengths={lengths} sum={int(lens.sum())}")
    N, H, D, B = 128, 8, 64, 16
    S = int(lens.max())
    q, K, V = normal((N, H, D), 20, np.float16), normal((N, H, S, D), 21, np.float16), normal((N, H, S, D), 22, np.float16)
    nb = sum((int(x) + B - 1) // B for x in lens)
    perm = np.random.default_rng(5).permutation(nb)          # free list handed out in seeded random order
    paged = run_batched(q, K, V, lens, H, B, KVC_F16, perm=perm)
    contig = run_batched(q, K, V, lens, H, B, KVC_F16, contiguous=True)
    np.testing.assert_array_equal(paged, contig)
    err = np.abs(paged - oracle_out(orc, q, K, V, lens)).max()
    assert err <= 2e-3, err


def test_merge_modes_agree(orc):
    say("merge modes 0/1/2")
    lens = np.array([1, 300, 2000, 777, 16, 5000], np.int32)
    N, Hq, Hkv, D, B = len(lens), 8, 2, 64, 16
    S = int(lens.max())
    q, K, V = normal((N, Hq, D), 30, np.float16), normal((N, Hkv, S, D), 31, np.float16), normal((N, Hkv, S, D), 32, np.float16)
    L = lib()
    outs = {}
    try:
        for mode in (0, 1, 2):   # merge kernel, fused behind fences, fused with coherent partials
            check(L.kvc_set_tuning(b"fused_merge", mode))
            outs[mode] = [run_batched(q, K, V, lens, Hkv, B, KVC_F16, split=sp) for sp in (256, 1024)]
    finally:
        check(L.kvc_set_tuning(b"fused_merge", -1))
    # the modes sum the chunk partials in different orders (fp32), so outputs agree
    # to within one fp16 rounding step
    for mode in (1, 2):
        for a, b in zip(outs[0], outs[mode]):
            assert np.abs(a - b).max() <= 1e-3
    assert np.abs(outs[0][0] - oracle_out(orc, q, K, V, lens)).max() <= 2e-3


# ---- GQA, split sizes, block sizes, head dims ----------------------------------------
@pytest.mark.parametrize("dtype", [KVC_F32, KVC_F16])
@pytest.mark.parametrize("split", [0, 16, 64, 512, 8192])
def test_gqa_split_sizes(orc, dtype, split):
    say(f"gqa 14/2 split={split} dtype={dtype}")
    lens = np.array([1, 15, 16, 17, 100, 1000, 3000], np.int32)
    N, Hq, Hkv, D, B = len(lens), 14, 2, 64, 16
    nt = as_np(dtype)
    S = int(lens.max())
    q, K, V = normal((N, Hq, D), 40, nt), normal((N, Hkv, S, D), 41, nt), normal((N, Hkv, S, D), 42, nt)
    got = run_batched(q, K, V, lens, Hkv, B, dtype, split=split, perm=np.random.default_rng(1).permutation(400))
    assert np.abs(got - oracle_out(orc, q, K, V, lens)).max() <= tol(dtype)


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (8, 4), (8, 2), (8, 1), (12, 4), (32, 4), (16, 1)])
def test_head_groupings(orc, Hq, Hkv):
    say(f"head grouping Hq={Hq} Hkv={Hkv}")
    lens = np.array([33, 260, 7], np.int32)
    N, D, B = 3, 64, 16
    q, K, V = normal((N, Hq, D), 50, np.float16), normal((N, Hkv, 260, D), 51, np.float16), normal((N, Hkv, 260, D), 52, np.float16)
    got = run_batched(q, K, V, lens, Hkv, B, KVC_F16, split=64)
    assert np.abs(got - oracle_out(orc, q, K, V, lens)).max() <= 2e-3


@pytest.mark.parametrize("dtype", [KVC_F32, KVC_F16])
@pytest.mark.parametrize("D", [32, 128, 256])
def test_head_dims(orc, dtype, D):
    say(f"head_dim D={D} dtype={dtype}")
    lens = np.array([5, 64, 200], np.int32)
    N, Hq, Hkv, B = 3, 4, 2, 16
    nt = as_np(dtype)
    q, K, V = normal((N, Hq, D), 60, nt), normal((N, Hkv, 200, D), 61, nt), normal((N, Hkv, 200, D), 62, nt)
    for split in (0, 32):
        paged = run_batched(q, K, V, lens, Hkv, B, dtype, split=split)
        contig = run_batched(q, K, V, lens, Hkv, B, dtype, split=split, contiguous=True)
        np.testing.assert_array_equal(paged, contig)
        assert np.abs(paged - oracle_out(orc, q, K, V, lens)).max() <= tol(dtype)


def test_small_blocks_per_lane_path_matches_uniform(orc):
    # BLOCK 4 < 8 tokens per fp16 wave-load -> per-lane table lookups; BLOCK 16 -> uniform
    say("block 4 (per-lane) vs block 16 (uniform)")
    lens = np.array([5, 8, 13, 130, 64], np.int32)
    N, H, D = len(lens), 8, 64
    q, K, V = normal((N, H, D), 70, np.float16), normal((N, H, 130, D), 71, np.float16), normal((N, H, 130, D), 72, np.float16)
    a = run_batched(q, K, V, lens, H, 4, KVC_F16, split=64, perm=np.random.default_rng(2).permutation(200))
    b = run_batched(q, K, V, lens, H, 16, KVC_F16, split=64)
    np.testing.assert_array_equal(a, b)
    assert np.abs(a - oracle_out(orc, q, K, V, lens)).max() <= 2e-3


def test_reference_paged_flash_case(orc):
    # test_paged_flash.cu:13-64: lens {5,8,13}, BLOCK 4, H 8, D 64, fp32
    say("reference test_paged_flash case")
    lens = np.array([5, 8, 13], np.int32)
    q, K, V = normal((3, 8, 64), 80), normal((3, 8, 13, 64), 81), normal((3, 8, 13, 64), 82)
    a = run_batched(q, K, V, lens, 8, 4, KVC_F32)
    assert np.abs(a - oracle_out(orc, q, K, V, lens)).max() <= 1e-5


def test_zero_and_one_token_sequences(orc):
    say("zero / one token sequences")
    lens = np.array([0, 1, 17, 0], np.int32)
    q, K, V = normal((4, 8, 64), 90), normal((4, 2, 17, 64), 91), normal((4, 2, 17, 64), 92)
    for split in (0, 16):
        got = run_batched(q, K, V, lens, 2, 16, KVC_F32, split=split)
        assert np.all(got[0] == 0) and np.all(got[3] == 0)
        np.testing.assert_allclose(got[1], np.repeat(V[1, :, 0].astype(np.float64), 4, axis=0), atol=1e-6)
        assert np.abs(got - oracle_out(orc, q, K, V, lens)).max() <= 1e-5


def test_caller_workspace_reuse_and_errors(orc):
    say("caller workspace")
    lens = np.array([700, 3, 1500], np.int32)
    q, K, V = normal((3, 8, 64), 100, np.float16), normal((3, 8, 1500, 64), 101, np.float16), normal((3, 8, 1500, 64), 102, np.float16)
    need = ops.decode_workspace_size(3, 8, 8, 64, 16, 1500, 128, KVC_F16)
    ws = DeviceBuffer(need)
    ws.upload(np.random.default_rng(3).integers(0, 256, need, dtype=np.uint8))  # garbage: must not matter
    ref = oracle_out(orc, q, K, V, lens)
    first = run_batched(q, K, V, lens, 8, 16, KVC_F16, split=128, workspace=ws)
    second = run_batched(q, K, V, lens, 8, 16, KVC_F16, split=128, workspace=ws)
    np.testing.assert_array_equal(first, second)
    assert np.abs(first - ref).max() <= 2e-3
    with pytest.raises(KvcError) as e:
        run_batched(q, K, V, lens, 8, 16, KVC_F16, split=128, workspace=(ws.ptr, need - 1))
    assert e.value.status == KVC_ERR_WORKSPACE


@pytest.mark.parametrize("D,dtype,Hq,Hkv,split", [(32, KVC_F32, 8, 2, 16), (64, KVC_F32, 8, 8, 16),
                                                   (128, KVC_F32, 4, 2, 16), (256, KVC_F32, 2, 2, 16),
                                                   (64, KVC_F16, 14, 2, 32), (128, KVC_F16, 14, 2, 32)])
def test_merge_kernel_chunk_batches_dirty_workspace(orc, D, dtype, Hq, Hkv, split):
    # The merge kernel reads 8 records per chunk group (512/D groups) ahead of the chunk
    # count, then folds later batches in with a rescale: 0, 1, 3, 19 and 132 chunks per
    # sequence cover the early exit, a partial first batch and (for every D) several
    # later batches; records past each sequence's count hold random bytes.
    say(f"merge kernel batches D={D} dtype={dtype} Hq={Hq} Hkv={Hkv} split={split}")
    lens = np.array([0, 1, 40, 300, 2100], np.int32)
    npdt = np.float32 if dtype == KVC_F32 else np.float16
    q = normal((5, Hq, D), 110 + D, npdt)
    K, V = normal((5, Hkv, 2100, D), 111 + D, npdt), normal((5, Hkv, 2100, D), 112 + D, npdt)
    need = ops.decode_workspace_size(5, Hq, Hkv, D, 16, 2100, split, dtype)
    ws = DeviceBuffer(need)
    ws.upload(np.random.default_rng(D).integers(0, 256, need, dtype=np.uint8))
    with tuning("fused_merge", 0):  # the standalone merge kernel
        got = run_batched(q, K, V, lens, Hkv, 16, dtype, split=split, workspace=ws)
    assert np.all(got[0] == 0)
    assert np.abs(got - oracle_out(orc, q, K, V, lens)).max() <= (1e-5 if dtype == KVC_F32 else 2e-3)


# ---- config 3: long-context split-K, Qwen2.5-0.5B attention shape --------------------
def test_c3_long_context_split_k(orc):
    lens = np.array([8192, 16384, 32768, 32768], np.int32)
    say(f"c3 long context split=512 lens={lens.tolist()}")
    N, Hq, Hkv, D, B = 4, 14, 2, 64, 16
    q = normal((N, Hq, D), 110, np.float16)
    K = normal((N, Hkv, 32768, D), 111, np.float16)
    V = normal((N, Hkv, 32768, D), 112, np.float16)
    nb = int(sum((int(x) + B - 1) // B for x in lens))
    perm = np.random.default_rng(7).permutation(nb)
    split = run_batched(q, K, V, lens, Hkv, B, KVC_F16, split=512, perm=perm)
    unsplit = run_batched(q, K, V, lens, Hkv, B, KVC_F16, split=32768, perm=perm)
    ref = oracle_out(orc, q, K, V, lens)
    assert np.abs(split - ref).max() <= 2e-3
    assert np.abs(unsplit - ref).max() <= 2e-3
    assert np.abs(split - unsplit).max() <= 2e-3


# ---- planned path (host-known lengths; the serving scheduler's path) ----------------
def run_planned(q, K, V, lens, Hkv, block, dtype, perm=None, target=0, workspace=None, inline=True, scale=None):
    N, Hq, D = q.shape
    scale = float(1.0 / np.sqrt(D)) if scale is None else float(scale)
    kp, vp, table, tab_off = paged_layout(K, V, lens, block, perm)
    work, nu, nr = ops.decode_plan(lens, Hq, Hkv, D, block, tab_off=tab_off, table=table if inline else None,
                                   dtype=dtype, target_tokens=target)
    out = DeviceBuffer(q.nbytes)
    ops.launch_batched_paged_planned(dev(q), dev(kp), dev(vp), dev(table), len(table), out, N, Hq, Hkv, D, block,
                                     scale, dev(work), nu, nr, dtype=dtype, workspace=workspace)
    return host(out, q.dtype, q.shape).astype(np.float64)


@pytest.mark.parametrize("Hq,Hkv,D,dtype", [(8, 8, 64, KVC_F16), (14, 2, 64, KVC_F16), (4, 2, 128, KVC_F32)])
def test_planned_many_chunks_fused_merge(orc, Hq, Hkv, D, dtype):
    # contexts of up to 20k tokens split into 20-31 chunks per (sequence, KV head),
    # merged by the last chunk to arrive; two launches on one workspace (arrival
    # counters left by the first, random bytes before) give identical outputs
    say(f"planned many chunks Hq={Hq} Hkv={Hkv} D={D} dtype={dtype}")
    lens = np.array([3000, 9000, 40, 20000], np.int32)
    npdt = np.float32 if dtype == KVC_F32 else np.float16
    q = normal((4, Hq, D), 200, npdt)
    K, V = normal((4, Hkv, 20000, D), 201, npdt), normal((4, Hkv, 20000, D), 202, npdt)
    work, nu, nr = ops.decode_plan(lens, Hq, Hkv, D, 16, dtype=dtype)
    assert nr > 8 * 2 * Hkv, "the plan splits the long contexts into more than 8 chunks"
    ws = DeviceBuffer(ops.planned_workspace_size(Hq, Hkv, D, nr, BLOCK=16, dtype=dtype))
    ws.upload(np.random.default_rng(9).integers(0, 256, ws.nbytes, dtype=np.uint8))
    perm = np.random.default_rng(12).permutation(sum((int(x) + 15) // 16 for x in lens))
    first = run_planned(q, K, V, lens, Hkv, 16, dtype, perm=perm, workspace=ws)
    second = run_planned(q, K, V, lens, Hkv, 16, dtype, perm=perm, workspace=ws)
    np.testing.assert_array_equal(first, second)
    assert np.abs(first - oracle_out(orc, q, K, V, lens)).max() <= (1e-5 if dtype == KVC_F32 else 2e-3)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("scale", [-0.2, 0.0, 0.5])
def test_planned_grouped_scale_sign(orc, D, scale):
    # the matrix-core kernel takes the tile max on raw scores and carries the sign of
    # the scale in q; a zero scale gives the plain mean of V
    say(f"planned grouped D={D} scale={scale}")
    lens = np.array([1, 17, 300, 1000], np.int32)
    N, Hq, Hkv, B = len(lens), 14, 2, 16
    q, K, V = normal((N, Hq, D), 190, np.float16), normal((N, Hkv, 1000, D), 191, np.float16), normal((N, Hkv, 1000, D), 192, np.float16)
    ref = orc.batched_contig(q, K, V, lens, float(scale))
    got = run_planned(q, K, V, lens, Hkv, B, KVC_F16, perm=np.random.default_rng(11).permutation(200), scale=scale)
    assert np.abs(got - ref).max() <= 2e-3


@pytest.mark.parametrize("lengths", ["reference", "loguniform"])
def test_planned_c2_ragged(orc, lengths):
    lens = W.ref_lengths() if lengths == "reference" else W.loguniform_lengths(128, 16, 2048, 7)
    say(f"planned c2 lengths={lengths}")
    N, H, D, B = 128, 8, 64, 16
    S = int(lens.max())
    q, K, V = normal((N, H, D), 120, np.float16), normal((N, H, S, D), 121, np.float16), normal((N, H, S, D), 122, np.float16)
    nb = sum((int(x) + B - 1) // B for x in lens)
    got = run_planned(q, K, V, lens, H, B, KVC_F16, perm=np.random.default_rng(5).permutation(nb))
    assert np.abs(got - oracle_out(orc, q, K, V, lens)).max() <= 2e-3


@pytest.mark.parametrize("dtype", [KVC_F32, KVC_F16])
@pytest.mark.parametrize("target", [0, 64, 256, 4096])
def test_planned_gqa_targets(orc, dtype, target):
    say(f"planned gqa target={target} dtype={dtype}")
    lens = np.array([0, 1, 15, 16, 17, 100, 1000, 3000, 2048], np.int32)
    N, Hq, Hkv, D, B = len(lens), 14, 2, 64, 16
    nt = as_np(dtype)
    S = int(lens.max())
    q, K, V = normal((N, Hq, D), 130, nt), normal((N, Hkv, S, D), 131, nt), normal((N, Hkv, S, D), 132, nt)
    ws = DeviceBuffer(1 << 22)
    ws.upload(np.random.default_rng(4).integers(0, 256, 1 << 22, dtype=np.uint8))  # never cleared
    got = run_planned(q, K, V, lens, Hkv, B, dtype, perm=np.random.default_rng(3).permutation(500), target=target,
                      workspace=ws)
    assert np.all(got[0] == 0)
    assert np.abs(got - oracle_out(orc, q, K, V, lens)).max() <= tol(dtype)


@pytest.mark.parametrize("D", [32, 128])
def test_planned_small_blocks_and_head_dims(orc, D):
    say(f"planned block 4 D={D}")
    lens = np.array([5, 8, 13, 700], np.int32)
    q, K, V = normal((4, 8, D), 140, np.float16), normal((4, 4, 700, D), 141, np.float16), normal((4, 4, 700, D), 142, np.float16)
    got = run_planned(q, K, V, lens, 4, 4, KVC_F16, perm=np.random.default_rng(6).permutation(300), target=128)
    assert np.abs(got - oracle_out(orc, q, K, V, lens)).max() <= 2e-3


def test_planned_c3_long_context(orc):
    lens = np.array([8192, 16384, 32768, 32768], np.int32)
    say("planned c3")
    N, Hq, Hkv, D, B = 4, 14, 2, 64, 16
    q = normal((N, Hq, D), 150, np.float16)
    K, V = normal((N, Hkv, 32768, D), 151, np.float16), normal((N, Hkv, 32768, D), 152, np.float16)
    got = run_planned(q, K, V, lens, Hkv, B, KVC_F16, target=512)
    assert np.abs(got - oracle_out(orc, q, K, V, lens)).max() <= 2e-3


# ---- grouped-query heads on the matrix cores (fp16, head_dim 64/128) ------------------
MFMA_LENS = np.array([0, 1, 15, 16, 17, 31, 33, 500, 1999], np.int32)


@pytest.mark.parametrize("Hq,Hkv", [(14, 2), (8, 2), (16, 1), (12, 4)])
@pytest.mark.parametrize("D", [64, 128])
def test_mfma_gqa_matches_valu_and_oracle(orc, Hq, Hkv, D):
    say(f"mfma gqa Hq={Hq} Hkv={Hkv} D={D}")
    lens = MFMA_LENS
    N, B = len(lens), 16
    S = int(lens.max())
    q, K, V = normal((N, Hq, D), 160, np.float16), normal((N, Hkv, S, D), 161, np.float16), normal((N, Hkv, S, D), 162, np.float16)
    ref = oracle_out(orc, q, K, V, lens)
    perm = np.random.default_rng(8).permutation(600)
    for split in (0, 32, 256):
        with tuning("mfma", 1):
            mf = run_batched(q, K, V, lens, Hkv, B, KVC_F16, split=split, perm=perm)
            mc = run_batched(q, K, V, lens, Hkv, B, KVC_F16, split=split, contiguous=True)
        with tuning("mfma", 0):
            va = run_batched(q, K, V, lens, Hkv, B, KVC_F16, split=split, perm=perm)
        np.testing.assert_array_equal(mf, mc)          # paged == contiguous, bit for bit
        assert np.all(mf[0] == 0)                      # empty sequence
        assert np.abs(mf - ref).max() <= 2e-3, split
        assert np.abs(mf - va).max() <= 2e-3, split
    with tuning("mfma", 1):
        pl = run_planned(q, K, V, lens, Hkv, B, KVC_F16, perm=perm)
        pn = run_planned(q, K, V, lens, Hkv, B, KVC_F16, perm=perm, inline=False)  # block ids from the table only
    assert np.abs(pl - ref).max() <= 2e-3
    np.testing.assert_array_equal(pl, pn)


@pytest.mark.parametrize("block", [8, 32, 48, 64])
def test_mfma_block_sizes(orc, block):
    # BLOCK 8 holds no whole 16-token subtile and BLOCK 48 is no power of two: the
    # grouped path falls back to the VALU kernel for both
    say(f"mfma block={block}")
    lens = np.array([3, 64, 100, 1000], np.int32)
    N, Hq, Hkv, D = len(lens), 14, 2, 64
    q, K, V = normal((N, Hq, D), 170, np.float16), normal((N, Hkv, 1000, D), 171, np.float16), normal((N, Hkv, 1000, D), 172, np.float16)
    ref = oracle_out(orc, q, K, V, lens)
    perm = np.random.default_rng(9).permutation(200)
    for split in (0, 128):
        got = run_batched(q, K, V, lens, Hkv, block, KVC_F16, split=split if split % block == 0 else 0, perm=perm)
        assert np.abs(got - ref).max() <= 2e-3
    got = run_planned(q, K, V, lens, Hkv, block, KVC_F16, perm=perm)
    assert np.abs(got - ref).max() <= 2e-3


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_mfma_merge_modes(orc, mode):
    say(f"mfma merge mode={mode}")
    lens = np.array([4000, 2047, 9, 3000], np.int32)
    N, Hq, Hkv, D, B = len(lens), 14, 2, 64, 16
    q, K, V = normal((N, Hq, D), 180, np.float16), normal((N, Hkv, 4000, D), 181, np.float16), normal((N, Hkv, 4000, D), 182, np.float16)
    ref = oracle_out(orc, q, K, V, lens)
    with tuning("fused_merge", mode):
        for split in (512, 1024):  # 8 and 4 chunks of the longest sequence
            got = run_batched(q, K, V, lens, Hkv, B, KVC_F16, split=split)
            assert np.abs(got - ref).max() <= 2e-3


# ---- prompt (prefill) attention: qk_paged_causal_attn (qwen_kernels.h:19-21) ---------
@pytest.mark.parametrize("dtype,Hq,Hkv", [(KVC_F16, 14, 2), (KVC_F16, 8, 8), (KVC_F32, 8, 2)])
@pytest.mark.parametrize("base,n", [(0, 1), (0, 37), (100, 64), (0, 600), (5000, 3)])
def test_paged_causal_attn(orc, dtype, Hq, Hkv, base, n):
    say(f"causal prefill dtype={dtype} Hq={Hq} Hkv={Hkv} base={base} n={n}")
    D, B = 64, 16
    nt = as_np(dtype)
    S = base + n
    nb = (S + B - 1) // B
    table = np.random.default_rng(base + n).permutation(nb + 9)[:nb].astype(np.int32)
    NB = int(table.max()) + 1
    kp, vp = normal((NB, Hkv, B, D), 190, nt), normal((NB, Hkv, B, D), 191, nt)
    q = normal((n, Hq, D), 192, nt)
    scale = float(1.0 / np.sqrt(D))
    out = DeviceBuffer(q.nbytes)
    ops.qk_paged_causal_attn(dev(q), out, dev(kp), dev(vp), dev(table), base, n, Hq, Hkv, D, B, scale, dtype=dtype)
    got = host(out, nt, q.shape).astype(np.float64)
    want = orc.paged_causal(q, kp, vp, table, base, Hkv, B, scale)
    assert np.abs(got - want).max() <= tol(dtype)
    if dtype == KVC_F16:  # the query-tiled matrix-core path against the per-query decode path
        with tuning("mfma", 0):
            alt = DeviceBuffer(q.nbytes)
            ops.qk_paged_causal_attn(dev(q), alt, dev(kp), dev(vp), dev(table), base, n, Hq, Hkv, D, B, scale)
        assert np.abs(got - host(alt, nt, q.shape).astype(np.float64)).max() <= 2e-3


def test_prefill_flow_write_then_causal_attn(orc):
    """The model path's prefill (qwen_serve.cu:106-108): write the P prompt rows of
    K/V through the sequence's table, then causal attention over them."""
    say("prefill flow")
    P, Hq, Hkv, D, B = 200, 14, 2, 64, 16
    nb = (P + B - 1) // B
    table = np.random.default_rng(11).permutation(40)[:nb].astype(np.int32)
    kp0 = np.zeros((40, Hkv, B, D), np.float16)
    K, V, q = normal((P, Hkv, D), 193, np.float16), normal((P, Hkv, D), 194, np.float16), normal((P, Hq, D), 195, np.float16)
    dk, dv, dt = dev(kp0), dev(kp0), dev(table)
    ops.qk_write_kv(dev(K), dev(V), dk, dv, dt, 0, P, Hkv, D, B)
    out = DeviceBuffer(q.nbytes)
    scale = float(1.0 / np.sqrt(D))
    ops.qk_paged_causal_attn(dev(q), out, dk, dv, dt, 0, P, Hq, Hkv, D, B, scale)
    got = host(out, np.float16, q.shape).astype(np.float64)
    # expected: causal attention over the contiguous rows
    Kc, Vc = K.transpose(1, 0, 2)[None], V.transpose(1, 0, 2)[None]          # [1, Hkv, P, D]
    want = np.stack([orc.batched_contig(q[i:i + 1], Kc, Vc, np.array([i + 1], np.int32), scale)[0] for i in range(P)])
    assert np.abs(got - want).max() <= 2e-3
