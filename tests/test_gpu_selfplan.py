"""Device-length decode planned by the kernel itself (the reference's launch_batched_paged /
qk_batched_paged_decode_attn take the lengths in device memory: batched.cu:140-147,
qwen_kernels.cu:293-326).

Every workgroup derives the host planner's units from the device lengths, so the
outputs must equal the host-planned launch's bit for bit (same chunks, same merge
order), whatever order the units run in and however many workgroups serve them; and
they must match the CPU oracle within the path's tolerance.  On the VALU kernel,
sequences of at most self_lead_tokens tokens are attended whole by the waves that
wait while wave 0 plans, and the plan leaves them out: the other sequences still
equal the host plan bit for bit, the short ones match the oracle, and paged equals
contiguous bit for bit.  No length is truncated:
a stated cap only sizes the launch, and the explicit-split path (whose grid is sized
by the cap) gives NaN rows, never a partial attention, for a sequence longer than it.
"""
import numpy as np
import pytest

from kvcache_amd import KVC_F16, KVC_F32, ops
from kvcache_amd import workloads as W
from kvcache_amd._native import KVC_ERR_ARG, KvcError
from kvcache_amd.device import DeviceBuffer

from _helpers import as_np, dev, host, normal, paged_layout, say, tol, tuning

pytestmark = pytest.mark.gpu


def inputs(lens, Hq, Hkv, D, dtype, seed):
    nt = as_np(dtype)
    S = max(int(max(lens)), 1)
    N = len(lens)
    return (normal((N, Hq, D), seed, nt), normal((N, Hkv, S, D), seed + 1, nt), normal((N, Hkv, S, D), seed + 2, nt))


def self_planned(q, kp, vp, table, tab_off, lens, Hkv, B, dtype, cap=0, workspace=None):
    N, Hq, D = q.shape
    out = DeviceBuffer(q.nbytes)
    ops.launch_batched_paged(dev(q), dev(kp), dev(vp), dev(table), dev(tab_off), dev(np.asarray(lens, np.int32)), out,
                             N, Hq, D, B, cap, float(1.0 / np.sqrt(D)), Hkv=Hkv, dtype=dtype, workspace=workspace)
    return host(out, q.dtype, q.shape).astype(np.float64)


def host_planned(q, kp, vp, table, tab_off, lens, Hkv, B, dtype):
    N, Hq, D = q.shape
    work, nu, nr = ops.decode_plan(lens, Hq, Hkv, D, B, tab_off=tab_off, table=table, dtype=dtype)
    out = DeviceBuffer(q.nbytes)
    ops.launch_batched_paged_planned(dev(q), dev(kp), dev(vp), dev(table), len(table), out, N, Hq, Hkv, D, B,
                                     float(1.0 / np.sqrt(D)), dev(work), nu, nr, dtype=dtype)
    return host(out, q.dtype, q.shape).astype(np.float64)


def oracle(orc, q, K, V, lens):
    return orc.batched_contig(q, K, V, np.asarray(lens, np.int32), float(1.0 / np.sqrt(q.shape[2])))


CASES = {
    # name: (lengths, Hq, Hkv, D, dtype)
    "c2_reference": (W.ref_lengths(), 8, 8, 64, KVC_F16),
    "c2_loguniform": (W.loguniform_lengths(128, 16, 2048, 7), 8, 8, 64, KVC_F16),
    "gqa_mfma_long": (np.array([8192, 16384, 300, 1, 0, 2500, 700, 1025], np.int32), 14, 2, 64, KVC_F16),
    "gqa_mfma_d128": (np.array([5, 1500, 4097, 33, 900], np.int32), 16, 2, 128, KVC_F16),
    "mha_fp32": (np.array([1, 17, 640, 961, 2000, 3000, 0, 64], np.int32), 8, 8, 64, KVC_F32),
    "gqa_valu_fp32": (np.array([1000, 15, 16, 17, 3000, 1], np.int32), 14, 2, 64, KVC_F32),
    "group2_fp16": (np.array([2048, 1024, 333, 5000, 7], np.int32), 8, 4, 64, KVC_F16),
    # every length within the largest short-sequence threshold: the plan has no units at all
    "short_mha": (np.array([1, 0, 700, 1024, 33, 64, 65, 1000], np.int32), 8, 8, 64, KVC_F16),
}


@pytest.mark.parametrize("case", list(CASES))
def test_self_planned_equals_host_planned(orc, case):
    lens, Hq, Hkv, D, dtype = CASES[case]
    say(f"self-planned vs host-planned: {case}")
    B = 16
    q, K, V = inputs(lens, Hq, Hkv, D, dtype, 300)
    nb = sum((int(x) + B - 1) // B for x in lens)
    kp, vp, table, tab_off = paged_layout(K, V, lens, B, np.random.default_rng(8).permutation(nb))
    with tuning("self_lead_tokens", 0):
        got = self_planned(q, kp, vp, table, tab_off, lens, Hkv, B, dtype, cap=int(max(lens)))
    ref = host_planned(q, kp, vp, table, tab_off, lens, Hkv, B, dtype)
    np.testing.assert_array_equal(got, ref)
    want = oracle(orc, q, K, V, lens)
    assert np.abs(got - want).max() <= tol(dtype)
    assert np.all(got[np.asarray(lens) == 0] == 0)
    lead = self_planned(q, kp, vp, table, tab_off, lens, Hkv, B, dtype, cap=int(max(lens)))  # short ones while planning
    assert np.abs(lead - want).max() <= tol(dtype)
    assert np.all(lead[np.asarray(lens) == 0] == 0)
    planned = np.asarray(lens) > 320  # (the default threshold; matrix-core shapes plan every sequence)
    np.testing.assert_array_equal(lead[planned], ref[planned])


@pytest.mark.parametrize("grid", [1, 7, 100])
def test_small_grids_serve_every_rank_once(orc, grid):
    """With fewer workgroups than units, each workgroup serves several ranks (rounds in
    alternating direction): the same outputs, bit for bit, on a first and a second
    launch over a never-cleared workspace (epoch-tagged arrival counters)."""
    say(f"self-planned, grid {grid}")
    lens, Hq, Hkv, D, dtype = np.array([1, 700, 2048, 90, 5000, 16, 1300], np.int32), 14, 2, 64, KVC_F16
    q, K, V = inputs(lens, Hq, Hkv, D, dtype, 310)
    kp, vp, table, tab_off = paged_layout(K, V, lens, 16)
    ws = DeviceBuffer(ops.decode_workspace_size(len(lens), Hq, Hkv, D, 16, 0, 0, dtype))
    ws.upload(np.random.default_rng(1).integers(0, 256, ws.nbytes, dtype=np.uint8))
    with tuning("self_lead_tokens", 0):  # (small grids run without lead chunks)
        ref = self_planned(q, kp, vp, table, tab_off, lens, Hkv, 16, dtype)
    with tuning("self_grid", grid):
        a = self_planned(q, kp, vp, table, tab_off, lens, Hkv, 16, dtype, workspace=ws)
        b = self_planned(q, kp, vp, table, tab_off, lens, Hkv, 16, dtype, workspace=ws)
    np.testing.assert_array_equal(a, ref)
    np.testing.assert_array_equal(b, ref)
    assert np.abs(ref - oracle(orc, q, K, V, lens)).max() <= 2e-3


def test_paged_and_contiguous_agree_bit_for_bit_gqa():
    """The reference's paged-vs-contiguous check (bench_throughput.cu:124-128) on the
    default launchers: both plan the same chunks from the device lengths."""
    say("self-planned paged vs contiguous, GQA fp16")
    lens = np.array([1, 16, 17, 1000, 4000, 2500, 64, 1023], np.int32)
    N, Hq, Hkv, D = len(lens), 14, 2, 64
    q, K, V = inputs(lens, Hq, Hkv, D, KVC_F16, 320)
    nb = sum((int(x) + 15) // 16 for x in lens)
    kp, vp, table, tab_off = paged_layout(K, V, lens, 16, np.random.default_rng(2).permutation(nb + 40))
    paged = self_planned(q, kp, vp, table, tab_off, lens, Hkv, 16, KVC_F16)
    out = DeviceBuffer(q.nbytes)
    S = K.shape[2]
    ops.launch_batched_decode(dev(q), dev(K), dev(V), dev(lens), out, N, Hq, D, S, int(lens.max()),
                              float(1.0 / np.sqrt(D)), Hkv=Hkv, dtype=KVC_F16)
    np.testing.assert_array_equal(paged, host(out, np.float16, q.shape).astype(np.float64))


def test_lengths_past_the_stated_cap_are_attended_whole(orc):
    """qk_batched_paged_decode_attn has no cap (qwen_kernels.h:35-37) and a cap is only a
    hint to launch_batched_paged: a 40k-token context (past the 32768 a fixed bound
    would have cut it at) and lengths above a cap of 100 are attended over their whole
    length."""
    say("no truncation past cap")
    lens = np.array([40000, 3, 1200], np.int32)
    Hq, Hkv, D = 14, 2, 64
    q, K, V = inputs(lens, Hq, Hkv, D, KVC_F16, 330)
    kp, vp, table, tab_off = paged_layout(K, V, lens, 16)
    out = DeviceBuffer(q.nbytes)
    ops.qk_batched_paged_decode_attn(dev(q), out, dev(kp), dev(vp), dev(table), dev(tab_off), dev(lens), len(lens),
                                     Hq, Hkv, D, 16, float(1.0 / np.sqrt(D)))
    got = host(out, np.float16, q.shape).astype(np.float64)
    ref = oracle(orc, q, K, V, lens)
    assert np.abs(got - ref).max() <= 2e-3
    hinted = self_planned(q, kp, vp, table, tab_off, lens, Hkv, 16, KVC_F16, cap=100)
    np.testing.assert_array_equal(hinted, got)
    # a prefix-only attention would differ from the whole-length one
    cut = oracle(orc, q, K[:, :, :32768], V[:, :, :32768], np.minimum(lens, 32768))
    assert np.abs(cut[0] - ref[0]).max() > 1e-2


def test_long_mean_context_within_the_stated_cap(orc):
    """One- and two-head units take chunks of at most 64 blocks and 64 partial records
    per (sequence, head) by default, so a batch whose mean context passes 63 x 1024
    tokens (BLOCK 16) cannot be planned without a bound: it gets NaN rows.  With the
    reference's own cap argument stated the record budget grows with it and the batch
    is attended whole."""
    say("mean context above the default record budget, MHA fp16")
    lens = np.array([70000, 75000], np.int32)
    Hq = Hkv = 2
    D = 64
    q, K, V = inputs(lens, Hq, Hkv, D, KVC_F16, 345)
    kp, vp, table, tab_off = paged_layout(K, V, lens, 16)
    got = self_planned(q, kp, vp, table, tab_off, lens, Hkv, 16, KVC_F16, cap=int(lens.max()))
    assert np.abs(got - oracle(orc, q, K, V, lens)).max() <= 2e-3
    unbounded = self_planned(q, kp, vp, table, tab_off, lens, Hkv, 16, KVC_F16, cap=0)
    assert np.all(np.isnan(unbounded))
    expect_device_error()


def test_explicit_split_past_cap_gives_nan_rows(orc):
    """The explicit-split path sizes its grid by cap: a longer sequence gets NaN rows
    (loud), the others their attention."""
    say("explicit split, length past cap")
    lens = np.array([50, 500, 80], np.int32)
    Hq, Hkv, D = 8, 8, 64
    q, K, V = inputs(lens, Hq, Hkv, D, KVC_F16, 340)
    kp, vp, table, tab_off = paged_layout(K, V, lens, 16)
    out = DeviceBuffer(q.nbytes)
    ops.launch_batched_paged(dev(q), dev(kp), dev(vp), dev(table), dev(tab_off), dev(lens), out, 3, Hq, D, 16, 100,
                             float(1.0 / np.sqrt(D)), dtype=KVC_F16, split=64)
    got = host(out, np.float16, q.shape).astype(np.float64)
    assert np.all(np.isnan(got[1]))
    ref = oracle(orc, q, K, V, lens)
    assert np.abs(got[[0, 2]] - ref[[0, 2]]).max() <= 2e-3
    expect_device_error(b"longer than its stated cap")


def test_contiguous_length_past_its_cache_gives_nan():
    say("contiguous length past MAXS")
    lens = np.array([10, 40], np.int32)
    Hq, Hkv, D, S = 8, 8, 64, 32
    q, K, V = normal((2, Hq, D), 350, np.float16), normal((2, Hkv, S, D), 351, np.float16), normal((2, Hkv, S, D), 352, np.float16)
    out = DeviceBuffer(q.nbytes)
    ops.launch_batched_decode(dev(q), dev(K), dev(V), dev(lens), out, 2, Hq, D, S, S, 0.125, Hkv=Hkv, dtype=KVC_F16)
    assert np.all(np.isnan(host(out, np.float16, q.shape).astype(np.float64)))
    expect_device_error()


def expect_device_error(text=b"NaN"):
    """The launch that wrote NaN rows also reported it: kvc_check_device_errors returns
    KVC_ERR_ARG once, then the report is cleared."""
    from kvcache_amd._native import lib
    with pytest.raises(KvcError) as e:
        ops.check_device_errors()
    assert e.value.status == KVC_ERR_ARG
    assert text in lib().kvc_last_error()
    ops.check_device_errors()


def test_device_error_fails_the_next_device_length_call(orc):
    """Without an explicit check, the next device-length decode call returns the report
    (KVC_ERR_ARG, nothing launched) and clears it; the call after that runs normally."""
    say("device error report surfaces at the next call")
    lens = np.array([50, 500, 80], np.int32)
    Hq, Hkv, D = 8, 8, 64
    q, K, V = inputs(lens, Hq, Hkv, D, KVC_F16, 341)
    kp, vp, table, tab_off = paged_layout(K, V, lens, 16)
    args = (dev(q), dev(kp), dev(vp), dev(table), dev(tab_off), dev(lens))
    out = DeviceBuffer(q.nbytes)
    ops.launch_batched_paged(*args, out, 3, Hq, D, 16, 100, float(1.0 / np.sqrt(D)), dtype=KVC_F16, split=64)
    host(out, np.float16, q.shape)  # the launch has finished: its report is in host memory
    with pytest.raises(KvcError) as e:
        ops.launch_batched_paged(*args, out, 3, Hq, D, 16, 0, float(1.0 / np.sqrt(D)), dtype=KVC_F16)
    assert e.value.status == KVC_ERR_ARG
    ops.launch_batched_paged(*args, out, 3, Hq, D, 16, 0, float(1.0 / np.sqrt(D)), dtype=KVC_F16)
    got = host(out, np.float16, q.shape).astype(np.float64)
    assert np.abs(got - oracle(orc, q, K, V, lens)).max() <= 2e-3
    ops.check_device_errors()


@pytest.mark.parametrize("case", ["gqa_mfma_600", "mha_valu_1100"])
def test_dropin_batches_past_one_launch(orc, case):
    """qk_batched_paged_decode_attn takes any N (a grid of N x Hq in the reference,
    qwen_kernels.cu:326-334) and no cap: more sequences than one self-planned launch plans
    (512 on the matrix cores, 1024 otherwise) run as consecutive launches, each attended
    whole."""
    rng = np.random.default_rng(370)
    N, Hq, Hkv, D, hi = (600, 14, 2, 64, 700) if case == "gqa_mfma_600" else (1100, 2, 2, 64, 200)
    say(f"drop-in batch of {N} sequences, {Hq}q/{Hkv}kv D{D}, cap 0")
    lens = rng.integers(0, hi, N).astype(np.int32)
    q, K, V = inputs(lens, Hq, Hkv, D, KVC_F16, 371)
    kp, vp, table, tab_off = paged_layout(K, V, lens, 16)
    out = DeviceBuffer(q.nbytes)
    ops.qk_batched_paged_decode_attn(dev(q), out, dev(kp), dev(vp), dev(table), dev(tab_off), dev(lens), N, Hq, Hkv,
                                     D, 16, float(1.0 / np.sqrt(D)))
    got = host(out, np.float16, q.shape).astype(np.float64)
    assert np.abs(got - oracle(orc, q, K, V, lens)).max() <= 2e-3
    ops.check_device_errors()


@pytest.mark.parametrize("B", [48, 4])
def test_dropin_block_without_self_plan_needs_no_cap(orc, B):
    """A BLOCK the self-planned kernel does not page (not a power of two, or smaller than a
    wave-load) with cap 0: the longest length is read from the device and sizes the grid,
    so every sequence is attended whole, as in the reference."""
    say(f"drop-in BLOCK {B}, cap 0")
    lens = np.array([1, 47, 48, 49, 1000, 3000, 0, 333], np.int32)
    Hq, Hkv, D = 14, 2, 64
    q, K, V = inputs(lens, Hq, Hkv, D, KVC_F16, 380 + B)
    kp, vp, table, tab_off = paged_layout(K, V, lens, B)
    out = DeviceBuffer(q.nbytes)
    ops.qk_batched_paged_decode_attn(dev(q), out, dev(kp), dev(vp), dev(table), dev(tab_off), dev(lens), len(lens),
                                     Hq, Hkv, D, B, float(1.0 / np.sqrt(D)))
    got = host(out, np.float16, q.shape).astype(np.float64)
    assert np.abs(got - oracle(orc, q, K, V, lens)).max() <= 2e-3
    ops.check_device_errors()


def test_device_position_variants(orc):
    """qkcuda_rope / qkcuda_write_kv / qkcuda_paged_causal_attn (qwen_kernels.h:42-47):
    positions read from device memory give the host-position results (rope and writes
    bit for bit; the prompt attention within tolerance of the CPU restatement)."""
    say("device-position rope / write / causal attention")
    rng = np.random.default_rng(360)
    Hq, Hkv, D, B, base, Nq = 14, 2, 64, 16, 1234, 5
    x = rng.standard_normal((Nq, Hq, D)).astype(np.float16)
    a, b = dev(x), dev(x)
    pos = dev(np.array([base], np.int32))
    ops.qk_rope(a, Nq, Hq, D, base, 1e6)
    ops.qkcuda_rope(b, Nq, Hq, D, pos, 1e6)
    np.testing.assert_array_equal(host(a, np.float16, x.shape), host(b, np.float16, x.shape))
    total = base + Nq
    nbk = (total + B - 1) // B
    table = rng.permutation(nbk + 7)[:nbk].astype(np.int32)
    kv = [rng.standard_normal((nbk + 7, Hkv, B, D)).astype(np.float16) for _ in range(2)]
    knew, vnew = (rng.standard_normal((Nq, Hkv, D)).astype(np.float16) for _ in range(2))
    p1, p2 = [dev(t) for t in kv], [dev(t) for t in kv]
    ops.qk_write_kv(dev(knew), dev(vnew), p1[0], p1[1], dev(table), base, Nq, Hkv, D, B)
    ops.qkcuda_write_kv(dev(knew), dev(vnew), p2[0], p2[1], dev(table), pos, Nq, Hkv, D, B)
    kp, vp = (host(t, np.float16, kv[0].shape) for t in p1)
    np.testing.assert_array_equal(kp, host(p2[0], np.float16, kv[0].shape))
    np.testing.assert_array_equal(vp, host(p2[1], np.float16, kv[0].shape))
    q = rng.standard_normal((Nq, Hq, D)).astype(np.float16)
    out = DeviceBuffer(q.nbytes)
    ops.qkcuda_paged_causal_attn(dev(q), out, p2[0], p2[1], dev(table), pos, Nq, Hq, Hkv, D, B, 0.125)
    got = host(out, np.float16, q.shape).astype(np.float64)
    ref = orc.paged_causal(q, kp, vp, table, base, Hkv, B, 0.125)
    assert np.abs(got - ref).max() <= 2e-3


@pytest.mark.parametrize("case", ["c2_reference", "gqa_mfma_long", "mha_fp32"])
def test_read_ahead_changes_no_output(case):
    """While the kernel plans, wave 1 of every workgroup reads the first blocks of every
    sequence ahead into an LDS sink (self_prefetch): no output may change, bit for bit,
    whatever the read-ahead budget -- none, the default, or one that covers whole
    sequences -- and with the minimum length at 0 (short sequences read ahead too)."""
    lens, Hq, Hkv, D, dtype = CASES[case]
    say(f"self-planned read-ahead on/off: {case}")
    B = 16
    q, K, V = inputs(lens, Hq, Hkv, D, dtype, 340)
    nb = sum((int(x) + B - 1) // B for x in lens)
    kp, vp, table, tab_off = paged_layout(K, V, lens, B, np.random.default_rng(9).permutation(nb))
    with tuning("self_lead_tokens", 0):  # (the read-ahead runs when there are no lead chunks)
        with tuning("self_prefetch_kib", 0):
            ref = self_planned(q, kp, vp, table, tab_off, lens, Hkv, B, dtype)
        for kib, min_len in ((32768, 256), (1 << 20, 0), (64, 1)):
            with tuning("self_prefetch_kib", kib), tuning("self_prefetch_min_len", min_len):
                got = self_planned(q, kp, vp, table, tab_off, lens, Hkv, B, dtype)
            np.testing.assert_array_equal(got, ref)


LEAD_CASES = ["c2_reference", "c2_loguniform", "mha_fp32", "gqa_valu_fp32", "group2_fp16", "short_mha"]


@pytest.mark.parametrize("case", LEAD_CASES)
def test_short_sequences_while_planning(orc, case):
    """Short-sequence thresholds -- one block, the default, more than most sequences,
    and the largest (a chunk's 64 blocks; larger requests are cut to it) -- against the
    oracle, on a first and a second launch over one never-cleared workspace; and paged
    against contiguous caches bit for bit (both cut the same chunks)."""
    lens, Hq, Hkv, D, dtype = CASES[case]
    say(f"self-planned, short sequences while planning: {case}")
    B = 16
    lens = np.asarray(lens, np.int32)
    N = len(lens)
    q, K, V = inputs(lens, Hq, Hkv, D, dtype, 350)
    nb = sum((int(x) + B - 1) // B for x in lens)
    kp, vp, table, tab_off = paged_layout(K, V, lens, B, np.random.default_rng(10).permutation(nb + 7))
    want = oracle(orc, q, K, V, lens)
    ws = DeviceBuffer(ops.decode_workspace_size(N, Hq, Hkv, D, B, 0, 0, dtype))
    ws.upload(np.random.default_rng(11).integers(0, 256, ws.nbytes, dtype=np.uint8))
    for lead in (16, 64, 1000, 1 << 20):
        with tuning("self_lead_tokens", lead):
            a = self_planned(q, kp, vp, table, tab_off, lens, Hkv, B, dtype, workspace=ws)
            b = self_planned(q, kp, vp, table, tab_off, lens, Hkv, B, dtype, workspace=ws)
            out = DeviceBuffer(q.nbytes)
            ops.launch_batched_decode(dev(q), dev(K), dev(V), dev(lens), out, N, Hq, D, K.shape[2], 0,
                                      float(1.0 / np.sqrt(D)), Hkv=Hkv, dtype=dtype)
            contig = host(out, q.dtype, q.shape).astype(np.float64)
        err = np.abs(a - want).max()
        say(f"  threshold {lead}: max |err| {err:.2e}")
        assert err <= tol(dtype)
        np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(a, contig)
        assert np.all(a[lens == 0] == 0)
