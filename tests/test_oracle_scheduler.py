"""Pins the oracle's workload generators and scheduling restatement.

Known answers come from the reference README (tests/golden/known_answers.json),
from its test programs (test_kv_manager.cu, demo_engine.cu) and from closed
forms of the policies (batch width 1 -> sequential, width >= n -> one wave).
The allocator is also compared with the reference's own block_alloc.h compiled
by oracle/Makefile (oracle/_ref) when the reference tree is present.
"""
import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())["published"]


def pub(key):
    return GOLDEN[key]["value"]


# ---- workload generators -------------------------------------------------------
def test_ragged_lengths_known_answers(orc):
    L = orc.ref_lengths(128, 2048, 12345)
    assert L.sum() == 83212 and L.max() == 2022 and L.min() >= 16
    assert round(L.mean()) == pub("ragged_batch_mean_len")
    H, D, B, LMAX, MB = 8, 64, 16, 2048, 1048576.0
    blocks = sum((int(x) + B - 1) // B for x in L)
    assert blocks == 5259
    reserved = 128 * H * LMAX * D * 4 * 2 / MB           # bench_throughput.cu:75
    used = L.sum() * H * D * 4 * 2 / MB                  # :76
    paged = (blocks * H * B * D * 4 * 2 + blocks * 4) / MB   # :77-78
    assert round(reserved) == pub("ragged_batch_reserved_mb_contiguous")
    assert round(used) == pub("ragged_batch_used_mb_contiguous")
    assert round(paged) == pub("ragged_batch_mb_paged")
    assert round(100 * used / reserved, 1) == pub("ragged_batch_util_pct_contiguous")
    budget = 4096 * MB                                    # :135-139
    per_seq_paged = ((int(L.mean()) + B - 1) // B) * H * B * D * 4 * 2
    assert int(budget / (H * LMAX * D * 4 * 2)) == pub("budget_4096mb_max_seqs_contiguous")
    assert int(budget / per_seq_paged) == pub("budget_4096mb_max_seqs_paged")


def test_continuous_trace_known_answers(orc):
    p, g, a = orc.ref_trace(256, 256, 512, 0.0, 2024)
    assert g.sum() == 48523 and abs(g.sum() - pub("offline_generated_tokens_approx")) < 100
    assert np.all(a == 0) and 16 <= p.min() and p.max() < 256 and 8 <= g.min() and g.max() < 512
    # online trace draws u after rp, rg (bench_continuous.cu:46), so lengths differ from offline
    p2, g2, a2 = orc.ref_trace(256, 256, 512, 400.0, 2024)
    assert np.all(np.diff(a2) > 0) and not np.array_equal(p2, p)
    assert abs(a2[-1] / 1e6 - 256 / 400) < 0.25      # ~256 arrivals at 400/s


def test_fill_rand_stream_gives_the_ragged_lengths():
    """bench_paged.cu:19-24 fills with x = 2r - 1 from the same LCG as the ragged lengths of
    bench_throughput.cu:50-57, so mapping its stream back through r = (x + 1) / 2 (exact in
    float32: r = k / 2^23) and L = 16 + (int)(2032 r^2) must give the README's batch
    (sum 83,212, max 2,022, 5,259 blocks of 16)."""
    from kvcache_amd import workloads as W
    x = W.fill_rand(128, 12345)
    assert x.dtype == np.float32 and -1.0 <= x.min() and x.max() < 1.0
    r = (x + np.float32(1.0)) / np.float32(2.0)
    L = np.array([16 + int(np.float32(2032.0) * ri * ri) for ri in r])
    assert L.sum() == 83212 and L.max() == 2022 and sum((int(v) + 15) // 16 for v in L) == 5259
    np.testing.assert_array_equal(L, W.ref_lengths(128, 2048, 12345))


def test_demo_trace_draws_glibc_rand():
    """demo_engine.cu:18-28 draws with srand(123)/rand(): the restated glibc generator must
    give the C library's own sequence (called through ctypes), and the trace takes the
    prompt draw before the generation draw of each request."""
    import ctypes
    import ctypes.util
    from kvcache_amd import workloads as W
    libc = ctypes.CDLL(ctypes.util.find_library("c"))
    if not hasattr(libc, "gnu_get_libc_version"):
        pytest.skip("C library is not glibc")
    for seed in (123, 0, 1, 2024, 0x80000005, 0xFFFFFFFF):
        libc.srand(ctypes.c_uint(seed))
        want = [libc.rand() for _ in range(600)]
        g = W.GlibcRand(seed)
        assert [g.rand() for _ in range(600)] == want, seed
    libc.srand(ctypes.c_uint(123))
    draws = [libc.rand() for _ in range(2 * 256)]
    p, g = W.demo_trace(256, 123)
    np.testing.assert_array_equal(p, [8 + d % 120 for d in draws[0::2]])
    np.testing.assert_array_equal(g, [16 + d % 200 for d in draws[1::2]])
    assert 8 <= p.min() and p.max() <= 127 and 16 <= g.min() and g.max() <= 215


def test_shuffle_perm_is_a_permutation():
    """main_paged.cu:28-37's table shuffle is an input generator: the paged == contiguous
    checks hold for any permutation, so only that it is one (and not the identity) matters."""
    from kvcache_amd import workloads as W
    for nb in (1, 2, 64, 5259):
        perm = W.shuffle_perm(nb, 42)
        assert sorted(perm.tolist()) == list(range(nb))
        assert nb < 64 or perm.tolist() != list(range(nb))


REF_GEN = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "ref_gen_driver"
_no_ref_gen = pytest.mark.skipif(not REF_GEN.exists(), reason="oracle/_ref/ref_gen_driver is built only where the "
                                                             "reference tree is present (oracle/Makefile, target ref)")


def _ref_gen(what):
    import subprocess
    return subprocess.run([str(REF_GEN), what], check=True, capture_output=True, text=True).stdout.splitlines()


@_no_ref_gen
def test_hval_equals_reference_generator():
    """workloads.hval against the reference's own hval (bench_throughput.cu:21-25,
    compiled from the reference tree into oracle/_ref): 864 argument tuples, large
    ones included (the hash wraps in uint32), bit for bit."""
    from kvcache_amd import workloads as W
    rows = [ln.split() for ln in _ref_gen("hval")]
    assert len(rows) == 864
    args = np.array([[int(x) for x in r[:5]] for r in rows], dtype=np.uint64)
    want = np.array([np.float32(float(r[5])) for r in rows], dtype=np.float32)
    got = np.array([W.hval(*a) for a in args], dtype=np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@_no_ref_gen
def test_shuffle_perm_equals_reference_generator():
    """workloads.shuffle_perm against the reference's table-shuffle loop (main_paged.cu:
    28-37, seed 42, compiled from the reference tree into oracle/_ref), element for
    element, for 1 .. 1000 blocks."""
    from kvcache_amd import workloads as W
    lines = _ref_gen("shuffle")
    assert len(lines) == 6
    for ln in lines:
        v = [int(x) for x in ln.split()]
        np.testing.assert_array_equal(W.shuffle_perm(v[0], 42), v[1:])


# ---- allocator / manager ---------------------------------------------------------
def test_kv_manager_known_answers(orc):
    # test_kv_manager.cu:13-55: 8 blocks x 4 tokens, Hkv 2, D 8
    k = orc.Kvm(8, 4, 2, 8)
    assert k.free_blocks() == 8
    assert k.allocate_prompt(0, 5) and len(k.table(0)) == 2 and k.cur_len(0) == 5
    assert k.free_blocks() == 6 and k.slack(0) == 3
    for _ in range(3):
        k.append_token(0)
    assert len(k.table(0)) == 2 and k.slack(0) == 0
    k.append_token(0)
    assert len(k.table(0)) == 3 and k.cur_len(0) == 9 and k.free_blocks() == 5
    assert k.allocate_prompt(1, 20) and k.free_blocks() == 0
    assert not k.allocate_prompt(2, 1) and k.table(2) == []
    assert not k.append_token(1)
    k.free(0)
    assert k.table(0) == [] and k.free_blocks() == 3
    assert k.append_token(1)
    # test_kv_manager.cu:53-55 expects (((3*2+1)*4+2)*8) = 240
    assert k.slot_offset(3, 1, 2) == 240
    # fresh pool hands out 0,1,2,...; A took 0,1 then 2; B took 3..7; A's free pushes
    # 0,1,2 so B's growth pops 2 (LIFO, block_alloc.h:16,25,31)
    assert k.table(1) == [3, 4, 5, 6, 7, 2]


def _random_script(seed, total=16, n=200):
    r = np.random.default_rng(seed)
    ops, args = [], []
    for _ in range(n):
        x = r.random()
        if x < 0.6:
            ops.append(0); args.append(0)
        elif x < 0.95:
            ops.append(-1); args.append(int(r.integers(1, 6)))
        else:
            ops.append(-2); args.append(0)
    return ops, args


def _script_text(total, ops, args):
    lines = [str(total)]
    for o, a in zip(ops, args):
        lines.append("A" if o == 0 else (f"F {a}" if o == -1 else "R"))
    return "\n".join(lines) + "\n"


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_alloc_oracle_matches_reference_code(orc, seed):
    if not orc.ref_driver_available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    ops, args = _random_script(seed)
    ours = orc.alloc_script(16, ops, args).tolist()
    ref = orc.run_ref_alloc_driver(_script_text(16, ops, args))
    assert ours == ref


def test_blocks_needed_and_done_against_reference_code(orc):
    if not orc.ref_driver_available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    cases = [(l, b) for l in (0, 1, 15, 16, 17, 31, 32, 33, 1000) for b in (1, 4, 16)]
    out = orc.run_ref_alloc_driver("1\n" + "".join(f"N {l} {b}\n" for l, b in cases))
    assert out == [(l + b - 1) // b for l, b in cases]
    out = orc.run_ref_alloc_driver("1\nD 5 9 4\nD 5 8 4\nD 0 0 0\n")
    assert out == [1, 0, 1]


# ---- scheduling ------------------------------------------------------------------
POOL = 32768  # bench_continuous.cu:33-34: 2048 MB / (8*16*64*2*4 B)


def test_static_offline_known_answers(orc):
    p, g, a = orc.ref_trace()
    rc, st, order = orc.sim_static(p, g, a, 16, POOL, 32)
    assert rc == 0 and st.iters == pub("offline_static_iters")
    assert round(100 * st.useful_steps / st.slot_steps, 1) == pub("offline_static_slot_util_pct")
    assert st.tokens == 48523 and st.finished == 256
    assert order[:3].tolist() == [176, 161, 162]     # libstdc++ introsort permutation of equal keys


def test_continuous_offline_known_answers(orc):
    p, g, a = orc.ref_trace()
    rc, st = orc.sim_engine(p, g, a, 16, POOL, 32)
    assert rc == 0 and st.iters == 1801 and st.tokens == 48523 and st.useful_steps == st.slot_steps
    # README.md:96's 1701 is the Engine fed in run_static's std::sort order
    _, _, order = orc.sim_static(p, g, a, 16, POOL, 32)
    rc, st2 = orc.sim_engine(p[order], g[order], a[order], 16, POOL, 32)
    assert st2.iters == pub("offline_continuous_iters_readme")
    assert 100 * st2.useful_steps / st2.slot_steps == pub("offline_continuous_slot_util_pct")


@pytest.mark.parametrize("kv_write", [False, True])
def test_policy_closed_forms(orc, kv_write):
    r = np.random.default_rng(3)
    n = 40
    p = r.integers(1, 60, n).astype(np.int32)
    g = r.integers(1, 50, n).astype(np.int32)
    a = np.zeros(n)
    # width 1: strictly sequential; latency of request k = sum of gen[0..k] steps of cost 1
    rc, st = orc.sim_engine(p, g, a, 16, 10000, 1, kv_write)
    assert st.iters == g.sum() and st.tokens == g.sum()
    lat = np.sort(np.cumsum(g).astype(np.float64))
    assert st.avg_latency_us == pytest.approx(lat.mean(), abs=1e-9)
    assert st.p99_latency_us == lat[min(int(n * 0.99), n - 1)]
    assert st.p50_latency_us == lat[min(int(n * 0.5), n - 1)]
    rc, ss, _ = orc.sim_static(p, g, a, 16, 10000, 1, kv_write)
    assert ss.iters == g.sum() and ss.tokens == g.sum()
    # width >= n: one wave of max(gen) steps for both policies
    rc, st = orc.sim_engine(p, g, a, 16, 10000, n, kv_write)
    assert st.iters == g.max()
    rc, ss, _ = orc.sim_static(p, g, a, 16, 10000, n, kv_write)
    assert ss.iters == g.max() and ss.slot_steps == n * g.max() and ss.useful_steps == g.sum()
    # one wave: after step t the sequences with gen >= t hold ceil((prompt + t)/16) blocks;
    # a sequence that finished at step t' < t was retired at the start of step t'+1
    peak = max(sum((int(pi) + t + 15) // 16 for pi, gi in zip(p, g) if gi >= t) for t in range(1, g.max() + 1))
    assert st.peak_blocks == peak


def test_isolated_poisson_arrivals(orc):
    # arrivals far apart: every request runs alone, latency = gen * c0
    n = 20
    p = np.full(n, 10, np.int32)
    g = np.arange(1, n + 1, dtype=np.int32)
    a = np.arange(n) * 1e6
    rc, st = orc.sim_engine(p, g, a, 16, 1000, 8, False, (5.0, 0.0, 0.0))
    lat = np.sort(g * 5.0)
    assert st.avg_latency_us == pytest.approx(lat.mean()) and st.iters == g.sum()
    assert st.wall_us == pytest.approx(a[-1] + g[-1] * 5.0)


def test_demo_engine_invariants(orc):
    # demo_engine.cu:14-42: 8 heads, D 64, BLOCK 16, 512 blocks, width 32, srand(123)
    from kvcache_amd import workloads as W
    p, g = W.demo_trace(256, 123)
    assert 8 <= p.min() and p.max() <= 127 and 16 <= g.min() and g.max() <= 215
    rc, st = orc.sim_engine(p, g, np.zeros(256), 16, 512, 32)
    assert rc == 0 and st.tokens == g.sum() and st.finished == 256 and st.peak_blocks <= 512


def test_never_admissible_request_is_reported(orc):
    # worst case ceil((prompt+gen)/16) = 7 blocks > pool of 5: the reference Engine would spin forever
    rc, st = orc.sim_engine([50], [50], [0.0], 16, 5, 4)
    assert rc == 1
    rc, st, _ = orc.sim_static([50], [50], [0.0], 16, 5, 4)
    assert rc == 1 and st.finished == 0


def test_bench_memory_report_matches_readme(orc):
    """bench.py's memory report (bench_throughput.cu:73-80,135-139) gives the README's
    numbers in the reference's fp32 layout for the config-2 batch."""
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    import bench
    m = bench.memory_accounting(orc.ref_lengths(128, 2048, 12345), 8, 64, 16)
    r = m["fp32_reference_layout"]
    assert m["blocks"] == 5259 and m["table_bytes"] == 5259 * 4
    assert round(r["contiguous_reserved_mb"]) == pub("ragged_batch_reserved_mb_contiguous")
    assert round(r["used_mb"]) == pub("ragged_batch_used_mb_contiguous")
    assert round(r["paged_mb"]) == pub("ragged_batch_mb_paged")
    assert r["contiguous_util_pct"] == pub("ragged_batch_util_pct_contiguous")
    assert r["seqs_in_4096mb_contiguous"] == pub("budget_4096mb_max_seqs_contiguous")
    assert r["seqs_in_4096mb_paged"] == pub("budget_4096mb_max_seqs_paged")
    assert m["fp16"]["used_mb"] * 2 == pytest.approx(r["used_mb"], abs=0.1)


def test_bench_reads_the_committed_profiles():
    """The bench line quotes the committed rocprofv3 summaries: every key it looks up is
    there, the profiled kernel times are plausible, and the roofline blocks follow
    from them (algorithmic bytes / time / 8 TB/s)."""
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    import bench
    pv = bench.profile_values()
    for key in ("headline_timed_mean_us", "device_lengths_timed_mean_us", "c4_layer_timed_mean_us",
                "c3_split512_split_kernel_mean_us", "c3_split512_merge_kernel_mean_us"):
        assert 1.0 < pv[key] < 100.0, key
    assert bench.profiled_launch_us() == pv["headline_timed_mean_us"]
    rb = bench.roofline_block(46174244, 17.0, "k", ("c3_split512_split_kernel_mean_us", "c3_split512_merge_kernel_mean_us"))
    us = pv["c3_split512_split_kernel_mean_us"] + pv["c3_split512_merge_kernel_mean_us"]
    assert rb["profile"]["kernel_us"] == pytest.approx(us, abs=1e-3)
    assert rb["profile"]["frac"] == pytest.approx(46174244 / (us * 1e-6) / 8e12, abs=1e-4)
    assert rb["frac"] == pytest.approx(46174244 / 17e-6 / 8e12, abs=1e-4)
    traffic, sym = bench.measured_traffic()
    assert traffic and 1.0 < traffic / 170702384 < 1.02 and "split_kernel" in sym
