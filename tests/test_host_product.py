"""The product's host logic (C++ BlockAllocator / Engine / run_static behind the
C ABI, and the Python workload generators) against the oracle -- bit-exact, on
the CPU.  The Engine runs in scheduling-only mode (device = 0, virtual clock):
no GPU, same decisions, same packed per-step metadata (digest)."""
import numpy as np
import pytest

from kvcache_amd import KVC_F16, KVC_F32
from kvcache_amd import workloads as W
from kvcache_amd._native import KVC_ERR_STATE, KvcError
from kvcache_amd.engine import BlockAllocator, Engine, EngineConfig, blocks_needed, run_continuous, run_static


def test_workload_generators_match_oracle(orc):
    np.testing.assert_array_equal(W.ref_lengths(), orc.ref_lengths())
    np.testing.assert_array_equal(W.ref_lengths(64, 4096, 99), orc.ref_lengths(64, 4096, 99))
    for rate in (0.0, 400.0):
        for a, b in zip(W.ref_trace(rate=rate), orc.ref_trace(rate=rate)):
            np.testing.assert_array_equal(a, b)
    s = np.arange(4)[:, None, None, None]
    h = np.arange(3)[None, :, None, None]
    pos = np.arange(5)[None, None, :, None]
    d = np.arange(8)[None, None, None, :]
    vec = W.hval(s, h, pos, d, 2)   # an input generator: deterministic values in [-1, 1)
    assert vec.shape == (4, 3, 5, 8) and vec.min() >= -1.0 and vec.max() < 1.0
    assert len(np.unique(vec)) > 400


def test_baseline_generators_are_seeded_and_shaped():
    a = W.loguniform_lengths(128, 16, 2048, 7)
    assert np.array_equal(a, W.loguniform_lengths(128, 16, 2048, 7)) and a.min() >= 16 and a.max() <= 2048
    p, g, arr = W.baseline_trace(256, 400.0, 11)
    assert p.min() >= 1 and p.max() <= 256 and g.min() >= 1 and g.max() <= 512 and np.all(np.diff(arr) > 0)
    assert 100 < g.mean() < 260


def _script(seed, n=300):
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


@pytest.mark.parametrize("seed", range(4))
def test_block_allocator_matches_oracle_and_reference(orc, seed):
    ops, args = _script(seed)
    a = BlockAllocator(16)
    held, out = [], []
    for o, k in zip(ops, args):
        if o == 0:
            b = a.alloc(); out.append(b)
            if b >= 0:
                held.append(b)
        elif o == -1:
            fr, held = held[:k], held[k:]
            a.free_blocks(fr); out.append(a.free_count())
        else:
            a.reset(); held = []; out.append(a.free_count())
    assert out == orc.alloc_script(16, ops, args).tolist()
    if orc.ref_driver_available():
        text = "16\n" + "".join("A\n" if o == 0 else (f"F {k}\n" if o == -1 else "R\n") for o, k in zip(ops, args))
        assert out == orc.run_ref_alloc_driver(text)


def test_allocator_basics_and_shuffle():
    a = BlockAllocator(8)
    assert [a.alloc() for _ in range(3)] == [0, 1, 2] and a.used_count() == 3
    a.free_blocks([1, 0])
    assert a.alloc() == 0 and a.alloc() == 1
    b = BlockAllocator(1000)
    b.shuffle(5)
    got = [b.alloc() for _ in range(1000)]
    assert sorted(got) == list(range(1000)) and got != list(range(1000)) and b.alloc() == -1
    assert blocks_needed(17, 16) == 2 and blocks_needed(0, 16) == 0


COST = (20.0, 1.5, 0.01)


def _cfg(block, num_blocks, width, kv_write, **kw):
    return EngineConfig(n_heads=8, head_dim=64, block_size=block, num_blocks=num_blocks, max_batch=width,
                        kv_write=kv_write, clock_mode=1, virt_c0=COST[0], virt_c1=COST[1], virt_c2=COST[2],
                        device=False, **kw)


def _same(ours, ref):
    assert ours.iters == ref.iters
    assert ours.tokens == ref.tokens
    assert ours.slot_steps == ref.slot_steps and ours.useful_steps == ref.useful_steps
    assert ours.peak_blocks == ref.peak_blocks and ours.finished == ref.finished
    assert ours.gpu_us == ref.gpu_us and ours.wall_us == ref.wall_us
    assert ours.avg_latency_us == ref.avg_latency_us
    assert ours.p50_latency_us == ref.p50_latency_us and ours.p99_latency_us == ref.p99_latency_us
    assert ours.step_digest == ref.digest


TRACES = {
    "ref_offline": lambda: W.ref_trace(),
    "ref_poisson400": lambda: W.ref_trace(rate=400.0),
    "baseline_offline": lambda: W.baseline_trace(256, 0.0, 11),
    "baseline_poisson400": lambda: W.baseline_trace(256, 400.0, 11),
}


@pytest.mark.parametrize("trace", sorted(TRACES))
@pytest.mark.parametrize("kv_write", [False, True])
def test_engine_and_static_match_oracle(orc, trace, kv_write):
    p, g, a = TRACES[trace]()
    for num_blocks in (32768, 600):  # roomy pool, and one where the reservation binds
        eng = Engine(_cfg(16, num_blocks, 32, kv_write))
        rc, ref = orc.sim_engine(p, g, a, 16, num_blocks, 32, kv_write, COST)
        assert rc == 0
        _same(run_continuous(p, g, a, eng), ref)
        rc, ref_s, _ = orc.sim_static(p, g, a, 16, num_blocks, 32, kv_write, COST)
        _same(run_static(p, g, a, eng, 32), ref_s)


def _random_trace(seed):
    r = np.random.default_rng(4000 + seed)
    n = int(r.integers(1, 121))
    prompt = r.integers(1, int(r.choice([8, 64, 256, 1024])) + 1, size=n).astype(np.int32)
    gmax = int(r.choice([4, 64, 512]))
    if r.random() < 0.5:
        gen = np.minimum(r.geometric(1.0 / max(gmax / 3, 1.5), size=n), gmax).astype(np.int32)
    else:
        gen = r.integers(1, gmax + 1, size=n).astype(np.int32)
    rate = float(r.choice([0.0, 20.0, 400.0, 5000.0]))
    arrival = np.cumsum(r.exponential(1e6 / rate, size=n)) if rate > 0 else np.zeros(n)
    block = int(r.choice([1, 4, 16, 32]))
    width = int(r.integers(1, 49))
    need = max(blocks_needed(int(a + b), block) for a, b in zip(prompt, gen))
    num_blocks = need + int(r.choice([0, 1, 3 * need, 100000]))
    return prompt, gen, arrival.astype(np.float64), block, num_blocks, width, bool(r.random() < 0.5)


@pytest.mark.parametrize("seed", range(20))
def test_engine_random_traces_match_oracle(orc, seed):
    """Seeded random traces (1-120 requests, prompts up to 1024, geometric or uniform
    generation lengths, offline or Poisson arrivals at 20-5000 req/s, blocks of 1-32
    tokens, widths 1-48, pools from the largest request's need up to roomy, with and
    without K/V writes): the continuous engine and the static batcher make the
    oracle's decisions step for step (engine.h:100-148, scheduler.h:182-238)."""
    p, g, a, block, num_blocks, width, kv_write = _random_trace(seed)
    eng = Engine(_cfg(block, num_blocks, width, kv_write))
    rc, ref = orc.sim_engine(p, g, a, block, num_blocks, width, kv_write, COST)
    assert rc == 0
    _same(run_continuous(p, g, a, eng), ref)
    rc, ref_s, _ = orc.sim_static(p, g, a, block, num_blocks, width, kv_write, COST)
    assert rc == 0
    _same(run_static(p, g, a, eng, width), ref_s)


def test_engine_reference_known_answers():
    p, g, a = W.ref_trace()
    eng = Engine(_cfg(16, 32768, 32, False))
    st = run_static(p, g, a, eng, 32)
    assert st.iters == 3898 and st.tokens == 48523 and round(100 * st.slot_util, 1) == 38.9
    co = run_continuous(p, g, a, eng)
    assert co.iters == 1801 and co.slot_util == 1.0


def test_engine_demo_invariants():
    p, g = W.demo_trace(256, 123)
    eng = Engine(_cfg(16, 512, 32, False))
    st = run_continuous(p, g, np.zeros(256), eng)
    assert st.tokens == g.sum() and st.finished == 256 and st.peak_blocks <= 512


def test_engine_step_api_and_reset():
    eng = Engine(_cfg(16, 100, 4, False))
    for i in range(6):
        eng.add_request(10, 3)
    steps = 0
    while eng.step():
        steps += 1
    st = eng.stats()
    assert st.finished == 6 and st.tokens == 18
    eng.reset()
    assert eng.stats().iters == 0


def test_never_admissible_request_raises():
    eng = Engine(_cfg(16, 5, 4, False))
    eng.add_request(50, 50)
    with pytest.raises(KvcError) as e:
        eng.run()
    assert e.value.status == KVC_ERR_STATE


def test_out_of_order_arrivals_rejected():
    eng = Engine(_cfg(16, 100, 4, False))
    eng.add_request(5, 5, 100.0)
    with pytest.raises(KvcError):
        eng.add_request(5, 5, 50.0)


@pytest.mark.parametrize("dtype", [KVC_F32, KVC_F16])
def test_gqa_layers_config_is_accepted_host_only(dtype):
    cfg = _cfg(16, 10922, 32, True, n_kv_heads=2, n_layers=24, dtype=dtype)
    cfg.n_heads = 14
    eng = Engine(cfg)
    p, g, a = W.ref_trace(nreq=64)
    st = run_continuous(p, g, a, eng)
    assert st.tokens == g.sum()


# ---- decode planner (host logic of the planned path) ---------------------------------
@pytest.mark.parametrize("case", ["ref", "loguniform", "uniform", "tiny", "gqa", "small_block"])
def test_decode_plan_covers_every_token_once(case):
    from kvcache_amd import ops
    Hq, Hkv, D, B = 8, 8, 64, 16
    if case == "ref":
        lens = W.ref_lengths()
    elif case == "loguniform":
        lens = W.loguniform_lengths(128, 16, 2048, 7)
    elif case == "uniform":
        lens = np.full(64, 650, np.int32)
    elif case == "tiny":
        lens = np.array([0, 1, 2, 15, 16, 17], np.int32)
    elif case == "gqa":
        lens, Hq, Hkv = np.array([8192, 16384, 32768, 32768], np.int32), 14, 2
    else:
        lens, B = np.array([5, 8, 13, 3000], np.int32), 4
    tab_off = np.concatenate([[0], np.cumsum([(int(x) + B - 1) // B for x in lens])]).astype(np.int32)
    table = np.random.default_rng(3).permutation(int(tab_off[-1]) + 5)[: tab_off[-1]].astype(np.int32)
    work, nu, nr = ops.decode_plan(lens, Hq, Hkv, D, B, tab_off=tab_off, table=table)
    assert nu == len(work) > 0
    # grouped-query fp16 units carry their first block ids after the 8-int header
    n_inl = work[:, 4] >> 16
    if work.shape[1] > 8:
        for row, k in zip(work, n_inl):
            nblk = (row[3] - 1) // B - row[2] // B + 1 if row[3] > row[2] else 0
            assert k == min(nblk, work.shape[1] - 8)
            np.testing.assert_array_equal(row[8: 8 + k], table[row[7]: row[7] + k])
    else:
        assert np.all(n_inl == 0)
    work = work[:, :8].copy()
    work[:, 4] &= 0xFFFF
    sizes = work[:, 3] - work[:, 2]
    split = work[:, 4] > 1
    # chunks of split sequences first (their merges overlap later units), each group longest first
    # in length buckets of a 42nd of the chunk target
    assert not np.any(np.diff(split.astype(int)) > 0), "split chunks precede whole sequences"
    T = ops.decode_plan_chunk(lens, Hq, Hkv, D, B)
    buckets = np.minimum(63, sizes.astype(np.int64) * 42 // T)
    assert np.all(np.diff(buckets[split]) <= 0) and np.all(np.diff(buckets[~split]) <= 0), "longest first"
    assert np.all(np.diff(sizes[split]) <= T // 42 + 1) and np.all(np.diff(sizes[~split]) <= T // 42 + 1)
    nsub = Hq // Hkv // (7 if Hq // Hkv == 7 else Hq // Hkv)
    hks = Hkv * nsub
    cover = {}
    groups = {}
    for s, hc, j0, j1, nc, rec, ctr, tab in work.tolist():
        h, c = hc & 0xFFFF, hc >> 16
        assert 0 <= s < len(lens) and 0 <= h < hks and 0 <= j0 <= j1 <= lens[s] and 0 <= c < nc
        assert tab == tab_off[s] + j0 // B
        cover.setdefault((s, h), []).append((j0, j1, c, nc))
        if nc > 1:
            assert j0 % B == 0 and rec >= 0 and ctr >= 0
            assert groups.setdefault((s, h), (rec, ctr, nc)) == (rec, ctr, nc)
        else:
            assert rec == -1 and ctr == -1
    for s in range(len(lens)):
        for h in range(hks):
            parts = sorted(cover[(s, h)])
            assert [c for _, _, c, _ in sorted(parts, key=lambda x: x[2])] == list(range(parts[0][3]))
            assert parts[0][0] == 0 and parts[-1][1] == lens[s]
            assert all(a[1] == b[0] for a, b in zip(parts, parts[1:])), "chunks tile [0, L) exactly"
    recs = sorted(v[0] + k for v in groups.values() for k in range(v[2]))
    assert recs == list(range(nr)), "record ids are dense and disjoint"
    assert sorted(v[1] for v in groups.values()) == list(range(len(groups)))


@pytest.mark.parametrize("Hq,Hkv,D,B,dtype", [(8, 8, 64, 16, 1), (14, 2, 64, 16, 1), (14, 2, 64, 16, 0),
                                              (8, 8, 64, 4, 1), (32, 8, 128, 16, 1)])
def test_decode_plan_capacity_bounds_every_plan(Hq, Hkv, D, B, dtype):
    """The graph-safe launches are sized by kvc_decode_plan_capacity(N, tokens): no plan
    of at most N sequences holding at most `tokens` tokens may need more units or
    partial records than it returns, whatever the length mix."""
    import ctypes as C

    from kvcache_amd import ops
    from kvcache_amd._native import lib
    rng = np.random.default_rng(Hq * 100 + D + B + dtype)
    N, tokens = 32, 32 * 2048
    cap = C.c_int(0)
    assert lib().kvc_decode_plan_capacity(N, tokens, Hq, Hkv, D, B, dtype, C.byref(cap)) == 0
    mixes = [np.full(N, tokens // N), np.r_[[tokens - (N - 1)], np.ones(N - 1, int)], np.ones(N, int),
             np.array([tokens // 2, tokens // 2]), np.array([tokens])]
    for _ in range(20):
        n = int(rng.integers(1, N + 1))
        cut = np.sort(rng.choice(np.arange(1, tokens), n - 1, replace=False)) if n > 1 else np.array([], int)
        mixes.append(np.diff(np.r_[0, cut, int(rng.integers(n, tokens + 1))]))
    planned = 0
    for lens in mixes:
        lens = np.maximum(np.asarray(lens, np.int32), 0)
        try:
            _, nu, nr = ops.decode_plan(lens, Hq, Hkv, D, B, dtype=dtype)
        except Exception as e:  # sequences too long for a path are refused by the planner itself
            assert "too long" in str(e) or "unsupported" in str(e).lower(), e
            continue
        planned += 1
        assert nu <= cap.value and nr <= cap.value, (lens.tolist()[:8], nu, nr, cap.value)
    assert planned >= len(mixes) - 2


def test_decode_plan_chunk_sizing():
    # one or two heads per unit: the automatic target is the batch's tokens per unit
    # slot capped at 640, and a sequence stays whole up to 1.5 targets; grouped-query
    # plans cut long contexts into ~1024-token units (planner rules of abi.hip)
    from kvcache_amd import ops
    for lens, Hq, Hkv, units, biggest in ((W.ref_lengths(), 8, 8, 1408, 960),
                                         (W.loguniform_lengths(128, 16, 2048, 7), 8, 8, 1392, 720),
                                         (np.array([8192, 16384, 32768, 32768], np.int32), 14, 2, 176, 1024)):
        work, nu, nr = ops.decode_plan(lens, Hq, Hkv, 64, 16, dtype=KVC_F16)
        sizes = work[:, 3] - work[:, 2]
        assert nu == units and sizes.max() <= biggest, (nu, int(sizes.max()))
