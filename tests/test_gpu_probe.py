"""The read-only probe kvc_read_probe_planned (a measurement aid: the practical ceiling
of the planned decode's access pattern, reported by bench.py).  It must accept every
plan the planner makes for the shapes it supports, touch only the pools and table it is
given (its loads are bounded by buffer descriptors), and write nothing but its sink
(left at zero unless a unit's xor hits the fixed constant)."""
import numpy as np
import pytest

from kvcache_amd import KVC_F16, KVC_F32, ops
from kvcache_amd._native import check, lib
from kvcache_amd.device import DeviceBuffer

from _helpers import dev, host, normal, paged_layout, say, tuning

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", ["mha_f16", "gqa_f16_512", "mha_f32", "group2_f16"])
def test_probe_runs_over_planner_work_lists(case):
    Hq, Hkv, D, dtype, min_chunk = {"mha_f16": (8, 8, 64, KVC_F16, None), "gqa_f16_512": (14, 2, 64, KVC_F16, 512),
                                    "mha_f32": (8, 8, 64, KVC_F32, None),
                                    "group2_f16": (8, 4, 64, KVC_F16, None)}[case]
    say(f"read probe over a planner work list: {case}")
    rng = np.random.default_rng(400)
    lens = rng.integers(0, 3000, 24).astype(np.int32)
    B = 16
    nt = np.float16 if dtype == KVC_F16 else np.float32
    K = normal((len(lens), Hkv, int(lens.max()), D), 401, nt)
    kp, vp, table, tab_off = paged_layout(K, K, lens, B, rng.permutation(int(sum((lens + B - 1) // B)) + 5))
    with tuning("mfma_min_chunk", min_chunk or 1024):
        work, nu, _ = ops.decode_plan(lens, Hq, Hkv, D, B, tab_off=tab_off, table=table, dtype=dtype,
                                      target_tokens=min_chunk or 0)
    # every buffer is held in a name for the whole call: a temporary's .ptr would be freed
    # before the kernel runs
    sink = dev(np.zeros(max(nu, 1), np.int32))
    dk, dv, dt, dw = dev(kp), dev(vp), dev(table), dev(work)
    check(lib().kvc_read_probe_planned(dk.ptr, dv.ptr, dt.ptr, len(table), dw.ptr, nu, Hq, Hkv, D, B, dtype,
                                       sink.ptr, None))
    assert nu > 0
    assert not host(sink, np.int32, (max(nu, 1),)).any()


def test_empty_launch_runs():
    """kvc_empty_launch (the launch-floor measurement) launches and completes for 1 and
    1024 workgroups."""
    from kvcache_amd.device import synchronize
    say("empty launches")
    for blocks in (1, 1024):
        check(lib().kvc_empty_launch(blocks, None))
    synchronize()
