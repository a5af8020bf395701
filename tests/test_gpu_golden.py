"""The HIP kernels against the committed golden attention cases
(tests/golden/attention_golden.npz, written by the CPU restatement): config 1 at full
size on the contiguous and paged paths (paged == contiguous bit for bit), config 2's
shape on 16 ragged sequences (device-lengths and host-planned paths), config 3's
shape (grouped-query, split contexts up to 8192 tokens) and causal prompt attention.
Bars: 1e-5 fp32, 2e-3 fp16 (max abs)."""
import sys
from pathlib import Path

import numpy as np
import pytest

from kvcache_amd import KVC_F16, KVC_F32, ops
from kvcache_amd.device import DeviceBuffer

from _helpers import dev, host, paged_layout, say

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import attention_cases as AC  # noqa: E402

pytestmark = pytest.mark.gpu
GOLD = np.load(Path(__file__).resolve().parent / "golden" / "attention_golden.npz")


def case(name):
    c = AC.inputs(name)
    assert str(GOLD[f"{name}/digest"]) == AC.digest(c)
    return c, GOLD[f"{name}/out"]


def test_golden_c1_contiguous_and_paged():
    say("golden c1")
    c, ref = case("c1")
    q, K, V = c["q"][0], c["K"][0], c["V"][0]
    H, S, D = K.shape
    scale = float(1.0 / np.sqrt(D))
    out = DeviceBuffer(q.nbytes)
    ops.launch_decode(dev(q), dev(K), dev(V), out, S, H, D, S, scale, dtype=KVC_F32)
    oc = host(out, np.float32, q.shape)
    assert np.abs(oc - ref[0]).max() <= 1e-5
    kp, vp, table, _ = paged_layout(K[None], V[None], [S], 16, c["perm"])
    outp = DeviceBuffer(q.nbytes)
    ops.launch_paged(dev(q), dev(kp), dev(vp), dev(table), outp, S, H, D, 16, scale, dtype=KVC_F32)
    np.testing.assert_array_equal(host(outp, np.float32, q.shape), oc)


@pytest.mark.parametrize("name", ["c2", "c3"])
def test_golden_batched_paths(name):
    say(f"golden {name}")
    c, ref = case(name)
    q, K, V, lens = c["q"], c["K"], c["V"], c["lens"]
    N, Hq, D = q.shape
    Hkv = c["Hkv"]
    scale = float(1.0 / np.sqrt(D))
    kp, vp, table, tab_off = paged_layout(K, V, lens, 16, c["perm"])
    dq, dk, dv, dt, do = dev(q), dev(kp), dev(vp), dev(table), dev(tab_off)
    out = DeviceBuffer(q.nbytes)
    ops.launch_batched_paged(dq, dk, dv, dt, do, dev(lens), out, N, Hq, D, 16, int(lens.max()), scale, Hkv=Hkv,
                             dtype=KVC_F16)
    assert np.abs(host(out, np.float16, q.shape) - ref).max() <= 2e-3
    work, nu, nr = ops.decode_plan(lens, Hq, Hkv, D, 16, tab_off=tab_off, table=table, dtype=KVC_F16)
    out2 = DeviceBuffer(q.nbytes)
    ops.launch_batched_paged_planned(dq, dk, dv, dt, len(table), out2, N, Hq, Hkv, D, 16, scale, dev(work), nu, nr,
                                     dtype=KVC_F16)
    assert np.abs(host(out2, np.float16, q.shape) - ref).max() <= 2e-3


def test_golden_causal_prompt_attention():
    say("golden causal")
    c, ref = case("causal")
    q, K, V = c["q"], c["K"], c["V"]
    P, Hq, D = q.shape
    L = K.shape[2]
    kp, vp, table, _ = paged_layout(K, V, [L], 16, c["perm"])
    out = DeviceBuffer(q.nbytes)
    ops.qk_paged_causal_attn(dev(q), out, dev(kp), dev(vp), dev(table), c["q_pos_base"], P, Hq, c["Hkv"], D, 16,
                             float(1.0 / np.sqrt(D)), dtype=KVC_F16)
    assert np.abs(host(out, np.float16, q.shape) - ref).max() <= 2e-3
