"""The allocation-free entry point kvc_paged_causal_attn_dev_noalloc (no counterpart in
the reference; for callers that cannot allocate, e.g. under HIP graph capture): its
split-K partials live in a static device array.  It must give the same outputs, bit for
bit, as kvc_paged_causal_attn_dev with a caller workspace -- the same kernels on the same
plan -- on two calls in a row, the second smaller (the array keeps the first call's
contents), and refuse sizes past the array."""
import ctypes as C

import numpy as np
import pytest

from kvcache_amd import KVC_F16
from kvcache_amd._native import KVC_ERR_UNSUPPORTED, check, lib
from kvcache_amd.device import DeviceBuffer

from _helpers import dev, host, say

pytestmark = pytest.mark.gpu
Hq, Hkv, D, B = 14, 2, 64, 16


def _case(rng, base, Nq):
    total = base + Nq
    nbk = (total + B - 1) // B
    table = rng.permutation(nbk + 9)[:nbk].astype(np.int32)
    kp = rng.standard_normal((nbk + 9, Hkv, B, D)).astype(np.float16)
    vp = rng.standard_normal((nbk + 9, Hkv, B, D)).astype(np.float16)
    q = rng.standard_normal((Nq, Hq, D)).astype(np.float16)
    return q, kp, vp, table


def test_noalloc_equals_workspace_entry_on_two_calls(orc):
    rng = np.random.default_rng(77)
    L = lib()
    for base, Nq in ((3000, 7), (40, 2)):  # the second call is smaller
        say(f"no-alloc prompt attention: base {base}, {Nq} queries")
        q, kp, vp, table = _case(rng, base, Nq)
        dq, dk, dv, dt, pos = dev(q), dev(kp), dev(vp), dev(table), dev(np.array([base], np.int32))
        ref_out, out = DeviceBuffer(q.nbytes), DeviceBuffer(q.nbytes)
        ws = DeviceBuffer(int(L.kvc_paged_causal_attn_dev_workspace_size(Nq, Hq, Hkv, D, B, KVC_F16)))
        check(L.kvc_paged_causal_attn_dev(dq.ptr, ref_out.ptr, dk.ptr, dv.ptr, dt.ptr, pos.ptr, Nq, Hq, Hkv, D, B,
                                          C.c_float(0.125), KVC_F16, ws.ptr, ws.nbytes, None))
        check(L.kvc_paged_causal_attn_dev_noalloc(dq.ptr, out.ptr, dk.ptr, dv.ptr, dt.ptr, pos.ptr, Nq, Hq, Hkv, D, B,
                                                  C.c_float(0.125), KVC_F16, None))
        got = host(out, np.float16, q.shape)
        np.testing.assert_array_equal(got, host(ref_out, np.float16, q.shape))
        ref = orc.paged_causal(q, kp, vp, table, base, Hkv, B, 0.125)
        assert np.abs(got.astype(np.float64) - ref).max() <= 2e-3


def test_noalloc_refuses_sizes_past_its_scratch():
    """A call whose partials would not fit the static array is refused.  Every buffer is
    real and large enough for the call, so even a refusal that came too late could not
    make the kernel read outside them."""
    say("no-alloc prompt attention: oversized call refused")
    L = lib()
    rng = np.random.default_rng(78)
    q, kp, vp, table = _case(rng, 0, 300)
    dq, dk, dv, dt, pos = dev(q), dev(kp), dev(vp), dev(table), dev(np.array([0], np.int32))
    out = DeviceBuffer(q.nbytes)
    rc = L.kvc_paged_causal_attn_dev_noalloc(dq.ptr, out.ptr, dk.ptr, dv.ptr, dt.ptr, pos.ptr, 300, Hq, Hkv, D, B,
                                             C.c_float(0.125), KVC_F16, None)
    assert rc == KVC_ERR_UNSUPPORTED
    assert b"static scratch" in L.kvc_last_error()
