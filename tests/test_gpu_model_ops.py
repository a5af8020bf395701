"""Decoder-step operations on the GPU against the CPU restatement (oracle/model.py)
on the same fp16 inputs (qwen_kernels.cu:13-107; linear layers through rocBLAS)."""
import numpy as np
import pytest

from kvcache_amd import KVC_F16, KVC_F32, ops
from kvcache_amd.device import DeviceBuffer
from oracle import model as M

from _helpers import dev, host, normal, say

pytestmark = pytest.mark.gpu


def close(got, ref, rel=2e-3):
    got = np.asarray(got, np.float64)
    assert np.all(np.abs(got - ref) <= rel * np.maximum(1.0, np.abs(ref))), np.abs(got - ref).max()


def test_embed_rmsnorm_bias_residual_silu():
    say("model ops: embed / rmsnorm / bias / residual / silu")
    V, H, L = 1000, 896, 7
    table = normal((V, H), 200, np.float16)
    ids = np.array([0, 999, 5, 123, -4, 1000, 77], np.int32)
    out = DeviceBuffer(L * H * 2)
    ops.qk_embed_gather(out, dev(table), dev(ids), L, H, V)
    np.testing.assert_array_equal(host(out, np.float16, (L, H)).astype(np.float64), M.embed_gather(table, ids))
    x, w = normal((L, H), 201, np.float16), (1 + 0.1 * normal((H,), 202)).astype(np.float16)
    y = DeviceBuffer(L * H * 2)
    ops.qk_rmsnorm(y, dev(x), dev(w), L, H, 1e-6)
    close(host(y, np.float16, (L, H)), M.rmsnorm(x, w, 1e-6))
    b = normal((H,), 203, np.float16)
    xb = dev(x)
    ops.qk_add_bias(xb, dev(b), L, H)
    close(host(xb, np.float16, (L, H)), x.astype(np.float64) + b)
    r = normal((L, H), 204, np.float16)
    ops.qk_add_residual(xb, dev(r), L * H)
    close(host(xb, np.float16, (L, H)), (x.astype(np.float64) + b).astype(np.float16).astype(np.float64) + r)
    g, u = normal((L, 4864), 205, np.float16), normal((L, 4864), 206, np.float16)
    o = DeviceBuffer(g.nbytes)
    ops.qk_silu_mul(o, dev(g), dev(u), g.size)
    close(host(o, np.float16, g.shape), M.silu_mul(g, u))


@pytest.mark.parametrize("per_row", [False, True])
def test_rope(per_row):
    say(f"model ops: rope per_row={per_row}")
    L, Hh, D, theta = 9, 14, 64, 1e6
    x = normal((L, Hh, D), 210, np.float16)
    dx = dev(x)
    if per_row:
        pos = np.array([0, 1, 7, 100, 255, 511, 4000, 31999, 3], np.int32)
        ops.qk_rope_pos(dx, L, Hh, D, dev(pos), theta)
    else:
        pos = 300 + np.arange(L)
        ops.qk_rope(dx, L, Hh, D, 300, theta)
    close(host(dx, np.float16, x.shape), M.rope(x, pos, D, theta))


def test_argmax_rows_and_ties():
    say("model ops: argmax")
    V = 151936
    lg = np.random.default_rng(7).standard_normal((3, V)).astype(np.float32)
    lg[1, 5] = lg[1, 150000] = 100.0          # tie: the first index wins
    lg[2, V - 1] = 50.0
    out = DeviceBuffer(3 * 4)
    ops.qk_argmax(dev(lg), 3, V, out)
    np.testing.assert_array_equal(host(out, np.int32, (3,)), M.argmax(lg))


@pytest.mark.parametrize("M_,N,K,odt", [(1, 896, 896, KVC_F16), (37, 128, 896, KVC_F16), (5, 4864, 896, KVC_F16),
                                        (16, 896, 4864, KVC_F16), (3, 2000, 896, KVC_F32)])
def test_linear(M_, N, K, odt):
    say(f"model ops: linear {M_}x{N}x{K} out={odt}")
    x, w = normal((M_, K), 220, np.float16), (0.02 * normal((N, K), 221)).astype(np.float16)
    nt = np.float16 if odt == KVC_F16 else np.float32
    y = DeviceBuffer(M_ * N * np.dtype(nt).itemsize)
    ops.linear(y, dev(x), dev(w), M_, N, K, out_dtype=odt)
    ref = M.linear(x, w)
    got = host(y, nt, (M_, N)).astype(np.float64)
    assert np.abs(got - ref).max() <= 2e-3 * max(1.0, np.abs(ref).max())
