"""Decode-step linear layers over at most 32 rows (fused matrix-core kernels) on the
GPU, checked against the CPU restatement (oracle/model.py) with the op-by-op
rounding points (fp16 GEMM result, then bias / residual / activation), and against
the op-by-op GPU path (rmsnorm + rocBLAS linear + elementwise kernels), which they
replace in the decode step (qwen_serve.cu:127-175)."""
import numpy as np
import pytest

from kvcache_amd import KVC_F16, KVC_F32, ops
from kvcache_amd.device import DeviceBuffer
from oracle import model as M
from oracle.model import _r16

from _helpers import dev, host, normal, say

pytestmark = pytest.mark.gpu
EPS = 1e-6


def close(got, ref, rel=4e-3):
    got = np.asarray(got, np.float64)
    err = np.abs(got - ref) - rel * np.maximum(1.0, np.abs(ref))
    assert np.all(err <= 0), (np.abs(got - ref).max(), np.unravel_index(np.argmax(err), err.shape))


def workspace(N, K):
    ws = DeviceBuffer(max(ops.rows_workspace_size(N, K), 1 << 20))
    ws.zero()
    return ws


def inputs(M_, K, seed):
    x = normal((M_, K), seed, np.float16)
    nw = (1 + 0.1 * normal((K,), seed + 1)).astype(np.float16)
    return x, nw


@pytest.mark.parametrize("M_", [1, 5, 16, 17, 32])
@pytest.mark.parametrize("norm", [False, True])
def test_rows_linear_store(M_, norm):
    say(f"rows linear store M={M_} norm={norm}")
    N, K = 896, 896
    x, nw = inputs(M_, K, 300 + M_)
    w = (0.03 * normal((N, K), 302)).astype(np.float16)
    y = DeviceBuffer(M_ * N * 2)
    ops.rows_linear(y, dev(x), dev(w), M_, N, K, norm_w=dev(nw) if norm else None, eps=EPS,
                    workspace=workspace(N, K))
    a = _r16(M.rmsnorm(x, nw, EPS)) if norm else x.astype(np.float32)
    ref = M.linear(a, w)
    close(host(y, np.float16, (M_, N)), ref)


@pytest.mark.parametrize("M_,K", [(3, 32), (32, 96), (17, 160), (32, 1024)])
@pytest.mark.parametrize("norm", [False, True])
def test_rows_linear_short_k(M_, K, norm):
    # K of 1, 3, 5 and 32 k steps: the whole-line loads read k steps in pairs, so a
    # wave whose range ends inside a pair masks the pair's second half
    say(f"rows linear store M={M_} K={K} norm={norm}")
    N = 64
    x, nw = inputs(M_, K, 320 + K)
    w = (0.1 * normal((N, K), 321)).astype(np.float16)
    y = DeviceBuffer(M_ * N * 2)
    ops.rows_linear(y, dev(x), dev(w), M_, N, K, norm_w=dev(nw) if norm else None, eps=EPS,
                    workspace=workspace(N, K))
    a = _r16(M.rmsnorm(x, nw, EPS)) if norm else x.astype(np.float32)
    close(host(y, np.float16, (M_, N)), M.linear(a, w))


@pytest.mark.parametrize("M_,K,splits", [(32, 896, -1), (7, 896, 1), (32, 4864, -1), (20, 4864, 7), (3, 4864, 40),
                                         (16, 4864, 5)])
def test_rows_linear_residual_splits(M_, K, splits):
    say(f"rows linear residual M={M_} K={K} splits={splits}")
    N = 896
    a = normal((M_, K), 310, np.float16)
    w = (0.03 * normal((N, K), 311)).astype(np.float16)
    x0 = normal((M_, N), 312, np.float16)
    ops.rows_set_tuning(splits=splits)  # before sizing: the workspace holds one partial per split
    try:
        ws = workspace(N, K)
        outs = []
        for _ in range(2):  # deterministic: the split partials are summed in a fixed order
            x = dev(x0)
            ops.rows_linear(x, dev(a), dev(w), M_, N, K, residual=True, workspace=ws)
            outs.append(host(x, np.float16, (M_, N)))
    finally:
        ops.rows_set_tuning()
    np.testing.assert_array_equal(outs[0], outs[1])
    ref = x0.astype(np.float64) + _r16(M.linear(a, w))
    close(outs[0], ref)
    # the op-by-op GPU path: rocBLAS linear, then the residual kernel
    y = DeviceBuffer(M_ * N * 2)
    ops.linear(y, dev(a), dev(w), M_, N, K)
    x = dev(x0)
    ops.qk_add_residual(x, y, M_ * N)
    d = np.abs(outs[0].astype(np.float64) - host(x, np.float16, (M_, N)))
    assert d.max() <= 4e-3 * max(1.0, np.abs(ref).max()), d.max()


@pytest.mark.parametrize("M_", [1, 9, 32])
def test_rows_qkv_rope(M_):
    say(f"rows qkv M={M_}")
    H, Hq, Hkv, D, theta = 896, 14, 2, 64, 1e6
    QD, KD = Hq * D, Hkv * D
    x, nw = inputs(M_, H, 320)
    w = (0.03 * normal((QD + 2 * KD, H), 322)).astype(np.float16)
    b = (0.5 * normal((QD + 2 * KD,), 323)).astype(np.float16)
    pos = np.random.default_rng(324).integers(0, 40000, M_).astype(np.int32)
    q, k, v = DeviceBuffer(M_ * QD * 2), DeviceBuffer(M_ * KD * 2), DeviceBuffer(M_ * KD * 2)
    ops.rows_qkv(q, k, v, dev(x), dev(w), dev(b), dev(pos), M_, H, Hq, Hkv, D, theta, norm_w=dev(nw), eps=EPS)
    n = _r16(M.rmsnorm(x, nw, EPS))
    y = _r16(_r16(M.linear(n, w)) + b.astype(np.float32))
    rq = M.rope(y[:, :QD].reshape(M_, Hq, D), pos, D, theta).reshape(M_, QD)
    rk = M.rope(y[:, QD:QD + KD].reshape(M_, Hkv, D), pos, D, theta).reshape(M_, KD)
    close(host(q, np.float16, (M_, QD)), rq)
    close(host(k, np.float16, (M_, KD)), rk)
    close(host(v, np.float16, (M_, KD)), y[:, QD + KD:])


@pytest.mark.parametrize("M_", [1, 12, 32])
def test_rows_swiglu(M_):
    say(f"rows swiglu M={M_}")
    H, I = 896, 4864
    x, nw = inputs(M_, H, 330)
    wgu = (0.03 * normal((2 * I, H), 332)).astype(np.float16)
    act = DeviceBuffer(M_ * I * 2)
    ops.rows_swiglu(act, dev(x), dev(wgu), M_, I, H, norm_w=dev(nw), eps=EPS)
    n = _r16(M.rmsnorm(x, nw, EPS))
    ref = M.silu_mul(_r16(M.linear(n, wgu[:I])), _r16(M.linear(n, wgu[I:])))
    close(host(act, np.float16, (M_, I)), ref)


@pytest.mark.parametrize("M_,V", [(1, 151936), (32, 151936), (19, 4096)])
def test_rows_lm_head(M_, V):
    say(f"rows lm_head M={M_} V={V}")
    H = 896
    x, nw = inputs(M_, H, 340)
    w = (0.03 * normal((V, H), 342)).astype(np.float16)
    w[V - 1] = w[5]  # identical rows: equal logits, the first index must win
    ws = workspace(V, H)
    logits, tok = DeviceBuffer(M_ * V * 4), DeviceBuffer(M_ * 4)
    ops.rows_lm_head(logits, tok, dev(x), dev(w), M_, V, H, norm_w=dev(nw), eps=EPS, workspace=ws)
    lg = host(logits, np.float32, (M_, V))
    ref = M.linear(_r16(M.rmsnorm(x, nw, EPS)), w)
    close(lg, ref)
    t = host(tok, np.int32, (M_,))
    np.testing.assert_array_equal(t, np.argmax(lg, axis=1))
    # without the logits buffer the tokens are the same
    tok2 = DeviceBuffer(M_ * 4)
    ops.rows_lm_head(None, tok2, dev(x), dev(w), M_, V, H, norm_w=dev(nw), eps=EPS, workspace=ws)
    np.testing.assert_array_equal(host(tok2, np.int32, (M_,)), t)


def test_rows_rejects_bad_shapes():
    say("rows: argument errors")
    from kvcache_amd import KvcError
    ws = workspace(896, 896)
    x, w, y = DeviceBuffer(64 * 896 * 2), DeviceBuffer(896 * 896 * 2), DeviceBuffer(64 * 896 * 2)
    for M_, N, K in [(0, 896, 896), (33, 896, 896), (4, 900, 896), (4, 896, 900)]:
        with pytest.raises(KvcError):
            ops.rows_linear(y, x, w, M_, N, K, workspace=ws)
    with pytest.raises(KvcError):
        ops.rows_linear(x, x, w, 4, 896, 896)  # y aliases x
    with pytest.raises(KvcError):  # split layer without a workspace
        ops.rows_linear(y, x, DeviceBuffer(896 * 4864 * 2), 4, 896, 4864, residual=True)


@pytest.mark.parametrize("n", [1, 7, 16, 17, 31])
def test_rows_dev_rows_equal_plain_calls(n):
    """The graph-safe form (row count read from device memory, M = 32 as capacity)
    gives bit for bit the plain call's rows and leaves the rows past the count
    untouched."""
    say(f"rows dev_rows n={n}")
    cap, H, I, QD, KD, V = 32, 896, 4864, 896, 128, 4096
    rng = np.random.default_rng(350 + n)
    x = rng.standard_normal((cap, H)).astype(np.float16)
    a = rng.standard_normal((cap, I)).astype(np.float16)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
    w = (0.03 * rng.standard_normal((H, H))).astype(np.float16)
    wd = (0.03 * rng.standard_normal((H, I))).astype(np.float16)
    wqkv = (0.03 * rng.standard_normal((QD + 2 * KD, H))).astype(np.float16)
    bqkv = (0.5 * rng.standard_normal(QD + 2 * KD)).astype(np.float16)
    wgu = (0.03 * rng.standard_normal((2 * I, H))).astype(np.float16)
    wl = (0.03 * rng.standard_normal((V, H))).astype(np.float16)
    pos = rng.integers(0, 3000, cap).astype(np.int32)
    dn = dev(np.array([n], np.int32))
    ws = workspace(V, I)
    sentinel = np.float16(7.25)

    def both(shape, dtype, call):
        """call(out, M, dev_rows) on a sentinel-filled buffer; returns (plain, graph-safe)."""
        outs = []
        for M_, d in ((n, None), (cap, dn)):
            buf = dev(np.full(shape, sentinel, dtype))
            call(buf, M_, d)
            outs.append(host(buf, dtype, shape))
        return outs

    p_, g_ = both((cap, H), np.float16, lambda o, M_, d: ops.rows_linear(
        o, dev(x), dev(w), M_, H, H, norm_w=dev(nw), eps=EPS, dev_rows=d, workspace=ws))
    np.testing.assert_array_equal(g_[:n], p_[:n]); assert np.all(g_[n:] == sentinel)
    # residual into x, K split across workgroups
    p_, g_ = [], []
    for M_, d in ((n, None), (cap, dn)):
        xb = dev(x)
        ops.rows_linear(xb, dev(a), dev(wd), M_, H, I, residual=True, dev_rows=d, workspace=ws)
        (p_ if d is None else g_).append(host(xb, np.float16, (cap, H)))
    np.testing.assert_array_equal(g_[0][:n], p_[0][:n]); np.testing.assert_array_equal(g_[0][n:], x[n:])
    # q|k|v + rotary
    res = []
    for M_, d in ((n, None), (cap, dn)):
        q, k, v = (dev(np.full((cap, c), sentinel, np.float16)) for c in (QD, KD, KD))
        ops.rows_qkv(q, k, v, dev(x), dev(wqkv), dev(bqkv), dev(pos), M_, H, 14, 2, 64, 1e6, norm_w=dev(nw),
                     eps=EPS, dev_rows=d)
        res.append([host(t, np.float16, (cap, c)) for t, c in ((q, QD), (k, KD), (v, KD))])
    for pt, gt in zip(*res):
        np.testing.assert_array_equal(gt[:n], pt[:n]); assert np.all(gt[n:] == sentinel)
    p_, g_ = both((cap, I), np.float16, lambda o, M_, d: ops.rows_swiglu(
        o, dev(x), dev(wgu), M_, I, H, norm_w=dev(nw), eps=EPS, dev_rows=d))
    np.testing.assert_array_equal(g_[:n], p_[:n]); assert np.all(g_[n:] == sentinel)
    p_, g_ = both((cap,), np.int32, lambda o, M_, d: ops.rows_lm_head(
        None, o, dev(x), dev(wl), M_, V, H, norm_w=dev(nw), eps=EPS, dev_rows=d, workspace=ws))
    np.testing.assert_array_equal(g_[:n], p_[:n])


# ---- layer chain (kvc_rows_chain): the linear layers between two attention launches as
# one launch with grid barriers; must equal the separate launches bit for bit ----------
H_, HQ, HKV, D_, I_ = 896, 14, 2, 64, 4864
QD, KD = HQ * D_, HKV * D_


def chain_weights(seed):
    w = {
        "w_o": (0.03 * normal((H_, QD), seed)).astype(np.float16),
        "ln2": (1 + 0.1 * normal((H_,), seed + 1)).astype(np.float16),
        "w_gate_up": (0.03 * normal((2 * I_, H_), seed + 2)).astype(np.float16),
        "w_down": (0.015 * normal((H_, I_), seed + 3)).astype(np.float16),
        "ln1": (1 + 0.1 * normal((H_,), seed + 4)).astype(np.float16),
        "w_qkv": (0.03 * normal((QD + 2 * KD, H_), seed + 5)).astype(np.float16),
        "b_qkv": (0.1 * normal((QD + 2 * KD,), seed + 6)).astype(np.float16),
    }
    return {k: dev(v) for k, v in w.items()}


def chain_separate(W, x, att, pos, M_, tail, head, rws):
    """The same layers as the separate fused launches (kvc_rows_linear / swiglu / qkv)."""
    act = DeviceBuffer(M_ * I_ * 2)
    q, k, v = DeviceBuffer(M_ * QD * 2), DeviceBuffer(M_ * KD * 2), DeviceBuffer(M_ * KD * 2)
    if tail:
        ops.rows_linear(x, att, W["w_o"], M_, H_, QD, residual=True, workspace=rws)
        ops.rows_swiglu(act, x, W["w_gate_up"], M_, I_, H_, norm_w=W["ln2"], eps=EPS)
        ops.rows_linear(x, act, W["w_down"], M_, H_, I_, residual=True, workspace=rws)
    if head:
        ops.rows_qkv(q, k, v, x, W["w_qkv"], W["b_qkv"], pos, M_, H_, HQ, HKV, D_, 1e6, norm_w=W["ln1"], eps=EPS)
    return act, q, k, v


def chain_run(W, x, att, pos, M_, tail, head, cws):
    act = DeviceBuffer(M_ * I_ * 2)
    q, k, v = DeviceBuffer(M_ * QD * 2), DeviceBuffer(M_ * KD * 2), DeviceBuffer(M_ * KD * 2)
    t = dict(att=att, w_o=W["w_o"], ln2=W["ln2"], w_gate_up=W["w_gate_up"], act=act, w_down=W["w_down"]) if tail else None
    h = dict(q=q, k=k, v=v, ln1=W["ln1"], w_qkv=W["w_qkv"], b_qkv=W["b_qkv"], pos=pos) if head else None
    rc = ops.rows_chain(x, M_, H_, HQ, HKV, D_, I_, eps=EPS, theta=1e6, tail=t, head=h, workspace=cws)
    return rc, act, q, k, v


def chain_workspace():
    cws = DeviceBuffer(ops.rows_chain_workspace_size(H_, I_))
    cws.zero()
    return cws


def test_chain_workspace_size():
    assert ops.rows_chain_workspace_size(H_, I_) > ops.rows_workspace_size(H_, I_)
    assert ops.rows_chain_workspace_size(H_, 100) == 0 and ops.rows_chain_workspace_size(0, I_) == 0


@pytest.mark.parametrize("parts", ["tail+head", "tail", "head"])
def test_chain_equals_separate_launches(parts):
    """Several calls in a row on one workspace (the barrier counters carry over), rows
    from 32 down to 1 (one and two 16-row tiles), each bit-exact with the separate
    launches on the same inputs."""
    from kvcache_amd._native import KVC_OK
    tail, head = "tail" in parts, "head" in parts
    W = chain_weights(700)
    rws = workspace(H_, I_)
    cws = chain_workspace()
    for M_ in (32, 17, 16, 5, 1, 32):
        say(f"layer chain {parts} M={M_}")
        x0 = normal((M_, H_), 710 + M_, np.float16)
        att = dev(normal((M_, QD), 720 + M_, np.float16))
        pos = dev(np.random.default_rng(730 + M_).integers(0, 4000, M_).astype(np.int32))
        xa, xb = dev(x0), dev(x0)
        ra = chain_separate(W, xa, att, pos, M_, tail, head, rws)
        rc, *rb = chain_run(W, xb, att, pos, M_, tail, head, cws)
        assert rc == KVC_OK
        assert np.array_equal(host(xa, np.uint16, (M_, H_)), host(xb, np.uint16, (M_, H_)))
        if tail:
            assert np.array_equal(host(ra[0], np.uint16, (M_, I_)), host(rb[0], np.uint16, (M_, I_)))
        if head:
            for a, b, n in zip(ra[1:], rb[1:], (QD, KD, KD)):
                assert np.array_equal(host(a, np.uint16, (M_, n)), host(b, np.uint16, (M_, n)))
    ops.check_device_errors()


def test_chain_against_oracle():
    """One tail + head at 9 rows against the CPU restatement with the op-by-op rounding
    points (the separate launches are pinned the same way elsewhere)."""
    from kvcache_amd._native import KVC_OK
    M_ = 9
    rng = np.random.default_rng(750)
    hw = {
        "w_o": (0.03 * normal((H_, QD), 751)).astype(np.float16),
        "ln2": (1 + 0.1 * normal((H_,), 752)).astype(np.float16),
        "w_gate_up": (0.03 * normal((2 * I_, H_), 753)).astype(np.float16),
        "w_down": (0.015 * normal((H_, I_), 754)).astype(np.float16),
        "ln1": (1 + 0.1 * normal((H_,), 755)).astype(np.float16),
        "w_qkv": (0.03 * normal((QD + 2 * KD, H_), 756)).astype(np.float16),
        "b_qkv": (0.1 * normal((QD + 2 * KD,), 757)).astype(np.float16),
    }
    W = {k: dev(v) for k, v in hw.items()}
    x0 = normal((M_, H_), 758, np.float16)
    att0 = normal((M_, QD), 759, np.float16)
    pos0 = rng.integers(0, 4000, M_).astype(np.int32)
    x = dev(x0)
    rc, act, q, k, v = chain_run(W, x, dev(att0), dev(pos0), M_, True, True, chain_workspace())
    assert rc == KVC_OK
    # CPU: the op-by-op rounding points of the decode step
    xr = _r16(x0.astype(np.float32) + _r16(M.linear(att0.astype(np.float32), hw["w_o"])))
    n2 = _r16(M.rmsnorm(xr, hw["ln2"], EPS))
    g = _r16(M.linear(n2, hw["w_gate_up"][:I_]))
    u = _r16(M.linear(n2, hw["w_gate_up"][I_:]))
    actr = _r16(g / (1 + np.exp(-g)) * u)
    xr2 = _r16(xr + _r16(M.linear(actr, hw["w_down"])))
    close(host(act, np.float16, (M_, I_)), actr)
    close(host(x, np.float16, (M_, H_)), xr2, rel=8e-3)
    n1 = _r16(M.rmsnorm(xr2, hw["ln1"], EPS))
    qkv = _r16(_r16(M.linear(n1, hw["w_qkv"])) + hw["b_qkv"].astype(np.float32))
    vr = qkv[:, QD + KD:]
    close(host(v, np.float16, (M_, KD)), vr, rel=8e-3)


def test_chain_barrier_give_up_reports_error():
    """A barrier wait that gives up (forced from the host with a spin limit of 0 polls:
    every wait ends at once, every wave exits normally) is reported through the device
    error word: kvc_check_device_errors and the next chain call say KVC_ERR_STATE, the
    call clears the counters, and the chain then works again."""
    from kvcache_amd._native import KVC_ERR_STATE, KVC_OK, KvcError
    from _helpers import tuning
    W = chain_weights(760)
    M_ = 8
    x0 = normal((M_, H_), 761, np.float16)
    att = dev(normal((M_, QD), 762, np.float16))
    pos = dev(np.arange(M_, dtype=np.int32))
    cws = chain_workspace()
    say("layer chain with a zero spin limit")
    with tuning("chain_spin", 0):
        rc, *_ = chain_run(W, dev(x0), att, pos, M_, True, True, cws)
        assert rc == KVC_OK  # the launch itself is fine; its barrier gives up on the device
        with pytest.raises(KvcError) as e:
            ops.check_device_errors()
        assert e.value.status == KVC_ERR_STATE
        # the report was taken by check_device_errors; give up again and let the next
        # chain call find it
        rc, *_ = chain_run(W, dev(x0), att, pos, M_, True, True, cws)
        assert rc == KVC_OK
        from kvcache_amd.device import synchronize
        synchronize()
        rc, *_ = chain_run(W, dev(x0), att, pos, M_, True, True, cws)
        assert rc == KVC_ERR_STATE
    say("layer chain after the reset")
    rws = workspace(H_, I_)
    xa, xb = dev(x0), dev(x0)
    ra = chain_separate(W, xa, att, pos, M_, True, True, rws)
    rc, *rb = chain_run(W, xb, att, pos, M_, True, True, cws)
    assert rc == KVC_OK
    assert np.array_equal(host(xa, np.uint16, (M_, H_)), host(xb, np.uint16, (M_, H_)))
    assert np.array_equal(host(ra[1], np.uint16, (M_, QD)), host(rb[1], np.uint16, (M_, QD)))
    ops.check_device_errors()


def test_chain_other_shape_and_refusal():
    """The chain at another decoder shape (hidden 512, 8q/2kv, SwiGLU 1536, 13 rows) equals
    the separate launches bit for bit; a shape outside its kernel shapes (SwiGLU 8960:
    three column groups per workgroup in the gate|up layer) is refused with
    KVC_ERR_UNSUPPORTED before anything is launched, and the separate launches still run it."""
    from kvcache_amd._native import KVC_ERR_UNSUPPORTED, KVC_OK
    H, Hq, Hkv, D = 512, 8, 2, 64
    qd, kd = Hq * D, Hkv * D
    for I, M_, expect in ((1536, 13, KVC_OK), (8960, 9, KVC_ERR_UNSUPPORTED)):
        say(f"layer chain H={H} I={I} M={M_}")
        w = {
            "w_o": dev((0.03 * normal((H, qd), 800)).astype(np.float16)),
            "ln2": dev((1 + 0.1 * normal((H,), 801)).astype(np.float16)),
            "w_gate_up": dev((0.03 * normal((2 * I, H), 802)).astype(np.float16)),
            "w_down": dev((0.015 * normal((H, I), 803)).astype(np.float16)),
            "ln1": dev((1 + 0.1 * normal((H,), 804)).astype(np.float16)),
            "w_qkv": dev((0.03 * normal((qd + 2 * kd, H), 805)).astype(np.float16)),
            "b_qkv": dev((0.1 * normal((qd + 2 * kd,), 806)).astype(np.float16)),
        }
        x0 = normal((M_, H), 807, np.float16)
        att = dev(normal((M_, qd), 808, np.float16))
        pos = dev(np.arange(M_, dtype=np.int32) * 37)
        xa, xb = dev(x0), dev(x0)
        rws = DeviceBuffer(max(ops.rows_workspace_size(H, I), 1 << 20))
        rws.zero()
        acta, actb = DeviceBuffer(M_ * I * 2), DeviceBuffer(M_ * I * 2)
        qa, ka, va = DeviceBuffer(M_ * qd * 2), DeviceBuffer(M_ * kd * 2), DeviceBuffer(M_ * kd * 2)
        qb, kb, vb = DeviceBuffer(M_ * qd * 2), DeviceBuffer(M_ * kd * 2), DeviceBuffer(M_ * kd * 2)
        ops.rows_linear(xa, att, w["w_o"], M_, H, qd, residual=True, workspace=rws)
        ops.rows_swiglu(acta, xa, w["w_gate_up"], M_, I, H, norm_w=w["ln2"], eps=EPS)
        ops.rows_linear(xa, acta, w["w_down"], M_, H, I, residual=True, workspace=rws)
        ops.rows_qkv(qa, ka, va, xa, w["w_qkv"], w["b_qkv"], pos, M_, H, Hq, Hkv, D, 1e6, norm_w=w["ln1"], eps=EPS)
        cws = DeviceBuffer(ops.rows_chain_workspace_size(H, I))
        cws.zero()
        rc = ops.rows_chain(xb, M_, H, Hq, Hkv, D, I, eps=EPS, theta=1e6, workspace=cws,
                            tail=dict(att=att, w_o=w["w_o"], ln2=w["ln2"], w_gate_up=w["w_gate_up"], act=actb,
                                      w_down=w["w_down"]),
                            head=dict(q=qb, k=kb, v=vb, ln1=w["ln1"], w_qkv=w["w_qkv"], b_qkv=w["b_qkv"], pos=pos))
        assert rc == expect
        if expect != KVC_OK:
            assert np.array_equal(host(xb, np.uint16, (M_, H)), x0.view(np.uint16))  # nothing ran
            continue
        assert np.array_equal(host(xa, np.uint16, (M_, H)), host(xb, np.uint16, (M_, H)))
        assert np.array_equal(host(acta, np.uint16, (M_, I)), host(actb, np.uint16, (M_, I)))
        for a, b, n in ((qa, qb, qd), (ka, kb, kd), (va, vb, kd)):
            assert np.array_equal(host(a, np.uint16, (M_, n)), host(b, np.uint16, (M_, n)))
