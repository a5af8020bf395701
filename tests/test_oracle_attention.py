"""Pins the CPU attention oracle (oracle/oracle.cpp) independently of its own text.

Each check is chosen so a plausible mistake fails it:
  * L = 1 gives V[0]                        -> wrong V row / length
  * q = 0 gives mean(V[:L])                 -> off-by-one length, wrong row range
  * two-token logistic closed form          -> wrong scale (1/D vs 1/sqrt(D)), sign of the score
  * joint K/V row permutation invariance    -> K and V indexed differently
  * score shift invariance at |shift| = 1e4 -> missing max subtraction (overflow)
  * linearity in V                          -> dropped / duplicated term
  * GQA == MHA with repeated KV heads       -> h % Hkv instead of h / (Hq/Hkv)
  * paged with shuffled table == contiguous -> wrong pool offset ((phys*H+h)*B+in)*D
  * scipy.special.softmax @ V               -> an independent library evaluation
  * split-K (flash) == two-pass for ns in {1,4,7,16,128}, including empty splits
"""
import numpy as np
import pytest
from scipy.special import expit, softmax

from kvcache_amd import workloads as W


def rng(seed=0):
    return np.random.default_rng(seed)


def contig(orc, q, K, V, L, scale):
    """q [H,D], K/V [H,S,D] single sequence through the batched contiguous oracle."""
    return orc.batched_contig(q[None], K[None], V[None], np.array([L], np.int32), scale)[0]


def test_single_token_returns_v0(orc):
    r = rng(1)
    q, K, V = r.standard_normal((4, 64)), r.standard_normal((4, 8, 64)), r.standard_normal((4, 8, 64))
    out = contig(orc, q, K, V, 1, 0.125)
    np.testing.assert_array_equal(out, V[:, 0].astype(np.float32).astype(np.float64))


def test_zero_query_gives_mean(orc):
    r = rng(2)
    K, V = r.standard_normal((3, 37, 32)), r.standard_normal((3, 37, 32))
    q = np.zeros((3, 32))
    for L in (1, 5, 36, 37):
        out = contig(orc, q, K, V, L, 0.2)
        ref = V[:, :L].astype(np.float32).astype(np.float64).mean(axis=1)
        np.testing.assert_allclose(out, ref, rtol=0, atol=1e-12)


def test_two_token_logistic_closed_form(orc):
    r = rng(3)
    D = 64
    scale = 1.0 / np.sqrt(D)
    q = r.standard_normal((2, D)).astype(np.float32)
    K = r.standard_normal((2, 2, D)).astype(np.float32)
    V = r.standard_normal((2, 2, D)).astype(np.float32)
    out = contig(orc, q, K, V, 2, scale)
    for h in range(2):
        s0 = float(np.dot(q[h].astype(np.float64), K[h, 0].astype(np.float64))) * scale
        s1 = float(np.dot(q[h].astype(np.float64), K[h, 1].astype(np.float64))) * scale
        w0 = expit(s0 - s1)
        ref = w0 * V[h, 0] + (1 - w0) * V[h, 1]
        np.testing.assert_allclose(out[h], ref, rtol=0, atol=1e-12)


def test_permutation_invariance(orc):
    r = rng(4)
    q, K, V = r.standard_normal((2, 64)), r.standard_normal((2, 50, 64)), r.standard_normal((2, 50, 64))
    perm = r.permutation(50)
    a = contig(orc, q, K, V, 50, 0.125)
    b = contig(orc, q, K[:, perm], V[:, perm], 50, 0.125)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)


def test_shift_invariance_large_scores(orc):
    r = rng(5)
    D = 16
    q = r.standard_normal((1, D)).astype(np.float32)
    q[0, 0] = 1.0
    K = (np.round(r.standard_normal((1, 20, D)) * 8) / 8).astype(np.float32)  # multiples of 1/8: k + 1e4 exact in fp32
    V = r.standard_normal((1, 20, D))
    shifted = K.copy()
    shifted[..., 0] += 1e4  # every score += exactly 1e4: exp would overflow without max-subtraction
    a = contig(orc, q, K, V, 20, 1.0)
    b = contig(orc, q, shifted, V, 20, 1.0)
    assert np.all(np.isfinite(b))
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-9)


def test_linearity_in_v(orc):
    r = rng(6)
    q, K = r.standard_normal((2, 32)), r.standard_normal((2, 30, 32))
    V1 = r.standard_normal((2, 30, 32)).astype(np.float32)
    V2 = r.standard_normal((2, 30, 32)).astype(np.float32)
    a = contig(orc, q, K, V1, 30, 0.3) + contig(orc, q, K, V2, 30, 0.3)
    b = contig(orc, q, K, (V1.astype(np.float64) + V2).astype(np.float32), 30, 0.3)
    np.testing.assert_allclose(a, b, rtol=0, atol=2e-6)  # V1+V2 rounded to fp32


def test_scipy_softmax_agreement(orc):
    r = rng(7)
    H, S, D = 8, 128, 64
    q = r.standard_normal((H, D)).astype(np.float32)
    K = r.standard_normal((H, S, D)).astype(np.float32)
    V = r.standard_normal((H, S, D)).astype(np.float32)
    scale = 1 / np.sqrt(D)
    out = contig(orc, q, K, V, S, scale)
    p = softmax(np.matmul(K.astype(np.float64), q.astype(np.float64)[:, :, None])[:, :, 0] * scale, axis=-1)
    ref = np.matmul(p[:, None, :], V.astype(np.float64))[:, 0]
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-12)


def test_gqa_equals_repeated_mha(orc):
    r = rng(8)
    N, Hq, Hkv, S, D = 3, 8, 2, 40, 64
    q = r.standard_normal((N, Hq, D)).astype(np.float32)
    K = r.standard_normal((N, Hkv, S, D)).astype(np.float32)
    V = r.standard_normal((N, Hkv, S, D)).astype(np.float32)
    lens = np.array([40, 17, 1], np.int32)
    g = orc.batched_contig(q, K, V, lens, 0.125)
    m = orc.batched_contig(q, np.repeat(K, Hq // Hkv, axis=1), np.repeat(V, Hq // Hkv, axis=1), lens, 0.125)
    np.testing.assert_array_equal(g, m)
    # and the map really is h -> h // (Hq/Hkv): a wrong map would pair q-head 1 with KV head 1
    wrong = orc.batched_contig(q, np.tile(K, (1, Hq // Hkv, 1, 1)), np.tile(V, (1, Hq // Hkv, 1, 1)), lens, 0.125)
    assert not np.allclose(g, wrong)


def test_paged_shuffled_equals_contiguous(orc, tmp_path):
    r = rng(9)
    N, H, D, B = 4, 8, 64, 16
    lens = np.array([1, 16, 17, 100], np.int32)
    S = int(lens.max())
    q = r.standard_normal((N, H, D)).astype(np.float32)
    K = r.standard_normal((N, H, S, D)).astype(np.float32)
    V = r.standard_normal((N, H, S, D)).astype(np.float32)
    nb = [(int(L) + B - 1) // B for L in lens]
    perm = W.shuffle_perm(sum(nb), 42)
    kp = np.zeros((sum(nb), H, B, D), np.float32)
    vp = np.zeros_like(kp)
    tab_off = np.concatenate([[0], np.cumsum(nb)]).astype(np.int32)
    table = perm.copy()
    for s in range(N):
        for pos in range(lens[s]):
            phys = table[tab_off[s] + pos // B]
            kp[phys, :, pos % B] = K[s, :, pos]
            vp[phys, :, pos % B] = V[s, :, pos]
    a = orc.batched_paged(q, kp, vp, table, tab_off, lens, H, B, 0.125)
    b = orc.batched_contig(q, K, V, lens, 0.125)
    np.testing.assert_array_equal(a, b)


def test_zero_length_gives_zero(orc):
    q = np.ones((1, 2, 32), np.float32)
    K = np.ones((1, 2, 4, 32), np.float32)
    out = orc.batched_contig(q, K, K, np.array([0], np.int32), 1.0)
    assert np.all(out == 0)


@pytest.mark.parametrize("ns", [1, 4, 7, 16, 128])
def test_flash_split_matches_two_pass(orc, ns):
    # main_flash.cu:36 split set; 7 does not divide 128, 128 = one token per split
    r = rng(10)
    H, S, D = 8, 128, 64
    q = r.standard_normal((H, D)).astype(np.float32)
    K = r.standard_normal((H, S, D)).astype(np.float32)
    V = r.standard_normal((H, S, D)).astype(np.float32)
    scale = 1 / np.sqrt(D)
    a = orc.flash_decode(q, K, V, S, scale, ns)
    b = contig(orc, q, K, V, S, scale)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)


def test_flash_empty_splits(orc):
    # L = 10, ns = 6 -> chunk 2, split 5 covers [10, 12) and is empty (flash_decode.cu:30-32)
    r = rng(11)
    H, S, D = 2, 10, 32
    q = r.standard_normal((H, D)).astype(np.float32)
    K = r.standard_normal((H, S, D)).astype(np.float32)
    V = r.standard_normal((H, S, D)).astype(np.float32)
    pa, pm, pl = orc.flash_split(q, K, V, 10, 0.5, 6)
    assert np.all(pl[:, 5] == 0) and np.all(pa[:, 5] == 0) and np.all(pm[:, 5] < -1e300)
    np.testing.assert_allclose(orc.flash_decode(q, K, V, 10, 0.5, 6), contig(orc, q, K, V, 10, 0.5), atol=1e-12)
    # num_splits is clamped to [1, L] (flash_decode.cu:106-107)
    np.testing.assert_allclose(orc.flash_decode(q, K, V, 10, 0.5, 50), contig(orc, q, K, V, 10, 0.5), atol=1e-12)


def test_fp16_inputs_decoded_exactly(orc):
    r = rng(12)
    q = r.standard_normal((2, 3, 64)).astype(np.float16)
    K = r.standard_normal((2, 1, 20, 64)).astype(np.float16)
    V = r.standard_normal((2, 1, 20, 64)).astype(np.float16)
    lens = np.array([20, 7], np.int32)
    a = orc.batched_contig(q, K, V, lens, 0.125)
    b = orc.batched_contig(q.astype(np.float32), K.astype(np.float32), V.astype(np.float32), lens, 0.125)
    np.testing.assert_array_equal(a, b)


# ---- prompt (prefill) attention: qwen_kernels.cu:146-181 ------------------------------
def _scatter(K, V, block, perm):
    """K/V [Hkv, S, D] of one sequence into a pool through table perm."""
    Hkv, S, D = K.shape
    nb = (S + block - 1) // block
    NB = int(perm[:nb].max()) + 1
    kp = np.zeros((NB, Hkv, block, D))
    vp = np.zeros_like(kp)
    for b in range(nb):
        t0, t1 = b * block, min(S, (b + 1) * block)
        kp[perm[b], :, : t1 - t0] = K[:, t0:t1]
        vp[perm[b], :, : t1 - t0] = V[:, t0:t1]
    return kp, vp, perm[:nb].astype(np.int32)


@pytest.mark.parametrize("base,n", [(0, 1), (0, 23), (40, 9)])
def test_paged_causal_against_masked_softmax(orc, base, n):
    """The causal restatement against a masked score matrix (-inf above the
    diagonal, row softmax): a different formulation of the same attention."""
    rng = np.random.default_rng(base + n)
    Hq, Hkv, D, B = 6, 2, 16, 4
    S = base + n
    # fp32 inputs (the restatement's storage type), compared in double
    q = rng.standard_normal((n, Hq, D)).astype(np.float32)
    K, V = rng.standard_normal((Hkv, S, D)).astype(np.float32), rng.standard_normal((Hkv, S, D)).astype(np.float32)
    kp, vp, table = _scatter(K, V, B, rng.permutation(64))
    kp, vp = kp.astype(np.float32), vp.astype(np.float32)
    q64, K, V = q.astype(np.float64), K.astype(np.float64), V.astype(np.float64)
    scale = 1 / np.sqrt(D)
    got = orc.paged_causal(q, kp, vp, table, base, Hkv, B, scale)
    g = Hq // Hkv
    for h in range(Hq):
        sc = q64[:, h] @ K[h // g].T * scale                     # [n, S]
        mask = np.arange(S)[None, :] > (base + np.arange(n))[:, None]
        sc[mask] = -np.inf
        want = softmax(sc, axis=1) @ V[h // g]
        np.testing.assert_allclose(got[:, h], want, rtol=1e-12, atol=1e-12)
    if base == 0:
        np.testing.assert_allclose(got[0], np.repeat(V[:, 0], g, axis=0), rtol=0, atol=0)  # first query sees only key 0
