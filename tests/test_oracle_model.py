"""The CPU restatement of the decoder-step operations (oracle/model.py), pinned by
properties the mathematics fixes rather than by retyping its formulas."""
import numpy as np

from oracle import model as M


def test_rope_properties():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 3, 8))
    np.testing.assert_allclose(M.rope(x, np.zeros(5), 8, 1e6), x, atol=0)          # position 0: identity
    y = M.rope(x, np.arange(5) * 7.0, 8, 1e6)
    n = lambda a: a[..., :4] ** 2 + a[..., 4:] ** 2                                  # each pair keeps its norm
    np.testing.assert_allclose(n(y), n(x), rtol=1e-12)
    a, b = np.arange(5) * 3.0, np.arange(5) * 11.0                                   # rotations compose additively
    np.testing.assert_allclose(M.rope(M.rope(x, a, 8, 1e4), b, 8, 1e4), M.rope(x, a + b, 8, 1e4), atol=1e-12)
    # pair 0 turns by exactly the position (frequency theta^0 = 1)
    e = np.zeros((1, 1, 8)); e[0, 0, 0] = 1.0
    r = M.rope(e, np.array([0.5]), 8, 1e6)
    np.testing.assert_allclose([r[0, 0, 0], r[0, 0, 4]], [np.cos(0.5), np.sin(0.5)], atol=1e-15)


def test_rmsnorm_silu_argmax_properties():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 16)) * 5
    y = M.rmsnorm(x, np.ones(16), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=1)), 1.0, rtol=1e-12)   # unit RMS
    np.testing.assert_allclose(M.rmsnorm(2 * x, np.ones(16), 0.0), y, rtol=1e-12)   # scale invariant
    assert M.silu_mul(np.array([0.0]), np.array([3.0]))[0] == 0.0
    np.testing.assert_allclose(M.silu_mul(np.array([40.0]), np.array([1.0])), [40.0], rtol=1e-15)
    assert M.argmax(np.array([[1.0, 3.0, 3.0, 2.0]]))[0] == 1                     # first of tied maxima
    assert (M.embed_gather(np.eye(3), [2, -1, 5]) == np.array([[0, 0, 1], [0, 0, 0], [0, 0, 0]])).all()
