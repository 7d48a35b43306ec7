"""The attention oracle (oracle/attention.py, imported as `attention`) pinned by closed forms, so that a
dropped bias, a flipped rel-shift or a wrong window bound fails here."""
import numpy as np
import pytest
from scipy.special import softmax

from attention import relpos_attention, window


def rnd(seed, *shape, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


def test_reduces_to_textbook_attention():
    """rk = 0 and bias_u = 0: plain multi-head softmax(q k^T / sqrt(dk)) v."""
    T, d, H = 11, 32, 4
    dk = d // H
    q, k, v = rnd(1, T, d), rnd(2, T, d), rnd(3, T, d)
    bv = rnd(4, d)  # bias_v only meets rk, which is zero
    ctx = relpos_attention(q, k, v, np.zeros((2 * T - 1, d)), np.zeros(d), bv, H)
    for h in range(H):
        sl = slice(h * dk, (h + 1) * dk)
        p = softmax(np.einsum("ti,ji->tj", q[:, sl], k[:, sl]) / np.sqrt(dk), axis=1)
        np.testing.assert_allclose(ctx[:, sl], p @ v[:, sl], rtol=1e-12, atol=1e-12)


def test_bias_u_shifts_every_query():
    """bias_u enters as q + bias_u in the content term (encoder.c:358-363)."""
    T, d, H = 7, 16, 2
    q, k, v = rnd(5, T, d), rnd(6, T, d), rnd(7, T, d)
    bu = rnd(8, d)
    a = relpos_attention(q, k, v, np.zeros((2 * T - 1, d)), bu, np.zeros(d), H)
    b = relpos_attention(q + bu, k, v, np.zeros((2 * T - 1, d)), np.zeros(d), np.zeros(d), H)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("delta", [-3, 0, 2])
def test_rel_shift_points_at_t_plus_delta(delta):
    """With k = 0 the scores come from bd only. Put all weight on position
    p* = T-1+delta: row t must attend to key j = t + delta (bd[t, T-1+j-t])."""
    T, H = 9, 1
    d = 16
    u = np.zeros(d)
    u[0] = 1.0
    rk = np.zeros((2 * T - 1, d))
    rk[T - 1 + delta, 0] = 60.0
    q = np.tile(u, (T, 1))
    v = np.zeros((T, d))
    v[np.arange(T), np.arange(T)] = 1.0          # v[j] = e_j
    ctx = relpos_attention(q, np.zeros((T, d)), v, rk, np.zeros(d), np.zeros(d), H)
    for t in range(T):
        j = t + delta
        if 0 <= j < T:
            assert ctx[t, j] > 0.999, (t, ctx[t, :T])


def test_window_bounds():
    """encoder.c:373-381: chunk = right + 1, row t sees [(tc-lc)*chunk, (tc+1)*chunk)."""
    j0, j1 = window(10, left=4, right=3)        # chunk 4, lc 1
    assert list(j0) == [0, 0, 0, 0, 0, 0, 0, 0, 4, 4]
    assert list(j1) == [4, 4, 4, 4, 8, 8, 8, 8, 10, 10]
    j0, j1 = window(5, left=-1, right=0)
    assert list(j0) == [0] * 5 and list(j1) == [5] * 5


def test_window_excludes_outside_keys():
    """A row's context depends on v only inside its window."""
    T, d, H = 12, 16, 2
    q, k, v, rk = rnd(9, T, d), rnd(10, T, d), rnd(11, T, d), rnd(12, 2 * T - 1, d)
    bu, bv = rnd(13, d), rnd(14, d)
    a = relpos_attention(q, k, v, rk, bu, bv, H, left=4, right=1)
    j0, j1 = window(T, 4, 1)
    t = 7
    v2 = v.copy()
    v2[: j0[t]] += 5.0
    v2[j1[t]:] += 5.0
    b = relpos_attention(q, k, v2, rk, bu, bv, H, left=4, right=1)
    np.testing.assert_array_equal(a[t], b[t])
    v3 = v.copy()
    v3[j0[t]] += 5.0
    c = relpos_attention(q, k, v3, rk, bu, bv, H, left=4, right=1)
    assert not np.allclose(a[t], c[t])
