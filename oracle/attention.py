"""attention.py — TEST INFRASTRUCTURE ONLY.

numpy restatement of the reference's relative-position self-attention core
(src/encoder.c): given the projected q, k, v (biases added), the projected
positions rk = pe . relk_w^T and the per-head biases bias_u, bias_v, it forms
per head h (dk = d / H, columns h*dk .. h*dk+dk-1):

    ac[t, j] = (q[t] + bias_u) . k[j]                      encoder.c:358-363
    bd[t, p] = (q[t] + bias_v) . rk[p],  p = 0 .. 2T-2     encoder.c:350-356
    s[t, j]  = (ac[t, j] + bd[t, T-1 + j - t]) / sqrt(dk)  encoder.c:383-386 (rel_shift in closed form)
    softmax over j in the row's window, ctx[t] = sum_j p[t, j] v[j]   :388-401

Window (encoder.c:373-381, 224-225, 287-292): left < 0 is full attention;
left >= 0 is chunked-limited with chunk = right + 1 and lc = left / chunk:
row t (chunk tc = t / chunk) sees keys [(tc - lc) * chunk, (tc + 1) * chunk)
clipped to [0, T). The banded path (encoder.c:220-313) computes the same
numbers block by block.

Computed in float64 (the reference's f32 arithmetic is checked against this
within the floating-point tolerance). Only tests/ and bench.py's checker
import this module.
"""
from __future__ import annotations

import numpy as np


def window(T: int, left: int, right: int):
    """Per-row key range [j0, j1) (encoder.c:373-381)."""
    t = np.arange(T)
    if left < 0:
        return np.zeros(T, np.int64), np.full(T, T, np.int64)
    chunk = right + 1
    lc = left // chunk
    tc = t // chunk
    j0 = np.maximum((tc - lc) * chunk, 0)
    j1 = np.minimum((tc + 1) * chunk, T)
    return j0, j1


def relpos_attention(q, k, v, rk, bias_u, bias_v, H: int, left: int = -1, right: int = 0):
    """ctx[T, d] (float64) — encoder.c:315-410 / 220-313."""
    q, k, v, rk = (np.asarray(a, np.float64) for a in (q, k, v, rk))
    bias_u, bias_v = np.asarray(bias_u, np.float64), np.asarray(bias_v, np.float64)
    T, d = q.shape
    dk = d // H
    assert rk.shape == (2 * T - 1, d)
    scaling = 1.0 / np.sqrt(float(np.float32(dk)))
    j0, j1 = window(T, left, right)
    tt = np.arange(T)[:, None]
    jj = np.arange(T)[None, :]
    shift = T - 1 + jj - tt                      # bd index of (t, j): 0 .. 2T-2
    mask = (jj >= j0[:, None]) & (jj < j1[:, None])
    ctx = np.zeros((T, d), np.float64)
    for h in range(H):
        sl = slice(h * dk, (h + 1) * dk)
        ac = (q[:, sl] + bias_u[sl]) @ k[:, sl].T
        bd = (q[:, sl] + bias_v[sl]) @ rk[:, sl].T
        s = (ac + np.take_along_axis(bd, shift, axis=1)) * scaling
        s = np.where(mask, s, -np.inf)
        s = s - s.max(axis=1, keepdims=True)
        e = np.where(mask, np.exp(s), 0.0)
        p = e / e.sum(axis=1, keepdims=True)
        ctx[:, sl] = p @ v[:, sl]
    return ctx
