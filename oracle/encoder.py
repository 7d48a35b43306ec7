"""encoder.py — TEST INFRASTRUCTURE ONLY.

numpy restatement, in float64, of one FastConformer encoder layer of the
reference (src/encoder.c), the checker of mynah_asr_hip_encoder_layer_dev:

    x += 0.5 * half_ffn(LN_ff1(x))                        encoder.c:492-494, 464-483
    x += attention(LN_att(x))                             :497-502, 315-410
    x += conv_module(LN_conv(x))                          :504-507, 413-462
    x += 0.5 * half_ffn(LN_ff2(x))                        :509-511
    x  = LN_out(x)                                        :513-515

Segments (the batched form, :901-946) share the products and layer norms;
attention and the depthwise conv run per segment. Weights are given as the
float64 values the products use (for quantized weights, the dequantized
values). Only tests/ and bench.py's checker import this module.
"""
from __future__ import annotations

import numpy as np

from attention import relpos_attention


def layer_norm(x, w, b):
    """encoder.c:25-37: mean and variance over the row, eps 1e-5."""
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + 1e-5) * w + b


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def silu(x):
    return x * sigmoid(x)


def linear(x, w, b=None):
    y = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    return y + b if b is not None else y


def half_ffn(x, p, which):
    """encoder.c:464-483: LN, linear1 (+b1), SiLU, linear2 (+b2)."""
    n = "ff2" if which else "ff1"
    h = silu(linear(layer_norm(x, p[f"ln_{n}_w"], p[f"ln_{n}_b"]), p[f"{n}_w1"], p.get(f"{n}_b1")))
    return linear(h, p[f"{n}_w2"], p.get(f"{n}_b2"))


def depthwise(g, w, bias, k, causal):
    """encoder.c:434-447 on one segment g [T, d]: out[t] = bias + sum over the
    taps j with 0 <= t - pc + j < T of w[:, j] * g[t - pc + j]."""
    T, d = g.shape
    pc = k - 1 if causal else (k - 1) // 2
    out = np.zeros((T, d), np.float64) + (bias if bias is not None else 0.0)
    for j in range(k):
        lo, hi = max(0, pc - j), min(T, T + pc - j)
        if lo < hi:
            out[lo:hi] += w[:, j] * g[lo - pc + j:hi - pc + j]
    return out


def conv_module(xn, p, T, nseq, k, causal):
    """encoder.c:413-462: pointwise 1 (+b), GLU, depthwise (+b), the conv
    norm (folded batch norm, else a layer norm), SiLU, pointwise 2 (+b)."""
    h = linear(xn, p["pw1_w"], p.get("pw1_b"))
    d = h.shape[1] // 2
    g = h[:, :d] * sigmoid(h[:, d:])
    c = np.concatenate([depthwise(g[s * T:(s + 1) * T], p["dw_w"], p.get("dw_b"), k, causal) for s in range(nseq)])
    if p.get("cnorm_scale") is not None:
        c = c * p["cnorm_scale"] + p["cnorm_shift"]
    else:
        c = layer_norm(c, p["cnorm_w"], p["cnorm_b"])
    return linear(silu(c), p["pw2_w"], p.get("pw2_b"))


def attention(xn, p, T, nseq, pe, H, left, right):
    """encoder.c:315-410 (left < 0) / 220-313: q, k, v (+biases), rk = pe .
    relk^T, the relative-position core per segment, the output projection."""
    q = linear(xn, p["q_w"], p.get("q_b"))
    k = linear(xn, p["k_w"], p.get("k_b"))
    v = linear(xn, p["v_w"], p.get("v_b"))
    rk = linear(pe, p["relk_w"])
    ctx = np.concatenate([relpos_attention(q[s * T:(s + 1) * T], k[s * T:(s + 1) * T], v[s * T:(s + 1) * T], rk,
                                           p["bias_u"], p["bias_v"], H, left, right) for s in range(nseq)])
    return linear(ctx, p["o_w"], p.get("o_b"))


def encoder_layer(x, p, T, nseq, pe, H, k, causal, left=-1, right=0):
    """encoder.c:485-521 on x [nseq * T, d] (returns the new x)."""
    x = np.array(x, np.float64)
    x = x + 0.5 * half_ffn(x, p, 0)
    x = x + attention(layer_norm(x, p["ln_att_w"], p["ln_att_b"]), p, T, nseq, pe, H, left, right)
    x = x + conv_module(layer_norm(x, p["ln_conv_w"], p["ln_conv_b"]), p, T, nseq, k, causal)
    x = x + 0.5 * half_ffn(x, p, 1)
    return layer_norm(x, p["ln_out_w"], p["ln_out_b"])


def pos_emb(T, d):
    """encoder.c:201-212: positions T-1 .. -(T-1), interleaved sin / cos."""
    pos = (T - 1 - np.arange(2 * T - 1, dtype=np.float64))[:, None]
    j = np.arange(d // 2, dtype=np.float64)[None, :]
    f = pos * np.power(10000.0, -2.0 * j / d)
    pe = np.empty((2 * T - 1, d), np.float64)
    pe[:, 0::2] = np.sin(f)
    pe[:, 1::2] = np.cos(f)
    return pe


# ------------------------------------------------------------ subsampling
def conv2d_s2(x, w, b, pl, pr, depthwise):
    """subsampling.c:109-200: 3x3 stride-2 conv of x [C_in, T, F] with zero
    pads (pl, pr) in time and frequency; w [C_out, C_in or 1, 3, 3]."""
    x = np.asarray(x, np.float64)
    Cin, T, F = x.shape
    xp = np.zeros((Cin, T + pl + pr, F + pl + pr))
    xp[:, pl:pl + T, pl:pl + F] = x
    To, Fo = (T + pl + pr - 3) // 2 + 1, (F + pl + pr - 3) // 2 + 1
    Cout = w.shape[0]
    out = np.zeros((Cout, To, Fo)) + np.asarray(b, np.float64)[:, None, None]
    for dt in range(3):
        for df in range(3):
            win = xp[:, dt:dt + 2 * To - 1:2, df:df + 2 * Fo - 1:2]          # [Cin, To, Fo]
            if depthwise:
                out += w[:, 0, dt, df][:, None, None] * win
            else:
                out += np.einsum("oi,itf->otf", w[:, :, dt, df], win)
    return out


def subsampling(feats, p, causal):
    """subsampling.c:208-268 on one segment feats [T, n_mels]: conv_in + ReLU,
    twice (depthwise, pointwise, ReLU), channel-major flatten, linear."""
    pl, pr = (2, 1) if causal else (1, 1)
    relu = lambda a: np.maximum(a, 0.0)
    a = relu(conv2d_s2(np.asarray(feats, np.float64)[None], p["conv_in_w"], p["conv_in_b"], pl, pr, False))
    for i in range(2):
        bb = conv2d_s2(a, p[f"dw_w{i}"], p[f"dw_b{i}"], pl, pr, True)
        a = relu(np.einsum("oc,ctf->otf", p[f"pw_w{i}"], bb) + np.asarray(p[f"pw_b{i}"], np.float64)[:, None, None])
    C, To, Fo = a.shape
    flat = a.transpose(1, 0, 2).reshape(To, C * Fo)                        # flat[t, c * Fo + f]
    return linear(flat, p["lin_w"], p["lin_b"])
