"""The encoder-layer oracle (oracle/encoder.py) pinned by closed forms and by
cases that reduce to textbook routines, so that a dropped term, a wrong
residual weight, a misplaced pad or a swapped GLU half fails one of them.
The attention core it calls is pinned in tests/test_oracle_attention.py."""
import numpy as np
import pytest

import encoder as E
from attention import relpos_attention


def rng(seed):
    return np.random.default_rng(seed)


def test_layer_norm_closed_form():
    """encoder.c:25-37: per row zero mean, unit variance (up to eps), then the
    affine; a constant row maps to b."""
    x = rng(0).standard_normal((7, 64)) * 3 + 5
    w, b = rng(1).standard_normal(64), rng(2).standard_normal(64)
    y = E.layer_norm(x, np.ones(64), np.zeros(64))
    assert np.allclose(y.mean(axis=1), 0, atol=1e-12)
    var = x.var(axis=1)
    assert np.allclose(y.var(axis=1), var / (var + 1e-5), rtol=1e-12)
    assert np.allclose(E.layer_norm(x, w, b), y * w + b)
    assert np.allclose(E.layer_norm(np.full((2, 64), 3.0), w, b), b)


def test_depthwise_taps_and_padding():
    """encoder.c:434-447: a one-hot tap j copies g shifted by j - pc, with
    zeros outside the segment; 'same' pads (k-1)/2, causal k-1."""
    T, d, k = 11, 8, 5
    g = rng(3).standard_normal((T, d))
    for causal, pc in ((0, 2), (1, 4)):
        for j in range(k):
            w = np.zeros((d, k))
            w[:, j] = 1.0
            out = E.depthwise(g, w, None, k, causal)
            want = np.zeros((T, d))
            for t in range(T):
                src = t - pc + j
                if 0 <= src < T:
                    want[t] = g[src]
            assert np.array_equal(out, want), (causal, j)
    # a general kernel is the sum of its taps, plus the bias
    w, bias = rng(4).standard_normal((d, k)), rng(5).standard_normal(d)
    parts = sum(E.depthwise(g, np.where(np.arange(k) == j, w, 0.0), None, k, 0) for j in range(k))
    assert np.allclose(E.depthwise(g, w, bias, k, 0), parts + bias)


def conv_params(d, k, rs):
    return {"pw1_w": rs.standard_normal((2 * d, d)) * 0.1, "pw1_b": rs.standard_normal(2 * d) * 0.1,
            "dw_w": rs.standard_normal((d, k)) * 0.3, "dw_b": rs.standard_normal(d) * 0.1,
            "cnorm_scale": 1 + 0.1 * rs.standard_normal(d), "cnorm_shift": 0.1 * rs.standard_normal(d),
            "pw2_w": rs.standard_normal((d, d)) * 0.1, "pw2_b": rs.standard_normal(d) * 0.1}


def test_conv_module_reduces_to_glu_and_silu():
    """encoder.c:413-462 with pw1 = [I; 0] (the gate half zero: sigmoid(0) =
    1/2), the centre tap one, the folded norm the identity and pw2 = I:
    out = silu(x / 2) — any swap of the GLU halves, tap order or norm order
    breaks it."""
    d, k, T = 16, 9, 13
    x = rng(6).standard_normal((T, d))
    w = np.zeros((d, k))
    w[:, (k - 1) // 2] = 1.0
    p = {"pw1_w": np.vstack([np.eye(d), np.zeros((d, d))]), "dw_w": w, "cnorm_scale": np.ones(d),
         "cnorm_shift": np.zeros(d), "pw2_w": np.eye(d)}
    assert np.allclose(E.conv_module(x, p, T, 1, k, 0), E.silu(x / 2))
    # a gate of +inf passes a through; of -inf blocks it
    p["pw1_w"] = np.vstack([np.eye(d), np.zeros((d, d))])
    p["pw1_b"] = np.concatenate([np.zeros(d), np.full(d, 50.0)])
    assert np.allclose(E.conv_module(x, p, T, 1, k, 0), E.silu(x), atol=1e-12)
    # the LN conv norm in place of the folded one
    q = dict(p)
    del q["cnorm_scale"]
    q["cnorm_w"], q["cnorm_b"] = np.ones(d), np.zeros(d)
    assert np.allclose(E.conv_module(x, q, T, 1, k, 0), E.silu(E.layer_norm(x, np.ones(d), np.zeros(d))), atol=1e-9)


def test_conv_module_segments_are_independent():
    """The depthwise conv does not cross a segment boundary (encoder.c:
    seg_worker runs it per segment): two segments packed give each segment's
    own result."""
    d, k, T = 16, 9, 10
    p = conv_params(d, k, rng(7))
    x = rng(8).standard_normal((2 * T, d))
    both = E.conv_module(x, p, T, 2, k, 1)
    assert np.allclose(both[:T], E.conv_module(x[:T], p, T, 1, k, 1))
    assert np.allclose(both[T:], E.conv_module(x[T:], p, T, 1, k, 1))


def layer_params(d, f, k, rs, biases):
    p = {}
    for n in ("ff1", "ff2", "att", "conv", "out"):
        p[f"ln_{n}_w"], p[f"ln_{n}_b"] = 1 + 0.1 * rs.standard_normal(d), 0.1 * rs.standard_normal(d)
    for n in ("ff1", "ff2"):
        p[f"{n}_w1"], p[f"{n}_w2"] = rs.standard_normal((f, d)) * 0.05, rs.standard_normal((d, f)) * 0.05
        if biases:
            p[f"{n}_b1"], p[f"{n}_b2"] = 0.1 * rs.standard_normal(f), 0.1 * rs.standard_normal(d)
    for n in ("q", "k", "v", "o", "relk"):
        p[f"{n}_w"] = rs.standard_normal((d, d)) * 0.05
        if biases and n != "relk":
            p[f"{n}_b"] = 0.1 * rs.standard_normal(d)
    p["bias_u"], p["bias_v"] = 0.1 * rs.standard_normal(d), 0.1 * rs.standard_normal(d)
    p.update(conv_params(d, k, rs))
    if not biases:
        for n in ("pw1_b", "dw_b", "pw2_b"):
            p.pop(n)
    return p


def test_layer_residual_structure():
    """encoder.c:485-521: with the attention, conv and second FFN outputs
    zeroed (o, pw2, ff2_w2 = 0) the layer is LN_out(x + ffn1(x)/2); with only
    the conv path live, LN_out(x' + conv(LN_conv(x'))) where x' carries the
    first FFN; the FFN terms weigh 1/2, the others 1."""
    d, f, k, T, H = 64, 128, 5, 9, 1
    p = layer_params(d, f, k, rng(9), biases=True)
    x = rng(10).standard_normal((T, d))
    pe = E.pos_emb(T, d)
    z = dict(p, o_w=np.zeros((d, d)), o_b=np.zeros(d), pw2_w=np.zeros((d, d)), pw2_b=np.zeros(d),
             ff2_w2=np.zeros((d, f)), ff2_b2=np.zeros(d))
    want = E.layer_norm(x + 0.5 * E.half_ffn(x, z, 0), z["ln_out_w"], z["ln_out_b"])
    assert np.allclose(E.encoder_layer(x, z, T, 1, pe, H, k, 0), want)
    c = dict(z, pw2_w=p["pw2_w"], pw2_b=p["pw2_b"])
    x1 = x + 0.5 * E.half_ffn(x, c, 0)
    x2 = x1 + E.conv_module(E.layer_norm(x1, c["ln_conv_w"], c["ln_conv_b"]), c, T, 1, k, 0)
    assert np.allclose(E.encoder_layer(x, c, T, 1, pe, H, k, 0), E.layer_norm(x2, c["ln_out_w"], c["ln_out_b"]))


def test_attention_is_the_core_between_projections():
    """encoder.c:315-410: q, k, v projections with their biases, rk = pe .
    relk^T, the core, the output projection: identity projections give the
    core itself."""
    d, T, H = 32, 6, 2
    x = rng(11).standard_normal((T, d))
    pe = E.pos_emb(T, d)
    bu, bv = rng(12).standard_normal(d) * 0.1, rng(13).standard_normal(d) * 0.1
    p = {"q_w": np.eye(d), "k_w": np.eye(d), "v_w": np.eye(d), "o_w": np.eye(d), "relk_w": np.eye(d),
         "bias_u": bu, "bias_v": bv}
    assert np.allclose(E.attention(x, p, T, 1, pe, H, -1, 0), relpos_attention(x, x, x, pe, bu, bv, H))


def test_pos_emb_closed_form():
    """encoder.c:201-212: row p is position T-1-p; sin at even, cos at odd
    columns; the middle row (position 0) is [0, 1, 0, 1, ...]."""
    T, d = 5, 8
    pe = E.pos_emb(T, d)
    assert pe.shape == (2 * T - 1, d)
    assert np.allclose(pe[T - 1], np.tile([0.0, 1.0], d // 2))
    p, j = 1, 2
    assert np.isclose(pe[p, 2 * j], np.sin((T - 1 - p) * 10000.0 ** (-2.0 * j / d)))
    assert np.isclose(pe[p, 2 * j + 1], np.cos((T - 1 - p) * 10000.0 ** (-2.0 * j / d)))


def conv2d_direct(x, w, b, pl, pr, depthwise):
    """The reference's direct loop (subsampling.c:169-197), element by
    element, for tiny inputs: the vectorized oracle must equal it."""
    Cin, T, F = x.shape
    To, Fo = (T + pl + pr - 3) // 2 + 1, (F + pl + pr - 3) // 2 + 1
    Cout = w.shape[0]
    out = np.zeros((Cout, To, Fo))
    for co in range(Cout):
        for ci in ([co] if depthwise else range(Cin)):
            ker = w[co, 0] if depthwise else w[co, ci]
            for to in range(To):
                for fo in range(Fo):
                    acc = 0.0
                    for dt in range(3):
                        t = 2 * to - pl + dt
                        if t < 0 or t >= T:
                            continue
                        for df in range(3):
                            f = 2 * fo - pl + df
                            if 0 <= f < F:
                                acc += ker[dt, df] * x[ci, t, f]
                    out[co, to, fo] += acc
        out[co] += b[co]
    return out


@pytest.mark.parametrize("pl,pr", [(1, 1), (2, 1)])
def test_conv2d_s2_equals_the_direct_loop(pl, pr):
    r = rng(20)
    x = r.standard_normal((3, 9, 7))
    w, b = r.standard_normal((4, 3, 3, 3)), r.standard_normal(4)
    assert np.allclose(E.conv2d_s2(x, w, b, pl, pr, False), conv2d_direct(x, w, b, pl, pr, False))
    wd = r.standard_normal((3, 1, 3, 3))
    assert np.allclose(E.conv2d_s2(x, wd, b[:3], pl, pr, True), conv2d_direct(x, wd, b[:3], pl, pr, True))
    # output sizes: (n + pl + pr - 3) // 2 + 1
    assert E.conv2d_s2(x, w, b, pl, pr, False).shape == (4, (9 + pl + pr - 3) // 2 + 1, (7 + pl + pr - 3) // 2 + 1)


def test_conv2d_s2_centre_tap_subsamples():
    """A kernel with only tap (pl, pl) picks x[2 to, 2 fo] (the stride)."""
    x = rng(21).standard_normal((1, 10, 8))
    for pl, pr in ((1, 1), (2, 1)):
        w = np.zeros((1, 1, 3, 3))
        w[0, 0, pl, pl] = 1.0
        out = E.conv2d_s2(x, w, np.zeros(1), pl, pr, False)
        To, Fo = out.shape[1:]
        want = np.zeros((To, Fo))            # positions past the end read the right pad (zero)
        sub = x[0, 0:2 * To:2, 0:2 * Fo:2]
        want[:sub.shape[0], :sub.shape[1]] = sub
        assert np.array_equal(out[0], want)


def test_subsampling_flatten_order():
    """subsampling.c:248-264: the linear sees flat[t, c * F' + f]. With
    identity-like convs (centre taps one, pointwise I, zero biases) and a
    positive input, the output picks the input at (8 t, 8 f) through the
    linear's column c * F' + f."""
    T, nm, C, d = 24, 16, 4, 5
    x = np.abs(rng(22).standard_normal((T, nm))) + 0.1
    p = {"conv_in_w": np.zeros((C, 1, 3, 3)), "conv_in_b": np.zeros(C), "lin_b": np.zeros(d)}
    p["conv_in_w"][:, 0, 1, 1] = 1.0
    for i in range(2):
        p[f"dw_w{i}"] = np.zeros((C, 1, 3, 3))
        p[f"dw_w{i}"][:, 0, 1, 1] = 1.0
        p[f"dw_b{i}"], p[f"pw_w{i}"], p[f"pw_b{i}"] = np.zeros(C), np.eye(C), np.zeros(C)
    Fo, To = 2, 3   # 16 -> 8 -> 4 -> 2; 24 -> 12 -> 6 -> 3
    for c in range(C):
        for f in range(Fo):
            lw = np.zeros((d, C * Fo))
            lw[0, c * Fo + f] = 1.0
            out = E.subsampling(x, dict(p, lin_w=lw), causal=0)
            assert out.shape == (To, d)
            assert np.allclose(out[:, 0], x[0:8 * To:8, 8 * f])
