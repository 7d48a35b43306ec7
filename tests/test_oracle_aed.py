"""The AED decoder oracle (oracle/aed.py, imported as `aed`) pinned by closed
forms and invariants: a dropped residual, a wrong normalisation, a causality
leak or a mis-scaled score fails here."""
import numpy as np
import pytest
from scipy.special import softmax

import aed


def rnd(seed, *shape, sc=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * sc


def test_ln_closed_form():
    y = aed.ln(np.array([1.0, 2.0, 3.0, 4.0]), np.ones(4), np.zeros(4))
    z = np.array([-1.5, -0.5, 0.5, 1.5]) / np.sqrt(1.25 + 1e-5)
    np.testing.assert_allclose(y, z, rtol=1e-15)
    x = rnd(1, 64)
    w, b = rnd(2, 64), rnd(3, 64)
    ref = (x - x.mean()) / np.sqrt(x.var() + 1e-5) * w + b
    np.testing.assert_allclose(aed.ln(x, w, b), ref, rtol=1e-13)


def test_attend_special_cases():
    d, H = 16, 2
    q = rnd(4, d)
    K, V = rnd(5, 1, d), rnd(6, 1, d)
    np.testing.assert_allclose(aed.attend(q, K, V, H), V[0])          # one key: its value
    K = np.zeros((5, d))
    V = rnd(7, 5, d)
    np.testing.assert_allclose(aed.attend(q, K, V, H), V.mean(0))    # equal scores: the mean
    K, Vr = rnd(8, 6, d), rnd(9, 6, d)
    out = aed.attend(q, K, Vr, H)
    for h in range(H):                                               # per head, scaled by 1/sqrt(dk)
        sl = slice(h * 8, h * 8 + 8)
        p = softmax(K[:, sl] @ q[sl] / np.sqrt(8.0))
        np.testing.assert_allclose(out[sl], p @ Vr[:, sl], rtol=1e-12)


def make_model(seed, d=16, H=2, ffn=24, vocab=20, n_layers=2, max_seq=12, zero_out=False):
    r = np.random.default_rng(seed)
    f = lambda *s, sc=0.3: r.standard_normal(s) * sc
    layers = []
    for _ in range(n_layers):
        L = {}
        for nm in ("sq", "sk", "sv", "so", "cq", "ck", "cv", "co"):
            L[nm], L[nm + "_b"] = f(d, d), f(d, sc=0.1)
        L["ff1"], L["ff1_b"], L["ff2"], L["ff2_b"] = f(ffn, d), f(ffn, sc=0.1), f(d, ffn), f(d, sc=0.1)
        for nm in ("self", "cross", "ffn"):
            L[f"ln_{nm}_w"], L[f"ln_{nm}_b"] = 1 + f(d, sc=0.1), f(d, sc=0.1)
        if zero_out:
            for nm in ("so", "co", "ff2"):
                L[nm] = np.zeros_like(L[nm])
                L[nm + "_b"] = np.zeros(d)
        layers.append(L)
    return aed.Model(f(vocab, d, sc=1.0), f(max_seq, d), 1 + f(d, sc=0.1), f(d, sc=0.1), 1 + f(d, sc=0.1),
                     f(d, sc=0.1), f(vocab, d, sc=1.0), f(vocab, sc=0.1), layers, H)


def test_sublayers_are_residual():
    """Output projections of zero: every layer passes x through unchanged, so
    the logits are those of the embedding alone (closed form)."""
    m = make_model(10, zero_out=True)
    enc = rnd(11, 7, 16)
    toks = [3, 5, 1, 7]
    got = m.forced(enc, toks)
    for p, t in enumerate(toks):
        x = aed.ln(m.emb[t] + m.pos[p], m.embln_w, m.embln_b)
        np.testing.assert_allclose(got[p], m.head @ aed.ln(x, m.fin_w, m.fin_b) + m.head_b, rtol=1e-12)


def test_causal():
    """Position p's logits do not depend on later tokens, and do depend on earlier ones."""
    m = make_model(12)
    enc = rnd(13, 9, 16)
    a = m.forced(enc, [1, 2, 3, 4, 5])
    b = m.forced(enc, [1, 2, 3, 9, 0])
    np.testing.assert_array_equal(a[:3], b[:3])
    assert not np.allclose(a[3:], b[3:])
    c = m.forced(enc, [6, 2, 3, 4, 5])
    assert not np.allclose(a[1:], c[1:])


def test_cross_attention_reads_encoder():
    m = make_model(14)
    e1, e2 = rnd(15, 9, 16), rnd(16, 9, 16)
    assert not np.allclose(m.forced(e1, [1, 2]), m.forced(e2, [1, 2]))
    # permuting the encoder frames does not change cross attention (no positions there)
    perm = np.random.default_rng(0).permutation(9)
    np.testing.assert_allclose(m.forced(e1, [1, 2]), m.forced(e1[perm], [1, 2]), rtol=1e-12)


def test_decode_follows_forced_argmax():
    """Greedy decoding = the argmax of the forced logits of its own prefix;
    prompt tokens are consumed without sampling; eos and cap stop it."""
    m = make_model(17)
    enc = rnd(18, 9, 16)
    prompt = [2, 4, 6]
    toks, _ = m.decode(enc, prompt, eos=-1, cap=5, max_seq=12)
    assert len(toks) == 5
    lg = m.forced(enc, prompt + toks[:-1])
    assert [int(np.argmax(l)) for l in lg[len(prompt) - 1:]] == toks
    eos = toks[2]
    toks2, _ = m.decode(enc, prompt, eos=eos, cap=5, max_seq=12)
    assert toks2 == toks[:toks.index(eos)]
    # positions stop at max_seq: the last prompt position already yields the first token
    toks3, _ = m.decode(enc, prompt, eos=-1, cap=5, max_seq=5)
    assert toks3 == toks[:5 - len(prompt) + 1]


# ------------------------------------------------------ closed-form layers
def _ln(x, w, b):
    # written out again (not aed.ln): mean, biased variance, eps 1e-5
    c = x - x.sum() / x.size
    return c / np.sqrt((c * c).sum() / x.size + 1e-5) * w + b


def _one_layer(seed, keep):
    """One layer whose sublayers outside `keep` have zero output projections."""
    m = make_model(seed, n_layers=1)
    L = m.layers[0]
    for sub, (w, b) in (("self", ("so", "so_b")), ("cross", ("co", "co_b")), ("ffn", ("ff2", "ff2_b"))):
        if sub not in keep:
            L[w] = np.zeros_like(L[w])
            L[b] = np.zeros_like(L[b])
    return m, L


def _logits(m, x):
    return m.head @ _ln(x, m.fin_w, m.fin_b) + m.head_b


def test_ffn_sublayer_closed_form():
    """decoder_aed.c:205-210: x + W2 relu(W1 LN_ffn(x) + b1) + b2, with the
    norm before the sublayer (pre-LN) and ReLU, not SiLU or GELU."""
    m, L = _one_layer(20, {"ffn"})
    enc = rnd(21, 5, 16)
    for p, t in enumerate([4, 9, 2]):
        x = _ln(m.emb[t] + m.pos[p], m.embln_w, m.embln_b)
        h = L["ff1"] @ _ln(x, L["ln_ffn_w"], L["ln_ffn_b"]) + L["ff1_b"]
        x = x + L["ff2"] @ np.where(h > 0, h, 0.0) + L["ff2_b"]
        np.testing.assert_allclose(m.forced(enc, [4, 9, 2][:p + 1])[p], _logits(m, x), rtol=1e-12, atol=1e-12)


def test_self_attention_at_position_zero_closed_form():
    """decoder_aed.c:186-198 at p = 0: one key (the position's own), so the
    attention output is its value: x + Wo (Wv LN_self(x) + bv) + bo."""
    m, L = _one_layer(22, {"self"})
    enc = rnd(23, 5, 16)
    t = 7
    x = _ln(m.emb[t] + m.pos[0], m.embln_w, m.embln_b)
    v = L["sv"] @ _ln(x, L["ln_self_w"], L["ln_self_b"]) + L["sv_b"]
    x = x + L["so"] @ v + L["so_b"]
    np.testing.assert_allclose(m.forced(enc, [t])[0], _logits(m, x), rtol=1e-12, atol=1e-12)


def test_cross_attention_one_frame_closed_form():
    """decoder_aed.c:199-204 over one encoder frame: the attention output is
    that frame's value, whatever the query: x + Wco (Wcv e + bcv) + bco."""
    m, L = _one_layer(24, {"cross"})
    e = rnd(25, 1, 16)
    toks = [3, 8]
    got = m.forced(e, toks)
    for p, t in enumerate(toks):
        x = _ln(m.emb[t] + m.pos[p], m.embln_w, m.embln_b)
        x = x + L["co"] @ (L["cv"] @ e[0] + L["cv_b"]) + L["co_b"]
        np.testing.assert_allclose(got[p], _logits(m, x), rtol=1e-12, atol=1e-12)


def test_layer_composition_order_closed_form():
    """All three sublayers at p = 0 over one encoder frame: self, then cross,
    then FFN, each pre-LN with a residual (decoder_aed.c:186-210). A swapped
    self/cross order or a post-LN layer gives other values."""
    m, L = _one_layer(26, {"self", "cross", "ffn"})
    e = rnd(27, 1, 16)
    t = 5
    x = _ln(m.emb[t] + m.pos[0], m.embln_w, m.embln_b)
    x = x + L["so"] @ (L["sv"] @ _ln(x, L["ln_self_w"], L["ln_self_b"]) + L["sv_b"]) + L["so_b"]
    x = x + L["co"] @ (L["cv"] @ e[0] + L["cv_b"]) + L["co_b"]
    h = L["ff1"] @ _ln(x, L["ln_ffn_w"], L["ln_ffn_b"]) + L["ff1_b"]
    x = x + L["ff2"] @ np.maximum(h, 0.0) + L["ff2_b"]
    want = _logits(m, x)
    np.testing.assert_allclose(m.forced(e, [t])[0], want, rtol=1e-12, atol=1e-12)
    # the swapped order is a different function here (so the test can tell)
    y = _ln(m.emb[t] + m.pos[0], m.embln_w, m.embln_b)
    y = y + L["co"] @ (L["cv"] @ e[0] + L["cv_b"]) + L["co_b"]
    y = y + L["so"] @ (L["sv"] @ _ln(y, L["ln_self_w"], L["ln_self_b"]) + L["sv_b"]) + L["so_b"]
    h = L["ff1"] @ _ln(y, L["ln_ffn_w"], L["ln_ffn_b"]) + L["ff1_b"]
    y = y + L["ff2"] @ np.maximum(h, 0.0) + L["ff2_b"]
    assert not np.allclose(_logits(m, y), want)
