"""aed.py — TEST INFRASTRUCTURE ONLY.

numpy float64 restatement of the reference's AED (Canary) greedy decoder,
src/decoder_aed.c, over weights given as dense matrices (the dequantized
blocks; W is [n, k] and a product is x . W^T as qmat_mul computes it):

    ln(x)        decoder_aed.c:21-28   mean and variance over d, eps 1e-5
    softmax      decoder_aed.c:30-37
    attend       decoder_aed.c:124-137 one query over n_kv keys, per head,
                                       scores scaled by 1/sqrt(dk)
    decode       decoder_aed.c:139-232 encoder projection, per-layer cross
                                       K/V, then per position: embedding +
                                       pos + LN, per layer pre-LN causal self
                                       attention (KV cache), cross attention,
                                       ReLU FFN, each with a residual; final
                                       LN, head, argmax (first maximum)

`forced` runs the same steps over a given token sequence and returns every
step's logits (the loop's own computation, with the tokens supplied instead
of chosen). Only tests/ import this module.
"""
from __future__ import annotations

import numpy as np


def ln(x, w, b):
    """decoder_aed.c:21-28 (double accumulation; the reference rounds the
    normalised value to f32 before the affine step)."""
    x = np.asarray(x, np.float64)
    mu = x.mean()
    var = ((x - mu) ** 2).mean()
    inv = 1.0 / np.sqrt(var + 1e-5)
    return (x - mu) * inv * w + b


def softmax(s):
    """decoder_aed.c:30-37."""
    e = np.exp(s - s.max())
    return e / e.sum()


def attend(q, K, V, H):
    """decoder_aed.c:124-137: q [d], K/V [n_kv, d] -> out [d]."""
    d = q.shape[0]
    dk = d // H
    scale = 1.0 / np.sqrt(float(np.float32(dk)))
    out = np.empty(d)
    for h in range(H):
        sl = slice(h * dk, (h + 1) * dk)
        p = softmax(scale * (K[:, sl] @ q[sl]))
        out[sl] = V[:, sl].T @ p
    return out


class Model:
    """The decoder's tensors as float64 arrays. `layers` is a list of dicts
    with the keys of mynah_asr_aed_layer (decoder_aed.h:12-22): weights
    sq sk sv so cq ck cv co ff1 ff2 ([n, k]), biases *_b, norms ln_*_w/_b.
    `proj` is None for the identity projection."""

    def __init__(self, emb, pos, embln_w, embln_b, fin_w, fin_b, head, head_b, layers, H,
                 proj=None, proj_b=None):
        f = lambda a: None if a is None else np.asarray(a, np.float64)
        self.emb, self.pos = f(emb), f(pos)
        self.embln_w, self.embln_b, self.fin_w, self.fin_b = f(embln_w), f(embln_b), f(fin_w), f(fin_b)
        self.head, self.head_b = f(head), f(head_b)
        self.proj, self.proj_b = f(proj), f(proj_b)
        self.layers = [{k: f(v) for k, v in L.items()} for L in layers]
        self.H = H

    def _cross(self, enc):
        encp = np.asarray(enc, np.float64)
        if self.proj is not None:
            encp = encp @ self.proj.T + self.proj_b
        return [(encp @ L["ck"].T + L["ck_b"], encp @ L["cv"].T + L["cv_b"]) for L in self.layers]

    def _step(self, tok, p, cross, cache):
        """One position (decoder_aed.c:181-212): returns the final x."""
        x = ln(self.emb[tok] + self.pos[p], self.embln_w, self.embln_b)
        for li, L in enumerate(self.layers):
            SK, SV = cache[li]
            xn = ln(x, L["ln_self_w"], L["ln_self_b"])
            q = L["sq"] @ xn + L["sq_b"]
            SK.append(L["sk"] @ xn + L["sk_b"])
            SV.append(L["sv"] @ xn + L["sv_b"])
            att = attend(q, np.array(SK), np.array(SV), self.H)
            x = x + (L["so"] @ att + L["so_b"])
            xn = ln(x, L["ln_cross_w"], L["ln_cross_b"])
            q = L["cq"] @ xn + L["cq_b"]
            att = attend(q, cross[li][0], cross[li][1], self.H)
            x = x + (L["co"] @ att + L["co_b"])
            xn = ln(x, L["ln_ffn_w"], L["ln_ffn_b"])
            ff = np.maximum(L["ff1"] @ xn + L["ff1_b"], 0.0)
            x = x + (L["ff2"] @ ff + L["ff2_b"])
        return x

    def logits(self, x):
        return self.head @ ln(x, self.fin_w, self.fin_b) + self.head_b

    def decode(self, enc, prompt, eos, cap, max_seq):
        """Greedy tokens (decoder_aed.c:139-232), with each chosen token's
        logit margin over the runner-up (for near-tie handling in tests)."""
        cross = self._cross(enc)
        cache = [([], []) for _ in self.layers]
        max_len = min(len(prompt) + cap, max_seq)
        out, margins, cur = [], [], prompt[0]
        for p in range(max_len):
            x = self._step(cur, p, cross, cache)
            if p + 1 < len(prompt):
                cur = prompt[p + 1]
                continue
            lg = self.logits(x)
            best = int(np.argmax(lg))            # first maximum, as the strict > scan
            top2 = np.sort(lg)[-2:]
            if best == eos or len(out) >= cap:
                break
            out.append(best)
            margins.append(float(top2[1] - top2[0]))
            cur = best
        return out, margins

    def forced(self, enc, tokens):
        """Logits [n, vocab] of every position for the given tokens."""
        cross = self._cross(enc)
        cache = [([], []) for _ in self.layers]
        return np.array([self.logits(self._step(t, p, cross, cache)) for p, t in enumerate(tokens)])
