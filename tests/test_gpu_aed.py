"""GPU parity of the device AED decoder (mynah_asr_hip_aed_forced_dev /
mynah_asr_hip_aed_decode_dev) against the oracle's float64 restatement of
src/decoder_aed.c:139-232 over the same (dequantized) weights.

Bar:
  * forced logits: |y - ref| <= 1e-4*|ref| + 1e-5*rms(ref) per element. The
    device computes in f32 (the products EXACT, LN and softmax in f32 with
    double LN sums, as the reference); the rms term covers logits near zero
    after the cancellations of two layers of residual sums;
  * greedy tokens: equal to the oracle's, except that a position where the
    oracle's top two logits are within 1e-4*|top| + 1e-5*rms may pick either
    (then the sequences are compared up to that position).
Inputs: weights N(0, 0.1) (linears quantized by the library's quantizers),
embeddings N(0, 1), encoder output N(0, 1), seeded.
"""
import sys

import numpy as np
import pytest

import aed
import mynah_hip as M
import oracle as O

pytestmark = pytest.mark.gpu
TO_ORC = {M.Q4_0: O.Q4_0, M.Q8_0: O.Q8_0, M.Q4_K: O.Q4_K, M.Q6_K: O.Q6_K}


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make_params(seed, d, H, ffn, vocab, n_layers, max_seq, d_enc=None):
    r = np.random.default_rng(seed)
    f = lambda *s, sc=0.1: (r.standard_normal(s) * sc).astype(np.float32)
    layers = []
    for _ in range(n_layers):
        L = {}
        for nm in ("sq", "sk", "sv", "so", "cq", "ck", "cv", "co"):
            L[nm], L[nm + "_b"] = f(d, d, sc=1.0 / np.sqrt(d)), f(d)
        L["ff1"], L["ff1_b"] = f(ffn, d, sc=1.0 / np.sqrt(d)), f(ffn)
        L["ff2"], L["ff2_b"] = f(d, ffn, sc=1.0 / np.sqrt(ffn)), f(d)
        for nm in ("self", "cross", "ffn"):
            L[f"ln_{nm}_w"], L[f"ln_{nm}_b"] = 1 + f(d), f(d)
        layers.append(L)
    p = {"emb": f(vocab, d, sc=1.0), "pos": f(max_seq, d, sc=0.3), "embln_w": 1 + f(d), "embln_b": f(d),
         "fin_w": 1 + f(d), "fin_b": f(d), "head": f(vocab, d, sc=1.0 / np.sqrt(d)), "head_b": f(vocab),
         "layers": layers, "proj": None, "proj_b": None}
    if d_enc:
        p["proj"], p["proj_b"] = f(d, d_enc, sc=1.0 / np.sqrt(d_enc)), f(d)
    return p


def dense(orc, w):
    if w.qtype == M.F32:
        return w.data.reshape(w.n, w.k)
    return orc.dequant(TO_ORC[w.qtype], w.data, w.n * w.k).reshape(w.n, w.k)


def oracle_model(orc, dev, params, H):
    """The oracle decoder over the weights exactly as the device holds them."""
    wt = {k: dense(orc, w) for k, w in dev.weights.items()}
    layers = []
    for i, L in enumerate(params["layers"]):
        Lo = dict(L)
        for nm in M.DeviceAed.LINEARS:
            Lo[nm] = wt[f"{i}.{nm}"]
        layers.append(Lo)
    return aed.Model(params["emb"], params["pos"], params["embln_w"], params["embln_b"], params["fin_w"],
                     params["fin_b"], wt["head"], params["head_b"], layers, H,
                     proj=wt.get("proj"), proj_b=params["proj_b"])


def check_logits(got, ref, what):
    rms = np.sqrt((ref ** 2).mean())
    lim = 1e-4 * np.abs(ref) + 1e-5 * rms
    err = np.abs(got - ref)
    assert np.isfinite(got).all(), what
    assert (err <= lim).all(), f"{what}: {int((err > lim).sum())} outside; worst ratio {(err / lim).max():.3g}"
    say(what, "worst err/limit %.3g" % float((err / lim).max()))


CASES = [
    # d, H, ffn, vocab, layers, T, qtype, d_enc
    (256, 2, 512, 1000, 2, 37, M.F32, None),     # head size 128
    (256, 4, 512, 1000, 2, 70, M.Q8_0, 128),     # head size 64, encoder projection
    (512, 4, 1024, 2048, 3, 130, M.Q4_K, None),  # K-quant linears, 3 splits of cross keys
    (256, 2, 2048, 500, 1, 20, M.Q8_0, None),    # ff2 with K = 2048: the split-K GEMV
    # d = 2048: each wave forms two chunks of the row and sums the layer norm
    # over two batches of x; 600 keys = 10 splits: the merge's second batch
    (2048, 16, 2048, 700, 1, 600, M.Q8_0, None),
]


@pytest.mark.parametrize("d,H,ffn,vocab,nl,T,qt,d_enc", CASES)
def test_aed_forced_logits(gpu, orc, d, H, ffn, vocab, nl, T, qt, d_enc):
    import torch
    say("aed forced", d, H, ffn, vocab, nl, T, M.NAMES[qt], d_enc)
    max_seq = 80
    params = make_params(d + T, d, H, ffn, vocab, nl, max_seq, d_enc)
    dev = M.DeviceAed(gpu, params, H, qt)
    enc = np.random.default_rng(7).standard_normal((T, d_enc or d)).astype(np.float32)
    denc = torch.from_numpy(enc).cuda()
    toks = list(np.random.default_rng(8).integers(0, vocab, 70))   # 70 positions: 2 self-attention splits
    got = dev.forced(denc.data_ptr(), T, toks)
    ref = oracle_model(orc, dev, params, H).forced(enc, toks)
    check_logits(got, ref, f"forced {M.NAMES[qt]} d={d} H={H}")
    again = dev.forced(denc.data_ptr(), T, toks)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "second call differs"
    dev.close()


@pytest.mark.parametrize("d,H,ffn,vocab,nl,T,qt,d_enc", CASES[:2])
def test_aed_greedy_tokens(gpu, orc, d, H, ffn, vocab, nl, T, qt, d_enc):
    import torch
    say("aed greedy", d, H, M.NAMES[qt])
    max_seq = 80
    params = make_params(3 * d + T, d, H, ffn, vocab, nl, max_seq, d_enc)
    dev = M.DeviceAed(gpu, params, H, qt)
    enc = np.random.default_rng(9).standard_normal((T, d_enc or d)).astype(np.float32)
    denc = torch.from_numpy(enc).cuda()
    prompt = [5, 17, 3, 250]
    om = oracle_model(orc, dev, params, H)
    ref, margins = om.decode(enc, prompt, eos=-1, cap=40, max_seq=max_seq)
    got = dev.decode(denc.data_ptr(), T, prompt, eos=-1, cap=40)
    assert len(got) == len(ref) == 40
    n = len(ref)
    for i, (a, b) in enumerate(zip(got, ref)):
        if a != b:
            lg = om.forced(enc, prompt + ref[:i])[-1]
            tol = 1e-4 * np.abs(lg).max() + 1e-5 * np.sqrt((lg ** 2).mean())
            assert margins[i] <= tol, f"token {i}: {a} vs {b} with margin {margins[i]:.3g}"
            n = i
            break
    say("tokens equal over", n, "of", len(ref))
    # eos stops it, excluded; cap bounds it
    eos = ref[5]
    got2 = dev.decode(denc.data_ptr(), T, prompt, eos=eos, cap=40)
    assert got2 == ref[:ref.index(eos)]
    assert dev.decode(denc.data_ptr(), T, prompt, eos=-1, cap=3) == ref[:3]
    dev.close()


def test_aed_rejects_unsupported(gpu):
    import torch
    params = make_params(1, 96, 1, 128, 100, 1, 8)   # head size 96
    dev = M.DeviceAed(gpu, params, 1, M.F32)
    enc = torch.zeros((4, 96), device="cuda")
    with pytest.raises(RuntimeError, match="head size"):
        dev.forced(enc.data_ptr(), 4, [1, 2])
    dev.close()
    params = make_params(2, 128, 2, 128, 100, 1, 8)
    dev = M.DeviceAed(gpu, params, 2, M.F32)
    enc = torch.zeros((4, 128), device="cuda")
    with pytest.raises(RuntimeError, match="vocabulary"):
        dev.forced(enc.data_ptr(), 4, [1, 100])
    with pytest.raises(RuntimeError, match="vocabulary"):
        dev.decode(enc.data_ptr(), 4, [-1], eos=0, cap=2)
    with pytest.raises(RuntimeError, match="bad argument"):
        dev.forced(enc.data_ptr(), 4, list(range(9)))      # more positions than max_seq
    # under a caller's stream capture both entry points refuse up front (they
    # capture their own step graph); the capture itself stays valid
    g, s = torch.cuda.CUDAGraph(), torch.cuda.Stream()
    z = torch.zeros(4, device="cuda")
    msgs = []
    with torch.cuda.graph(g, stream=s):
        z.add_(1.0)
        for call in (lambda: dev.forced(enc.data_ptr(), 4, [1, 2], stream=s.cuda_stream),
                     lambda: dev.decode(enc.data_ptr(), 4, [1], eos=0, cap=2, stream=s.cuda_stream)):
            try:
                call()
                msgs.append("no error")
            except RuntimeError as ex:
                msgs.append(str(ex))
    g.replay()
    torch.cuda.synchronize()
    assert all("stream capture" in m for m in msgs), msgs
    assert torch.equal(z, torch.ones(4, device="cuda"))
    dev.close()


@pytest.mark.parametrize("nl,T", [(0, 5), (1, 1)])
def test_aed_edge_shapes(gpu, orc, nl, T):
    """No decoder layers (embedding, final norm and head only); a one-frame
    encoder output (cross attention over a single key)."""
    import torch
    say("aed edge", nl, T)
    d, H, ffn, vocab, max_seq = 128, 2, 256, 300, 16
    params = make_params(40 + nl, d, H, ffn, vocab, nl, max_seq)
    dev = M.DeviceAed(gpu, params, H, M.Q8_0)
    enc = np.random.default_rng(41).standard_normal((T, d)).astype(np.float32)
    denc = torch.from_numpy(enc).cuda()
    toks = [3, 1, 4, 1, 5, 9, 2, 6]
    got = dev.forced(denc.data_ptr(), T, toks)
    check_logits(got, oracle_model(orc, dev, params, H).forced(enc, toks), f"edge layers={nl} T={T}")
    dev.close()
