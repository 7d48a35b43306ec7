"""The device encoder layer (mynah_asr_hip_encoder_layer_dev) against the
float64 restatement of src/encoder.c:485-521 (oracle/encoder.py), over the
dequantized values of the weights it runs with, and its segments' rows
bit-identical to each segment run alone (encoder.c:876-878: the batched
form is bit-identical to the serial loop).

Bar: |y - ref| <= 2e-6 * (1 + |ref|) per element (the layer ends in a layer
norm, so its outputs are O(1)): the measured worst over these cases is
3.1e-7 (Q8_0 and Q4_K weights, biases or none, folded batch norm or layer
norm, causal or 'same' conv, full or chunked attention). Each case prints
its own."""
import sys

import numpy as np
import pytest

import encoder as E
import mynah_hip as M
import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make_params(seed, d, f, k, biases, bn):
    r = np.random.default_rng(seed)
    g = lambda *s: r.standard_normal(s).astype(np.float32)
    p = {}
    for n in ("ff1", "ff2", "att", "conv", "out"):
        p[f"ln_{n}_w"], p[f"ln_{n}_b"] = 1 + 0.1 * g(d), 0.1 * g(d)
    for n in ("ff1", "ff2"):
        p[f"{n}_w1"], p[f"{n}_w2"] = 0.02 * g(f, d), 0.02 * g(d, f)
        if biases:
            p[f"{n}_b1"], p[f"{n}_b2"] = 0.1 * g(f), 0.1 * g(d)
    for n in ("q", "k", "v", "o", "relk"):
        p[f"{n}_w"] = 0.02 * g(d, d)
        if biases and n != "relk":
            p[f"{n}_b"] = 0.1 * g(d)
    p["bias_u"], p["bias_v"] = 0.1 * g(d), 0.1 * g(d)
    p["pw1_w"], p["pw2_w"], p["dw_w"] = 0.02 * g(2 * d, d), 0.02 * g(d, d), 0.3 * g(d, k)
    if biases:
        p["pw1_b"], p["dw_b"], p["pw2_b"] = 0.1 * g(2 * d), 0.1 * g(d), 0.1 * g(d)
    if bn:
        p["cnorm_scale"], p["cnorm_shift"] = 1 + 0.1 * g(d), 0.1 * g(d)
    else:
        p["cnorm_w"], p["cnorm_b"] = 1 + 0.1 * g(d), 0.1 * g(d)
    return p


def oracle_params(orc, dev, p, qt):
    """The float64 values the device products use: quantized linears
    dequantized by the oracle, relk_w as given (F32)."""
    q = {}
    for f, a in p.items():
        if f in M.DeviceEncoderLayer.LINEARS and f != "relk_w":
            w = dev.weights[f]
            oq = {M.Q8_0: O.Q8_0, M.Q4_K: O.Q4_K}[qt]
            q[f] = orc.dequant(oq, w.data, w.n * w.k).reshape(w.n, w.k).astype(np.float64)
        else:
            q[f] = np.asarray(a, np.float64)
    return q


CASES = [
    # d, H, f, k, T, nseq, causal, biases, bn, left, right, qt
    (256, 4, 512, 9, 37, 3, 0, False, True, -1, 0, M.Q8_0),
    (256, 4, 512, 9, 29, 2, 1, True, False, -1, 0, M.Q8_0),
    (256, 2, 768, 5, 41, 2, 0, True, True, 12, 3, M.Q4_K),
    (1024, 8, 4096, 9, 120, 2, 0, False, True, -1, 0, M.Q8_0),
    (256, 2, 512, 31, 45, 2, 1, True, True, -1, 0, M.Q8_0),   # k 31: the untiled depthwise conv
    (256, 2, 512, 9, 7, 2, 0, False, True, -1, 0, M.Q8_0),    # M = 14: every product on the GEMV
    (512, 4, 1024, 9, 50, 2, 0, False, True, -1, 0, M.Q8_0),
    (2048, 16, 2048, 9, 40, 2, 0, False, True, -1, 0, M.Q8_0),  # the widest fused layer norm
]


@pytest.mark.parametrize("case", CASES, ids=[f"d{c[0]}-T{c[4]}x{c[5]}-{'causal' if c[6] else 'same'}"
                                             f"-{'bias' if c[7] else 'nobias'}-{'bn' if c[8] else 'ln'}"
                                             f"-L{c[9]}" for c in CASES])
def test_encoder_layer_matches_oracle(gpu, orc, case):
    import torch
    d, H, f, k, T, nseq, causal, biases, bn, left, right, qt = case
    say("encoder layer", case)
    p = make_params(7, d, f, k, biases, bn)
    dev = M.DeviceEncoderLayer(gpu, p, qt)
    try:
        x = np.random.default_rng(8).standard_normal((nseq * T, d)).astype(np.float32)
        pe = E.pos_emb(T, d).astype(np.float32)
        xd, ped = torch.from_numpy(x).cuda(), torch.from_numpy(pe).cuda()
        dev.run(xd.data_ptr(), T, nseq, ped.data_ptr(), d, H, k, causal, left, right)
        torch.cuda.synchronize()
        y = xd.cpu().numpy()
        ref = E.encoder_layer(x, oracle_params(orc, dev, p, qt), T, nseq, pe, H, k, causal, left, right)
        err = np.abs(y - ref)
        say(f"  max |y - ref| {err.max():.3g}, max err / (1 + |ref|) {(err / (1 + np.abs(ref))).max():.3g}")
        assert np.isfinite(y).all()
        assert (err <= 2e-6 * (1 + np.abs(ref))).all()
    finally:
        dev.close()


def test_encoder_layer_segments_are_independent(gpu):
    """Three segments packed: each segment's rows carry the bits of that
    segment run alone (products are row-stable; layer norms are per row;
    attention and the depthwise conv are per segment)."""
    import torch
    say("encoder layer segments")
    d, H, f, k, T = 256, 4, 512, 9, 33
    p = make_params(9, d, f, k, True, True)
    dev = M.DeviceEncoderLayer(gpu, p, M.Q8_0)
    try:
        x = np.random.default_rng(10).standard_normal((3 * T, d)).astype(np.float32)
        ped = torch.from_numpy(E.pos_emb(T, d).astype(np.float32)).cuda()
        xa = torch.from_numpy(x).cuda()
        dev.run(xa.data_ptr(), T, 3, ped.data_ptr(), d, H, k, 0)
        for s in range(3):
            xs = torch.from_numpy(x[s * T:(s + 1) * T].copy()).cuda()
            dev.run(xs.data_ptr(), T, 1, ped.data_ptr(), d, H, k, 0)
            torch.cuda.synchronize()
            assert torch.equal(xs.view(torch.int32), xa[s * T:(s + 1) * T].view(torch.int32)), s
    finally:
        dev.close()


@pytest.mark.parametrize("d,f,biases,qt,T,nseq", [(1024, 4096, False, M.Q8_0, 150, 2), (256, 512, True, M.Q8_0, 150, 2),
                                                  (512, 1024, False, M.Q4_K, 150, 2),
                                                  (256, 512, False, M.Q8_0, 128, 256),   # 8-wave attention
                                                  (2048, 2048, True, M.Q8_0, 70, 2), (2048, 4096, False, M.Q8_0, 64, 3)])
def test_encoder_layer_ln_prep_bit_identical(gpu, monkeypatch, d, f, biases, qt, T, nseq):
    """The layer's fused hand-offs give the bits of the layer without them
    (MYNAH_ASR_HIP_LN_PREP=0): layer norms, the attention core and the
    depthwise conv writing their products' prepared input directly (the same
    split of the same values), and products without bias adding their output
    into x in their epilogue (the layer norm's own residual fma). Q4_K
    products read row sums, so that layer keeps f32 rows but still takes the
    residual epilogues."""
    import torch
    say("encoder layer ln prep", d, f, biases, qt, T, nseq)
    H, k = d // 128, 9
    p = make_params(11, d, f, k, biases, True)
    dev = M.DeviceEncoderLayer(gpu, p, qt)
    try:
        x = np.random.default_rng(12).standard_normal((nseq * T, d)).astype(np.float32)
        ped = torch.from_numpy(E.pos_emb(T, d).astype(np.float32)).cuda()
        outs = []
        for flag in ("1", "0"):
            monkeypatch.setenv("MYNAH_ASR_HIP_LN_PREP", flag)
            xd = torch.from_numpy(x).cuda()
            dev.run(xd.data_ptr(), T, nseq, ped.data_ptr(), d, H, k, 0)
            torch.cuda.synchronize()
            outs.append(xd)
        assert torch.isfinite(outs[0]).all()
        assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    finally:
        dev.close()


def test_encoder_layer_refuses_bad_shapes(gpu):
    import torch
    say("encoder layer refusals")
    d, H, f, k, T = 256, 4, 512, 9, 8
    p = make_params(11, d, f, k, False, True)
    dev = M.DeviceEncoderLayer(gpu, p, M.Q8_0)
    try:
        x = torch.zeros((T, d), dtype=torch.float32, device="cuda")
        pe = torch.zeros((2 * T - 1, d), dtype=torch.float32, device="cuda")
        with pytest.raises(RuntimeError, match="head size"):
            dev.run(x.data_ptr(), T, 1, pe.data_ptr(), d, 1, k, 0)      # dk = 256
        with pytest.raises(RuntimeError, match="q/k/v/o"):
            dev.run(x.data_ptr(), T, 1, pe.data_ptr(), 512, 8, k, 0)    # weights are [256, 256]
        with pytest.raises(RuntimeError, match="256 times"):
            dev.run(x.data_ptr(), T, 1, pe.data_ptr(), 2304, 18, k, 0)  # no layer-norm width for 9 x 256
        c = dev.c
        saved, c.cnorm_shift = c.cnorm_shift, None
        with pytest.raises(RuntimeError, match="conv norm"):
            dev.run(x.data_ptr(), T, 1, pe.data_ptr(), d, H, k, 0)
        c.cnorm_shift = saved
    finally:
        dev.close()


def ss_params(seed, C, n_mels, d, causal):
    r = np.random.default_rng(seed)
    g = lambda *s: r.standard_normal(s).astype(np.float32)
    F = n_mels
    for _ in range(3):
        F = (F + (3 if causal else 2) - 3) // 2 + 1
    return {"conv_in_w": 0.3 * g(C, 1, 3, 3), "conv_in_b": 0.1 * g(C),
            "dw_w0": 0.3 * g(C, 1, 3, 3), "dw_b0": 0.1 * g(C), "pw_w0": 0.1 * g(C, C), "pw_b0": 0.1 * g(C),
            "dw_w1": 0.3 * g(C, 1, 3, 3), "dw_b1": 0.1 * g(C), "pw_w1": 0.1 * g(C, C), "pw_b1": 0.1 * g(C),
            "lin_w": 0.05 * g(d, C * F), "lin_b": 0.1 * g(d)}


@pytest.mark.parametrize("causal,C", [(0, 64), (1, 64), (0, 320)])
def test_subsampling_matches_oracle(gpu, causal, C):
    """mynah_asr_hip_subsampling_dev against the float64 restatement of
    src/subsampling.c:208-268 (oracle/encoder.py, pinned against the
    reference's direct loop): 3 segments of 203 frames of 80 mel features,
    C = 64 (and 320: the fused first stage's lanes take channels 4 at a
    time, 256 per pass), d_model 256, xscale 2. Bar: |y - ref| <= 5e-6 * (|ref| + rms(ref))
    (measured worst 8.2e-7: f32-weight products and 9-term f32 convolution
    sums)."""
    import torch
    say("subsampling, causal", causal, "channels", C)
    nm, d, T, nseq = 80, 256, 203, 3
    p = ss_params(12, C, nm, d, causal)
    dev = M.DeviceSubsampling(gpu, p, causal)
    try:
        x = np.random.default_rng(13).standard_normal((nseq * T, nm)).astype(np.float32)
        To = (T + (3 if causal else 2) - 3) // 2 + 1
        for _ in range(2):
            To = (To + (3 if causal else 2) - 3) // 2 + 1
        out = torch.full((nseq * To, d), float("nan"), dtype=torch.float32, device="cuda")
        xd = torch.from_numpy(x).cuda()
        t_out = dev.run(xd.data_ptr(), T, nseq, nm, out.data_ptr(), xscale=2.0)
        torch.cuda.synchronize()
        assert t_out == To
        y = out.cpu().numpy()
        pp = {k: (v.reshape(v.shape[0], -1) if k.startswith("pw_w") else v) for k, v in p.items()}
        ref = np.concatenate([2.0 * E.subsampling(x[s * T:(s + 1) * T], pp, causal) for s in range(nseq)])
        err = np.abs(y - ref)
        rms = float(np.sqrt((ref ** 2).mean()))
        say(f"  max |y - ref| {err.max():.3g} (rms ref {rms:.3g}), worst / (|ref| + rms) "
            f"{(err / (np.abs(ref) + rms)).max():.3g}")
        assert (err <= 5e-6 * (np.abs(ref) + rms)).all()
    finally:
        dev.close()


@pytest.mark.parametrize("mode", [M.INT8ACT, M.QMAT], ids=["int8act", "qmat"])
def test_encoder_layer_in_other_numerics(gpu, mode):
    """Each product of the layer runs in the current numerics mode (the
    f32 position projection stays f32, as the reference keeps relk_w): in
    INT8ACT (Q8_0: per-row int8 activations) the layer stays within the int8
    path's budget of the EXACT layer (relative L2 < 1e-2; the output is a
    layer norm, O(1)); QMAT numerics runs Q8_0 products EXACT (qmat.c's
    dispatch takes the int8 path for INT8/INT4 weights only), so its output
    has the EXACT layer's bits."""
    import torch
    say("encoder layer, numerics", mode)
    d, H, f, k, T, nseq = 256, 4, 512, 9, 40, 2
    p = make_params(14, d, f, k, True, True)
    dev = M.DeviceEncoderLayer(gpu, p, M.Q8_0)
    try:
        x = np.random.default_rng(15).standard_normal((nseq * T, d)).astype(np.float32)
        ped = torch.from_numpy(E.pos_emb(T, d).astype(np.float32)).cuda()
        ys = {}
        for m in (M.EXACT, mode):
            assert gpu.set_numerics(m) == m
            xd = torch.from_numpy(x).cuda()
            dev.run(xd.data_ptr(), T, nseq, ped.data_ptr(), d, H, k, 0)
            torch.cuda.synchronize()
            ys[m] = xd.cpu().numpy()
        gpu.set_numerics(M.EXACT)
        y, ex = ys[mode], ys[M.EXACT]
        assert np.isfinite(y).all()
        if mode == M.QMAT:
            assert np.array_equal(y.view(np.uint32), ex.view(np.uint32))
        else:
            rel = float(np.linalg.norm(y - ex) / np.linalg.norm(ex))
            say(f"  relative L2 vs EXACT {rel:.3g}")
            assert 0 < rel < 1e-2
    finally:
        gpu.set_numerics(M.EXACT)
        dev.close()
