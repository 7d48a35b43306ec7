#!/usr/bin/env python3
"""bench.py — throughput of the MI355X linear-layer backend on the benchmark's shapes.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

A step is one pass over the FastConformer-0.6B encoder linear set at
M = 8 segments x 750 frames = 6000 rows (benchmark config 2's shapes:
1024->4096, 4096->1024 and five 1024->1024 for Q, K, V, out, pos), every
weight Q8_0 (the headline metric), EXACT numerics (the default). Inputs are
resident in HBM before the timed region; the products go through the
library's device entry points the way an encoder layer calls them
(src/encoder.c): the FFN pair through qffn_dev (the first product prepares
the intermediate for the second), q/k/v through qqkv_dev (one preparation of
their shared input), out and pos through qgemm_dev (preparation + product).
`value` = dense-equivalent 2*M*N*K operations per second, summed over the
step, in TOPS.

Also reported (not `value`): per-kernel roofline fractions, the same step in
INT8ACT numerics (int8 activations on the i8 MFMA, against 5.0 POP/s), each of
Q2_K, Q3_K, Q4_K, Q5_K and Q6_K at benchmark config 4's M = 12000 shapes, decoder GEMVs (config 3) in HBM GB/s with >= 512
MB of rotating weight copies (defeats the 256 MB MALL), timed as one HIP graph
of all the launches (kernel_us; call_us = the same launches issued one by one
from the host), products of 16 to 750 rows on one stream (qgemm_dev calls: few tiles,
K split over workgroups), the f32-weight GEMM, the relative-position attention core at T = 750
(16 segments as in benchmark config 5, d 1024, 8 heads; full and chunked-limited [70, 13] windows;
useful flops = 6 * dk per visible (row, key) pair, against the 157.3 TFLOP/s
fp32 MFMA peak; full attention forms its products on the f16 MFMA from split
hi + lo operands, three f16 products per f32 one), and the reference CPU path timed on this host (ingot dequant, compiled from
the reference's sources, + OpenBLAS sgemm, as src/weights.c:103-114 +
src/backend.c:79 do).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mynah-asr_amd"))

PEAK_FP16 = 2500.0  # TFLOP/s dense (MI355X)
PEAK_HBM = 8000.0   # GB/s
PEAK_INT8 = 5000.0  # TOPS dense int8 (MI355X)
METRIC = "Q8_0/Q4_K GEMM TOPS & % roofline at FastConformer-0.6B shapes; GEMV HBM GB/s"

ENC_SHAPES = [("ffn1", 1024, 4096), ("ffn2", 4096, 1024), ("q", 1024, 1024), ("k", 1024, 1024),
              ("v", 1024, 1024), ("out", 1024, 1024), ("pos", 1024, 1024)]
KQ_SHAPES = [("ffn1", 1024, 4096), ("ffn2", 4096, 1024), ("q", 1024, 1024), ("k", 1024, 1024),
             ("v", 1024, 1024), ("out", 1024, 1024)]
GEMV_SHAPES = [(1024, 1024), (1024, 4096), (4096, 1024), (1024, 16384)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def roof_time_s(flops: float, nbytes: float) -> float:
    return max(flops / (PEAK_FP16 * 1e12), nbytes / (PEAK_HBM * 1e9))


class Bench:
    def __init__(self, lib, torch):
        self.lib, self.torch = lib, torch
        self.stream = torch.cuda.Stream()  # default priority
        self.sp = self.stream.cuda_stream

    def sync(self):
        self.torch.cuda.synchronize()

    def dev(self, a: np.ndarray):
        return self.torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def empty(self, *shape):
        return self.torch.empty(shape, dtype=self.torch.float32, device="cuda")

    def kernel_ms(self, dw, M: int, x, y, reps: int) -> float:
        """Average duration of the GEMM kernel alone (input prepared once),
        HIP events on the stream the kernel runs on."""
        torch = self.torch
        dw.prep(x.data_ptr(), M, self.sp)
        dw.gemm_prepped(y.data_ptr(), M, 0, self.sp)  # warm
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(self.stream)
        for _ in range(reps):
            dw.gemm_prepped(y.data_ptr(), M, 0, self.sp)
        e1.record(self.stream)
        self.sync()
        return e0.elapsed_time(e1) / reps


def gemm_row(name, qt, M, k, n, ms, M_):
    flops = 2.0 * M * n * k
    nbytes = 4.0 * M * k + M_.weight_bytes(qt, n, k) + 4.0 * M * n
    t = ms * 1e-3
    return {"gemm": name, "M": M, "k": k, "n": n, "format": M_.NAMES[qt], "kernel_us": round(ms * 1e3, 2),
            "tflops": round(flops / t / 1e12, 2), "gbps": round(nbytes / t / 1e9, 1),
            "roofline_frac": round(roof_time_s(flops, nbytes) / t, 4),
            "mfma_frac": round(flops / t / 1e12 / PEAK_FP16, 4)}


def run_encoder_set(B, M_, qt, M, shapes, steps, warmup, seed0):
    lib = B.lib
    ws, dws, xs, ys = [], [], {}, []
    for i, (name, k, n) in enumerate(shapes):
        w = M_.Weight.make(lib, qt, lib.randn(seed0 + i, 0.02, (n, k)))
        ws.append(w)
        dws.append(M_.DeviceWeight(lib, w))
        if k not in xs:
            xs[k] = B.dev(lib.randn(1, 1.0, (M, k)))
        ys.append(B.empty(M, n))
    B.sync()

    idx = {name: i for i, (name, _, _) in enumerate(shapes)}
    fused = {"ffn1", "ffn2"} <= idx.keys()
    qkv = {"q", "k", "v"} <= idx.keys()

    def step():
        # the encoder layer's call pattern (src/encoder.c): the FFN through the
        # fused entry point, q/k/v on one prepared input, the rest one by one
        done = set()
        if fused:
            i1, i2 = idx["ffn1"], idx["ffn2"]
            M_.ffn_dev(lib, dws[i1], dws[i2], xs[shapes[i1][1]].data_ptr(), ys[i2].data_ptr(), M, B.sp)
            done |= {i1, i2}
        if qkv:
            ii = [idx["q"], idx["k"], idx["v"]]
            M_.qkv_dev(lib, [dws[i] for i in ii], xs[shapes[ii[0]][1]].data_ptr(), [ys[i].data_ptr() for i in ii],
                       M, B.sp)
            done |= set(ii)
        for i, (dw, (name, k, n), y) in enumerate(zip(dws, shapes, ys)):
            if i not in done:
                dw.gemm(xs[k].data_ptr(), y.data_ptr(), M, 0, B.sp)

    for _ in range(warmup):
        step()
    B.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    B.sync()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / steps
    flops = sum(2.0 * M * n * k for _, k, n in shapes)
    rows = []
    for dw, (name, k, n), y in zip(dws, shapes, ys):
        ms = B.kernel_ms(dw, M, xs[k], y, reps=10)
        rows.append(gemm_row(name, qt, M, k, n, ms, M_))
    for dw in dws:
        dw.close()
    return ms_step, flops, rows


def run_int8act(B, M_, M):
    """INT8ACT numerics: the qmat INT8 encoder set at M = 6000 (the reference's
    own int8 GEMM, qmat.c:464-500, 598-643: int8 MFMA, one int32 sum per
    output), the Q8_0 encoder set at M = 6000 (per-row int8
    activations, qmat.c:186-202) and the Q4_K / Q5_K layer sets at config 4's
    M = 12000 (per-super-block int8 activations, ingot's int8 path,
    third_party/ingot/src/kernels.c:719-750, 1649-1795). The block formats'
    products run on the f16 MFMA with the int8 values as single exact terms;
    the fractions are given against both the int8 (5.0 POP/s) and the f16
    (2.5 PF) peak."""
    lib = B.lib
    out = {}
    lib.set_numerics(1)
    try:
        for name, qt, MM, shapes, seed in (("int8act_int8_m6000", M_.INT8, M, ENC_SHAPES, 0),
                                           ("int8act_q8_0_m6000", M_.Q8_0, M, ENC_SHAPES, 0),
                                           ("int8act_q4_k_m12000", M_.Q4_K, 12000, KQ_SHAPES, 100),
                                           ("int8act_q5_k_m12000", M_.Q5_K, 12000, KQ_SHAPES, 100)):
            log(f"[bench] {name}")
            ms8, fl8, rows8 = run_encoder_set(B, M_, qt, MM, shapes, 5, 2, seed)
            tops = fl8 / (ms8 * 1e-3) / 1e12
            for r in rows8:
                r["int8_mfma_frac"] = round(r["tflops"] / PEAK_INT8, 4)
            out[name] = {"tops": round(tops, 2), "ms_per_step": round(ms8, 4),
                         "int8_mfma_frac": round(tops / PEAK_INT8, 4), "f16_mfma_frac": round(tops / PEAK_FP16, 4),
                         "rows": rows8}
    finally:
        lib.set_numerics(0)
    out["int8act_note"] = ("int8 activations (Q8_0: per row as qmat.c:186-202; K-quants: per 256-element "
                           "super-block as ingot's int8 path), exact integer sums, f32 combine; outputs match "
                           "that path (ingot's 5e-3 budget against the f32 product), not the f32 product")
    return out


def run_config5(B, M_, reps=3):
    """The parts of one FastConformer-0.6B encoder layer this build runs, at
    benchmark config 5's batch (16 segments x 750 frames = 12000 rows, d 1024,
    FFN 4096, 8 heads; src/encoder.c:901-946 for the layer's order), Q8_0
    weights, EXACT numerics, one stream: the two macaron FFNs (qffn_dev),
    q/k/v (qqkv_dev), the attention output projection, the pos projection
    (2T-1 = 1499 rows of the sinusoidal table: the reference forms it per
    segment, 16 x 1499 rows; one product over the 1499 shared rows gives the
    same values), the relative-position attention core over the 16 segments,
    and the conv module's pointwise convolutions (1024->2048 before the GLU,
    1024->1024 after). Each call is timed with HIP events on the stream
    (preparation included), for the per-GEMM roofline fractions; the whole
    forward is run_config5_forward's."""
    torch, lib = B.torch, B.lib
    Mr, T, nseq, d, H = 12000, 750, 16, 1024, 8
    mk = lambda seed, n, k: M_.DeviceWeight(lib, M_.Weight.make(lib, M_.Q8_0, lib.randn(seed, 0.02, (n, k))))
    W = {"ffa1": mk(500, 4096, d), "ffa2": mk(501, d, 4096), "ffb1": mk(502, 4096, d), "ffb2": mk(503, d, 4096),
         "q": mk(504, d, d), "k": mk(505, d, d), "v": mk(506, d, d), "out": mk(507, d, d), "pos": mk(508, d, d),
         "pw1": mk(509, 2 * d, d), "pw2": mk(510, d, d)}
    x = B.dev(lib.randn(511, 1.0, (Mr, d)))
    pe = B.dev(lib.randn(512, 1.0, (2 * T - 1, d)))
    y, q, kk, v, ctx = (B.empty(Mr, d) for _ in range(5))
    rk = B.empty(2 * T - 1, d)
    y2 = B.empty(Mr, 2 * d)
    bu, bv = B.dev(lib.randn(513, 0.1, (d,))), B.dev(lib.randn(514, 0.1, (d,)))
    sp = B.sp
    steps = [
        ("ffn_a (1024->4096->1024)", 2 * Mr * 2 * 4096 * d,
         lambda: M_.ffn_dev(lib, W["ffa1"], W["ffa2"], x.data_ptr(), y.data_ptr(), Mr, sp)),
        ("q/k/v (3 x 1024->1024)", 3 * 2 * Mr * d * d,
         lambda: M_.qkv_dev(lib, [W["q"], W["k"], W["v"]], x.data_ptr(), [q.data_ptr(), kk.data_ptr(), v.data_ptr()],
                            Mr, sp)),
        ("pos (1499 x 1024->1024)", 2 * (2 * T - 1) * d * d,
         lambda: W["pos"].gemm(pe.data_ptr(), rk.data_ptr(), 2 * T - 1, 0, sp)),
        ("rel-pos attention core (16 x 750)", attn_flops(T, H, d // H, -1, 0, nseq),
         lambda: M_.relpos_attention_dev(lib, q.data_ptr(), kk.data_ptr(), v.data_ptr(), rk.data_ptr(), bu.data_ptr(),
                                         bv.data_ptr(), ctx.data_ptr(), T, d, H, -1, 0, nseq, sp)),
        ("out (1024->1024)", 2 * Mr * d * d, lambda: W["out"].gemm(ctx.data_ptr(), y.data_ptr(), Mr, 0, sp)),
        ("conv pw1 (1024->2048)", 2 * Mr * 2 * d * d, lambda: W["pw1"].gemm(x.data_ptr(), y2.data_ptr(), Mr, 0, sp)),
        ("conv pw2 (1024->1024)", 2 * Mr * d * d, lambda: W["pw2"].gemm(x.data_ptr(), y.data_ptr(), Mr, 0, sp)),
        ("ffn_b (1024->4096->1024)", 2 * Mr * 2 * 4096 * d,
         lambda: M_.ffn_dev(lib, W["ffb1"], W["ffb2"], x.data_ptr(), y.data_ptr(), Mr, sp)),
    ]
    for _, _, f in steps:
        f()
    B.sync()
    rows, total = [], 0.0
    for name, fl, f in steps:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(B.stream)
        for _ in range(reps):
            f()
        e1.record(B.stream)
        B.sync()
        us = e0.elapsed_time(e1) / reps * 1e3
        total += us
        peak = PEAK_FP32 if "attention" in name else PEAK_FP16
        rows.append({"step": name, "us": round(us, 1), "gflop": round(fl / 1e9, 1),
                     "tflops": round(fl / us / 1e6, 1), "mfma_frac": round(fl / us / 1e6 / peak, 4),
                     "peak": "fp32 MFMA 157.3" if "attention" in name else "f16 MFMA 2500"})
    # the whole layer as one back-to-back sequence
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(B.stream)
    for _ in range(reps):
        for _, _, f in steps:
            f()
    e1.record(B.stream)
    B.sync()
    seq_us = e0.elapsed_time(e1) / reps * 1e3
    for w in W.values():
        w.close()
    fwd_ms = 24 * seq_us / 1e3
    return {"rows": Mr, "segments": nseq, "frames": T, "layers": 24, "format": "Q8_0", "numerics": "EXACT",
            "steps": rows, "layer_us_sum_of_steps": round(total, 1), "layer_us_sequence": round(seq_us, 1),
            "products_attention_24_layers_ms": round(fwd_ms, 2),
            "note": "the products and attention core of one layer, step by step; the whole encoder forward "
                    "(subsampling, layer norms, GLU, depthwise conv, residuals): config5_forward"}


def run_config5_forward(B, M_, reps=3):
    """BASELINE config 5 end to end, on the device: a random-init
    FastConformer-0.6B encoder (24 layers, d_model 1024, 8 heads, FFN 4096
    macaron, depthwise conv kernel 9, dw_striding 8x subsampling with 256
    channels) over 16 segments of 60 s (6000 log-mel frames of 80 features,
    N(0, 1)), all 16 segments as one batch of 12000 encoder rows: the
    subsampling (mynah_asr_hip_subsampling_dev), then the 24 layers
    (mynah_asr_hip_encoder_layer_dev; src/encoder.c:948-1010 forward_batch
    without its final projection). Linears Q8_0 (EXACT numerics), the
    position projection and the subsampling's pointwise convs and linear f32;
    no linear biases (the reference's fused-FFN path), the folded batch norm,
    'same' conv padding, full attention, xscale 1. Every layer has its own
    weights (624 MB resident). Timed with HIP events on the bench stream;
    RTF = forward time / 960 s of audio."""
    torch, lib = B.torch, B.lib
    nseq, Tm, nm, d, H, f, k, C, L = 16, 6000, 80, 1024, 8, 4096, 9, 256, 24
    r = np.random.default_rng(600)
    g = lambda *shape: r.standard_normal(shape).astype(np.float32)
    t0 = time.perf_counter()
    layers = []
    for li in range(L):
        sd = 1000 + 100 * li
        p = {"relk_w": lib.randn(sd + 9, 0.02, (d, d)), "bias_u": 0.1 * g(d), "bias_v": 0.1 * g(d),
             "dw_w": 0.3 * g(d, k), "cnorm_scale": 1 + 0.1 * g(d), "cnorm_shift": 0.1 * g(d)}
        for n in ("ff1", "att", "conv", "ff2", "out"):
            p[f"ln_{n}_w"], p[f"ln_{n}_b"] = 1 + 0.1 * g(d), 0.1 * g(d)
        for j, (n, shape) in enumerate((("ff1_w1", (f, d)), ("ff1_w2", (d, f)), ("ff2_w1", (f, d)), ("ff2_w2", (d, f)),
                                        ("q_w", (d, d)), ("k_w", (d, d)), ("v_w", (d, d)), ("o_w", (d, d)),
                                        ("pw1_w", (2 * d, d)), ("pw2_w", (d, d)))):
            p[n] = lib.randn(sd + j, 0.02, shape)
        layers.append(M_.DeviceEncoderLayer(lib, p, M_.Q8_0))
    Fo = nm
    for _ in range(3):
        Fo = (Fo + 2 - 3) // 2 + 1
    ssp = {"conv_in_w": 0.3 * g(C, 1, 3, 3), "conv_in_b": 0.1 * g(C), "lin_w": lib.randn(1999, 0.02, (d, C * Fo)),
           "lin_b": 0.1 * g(d)}
    for i in range(2):
        ssp[f"dw_w{i}"], ssp[f"dw_b{i}"] = 0.3 * g(C, 1, 3, 3), 0.1 * g(C)
        ssp[f"pw_w{i}"], ssp[f"pw_b{i}"] = lib.randn(1998 - i, 0.05, (C, C)), 0.1 * g(C)
    ss = M_.DeviceSubsampling(lib, ssp, 0)
    setup_s = time.perf_counter() - t0
    mel = B.dev(lib.randn(1997, 1.0, (nseq * Tm, nm)))
    T = (Tm - 1) // 2 + 1
    T = (T - 1) // 2 + 1
    T = (T - 1) // 2 + 1
    # the relative positional embedding (encoder.c:201-212), formed on the host as the reference does
    pos = (T - 1 - np.arange(2 * T - 1, dtype=np.float64))[:, None]
    fr = pos * np.power(10000.0, -2.0 * np.arange(d // 2, dtype=np.float64)[None, :] / d)
    pe_h = np.empty((2 * T - 1, d), np.float32)
    pe_h[:, 0::2], pe_h[:, 1::2] = np.sin(fr), np.cos(fr)
    pe = B.dev(pe_h)
    x = B.empty(nseq * T, d)
    sp = B.sp

    def forward():
        t_out = ss.run(mel.data_ptr(), Tm, nseq, nm, x.data_ptr(), 1.0, sp)
        assert t_out == T
        for ly in layers:
            ly.run(x.data_ptr(), T, nseq, pe.data_ptr(), d, H, k, 0, -1, 0, sp)

    forward()
    B.sync()
    ev = lambda: torch.cuda.Event(enable_timing=True)
    e0, e1, e2 = ev(), ev(), ev()
    e0.record(B.stream)
    for _ in range(reps):
        forward()
    e1.record(B.stream)
    B.sync()
    fwd_ms = e0.elapsed_time(e1) / reps
    # the subsampling alone and one layer alone, for the split
    e0.record(B.stream)
    for _ in range(reps):
        ss.run(mel.data_ptr(), Tm, nseq, nm, x.data_ptr(), 1.0, sp)
    e1.record(B.stream)
    for _ in range(reps):
        layers[0].run(x.data_ptr(), T, nseq, pe.data_ptr(), d, H, k, 0, -1, 0, sp)
    e2.record(B.stream)
    B.sync()
    ss_ms, layer_ms = e0.elapsed_time(e1) / reps, e1.elapsed_time(e2) / reps
    finite = bool(torch.isfinite(x).all().item())
    for ly in layers:
        ly.close()
    ss.close()
    return {"segments": nseq, "mel_frames": Tm, "encoder_frames": T, "rows": nseq * T, "layers": L,
            "format": "Q8_0", "numerics": "EXACT", "forward_ms": round(fwd_ms, 2),
            "subsampling_ms": round(ss_ms, 3), "layer_ms": round(layer_ms, 3),
            "rtf": float(f"{fwd_ms / 1e3 / (nseq * 60.0):.3g}"), "output_finite": finite,
            "weights_setup_s": round(setup_s, 1)}


def read_floor_us(B, nbytes, copies):
    """The one-launch floor for nbytes: a plain streaming read of that many
    bytes (mynah_asr_hip_read_floor_dev, no compute), over `copies` distinct
    buffers in turn, replayed from one HIP graph as the GEMVs are."""
    torch = B.torch
    try:
        buf = torch.empty(copies * nbytes // 4, dtype=torch.float32, device="cuda")
        buf.zero_()
        g = torch.cuda.CUDAGraph()
        cs = torch.cuda.Stream()
        with torch.cuda.graph(g, stream=cs):
            for i in range(copies):
                B.lib.read_floor(buf.data_ptr() + i * nbytes, nbytes, cs.cuda_stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(cs):
            g.replay()
            B.sync()
            e0.record(cs)
            for _ in range(3):
                g.replay()
            e1.record(cs)
        B.sync()
        us = e0.elapsed_time(e1) / (3 * copies) * 1e3
        del g, buf
        return round(us, 2)
    except Exception as ex:
        log(f"[bench] read floor not measured ({ex})")
        return None


floor = {}


def run_gemv(B, M_, qt, n, k, Ms, min_bytes=512 << 20, max_copies=512):
    lib = B.lib
    w = M_.Weight.make(lib, qt, lib.randn(0, 0.02, (n, k)))
    wb = M_.weight_bytes(qt, n, k)
    copies = int(min(max_copies, max(4, -(-min_bytes // wb))))
    dws = [M_.DeviceWeight(lib, w) for _ in range(copies)]
    out = []
    torch = B.torch
    for M in Ms:
        x = B.dev(lib.randn(1, 1.0, (M, k)))
        y = B.empty(M, n)
        # the full call, as a decoder step issues it: for M <= 16 it is one
        # kernel (the GEMV splits x in registers), every copy in turn
        for dw in dws[:4]:
            dw.gemm(x.data_ptr(), y.data_ptr(), M, 0, B.sp)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(B.stream)
        for dw in dws:
            dw.gemm(x.data_ptr(), y.data_ptr(), M, 0, B.sp)
        e1.record(B.stream)
        B.sync()
        call_ms = e0.elapsed_time(e1) / copies
        # the same launches captured once in a HIP graph and replayed: the
        # GPU-side time per GEMV without the host's launch cost in the way
        kms = call_ms
        try:
            g = torch.cuda.CUDAGraph()
            cs = torch.cuda.Stream()
            with torch.cuda.graph(g, stream=cs):
                for dw in dws:
                    dw.gemm(x.data_ptr(), y.data_ptr(), M, 0, cs.cuda_stream)
            with torch.cuda.stream(cs):  # replay on the stream the events mark
                g.replay()
                B.sync()
                e0.record(cs)
                for _ in range(3):
                    g.replay()
                e1.record(cs)
            B.sync()
            kms = e0.elapsed_time(e1) / (3 * copies)
            del g
        except Exception as ex:  # keep the stream figure
            log(f"[bench] graph capture failed ({ex}); GEMV time from stream launches")
        nbytes = wb + 4.0 * M * k + 4.0 * M * n
        fus = floor.get(int(nbytes) // 16 * 16)
        if fus is None:
            fus = floor[int(nbytes) // 16 * 16] = read_floor_us(B, int(nbytes) // 16 * 16, copies)
        out.append({"format": M_.NAMES[qt], "M": M, "k": k, "n": n, "copies": copies,
                    "read_floor_us": fus, "kernel_vs_floor": round(fus / (kms * 1e3), 3) if fus else None,
                    "rotated_mb": round(copies * wb / 2**20), "kernel_us": round(kms * 1e3, 2),
                    "call_us": round(call_ms * 1e3, 2),
                    "kernel_gbps": round(nbytes / (kms * 1e-3) / 1e9, 1),
                    "kernel_hbm_frac": round(nbytes / (kms * 1e-3) / 1e9 / PEAK_HBM, 4)})
    for dw in dws:
        dw.close()
    return out


def host_cpu() -> dict:
    """The host's CPU model, the logical CPUs this process may use, and the
    physical cores among them (from /proc/cpuinfo)."""
    model, cores, allowed, ids = "unknown", set(), sorted(os.sched_getaffinity(0)), {}
    try:
        phys = core = proc = None
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "processor":
                proc = int(v)
            elif k == "model name":
                model = v
            elif k in ("vendor_id", "cpu family", "model", "stepping") and k not in ids:
                ids[k] = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
                if proc in allowed:
                    cores.add((phys, core))
    except OSError:
        pass
    # the model name a VM reports can be bare ("AMD EPYC"); family/model/stepping pin the part
    cpuid = " ".join(f"{k}={v}" for k, v in ids.items())
    return {"model": model, "cpuid": cpuid, "logical_cpus": len(allowed), "physical_cores": len(cores) or None}


def _median_time(fn, budget_s, max_reps=5, min_reps=1):
    t_all, start = [], time.perf_counter()
    while len(t_all) < max_reps and (len(t_all) < min_reps or time.perf_counter() - start < budget_s):
        t0 = time.perf_counter()
        fn()
        t_all.append(time.perf_counter() - t0)
    return float(np.median(t_all)), len(t_all)


def cpu_baseline(M_, lib, seconds_budget=20.0):
    """The reference CPU path on this host's cores, on bounded samples of the
    benchmark's workloads. `value`: the Q8_0 encoder set at M = 6000 as the
    reference runs GGUF weights: ingot decodes the blocks to f32 once
    (src/weights.c:103-114; oracle/_ref is the reference's ingot sources
    compiled unmodified, or the oracle's restatement when _ref is absent),
    then every product is cblas_sgemm (src/backend.c:79; numpy's OpenBLAS).
    `variants`: the same at one thread; qmat's INT8 large-T default (per-call
    dequant + sgemm, src/qmat.c:644-650) at config 1; the reference's own
    SIMD CPU GEMMs straight off the blocks (ingot_q8_0_matmat,
    ingot_q4_k_matmat_exact, and the int8-activation ingot_q4_k_matmat,
    third_party/ingot/src/kernels.c:1758-1795, 2392-2400; built with its x86
    SIMD flags) at config 1; and the decoder GEMVs (config 3, M = 1) as the
    reference runs them (f32 weights through sgemv) and through ingot's Q8_0
    matvec, with the AED step's linears summed."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    kind = "reference"
    if O.IngotRef.available():
        dec = O.IngotRef()
        decoder = "oracle/_ref ingot_dequant (reference sources)"
    else:
        dec = O.Oracle()
        kind = "port"
        decoder = "oracle restatement of ingot dequant"
    host = host_cpu()
    try:
        from threadpoolctl import threadpool_info, threadpool_limits
        threads = max([i.get("num_threads", 1) for i in threadpool_info()
                       if i.get("user_api") == "blas"] or [1])
    except Exception:
        threadpool_limits = None
        threads = host["logical_cpus"]
    M = 6000
    wd, raws = {}, {}
    for i, (name, k, n) in enumerate(ENC_SHAPES):
        raw = lib.quantize(M_.Q8_0, lib.randn(i, 0.02, (n, k)))
        raws[name] = raw
        wd[name] = dec.dequant(O.Q8_0, raw, n * k).reshape(n, k)
    xs = {k: lib.randn(1, 1.0, (M, k)) for k in (1024, 4096)}

    def step(rows):
        for name, k, n in ENC_SHAPES:
            np.matmul(xs[k][:rows], wd[name].T)

    step(750)  # warm the BLAS pool
    flops = sum(2.0 * M * n * k for _, k, n in ENC_SHAPES)
    med, reps = _median_time(lambda: step(M), seconds_budget * 0.4)
    variants = []
    if threadpool_limits is not None:
        with threadpool_limits(limits=1, user_api="blas"):
            med1, _ = _median_time(lambda: step(M), 0.0, max_reps=1)
        variants.append({"variant": "ingot dequant once + OpenBLAS sgemm, encoder set M=6000", "threads": 1,
                         "ms": round(med1 * 1e3, 1), "tops": round(flops / med1 / 1e12, 4)})
    # config 1: Q8_0 M=750, 1024 -> 4096
    c1x = xs[1024][:750]
    c1f = 2.0 * 750 * 4096 * 1024
    raw1, wd1 = raws["ffn1"], wd["ffn1"]
    q8, s8 = O.Oracle().qmat_quantize_int8(wd1)
    orc = O.Oracle()

    def qmat_default():   # qmat.c:644-650: dequant_row per call (one thread), then sgemm
        np.matmul(c1x, orc.qmat_dequant(1, q8, s8, 4096, 1024).T)

    t, _ = _median_time(qmat_default, 2.0, max_reps=3)
    variants.append({"variant": "qmat INT8 per-call dequant + OpenBLAS sgemm (qmat.c:644-650), config 1 M=750 "
                                "1024->4096 (dequant: oracle restatement, one thread)", "threads": int(threads),
                     "kind": "port", "ms": round(t * 1e3, 2), "gflops": round(c1f / t / 1e9, 1)})
    gemv_cpu = []
    if os.path.exists(O.REF_AVX2_PATH):
        R = O.IngotRef(O.REF_AVX2_PATH)
        R.set_threads(host["logical_cpus"])
        raw4 = lib.quantize(M_.Q4_K, lib.randn(0, 0.02, (4096, 1024)))
        for name, raw, label in (("ingot_q8_0_matmat", raw1, "Q8_0"), ("ingot_q4_k_matmat_exact", raw4, "Q4_K"),
                                 ("ingot_q4_k_matmat", raw4, "Q4_K int8 activations")):
            R.kernel(name, raw, 4096, 1024, c1x[:64])
            t, _ = _median_time(lambda: R.kernel(name, raw, 4096, 1024, c1x), 3.0, max_reps=3)
            variants.append({"variant": f"{name} ({label}), config 1 M=750 1024->4096", "kind": "reference",
                             "threads": host["logical_cpus"], "ms": round(t * 1e3, 2),
                             "gflops": round(c1f / t / 1e9, 1)})
        # decoder GEMVs: M = 1 (ingot's Q8_0 matvec) and M = 4, 16 (its matmat)
        for k, n in [(s[0], s[1]) for s in GEMV_SHAPES]:
            raw = lib.quantize(M_.Q8_0, lib.randn(0, 0.02, (n, k)))
            wf = dec.dequant(O.Q8_0, raw, n * k).reshape(n, k)
            xg = lib.randn(1, 1.0, (16, k))
            for Mg in (1, 4, 16):
                t_s, _ = _median_time(lambda: np.matmul(xg[:Mg], wf.T), 0.3, max_reps=20, min_reps=5)
                qb = M_.weight_bytes(M_.Q8_0, n, k) + 4.0 * Mg * (k + n)
                row = {"M": Mg, "k": k, "n": n, "sgemv_f32_us": round(t_s * 1e6, 1)}
                # ingot's own thread split (a persistent pool: no thread
                # creation per call); M = 1 is its serial matvec at any count
                for th in (1, host["logical_cpus"]):
                    R.set_threads(th)
                    R.kernel("ingot_q8_0_matmat", raw, n, k, xg[:Mg])
                    t_i, _ = _median_time(lambda: R.kernel("ingot_q8_0_matmat", raw, n, k, xg[:Mg]), 0.3,
                                          max_reps=20, min_reps=5)
                    tag = "1t" if th == 1 else f"{th}t"
                    row[f"ingot_q8_0_{tag}_us"] = round(t_i * 1e6, 1)
                    row[f"ingot_q8_0_{tag}_gbps"] = round(qb / t_i / 1e9, 2)
                gemv_cpu.append(row)
        R.set_threads(host["logical_cpus"])
    # the AED step's linears at M = 1 through sgemv (4 layers of 6 x 1024^2 +
    # 1024x4096 + 4096x1024, then the 16384-row head): the CPU floor of a step
    sg = {(g["k"], g["n"]): g["sgemv_f32_us"] for g in gemv_cpu if g["M"] == 1}
    aed_us = None
    if sg:
        aed_us = round(4 * (6 * sg[(1024, 1024)] + sg[(1024, 4096)] + sg[(4096, 1024)]) + sg[(1024, 16384)], 1)
    return {"value": round(flops / med / 1e12, 4), "unit": "TOPS", "cores": int(threads),
            "kind": kind, "host": host,
            "sample": f"{reps} whole steps (7 GEMMs at M=6000, median {med*1e3:.0f} ms): "
                      f"{decoder} once + OpenBLAS sgemm per product, {threads} BLAS threads on "
                      f"{host['logical_cpus']} logical CPUs ({host['physical_cores']} physical cores) of {host['model']} ({host['cpuid']})",
            "sample_short": f"{reps} steps (7 GEMMs, M=6000): ingot dequant once + OpenBLAS sgemm, "
                            f"{threads} threads, {host['model']} ({host['cpuid']})",
            "variants": variants, "gemv": gemv_cpu,
            "aed_step_linears_sgemv_us": aed_us}


PEAK_FP32 = 157.3  # TFLOP/s dense fp32 MFMA (MI355X)


def headline_summary(details: dict, rows: list) -> dict:
    """A few figures from the detail tree, small enough for the contract line."""
    s = {"gemm_us": {r["gemm"]: round(r["kernel_us"], 1) for r in rows if r["gemm"] in ("ffn1", "ffn2", "q")}}
    if "gemv_hbm_frac_mean_large" in details:
        s["gemv_hbm_frac_large"] = details["gemv_hbm_frac_mean_large"]
        g1 = [g for g in details["gemv"] if g["format"] == "Q8_0" and g["M"] == 1 and g["n"] == 16384]
        if g1:
            s["gemv_q8_0_1024x16384_m1_us"] = g1[0]["kernel_us"]
    if "aed_decoder" in details:
        s["aed_us_per_pos"] = details["aed_decoder"].get("forced_us_per_position")
    if "vendor_gemm" in details:
        v = {r["gemm"].split()[0]: r["us"] for r in details["vendor_gemm"]
             if r["dtype"] == "f16" and r["gemm"] in ("ffn2 volume", "ffn1 volume")}
        if v:
            s["hipblaslt_f16_same_mfma_us"] = v
    if "gemm_small_m" in details:
        c1 = [r for r in details["gemm_small_m"] if r.get("M") == 750 and r.get("k") == 1024
              and r.get("n") == 4096]
        if c1:
            s["config1_us_per_call"] = c1[0].get("call_us")
    if "config5_forward" in details:
        s["config5_rtf"] = details["config5_forward"]["rtf"]
    if "int8act_int8_m6000" in details:
        s["int8_qmat_set_tops"] = details["int8act_int8_m6000"]["tops"]
    return s


def attn_flops(T, H, dk, left, right, nseq):
    """Useful flops of the attention core: per (row, visible key) pair, the
    content and position dot products and the context update, 2*dk each."""
    t = np.arange(T)
    if left < 0:
        pairs = T * T
    else:
        chunk = right + 1
        lc = left // chunk
        pairs = int((np.minimum((t // chunk + 1) * chunk, T) - np.maximum((t // chunk - lc) * chunk, 0)).sum())
    return 6.0 * dk * pairs * H * nseq


def run_small_m(B, M_, reps=50):
    """Products of few rows on one stream (the streaming encoder's chunks, one
    segment's out / pos products, the decoder's cross K/V): qgemm_dev calls
    (preparation + product, K split over workgroups where the product has few
    tiles), HIP events on the stream, Q8_0 weights."""
    torch = B.torch
    lib = B.lib
    out = []
    for (k, n) in [(1024, 1024), (4096, 1024), (1024, 4096)]:
        dw = M_.DeviceWeight(lib, M_.Weight.make(lib, M_.Q8_0, lib.randn(0, 0.02, (n, k))))
        for M in (16, 17, 64, 256, 750):
            x = B.dev(lib.randn(1, 1.0, (M, k)))
            y = B.empty(M, n)
            for _ in range(5):
                dw.gemm(x.data_ptr(), y.data_ptr(), M, 0, B.sp)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(B.stream)
            for _ in range(reps):
                dw.gemm(x.data_ptr(), y.data_ptr(), M, 0, B.sp)
            e1.record(B.stream)
            B.sync()
            us = e0.elapsed_time(e1) / reps * 1e3
            out.append({"M": M, "k": k, "n": n, "format": "Q8_0", "call_us": round(us, 2),
                        "tflops": round(2.0 * M * n * k / us / 1e6, 2)})
        dw.close()
    return out


def run_vendor_gemm(B, reps=50):
    """The vendor's plain GEMM (torch.matmul -> hipBLASLt) at the MFMA volume of
    this build's EXACT products: a plain f16 / bf16 GEMM with K doubled issues
    the same MFMA work as two f16 terms per useful product (ffn2: M=6000,
    K=2*4096, N=1024; ffn1: K=2*1024, N=4096), and the single-term shapes
    themselves. A calibration of what this box's MFMA sustains on these
    shapes, not a parity path (no rounding contract, no row stability)."""
    torch = B.torch
    out = []
    for name, (M, K, N) in (("ffn2 volume", (6000, 8192, 1024)), ("ffn1 volume", (6000, 2048, 4096)),
                            ("4096->1024 plain", (6000, 4096, 1024)), ("1024->4096 plain", (6000, 1024, 4096)),
                            ("config 1 volume", (750, 2048, 4096)), ("4096->1024 M=750 volume", (750, 8192, 1024))):
        for dt, dn in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
            g = torch.Generator(device="cuda").manual_seed(5)
            a = torch.randn(M, K, device="cuda", dtype=dt, generator=g)
            b = torch.randn(K, N, device="cuda", dtype=dt, generator=g)
            with torch.cuda.stream(B.stream):
                for _ in range(5):
                    c = a @ b
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(B.stream)
                for _ in range(reps):
                    c = a @ b
                e1.record(B.stream)
            B.sync()
            us = e0.elapsed_time(e1) / reps * 1e3
            tf = 2.0 * M * N * K / us / 1e6
            out.append({"gemm": name, "M": M, "K": K, "N": N, "dtype": dn, "us": round(us, 2),
                        "tflops": round(tf, 1), "mfma_frac": round(tf / PEAK_FP16, 4)})
            del a, b, c
    return out


def run_attention(B, M_, T=750, d=1024, H=8, nseq=16, reps=10):
    """The rel-pos attention core (src/encoder.c:315-410 / 220-313) on one
    layer's q, k, v of nseq segments, full and chunked-limited windows."""
    torch, lib = B.torch, B.lib
    q, k, v = (B.dev(lib.randn(300 + i, 1.0, (nseq, T, d))) for i in range(3))
    rk = B.dev(lib.randn(303, 1.0, (2 * T - 1, d)))
    bu, bv = B.dev(lib.randn(304, 0.1, (d,))), B.dev(lib.randn(305, 0.1, (d,)))
    ctx = B.empty(nseq, T, d)
    out = []
    for left, right in ((-1, 0), (70, 13)):
        def call():
            M_.relpos_attention_dev(lib, q.data_ptr(), k.data_ptr(), v.data_ptr(), rk.data_ptr(), bu.data_ptr(),
                                    bv.data_ptr(), ctx.data_ptr(), T, d, H, left, right, nseq, B.sp)
        call()
        B.sync()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(B.stream)
        for _ in range(reps):
            call()
        e1.record(B.stream)
        B.sync()
        ms = e0.elapsed_time(e1) / reps
        fl = attn_flops(T, H, d // H, left, right, nseq)
        out.append({"T": T, "d": d, "heads": H, "segments": nseq, "left": left, "right": right,
                    "kernel_us": round(ms * 1e3, 2), "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
                    "fp32_mfma_frac": round(fl / (ms * 1e-3) / 1e12 / PEAK_FP32, 4),
                    "products_on": "f32 MFMA" if left >= 0 else "f16 MFMA, split operands"})
    return out


def run_aed(B, M_, d=1024, H=8, ffn=4096, vocab=16384, n_layers=4, T=750, cap=64, qt=None):
    """The AED decoder on the device (src/decoder_aed.c:139-232) at benchmark
    config 3's shapes: greedy decoding of `cap` tokens after a 4-token prompt
    (a host read-back per token for the EOS check), and the same steps
    teacher-forced (no read-back: the graph replays back to back)."""
    torch, lib = B.torch, B.lib
    qt = M_.Q8_0 if qt is None else qt
    r = np.random.default_rng(400)
    f = lambda *s, sc=0.02: (r.standard_normal(s) * sc).astype(np.float32)
    layers = []
    for _ in range(n_layers):
        L = {nm: f(d, d) for nm in ("sq", "sk", "sv", "so", "cq", "ck", "cv", "co")}
        L.update({nm + "_b": f(d) for nm in ("sq", "sk", "sv", "so", "cq", "ck", "cv", "co")})
        L.update(ff1=f(ffn, d), ff1_b=f(ffn), ff2=f(d, ffn), ff2_b=f(d))
        for nm in ("self", "cross", "ffn"):
            L[f"ln_{nm}_w"], L[f"ln_{nm}_b"] = 1 + f(d), f(d)
        layers.append(L)
    max_seq = 4 + cap + 1
    params = {"emb": f(vocab, d, sc=1.0), "pos": f(max_seq, d, sc=0.3), "embln_w": 1 + f(d), "embln_b": f(d),
              "fin_w": 1 + f(d), "fin_b": f(d), "head": f(vocab, d), "head_b": f(vocab), "layers": layers}
    dev = M_.DeviceAed(lib, params, H, qt)
    enc = B.dev(f(T, d, sc=1.0))
    prompt = [1, 2, 3, 4]
    dev.decode(enc.data_ptr(), T, prompt, -1, 4)   # warm
    B.sync()
    t0 = time.perf_counter()
    toks = dev.decode(enc.data_ptr(), T, prompt, -1, cap)
    t1 = time.perf_counter()
    forced = prompt + toks[:cap - 1]
    dev.forced(enc.data_ptr(), T, forced)
    t2 = time.perf_counter()
    dev.forced(enc.data_ptr(), T, forced)
    t3 = time.perf_counter()
    positions = len(prompt) - 1 + len(toks)
    # bytes one position streams: the step's linears, the cross K/V, the self cache (mean length)
    wb = lambda n, k: M_.weight_bytes(qt, n, k)
    per_layer = 6 * wb(d, d) + wb(ffn, d) + wb(d, ffn) + 2 * 4 * T * d + 2 * 4 * d * (len(forced) / 2)
    step_bytes = n_layers * per_layer + wb(vocab, d)
    us_forced = (t3 - t2) * 1e6 / len(forced)
    dev.close()
    return {"d": d, "heads": H, "ffn": ffn, "vocab": vocab, "layers": n_layers, "T": T, "format": M_.NAMES[qt],
            "tokens": len(toks), "greedy_us_per_token": round((t1 - t0) * 1e6 / positions, 1),
            "forced_us_per_position": round(us_forced, 1), "bytes_per_position": int(step_bytes),
            "forced_hbm_gbps": round(step_bytes / (us_forced * 1e-6) / 1e9, 1),
            "note": "host wall clock around one call (graph capture, cross K/V products and copies included)"}


COUNTERS = os.path.join(ROOT, "profiles", "counters_q8_0_gemm_and_gemv.md")


def profiled_counters() -> dict:
    """Per-kernel counter figures recorded by the rocprofv3 --pmc passes under
    profiles/ (MFMA busy %, useful MFMA %, HBM MB read / written per launch,
    GB/s): {name: {field: value}}; {} if absent."""
    out = {}
    try:
        for line in open(COUNTERS):
            if line.startswith("counter ") and ":" in line:
                name, rest = line[len("counter "):].split(":", 1)
                out[name.strip()] = {k: float(v) for k, v in (f.split("=") for f in rest.split())}
    except OSError:
        pass
    return out


def profiled_traffic():
    """HBM bytes per launch of the roofline kernel (ffn2), from the counters."""
    c = profiled_counters().get("ffn2")
    return int((c["hbm_read_mb"] + c["hbm_write_mb"]) * 1e6) if c else None


def run_profile(B, M_):
    """Counter runs for rocprofv3 --pmc: a 256 MiB device copy (calibrates
    FETCH_SIZE / WRITE_SIZE), then each kernel the bench line reports, three
    launches each on inputs prepared once: the EXACT Q8_0 products at M = 6000
    (1024->4096, 4096->1024, 1024->1024), the INT8ACT Q4_K 4096->1024 product at
    M = 12000, and the decoder GEMVs (Q8_0, M = 1: 1024->16384, 4096->1024
    split K, 1024->1024) over rotating weight copies."""
    torch, lib = B.torch, B.lib
    src = torch.empty(64 << 20, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    with torch.cuda.stream(B.stream):
        for _ in range(3):
            dst.copy_(src)
    B.sync()
    del src, dst
    for qt, k, n, M, num in ((M_.Q8_0, 1024, 4096, 6000, 0), (M_.Q8_0, 4096, 1024, 6000, 0),
                             (M_.Q8_0, 1024, 1024, 6000, 0), (M_.Q4_K, 4096, 1024, 12000, 1)):
        lib.set_numerics(num)
        try:
            dw = M_.DeviceWeight(lib, M_.Weight.make(lib, qt, lib.randn(1, 0.02, (n, k))))
            x, y = B.dev(lib.randn(1, 1.0, (M, k))), B.empty(M, n)
            dw.prep(x.data_ptr(), M, B.sp)
            for _ in range(3):
                dw.gemm_prepped(y.data_ptr(), M, 0, B.sp)
            B.sync()
            dw.close()
        finally:
            lib.set_numerics(0)
        log(f"[bench] profile: {M_.NAMES[qt]} {k}->{n} M={M} numerics={num} x3")
    for k, n in ((1024, 16384), (4096, 1024), (1024, 1024)):
        w = M_.Weight.make(lib, M_.Q8_0, lib.randn(0, 0.02, (n, k)))
        dws = [M_.DeviceWeight(lib, w) for _ in range(3)]
        x, y = B.dev(lib.randn(1, 1.0, (1, k))), B.empty(1, n)
        for dw in dws:
            dw.gemm(x.data_ptr(), y.data_ptr(), 1, 0, B.sp)
        B.sync()
        for dw in dws:
            dw.close()
        log(f"[bench] profile: GEMV Q8_0 {k}->{n} M=1 x3")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extras", action="store_true", help="primary workload only")
    ap.add_argument("--attention", action="store_true",
                    help="only the rel-pos attention core (T=750, 16 segments, full and [70, 13] windows), "
                         "one JSON line")
    ap.add_argument("--small-m", action="store_true",
                    help="only the few-row products on one stream (M = 16 .. 750), one JSON line")
    ap.add_argument("--aed", action="store_true",
                    help="only the AED decoder (config 3 shapes, 4 layers, T=750, Q8_0), one JSON line")
    ap.add_argument("--int8act", action="store_true",
                    help="only the INT8ACT layer sets (Q8_0 M=6000, Q4_K and Q5_K M=12000), one JSON line")
    ap.add_argument("--vendor", action="store_true",
                    help="only the vendor GEMM calibration (torch.matmul / hipBLASLt at the EXACT products' "
                         "MFMA volume), one JSON line")
    ap.add_argument("--config5", action="store_true",
                    help="only the built parts of one encoder layer at config 5's batch (M=12000), one JSON line")
    ap.add_argument("--profile", action="store_true",
                    help="counter run for rocprofv3 --pmc: a 256 MiB device copy, then each kernel the "
                         "bench line reports (GEMMs and decoder GEMVs), 3 launches each")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are out of scope "
                                   "(the path shards by rows with no communication)",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    import mynah_hip as M_
    lib = M_.HipLib()
    if not lib.available():
        raise SystemExit("bench: no usable gfx950 device: " + lib.last_error())
    B = Bench(lib, torch)
    M = 6000
    if args.profile:
        run_profile(B, M_)
        return
    if args.attention:
        print(json.dumps({"relpos_attention": run_attention(B, M_)}), flush=True)
        return
    if args.small_m:
        print(json.dumps({"gemm_small_m": run_small_m(B, M_)}), flush=True)
        return
    if args.aed:
        print(json.dumps({"aed_decoder": run_aed(B, M_)}), flush=True)
        return
    if args.int8act:
        print(json.dumps(run_int8act(B, M_, M)), flush=True)
        return
    if args.config5:
        print(json.dumps({"config5_layer": run_config5(B, M_), "config5_forward": run_config5_forward(B, M_)}),
              flush=True)
        return
    if args.vendor:
        print(json.dumps({"vendor_gemm": run_vendor_gemm(B)}), flush=True)
        return

    log("[bench] q8_0 set")
    ms_step, flops, rows = run_encoder_set(B, M_, M_.Q8_0, M, ENC_SHAPES, args.steps, args.warmup, 0)
    value = flops / (ms_step * 1e-3) / 1e12
    # the roofline entry follows the 4096->1024 product: with 1024->4096 the
    # longest launch of the step; its HBM traffic and MFMA busy fraction are
    # measured under profiles/ (counters_q8_0_gemm_and_gemv.md)
    dom = next(r for r in rows if r["gemm"] == "ffn2")
    dom_flops = 2.0 * M * dom["n"] * dom["k"]
    achieved = dom_flops / (dom["kernel_us"] * 1e-6) / 1e12
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP16, 4), "traffic": profiled_traffic(),
                "kernel": f"k_gemm<Q8_0> {dom['gemm']} {dom['k']}->{dom['n']} M={M}"}
    counters = profiled_counters()
    for r in rows:
        c = counters.get("qkvo" if r["gemm"] in ("q", "k", "v", "out", "pos") else r["gemm"])
        if c:
            r["counter_mfma_busy_pct"], r["counter_useful_mfma_pct"] = c["mfma_util"], c["useful_mfma"]
    details = {"encoder_q8_0_m6000": rows, "counters": {
        "source": "profiles/counters_q8_0_gemm_and_gemv.md (rocprofv3 --pmc passes over bench.py --profile)",
        "kernels": counters}}

    if not args.no_extras:
        kq = {}
        for qt in (M_.Q2_K, M_.Q3_K, M_.Q4_K, M_.Q5_K, M_.Q6_K):
            log(f"[bench] {M_.NAMES[qt]}")
            ms4, fl4, rows4 = run_encoder_set(B, M_, qt, 12000, KQ_SHAPES, 3, 1, 100)
            kq[M_.NAMES[qt]] = {"tops_per_layer_set": round(fl4 / (ms4 * 1e-3) / 1e12, 2),
                                "ms_per_layer_set": round(ms4, 3), "rows": rows4}
        details["kquant_m12000"] = kq
        details.update(run_int8act(B, M_, M))
        log("[bench] f32")
        msf, flf, rowsf = run_encoder_set(B, M_, M_.F32, M, ENC_SHAPES[:2], 3, 1, 200)
        details["f32_m6000"] = {"tflops": round(flf / (msf * 1e-3) / 1e12, 2), "rows": rowsf}
        log("[bench] attention")
        details["relpos_attention"] = run_attention(B, M_)
        log("[bench] aed")
        details["aed_decoder"] = run_aed(B, M_)
        log("[bench] gemv")
        gv = []
        for qt in (M_.Q8_0, M_.Q4_0, M_.Q4_K):
            for n, k in [(s[1], s[0]) for s in GEMV_SHAPES]:
                gv += run_gemv(B, M_, qt, n, k, (1, 4, 16))
        details["gemv"] = gv
        big = [g for g in gv if g["n"] * g["k"] >= 4 << 20]
        details["gemv_hbm_frac_mean_large"] = round(float(np.mean([g["kernel_hbm_frac"] for g in big])), 4)
        vf = [g["kernel_vs_floor"] for g in big if g.get("kernel_vs_floor")]
        if vf:   # the same GEMVs against a plain streaming read of their bytes, one launch each
            details["gemv_vs_read_floor_mean_large"] = round(float(np.mean(vf)), 3)
        log("[bench] small m")
        details["gemm_small_m"] = run_small_m(B, M_)
        log("[bench] config5")
        details["config5_layer"] = run_config5(B, M_)
        log("[bench] config5 forward")
        details["config5_forward"] = run_config5_forward(B, M_)
        log("[bench] vendor gemm")
        details["vendor_gemm"] = run_vendor_gemm(B)

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu")
        cpu = cpu_baseline(M_, lib)

    line = {"metric": METRIC, "value": round(value, 3), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f16x2-mfma/f32",
            "data": "synthetic (weights N(0,0.02) seed 0.., activations N(0,1) seed 1)",
            "config": {"workload": "FastConformer-0.6B encoder linear set, Q8_0 weights, M=6000 "
                                   "(1024->4096, 4096->1024, 5x 1024->1024), EXACT numerics",
                       "M": M, "weights": "Q8_0"},
            "roofline": roofline, "cpu_baseline": cpu}
    # The full tree goes to a file (gpurun_out/ when the run has one); stdout
    # gets the contract line alone, kept short (about 1 KB) so that a reader
    # of the output's last lines gets all of it.
    full = dict(line, details=details)
    path = os.path.join(ROOT, "gpurun_out", "bench_details.json")
    try:
        os.makedirs(os.path.dirname(path), exist_ok=True)
        with open(path, "w") as f:
            json.dump(full, f)
        log(f"[bench] details: {os.path.relpath(path, ROOT)}")
    except OSError as ex:
        log(f"[bench] details not written ({ex})")
    line["summary"] = headline_summary(details, rows)
    if cpu is not None:
        line["cpu_baseline"] = {k: cpu[k] for k in ("value", "unit", "cores", "kind")}
        line["cpu_baseline"]["sample"] = cpu["sample_short"]
    print(json.dumps(line, separators=(",", ":")), flush=True)

if __name__ == "__main__":
    main()
