"""GPU parity of the HIP backend against the CPU oracle (EXACT numerics).

Bar (stated where it is checked):
  * dequantized weights: bit-exact (the reference's llama.cpp fixtures and the
    oracle's decoders);
  * f32 outputs: |y - ref| <= 1e-4*|ref| + 1e-6 per element, ref = the product
    of the dequantized weights and the f32 inputs accumulated in double
    (the reference's own self-test pattern, tests/test_qmat.c:39-45);
  * rows: bit-identical across batch sizes M.
Inputs: weights N(0, 0.02) seed 0 (quantized by the library's quantizers,
pinned bit-exact to the reference's by test_host_lib), activations N(0, 1)
seed 1.
"""
import os
import sys

import numpy as np
import pytest

import mynah_hip as M
import oracle as O

pytestmark = pytest.mark.gpu

FIX = os.path.join(os.path.dirname(__file__), "golden", "ingot_fixtures")
TO_ORC = {M.Q4_0: O.Q4_0, M.Q8_0: O.Q8_0, M.Q2_K: O.Q2_K, M.Q3_K: O.Q3_K, M.Q4_K: O.Q4_K,
          M.Q5_K: O.Q5_K, M.Q6_K: O.Q6_K}
ALL = [M.F32, M.INT8, M.INT4, M.Q4_0, M.Q8_0, M.Q2_K, M.Q3_K, M.Q4_K, M.Q5_K, M.Q6_K]
RTOL, ATOL = 1e-4, 1e-6


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def oracle_dequant(orc, w: M.Weight) -> np.ndarray:
    if w.qtype == M.F32:
        return w.data.reshape(w.n, w.k)
    if w.qtype in (M.INT8, M.INT4):
        return orc.qmat_dequant(w.qtype, w.data, w.scales, w.n, w.k)
    return orc.dequant(TO_ORC[w.qtype], w.data, w.n * w.k).reshape(w.n, w.k)


def check_close(y, ref, what):
    err = np.abs(y.astype(np.float64) - ref)
    bound = RTOL * np.abs(ref) + ATOL
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside 1e-4*|ref|+1e-6; "
                             f"worst at {i}: y={y[i]!r} ref={ref[i]!r}")


def kdim(qt):
    return 1024 if qt in (M.Q2_K, M.Q3_K, M.Q4_K, M.Q5_K, M.Q6_K) else 1056


# ---------------------------------------------------------------- dequant
def _fixture_list():
    out = []
    for line in open(os.path.join(FIX, "manifest.txt")):
        name, t, be, bb, nb = line.split()
        out.append((name, int(t) + 16, int(be), int(nb)))
    return out


@pytest.mark.parametrize("name,qt,be,nb", _fixture_list())
def test_dequant_reference_fixtures(gpu, name, qt, be, nb):
    say("dequant fixture", name)
    raw = np.fromfile(os.path.join(FIX, name + ".bin"), dtype=np.uint8)
    ref = np.fromfile(os.path.join(FIX, name + ".ref"), dtype=np.float32)
    k = 1024 if be == 256 else 512
    n = nb * be // k
    w = M.Weight(qt, n, k, raw)
    got = M.host_dequant(gpu, w)
    assert np.array_equal(got.ravel().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("qt", [q for q in ALL if q != M.F32], ids=lambda q: M.NAMES[q])
def test_dequant_random_weights(gpu, orc, qt):
    say("dequant random", M.NAMES[qt])
    k = kdim(qt)
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (200, k)))
    got = M.host_dequant(gpu, w)
    want = oracle_dequant(orc, w)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("T", [1, 3, 16, 17, 40, 300])
@pytest.mark.parametrize("qt", ALL, ids=lambda q: M.NAMES[q])
def test_gemm_matches_oracle(gpu, orc, qt, T):
    say("gemm", M.NAMES[qt], "T", T)
    k = kdim(qt)
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (200, k)))
    x = gpu.randn(1, 1.0, (T, k))
    y = M.host_qgemm(gpu, w, x)
    ref = orc.gemm_f64(x, oracle_dequant(orc, w))
    check_close(y, ref, f"{M.NAMES[qt]} T={T}")


def _sweep_cases(n_cases=40, seed=2024):
    """Seeded random shapes: every format, ragged n, several K per format (block
    multiples for the block formats, any K for F32 / INT8), M on both sides of
    the GEMV / GEMM boundary, weight scales small and large, and activations
    with or without outliers (one entry in 64 scaled by 300: a wide range
    inside each 128-chunk for its shift and split)."""
    r = np.random.default_rng(seed)
    ks = {M.F32: [7, 100, 1000], M.INT8: [13, 256, 1100], M.INT4: [32, 224, 1056],
          M.Q4_0: [32, 96, 544, 2080], M.Q8_0: [32, 96, 544, 2080]}
    kq = [256, 768, 2304]
    out = []
    for i in range(n_cases):
        qt = ALL[i % len(ALL)]
        k = int(r.choice(ks.get(qt, kq)))
        n = int(r.integers(1, 700))
        T = int(r.choice([1, 2, 5, 16, 17, 31, 64, 129, 777]))
        out.append((i, qt, n, k, T, float(r.choice([0.02, 3.0])), bool(r.integers(0, 2))))
    return out


@pytest.mark.parametrize("i,qt,n,k,T,wsc,outliers", _sweep_cases())
def test_gemm_shape_sweep(gpu, orc, i, qt, n, k, T, wsc, outliers):
    say("sweep", i, M.NAMES[qt], "n", n, "k", k, "T", T, "wsc", wsc, "outliers", outliers)
    w = M.Weight.make(gpu, qt, gpu.randn(100 + i, wsc, (n, k)))
    x = gpu.randn(200 + i, 1.0, (T, k))
    if outliers:
        x[:, ::64] *= 300.0
    y = M.host_qgemm(gpu, w, x)
    wd = oracle_dequant(orc, w)
    ref = orc.gemm_f64(x, wd)
    # Large weights and outliers make outputs that cancel: there the f32
    # rounding of the terms, not the result's own size, sets what any f32
    # product can reach. The reference's product (f32 sgemm over the
    # dequantized weights) misses 1e-4*|ref| + 1e-6 on such elements too, by up
    # to 18.5 * 2^-24 * sum_k |x||w| on these cases (measured with numpy's
    # float32 matmul), and this backend by up to 30.1 (its activations carry 22
    # bits as an f16 pair). So the bar adds 32 * 2^-24 * sum_k |x||w|: just
    # above the measured worst, so that a regression still fails.
    unit = 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(wd).astype(np.float64).T)
    floor = 32 * unit
    err = np.abs(y.astype(np.float64) - ref)
    bound = RTOL * np.abs(ref) + ATOL + floor
    ratio = float((err / np.maximum(unit, 1e-300)).max())
    say(f"  worst err / (2^-24 sum|x||w|) = {ratio:.3g}")
    bad = err > bound
    assert not bad.any(), (f"sweep {i} {M.NAMES[qt]} n={n} k={k} T={T}: {int(bad.sum())} outside; "
                           f"worst ratio {ratio:.3g}")


def test_gemm_zero_and_tiny_rows(gpu, orc):
    say("gemm special rows")
    w = M.Weight.make(gpu, M.Q8_0, gpu.randn(0, 0.02, (64, 256)))
    x = gpu.randn(1, 1.0, (5, 256))
    x[1] = 0.0
    x[2] *= 1e-30
    x[3] *= 1e20
    y = M.host_qgemm(gpu, w, x)
    ref = orc.gemm_f64(x, oracle_dequant(orc, w))
    assert not y[1].any()
    # the absolute term of the bound is for unit-scale inputs: compare each
    # scaled row in its own units
    for r, scale in ((0, 1.0), (2, 1e-30), (3, 1e20), (4, 1.0)):
        check_close((y[r] / np.float32(scale)).astype(np.float32), ref[r] / scale, f"row {r}")


@pytest.mark.parametrize("T", [3, 40])
def test_gemm_nonfinite_rows_stay_in_their_rows(gpu, orc, T):
    """A row holding NaN or +-inf gives non-finite outputs (NaN for a NaN, as
    the f32 product; for an infinity the f32 product's +-inf or NaN, here NaN:
    the infinity's f16 pair is inf + NaN) and leaves every other row's bits
    as they are without it (GEMV at T = 3, GEMM at T = 40)."""
    say("gemm non-finite rows T", T)
    w = M.Weight.make(gpu, M.Q8_0, gpu.randn(0, 0.02, (64, 512)))
    x = gpu.randn(1, 1.0, (T, 512))
    clean = M.host_qgemm(gpu, w, x, keep=True)
    x[0, 7] = np.nan
    x[2, 300] = np.inf
    y = M.host_qgemm(gpu, w, x)
    assert np.isnan(y[0]).all()
    assert not np.isfinite(y[2]).any()
    others = [r for r in range(T) if r not in (0, 2)]
    assert np.array_equal(y[others].view(np.uint32), clean[others].view(np.uint32))


@pytest.mark.parametrize("n,k", [(1024, 4096), (4096, 1024), (16384, 1024)])
@pytest.mark.parametrize("qt", [M.Q8_0, M.Q4_0], ids=lambda q: M.NAMES[q])
def test_decoder_gemv_shapes(gpu, orc, qt, n, k):
    """Benchmark config 3 shapes at M in {1, 4, 16}."""
    say("gemv", M.NAMES[qt], n, k)
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (n, k)))
    wd = oracle_dequant(orc, w)
    for T in (1, 4, 16):
        x = gpu.randn(1, 1.0, (T, k))
        check_close(M.host_qgemm(gpu, w, x), orc.gemm_f64(x, wd), f"{n}x{k} T={T}")


# --------------------------------------------------------- row stability
@pytest.mark.parametrize("qt,n,k", [(M.Q8_0, 4096, 1024), (M.Q4_K, 1024, 4096), (M.F32, 1024, 1024)],
                         ids=["Q8_0-1024to4096", "Q4_K-4096to1024", "F32-1024to1024"])
def test_rows_bit_identical_across_M(gpu, orc, qt, n, k):
    """A row's output bits do not depend on the batch size (M = 1, 7, 750, 6000)."""
    import torch
    say("row stability", M.NAMES[qt], n, k)
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (n, k)))
    dw = M.DeviceWeight(gpu, w)
    x = gpu.randn(1, 1.0, (6000, k))
    xd = torch.from_numpy(x).cuda()
    outs = {}
    for T in (6000, 750, 7, 1):
        yd = torch.empty((T, n), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        dw.gemm(xd.data_ptr(), yd.data_ptr(), T)
        torch.cuda.synchronize()
        outs[T] = yd.cpu().numpy()
    # the single-row case also for a row that sits mid-tile in the big runs
    for r in (5, 4321):
        yd = torch.empty((1, n), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        dw.gemm(xd[r:r + 1].data_ptr(), yd.data_ptr(), 1)
        torch.cuda.synchronize()
        assert np.array_equal(yd.cpu().numpy()[0].view(np.uint32), outs[6000][r].view(np.uint32)), r
    for T in (750, 7, 1):
        assert np.array_equal(outs[T].view(np.uint32), outs[6000][:T].view(np.uint32)), T
    # and the big run is right
    check_close(outs[6000][:64], orc.gemm_f64(x[:64], oracle_dequant(orc, w)), "rows 0..63")
    dw.close()


@pytest.mark.parametrize("qt", ALL, ids=lambda q: M.NAMES[q])
def test_split_k_gemv_rows_match_gemm(gpu, orc, qt):
    """K = 2048 over N = 96 (4 column groups): M <= 16 runs the split-K GEMV
    (chunk results, then their fold in chunk order), M = 40 the GEMM. Every
    format's rows must be the same bits either way, and right."""
    import torch
    say("split-K GEMV rows", M.NAMES[qt])
    n, k = 96, 2048
    w = M.Weight.make(gpu, qt, gpu.randn(3, 0.02, (n, k)))
    dw = M.DeviceWeight(gpu, w)
    x = gpu.randn(4, 1.0, (40, k))
    xd = torch.from_numpy(x).cuda()
    outs = {}
    for T in (40, 16, 3, 1):
        yd = torch.empty((T, n), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        dw.gemm(xd.data_ptr(), yd.data_ptr(), T)
        torch.cuda.synchronize()
        outs[T] = yd.cpu().numpy()
    for T in (16, 3, 1):
        assert np.array_equal(outs[T].view(np.uint32), outs[40][:T].view(np.uint32)), T
    check_close(outs[40], orc.gemm_f64(x, oracle_dequant(orc, w)), f"{M.NAMES[qt]} K=2048")
    dw.close()


@pytest.mark.parametrize("qt", [M.Q8_0, M.Q4_K, M.Q6_K], ids=lambda q: M.NAMES[q])
def test_split_k_gemv_in_place_and_repeated(gpu, orc, qt):
    """K = N = 2048 (64 column groups, the most the split-K GEMV takes): eight
    calls in a row on changing inputs sharing one workspace, then one in place
    (x aliasing y, as qgemm allows: every chunk result is formed before the
    fold writes y). Each must be the same bits as the rows of a GEMM (M = 40)."""
    import torch
    say("split-K GEMV in place / repeated", M.NAMES[qt])
    n = k = 2048
    dw = M.DeviceWeight(gpu, M.Weight.make(gpu, qt, gpu.randn(5, 0.02, (n, k))))
    x = torch.from_numpy(gpu.randn(6, 1.0, (40, k))).cuda()
    ref = torch.empty((40, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    dw.gemm(x.data_ptr(), ref.data_ptr(), 40)
    torch.cuda.synchronize()
    for T in (1, 5, 16):
        ys = [torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda") for _ in range(8)]
        xs = [x[i:i + T].contiguous() for i in range(8)]
        torch.cuda.synchronize()
        for xi, yi in zip(xs, ys):
            dw.gemm(xi.data_ptr(), yi.data_ptr(), T)
        z = x[:T].clone()
        torch.cuda.synchronize()
        dw.gemm(z.data_ptr(), z.data_ptr(), T)
        torch.cuda.synchronize()
        rb = ref.cpu().numpy().view(np.uint32)
        for i, yi in enumerate(ys):
            assert np.array_equal(yi.cpu().numpy().view(np.uint32), rb[i:i + T]), (T, i)
        assert np.array_equal(z.cpu().numpy().view(np.uint32), rb[:T]), (T, "in place")
    check_close(ref.cpu().numpy(), orc.gemm_f64(x.cpu().numpy(), oracle_dequant(orc, dw.w)), f"{M.NAMES[qt]} 2048x2048")
    dw.close()


@pytest.mark.parametrize("qt", ALL, ids=lambda q: M.NAMES[q])
def test_split_k_gemm_rows_match_gemm(gpu, orc, qt):
    """A product with few tiles splits K over workgroups (chunk results to a
    workspace, then their fold in chunk order); its rows must carry the bits
    of the same rows in a product with enough tiles to run unsplit. K = 2048,
    N = 1024: M = 40 and 700 split (8 and 88 tiles), M = 2100 does not (264
    tiles); with and without SiLU."""
    import torch
    say("split-K gemm", M.NAMES[qt])
    k, n = 2048, 1024
    dw = M.DeviceWeight(gpu, M.Weight.make(gpu, qt, gpu.randn(80, 0.02, (n, k))))
    x = torch.from_numpy(gpu.randn(81, 1.0, (2100, k))).cuda()
    for act in (0, 1):
        ys = {}
        for T in (2100, 700, 40):
            y = torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            dw.gemm(x.data_ptr(), y.data_ptr(), T, act)
            torch.cuda.synchronize()
            ys[T] = y
        for T in (700, 40):
            assert torch.equal(ys[T].view(torch.int32), ys[2100][:T].view(torch.int32)), f"M={T} act={act}"
    if qt == M.Q8_0:
        ref = orc.gemm_f64(x[:40].cpu().numpy(), oracle_dequant(orc, dw.w))
        check_close(ys[40].cpu().numpy(), ref / (1.0 + np.exp(-ref)), "split-K Q8_0 SiLU")
    dw.close()


# ------------------------------------------------------ fused entry points
def test_ffn_and_qkv(gpu, orc):
    import ctypes as C
    say("ffn / qkv")
    k, n1 = 256, 512
    w1 = M.Weight.make(gpu, M.Q8_0, gpu.randn(0, 0.02, (n1, k)))
    w2 = M.Weight.make(gpu, M.Q4_K, gpu.randn(2, 0.02, (k, n1)))
    x = gpu.randn(1, 1.0, (37, k))
    out = x.copy()  # aliasing as encoder.c:474 does
    rc = gpu.L.mynah_asr_hip_qffn(C.byref(w1.desc), C.byref(w2.desc), out.ctypes.data, out.ctypes.data, 37)
    assert rc == 0, gpu.last_error()
    h = orc.gemm_f64(x, oracle_dequant(orc, w1))
    h = (h / (1.0 + np.exp(-h))).astype(np.float32)
    ref = orc.gemm_f64(h, oracle_dequant(orc, w2))
    err = np.abs(out - ref)
    M.evict(gpu, w1)
    M.evict(gpu, w2)
    assert (err <= 1e-4 * np.abs(ref) + 1e-5).all(), err.max()

    ws = [M.Weight.make(gpu, qt, gpu.randn(10 + i, 0.02, (96, k))) for i, qt in
          enumerate((M.Q8_0, M.Q6_K, M.F32))]
    outs = [np.empty((37, 96), np.float32) for _ in range(3)]
    rc = gpu.L.mynah_asr_hip_qqkv(*[C.byref(w.desc) for w in ws], x.ctypes.data,
                                  *[o.ctypes.data for o in outs], 37)
    assert rc == 0, gpu.last_error()
    for w, o in zip(ws, outs):
        check_close(o, orc.gemm_f64(x, oracle_dequant(orc, w)), "qkv " + M.NAMES[w.qtype])
        assert np.array_equal(o, M.host_qgemm(gpu, w, x))  # evicts w


@pytest.mark.parametrize("T", [300, 5])
@pytest.mark.parametrize("q1,q2", [(M.Q8_0, M.Q8_0), (M.Q4_K, M.Q4_K), (M.Q8_0, M.Q2_K), (M.F32, M.Q4_0)],
                         ids=lambda q: M.NAMES[q] if isinstance(q, int) else q)
def test_ffn_dev_matches_two_products(gpu, q1, q2, T):
    """The fused FFN (first product preparing the second's input in its epilogue)
    is bit-identical to SiLU product + product; x may alias out."""
    import torch
    say("ffn_dev", M.NAMES[q1], M.NAMES[q2], T)
    k, n1 = 512, 1024
    w1 = M.DeviceWeight(gpu, M.Weight.make(gpu, q1, gpu.randn(3, 0.02, (n1, k))))
    w2 = M.DeviceWeight(gpu, M.Weight.make(gpu, q2, gpu.randn(4, 0.02, (k, n1))))
    x = torch.from_numpy(gpu.randn(5, 1.0, (T, k))).cuda()
    h = torch.empty((T, n1), dtype=torch.float32, device="cuda")
    ref = torch.empty((T, k), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    w1.gemm(x.data_ptr(), h.data_ptr(), T, act=1)
    w2.gemm(h.data_ptr(), ref.data_ptr(), T)
    out = x.clone()
    torch.cuda.synchronize()
    M.ffn_dev(gpu, w1, w2, out.data_ptr(), out.data_ptr(), T)
    torch.cuda.synchronize()
    a, b = out.cpu().numpy(), ref.cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{int((a != b).sum())} differ"
    qs = [M.DeviceWeight(gpu, M.Weight.make(gpu, qt, gpu.randn(20 + i, 0.02, (96, k))))
          for i, qt in enumerate((M.Q8_0, M.Q4_K, M.F32))]
    ys = [torch.empty((T, 96), dtype=torch.float32, device="cuda") for _ in range(3)]
    M.qkv_dev(gpu, qs, x.data_ptr(), [y.data_ptr() for y in ys], T)
    for q, y in zip(qs, ys):
        r = torch.empty((T, 96), dtype=torch.float32, device="cuda")
        q.gemm(x.data_ptr(), r.data_ptr(), T)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), r.view(torch.int32)), M.NAMES[q.w.qtype] if hasattr(q, "w") else ""
        q.close()
    w1.close()
    w2.close()


@pytest.mark.parametrize("qt", ALL, ids=lambda q: M.NAMES[q])
def test_qkv_one_launch_matches_products(gpu, qt):
    """Three weights of one format and shape run as one GEMM launch over one
    prepared input; each output is bit-identical to the weight's own product
    (two row counts: several row bands, and a ragged last band; N = 200 pads)."""
    import torch
    say("qkv one launch", M.NAMES[qt])
    k, n = 512, 200
    qs = [M.DeviceWeight(gpu, M.Weight.make(gpu, qt, gpu.randn(30 + i, 0.02, (n, k)))) for i in range(3)]
    for T in (700, 70):
        x = torch.from_numpy(gpu.randn(T, 1.0, (T, k))).cuda()
        ys = [torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda") for _ in range(3)]
        torch.cuda.synchronize()
        M.qkv_dev(gpu, qs, x.data_ptr(), [y.data_ptr() for y in ys], T)
        for i, (q, y) in enumerate(zip(qs, ys)):
            r = torch.empty((T, n), dtype=torch.float32, device="cuda")
            q.gemm(x.data_ptr(), r.data_ptr(), T)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int32), r.view(torch.int32)), f"T={T} output {i}"
    for q in qs:
        q.close()


class XorShift:
    """The reference self-test's generator (tests/test_qmat.c:13-19)."""

    def __init__(self, seed=42):
        self.s = seed

    def frand(self, n):
        out = np.empty(n, dtype=np.float32)
        s, m = self.s, (1 << 64) - 1
        for i in range(n):
            s ^= (s << 13) & m
            s ^= s >> 7
            s ^= (s << 17) & m
            out[i] = np.float32(s % 200001) / np.float32(100000.0) - np.float32(1.0)
        self.s = s
        return out


def _rel_err(a, ref):
    d = a.astype(np.float64) - ref
    r2 = (ref.astype(np.float64) ** 2).sum()
    return float(np.sqrt((d * d).sum() / (r2 if r2 > 0 else 1.0)))


@pytest.mark.parametrize("name,qtype,n,k,T,tol", [
    ("q8 small-T", 1, 96, 1024, 1, 0.03), ("q8 small-T multi", 1, 64, 4096, 4, 0.03),
    ("q4 small-T", 2, 96, 1024, 1, 0.08), ("q4 small-T multi", 2, 64, 4096, 4, 0.08),
    ("q8 large-T", 1, 96, 1024, 48, 0.02), ("q4 large-T", 2, 96, 1024, 48, 0.08),
    ("f32 passthrough", 0, 96, 1024, 8, 1e-6)])
def test_reference_selftest_cases(gpu, name, qtype, n, k, T, tol):
    """tests/test_qmat.c:48-71, case for case, through the qmat.h API: the
    product of the quantized weight against the f32 GEMM in double, relative
    L2 within the reference's own budgets. Every case also meets 1e-6 against
    the dequantized weight (the quantization error is all that remains)."""
    import ctypes as C
    say("reference self-test", name)
    rng = XorShift()
    w = rng.frand(n * k).reshape(n, k)
    x = rng.frand(T * k).reshape(T, k)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    H = gpu.H
    assert H.mynah_asr_set_backend(b"hip") == 3
    m = M.QMat()
    assert H.mynah_asr_qmat_init(C.byref(m), w.ctypes.data, n, k, qtype) == 0
    out = np.zeros((T, n), np.float32)
    H.mynah_asr_qmat_mul(C.byref(m), x.ctypes.data, out.ctypes.data, T)
    wd = np.empty((n, k), np.float32)
    H.mynah_asr_qmat_dequant(C.byref(m), wd.ctypes.data)
    H.mynah_asr_qmat_free(C.byref(m))
    assert _rel_err(out, ref) <= tol
    assert _rel_err(out, x.astype(np.float64) @ wd.astype(np.float64).T) <= 1e-6


def test_qmat_api_mirror(gpu, orc):
    """The qmat.h entry points (the reference's own API) on the HIP backend."""
    import ctypes as C
    say("qmat mirror")
    H = gpu.H
    assert H.mynah_asr_set_backend(b"hip") == 3
    rng_w = gpu.randn(0, 0.02, (96, 1024))
    x = gpu.randn(1, 1.0, (48, 1024))
    for qt in (0, 1, 2):
        m = M.QMat()
        assert H.mynah_asr_qmat_init(C.byref(m), rng_w.ctypes.data, 96, 1024, qt) == 0
        out = np.empty((48, 96), np.float32)
        H.mynah_asr_qmat_mul(C.byref(m), x.ctypes.data, out.ctypes.data, 48)
        wd = np.empty((96, 1024), np.float32)
        H.mynah_asr_qmat_dequant(C.byref(m), wd.ctypes.data)
        if qt == 0:
            assert np.array_equal(wd, rng_w)
        else:
            q = np.ctypeslib.as_array(C.cast(m.q8 if qt == 1 else m.q4, C.POINTER(C.c_uint8)),
                                      shape=(96 * (1024 if qt == 1 else 512),))
            s = np.ctypeslib.as_array(C.cast(m.scales, C.POINTER(C.c_float)),
                                      shape=(96 if qt == 1 else 96 * 32,))
            assert np.array_equal(wd, orc.qmat_dequant(qt, q.copy(), s.copy(), 96, 1024))
        check_close(out, orc.gemm_f64(x, wd), f"qmat_mul qtype {qt}")
        H.mynah_asr_qmat_free(C.byref(m))
    # ggml blocks straight through qmat_init_blocks
    raw = gpu.quantize(M.Q4_K, rng_w)
    m = M.QMat()
    assert H.mynah_asr_qmat_init_blocks(C.byref(m), raw.ctypes.data, 96, 1024, M.Q4_K) == 0
    out = np.empty((48, 96), np.float32)
    H.mynah_asr_qmat_mul(C.byref(m), x.ctypes.data, out.ctypes.data, 48)
    check_close(out, orc.gemm_f64(x, orc.dequant(O.Q4_K, raw, 96 * 1024).reshape(96, 1024)), "blocks")
    H.mynah_asr_qmat_free(C.byref(m))


# ------------------------------------------------------------- threading
def test_concurrent_callers_match_serial(gpu, orc):
    """The reference calls the qmat entry points from several threads at once
    (server workers, and segment workers inside parallel_for:
    src/encoder.c:928,934; the CUDA unit keeps a per-thread stream and buffers,
    src/cuda_gemm.cu:50-90, and locks only its weight cache, :92-130). Six
    threads call the host-pointer qgemm and qqkv entry points on shared
    weights, each first uploaded while the threads contend for it, and on
    inputs of their own (M = 1, 5, 40, 300). Every result must carry the same
    bits as the same call made from one thread."""
    import ctypes as C
    import threading
    say("concurrent callers")
    k = 512
    ws = [M.Weight.make(gpu, qt, gpu.randn(60 + i, 0.02, (192, k))) for i, qt in
          enumerate((M.Q8_0, M.Q4_K, M.F32, M.Q6_K))]
    qkv = [M.Weight.make(gpu, M.Q8_0, gpu.randn(70 + i, 0.02, (128, k))) for i in range(3)]
    Ts = (1, 5, 40, 300)
    cases = [(t, j) for t in range(6) for j in range(8)]

    def inputs(t, j):
        return gpu.randn(1000 + 8 * t + j, 1.0, (Ts[(t + j) % 4], k))

    def run_qkv(x):
        outs = [np.empty((x.shape[0], 128), np.float32) for _ in range(3)]
        rc = gpu.L.mynah_asr_hip_qqkv(*[C.byref(w.desc) for w in qkv], x.ctypes.data,
                                      *[o.ctypes.data for o in outs], x.shape[0])
        return rc, outs

    # one thread (weights evicted after each call, so the threads upload them again)
    serial = {}
    for t, j in cases:
        x = inputs(t, j)
        if j % 4 == 3:
            rc, outs = run_qkv(x)
            assert rc == 0, gpu.last_error()
            serial[(t, j)] = outs
            for w in qkv:
                M.evict(gpu, w)
        else:
            serial[(t, j)] = [M.host_qgemm(gpu, ws[(t + j) % 4], x)]

    got, errors = {}, []

    def worker(t):
        try:
            for j in range(8):
                x = inputs(t, j)
                if j % 4 == 3:
                    rc, outs = run_qkv(x)
                    if rc != 0:
                        raise RuntimeError(gpu.last_error())
                    got[(t, j)] = outs
                else:
                    got[(t, j)] = [M.host_qgemm(gpu, ws[(t + j) % 4], x, keep=True)]
        except Exception as e:  # reported by the main thread
            errors.append(f"thread {t}: {e!r}")

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(6)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads), "a caller thread did not finish"
    for w in ws + qkv:
        M.evict(gpu, w)
    assert not errors, errors
    for key in cases:
        for a, b in zip(got[key], serial[key]):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"case {key} differs"


# ------------------------------------------------- largest K, empty inputs
@pytest.mark.parametrize("qt", [M.Q8_0, M.Q4_K, M.INT8], ids=lambda q: M.NAMES[q])
def test_largest_k(gpu, orc, qt):
    """K = 8192 (QMAT_K_MAX, the reference's largest K for its native int8
    paths, src/qmat.c:181, 515-517) and beyond it (K = 8448, where the
    reference's small-T path leaves SIMD for its scalar loop, the same
    arithmetic): the GEMV (M = 1, 16, K split over workgroups) and the GEMM
    (M = 40, split K; M = 300) against the oracle in EXACT numerics; the
    qmat INT8 format also bit-exact with the reference's small-T int8 path in
    INT8ACT numerics; rows bit-identical across M.
    Bar: 1e-4*|ref| + 1e-6 plus 4 * 2^-24 * sum_k |x||w| per element: at
    K = 8192 some outputs cancel to far below their terms, and there no f32
    product meets the plain bar (the reference's own sgemm misses it at
    K = 4096 by up to 3.3 of these units; tests/test_gpu_configs.py)."""
    say("largest K", M.NAMES[qt])
    for k in (8192, 8448):
        w = M.Weight.make(gpu, qt, gpu.randn(3, 0.02, (96, k)))
        x = gpu.randn(4, 1.0, (300, k))
        wd = oracle_dequant(orc, w)
        y300 = M.host_qgemm(gpu, w, x, keep=True)
        ref = orc.gemm_f64(x[:24], wd)
        unit = 2.0 ** -24 * (np.abs(x[:24]).astype(np.float64) @ np.abs(wd).astype(np.float64).T)
        err = np.abs(y300[:24].astype(np.float64) - ref)
        say(f"  K={k}: worst err / (2^-24 sum|x||w|) = {float((err / unit).max()):.3g}")
        assert (err <= RTOL * np.abs(ref) + ATOL + 4.0 * unit).all(), f"K={k} M=300"
        for T in (1, 16, 40):
            yT = M.host_qgemm(gpu, w, x[:T], keep=True)
            assert np.array_equal(yT.view(np.uint32), y300[:T].view(np.uint32)), f"K={k} M={T}"
        if qt == M.INT8:
            assert gpu.set_numerics(M.INT8ACT) == M.INT8ACT
            try:
                for T in (1, 16, 300):
                    y8 = M.host_qgemm(gpu, w, x[:T], keep=True)
                    ref, _ = orc.qmat_int8_path(w.qtype, w.data, w.scales, w.n, w.k, x[:T])
                    assert np.array_equal(y8.view(np.uint32), ref.view(np.uint32)), f"INT8ACT K={k} M={T}"
            finally:
                gpu.set_numerics(M.EXACT)
        M.evict(gpu, w)


def test_empty_inputs(gpu):
    """T = 0 is done (0) and touches nothing, through the host-pointer and the
    device-pointer entry points, as the reference's loops do nothing for it."""
    import ctypes as C
    import torch
    say("empty inputs")
    w = M.Weight.make(gpu, M.Q8_0, gpu.randn(0, 0.02, (64, 256)))
    out = np.full((1, 64), 7.0, np.float32)
    x = np.zeros((1, 256), np.float32)
    assert gpu.L.mynah_asr_hip_qgemm(C.byref(w.desc), x.ctypes.data, out.ctypes.data, 0) == 0
    assert (out == 7.0).all()
    dw = M.DeviceWeight(gpu, w)
    try:
        xd = torch.zeros((1, 256), device="cuda")
        yd = torch.full((1, 64), 7.0, device="cuda")
        torch.cuda.synchronize()
        assert gpu.L.mynah_asr_hip_qgemm_dev(dw.h, xd.data_ptr(), yd.data_ptr(), 0, 0, None) == 0
        torch.cuda.synchronize()
        assert bool((yd == 7.0).all())
    finally:
        dw.close()
    M.evict(gpu, w)


@pytest.mark.parametrize("T", [700, 5])   # the GEMM and the GEMV paths
def test_public_act_values_other_than_one_mean_silu(gpu, T):
    """The C ABI's act is 0 (none) or anything else (SiLU): act values that the
    library uses internally for its residual epilogues (2, 3) give SiLU at
    the public entry points, bit-identical to act = 1, and never touch y's
    previous contents."""
    import torch
    say("public act", T)
    w = M.DeviceWeight(gpu, M.Weight.make(gpu, M.Q8_0, gpu.randn(6, 0.02, (256, 1024))))
    x = torch.from_numpy(gpu.randn(7, 1.0, (T, 1024))).cuda()
    try:
        outs = []
        for act in (1, 2, 3, -1):
            y = torch.full((T, 256), 123.0, dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            w.gemm(x.data_ptr(), y.data_ptr(), T, act=act)
            torch.cuda.synchronize()
            outs.append(y)
        for y in outs[1:]:
            assert torch.equal(y.view(torch.int32), outs[0].view(torch.int32))
    finally:
        w.close()
