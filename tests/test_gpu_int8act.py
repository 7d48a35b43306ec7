"""INT8ACT numerics on the GPU for every M.

Bars:
  * INT8 / INT4 (qmat formats): the reference's small-T int8 path
    (src/qmat.c:508-552), bit-exact with orc_qmat_int8_path: exact int32 sums,
    the f32 combine in qmat.c's order.
  * ggml block formats (Q8_0, Q4_0 with per-row activations as qmat.c:186-202;
    the K-quants with ingot's per-super-block activations,
    third_party/ingot/src/kernels.c:719-750): bit-exact with
    orc_int8act_blocks, whose integer sums and evaluation order are pinned in
    tests/test_oracle_int8act.py (to the reference's own int8 path among
    others).
  * the reference's precision contract for its int8 path
    (third_party/ingot/tests/test_quant.c:157-205): within 5e-3 relative L2 of
    the exact product on that test's case, and within 1e-6 of the reference's
    int8 path itself (oracle/_ref built with its SIMD flags, where present).
  * rows bit-identical across M.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import mynah_hip as M
import oracle as O

pytestmark = pytest.mark.gpu

TO_ORC = {M.Q8_0: O.Q8_0, M.Q4_0: O.Q4_0, M.Q2_K: O.Q2_K, M.Q3_K: O.Q3_K, M.Q4_K: O.Q4_K, M.Q5_K: O.Q5_K,
          M.Q6_K: O.Q6_K}
BLOCKS = [M.Q8_0, M.Q4_0, M.Q2_K, M.Q3_K, M.Q4_K, M.Q5_K, M.Q6_K]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture
def int8act(gpu):
    assert gpu.set_numerics(M.INT8ACT) == M.INT8ACT
    try:
        yield gpu
    finally:
        gpu.set_numerics(M.EXACT)


def oracle_int8(orc, w: M.Weight, x: np.ndarray) -> np.ndarray:
    if w.qtype in (M.INT8, M.INT4):
        out, _ = orc.qmat_int8_path(w.qtype, w.data, w.scales, w.n, w.k, x)
        return out
    out, _ = orc.int8act_blocks(TO_ORC[w.qtype], w.data, w.n, w.k, x)
    return out


def kdim(qt):
    return 1024 if qt in (M.Q2_K, M.Q3_K, M.Q4_K, M.Q5_K, M.Q6_K) else 1056


@pytest.mark.parametrize("T", [1, 4, 16, 17, 300])
@pytest.mark.parametrize("qt", [M.INT8, M.INT4] + BLOCKS, ids=lambda q: M.NAMES[q])
def test_int8act_bit_exact(int8act, orc, qt, T):
    say("int8act", M.NAMES[qt], "T", T)
    gpu = int8act
    k = kdim(qt)
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (200, k)))
    x = gpu.randn(1, 1.0, (T, k))
    x[0, :5] = 0.0
    if T > 2:
        x[2] = 0.0                                       # all-zero row: scale 0
    if T > 3:
        x[3, 256:512] = 0.0                              # an all-zero super-block
        x[3, 700] = 40.0                                 # and one with a far larger maximum
    y = M.host_qgemm(gpu, w, x)
    ref = oracle_int8(orc, w, x)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), \
        f"{int((y != ref).sum())} of {y.size} differ; max abs {np.abs(y - ref).max()}"


@pytest.mark.parametrize("qt", [M.Q4_K, M.Q5_K, M.Q6_K, M.Q8_0, M.Q4_0], ids=lambda q: M.NAMES[q])
def test_int8act_large_products_bit_exact(int8act, orc, qt):
    """The encoder's widest shapes (split-K and unsplit launches, three
    workgroups per CU; for Q8_0 / Q4_0 the one-pass row preparation at
    K = 1024 and 4096), sampled rows against the oracle."""
    import torch
    say("int8act large", M.NAMES[qt])
    gpu = int8act
    for (n, k, T) in ((4096, 1024, 2000), (1024, 4096, 700)):
        w = M.Weight.make(gpu, qt, gpu.randn(5, 0.02, (n, k)))
        dw = M.DeviceWeight(gpu, w)
        x = gpu.randn(6, 1.0, (T, k))
        xd = torch.from_numpy(x).cuda()
        y = torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        dw.gemm(xd.data_ptr(), y.data_ptr(), T)
        torch.cuda.synchronize()
        rows = np.r_[0:8, T - 8:T]
        ref = oracle_int8(orc, w, x[rows])
        got = y.cpu().numpy()[rows]
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (n, k, T)
        dw.close()


def test_int8act_int8_tiled_rows_match(int8act, orc):
    """qmat INT8 weights above 64 rows run the tiled int8 GEMM (96 x 256 or
    64 x 256 tiles), at most 64 rows the one-wave form: the same exact int32
    sums and epilogue, so every row must carry the same bits at every M
    (ragged N and K, M = 2100 down to 1), and sampled rows match the
    reference's int8 path (qmat.c:464-500) restated in the oracle. The
    preparation runs in one pass for 16-byte rows with K <= 4096 and in two
    otherwise (K = 1001, 8192)."""
    import torch
    say("int8act INT8 tiled vs one-wave")
    gpu = int8act
    for (n, k) in ((1000, 1056), (4096, 1024), (1024, 4096), (96, 2080), (200, 1001), (64, 8192)):
        w = M.Weight.make(gpu, M.INT8, gpu.randn(7, 0.02, (n, k)))
        dw = M.DeviceWeight(gpu, w)
        x = gpu.randn(8, 1.0, (2100, k))
        x[5] = 0.0
        xd = torch.from_numpy(x).cuda()
        outs = {}
        for T in (2100, 700, 129, 65, 64, 16, 1):
            y = torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            dw.gemm(xd.data_ptr(), y.data_ptr(), T)
            torch.cuda.synchronize()
            outs[T] = y.cpu().numpy()
        for T in (700, 129, 65, 64, 16, 1):
            assert np.array_equal(outs[T].view(np.uint32), outs[2100][:T].view(np.uint32)), (n, k, T)
        rows = np.r_[0:8, 1000:1004, 2092:2100]
        ref = oracle_int8(orc, w, x[rows])
        assert np.array_equal(outs[2100][rows].view(np.uint32), ref.view(np.uint32)), (n, k)
        dw.close()


@pytest.mark.parametrize("name", ["Q4_K", "Q5_K", "Q8_0", "Q4_0", "Q2_K", "Q3_K", "Q6_K"])
def test_int8act_reference_budget(int8act, orc, name):
    """test_quant.c:157-205: 37 rows of 0.02 * uniform(-1, 1), 131 tokens of
    uniform(-1, 1), 256 columns: relative L2 against the exact product below
    the reference's int8 budget, 5e-3. The reference has this path for Q4_K
    and Q5_K only (checked against it below when oracle/_ref is built); for
    the other formats INT8ACT is this build's extension and the budget is
    the check that pins it. Q4_K through the reference's own quantizer
    (restated in the oracle), the others through the build's."""
    say("int8act budget", name)
    gpu = int8act
    r = np.random.default_rng(0xC0FFEE)
    wf = (0.02 * r.uniform(-1, 1, (37, 256))).astype(np.float32)
    oq, mq = getattr(O, name), getattr(M, name)
    raw = orc.quantize(O.Q4_K, wf) if name == "Q4_K" else gpu.quantize(mq, wf)
    x = r.uniform(-1, 1, (131, 256)).astype(np.float32)
    w = M.Weight(mq, 37, 256, raw)
    y = M.host_qgemm(gpu, w, x)
    ex = orc.gemm_f64(x, orc.dequant(oq, raw, 37 * 256).reshape(37, 256))
    rel = float(np.linalg.norm(y - ex) / np.linalg.norm(ex))
    say(f"  rel L2 vs exact {rel:.3g}")
    assert rel < 5e-3
    ref_path = os.path.join(os.path.dirname(O.__file__), "_ref", "libingot_ref_avx2.so")
    if name in ("Q4_K", "Q5_K") and os.path.exists(ref_path):
        R = O.IngotRef(ref_path)
        if not R.is_exact(131):
            ri = R.kernel("ingot_%s_matmat" % name.lower(), raw, 37, 256, x)
            rel_i = float(np.linalg.norm(y - ri) / np.linalg.norm(ri))
            say(f"  rel L2 vs the reference's int8 path {rel_i:.3g}")
            assert rel_i < 1e-6


@pytest.mark.parametrize("qt", [M.Q8_0, M.Q4_K], ids=lambda q: M.NAMES[q])
def test_int8act_rows_bit_identical_across_M(int8act, qt):
    import torch
    say("int8act row stability", M.NAMES[qt])
    gpu = int8act
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (1024, 1024)))
    dw = M.DeviceWeight(gpu, w)
    x = gpu.randn(1, 1.0, (750, 1024))
    xd = torch.from_numpy(x).cuda()
    outs = {}
    for T in (750, 7, 1):
        yd = torch.empty((T, 1024), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        dw.gemm(xd.data_ptr(), yd.data_ptr(), T)
        torch.cuda.synchronize()
        outs[T] = yd.cpu().numpy()
    for T in (7, 1):
        assert np.array_equal(outs[T].view(np.uint32), outs[750][:T].view(np.uint32)), T
    dw.close()


def test_int8act_qkv_one_launch_matches_products(int8act):
    """Three K-quant products of one prepared input as one launch: each
    output the bits of its own product."""
    import torch
    say("int8act qkv")
    gpu = int8act
    k = n = 1024
    ws = [M.DeviceWeight(gpu, M.Weight.make(gpu, M.Q4_K, gpu.randn(60 + i, 0.02, (n, k)))) for i in range(3)]
    for T in (17, 900):
        x = torch.from_numpy(gpu.randn(63, 1.0, (T, k))).cuda()
        ys = [torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda") for _ in range(3)]
        torch.cuda.synchronize()
        M.qkv_dev(gpu, ws, x.data_ptr(), [y.data_ptr() for y in ys], T)
        torch.cuda.synchronize()
        for i, (w, y) in enumerate(zip(ws, ys)):
            r = torch.empty((T, n), dtype=torch.float32, device="cuda")
            w.gemm(x.data_ptr(), r.data_ptr(), T)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int32), r.view(torch.int32)), f"T={T} output {i}"
    for w in ws:
        w.close()


def test_int8act_f32_weights_fall_back(int8act):
    say("int8act f32")
    gpu = int8act
    w = M.Weight.make(gpu, M.F32, gpu.randn(0, 0.02, (64, 256)))
    x = gpu.randn(1, 1.0, (3, 256))
    out = np.zeros((3, 64), np.float32)
    rc = gpu.L.mynah_asr_hip_qgemm(C.byref(w.desc), x.ctypes.data, out.ctypes.data, 3)
    M.evict(gpu, w)
    assert rc == -1 and "INT8ACT" in gpu.last_error()
