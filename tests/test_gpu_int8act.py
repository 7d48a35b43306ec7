"""INT8ACT numerics: the reference's small-T int8 path (src/qmat.c:508-552) on the
GPU for every M. Bar: bit-exact with the oracle — the int32 sums are exact
and the f32 combine follows the same order (qmat.c's for INT8/INT4, the
oracle's block semantics for Q8_0/Q4_0), so every output bit matches.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import mynah_hip as M
import oracle as O

pytestmark = pytest.mark.gpu


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
    out, _ = orc.block_int8_path({M.Q8_0: O.Q8_0, M.Q4_0: O.Q4_0}[w.qtype], w.data, w.n, w.k, x)
    return out


@pytest.mark.parametrize("T", [1, 4, 16, 17, 300])
@pytest.mark.parametrize("qt", [M.INT8, M.INT4, M.Q8_0, M.Q4_0], ids=lambda q: M.NAMES[q])
def test_int8act_bit_exact(int8act, orc, qt, T):
    say("int8act", M.NAMES[qt], "T", T)
    gpu = int8act
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (200, 1056)))
    x = gpu.randn(1, 1.0, (T, 1056))
    x[0, :5] = 0.0
    if T > 2:
        x[2] = 0.0                                       # all-zero row: scale 0
    y = M.host_qgemm(gpu, w, x)
    ref = oracle_int8(orc, w, x)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), \
        f"{int((y != ref).sum())} of {y.size} differ; max abs {np.abs(y - ref).max()}"


def test_int8act_rows_bit_identical_across_M(int8act):
    import torch
    say("int8act row stability")
    gpu = int8act
    w = M.Weight.make(gpu, M.Q8_0, gpu.randn(0, 0.02, (1024, 1024)))
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


def test_int8act_unsupported_format_falls_back(int8act):
    say("int8act unsupported")
    gpu = int8act
    w = M.Weight.make(gpu, M.Q4_K, gpu.randn(0, 0.02, (64, 256)))
    x = gpu.randn(1, 1.0, (3, 256))
    out = np.zeros((3, 64), np.float32)
    rc = gpu.L.mynah_asr_hip_qgemm(C.byref(w.desc), x.ctypes.data, out.ctypes.data, 3)
    M.evict(gpu, w)
    assert rc == -1 and "INT8ACT" in gpu.last_error()
