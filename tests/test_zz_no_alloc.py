"""The allocation-free product (mynah_asr_hip_qgemm_noalloc_dev) against
mynah_asr_hip_qgemm_dev, through the C ABI.

Bar: bit-identical outputs (the same kernels on the same data; the only
differences are where the prepared input lives and that K is not split), on
two calls in a row, the second with fewer rows, so the second reads a scratch
array the first left holding larger contents. Also: the size limit refuses
what does not fit, and the GEMV rows (M <= 16) need no scratch.
Inputs: weights N(0, 0.02) seed 0 quantized by the library's quantizers,
activations N(0, 1).
"""
import sys

import numpy as np
import pytest

import mynah_hip as M

pytestmark = pytest.mark.gpu

LIMIT = 32 << 20


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _run(torch, dw, x, T, n, act, noalloc):
    y = torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    if noalloc:
        dw.gemm_noalloc(x.data_ptr(), y.data_ptr(), T, act)
    else:
        dw.gemm(x.data_ptr(), y.data_ptr(), T, act)
    torch.cuda.synchronize()
    return y


# (format, n, k, first M, second M): GEMM sizes on both calls, one pair that
# would split K in qgemm_dev (M = 40 at K = 4096), pairs crossing to the GEMV
# (Q8_0 4096 -> 1024 at M = 4: qgemm_dev runs the split-K GEMV there, the
# allocation-free entry the one-launch GEMV, which must give the same bits)
CASES = [
    (M.Q8_0, 1024, 1024, 2000, 300),
    (M.Q8_0, 1024, 4096, 300, 4),
    (M.Q4_K, 512, 4096, 700, 40),
    (M.F32, 256, 1024, 600, 17),
    (M.Q6_K, 256, 1024, 130, 9),
    (M.INT4, 384, 1056, 256, 100),
]


@pytest.mark.parametrize("qt,n,k,m1,m2", CASES, ids=[f"{M.NAMES[c[0]]}-{c[1]}x{c[2]}" for c in CASES])
def test_noalloc_matches_qgemm_dev(gpu, qt, n, k, m1, m2):
    import torch
    say("noalloc", M.NAMES[qt], n, k, m1, m2)
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (n, k)))
    dw = M.DeviceWeight(gpu, w)
    x = torch.from_numpy(gpu.randn(7, 1.0, (m1, k))).cuda()
    try:
        for T, act in ((m1, 0), (m2, 1)):
            assert dw.noalloc_bytes(T) <= LIMIT
            ref = _run(torch, dw, x, T, n, act, False)
            got = _run(torch, dw, x, T, n, act, True)
            assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), f"M={T} act={act}"
    finally:
        dw.close()


# INT8ACT's three activation forms: per-row (Q8_0), per-super-block with the
# mins operand (Q4_K), and the qmat INT4 form on the i8 MFMA; calls of 900, 33
# and 5 rows in a row (the last takes the M <= 16 path)
@pytest.mark.parametrize("qt", [M.Q8_0, M.Q4_K, M.INT4, M.INT8], ids=lambda q: M.NAMES[q])
def test_noalloc_int8act_matches_qgemm_dev(gpu, qt):
    import torch
    say("noalloc INT8ACT", M.NAMES[qt])
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (512, 1024)))
    dw = M.DeviceWeight(gpu, w)
    x = torch.from_numpy(gpu.randn(8, 1.0, (900, 1024))).cuda()
    gpu.set_numerics(M.INT8ACT)
    try:
        for T in (900, 33, 5):
            ref = _run(torch, dw, x, T, 512, 0, False)
            got = _run(torch, dw, x, T, 512, 0, True)
            assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), f"M={T}"
    finally:
        gpu.set_numerics(M.EXACT)
        dw.close()


def test_noalloc_refuses_beyond_limit(gpu):
    import torch
    say("noalloc limit")
    w = M.Weight.make(gpu, M.Q8_0, gpu.randn(0, 0.02, (128, 4096)))
    dw = M.DeviceWeight(gpu, w)
    try:
        T = 2100   # 2112 rows x 4096 x 4 B of prepared input alone is 33 MiB
        assert dw.noalloc_bytes(T) > LIMIT
        assert dw.noalloc_bytes(16) == 0   # the GEMV path prepares nothing
        x = torch.zeros((T, 4096), dtype=torch.float32, device="cuda")
        y = torch.zeros((T, 128), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        rc = gpu.L.mynah_asr_hip_qgemm_noalloc_dev(dw.h, x.data_ptr(), y.data_ptr(), T, 0, None)
        assert rc == -1 and "32 MiB" in gpu.last_error()
    finally:
        dw.close()
