"""QMAT numerics: the reference's own qmat.c dispatch, product by product.

src/qmat.c:503-651 chooses the arithmetic of each product from its weight
format, K and row count T: INT8 / INT4 weights with K <= 8192 (QMAT_K_MAX,
:181) take the int8-activation dots for T <= 16 (:508-552) and, with
MYNAH_ASR_QGEMM=1, the int8 GEMM for every T (:598-643, bit-identical to the
dots by construction, :447-450); everything else is dequant + sgemm (:644-650).
Bars:
  * the int8 products bit-exact with the reference's int8 path restated in
    the oracle (orc_qmat_int8_path, pinned in tests/test_oracle.py);
  * every other product bit-identical to this unit's EXACT numerics (whose
    own bar against the f32 product is tests/test_gpu_parity.py's);
  * the reference's callers see the same through the qmat.h mirror
    (mynah_asr_qmat_mul), the fused FFN and Q/K/V entry points (each product
    in its own mode, as qmat_ffn / qmat_qkv call qmat_mul).
Inputs: weights N(0, 0.02) quantized by the library, activations N(0, 1).
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import mynah_hip as M

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture
def qmat_mode(gpu):
    assert gpu.set_numerics(M.QMAT) == M.QMAT
    try:
        yield gpu
    finally:
        gpu.set_numerics(M.EXACT)


def int8_ref(orc, w, x):
    out, _ = orc.qmat_int8_path(w.qtype, w.data, w.scales, w.n, w.k, x)
    return out


def in_mode(gpu, mode, w, x):
    prev = gpu.numerics()
    gpu.set_numerics(mode)
    try:
        return M.host_qgemm(gpu, w, x, keep=True)
    finally:
        gpu.set_numerics(prev)


@pytest.mark.parametrize("qt", [M.INT8, M.INT4], ids=lambda q: M.NAMES[q])
def test_int8_formats_follow_qmat_dispatch(qmat_mode, orc, qt):
    say("qmat dispatch", M.NAMES[qt])
    gpu = qmat_mode
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (200, 1056)))
    x = gpu.randn(1, 1.0, (300, 1056))
    x[2] = 0.0
    for T in (1, 5, 16):
        y = M.host_qgemm(gpu, w, x[:T], keep=True)
        ref = int8_ref(orc, w, x[:T])
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), f"T={T}"
    for T in (17, 300):
        y = M.host_qgemm(gpu, w, x[:T], keep=True)
        ex = in_mode(gpu, M.EXACT, w, x[:T])
        assert np.array_equal(y.view(np.uint32), ex.view(np.uint32)), f"T={T}"
    M.evict(gpu, w)


@pytest.mark.parametrize("qt", [M.F32, M.Q8_0, M.Q4_K], ids=lambda q: M.NAMES[q])
def test_other_formats_are_exact(qmat_mode, qt):
    say("qmat dispatch, EXACT formats", M.NAMES[qt])
    gpu = qmat_mode
    w = M.Weight.make(gpu, qt, gpu.randn(0, 0.02, (160, 1024)))
    x = gpu.randn(1, 1.0, (300, 1024))
    for T in (1, 16, 300):
        y = M.host_qgemm(gpu, w, x[:T], keep=True)
        ex = in_mode(gpu, M.EXACT, w, x[:T])
        assert np.array_equal(y.view(np.uint32), ex.view(np.uint32)), f"T={T}"
    M.evict(gpu, w)


def test_beyond_qmat_k_max_is_exact(qmat_mode):
    """K > 8192: the reference leaves its native int8 dots for an f32 loop."""
    say("qmat dispatch, K = 8448")
    gpu = qmat_mode
    w = M.Weight.make(gpu, M.INT8, gpu.randn(0, 0.02, (64, 8448)))
    x = gpu.randn(1, 1.0, (4, 8448))
    y = M.host_qgemm(gpu, w, x, keep=True)
    ex = in_mode(gpu, M.EXACT, w, x)
    assert np.array_equal(y.view(np.uint32), ex.view(np.uint32))
    M.evict(gpu, w)


def test_qmat_mirror_api(qmat_mode, orc):
    """mynah_asr_qmat_mul (the reference's API, host/qmat.c) on the HIP
    backend: the int8 path at T = 4, EXACT at T = 40."""
    say("qmat dispatch through qmat.h")
    gpu = qmat_mode
    H = gpu.H
    assert H.mynah_asr_set_backend(b"hip") == 3
    n, k = 96, 1024
    wf = gpu.randn(3, 0.02, (n, k))
    m = M.QMat()
    assert H.mynah_asr_qmat_init(C.byref(m), wf.ctypes.data, n, k, M.INT8) == 0
    try:
        q, s = gpu.quantize_int8(wf)
        w = M.Weight(M.INT8, n, k, q, s)
        x = gpu.randn(4, 1.0, (40, k))
        for T in (4, 40):
            out = np.zeros((T, n), np.float32)
            H.mynah_asr_qmat_mul(C.byref(m), x[:T].ctypes.data, out.ctypes.data, T)
            ref = int8_ref(orc, w, x[:T]) if T <= 16 else in_mode(gpu, M.EXACT, w, x[:T])
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), f"T={T}"
        M.evict(gpu, w)
    finally:
        H.mynah_asr_qmat_free(C.byref(m))


def test_ffn_and_qkv_products_in_their_own_modes(qmat_mode):
    """qffn_dev with an INT8 first weight and a Q8_0 second one at T = 8: the
    first product takes the int8 path (SiLU applied), the second EXACT; qqkv_dev
    with INT8 q and Q8_0 k, v: each as its own product."""
    import torch
    say("qmat dispatch, ffn / qkv")
    gpu = qmat_mode
    T, d, f = 8, 1024, 2048
    w1 = M.Weight.make(gpu, M.INT8, gpu.randn(1, 0.02, (f, d)))
    w2 = M.Weight.make(gpu, M.Q8_0, gpu.randn(2, 0.02, (d, f)))
    d1, d2 = M.DeviceWeight(gpu, w1), M.DeviceWeight(gpu, w2)
    x = torch.from_numpy(gpu.randn(5, 1.0, (T, d))).cuda()
    try:
        h = torch.empty((T, f), dtype=torch.float32, device="cuda")
        want = torch.empty((T, d), dtype=torch.float32, device="cuda")
        got = torch.empty((T, d), dtype=torch.float32, device="cuda")
        d1.gemm(x.data_ptr(), h.data_ptr(), T, 1)        # int8 path, SiLU
        d2.gemm(h.data_ptr(), want.data_ptr(), T, 0)     # EXACT
        rc = gpu.L.mynah_asr_hip_qffn_dev(d1.h, d2.h, x.data_ptr(), got.data_ptr(), T, None)
        assert rc == 0, gpu.last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))
        wk = M.Weight.make(gpu, M.Q8_0, gpu.randn(3, 0.02, (d, d)))
        wq = M.Weight.make(gpu, M.INT8, gpu.randn(4, 0.02, (d, d)))
        dq, dk = M.DeviceWeight(gpu, wq), M.DeviceWeight(gpu, wk)
        ys = [torch.empty((T, d), dtype=torch.float32, device="cuda") for _ in range(3)]
        rc = gpu.L.mynah_asr_hip_qqkv_dev(dq.h, dk.h, dk.h, x.data_ptr(), ys[0].data_ptr(), ys[1].data_ptr(),
                                          ys[2].data_ptr(), T, None)
        assert rc == 0, gpu.last_error()
        for dw, y in ((dq, ys[0]), (dk, ys[1]), (dk, ys[2])):
            r = torch.empty((T, d), dtype=torch.float32, device="cuda")
            dw.gemm(x.data_ptr(), r.data_ptr(), T, 0)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int32), r.view(torch.int32))
        dq.close()
        dk.close()
    finally:
        d1.close()
        d2.close()


def test_qgemm_env_takes_int8_for_every_t(qmat_mode, orc):
    """MYNAH_ASR_QGEMM=1 (qmat.c:598-643): INT8 weights take the int8 path at
    T = 300 too; Q8_0 stays EXACT."""
    say("qmat dispatch, MYNAH_ASR_QGEMM=1")
    gpu = qmat_mode
    w = M.Weight.make(gpu, M.INT8, gpu.randn(0, 0.02, (96, 1024)))
    wq = M.Weight.make(gpu, M.Q8_0, gpu.randn(0, 0.02, (96, 1024)))
    x = gpu.randn(1, 1.0, (300, 1024))
    os.environ["MYNAH_ASR_QGEMM"] = "1"
    try:
        y = M.host_qgemm(gpu, w, x, keep=True)
        yq = M.host_qgemm(gpu, wq, x, keep=True)
    finally:
        del os.environ["MYNAH_ASR_QGEMM"]
    ref = int8_ref(orc, w, x)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    ex = in_mode(gpu, M.EXACT, wq, x)
    assert np.array_equal(yq.view(np.uint32), ex.view(np.uint32))
    M.evict(gpu, w)
    M.evict(gpu, wq)


def test_device_decoder_in_qmat_mode(qmat_mode):
    """The device AED decoder runs EXACT products only: in QMAT numerics it
    refuses INT8 linears (their one-row products would take the int8 path) and
    runs Q8_0 ones with the same bits as in EXACT numerics."""
    import torch
    from test_gpu_aed import make_params
    say("qmat dispatch, AED decoder")
    gpu = qmat_mode
    d, H, T = 256, 2, 20
    params = make_params(11, d, H, 512, 300, 1, 16)
    enc = torch.from_numpy(np.random.default_rng(3).standard_normal((T, d)).astype(np.float32)).cuda()
    dev8 = M.DeviceAed(gpu, params, H, M.INT8)
    try:
        with pytest.raises(RuntimeError, match="QMAT numerics"):
            dev8.forced(enc.data_ptr(), T, [1, 2, 3])
    finally:
        dev8.close()
    devq = M.DeviceAed(gpu, params, H, M.Q8_0)
    try:
        got = devq.forced(enc.data_ptr(), T, [1, 2, 3])
        gpu.set_numerics(M.EXACT)
        want = devq.forced(enc.data_ptr(), T, [1, 2, 3])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        devq.close()


def test_threads_each_get_their_products_mode(qmat_mode, orc):
    """Four threads at once, INT8 weights at T = 4 (int8 path) and T = 40
    (EXACT) interleaved: each call's mode is its own (the effective mode is
    per call and per thread), so every result matches its serial twin."""
    import threading
    say("qmat dispatch, concurrent callers")
    gpu = qmat_mode
    w = M.Weight.make(gpu, M.INT8, gpu.randn(0, 0.02, (128, 1024)))
    x = gpu.randn(1, 1.0, (40, 1024))
    want = {4: int8_ref(orc, w, x[:4]), 40: in_mode(gpu, M.EXACT, w, x[:40])}
    gpu.set_numerics(M.QMAT)
    errors = []

    def work(i):
        try:
            for r in range(6):
                T = 4 if (i + r) % 2 == 0 else 40
                y = M.host_qgemm(gpu, w, x[:T], keep=True)
                if not np.array_equal(y.view(np.uint32), want[T].view(np.uint32)):
                    errors.append((i, r, T))
        except Exception as ex:   # surfaced below
            errors.append((i, repr(ex)))

    th = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    M.evict(gpu, w)
    assert not errors, errors
