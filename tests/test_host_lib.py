"""CPU-side checks of the product libraries: they load, they export every
symbol their headers declare, and the load-time helpers (quantizers, the
synthetic-input generator) agree with the oracle. No GPU compute here."""
import json
import os
import re

import numpy as np
import pytest

import mynah_hip as M
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _declared(header):
    txt = open(header).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(mynah_(?:asr|synth|gguf)_\w+)\s*\(", txt)) - {"mynah_asr_sigmoid"})


def test_hip_library_exports_every_declared_symbol(lib):
    names = _declared(os.path.join(ROOT, "include", "mynah_asr_hip.h"))
    assert names, "no declarations parsed"
    assert sorted(names) == sorted(M.HIP_SYMBOLS)
    for n in names:
        assert hasattr(lib.L, n), n


def test_host_library_exports_every_declared_symbol(lib):
    host = os.path.join(ROOT, "mynah-asr_amd", "host")
    names = []
    for h in ("qmat.h", "backend.h", "synth.h", "gguf.h"):
        names += _declared(os.path.join(host, h))
    assert sorted(names) == sorted(M.HOST_SYMBOLS)
    for n in names:
        assert hasattr(lib.H, n), n


def test_no_device_here_means_cpu_backend(lib):
    if lib.available():
        pytest.skip("a GPU is present")
    assert lib.L.mynah_asr_hip_available() == 0
    assert lib.H.mynah_asr_set_backend(b"hip") == 0  # falls back to CPU with a note
    assert lib.L.mynah_asr_hip_qgemm(None, None, None, 1) == -1
    assert lib.last_error()


def test_randn_golden_prefix(lib):
    ref = json.load(open(os.path.join(GOLDEN, "randn_prefix.json")))
    for case in ref:
        got = lib.randn(case["seed"], case["sigma"], (len(case["values"]),))
        want = np.array(case["values"], dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), case["seed"]


def test_randn_statistics(lib):
    x = lib.randn(0, 0.02, (1 << 20,)).astype(np.float64)
    assert abs(x.mean()) < 1e-4 and abs(x.std() - 0.02) < 1e-4
    y = lib.randn(1, 1.0, (1 << 20,)).astype(np.float64)
    assert abs(y.std() - 1.0) < 3e-3
    assert not np.array_equal(lib.randn(0, 1.0, (64,)), lib.randn(1, 1.0, (64,)))


@pytest.mark.parametrize("qt,ot", [(M.Q8_0, O.Q8_0), (M.Q4_0, O.Q4_0), (M.Q4_K, O.Q4_K), (M.Q6_K, O.Q6_K)])
def test_reference_quantizers_bit_exact(lib, orc, qt, ot):
    w = lib.randn(0, 0.02, (64, 1024))
    w[3] = 0.0
    assert np.array_equal(lib.quantize(qt, w), orc.quantize(ot, w.ravel()))


@pytest.mark.parametrize("qt,ot,budget", [(M.Q2_K, O.Q2_K, 0.45), (M.Q3_K, O.Q3_K, 0.25),
                                          (M.Q5_K, O.Q5_K, 0.06)])
def test_own_kquant_quantizers_round_trip(lib, orc, qt, ot, budget):
    """Q2_K/Q3_K/Q5_K quantizers are this library's own; the oracle's decoder
    (pinned on the reference fixtures) reads them back within the bit budget."""
    w = lib.randn(0, 0.02, (32, 1024))
    raw = lib.quantize(qt, w)
    wd = orc.dequant(ot, raw, w.size).reshape(w.shape)
    rel = np.linalg.norm(wd - w) / np.linalg.norm(w)
    assert rel < budget, rel


def test_qmat_quantizers_match_oracle(lib, orc):
    w = lib.randn(4, 0.5, (33, 256))
    w[5] = 0.0
    q, s = lib.quantize_int8(w)
    q2, s2 = orc.qmat_quantize_int8(w)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    q, s = lib.quantize_int4(w)
    q2, s2 = orc.qmat_quantize_int4(w)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_weight_bytes_accounting():
    assert M.weight_bytes(M.Q8_0, 4096, 1024) == 4456448
    assert M.weight_bytes(M.Q4_0, 4096, 1024) == 2359296
    assert M.weight_bytes(M.Q8_0, 16384, 1024) == 17825792
    for qt, bits in M.BITS.items():
        if qt in M.BLOCK:
            assert M.weight_bytes(qt, 1024, 1024) * 8 == int(bits * 1024 * 1024)
