"""bench.py's contract line stays short (CPU only).

The driver reads the bench's result from the tail of its output: the last
stdout line must carry every contract key and fit well inside that tail. The
detail tree goes to a file instead. Also: the oracle's persistent thread pool
(the CPU baseline's ingot runs) gives the serial results bit for bit.
"""
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

CONTRACT = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
            "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline")


def _fake_details():
    rows = [{"gemm": g, "kernel_us": 120.123, "mfma_frac": 0.1712, "k": 1024, "n": 4096}
            for g in ("ffn1", "ffn2", "q", "k", "v", "out", "pos")]
    gemv = [{"format": f, "M": m, "k": k, "n": n, "kernel_us": 7.06}
            for f in ("Q8_0", "Q4_0", "Q4_K") for m in (1, 4, 16)
            for k, n in ((1024, 1024), (1024, 4096), (4096, 1024), (1024, 16384))]
    return rows, {"gemv": gemv, "gemv_hbm_frac_mean_large": 0.1103,
                  "aed_decoder": {"forced_us_per_position": 248.3},
                  "gemm_small_m": [{"M": 750, "k": 1024, "n": 4096, "call_us": 27.59}],
                  "kquant_m12000": {"Q4_K": {"tops_per_layer_set": 332.0}},
                  "vendor_gemm": [{"gemm": g, "dtype": d, "us": 125.43}
                                  for g in ("ffn2 volume", "ffn1 volume", "4096->1024 plain", "config 1 volume",
                                            "4096->1024 M=750 volume")
                                  for d in ("f16", "bf16")]}


def test_contract_line_is_short():
    import bench
    rows, details = _fake_details()
    s = bench.headline_summary(details, rows)
    assert s["gemv_q8_0_1024x16384_m1_us"] == 7.06 and s["config1_us_per_call"] == 27.59
    assert s["hipblaslt_f16_same_mfma_us"] == {"ffn2": 125.43, "ffn1": 125.43}
    line = {k: None for k in CONTRACT}
    line.update(metric=bench.METRIC, value=316.122, unit="TOPS", n_gpus=1, steps=20, warmup=5,
                ms_per_step=0.5175, higher_is_better=True, scaling="weak", dtype="f16x2-mfma/f32",
                data="synthetic (weights N(0,0.02) seed 0.., activations N(0,1) seed 1)",
                config={"workload": "FastConformer-0.6B encoder linear set, Q8_0 weights, M=6000 "
                                    "(1024->4096, 4096->1024, 5x 1024->1024), EXACT numerics",
                        "M": 6000, "weights": "Q8_0"},
                roofline={"bound": "mfma", "achieved": 427.95, "peak": 2500.0, "unit": "TFLOP/s", "frac": 0.1712,
                          "traffic": 208000000, "kernel": "k_gemm<Q8_0> ffn2 4096->1024 M=6000"},
                cpu_baseline={"value": 3.4613, "unit": "TOPS", "cores": 16, "kind": "reference",
                              "sample": "5 steps (7 GEMMs, M=6000): ingot dequant once + OpenBLAS sgemm, 16 "
                                        "threads, AMD EPYC (vendor_id=AuthenticAMD cpu family=26 model=2 stepping=1)"},
                summary=s)
    text = json.dumps(line, separators=(",", ":"))
    assert len(text) < 1400, len(text)
    assert set(CONTRACT) <= set(json.loads(text))


def test_persistent_pool_matches_serial():
    import oracle as O
    if not os.path.exists(O.REF_AVX2_PATH):
        pytest.skip("oracle/_ref not built (needs the reference tree at build time)")
    import mynah_hip as M
    lib = M.HipLib()
    R = O.IngotRef(O.REF_AVX2_PATH)
    raw = lib.quantize(M.Q8_0, lib.randn(0, 0.02, (96, 512)))
    x = lib.randn(1, 1.0, (7, 512))
    R.set_threads(1)
    one = R.kernel("ingot_q8_0_matmat", raw, 96, 512, x)
    outs = []
    for th in (4, 3, 8, 2):   # grow, shrink, grow again: workers stay, ranges follow the count
        R.set_threads(th)
        outs.append(R.kernel("ingot_q8_0_matmat", raw, 96, 512, x))
    for i in range(200):   # many short jobs, the count changing between them
        R.set_threads(1 + i % 6)
        o = R.kernel("ingot_q8_0_matmat", raw, 96, 512, x)
        if i % 50 == 0:
            outs.append(o)
    R.set_threads(1)
    for o in outs:
        assert np.array_equal(o.view(np.uint32), one.view(np.uint32))
