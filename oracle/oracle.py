"""oracle.py — TEST INFRASTRUCTURE ONLY.

ctypes view of ``liboracle.so`` (this build's C restatement of the reference
CPU path, ``oracle.c``) and of ``_ref/libingot_ref.so`` (the reference's own
ingot sources compiled unmodified, built only where ``/root/reference`` exists).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, and only as the checker.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libingot_ref.so")
REF_AVX2_PATH = os.path.join(HERE, "_ref", "libingot_ref_avx2.so")

F32, Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 2, 8, 10, 11, 12, 13, 14
GEOMETRY = {F32: (1, 4), Q4_0: (32, 18), Q8_0: (32, 34), Q2_K: (256, 84),
            Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K",
         Q5_K: "Q5_K", Q6_K: "Q6_K", F32: "F32"}

_P = C.c_void_p


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and _ref when the reference tree is mounted)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if ref and os.path.isdir("/root/reference/third_party/ingot/src"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_P)


class Oracle:
    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            build(ref=False)
        L = C.CDLL(path)
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_quantize.argtypes = [C.c_int, _P, C.c_size_t, _P]
        L.orc_dequant.argtypes = [C.c_int, _P, C.c_size_t, _P]
        L.orc_qmat_quantize_int8.argtypes = [_P, C.c_int, C.c_int, _P, _P]
        L.orc_qmat_quantize_int4.argtypes = [_P, C.c_int, C.c_int, _P, _P]
        L.orc_qmat_dequant.argtypes = [C.c_int, _P, _P, C.c_int, C.c_int, _P]
        L.orc_act_quant_int8.restype = C.c_float
        L.orc_act_quant_int8.argtypes = [_P, C.c_int, _P]
        L.orc_qmat_int8_path.argtypes = [C.c_int, _P, _P, C.c_int, C.c_int, _P, C.c_int, _P, _P]
        L.orc_gemm_f64.argtypes = [_P, _P, C.c_int, C.c_int, C.c_int, _P, C.c_int]
        L.orc_kquant_ints.argtypes = [C.c_int, _P, _P, _P, _P, _P, _P]
        L.orc_act_quant_sb.restype = C.c_float
        L.orc_act_quant_sb.argtypes = [_P, _P]
        L.orc_int8act_blocks.argtypes = [C.c_int, _P, C.c_int, C.c_int, _P, C.c_int, _P, _P]
        L.orc_ingot_install_pool.argtypes = [_P, C.c_int]
        self.L = L

    # ---- conversions
    def f16_to_f32(self, h: int) -> float:
        return self.L.orc_f16_to_f32(h)

    def f32_to_f16(self, f: float) -> int:
        return self.L.orc_f32_to_f16(f)

    # ---- blocks
    @staticmethod
    def nbytes(qtype: int, count: int) -> int:
        be, bb = GEOMETRY[qtype]
        assert count % be == 0
        return count // be * bb

    def quantize(self, qtype: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(self.nbytes(qtype, x.size), dtype=np.uint8)
        rc = self.L.orc_quantize(qtype, _ptr(x), x.size, _ptr(out))
        assert rc == 0, f"orc_quantize({qtype}) failed"
        return out

    def dequant(self, qtype: int, raw: np.ndarray, count: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        out = np.zeros(count, dtype=np.float32)
        rc = self.L.orc_dequant(qtype, _ptr(raw), count, _ptr(out))
        assert rc == 0, f"orc_dequant({qtype}) failed"
        return out

    # ---- qmat formats
    def qmat_quantize_int8(self, w: np.ndarray):
        n, k = w.shape
        w = np.ascontiguousarray(w, dtype=np.float32)
        q = np.zeros((n, k), dtype=np.int8)
        s = np.zeros(n, dtype=np.float32)
        self.L.orc_qmat_quantize_int8(_ptr(w), n, k, _ptr(q), _ptr(s))
        return q, s

    def qmat_quantize_int4(self, w: np.ndarray):
        n, k = w.shape
        w = np.ascontiguousarray(w, dtype=np.float32)
        q = np.zeros((n, k // 2), dtype=np.uint8)
        s = np.zeros((n, k // 32), dtype=np.float32)
        self.L.orc_qmat_quantize_int4(_ptr(w), n, k, _ptr(q), _ptr(s))
        return q, s

    def qmat_dequant(self, qtype: int, q: np.ndarray, s: np.ndarray, n: int, k: int):
        out = np.zeros((n, k), dtype=np.float32)
        self.L.orc_qmat_dequant(qtype, _ptr(q), _ptr(s), n, k, _ptr(out))
        return out

    def act_quant_int8(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.zeros(x.size, dtype=np.int8)
        s = self.L.orc_act_quant_int8(_ptr(x), x.size, _ptr(q))
        return q, s

    def qmat_int8_path(self, qtype, q, s, n, k, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        out = np.zeros((T, n), dtype=np.float32)
        sums = np.zeros((T, n) if qtype == 1 else (T, n, k // 32), dtype=np.int32)
        self.L.orc_qmat_int8_path(qtype, _ptr(q), _ptr(s), n, k, _ptr(x), T, _ptr(out), _ptr(sums))
        return out, sums

    def kquant_ints(self, qtype: int, block: np.ndarray):
        """(q[256], f[16], m[16], d, dmin) of one K-quant super-block."""
        block = np.ascontiguousarray(block, dtype=np.uint8)
        q = np.zeros(256, np.int32)
        f = np.zeros(16, np.int32)
        m = np.zeros(16, np.int32)
        d, dmin = C.c_float(), C.c_float()
        assert self.L.orc_kquant_ints(qtype, _ptr(block), _ptr(q), _ptr(f), _ptr(m), C.byref(d), C.byref(dmin)) == 0
        return q, f, m, np.float32(d.value), np.float32(dmin.value)

    def act_quant_sb(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        assert x.size == 256
        q = np.zeros(256, np.int8)
        s = self.L.orc_act_quant_sb(_ptr(x), _ptr(q))
        return q, np.float32(s)

    def int8act_blocks(self, qtype: int, blocks: np.ndarray, n: int, k: int, x: np.ndarray):
        """INT8ACT over ggml blocks in the HIP unit's order: (out [T, n],
        chunk integers [T, n, k/128, 2] of the K-quants)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        out = np.zeros((T, n), np.float32)
        ints = np.zeros((T, n, (k + 127) // 128, 2), np.int64)
        self.L.orc_int8act_blocks(qtype, _ptr(np.ascontiguousarray(blocks, dtype=np.uint8)), n, k, _ptr(x), T,
                                  _ptr(out), _ptr(ints))
        return out, ints

    def gemm_f64(self, x: np.ndarray, wd: np.ndarray, threads: int = 0) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        wd = np.ascontiguousarray(wd, dtype=np.float32)
        T, k = x.shape
        n = wd.shape[0]
        out = np.zeros((T, n), dtype=np.float64)
        self.L.orc_gemm_f64(_ptr(x), _ptr(wd), T, n, k, _ptr(out), threads)
        return out


class IngotRef:
    """The reference's own ingot block-format code, compiled from its sources
    (REF_AVX2_PATH: with the reference's x86 SIMD flags)."""

    def __init__(self, path: str = REF_PATH):
        L = C.CDLL(path)
        self.path = path
        L.ingot_f16_to_f32.restype = C.c_float
        L.ingot_f16_to_f32.argtypes = [C.c_uint16]
        L.ingot_f32_to_f16.restype = C.c_uint16
        L.ingot_f32_to_f16.argtypes = [C.c_float]
        L.ingot_quantize.argtypes = [C.c_int, _P, C.c_size_t, _P]
        L.ingot_dequant.argtypes = [C.c_int, _P, C.c_size_t, _P]
        L.ingot_matmat.argtypes = [C.c_int, _P, C.c_size_t, C.c_size_t, _P, _P, C.c_size_t]
        for fn in ("ingot_q4_k_matmat_exact", "ingot_q5_k_matmat_exact", "ingot_q4_k_matmat", "ingot_q5_k_matmat",
                   "ingot_q8_0_matmat"):
            getattr(L, fn).argtypes = [_P, C.c_size_t, C.c_size_t, _P, _P, C.c_size_t]
        L.ingot_matmat_is_exact.argtypes = [C.c_size_t]
        self.L = L

    def set_threads(self, threads: int) -> None:
        """Run ingot's row loops on `threads` host threads (its default is serial)."""
        Oracle().L.orc_ingot_install_pool(C.cast(self.L.ingot_set_parallel_for, _P), threads)

    def is_exact(self, tokens: int) -> bool:
        return bool(self.L.ingot_matmat_is_exact(tokens))

    def kernel(self, name: str, raw: np.ndarray, rows: int, cols: int, x: np.ndarray):
        """One of the named ingot_*_matmat entry points."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros((x.shape[0], rows), dtype=np.float32)
        assert getattr(self.L, name)(_ptr(np.ascontiguousarray(raw, dtype=np.uint8)), rows, cols, _ptr(x), _ptr(out),
                                     x.shape[0]) == 0, name
        return out

    @staticmethod
    def available(path: str = REF_PATH) -> bool:
        return os.path.exists(path)

    def quantize(self, qtype: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(Oracle.nbytes(qtype, x.size), dtype=np.uint8)
        assert self.L.ingot_quantize(qtype, _ptr(x), x.size, _ptr(out)) == 0
        return out

    def dequant(self, qtype: int, raw: np.ndarray, count: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        out = np.zeros(count, dtype=np.float32)
        assert self.L.ingot_dequant(qtype, _ptr(raw), count, _ptr(out)) == 0
        return out

    def matmat(self, qtype: int, raw: np.ndarray, rows: int, cols: int, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros((x.shape[0], rows), dtype=np.float32)
        assert self.L.ingot_matmat(qtype, _ptr(raw), rows, cols, _ptr(x), _ptr(out),
                                   x.shape[0]) == 0
        return out
