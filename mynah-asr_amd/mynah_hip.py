"""ctypes view of the MI355X backend unit and its C11 host mirror.

Loads the in-tree libraries built by ``build.py``:
  lib/libmynah_asr_hip.so  include/mynah_asr_hip.h (kernels + C ABI)
  lib/libmynah_asr.so      the qmat.h / backend.h mirror and synth.h
Loading fails loudly when they are missing: there is no Python or CPU
fallback for any product.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
HIP_LIB = os.path.join(PKG, "lib", "libmynah_asr_hip.so")
HOST_LIB = os.path.join(PKG, "lib", "libmynah_asr.so")

F32, INT8, INT4 = 0, 1, 2
Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 18, 24, 26, 27, 28, 29, 30
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
NAMES = {F32: "F32", INT8: "INT8", INT4: "INT4", Q4_0: "Q4_0", Q8_0: "Q8_0", Q2_K: "Q2_K",
         Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}
# bits per weight as stored (algorithmic HBM bytes of a weight = n*k*bits/8)
BITS = {F32: 32.0, INT8: 8.0, INT4: 5.0, Q4_0: 4.5, Q8_0: 8.5, Q2_K: 2.625, Q3_K: 3.4375,
        Q4_K: 4.5, Q5_K: 5.5, Q6_K: 6.5625}
EXACT, INT8ACT, QMAT = 0, 1, 2

# every symbol include/mynah_asr_hip.h declares
HIP_SYMBOLS = [
    "mynah_asr_hip_available", "mynah_asr_hip_set_numerics", "mynah_asr_hip_numerics",
    "mynah_asr_hip_gemm_wt", "mynah_asr_hip_ffn_wt", "mynah_asr_hip_gemm3_wt",
    "mynah_asr_hip_qgemm", "mynah_asr_hip_qffn", "mynah_asr_hip_qqkv", "mynah_asr_hip_dequant",
    "mynah_asr_hip_evict", "mynah_asr_hip_evict_all", "mynah_asr_hip_last_error",
    "mynah_asr_hip_weight_create", "mynah_asr_hip_weight_destroy", "mynah_asr_hip_weight_bytes",
    "mynah_asr_hip_qgemm_dev", "mynah_asr_hip_dequant_dev", "mynah_asr_hip_prep_dev",
    "mynah_asr_hip_qgemm_prepped_dev", "mynah_asr_hip_qffn_dev", "mynah_asr_hip_qqkv_dev",
    "mynah_asr_hip_relpos_attention_dev", "mynah_asr_hip_relpos_attention",
    "mynah_asr_hip_aed_decode_dev", "mynah_asr_hip_aed_forced_dev",
    "mynah_asr_hip_qgemm_noalloc_dev", "mynah_asr_hip_noalloc_bytes", "mynah_asr_hip_read_floor_dev",
    "mynah_asr_hip_encoder_layer_dev", "mynah_asr_hip_subsampling_dev",
]
HOST_SYMBOLS = [
    "mynah_asr_set_backend", "mynah_asr_backend", "mynah_asr_gemm_wt", "mynah_asr_silu",
    "mynah_asr_ffn_wt", "mynah_asr_gemm3_wt", "mynah_asr_set_cpu_fallback",
    "mynah_asr_qmat_init", "mynah_asr_qmat_init_blocks", "mynah_asr_qmat_free",
    "mynah_asr_qmat_mul", "mynah_asr_qmat_ffn", "mynah_asr_qmat_qkv", "mynah_asr_qmat_dequant",
    "mynah_asr_quantize_int8", "mynah_asr_quantize_int4",
    "mynah_synth_randn", "mynah_synth_quantize", "mynah_synth_nbytes",
    "mynah_gguf_open", "mynah_gguf_close", "mynah_gguf_version", "mynah_gguf_alignment", "mynah_gguf_count",
    "mynah_gguf_at", "mynah_gguf_find", "mynah_asr_qmat_init_gguf",
]

_P = C.c_void_p


class AedLayerC(C.Structure):
    """mynah_asr_hip_aed_layer (include/mynah_asr_hip.h)."""
    _fields_ = [(f, C.c_void_p) for f in (
        "ln_self_w", "ln_self_b", "sq", "sk", "sv", "so", "sq_b", "sk_b", "sv_b", "so_b",
        "ln_cross_w", "ln_cross_b", "cq", "ck", "cv", "co", "cq_b", "ck_b", "cv_b", "co_b",
        "ln_ffn_w", "ln_ffn_b", "ff1", "ff2", "ff1_b", "ff2_b")]


class AedC(C.Structure):
    """mynah_asr_hip_aed (include/mynah_asr_hip.h)."""
    _fields_ = [("n_layers", C.c_int), ("d", C.c_int), ("n_heads", C.c_int), ("ffn", C.c_int),
                ("vocab", C.c_int), ("max_seq", C.c_int)] + \
               [(f, C.c_void_p) for f in ("proj", "proj_b", "emb", "pos", "embln_w", "embln_b", "fin_w", "fin_b",
                                          "head", "head_b")] + [("layers", C.POINTER(AedLayerC))]


class EncLayerC(C.Structure):
    """mynah_asr_hip_enc_layer (include/mynah_asr_hip.h; src/encoder.h:12-32)."""
    FIELDS = ("ln_ff1_w", "ln_ff1_b", "ff1_w1", "ff1_w2", "ln_att_w", "ln_att_b", "q_w", "k_w", "v_w", "o_w",
              "relk_w", "bias_u", "bias_v", "ln_conv_w", "ln_conv_b", "pw1_w", "pw2_w", "dw_w", "cnorm_w", "cnorm_b",
              "ff1_b1", "ff1_b2", "ff2_b1", "ff2_b2", "q_b", "k_b", "v_b", "o_b", "pw1_b", "dw_b", "pw2_b",
              "cnorm_scale", "cnorm_shift", "ln_ff2_w", "ln_ff2_b", "ff2_w1", "ff2_w2", "ln_out_w", "ln_out_b")
    _fields_ = [(f, C.c_void_p) for f in FIELDS]


class SubsamplingC(C.Structure):
    """mynah_asr_hip_subsampling (include/mynah_asr_hip.h; src/subsampling.h:12-21)."""
    _fields_ = [("conv_in_w", C.c_void_p), ("conv_in_b", C.c_void_p), ("dw_w", C.c_void_p * 2),
                ("dw_b", C.c_void_p * 2), ("pw_w", C.c_void_p * 2), ("pw_b", C.c_void_p * 2),
                ("lin_w", C.c_void_p), ("lin_b", C.c_void_p), ("channels", C.c_int), ("d_model", C.c_int),
                ("causal", C.c_int)]


class WDesc(C.Structure):
    _fields_ = [("qtype", C.c_int), ("n", C.c_int), ("k", C.c_int),
                ("data", C.c_void_p), ("scales", C.c_void_p)]


class QMat(C.Structure):
    """mynah_asr_qmat (host/qmat.h)."""
    _fields_ = [("f32", C.c_void_p), ("q8", C.c_void_p), ("q4", C.c_void_p),
                ("scales", C.c_void_p), ("owned_q", C.c_void_p), ("owned_s", C.c_void_p),
                ("qtype", C.c_int), ("n", C.c_int), ("k", C.c_int), ("blocks", C.c_void_p)]


class GgufTensor(C.Structure):
    """mynah_gguf_tensor (host/gguf.h)."""
    _fields_ = [("name", C.c_char_p), ("ggml_type", C.c_int), ("rank", C.c_int), ("ne", C.c_int64 * 4),
                ("data", C.c_void_p), ("nbytes", C.c_uint64)]


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_P)


def weight_bytes(qtype: int, n: int, k: int) -> int:
    """Algorithmic bytes of a weight as the caller stores it."""
    if qtype in BLOCK:
        be, bb = BLOCK[qtype]
        return n * (k // be) * bb
    if qtype == F32:
        return 4 * n * k
    if qtype == INT8:
        return n * k + 4 * n
    return n * k // 2 + 4 * n * (k // 32)


class HipLib:
    def __init__(self, path: str = HIP_LIB, host_path: str = HOST_LIB):
        if not os.path.exists(path) or not os.path.exists(host_path):
            raise RuntimeError(f"backend libraries not built ({path}); run mynah-asr_amd/build.py")
        L = C.CDLL(path, mode=C.RTLD_GLOBAL)
        H = C.CDLL(host_path)
        self.L, self.H, self.path, self.host_path = L, H, path, host_path
        L.mynah_asr_hip_last_error.restype = C.c_char_p
        L.mynah_asr_hip_weight_create.restype = _P
        L.mynah_asr_hip_weight_create.argtypes = [C.POINTER(WDesc)]
        L.mynah_asr_hip_weight_destroy.argtypes = [_P]
        L.mynah_asr_hip_weight_bytes.restype = C.c_size_t
        L.mynah_asr_hip_weight_bytes.argtypes = [_P]
        L.mynah_asr_hip_qgemm_dev.argtypes = [_P, _P, _P, C.c_int, C.c_int, _P]
        L.mynah_asr_hip_dequant_dev.argtypes = [_P, _P, _P]
        if hasattr(L, "mynah_asr_hip_qgemm_noalloc_dev"):
            L.mynah_asr_hip_qgemm_noalloc_dev.argtypes = [_P, _P, _P, C.c_int, C.c_int, _P]
            L.mynah_asr_hip_noalloc_bytes.restype = C.c_size_t
            L.mynah_asr_hip_noalloc_bytes.argtypes = [_P, C.c_int]
        if hasattr(L, "mynah_asr_hip_read_floor_dev"):
            L.mynah_asr_hip_read_floor_dev.argtypes = [_P, C.c_size_t, _P]
        if hasattr(L, "mynah_asr_hip_prep_dev"):  # absent from older builds
            L.mynah_asr_hip_prep_dev.argtypes = [_P, _P, C.c_int, _P]
            L.mynah_asr_hip_qgemm_prepped_dev.argtypes = [_P, _P, C.c_int, C.c_int, _P]
        if hasattr(L, "mynah_asr_hip_qffn_dev"):
            L.mynah_asr_hip_qffn_dev.argtypes = [_P, _P, _P, _P, C.c_int, _P]
            L.mynah_asr_hip_qqkv_dev.argtypes = [_P, _P, _P, _P, _P, _P, _P, C.c_int, _P]
        if hasattr(L, "mynah_asr_hip_relpos_attention_dev"):
            L.mynah_asr_hip_relpos_attention_dev.argtypes = [_P] * 7 + [C.c_int] * 6 + [_P]
            L.mynah_asr_hip_relpos_attention.argtypes = [_P] * 7 + [C.c_int] * 5
        if hasattr(L, "mynah_asr_hip_encoder_layer_dev"):
            L.mynah_asr_hip_encoder_layer_dev.argtypes = [C.POINTER(EncLayerC), _P, C.c_int, C.c_int, _P] + \
                [C.c_int] * 6 + [_P]
        if hasattr(L, "mynah_asr_hip_subsampling_dev"):
            L.mynah_asr_hip_subsampling_dev.argtypes = [C.POINTER(SubsamplingC), _P, C.c_int, C.c_int, C.c_int,
                                                        C.c_float, _P, C.POINTER(C.c_int), _P]
        if hasattr(L, "mynah_asr_hip_aed_decode_dev"):
            L.mynah_asr_hip_aed_decode_dev.argtypes = [C.POINTER(AedC), _P, C.c_int, _P, C.c_int, C.c_int, _P,
                                                       C.c_int, _P]
            L.mynah_asr_hip_aed_forced_dev.argtypes = [C.POINTER(AedC), _P, C.c_int, _P, C.c_int, _P, _P]
        L.mynah_asr_hip_qgemm.argtypes = [C.POINTER(WDesc), _P, _P, C.c_int]
        L.mynah_asr_hip_qffn.argtypes = [C.POINTER(WDesc), C.POINTER(WDesc), _P, _P, C.c_int]
        L.mynah_asr_hip_qqkv.argtypes = [C.POINTER(WDesc)] * 3 + [_P] * 4 + [C.c_int]
        L.mynah_asr_hip_dequant.argtypes = [C.POINTER(WDesc), _P]
        L.mynah_asr_hip_gemm_wt.argtypes = [_P, _P, _P, C.c_int, C.c_int, C.c_int]
        L.mynah_asr_hip_evict.argtypes = [_P]
        H.mynah_synth_randn.argtypes = [C.c_uint64, C.c_double, _P, C.c_size_t]
        H.mynah_synth_quantize.restype = C.c_size_t
        H.mynah_synth_quantize.argtypes = [C.c_int, _P, C.c_size_t, _P]
        H.mynah_synth_nbytes.restype = C.c_size_t
        H.mynah_synth_nbytes.argtypes = [C.c_int, C.c_size_t]
        H.mynah_asr_set_backend.argtypes = [C.c_char_p]
        H.mynah_asr_qmat_init.argtypes = [C.POINTER(QMat), _P, C.c_int, C.c_int, C.c_int]
        H.mynah_asr_qmat_init_blocks.argtypes = [C.POINTER(QMat), _P, C.c_int, C.c_int, C.c_int]
        H.mynah_gguf_open.restype = _P
        H.mynah_gguf_open.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
        H.mynah_gguf_close.argtypes = [_P]
        H.mynah_gguf_version.restype = C.c_uint32
        H.mynah_gguf_version.argtypes = [_P]
        H.mynah_gguf_alignment.restype = C.c_uint64
        H.mynah_gguf_alignment.argtypes = [_P]
        H.mynah_gguf_count.restype = C.c_size_t
        H.mynah_gguf_count.argtypes = [_P]
        H.mynah_gguf_at.restype = C.POINTER(GgufTensor)
        H.mynah_gguf_at.argtypes = [_P, C.c_size_t]
        H.mynah_gguf_find.restype = C.POINTER(GgufTensor)
        H.mynah_gguf_find.argtypes = [_P, C.c_char_p]
        H.mynah_asr_qmat_init_gguf.argtypes = [C.POINTER(QMat), _P, C.c_char_p]
        H.mynah_asr_qmat_free.argtypes = [C.POINTER(QMat)]
        H.mynah_asr_qmat_mul.argtypes = [C.POINTER(QMat), _P, _P, C.c_int]
        H.mynah_asr_qmat_ffn.argtypes = [C.POINTER(QMat), C.POINTER(QMat), _P, _P, C.c_int, _P]
        H.mynah_asr_qmat_qkv.argtypes = [C.POINTER(QMat)] * 3 + [_P] * 4 + [C.c_int]
        H.mynah_asr_qmat_dequant.argtypes = [C.POINTER(QMat), _P]
        H.mynah_asr_gemm_wt.argtypes = [_P, _P, _P, C.c_int, C.c_int, C.c_int]
        H.mynah_asr_quantize_int8.argtypes = [_P, C.c_int, C.c_int, _P, _P]
        H.mynah_asr_quantize_int4.argtypes = [_P, C.c_int, C.c_int, _P, _P]

    # ------------------------------------------------------------- basics
    def available(self) -> bool:
        return bool(self.L.mynah_asr_hip_available())

    def last_error(self) -> str:
        return self.L.mynah_asr_hip_last_error().decode()

    def read_floor(self, ptr: int, nbytes: int, stream: int = 0) -> None:
        """One streaming read of nbytes at a device pointer (a measurement aid)."""
        self._check(self.L.mynah_asr_hip_read_floor_dev(ptr, nbytes, stream or None), "read_floor_dev")

    def set_numerics(self, mode: int) -> int:
        return self.L.mynah_asr_hip_set_numerics(mode)

    def numerics(self) -> int:
        return self.L.mynah_asr_hip_numerics()

    def _check(self, rc: int, what: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{what} failed: {self.last_error()}")

    # ------------------------------------------------------ synthetic data
    def randn(self, seed: int, sigma: float, shape) -> np.ndarray:
        out = np.empty(int(np.prod(shape)), dtype=np.float32)
        self.H.mynah_synth_randn(seed, sigma, _ptr(out), out.size)
        return out.reshape(shape)

    def quantize(self, qtype: int, w: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32)
        nb = self.H.mynah_synth_nbytes(qtype, w.size)
        if nb == 0:
            raise ValueError(f"cannot quantize {w.size} values to {NAMES.get(qtype, qtype)}")
        out = np.empty(nb, dtype=np.uint8)
        assert self.H.mynah_synth_quantize(qtype, _ptr(w), w.size, _ptr(out)) == nb
        return out

    def quantize_int8(self, w: np.ndarray):
        n, k = w.shape
        w = np.ascontiguousarray(w, dtype=np.float32)
        q = np.empty((n, k), dtype=np.int8)
        s = np.empty(n, dtype=np.float32)
        self.H.mynah_asr_quantize_int8(_ptr(w), n, k, _ptr(q), _ptr(s))
        return q, s

    def quantize_int4(self, w: np.ndarray):
        n, k = w.shape
        w = np.ascontiguousarray(w, dtype=np.float32)
        q = np.empty((n, k // 2), dtype=np.uint8)
        s = np.empty((n, k // 32), dtype=np.float32)
        self.H.mynah_asr_quantize_int4(_ptr(w), n, k, _ptr(q), _ptr(s))
        return q, s


class Weight:
    """A host weight (numpy arrays kept alive) + its descriptor."""

    def __init__(self, qtype: int, n: int, k: int, data: np.ndarray, scales: np.ndarray | None = None):
        self.qtype, self.n, self.k = qtype, n, k
        self.data = np.ascontiguousarray(data)
        self.scales = None if scales is None else np.ascontiguousarray(scales, dtype=np.float32)
        self.desc = WDesc(qtype, n, k, self.data.ctypes.data,
                          self.scales.ctypes.data if self.scales is not None else None)

    @staticmethod
    def make(lib: HipLib, qtype: int, w: np.ndarray) -> "Weight":
        """Quantize an f32 [n, k] matrix into `qtype` with the library's quantizers."""
        n, k = w.shape
        if qtype == F32:
            return Weight(F32, n, k, np.ascontiguousarray(w, dtype=np.float32))
        if qtype == INT8:
            q, s = lib.quantize_int8(w)
            return Weight(INT8, n, k, q, s)
        if qtype == INT4:
            q, s = lib.quantize_int4(w)
            return Weight(INT4, n, k, q, s)
        return Weight(qtype, n, k, lib.quantize(qtype, w))

    def nbytes(self) -> int:
        return weight_bytes(self.qtype, self.n, self.k)


class DeviceWeight:
    """Resident copy created through mynah_asr_hip_weight_create."""

    def __init__(self, lib: HipLib, w: Weight):
        self.lib, self.w = lib, w
        self.h = lib.L.mynah_asr_hip_weight_create(C.byref(w.desc))
        if not self.h:
            raise RuntimeError(f"weight_create failed: {lib.last_error()}")

    def close(self) -> None:
        if self.h:
            self.lib.L.mynah_asr_hip_weight_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def gemm(self, dx_ptr: int, dy_ptr: int, T: int, act: int = 0, stream: int = 0) -> None:
        rc = self.lib.L.mynah_asr_hip_qgemm_dev(self.h, dx_ptr, dy_ptr, T, act, stream or None)
        self.lib._check(rc, "qgemm_dev")

    def gemm_noalloc(self, dx_ptr: int, dy_ptr: int, T: int, act: int = 0, stream: int = 0) -> None:
        """qgemm_dev through the allocation-free entry point (its scratch array)."""
        rc = self.lib.L.mynah_asr_hip_qgemm_noalloc_dev(self.h, dx_ptr, dy_ptr, T, act, stream or None)
        self.lib._check(rc, "qgemm_noalloc_dev")

    def noalloc_bytes(self, T: int) -> int:
        return int(self.lib.L.mynah_asr_hip_noalloc_bytes(self.h, T))

    def prep(self, dx_ptr: int, T: int, stream: int = 0) -> None:
        self.lib._check(self.lib.L.mynah_asr_hip_prep_dev(self.h, dx_ptr, T, stream or None), "prep_dev")

    def gemm_prepped(self, dy_ptr: int, T: int, act: int = 0, stream: int = 0) -> None:
        rc = self.lib.L.mynah_asr_hip_qgemm_prepped_dev(self.h, dy_ptr, T, act, stream or None)
        self.lib._check(rc, "qgemm_prepped_dev")

    def dequant(self, dwd_ptr: int, stream: int = 0) -> None:
        rc = self.lib.L.mynah_asr_hip_dequant_dev(self.h, dwd_ptr, stream or None)
        self.lib._check(rc, "dequant_dev")


def ffn_dev(lib, w1: "DeviceWeight", w2: "DeviceWeight", dx_ptr: int, dy_ptr: int, T: int, stream: int = 0):
    """dy = SiLU(dx . W1^T) . W2^T on device buffers (mynah_asr_hip_qffn_dev)."""
    lib._check(lib.L.mynah_asr_hip_qffn_dev(w1.h, w2.h, dx_ptr, dy_ptr, T, stream or None), "qffn_dev")


def qkv_dev(lib, ws, dx_ptr: int, dys, T: int, stream: int = 0):
    """Three products of one input, prepared once (mynah_asr_hip_qqkv_dev)."""
    rc = lib.L.mynah_asr_hip_qqkv_dev(ws[0].h, ws[1].h, ws[2].h, dx_ptr, dys[0], dys[1], dys[2], T, stream or None)
    lib._check(rc, "qqkv_dev")


def relpos_attention_dev(lib, q, k, v, rk, bias_u, bias_v, ctx, T: int, d: int, H: int,
                        left: int = -1, right: int = 0, nseq: int = 1, stream: int = 0):
    """Relative-position attention core on device pointers
    (mynah_asr_hip_relpos_attention_dev; src/encoder.c:315-410, 220-313)."""
    rc = lib.L.mynah_asr_hip_relpos_attention_dev(q, k, v, rk, bias_u, bias_v, ctx, T, d, H, left, right,
                                                 nseq, stream or None)
    lib._check(rc, "relpos_attention_dev")


def host_relpos_attention(lib, q, k, v, rk, bias_u, bias_v, H: int, left: int = -1, right: int = 0):
    """One segment on host arrays (mynah_asr_hip_relpos_attention): ctx [T, d]."""
    q, k, v, rk, bias_u, bias_v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, rk, bias_u, bias_v))
    T, d = q.shape
    ctx = np.empty((T, d), dtype=np.float32)
    rc = lib.L.mynah_asr_hip_relpos_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(rk), _ptr(bias_u), _ptr(bias_v),
                                             _ptr(ctx), T, d, H, left, right)
    lib._check(rc, "relpos_attention")
    return ctx


class Gguf:
    """A mapped GGUF file (host/gguf.h): `tensors()` lists (name, ggml type,
    ne, bytes); `qmat(name)` is the zero-copy qmat of one weight."""

    def __init__(self, lib: "HipLib", path: str):
        self.lib = lib
        err = C.create_string_buffer(256)
        self.h = lib.H.mynah_gguf_open(path.encode(), err, 256)
        if not self.h:
            raise ValueError(err.value.decode())

    def version(self) -> int:
        return int(self.lib.H.mynah_gguf_version(self.h))

    def alignment(self) -> int:
        return int(self.lib.H.mynah_gguf_alignment(self.h))

    def tensors(self):
        out = []
        for i in range(self.lib.H.mynah_gguf_count(self.h)):
            t = self.lib.H.mynah_gguf_at(self.h, i).contents
            raw = C.string_at(t.data, t.nbytes) if t.nbytes else b""
            out.append((t.name.decode("utf-8", "replace"), t.ggml_type, tuple(t.ne[:t.rank]), raw, t.data))
        return out

    def qmat(self, name: str) -> QMat:
        m = QMat()
        if self.lib.H.mynah_asr_qmat_init_gguf(C.byref(m), self.h, name.encode()) != 0:
            raise KeyError(name)
        return m

    def close(self):
        if self.h:
            self.lib.H.mynah_gguf_close(self.h)
            self.h = None


class DeviceAed:
    """An AED decoder on the device. `params` holds the reference's tensors
    (src/decoder_aed.h:12-36) as f32 arrays: emb, pos, embln_w/_b, fin_w/_b,
    head, head_b, optional proj/proj_b, and `layers`, a list of dicts with
    sq..ff2 ([n, k] weights), their *_b biases and ln_{self,cross,ffn}_{w,b}.
    Linears are quantized to `qtype` by the library's quantizers and made
    resident; everything else is copied to device tensors (torch)."""

    LINEARS = ("sq", "sk", "sv", "so", "cq", "ck", "cv", "co", "ff1", "ff2")

    def __init__(self, lib: "HipLib", params: dict, n_heads: int, qtype: int):
        import torch
        self.lib, self.torch = lib, torch
        self._keep = []
        self.weights = {}       # name -> Weight (host blocks, for the oracle's decoder)

        def dev(a):
            if a is None:
                return None
            t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()
            self._keep.append(t)
            return t.data_ptr()

        def lin(name, w):
            if w is None:
                return None
            hw = Weight.make(lib, qtype, np.asarray(w, np.float32))
            dw = DeviceWeight(lib, hw)
            self.weights[name] = hw
            self._keep.append(dw)
            return dw.h

        layers = params["layers"]
        self._layers = (AedLayerC * max(len(layers), 1))()
        for i, Ld in enumerate(layers):
            Lc = self._layers[i]
            for f, _ in AedLayerC._fields_:
                setattr(Lc, f, lin(f"{i}.{f}", Ld[f]) if f in self.LINEARS else dev(Ld[f]))
        d = params["emb"].shape[1]
        self.c = AedC(len(layers), d, n_heads, layers[0]["ff1"].shape[0] if layers else 1,
                      params["emb"].shape[0], params["pos"].shape[0])
        self.c.proj = lin("proj", params.get("proj"))
        self.c.proj_b = dev(params.get("proj_b"))
        for f in ("emb", "pos", "embln_w", "embln_b", "fin_w", "fin_b", "head_b"):
            setattr(self.c, f, dev(params[f]))
        self.c.head = lin("head", params["head"])
        self.c.layers = self._layers
        torch.cuda.synchronize()

    def forced(self, enc_ptr: int, T: int, tokens, stream: int = 0) -> np.ndarray:
        """Logits [n, vocab] of every position (mynah_asr_hip_aed_forced_dev)."""
        torch = self.torch
        tok = np.ascontiguousarray(tokens, dtype=np.int32)
        out = torch.empty((len(tok), self.c.vocab), dtype=torch.float32, device="cuda")
        rc = self.lib.L.mynah_asr_hip_aed_forced_dev(C.byref(self.c), enc_ptr, T, tok.ctypes.data, len(tok),
                                                     out.data_ptr(), stream or None)
        self.lib._check(rc, "aed_forced_dev")
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def decode(self, enc_ptr: int, T: int, prompt, eos: int, cap: int, stream: int = 0) -> list:
        """Greedy tokens (mynah_asr_hip_aed_decode_dev)."""
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        toks = np.zeros(max(cap, 1), dtype=np.int32)
        n = self.lib.L.mynah_asr_hip_aed_decode_dev(C.byref(self.c), enc_ptr, T, pr.ctypes.data, len(pr), eos,
                                                    toks.ctypes.data, cap, stream or None)
        if n < 0:
            raise RuntimeError(f"aed_decode_dev failed: {self.lib.last_error()}")
        return [int(t) for t in toks[:n]]

    def close(self):
        for k in self._keep:
            if isinstance(k, DeviceWeight):
                k.close()
        self._keep = []


class DeviceEncoderLayer:
    """One FastConformer encoder layer on the device. `params` holds the
    reference's tensors by their mynah_asr_enc_layer names (src/encoder.h:
    12-32) as f32 arrays ([n, k] weights; absent biases omitted or None).
    The linears are quantized to `qtype` by the library's quantizers and made
    resident, relk_w as an F32 weight (the reference keeps it f32); the rest
    are copied to device tensors. `weights` keeps the host blocks, for the
    oracle's dequantization."""

    LINEARS = ("ff1_w1", "ff1_w2", "q_w", "k_w", "v_w", "o_w", "relk_w", "pw1_w", "pw2_w", "ff2_w1", "ff2_w2")

    def __init__(self, lib: "HipLib", params: dict, qtype: int):
        import torch
        self.lib, self.torch = lib, torch
        self._keep, self.weights = [], {}
        self.c = EncLayerC()
        for f in EncLayerC.FIELDS:
            a = params.get(f)
            if a is None:
                continue
            if f in self.LINEARS:
                hw = Weight.make(lib, F32 if f == "relk_w" else qtype, np.asarray(a, np.float32))
                dw = DeviceWeight(lib, hw)
                self.weights[f] = hw
                self._keep.append(dw)
                setattr(self.c, f, dw.h)
            else:
                t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()
                self._keep.append(t)
                setattr(self.c, f, t.data_ptr())
        torch.cuda.synchronize()

    def run(self, x_ptr: int, T: int, nseq: int, pe_ptr: int, d: int, H: int, conv_k: int, causal: int,
            left: int = -1, right: int = 0, stream: int = 0) -> None:
        """mynah_asr_hip_encoder_layer_dev on x [nseq * T, d] in place."""
        rc = self.lib.L.mynah_asr_hip_encoder_layer_dev(C.byref(self.c), x_ptr, T, nseq, pe_ptr, d, H, conv_k, causal,
                                                        left, right, stream or None)
        self.lib._check(rc, "encoder_layer_dev")

    def close(self):
        for k in self._keep:
            if isinstance(k, DeviceWeight):
                k.close()
        self._keep = []


class DeviceSubsampling:
    """The dw_striding subsampling on the device. `params`: conv_in_w [C, 1,
    3, 3], conv_in_b, dw_w0/dw_w1 [C, 1, 3, 3], dw_b0/dw_b1, pw_w0/pw_w1
    [C, C] (or [C, C, 1, 1]), pw_b0/pw_b1, lin_w [d_model, C * F'], lin_b, as
    f32 arrays (src/subsampling.h:12-21). The pointwise convs and the linear
    become resident F32 weights."""

    def __init__(self, lib: "HipLib", params: dict, causal: int):
        import torch
        self.lib, self.torch = lib, torch
        self._keep = []

        def dev(a):
            t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32).reshape(-1)).cuda()
            self._keep.append(t)
            return t.data_ptr()

        def lin(a):
            a = np.asarray(a, np.float32)
            dw = DeviceWeight(lib, Weight.make(lib, F32, a.reshape(a.shape[0], -1)))
            self._keep.append(dw)
            return dw.h

        c = self.c = SubsamplingC()
        c.conv_in_w, c.conv_in_b = dev(params["conv_in_w"]), dev(params["conv_in_b"])
        for i in range(2):
            c.dw_w[i], c.dw_b[i] = dev(params[f"dw_w{i}"]), dev(params[f"dw_b{i}"])
            c.pw_w[i], c.pw_b[i] = lin(params[f"pw_w{i}"]), dev(params[f"pw_b{i}"])
        c.lin_w, c.lin_b = lin(params["lin_w"]), dev(params["lin_b"])
        c.channels, c.d_model, c.causal = params["conv_in_w"].shape[0], params["lin_w"].shape[0], causal
        torch.cuda.synchronize()

    def run(self, feats_ptr: int, T: int, nseq: int, n_mels: int, out_ptr: int, xscale: float = 1.0,
            stream: int = 0) -> int:
        """mynah_asr_hip_subsampling_dev: returns T' (rows per segment of out)."""
        t_out = C.c_int(0)
        rc = self.lib.L.mynah_asr_hip_subsampling_dev(C.byref(self.c), feats_ptr, T, nseq, n_mels, xscale, out_ptr,
                                                      C.byref(t_out), stream or None)
        self.lib._check(rc, "subsampling_dev")
        return t_out.value

    def close(self):
        for k in self._keep:
            if isinstance(k, DeviceWeight):
                k.close()
        self._keep = []


def evict(lib: HipLib, w: Weight) -> None:
    """Drop the resident copy keyed by w's host buffer (call before the buffer
    is freed: the cache is keyed by address, which numpy reuses)."""
    lib.L.mynah_asr_hip_evict(w.data.ctypes.data)


def host_qgemm(lib: HipLib, w: Weight, x: np.ndarray, keep: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty((x.shape[0], w.n), dtype=np.float32)
    rc = lib.L.mynah_asr_hip_qgemm(C.byref(w.desc), _ptr(x), _ptr(out), x.shape[0])
    if not keep:
        evict(lib, w)
    lib._check(rc, "qgemm")
    return out


def host_dequant(lib: HipLib, w: Weight, keep: bool = False) -> np.ndarray:
    out = np.empty((w.n, w.k), dtype=np.float32)
    rc = lib.L.mynah_asr_hip_dequant(C.byref(w.desc), _ptr(out))
    if not keep:
        evict(lib, w)
    lib._check(rc, "dequant")
    return out
