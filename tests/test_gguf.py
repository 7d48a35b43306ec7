"""The host mirror's GGUF reader (mynah-asr_amd/host/gguf.c) and
mynah_asr_qmat_init_gguf, pinned against the reference's own GGUF writer and
reader (third_party/ingot/src/write.c, gguf.c, compiled unmodified into
oracle/_ref): files written by ingot are read back tensor by tensor, byte for
byte, and files written by this test's own spec writer (other alignments,
version 2, every KV type) are read identically by both readers. Malformed
files are refused, never read past their end."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import mynah_hip as M
import oracle as O

GGML = {"F32": 0, "F16": 1, "BF16": 30, "Q4_0": 2, "Q8_0": 8, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}
QT_OF = {GGML["Q4_0"]: M.Q4_0, GGML["Q8_0"]: M.Q8_0, GGML["Q4_K"]: M.Q4_K, GGML["Q6_K"]: M.Q6_K,
         GGML["Q2_K"]: M.Q2_K}


# ------------------------------------------------------------ spec writer
def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, typ, val):
    out = _str(key) + struct.pack("<I", typ)
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
    if typ == 8:
        return out + _str(val)
    if typ == 9:
        et, items = val
        out += struct.pack("<IQ", et, len(items))
        return out + b"".join(_str(v) if et == 8 else struct.pack(fmt[et], v) for v in items)
    return out + struct.pack(fmt[typ], val)


def write_gguf(path, tensors, kvs=(), alignment=None, version=3):
    """tensors: (name, ggml type, ne tuple (ne[0] fastest), raw bytes)."""
    kv = list(kvs)
    if alignment is not None:
        kv.append(("general.alignment", 4, alignment))
    align = alignment or 32
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    head += b"".join(_kv(*e) for e in kv)
    off, offs = 0, []
    for _, _, _, raw in tensors:
        offs.append(off)
        off = (off + len(raw) + align - 1) // align * align
    for (name, typ, ne, raw), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
        head += struct.pack("<IQ", typ, o)
    data0 = (len(head) + align - 1) // align * align
    buf = bytearray(head + bytes(data0 - len(head)))
    for (_, _, _, raw), o in zip(tensors, offs):
        buf += bytes(data0 + o - len(buf)) + raw
    with open(path, "wb") as f:
        f.write(bytes(buf))


def sample_tensors(lib):
    w8 = lib.quantize(M.Q8_0, lib.randn(1, 0.02, (64, 256)))
    w4k = lib.quantize(M.Q4_K, lib.randn(2, 0.02, (32, 512)))
    w6k = lib.quantize(M.Q6_K, lib.randn(3, 0.02, (16, 256)))
    w40 = lib.quantize(M.Q4_0, lib.randn(4, 0.02, (8, 64)))
    f = lib.randn(5, 1.0, (8, 16))
    b = lib.randn(6, 1.0, (16,))
    return [("enc.l0.ffn1.weight", GGML["Q8_0"], (256, 64), w8.tobytes()),
            ("enc.l0.ffn2.weight", GGML["Q4_K"], (512, 32), w4k.tobytes()),
            ("dec.head.weight", GGML["Q6_K"], (256, 16), w6k.tobytes()),
            ("dec.small.weight", GGML["Q4_0"], (64, 8), w40.tobytes()),
            ("pos.weight", GGML["F32"], (16, 8), f.tobytes()),
            ("pos.bias", GGML["F32"], (16,), b.tobytes())]


# ------------------------------------------------------------ ingot (reference) side
def ingot_lib():
    if not O.IngotRef.available():
        pytest.skip("oracle/_ref not built (needs the reference tree at build time)")
    L = C.CDLL(O.REF_PATH)
    P = C.c_void_p
    L.ingot_gguf_writer_new.restype = P
    L.ingot_gguf_writer_free.argtypes = [P]
    L.ingot_gguf_kv_string.argtypes = [P, C.c_char_p, C.c_char_p]
    L.ingot_gguf_kv_u32.argtypes = [P, C.c_char_p, C.c_uint32]
    L.ingot_gguf_kv_f32.argtypes = [P, C.c_char_p, C.c_float]
    L.ingot_gguf_kv_bool.argtypes = [P, C.c_char_p, C.c_int]
    L.ingot_gguf_kv_array_string.argtypes = [P, C.c_char_p, C.POINTER(C.c_char_p), C.c_size_t]
    L.ingot_gguf_kv_array_f32.argtypes = [P, C.c_char_p, P, C.c_size_t]
    L.ingot_gguf_add_tensor.argtypes = [P, C.c_char_p, C.c_int, C.c_uint32, C.POINTER(C.c_uint64), P]
    L.ingot_gguf_writer_save.argtypes = [P, C.c_char_p, C.c_char_p, C.c_size_t]
    L.ingot_gguf_open.argtypes = [C.POINTER(P), C.c_char_p, C.c_char_p, C.c_size_t]
    L.ingot_gguf_close.argtypes = [P]
    L.ingot_gguf_count.restype = C.c_size_t
    L.ingot_gguf_count.argtypes = [P]
    L.ingot_gguf_at.restype = C.POINTER(IngotTensor)
    L.ingot_gguf_at.argtypes = [P, C.c_size_t]
    L.ingot_gguf_data.restype = P
    L.ingot_gguf_data.argtypes = [P, C.POINTER(IngotTensor)]
    return L


class IngotTensor(C.Structure):
    """ingot_tensor (third_party/ingot/include/ingot/gguf.h:40-49)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("rank", C.c_uint32), ("ne", C.c_uint64 * 8),
                ("nelem", C.c_uint64), ("nbytes", C.c_uint64), ("offset", C.c_uint64), ("shard", C.c_uint32)]


def ingot_read(L, path):
    g = C.c_void_p()
    err = C.create_string_buffer(256)
    assert L.ingot_gguf_open(C.byref(g), path.encode(), err, 256) == 0, err.value
    out = []
    for i in range(L.ingot_gguf_count(g)):
        tp = L.ingot_gguf_at(g, i)
        t = tp.contents
        out.append((t.name.decode("utf-8", "replace"), t.type, tuple(t.ne[:t.rank]),
                    C.string_at(L.ingot_gguf_data(g, tp), t.nbytes)))
    L.ingot_gguf_close(g)
    return out


def ours(lib, path):
    g = M.Gguf(lib, path)
    t = [(n, ty, ne, raw) for n, ty, ne, raw, _ in g.tensors()]
    v, a = g.version(), g.alignment()
    g.close()
    return t, v, a


# ------------------------------------------------------------ tests
def test_reads_files_written_by_the_reference_writer(lib, tmp_path):
    L = ingot_lib()
    tens = sample_tensors(lib)
    w = L.ingot_gguf_writer_new()
    assert L.ingot_gguf_kv_string(w, b"general.architecture", b"fastconformer") == 0
    assert L.ingot_gguf_kv_u32(w, b"enc.n_layers", 24) == 0
    assert L.ingot_gguf_kv_f32(w, b"enc.eps", 1e-5) == 0
    assert L.ingot_gguf_kv_bool(w, b"enc.causal", 0) == 0
    toks = (C.c_char_p * 3)(b"<pad>", b"<s>", b"</s>")
    assert L.ingot_gguf_kv_array_string(w, b"tokenizer.tokens", toks, 3) == 0
    arr = np.arange(5, dtype=np.float32)
    assert L.ingot_gguf_kv_array_f32(w, b"enc.scales", arr.ctypes.data, 5) == 0
    keep = []
    for name, typ, ne, raw in tens:
        buf = np.frombuffer(raw, dtype=np.uint8).copy()
        keep.append(buf)
        nea = (C.c_uint64 * len(ne))(*ne)
        assert L.ingot_gguf_add_tensor(w, name.encode(), typ, len(ne), nea, buf.ctypes.data) == 0, name
    path = str(tmp_path / "ingot.gguf")
    err = C.create_string_buffer(256)
    assert L.ingot_gguf_writer_save(w, path.encode(), err, 256) == 0, err.value
    L.ingot_gguf_writer_free(w)
    got, version, align = ours(lib, path)
    assert version == 3 and align == 32
    assert got == [(n, t, ne, raw) for n, t, ne, raw in tens]
    assert got == ingot_read(L, path)


@pytest.mark.parametrize("alignment,version", [(None, 3), (64, 3), (256, 2), (8, 3)])
def test_agrees_with_the_reference_reader(lib, tmp_path, alignment, version):
    L = ingot_lib()
    tens = sample_tensors(lib)
    kvs = [("general.name", 8, "t"), ("u8", 0, 7), ("i8", 1, -3), ("u16", 2, 9), ("i16", 3, -9),
           ("u32", 4, 11), ("i32", 5, -11), ("f32", 6, 0.5), ("b", 7, True), ("u64", 10, 1 << 40),
           ("i64", 11, -(1 << 40)), ("f64", 12, 0.25), ("strs", 9, (8, ["a", "bc", ""])),
           ("ints", 9, (5, [1, 2, 3]))]
    path = str(tmp_path / f"own_{alignment}_{version}.gguf")
    write_gguf(path, tens, kvs, alignment, version)
    got, v, a = ours(lib, path)
    assert v == version and a == (alignment or 32)
    assert got == [(n, t, ne, raw) for n, t, ne, raw in tens]
    assert got == ingot_read(L, path)


def test_malformed_files_are_refused(lib, tmp_path):
    tens = sample_tensors(lib)[:2]
    good = str(tmp_path / "good.gguf")
    write_gguf(good, tens, [("general.name", 8, "x")])
    blob = open(good, "rb").read()
    cases = {
        "magic": b"GGUX" + blob[4:],
        "version1": blob[:4] + struct.pack("<I", 1) + blob[8:],
        "header": blob[:20],
        "kv": blob[:40],
        "infos": blob[:120],
        "data": blob[:len(blob) - 100],
        "count": blob[:8] + struct.pack("<Q", 1 << 40) + blob[16:],
    }
    bad_align = str(tmp_path / "align.gguf")
    write_gguf(bad_align, tens, [], alignment=48)
    cases["alignment48"] = open(bad_align, "rb").read()
    # element counts whose byte size passes 2^64 (2^63 f32 elements: 2^65 bytes,
    # which wraps to 0 in 64 bits) over a zero-length payload
    wrap = str(tmp_path / "wrap.gguf")
    write_gguf(wrap, [("wrap", GGML["F32"], (1 << 62, 2, 1), b"")], [])
    cases["size_wraps"] = open(wrap, "rb").read()
    wrapq = str(tmp_path / "wrapq.gguf")
    write_gguf(wrapq, [("wrapq", GGML["Q8_0"], (1 << 58, 32), b"")], [])
    cases["block_size_wraps"] = open(wrapq, "rb").read()
    for what, data in cases.items():
        p = str(tmp_path / f"bad_{what}.gguf")
        with open(p, "wb") as f:
            f.write(data)
        with pytest.raises(ValueError):
            M.Gguf(lib, p)
    with pytest.raises(ValueError, match="cannot open"):
        M.Gguf(lib, str(tmp_path / "missing.gguf"))


def test_qmat_from_gguf_is_zero_copy(lib, tmp_path):
    tens = sample_tensors(lib)
    path = str(tmp_path / "w.gguf")
    write_gguf(path, tens)
    g = M.Gguf(lib, path)
    ptrs = {n: p for n, _, _, _, p in g.tensors()}
    m = g.qmat("enc.l0.ffn1.weight")
    assert (m.qtype, m.n, m.k) == (M.Q8_0, 64, 256) and m.blocks == ptrs["enc.l0.ffn1.weight"]
    m = g.qmat("enc.l0.ffn2.weight")
    assert (m.qtype, m.n, m.k) == (M.Q4_K, 32, 512) and m.blocks == ptrs["enc.l0.ffn2.weight"]
    m = g.qmat("pos.weight")
    assert (m.qtype, m.n, m.k) == (M.F32, 8, 16) and m.f32 == ptrs["pos.weight"]
    with pytest.raises(KeyError):
        g.qmat("pos.bias")          # 1-D: not a weight matrix
    with pytest.raises(KeyError):
        g.qmat("nope")
    g.close()


def test_half_tensors_decode_to_owned_f32(lib, tmp_path):
    """F16 and BF16 tensors become F32 qmats over an owned decoded copy, as
    the reference's loader decodes every non-F32 GGUF tensor at load
    (src/weights.c:90-104). The decoded values are checked against numpy's
    float16 conversion and, for BF16, against the f32 whose top half it is;
    every f16 bit pattern appears once (subnormals, infinities, NaNs)."""
    import ctypes as C
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(256, 256)
    f = np.random.default_rng(5).standard_normal((32, 64)).astype(np.float32)
    bf = (f.view(np.uint32) >> 16).astype(np.uint16)
    path = str(tmp_path / "h.gguf")
    write_gguf(path, [("h", GGML["F16"], (256, 256), h.tobytes()),
                      ("b", GGML["BF16"], (64, 32), bf.tobytes())])
    g = M.Gguf(lib, path)
    ptrs = {n: p for n, _, _, _, p in g.tensors()}
    for name, shape, want in (("h", (256, 256), h.view(np.float16).astype(np.float32)),
                              ("b", (32, 64), (bf.astype(np.uint32) << 16).view(np.float32))):
        m = g.qmat(name)
        try:
            assert (m.qtype, m.n, m.k) == (M.F32, shape[0], shape[1])
            assert m.f32 and m.f32 != ptrs[name]          # an owned copy, not the mapping
            got = np.ctypeslib.as_array(C.cast(m.f32, C.POINTER(C.c_uint32)), shape=shape).copy()
            nan = np.isnan(want)
            assert np.array_equal(got[~nan], want.view(np.uint32)[~nan])
            assert np.isnan(got.view(np.float32)[nan]).all()
            assert np.array_equal(got[nan] >> 31, want.view(np.uint32)[nan] >> 31)
        finally:
            lib.H.mynah_asr_qmat_free(C.byref(m))
    g.close()


@pytest.mark.gpu
def test_gguf_weights_on_the_device(gpu, orc, tmp_path):
    """Products from GGUF-mapped blocks equal the oracle's product over the
    decoded blocks (and the direct-blocks path bit for bit)."""
    H = gpu.H
    assert H.mynah_asr_set_backend(b"hip") == 3
    tens = [("a", GGML["Q8_0"], (1024, 96), gpu.quantize(M.Q8_0, gpu.randn(7, 0.02, (96, 1024))).tobytes()),
            ("b", GGML["Q4_K"], (1024, 64), gpu.quantize(M.Q4_K, gpu.randn(8, 0.02, (64, 1024))).tobytes())]
    path = str(tmp_path / "dev.gguf")
    write_gguf(path, tens)
    g = M.Gguf(gpu, path)
    x = gpu.randn(9, 1.0, (40, 1024))
    for name, typ, ne, raw in tens:
        n, k = ne[1], ne[0]
        m = g.qmat(name)
        out = np.empty((40, n), np.float32)
        H.mynah_asr_qmat_mul(C.byref(m), x.ctypes.data, out.ctypes.data, 40)
        blk = np.frombuffer(raw, dtype=np.uint8).copy()
        m2 = M.QMat()
        assert H.mynah_asr_qmat_init_blocks(C.byref(m2), blk.ctypes.data, n, k, QT_OF[typ]) == 0
        out2 = np.empty((40, n), np.float32)
        H.mynah_asr_qmat_mul(C.byref(m2), x.ctypes.data, out2.ctypes.data, 40)
        assert np.array_equal(out.view(np.uint32), out2.view(np.uint32)), name
        oq = {GGML["Q8_0"]: O.Q8_0, GGML["Q4_K"]: O.Q4_K}[typ]
        ref = orc.gemm_f64(x, orc.dequant(oq, blk, n * k).reshape(n, k))
        err = np.abs(out - ref)
        assert (err <= 1e-4 * np.abs(ref) + 1e-6).all(), name
        H.mynah_asr_qmat_free(C.byref(m))
        H.mynah_asr_qmat_free(C.byref(m2))
    g.close()
    # an F16 tensor: the decoded f32 copy runs on the device as an F32 qmat
    wh = gpu.randn(10, 0.02, (48, 1024)).astype(np.float16)
    write_gguf(path, [("h", GGML["F16"], (1024, 48), wh.tobytes())])
    g = M.Gguf(gpu, path)
    m = g.qmat("h")
    out = np.empty((40, 48), np.float32)
    H.mynah_asr_qmat_mul(C.byref(m), x.ctypes.data, out.ctypes.data, 40)
    ref = orc.gemm_f64(x, wh.astype(np.float32))
    assert (np.abs(out - ref) <= 1e-4 * np.abs(ref) + 1e-6).all()
    H.mynah_asr_qmat_free(C.byref(m))
    g.close()


def test_mutated_files_never_read_outside(lib, tmp_path):
    """Seeded mutation fuzz (as the reference fuzzes its reader,
    third_party/ingot/tests/fuzz_mutate.c): flipped bytes, overwritten
    length fields and truncations are either refused or parsed into tensors
    whose bytes lie inside the file; where both readers accept a file they
    agree on it."""
    L = ingot_lib() if O.IngotRef.available() else None
    tens = sample_tensors(lib)[:3]
    good = str(tmp_path / "seed.gguf")
    write_gguf(good, tens, [("general.name", 8, "x"), ("arr", 9, (8, ["a", "b"]))], alignment=64)
    blob = bytearray(open(good, "rb").read())
    rng = np.random.default_rng(1234)
    accepted = 0
    for i in range(300):
        b = bytearray(blob)
        kind = i % 3
        if kind == 0:                      # a few random byte flips in the header and tables
            for _ in range(rng.integers(1, 4)):
                b[rng.integers(0, min(len(b), 600))] ^= int(rng.integers(1, 256))
        elif kind == 1:                    # a huge or odd value over an 8-byte field
            o = int(rng.integers(8, min(len(b), 600) - 8))
            vals = [0, 1, 1 << 31, 1 << 40, (1 << 64) - 1]
            b[o:o + 8] = struct.pack("<Q", vals[int(rng.integers(0, len(vals)))])
        else:                              # truncation
            b = b[:int(rng.integers(0, len(b)))]
        p = str(tmp_path / f"m{i}.gguf")
        with open(p, "wb") as f:
            f.write(bytes(b))
        try:
            g = M.Gguf(lib, p)
        except ValueError:
            continue
        accepted += 1
        for name, typ, ne, raw, ptr in g.tensors():
            assert len(raw) <= len(b)
        g.close()
        if L is not None:
            gi = C.c_void_p()
            err = C.create_string_buffer(256)
            if L.ingot_gguf_open(C.byref(gi), p.encode(), err, 256) == 0:
                L.ingot_gguf_close(gi)
                ours_t, _, _ = ours(lib, p)
                theirs = ingot_read(L, p)
                # names, types and shapes agree wherever both read every tensor
                assert [(n, t, ne) for n, t, ne, _ in ours_t] == [(n, t, ne) for n, t, ne, _ in theirs]
    assert accepted > 0   # some mutations (in payload bytes, unused fields) still parse
