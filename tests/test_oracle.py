"""Pins the CPU oracle before anything is compared against it.

Every oracle function is checked against something that is not the oracle:
the reference's own known-answer fixtures (llama.cpp dequantizer output,
third_party/ingot/tests/fixtures), the reference's ingot sources compiled from
/root/reference (oracle/_ref), brute force in Python integers, and closed forms.
"""
import os

import numpy as np
import pytest

import oracle as O

FIX = os.path.join(os.path.dirname(__file__), "golden", "ingot_fixtures")


def _fixtures():
    out = []
    for line in open(os.path.join(FIX, "manifest.txt")):
        name, t, be, bb, nb = line.split()
        out.append((name, int(t), int(be), int(bb), int(nb)))
    return out


@pytest.mark.parametrize("name,t,be,bb,nb", _fixtures())
def test_decoders_match_llamacpp_fixtures(orc, name, t, be, bb, nb):
    """ingot tests/test_oracle.c:149-157 gates at rel 1e-5; decoded values are
    exact products, so the oracle must match bit for bit."""
    raw = np.fromfile(os.path.join(FIX, name + ".bin"), dtype=np.uint8)
    ref = np.fromfile(os.path.join(FIX, name + ".ref"), dtype=np.float32)
    assert raw.size == nb * bb and ref.size == nb * be  # geometry (fixtures/geometry.txt)
    got = orc.dequant(t, raw, nb * be)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_f16_decode_exhaustive(orc, ingot_ref):
    for h in range(65536):
        a = np.float32(orc.f16_to_f32(h)).view(np.uint32)
        b = np.float32(ingot_ref.L.ingot_f16_to_f32(h)).view(np.uint32)
        assert a == b, hex(h)


def test_f16_known_values(orc):
    assert orc.f16_to_f32(0x3C00) == 1.0
    assert orc.f16_to_f32(0xC000) == -2.0
    assert orc.f16_to_f32(0x7BFF) == 65504.0
    assert orc.f16_to_f32(0x0001) == 2.0 ** -24
    assert orc.f16_to_f32(0x7C00) == float("inf")
    assert np.isnan(orc.f16_to_f32(0x7E00))
    assert orc.f32_to_f16(1.0) == 0x3C00
    assert orc.f32_to_f16(65520.0) == 0x7C00          # rounds past the largest finite
    assert orc.f32_to_f16(1.0 + 2.0 ** -11) == 0x3C00  # tie to even
    assert orc.f32_to_f16(1.0 + 3 * 2.0 ** -11) == 0x3C02


def test_f16_encode_vs_reference(orc, ingot_ref):
    rng = np.random.default_rng(7)
    xs = np.concatenate([rng.standard_normal(4000).astype(np.float32) * s
                         for s in (1e-9, 3e-6, 1e-4, 1e-2, 1.0, 300.0, 7e4)])
    for v in xs:
        assert orc.f32_to_f16(float(v)) == ingot_ref.L.ingot_f32_to_f16(float(v))


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.Q4_K, O.Q6_K])
def test_quantizers_match_reference(orc, ingot_ref, t):
    rng = np.random.default_rng(11 + t)
    x = (rng.standard_normal(256 * 96) * 0.02).astype(np.float32)
    x[:256] = 0.0                                   # all-zero block
    x[256:512] = np.abs(x[256:512])                  # one-signed block
    x[512:768] = np.round(x[512:768] * 1000) / 1000  # ties
    assert np.array_equal(orc.quantize(t, x), ingot_ref.quantize(t, x))


@pytest.mark.parametrize("t", [O.Q4_0, O.Q8_0, O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K])
def test_decoders_match_reference_on_random_blocks(orc, ingot_ref, t):
    be, bb = O.GEOMETRY[t]
    rng = np.random.default_rng(100 + t)
    raw = rng.integers(0, 256, size=bb * 40, dtype=np.uint8)
    # keep the f16 factors finite and moderate (the gen_kquant_ref recipe)
    for b in range(40):
        blk = raw[b * bb:(b + 1) * bb]
        for off in {O.Q4_0: [0], O.Q8_0: [0], O.Q2_K: [80, 82], O.Q3_K: [108],
                    O.Q4_K: [0, 2], O.Q5_K: [0, 2], O.Q6_K: [208]}[t]:
            blk[off:off + 2] = np.frombuffer(np.float16(rng.uniform(1e-3, 1e-1)).tobytes(), np.uint8)
    a = orc.dequant(t, raw, 40 * be)
    b = ingot_ref.dequant(t, raw, 40 * be)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q8_0_quantizer_closed_form(orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 200) * 0.02).astype(np.float32)
    raw = orc.quantize(O.Q8_0, x).reshape(200, 34)
    for b in range(200):
        blk = x[32 * b:32 * b + 32]
        d16 = raw[b, :2].view(np.float16)[0]
        q = raw[b, 2:].view(np.int8).astype(np.int32)
        amax = np.abs(blk).max()
        assert d16 == np.float16(amax / np.float32(127))
        assert np.abs(q).max() == 127 and q[np.argmax(np.abs(blk))] == np.sign(blk[np.argmax(np.abs(blk))]) * 127
        # q = lroundf(x * (1/d)) with the f32 d before f16 rounding
        d = np.float32(amax) / np.float32(127)
        id_ = np.float32(1) / d
        v = (blk * id_).astype(np.float64)
        want = np.where(v >= 0, np.floor(v + 0.5), -np.floor(-v + 0.5)).astype(np.int32)
        assert np.array_equal(q, np.clip(want, -127, 127))


def test_q8_0_ties_round_away(orc):
    x = np.zeros(32, dtype=np.float32)
    x[0] = 127.0
    x[1] = 2.5
    x[2] = -2.5
    x[3] = 0.5
    raw = orc.quantize(O.Q8_0, x)
    q = raw[2:].view(np.int8)
    assert list(q[:4]) == [127, 3, -3, 1]


def test_qmat_int8_quantizer_brute(orc):
    rng = np.random.default_rng(5)
    w = rng.uniform(-1, 1, size=(7, 64)).astype(np.float32)
    w[3] = 0.0
    q, s = orc.qmat_quantize_int8(w)
    for r in range(7):
        amax = np.float32(np.abs(w[r]).max())
        sc = amax / np.float32(127) if amax > 0 else np.float32(1)
        assert s[r] == sc
        inv = np.float32(1) / sc
        for j in range(64):
            v = np.float32(w[r, j] * inv)
            want = int(v + np.float32(0.5)) if v >= 0 else int(v - np.float32(0.5))
            assert q[r, j] == want


def test_qmat_int4_layout_and_range(orc):
    rng = np.random.default_rng(6)
    w = rng.uniform(-1, 1, size=(3, 64)).astype(np.float32)
    q, s = orc.qmat_quantize_int4(w)
    wd = orc.qmat_dequant(2, q, s, 3, 64)
    # element 2j in the low nibble of byte j, 2j+1 in the high nibble
    lo = (q & 15).astype(np.int32) - 8
    hi = (q >> 4).astype(np.int32) - 8
    vals = np.empty((3, 64), dtype=np.int32)
    vals[:, 0::2], vals[:, 1::2] = lo, hi
    assert vals.min() >= -8 and vals.max() <= 7
    expect = vals.astype(np.float32) * np.repeat(s, 32, axis=1)
    assert np.array_equal(wd, expect)
    assert np.abs(wd - w).max() <= np.repeat(s, 32, axis=1).max() * 0.5 + 1e-7


def test_act_quant_special_cases(orc):
    q, s = orc.act_quant_int8(np.zeros(16, np.float32))
    assert s == 0.0 and not q.any()
    x = np.array([127.0, 63.5, -63.5, 0.49, -127.0] + [0.0] * 11, dtype=np.float32)
    q, s = orc.act_quant_int8(x)
    assert s == np.float32(1.0)
    assert list(q[:5]) == [127, 64, -64, 0, -127]   # half away from zero


@pytest.mark.parametrize("qtype", [1, 2])
def test_int8_path_sums_brute(orc, qtype):
    rng = np.random.default_rng(9 + qtype)
    n, k, T = 5, 96, 3
    w = rng.uniform(-1, 1, size=(n, k)).astype(np.float32)
    x = rng.standard_normal((T, k)).astype(np.float32)
    q, s = (orc.qmat_quantize_int8 if qtype == 1 else orc.qmat_quantize_int4)(w)
    out, sums = orc.qmat_int8_path(qtype, q, s, n, k, x)
    for t in range(T):
        qx, sx = orc.act_quant_int8(x[t])
        qx = qx.astype(np.int64)
        for r in range(n):
            if qtype == 1:
                assert sums[t, r] == int((q[r].astype(np.int64) * qx).sum())
                assert out[t, r] == np.float32(np.float32(sums[t, r]) * s[r]) * np.float32(sx)
            else:
                vals = np.empty(k, dtype=np.int64)
                vals[0::2] = (q[r] & 15).astype(np.int64) - 8
                vals[1::2] = (q[r] >> 4).astype(np.int64) - 8
                for g in range(k // 32):
                    assert sums[t, r, g] == int((vals[32 * g:32 * g + 32] * qx[32 * g:32 * g + 32]).sum())


def test_gemm_f64_closed_forms(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 40)).astype(np.float32)
    eye = np.eye(40, dtype=np.float32)
    assert np.array_equal(orc.gemm_f64(x, eye), x.astype(np.float64))       # identity
    onehot = np.zeros((3, 40), np.float32)
    onehot[0, 5] = 2.0
    onehot[1, 39] = -1.0
    y = orc.gemm_f64(x, onehot)
    assert np.array_equal(y[:, 0], 2.0 * x[:, 5].astype(np.float64))
    assert np.array_equal(y[:, 1], -x[:, 39].astype(np.float64))
    assert not y[:, 2].any()
    u = rng.standard_normal(40).astype(np.float32)                            # rank one
    v = rng.standard_normal(3).astype(np.float32)
    w = np.outer(v, u).astype(np.float32)
    y = orc.gemm_f64(x, w)
    np.testing.assert_allclose(y, x.astype(np.float64) @ w.T.astype(np.float64), rtol=1e-12, atol=1e-12)
