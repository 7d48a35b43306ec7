"""The oracle's INT8ACT over ggml block formats (orc_int8act_blocks,
orc_kquant_ints, orc_act_quant_sb) pinned:
  * the integer decode of every K-quant rebuilds the reference decoders'
    f32 output bit for bit (the decoders are pinned to llama.cpp fixtures);
  * ingot's activation quantizer by closed forms (round-to-nearest-even, the
    block maximum maps to +-127, all-zero blocks);
  * the whole product against the reference's own int8-activation path
    (ingot_q4_k_matmat / ingot_q5_k_matmat, compiled from the reference's
    sources with its x86 SIMD flags): the same integer sums, another f32
    order, so within 1e-6 relative L2;
  * the f32 evaluation order by an independent restatement in exact rational
    arithmetic (every f32 operation rounded once, as IEEE does), bit for bit;
  * the precision contract of the reference's int8 path: relative L2 error
    against the exact product below 5e-3 on the reference's own test case
    (third_party/ingot/tests/test_quant.c:157-205)."""
import os
import sys
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "mynah-asr_amd"))

KQ = [O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K]
FIX = os.path.join(os.path.dirname(__file__), "golden", "ingot_fixtures")


def random_blocks(qt, nblocks, seed):
    """Random bytes with small finite f16 scales (the recipe of the reference's
    tools/gen_kquant_ref.py: any bit pattern is a valid block)."""
    r = np.random.default_rng(seed)
    be, bb = O.GEOMETRY[qt]
    raw = r.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    offs = {O.Q2_K: (80, 82), O.Q3_K: (108,), O.Q4_K: (0, 2), O.Q5_K: (0, 2), O.Q6_K: (208,), O.Q8_0: (0,),
            O.Q4_0: (0,)}[qt]
    for o in offs:
        h = (r.standard_normal(nblocks) * 0.01).astype(np.float16)
        raw[:, o:o + 2] = h.view(np.uint8).reshape(nblocks, 2)
    return raw.ravel()


@pytest.mark.parametrize("qt", KQ, ids=lambda q: O.NAMES[q])
def test_kquant_ints_rebuild_the_decoder(orc, qt):
    be, bb = O.GEOMETRY[qt]
    blocks = [random_blocks(qt, 40, 7 + qt).reshape(40, bb)]
    fx = os.path.join(FIX, O.NAMES[qt] + ".bin")
    if os.path.exists(fx):
        blocks.append(np.fromfile(fx, dtype=np.uint8).reshape(-1, bb))
    sub = 32 if qt in (O.Q4_K, O.Q5_K) else 16
    for bl in blocks:
        ref = orc.dequant(qt, bl.ravel(), bl.shape[0] * 256).reshape(-1, 256)
        for i in range(bl.shape[0]):
            q, f, m, d, dmin = orc.kquant_ints(qt, bl[i])
            fj = np.repeat(f[:256 // sub], sub).astype(np.float32)
            mj = np.repeat(m[:256 // sub], sub).astype(np.float32)
            sc = (d * fj).astype(np.float32)
            w = (sc * q.astype(np.float32)).astype(np.float32)
            if qt in (O.Q2_K, O.Q4_K, O.Q5_K):
                w = (w - (dmin * mj).astype(np.float32)).astype(np.float32)
            assert np.array_equal(w.view(np.uint32), ref[i].view(np.uint32)), (O.NAMES[qt], i)


def test_act_quant_sb_closed_forms(orc):
    # amax 127: the scale is 1 and inverse 1, so q = rne(x)
    x = np.zeros(256, np.float32)
    x[0] = 127.0
    x[1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.49999988, -126.5]
    q, s = orc.act_quant_sb(x)
    assert s == np.float32(1.0)
    assert list(q[:9]) == [127, 2, 4, -2, -4, 0, 0, 1, -126]
    # the block maximum maps to +-127, everything within [-127, 127]
    r = np.random.default_rng(3).standard_normal(256).astype(np.float32) * 3
    q, s = orc.act_quant_sb(r)
    i = int(np.argmax(np.abs(r)))
    assert q[i] == np.sign(r[i]) * 127 and np.abs(q).max() == 127
    assert s == np.float32(np.float32(np.abs(r).max()) / np.float32(127.0))
    inv = np.float32(127.0) / np.float32(np.abs(r).max())
    assert np.array_equal(q, np.rint((r * inv).astype(np.float32)).astype(np.int8))
    q, s = orc.act_quant_sb(np.zeros(256, np.float32))
    assert s == 0.0 and not q.any()


# ------------------------------------------------ exact-arithmetic restatement
def rnd32(v) -> np.float32:
    """A rational rounded to the nearest f32 (ties to even)."""
    v = Fraction(v)
    if v == 0:
        return np.float32(0.0)
    sgn, a = (-1 if v < 0 else 1), abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    qn, rem = divmod(a.numerator * ulp.denominator, a.denominator * ulp.numerator)
    twice = 2 * rem
    den = a.denominator * ulp.numerator
    if twice > den or (twice == den and qn % 2):
        qn += 1
    return np.float32(sgn * float(qn * ulp))


def fma32(a, b, c):
    return rnd32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def mul32(a, b):
    return rnd32(Fraction(float(a)) * Fraction(float(b)))


def restated(orc, qt, raw, n, k, x):
    """orc_int8act_blocks' order, restated independently."""
    be, bb = O.GEOMETRY[qt]
    T = x.shape[0]
    Kc = (k + 127) // 128
    out = np.zeros((T, n), np.float32)
    for t in range(T):
        if be == 32:
            qx, sx = orc.act_quant_int8(x[t])
            qx = np.concatenate([qx.astype(np.int64), np.zeros(Kc * 128 - k, np.int64)])
        else:
            qs = [orc.act_quant_sb(x[t, 256 * b:256 * b + 256]) for b in range(k // 256)]
        for r in range(n):
            total = np.float32(0.0)
            for c in range(Kc):
                if be == 32:
                    acc = np.float32(0.0)
                    for b in range(4 * c, min(4 * c + 4, k // 32)):
                        blk = raw[(r * (k // 32) + b) * bb:(r * (k // 32) + b + 1) * bb]
                        d = np.frombuffer(blk[:2].tobytes(), np.float16)[0].astype(np.float32)
                        if qt == O.Q8_0:
                            qw = blk[2:34].view(np.int8).astype(np.int64)
                        else:
                            qw = np.concatenate([blk[2:18] & 15, blk[2:18] >> 4]).astype(np.int64) - 8
                        tb = int((qw * qx[32 * b:32 * b + 32]).sum())
                        acc = fma32(d, np.float32(tb), acc)
                    total = fma32(np.float32(sx), acc, total)
                else:
                    B, e0 = c // 2, 128 * (c % 2)
                    blk = raw[(r * (k // 256) + B) * bb:(r * (k // 256) + B + 1) * bb]
                    q, f, m, d, dmin = orc.kquant_ints(qt, blk)
                    xq, xs = qs[B]
                    xq = xq.astype(np.int64)
                    sub = 32 if qt in (O.Q4_K, O.Q5_K) else 16
                    if qt == O.Q6_K:
                        acc = np.float32(0.0)
                        for j in range(e0 // 16, e0 // 16 + 8):
                            tj = int((q[16 * j:16 * j + 16].astype(np.int64) * xq[16 * j:16 * j + 16]).sum())
                            acc = fma32(mul32(d, np.float32(f[j])), np.float32(tj), acc)
                    else:
                        A = sum(int(q[e]) * int(f[e // sub]) * int(xq[e]) for e in range(e0, e0 + 128))
                        Af = rnd32(A)      # one rounding of the exact integer (exact below 2^24)
                        if qt == O.Q3_K:
                            acc = mul32(d, Af)
                        else:
                            Bm = sum(int(m[j]) * int(xq[sub * j:sub * j + sub].sum())
                                     for j in range(e0 // sub, (e0 + 128) // sub))
                            acc = fma32(-mul32(dmin, np.float32(32.0)), rnd32(Fraction(Bm, 32)), mul32(d, Af))
                    total = fma32(xs, acc, total)
            out[t, r] = total
    return out


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_0] + KQ, ids=lambda q: O.NAMES[q])
def test_int8act_order_restated_exactly(orc, qt):
    be, _ = O.GEOMETRY[qt]
    n, T = 3, 2
    k = 288 if be == 32 else 512          # Q8_0 / Q4_0: a ragged last chunk
    raw = random_blocks(qt, n * k // be, 90 + qt)
    x = np.random.default_rng(91).standard_normal((T, k)).astype(np.float32)
    x[1, :40] *= 50.0                      # one block with a far larger maximum
    got, _ = orc.int8act_blocks(qt, raw, n, k, x)
    want = restated(orc, qt, raw, n, k, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (got, want)


@pytest.mark.parametrize("qt", [O.Q4_K, O.Q5_K], ids=lambda q: O.NAMES[q])
def test_int8act_matches_reference_int8_path(orc, qt):
    if not os.path.exists(O.REF_AVX2_PATH):
        pytest.skip("oracle/_ref not built (needs the reference tree at build time)")
    R = O.IngotRef(O.REF_AVX2_PATH)
    if R.is_exact(2):
        pytest.skip("this host's CPU lacks AVX2: the reference's int8 path is not compiled in")
    import mynah_hip as M
    lib = M.HipLib()
    n, k = 96, 1024
    raw = lib.quantize({O.Q4_K: M.Q4_K, O.Q5_K: M.Q5_K}[qt], lib.randn(0, 0.02, (n, k)))
    x = lib.randn(1, 1.0, (33, k))
    ours, _ = orc.int8act_blocks(qt, raw, n, k, x)
    ref = R.kernel({O.Q4_K: "ingot_q4_k_matmat", O.Q5_K: "ingot_q5_k_matmat"}[qt], raw, n, k, x)
    rel = np.linalg.norm(ours - ref) / np.linalg.norm(ref)
    assert rel < 1e-6, rel


def test_int8act_budget_on_reference_case(orc):
    """test_quant.c:157-205: 37 rows of 0.02 * uniform(-1, 1) quantized to Q4_K,
    131 tokens of uniform(-1, 1); the int8 path within 5e-3 relative L2 of the
    exact product."""
    r = np.random.default_rng(0xC0FFEE)
    w = (0.02 * r.uniform(-1, 1, (37, 256))).astype(np.float32)
    raw = orc.quantize(O.Q4_K, w)
    x = r.uniform(-1, 1, (131, 256)).astype(np.float32)
    ours, _ = orc.int8act_blocks(O.Q4_K, raw, 37, 256, x)
    ex = orc.gemm_f64(x, orc.dequant(O.Q4_K, raw, 37 * 256).reshape(37, 256))
    rel = np.linalg.norm(ours - ex) / np.linalg.norm(ex)
    assert rel < 5e-3, rel


BLOCK_FORMATS = ["Q8_0", "Q4_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]


def _budget_case(orc, lib, name, rows, cols, tokens, weights, acts):
    import mynah_hip as M
    raw = lib.quantize(getattr(M, name), weights)
    oq = getattr(O, name)
    ours, _ = orc.int8act_blocks(oq, raw, rows, cols, acts)
    ex = orc.gemm_f64(acts, orc.dequant(oq, raw, rows * cols).reshape(rows, cols))
    return float(np.linalg.norm(ours - ex) / np.linalg.norm(ex))


@pytest.mark.parametrize("name", BLOCK_FORMATS)
def test_int8act_budget_every_block_format(orc, name):
    """The reference's int8 precision contract (test_quant.c:157-205: 37 rows
    of 0.02 * uniform(-1, 1), 131 tokens of uniform(-1, 1), 256 columns,
    relative L2 against the exact product below 5e-3) for every block format.
    Only Q4_K and Q5_K have an int8 path in the reference
    (kernels.c:1767-1791, 2325-2353); for Q8_0, Q4_0, Q2_K, Q3_K and Q6_K the
    INT8ACT form is this build's own extension, and this is the check that
    pins its error. Weights through the build's quantizers (host/synth.c).
    Measured: 3.86e-3 for every format. The same activations drawn N(0, 1) at
    K = 1024 give 6.9e-3 (K-quants, per-256 activation scales) and 7.8e-3
    (Q8_0 / Q4_0, per-row scales): the 5e-3 figure holds for the reference's
    case, not for any input; that second case is bounded at 1e-2 here."""
    import mynah_hip as M
    lib = M.HipLib()
    r = np.random.default_rng(0xC0FFEE)
    w = (0.02 * r.uniform(-1, 1, (37, 256))).astype(np.float32)
    x = r.uniform(-1, 1, (131, 256)).astype(np.float32)
    rel = _budget_case(orc, lib, name, 37, 256, 131, w, x)
    assert rel < 5e-3, rel
    w2 = lib.randn(0, 0.02, (64, 1024))
    x2 = lib.randn(1, 1.0, (64, 1024))
    rel2 = _budget_case(orc, lib, name, 64, 1024, 64, w2, x2)
    assert 5e-3 < rel2 < 1e-2, rel2
