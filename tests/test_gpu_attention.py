"""GPU parity of the relative-position attention core
(mynah_asr_hip_relpos_attention_dev) against the oracle's float64 restatement
of src/encoder.c:315-410 (full) and :220-313 (chunked-limited).

Bar: |ctx - ref| <= 1e-4*|ref| + 1e-5*max|v| per element. The kernel computes
in f32 like the reference, with another summation order and base-2
exponentials (full attention forms its scores from f16 hi + lo splits of
row-scaled operands, 22 bits of each row's maximum), so a context element near
zero (a cancelling weighted sum of v) carries an absolute error of order
1e-6 * max|v| — the scale term covers that.
Inputs: q, k, v, rk N(0, 1) and bias_u, bias_v N(0, 0.1), seeded.
"""
import sys

import numpy as np
import pytest

import mynah_hip as M
from attention import relpos_attention

pytestmark = pytest.mark.gpu
RTOL, VTOL = 1e-4, 1e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make(seed, T, d, nseq=1):
    r = np.random.default_rng(seed)
    f = lambda *s, sc=1.0: (r.standard_normal(s) * sc).astype(np.float32)
    return (f(nseq, T, d), f(nseq, T, d), f(nseq, T, d), f(2 * T - 1, d), f(d, sc=0.1), f(d, sc=0.1))


def run_gpu(gpu, arrs, T, d, H, left, right, nseq):
    import torch
    q, k, v, rk, bu, bv = (torch.from_numpy(a).cuda() for a in arrs)
    ctx = torch.full((nseq, T, d), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    M.relpos_attention_dev(gpu, q.data_ptr(), k.data_ptr(), v.data_ptr(), rk.data_ptr(), bu.data_ptr(),
                           bv.data_ptr(), ctx.data_ptr(), T, d, H, left, right, nseq)
    torch.cuda.synchronize()
    return ctx.cpu().numpy()


def check(out, arrs, H, left, right):
    q, k, v, rk, bu, bv = arrs
    for s in range(q.shape[0]):
        ref = relpos_attention(q[s], k[s], v[s], rk, bu, bv, H, left, right)
        err = np.abs(out[s] - ref)
        lim = RTOL * np.abs(ref) + VTOL * np.abs(v[s]).max()
        assert np.isfinite(out[s]).all()
        assert (err <= lim).all(), (f"seg {s}: {int((err > lim).sum())} outside, max err {err.max():.3g}, "
                                    f"worst ratio {(err / lim).max():.3g}")


@pytest.mark.parametrize("T,d,H,left,right,nseq", [
    (1, 128, 2, -1, 0, 1),        # one frame
    (37, 128, 2, -1, 0, 1),       # dk 64, ragged tiles
    (64, 256, 2, -1, 0, 1),       # dk 128, one exact row block
    (65, 256, 2, -1, 0, 2),       # one row past a block, two segments
    (130, 256, 2, 32, 7, 1),      # chunked: chunk 8, 4 chunks of left context
    (130, 256, 2, 4, 3, 3),       # chunked: chunk 4, one chunk of left context
    (200, 512, 4, 0, 0, 1),       # chunk 1, no left context: each row sees itself only
    (300, 256, 4, 70, 13, 1),     # chunk 14, lc 5, T not a multiple of the chunk
    (300, 512, 4, 1000, 299, 1),  # one chunk covering all rows: equals full attention
])
def test_relpos_attention_matches_oracle(gpu, T, d, H, left, right, nseq):
    say("attention", T, d, H, left, right, nseq)
    arrs = make(T * 7 + d, T, d, nseq)
    out = run_gpu(gpu, arrs, T, d, H, left, right, nseq)
    check(out, arrs, H, left, right)


def test_relpos_attention_fastconformer_segment(gpu):
    """FastConformer-0.6B: d_model 1024, 8 heads (dk 128), one 750-frame
    segment, full attention and the streaming chunked-limited window."""
    T, d, H = 750, 1024, 8
    arrs = make(11, T, d, 2)
    for left, right in ((-1, 0), (70, 13)):
        say("attention fastconformer", T, left, right)
        out = run_gpu(gpu, arrs, T, d, H, left, right, 2)
        check(out, arrs, H, left, right)


@pytest.mark.parametrize("d", [256, 128])
def test_relpos_attention_many_segments(gpu, d):
    """Enough segments for the eight-wave (128-row) kernel variant, dk 128 and 64."""
    T, H, nseq = 200, 2, 128
    say("attention many segments", T, d, H, nseq)
    arrs = make(21 + d, T, d, nseq)
    out = run_gpu(gpu, arrs, T, d, H, -1, 0, nseq)
    check(out, arrs, H, -1, 0)


@pytest.mark.parametrize("left,right", [(-1, 0), (1000, 299)])
def test_relpos_attention_wide_row_scales(gpu, left, right):
    """Rows of q, k and rk scaled by 2^-30 .. 2^30, rows of zeros, and rows
    with one feature 1e4 times the rest; V's features scaled by 2^-20 .. 2^20
    with a zero key tile: the split operands carry each row's (V: each key
    tile and feature's) own scale, so the bar holds as for N(0, 1) inputs
    (full attention on the split path, and the one-chunk window, the same
    products on the f32 path)."""
    T, d, H = 150, 256, 2
    r = np.random.default_rng(77)
    q, k, v, rk, bu, bv = make(41, T, d, 1)
    for a, n in ((q[0], T), (k[0], T), (rk, 2 * T - 1)):
        a *= np.exp2(r.integers(-30, 31, size=(n, 1))).astype(np.float32)
        a[r.integers(0, n, size=5)] = 0.0
        a[r.integers(0, n, size=5), r.integers(0, d, size=5)] *= 1e4
    # V: features scaled by 2^-20 .. 2^20 (its split carries one exponent per
    # key tile and feature), a zero tile of keys, zero rows
    v[0] *= np.exp2(r.integers(-20, 21, size=(1, d))).astype(np.float32)
    v[0, 32:64] = 0.0
    v[0, r.integers(0, T, size=5)] = 0.0
    bu[:] = 0.0
    bv[:] = 0.0
    say("attention wide row scales", left, right)
    arrs = (q, k, v, rk, bu, bv)
    out = run_gpu(gpu, arrs, T, d, H, left, right, 1)
    # the bar per feature: a context column's error scales with that column of V
    ref = relpos_attention(q[0], k[0], v[0], rk, bu, bv, H, left, right)
    err = np.abs(out[0] - ref)
    lim = RTOL * np.abs(ref) + VTOL * np.abs(v[0]).max(axis=0, keepdims=True)
    assert np.isfinite(out[0]).all()
    assert (err <= lim).all(), f"{int((err > lim).sum())} outside, worst ratio {(err / lim).max():.3g}"


def test_relpos_attention_segments_independent(gpu):
    """A segment's context does not depend on the other segments of the call
    (bit-identical to running it alone)."""
    T, d, H = 97, 256, 2
    for nseq in (3, 256):   # the four- and the eight-wave kernel
        arrs = make(5, T, d, nseq)
        many = run_gpu(gpu, arrs, T, d, H, -1, 0, nseq)
        one = run_gpu(gpu, tuple(a[1:2] if a.ndim == 3 else a for a in arrs), T, d, H, -1, 0, 1)
        assert np.array_equal(many[1].view(np.uint32), one[0].view(np.uint32))


def test_relpos_attention_host_entry(gpu):
    """The host-pointer entry point gives the device entry point's bits."""
    T, d, H = 150, 256, 2
    arrs = make(31, T, d, 1)
    for left, right in ((-1, 0), (20, 4)):
        dev = run_gpu(gpu, arrs, T, d, H, left, right, 1)[0]
        q, k, v, rk, bu, bv = arrs
        host = M.host_relpos_attention(gpu, q[0], k[0], v[0], rk, bu, bv, H, left, right)
        assert np.array_equal(host.view(np.uint32), dev.view(np.uint32))


def test_relpos_attention_rejects_bad_arguments(gpu):
    import torch
    x = torch.zeros((4, 192), dtype=torch.float32, device="cuda")
    p = x.data_ptr()
    with pytest.raises(RuntimeError, match="head size"):
        M.relpos_attention_dev(gpu, p, p, p, p, p, p, x[1:].data_ptr(), 1, 192, 2)   # dk 96
    with pytest.raises(RuntimeError, match="right"):
        M.relpos_attention_dev(gpu, p, p, p, p, p, p, x[1:].data_ptr(), 1, 128, 2, 4, -1)
    with pytest.raises(RuntimeError, match="alias"):
        M.relpos_attention_dev(gpu, p, p, p, p, p, p, p, 1, 128, 2)
