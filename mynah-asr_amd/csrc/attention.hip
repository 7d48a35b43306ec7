// attention.hip — the relative-position self-attention core of the FastConformer
// encoder layer (the reference's src/encoder.c:315-410 for full attention and
// its banded twin encoder.c:220-313 for chunked-limited attention), on the
// MFMA of gfx950: fp32 (v_mfma_f32_16x16x4_f32) for chunked windows, f16
// (v_mfma_f32_16x16x32_f16) on split operands for full attention.
//
// Per head h (columns h*DK .. h*DK+DK-1 of the [T, d] buffers):
//   s[t, j] = ((q[t] + bias_u) . k[j] + (q[t] + bias_v) . rk[T-1 + j - t]) / sqrt(DK)
//   ctx[t]  = sum_j softmax_j(s[t, j]) v[j],  j over the row's window
// rk = pe . relk_w^T is [2T-1, d] (the pos projection's output, shared by the
// segments of one call). The window is all of [0, T) for left < 0, else
// chunked-limited: chunk = right + 1, lc = left / chunk, row t (chunk t/chunk)
// sees [(t/chunk - lc) * chunk, (t/chunk + 1) * chunk) clipped to [0, T)
// (encoder.c:373-381).
//
// One workgroup = NW waves (4 or 8) = 16 NW query rows of one head of one
// segment; wave w owns rows t0 + 16w .. +15. Keys are visited in tiles of 32 (only the tiles
// the block's rows can see); each tile's K and V are staged in LDS, and the
// 16 NW + 16 rk rows of the block's position columns stay in an LDS ring that
// takes 32 new rows per tile; every wave
//   1. forms the content scores (16 x 32) with its (q + bias_u) held in registers,
//   2. forms the position scores (q + bias_v) . rk for its 16 rows in tiles of
//      16 offsets delta = j - t: a key tile needs 47 offsets (three tiles),
//      the first of which the previous key tile computed as its last (carried
//      in registers), so each key tile costs two position tiles, no more MFMA
//      work than the content scores,
//   3. applies the rel-shift through a per-wave LDS scratch (row i, key jj
//      reads band column jj - i + 15),
//   4. runs an online softmax (running row max and sum, base-2 exponentials of
//      scores pre-scaled by log2(e)/sqrt(DK)), and
//   5. multiplies the probabilities (re-laid out as an MFMA A operand through
//      LDS) by the V tile into its 16 x DK context accumulator.
// fp32 products and sums throughout (SPL = false): the result is the
// reference's f32 computation up to summation order and the exponential's
// rounding.
//
// SPL = FULL = true (full attention) forms the products on the f16 MFMA
// instead. Each q, K and rk row is scaled by a power of two 2^e that puts its
// largest magnitude in [2^14, 2^15) and split into f16 pairs hi + lo (hi =
// f16(x 2^e), lo = f16(x 2^e - hi)), which hold x to 2^-22 of the row's
// maximum; a score is hi.hi + hi.lo + lo.hi summed in f32 (the dropped lo.lo
// is below 2^-22 of the same scale) and multiplied by 2^-(e_q + e_k), which is
// exact. The content scores are formed transposed (K . q^T: a lane holds 8
// keys of one query), so the probabilities are already the context update's
// A operand; that update splits them (<= 256: the running maximum moves only
// by steps above 2^8) at the fixed scale 2^6 and V per (tile of 32 keys,
// feature, keys stored in the A operand's order), and undoes both per tile
// with one exact power of two. K, rk and V are split once per call by a
// pre-pass (k_attn_split, one launch); the q rows once per wave. The softmax
// stays fp32. With dk = 128 the context can be written directly as the
// output projection's prepared input (SplitIn::xp) instead of as f32 rows.
//
// MFMA 16x16x4 f32 operand layout (lane l, c = l & 15, g = l >> 4):
//   A: row c, k-slot g;  B: column c, k-slot g;  D: rows 4g + e (e = 0..3), column c.
// The reduction index of the score products is permuted so each lane reads a
// contiguous run: step s, slot g carries feature NS*g + s (NS = DK / 4).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "fmt.h"
#include "launch.h"

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

constexpr int KT = 32;           // keys per tile

// NW waves per workgroup, 16 query rows each. SPL: the scores on split
// operands, K and the rk ring holding f16 (hi, lo) pairs (rows of KSH halves
// each, hi rows then lo rows) and each row's exponent (EK, ER) in place of
// f32 rows. FULL (implies SPL): the full window, with V split too (planes
// of VTH halves per feature, a scale per feature in EV).
template <int DK, int NW, bool SPL = false, bool FULL = SPL>
struct AttnLds {
    static constexpr int NTH = 64 * NW;
    static constexpr int RB = 16 * NW;        // query rows per workgroup
    static constexpr int NB = RB + KT - 16;   // rk rows a key tile reads (all waves' position columns): the ring
    static constexpr int KS = DK + 4;   // K / rk row stride (16-byte rows, conflict-free b128 reads)
    static constexpr int KSH = DK + 8;  // SPL: the same in halves
    static constexpr int RS = SPL ? KSH : KS;   // floats per K / rk row (SPL: two rows of KSH halves)
    static constexpr int VT = KT + 4;   // V is stored transposed, [DK][VT]: conflict-free b128 reads
    static constexpr int VTH = KT + 8;  // SPL: the same in halves, hi plane then lo plane
    static constexpr int VSZ = FULL ? DK * VTH : DK * VT;   // floats
    static constexpr int BS = 53;       // band scratch row stride
    static constexpr int PS = 36;       // probability scratch row stride
    static constexpr int K0 = 0;
    static constexpr int V0 = K0 + KT * RS;
    static constexpr int R0 = V0 + VSZ;
    static constexpr int EK0 = R0 + NB * RS;            // SPL: key rows' exponents, then rk rows' (negated)
    static constexpr int ER0 = EK0 + (SPL ? KT : 0);
    static constexpr int EV0 = ER0 + (SPL ? NB : 0);     // FULL: the V tile's scale per feature
    static constexpr int W0 = (EV0 + (FULL ? DK : 0) + 3) / 4 * 4;
    static constexpr int WB = 16 * BS;
    static constexpr int WSZ = WB;      // the probabilities reuse the band scratch
    static constexpr int TOTAL = W0 + NW * WSZ;   // floats
};

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f4 mfma16h(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The exponent s that puts a row's largest magnitude amax in [2^14, 2^15)
// (0 for a row of zeros or a non-finite amax: its products are then what
// f16 makes of them, as the f32 products would be infinite or NaN)
__device__ __forceinline__ int row_exp(float amax) {
    if (!(amax > 0.0f) || !(amax < INFINITY)) return 0;
    int E;
    (void)frexpf(amax, &E);
    return min(max(15 - E, -120), 120);
}

// x * 2^s as an f16 pair: hi = f16(y), lo = f16(y - hi); y - hi is exact in
// f32, so hi + lo keeps 22 bits of x (the products of the score MFMAs drop
// only lo * lo, 2^-22 of a term)
__device__ __forceinline__ void split_h(float x, int s, _Float16 &hi, _Float16 &lo) {
    const float y = ldexpf(x, s);
    hi = (_Float16)y;
    lo = (_Float16)(y - (float)hi);
}

// SPL: K and rk as f16 (hi, lo) planes ([rows][d] each, the f32 tensors'
// indexing) and each (row, head)'s exponent ([rows][H]), formed once per
// call by k_attn_split instead of by every workgroup that stages a row
// V likewise, per tile of 32 keys (from key 0) and transposed: planes
// [segment][tile][d][32], and per (segment, tile, feature) the scale
// 2^-(6 + e) that undoes both the feature's exponent e and the
// probabilities' fixed 2^6
//
// xp (DK = 128, may be null): the context is written as the EXACT products'
// prepared input (the f16 split of each row's 128-element chunks, a chunk
// being one head, with the fold factors xpf, for M = nseq T rows padded to
// mh_mpad(M)) in place of ctx, for the output projection.
struct SplitIn {
    const _Float16 *kh, *kl, *rh, *rl;
    const int *ke, *re;
    const _Float16 *vh, *vl;
    const float *vs;
    uint8_t *xp;
    float *xpf;
};

__device__ __forceinline__ f4 mfma16(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Reductions over the 16 lanes of a DPP row (the lanes holding one score row):
// swap neighbours, swap pairs, mirror within 8, mirror within 16. Every lane
// ends with the same value (each step combines a and b symmetrically).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float max16(float x) {
    x = fmaxf(x, dpp<0xB1>(x));    // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp<0x4E>(x));    // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp<0x141>(x));   // row_half_mirror
    x = fmaxf(x, dpp<0x140>(x));   // row_mirror
    return x;
}

__device__ __forceinline__ float sum16(float x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    x += dpp<0x140>(x);
    return x;
}

// Compiler-level ordering of a wave's own LDS writes and reads (the LDS
// executes one wave's operations in issue order).
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct Window {
    int lim, chunk, lc, T;
    __device__ int j0(int t) const { return lim ? max((t / chunk - lc) * chunk, 0) : 0; }
    __device__ int j1(int t) const { return lim ? min((t / chunk + 1) * chunk, T) : T; }
};

template <int DK, int NW, bool SPL, bool FULL>
__global__ __launch_bounds__(64 * NW, 1) void k_relpos_attn(const float *__restrict__ q, const float *__restrict__ k,
                                                        const float *__restrict__ v, const float *__restrict__ rk,
                                                        const float *__restrict__ bu, const float *__restrict__ bv,
                                                        float *__restrict__ ctx, int T, int d, int left, int right,
                                                        float kscale, SplitIn sp) {
    using L = AttnLds<DK, NW, SPL, FULL>;
    static_assert(SPL || !FULL, "the full-window path splits every product");
    constexpr int NTH = L::NTH, RB = L::RB, NB = L::NB;
    constexpr int NS = DK / 4;    // reduction steps of a score product (f32 MFMA)
    constexpr int NKS = DK / 32;  // SPL: reduction steps of the f16 score MFMAs
    constexpr int NT = DK / 16;   // context column tiles
    extern __shared__ float lds[];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = lane & 15, g = lane >> 4;
    // XCD-aware order (query block bx, head by, segment bz): the query blocks
    // of one (segment, head) read the same K and V planes, and the segments of
    // one head the same rk rows, so they run on one XCD and share its L2
    int bx, by, bz;
    xcd_order(bx, by, bz);
    const int ho = by * DK;
    const size_t so = (size_t)bz * (size_t)T * (size_t)d;
    q += so;
    k += so;
    v += so;
    ctx += so;
    const int H = d / DK;
    const int ntile = (T + KT - 1) / KT;
    if constexpr (SPL) {
        sp.kh += so;
        sp.kl += so;
        sp.ke += (size_t)bz * T * H;
    }
    if constexpr (FULL) {
        sp.vh += (size_t)bz * ntile * d * KT;
        sp.vl += (size_t)bz * ntile * d * KT;
        sp.vs += (size_t)bz * ntile * d;
    }
    const int t0 = bx * RB, tw = t0 + 16 * w;
    Window win;
    win.lim = left >= 0;
    win.chunk = win.lim ? right + 1 : 1;
    win.lc = win.lim ? left / win.chunk : 0;
    win.T = T;
    const int ja = win.j0(t0), jb = win.j1(min(t0 + RB - 1, T - 1));

    // SPL: (q + bias_u), (q + bias_v) of query row tw + c, features 32 i +
    // 8 g .. +7 of step i, as f16 pairs scaled by the row's 2^e; the
    // exponents of this lane's output rows 4 g + e, negated
    h8 qah[SPL ? NKS : 1], qal[SPL ? NKS : 1], qbh[SPL ? NKS : 1], qbl[SPL ? NKS : 1];
    int eqa[4], eqb[4];
    int eqo = 0;   // FULL: the negated exponent of this lane's own query row tw + c
    if constexpr (SPL) {
        const int t = tw + c;
        float xa[SPL ? DK / 4 : 1], xb[SPL ? DK / 4 : 1];
        float ma = 0.0f, mb = 0.0f;
#pragma unroll
        for (int i = 0; i < NKS; i++)
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const int f = ho + 32 * i + 8 * g + 4 * hf;
                f4 u = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
                if (t < T) {
                    const f4 x = *(const f4 *)(q + (size_t)t * d + f);
                    u = x + *(const f4 *)(bu + f);
                    b = x + *(const f4 *)(bv + f);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    xa[8 * i + 4 * hf + j] = u[j];
                    xb[8 * i + 4 * hf + j] = b[j];
                    ma = fmaxf(ma, fabsf(u[j]));
                    mb = fmaxf(mb, fabsf(b[j]));
                }
            }
        ma = fmaxf(ma, __shfl_xor(ma, 16));
        ma = fmaxf(ma, __shfl_xor(ma, 32));
        mb = fmaxf(mb, __shfl_xor(mb, 16));
        mb = fmaxf(mb, __shfl_xor(mb, 32));
        const int ea = row_exp(ma), eb = row_exp(mb);
#pragma unroll
        for (int i = 0; i < NKS; i++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                _Float16 h, l;
                split_h(xa[8 * i + j], ea, h, l);
                qah[i][j] = h;
                qal[i][j] = l;
                split_h(xb[8 * i + j], eb, h, l);
                qbh[i][j] = h;
                qbl[i][j] = l;
            }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            eqa[e] = -__shfl(ea, 4 * g + e);   // negated: the unscale adds them
            eqb[e] = -__shfl(eb, 4 * g + e);
        }
        eqo = -ea;
    }
    // (q + bias_u), (q + bias_v) of query row tw + c, features NS*g .. NS*g + NS-1
    float qa[SPL ? 1 : NS], qb[SPL ? 1 : NS];
    if constexpr (!SPL) {
        const int t = tw + c;
        const int f = ho + NS * g;
#pragma unroll
        for (int i = 0; i < NS / 4; i++) {
            f4 x = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
            if (t < T) {
                x = *(const f4 *)(q + (size_t)t * d + f + 4 * i);
                u = x + *(const f4 *)(bu + f + 4 * i);
                b = x + *(const f4 *)(bv + f + 4 * i);
            }
            qa[4 * i + 0] = u.x; qa[4 * i + 1] = u.y; qa[4 * i + 2] = u.z; qa[4 * i + 3] = u.w;
            qb[4 * i + 0] = b.x; qb[4 * i + 1] = b.y; qb[4 * i + 2] = b.z; qb[4 * i + 3] = b.w;
        }
    }
    // this lane's output rows tw + 4g + e and their windows
    int rj0[4], rj1[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int t = min(tw + 4 * g + e, T - 1);
        rj0[e] = win.j0(t);
        rj1[e] = win.j1(t);
    }
    float m[4], l[4];
    f4 acc[NT];
#pragma unroll
    for (int e = 0; e < 4; e++) m[e] = -1e30f, l[e] = 0.f;
#pragma unroll
    for (int n = 0; n < NT; n++) acc[n] = f4{0.f, 0.f, 0.f, 0.f};

    float *Ks = lds + L::K0, *Vs = lds + L::V0, *Rs = lds + L::R0;
    // SPL: the same K and rk rows as f16 pairs and their exponents
    _Float16 *Kh = (_Float16 *)(lds + L::K0), *Kl = Kh + KT * L::KSH;
    _Float16 *Rh = (_Float16 *)(lds + L::R0), *Rl = Rh + NB * L::KSH;
    _Float16 *Vh = (_Float16 *)(lds + L::V0), *Vl = Vh + DK * L::VTH;
    float *EVs = lds + L::EV0;
    int *EK = (int *)(lds + L::EK0), *ER = (int *)(lds + L::ER0);
    float *Bw = lds + L::W0 + w * L::WSZ, *Pw = Bw;
    const int P = 2 * T - 1;

    // The next tile's K, V and rk rows are loaded into registers while the
    // current tile computes, then written to LDS between two barriers. Rows
    // past the ends are clamped, not zeroed: a key j outside [0, T) is masked
    // out of every score, and an rk row p outside [0, 2T-2] only pairs a query
    // row t >= T (never stored) or a masked key.
    //
    // The rk rows form a ring of NB rows: key tile ti (0 = the tile before
    // the first) reads window rows 32 ti .. 32 ti + NB - 1 (absolute rk row
    // pb0 + v for window row v), in slot v mod NB; moving to the next tile
    // retires the 32 lowest and stages 32 new ones into their slots.
    constexpr int UKV = KT * DK / 4 / NTH, UR = KT * DK / 4 / NTH;
    static_assert(UKV * NTH == KT * DK / 4, "staging split");
    // SPL: V tile pieces of 16 bytes (8 keys of one feature, hi or lo plane)
    constexpr int NVP = 2 * DK * 4, UVP = (NVP + NTH - 1) / NTH;
    f4 gk[SPL ? 1 : UKV], gv[FULL ? 1 : UKV], gr[SPL ? 1 : UR];
    uint4 svp[FULL ? UVP : 1];
    float svs = 0.0f;
    uint4 sk[SPL ? UKV : 1], sr[SPL ? UR : 1];   // SPL: (hi, lo) halves of the same 4 features
    int ek[SPL ? UKV : 1], er[SPL ? UR : 1];
    const int pb0 = T + (ja - KT) - t0 - (RB - 16);
    // SPL: the (hi, lo) halves and the (row, head) exponent of row `row` of a split tensor
    auto sload = [&](const _Float16 *hp, const _Float16 *lp, const int *ep, int row, int cc, uint4 &o, int &e) {
        const unsigned off = (unsigned)(row * d + ho + cc);   // < 2^31: checked at launch
        const uint2 a = *(const uint2 *)(hp + off), b = *(const uint2 *)(lp + off);
        o = make_uint4(a.x, a.y, b.x, b.y);
        e = ep[(unsigned)(row * H) + by];
    };
    auto sstore = [&](const uint4 &o, int e, int row, int cc, _Float16 *Hd, _Float16 *Ld, int *E) {
        *(uint2 *)(Hd + row * L::KSH + cc) = make_uint2(o.x, o.y);
        *(uint2 *)(Ld + row * L::KSH + cc) = make_uint2(o.z, o.w);
        if (cc == 0) E[row] = -e;   // negated: the unscale adds them
    };
    auto gload = [&](int jt, int ti) {
#pragma unroll
        for (int u = 0; u < UKV; u++) {
            const int i = tid + NTH * u;
            const int r = i / (DK / 4), cc = 4 * (i % (DK / 4));
            const int kr = min(max(jt + r, 0), T - 1);
            if constexpr (SPL) sload(sp.kh, sp.kl, sp.ke, kr, cc, sk[u], ek[u]);
            else gk[u] = *(const f4 *)(k + (unsigned)(kr * d + ho + cc));
            if constexpr (!FULL) {
                const int rv = i % KT, cv = 4 * (i / KT);   // V: lanes along keys (transposed store)
                gv[u] = *(const f4 *)(v + (unsigned)(min(max(jt + rv, 0), T - 1) * d + ho + cv));
            }
        }
        if constexpr (FULL) {
            const int vt = jt / KT;   // full attention: tiles start at key 0
#pragma unroll
            for (int u = 0; u < UVP; u++) {
                const int pc = tid + NTH * u;
                if (NVP % NTH == 0 || pc < NVP) {
                    const int f = (pc >> 2) % DK, part = pc & 3;
                    const _Float16 *pl = pc < DK * 4 ? sp.vh : sp.vl;
                    svp[u] = *(const uint4 *)(pl + ((unsigned)(vt * d + ho + f) * KT + 8 * part));
                }
            }
            if (tid < DK) svs = sp.vs[(unsigned)(vt * d + ho + tid)];
        }
#pragma unroll
        for (int u = 0; u < UR; u++) {
            const int i = tid + NTH * u, r = i / (DK / 4), cc = 4 * (i % (DK / 4));
            const int p = min(max(pb0 + 32 * ti + NB - 32 + r, 0), P - 1);
            if constexpr (SPL) sload(sp.rh, sp.rl, sp.re, p, cc, sr[u], er[u]);
            else gr[u] = *(const f4 *)(rk + (unsigned)(p * d + ho + cc));
        }
    };
    auto lstore = [&](int ti) {
#pragma unroll
        for (int u = 0; u < UKV; u++) {
            const int i = tid + NTH * u, r = i / (DK / 4), cc = 4 * (i % (DK / 4));
            if constexpr (SPL) sstore(sk[u], ek[u], r, cc, Kh, Kl, EK);
            else *(f4 *)(Ks + r * L::KS + cc) = gk[u];
            if constexpr (!FULL) {
                const int rv = i % KT, cv = 4 * (i / KT);
#pragma unroll
                for (int e = 0; e < 4; e++) Vs[(cv + e) * L::VT + rv] = gv[u][e];
            }
        }
        if constexpr (FULL) {
#pragma unroll
            for (int u = 0; u < UVP; u++) {
                const int pc = tid + NTH * u;
                if (NVP % NTH == 0 || pc < NVP) {
                    const int f = (pc >> 2) % DK, part = pc & 3;
                    _Float16 *pl = pc < DK * 4 ? Vh : Vl;
                    *(uint4 *)(pl + f * L::VTH + 8 * part) = svp[u];
                }
            }
            if (tid < DK) EVs[tid] = svs;
        }
#pragma unroll
        for (int u = 0; u < UR; u++) {
            const int i = tid + NTH * u, r = i / (DK / 4), cc = 4 * (i % (DK / 4));
            const int slot = (32 * ti + NB - 32 + r) % NB;
            if constexpr (SPL) sstore(sr[u], er[u], slot, cc, Rh, Rl, ER);
            else *(f4 *)(Rs + slot * L::KS + cc) = gr[u];
        }
    };
    // Position columns are computed in tiles of 16 offsets delta = j - t.
    // For key tile jt the wave needs delta in [b, b+47), b = jt - tw - 15:
    // tiles D0 = [b, b+16), D1, D2. The next key tile's D0 is this tile's D2,
    // so it is carried in registers and every tile computes only D1 and D2
    // (rk rows T-1 + b + 16 .. + 47: staged row (RB - 16) - 16w + col).
    const int prow = (RB - 16) - 16 * w;
    // ring slots of this lane's window rows prow + 16n + c at tile ti
    auto rrow = [&](int ti, int n) { return (32 * ti + prow + 16 * n + c) % NB; };
    auto bd_tiles = [&](f4 *bd, int n0) {   // tile 0
        if constexpr (SPL) {
#pragma unroll
            for (int i = 0; i < NKS; i++)
#pragma unroll
                for (int n = n0; n < 2; n++) {
                    const int o = rrow(0, n) * L::KSH + 32 * i + 8 * g;
                    const h8 rh = *(const h8 *)(Rh + o), rl = *(const h8 *)(Rl + o);
                    bd[n] = mfma16h(qbh[i], rh, bd[n]);
                    bd[n] = mfma16h(qbh[i], rl, bd[n]);
                    bd[n] = mfma16h(qbl[i], rh, bd[n]);
                }
#pragma unroll
            for (int n = n0; n < 2; n++) {
                const int er = ER[rrow(0, n)];
#pragma unroll
                for (int e = 0; e < 4; e++) bd[n][e] = ldexpf(bd[n][e], eqb[e] + er);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < NS / 4; i++) {
            f4 rx[2];
#pragma unroll
            for (int n = n0; n < 2; n++) rx[n] = *(const f4 *)(Rs + rrow(0, n) * L::KS + NS * g + 4 * i);
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int n = n0; n < 2; n++) bd[n] = mfma16(qb[4 * i + u], rx[n][u], bd[n]);
        }
    };
    f4 carry = {0.f, 0.f, 0.f, 0.f};
    {
        // D0 of the first tile = D2 of the tile before it: tile 0's whole
        // window of rk rows (slots 0 .. NB-1), then its position tile D2
        for (int i = tid; i < NB * DK / 4; i += NTH) {
            const int r = i / (DK / 4), cc = 4 * (i % (DK / 4));
            const int p = min(max(pb0 + r, 0), P - 1);
            if constexpr (SPL) {
                uint4 o;
                int e;
                sload(sp.rh, sp.rl, sp.re, p, cc, o, e);
                sstore(o, e, r, cc, Rh, Rl, ER);
            } else {
                *(f4 *)(Rs + r * L::KS + cc) = *(const f4 *)(rk + (size_t)p * d + ho + cc);
            }
        }
        __syncthreads();
        f4 bd[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        bd_tiles(bd, 1);
        carry = bd[1];
        gload(ja, 1);
    }

    // ring slots of this lane's window rows at tile ti, carried from tile to
    // tile (each tile moves them 32 rows on)
    int rb0 = (32 + prow + c) % NB;
    for (int jt = ja, ti = 1; jt < jb; jt += KT, ti++) {
        const int rr[2] = {rb0, rb0 + 16 >= NB ? rb0 + 16 - NB : rb0 + 16};
        rb0 = rb0 + 32 >= NB ? rb0 + 32 - NB : rb0 + 32;
        __syncthreads();   // every wave is done with the previous tile
        lstore(ti);
        __syncthreads();
        if (jt + KT < jb) gload(jt + KT, ti + 1);

        // 1. content scores (16 rows x 32 keys), 2. position tiles D1, D2
        f4 s[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        f4 bd[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        if constexpr (SPL) {
            // three f16 MFMAs per product (hi.hi, hi.lo, lo.hi), then the
            // rows' scales undone (exact: powers of two)
#pragma unroll
            for (int i = 0; i < NKS; i++) {
                h8 kh[2], kl[2], rh[2], rl[2];
#pragma unroll
                for (int n = 0; n < 2; n++) {
                    const int ok = (16 * n + c) * L::KSH + 32 * i + 8 * g;
                    kh[n] = *(const h8 *)(Kh + ok);
                    kl[n] = *(const h8 *)(Kl + ok);
                    const int orr = rr[n] * L::KSH + 32 * i + 8 * g;
                    rh[n] = *(const h8 *)(Rh + orr);
                    rl[n] = *(const h8 *)(Rl + orr);
                }
#pragma unroll
                for (int n = 0; n < 2; n++) {
                    if constexpr (FULL) {
                        // transposed: rows = keys 16n + 4g + e, column = query c
                        s[n] = mfma16h(kh[n], qah[i], s[n]);
                        s[n] = mfma16h(kl[n], qah[i], s[n]);
                        s[n] = mfma16h(kh[n], qal[i], s[n]);
                    } else {
                        s[n] = mfma16h(qah[i], kh[n], s[n]);
                        s[n] = mfma16h(qah[i], kl[n], s[n]);
                        s[n] = mfma16h(qal[i], kh[n], s[n]);
                    }
                    bd[n] = mfma16h(qbh[i], rh[n], bd[n]);
                    bd[n] = mfma16h(qbh[i], rl[n], bd[n]);
                    bd[n] = mfma16h(qbl[i], rh[n], bd[n]);
                }
            }
#pragma unroll
            for (int n = 0; n < 2; n++) {
                const int ek = EK[16 * n + c], er = ER[rr[n]];
                int4 ek4 = {0, 0, 0, 0};
                if constexpr (FULL) ek4 = *(const int4 *)(EK + 16 * n + 4 * g);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if constexpr (FULL) s[n][e] = ldexpf(s[n][e], eqo + ek4[e]);
                    else s[n][e] = ldexpf(s[n][e], eqa[e] + ek);
                    bd[n][e] = ldexpf(bd[n][e], eqb[e] + er);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < (SPL ? 0 : NS / 4); i++) {
            f4 kx[2], rx[2];
#pragma unroll
            for (int n = 0; n < 2; n++) kx[n] = *(const f4 *)(Ks + (16 * n + c) * L::KS + NS * g + 4 * i);
#pragma unroll
            for (int n = 0; n < 2; n++) rx[n] = *(const f4 *)(Rs + rr[n] * L::KS + NS * g + 4 * i);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                s[0] = mfma16(qa[4 * i + u], kx[0][u], s[0]);
                s[1] = mfma16(qa[4 * i + u], kx[1][u], s[1]);
                bd[0] = mfma16(qb[4 * i + u], rx[0][u], bd[0]);
                bd[1] = mfma16(qb[4 * i + u], rx[1][u], bd[1]);
            }
        }
        // 3. rel-shift: row i = 4g + e, key jj = 16n + c takes band column jj - i + 15
        //    (delta = jt + jj - (tw + i) = b + (jj - i + 15))
#pragma unroll
        for (int e = 0; e < 4; e++) {
            Bw[(4 * g + e) * L::BS + c] = carry[e];
            Bw[(4 * g + e) * L::BS + 16 + c] = bd[0][e];
            Bw[(4 * g + e) * L::BS + 32 + c] = bd[1][e];
        }
        carry = bd[1];
        wave_lds_order();
        float sv[2][4];
#pragma unroll
        for (int n = 0; n < 2; n++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if constexpr (FULL) {   // key 16n + 4g + e of query c
                    sv[n][e] = Bw[c * L::BS + 16 * n + 4 * g + e - c + 15];
                } else {
                    const int i = 4 * g + e;
                    sv[n][e] = Bw[i * L::BS + 16 * n + c - i + 15];
                }
            }
        if constexpr (FULL) {
            // full attention: every key below T is visible, and only the
            // last tile reaches past T
#pragma unroll
            for (int n = 0; n < 2; n++)
#pragma unroll
                for (int e = 0; e < 4; e++) sv[n][e] = (s[n][e] + sv[n][e]) * kscale;
            if (jt + KT > T) {
#pragma unroll
                for (int n = 0; n < 2; n++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (jt + 16 * n + 4 * g + e >= T) sv[n][e] = -INFINITY;
            }
        } else {
#pragma unroll
            for (int n = 0; n < 2; n++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int j = jt + 16 * n + c;
                    const float x = (s[n][e] + sv[n][e]) * kscale;
                    sv[n][e] = (unsigned)(j - rj0[e]) < (unsigned)(rj1[e] - rj0[e]) ? x : -INFINITY;
                }
        }
        // 4. online softmax over the tile
        if constexpr (FULL) {
            // One query per lane (column c; the 4 lanes of a column hold its
            // 32 keys): its running maximum and sum in m[0], l[0]. The maxima
            // move only when some query of the wave would exceed its maximum
            // by more than 2^8 (base 2): the probabilities stay <= 256, the
            // context and the sum carry the same maximum, and most tiles skip
            // the rescale (whose factors go to the context's rows 4g + e).
            float mx = -INFINITY;
#pragma unroll
            for (int n = 0; n < 2; n++)
#pragma unroll
                for (int e = 0; e < 4; e++) mx = fmaxf(mx, sv[n][e]);
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            if (__any(mx > m[0] + 8.0f)) {
                const float mn = fmaxf(m[0], mx), alpha = exp2f(m[0] - mn);
                m[0] = mn;
                l[0] *= alpha;
                float ae[4];
#pragma unroll
                for (int e = 0; e < 4; e++) ae[e] = __shfl(alpha, 4 * g + e);
#pragma unroll
                for (int n = 0; n < NT; n++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[n][e] *= ae[e];
            }
            float ls = 0.0f;
#pragma unroll
            for (int n = 0; n < 2; n++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    sv[n][e] = exp2f(sv[n][e] - m[0]);
                    ls += sv[n][e];
                }
            ls += __shfl_xor(ls, 16);
            ls += __shfl_xor(ls, 32);
            l[0] += ls;
        } else {
            float alpha[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float mx = max16(fmaxf(sv[0][e], sv[1][e]));
                const float mn = fmaxf(m[e], mx);
                alpha[e] = exp2f(m[e] - mn);
                m[e] = mn;
                sv[0][e] = exp2f(sv[0][e] - mn);
                sv[1][e] = exp2f(sv[1][e] - mn);
                l[e] = l[e] * alpha[e] + sum16(sv[0][e] + sv[1][e]);
            }
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[n][e] *= alpha[e];
        }
        if constexpr (FULL) {
            // probabilities (<= 256) split at the fixed scale 2^6, V split by
            // the pre-pass; the tile's scales undone by an exact power of two
            // The A operand straight from the scores' layout: this lane's
            // query c and its keys 4g .. 4g+3, 16+4g .. 16+4g+3 (the V planes
            // hold a tile's keys in that order)
            h8 ph, pl;
#pragma unroll
            for (int u = 0; u < 8; u++) {
                _Float16 hh, ll;
                split_h(sv[u >> 2][u & 3], 6, hh, ll);
                ph[u] = hh;
                pl[u] = ll;
            }
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const int o = (16 * n + c) * L::VTH + 8 * g;
                const h8 vh = *(const h8 *)(Vh + o), vl = *(const h8 *)(Vl + o);
                f4 t = {0.f, 0.f, 0.f, 0.f};
                t = mfma16h(ph, vh, t);
                t = mfma16h(ph, vl, t);
                t = mfma16h(pl, vh, t);
                const float sc = EVs[16 * n + c];
#pragma unroll
                for (int e = 0; e < 4; e++) acc[n][e] = fmaf(t[e], sc, acc[n][e]);
            }
            continue;
        }
        // 5. (f32 path) probabilities to the A layout (row c, keys 8g .. 8g+7), then P . V
        wave_lds_order();   // the band reads above precede these writes
#pragma unroll
        for (int n = 0; n < 2; n++)
#pragma unroll
            for (int e = 0; e < 4; e++) Pw[(4 * g + e) * L::PS + 16 * n + c] = sv[n][e];
        wave_lds_order();
        const f4 pa0 = *(const f4 *)(Pw + c * L::PS + 8 * g);
        const f4 pa1 = *(const f4 *)(Pw + c * L::PS + 8 * g + 4);
        const float pa[8] = {pa0.x, pa0.y, pa0.z, pa0.w, pa1.x, pa1.y, pa1.z, pa1.w};
        // B operand: column 16n + c, keys 8g .. 8g+7 of the transposed V tile
        f4 vb[2][2];
        auto rdv = [&](int n, f4 *vx) {
            const float *vr = Vs + (16 * n + c) * L::VT + 8 * g;
            vx[0] = *(const f4 *)vr;
            vx[1] = *(const f4 *)(vr + 4);
        };
        rdv(0, vb[0]);
#pragma unroll
        for (int n = 0; n < NT; n++) {
            if (n + 1 < NT) rdv(n + 1, vb[(n + 1) & 1]);
            const f4 *vx = vb[n & 1];
#pragma unroll
            for (int u = 0; u < 8; u++) acc[n] = mfma16(pa[u], vx[u >> 2][u & 3], acc[n]);
        }
    }

    if constexpr (FULL) {
        // the per-query sums (lane column c) to the context's rows 4g + e
        const float lc = l[0];
#pragma unroll
        for (int e = 0; e < 4; e++) l[e] = __shfl(lc, 4 * g + e);
    }
    if constexpr (FULL && DK == 128) {
        if (sp.xp) {
            // The context rows as the output projection's prepared input: the
            // values ctx would hold, split per (row, head) exactly as the
            // products' preparation splits a 128-element chunk, re-laid out
            // through LDS (free once every wave is past its last tile) into
            // 16-byte fragment slots.
            const int Kc = d / 128, chunk = by;
            __syncthreads();
            _Float16 *ph = (_Float16 *)lds + w * 4096, *pl = ph + 2048;   // [16 rows][128], hi then lo
            float fold[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = tw + 4 * g + e;
                const float inv = t < T ? 1.0f / l[e] : 0.0f;
                float vv[NT], a = 0.0f;
#pragma unroll
                for (int n = 0; n < NT; n++) {
                    vv[n] = acc[n][e] * inv;
                    a = fmaxf(a, fabsf(vv[n]));
                }
                a = max16(a);
                const int sh = chunk_shift(a);
                fold[e] = ldexpf(1.0f, -sh);
#pragma unroll
                for (int n = 0; n < NT; n++) {
                    const float xs = ldexpf(vv[n], sh);
                    const _Float16 hh = (_Float16)xs;
                    ph[(4 * g + e) * 128 + 16 * n + c] = hh;
                    pl[(4 * g + e) * 128 + 16 * n + c] = (_Float16)(xs - (float)hh);
                }
            }
            wave_lds_order();
            const size_t mb = (size_t)bz * T;
            // 512 slots per wave: lanes run along the 16 rows, so a store covers
            // consecutive slots of one (half-step, term, half)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int pc = lane + 64 * i, r16 = pc & 15, q = pc >> 4;
                const int plane = q >> 4, hu = (q >> 1) & 7, hh = q & 1;
                const int t = tw + r16;
                if (t < T) {
                    const size_t m = mb + t;
                    const uint4 val = *(const uint4 *)((plane ? pl : ph) + r16 * 128 + 16 * hu + 8 * hh);
                    *(uint4 *)(sp.xp + ((((m >> 5) * Kc + chunk) * 8 + hu) * 2 * 64 + plane * 64 + (m & 31) +
                                        32 * hh) * 16) = val;
                }
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = tw + 4 * g + e;
                if (t < T && c == 0) {
                    const size_t m = mb + t;
                    sp.xpf[((m >> 5) * Kc + chunk) * 32 + (m & 31)] = fold[e];
                }
            }
            // the rows past M up to the 64-row padding: zeros (fold factor 1),
            // as the preparation pads; by the last block of the last segment
            if (bz == gridDim.z - 1 && bx == gridDim.x - 1 && w == 0) {
                const size_t M = (size_t)gridDim.z * T, Mp = (M + 63) / 64 * 64;
                for (size_t i = lane; i < (Mp - M) * 32; i += 64) {
                    const size_t m = M + (i >> 5);
                    const int q = (int)(i & 31), plane = q >> 4, hu = (q >> 1) & 7, hh = q & 1;
                    *(uint4 *)(sp.xp + ((((m >> 5) * Kc + chunk) * 8 + hu) * 2 * 64 + plane * 64 + (m & 31) +
                                        32 * hh) * 16) = make_uint4(0, 0, 0, 0);
                    if (q == 0) sp.xpf[((m >> 5) * Kc + chunk) * 32 + (m & 31)] = 1.0f;
                }
            }
            return;
        }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int t = tw + 4 * g + e;
        if (t < T) {
            const float inv = 1.0f / l[e];
            float *o = ctx + (size_t)t * d + ho + c;
#pragma unroll
            for (int n = 0; n < NT; n++) o[16 * n] = acc[n][e] * inv;
        }
    }
}

// The split of rows of DK features (x [rows][d], heads of DK columns): per
// (row, head) the exponent e that puts the largest magnitude in [2^14, 2^15)
// and the planes hi = f16(x 2^e), lo = f16(x 2^e - hi), as the attention
// kernel's q split forms them. Thread = 4 features; the DK / 4 threads of a
// (row, head) are consecutive lanes.
template <int DK>
__device__ __forceinline__ void split_rows(const float *__restrict__ x, size_t n4, _Float16 *__restrict__ hi,
                                           _Float16 *__restrict__ lo, int *__restrict__ ex, size_t idx) {
    constexpr int TPR = DK / 4;
    if (idx >= n4) return;   // whole (row, head) groups only: n4 is a multiple of TPR
    const f4 v = *(const f4 *)(x + 4 * idx);
    float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int o = TPR / 2; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));
    const int e = row_exp(a);
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 hv, lv;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        _Float16 hh, ll;
        split_h(v[j], e, hh, ll);
        hv[j] = hh;
        lv[j] = ll;
    }
    *(h4 *)(hi + 4 * idx) = hv;
    *(h4 *)(lo + 4 * idx) = lv;
    if (idx % TPR == 0) ex[idx / TPR] = e;   // [row][head]: (4 idx / d) * (d / DK) + head
}

// V per tile of 32 keys (from key 0), transposed. Per feature the exponent
// e that puts the tile's largest magnitude in [2^14, 2^15) (clamped to
// [-100, 100], so that the scale below stays a normal float), the planes
// hi = f16(v 2^e), lo = f16(v 2^e - hi) as [segment][tile][d][32] (keys past
// T zero; within a tile in the order the kernel's P operand takes them: keys
// 4q .. 4q+3, 16+4q .. 16+4q+3 at positions 8q .. 8q+7), and the scale
// 2^-(6 + e). Thread = (segment, tile, feature, 8 positions): the 4 threads of
// a feature are consecutive lanes (the maximum is a quad reduction), and a
// wave's stores cover 16 features' 64-byte rows.
__device__ __forceinline__ void split_v(const float *__restrict__ v, int T, int d, int nseq,
                                        _Float16 *__restrict__ hi, _Float16 *__restrict__ lo,
                                        float *__restrict__ vs, size_t idx) {
    const int ntile = (T + KT - 1) / KT;
    if (idx >= (size_t)nseq * ntile * d * 4) return;   // whole quads only
    const int part = (int)(idx & 3);
    const size_t fi = idx >> 2;   // (segment, tile, feature)
    const int f = (int)(fi % d), tile = (int)((fi / d) % ntile), s = (int)(fi / ((size_t)d * ntile));
    // stored position 8 part + jj holds key 4 part + jj (jj < 4), else
    // 16 + 4 part + jj - 4: the keys one lane of the attention kernel's
    // score layout holds for its query
    const float *vs0 = v + ((size_t)s * T + (size_t)tile * KT) * d + f;
    float x[8];
    float a = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
        const int key = (jj < 4 ? 4 * part + jj : 16 + 4 * part + jj - 4);
        x[jj] = tile * KT + key < T ? vs0[(size_t)key * d] : 0.0f;
        a = fmaxf(a, fabsf(x[jj]));
    }
    a = fmaxf(a, __shfl_xor(a, 1));
    a = fmaxf(a, __shfl_xor(a, 2));
    const int ex = min(max(row_exp(a), -100), 100);
    h8 hv, lv;
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
        _Float16 hh, ll;
        split_h(x[jj], ex, hh, ll);
        hv[jj] = hh;
        lv[jj] = ll;
    }
    *(h8 *)(hi + fi * KT + 8 * part) = hv;
    *(h8 *)(lo + fi * KT + 8 * part) = lv;
    if (part == 0) vs[fi] = __int_as_float((127 - 6 - ex) << 23);
}

// The three splits in one launch: workgroups [0, bk) split K, the next br
// rk, the rest V (a workgroup's waves all take the same task).
struct SplitJobs {
    const float *k, *rk, *v;
    size_t nk4, nr4;
    unsigned bk, br;
    int T, d, nseq;
    _Float16 *kh, *kl, *rh, *rl, *vh, *vl;
    int *ke, *re;
    float *vs;
};

template <int DK>
__global__ __launch_bounds__(256) void k_attn_split(SplitJobs J) {
    const unsigned b = blockIdx.x;
    if (b < J.bk) {
        split_rows<DK>(J.k, J.nk4, J.kh, J.kl, J.ke, (size_t)b * 256 + threadIdx.x);
    } else if (b < J.bk + J.br) {
        split_rows<DK>(J.rk, J.nr4, J.rh, J.rl, J.re, (size_t)(b - J.bk) * 256 + threadIdx.x);
    } else {
        split_v(J.v, J.T, J.d, J.nseq, J.vh, J.vl, J.vs, (size_t)(b - J.bk - J.br) * 256 + threadIdx.x);
    }
}

size_t al256(size_t b) { return (b + 255) / 256 * 256; }

// the workspace of the split path: K planes and exponents, then rk's
struct SplitWs {
    size_t kp, ke, rp, re, vp, vs, total;
    SplitWs(int T, int d, int H, int nseq) {
        const size_t kr = (size_t)nseq * T, pr = (size_t)(2 * T - 1);
        const size_t vt = (size_t)nseq * ((T + KT - 1) / KT);
        kp = al256(kr * d * sizeof(_Float16));
        ke = al256(kr * H * sizeof(int));
        rp = al256(pr * d * sizeof(_Float16));
        re = al256(pr * H * sizeof(int));
        vp = al256(vt * d * KT * sizeof(_Float16));
        vs = al256(vt * d * sizeof(float));
        total = 2 * kp + ke + 2 * rp + re + 2 * vp + vs;
    }
};


template <int DK, int NW, bool SPL, bool FULL = SPL>
hipError_t launch_attn(const float *q, const float *k, const float *v, const float *rk, const float *bu,
                         const float *bv, float *ctx, int T, int d, int H, int left, int right, int nseq,
                         void *ws, uint8_t *xp, float *xpf, hipStream_t st) {
    if ((size_t)(2 * (size_t)T) * d >= 0x7fffffffu) return hipErrorInvalidValue;   // 32-bit row offsets
    if (FULL && left >= 0) return hipErrorInvalidValue;   // the full-window path
    if (xp && !(FULL && DK == 128)) return hipErrorInvalidValue;   // the prepared output: full window, dk 128
    SplitIn sp{};
    if constexpr (SPL) {
        if (!ws) return hipErrorInvalidValue;
        const SplitWs W(T, d, H, nseq);
        uint8_t *b = (uint8_t *)ws;
        _Float16 *kh = (_Float16 *)b, *kl = (_Float16 *)(b + W.kp);
        int *ke = (int *)(b + 2 * W.kp);
        _Float16 *rh = (_Float16 *)(b + 2 * W.kp + W.ke), *rl = (_Float16 *)(b + 2 * W.kp + W.ke + W.rp);
        int *re = (int *)(b + 2 * W.kp + W.ke + 2 * W.rp);
        uint8_t *vb = b + 2 * W.kp + W.ke + 2 * W.rp + W.re;
        _Float16 *vh = (_Float16 *)vb, *vl = (_Float16 *)(vb + W.vp);
        float *vsc = (float *)(vb + 2 * W.vp);
        SplitJobs J{};
        J.k = k;
        J.rk = rk;
        J.v = v;
        J.nk4 = (size_t)nseq * T * (d / 4);
        J.nr4 = (size_t)(2 * T - 1) * (d / 4);
        J.bk = (unsigned)((J.nk4 + 255) / 256);
        J.br = (unsigned)((J.nr4 + 255) / 256);
        J.T = T;
        J.d = d;
        J.nseq = nseq;
        J.kh = kh, J.kl = kl, J.ke = ke, J.rh = rh, J.rl = rl, J.re = re, J.vh = vh, J.vl = vl, J.vs = vsc;
        const size_t nv = FULL ? (size_t)nseq * ((T + KT - 1) / KT) * d * 4 : 0;
        const unsigned bv = (unsigned)((nv + 255) / 256);
        hipLaunchKernelGGL(k_attn_split<DK>, dim3(J.bk + J.br + bv), dim3(256), 0, st, J);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        sp = SplitIn{kh, kl, rh, rl, ke, re, vh, vl, vsc, DK == 128 ? xp : nullptr, xpf};
    }
    using L = AttnLds<DK, NW, SPL, FULL>;
    const size_t bytes = sizeof(float) * L::TOTAL;
    // set once per instantiation (thread-safe static initialisation)
    static const hipError_t attr = hipFuncSetAttribute((const void *)k_relpos_attn<DK, NW, SPL, FULL>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (attr != hipSuccess) return attr;
    // exponentials are base 2: scores carry log2(e) / sqrt(DK)
    const float kscale = (1.0f / sqrtf((float)DK)) * 1.4426950408889634f;
    dim3 grid((T + L::RB - 1) / L::RB, H, nseq);
    hipLaunchKernelGGL((k_relpos_attn<DK, NW, SPL, FULL>), grid, dim3(L::NTH), bytes, st, q, k, v, rk, bu, bv, ctx, T, d,
                       left, right, kscale, sp);
    return hipGetLastError();
}

// Eight waves (two per SIMD, one 128-row block) run full attention faster
// once there are at least two rounds of such blocks for the 256 CUs; with
// fewer blocks four waves (64 rows) balance better. Chunked windows take two
// waves (32 rows): a block visits the union of its rows' windows, so
// narrower blocks skip more of the keys their rows cannot see.
bool use8(int T, int H, int left, int nseq) {
    return left < 0 && (long)((T + 127) / 128) * H * nseq >= 512;
}

template <int DK>
hipError_t launch_dk(const float *q, const float *k, const float *v, const float *rk, const float *bu,
                     const float *bv, float *ctx, int T, int d, int H, int left, int right, int nseq, void *ws,
                     uint8_t *xp, float *xpf, hipStream_t st) {
    // Full attention computes its scores on the f16 MFMA from split operands
    // (18% faster at T = 750); chunked windows stage as many K / rk rows per
    // score they keep, so the splitting costs more than it saves there.
    if (use8(T, H, left, nseq))
        return launch_attn<DK, 8, true>(q, k, v, rk, bu, bv, ctx, T, d, H, left, right, nseq, ws, xp, xpf, st);
    if (left >= 0) return launch_attn<DK, 2, false>(q, k, v, rk, bu, bv, ctx, T, d, H, left, right, nseq, ws, xp, xpf, st);
    return launch_attn<DK, 4, true>(q, k, v, rk, bu, bv, ctx, T, d, H, left, right, nseq, ws, xp, xpf, st);
}

}  // namespace

bool mh_attn_supported(int dk) { return dk == 64 || dk == 128; }

size_t mh_attn_ws_bytes(int T, int d, int H, int nseq, int left) {
    if (left >= 0 || T <= 0 || nseq <= 0 || H <= 0) return 0;   // chunked windows: all f32, no split
    return SplitWs(T, d, H, nseq).total;
}

hipError_t mh_launch_relpos_attn(const float *q, const float *k, const float *v, const float *rk,
                                 const float *bias_u, const float *bias_v, float *ctx, int T, int d, int H,
                                 int left, int right, int nseq, void *ws, uint8_t *xp, float *xpf,
                                 hipStream_t st) {
    const int dk = d / H;
    if (dk == 128)
        return launch_dk<128>(q, k, v, rk, bias_u, bias_v, ctx, T, d, H, left, right, nseq, ws, xp, xpf, st);
    if (dk == 64 && !xp)
        return launch_dk<64>(q, k, v, rk, bias_u, bias_v, ctx, T, d, H, left, right, nseq, ws, nullptr, nullptr, st);
    return hipErrorInvalidValue;
}

bool mh_attn_preps_out(int d, int H, int left) { return left < 0 && H > 0 && d / H == 128; }
