/* oracle.c — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates, in plain scalar C, the arithmetic of the reference CPU path that
 * the HIP backend replaces. Every function cites the reference file:line it
 * follows (paths relative to the mynah-asr tree). Built with
 * -ffp-contract=off so that every float operation rounds exactly where the C
 * source says it does.
 *
 * How each part is pinned (the tests in tests/test_oracle_*.py):
 *   f16 conversion      — exhaustive over all 65536 halves vs the reference's
 *                         ingot_f16_to_f32 / ingot_f32_to_f16 (oracle/_ref),
 *                         plus textbook values (1, -2, 65504, 2^-24, inf, nan).
 *   block decoders      — the reference's known-answer fixtures
 *                         (ingot/tests/fixtures/<TYPE>.{bin,ref}, from llama.cpp's
 *                         dequantizer), bit for bit, plus oracle/_ref.
 *   block quantizers    — oracle/_ref bit for bit on seeded inputs, plus closed
 *                         form invariants (|q| <= 127, amax maps to +-127 ...).
 *   qmat INT8/INT4      — closed form invariants and brute force on tiny rows
 *                         (qmat.c cannot be compiled here: it includes <cblas.h>,
 *                         which this image does not have).
 *   int8 dot path       — int64 brute force of the integer sums.
 *   f64 GEMM            — closed forms (identity / one-hot weights, rank-1).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ util */
static uint16_t ld16(const unsigned char *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void st16(unsigned char *p, uint16_t v) {
    p[0] = (unsigned char)(v & 0xff);
    p[1] = (unsigned char)(v >> 8);
}
static float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

int orc_geometry(int type, int *be, int *bb) {
    int e, b;
    switch (type) {
    case ORC_F32:  e = 1;   b = 4;   break;
    case ORC_Q4_0: e = 32;  b = 18;  break;
    case ORC_Q8_0: e = 32;  b = 34;  break;
    case ORC_Q2_K: e = 256; b = 84;  break;
    case ORC_Q3_K: e = 256; b = 110; break;
    case ORC_Q4_K: e = 256; b = 144; break;
    case ORC_Q5_K: e = 256; b = 176; break;
    case ORC_Q6_K: e = 256; b = 210; break;
    default: return -1;
    }
    if (be) *be = e;
    if (bb) *bb = b;
    return 0;
}

/* ------------------------------------------------------- f16 conversions
 * Follows ingot dtype.c:218-244 (decode: subnormals normalised, NaN quieted)
 * and dtype.c:246-268 (encode: nearest-even for normals, half-up for the
 * subnormal range, overflow to inf, NaN keeps a payload bit). */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int e = (h >> 10) & 31;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bits_f(sign);
        e = 1;                                  /* normalise the subnormal */
        while (!(m & 0x400u)) { m <<= 1; e--; }
        return bits_f(sign | ((uint32_t)(e + 112) << 23) | ((m & 0x3ffu) << 13));
    }
    if (e == 31) return bits_f(sign | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0u));
    return bits_f(sign | ((uint32_t)(e + 112) << 23) | (m << 13));
}

uint16_t orc_f32_to_f16(float f) {
    const uint32_t u = f_bits(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int e = (int)((u >> 23) & 0xff) - 127;
    uint32_t m = u & 0x7fffffu;
    if (e == 128) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e < -24) return (uint16_t)sign;
    if (e < -14) {                              /* lands in the f16 subnormals */
        m |= 0x800000u;
        const int sh = -e - 14;
        uint32_t r = m >> (13 + sh);
        if ((m >> (12 + sh)) & 1u) r++;         /* half rounds up here */
        return (uint16_t)(sign | r);
    }
    uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
    const uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* The Q4_K quantizer carries its own pair of converters (ingot
 * kernels.c:61-78 and :150-168): the encoder adds half an ulp to the magnitude
 * (ties away from zero) and saturates to inf; the decoder does not quiet NaNs. */
static float q4k_h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int e = (h >> 10) & 31;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bits_f(sign);
        e = 1;
        while (!(m & 0x400u)) { m <<= 1; e--; }
        return bits_f(sign | ((uint32_t)(e + 112) << 23) | ((m & 0x3ffu) << 13));
    }
    if (e == 31) return bits_f(sign | 0x7f800000u | (m << 13));
    return bits_f(sign | ((uint32_t)(e + 112) << 23) | (m << 13));
}

static uint16_t q4k_f2h(float f) {
    const uint32_t u = f_bits(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    int e = (int)((u >> 23) & 0xff) - 127 + 15;
    uint32_t m = u & 0x7fffffu;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m |= 0x800000u;
        const uint32_t sh = (uint32_t)(14 - e);
        return (uint16_t)(sign | ((m + (1u << (sh - 1))) >> sh));
    }
    uint32_t r = (m + 0x1000u) >> 13;
    if (r > 0x3ffu) {
        r = 0;
        e++;
        if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | r);
}

static float h2f(const unsigned char *p) { return orc_f16_to_f32(ld16(p)); }

/* --------------------------------------------------------------- decoders */

/* Q4_0 (ingot dequant.c:73-83): 18 B = f16 d + 16 B; byte i carries element i
 * in its low nibble and element i+16 in its high nibble; x = d * (nib - 8). */
static void dq_q4_0(const unsigned char *s, size_t nb, float *y) {
    for (size_t b = 0; b < nb; b++, s += 18, y += 32) {
        const float d = h2f(s);
        for (int i = 0; i < 16; i++) {
            y[i] = d * (float)((s[2 + i] & 15) - 8);
            y[i + 16] = d * (float)((s[2 + i] >> 4) - 8);
        }
    }
}

/* Q8_0 (dequant.c:132-156): 34 B = f16 d + 32 int8; x = d * q. */
static void dq_q8_0(const unsigned char *s, size_t nb, float *y) {
    for (size_t b = 0; b < nb; b++, s += 34, y += 32) {
        const float d = h2f(s);
        for (int i = 0; i < 32; i++) y[i] = d * (float)(signed char)s[2 + i];
    }
}

/* Q2_K (dequant.c:164-184): 84 B = 16 B scale/min nibbles, 64 B of 2-bit
 * quants, f16 d, f16 dmin. Sixteen sub-blocks of 16. Element e of the super-
 * block: half h = e/128, within it r = e%128, field f = r/32 (bit shift 2f),
 * lane l = r%32 (byte 32h + l); sub-block index 8h + 2f + l/16. */
static void dq_q2_k(const unsigned char *s, size_t nb, float *y) {
    for (size_t b = 0; b < nb; b++, s += 84, y += 256) {
        const float d = h2f(s + 80), dmin = h2f(s + 82);
        for (int e = 0; e < 256; e++) {
            const int h = e / 128, r = e % 128, f = r / 32, l = r % 32;
            const int sb = 8 * h + 2 * f + l / 16;
            const int q = (s[16 + 32 * h + l] >> (2 * f)) & 3;
            const float dl = d * (float)(s[sb] & 15);
            const float ml = dmin * (float)(s[sb] >> 4);
            y[e] = dl * (float)q - ml;
        }
    }
}

/* Q3_K (dequant.c:190-220): 110 B = 32 B hmask, 64 B 2-bit quants, 12 B of
 * packed 6-bit scales, f16 d. Same element walk as Q2_K; the high bit of
 * element e is bit (4h + f) of hmask[l] and is INVERTED (clear => subtract 4).
 * Scale j: low nibble from byte j (j<8) or high nibble of byte j-8, top two
 * bits from byte 8 + j%4 at shift 2*(j/4); value minus 32. */
static int q3k_scale(const unsigned char *sc, int j) {
    const int lo = j < 8 ? (sc[j] & 15) : (sc[j - 8] >> 4);
    const int hi = (sc[8 + (j % 4)] >> (2 * (j / 4))) & 3;
    return (lo | (hi << 4)) - 32;
}
static void dq_q3_k(const unsigned char *s, size_t nb, float *y) {
    for (size_t b = 0; b < nb; b++, s += 110, y += 256) {
        const float d = h2f(s + 108);
        for (int e = 0; e < 256; e++) {
            const int h = e / 128, r = e % 128, f = r / 32, l = r % 32;
            const int sb = 8 * h + 2 * f + l / 16;
            const int q = (s[32 + 32 * h + l] >> (2 * f)) & 3;
            const int hb = (s[l] >> (4 * h + f)) & 1;
            const float dl = d * (float)q3k_scale(s + 96, sb);
            y[e] = dl * (float)(q - (hb ? 0 : 4));
        }
    }
}

/* Q4_K / Q5_K 6-bit scale+min unpacking (dequant.c:59-68). */
static void k4_sm(const unsigned char *sc, int j, int *s, int *m) {
    if (j < 4) {
        *s = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
        *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

/* Q4_K (dequant.c:224-273): 144 B = f16 d, f16 dmin, 12 B scales, 128 B
 * nibbles. Sub-block j (32 elements): pair p = j/2 uses bytes 32p..32p+31,
 * low nibbles for even j, high for odd j. x = (d*sc)*q - dmin*m. */
static void dq_q4_k(const unsigned char *s, size_t nb, float *y) {
    for (size_t b = 0; b < nb; b++, s += 144, y += 256) {
        const float d = h2f(s), dmin = h2f(s + 2);
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            k4_sm(s + 4, j, &sc, &mn);
            const float dl = d * (float)sc, ml = dmin * (float)mn;
            const unsigned char *q = s + 16 + 32 * (j / 2);
            for (int i = 0; i < 32; i++) {
                const int v = (j & 1) ? (q[i] >> 4) : (q[i] & 15);
                y[32 * j + i] = dl * (float)v - ml;
            }
        }
    }
}

/* Q5_K (dequant.c:278-350): 176 B = f16 d, f16 dmin, 12 B scales, 32 B qh,
 * 128 B nibbles. As Q4_K plus a fifth bit: element i of sub-block j takes
 * bit j of qh[i] as its value 16. */
static void dq_q5_k(const unsigned char *s, size_t nb, float *y) {
    for (size_t b = 0; b < nb; b++, s += 176, y += 256) {
        const float d = h2f(s), dmin = h2f(s + 2);
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            k4_sm(s + 4, j, &sc, &mn);
            const float dl = d * (float)sc, ml = dmin * (float)mn;
            const unsigned char *q = s + 48 + 32 * (j / 2);
            for (int i = 0; i < 32; i++) {
                int v = (j & 1) ? (q[i] >> 4) : (q[i] & 15);
                if ((s[16 + i] >> j) & 1) v += 16;
                y[32 * j + i] = dl * (float)v - ml;
            }
        }
    }
}

/* Q6_K (dequant.c:354-445): 210 B = 128 B low nibbles ql, 64 B high bit pairs
 * qh, 16 int8 scales, f16 d. Element e: half h = e/128, r = e%128, quarter
 * f = r/32, l = r%32; low nibble from ql[64h + 32(f&1) + l] (high nibble when
 * f >= 2), two high bits from qh[32h + l] at shift 2f; sub-block 8h + 2f + l/16.
 * x = d * sc * (q - 32), evaluated (d*sc)*(q-32). */
static void dq_q6_k(const unsigned char *s, size_t nb, float *y) {
    for (size_t b = 0; b < nb; b++, s += 210, y += 256) {
        const float d = h2f(s + 208);
        const signed char *sc = (const signed char *)(s + 192);
        for (int e = 0; e < 256; e++) {
            const int h = e / 128, r = e % 128, f = r / 32, l = r % 32;
            const unsigned char lb = s[64 * h + 32 * (f & 1) + l];
            const int lo = (f >= 2) ? (lb >> 4) : (lb & 15);
            const int hi = (s[128 + 32 * h + l] >> (2 * f)) & 3;
            const int q = (lo | (hi << 4)) - 32;
            y[e] = d * (float)sc[8 * h + 2 * f + l / 16] * (float)q;
        }
    }
}

int orc_dequant(int type, const void *src, size_t count, float *dst) {
    int be, bb;
    if (!src || !dst || orc_geometry(type, &be, &bb) != 0 || count % (size_t)be) return -1;
    const unsigned char *s = (const unsigned char *)src;
    const size_t nb = count / (size_t)be;
    switch (type) {
    case ORC_F32: memcpy(dst, src, count * 4); return 0;
    case ORC_Q4_0: dq_q4_0(s, nb, dst); return 0;
    case ORC_Q8_0: dq_q8_0(s, nb, dst); return 0;
    case ORC_Q2_K: dq_q2_k(s, nb, dst); return 0;
    case ORC_Q3_K: dq_q3_k(s, nb, dst); return 0;
    case ORC_Q4_K: dq_q4_k(s, nb, dst); return 0;
    case ORC_Q5_K: dq_q5_k(s, nb, dst); return 0;
    case ORC_Q6_K: dq_q6_k(s, nb, dst); return 0;
    }
    return -1;
}

/* ------------------------------------------------------------- quantizers */

/* Q8_0 (ingot quantize.c:49-57): d = amax/127 (f32), id = 1/d, the stored
 * scale is f16(d); q = clamp(lroundf(x*id), -127, 127) (ties away from 0). */
static void q_q8_0(const float *x, unsigned char *o) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) if (fabsf(x[i]) > amax) amax = fabsf(x[i]);
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    st16(o, orc_f32_to_f16(d));
    for (int i = 0; i < 32; i++)
        o[2 + i] = (unsigned char)(signed char)clampi((int)lroundf(x[i] * id), -127, 127);
}

/* The element of largest magnitude, keeping its sign; the first one wins a
 * tie (quantize.c:26-33). */
static float signed_absmax(const float *x, int n) {
    float amax = 0.0f, v = 0.0f;
    for (int i = 0; i < n; i++)
        if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); v = x[i]; }
    return v;
}

/* Q4_0 (quantize.c:60-71): d = max/-8 where max is the signed extreme;
 * q = clamp((int)(x*id + 8.5), 0, 15); element i low nibble, i+16 high. */
static void q_q4_0(const float *x, unsigned char *o) {
    const float d = signed_absmax(x, 32) / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    st16(o, orc_f32_to_f16(d));
    for (int i = 0; i < 16; i++) {
        const int lo = clampi((int)(x[i] * id + 8.5f), 0, 15);
        const int hi = clampi((int)(x[i + 16] * id + 8.5f), 0, 15);
        o[2 + i] = (unsigned char)(lo | (hi << 4));
    }
}

/* Q6_K (quantize.c:129-168): per sub-block of 16 a signed scale max/-32; the
 * super-scale d = (the sub-scale of largest magnitude)/-128; sc = clamp(
 * lroundf(scale/d)) to int8; q = clamp(lroundf(x / (d*sc)) + 32, 0, 63),
 * scattered into ql/qh exactly where dq_q6_k reads it. */
static void q_q6_k(const float *x, unsigned char *o) {
    float sub[16], big = 0.0f;
    for (int j = 0; j < 16; j++) {
        sub[j] = signed_absmax(x + 16 * j, 16) / -32.0f;
        if (fabsf(sub[j]) > fabsf(big)) big = sub[j];
    }
    const float d = big / -128.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    signed char sc[16];
    for (int j = 0; j < 16; j++) sc[j] = (signed char)clampi((int)lroundf(sub[j] * id), -128, 127);
    unsigned char ql[128], qh[64];
    memset(ql, 0, sizeof ql);
    memset(qh, 0, sizeof qh);
    for (int e = 0; e < 256; e++) {
        const int j = e / 16;
        const float ds = d * (float)sc[j];
        const float ids = ds != 0.0f ? 1.0f / ds : 0.0f;
        const int q = clampi((int)lroundf(x[e] * ids) + 32, 0, 63);
        const int h = e / 128, r = e % 128, f = r / 32, l = r % 32;
        ql[64 * h + 32 * (f & 1) + l] |= (unsigned char)((q & 15) << (4 * (f / 2)));
        qh[32 * h + l] |= (unsigned char)(((q >> 4) & 3) << (2 * f));
    }
    memcpy(o, ql, 128);
    memcpy(o + 128, qh, 64);
    memcpy(o + 192, sc, 16);
    st16(o + 208, orc_f32_to_f16(d));
}

/* Q4_K (ingot kernels.c:175-318). Per sub-block of 32: the range [lo, hi]
 * (widened to include 0) is tried at six shrink factors 1 - 0.04c around its
 * centre; each candidate gets two rounds of level assignment (lrintf) and a
 * least-squares refit of (step, base), with base pinned to <= 0; the candidate
 * with the smallest squared error wins (first on ties). Then d = f16(max step
 * / 63), dmin = f16(max offset / 63) with this file's own f16 encoder; the
 * 6-bit sc/m are lrintf(step/d), lrintf(offset/dmin) against the ROUNDED
 * factors; quants are lrintf((x + dmin*m) / (d*sc)) clamped to 0..15. */
static void q_q4_k(const float *x, unsigned char *o) {
    float steps[8], offs[8], max_step = 0.0f, max_off = 0.0f;
    for (int j = 0; j < 8; j++) {
        const float *v = x + 32 * j;
        float lo = v[0], hi = v[0];
        for (int i = 1; i < 32; i++) {
            if (v[i] < lo) lo = v[i];
            if (v[i] > hi) hi = v[i];
        }
        if (lo > 0.0f) lo = 0.0f;
        if (hi < 0.0f) hi = 0.0f;
        float best_step = (hi - lo) / 15.0f, best_off = -lo, best_err = -1.0f;
        for (int c = 0; c <= 5; c++) {
            const float shrink = 1.0f - 0.04f * (float)c;
            const float mid = 0.5f * (hi + lo);
            const float half = 0.5f * shrink * (hi - lo);
            float a = mid - half, bnd = mid + half;
            if (a > 0.0f) a = 0.0f;
            if (bnd < 0.0f) bnd = 0.0f;
            float step = (bnd - a) / 15.0f;
            if (!(step > 0.0f)) continue;
            for (int round = 0; round < 2; round++) {
                float sq = 0.0f, sqq = 0.0f, sx = 0.0f, sxq = 0.0f;
                for (int i = 0; i < 32; i++) {
                    long lv = lrintf((v[i] - a) / step);
                    if (lv < 0) lv = 0;
                    if (lv > 15) lv = 15;
                    const float q = (float)lv;
                    sq += q;
                    sqq += q * q;
                    sx += v[i];
                    sxq += v[i] * q;
                }
                const float det = 32.0f * sqq - sq * sq;
                if (!(fabsf(det) > 1e-12f)) break;
                float fit = (32.0f * sxq - sq * sx) / det;
                float base = (sx - fit * sq) / 32.0f;
                if (base > 0.0f) {
                    base = 0.0f;
                    if (sqq > 0.0f) fit = sxq / sqq;
                }
                if (!(fit > 0.0f)) break;
                step = fit;
                a = base;
            }
            float err = 0.0f;
            for (int i = 0; i < 32; i++) {
                long q = lrintf((v[i] - a) / step);
                if (q < 0) q = 0;
                if (q > 15) q = 15;
                const float diff = step * (float)q + a - v[i];
                err += diff * diff;
            }
            if (best_err < 0.0f || err < best_err) {
                best_err = err;
                best_step = step;
                best_off = -a;
            }
        }
        steps[j] = best_step;
        offs[j] = best_off;
        if (steps[j] > max_step) max_step = steps[j];
        if (offs[j] > max_off) max_off = offs[j];
    }
    const uint16_t dh = q4k_f2h(max_step / 63.0f), mh = q4k_f2h(max_off / 63.0f);
    st16(o, dh);
    st16(o + 2, mh);
    const float d = q4k_h2f(dh), dmin = q4k_h2f(mh);
    unsigned char sb[8], mb[8];
    for (int j = 0; j < 8; j++) {
        long s = d > 0.0f ? lrintf(steps[j] / d) : 0;
        long m = dmin > 0.0f ? lrintf(offs[j] / dmin) : 0;
        sb[j] = (unsigned char)(s < 0 ? 0 : (s > 63 ? 63 : s));
        mb[j] = (unsigned char)(m < 0 ? 0 : (m > 63 ? 63 : m));
    }
    unsigned char *sc = o + 4;
    for (int j = 0; j < 4; j++) {
        sc[j] = (unsigned char)(sb[j] | ((sb[j + 4] >> 4) << 6));
        sc[j + 4] = (unsigned char)(mb[j] | ((mb[j + 4] >> 4) << 6));
        sc[j + 8] = (unsigned char)((sb[j + 4] & 15) | ((mb[j + 4] & 15) << 4));
    }
    for (int p = 0; p < 4; p++) {
        const int jl = 2 * p, jh = 2 * p + 1;
        const float sl = d * sb[jl], sh = d * sb[jh];
        const float ol = dmin * mb[jl], oh = dmin * mb[jh];
        for (int i = 0; i < 32; i++) {
            long l = sl > 0.0f ? lrintf((x[32 * jl + i] + ol) / sl) : 0;
            long h = sh > 0.0f ? lrintf((x[32 * jh + i] + oh) / sh) : 0;
            l = l < 0 ? 0 : (l > 15 ? 15 : l);
            h = h < 0 ? 0 : (h > 15 ? 15 : h);
            o[16 + 32 * p + i] = (unsigned char)((unsigned)l | ((unsigned)h << 4));
        }
    }
}

int orc_quantize(int type, const float *x, size_t count, void *out) {
    int be, bb;
    if (!x || !out || orc_geometry(type, &be, &bb) != 0 || count % (size_t)be) return -1;
    void (*fn)(const float *, unsigned char *) = NULL;
    switch (type) {
    case ORC_F32: memcpy(out, x, count * 4); return 0;
    case ORC_Q8_0: fn = q_q8_0; break;
    case ORC_Q4_0: fn = q_q4_0; break;
    case ORC_Q4_K: fn = q_q4_k; break;
    case ORC_Q6_K: fn = q_q6_k; break;
    default: return -1;
    }
    unsigned char *o = (unsigned char *)out;
    for (size_t b = 0; b < count / (size_t)be; b++) fn(x + b * (size_t)be, o + b * (size_t)bb);
    return 0;
}

/* ------------------------------------------------------- qmat INT8 / INT4 */

/* qmat.c:19-36: per row scale = amax/127 (1 when the row is all zero);
 * q = (int8)(v +- 0.5) with v = w * (1/scale), truncation toward zero. */
void orc_qmat_quantize_int8(const float *w, int n, int k, int8_t *q, float *scales) {
    for (int r = 0; r < n; r++) {
        const float *row = w + (size_t)r * k;
        float amax = 0.0f;
        for (int j = 0; j < k; j++) if (fabsf(row[j]) > amax) amax = fabsf(row[j]);
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / s;
        scales[r] = s;
        for (int j = 0; j < k; j++) {
            const float v = row[j] * inv;
            q[(size_t)r * k + j] = (int8_t)(v >= 0.0f ? v + 0.5f : v - 0.5f);
        }
    }
}

/* qmat.c:38-67: per group of 32 scale = amax/7 (1 when zero); q clamped to
 * [-8, 7] and stored +8; byte j of a group holds elements 2j (low nibble) and
 * 2j+1 (high nibble). */
void orc_qmat_quantize_int4(const float *w, int n, int k, uint8_t *q, float *scales) {
    const int G = k / 32;
    for (int r = 0; r < n; r++) {
        for (int g = 0; g < G; g++) {
            const float *v = w + (size_t)r * k + 32 * g;
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) if (fabsf(v[j]) > amax) amax = fabsf(v[j]);
            const float s = amax > 0.0f ? amax / 7.0f : 1.0f;
            const float inv = 1.0f / s;
            scales[(size_t)r * G + g] = s;
            for (int j = 0; j < 32; j += 2) {
                const float a = v[j] * inv, b = v[j + 1] * inv;
                const int qa = clampi((int)(a >= 0.0f ? a + 0.5f : a - 0.5f), -8, 7);
                const int qb = clampi((int)(b >= 0.0f ? b + 0.5f : b - 0.5f), -8, 7);
                q[(size_t)r * (k / 2) + 16 * g + j / 2] = (uint8_t)((qa + 8) | ((qb + 8) << 4));
            }
        }
    }
}

/* qmat.c:152-169: w = (float)q * s. */
void orc_qmat_dequant(int qtype, const void *qv, const float *scales, int n, int k, float *wd) {
    for (int r = 0; r < n; r++) {
        float *o = wd + (size_t)r * k;
        if (qtype == 1) {
            const int8_t *q = (const int8_t *)qv + (size_t)r * k;
            for (int j = 0; j < k; j++) o[j] = (float)q[j] * scales[r];
        } else {
            const uint8_t *q = (const uint8_t *)qv + (size_t)r * (k / 2);
            const float *s = scales + (size_t)r * (k / 32);
            for (int j = 0; j < k; j += 2) {
                o[j] = (float)((q[j / 2] & 15) - 8) * s[j / 32];
                o[j + 1] = (float)((q[j / 2] >> 4) - 8) * s[j / 32];
            }
        }
    }
}

/* qmat.c:186-202: amax over the row; all-zero row -> zeros and scale 0;
 * inv = 127/amax; q = (int)(v +- 0.5) clamped to +-127; scale = amax/127. */
float orc_act_quant_int8(const float *x, int k, int8_t *qx) {
    float amax = 0.0f;
    for (int j = 0; j < k; j++) if (fabsf(x[j]) > amax) amax = fabsf(x[j]);
    if (amax == 0.0f) { memset(qx, 0, (size_t)k); return 0.0f; }
    const float inv = 127.0f / amax;
    for (int j = 0; j < k; j++) {
        const float v = x[j] * inv;
        qx[j] = (int8_t)clampi((int)(v >= 0.0f ? v + 0.5f : v - 0.5f), -127, 127);
    }
    return amax / 127.0f;
}

/* qmat.c:519-551 (dot_q8_* :212-220, :285-322; dot_q4_* :222-236, :341-364):
 * every SIMD flavour yields the same exact int32 sums; the float combine is
 * (float)s * ws * sx for INT8 and acc += (float)ig * sg, acc * sx for INT4. */
void orc_qmat_int8_path(int qtype, const void *qv, const float *scales, int n, int k,
                        const float *x, int T, float *out, int32_t *int_sums) {
    int8_t *qx = (int8_t *)malloc((size_t)k);
    const int G = k / 32;
    for (int t = 0; t < T; t++) {
        const float sx = orc_act_quant_int8(x + (size_t)t * k, k, qx);
        for (int r = 0; r < n; r++) {
            if (qtype == 1) {
                const int8_t *q = (const int8_t *)qv + (size_t)r * k;
                int64_t s = 0;
                for (int j = 0; j < k; j++) s += (int64_t)q[j] * qx[j];
                if (int_sums) int_sums[(size_t)t * n + r] = (int32_t)s;
                out[(size_t)t * n + r] = (float)(int32_t)s * scales[r] * sx;
            } else {
                const uint8_t *q = (const uint8_t *)qv + (size_t)r * (k / 2);
                float acc = 0.0f;
                for (int g = 0; g < G; g++) {
                    int64_t ig = 0;
                    for (int j = 0; j < 32; j += 2) {
                        const uint8_t b = q[16 * g + j / 2];
                        ig += (int64_t)((b & 15) - 8) * qx[32 * g + j];
                        ig += (int64_t)((b >> 4) - 8) * qx[32 * g + j + 1];
                    }
                    if (int_sums) int_sums[((size_t)t * n + r) * G + g] = (int32_t)ig;
                    acc += (float)(int32_t)ig * scales[(size_t)r * G + g];
                }
                out[(size_t)t * n + r] = acc * sx;
            }
        }
    }
    free(qx);
}

/* ------------------------------------------ INT8ACT over ggml block formats
 * Integer form of one K-quant super-block: quant q[e] (offsets applied, e.g.
 * Q3_K q - 4*!hbit, Q6_K q - 32), sub-block factor f and min m of the
 * sub-block holding e (16 elements for Q2_K, Q3_K, Q6_K; 32 for Q4_K, Q5_K),
 * super-block factors d, dmin. The decoders above are these integers put
 * together in f32: (d * f) * q - dmin * m (Q2_K, Q4_K, Q5_K), (d * f) * q
 * (Q3_K, Q6_K); orc_kquant_ints returns them so that a test can rebuild the
 * decoder's output from them bit for bit. */
static int kq_sub(int type) { return (type == ORC_Q4_K || type == ORC_Q5_K) ? 32 : 16; }

int orc_kquant_ints(int type, const void *block, int32_t *q, int32_t *f, int32_t *m, float *d, float *dmin) {
    const unsigned char *s = (const unsigned char *)block;
    switch (type) {
    case ORC_Q2_K:
        *d = h2f(s + 80), *dmin = h2f(s + 82);
        for (int e = 0; e < 256; e++) {
            const int h = e / 128, r = e % 128, fi = r / 32, l = r % 32;
            q[e] = (s[16 + 32 * h + l] >> (2 * fi)) & 3;
        }
        for (int j = 0; j < 16; j++) f[j] = s[j] & 15, m[j] = s[j] >> 4;
        return 0;
    case ORC_Q3_K:
        *d = h2f(s + 108), *dmin = 0.0f;
        for (int e = 0; e < 256; e++) {
            const int h = e / 128, r = e % 128, fi = r / 32, l = r % 32;
            const int v = (s[32 + 32 * h + l] >> (2 * fi)) & 3;
            q[e] = v - (((s[l] >> (4 * h + fi)) & 1) ? 0 : 4);
        }
        for (int j = 0; j < 16; j++) f[j] = q3k_scale(s + 96, j), m[j] = 0;
        return 0;
    case ORC_Q4_K:
    case ORC_Q5_K: {
        *d = h2f(s), *dmin = h2f(s + 2);
        const unsigned char *qs = s + (type == ORC_Q4_K ? 16 : 48);
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            k4_sm(s + 4, j, &sc, &mn);
            f[j] = sc, m[j] = mn;
            for (int i = 0; i < 32; i++) {
                int v = (j & 1) ? (qs[32 * (j / 2) + i] >> 4) : (qs[32 * (j / 2) + i] & 15);
                if (type == ORC_Q5_K && ((s[16 + i] >> j) & 1)) v += 16;
                q[32 * j + i] = v;
            }
        }
        return 0;
    }
    case ORC_Q6_K:
        *d = h2f(s + 208), *dmin = 0.0f;
        for (int e = 0; e < 256; e++) {
            const int h = e / 128, r = e % 128, fi = r / 32, l = r % 32;
            const unsigned char lb = s[64 * h + 32 * (fi & 1) + l];
            const int lo = (fi >= 2) ? (lb >> 4) : (lb & 15);
            const int hi = (s[128 + 32 * h + l] >> (2 * fi)) & 3;
            q[e] = (lo | (hi << 4)) - 32;
        }
        for (int j = 0; j < 16; j++) f[j] = (signed char)s[192 + j], m[j] = 0;
        return 0;
    }
    return -1;
}

/* ingot's int8 activations for the K-quants (third_party/ingot/src/kernels.c:
 * 719-750, q4_k_quantize_activation): per 256-element super-block, scale =
 * amax/127, q = round-to-nearest-even(x * (127/amax)) saturated to int8
 * (CVTPS2DQ and the saturating packs); an all-zero block gives q = 0, scale 0.
 * Returns the scale. */
float orc_act_quant_sb(const float *x, int8_t *qx) {
    float amax = 0.0f;
    for (int i = 0; i < 256; i++) if (fabsf(x[i]) > amax) amax = fabsf(x[i]);
    if (!(amax > 0.0f)) { memset(qx, 0, 256); return 0.0f; }
    const float inv = 127.0f / amax;
    for (int i = 0; i < 256; i++) qx[i] = (int8_t)clampi((int)nearbyintf(x[i] * inv), -128, 127);
    return amax / 127.0f;
}

/* INT8ACT over the ggml block formats, in the order the HIP unit evaluates it
 * (this build's definition: the reference has an int8 path over ggml blocks
 * only for Q4_K/Q5_K, kernels.c:1649-1795, whose f32 combine runs in another
 * order; that path is the check against the reference, within its own budget).
 * K is cut into chunks of 128 (4 blocks of 32, or half a super-block).
 *   Q8_0 / Q4_0: activations per row as quantize_act_int8 (scale sx); per chunk
 *     acc = 0, acc = fmaf(d_b, (float)t_b, acc) over its blocks, t_b = sum
 *     q_w * q_x (exact); total = fmaf(sx, acc, total), chunks in order.
 *   K-quants: activations per super-block (orc_act_quant_sb, scale s_B); per
 *     chunk the exact integers A = sum_j f_j sum_{e in j} q_e qx_e and
 *     Bm = sum_j m_j * xsum_j (xsum_j = sum of qx over sub-block j), then
 *       Q2_K, Q4_K, Q5_K: acc = fmaf(-(32 dmin), (float)Bm / 32, d * (float)A)
 *       Q3_K:             acc = d * (float)A
 *       Q6_K:             acc = 0, acc = fmaf(d * f_j, (float)t_j, acc) over
 *                         its 16-element sub-blocks j in order
 *     ((float)A is exact: |A| < 2^24; for Q5_K A is the int32 sum of the
 *     chunk's two 64-element halves, each below 2^24, converted once);
 *     total = fmaf(s_B, acc, total), chunks in order.
 * chunk_ints (optional) [T, n, k/128, 2] receives (A, Bm) of the K-quants. */
void orc_int8act_blocks(int type, const void *blocks, int n, int k, const float *x, int T, float *out,
                        int64_t *chunk_ints) {
    int be, bb;
    orc_geometry(type, &be, &bb);
    const int nblk = k / be, Kc = (k + 127) / 128;
    const unsigned char *w = (const unsigned char *)blocks;
    int8_t *qx = (int8_t *)calloc((size_t)Kc * 128 + 256, 1);
    float *xs = (float *)calloc((size_t)nblk + 1, sizeof(float));
    int32_t qi[256], fi[16], mi[16];
    for (int t = 0; t < T; t++) {
        const float *xr = x + (size_t)t * k;
        float sx = 0.0f;
        if (be == 32) {
            memset(qx, 0, (size_t)Kc * 128);
            sx = orc_act_quant_int8(xr, k, qx);
        } else {
            for (int b = 0; b < nblk; b++) xs[b] = orc_act_quant_sb(xr + 256 * b, qx + 256 * b);
        }
        for (int r = 0; r < n; r++) {
            const unsigned char *row = w + (size_t)r * nblk * bb;
            float total = 0.0f;
            if (be == 32) {
                for (int c = 0; c < Kc; c++) {
                    float acc = 0.0f;
                    for (int b = 4 * c; b < 4 * c + 4 && b < nblk; b++) {
                        const unsigned char *blk = row + (size_t)b * bb;
                        const float d = h2f(blk);
                        int64_t tb = 0;
                        for (int i = 0; i < 32; i++) {
                            const int qv = type == ORC_Q8_0 ? (signed char)blk[2 + i]
                                                            : (i < 16 ? (blk[2 + i] & 15) : (blk[2 + i - 16] >> 4)) - 8;
                            tb += (int64_t)qv * qx[32 * b + i];
                        }
                        acc = fmaf(d, (float)tb, acc);
                    }
                    total = fmaf(sx, acc, total);
                }
            } else {
                const int sub = kq_sub(type);
                float d = 0.0f, dmin = 0.0f;
                for (int c = 0; c < Kc; c++) {
                    const int B = c / 2, e0 = 128 * (c & 1);
                    orc_kquant_ints(type, row + (size_t)B * bb, qi, fi, mi, &d, &dmin);
                    const int8_t *xq = qx + 256 * B;
                    float acc = 0.0f;
                    if (type == ORC_Q6_K) {
                        for (int j = e0 / 16; j < e0 / 16 + 8; j++) {
                            int64_t tj = 0;
                            for (int i = 16 * j; i < 16 * j + 16; i++) tj += (int64_t)qi[i] * xq[i];
                            acc = fmaf(d * (float)fi[j], (float)tj, acc);
                        }
                    } else {
                        int64_t A0 = 0, A1 = 0, Bm = 0;
                        for (int e = e0; e < e0 + 128; e++) {
                            const int64_t p = (int64_t)qi[e] * fi[e / sub] * xq[e];
                            if (e < e0 + 64) A0 += p; else A1 += p;
                        }
                        for (int j = e0 / sub; j < (e0 + 128) / sub; j++) {
                            int64_t xsum = 0;
                            for (int i = sub * j; i < sub * j + sub; i++) xsum += xq[i];
                            Bm += (int64_t)mi[j] * xsum;
                        }
                        const float Af = type == ORC_Q5_K ? (float)(int32_t)(A0 + A1) : (float)(A0 + A1);
                        if (type == ORC_Q3_K) acc = d * Af;
                        else acc = fmaf(-(dmin * 32.0f), (float)((double)Bm / 32.0), d * Af);
                        if (chunk_ints) {
                            chunk_ints[(((size_t)t * n + r) * Kc + c) * 2] = A0 + A1;
                            chunk_ints[(((size_t)t * n + r) * Kc + c) * 2 + 1] = Bm;
                        }
                    }
                    total = fmaf(xs[B], acc, total);
                }
            }
            out[(size_t)t * n + r] = total;
        }
    }
    free(qx);
    free(xs);
}

/* ---------------------------------------------------- double reference GEMM
 * The pattern of the reference's own self-test (tests/test_qmat.c:39-45):
 * every output accumulated in double from the f32 operands. */
typedef struct {
    const float *x, *wd;
    int T, n, k, t0, t1;
    double *out;
} gemm_job;

static void *gemm_rows(void *arg) {
    const gemm_job *g = (const gemm_job *)arg;
    for (int t = g->t0; t < g->t1; t++) {
        const float *xr = g->x + (size_t)t * g->k;
        for (int r = 0; r < g->n; r++) {
            const float *wr = g->wd + (size_t)r * g->k;
            double acc = 0.0;
            for (int j = 0; j < g->k; j++) acc += (double)xr[j] * (double)wr[j];
            g->out[(size_t)t * g->n + r] = acc;
        }
    }
    return NULL;
}

void orc_gemm_f64(const float *x, const float *wd, int T, int n, int k, double *out,
                  int threads) {
    if (threads <= 0) threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (threads > 64) threads = 64;
    if (threads > T) threads = T > 0 ? T : 1;
    pthread_t tid[64];
    gemm_job job[64];
    for (int i = 0; i < threads; i++) {
        job[i] = (gemm_job){x, wd, T, n, k, (int)((long)T * i / threads),
                            (int)((long)T * (i + 1) / threads), out};
        pthread_create(&tid[i], NULL, gemm_rows, &job[i]);
    }
    for (int i = 0; i < threads; i++) pthread_join(tid[i], NULL);
}

/* ----------------------------------------- a thread pool for oracle/_ref
 * ingot runs its row loops through a parallel_for its host installs
 * (ingot_set_parallel_for, third_party/ingot/src/cpu.c:217-230; serial by
 * default). For timing the reference's CPU kernels on all host cores, this
 * installs one that splits [0, count) into `threads` contiguous ranges. The
 * workers are started once and stay alive; they spin on a generation counter
 * for a while after each job, then sleep on a condition variable, so a call
 * costs a wake-up, not a thread creation, and an idle pool uses no CPU. The calling
 * thread runs range 0 itself. Calls are serialised by the caller (timing runs
 * one kernel at a time). */
typedef void (*orc_range_fn)(size_t begin, size_t end, void *user);
typedef void (*orc_set_pf_fn)(void (*)(size_t, orc_range_fn, void *));
#define ORC_POOL_MAX 256
static struct {
    int threads;                 /* workers + the caller */
    int started;                 /* workers running */
    _Atomic unsigned long gen;   /* bumped per job */
    _Atomic int pending;         /* workers still on the current job */
    orc_range_fn fn;
    void *user;
    size_t count;
    int nt;                      /* ranges of the current job */
    pthread_t th[ORC_POOL_MAX];
    pthread_mutex_t mu;
    pthread_cond_t cv;
} g_pool = {1, 0, 0, 0, NULL, NULL, 0, 1, {0}, PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER};

/* a worker's id and the generation current when it was created: the next
 * job published is the first it joins */
static struct { int id; unsigned long gen0; } g_pool_start[ORC_POOL_MAX];

static void *orc_pool_worker(void *arg) {
    const int id = ((const int *)arg)[0];     /* 1 .. threads-1 */
    unsigned long seen = g_pool_start[id].gen0;
    for (;;) {
        unsigned long g;
        int spins = 0;
        while ((g = atomic_load_explicit(&g_pool.gen, memory_order_acquire)) == seen) {
            if (++spins > 200000) {
                pthread_mutex_lock(&g_pool.mu);
                while ((g = atomic_load_explicit(&g_pool.gen, memory_order_acquire)) == seen)
                    pthread_cond_wait(&g_pool.cv, &g_pool.mu);
                pthread_mutex_unlock(&g_pool.mu);
                break;
            }
        }
        seen = g;
        if (id < g_pool.nt) {
            const size_t b = g_pool.count * (size_t)id / (size_t)g_pool.nt;
            const size_t e = g_pool.count * (size_t)(id + 1) / (size_t)g_pool.nt;
            if (b < e) g_pool.fn(b, e, g_pool.user);
        }
        atomic_fetch_sub_explicit(&g_pool.pending, 1, memory_order_acq_rel);
    }
    return NULL;
}

static void orc_parallel_for(size_t count, orc_range_fn fn, void *user) {
    int nt = g_pool.threads < g_pool.started + 1 ? g_pool.threads : g_pool.started + 1;
    if ((size_t)nt > count) nt = (int)count;
    if (nt <= 1) { if (count) fn(0, count, user); return; }
    g_pool.fn = fn, g_pool.user = user, g_pool.count = count, g_pool.nt = nt;
    atomic_store_explicit(&g_pool.pending, g_pool.started, memory_order_relaxed);
    atomic_fetch_add_explicit(&g_pool.gen, 1, memory_order_release);
    pthread_mutex_lock(&g_pool.mu);
    pthread_cond_broadcast(&g_pool.cv);
    pthread_mutex_unlock(&g_pool.mu);
    fn(0, count / (size_t)nt, user);
    while (atomic_load_explicit(&g_pool.pending, memory_order_acquire) > 0) { }
}

static void orc_pool_grow(int threads) {
    if (threads > ORC_POOL_MAX) threads = ORC_POOL_MAX;
    while (g_pool.started + 1 < threads) {
        const int id = g_pool.started + 1;
        /* no job is in flight here (the caller is between jobs) */
        g_pool_start[id].id = id;
        g_pool_start[id].gen0 = atomic_load_explicit(&g_pool.gen, memory_order_relaxed);
        if (pthread_create(&g_pool.th[id], NULL, orc_pool_worker, &g_pool_start[id].id) != 0) break;
        g_pool.started++;
    }
}

/* Range count of the next jobs: at most the threads started so far (workers
 * are never stopped; a smaller count leaves the extra workers idle). */
static void orc_pool_use(int threads) {
    if (threads < 1) threads = 1;
    orc_pool_grow(threads);
    g_pool.threads = threads;
}

void orc_ingot_install_pool(void *set_parallel_for, int threads) {
    orc_pool_use(threads);
    ((orc_set_pf_fn)set_parallel_for)(orc_parallel_for);
}
