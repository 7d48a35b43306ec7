/* synth.c — see synth.h. */
#include "synth.h"

#include <math.h>
#include <string.h>

#include "mynah_asr_hip.h"

/* ------------------------------------------------------------ generator */
static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void mynah_synth_randn(uint64_t seed, double sigma, float *out, size_t n) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        /* u1 in (0, 1], u2 in [0, 1): 53-bit uniforms */
        const double u1 = (double)((splitmix64(&s) >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double)(splitmix64(&s) >> 11) * 0x1.0p-53;
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(sigma * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(sigma * r * sin(two_pi * u2));
    }
}

/* ------------------------------------------------------------ f16 helpers */
static uint16_t to_f16(float f) {
    /* nearest-even for normals, half-up in the subnormal range, as ingot's
     * ingot_f32_to_f16 (dtype.c:246-268) */
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int e = (int)((u >> 23) & 0xff) - 127;
    uint32_t m = u & 0x7fffffu;
    if (e == 128) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e < -24) return (uint16_t)sign;
    if (e < -14) {
        m |= 0x800000u;
        const int sh = -e - 14;
        uint32_t r = m >> (13 + sh);
        if ((m >> (12 + sh)) & 1u) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
    const uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* ingot kernels.c:150-168: the Q4_K quantizer's own encoder (half-up on the
 * magnitude, saturating) */
static uint16_t to_f16_q4k(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    int e = (int)((u >> 23) & 0xff) - 112;
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
        if (++e >= 31) return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | r);
}

static float from_f16(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int e = (h >> 10) & 31;
    uint32_t m = h & 0x3ffu, b;
    if (e == 0) {
        if (m == 0) b = sign;
        else {
            e = 1;
            while (!(m & 0x400u)) { m <<= 1; e--; }
            b = sign | ((uint32_t)(e + 112) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) b = sign | 0x7f800000u | (m << 13);
    else b = sign | ((uint32_t)(e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &b, 4);
    return f;
}

static void put16(unsigned char *p, uint16_t v) { p[0] = (unsigned char)v; p[1] = (unsigned char)(v >> 8); }
static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }
static long clampl(long v, long lo, long hi) { return v < lo ? lo : v > hi ? hi : v; }

/* largest magnitude keeping its sign, first wins (ingot quantize.c:26-33) */
static float extreme(const float *x, int n) {
    float a = 0.0f, v = 0.0f;
    for (int i = 0; i < n; i++)
        if (fabsf(x[i]) > a) { a = fabsf(x[i]); v = x[i]; }
    return v;
}

/* ------------------------------------------------- reference quantizers */
static void q8_0(const float *x, unsigned char *o) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fabsf(x[i]) > amax ? fabsf(x[i]) : amax;
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(o, to_f16(d));
    for (int i = 0; i < 32; i++) o[2 + i] = (unsigned char)(signed char)clampi((int)lroundf(x[i] * id), -127, 127);
}

static void q4_0(const float *x, unsigned char *o) {
    const float d = extreme(x, 32) / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(o, to_f16(d));
    for (int i = 0; i < 16; i++)
        o[2 + i] = (unsigned char)(clampi((int)(x[i] * id + 8.5f), 0, 15) |
                                   (clampi((int)(x[i + 16] * id + 8.5f), 0, 15) << 4));
}

static void q6_k(const float *x, unsigned char *o) {
    float s[16], big = 0.0f;
    for (int j = 0; j < 16; j++) {
        s[j] = extreme(x + 16 * j, 16) / -32.0f;
        if (fabsf(s[j]) > fabsf(big)) big = s[j];
    }
    const float d = big / -128.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    signed char sc[16];
    for (int j = 0; j < 16; j++) sc[j] = (signed char)clampi((int)lroundf(s[j] * id), -128, 127);
    memset(o, 0, 192);
    for (int e = 0; e < 256; e++) {
        const float ds = d * (float)sc[e / 16], ids = ds != 0.0f ? 1.0f / ds : 0.0f;
        const int q = clampi((int)lroundf(x[e] * ids) + 32, 0, 63);
        const int h = e / 128, f = (e % 128) / 32, l = e % 32;
        o[64 * h + 32 * (f & 1) + l] |= (unsigned char)((q & 15) << (4 * (f / 2)));
        o[128 + 32 * h + l] |= (unsigned char)((q >> 4) << (2 * f));
    }
    memcpy(o + 192, sc, 16);
    put16(o + 208, to_f16(d));
}

/* one sub-block fit of the Q4_K quantizer (kernels.c:180-282) */
static void q4k_fit(const float *v, float *step_out, float *off_out) {
    float lo = v[0], hi = v[0];
    for (int i = 1; i < 32; i++) { lo = v[i] < lo ? v[i] : lo; hi = v[i] > hi ? v[i] : hi; }
    if (lo > 0.0f) lo = 0.0f;
    if (hi < 0.0f) hi = 0.0f;
    float best_step = (hi - lo) / 15.0f, best_off = -lo, best_err = -1.0f;
    for (int c = 0; c <= 5; c++) {
        const float shrink = 1.0f - 0.04f * (float)c;
        const float mid = 0.5f * (hi + lo), half = 0.5f * shrink * (hi - lo);
        float a = mid - half, b = mid + half;
        if (a > 0.0f) a = 0.0f;
        if (b < 0.0f) b = 0.0f;
        float step = (b - a) / 15.0f;
        if (!(step > 0.0f)) continue;
        for (int round = 0; round < 2; round++) {
            float sq = 0.0f, sqq = 0.0f, sx = 0.0f, sxq = 0.0f;
            for (int i = 0; i < 32; i++) {
                const float q = (float)clampl(lrintf((v[i] - a) / step), 0, 15);
                sq += q; sqq += q * q; sx += v[i]; sxq += v[i] * q;
            }
            const float det = 32.0f * sqq - sq * sq;
            if (!(fabsf(det) > 1e-12f)) break;
            float fit = (32.0f * sxq - sq * sx) / det, base = (sx - fit * sq) / 32.0f;
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
            const float q = (float)clampl(lrintf((v[i] - a) / step), 0, 15);
            const float diff = step * q + a - v[i];
            err += diff * diff;
        }
        if (best_err < 0.0f || err < best_err) { best_err = err; best_step = step; best_off = -a; }
    }
    *step_out = best_step;
    *off_out = best_off;
}

static void q4_k(const float *x, unsigned char *o) {
    float st[8], of[8], mst = 0.0f, mof = 0.0f;
    for (int j = 0; j < 8; j++) {
        q4k_fit(x + 32 * j, &st[j], &of[j]);
        mst = st[j] > mst ? st[j] : mst;
        mof = of[j] > mof ? of[j] : mof;
    }
    const uint16_t dh = to_f16_q4k(mst / 63.0f), mh = to_f16_q4k(mof / 63.0f);
    put16(o, dh);
    put16(o + 2, mh);
    const float d = from_f16(dh), dmin = from_f16(mh);
    unsigned char sb[8], mb[8];
    for (int j = 0; j < 8; j++) {
        sb[j] = (unsigned char)clampl(d > 0.0f ? lrintf(st[j] / d) : 0, 0, 63);
        mb[j] = (unsigned char)clampl(dmin > 0.0f ? lrintf(of[j] / dmin) : 0, 0, 63);
    }
    for (int j = 0; j < 4; j++) {
        o[4 + j] = (unsigned char)(sb[j] | ((sb[j + 4] >> 4) << 6));
        o[8 + j] = (unsigned char)(mb[j] | ((mb[j + 4] >> 4) << 6));
        o[12 + j] = (unsigned char)((sb[j + 4] & 15) | ((mb[j + 4] & 15) << 4));
    }
    for (int p = 0; p < 4; p++) {
        const float sl = d * sb[2 * p], sh = d * sb[2 * p + 1];
        const float ol = dmin * mb[2 * p], oh = dmin * mb[2 * p + 1];
        for (int i = 0; i < 32; i++) {
            const long l = clampl(sl > 0.0f ? lrintf((x[64 * p + i] + ol) / sl) : 0, 0, 15);
            const long h = clampl(sh > 0.0f ? lrintf((x[64 * p + 32 + i] + oh) / sh) : 0, 0, 15);
            o[16 + 32 * p + i] = (unsigned char)(l | (h << 4));
        }
    }
}

/* ------------------------------------ this library's own K-quant fits
 * Plain range fits with no search, enough to make realistic test weights. */

/* Q5_K: per 32-sub-block affine fit over 32 levels; scale/min 6-bit against
 * f16 super factors; layout as ingot dequant.c:278-350 reads it. */
static void q5_k(const float *x, unsigned char *o) {
    float st[8], of[8], mst = 0.0f, mof = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = 0.0f, hi = 0.0f;
        for (int i = 0; i < 32; i++) { lo = fminf(lo, x[32 * j + i]); hi = fmaxf(hi, x[32 * j + i]); }
        st[j] = (hi - lo) / 31.0f;
        of[j] = -lo;
        mst = fmaxf(mst, st[j]);
        mof = fmaxf(mof, of[j]);
    }
    const uint16_t dh = to_f16(mst / 63.0f), mh = to_f16(mof / 63.0f);
    put16(o, dh);
    put16(o + 2, mh);
    const float d = from_f16(dh), dmin = from_f16(mh);
    unsigned char sb[8], mb[8];
    for (int j = 0; j < 8; j++) {
        sb[j] = (unsigned char)clampl(d > 0.0f ? lrintf(st[j] / d) : 0, 0, 63);
        mb[j] = (unsigned char)clampl(dmin > 0.0f ? lrintf(of[j] / dmin) : 0, 0, 63);
    }
    for (int j = 0; j < 4; j++) {
        o[4 + j] = (unsigned char)(sb[j] | ((sb[j + 4] >> 4) << 6));
        o[8 + j] = (unsigned char)(mb[j] | ((mb[j + 4] >> 4) << 6));
        o[12 + j] = (unsigned char)((sb[j + 4] & 15) | ((mb[j + 4] & 15) << 4));
    }
    memset(o + 16, 0, 160);
    for (int j = 0; j < 8; j++) {
        const float s = d * sb[j], m = dmin * mb[j];
        for (int i = 0; i < 32; i++) {
            const long q = clampl(s > 0.0f ? lrintf((x[32 * j + i] + m) / s) : 0, 0, 31);
            o[48 + 32 * (j / 2) + i] |= (unsigned char)((q & 15) << (4 * (j & 1)));
            o[16 + i] |= (unsigned char)(((q >> 4) & 1) << j);
        }
    }
}

/* Q3_K: symmetric per 16-sub-block, q in [-4, 3]; 6-bit signed scales (stored
 * +32) against one f16 factor; layout as dequant.c:190-220 reads it. */
static void q3_k(const float *x, unsigned char *o) {
    float s[16], big = 0.0f;
    for (int j = 0; j < 16; j++) {
        s[j] = extreme(x + 16 * j, 16) / -4.0f;
        if (fabsf(s[j]) > fabsf(big)) big = s[j];
    }
    const float d = fabsf(big) / 31.0f;
    const uint16_t dh = to_f16(d);
    const float dq = from_f16(dh);
    int sc[16];
    for (int j = 0; j < 16; j++) sc[j] = clampi(dq > 0.0f ? (int)lrintf(s[j] / dq) : 0, -32, 31);
    memset(o, 0, 110);
    for (int j = 0; j < 16; j++) {
        const int v = sc[j] + 32;
        if (j < 8) o[96 + j] |= (unsigned char)(v & 15);
        else o[96 + j - 8] |= (unsigned char)((v & 15) << 4);
        o[104 + (j % 4)] |= (unsigned char)(((v >> 4) & 3) << (2 * (j / 4)));
    }
    for (int e = 0; e < 256; e++) {
        const float ds = dq * (float)sc[e / 16];
        const int q = clampi(ds != 0.0f ? (int)lrintf(x[e] / ds) : 0, -4, 3) + 4;
        const int h = e / 128, f = (e % 128) / 32, l = e % 32;
        o[32 + 32 * h + l] |= (unsigned char)((q & 3) << (2 * f));
        if (q >> 2) o[l] |= (unsigned char)(1u << (4 * h + f));
    }
    put16(o + 108, dh);
}

/* Q2_K: affine per 16-sub-block over 4 levels; 4-bit scale and min against
 * f16 factors; layout as dequant.c:164-184 reads it. */
static void q2_k(const float *x, unsigned char *o) {
    float st[16], of[16], mst = 0.0f, mof = 0.0f;
    for (int j = 0; j < 16; j++) {
        float lo = 0.0f, hi = 0.0f;
        for (int i = 0; i < 16; i++) { lo = fminf(lo, x[16 * j + i]); hi = fmaxf(hi, x[16 * j + i]); }
        st[j] = (hi - lo) / 3.0f;
        of[j] = -lo;
        mst = fmaxf(mst, st[j]);
        mof = fmaxf(mof, of[j]);
    }
    const uint16_t dh = to_f16(mst / 15.0f), mh = to_f16(mof / 15.0f);
    const float d = from_f16(dh), dmin = from_f16(mh);
    memset(o, 0, 84);
    for (int j = 0; j < 16; j++) {
        const int s = (int)clampl(d > 0.0f ? lrintf(st[j] / d) : 0, 0, 15);
        const int m = (int)clampl(dmin > 0.0f ? lrintf(of[j] / dmin) : 0, 0, 15);
        o[j] = (unsigned char)(s | (m << 4));
        const float ds = d * (float)s, dm = dmin * (float)m;
        for (int i = 0; i < 16; i++) {
            const int e = 16 * j + i;
            const int q = (int)clampl(ds > 0.0f ? lrintf((x[e] + dm) / ds) : 0, 0, 3);
            const int h = e / 128, f = (e % 128) / 32, l = e % 32;
            o[16 + 32 * h + l] |= (unsigned char)(q << (2 * f));
        }
    }
    put16(o + 80, dh);
    put16(o + 82, mh);
}

/* ---------------------------------------------------------------- entry */
static int geometry(int qtype, int *be, int *bb) {
    switch (qtype) {
    case MYNAH_ASR_HIP_Q4_0: *be = 32; *bb = 18; return 0;
    case MYNAH_ASR_HIP_Q8_0: *be = 32; *bb = 34; return 0;
    case MYNAH_ASR_HIP_Q2_K: *be = 256; *bb = 84; return 0;
    case MYNAH_ASR_HIP_Q3_K: *be = 256; *bb = 110; return 0;
    case MYNAH_ASR_HIP_Q4_K: *be = 256; *bb = 144; return 0;
    case MYNAH_ASR_HIP_Q5_K: *be = 256; *bb = 176; return 0;
    case MYNAH_ASR_HIP_Q6_K: *be = 256; *bb = 210; return 0;
    }
    return -1;
}

size_t mynah_synth_nbytes(int qtype, size_t count) {
    int be, bb;
    if (geometry(qtype, &be, &bb) || count % (size_t)be) return 0;
    return count / (size_t)be * (size_t)bb;
}

size_t mynah_synth_quantize(int qtype, const float *x, size_t count, void *out) {
    int be, bb;
    if (!x || !out || geometry(qtype, &be, &bb) || count % (size_t)be) return 0;
    void (*fn)(const float *, unsigned char *) = 0;
    switch (qtype) {
    case MYNAH_ASR_HIP_Q4_0: fn = q4_0; break;
    case MYNAH_ASR_HIP_Q8_0: fn = q8_0; break;
    case MYNAH_ASR_HIP_Q2_K: fn = q2_k; break;
    case MYNAH_ASR_HIP_Q3_K: fn = q3_k; break;
    case MYNAH_ASR_HIP_Q4_K: fn = q4_k; break;
    case MYNAH_ASR_HIP_Q5_K: fn = q5_k; break;
    case MYNAH_ASR_HIP_Q6_K: fn = q6_k; break;
    }
    unsigned char *o = (unsigned char *)out;
    const size_t nb = count / (size_t)be;
    for (size_t b = 0; b < nb; b++) fn(x + b * (size_t)be, o + b * (size_t)bb);
    return nb * (size_t)bb;
}
