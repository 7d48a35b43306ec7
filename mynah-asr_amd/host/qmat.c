/* qmat.c — the quantized linear op (src/qmat.c) with the HIP backend as its
 * compute path. The load-time quantizers are the reference's arithmetic
 * (src/qmat.c:19-67); every product goes to include/mynah_asr_hip.h. */
#include "qmat.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "backend.h"

void mynah_asr__cpu_or_die(const mynah_asr_qmat *m, const float *x, float *out, int T, const char *op);

/* per-row scale amax/127 (1 for a zero row); q = (int8)(v +- 0.5) */
void mynah_asr_quantize_int8(const float *w, int n, int k, int8_t *out_q, float *out_scales) {
    for (int i = 0; i < n; i++) {
        const float *row = w + (size_t)i * (size_t)k;
        float amax = 0.0f;
        for (int j = 0; j < k; j++) amax = fabsf(row[j]) > amax ? fabsf(row[j]) : amax;
        const float scale = amax > 0.0f ? amax / 127.0f : 1.0f, inv = 1.0f / scale;
        out_scales[i] = scale;
        for (int j = 0; j < k; j++) {
            const float v = row[j] * inv;
            out_q[(size_t)i * k + j] = (int8_t)(v >= 0.0f ? v + 0.5f : v - 0.5f);
        }
    }
}

/* per-32 group scale amax/7 (1 for a zero group); q in [-8, 7] stored +8,
 * elements 2j (low nibble) and 2j+1 (high) share byte j of the group */
void mynah_asr_quantize_int4(const float *w, int n, int k, uint8_t *out_q, float *out_scales) {
    const int G = MYNAH_ASR_Q4_GROUP, groups = k / G;
    for (int i = 0; i < n; i++)
        for (int g = 0; g < groups; g++) {
            const float *v = w + (size_t)i * k + g * G;
            float amax = 0.0f;
            for (int j = 0; j < G; j++) amax = fabsf(v[j]) > amax ? fabsf(v[j]) : amax;
            const float scale = amax > 0.0f ? amax / 7.0f : 1.0f, inv = 1.0f / scale;
            out_scales[(size_t)i * groups + g] = scale;
            for (int j = 0; j < G; j += 2) {
                const float a = v[j] * inv, b = v[j + 1] * inv;
                int qa = (int)(a >= 0.0f ? a + 0.5f : a - 0.5f), qb = (int)(b >= 0.0f ? b + 0.5f : b - 0.5f);
                qa = qa < -8 ? -8 : qa > 7 ? 7 : qa;
                qb = qb < -8 ? -8 : qb > 7 ? 7 : qb;
                out_q[(size_t)i * (k / 2) + (g * G + j) / 2] = (uint8_t)((qa + 8) | ((qb + 8) << 4));
            }
        }
}

int mynah_asr_qmat_init(mynah_asr_qmat *m, const float *w, int n, int k, int qtype) {
    memset(m, 0, sizeof(*m));
    m->f32 = w;
    m->n = n;
    m->k = k;
    m->qtype = MYNAH_ASR_Q_F32;
    if (qtype == MYNAH_ASR_Q_F32 || !w) return 0;
    if (qtype == MYNAH_ASR_Q_INT8) {
        int8_t *q = malloc((size_t)n * (size_t)k);
        float *s = malloc((size_t)n * sizeof(float));
        if (!q || !s) { free(q); free(s); return -1; }
        mynah_asr_quantize_int8(w, n, k, q, s);
        m->q8 = q;
        m->scales = s;
        m->owned_q = q;
        m->owned_s = s;
        m->qtype = MYNAH_ASR_Q_INT8;
    } else if (qtype == MYNAH_ASR_Q_INT4) {
        if (k % MYNAH_ASR_Q4_GROUP != 0) return 0; /* stays f32 */
        uint8_t *q = malloc((size_t)n * (size_t)k / 2);
        float *s = malloc((size_t)n * (size_t)(k / MYNAH_ASR_Q4_GROUP) * sizeof(float));
        if (!q || !s) { free(q); free(s); return -1; }
        mynah_asr_quantize_int4(w, n, k, q, s);
        m->q4 = q;
        m->scales = s;
        m->owned_q = q;
        m->owned_s = s;
        m->qtype = MYNAH_ASR_Q_INT4;
    }
    return 0;
}

int mynah_asr_qmat_init_blocks(mynah_asr_qmat *m, const void *blocks, int n, int k, int qtype) {
    memset(m, 0, sizeof(*m));
    const int be = (qtype == MYNAH_ASR_Q_Q4_0 || qtype == MYNAH_ASR_Q_Q8_0) ? 32 : 256;
    if (!blocks || n <= 0 || k <= 0 || k % be != 0) return -1;
    switch (qtype) {
    case MYNAH_ASR_Q_Q4_0: case MYNAH_ASR_Q_Q8_0: case MYNAH_ASR_Q_Q2_K: case MYNAH_ASR_Q_Q3_K:
    case MYNAH_ASR_Q_Q4_K: case MYNAH_ASR_Q_Q5_K: case MYNAH_ASR_Q_Q6_K: break;
    default: return -1;
    }
    m->blocks = blocks;
    m->qtype = qtype;
    m->n = n;
    m->k = k;
    return 0;
}

static const void *key_of(const mynah_asr_qmat *m) {
    switch (m->qtype) {
    case MYNAH_ASR_Q_F32: return m->f32;
    case MYNAH_ASR_Q_INT8: return m->q8;
    case MYNAH_ASR_Q_INT4: return m->q4;
    default: return m->blocks;
    }
}

void mynah_asr_qmat_free(mynah_asr_qmat *m) {
    /* the device copy is keyed by this pointer, which may be reused after free
     * (also for borrowed f32 weights: a later allocation at the same address
     * must not find this copy) */
    if (key_of(m)) mynah_asr_hip_evict(key_of(m));
    free(m->owned_q);
    free(m->owned_s);
    memset(m, 0, sizeof(*m));
}

static mynah_asr_hip_wdesc desc_of(const mynah_asr_qmat *m) {
    mynah_asr_hip_wdesc d;
    d.qtype = m->qtype;
    d.n = m->n;
    d.k = m->k;
    d.data = key_of(m);
    d.scales = m->scales;
    return d;
}

static int on_hip(void) { return mynah_asr_backend() == MYNAH_ASR_BACKEND_HIP; }

void mynah_asr_qmat_mul(const mynah_asr_qmat *m, const float *x, float *out, int T) {
    if (on_hip()) {
        const mynah_asr_hip_wdesc d = desc_of(m);
        if (mynah_asr_hip_qgemm(&d, x, out, T) == 0) return;
    }
    mynah_asr__cpu_or_die(m, x, out, T, "qmat_mul");
}

void mynah_asr_qmat_ffn(const mynah_asr_qmat *w1, const mynah_asr_qmat *w2, const float *x, float *out,
                        int T, float *scratch) {
    if (on_hip()) {
        const mynah_asr_hip_wdesc d1 = desc_of(w1), d2 = desc_of(w2);
        if (mynah_asr_hip_qffn(&d1, &d2, x, out, T) == 0) return;
    }
    mynah_asr_qmat_mul(w1, x, scratch, T);
    mynah_asr_silu(scratch, (size_t)T * (size_t)w1->n);
    mynah_asr_qmat_mul(w2, scratch, out, T);
}

void mynah_asr_qmat_qkv(const mynah_asr_qmat *wq, const mynah_asr_qmat *wk, const mynah_asr_qmat *wv,
                        const float *x, float *oq, float *ok, float *ov, int T) {
    if (on_hip()) {
        const mynah_asr_hip_wdesc a = desc_of(wq), b = desc_of(wk), c = desc_of(wv);
        if (mynah_asr_hip_qqkv(&a, &b, &c, x, oq, ok, ov, T) == 0) return;
    }
    mynah_asr_qmat_mul(wq, x, oq, T);
    mynah_asr_qmat_mul(wk, x, ok, T);
    mynah_asr_qmat_mul(wv, x, ov, T);
}

void mynah_asr_qmat_dequant(const mynah_asr_qmat *m, float *wd) {
    if (m->qtype == MYNAH_ASR_Q_F32) {
        memcpy(wd, m->f32, (size_t)m->n * (size_t)m->k * sizeof(float));
        return;
    }
    if (on_hip()) {
        const mynah_asr_hip_wdesc d = desc_of(m);
        if (mynah_asr_hip_dequant(&d, wd) == 0) return;
    }
    fprintf(stderr, "mynah-asr: qmat_dequant: %s\n",
            on_hip() ? mynah_asr_hip_last_error() : "HIP backend not active");
    abort();
}
