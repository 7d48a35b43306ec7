/* qmat.h — mynah-asr's quantized linear-op API (src/qmat.h), as this library
 * provides it on MI355X. Names, argument meaning and the struct's leading
 * fields are the reference's; two additions carry ggml blocks straight to the
 * device (the reference decodes them to f32 at load, src/weights.c:103-114):
 * the block qtypes below and mynah_asr_qmat_init_blocks().
 *
 * Dispatch: with the "hip" backend active every product runs on the GPU
 * through include/mynah_asr_hip.h. This library carries no CPU GEMM: when the
 * GPU call cannot run, the registered CPU fallback (mynah_asr_set_cpu_fallback,
 * in the full program the reference's own qmat.c/backend.c CPU code) is used;
 * with none registered the call prints the reason and aborts. */
#ifndef MYNAH_ASR_QMAT_H
#define MYNAH_ASR_QMAT_H

#include <math.h>
#include <stddef.h>
#include <stdint.h>

#include "mynah_asr_hip.h"

enum {
    MYNAH_ASR_Q_F32 = 0, MYNAH_ASR_Q_INT8 = 1, MYNAH_ASR_Q_INT4 = 2,
    /* ggml block formats, raw GGUF bytes (same ids as MYNAH_ASR_HIP_*) */
    MYNAH_ASR_Q_Q4_0 = MYNAH_ASR_HIP_Q4_0, MYNAH_ASR_Q_Q8_0 = MYNAH_ASR_HIP_Q8_0,
    MYNAH_ASR_Q_Q2_K = MYNAH_ASR_HIP_Q2_K, MYNAH_ASR_Q_Q3_K = MYNAH_ASR_HIP_Q3_K,
    MYNAH_ASR_Q_Q4_K = MYNAH_ASR_HIP_Q4_K, MYNAH_ASR_Q_Q5_K = MYNAH_ASR_HIP_Q5_K,
    MYNAH_ASR_Q_Q6_K = MYNAH_ASR_HIP_Q6_K
};

/* stable sigmoid (src/qmat.h:31-35) */
static inline float mynah_asr_sigmoid(float x) {
    if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
    const float e = expf(x);
    return e / (1.0f + e);
}

#define MYNAH_ASR_Q4_GROUP 32

typedef struct {
    const float *f32;        /* F32 [n, k] */
    const int8_t *q8;        /* INT8 [n, k] */
    const uint8_t *q4;       /* INT4 packed [n, k/2] */
    const float *scales;     /* INT8: [n]; INT4: [n, k/32] */
    void *owned_q, *owned_s; /* buffers quantized at load, freed by qmat_free */
    int qtype;
    int n, k;
    const void *blocks;      /* ggml block qtypes: [n, k/block] raw blocks */
} mynah_asr_qmat;

/* src/qmat.c:80-112 (quantize on load for INT8/INT4) */
int mynah_asr_qmat_init(mynah_asr_qmat *m, const float *w, int n, int k, int qtype);
/* ggml blocks as stored in a GGUF (borrowed, must outlive m). 0 ok, -1 bad. */
int mynah_asr_qmat_init_blocks(mynah_asr_qmat *m, const void *blocks, int n, int k, int qtype);
void mynah_asr_qmat_free(mynah_asr_qmat *m);

/* out[T, n] = x[T, k] @ W^T */
void mynah_asr_qmat_mul(const mynah_asr_qmat *m, const float *x, float *out, int T);
/* out = SiLU(x @ W1^T) @ W2^T; scratch >= T*w1->n floats (used only by the CPU fallback) */
void mynah_asr_qmat_ffn(const mynah_asr_qmat *w1, const mynah_asr_qmat *w2, const float *x,
                        float *out, int T, float *scratch);
void mynah_asr_qmat_qkv(const mynah_asr_qmat *wq, const mynah_asr_qmat *wk, const mynah_asr_qmat *wv,
                        const float *x, float *oq, float *ok, float *ov, int T);
void mynah_asr_qmat_dequant(const mynah_asr_qmat *m, float *wd);

/* src/qmat.c:19-67 */
void mynah_asr_quantize_int8(const float *w, int n, int k, int8_t *out_q, float *out_scales);
void mynah_asr_quantize_int4(const float *w, int n, int k, uint8_t *out_q, float *out_scales);

#endif
