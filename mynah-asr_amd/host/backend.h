/* backend.h — mynah-asr's backend selection and f32 GEMM API (src/backend.h),
 * with the HIP backend registered next to the reference's cpu/metal/cuda. */
#ifndef MYNAH_ASR_BACKEND_H
#define MYNAH_ASR_BACKEND_H

#include <stddef.h>

enum {
    MYNAH_ASR_BACKEND_CPU = 0, MYNAH_ASR_BACKEND_METAL = 1, MYNAH_ASR_BACKEND_CUDA = 2,
    MYNAH_ASR_BACKEND_HIP = 3
};

/* "cpu" | "hip" (others resolve to cpu here). Returns the EFFECTIVE backend;
 * an unavailable request falls back to CPU with a note on stderr
 * (src/backend.c:33-64). */
int mynah_asr_set_backend(const char *name);
int mynah_asr_backend(void);

/* out[T,n] = x[T,k] @ W[n,k]^T */
void mynah_asr_gemm_wt(const float *x, const float *w, float *out, int T, int n, int k);
void mynah_asr_silu(float *x, size_t n);
void mynah_asr_ffn_wt(const float *x, const float *w1, int n1, const float *w2, int n2,
                      float *out, int T, int k, float *scratch);
void mynah_asr_gemm3_wt(const float *x, const float *wa, const float *wb, const float *wc,
                        float *oa, float *ob, float *oc, int T, int n, int k);

/* The CPU path the embedding program provides (in mynah-asr: qmat.c's dot
 * kernels + cblas_sgemm). Receives the failed operation's name and arguments
 * as the generic product `out[T,n] = x[T,k] @ dequant(m)^T`. */
typedef void (*mynah_asr_cpu_gemm_fn)(const void *qmat /* const mynah_asr_qmat* */, const float *x,
                                      float *out, int T);
void mynah_asr_set_cpu_fallback(mynah_asr_cpu_gemm_fn fn);

#endif
