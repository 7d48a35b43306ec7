/* backend.c — backend selection and the f32 GEMM entry points
 * (src/backend.c:33-132), with a HIP branch in place of the reference's
 * Metal/CUDA ones. */
#include "backend.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mynah_asr_hip.h"
#include "qmat.h"

static int g_backend = MYNAH_ASR_BACKEND_CPU;
static mynah_asr_cpu_gemm_fn g_cpu = NULL;

int mynah_asr_set_backend(const char *name) {
    if (name && strcmp(name, "hip") == 0) {
        if (mynah_asr_hip_available()) {
            g_backend = MYNAH_ASR_BACKEND_HIP;
            fprintf(stderr, "mynah-asr: HIP backend active (gfx950, every linear on the GPU)\n");
            return g_backend;
        }
        fprintf(stderr, "mynah-asr: HIP requested but no gfx950 device available -> CPU\n");
    } else if (name && strcmp(name, "cpu") != 0) {
        fprintf(stderr, "mynah-asr: backend '%s' is not part of this build -> CPU\n", name);
    }
    g_backend = MYNAH_ASR_BACKEND_CPU;
    return g_backend;
}

int mynah_asr_backend(void) { return g_backend; }

void mynah_asr_set_cpu_fallback(mynah_asr_cpu_gemm_fn fn) { g_cpu = fn; }

/* Called when the GPU path cannot run: hand over to the program's CPU path,
 * or stop loudly — this library never computes a product on the CPU. */
void mynah_asr__cpu_or_die(const mynah_asr_qmat *m, const float *x, float *out, int T, const char *op);
void mynah_asr__cpu_or_die(const mynah_asr_qmat *m, const float *x, float *out, int T, const char *op) {
    if (g_cpu) {
        g_cpu(m, x, out, T);
        return;
    }
    fprintf(stderr, "mynah-asr: %s: %s; no CPU fallback registered (backend %d)\n", op,
            g_backend == MYNAH_ASR_BACKEND_HIP ? mynah_asr_hip_last_error() : "HIP backend not active",
            g_backend);
    abort();
}

static mynah_asr_qmat f32_qmat(const float *w, int n, int k) {
    mynah_asr_qmat m;
    memset(&m, 0, sizeof m);
    m.f32 = w;
    m.n = n;
    m.k = k;
    m.qtype = MYNAH_ASR_Q_F32;
    return m;
}

void mynah_asr_gemm_wt(const float *x, const float *w, float *out, int T, int n, int k) {
    if (g_backend == MYNAH_ASR_BACKEND_HIP && mynah_asr_hip_gemm_wt(x, w, out, T, n, k) == 0) return;
    const mynah_asr_qmat m = f32_qmat(w, n, k);
    mynah_asr__cpu_or_die(&m, x, out, T, "gemm_wt");
}

void mynah_asr_silu(float *x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = x[i] * mynah_asr_sigmoid(x[i]);
}

void mynah_asr_ffn_wt(const float *x, const float *w1, int n1, const float *w2, int n2, float *out,
                      int T, int k, float *scratch) {
    if (g_backend == MYNAH_ASR_BACKEND_HIP && mynah_asr_hip_ffn_wt(x, w1, n1, w2, n2, out, T, k) == 0)
        return;
    mynah_asr_gemm_wt(x, w1, scratch, T, n1, k);
    mynah_asr_silu(scratch, (size_t)T * (size_t)n1);
    mynah_asr_gemm_wt(scratch, w2, out, T, n2, n1);
}

void mynah_asr_gemm3_wt(const float *x, const float *wa, const float *wb, const float *wc, float *oa,
                        float *ob, float *oc, int T, int n, int k) {
    if (g_backend == MYNAH_ASR_BACKEND_HIP &&
        mynah_asr_hip_gemm3_wt(x, wa, wb, wc, oa, ob, oc, T, n, k) == 0)
        return;
    mynah_asr_gemm_wt(x, wa, oa, T, n, k);
    mynah_asr_gemm_wt(x, wb, ob, T, n, k);
    mynah_asr_gemm_wt(x, wc, oc, T, n, k);
}
