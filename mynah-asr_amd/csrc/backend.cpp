// backend.cpp — the C ABI of include/mynah_asr_hip.h.
//
// Structure (the roles of src/cuda_gemm.cu, built the MI355X way):
//   * a process-wide resident weight cache keyed by the caller's host pointer,
//     holding each weight in the repacked device layout (repack.cpp), guarded
//     by one mutex held only around the cache (src/cuda_gemm.cu:92-130);
//   * a per-thread context: one HIP stream (default priority) and grow-only
//     device buffers for activations, outputs and the prepared-activation
//     workspace (src/cuda_gemm.cu:50-90);
//   * every host-pointer entry point = H2D copy of x, prep + GEMM kernels on the
//     thread's stream, D2H copy of out, stream sync. 0 = done, -1 = the caller
//     runs its CPU path (src/backend.c:74-77).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <vector>

#include "fmt.h"
#include "launch.h"
#include "mynah_asr_hip.h"
#include "repack.h"

struct mynah_asr_hip_weight {
    DevW dw;
    int qtype;
    void *mem;
    size_t bytes;
};

namespace {

std::mutex g_mu;
int g_ready = -1;
// the process-wide numerics mode (-1: not yet read from the environment);
// atomic: set_numerics may run while other threads' calls read it
std::atomic<int> g_numerics{-1};

struct CacheEnt {
    const void *key;
    int qtype, n, k;
    mynah_asr_hip_weight *w;
};
std::vector<CacheEnt> g_cache;

thread_local char t_err[256];

int fail(const char *msg, const char *detail = nullptr) {
    snprintf(t_err, sizeof t_err, "%s%s%s", msg, detail ? ": " : "", detail ? detail : "");
    return -1;
}

// Set once the calling thread has issued a _dev call on a stream under capture:
// a HIP graph may then hold pointers into this thread's buffers, so a buffer
// that grows afterwards keeps its old allocation alive (t_retired, held until
// the process ends) instead of freeing it, and the graph's replays keep
// writing and reading memory of their own.
thread_local bool t_captured = false;
thread_local std::vector<void *> t_retired;

void note_capture(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs == hipStreamCaptureStatusActive) t_captured = true;
}

// grow-only device buffer
struct DBuf {
    void *p = nullptr;
    size_t cap = 0;
    void *get(size_t bytes) {
        if (bytes == 0) bytes = 256;
        if (p && cap >= bytes) return p;
        size_t want = cap ? cap : ((size_t)1 << 20);
        while (want < bytes) want *= 2;
        if (p) {
            if (t_captured) t_retired.push_back(p);
            else (void)hipFree(p);
        }
        p = nullptr;
        cap = 0;
        if (hipMalloc(&p, want) != hipSuccess) { p = nullptr; return nullptr; }
        cap = want;
        return p;
    }
};

// a prepared input: the buffers and what they hold now (i8: 0 = EXACT, else
// the INT8ACT activation form, MH_I8_QMAT / _ROW / _SB)
struct PrepBuf {
    DBuf xp, xs16, xpf;
    int T = -1, Kp = 0, xsum = 0, i8 = 0;
    // non-null: the activations whose EXACT preparation (no row sums) these
    // buffers hold, written by the layer norm that produced them in place
    // of f32 rows; a preparation of those activations is then skipped
    const void *src = nullptr;
};

struct Ctx {
    int state = 0;  // 0 uninitialised, 1 ok, -1 failed
    hipStream_t st = nullptr;
    DBuf x, y, h;
    DBuf att;    // the host-pointer attention call's q, k, v, rk, biases and ctx
    DBuf attw;   // the attention core's workspace (K and rk split into f16 planes)
    DBuf aed;    // the AED decoder's caches and vectors
    DBuf enc;    // the encoder layer's activations
    DBuf ssb;    // the subsampling's activations
    DBuf gs;     // split-K GEMV workspace
    DBuf gk;     // split-K GEMM workspace (chunk results)
    int *pin = nullptr;   // pinned host int[2][2]: the step state of two positions read back
    hipEvent_t pev[2] = {nullptr, nullptr};   // their copies' completion
    PrepBuf pa;  // the products' input (prep_dev / qgemm_prepped_dev use this one)
    PrepBuf pb;  // the FFN's intermediate, prepared by the first product
};
thread_local Ctx t_ctx;

Ctx *ctx() {
    if (t_ctx.state == 0)
        t_ctx.state = hipStreamCreateWithFlags(&t_ctx.st, hipStreamNonBlocking) == hipSuccess ? 1 : -1;
    return t_ctx.state == 1 ? &t_ctx : nullptr;
}

hipStream_t pick_stream(void *s) {
    if (s) return (hipStream_t)s;
    Ctx *c = ctx();
    return c ? c->st : nullptr;
}

// row sums of x the EXACT products with this format read: 0 none, 1 per
// 16-element sub-block (Q2_K), 2 per 32-element sub-block (Q4_K, Q5_K)
int wants_xsum(int qtype) {
    if (qtype == MYNAH_ASR_HIP_Q2_K) return 1;
    return qtype == MYNAH_ASR_HIP_Q4_K || qtype == MYNAH_ASR_HIP_Q5_K ? 2 : 0;
}

mynah_asr_hip_weight *upload(const mynah_asr_hip_wdesc *w) {
    HostLayout L;
    if (mh_repack(w, &L) != 0) {
        fail("unsupported weight format or shape");
        return nullptr;
    }
    size_t off[4];
    const size_t bytes = mh_layout_bytes(L, off);
    void *mem = nullptr;
    if (hipMalloc(&mem, bytes) != hipSuccess) {
        fail("hipMalloc for a weight failed");
        return nullptr;
    }
    uint8_t *b = (uint8_t *)mem;
    hipError_t e = hipSuccess;
    if (!L.p0.empty()) e = hipMemcpy(b + off[0], L.p0.data(), L.p0.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && !L.p1.empty()) e = hipMemcpy(b + off[1], L.p1.data(), L.p1.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && !L.h.empty()) e = hipMemcpy(b + off[2], L.h.data(), L.h.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && !L.h2.empty())
        e = hipMemcpy(b + off[3], L.h2.data(), L.h2.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(mem);
        fail("weight upload failed", hipGetErrorString(e));
        return nullptr;
    }
    auto *W = new mynah_asr_hip_weight;
    W->qtype = w->qtype;
    W->mem = mem;
    W->bytes = bytes;
    W->dw.p0 = b + off[0];
    W->dw.p1 = b + off[1];
    W->dw.h = b + off[2];
    W->dw.h2 = (const float *)(b + off[3]);
    W->dw.n = w->n;
    W->dw.k = w->k;
    W->dw.Np = L.Np;
    W->dw.Kp = L.Kp;
    return W;
}

// resident copy for a host weight (uploaded on first use)
const mynah_asr_hip_weight *resident(const mynah_asr_hip_wdesc *w) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto &e : g_cache)
        if (e.key == w->data && e.qtype == w->qtype && e.n == w->n && e.k == w->k) return e.w;
    mynah_asr_hip_weight *W = upload(w);
    if (!W) return nullptr;
    g_cache.push_back({w->data, w->qtype, w->n, w->k, W});
    return W;
}

// The numerics of the product being run. The process mode (set_numerics)
// applies as it is, except MYNAH_ASR_HIP_QMAT, which follows the reference's
// qmat.c dispatch per product (src/qmat.c:508-552, 598-650): INT8 / INT4
// weights with K <= 8192 (QMAT_K_MAX, :181) take the int8-activation path
// for T <= 16 (QMAT_SMALL_T, :180) and, with MYNAH_ASR_QGEMM=1 in the
// environment (:607-611; read at each call here, once per process there),
// for every T; every other product runs EXACT. Entry points set the effective mode for the call (NumScope).
thread_local int t_num = -1;
int num_now() { return t_num >= 0 ? t_num : mynah_asr_hip_numerics(); }
int eff_num(int qtype, int k, int T) {
    const int m = mynah_asr_hip_numerics();
    if (m != MYNAH_ASR_HIP_QMAT) return m;
    if ((qtype != MYNAH_ASR_HIP_INT8 && qtype != MYNAH_ASR_HIP_INT4) || k > 8192) return MYNAH_ASR_HIP_EXACT;
    if (T <= 16) return MYNAH_ASR_HIP_INT8ACT;
    const char *e = getenv("MYNAH_ASR_QGEMM");
    return (e && e[0] == '1') ? MYNAH_ASR_HIP_INT8ACT : MYNAH_ASR_HIP_EXACT;
}
struct NumScope {
    int prev;
    explicit NumScope(int m) : prev(t_num) { t_num = m; }
    ~NumScope() { t_num = prev; }
};

int check_numerics_supported(int qtype, int k, int T) {
    if (eff_num(qtype, k, T) == MYNAH_ASR_HIP_EXACT) return 0;
    if (mh_i8_supported(qtype)) return 0;
    return fail("INT8ACT numerics: f32 weights have no int8 form (the reference multiplies them in f32)");
}

// the prepared-input form a product of this format reads in the current mode
int prep_kind(int qtype) {
    return num_now() == MYNAH_ASR_HIP_INT8ACT ? mh_i8_kind(qtype) : 0;
}

// bytes of the three prepared-input buffers (xp, xs16, xpf) for one form
void prep_sizes(int kind, int Mpad, int Kp, size_t b[3]) {
    b[0] = (size_t)Mpad * Kp * (kind == MH_I8_QMAT ? 1 : (kind ? 2 : 4));
    b[1] = (size_t)Mpad * (kind == MH_I8_QMAT ? 1 : Kp / 16) * sizeof(float);
    b[2] = (size_t)Mpad * (Kp / 128) * sizeof(float);
}

// Launch the preparation of x for products of W's format and inner size into
// (xp, xs16, xpf), sized by prep_sizes:
//   EXACT:           xp = f16 (hi, lo) A fragments, xs16 = the mins operand of
//                    the affine formats, xpf = chunk fold factors
//   INT8ACT QMAT:    xp = int8 A fragments, xs16 = row scales sx (xpf holds
//                    each row's factor 127 / amax while the preparation runs)
//   INT8ACT ROW/SB:  xp = int8 values as f16 A fragments, xpf = their scales
//                    per chunk, xs16 = the mins operand of the affine formats
hipError_t launch_prep(int kind, const mynah_asr_hip_weight *W, const float *dx, int T, uint8_t *xp, float *xs16,
                       float *xpf, hipStream_t st) {
    const int Mpad = mh_mpad(T), Kp = W->dw.Kp, k = W->dw.k;
    if (kind == MH_I8_QMAT) return mh_launch_prep_i8(dx, T, k, Kp, Mpad, xp, xs16, xpf, st);   // (xpf: Mpad * Kp / 128 floats)
    if (kind) return mh_launch_prep_a1(kind, dx, T, k, Kp, Mpad, xp, xs16, xpf, wants_xsum(W->qtype), st);
    const int vec = (k % 8 == 0) && (((uintptr_t)dx & 15) == 0);
    return mh_launch_prep(dx, T, k, Kp, Mpad, xp, xs16, xpf, wants_xsum(W->qtype), vec, st);
}

// Prepare x for products with W in the current numerics mode into the
// calling thread's workspace P.
int prep_into(PrepBuf &P, const mynah_asr_hip_weight *W, const float *dx, int T, hipStream_t st) {
    const int Mpad = mh_mpad(T), Kp = W->dw.Kp;
    const int kind = prep_kind(W->qtype);
    if (P.src && P.src == dx && kind == 0 && !wants_xsum(W->qtype) && P.T == T && P.Kp == Kp && P.i8 == 0)
        return 0;
    P.src = nullptr;
    size_t b[3];
    prep_sizes(kind, Mpad, Kp, b);
    uint8_t *xp = (uint8_t *)P.xp.get(b[0]);
    float *xs16 = (float *)P.xs16.get(b[1]);
    float *xpf = (float *)P.xpf.get(b[2]);
    if (!xp || !xs16 || !xpf) return fail("workspace allocation failed");
    hipError_t e = launch_prep(kind, W, dx, T, xp, xs16, xpf, st);
    if (e != hipSuccess) return fail("prep launch failed", hipGetErrorString(e));
    P.T = T;
    P.Kp = Kp;
    P.xsum = kind == MH_I8_QMAT ? 0 : wants_xsum(W->qtype);
    P.i8 = kind;
    return 0;
}
int prep_for(Ctx *c, const mynah_asr_hip_weight *W, const float *dx, int T, hipStream_t st) {
    return prep_into(c->pa, W, dx, T, st);
}

bool fits(const PrepBuf &P, const mynah_asr_hip_weight *W, int T) {
    const int kind = prep_kind(W->qtype);
    return P.T == T && P.Kp == W->dw.Kp && P.i8 == kind &&
           (kind == MH_I8_QMAT || !wants_xsum(W->qtype) || P.xsum == wants_xsum(W->qtype));
}
bool prep_fits(const Ctx *c, const mynah_asr_hip_weight *W, int T) { return fits(c->pa, W, T); }

// the product on a prepared input
// act: 0 none, 1 SiLU; 2 and 3 (internal, the EXACT GEMM path only) add the
// product, or half of it, into dy (the encoder layer's residual adds)
int run_from(Ctx *c, const PrepBuf &P, const mynah_asr_hip_weight *W, float *dy, int T, int act, hipStream_t st) {
    hipError_t e;
    if (act >= 2 && P.i8 != 0) return fail("internal: a residual epilogue outside the EXACT GEMM path");
    if (P.i8 == MH_I8_QMAT) {
        e = mh_launch_gemm_i8(W->qtype, W->dw, (const uint8_t *)P.xp.p, (const float *)P.xs16.p, dy, T, act, st);
    } else {
        // few tiles: K split over workgroups, through the calling thread's workspace
        const size_t n = mh_gemm_ws_floats(W->dw, T);
        float *ws = n ? (float *)c->gk.get(n * sizeof(float)) : nullptr;
        e = mh_launch_gemm(W->qtype, W->dw, (const uint8_t *)P.xp.p, (const float *)P.xs16.p,
                           (const float *)P.xpf.p, dy, T, act, ws, st, P.i8 != 0);
    }
    if (e != hipSuccess) return fail("gemm launch failed", hipGetErrorString(e));
    return 0;
}
int run_prepped(Ctx *c, const mynah_asr_hip_weight *W, float *dy, int T, int act, hipStream_t st) {
    return run_from(c, c->pa, W, dy, T, act, st);
}

// the calling thread's split-K GEMV workspace for W (null: the one-launch GEMV)
float *gemv_ws(Ctx *c, const mynah_asr_hip_weight *W) {
    const size_t n = mh_gemv_ws_floats(W->dw);
    return n ? (float *)c->gs.get(n * sizeof(float)) : nullptr;
}

int gemm_dev(Ctx *c, const mynah_asr_hip_weight *W, const float *dx, float *dy, int T, int act,
             hipStream_t st) {
    if (num_now() == MYNAH_ASR_HIP_EXACT && mh_use_gemv(W->dw, T)) {
        if (act >= 2) return fail("internal: a residual epilogue outside the EXACT GEMM path");
        const int vec = (W->dw.k % 8 == 0) && (((uintptr_t)dx & 15) == 0);
        hipError_t e = mh_launch_gemv(W->qtype, W->dw, dx, T, vec, dy, act, gemv_ws(c, W), st);
        if (e != hipSuccess) return fail("gemv launch failed", hipGetErrorString(e));
        return 0;
    }
    if (prep_for(c, W, dx, T, st)) return -1;
    return run_prepped(c, W, dy, T, act, st);
}

// out = SiLU(x . W1^T) . W2^T on device buffers (dx may alias dy). In EXACT
// numerics on the GEMM path, when W2's chunks are W1's column tiles, the
// first product prepares the intermediate for the second in its epilogue
// (no f32 intermediate, no preparation pass); otherwise two products.
int ffn_dev(Ctx *c, const mynah_asr_hip_weight *W1, const mynah_asr_hip_weight *W2, const float *dx, float *dy,
            int T, hipStream_t st, int act2 = 0) {
    const int n1 = eff_num(W1->qtype, W1->dw.k, T), n2 = eff_num(W2->qtype, W2->dw.k, T);
    if (n1 != n2) {
        // (QMAT numerics: each product in its own mode, as qmat_ffn's two qmat_mul calls)
        float *dh = (float *)c->h.get((size_t)T * W1->dw.n * sizeof(float));
        if (!dh) return fail("device buffer allocation failed");
        {
            NumScope s1(n1);
            if (gemm_dev(c, W1, dx, dh, T, 1, st)) return -1;
        }
        NumScope s2(n2);
        return gemm_dev(c, W2, dh, dy, T, act2, st);
    }
    NumScope sc(n1);
    const bool fuse = num_now() == MYNAH_ASR_HIP_EXACT && !mh_use_gemv(W1->dw, T) &&
                      W2->dw.Kp == W1->dw.Np;
    if (fuse) {
        if (prep_into(c->pa, W1, dx, T, st)) return -1;
        PrepBuf &P = c->pb;
        const int Mpad = mh_mpad(T), Kp = W2->dw.Kp;
        const int xsum = wants_xsum(W2->qtype);
        uint8_t *xp = (uint8_t *)P.xp.get((size_t)Mpad * Kp * 4);
        float *xs16 = (float *)P.xs16.get((size_t)Mpad * (Kp / 16) * sizeof(float));
        float *xpf = (float *)P.xpf.get((size_t)Mpad * (Kp / 128) * sizeof(float));
        if (!xp || !xs16 || !xpf) return fail("workspace allocation failed");
        hipError_t e = mh_launch_gemm_prep_out(W1->qtype, W1->dw, (const uint8_t *)c->pa.xp.p,
                                               (const float *)c->pa.xs16.p, (const float *)c->pa.xpf.p, T, xp, xs16,
                                               xpf, Kp / 128, xsum, st);
        if (e != hipSuccess) return fail("gemm launch failed", hipGetErrorString(e));
        P.T = T;
        P.Kp = Kp;
        P.xsum = xsum;
        P.i8 = 0;
        return run_from(c, P, W2, dy, T, act2, st);
    }
    float *dh = (float *)c->h.get((size_t)T * W1->dw.n * sizeof(float));
    if (!dh) return fail("device buffer allocation failed");
    if (gemm_dev(c, W1, dx, dh, T, 1, st)) return -1;
    return gemm_dev(c, W2, dh, dy, T, act2, st);
}

// three products of one input: prepared once whenever it fits them all
int qkv_dev(Ctx *c, const mynah_asr_hip_weight *const W[3], const float *dx, float *const dy[3], int T,
            hipStream_t st) {
    const int nq = eff_num(W[0]->qtype, W[0]->dw.k, T);
    if (eff_num(W[1]->qtype, W[1]->dw.k, T) != nq || eff_num(W[2]->qtype, W[2]->dw.k, T) != nq) {
        // (QMAT numerics: each product in its own mode, as qmat_qkv's three qmat_mul calls)
        for (int i = 0; i < 3; i++) {
            NumScope si(eff_num(W[i]->qtype, W[i]->dw.k, T));
            if (gemm_dev(c, W[i], dx, dy[i], T, 0, st)) return -1;
        }
        return 0;
    }
    NumScope sc(nq);
    // GEMMs of one format and shape: one preparation, one launch
    const bool exact = num_now() == MYNAH_ASR_HIP_EXACT;
    if ((!exact || !mh_use_gemv(W[0]->dw, T)) &&
        W[1]->qtype == W[0]->qtype && W[2]->qtype == W[0]->qtype && W[1]->dw.n == W[0]->dw.n &&
        W[2]->dw.n == W[0]->dw.n && W[1]->dw.k == W[0]->dw.k && W[2]->dw.k == W[0]->dw.k &&
        W[1]->dw.Np == W[0]->dw.Np && W[2]->dw.Np == W[0]->dw.Np) {
        if (prep_for(c, W[0], dx, T, st)) return -1;
        if (c->pa.i8 == MH_I8_QMAT) {
            for (int i = 0; i < 3; i++)
                if (run_prepped(c, W[i], dy[i], T, 0, st)) return -1;
            return 0;
        }
        GemmJobs J{};
        for (int i = 0; i < 3; i++) {
            J.W[i] = W[i]->dw;
            J.y[i] = dy[i];
        }
        J.n = 3;
        const PrepBuf &P = c->pa;
        const size_t n = mh_gemm_ws_floats(W[0]->dw, T, 3);
        float *ws = n ? (float *)c->gk.get(n * sizeof(float)) : nullptr;
        hipError_t e = mh_launch_gemm_jobs(W[0]->qtype, J, (const uint8_t *)P.xp.p, (const float *)P.xs16.p,
                                           (const float *)P.xpf.p, T, ws, st, P.i8 != 0);
        if (e != hipSuccess) return fail("gemm launch failed", hipGetErrorString(e));
        return 0;
    }
    bool prepared = false;
    for (int i = 0; i < 3; i++) {
        if (num_now() == MYNAH_ASR_HIP_EXACT && mh_use_gemv(W[i]->dw, T)) {
            if (gemm_dev(c, W[i], dx, dy[i], T, 0, st)) return -1;
            continue;
        }
        if (!prepared || !prep_fits(c, W[i], T))
            if (prep_for(c, W[i], dx, T, st)) return -1;
        prepared = true;
        if (run_prepped(c, W[i], dy[i], T, 0, st)) return -1;
    }
    return 0;
}

int h2d(Ctx *c, DBuf &b, const float *x, size_t n, float **d) {
    *d = (float *)b.get(n * sizeof(float));
    if (!*d) return fail("device buffer allocation failed");
    if (hipMemcpyAsync(*d, x, n * sizeof(float), hipMemcpyHostToDevice, c->st) != hipSuccess)
        return fail("H2D copy failed");
    return 0;
}

int d2h_sync(Ctx *c, float *out, const float *d, size_t n) {
    if (hipMemcpyAsync(out, d, n * sizeof(float), hipMemcpyDeviceToHost, c->st) != hipSuccess)
        return fail("D2H copy failed");
    hipError_t e = hipStreamSynchronize(c->st);
    if (e != hipSuccess) return fail("stream sync failed", hipGetErrorString(e));
    return 0;
}

// ---------------------------------------------------------------------------
// AED decoder (decoder_aed.c:139-232) on the device.

struct AedBufs {
    float *encp, *ckv, *skv, *x, *xn, *q, *att, *kn, *vn, *ff, *logits, *opart, *ml;
    int *st, *prompt;
    int nsplit;
};

bool gemv_ok(const mynah_asr_hip_weight *W, int n, int k) {
    return W && W->dw.n == n && W->dw.k == k && mh_use_gemv(W->dw, 1);
}

int aed_check(const mynah_asr_hip_aed *a, int T) {
    if (!a || !a->layers || a->n_layers < 0 || a->d <= 0 || a->n_heads <= 0 || a->d % a->n_heads || T <= 0 ||
        a->vocab <= 0 || a->ffn <= 0 || a->max_seq <= 0)
        return fail("bad argument");
    const int d = a->d, dk = d / a->n_heads;
    if (dk != 64 && dk != 128) return fail("decoder head size must be 64 or 128");
    if (d > 4096 || d % 4) return fail("decoder width must be a multiple of 4, at most 4096");
    if (mynah_asr_hip_numerics() == MYNAH_ASR_HIP_INT8ACT) return fail("the device decoder runs EXACT numerics only");
    if (!a->emb || !a->pos || !a->embln_w || !a->embln_b || !a->fin_w || !a->fin_b || !a->head_b)
        return fail("bad argument: a decoder tensor is NULL");
    if (!gemv_ok(a->head, a->vocab, d)) return fail("head weight shape or GEMV limits");
    if (a->proj && a->proj->dw.n != d) return fail("proj weight shape");
    for (int li = 0; li < a->n_layers; li++) {
        const mynah_asr_hip_aed_layer *L = &a->layers[li];
        const mynah_asr_hip_weight *sq[8] = {L->sq, L->sk, L->sv, L->so, L->cq, L->ck, L->cv, L->co};
        for (int i = 0; i < 8; i++)
            if (!sq[i] || sq[i]->dw.n != d || sq[i]->dw.k != d || (i != 5 && i != 6 && !mh_use_gemv(sq[i]->dw, 1)))
                return fail("attention weight shape or GEMV limits");
        if (!gemv_ok(L->ff1, a->ffn, d) || !gemv_ok(L->ff2, d, a->ffn)) return fail("FFN weight shape or GEMV limits");
        const float *v[16] = {L->ln_self_w, L->ln_self_b, L->sq_b, L->sk_b, L->sv_b, L->so_b, L->ln_cross_w,
                              L->ln_cross_b, L->cq_b, L->ck_b, L->cv_b, L->co_b, L->ln_ffn_w, L->ln_ffn_b,
                              L->ff1_b, L->ff2_b};
        for (int i = 0; i < 16; i++)
            if (!v[i]) return fail("bad argument: a decoder layer tensor is NULL");
    }
    // QMAT numerics: the decoder's one-row products of INT8/INT4 weights would
    // take the reference's int8 path, which the device decoder does not run
    if (mynah_asr_hip_numerics() == MYNAH_ASR_HIP_QMAT) {
        auto int8_path = [](const mynah_asr_hip_weight *W) {
            return W && eff_num(W->qtype, W->dw.k, 1) != MYNAH_ASR_HIP_EXACT;
        };
        bool any = int8_path(a->head) || int8_path(a->proj);
        for (int li = 0; li < a->n_layers && !any; li++) {
            const mynah_asr_hip_aed_layer *L = &a->layers[li];
            const mynah_asr_hip_weight *ws[10] = {L->sq, L->sk, L->sv, L->so, L->cq, L->ck, L->cv, L->co, L->ff1, L->ff2};
            for (int i = 0; i < 10; i++) any = any || int8_path(ws[i]);
        }
        if (any)
            return fail("QMAT numerics: INT8/INT4 decoder weights take the reference's int8 path, which the device "
                        "decoder does not run");
    }
    return 0;
}

int gemv_epi(const mynah_asr_hip_weight *W, const float *x, float *y, int act, const float *bias, const float *res,
             hipStream_t st) {
    const int vec = (W->dw.k % 8 == 0) && (((uintptr_t)x & 15) == 0);
    Ctx *c = ctx();
    hipError_t e = mh_launch_gemv_epi(W->qtype, W->dw, x, 1, vec, y, GEpi{act, bias, res},
                                      c ? gemv_ws(c, W) : nullptr, st);
    return e == hipSuccess ? 0 : fail("gemv launch failed", hipGetErrorString(e));
}

#define AED_TRY(expr)                                                             \
    do {                                                                          \
        hipError_t e_ = (expr);                                                   \
        if (e_ != hipSuccess) return fail("decoder launch failed", hipGetErrorString(e_)); \
    } while (0)

// One decoding position: every launch reads p and the token from b.st. The
// layer norms and the merge of the attention splits run as the prologue of
// the GEMV that consumes them; q, k and v are one launch.
int aed_gemv(const mynah_asr_hip_weight *const *Ws, float *const *ys, const GEpi *eps, int n, const GPro &pro,
             const float *x, hipStream_t st) {
    GJobs J{};
    for (int i = 0; i < 3; i++) {
        const int j = i < n ? i : 0;
        J.W[i] = Ws[j]->dw;
        J.y[i] = ys[j];
        J.ep[i] = eps[j];
    }
    J.n = n;
    const int vec = x && (Ws[0]->dw.k % 8 == 0) && (((uintptr_t)x & 15) == 0);
    Ctx *c = ctx();
    // one product of a plain input may split K (ff2); the workspace is sized by
    // the eager first step, before the step is captured
    float *ws = n == 1 && pro.kind == GPRO_NONE && c ? gemv_ws(c, Ws[0]) : nullptr;
    hipError_t e = ws ? mh_launch_gemv_epi(Ws[0]->qtype, J.W[0], x, 1, vec, J.y[0], J.ep[0], ws, st)
                      : mh_launch_gemv_jobs(Ws[0]->qtype, J, x, 1, vec, pro, st);
    return e == hipSuccess ? 0 : fail("gemv launch failed", hipGetErrorString(e));
}

GPro pro_ln(const float *x, const float *w, const float *b) {
    GPro p{};
    p.kind = GPRO_LN;
    p.x = x, p.w = w, p.b = b;
    return p;
}

GPro pro_comb(const AedBufs &b, int n_fixed, int H) {
    GPro p{};
    p.kind = GPRO_COMB;
    p.opart = b.opart, p.ml = b.ml, p.st = b.st, p.n_fixed = n_fixed, p.nsplit = b.nsplit, p.H = H;
    return p;
}

int aed_one(const mynah_asr_hip_weight *W, float *y, GEpi ep, const GPro &pro, hipStream_t st) {
    return aed_gemv(&W, &y, &ep, 1, pro, nullptr, st);
}

// One position. Its input row x is formed by the previous step's argmax
// kernel, so only the first step (first = true) embeds its own.
int aed_step(const mynah_asr_hip_aed *a, const AedBufs &b, int T, int max_len, int n_prompt, float *logits_out,
             bool first, hipStream_t st) {
    const int d = a->d, H = a->n_heads;
    const size_t td = (size_t)T * d, md = (size_t)max_len * d;
    if (first) AED_TRY(mh_launch_embed_ln(a->emb, a->pos, b.prompt, n_prompt, b.st, a->embln_w, a->embln_b, b.x, d, st));
    for (int li = 0; li < a->n_layers; li++) {
        const mynah_asr_hip_aed_layer *L = &a->layers[li];
        float *SK = b.skv + 2 * (size_t)li * md, *SV = SK + md;
        float *CK = b.ckv + 2 * (size_t)li * td, *CV = CK + td;
        // causal self attention, its k and v rows appended to the cache at p
        const mynah_asr_hip_weight *qkv[3] = {L->sq, L->sk, L->sv};
        float *const qkv_y[3] = {b.q, b.kn, b.vn};
        const GEpi qkv_ep[3] = {{0, L->sq_b, nullptr}, {0, L->sk_b, nullptr}, {0, L->sv_b, nullptr}};
        const bool same = L->sk->qtype == L->sq->qtype && L->sv->qtype == L->sq->qtype;
        const GPro ln_self = pro_ln(b.x, L->ln_self_w, L->ln_self_b);
        if (same) {
            if (aed_gemv(qkv, qkv_y, qkv_ep, 3, ln_self, nullptr, st)) return -1;
        } else {
            for (int i = 0; i < 3; i++)
                if (aed_one(qkv[i], qkv_y[i], qkv_ep[i], ln_self, st)) return -1;
        }
        AED_TRY(mh_launch_attend1(b.q, SK, SV, b.kn, b.vn, b.st, 0, d, H, b.opart, b.ml, b.nsplit, nullptr, st));
        if (aed_one(L->so, b.x, GEpi{0, L->so_b, b.x}, pro_comb(b, 0, H), st)) return -1;
        // cross attention over the projected encoder output
        if (aed_one(L->cq, b.q, GEpi{0, L->cq_b, nullptr}, pro_ln(b.x, L->ln_cross_w, L->ln_cross_b), st)) return -1;
        AED_TRY(mh_launch_attend1(b.q, CK, CV, nullptr, nullptr, b.st, T, d, H, b.opart, b.ml, b.nsplit, nullptr, st));
        if (aed_one(L->co, b.x, GEpi{0, L->co_b, b.x}, pro_comb(b, T, H), st)) return -1;
        // ReLU FFN
        const GEpi ff2_ep{0, L->ff2_b, b.x};
        if (aed_one(L->ff1, b.ff, GEpi{2, L->ff1_b, nullptr}, pro_ln(b.x, L->ln_ffn_w, L->ln_ffn_b), st) ||
            aed_gemv(&L->ff2, &b.x, &ff2_ep, 1, GPro{}, b.ff, st))
            return -1;
    }
    if (aed_one(a->head, b.logits, GEpi{0, a->head_b, nullptr}, pro_ln(b.x, a->fin_w, a->fin_b), st)) return -1;
    const MhEmbNext en{a->emb, a->pos, b.prompt, n_prompt, max_len, a->embln_w, a->embln_b, b.x, d};
    AED_TRY(mh_launch_argmax(b.logits, a->vocab, b.st, logits_out, &en, st));
    return 0;
}

// Shared body of decode (greedy, tokens != NULL) and forced (logits_out != NULL).
int aed_run(Ctx *c, const mynah_asr_hip_aed *a, const float *enc, int T, const int *prompt, int n_prompt,
            int max_len, int eos, int *tokens, int cap, float *logits_out, hipStream_t st) {
    const int d = a->d, nl = a->n_layers;
    const size_t td = (size_t)T * d, md = (size_t)max_len * d;
    AedBufs b;
    b.nsplit = mh_att_splits(T > max_len ? T : max_len);
    auto al = [](size_t n) { return (n + 63) / 64 * 64; };   // floats, 256-byte pieces
    const size_t nenc = a->proj ? al(td) : 0, nckv = al(2 * (size_t)nl * td), nskv = al(2 * (size_t)nl * md);
    const size_t nvec = 6 * al(d) + al(a->ffn) + al(a->vocab) + al((size_t)b.nsplit * d) +
                        al((size_t)b.nsplit * a->n_heads * 2) + al(2 + (size_t)n_prompt);
    float *base = (float *)c->aed.get((nenc + nckv + nskv + nvec) * sizeof(float));
    if (!base) return fail("device buffer allocation failed");
    float *cur = base;
    auto take = [&](size_t n) { float *r = cur; cur += al(n); return r; };
    b.encp = a->proj ? take(td) : (float *)enc;
    b.ckv = take(2 * (size_t)nl * td);
    b.skv = take(2 * (size_t)nl * md);
    b.x = take(d), b.xn = take(d), b.q = take(d), b.att = take(d), b.kn = take(d), b.vn = take(d);
    b.ff = take(a->ffn), b.logits = take(a->vocab);
    b.opart = take((size_t)b.nsplit * d), b.ml = take((size_t)b.nsplit * a->n_heads * 2);
    b.st = (int *)take(2 + (size_t)n_prompt);
    b.prompt = b.st + 2;
    if (!c->pin && hipHostMalloc((void **)&c->pin, 4 * sizeof(int)) != hipSuccess) {
        c->pin = nullptr;
        return fail("pinned host allocation failed");
    }
    for (int i = 0; i < 2; i++)
        if (!c->pev[i] && hipEventCreateWithFlags(&c->pev[i], hipEventDisableTiming) != hipSuccess) {
            c->pev[i] = nullptr;
            return fail("event creation failed");
        }

    // encoder projection and the per-layer cross K/V (decoder_aed.c:150-175)
    if (a->proj) {
        if (gemm_dev(c, a->proj, enc, b.encp, T, 0, st)) return -1;
        if (a->proj_b) AED_TRY(mh_launch_bias_rows(b.encp, a->proj_b, T, d, st));
    }
    for (int li = 0; li < nl; li++) {
        const mynah_asr_hip_aed_layer *L = &a->layers[li];
        float *CK = b.ckv + 2 * (size_t)li * td, *CV = CK + td;
        if (gemm_dev(c, L->ck, b.encp, CK, T, 0, st) || gemm_dev(c, L->cv, b.encp, CV, T, 0, st)) return -1;
        AED_TRY(mh_launch_bias_rows(CK, L->ck_b, T, d, st));
        AED_TRY(mh_launch_bias_rows(CV, L->cv_b, T, d, st));
    }
    if (hipMemcpyAsync(b.prompt, prompt, n_prompt * sizeof(int), hipMemcpyHostToDevice, st) != hipSuccess)
        return fail("H2D copy failed");
    AED_TRY(mh_launch_set_state(b.st, 0, prompt[0], st));

    // position 0 eagerly, then the step captured once and replayed. Greedy
    // decoding reads each position's token back while the next position runs:
    // the step's argmax already formed the next input row on the device, so
    // position p+1 is enqueued before the host sees p's token (a position
    // enqueued past an EOS or the cap only extends the internal cache by one
    // row, within max_len, and its token is never read).
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int n_out = 0, rc = 0, pending = -1;
    bool stop = false;
    auto resolve = [&](int q) {   // position q's token: the loop's EOS / cap test (decoder_aed.c:215-221)
        if (hipEventSynchronize(c->pev[q & 1]) != hipSuccess) {
            rc = fail("token read-back failed");
            return true;
        }
        const int best = c->pin[2 * (q & 1) + 1];
        if (best == eos || n_out >= cap) return true;
        tokens[n_out++] = best;
        return false;
    };
    for (int p = 0; p < max_len && !stop; p++) {
        if (p == 0) {
            if (aed_step(a, b, T, max_len, n_prompt, logits_out, true, st)) return -1;
        } else {
            if (!exec) {
                if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess)
                    return fail("stream capture failed");
                const int r = aed_step(a, b, T, max_len, n_prompt, logits_out, false, st);
                hipError_t e = hipStreamEndCapture(st, &graph);
                if (r || e != hipSuccess) {
                    if (graph) (void)hipGraphDestroy(graph);
                    return r ? -1 : fail("stream capture failed", hipGetErrorString(e));
                }
                if (hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
                    (void)hipGraphDestroy(graph);
                    return fail("graph instantiation failed");
                }
            }
            if (hipGraphLaunch(exec, st) != hipSuccess) { rc = fail("graph launch failed"); break; }
        }
        if (!tokens || p + 1 < n_prompt) continue;   // prompt positions: no sampling
        if (hipMemcpyAsync(c->pin + 2 * (p & 1), b.st, 2 * sizeof(int), hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipEventRecord(c->pev[p & 1], st) != hipSuccess) {
            rc = fail("token read-back failed");
            break;
        }
        if (pending >= 0) stop = resolve(pending);
        pending = p;
    }
    if (pending >= 0 && !stop && rc == 0) resolve(pending);
    if (hipStreamSynchronize(st) != hipSuccess && rc == 0) rc = fail("stream sync failed");
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    return rc ? -1 : n_out;
}

// ---------------------------------------------------------------------------
// The allocation-free product (mynah_asr_hip_qgemm_noalloc_dev). Its prepared
// input lives in `scratch`, a file-scope device array: every device the
// library runs on holds one copy, at its own address, until the process ends.
// In host code `scratch` names a host-side stand-in, never the device memory:
// the device address comes from hipGetSymbolAddress, once per device, and is
// the only form host code passes to kernels.
constexpr size_t kNoAllocBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

constexpr int kMaxDevices = 64;
void *g_scratch_dev[kMaxDevices];   // device address of `scratch` per device (null: not yet looked up)

// the scratch address on the current device (null + t_err on failure)
uint8_t *noalloc_scratch() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        fail("no current device for the scratch buffer");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch_dev[dev]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            fail("hipGetSymbolAddress(scratch) failed", hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_dev[dev] = ptr;
    }
    return (uint8_t *)g_scratch_dev[dev];
}

inline size_t al256(size_t b) { return (b + 255) / 256 * 256; }

// Bytes of scratch a product of W over T rows needs in the current numerics
// mode (0: the GEMV path, which uses none); what prep_into would allocate.
size_t noalloc_need(const mynah_asr_hip_weight *W, int T, size_t *o_xs16, size_t *o_xpf) {
    const int kind = prep_kind(W->qtype);
    if (!kind && mh_use_gemv(W->dw, T)) return 0;
    size_t b[3];
    prep_sizes(kind, mh_mpad(T), W->dw.Kp, b);
    const size_t xp = al256(b[0]), xs16 = al256(b[1]), xpf = al256(b[2]);
    *o_xs16 = xp;
    *o_xpf = xp + xs16;
    return xp + xs16 + xpf;
}

// qgemm_dev's product with its prepared input in `scratch` and K unsplit (the
// split-K launches need a workspace of their own): the same kernels on the
// same data, so the same bits.
int gemm_noalloc(const mynah_asr_hip_weight *W, const float *dx, float *dy, int T, int act, hipStream_t st) {
    size_t o_xs16 = 0, o_xpf = 0;
    const size_t need = noalloc_need(W, T, &o_xs16, &o_xpf);
    const int kind = prep_kind(W->qtype);
    hipError_t e;
    if (need == 0) {
        const int vec = (W->dw.k % 8 == 0) && (((uintptr_t)dx & 15) == 0);
        e = mh_launch_gemv(W->qtype, W->dw, dx, T, vec, dy, act, nullptr, st);
        return e == hipSuccess ? 0 : fail("gemv launch failed", hipGetErrorString(e));
    }
    if (need > kNoAllocBytes) return fail("input too large for the 32 MiB no-allocation scratch");
    uint8_t *base = noalloc_scratch();
    if (!base) return -1;
    uint8_t *xp = base;
    float *xs16 = (float *)(base + o_xs16), *xpf = (float *)(base + o_xpf);
    e = launch_prep(kind, W, dx, T, xp, xs16, xpf, st);
    if (e == hipSuccess) {
        if (kind == MH_I8_QMAT) e = mh_launch_gemm_i8(W->qtype, W->dw, xp, xs16, dy, T, act, st);
        else e = mh_launch_gemm(W->qtype, W->dw, xp, xs16, xpf, dy, T, act, nullptr, st, kind != 0);
    }
    return e == hipSuccess ? 0 : fail("launch failed", hipGetErrorString(e));
}

// ---------------------------------------------------------------- encoder layer
// The steps of src/encoder.c:485-521 (encoder_layer; batched, :901-946) on
// device buffers: every product through the same entry points the callers
// use one by one (each in the current numerics mode), the rest through the
// encoder.hip kernels.
int enc_check(const mynah_asr_hip_enc_layer *L, int T, int nseq, int d, int H, int conv_k) {
    if (!L || T < 0 || nseq < 0 || d <= 0 || H <= 0 || d % H != 0 || conv_k <= 0) return fail("bad argument");
    if (!mh_enc_d_supported(d)) return fail("encoder layer: d must be 256 times 1 to 8, 12 or 16");
    if (!mh_attn_supported(d / H)) return fail("head size must be 64 or 128");
    if ((size_t)2 * T * d >= 0x7fffffffu) return fail("attention: 2 T d must stay below 2^31");
    const mynah_asr_hip_weight *sq[] = {L->q_w, L->k_w, L->v_w, L->o_w, L->relk_w, L->pw2_w};
    for (const mynah_asr_hip_weight *w : sq)
        if (!w || w->dw.n != d || w->dw.k != d) return fail("encoder layer: q/k/v/o/relk/pw2 must be [d, d]");
    if (!L->pw1_w || L->pw1_w->dw.n != 2 * d || L->pw1_w->dw.k != d) return fail("encoder layer: pw1 must be [2d, d]");
    const mynah_asr_hip_weight *ff[] = {L->ff1_w1, L->ff1_w2, L->ff2_w1, L->ff2_w2};
    for (const mynah_asr_hip_weight *w : ff)
        if (!w) return fail("encoder layer: missing FFN weight");
    if (L->ff1_w1->dw.k != d || L->ff1_w2->dw.n != d || L->ff1_w2->dw.k != L->ff1_w1->dw.n ||
        L->ff2_w1->dw.k != d || L->ff2_w2->dw.n != d || L->ff2_w2->dw.k != L->ff2_w1->dw.n)
        return fail("encoder layer: FFN weights must be [f, d] and [d, f]");
    const float *req[] = {L->ln_ff1_w, L->ln_ff1_b, L->ln_att_w, L->ln_att_b, L->bias_u, L->bias_v,
                          L->ln_conv_w, L->ln_conv_b, L->dw_w, L->ln_ff2_w, L->ln_ff2_b, L->ln_out_w, L->ln_out_b};
    for (const float *p : req)
        if (!p) return fail("encoder layer: missing tensor");
    if (L->cnorm_scale ? !L->cnorm_shift : (!L->cnorm_w || !L->cnorm_b))
        return fail("encoder layer: the conv norm needs cnorm_scale and cnorm_shift, or cnorm_w and cnorm_b");
    return 0;
}

int bias_add(float *y, const float *b, size_t rows, int n, hipStream_t st) {
    if (!b) return 0;
    hipError_t e = mh_launch_bias_rows(y, b, rows, n, st);
    return e == hipSuccess ? 0 : fail("bias launch failed", hipGetErrorString(e));
}

// half_ffn (encoder.c:464-483) on xn: the fused FFN when both biases are
// absent, else product, bias, SiLU, product, bias
int enc_half_ffn(Ctx *c, const mynah_asr_hip_weight *w1, const mynah_asr_hip_weight *w2, const float *b1,
                 const float *b2, const float *xn, float *out, float *h, int M, hipStream_t st, int act2 = 0) {
    if (!b1 && !b2) return ffn_dev(c, w1, w2, xn, out, M, st, act2);
    const int f = w1->dw.n;
    {
        NumScope s1(eff_num(w1->qtype, w1->dw.k, M));
        if (gemm_dev(c, w1, xn, h, M, 0, st)) return -1;
    }
    if (bias_add(h, b1, M, f, st)) return -1;
    hipError_t e = mh_launch_silu(h, (size_t)M * f, st);
    if (e != hipSuccess) return fail("silu launch failed", hipGetErrorString(e));
    {
        NumScope s2(eff_num(w2->qtype, w2->dw.k, M));
        if (gemm_dev(c, w2, h, out, M, 0, st)) return -1;
    }
    return bias_add(out, b2, M, w2->dw.n, st);
}

// Whether the products W[0..n) of one layer-norm output xn all read it as
// the EXACT GEMM path's prepared input (no GEMV, no row sums, K = Kp = d):
// then the layer norm writes that input directly.
// The encoder layer's fused hand-offs (prepared inputs written by their
// producers, residual adds in the products' epilogues) are on unless
// MYNAH_ASR_HIP_LN_PREP=0 (f32 rows and separate passes: the same bits).
bool enc_fused() {
    const char *env = getenv("MYNAH_ASR_HIP_LN_PREP");
    return !(env && env[0] == '0');
}

bool ln_preps(const mynah_asr_hip_weight *const *W, int n, int M, int d) {
    if (!enc_fused() || !mh_add_ln_prep_supported(d)) return false;
    for (int i = 0; i < n; i++)
        if (eff_num(W[i]->qtype, W[i]->dw.k, M) != MYNAH_ASR_HIP_EXACT || mh_use_gemv(W[i]->dw, M) ||
            wants_xsum(W[i]->qtype) || W[i]->dw.k != d || W[i]->dw.Kp != d)
            return false;
    return true;
}

// xn = LN(x += alpha res) for the products W[0..n): as their prepared input
// (c->pa, tagged xn; xn itself is then not written) when ln_preps allows,
// else as f32 rows
int enc_add_ln(Ctx *c, float *x, const float *res, float alpha, const float *w, const float *b, float *xn, int M,
               int d, const mynah_asr_hip_weight *const *W, int n, hipStream_t st) {
    hipError_t e;
    c->pa.src = nullptr;
    if (ln_preps(W, n, M, d)) {
        const int Mpad = mh_mpad(M);
        size_t bs[3];
        prep_sizes(0, Mpad, d, bs);
        uint8_t *xp = (uint8_t *)c->pa.xp.get(bs[0]);
        float *xs16 = (float *)c->pa.xs16.get(bs[1]);
        float *xpf = (float *)c->pa.xpf.get(bs[2]);
        if (!xp || !xs16 || !xpf) return fail("workspace allocation failed");
        e = mh_launch_add_ln_prep(x, res, alpha, w, b, M, d, xp, xpf, st);
        if (e != hipSuccess) return fail("encoder layer launch failed", hipGetErrorString(e));
        c->pa.T = M;
        c->pa.Kp = d;
        c->pa.xsum = 0;
        c->pa.i8 = 0;
        c->pa.src = xn;
        return 0;
    }
    e = mh_launch_add_ln(x, res, alpha, w, b, xn, M, d, st);
    return e == hipSuccess ? 0 : fail("encoder layer launch failed", hipGetErrorString(e));
}

int encoder_layer_dev(Ctx *c, const mynah_asr_hip_enc_layer *L, float *x, int T, int nseq, const float *pe, int d,
                      int H, int conv_k, int causal, int left, int right, hipStream_t st) {
    const int M = T * nseq, P = 2 * T - 1;
    // the prepared-input tag never outlives this call (an error return included)
    struct TagClear {
        PrepBuf &pa;
        ~TagClear() { pa.src = nullptr; }
    } tag_clear{c->pa};
    const int f = L->ff1_w1->dw.n > L->ff2_w1->dw.n ? L->ff1_w1->dw.n : L->ff2_w1->dw.n;
    const bool biased_ffn = L->ff1_b1 || L->ff1_b2 || L->ff2_b1 || L->ff2_b2;
    const size_t md = (size_t)M * d;
    // xn, tmp, q, k, v, ctx [M, d]; h [M, 2d] (pw1, GLU); rk [P, d]; the FFN
    // intermediate [M, f] only with FFN biases
    const size_t need = 6 * md + 2 * md + (size_t)P * d + (biased_ffn ? (size_t)M * f : 0);
    float *base = (float *)c->enc.get(need * sizeof(float));
    if (!base) return fail("device buffer allocation failed");
    float *xn = base, *tmp = xn + md, *q = tmp + md, *k = q + md, *v = k + md, *ctx = v + md, *h = ctx + md,
          *rk = h + 2 * md, *hf = rk + (size_t)P * d;
    hipError_t e;
#define ENC_TRY(expr)                                                                   \
    do {                                                                                \
        e = (expr);                                                                     \
        if (e != hipSuccess) return fail("encoder layer launch failed", hipGetErrorString(e)); \
    } while (0)
    // 1/2 FFN1 (:492-494)
    // (each layer norm whose output only feeds products tags the prepared
    // input with xn; the tag is cleared once those products have run)
    //
    // A product with no bias on the EXACT GEMM path adds its output into x
    // itself (x += tmp or x += tmp / 2, the same operations as the layer
    // norm's residual add), and the next layer norm reads x alone.
    auto res_ok = [&](const mynah_asr_hip_weight *W, bool biased) {
        return !biased && enc_fused() && eff_num(W->qtype, W->dw.k, M) == MYNAH_ASR_HIP_EXACT &&
               !mh_use_gemv(W->dw, M);
    };
    if (enc_add_ln(c, x, nullptr, 0.0f, L->ln_ff1_w, L->ln_ff1_b, xn, M, d, &L->ff1_w1, 1, st)) return -1;
    const bool r1 = res_ok(L->ff1_w2, L->ff1_b1 || L->ff1_b2);
    if (enc_half_ffn(c, L->ff1_w1, L->ff1_w2, L->ff1_b1, L->ff1_b2, xn, r1 ? x : tmp, hf, M, st, r1 ? 3 : 0))
        return -1;
    c->pa.src = nullptr;
    // x += 0.5 tmp; MHSA on LN(x) (:495-502)
    const mynah_asr_hip_weight *W3[3] = {L->q_w, L->k_w, L->v_w};
    if (enc_add_ln(c, x, r1 ? nullptr : tmp, r1 ? 0.0f : 0.5f, L->ln_att_w, L->ln_att_b, xn, M, d, W3, 3, st))
        return -1;
    float *const y3[3] = {q, k, v};
    if (qkv_dev(c, W3, xn, y3, M, st)) return -1;
    c->pa.src = nullptr;
    if (bias_add(q, L->q_b, M, d, st) || bias_add(k, L->k_b, M, d, st) || bias_add(v, L->v_b, M, d, st)) return -1;
    {
        // rk = pe . relk^T (:336): the segments share T, so one product serves
        // them all; in f32 arithmetic whatever the mode (relk_w stays f32 in
        // the reference, encoder.h:17)
        NumScope sp(MYNAH_ASR_HIP_EXACT);
        if (gemm_dev(c, L->relk_w, pe, rk, P, 0, st)) return -1;
    }
    {
        const size_t wb = mh_attn_ws_bytes(T, d, H, nseq, left);
        void *ws = wb ? c->attw.get(wb) : nullptr;
        if (wb && !ws) return fail("device buffer allocation failed");
        // the context as the output projection's prepared input (tagged ctx),
        // when that product takes the EXACT GEMM path
        uint8_t *xp = nullptr;
        float *xpf = nullptr;
        c->pa.src = nullptr;
        if (mh_attn_preps_out(d, H, left) && ln_preps(&L->o_w, 1, M, d)) {
            size_t bs[3];
            prep_sizes(0, mh_mpad(M), d, bs);
            xp = (uint8_t *)c->pa.xp.get(bs[0]);
            float *xs16 = (float *)c->pa.xs16.get(bs[1]);
            xpf = (float *)c->pa.xpf.get(bs[2]);
            if (!xp || !xs16 || !xpf) return fail("workspace allocation failed");
        }
        ENC_TRY(mh_launch_relpos_attn(q, k, v, rk, L->bias_u, L->bias_v, ctx, T, d, H, left, right, nseq, ws, xp,
                                      xpf, st));
        if (xp) {
            c->pa.T = M;
            c->pa.Kp = d;
            c->pa.xsum = 0;
            c->pa.i8 = 0;
            c->pa.src = ctx;
        }
    }
    const bool r2 = res_ok(L->o_w, L->o_b != nullptr);
    {
        NumScope so(eff_num(L->o_w->qtype, d, M));
        if (gemm_dev(c, L->o_w, ctx, r2 ? x : tmp, M, r2 ? 2 : 0, st)) return -1;
    }
    c->pa.src = nullptr;
    if (bias_add(tmp, L->o_b, M, d, st)) return -1;
    // x += tmp; conv module on LN(x) (:503-507, 413-462)
    if (enc_add_ln(c, x, r2 ? nullptr : tmp, r2 ? 0.0f : 1.0f, L->ln_conv_w, L->ln_conv_b, xn, M, d, &L->pw1_w, 1,
                   st))
        return -1;
    {
        NumScope s1(eff_num(L->pw1_w->qtype, d, M));
        if (gemm_dev(c, L->pw1_w, xn, h, M, 0, st)) return -1;
    }
    c->pa.src = nullptr;
    if (bias_add(h, L->pw1_b, M, 2 * d, st)) return -1;
    // the GLU (g = q, free now) folded into the depthwise conv where it can be
    const bool glu_dw = mh_glu_dwconv_supported(d, conv_k);
    if (!glu_dw) ENC_TRY(mh_launch_glu(h, q, M, d, st));
    auto dwconv = [&](const float *sc, const float *sh, float *o, uint8_t *xp, float *xpf) {
        return glu_dw ? mh_launch_glu_dwconv(h, L->dw_w, L->dw_b, sc, sh, o, T, nseq, d, conv_k, causal, xp, xpf, st)
                      : mh_launch_dwconv(q, L->dw_w, L->dw_b, sc, sh, o, T, nseq, d, conv_k, causal, st);
    };
    if (L->cnorm_scale) {
        // with the folded batch norm the conv's output feeds only pw2: written
        // as its prepared input (tagged k) when pw2 takes the EXACT GEMM path
        uint8_t *xp = nullptr;
        float *xpf = nullptr;
        c->pa.src = nullptr;
        if (glu_dw && ln_preps(&L->pw2_w, 1, M, d)) {
            size_t bs[3];
            prep_sizes(0, mh_mpad(M), d, bs);
            xp = (uint8_t *)c->pa.xp.get(bs[0]);
            float *xs16 = (float *)c->pa.xs16.get(bs[1]);
            xpf = (float *)c->pa.xpf.get(bs[2]);
            if (!xp || !xs16 || !xpf) return fail("workspace allocation failed");
        }
        ENC_TRY(dwconv(L->cnorm_scale, L->cnorm_shift, k, xp, xpf));
        if (xp) {
            c->pa.T = M;
            c->pa.Kp = d;
            c->pa.xsum = 0;
            c->pa.i8 = 0;
            c->pa.src = k;
        }
    } else {
        ENC_TRY(dwconv(nullptr, nullptr, v, nullptr, nullptr));
        ENC_TRY(mh_launch_add_ln(v, nullptr, 0.0f, L->cnorm_w, L->cnorm_b, k, M, d, st));
        ENC_TRY(mh_launch_silu(k, md, st));
    }
    const bool r3 = res_ok(L->pw2_w, L->pw2_b != nullptr);
    {
        NumScope s2(eff_num(L->pw2_w->qtype, d, M));
        if (gemm_dev(c, L->pw2_w, k, r3 ? x : tmp, M, r3 ? 2 : 0, st)) return -1;
    }
    c->pa.src = nullptr;
    if (bias_add(tmp, L->pw2_b, M, d, st)) return -1;
    // x += tmp; 1/2 FFN2 on LN(x) (:508-511)
    if (enc_add_ln(c, x, r3 ? nullptr : tmp, r3 ? 0.0f : 1.0f, L->ln_ff2_w, L->ln_ff2_b, xn, M, d, &L->ff2_w1, 1,
                   st))
        return -1;
    const bool r4 = res_ok(L->ff2_w2, L->ff2_b1 || L->ff2_b2);
    if (enc_half_ffn(c, L->ff2_w1, L->ff2_w2, L->ff2_b1, L->ff2_b2, xn, r4 ? x : tmp, hf, M, st, r4 ? 3 : 0))
        return -1;
    c->pa.src = nullptr;
    // x += 0.5 tmp; x = LN_out(x) (:511-515)
    ENC_TRY(mh_launch_add_ln(x, r4 ? nullptr : tmp, r4 ? 0.0f : 0.5f, L->ln_out_w, L->ln_out_b, x, M, d, st));
#undef ENC_TRY
    return 0;
}

// mynah_asr_subsampling_forward (src/subsampling.c:208-268) on device
// buffers, activations channel-last; every product in f32 arithmetic.
int subsampling_dev(Ctx *c, const mynah_asr_hip_subsampling *ss, const float *feats, int T, int nseq, int F,
                    float xscale, float *out, int *t_out, hipStream_t st) {
    const int C = ss->channels, cz = ss->causal;
    const int T1 = mh_ss_out_len(T, cz), F1 = mh_ss_out_len(F, cz);
    const int T2 = mh_ss_out_len(T1, cz), F2 = mh_ss_out_len(F1, cz);
    const int T3 = mh_ss_out_len(T2, cz), F3 = mh_ss_out_len(F2, cz);
    *t_out = T3;
    if (T3 <= 0 || F3 <= 0) return fail("subsampling: input too short for three stride-2 stages");
    if (ss->lin_w->dw.k != C * F3) return fail("subsampling: lin_w must be [d_model, channels * F']");
    // A holds the pointwise outputs; B the depthwise outputs, then the
    // flattened rows (the first conv's output is never stored)
    const size_t a = (size_t)nseq * T2 * F2 * C, b = a, tw = (size_t)27 * C;
    float *A = (float *)c->ssb.get((a + b + tw) * sizeof(float));
    if (!A) return fail("device buffer allocation failed");
    float *B = A + a, *w0 = B + b, *w1 = w0 + 9 * (size_t)C, *w2 = w1 + 9 * (size_t)C;   // taps tap-major
    hipError_t e;
#define SS_TRY(expr)                                                                 \
    do {                                                                             \
        e = (expr);                                                                  \
        if (e != hipSuccess) return fail("subsampling launch failed", hipGetErrorString(e)); \
    } while (0)
    NumScope sc(MYNAH_ASR_HIP_EXACT);
    SS_TRY(mh_launch_transpose_taps(ss->conv_in_w, w0, C, 9, st));
    SS_TRY(mh_launch_transpose_taps(ss->dw_w[0], w1, C, 9, st));
    SS_TRY(mh_launch_transpose_taps(ss->dw_w[1], w2, C, 9, st));
    SS_TRY(mh_launch_conv_in_dw(feats, w0, ss->conv_in_b, w1, ss->dw_b[0], B, nseq, T, F, C, cz, st));
    if (gemm_dev(c, ss->pw_w[0], B, A, nseq * T2 * F2, 0, st)) return -1;
    SS_TRY(mh_launch_dw_s2(A, ss->pw_b[0], w2, ss->dw_b[1], B, nseq, T2, F2, C, cz, st));
    if (gemm_dev(c, ss->pw_w[1], B, A, nseq * T3 * F3, 0, st)) return -1;
    SS_TRY(mh_launch_flatten(A, ss->pw_b[1], B, (size_t)nseq * T3, F3, C, st));
    if (gemm_dev(c, ss->lin_w, B, out, nseq * T3, 0, st)) return -1;
    SS_TRY(mh_launch_bias_scale(out, ss->lin_b, (size_t)nseq * T3, ss->d_model, xscale, st));
#undef SS_TRY
    return 0;
}

int begin(Ctx **c) {
    t_err[0] = 0;
    if (!mynah_asr_hip_available()) return fail("no gfx950 device");
    *c = ctx();
    if (!*c) return fail("stream creation failed");
    return 0;
}

}  // namespace

extern "C" {

int mynah_asr_hip_available(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ready < 0) {
        int n = 0;
        g_ready = 0;
        if (hipGetDeviceCount(&n) == hipSuccess && n > 0) {
            hipDeviceProp_t p;
            if (hipGetDeviceProperties(&p, 0) == hipSuccess && strncmp(p.gcnArchName, "gfx950", 6) == 0)
                g_ready = 1;
        }
    }
    return g_ready == 1;
}

int mynah_asr_hip_set_numerics(int mode) {
    if (mode == MYNAH_ASR_HIP_EXACT || mode == MYNAH_ASR_HIP_INT8ACT || mode == MYNAH_ASR_HIP_QMAT)
        g_numerics.store(mode, std::memory_order_relaxed);
    return mynah_asr_hip_numerics();
}

int mynah_asr_hip_numerics(void) {
    int m = g_numerics.load(std::memory_order_relaxed);
    if (m < 0) {
        const char *e = getenv("MYNAH_ASR_HIP_NUMERICS");
        m = (e && strcmp(e, "int8") == 0)   ? MYNAH_ASR_HIP_INT8ACT
            : (e && strcmp(e, "qmat") == 0) ? MYNAH_ASR_HIP_QMAT
                                            : MYNAH_ASR_HIP_EXACT;
        int expect = -1;   // a concurrent first call or set_numerics may have won: keep theirs
        if (!g_numerics.compare_exchange_strong(expect, m, std::memory_order_relaxed)) m = expect;
    }
    return m;
}

const char *mynah_asr_hip_last_error(void) { return t_err; }

mynah_asr_hip_weight *mynah_asr_hip_weight_create(const mynah_asr_hip_wdesc *w) {
    t_err[0] = 0;
    if (!mynah_asr_hip_available()) { fail("no gfx950 device"); return nullptr; }
    return upload(w);
}

void mynah_asr_hip_weight_destroy(mynah_asr_hip_weight *w) {
    if (!w) return;
    (void)hipFree(w->mem);
    delete w;
}

size_t mynah_asr_hip_weight_bytes(const mynah_asr_hip_weight *w) { return w ? w->bytes : 0; }

int mynah_asr_hip_qgemm_dev(const mynah_asr_hip_weight *w, const float *dx, float *dy, int T, int act,
                            void *stream) {
    act = act != 0;   // 0 none, anything else SiLU (the residual modes are internal)
    Ctx *c;
    if (begin(&c)) return -1;
    note_capture(pick_stream(stream));
    if (!w || !dx || !dy || T < 0) return fail("bad argument");
    if (T == 0) return 0;
    if (check_numerics_supported(w->qtype, w->dw.k, T)) return -1;
    NumScope sc(eff_num(w->qtype, w->dw.k, T));
    return gemm_dev(c, w, dx, dy, T, act, pick_stream(stream));
}

int mynah_asr_hip_qgemm_noalloc_dev(const mynah_asr_hip_weight *w, const float *dx, float *dy, int T, int act,
                                    void *stream) {
    act = act != 0;   // 0 none, anything else SiLU (the residual modes are internal)
    // no begin(): that creates the thread's stream; this call uses `stream`
    // as given (NULL = the null stream) and allocates nothing
    t_err[0] = 0;
    if (!mynah_asr_hip_available()) return fail("no gfx950 device");
    if (!w || !dx || !dy || T < 0) return fail("bad argument");
    if (T == 0) return 0;
    if (check_numerics_supported(w->qtype, w->dw.k, T)) return -1;
    NumScope sc(eff_num(w->qtype, w->dw.k, T));
    return gemm_noalloc(w, dx, dy, T, act, (hipStream_t)stream);
}

size_t mynah_asr_hip_noalloc_bytes(const mynah_asr_hip_weight *w, int T) {
    if (!w || T <= 0) return 0;
    NumScope sc(eff_num(w->qtype, w->dw.k, T));
    size_t a, b;
    return noalloc_need(w, T, &a, &b);
}

int mynah_asr_hip_prep_dev(const mynah_asr_hip_weight *w, const float *dx, int T, void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    note_capture(pick_stream(stream));
    if (!w || !dx || T <= 0) return fail("bad argument");
    if (check_numerics_supported(w->qtype, w->dw.k, T)) return -1;
    NumScope sc(eff_num(w->qtype, w->dw.k, T));
    return prep_for(c, w, dx, T, pick_stream(stream));
}

int mynah_asr_hip_qgemm_prepped_dev(const mynah_asr_hip_weight *w, float *dy, int T, int act,
                                    void *stream) {
    act = act != 0;   // 0 none, anything else SiLU (the residual modes are internal)
    Ctx *c;
    if (begin(&c)) return -1;
    note_capture(pick_stream(stream));
    if (!w || !dy || T <= 0) return fail("bad argument");
    if (check_numerics_supported(w->qtype, w->dw.k, T)) return -1;
    NumScope sc(eff_num(w->qtype, w->dw.k, T));
    if (!prep_fits(c, w, T)) return fail("the prepared input does not fit this weight");
    return run_prepped(c, w, dy, T, act, pick_stream(stream));
}

int mynah_asr_hip_qffn_dev(const mynah_asr_hip_weight *w1, const mynah_asr_hip_weight *w2, const float *dx,
                           float *dy, int T, void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    note_capture(pick_stream(stream));
    if (!w1 || !w2 || !dx || !dy || T < 0 || w2->dw.k != w1->dw.n) return fail("bad argument");
    if (T == 0) return 0;
    if (check_numerics_supported(w1->qtype, w1->dw.k, T) || check_numerics_supported(w2->qtype, w2->dw.k, T)) return -1;
    return ffn_dev(c, w1, w2, dx, dy, T, pick_stream(stream));
}

int mynah_asr_hip_qqkv_dev(const mynah_asr_hip_weight *wq, const mynah_asr_hip_weight *wk,
                           const mynah_asr_hip_weight *wv, const float *dx, float *dq, float *dk, float *dv, int T,
                           void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    note_capture(pick_stream(stream));
    if (!wq || !wk || !wv || !dx || !dq || !dk || !dv || T < 0 || wk->dw.k != wq->dw.k || wv->dw.k != wq->dw.k)
        return fail("bad argument");
    if (T == 0) return 0;
    const mynah_asr_hip_weight *W[3] = {wq, wk, wv};
    float *const dy[3] = {dq, dk, dv};
    for (int i = 0; i < 3; i++)
        if (check_numerics_supported(W[i]->qtype, W[i]->dw.k, T)) return -1;
    return qkv_dev(c, W, dx, dy, T, pick_stream(stream));
}

int mynah_asr_hip_dequant_dev(const mynah_asr_hip_weight *w, float *dwd, void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    if (!w || !dwd) return fail("bad argument");
    if (w->qtype == MYNAH_ASR_HIP_F32) return fail("F32 weights are not decoded (plain copy)");
    hipError_t e = mh_launch_dequant(w->qtype, w->dw, dwd, pick_stream(stream));
    if (e != hipSuccess) return fail("dequant launch failed", hipGetErrorString(e));
    return 0;
}

int mynah_asr_hip_read_floor_dev(const void *p, size_t bytes, void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    if (!p || ((uintptr_t)p & 15) || (bytes & 15)) return fail("bad argument: 16-byte aligned pointer and size");
    hipError_t e = mh_launch_read_floor(p, bytes, pick_stream(stream));
    if (e != hipSuccess) return fail("read launch failed", hipGetErrorString(e));
    return 0;
}

int mynah_asr_hip_relpos_attention_dev(const float *q, const float *k, const float *v, const float *rk,
                                       const float *bias_u, const float *bias_v, float *ctx, int T, int d,
                                       int H, int left, int right, int nseq, void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    note_capture(pick_stream(stream));   // the split workspace may grow
    if (!q || !k || !v || !rk || !bias_u || !bias_v || !ctx || T < 0 || nseq < 0 || H <= 0 || d <= 0 ||
        d % H != 0)
        return fail("bad argument");
    if (!mh_attn_supported(d / H)) return fail("head size must be 64 or 128");
    if (left >= 0 && right < 0) return fail("chunked attention needs right >= 0");
    const void *ptrs[7] = {q, k, v, rk, bias_u, bias_v, ctx};
    for (const void *p : ptrs)
        if ((uintptr_t)p % 16) return fail("attention buffers must be 16-byte aligned");
    if (ctx == q || ctx == k || ctx == v) return fail("ctx may not alias q, k or v");
    if ((size_t)2 * T * d >= 0x7fffffffu) return fail("attention: 2 T d must stay below 2^31");
    if (T == 0 || nseq == 0) return 0;
    const size_t wb = mh_attn_ws_bytes(T, d, H, nseq, left);
    void *ws = wb ? c->attw.get(wb) : nullptr;
    if (wb && !ws) return fail("device buffer allocation failed");
    hipError_t e = mh_launch_relpos_attn(q, k, v, rk, bias_u, bias_v, ctx, T, d, H, left, right, nseq, ws,
                                         nullptr, nullptr, pick_stream(stream));
    if (e != hipSuccess) return fail("attention launch failed", hipGetErrorString(e));
    return 0;
}

int mynah_asr_hip_relpos_attention(const float *q, const float *k, const float *v, const float *rk,
                                   const float *bias_u, const float *bias_v, float *ctx, int T, int d, int H,
                                   int left, int right) {
    Ctx *c;
    if (begin(&c)) return -1;
    if (!q || !k || !v || !rk || !bias_u || !bias_v || !ctx || T < 0 || H <= 0 || d <= 0 || d % H != 0)
        return fail("bad argument");
    if (!mh_attn_supported(d / H)) return fail("head size must be 64 or 128");
    if (T == 0) return 0;
    const size_t td = (size_t)T * d, pd = (size_t)(2 * T - 1) * d;
    float *base = (float *)c->att.get((4 * td + pd + 2 * (size_t)d) * sizeof(float));
    if (!base) return fail("device buffer allocation failed");
    float *dq = base, *dk = dq + td, *dv = dk + td, *dctx = dv + td, *drk = dctx + td, *dbu = drk + pd,
          *dbv = dbu + d;
    const float *src[6] = {q, k, v, rk, bias_u, bias_v};
    float *dst[6] = {dq, dk, dv, drk, dbu, dbv};
    const size_t n[6] = {td, td, td, pd, (size_t)d, (size_t)d};
    for (int i = 0; i < 6; i++)
        if (hipMemcpyAsync(dst[i], src[i], n[i] * sizeof(float), hipMemcpyHostToDevice, c->st) != hipSuccess)
            return fail("H2D copy failed");
    if (mynah_asr_hip_relpos_attention_dev(dq, dk, dv, drk, dbu, dbv, dctx, T, d, H, left, right, 1, c->st))
        return -1;
    return d2h_sync(c, ctx, dctx, td);
}

int mynah_asr_hip_encoder_layer_dev(const mynah_asr_hip_enc_layer *L, float *x, int T, int nseq, const float *pe,
                                    int d, int H, int conv_k, int causal, int left, int right, void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    note_capture(pick_stream(stream));
    if (enc_check(L, T, nseq, d, H, conv_k)) return -1;
    if (!x || !pe) return fail("bad argument");
    if (left >= 0 && right < 0) return fail("chunked attention needs right >= 0");
    if (((uintptr_t)x | (uintptr_t)pe) % 16) return fail("encoder layer buffers must be 16-byte aligned");
    if (T == 0 || nseq == 0) return 0;
    const mynah_asr_hip_weight *lin[] = {L->ff1_w1, L->ff1_w2, L->q_w, L->k_w, L->v_w, L->o_w,
                                         L->pw1_w, L->pw2_w, L->ff2_w1, L->ff2_w2};
    for (const mynah_asr_hip_weight *w : lin)
        if (check_numerics_supported(w->qtype, w->dw.k, T * nseq)) return -1;
    return encoder_layer_dev(c, L, x, T, nseq, pe, d, H, conv_k, causal, left, right, pick_stream(stream));
}

int mynah_asr_hip_subsampling_dev(const mynah_asr_hip_subsampling *ss, const float *feats, int T, int nseq,
                                  int n_mels, float xscale, float *out, int *t_out, void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    note_capture(pick_stream(stream));
    if (!ss || !feats || !out || !t_out || T < 0 || nseq < 0 || n_mels <= 0) return fail("bad argument");
    const int C = ss->channels;
    if (C <= 0 || C % 4 || ss->d_model <= 0) return fail("subsampling: channels must be a multiple of 4");
    if (!ss->conv_in_w || !ss->conv_in_b || !ss->lin_w || !ss->lin_b) return fail("subsampling: missing tensor");
    for (int i = 0; i < 2; i++)
        if (!ss->dw_w[i] || !ss->dw_b[i] || !ss->pw_w[i] || !ss->pw_b[i]) return fail("subsampling: missing tensor");
    for (int i = 0; i < 2; i++)
        if (ss->pw_w[i]->dw.n != C || ss->pw_w[i]->dw.k != C) return fail("subsampling: pw_w must be [C, C]");
    if (ss->lin_w->dw.n != ss->d_model) return fail("subsampling: lin_w must be [d_model, channels * F']");
    if (((uintptr_t)feats | (uintptr_t)out) % 16) return fail("subsampling buffers must be 16-byte aligned");
    if (T == 0 || nseq == 0) {
        *t_out = 0;
        return 0;
    }
    return subsampling_dev(c, ss, feats, T, nseq, n_mels, xscale, out, t_out, pick_stream(stream));
}

// The decoder entry points cannot run under a caller's graph capture: each
// captures (and replays) its own step graph on the stream, reads tokens back
// on the host (decode) and grows its thread buffers between calls. Refused
// up front with a clear message rather than failing inside the capture.
static int aed_refuse_capture(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return fail("stream capture query failed");
    if (cs != hipStreamCaptureStatusNone)
        return fail("the AED decoder entry points cannot be called under stream capture (they capture their own "
                    "step graph)");
    return 0;
}

int mynah_asr_hip_aed_decode_dev(const mynah_asr_hip_aed *a, const float *enc, int T, const int *prompt,
                                 int n_prompt, int eos, int *tokens, int cap, void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    if (aed_refuse_capture(pick_stream(stream))) return -1;
    if (aed_check(a, T)) return -1;
    NumScope sc(MYNAH_ASR_HIP_EXACT);
    if (!enc || !prompt || n_prompt <= 0 || !tokens || cap < 0) return fail("bad argument");
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= a->vocab) return fail("prompt token outside the vocabulary");
    int max_len = n_prompt + cap;
    if (max_len > a->max_seq) max_len = a->max_seq;
    return aed_run(c, a, enc, T, prompt, n_prompt, max_len, eos, tokens, cap, nullptr, pick_stream(stream));
}

int mynah_asr_hip_aed_forced_dev(const mynah_asr_hip_aed *a, const float *enc, int T, const int *tokens, int n,
                                 float *logits, void *stream) {
    Ctx *c;
    if (begin(&c)) return -1;
    if (aed_refuse_capture(pick_stream(stream))) return -1;
    if (aed_check(a, T)) return -1;
    NumScope sc(MYNAH_ASR_HIP_EXACT);
    if (!enc || !tokens || n <= 0 || n > a->max_seq || !logits) return fail("bad argument");
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= a->vocab) return fail("token outside the vocabulary");
    const int r = aed_run(c, a, enc, T, tokens, n, n, -1, nullptr, 0, logits, pick_stream(stream));
    return r < 0 ? -1 : 0;
}

int mynah_asr_hip_qgemm(const mynah_asr_hip_wdesc *w, const float *x, float *out, int T) {
    Ctx *c;
    if (begin(&c)) return -1;
    if (!w || !x || !out || T < 0) return fail("bad argument");
    if (T == 0) return 0;
    if (check_numerics_supported(w->qtype, w->k, T)) return -1;
    NumScope sc(eff_num(w->qtype, w->k, T));
    const mynah_asr_hip_weight *W = resident(w);
    if (!W) return -1;
    float *dx, *dy = (float *)c->y.get((size_t)T * w->n * sizeof(float));
    if (!dy) return fail("device buffer allocation failed");
    if (h2d(c, c->x, x, (size_t)T * w->k, &dx)) return -1;
    if (gemm_dev(c, W, dx, dy, T, 0, c->st)) return -1;
    return d2h_sync(c, out, dy, (size_t)T * w->n);
}

int mynah_asr_hip_qffn(const mynah_asr_hip_wdesc *w1, const mynah_asr_hip_wdesc *w2, const float *x,
                       float *out, int T) {
    Ctx *c;
    if (begin(&c)) return -1;
    if (!w1 || !w2 || !x || !out || T < 0 || w2->k != w1->n) return fail("bad argument");
    if (T == 0) return 0;
    if (check_numerics_supported(w1->qtype, w1->k, T) || check_numerics_supported(w2->qtype, w2->k, T)) return -1;
    const mynah_asr_hip_weight *W1 = resident(w1), *W2 = resident(w2);
    if (!W1 || !W2) return -1;
    float *dx, *dy = (float *)c->y.get((size_t)T * w2->n * sizeof(float));
    if (!dy) return fail("device buffer allocation failed");
    if (h2d(c, c->x, x, (size_t)T * w1->k, &dx)) return -1;  // x is consumed before out is written
    if (ffn_dev(c, W1, W2, dx, dy, T, c->st)) return -1;
    return d2h_sync(c, out, dy, (size_t)T * w2->n);
}

int mynah_asr_hip_qqkv(const mynah_asr_hip_wdesc *wq, const mynah_asr_hip_wdesc *wk,
                       const mynah_asr_hip_wdesc *wv, const float *x, float *oq, float *ok, float *ov,
                       int T) {
    Ctx *c;
    if (begin(&c)) return -1;
    if (!wq || !wk || !wv || !x || !oq || !ok || !ov || T < 0 || wk->k != wq->k || wv->k != wq->k)
        return fail("bad argument");
    if (T == 0) return 0;
    const mynah_asr_hip_wdesc *ws[3] = {wq, wk, wv};
    float *outs[3] = {oq, ok, ov};
    const mynah_asr_hip_weight *W[3];
    for (int i = 0; i < 3; i++) {
        if (check_numerics_supported(ws[i]->qtype, ws[i]->k, T)) return -1;
        if (!(W[i] = resident(ws[i]))) return -1;
    }
    float *dx;
    if (h2d(c, c->x, x, (size_t)T * wq->k, &dx)) return -1;
    // one prepared input serves the three products whenever it fits them
    bool prepared = false;
    for (int i = 0; i < 3; i++) {
        float *dy = (float *)c->y.get((size_t)T * ws[i]->n * sizeof(float));
        if (!dy) return fail("device buffer allocation failed");
        NumScope si(eff_num(ws[i]->qtype, ws[i]->k, T));
        if (num_now() == MYNAH_ASR_HIP_EXACT && mh_use_gemv(W[i]->dw, T)) {
            if (gemm_dev(c, W[i], dx, dy, T, 0, c->st)) return -1;
        } else {
            if (!prepared || !prep_fits(c, W[i], T))
                if (prep_for(c, W[i], dx, T, c->st)) return -1;
            prepared = true;
            if (run_prepped(c, W[i], dy, T, 0, c->st)) return -1;
        }
        if (d2h_sync(c, outs[i], dy, (size_t)T * ws[i]->n)) return -1;
    }
    return 0;
}

int mynah_asr_hip_dequant(const mynah_asr_hip_wdesc *w, float *wd) {
    Ctx *c;
    if (begin(&c)) return -1;
    if (!w || !wd) return fail("bad argument");
    if (w->qtype == MYNAH_ASR_HIP_F32) return fail("F32 weights are not decoded (plain copy)");
    const mynah_asr_hip_weight *W = resident(w);
    if (!W) return -1;
    float *dw = (float *)c->y.get((size_t)w->n * w->k * sizeof(float));
    if (!dw) return fail("device buffer allocation failed");
    hipError_t e = mh_launch_dequant(W->qtype, W->dw, dw, c->st);
    if (e != hipSuccess) return fail("dequant launch failed", hipGetErrorString(e));
    return d2h_sync(c, wd, dw, (size_t)w->n * w->k);
}

static mynah_asr_hip_wdesc f32_desc(const float *w, int n, int k) {
    mynah_asr_hip_wdesc d;
    d.qtype = MYNAH_ASR_HIP_F32;
    d.n = n;
    d.k = k;
    d.data = w;
    d.scales = nullptr;
    return d;
}

int mynah_asr_hip_gemm_wt(const float *x, const float *w, float *out, int T, int n, int k) {
    const mynah_asr_hip_wdesc d = f32_desc(w, n, k);
    return mynah_asr_hip_qgemm(&d, x, out, T);
}

int mynah_asr_hip_ffn_wt(const float *x, const float *w1, int n1, const float *w2, int n2, float *out,
                         int T, int k) {
    const mynah_asr_hip_wdesc d1 = f32_desc(w1, n1, k), d2 = f32_desc(w2, n2, n1);
    return mynah_asr_hip_qffn(&d1, &d2, x, out, T);
}

int mynah_asr_hip_gemm3_wt(const float *x, const float *wa, const float *wb, const float *wc, float *oa,
                           float *ob, float *oc, int T, int n, int k) {
    const mynah_asr_hip_wdesc a = f32_desc(wa, n, k), b = f32_desc(wb, n, k), c = f32_desc(wc, n, k);
    return mynah_asr_hip_qqkv(&a, &b, &c, x, oa, ob, oc, T);
}

void mynah_asr_hip_evict(const void *data) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (size_t i = 0; i < g_cache.size();) {
        if (g_cache[i].key == data) {
            mynah_asr_hip_weight_destroy(g_cache[i].w);
            g_cache.erase(g_cache.begin() + i);
        } else {
            i++;
        }
    }
}

void mynah_asr_hip_evict_all(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto &e : g_cache) mynah_asr_hip_weight_destroy(e.w);
    g_cache.clear();
}

}  // extern "C"
