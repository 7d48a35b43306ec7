/* mynah_asr_hip.h — C ABI of the MI355X (gfx950) backend unit for mynah-asr's
 * linear-layer hot path.
 *
 * The unit plays the role src/cuda_gemm.cu plays for CUDA: backend.c and qmat.c
 * call these functions first and fall back to their CPU code when one returns
 * -1 (src/backend.c:74-77). Every entry point takes plain host pointers and
 * sizes; nothing here exposes a HIP or torch type (streams travel as void*).
 *
 * Numerics. Three modes, chosen process-wide with mynah_asr_hip_set_numerics():
 *   EXACT (default): every output row matches an f32 GEMM over the
 *     dequantized weights to |y - ref| <= 1e-4*|ref| + 1e-6 (ref accumulated in
 *     double), and a row's bits never depend on how many rows share the call.
 *   INT8ACT: int8 activations and exact integer sums, for every M.
 *     INT8 / INT4: the reference's small-T path (qmat.c:186-202, 508-552),
 *     its f32 combine order included. Q4_K / Q5_K: ingot's int8 path
 *     (third_party/ingot/src/kernels.c:719-750, 1767-1791, 2325-2353;
 *     activations per 256-element super-block), within 1e-7 of it. Q8_0 /
 *     Q4_0 (activations per row as qmat.c:186-202) and Q2_K, Q3_K, Q6_K (per
 *     super-block, as Q4_K): this unit's own extension; the reference has no
 *     int8 path for them (its matmat is exact f32 there). Error against the
 *     f32 product, measured on the reference's own int8 test case
 *     (tests/test_quant.c:157-205, uniform(-1, 1) activations): 3.9e-3
 *     relative L2 for every block format, under that test's 5e-3 budget; this
 *     is a measurement on that case, not a bound (N(0, 1) activations at
 *     K = 1024 give 6.9e-3 to 7.8e-3). F32 weights return -1.
 *   QMAT: qmat.c's own choice per product (src/qmat.c:503-651): INT8ACT for
 *     INT8/INT4 weights with K <= 8192 at T <= 16 (and at every T with
 *     MYNAH_ASR_QGEMM=1), EXACT for everything else. Bit-exact with the
 *     reference wherever it computes in int8; not row-stable across T = 16.
 *
 * Return values: 0 = done, -1 = not done (the caller runs its CPU path);
 * mynah_asr_hip_last_error() names the reason for the calling thread.
 * Thread safety: every entry point may be called from many threads at once;
 * each thread gets its own HIP stream and device buffers, and the weight cache
 * is shared under a lock. */
#ifndef MYNAH_ASR_HIP_H
#define MYNAH_ASR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight formats. 0..2 are qmat.h's own (src/qmat.h:23); the ggml block formats
 * are 16 + their GGML type id (third_party/ingot/tests/fixtures/geometry.txt). */
enum {
    MYNAH_ASR_HIP_F32 = 0,   /* float [n, k] */
    MYNAH_ASR_HIP_INT8 = 1,  /* qmat per-row: int8 [n, k] + float scales [n] */
    MYNAH_ASR_HIP_INT4 = 2,  /* qmat group-32: uint8 [n, k/2] (elements 2j | 2j+1<<4) + float [n, k/32] */
    MYNAH_ASR_HIP_Q4_0 = 18, /* ggml blocks, GGUF byte layout, row-major [n, k/block] */
    MYNAH_ASR_HIP_Q8_0 = 24,
    MYNAH_ASR_HIP_Q2_K = 26,
    MYNAH_ASR_HIP_Q3_K = 27,
    MYNAH_ASR_HIP_Q4_K = 28,
    MYNAH_ASR_HIP_Q5_K = 29,
    MYNAH_ASR_HIP_Q6_K = 30
};

enum { MYNAH_ASR_HIP_EXACT = 0, MYNAH_ASR_HIP_INT8ACT = 1, MYNAH_ASR_HIP_QMAT = 2 };

/* A weight matrix as the caller holds it in host memory: the fields of
 * mynah_asr_qmat (src/qmat.h:39-47) plus the raw ggml block pointer. `data` is
 * also the cache key: it must stay valid and unchanged until evicted
 * (src/backend.h:16-18). */
typedef struct {
    int qtype;
    int n, k;
    const void *data;     /* F32 floats, INT8/INT4 quants, or ggml block bytes */
    const float *scales;  /* INT8 [n], INT4 [n, k/32]; NULL for the other formats */
} mynah_asr_hip_wdesc;

/* 1 when a gfx950 device is present and usable. Replaces
 * mynah_asr_cuda_available (src/cuda_gemm.cu:62, declared src/backend.c:24). */
int mynah_asr_hip_available(void);

/* Process-wide numerics mode (MYNAH_ASR_HIP_EXACT / _INT8ACT / _QMAT). Returns
 * the mode now in force. The environment variable MYNAH_ASR_HIP_NUMERICS=int8
 * selects INT8ACT at first use, =qmat QMAT. No reference counterpart: EXACT
 * and INT8ACT expose the choice qmat.c makes by row count (src/qmat.c:180,
 * 508, 644) as a fixed setting, so a row's result never depends on the batch
 * size. QMAT instead makes that choice per product as qmat.c does
 * (src/qmat.c:503-651): INT8/INT4 weights with K <= 8192 take the
 * int8-activation path (INT8ACT's, bit-exact with the reference's) for
 * T <= 16, and for every T when MYNAH_ASR_QGEMM=1 is set (qmat.c:598-643;
 * read at each product, where qmat.c reads it once); every other product is
 * EXACT (the reference's dequant + sgemm,
 * to the tolerance above). Like the reference it is not row-stable across
 * T = 16 for INT8/INT4 weights. The device AED decoder refuses INT8/INT4
 * weights in QMAT (their one-row products would take the int8 path). */
int mynah_asr_hip_set_numerics(int mode);
int mynah_asr_hip_numerics(void);

/* ---- host-pointer entry points (the drop-in boundary) ---------------------- */

/* out[T,n] = x[T,k] . w[n,k]^T with f32 weights. Replaces
 * mynah_asr_cuda_gemm_wt (src/cuda_gemm.cu:144-190); caller mynah_asr_gemm_wt
 * (src/backend.c:68-81). */
int mynah_asr_hip_gemm_wt(const float *x, const float *w, float *out, int T, int n, int k);

/* out[T,n2] = SiLU(x . w1^T) . w2^T, the intermediate kept on the device.
 * Same contract as mynah_asr_metal_ffn_wt (src/backend.c:17-18); caller
 * mynah_asr_ffn_wt (src/backend.c:110-120). x may alias out. */
int mynah_asr_hip_ffn_wt(const float *x, const float *w1, int n1, const float *w2, int n2,
                         float *out, int T, int k);

/* Three GEMMs over one input. Same contract as mynah_asr_metal_gemm3_wt
 * (src/backend.c:19-21); caller mynah_asr_gemm3_wt (src/backend.c:122-132). */
int mynah_asr_hip_gemm3_wt(const float *x, const float *wa, const float *wb, const float *wc,
                           float *oa, float *ob, float *oc, int T, int n, int k);

/* out[T,n] = x[T,k] . W^T for any supported format. The HIP branch of
 * mynah_asr_qmat_mul (src/qmat.c:503-651). */
int mynah_asr_hip_qgemm(const mynah_asr_hip_wdesc *w, const float *x, float *out, int T);

/* out = SiLU(x . W1^T) . W2^T. The HIP branch of mynah_asr_qmat_ffn
 * (src/qmat.c:654-663). x may alias out (src/encoder.c:474 passes the same
 * buffer). */
int mynah_asr_hip_qffn(const mynah_asr_hip_wdesc *w1, const mynah_asr_hip_wdesc *w2,
                       const float *x, float *out, int T);

/* q/k/v over one input (the input is prepared once). The HIP branch of
 * mynah_asr_qmat_qkv (src/qmat.c:665-674). */
int mynah_asr_hip_qqkv(const mynah_asr_hip_wdesc *wq, const mynah_asr_hip_wdesc *wk,
                       const mynah_asr_hip_wdesc *wv, const float *x, float *oq, float *ok,
                       float *ov, int T);

/* wd[n,k] = the dequantized weight, decoded on the device from the resident
 * copy (bit-identical to ingot's dequant.c and qmat.c:152-169). The HIP branch
 * of mynah_asr_qmat_dequant (src/qmat.c:171-177). */
int mynah_asr_hip_dequant(const mynah_asr_hip_wdesc *w, float *wd);

/* Drop resident copies. The reference's CUDA unit never evicts
 * (src/cuda_gemm.cu:92-130); the Metal one evicts on model free
 * (mynah_asr_metal_weights_evict, src/backend.h:55-57). Call from
 * mynah_asr_qmat_free / mynah_asr_free. */
void mynah_asr_hip_evict(const void *data);
void mynah_asr_hip_evict_all(void);

/* Reason for the last -1 returned on this thread ("" when none). */
const char *mynah_asr_hip_last_error(void);

/* ---- device-resident entry points ----------------------------------------
 * For callers that keep activations on the device (the fused encoder layer,
 * the AED decoder loop, benchmarks). `dx`/`dy` are device pointers, `stream`
 * a hipStream_t (NULL = the calling thread's stream). No reference
 * counterpart: the reference copies activations per call
 * (src/cuda_gemm.cu:167-188). */
typedef struct mynah_asr_hip_weight mynah_asr_hip_weight;

/* Upload + repack into the device layout; NULL on failure. */
mynah_asr_hip_weight *mynah_asr_hip_weight_create(const mynah_asr_hip_wdesc *w);
void mynah_asr_hip_weight_destroy(mynah_asr_hip_weight *w);
/* Device bytes the resident copy occupies. */
size_t mynah_asr_hip_weight_bytes(const mynah_asr_hip_weight *w);

/* dy[T,n] = dx[T,k] . W^T; act = 0 none, 1 SiLU applied to the output. */
int mynah_asr_hip_qgemm_dev(const mynah_asr_hip_weight *w, const float *dx, float *dy, int T,
                            int act, void *stream);
/* The two halves of qgemm_dev, for callers that feed one input to several
 * weights (q/k/v) or time the product kernel alone: prep_dev prepares dx for
 * weights of w's inner size into the calling thread's workspace;
 * qgemm_prepped_dev runs the product on the last input this thread prepared
 * (-1 when it does not fit w). Both on `stream`, in order. */
int mynah_asr_hip_prep_dev(const mynah_asr_hip_weight *w, const float *dx, int T, void *stream);
int mynah_asr_hip_qgemm_prepped_dev(const mynah_asr_hip_weight *w, float *dy, int T, int act,
                                    void *stream);
/* dy = SiLU(dx . W1^T) . W2^T (the device twin of mynah_asr_hip_qffn; dx may
 * alias dy). On the GEMM path in EXACT numerics the first product hands the
 * intermediate to the second already prepared (no f32 intermediate is
 * stored); results are bit-identical to two qgemm_dev calls. */
int mynah_asr_hip_qffn_dev(const mynah_asr_hip_weight *w1, const mynah_asr_hip_weight *w2, const float *dx,
                           float *dy, int T, void *stream);
/* dq, dk, dv = dx . Wq^T, Wk^T, Wv^T with one preparation of dx (the device
 * twin of mynah_asr_hip_qqkv). */
int mynah_asr_hip_qqkv_dev(const mynah_asr_hip_weight *wq, const mynah_asr_hip_weight *wk,
                           const mynah_asr_hip_weight *wv, const float *dx, float *dq, float *dk, float *dv, int T,
                           void *stream);
/* qgemm_dev without any allocation, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. The same product and
 * the same bits as mynah_asr_hip_qgemm_dev; the prepared input goes to a
 * 32 MiB device array that each GPU holds from the library's first such call
 * until the process ends, and K is never split over workgroups (the split-K
 * launches need a workspace of their own). `stream` is used as given (NULL =
 * the null stream; no per-thread stream is created). Returns -1 when the
 * prepared input of T rows does not fit the 32 MiB (see
 * mynah_asr_hip_noalloc_bytes). Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (two streams, two threads) race, so the
 * caller orders them. */
int mynah_asr_hip_qgemm_noalloc_dev(const mynah_asr_hip_weight *w, const float *dx, float *dy, int T, int act,
                                    void *stream);
/* Scratch bytes qgemm_noalloc_dev needs for w over T rows in the current
 * numerics mode (0 for the GEMV path, M <= 16, which needs none); calls above
 * 32 MiB (33554432) are refused. */
size_t mynah_asr_hip_noalloc_bytes(const mynah_asr_hip_weight *w, int T);
/* dwd[n,k] = dequantized weight. */
int mynah_asr_hip_dequant_dev(const mynah_asr_hip_weight *w, float *dwd, void *stream);
/* No counterpart in the reference: a measurement aid for benchmarks. One
 * launch that streams `bytes` from device memory at p (16-byte aligned, size a
 * multiple of 16) and computes nothing from them: the one-launch floor a
 * memory-bound product over the same bytes (a decoder GEMV) is compared with. */
int mynah_asr_hip_read_floor_dev(const void *p, size_t bytes, void *stream);

/* Relative-position self-attention core of one encoder layer on device buffers:
 * the computation of src/encoder.c:315-410 (left < 0, full attention) and
 * src/encoder.c:220-313 (left >= 0, chunked-limited attention with chunk =
 * right + 1) from the point where q, k, v carry their biases and
 * rk = pe . relk_w^T (encoder.c:336, 233) has been formed:
 *   ctx[t, h] = sum_j softmax_j(((q[t,h] + bias_u[h]) . k[j,h]
 *                               + (q[t,h] + bias_v[h]) . rk[T-1+j-t, h]) / sqrt(dk)) v[j,h]
 * q, k, v, ctx: nseq segments of [T, d] floats each (row stride d, segment
 * stride T*d); rk: [2T-1, d], shared by the segments; bias_u, bias_v: [d]
 * (head h at columns h*dk .. h*dk+dk-1, dk = d / H, 64 or 128). nseq > 1 runs
 * independent equal-length segments in one launch (the reference calls the
 * layer once per segment). All pointers 16-byte aligned. ctx may not alias
 * q, k or v. Outputs are f32 sums in another order than the reference's BLAS
 * (full attention forms its products from f16 hi + lo splits scaled by
 * powers of two, 22 bits of each row's, or V tile column's, maximum): equal
 * within |y - ref| <= 1e-4*|ref| + 1e-5*max|v|. Full attention first splits
 * K, rk and V into the calling thread's workspace (the size of K + V + rk,
 * grown as needed, as the other _dev calls' buffers are); 2T * d must stay
 * below 2^31. */
/* The same on host buffers, one segment (the call encoder.c's attention() and
 * attention_banded() would make in place of their per-head loops, after rk is
 * formed): copies in, computes, copies ctx out. d must be a multiple of 4. */
int mynah_asr_hip_relpos_attention(const float *q, const float *k, const float *v, const float *rk,
                                   const float *bias_u, const float *bias_v, float *ctx, int T, int d, int H,
                                   int left, int right);
int mynah_asr_hip_relpos_attention_dev(const float *q, const float *k, const float *v, const float *rk,
                                       const float *bias_u, const float *bias_v, float *ctx, int T, int d,
                                       int H, int left, int right, int nseq, void *stream);

/* One FastConformer encoder layer on the device: the device twin of
 * mynah_asr_encoder_layer (src/encoder.c:485-521) in its batched form
 * encoder_layer_batch (:901-946). The fields follow mynah_asr_enc_layer
 * (src/encoder.h:12-32): linears are resident weights (relk_w, the position
 * projection, too: the reference keeps it f32, and an F32 weight here does
 * the same), every other tensor is a device pointer of f32, and a NULL bias
 * is absent. The conv norm is the folded batch norm (cnorm_scale,
 * cnorm_shift) or, when cnorm_scale is NULL, a layer norm (cnorm_w, cnorm_b). */
typedef struct {
    const float *ln_ff1_w, *ln_ff1_b;
    const mynah_asr_hip_weight *ff1_w1, *ff1_w2;
    const float *ln_att_w, *ln_att_b;
    const mynah_asr_hip_weight *q_w, *k_w, *v_w, *o_w, *relk_w;
    const float *bias_u, *bias_v;
    const float *ln_conv_w, *ln_conv_b;
    const mynah_asr_hip_weight *pw1_w, *pw2_w;
    const float *dw_w, *cnorm_w, *cnorm_b;
    const float *ff1_b1, *ff1_b2, *ff2_b1, *ff2_b2;
    const float *q_b, *k_b, *v_b, *o_b;
    const float *pw1_b, *dw_b, *pw2_b;
    const float *cnorm_scale, *cnorm_shift;
    const float *ln_ff2_w, *ln_ff2_b;
    const mynah_asr_hip_weight *ff2_w1, *ff2_w2;
    const float *ln_out_w, *ln_out_b;
} mynah_asr_hip_enc_layer;

/* The layer in place on x: nseq segments of T frames packed back to back
 * ([nseq * T, d], the reference's padding-free batch with equal lengths).
 * The products and layer norms run over all rows; attention and the
 * depthwise conv per segment. pe [2T-1, d]: the segments' relative positional
 * embedding (mynah_asr_pos_emb). d: the model width, 256 times 1 to 8, 12 or
 * 16 (up to 4096); H heads of 64 or 128; conv_k the depthwise kernel (causal: left pad
 * conv_k - 1, else (conv_k - 1) / 2 per side); left / right the attention
 * context as mynah_asr_encoder_layer's (left < 0: full). Each product runs in
 * the current numerics mode; -1 and the reason (mynah_asr_hip_last_error) on
 * a bad argument or a failed launch. */
int mynah_asr_hip_encoder_layer_dev(const mynah_asr_hip_enc_layer *L, float *x, int T, int nseq, const float *pe,
                                    int d, int H, int conv_k, int causal, int left, int right, void *stream);

/* The dw_striding 8x subsampling on the device (the device twin of
 * mynah_asr_subsampling_forward, src/subsampling.c:208-268; tensors of
 * mynah_asr_subsampling, src/subsampling.h:12-21): the 3x3 stride-2 conv
 * 1 -> C channels + ReLU, twice (depthwise 3x3 stride 2, pointwise 1x1, ReLU),
 * the channel-major flatten and the linear to d_model. The pointwise convs and
 * the linear are resident weights (f32 arithmetic: the reference multiplies
 * them in f32); the rest are device pointers. */
typedef struct {
    const float *conv_in_w, *conv_in_b;      /* [C, 1, 3, 3], [C] */
    const float *dw_w[2], *dw_b[2];          /* [C, 1, 3, 3], [C] */
    const mynah_asr_hip_weight *pw_w[2];     /* [C, C] */
    const float *pw_b[2];                    /* [C] */
    const mynah_asr_hip_weight *lin_w;       /* [d_model, C * F'], F' the features after three stages */
    const float *lin_b;                      /* [d_model] */
    int channels, d_model, causal;           /* causal: pads (2, 1), else (1, 1) */
} mynah_asr_hip_subsampling;

/* feats: nseq segments of T frames of n_mels features ([nseq * T, n_mels],
 * equal lengths) -> out [nseq * T', d_model], each row times xscale (the
 * encoder's layer input scale, encoder.c:958-959; 1 for none). *t_out = T'.
 * C a multiple of 4; 16-byte aligned buffers. */
int mynah_asr_hip_subsampling_dev(const mynah_asr_hip_subsampling *ss, const float *feats, int T, int nseq,
                                  int n_mels, float xscale, float *out, int *t_out, void *stream);

/* AED (Canary) decoder on the device: src/decoder_aed.h:12-36 with every
 * linear a resident weight (mynah_asr_hip_weight_create) and every other tensor
 * a device pointer. Biases may not be NULL except proj_b. */
typedef struct {
    const float *ln_self_w, *ln_self_b;
    const mynah_asr_hip_weight *sq, *sk, *sv, *so;
    const float *sq_b, *sk_b, *sv_b, *so_b;
    const float *ln_cross_w, *ln_cross_b;
    const mynah_asr_hip_weight *cq, *ck, *cv, *co;
    const float *cq_b, *ck_b, *cv_b, *co_b;
    const float *ln_ffn_w, *ln_ffn_b;
    const mynah_asr_hip_weight *ff1, *ff2;
    const float *ff1_b, *ff2_b;
} mynah_asr_hip_aed_layer;

typedef struct {
    int n_layers, d, n_heads, ffn, vocab, max_seq;
    const mynah_asr_hip_weight *proj;      /* enc_dec_proj [d, d_enc]; NULL = identity */
    const float *proj_b;                   /* may be NULL */
    const float *emb;                      /* [vocab, d] */
    const float *pos;                      /* [max_seq, d] */
    const float *embln_w, *embln_b;
    const float *fin_w, *fin_b;
    const mynah_asr_hip_weight *head;      /* [vocab, d] */
    const float *head_b;
    const mynah_asr_hip_aed_layer *layers; /* host array of n_layers */
} mynah_asr_hip_aed;

/* Greedy decoding, the device twin of mynah_asr_aed_decode (src/decoder_aed.c:139-232):
 * enc = device [T, d_enc]; prompt (host, n_prompt >= 1), eos, tokens (host, cap):
 * returns the generated token count (prompt and EOS excluded) or -1. The self and
 * cross K/V caches stay on the device; a decoding step is one HIP graph replay
 * (the step's position and token live in device memory). d <= 4096, head size 64
 * or 128, EXACT numerics, every linear on the GEMV path (K <= 8192). */
int mynah_asr_hip_aed_decode_dev(const mynah_asr_hip_aed *a, const float *enc, int T, const int *prompt,
                                 int n_prompt, int eos, int *tokens, int cap, void *stream);
/* The same steps over given tokens (host, n <= max_seq): logits (device,
 * [n, vocab]) of every position, as the decode loop computes them before its
 * argmax. 0 or -1. */
int mynah_asr_hip_aed_forced_dev(const mynah_asr_hip_aed *a, const float *enc, int T, const int *tokens, int n,
                                 float *logits, void *stream);

#ifdef __cplusplus
}
#endif
#endif
