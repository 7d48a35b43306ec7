// launch.h — host-side launchers of kernels.hip (C++ linkage, library-internal).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "fmt.h"   // DevW

// Rows the prepared-activation buffer must hold for an M-row product: the
// kernels read whole row groups up to this count.
static inline int mh_mpad(int M) { return (M + 63) / 64 * 64; }

// x -> prepared activations: xp (f16 A fragments), xpf (fold factors) and,
// for want_xsum 1 / 2, in xs16 (Mpad * Kp / 4 bytes) the mins operands of the
// affine formats with 16- / 32-element sub-blocks
hipError_t mh_launch_prep(const float *x, int M, int K, int Kp, int Mpad, uint8_t *xp, float *xs16,
                          float *xpf, int want_xsum, int vec, hipStream_t st);
// M <= 16 (and K small enough for the LDS partials): the preparation-free GEMV
bool mh_use_gemv(const DevW &W, int M);
// Floats of device workspace that let a GEMV of W split K over workgroups (0:
// it never does). The launchers below take such a workspace (or null) in `ws`;
// with it, K >= 2048 over N <= 2048 runs as two launches (chunk results, then
// their fold in chunk order: the same bits as without). Calls sharing one
// workspace must be ordered on one stream.
size_t mh_gemv_ws_floats(const DevW &W);
hipError_t mh_launch_gemv(int qtype, const DevW &W, const float *x, int M, int vec, float *y, int act,
                          float *ws, hipStream_t st);
// GEMV epilogue: y = act(W x + bias) + res; act 0 none, 1 SiLU, 2 ReLU; bias [n]
// and res [M, n] may be null; res may alias y
struct GEpi {
    int act;
    const float *bias;
    const float *res;
};
hipError_t mh_launch_gemv_epi(int qtype, const DevW &W, const float *x, int M, int vec, float *y, GEpi ep,
                              float *ws, hipStream_t st);
// The input row of a one-row GEMV built per workgroup: GPRO_LN = the layer norm
// of x (w, b); GPRO_COMB = the attention splits merged (opart [H][nsplit][dk],
// ml [H][nsplit][2], n keys = n_fixed, or st[0] + 1 when n_fixed == 0).
enum { GPRO_NONE = 0, GPRO_LN = 1, GPRO_COMB = 2 };
struct GPro {
    int kind;
    const float *x, *w, *b;
    const float *opart, *ml;
    const int *st;
    int n_fixed, nsplit, H;
};
// up to three products of one input, same format and shape
struct GJobs {
    DevW W[3];
    float *y[3];
    GEpi ep[3];
    int n;
};
hipError_t mh_launch_gemv_jobs(int qtype, const GJobs &J, const float *x, int M, int vec, const GPro &pro,
                               hipStream_t st);
// keys per attention split of the decoder step
constexpr int MH_ATT_KC = 64;
__host__ __device__ inline int mh_att_splits_dev(int n) { return (n + MH_ATT_KC - 1) / MH_ATT_KC; }
// Floats of device workspace that let a product of W over M rows split K over
// workgroups (0: it never does). It does when the product has at most 256
// tiles of 64 x 128 (one workgroup per CU or fewer): each chunk's results go
// to the workspace and a second launch folds them in chunk order (the same
// bits as without). Calls sharing one workspace must be ordered on one stream.
size_t mh_gemm_ws_floats(const DevW &W, int M, int jobs = 1);
// a1: the INT8ACT form of the product, on activations prepared by mh_launch_prep_a1
hipError_t mh_launch_gemm(int qtype, const DevW &W, const uint8_t *xp, const float *xs16,
                          const float *xpf, float *y, int M, int act, float *ws, hipStream_t st, bool a1 = false);
// up to three products (same shape) of one prepared input in one launch
struct GemmJobs {
    DevW W[3];
    float *y[3];
    int n;
};
// (ws: as for mh_launch_gemm, sized by mh_gemm_ws_floats(W, M, J.n), or null)
hipError_t mh_launch_gemm_jobs(int qtype, const GemmJobs &J, const uint8_t *xp, const float *xs16,
                               const float *xpf, int M, float *ws, hipStream_t st, bool a1 = false);
// The FFN's first product with SiLU, its output prepared as the input of a
// product with Kp = 128 * oKc (oKc = the first product's column tiles):
// (oxp, oxs16, oxpf) as mh_launch_prep would write them.
hipError_t mh_launch_gemm_prep_out(int qtype, const DevW &W, const uint8_t *xp, const float *xs16,
                                   const float *xpf, int M, uint8_t *oxp, float *oxs16, float *oxpf, int oKc,
                                   int oxsum, hipStream_t st);
hipError_t mh_launch_dequant(int qtype, const DevW &W, float *out, hipStream_t st);
// a plain streaming read of `bytes` (16-byte aligned), nothing written
hipError_t mh_launch_read_floor(const void *p, size_t bytes, hipStream_t st);
hipError_t mh_launch_silu(float *x, size_t n, hipStream_t st);

// INT8ACT numerics (every format but F32). Three activation forms:
//   MH_I8_QMAT (INT8, INT4): int8 bytes for k_gemm_i8, one scale per row
//     (mh_launch_prep_i8), the reference's qmat int8 path;
//   MH_I8_ROW (Q8_0, Q4_0): int8 values as f16 for the A1 GEMM, one scale per
//     row, quantized as the qmat path quantizes;
//   MH_I8_SB (the K-quants): the same, one scale per 256-element super-block
//     (ingot's int8-activation semantics).
enum { MH_I8_QMAT = 1, MH_I8_ROW = 2, MH_I8_SB = 3 };
bool mh_i8_supported(int qtype);
int mh_i8_kind(int qtype);
// xp: Mpad * Kp * 2 bytes; xpf: Mpad * Kp / 128 floats; xs16: the mins operand
// (Mpad * Kp / 4 bytes) when want_xsum (MH_I8_SB only)
hipError_t mh_launch_prep_a1(int kind, const float *x, int M, int K, int Kp, int Mpad, uint8_t *xp, float *xs16,
                             float *xpf, int want_xsum, hipStream_t st);
// MH_I8_QMAT: qx (Mpad * Kp bytes), sx (Mpad floats); inv: Mpad floats of
// scratch (each row's 127 / amax, between the two launches)
hipError_t mh_launch_prep_i8(const float *x, int M, int K, int Kp, int Mpad, uint8_t *qx, float *sx, float *inv,
                             hipStream_t st);
hipError_t mh_launch_gemm_i8(int qtype, const DevW &W, const uint8_t *qx, const float *sx, float *y, int M,
                             int act, hipStream_t st);

// Relative-position self-attention core (attention.hip): head size d / H of 64 or 128
bool mh_attn_supported(int dk);
// ws: mh_attn_ws_bytes of device workspace (full attention splits K, rk and
// V into f16 planes there first; may be null when that is 0). xp, xpf (null,
// or when mh_attn_preps_out): the context written as the EXACT products'
// prepared input of the M = nseq T rows (xp: mh_mpad(M) * d * 4 bytes, xpf:
// mh_mpad(M) * d / 128 floats) instead of into ctx.
size_t mh_attn_ws_bytes(int T, int d, int H, int nseq, int left);
bool mh_attn_preps_out(int d, int H, int left);
hipError_t mh_launch_relpos_attn(const float *q, const float *k, const float *v, const float *rk,
                                 const float *bias_u, const float *bias_v, float *ctx, int T, int d, int H,
                                 int left, int right, int nseq, void *ws, uint8_t *xp, float *xpf,
                                 hipStream_t st);

// Encoder layer steps around the products (encoder.hip). d: 256 * {1..8, 12,
// 16} for the layer norm (mh_enc_d_supported), a multiple of 4 for the rest.
bool mh_enc_d_supported(int d);
// x += alpha * res (res may be null: no add), then out = LN(x) (w, b) per row;
// out may be x
hipError_t mh_launch_add_ln(float *x, const float *res, float alpha, const float *w, const float *b, float *out,
                            int rows, int d, hipStream_t st);
// the same, its output as the EXACT products' prepared input (xp: mh_mpad(rows)
// * d * 4 bytes, xpf: mh_mpad(rows) * d / 128 floats) in place of f32 rows;
// for d a multiple of 256 up to 2048
bool mh_add_ln_prep_supported(int d);
hipError_t mh_launch_add_ln_prep(float *x, const float *res, float alpha, const float *w, const float *b, int rows,
                                 int d, uint8_t *xp, float *xpf, hipStream_t st);
// g [rows, d] = h[:, :d] * sigmoid(h[:, d:]) for h [rows, 2d]
hipError_t mh_launch_glu(const float *h, float *g, size_t rows, int d, hipStream_t st);
// depthwise conv over time in each of nseq segments of T rows (w: the taps
// in the reference's order, [d, k]);
// causal: left pad k - 1, else (k - 1) / 2 per side), + bias (or null); with
// scale: silu(c * scale + shift)
hipError_t mh_launch_dwconv(const float *g, const float *w, const float *bias, const float *scale,
                            const float *shift, float *out, int T, int nseq, int d, int k, int causal,
                            hipStream_t st);
// GLU and the depthwise conv in one pass: h = pw1's output [rows][2d],
// g = h[:, :d] * sigmoid(h[:, d:]) formed as it is read (bit-identical to
// mh_launch_glu, then mh_launch_dwconv); for d a multiple of 256, k <= 16.
// xp, xpf (or null): the output as the EXACT products' prepared input
// (mh_mpad(M) * d * 4 bytes, mh_mpad(M) * d / 128 floats, M = nseq T) in
// place of out.
bool mh_glu_dwconv_supported(int d, int k);
hipError_t mh_launch_glu_dwconv(const float *h, const float *w, const float *bias, const float *scale,
                                const float *shift, float *out, int T, int nseq, int d, int k, int causal,
                                uint8_t *xp, float *xpf, hipStream_t st);

// The dw_striding subsampling's steps (encoder.hip), channel-last activations
// [segment][time][freq][channel] (C a multiple of 4); causal pads (2, 1),
// else (1, 1), in time and frequency alike.
int mh_ss_out_len(int n, int causal);   // the length after one stride-2 stage
// the first conv (1 -> C, + b0, ReLU) and the first depthwise conv (+ b1) in
// one pass: x [nseq][T][F] -> out [nseq][T2][F2][C]
hipError_t mh_launch_conv_in_dw(const float *x, const float *w0, const float *b0, const float *w1, const float *b1,
                                float *out, int nseq, int T, int F, int C, int causal, hipStream_t st);
// pb (or null): the previous pointwise conv's bias, applied with ReLU on load
hipError_t mh_launch_dw_s2(const float *in, const float *pb, const float *w, const float *b, float *out, int nseq,
                           int T, int F, int C, int causal, hipStream_t st);
hipError_t mh_launch_flatten(const float *in, const float *pb, float *flat, size_t rows, int Fo, int C,
                             hipStream_t st);
// wt [k][C] = the taps of w [C][k] tap-major (the layout k_conv_in_dw and
// k_dw_s2 read: w, the argument of their launchers, is this copy)
hipError_t mh_launch_transpose_taps(const float *w, float *wt, int C, int k, hipStream_t st);
// y = (y + b) * scale per row (scale 1: the bias alone)
hipError_t mh_launch_bias_scale(float *y, const float *b, size_t rows, int d, float scale, hipStream_t st);

// AED decoder step kernels (decoder.hip); st = device int[2]: position p, last argmax
int mh_att_splits(int n);   // attention splits for n keys
hipError_t mh_launch_embed_ln(const float *emb, const float *pos, const int *prompt, int n_prompt, const int *st,
                              const float *w, const float *b, float *x, int d, hipStream_t s);
// out = attention of q over n keys (n_fixed, or p + 1 with the cache append of kn, vn when n_fixed == 0);
// out == NULL: the splits only (merged by a GPRO_COMB prologue);
// o_part [H][nsplit][dk], ml_part [H][nsplit][2]
hipError_t mh_launch_attend1(const float *q, float *K, float *V, const float *kn, const float *vn, const int *st,
                             int n_fixed, int d, int H, float *o_part, float *ml_part, int nsplit, float *out,
                             hipStream_t s);
// The next position's input row, formed by the argmax kernel once it has the
// token: x = LN(emb[tok] + pos[q]) for q = p + 1 < max_pos, tok = prompt[q]
// while q < n_prompt, else the argmax (d <= 4096)
struct MhEmbNext {
    const float *emb, *pos;
    const int *prompt;
    int n_prompt, max_pos;
    const float *w, *b;
    float *x;
    int d;
};
// first maximum of the logits into st[1], st[0] advanced; logits_out (if not
// null) receives row p of the logits; en (if not null) as above
hipError_t mh_launch_argmax(const float *logits, int vocab, int *st, float *logits_out, const MhEmbNext *en,
                            hipStream_t s);
hipError_t mh_launch_bias_rows(float *y, const float *b, size_t rows, int d, hipStream_t s);
hipError_t mh_launch_set_state(int *st, int p, int cur, hipStream_t s);
