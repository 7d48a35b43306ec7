/* oracle.h — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference CPU path for the encoder/decoder
 * linear layers of mynah-asr: the ggml block decoders and quantizers of the
 * vendored ingot library, the qmat INT8/INT4 quantizers, the qmat small-T
 * int8 dot path and a double-accumulated reference GEMM.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker. The product (the HIP backend and the
 * C host mirror) never links it.
 *
 * Parity status of each function (how it is pinned) is recorded next to its
 * definition in oracle.c. Block type ids are the GGML ids used by the
 * reference's fixtures (third_party/ingot/tests/fixtures/manifest.txt):
 * F32 0, Q4_0 2, Q8_0 8, Q2_K 10, Q3_K 11, Q4_K 12, Q5_K 13, Q6_K 14. */
#ifndef MYNAH_ORACLE_H
#define MYNAH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

enum {
    ORC_F32 = 0, ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q2_K = 10, ORC_Q3_K = 11,
    ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14
};

/* geometry: elements and bytes per block; -1 for an unknown type */
int orc_geometry(int type, int *block_elems, int *block_bytes);

float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* f32 -> blocks (Q8_0, Q4_0, Q4_K, Q6_K); count multiple of the block size */
int orc_quantize(int type, const float *x, size_t count, void *out);
/* blocks -> f32 (Q4_0, Q8_0, Q2_K..Q6_K, F32) */
int orc_dequant(int type, const void *src, size_t count, float *dst);

/* qmat per-row INT8 / group-32 INT4 (qmat.c:19-67, 152-169) */
void orc_qmat_quantize_int8(const float *w, int n, int k, int8_t *q, float *scales);
void orc_qmat_quantize_int4(const float *w, int n, int k, uint8_t *q, float *scales);
/* qtype 1 = INT8, 2 = INT4 */
void orc_qmat_dequant(int qtype, const void *q, const float *scales, int n, int k, float *wd);

/* per-row activation quantization (qmat.c:186-202); returns the scale */
float orc_act_quant_int8(const float *x, int k, int8_t *qx);

/* The qmat small-T int8 path (qmat.c:508-552) for every row t < T:
 * INT8: out = (float)s * ws * sx; INT4: acc += (float)ig * sg; out = acc * sx.
 * int_sums (optional, may be NULL) receives the exact int32 sums:
 * INT8 [T, n]; INT4 [T, n, k/32]. */
void orc_qmat_int8_path(int qtype, const void *q, const float *scales, int n, int k,
                        const float *x, int T, float *out, int32_t *int_sums);

/* K-quant super-block as integers (quants with offsets, sub-block factors
 * and mins, d, dmin); 0 or -1 for other types */
int orc_kquant_ints(int type, const void *block, int32_t *q, int32_t *f, int32_t *m, float *d, float *dmin);
/* ingot's per-super-block int8 activation quantizer (256 values); returns the scale */
float orc_act_quant_sb(const float *x, int8_t *qx);
/* INT8ACT over ggml blocks in the HIP unit's evaluation order (see oracle.c);
 * chunk_ints (optional) [T, n, k/128, 2] = the K-quants' exact chunk integers */
void orc_int8act_blocks(int type, const void *blocks, int n, int k, const float *x, int T, float *out,
                        int64_t *chunk_ints);

/* out[T, n] = x[T, k] . wd[n, k]^T accumulated in double (threads: 0 = all) */
void orc_gemm_f64(const float *x, const float *wd, int T, int n, int k, double *out,
                  int threads);

/* install a pthread parallel_for of `threads` ranges into an ingot build
 * (set_parallel_for = that library's ingot_set_parallel_for) */
void orc_ingot_install_pool(void *set_parallel_for, int threads);

#endif
