/* gguf.h — a read-only GGUF (v2, v3) mapping for the host mirror, so GGUF block
 * tensors reach the device as raw blocks instead of the reference's decode to
 * f32 at load (src/weights.c:82-116, through third_party/ingot/src/gguf.c).
 *
 * The file is mapped read-only; tensor data pointers point into the mapping and
 * stay valid until mynah_gguf_close(). Layout (GGUF v3, also read by v2):
 *   magic "GGUF", u32 version, u64 tensor count, u64 KV count,
 *   KV pairs (string key, u32 type, value; arrays: u32 element type, u64 count),
 *   tensor infos (string name, u32 rank, u64 ne[rank] with ne[0] fastest,
 *   u32 ggml type, u64 offset), then the data section at the next multiple of
 *   general.alignment (32 when absent); tensor i at data + offset_i. */
#ifndef MYNAH_GGUF_H
#define MYNAH_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "qmat.h"

#ifdef __cplusplus
extern "C" {
#endif

#define MYNAH_GGUF_MAX_RANK 4

typedef struct {
    const char *name;
    int ggml_type;                    /* GGML type id (0 F32, 8 Q8_0, 12 Q4_K, ...) */
    int rank;
    int64_t ne[MYNAH_GGUF_MAX_RANK];  /* ggml order: ne[0] is the fastest dimension */
    const void *data;                 /* inside the mapping */
    uint64_t nbytes;                  /* 0 for a type this reader does not size */
} mynah_gguf_tensor;

typedef struct mynah_gguf mynah_gguf;

/* NULL on failure, with the reason in err (if given). */
mynah_gguf *mynah_gguf_open(const char *path, char *err, size_t errsz);
void mynah_gguf_close(mynah_gguf *g);
uint32_t mynah_gguf_version(const mynah_gguf *g);
uint64_t mynah_gguf_alignment(const mynah_gguf *g);
size_t mynah_gguf_count(const mynah_gguf *g);
const mynah_gguf_tensor *mynah_gguf_at(const mynah_gguf *g, size_t i);
const mynah_gguf_tensor *mynah_gguf_find(const mynah_gguf *g, const char *name);

/* The qmat_init_st of a GGUF (src/qmat.c:114-143 for safetensors): a 2-D
 * tensor [n, k] (ne = {k, n}) of a block type the unit runs (Q4_0, Q8_0,
 * Q2_K..Q6_K) becomes a block qmat over the mapped bytes (zero-copy, borrowed:
 * the mapping must outlive m); an F32 tensor becomes an F32 qmat (borrowed);
 * an F16 or BF16 tensor is decoded to an owned f32 copy (src/weights.c:90-104
 * decodes every non-F32 GGUF tensor at load), freed by mynah_asr_qmat_free.
 * 0 ok, -1 missing or unsupported. */
int mynah_asr_qmat_init_gguf(mynah_asr_qmat *m, const mynah_gguf *g, const char *name);

#ifdef __cplusplus
}
#endif

#endif
