/* gguf.c — read-only GGUF mapping (see gguf.h). Every read is bounds-checked
 * against the file size; a malformed file is refused with a message, never read
 * past its end. The GGUF layout follows the published format, as ingot's reader
 * parses it (third_party/ingot/src/gguf.c:141-246 KV pairs, :298-465 tensor
 * table and data section). */
#define _DEFAULT_SOURCE
#include "gguf.h"

#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

struct mynah_gguf {
    void *map;
    size_t size;
    uint32_t version;
    uint64_t alignment;
    size_t count;
    mynah_gguf_tensor *t;
    char *names;   /* all tensor names, NUL-terminated, back to back */
};

typedef struct {
    const unsigned char *p;
    size_t off, size;
} cur_t;

static int seterr(char *err, size_t errsz, const char *fmt, ...) {
    if (err && errsz) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, errsz, fmt, ap);
        va_end(ap);
    }
    return -1;
}

static int take(cur_t *c, uint64_t n, const unsigned char **out) {
    if (n > c->size - c->off) return -1;
    *out = c->p + c->off;
    c->off += (size_t)n;
    return 0;
}

static int rd_u32(cur_t *c, uint32_t *v) {
    const unsigned char *b;
    if (take(c, 4, &b)) return -1;
    memcpy(v, b, 4);   /* GGUF is little-endian, as this host */
    return 0;
}

static int rd_u64(cur_t *c, uint64_t *v) {
    const unsigned char *b;
    if (take(c, 8, &b)) return -1;
    memcpy(v, b, 8);
    return 0;
}

static int rd_str(cur_t *c, const char **s, uint64_t *len) {
    const unsigned char *b;
    if (rd_u64(c, len) || take(c, *len, &b)) return -1;
    *s = (const char *)b;
    return 0;
}

/* KV value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool,
 * 8 string, 9 array, 10 u64, 11 i64, 12 f64 */
static int scalar_bytes(uint32_t type) {
    switch (type) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return -1;
    }
}

/* skip one KV value of `type` (an array of arrays is refused) */
static int skip_value(cur_t *c, uint32_t type, int depth) {
    const unsigned char *b;
    if (type == 8) {
        const char *s;
        uint64_t n;
        return rd_str(c, &s, &n);
    }
    if (type == 9) {
        uint32_t et;
        uint64_t n;
        if (depth > 0 || rd_u32(c, &et) || rd_u64(c, &n)) return -1;
        if (et == 8 || et == 9) {
            for (uint64_t i = 0; i < n; i++)
                if (skip_value(c, et, depth + 1)) return -1;
            return 0;
        }
        const int sb = scalar_bytes(et);
        if (sb < 0 || n > (c->size - c->off) / (uint64_t)sb) return -1;
        return take(c, n * (uint64_t)sb, &b);
    }
    const int sb = scalar_bytes(type);
    return sb < 0 ? -1 : take(c, (uint64_t)sb, &b);
}

/* bytes of `nelem` elements of ggml `type` (0 when not sized here, UINT64_MAX when
 * beyond 64 bits) */
static uint64_t type_nbytes(int type, uint64_t nelem) {
    uint64_t bs = 0, be = 1;
    switch (type) {
    case 0: bs = 4; break;                  /* F32 */
    case 1: bs = 2; break;                  /* F16 */
    case 2: bs = 18; be = 32; break;        /* Q4_0 */
    case 3: bs = 20; be = 32; break;        /* Q4_1 */
    case 6: bs = 22; be = 32; break;        /* Q5_0 */
    case 7: bs = 24; be = 32; break;        /* Q5_1 */
    case 8: bs = 34; be = 32; break;        /* Q8_0 */
    case 9: bs = 36; be = 32; break;        /* Q8_1 */
    case 10: bs = 84; be = 256; break;      /* Q2_K */
    case 11: bs = 110; be = 256; break;     /* Q3_K */
    case 12: bs = 144; be = 256; break;     /* Q4_K */
    case 13: bs = 176; be = 256; break;     /* Q5_K */
    case 14: bs = 210; be = 256; break;     /* Q6_K */
    case 15: bs = 292; be = 256; break;     /* Q8_K */
    case 24: bs = 1; break;                 /* I8 */
    case 25: bs = 2; break;                 /* I16 */
    case 26: bs = 4; break;                 /* I32 */
    case 27: bs = 8; break;                 /* I64 */
    case 28: bs = 8; break;                 /* F64 */
    case 30: bs = 2; break;                 /* BF16 */
    default: return 0;
    }
    if (nelem % be) return 0;
    /* a size past 2^64 cannot lie inside any file: UINT64_MAX fails the bounds check */
    if (nelem / be > UINT64_MAX / bs) return UINT64_MAX;
    return nelem / be * bs;
}

void mynah_gguf_close(mynah_gguf *g) {
    if (!g) return;
    if (g->map && g->map != MAP_FAILED) munmap(g->map, g->size);
    free(g->t);
    free(g->names);
    free(g);
}

mynah_gguf *mynah_gguf_open(const char *path, char *err, size_t errsz) {
    mynah_gguf *g = calloc(1, sizeof(*g));
    if (!g) { seterr(err, errsz, "out of memory"); return NULL; }
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { seterr(err, errsz, "cannot open %s", path); free(g); return NULL; }
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 24) {
        close(fd);
        seterr(err, errsz, "%s: too short for a GGUF header", path);
        free(g);
        return NULL;
    }
    g->size = (size_t)sb.st_size;
    g->map = mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (g->map == MAP_FAILED) { seterr(err, errsz, "%s: mmap failed", path); g->map = NULL; mynah_gguf_close(g); return NULL; }

    cur_t c = {(const unsigned char *)g->map, 0, g->size};
    uint32_t magic;
    uint64_t nt, nkv;
    if (rd_u32(&c, &magic) || memcmp(&magic, "GGUF", 4) != 0) {
        seterr(err, errsz, "%s: not a GGUF file", path);
        goto fail;
    }
    if (rd_u32(&c, &g->version) || (g->version != 2 && g->version != 3)) {
        seterr(err, errsz, "%s: GGUF version %u not supported (2, 3)", path, g->version);
        goto fail;
    }
    if (rd_u64(&c, &nt) || rd_u64(&c, &nkv)) { seterr(err, errsz, "%s: truncated header", path); goto fail; }
    g->alignment = 32;
    for (uint64_t i = 0; i < nkv; i++) {
        const char *key;
        uint64_t klen;
        uint32_t type;
        if (rd_str(&c, &key, &klen) || rd_u32(&c, &type)) { seterr(err, errsz, "%s: truncated KV %llu", path, (unsigned long long)i); goto fail; }
        if (klen == 17 && memcmp(key, "general.alignment", 17) == 0 && type == 4) {
            uint32_t a;
            if (rd_u32(&c, &a)) { seterr(err, errsz, "%s: truncated alignment", path); goto fail; }
            if (a == 0 || (a & (a - 1))) { seterr(err, errsz, "%s: alignment %u is not a power of two", path, a); goto fail; }
            g->alignment = a;
            continue;
        }
        if (skip_value(&c, type, 0)) { seterr(err, errsz, "%s: bad or truncated KV value (type %u)", path, type); goto fail; }
    }
    /* each tensor info takes at least 8 (name length) + 4 + 4 + 8 bytes */
    if (nt > (c.size - c.off) / 24) { seterr(err, errsz, "%s: tensor count %llu does not fit the file", path, (unsigned long long)nt); goto fail; }
    g->count = (size_t)nt;
    g->t = calloc(g->count ? g->count : 1, sizeof(*g->t));
    size_t names_len = 0;
    uint64_t *offs = calloc(g->count ? g->count : 1, sizeof(uint64_t));
    const char **nm = calloc(g->count ? g->count : 1, sizeof(char *));
    uint64_t *nl = calloc(g->count ? g->count : 1, sizeof(uint64_t));
    if (!g->t || !offs || !nm || !nl) { free(offs); free(nm); free(nl); seterr(err, errsz, "out of memory"); goto fail; }
    for (size_t i = 0; i < g->count; i++) {
        mynah_gguf_tensor *t = &g->t[i];
        uint32_t rank, type;
        if (rd_str(&c, &nm[i], &nl[i]) || rd_u32(&c, &rank)) goto bad_info;
        if (rank == 0 || rank > MYNAH_GGUF_MAX_RANK) {
            free(offs); free(nm); free(nl);
            seterr(err, errsz, "%s: tensor %zu has rank %u (1..%d)", path, i, rank, MYNAH_GGUF_MAX_RANK);
            goto fail;
        }
        uint64_t nelem = 1;
        for (uint32_t d = 0; d < MYNAH_GGUF_MAX_RANK; d++) t->ne[d] = 1;
        for (uint32_t d = 0; d < rank; d++) {
            uint64_t ne;
            if (rd_u64(&c, &ne) || ne == 0 || ne > INT64_MAX || (nelem && ne > UINT64_MAX / nelem)) goto bad_info;
            t->ne[d] = (int64_t)ne;
            nelem *= ne;
        }
        if (rd_u32(&c, &type) || rd_u64(&c, &offs[i])) goto bad_info;
        t->rank = (int)rank;
        t->ggml_type = (int)type;
        t->nbytes = type_nbytes((int)type, nelem);
        names_len += (size_t)nl[i] + 1;
        continue;
    bad_info:
        free(offs); free(nm); free(nl);
        seterr(err, errsz, "%s: bad or truncated tensor info %zu", path, i);
        goto fail;
    }
    /* data section: the next multiple of the alignment after the infos */
    const uint64_t data0 = ((uint64_t)c.off + g->alignment - 1) / g->alignment * g->alignment;
    g->names = malloc(names_len ? names_len : 1);
    if (!g->names) { free(offs); free(nm); free(nl); seterr(err, errsz, "out of memory"); goto fail; }
    size_t np = 0;
    for (size_t i = 0; i < g->count; i++) {
        mynah_gguf_tensor *t = &g->t[i];
        memcpy(g->names + np, nm[i], (size_t)nl[i]);
        g->names[np + nl[i]] = 0;
        t->name = g->names + np;
        np += (size_t)nl[i] + 1;
        const uint64_t start = data0 + offs[i];
        if (offs[i] % g->alignment || start < data0 || start > g->size || t->nbytes > g->size - start) {
            seterr(err, errsz, "%s: tensor '%s' lies outside the file or off the alignment", path, t->name);
            free(offs); free(nm); free(nl);
            goto fail;
        }
        t->data = (const unsigned char *)g->map + start;
    }
    free(offs); free(nm); free(nl);
    return g;
fail:
    mynah_gguf_close(g);
    return NULL;
}

uint32_t mynah_gguf_version(const mynah_gguf *g) { return g ? g->version : 0; }
uint64_t mynah_gguf_alignment(const mynah_gguf *g) { return g ? g->alignment : 0; }
size_t mynah_gguf_count(const mynah_gguf *g) { return g ? g->count : 0; }

const mynah_gguf_tensor *mynah_gguf_at(const mynah_gguf *g, size_t i) {
    return g && i < g->count ? &g->t[i] : NULL;
}

const mynah_gguf_tensor *mynah_gguf_find(const mynah_gguf *g, const char *name) {
    if (!g || !name) return NULL;
    for (size_t i = 0; i < g->count; i++)
        if (strcmp(g->t[i].name, name) == 0) return &g->t[i];
    return NULL;
}

/* IEEE binary16 -> binary32, exact for every input (subnormals normalised,
 * inf / NaN kept) */
static float half_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    int e = (int)((h >> 10) & 31);
    uint32_t mant = h & 0x3ffu, b;
    if (e == 0) {
        if (mant == 0) b = sign;
        else {
            e = 1;
            while (!(mant & 0x400u)) { mant <<= 1; e--; }
            b = sign | ((uint32_t)(e + 112) << 23) | ((mant & 0x3ffu) << 13);
        }
    } else if (e == 31) b = sign | 0x7f800000u | (mant << 13);
    else b = sign | ((uint32_t)(e + 112) << 23) | (mant << 13);
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* bfloat16 is the top half of a binary32 */
static float bf16_to_f32(uint32_t h) {
    const uint32_t b = h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

int mynah_asr_qmat_init_gguf(mynah_asr_qmat *m, const mynah_gguf *g, const char *name) {
    memset(m, 0, sizeof(*m));
    const mynah_gguf_tensor *t = mynah_gguf_find(g, name);
    if (!t || t->rank != 2 || t->nbytes == 0 || t->ne[0] > INT32_MAX || t->ne[1] > INT32_MAX) return -1;
    const int k = (int)t->ne[0], n = (int)t->ne[1];
    if (t->ggml_type == 0) {                 /* F32: borrowed, as qmat_init with F32 */
        m->f32 = (const float *)t->data;
        m->qtype = MYNAH_ASR_Q_F32;
        m->n = n;
        m->k = k;
        return 0;
    }
    if (t->ggml_type == 1 || t->ggml_type == 30) {
        /* F16 / BF16: decoded to an owned f32 copy at load, as the reference's
         * loader does for every non-F32 GGUF tensor (src/weights.c:90-104) */
        const size_t ne = (size_t)n * (size_t)k;
        if (t->nbytes < ne * 2) return -1;
        float *f = (float *)malloc(ne * sizeof(float));
        if (!f) return -1;
        const unsigned char *p = (const unsigned char *)t->data;
        for (size_t i = 0; i < ne; i++) {
            const uint32_t h = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 8);
            f[i] = t->ggml_type == 1 ? half_to_f32(h) : bf16_to_f32(h);
        }
        m->owned_q = f;
        m->f32 = f;
        m->qtype = MYNAH_ASR_Q_F32;
        m->n = n;
        m->k = k;
        return 0;
    }
    /* block qtypes are 16 + the GGML type id */
    return mynah_asr_qmat_init_blocks(m, t->data, n, k, 16 + t->ggml_type);
}
