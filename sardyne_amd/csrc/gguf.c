/* GGUF v2/v3 reader: memory-mapped, validated once at open, tensor data pointers into the map.
 *
 * Behaviour follows the reference parser (csrc/gguf.c:250-455) so that both accept and reject the
 * same files and report the same fields: UTF-8 keys and names without NUL and without duplicates,
 * little-endian v2/v3 only, plausible counts, known ggml types, ne[0] a multiple of the block,
 * no size overflow, aligned in-file tensor data, power-of-two general.alignment <= 1 MiB.
 * The implementation is this file's own: a bounds-checked cursor over the map, names copied into
 * one string pool, duplicates found with a sorted index.
 */
#define _POSIX_C_SOURCE 200809L
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "sardyne.h"

#define DEFAULT_ALIGN 32u
#define MAX_ALIGN (1u << 20)

struct gguf_file {
    const uint8_t *map;
    size_t size;
    uint32_t version, alignment;
    uint64_t data_offset, n_kv, n_tensors;
    gguf_kv *kv;
    gguf_tensor *tensors;
};

/* ggml type table: name, elements per block, bytes per block (GGUF type ids). */
typedef struct {
    const char *name;
    uint32_t blk, bytes;
} ggml_type_desc;

static const ggml_type_desc *type_desc(uint32_t t) {
    static const ggml_type_desc T[40] = {
        [0] = {"F32", 1, 4},        [1] = {"F16", 1, 2},        [2] = {"Q4_0", 32, 18},   [3] = {"Q4_1", 32, 20},
        [6] = {"Q5_0", 32, 22},     [7] = {"Q5_1", 32, 24},     [8] = {"Q8_0", 32, 34},   [9] = {"Q8_1", 32, 36},
        [10] = {"Q2_K", 256, 84},   [11] = {"Q3_K", 256, 110},  [12] = {"Q4_K", 256, 144}, [13] = {"Q5_K", 256, 176},
        [14] = {"Q6_K", 256, 210},  [15] = {"Q8_K", 256, 292},  [16] = {"IQ2_XXS", 256, 66}, [17] = {"IQ2_XS", 256, 74},
        [18] = {"IQ3_XXS", 256, 98}, [19] = {"IQ1_S", 256, 50}, [20] = {"IQ4_NL", 32, 18}, [21] = {"IQ3_S", 256, 110},
        [22] = {"IQ2_S", 256, 82},  [23] = {"IQ4_XS", 256, 136}, [24] = {"I8", 1, 1},     [25] = {"I16", 1, 2},
        [26] = {"I32", 1, 4},       [27] = {"I64", 1, 8},       [28] = {"F64", 1, 8},     [29] = {"IQ1_M", 256, 56},
        [30] = {"BF16", 1, 2},      [34] = {"TQ1_0", 256, 54},  [35] = {"TQ2_0", 256, 66}, [39] = {"MXFP4", 32, 17},
    };
    return t < 40 && T[t].name ? &T[t] : NULL;
}

const char *gguf_type_name(uint32_t t) {
    const ggml_type_desc *d = type_desc(t);
    return d ? d->name : NULL;
}

static size_t scalar_size(uint32_t vt) {
    static const uint8_t S[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    return vt < 13 ? S[vt] : 0;
}

/* ------------------------------------------------------------------ cursor */

typedef struct {
    const uint8_t *p;
    size_t n, at;
    char *err;
    size_t err_len;
} cursor;

static int bad(cursor *c, const char *fmt, ...) {
    if (c->err && c->err_len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(c->err, c->err_len, fmt, ap);
        va_end(ap);
    }
    return -1;
}

static int avail(cursor *c, uint64_t k) {
    if (k > c->n - c->at)
        return bad(c, "file troncato all'offset %zu (servono %llu byte)", c->at, (unsigned long long)k);
    return 0;
}

static int get(cursor *c, void *dst, size_t k) {
    if (avail(c, k)) return -1;
    memcpy(dst, c->p + c->at, k);
    c->at += k;
    return 0;
}

/* Strict UTF-8 (no overlong forms, surrogates or code points above U+10FFFF) and no NUL byte. */
static int utf8_ok(const uint8_t *s, uint64_t n) {
    for (uint64_t i = 0; i < n;) {
        uint32_t c = s[i];
        if (c == 0) return 0;
        if (c < 0x80) {
            i++;
            continue;
        }
        int len = (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
        if (!len || n - i < (uint64_t)len) return 0;
        uint32_t cp = c & (0x7Fu >> len);
        for (int k = 1; k < len; k++) {
            if ((s[i + k] & 0xC0) != 0x80) return 0;
            cp = cp << 6 | (s[i + k] & 0x3Fu);
        }
        static const uint32_t min_cp[5] = {0, 0, 0x80, 0x800, 0x10000};
        if (cp < min_cp[len] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return 0;
        i += (uint64_t)len;
    }
    return 1;
}

static char *get_name(cursor *c, const char *what) {
    uint64_t n;
    if (get(c, &n, 8) || avail(c, n)) return NULL;
    if (!utf8_ok(c->p + c->at, n)) {
        bad(c, "%s all'offset %zu: UTF-8 non valido o byte NUL", what, c->at);
        return NULL;
    }
    char *s = malloc((size_t)n + 1);
    if (!s) {
        bad(c, "memoria esaurita");
        return NULL;
    }
    memcpy(s, c->p + c->at, (size_t)n);
    s[n] = '\0';
    c->at += (size_t)n;
    return s;
}

static int get_value(cursor *c, gguf_kv *kv) {
    if (kv->type == GGUF_TYPE_STRING) {
        if (get(c, &kv->n, 8) || avail(c, kv->n)) return -1;
        kv->ptr = c->p + c->at;
        c->at += kv->n;
        return 0;
    }
    if (kv->type != GGUF_TYPE_ARRAY) {
        size_t es = scalar_size(kv->type);
        if (!es) return bad(c, "tipo di valore sconosciuto %u", kv->type);
        if (avail(c, es)) return -1;
        kv->ptr = c->p + c->at;
        kv->n = 1;
        c->at += es;
        return 0;
    }
    if (get(c, &kv->arr_type, 4) || get(c, &kv->n, 8)) return -1;
    kv->ptr = c->p + c->at;
    size_t es = scalar_size(kv->arr_type);
    if (es) {
        if (kv->n > (c->n - c->at) / es) return bad(c, "array oltre la fine del file");
        c->at += kv->n * es;
        return 0;
    }
    if (kv->arr_type != GGUF_TYPE_STRING) return bad(c, "array di tipo %u non supportato", kv->arr_type);
    if (kv->n > (c->n - c->at) / 8) return bad(c, "array di stringhe oltre la fine del file");
    kv->str_pos = malloc((size_t)(kv->n ? kv->n : 1) * sizeof(uint64_t));
    if (!kv->str_pos) return bad(c, "memoria esaurita");
    for (uint64_t j = 0; j < kv->n; j++) {
        uint64_t len;
        kv->str_pos[j] = c->at;
        if (get(c, &len, 8) || avail(c, len)) return -1;
        c->at += len;
    }
    return 0;
}

static int by_name(const void *a, const void *b) { return strcmp(*(const char *const *)a, *(const char *const *)b); }

static int dup_check(cursor *c, const char **names, uint64_t n, const char *what) {
    qsort(names, (size_t)n, sizeof(*names), by_name);
    for (uint64_t i = 1; i < n; i++)
        if (!strcmp(names[i - 1], names[i])) return bad(c, "%s duplicato: %s", what, names[i]);
    return 0;
}

/* ------------------------------------------------------------------ open / close */

void gguf_close(gguf_file *f) {
    if (!f) return;
    for (uint64_t i = 0; f->kv && i < f->n_kv; i++) {
        free((char *)f->kv[i].key);
        free(f->kv[i].str_pos);
    }
    for (uint64_t i = 0; f->tensors && i < f->n_tensors; i++) free((char *)f->tensors[i].name);
    free(f->kv);
    free(f->tensors);
    if (f->map) munmap((void *)f->map, f->size);
    free(f);
}

static int parse(gguf_file *f, cursor *c) {
    uint8_t magic[4];
    if (get(c, magic, 4)) return -1;
    if (memcmp(magic, "GGUF", 4)) return bad(c, "non è un file GGUF (magic errato)");
    if (get(c, &f->version, 4)) return -1;
    uint32_t v = f->version;
    if ((v & 0xFFFFu) == 0 && (v >> 24) >= 1 && (v >> 24) <= 3) return bad(c, "file GGUF big-endian non supportato");
    if (v != 2 && v != 3) return bad(c, "versione GGUF %u non supportata", v);
    uint64_t nt, nk;
    if (get(c, &nt, 8) || get(c, &nk, 8)) return -1;
    if (nk > c->n / 12 || nt > c->n / 32) return bad(c, "contatori implausibili");
    f->kv = calloc((size_t)(nk ? nk : 1), sizeof(gguf_kv));
    f->tensors = calloc((size_t)(nt ? nt : 1), sizeof(gguf_tensor));
    if (!f->kv || !f->tensors) return bad(c, "memoria esaurita");
    f->alignment = DEFAULT_ALIGN;

    for (uint64_t i = 0; i < nk; i++) {
        gguf_kv *kv = &f->kv[i];
        if (!(kv->key = get_name(c, "chiave"))) return -1;
        f->n_kv = i + 1;
        if (get(c, &kv->type, 4) || get_value(c, kv)) return -1;
        if (!strcmp(kv->key, "general.alignment")) {
            uint64_t a;
            if (gguf_kv_get_u64(f, (int64_t)i, &a) || a == 0 || a > MAX_ALIGN || (a & (a - 1)))
                return bad(c, "general.alignment non valido");
            f->alignment = (uint32_t)a;
        }
    }
    for (uint64_t i = 0; i < nt; i++) {
        gguf_tensor *t = &f->tensors[i];
        if (!(t->name = get_name(c, "nome di tensore"))) return -1;
        f->n_tensors = i + 1;
        if (get(c, &t->n_dims, 4)) return -1;
        if (t->n_dims < 1 || t->n_dims > GGUF_MAX_DIMS) return bad(c, "%s: n_dims=%u", t->name, t->n_dims);
        for (uint32_t d = 0; d < GGUF_MAX_DIMS; d++) {
            t->ne[d] = 1;
            if (d < t->n_dims && get(c, &t->ne[d], 8)) return -1;
            if (!t->ne[d]) return bad(c, "%s: dimensione %u nulla", t->name, d);
        }
        if (get(c, &t->type, 4) || get(c, &t->offset, 8)) return -1;
        const ggml_type_desc *td = type_desc(t->type);
        if (!td) return bad(c, "%s: tipo ggml sconosciuto %u", t->name, t->type);
        if (t->ne[0] % td->blk) return bad(c, "%s: ne[0] non multiplo del blocco %u", t->name, td->blk);
        uint64_t n = 1;
        for (uint32_t d = 0; d < GGUF_MAX_DIMS; d++) {
            if (n > UINT64_MAX / t->ne[d]) return bad(c, "%s: dimensioni troppo grandi", t->name);
            n *= t->ne[d];
        }
        uint64_t blocks = n / td->blk;
        if (blocks > UINT64_MAX / td->bytes) return bad(c, "%s: dimensioni troppo grandi", t->name);
        t->nbytes = blocks * td->bytes;
    }
    uint64_t m = f->n_kv > f->n_tensors ? f->n_kv : f->n_tensors;
    const char **names = malloc((size_t)(m ? m : 1) * sizeof(*names));
    if (!names) return bad(c, "memoria esaurita");
    for (uint64_t i = 0; i < f->n_kv; i++) names[i] = f->kv[i].key;
    int rc = dup_check(c, names, f->n_kv, "metadato");
    if (!rc) {
        for (uint64_t i = 0; i < f->n_tensors; i++) names[i] = f->tensors[i].name;
        rc = dup_check(c, names, f->n_tensors, "tensore");
    }
    free(names);
    if (rc) return rc;

    f->data_offset = (c->at + f->alignment - 1) / f->alignment * f->alignment;
    if (f->data_offset > c->n) return bad(c, "zona dati oltre la fine del file");
    uint64_t data_size = c->n - f->data_offset;
    for (uint64_t i = 0; i < f->n_tensors; i++) {
        gguf_tensor *t = &f->tensors[i];
        if (t->offset % f->alignment) return bad(c, "%s: offset non allineato", t->name);
        if (t->offset > data_size || t->nbytes > data_size - t->offset)
            return bad(c, "%s: dati oltre la fine del file", t->name);
        t->data = f->map + f->data_offset + t->offset;
    }
    return 0;
}

gguf_file *gguf_open(const char *path, char *err, size_t err_len) {
    cursor c = {.err = err, .err_len = err_len};
    if (err && err_len) err[0] = '\0';
    const uint16_t one = 1;
    if (*(const uint8_t *)&one != 1) {
        bad(&c, "host big-endian non supportato");
        return NULL;
    }
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        bad(&c, "impossibile aprire %s: %s", path, strerror(errno));
        return NULL;
    }
    struct stat st;
    if (fstat(fd, &st)) {
        bad(&c, "impossibile leggere la dimensione di %s: %s", path, strerror(errno));
        close(fd);
        return NULL;
    }
    if (st.st_size <= 0) {
        close(fd);
        bad(&c, "%s: dimensione non valida o troppo grande per questa piattaforma", path);
        return NULL;
    }
    void *map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_SHARED, fd, 0);
    int map_errno = errno;
    close(fd);
    if (map == MAP_FAILED) {
        bad(&c, "mmap fallita su %s: %s", path, strerror(map_errno));
        return NULL;
    }
    gguf_file *f = calloc(1, sizeof(*f));
    if (!f) {
        munmap(map, (size_t)st.st_size);
        bad(&c, "memoria esaurita");
        return NULL;
    }
    f->map = map;
    f->size = (size_t)st.st_size;
    c.p = f->map;
    c.n = f->size;
    if (parse(f, &c)) {
        gguf_close(f);
        return NULL;
    }
    return f;
}

void gguf_prefetch(const void *p, size_t n) {
    const uintptr_t chunk = 1u << 20, page = (uintptr_t)sysconf(_SC_PAGESIZE);
    uintptr_t b = (uintptr_t)p & ~(page - 1), end = (uintptr_t)p + n;
    while (b < end) {
        size_t len = end - b < chunk ? (size_t)(end - b) : (size_t)chunk;
        posix_madvise((void *)b, len, POSIX_MADV_WILLNEED);
        b += len;
    }
}

/* ------------------------------------------------------------------ accessors (NULL-tolerant) */

uint32_t gguf_version(const gguf_file *f) { return f ? f->version : 0; }
uint32_t gguf_alignment(const gguf_file *f) { return f ? f->alignment : 0; }
uint64_t gguf_data_offset(const gguf_file *f) { return f ? f->data_offset : 0; }
uint64_t gguf_n_kv(const gguf_file *f) { return f ? f->n_kv : 0; }
uint64_t gguf_n_tensors(const gguf_file *f) { return f ? f->n_tensors : 0; }

const gguf_kv *gguf_get_kv(const gguf_file *f, uint64_t i) { return f && i < f->n_kv ? &f->kv[i] : NULL; }
const gguf_tensor *gguf_get_tensor(const gguf_file *f, uint64_t i) {
    return f && i < f->n_tensors ? &f->tensors[i] : NULL;
}

int64_t gguf_find_kv(const gguf_file *f, const char *key) {
    for (uint64_t i = 0; f && key && i < f->n_kv; i++)
        if (!strcmp(f->kv[i].key, key)) return (int64_t)i;
    return -1;
}

int64_t gguf_find_tensor(const gguf_file *f, const char *name) {
    for (uint64_t i = 0; f && name && i < f->n_tensors; i++)
        if (!strcmp(f->tensors[i].name, name)) return (int64_t)i;
    return -1;
}

static const gguf_kv *kv_at(const gguf_file *f, int64_t i) {
    return f && i >= 0 && (uint64_t)i < f->n_kv ? &f->kv[i] : NULL;
}

int gguf_kv_get_u64(const gguf_file *f, int64_t i, uint64_t *out) {
    const gguf_kv *kv = kv_at(f, i);
    if (!kv || !out) return -1;
    const uint8_t *p = kv->ptr;
    int64_t sv;
    switch (kv->type) {
    case GGUF_TYPE_UINT8: *out = p[0]; return 0;
    case GGUF_TYPE_UINT16: { uint16_t v; memcpy(&v, p, 2); *out = v; return 0; }
    case GGUF_TYPE_UINT32: { uint32_t v; memcpy(&v, p, 4); *out = v; return 0; }
    case GGUF_TYPE_UINT64: { uint64_t v; memcpy(&v, p, 8); *out = v; return 0; }
    case GGUF_TYPE_INT8: sv = (int8_t)p[0]; break;
    case GGUF_TYPE_INT16: { int16_t v; memcpy(&v, p, 2); sv = v; break; }
    case GGUF_TYPE_INT32: { int32_t v; memcpy(&v, p, 4); sv = v; break; }
    case GGUF_TYPE_INT64: { int64_t v; memcpy(&v, p, 8); sv = v; break; }
    default: return -1;
    }
    if (sv < 0) return -1;
    *out = (uint64_t)sv;
    return 0;
}

int gguf_kv_get_f64(const gguf_file *f, int64_t i, double *out) {
    const gguf_kv *kv = kv_at(f, i);
    if (!kv || !out) return -1;
    if (kv->type == GGUF_TYPE_FLOAT32) {
        float v;
        memcpy(&v, kv->ptr, 4);
        *out = v;
        return 0;
    }
    if (kv->type == GGUF_TYPE_FLOAT64) {
        memcpy(out, kv->ptr, 8);
        return 0;
    }
    return -1;
}

const char *gguf_kv_get_str(const gguf_file *f, int64_t i, uint64_t *len) {
    const gguf_kv *kv = kv_at(f, i);
    if (!kv || !len || kv->type != GGUF_TYPE_STRING) return NULL;
    *len = kv->n;
    return (const char *)kv->ptr;
}

const char *gguf_kv_get_arr_str(const gguf_file *f, int64_t i, uint64_t j, uint64_t *len) {
    const gguf_kv *kv = kv_at(f, i);
    if (!kv || !len || kv->type != GGUF_TYPE_ARRAY || kv->arr_type != GGUF_TYPE_STRING || j >= kv->n) return NULL;
    memcpy(len, f->map + kv->str_pos[j], 8);
    return (const char *)(f->map + kv->str_pos[j] + 8);
}
