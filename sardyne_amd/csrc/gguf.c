/* GGUF v2/v3 reader: the file is memory-mapped read-only, its header is scanned and validated once
 * at open, and tensor data pointers point into the map (no copy).
 *
 * Accepted files (the contract of the reference reader, csrc/gguf.h:4-17, so that both take and
 * refuse the same files): little-endian GGUF version 2 or 3; keys and tensor names valid UTF-8
 * without NUL and without duplicates; scalar, string, scalar-array and string-array values;
 * general.alignment, when present, an integer power of two <= 1 MiB; tensors of 1..4 non-zero
 * dimensions of a known ggml type, ne[0] a multiple of the type's block, sizes without overflow,
 * data aligned and inside the file.
 *
 * How this reader is organised:
 *   - one forward scan over the header with a bounds-checked cursor. Scalars are decoded from
 *     little-endian bytes explicitly, so the host byte order does not matter;
 *   - the scan grows its kv and tensor tables as entries are read, so a hostile count costs
 *     nothing until the bytes that back it are actually present;
 *   - keys and names are recorded as offsets into the map. When the scan ends they are copied
 *     into one pool of NUL-terminated strings, and every string-array element position goes into
 *     one shared table;
 *   - an open-addressing hash index (FNV-1a) over keys and names finds duplicates while it is
 *     built, and serves gguf_find_kv / gguf_find_tensor in O(1).
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

enum { ALIGN_DEFAULT = 32, ALIGN_MAX = 1 << 20 };

/* ggml type ids -> name, elements per block, bytes per block (the GGUF type table, csrc/gguf.c:30-43). */
typedef struct {
    const char *name;
    uint16_t per_block, block_bytes;
} ggml_type;

static const ggml_type GGML[] = {
    [0] = {"F32", 1, 4},        [1] = {"F16", 1, 2},        [2] = {"Q4_0", 32, 18},    [3] = {"Q4_1", 32, 20},
    [6] = {"Q5_0", 32, 22},     [7] = {"Q5_1", 32, 24},     [8] = {"Q8_0", 32, 34},    [9] = {"Q8_1", 32, 36},
    [10] = {"Q2_K", 256, 84},   [11] = {"Q3_K", 256, 110},  [12] = {"Q4_K", 256, 144}, [13] = {"Q5_K", 256, 176},
    [14] = {"Q6_K", 256, 210},  [15] = {"Q8_K", 256, 292},  [16] = {"IQ2_XXS", 256, 66},
    [17] = {"IQ2_XS", 256, 74}, [18] = {"IQ3_XXS", 256, 98}, [19] = {"IQ1_S", 256, 50}, [20] = {"IQ4_NL", 32, 18},
    [21] = {"IQ3_S", 256, 110}, [22] = {"IQ2_S", 256, 82},  [23] = {"IQ4_XS", 256, 136}, [24] = {"I8", 1, 1},
    [25] = {"I16", 1, 2},       [26] = {"I32", 1, 4},       [27] = {"I64", 1, 8},      [28] = {"F64", 1, 8},
    [29] = {"IQ1_M", 256, 56},  [30] = {"BF16", 1, 2},      [34] = {"TQ1_0", 256, 54}, [35] = {"TQ2_0", 256, 66},
    [39] = {"MXFP4", 32, 17},
};

const char *gguf_type_name(uint32_t t) {
    return t < sizeof GGML / sizeof *GGML ? GGML[t].name : NULL;
}

/* Byte width of a scalar value type; 0 for strings, arrays and unknown types. */
static unsigned scalar_width(uint32_t vt) {
    static const unsigned char W[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    return vt < 13 ? W[vt] : 0;
}

static uint64_t le_bytes(const uint8_t *p, unsigned n) {
    uint64_t v = 0;
    while (n--) v = v << 8 | p[n];
    return v;
}

/* Strict UTF-8 without NUL: no overlong forms, no surrogates, nothing above U+10FFFF. */
static int utf8_clean(const uint8_t *s, uint64_t n) {
    static const uint32_t least[4] = {0, 0x80, 0x800, 0x10000};
    for (uint64_t i = 0; i < n;) {
        uint32_t c = s[i];
        if (c >= 1 && c < 0x80) {
            i++;
            continue;
        }
        if (c < 0xC0 || c > 0xF4) return 0; /* NUL, a stray continuation byte, or no valid lead */
        unsigned more = c >= 0xF0 ? 3 : c >= 0xE0 ? 2 : 1;
        if (n - i <= more) return 0;
        uint32_t cp = c & (0x3Fu >> more);
        for (unsigned k = 1; k <= more; k++) {
            uint32_t b = s[i + k];
            if ((b & 0xC0) != 0x80) return 0;
            cp = cp << 6 | (b & 0x3F);
        }
        if (cp < least[more] || cp > 0x10FFFF || (cp >> 11) == 0x1B) return 0;
        i += more + 1;
    }
    return 1;
}

/* ------------------------------------------------------------------ file state */

typedef struct {
    uint64_t at, len;
} span; /* a byte range of the map */

typedef struct {
    uint64_t *slot; /* entry index + 1, 0 = empty */
    uint64_t mask;
} name_index;

struct gguf_file {
    const uint8_t *map;
    size_t size;
    uint32_t version, alignment;
    uint64_t data_offset, n_kv, n_tensors;
    gguf_kv *kv;
    gguf_tensor *tensors;
    char *pool;          /* every key and tensor name, NUL-terminated */
    uint64_t *positions; /* element positions of every string array */
    name_index kv_idx, t_idx;
};

/* ------------------------------------------------------------------ scanning */

typedef struct {
    const uint8_t *base;
    uint64_t size, at;
    char *err;
    size_t err_len;
    /* recorded during the scan, resolved to pointers afterwards */
    span *kv_name, *t_name;
    uint64_t *arr_first;    /* string arrays: index of their first position */
    uint64_t *pos;
    uint64_t n_pos, cap_pos, cap_kv, cap_t, pool_bytes;
} scan;

static int complain(scan *s, const char *fmt, ...) {
    if (s->err && s->err_len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(s->err, s->err_len, fmt, ap);
        va_end(ap);
    }
    return -1;
}

/* Pointer to the next n bytes, or NULL (and the error) when the file ends first. */
static const uint8_t *take(scan *s, uint64_t n) {
    if (n > s->size - s->at) {
        complain(s, "file troncato all'offset %llu (servono %llu byte)", (unsigned long long)s->at,
                 (unsigned long long)n);
        return NULL;
    }
    const uint8_t *p = s->base + s->at;
    s->at += n;
    return p;
}

static int take_u32(scan *s, uint32_t *v) {
    const uint8_t *p = take(s, 4);
    if (p) *v = (uint32_t)le_bytes(p, 4);
    return p ? 0 : -1;
}

static int take_u64(scan *s, uint64_t *v) {
    const uint8_t *p = take(s, 8);
    if (p) *v = le_bytes(p, 8);
    return p ? 0 : -1;
}

/* Makes room for entry i of the kv tables (f->kv, the recorded key spans, the string-array first
 * positions) or of the tensor tables; capacities double, so a hostile count costs nothing until
 * the bytes behind its entries have been read. */
static int grow_kv(scan *s, gguf_file *f, uint64_t i) {
    if (i < s->cap_kv) return 0;
    const uint64_t c = s->cap_kv ? 2 * s->cap_kv : 16;
    gguf_kv *kv = realloc(f->kv, c * sizeof *kv);
    if (kv) f->kv = kv;
    span *kn = kv ? realloc(s->kv_name, c * sizeof *kn) : NULL;
    if (kn) s->kv_name = kn;
    uint64_t *af = kn ? realloc(s->arr_first, c * sizeof *af) : NULL;
    if (af) s->arr_first = af;
    if (!af) return complain(s, "memoria esaurita");
    s->cap_kv = c;
    return 0;
}

static int grow_tensors(scan *s, gguf_file *f, uint64_t i) {
    if (i < s->cap_t) return 0;
    const uint64_t c = s->cap_t ? 2 * s->cap_t : 16;
    gguf_tensor *t = realloc(f->tensors, c * sizeof *t);
    if (t) f->tensors = t;
    span *tn = t ? realloc(s->t_name, c * sizeof *tn) : NULL;
    if (tn) s->t_name = tn;
    if (!tn) return complain(s, "memoria esaurita");
    s->cap_t = c;
    return 0;
}

static int push_position(scan *s, uint64_t at) {
    if (s->n_pos == s->cap_pos) {
        const uint64_t c = s->cap_pos ? 2 * s->cap_pos : 64;
        uint64_t *p = realloc(s->pos, c * sizeof *p);
        if (!p) return complain(s, "memoria esaurita");
        s->pos = p;
        s->cap_pos = c;
    }
    s->pos[s->n_pos++] = at;
    return 0;
}

static int take_name(scan *s, span *out, const char *what) {
    uint64_t n;
    if (take_u64(s, &n)) return -1;
    uint64_t at = s->at;
    const uint8_t *p = take(s, n);
    if (!p) return -1;
    if (!utf8_clean(p, n)) return complain(s, "%s all'offset %llu: UTF-8 non valido o byte NUL", what,
                                           (unsigned long long)at);
    out->at = at;
    out->len = n;
    s->pool_bytes += n + 1;
    return 0;
}

static int take_value(scan *s, gguf_file *f, uint64_t i) {
    gguf_kv *kv = &f->kv[i];
    if (take_u32(s, &kv->type)) return -1;
    unsigned w = scalar_width(kv->type);
    if (w) {
        kv->n = 1;
        return (kv->ptr = take(s, w)) ? 0 : -1;
    }
    if (kv->type == GGUF_TYPE_STRING) {
        if (take_u64(s, &kv->n)) return -1;
        return (kv->ptr = take(s, kv->n)) ? 0 : -1;
    }
    if (kv->type != GGUF_TYPE_ARRAY) return complain(s, "tipo di valore sconosciuto %u", kv->type);
    if (take_u32(s, &kv->arr_type) || take_u64(s, &kv->n)) return -1;
    kv->ptr = s->base + s->at;
    if ((w = scalar_width(kv->arr_type))) {
        if (kv->n > (s->size - s->at) / w) return complain(s, "array oltre la fine del file");
        s->at += kv->n * w;
        return 0;
    }
    if (kv->arr_type != GGUF_TYPE_STRING) return complain(s, "array di tipo %u non supportato", kv->arr_type);
    s->arr_first[i] = s->n_pos;
    for (uint64_t j = 0; j < kv->n; j++) {
        uint64_t len;
        if (push_position(s, s->at) || take_u64(s, &len) || !take(s, len)) return -1;
    }
    return 0;
}

static int take_tensor(scan *s, gguf_tensor *t, span *name) {
    if (take_name(s, name, "nome di tensore") || take_u32(s, &t->n_dims)) return -1;
    /* the name is resolved later; keep a printable copy for messages until then */
    char shown[96];
    uint64_t sl = name->len < sizeof shown - 1 ? name->len : sizeof shown - 1;
    memcpy(shown, s->base + name->at, sl);
    shown[sl] = '\0';
    if (t->n_dims - 1u >= GGUF_MAX_DIMS) return complain(s, "%s: n_dims=%u", shown, t->n_dims);
    uint64_t count = 1;
    int overflow = 0;
    for (uint32_t d = 0; d < GGUF_MAX_DIMS; d++) {
        t->ne[d] = 1;
        if (d < t->n_dims && take_u64(s, &t->ne[d])) return -1;
        if (!t->ne[d]) return complain(s, "%s: dimensione %u nulla", shown, d);
        if (count > UINT64_MAX / t->ne[d]) overflow = 1;
        else count *= t->ne[d];
    }
    if (take_u32(s, &t->type) || take_u64(s, &t->offset)) return -1;
    const char *tn = gguf_type_name(t->type);
    if (!tn) return complain(s, "%s: tipo ggml sconosciuto %u", shown, t->type);
    const ggml_type *g = &GGML[t->type];
    if (t->ne[0] % g->per_block) return complain(s, "%s: ne[0] non multiplo del blocco %u", shown, g->per_block);
    uint64_t blocks = count / g->per_block;
    if (overflow || blocks > UINT64_MAX / g->block_bytes) return complain(s, "%s: dimensioni troppo grandi", shown);
    t->nbytes = blocks * g->block_bytes;
    return 0;
}

/* ------------------------------------------------------------------ name index */

static uint64_t fnv1a(const char *p) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (; *p; p++) h = (h ^ (uint8_t)*p) * 0x100000001b3ull;
    return h;
}

/* Builds the index over n names (name(i) for entry i); -1 on a duplicate or memory exhaustion. */
static int index_names(scan *s, name_index *ix, uint64_t n, const char *(*name)(const gguf_file *, uint64_t),
                       const gguf_file *f, const char *what) {
    uint64_t cap = 16;
    while (cap < 2 * n) cap *= 2;
    if (!(ix->slot = calloc(cap, sizeof *ix->slot))) return complain(s, "memoria esaurita");
    ix->mask = cap - 1;
    for (uint64_t i = 0; i < n; i++) {
        const char *nm = name(f, i);
        for (uint64_t h = fnv1a(nm) & ix->mask;; h = (h + 1) & ix->mask) {
            if (!ix->slot[h]) {
                ix->slot[h] = i + 1;
                break;
            }
            if (!strcmp(name(f, ix->slot[h] - 1), nm)) return complain(s, "%s duplicato: %s", what, nm);
        }
    }
    return 0;
}

static int64_t index_find(const name_index *ix, const char *nm, const char *(*name)(const gguf_file *, uint64_t),
                          const gguf_file *f) {
    if (!ix->slot) return -1;
    for (uint64_t h = fnv1a(nm) & ix->mask; ix->slot[h]; h = (h + 1) & ix->mask)
        if (!strcmp(name(f, ix->slot[h] - 1), nm)) return (int64_t)(ix->slot[h] - 1);
    return -1;
}

static const char *kv_name(const gguf_file *f, uint64_t i) { return f->kv[i].key; }
static const char *tensor_name(const gguf_file *f, uint64_t i) { return f->tensors[i].name; }

/* ------------------------------------------------------------------ open / close */

void gguf_close(gguf_file *f) {
    if (!f) return;
    free(f->kv);
    free(f->tensors);
    free(f->pool);
    free(f->positions);
    free(f->kv_idx.slot);
    free(f->t_idx.slot);
    if (f->map) munmap((void *)f->map, f->size);
    free(f);
}

/* Copies the recorded names into the pool and points keys, names and string arrays at it. */
static int resolve(scan *s, gguf_file *f) {
    char *p = f->pool = malloc(s->pool_bytes ? s->pool_bytes : 1);
    if (!p) return complain(s, "memoria esaurita");
    for (int pass = 0; pass < 2; pass++) {
        uint64_t n = pass ? f->n_tensors : f->n_kv;
        for (uint64_t i = 0; i < n; i++) {
            const span *sp = pass ? &s->t_name[i] : &s->kv_name[i];
            memcpy(p, s->base + sp->at, sp->len);
            p[sp->len] = '\0';
            if (pass) f->tensors[i].name = p;
            else f->kv[i].key = p;
            p += sp->len + 1;
        }
    }
    f->positions = s->pos;
    s->pos = NULL;
    for (uint64_t i = 0; i < f->n_kv; i++)
        if (f->kv[i].type == GGUF_TYPE_ARRAY && f->kv[i].arr_type == GGUF_TYPE_STRING)
            f->kv[i].str_pos = f->positions + s->arr_first[i];
    return 0;
}

static int read_header(scan *s, gguf_file *f) {
    const uint8_t *magic = take(s, 4);
    if (!magic) return -1;
    if (memcmp(magic, "GGUF", 4)) return complain(s, "non è un file GGUF (magic errato)");
    if (take_u32(s, &f->version)) return -1;
    /* a big-endian writer's 1..3 reads as 0x01000000..0x03000000 here */
    if ((f->version & 0xFFFFu) == 0 && f->version >> 24 && f->version >> 24 <= 3)
        return complain(s, "file GGUF big-endian non supportato");
    if (f->version != 2 && f->version != 3) return complain(s, "versione GGUF %u non supportata", f->version);
    uint64_t n_tensors, n_kv;
    if (take_u64(s, &n_tensors) || take_u64(s, &n_kv)) return -1;

    f->alignment = ALIGN_DEFAULT;
    for (uint64_t i = 0; i < n_kv; i++) {
        if (grow_kv(s, f, i)) return -1;
        memset(&f->kv[i], 0, sizeof f->kv[i]);
        if (take_name(s, &s->kv_name[i], "chiave")) return -1;
        f->n_kv = i + 1;
        if (take_value(s, f, i)) return -1;
        const span *k = &s->kv_name[i];
        if (k->len == 17 && !memcmp(s->base + k->at, "general.alignment", 17)) {
            uint64_t a;
            if (gguf_kv_get_u64(f, (int64_t)i, &a) || a == 0 || a > ALIGN_MAX || (a & (a - 1)))
                return complain(s, "general.alignment non valido");
            f->alignment = (uint32_t)a;
        }
    }
    for (uint64_t i = 0; i < n_tensors; i++) {
        if (grow_tensors(s, f, i)) return -1;
        memset(&f->tensors[i], 0, sizeof f->tensors[i]);
        if (take_tensor(s, &f->tensors[i], &s->t_name[i])) return -1;
        f->n_tensors = i + 1;
    }
    if (resolve(s, f) || index_names(s, &f->kv_idx, f->n_kv, kv_name, f, "metadato") ||
        index_names(s, &f->t_idx, f->n_tensors, tensor_name, f, "tensore"))
        return -1;

    /* tensor data starts at the first multiple of the alignment after the header */
    f->data_offset = (s->at + f->alignment - 1) / f->alignment * f->alignment;
    if (f->data_offset > s->size) return complain(s, "zona dati oltre la fine del file");
    const uint64_t room = s->size - f->data_offset;
    for (uint64_t i = 0; i < f->n_tensors; i++) {
        gguf_tensor *t = &f->tensors[i];
        if (t->offset % f->alignment) return complain(s, "%s: offset non allineato", t->name);
        if (t->offset > room || t->nbytes > room - t->offset)
            return complain(s, "%s: dati oltre la fine del file", t->name);
        t->data = f->map + f->data_offset + t->offset;
    }
    return 0;
}

gguf_file *gguf_open(const char *path, char *err, size_t err_len) {
    scan s = {.err = err, .err_len = err_len};
    if (err && err_len) err[0] = '\0';
    int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        complain(&s, "impossibile aprire %s: %s", path, strerror(errno));
        return NULL;
    }
    struct stat st;
    void *map = MAP_FAILED;
    if (fstat(fd, &st)) complain(&s, "impossibile leggere la dimensione di %s: %s", path, strerror(errno));
    else if (st.st_size <= 0 || (uintmax_t)st.st_size > SIZE_MAX)
        complain(&s, "%s: dimensione non valida o troppo grande per questa piattaforma", path);
    else if ((map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_SHARED, fd, 0)) == MAP_FAILED)
        complain(&s, "mmap fallita su %s: %s", path, strerror(errno));
    close(fd); /* a mapping outlives its descriptor */
    if (map == MAP_FAILED) return NULL;
    gguf_file *f = calloc(1, sizeof *f);
    if (!f) {
        munmap(map, (size_t)st.st_size);
        complain(&s, "memoria esaurita");
        return NULL;
    }
    f->map = map;
    f->size = (size_t)st.st_size;
    s.base = f->map;
    s.size = f->size;
    int rc = read_header(&s, f);
    free(s.kv_name);
    free(s.t_name);
    free(s.arr_first);
    free(s.pos);
    if (rc) {
        gguf_close(f); /* keys and names live in the pool: nothing per entry to free */
        return NULL;
    }
    return f;
}

void gguf_prefetch(const void *p, size_t n) {
    /* one advisory request over the whole page-aligned range; the kernel issues the read-ahead
       in pieces itself and this call does not wait for it */
    if (!p || !n) return;
    const uintptr_t page = (uintptr_t)sysconf(_SC_PAGESIZE);
    const uintptr_t lo = (uintptr_t)p & ~(page - 1);
    posix_madvise((void *)lo, (uintptr_t)p + n - lo, POSIX_MADV_WILLNEED);
}

/* ------------------------------------------------------------------ accessors (NULL-tolerant) */

uint32_t gguf_version(const gguf_file *f) { return f ? f->version : 0; }
uint32_t gguf_alignment(const gguf_file *f) { return f ? f->alignment : 0; }
uint64_t gguf_data_offset(const gguf_file *f) { return f ? f->data_offset : 0; }
uint64_t gguf_n_kv(const gguf_file *f) { return f ? f->n_kv : 0; }
uint64_t gguf_n_tensors(const gguf_file *f) { return f ? f->n_tensors : 0; }

const gguf_kv *gguf_get_kv(const gguf_file *f, uint64_t i) { return f && i < f->n_kv ? f->kv + i : NULL; }
const gguf_tensor *gguf_get_tensor(const gguf_file *f, uint64_t i) {
    return f && i < f->n_tensors ? f->tensors + i : NULL;
}

int64_t gguf_find_kv(const gguf_file *f, const char *key) {
    return f && key ? index_find(&f->kv_idx, key, kv_name, f) : -1;
}

int64_t gguf_find_tensor(const gguf_file *f, const char *name) {
    return f && name ? index_find(&f->t_idx, name, tensor_name, f) : -1;
}

static const gguf_kv *kv_at(const gguf_file *f, int64_t i) {
    return f && i >= 0 && (uint64_t)i < f->n_kv ? f->kv + i : NULL;
}

int gguf_kv_get_u64(const gguf_file *f, int64_t i, uint64_t *out) {
    const gguf_kv *kv = kv_at(f, i);
    if (!kv || !out) return -1;
    static const signed char SIGNED[13] = {0, 1, 0, 1, 0, 1, -1, -1, -1, -1, 0, 1, -1}; /* -1: not an integer */
    if (kv->type >= 13 || SIGNED[kv->type] < 0) return -1;
    unsigned w = scalar_width(kv->type);
    uint64_t v = le_bytes(kv->ptr, w);
    if (SIGNED[kv->type] && w < 8 && (v >> (8 * w - 1))) return -1; /* negative narrow integer */
    if (SIGNED[kv->type] && w == 8 && (v >> 63)) return -1;
    *out = v;
    return 0;
}

int gguf_kv_get_f64(const gguf_file *f, int64_t i, double *out) {
    const gguf_kv *kv = kv_at(f, i);
    if (!kv || !out) return -1;
    if (kv->type == GGUF_TYPE_FLOAT32) {
        uint32_t b = (uint32_t)le_bytes(kv->ptr, 4);
        float v;
        memcpy(&v, &b, 4);
        *out = v;
        return 0;
    }
    if (kv->type == GGUF_TYPE_FLOAT64) {
        uint64_t b = le_bytes(kv->ptr, 8);
        memcpy(out, &b, 8);
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
    *len = le_bytes(f->map + kv->str_pos[j], 8);
    return (const char *)(f->map + kv->str_pos[j] + 8);
}
