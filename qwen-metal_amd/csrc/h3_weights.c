/* Safetensors shards and the component weight store (reference
 * h3_safetensors.c, h3_weights.c), written for this build: a bounded
 * recursive-descent reader of the JSON header that keeps only what the
 * loader needs (dtype, shape, data_offsets), strict validation of every
 * byte range against the file, and payload reads in bounded host chunks
 * straight into device tensors. Host code only; no GPU work except the
 * uploads. */
#define _DEFAULT_SOURCE
#include "../../include/h3_weights.h"

#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#define ST_MAX_HEADER (256ull << 20) /* bytes of JSON header accepted */
#define ST_MAX_DEPTH 64              /* nesting accepted inside skipped values */
#define ST_CHUNK (32u << 20)         /* host staging per upload */

static int fail(char *error, size_t n, const char *fmt, ...) {
    if (error && n) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(error, n, fmt, ap);
        va_end(ap);
    }
    return 0;
}

/* ---------------------------------------------------------------- dtypes */

static const struct {
    const char *name;
    h3_dtype dtype;
    size_t size;
} k_dtypes[] = {
    {"BOOL", H3_DTYPE_BOOL, 1}, {"I8", H3_DTYPE_I8, 1},     {"U8", H3_DTYPE_U8, 1},
    {"I16", H3_DTYPE_I16, 2},   {"U16", H3_DTYPE_U16, 2},   {"F16", H3_DTYPE_F16, 2},
    {"BF16", H3_DTYPE_BF16, 2}, {"I32", H3_DTYPE_I32, 4},   {"U32", H3_DTYPE_U32, 4},
    {"F32", H3_DTYPE_F32, 4},   {"I64", H3_DTYPE_I64, 8},   {"U64", H3_DTYPE_U64, 8},
    {"F64", H3_DTYPE_F64, 8},
};
#define N_DTYPES (sizeof(k_dtypes) / sizeof(k_dtypes[0]))

size_t h3_dtype_size(h3_dtype dtype) {
    for (size_t i = 0; i < N_DTYPES; i++)
        if (k_dtypes[i].dtype == dtype) return k_dtypes[i].size;
    return 0;
}

const char *h3_dtype_name(h3_dtype dtype) {
    for (size_t i = 0; i < N_DTYPES; i++)
        if (k_dtypes[i].dtype == dtype) return k_dtypes[i].name;
    return "UNKNOWN";
}

static h3_dtype dtype_of(const char *name) {
    for (size_t i = 0; i < N_DTYPES; i++)
        if (strcmp(k_dtypes[i].name, name) == 0) return k_dtypes[i].dtype;
    return H3_DTYPE_UNKNOWN;
}

/* ------------------------------------------------------------ JSON reader */

typedef struct {
    const unsigned char *p, *end, *begin;
    char *error;
    size_t error_size;
} jr;

static int jr_fail(jr *r, const char *what) {
    return fail(r->error, r->error_size, "safetensors header: %s at byte %zu", what,
                (size_t)(r->p - r->begin));
}

static void jr_space(jr *r) {
    while (r->p < r->end && (*r->p == ' ' || *r->p == '\t' || *r->p == '\n' || *r->p == '\r'))
        r->p++;
}

/* next non-space byte, or 0 at the end */
static int jr_peek(jr *r) {
    jr_space(r);
    return r->p < r->end ? *r->p : 0;
}

static int jr_expect(jr *r, int c) {
    if (jr_peek(r) != c) return 0;
    r->p++;
    return 1;
}

static void utf8_put(char *out, size_t *n, unsigned cp) {
    if (cp < 0x80) {
        out[(*n)++] = (char)cp;
    } else if (cp < 0x800) {
        out[(*n)++] = (char)(0xC0 | (cp >> 6));
        out[(*n)++] = (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        out[(*n)++] = (char)(0xE0 | (cp >> 12));
        out[(*n)++] = (char)(0x80 | ((cp >> 6) & 0x3F));
        out[(*n)++] = (char)(0x80 | (cp & 0x3F));
    } else {
        out[(*n)++] = (char)(0xF0 | (cp >> 18));
        out[(*n)++] = (char)(0x80 | ((cp >> 12) & 0x3F));
        out[(*n)++] = (char)(0x80 | ((cp >> 6) & 0x3F));
        out[(*n)++] = (char)(0x80 | (cp & 0x3F));
    }
}

static int hex4(const unsigned char *s, unsigned *v) {
    *v = 0;
    for (int i = 0; i < 4; i++) {
        const unsigned c = s[i];
        unsigned d;
        if (c >= '0' && c <= '9') d = c - '0';
        else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
        else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
        else return 0;
        *v = *v * 16 + d;
    }
    return 1;
}

/* A JSON string, unescaped into a new NUL-terminated buffer (UTF-8; the
 * result is never longer than the quoted text). NUL characters are
 * rejected, since names are C strings. */
static char *jr_string(jr *r) {
    if (!jr_expect(r, '"')) {
        jr_fail(r, "expected a string");
        return NULL;
    }
    const unsigned char *start = r->p;
    while (r->p < r->end && *r->p != '"') r->p += (*r->p == '\\' && r->p + 1 < r->end) ? 2 : 1;
    if (r->p >= r->end) {
        jr_fail(r, "unterminated string");
        return NULL;
    }
    const size_t span = (size_t)(r->p - start);
    r->p++; /* closing quote */
    char *out = malloc(span + 1);
    if (!out) {
        fail(r->error, r->error_size, "out of memory");
        return NULL;
    }
    size_t n = 0;
    for (const unsigned char *s = start; s < start + span;) {
        if (*s < 0x20) goto bad;
        if (*s != '\\') {
            out[n++] = (char)*s++;
            continue;
        }
        const unsigned char e = s[1];
        s += 2;
        switch (e) {
        case '"': out[n++] = '"'; break;
        case '\\': out[n++] = '\\'; break;
        case '/': out[n++] = '/'; break;
        case 'b': out[n++] = '\b'; break;
        case 'f': out[n++] = '\f'; break;
        case 'n': out[n++] = '\n'; break;
        case 'r': out[n++] = '\r'; break;
        case 't': out[n++] = '\t'; break;
        case 'u': {
            unsigned cp;
            if (s + 4 > start + span || !hex4(s, &cp)) goto bad;
            s += 4;
            if (cp >= 0xD800 && cp < 0xDC00) { /* surrogate pair */
                unsigned lo;
                if (s + 6 > start + span || s[0] != '\\' || s[1] != 'u' || !hex4(s + 2, &lo) ||
                    lo < 0xDC00 || lo >= 0xE000)
                    goto bad;
                s += 6;
                cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            } else if (cp >= 0xDC00 && cp < 0xE000) {
                goto bad;
            }
            if (cp == 0) goto bad;
            utf8_put(out, &n, cp);
            break;
        }
        default: goto bad;
        }
    }
    out[n] = '\0';
    return out;
bad:
    free(out);
    jr_fail(r, "invalid string");
    return NULL;
}

/* an unsigned integer that fits 64 bits (no sign, fraction or exponent) */
static int jr_uint(jr *r, uint64_t *v) {
    jr_space(r);
    if (r->p >= r->end || *r->p < '0' || *r->p > '9') return jr_fail(r, "expected an integer");
    uint64_t x = 0;
    const unsigned char *start = r->p;
    while (r->p < r->end && *r->p >= '0' && *r->p <= '9') {
        const unsigned d = *r->p - '0';
        if (x > (UINT64_MAX - d) / 10) return jr_fail(r, "integer overflow");
        x = x * 10 + d;
        r->p++;
    }
    if (r->p - start > 1 && *start == '0') return jr_fail(r, "leading zero");
    if (r->p < r->end && (*r->p == '.' || *r->p == 'e' || *r->p == 'E'))
        return jr_fail(r, "expected an integer");
    *v = x;
    return 1;
}

/* any JSON value, checked and discarded */
static int jr_skip(jr *r, int depth) {
    if (depth > ST_MAX_DEPTH) return jr_fail(r, "nesting too deep");
    const int c = jr_peek(r);
    if (c == '"') {
        char *s = jr_string(r);
        const int ok = s != NULL;
        free(s);
        return ok;
    }
    if (c == '{' || c == '[') {
        const int close = c == '{' ? '}' : ']';
        r->p++;
        if (jr_expect(r, close)) return 1;
        for (;;) {
            if (c == '{') {
                char *k = jr_string(r);
                if (!k) return 0;
                free(k);
                if (!jr_expect(r, ':')) return jr_fail(r, "expected ':'");
            }
            if (!jr_skip(r, depth + 1)) return 0;
            if (jr_expect(r, ',')) continue;
            if (jr_expect(r, close)) return 1;
            return jr_fail(r, "expected ',' or a closing bracket");
        }
    }
    static const char *const words[] = {"true", "false", "null"};
    for (int i = 0; i < 3; i++) {
        const size_t n = strlen(words[i]);
        if ((size_t)(r->end - r->p) >= n && memcmp(r->p, words[i], n) == 0) {
            r->p += n;
            return 1;
        }
    }
    if (c == '-' || (c >= '0' && c <= '9')) { /* number: sign, digits, fraction, exponent */
        if (*r->p == '-') r->p++;
        int digits = 0;
        while (r->p < r->end && ((*r->p >= '0' && *r->p <= '9') || *r->p == '.' ||
                                 *r->p == 'e' || *r->p == 'E' || *r->p == '+' || *r->p == '-')) {
            digits += *r->p >= '0' && *r->p <= '9';
            r->p++;
        }
        return digits ? 1 : jr_fail(r, "invalid number");
    }
    return jr_fail(r, "unexpected character");
}

/* [u, u, ...] with at most max entries */
static int jr_uint_array(jr *r, uint64_t *out, int max, int *count) {
    if (!jr_expect(r, '[')) return jr_fail(r, "expected '['");
    *count = 0;
    if (jr_expect(r, ']')) return 1;
    for (;;) {
        uint64_t v = 0;
        if (!jr_uint(r, &v)) return 0;
        if (*count >= max) return jr_fail(r, "too many entries");
        out[(*count)++] = v;
        if (jr_expect(r, ',')) continue;
        if (jr_expect(r, ']')) return 1;
        return jr_fail(r, "expected ',' or ']'");
    }
}

/* one tensor entry: {"dtype": ..., "shape": [...], "data_offsets": [b, e]} */
static int jr_tensor(jr *r, h3_st_tensor *t) {
    if (!jr_expect(r, '{')) return jr_fail(r, "expected a tensor object");
    int have_dtype = 0, have_shape = 0, have_offsets = 0;
    if (!jr_expect(r, '}')) {
        for (;;) {
            char *key = jr_string(r);
            if (!key) return 0;
            if (!jr_expect(r, ':')) {
                free(key);
                return jr_fail(r, "expected ':'");
            }
            int ok;
            if (strcmp(key, "dtype") == 0) {
                char *dt = jr_string(r);
                ok = dt != NULL;
                if (ok) {
                    t->dtype = dtype_of(dt);
                    if (t->dtype == H3_DTYPE_UNKNOWN)
                        ok = fail(r->error, r->error_size, "safetensors header: unknown dtype %s",
                                  dt);
                }
                free(dt);
                have_dtype = 1;
            } else if (strcmp(key, "shape") == 0) {
                ok = jr_uint_array(r, t->shape, 8, &t->ndim);
                have_shape = 1;
            } else if (strcmp(key, "data_offsets") == 0) {
                uint64_t o[2];
                int n = 0;
                ok = jr_uint_array(r, o, 2, &n);
                if (ok && n != 2) ok = jr_fail(r, "data_offsets needs two entries");
                if (ok) {
                    t->data_begin = o[0];
                    t->data_end = o[1];
                }
                have_offsets = 1;
            } else {
                ok = jr_skip(r, 1);
            }
            free(key);
            if (!ok) return 0;
            if (jr_expect(r, ',')) continue;
            if (jr_expect(r, '}')) break;
            return jr_fail(r, "expected ',' or '}'");
        }
    }
    if (!have_dtype || !have_shape || !have_offsets)
        return jr_fail(r, "tensor entry lacks dtype, shape or data_offsets");
    return 1;
}

/* ----------------------------------------------------------- the header */

void h3_st_free_header(h3_st_header *h) {
    if (!h) return;
    for (size_t i = 0; i < h->tensor_count; i++) free(h->tensors[i].name);
    free(h->tensors);
    free(h->path);
    memset(h, 0, sizeof(*h));
}

uint64_t h3_st_tensor_elements(const h3_st_tensor *t) {
    if (!t) return 0;
    uint64_t n = 1;
    for (int i = 0; i < t->ndim; i++) {
        if (t->shape[i] && n > UINT64_MAX / t->shape[i]) return UINT64_MAX;
        n *= t->shape[i];
    }
    return n;
}

static int read_full(int fd, void *buf, size_t n, uint64_t off) {
    unsigned char *p = buf;
    while (n) {
        const ssize_t got = pread(fd, p, n, (off_t)off);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return 0;
        p += got;
        n -= (size_t)got;
        off += (uint64_t)got;
    }
    return 1;
}

static int name_cmp(const void *a, const void *b) {
    return strcmp(((const h3_st_tensor *)a)->name, ((const h3_st_tensor *)b)->name);
}

int h3_st_read_header(const char *path, h3_st_header *h, char *error, size_t error_size) {
    if (error && error_size) error[0] = '\0';
    if (!path || !h) return fail(error, error_size, "safetensors: missing path or header");
    memset(h, 0, sizeof(*h));
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(error, error_size, "%s: %s", path, strerror(errno));
    struct stat st;
    unsigned char len8[8];
    unsigned char *json = NULL;
    int ok = 0;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode) || st.st_size < 8) {
        fail(error, error_size, "%s: not a safetensors file", path);
        goto out;
    }
    if (!read_full(fd, len8, 8, 0)) {
        fail(error, error_size, "%s: cannot read the header length", path);
        goto out;
    }
    uint64_t hs = 0;
    for (int i = 7; i >= 0; i--) hs = (hs << 8) | len8[i];
    const uint64_t fsize = (uint64_t)st.st_size;
    if (hs < 2 || hs > ST_MAX_HEADER || hs > fsize - 8) {
        fail(error, error_size, "%s: invalid header length %llu", path, (unsigned long long)hs);
        goto out;
    }
    json = malloc((size_t)hs);
    if (!json) {
        fail(error, error_size, "out of memory");
        goto out;
    }
    if (!read_full(fd, json, (size_t)hs, 8)) {
        fail(error, error_size, "%s: cannot read the header", path);
        goto out;
    }
    const uint64_t payload = fsize - 8 - hs;
    jr r = {json, json + hs, json, error, error_size};
    size_t cap = 0;
    if (!jr_expect(&r, '{')) {
        jr_fail(&r, "expected a JSON object");
        goto out;
    }
    if (!jr_expect(&r, '}')) {
        for (;;) {
            char *key = jr_string(&r);
            if (!key) goto out;
            if (!jr_expect(&r, ':')) {
                free(key);
                jr_fail(&r, "expected ':'");
                goto out;
            }
            if (strcmp(key, "__metadata__") == 0) {
                free(key);
                if (!jr_skip(&r, 1)) goto out;
            } else {
                if (h->tensor_count == cap) {
                    cap = cap ? 2 * cap : 64;
                    h3_st_tensor *t = realloc(h->tensors, cap * sizeof(*t));
                    if (!t) {
                        free(key);
                        fail(error, error_size, "out of memory");
                        goto out;
                    }
                    h->tensors = t;
                }
                h3_st_tensor *t = &h->tensors[h->tensor_count];
                memset(t, 0, sizeof(*t));
                t->name = key;
                h->tensor_count++;
                if (!jr_tensor(&r, t)) goto out;
                const uint64_t n = h3_st_tensor_elements(t);
                const uint64_t es = h3_dtype_size(t->dtype);
                if (t->data_end < t->data_begin || t->data_end > payload) {
                    fail(error, error_size, "%s: tensor %s: data_offsets [%llu, %llu] outside the "
                         "%llu-byte payload", path, key, (unsigned long long)t->data_begin,
                         (unsigned long long)t->data_end, (unsigned long long)payload);
                    goto out;
                }
                if (n == UINT64_MAX || n > UINT64_MAX / es || n * es != t->data_end - t->data_begin) {
                    fail(error, error_size, "%s: tensor %s: %llu bytes do not hold a %s tensor of "
                         "%llu elements", path, key,
                         (unsigned long long)(t->data_end - t->data_begin), h3_dtype_name(t->dtype),
                         (unsigned long long)n);
                    goto out;
                }
                t->file_offset = 8 + hs + t->data_begin;
            }
            if (jr_expect(&r, ',')) continue;
            if (jr_expect(&r, '}')) break;
            jr_fail(&r, "expected ',' or '}'");
            goto out;
        }
    }
    if (jr_peek(&r) != 0) {
        jr_fail(&r, "trailing bytes after the header object");
        goto out;
    }
    /* sorted by name: h3_st_find bisects, duplicates become neighbours */
    if (h->tensor_count) qsort(h->tensors, h->tensor_count, sizeof(h3_st_tensor), name_cmp);
    for (size_t i = 1; i < h->tensor_count; i++)
        if (strcmp(h->tensors[i - 1].name, h->tensors[i].name) == 0) {
            fail(error, error_size, "%s: tensor %s appears twice", path, h->tensors[i].name);
            goto out;
        }
    h->path = strdup(path);
    if (!h->path) {
        fail(error, error_size, "out of memory");
        goto out;
    }
    h->file_size = fsize;
    h->header_size = hs;
    ok = 1;
out:
    free(json);
    close(fd);
    if (!ok) h3_st_free_header(h);
    return ok;
}

const h3_st_tensor *h3_st_find(const h3_st_header *h, const char *name) {
    if (!h || !name || !h->tensor_count) return NULL;
    size_t lo = 0, hi = h->tensor_count;
    while (lo < hi) {
        const size_t mid = lo + (hi - lo) / 2;
        const int c = strcmp(h->tensors[mid].name, name);
        if (c == 0) return &h->tensors[mid];
        if (c < 0) lo = mid + 1;
        else hi = mid;
    }
    return NULL;
}

int h3_st_read_data(const h3_st_header *h, const h3_st_tensor *t, void *data, size_t bytes,
                    char *error, size_t error_size) {
    if (error && error_size) error[0] = '\0';
    if (!h || !t || (!data && bytes)) return fail(error, error_size, "invalid tensor read request");
    if ((uint64_t)bytes != t->data_end - t->data_begin)
        return fail(error, error_size, "%s: expected %llu bytes, got %zu", t->name,
                    (unsigned long long)(t->data_end - t->data_begin), bytes);
    const int fd = open(h->path, O_RDONLY);
    if (fd < 0) return fail(error, error_size, "%s: %s", h->path, strerror(errno));
    const int ok = read_full(fd, data, bytes, t->file_offset);
    close(fd);
    return ok ? 1 : fail(error, error_size, "%s: cannot read %s", h->path, t->name);
}

/* ------------------------------------------------------------ the store */

struct h3_weight_store {
    h3_st_header *shards;
    size_t count;
};

static int is_shard(const char *name) {
    static const char suffix[] = ".safetensors";
    const size_t n = strlen(name), s = sizeof(suffix) - 1;
    return n > s && strcmp(name + n - s, suffix) == 0;
}

static int str_cmp(const void *a, const void *b) {
    return strcmp(*(char *const *)a, *(char *const *)b);
}

void h3_weight_store_free(h3_weight_store *s) {
    if (!s) return;
    for (size_t i = 0; i < s->count; i++) h3_st_free_header(&s->shards[i]);
    free(s->shards);
    free(s);
}

size_t h3_weight_store_shards(const h3_weight_store *s) { return s ? s->count : 0; }

h3_weight_store *h3_weight_store_open(const char *dir, char *error, size_t error_size) {
    if (error && error_size) error[0] = '\0';
    if (!dir) {
        fail(error, error_size, "weight store: missing directory");
        return NULL;
    }
    DIR *d = opendir(dir);
    if (!d) {
        fail(error, error_size, "%s: %s", dir, strerror(errno));
        return NULL;
    }
    char **names = NULL;
    size_t n = 0, cap = 0;
    int ok = 1;
    for (struct dirent *e; ok && (e = readdir(d));) {
        if (!is_shard(e->d_name)) continue;
        if (n == cap) {
            cap = cap ? 2 * cap : 16;
            char **m = realloc(names, cap * sizeof(*m));
            if (!m) {
                ok = 0;
                break;
            }
            names = m;
        }
        names[n] = strdup(e->d_name);
        ok = names[n] != NULL;
        n += ok;
    }
    closedir(d);
    h3_weight_store *s = ok ? calloc(1, sizeof(*s)) : NULL;
    if (s && n) s->shards = calloc(n, sizeof(h3_st_header));
    if (!s || (n && !s->shards)) {
        fail(error, error_size, "out of memory");
        ok = 0;
    } else if (!n) {
        fail(error, error_size, "%s: no safetensors files", dir);
        ok = 0;
    }
    if (ok) qsort(names, n, sizeof(*names), str_cmp);
    for (size_t i = 0; ok && i < n; i++) {
        const size_t len = strlen(dir) + strlen(names[i]) + 2;
        char *path = malloc(len);
        if (!path) {
            ok = fail(error, error_size, "out of memory");
            break;
        }
        snprintf(path, len, "%s/%s", dir, names[i]);
        ok = h3_st_read_header(path, &s->shards[i], error, error_size);
        free(path);
        if (ok) s->count = i + 1;
    }
    /* a tensor name in two shards is ambiguous */
    for (size_t i = 0; ok && i < s->count; i++)
        for (size_t t = 0; ok && t < s->shards[i].tensor_count; t++)
            for (size_t j = i + 1; ok && j < s->count; j++)
                if (h3_st_find(&s->shards[j], s->shards[i].tensors[t].name))
                    ok = fail(error, error_size, "%s: tensor %s is in %s and %s", dir,
                              s->shards[i].tensors[t].name, s->shards[i].path, s->shards[j].path);
    for (size_t i = 0; i < n; i++) free(names[i]);
    free(names);
    if (!ok) {
        h3_weight_store_free(s);
        return NULL;
    }
    return s;
}

const h3_st_tensor *h3_weight_find(const h3_weight_store *s, const char *name,
                                   const h3_st_header **header) {
    if (header) *header = NULL;
    if (!s || !name) return NULL;
    for (size_t i = 0; i < s->count; i++) {
        const h3_st_tensor *t = h3_st_find(&s->shards[i], name);
        if (t) {
            if (header) *header = &s->shards[i];
            return t;
        }
    }
    return NULL;
}

static void shape_text(char *out, size_t n, int ndim, const uint64_t *shape) {
    size_t used = (size_t)snprintf(out, n, "[");
    for (int i = 0; i < ndim && used < n; i++)
        used += (size_t)snprintf(out + used, n - used, i ? ", %llu" : "%llu",
                                 (unsigned long long)shape[i]);
    if (used < n) snprintf(out + used, n - used, "]");
}

/* the named tensor, checked against dtype and shape */
static const h3_st_tensor *checked(const h3_weight_store *s, const char *name, h3_dtype dtype,
                                   int ndim, const uint64_t *shape, const h3_st_header **h,
                                   char *error, size_t error_size) {
    const h3_st_tensor *t = h3_weight_find(s, name, h);
    if (!t) {
        fail(error, error_size, "missing tensor %s", name ? name : "(null)");
        return NULL;
    }
    if (t->dtype != dtype) {
        fail(error, error_size, "tensor %s: dtype %s, expected %s", name, h3_dtype_name(t->dtype),
             h3_dtype_name(dtype));
        return NULL;
    }
    int same = t->ndim == ndim;
    for (int i = 0; same && i < ndim; i++) same = t->shape[i] == shape[i];
    if (!same) {
        char got[160], want[160];
        shape_text(got, sizeof(got), t->ndim, t->shape);
        shape_text(want, sizeof(want), ndim, shape);
        fail(error, error_size, "tensor %s: shape %s, expected %s", name, got, want);
        return NULL;
    }
    return t;
}

/* payload -> dst[offset ...] through a bounded host buffer */
static int upload(const h3_st_header *h, const h3_st_tensor *t, h3_gpu_tensor *dst,
                  size_t offset, size_t esize, char *error, size_t error_size) {
    const uint64_t bytes = t->data_end - t->data_begin;
    const size_t chunk = (size_t)(bytes < ST_CHUNK ? bytes : ST_CHUNK);
    unsigned char *buf = chunk ? malloc(chunk) : NULL;
    if (chunk && !buf) return fail(error, error_size, "out of memory");
    const int fd = open(h->path, O_RDONLY);
    if (fd < 0) {
        free(buf);
        return fail(error, error_size, "%s: %s", h->path, strerror(errno));
    }
    int ok = 1;
    for (uint64_t done = 0; ok && done < bytes;) {
        const size_t n = (size_t)(bytes - done < chunk ? bytes - done : chunk);
        ok = read_full(fd, buf, n, t->file_offset + done);
        if (!ok) {
            fail(error, error_size, "%s: cannot read %s", h->path, t->name);
            break;
        }
        const size_t at = offset + (size_t)(done / esize);
        ok = esize == 2 ? h3_gpu_tensor_write_bf16_range(dst, at, (const uint16_t *)buf, n / 2)
                        : h3_gpu_tensor_write_f32_range(dst, at, (const float *)buf, n / 4);
        if (!ok) fail(error, error_size, "tensor %s: upload failed", t->name);
        done += n;
    }
    close(fd);
    free(buf);
    return ok;
}

int h3_weight_read_bf16_into(const h3_weight_store *s, const char *name, int ndim,
                             const uint64_t *shape, h3_gpu_tensor *dst, size_t offset,
                             char *error, size_t error_size) {
    const h3_st_header *h;
    const h3_st_tensor *t = checked(s, name, H3_DTYPE_BF16, ndim, shape, &h, error, error_size);
    if (!t) return 0;
    if (!dst || h3_gpu_tensor_dtype(dst) != H3_GPU_BF16 ||
        h3_gpu_tensor_elements(dst) < offset + h3_st_tensor_elements(t))
        return fail(error, error_size, "tensor %s: destination too small", name);
    return upload(h, t, dst, offset, 2, error, error_size);
}

static h3_gpu_tensor *load(const h3_weight_store *s, h3_gpu *gpu, const char *name, int ndim,
                           const uint64_t *shape, h3_dtype dtype, char *error,
                           size_t error_size) {
    const h3_st_header *h;
    const h3_st_tensor *t = checked(s, name, dtype, ndim, shape, &h, error, error_size);
    if (!t) return NULL;
    const size_t n = (size_t)h3_st_tensor_elements(t);
    h3_gpu_tensor *out = dtype == H3_DTYPE_BF16 ? h3_gpu_tensor_new_bf16(gpu, n)
                                                : h3_gpu_tensor_new_f32(gpu, n);
    if (!out) {
        fail(error, error_size, "tensor %s: device allocation failed", name);
        return NULL;
    }
    if (!upload(h, t, out, 0, h3_dtype_size(dtype), error, error_size)) {
        h3_gpu_tensor_free(out);
        return NULL;
    }
    return out;
}

h3_gpu_tensor *h3_weight_load_bf16(const h3_weight_store *s, h3_gpu *gpu, const char *name,
                                   int ndim, const uint64_t *shape, char *error,
                                   size_t error_size) {
    return load(s, gpu, name, ndim, shape, H3_DTYPE_BF16, error, error_size);
}

h3_gpu_tensor *h3_weight_load_f32(const h3_weight_store *s, h3_gpu *gpu, const char *name,
                                  int ndim, const uint64_t *shape, char *error,
                                  size_t error_size) {
    return load(s, gpu, name, ndim, shape, H3_DTYPE_F32, error, error_size);
}
