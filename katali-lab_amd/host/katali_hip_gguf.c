/* katali_hip_gguf.c — GGUF reader, device weight cache, MoE layer assembly
 * and expert VRAM tier (declarations and contracts in katali_hip_gguf.h).
 *
 * The reader maps the file read-only and parses it from the public GGUF
 * layout in four passes (header, metadata, tensor directory, data layout);
 * every count, length and offset read from the file is checked against the
 * bytes left before it is used, and the first refusal is reported with its
 * byte position. It accepts and refuses the same files as the engine's reader
 * (V/src/gguf_reader.c:351-543), so a file the engine opens opens here too.
 * Little-endian host (x86-64, as the engine).
 */
#ifndef _POSIX_C_SOURCE
#define _POSIX_C_SOURCE 200809L
#endif
#include "katali_hip_gguf.h"

#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "katali_hip_loader.h"

static char g_err[256];

static int gguf_fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

const char *katali_hip_gguf_last_error(void) { return g_err; }

/* ---- ggml block sizes (public ggml type table) -------------------------- */
static void type_block(uint32_t t, uint64_t *elems, uint64_t *bytes) {
    static const struct { uint32_t t; uint16_t e, b; } k[] = {
        {0, 1, 4},     {1, 1, 2},     {2, 32, 18},   {3, 32, 20},   {6, 32, 22},  {7, 32, 24},
        {8, 32, 34},   {9, 32, 36},   {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {15, 256, 292}, {24, 1, 1},  {25, 1, 2},    {26, 1, 4},   {27, 1, 8},
        {28, 1, 8},    {30, 1, 2},
    };
    *elems = *bytes = 0;
    for (size_t i = 0; i < sizeof k / sizeof k[0]; i++)
        if (k[i].t == t) { *elems = k[i].e; *bytes = k[i].b; return; }
}

uint64_t katali_hip_ggml_row_bytes(uint32_t type, uint64_t n) {
    uint64_t e, b;
    type_block(type, &e, &b);
    if (!e || n % e || n / e > UINT64_MAX / b) return 0;
    return n / e * b;
}

/* ---- the file ------------------------------------------------------------ */
/* GGUF metadata value types (the public GGUF format) */
enum {
    VT_U8 = 0, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STRING, VT_ARRAY, VT_U64, VT_I64, VT_F64,
    VT_COUNT
};

/* bytes of one fixed-size value, 0 for strings, arrays and unknown types */
static unsigned value_width(uint32_t vt) {
    static const uint8_t w[VT_COUNT] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    return vt < VT_COUNT ? w[vt] : 0;
}
static int value_signed(uint32_t vt) { return vt == VT_I8 || vt == VT_I16 || vt == VT_I32 || vt == VT_I64; }
static int value_float(uint32_t vt) { return vt == VT_F32 || vt == VT_F64; }

/* A metadata entry as kept: a number as int64 and double, a string as bytes
 * in the map; arrays are validated and skipped (nothing here reads them). */
typedef struct Meta {
    char *key;
    uint32_t vt;
    int64_t num;       /* integers and bools (unsigned 64-bit kept as its bits) */
    double real;       /* F32 / F64 */
    const uint8_t *str;
    uint64_t str_len;
} Meta;

struct KataliHipGguf {
    const uint8_t *map;
    uint64_t size;
    uint32_t version;
    uint64_t n_meta, n_tensors, alignment, data_offset;
    Meta *meta;
    KataliHipGgufTensor *t;
};

/* The parser: a read position over the mapped file and the first refusal. */
typedef struct Reader {
    const uint8_t *base;
    uint64_t size, at;
    char *why;
    size_t why_cap;
    int refused;
} Reader;

static int refuse(Reader *r, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static int refuse(Reader *r, const char *fmt, ...) {
    if (!r->refused && r->why && r->why_cap) {
        va_list ap;
        va_start(ap, fmt);
        const int n = vsnprintf(r->why, r->why_cap, fmt, ap);
        va_end(ap);
        if (n >= 0 && (size_t)n < r->why_cap)
            snprintf(r->why + n, r->why_cap - (size_t)n, " [byte %llu of %llu]", (unsigned long long)r->at,
                     (unsigned long long)r->size);
    }
    r->refused = 1;
    return -1;
}

static uint64_t left(const Reader *r) { return r->size - r->at; }

/* n little-endian bytes (n <= 8) as an unsigned number */
static int fixed(Reader *r, unsigned n, uint64_t *v, const char *what) {
    *v = 0;
    if (left(r) < n) return refuse(r, "file ends inside %s", what);
    uint64_t x = 0;
    for (unsigned k = 0; k < n; k++) x |= (uint64_t)r->base[r->at + k] << (8 * k);
    r->at += n;
    *v = x;
    return 0;
}
static int u32_at(Reader *r, uint32_t *v, const char *what) {
    uint64_t x;
    if (fixed(r, 4, &x, what)) return -1;
    *v = (uint32_t)x;
    return 0;
}

/* a GGUF string: u64 length, then that many bytes, all inside the file */
static int string_at(Reader *r, const uint8_t **p, uint64_t *len, const char *what) {
    uint64_t n;
    if (fixed(r, 8, &n, what)) return -1;
    if (n > left(r)) return refuse(r, "%s claims %llu bytes, %llu remain", what, (unsigned long long)n,
                                   (unsigned long long)left(r));
    *p = r->base + r->at;
    *len = n;
    r->at += n;
    return 0;
}

static char *c_string(const uint8_t *p, uint64_t n) {
    char *s = (char *)malloc(n + 1);
    if (s) {
        memcpy(s, p, n);
        s[n] = 0;
    }
    return s;
}

/* An array value: element type, count, then the elements. Arrays of arrays
 * are refused; the count may not exceed the bytes left (a cheap bound before
 * any element is read), fixed-size payloads must fit, and strings are walked
 * one by one. */
static int skip_array(Reader *r, const char *key) {
    uint32_t et;
    uint64_t count;
    if (u32_at(r, &et, "an array's element type") || fixed(r, 8, &count, "an array's length")) return -1;
    if (et == VT_ARRAY) return refuse(r, "metadata '%s': arrays of arrays are not read", key);
    if (count > left(r)) return refuse(r, "metadata '%s': array of %llu elements in %llu bytes", key,
                                       (unsigned long long)count, (unsigned long long)left(r));
    const unsigned w = value_width(et);
    if (w) {
        if (count > left(r) / w)
            return refuse(r, "metadata '%s': %llu elements of %u bytes overrun the file", key,
                          (unsigned long long)count, w);
        r->at += count * w;
        return 0;
    }
    if (et != VT_STRING) return refuse(r, "metadata '%s': array element type %u is not a GGUF type", key, et);
    for (uint64_t k = 0; k < count; k++) {
        const uint8_t *p;
        uint64_t n;
        if (string_at(r, &p, &n, "a string element")) return -1;
    }
    return 0;
}

static int read_meta(Reader *r, Meta *m) {
    const uint8_t *kp;
    uint64_t kn;
    if (string_at(r, &kp, &kn, "a metadata key")) return -1;
    if (!(m->key = c_string(kp, kn))) return refuse(r, "out of memory");
    if (u32_at(r, &m->vt, "a metadata value type")) return -1;
    if (m->vt == VT_ARRAY) return skip_array(r, m->key);
    if (m->vt == VT_STRING) return string_at(r, &m->str, &m->str_len, "a metadata string");
    const unsigned w = value_width(m->vt);
    if (!w) return refuse(r, "metadata '%s': value type %u is not a GGUF type", m->key, m->vt);
    uint64_t bits;
    if (fixed(r, w, &bits, "a metadata value")) return -1;
    if (m->vt == VT_F32) {
        float f;
        const uint32_t b32 = (uint32_t)bits;
        memcpy(&f, &b32, 4);
        m->real = f;
    } else if (m->vt == VT_F64) {
        memcpy(&m->real, &bits, 8);
    } else if (m->vt == VT_BOOL) {
        m->num = bits != 0;
    } else if (value_signed(m->vt)) {
        const unsigned sh = 64 - 8 * w;   /* sign-extend from w bytes */
        m->num = (int64_t)(bits << sh) >> sh;
    } else {
        m->num = (int64_t)bits;
    }
    return 0;
}

/* One tensor directory record: name, rank 1..4, dims (none zero, product
 * in 64 bits), ggml type, offset into the data section. */
static int read_tensor(Reader *r, KataliHipGgufTensor *t) {
    const uint8_t *np;
    uint64_t nn;
    if (string_at(r, &np, &nn, "a tensor name")) return -1;
    if (!(t->name = c_string(np, nn))) return refuse(r, "out of memory");
    if (u32_at(r, &t->n_dims, "a tensor rank")) return -1;
    if (t->n_dims == 0 || t->n_dims > 4) return refuse(r, "tensor '%s': rank %u (1 to 4)", t->name, t->n_dims);
    for (uint32_t d = 0; d < t->n_dims; d++)
        if (fixed(r, 8, &t->dims[d], "a tensor dimension")) return -1;
    uint64_t elems = 1;
    for (uint32_t d = 0; d < t->n_dims; d++) {
        if (t->dims[d] == 0) return refuse(r, "tensor '%s': dimension %u is 0", t->name, d);
        if (elems > UINT64_MAX / t->dims[d]) return refuse(r, "tensor '%s': more than 2^64 elements", t->name);
        elems *= t->dims[d];
    }
    if (u32_at(r, &t->type, "a tensor type") || fixed(r, 8, &t->offset, "a tensor offset")) return -1;
    t->nbytes = elems;   /* elements until the layout is resolved */
    return 0;
}

static const Meta *meta_find(const KataliHipGguf *g, const char *key) {
    for (uint64_t k = 0; k < g->n_meta; k++)
        if (g->meta[k].key && strcmp(g->meta[k].key, key) == 0) return &g->meta[k];
    return NULL;
}

void katali_hip_gguf_close(KataliHipGguf *g) {
    if (!g) return;
    for (uint64_t k = 0; g->meta && k < g->n_meta; k++) free(g->meta[k].key);
    for (uint64_t k = 0; g->t && k < g->n_tensors; k++) free((char *)g->t[k].name);
    free(g->meta);
    free(g->t);
    if (g->map) munmap((void *)g->map, g->size);
    free(g);
}

/* The file in four passes: header, metadata, tensor directory, layout. */
static int parse(KataliHipGguf *g, char *why, size_t why_cap) {
    Reader r = {g->map, g->size, 0, why, why_cap, 0};
    uint32_t magic = 0;
    if (left(&r) < 4) return refuse(&r, "too short for a GGUF header");
    u32_at(&r, &magic, "the magic");
    if (magic != 0x46554747u) return refuse(&r, "no GGUF magic at the start of the file");
    if (u32_at(&r, &g->version, "the version")) return -1;
    if (g->version < 1 || g->version > 3) return refuse(&r, "GGUF version %u (versions 1 to 3 are read)", g->version);
    if (fixed(&r, 8, &g->n_tensors, "the tensor count") || fixed(&r, 8, &g->n_meta, "the metadata count"))
        return -1;
    /* every entry takes at least one byte: larger counts cannot be real */
    if (g->n_tensors > g->size || g->n_meta > g->size)
        return refuse(&r, "%llu tensors / %llu metadata entries in a %llu-byte file",
                      (unsigned long long)g->n_tensors, (unsigned long long)g->n_meta, (unsigned long long)g->size);
    g->meta = (Meta *)calloc(g->n_meta ? g->n_meta : 1, sizeof(Meta));
    g->t = (KataliHipGgufTensor *)calloc(g->n_tensors ? g->n_tensors : 1, sizeof(KataliHipGgufTensor));
    if (!g->meta || !g->t) return refuse(&r, "out of memory");

    for (uint64_t k = 0; k < g->n_meta; k++)
        if (read_meta(&r, &g->meta[k])) return -1;
    /* general.alignment, when an integer in [8, 2^20]; 32 otherwise */
    g->alignment = 32;
    const Meta *al = meta_find(g, "general.alignment");
    if (al && !value_float(al->vt) && value_width(al->vt) && (uint64_t)al->num >= 8 &&
        (uint64_t)al->num <= (1u << 20))
        g->alignment = (uint64_t)al->num;

    for (uint64_t k = 0; k < g->n_tensors; k++)
        if (read_tensor(&r, &g->t[k])) return -1;

    /* data section: the directory's end rounded up to the alignment */
    g->data_offset = (r.at + g->alignment - 1) / g->alignment * g->alignment;
    if (g->data_offset > g->size) return refuse(&r, "the data section would start past the end of the file");
    const uint64_t data = g->size - g->data_offset;
    for (uint64_t k = 0; k < g->n_tensors; k++) {
        KataliHipGgufTensor *t = &g->t[k];
        if (t->offset > data)
            return refuse(&r, "tensor '%s' starts %llu bytes into a %llu-byte data section", t->name,
                          (unsigned long long)t->offset, (unsigned long long)data);
        const uint64_t bytes = katali_hip_ggml_row_bytes(t->type, t->nbytes);
        if (bytes == 0) {          /* a type this library has no block size for: listed, no data */
            t->nbytes = 0;
            t->data = NULL;
            continue;
        }
        if (bytes > data - t->offset)
            return refuse(&r, "tensor '%s' needs %llu bytes, %llu remain after its offset", t->name,
                          (unsigned long long)bytes, (unsigned long long)(data - t->offset));
        t->nbytes = bytes;
        t->data = g->map + g->data_offset + t->offset;
    }
    return 0;
}

int katali_hip_gguf_open(const char *path, KataliHipGguf **out, char *err, size_t cap) {
    if (!path || !out) return -1;
    *out = NULL;
    const int fd = open(path, O_RDONLY);
    struct stat st;
    const char *why = fd < 0 ? "open failed" : fstat(fd, &st) != 0 ? "stat failed" : st.st_size <= 0 ? "empty file" : NULL;
    if (why) {
        if (fd >= 0) close(fd);
        if (err && cap) snprintf(err, cap, "%s: %s", path, why);
        return -1;
    }
    void *m = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        if (err && cap) snprintf(err, cap, "%s: mmap failed", path);
        return -1;
    }
    KataliHipGguf *g = (KataliHipGguf *)calloc(1, sizeof *g);
    if (!g) {
        munmap(m, (size_t)st.st_size);
        return -1;
    }
    g->map = (const uint8_t *)m;
    g->size = (uint64_t)st.st_size;
    if (parse(g, err, cap) != 0) {
        katali_hip_gguf_close(g);
        return -1;
    }
    *out = g;
    return 0;
}

uint32_t katali_hip_gguf_version(const KataliHipGguf *g) { return g ? g->version : 0; }
uint64_t katali_hip_gguf_tensor_count(const KataliHipGguf *g) { return g ? g->n_tensors : 0; }
uint64_t katali_hip_gguf_alignment(const KataliHipGguf *g) { return g ? g->alignment : 0; }
uint64_t katali_hip_gguf_data_offset(const KataliHipGguf *g) { return g ? g->data_offset : 0; }
const uint8_t *katali_hip_gguf_base(const KataliHipGguf *g) { return g ? g->map : NULL; }

int katali_hip_gguf_tensor(const KataliHipGguf *g, uint64_t i, KataliHipGgufTensor *out) {
    if (!g || !out || i >= g->n_tensors) return -1;
    *out = g->t[i];
    return 0;
}

static const KataliHipGgufTensor *find(const KataliHipGguf *g, const char *name) {
    for (uint64_t k = 0; g && name && k < g->n_tensors; k++)
        if (strcmp(g->t[k].name, name) == 0) return &g->t[k];
    return NULL;
}

int katali_hip_gguf_find(const KataliHipGguf *g, const char *name, KataliHipGgufTensor *out) {
    const KataliHipGgufTensor *t = find(g, name);
    if (!t || !out) return -1;
    *out = *t;
    return 0;
}

int64_t katali_hip_gguf_get_int(const KataliHipGguf *g, const char *key, int64_t def) {
    const Meta *m = g ? meta_find(g, key) : NULL;
    if (!m || m->vt == VT_ARRAY || m->vt == VT_STRING) return def;
    return value_float(m->vt) ? (int64_t)m->real : m->num;
}

double katali_hip_gguf_get_float(const KataliHipGguf *g, const char *key, double def) {
    const Meta *m = g ? meta_find(g, key) : NULL;
    if (!m || m->vt == VT_ARRAY || m->vt == VT_STRING) return def;
    return value_float(m->vt) ? m->real : (double)m->num;
}

const char *katali_hip_gguf_get_str(const KataliHipGguf *g, const char *key, size_t *len_out) {
    const Meta *m = g ? meta_find(g, key) : NULL;
    if (!m || m->vt != VT_STRING) return NULL;
    if (len_out) *len_out = (size_t)m->str_len;
    return (const char *)m->str;
}

/* ---- device weight cache --------------------------------------------------- */
static uint64_t budget_from_env(uint64_t b) {
    if (b) return b;
    const char *e = getenv("KATALI_VRAM_GB");
    const double gb = e ? atof(e) : 0.0;
    return gb > 0 ? (uint64_t)(gb * 1073741824.0) : 0;   /* 0: no cap */
}

struct KataliHipWeights {
    const KataliHipGguf *g;
    uint64_t budget, resident;
    void **dev;   /* per tensor index */
};

int katali_hip_weights_create(const KataliHipGguf *g, uint64_t budget, KataliHipWeights **out) {
    if (!g || !out) return gguf_fail("null argument");
    KataliHipWeights *w = (KataliHipWeights *)calloc(1, sizeof *w);
    if (!w || !(w->dev = (void **)calloc(g->n_tensors ? g->n_tensors : 1, sizeof(void *)))) {
        free(w);
        return gguf_fail("out of memory");
    }
    w->g = g;
    w->budget = budget_from_env(budget);
    *out = w;
    return 0;
}

void katali_hip_weights_destroy(KataliHipWeights *w) {
    if (!w) return;
    for (uint64_t k = 0; k < w->g->n_tensors; k++)
        if (w->dev[k]) katali_gpu_free(w->dev[k]);
    free(w->dev);
    free(w);
}

const void *katali_hip_weights_get(KataliHipWeights *w, const char *name) {
    if (!w) return NULL;
    const KataliHipGgufTensor *t = find(w->g, name);
    if (!t) { gguf_fail("tensor '%s' not in the file", name ? name : "(null)"); return NULL; }
    const uint64_t k = (uint64_t)(t - w->g->t);
    if (w->dev[k]) return w->dev[k];
    if (!t->data) { gguf_fail("tensor '%s' has no known block size (type %u)", t->name, t->type); return NULL; }
    if (w->budget && w->resident + t->nbytes > w->budget) {
        gguf_fail("tensor '%s' (%llu bytes) passes the VRAM budget (%llu of %llu held)", t->name,
                  (unsigned long long)t->nbytes, (unsigned long long)w->resident, (unsigned long long)w->budget);
        return NULL;
    }
    void *d = NULL;
    if (katali_gpu_malloc(&d, (size_t)t->nbytes) != KATALI_GPU_OK) {
        gguf_fail("device allocation of %llu bytes for '%s': %s", (unsigned long long)t->nbytes, t->name,
                  katali_gpu_last_error());
        return NULL;
    }
    if (katali_gpu_upload(d, t->data, (size_t)t->nbytes) != KATALI_GPU_OK) {
        katali_gpu_free(d);
        gguf_fail("upload of '%s': %s", t->name, katali_gpu_last_error());
        return NULL;
    }
    w->dev[k] = d;
    w->resident += t->nbytes;
    return d;
}

uint64_t katali_hip_weights_resident_bytes(const KataliHipWeights *w) { return w ? w->resident : 0; }

/* ---- MoE layer assembly ------------------------------------------------------ */
static const KataliHipGgufTensor *blk(const KataliHipGguf *g, uint32_t layer, const char *what) {
    char name[96];
    snprintf(name, sizeof name, "blk.%u.%s.weight", layer, what);
    return find(g, name);
}

static int quant_ok(uint32_t t) { return t == KATALI_HIP_TYPE_Q4_K || t == KATALI_HIP_TYPE_Q6_K; }

/* Shape of a layer's expert stacks: gate/up [n_expert][ffn][hidden],
 * down [n_expert][hidden][ffn] (GGUF dims reversed), gate type == up type. */
static int expert_shape(const KataliHipGguf *g, uint32_t layer, KataliHipMoe *m, const KataliHipGgufTensor **ts) {
    const KataliHipGgufTensor *gt = blk(g, layer, "ffn_gate_exps"), *ut = blk(g, layer, "ffn_up_exps"),
                              *dt = blk(g, layer, "ffn_down_exps");
    if (!gt || !ut || !dt) return gguf_fail("layer %u: ffn_{gate,up,down}_exps missing", layer);
    if (gt->n_dims != 3 || ut->n_dims != 3 || dt->n_dims != 3)
        return gguf_fail("layer %u: expert stacks are not 3-D", layer);
    const uint64_t hidden = gt->dims[0], ffn = gt->dims[1], ne = gt->dims[2];
    if (ut->dims[0] != hidden || ut->dims[1] != ffn || ut->dims[2] != ne || dt->dims[0] != ffn ||
        dt->dims[1] != hidden || dt->dims[2] != ne)
        return gguf_fail("layer %u: gate/up/down expert shapes disagree", layer);
    if (!quant_ok(gt->type) || gt->type != ut->type || !quant_ok(dt->type))
        return gguf_fail("layer %u: expert types %u/%u/%u (Q4_K or Q6_K, gate == up)", layer, gt->type, ut->type,
                         dt->type);
    if (hidden % 256 || ffn % 256 || ne == 0 || ne > 512 || hidden > 65536 || ffn > 65536)
        return gguf_fail("layer %u: hidden %llu, ffn %llu, %llu experts do not fit the fused layer", layer,
                         (unsigned long long)hidden, (unsigned long long)ffn, (unsigned long long)ne);
    memset(m, 0, sizeof *m);
    m->struct_size = sizeof *m;
    m->gate_type = gt->type;
    m->up_type = ut->type;
    m->down_type = dt->type;
    m->hidden = (uint32_t)hidden;
    m->ffn = (uint32_t)ffn;
    m->n_expert = (uint32_t)ne;
    ts[0] = gt;
    ts[1] = ut;
    ts[2] = dt;
    return 0;
}

int katali_hip_gguf_moe_layer(KataliHipWeights *w, uint32_t layer, KataliHipMoe *moe, const float **router,
                              const float **norm_w) {
    if (!w || !moe) return gguf_fail("null argument");
    const KataliHipGguf *g = w->g;
    const KataliHipGgufTensor *ts[3];
    KataliHipMoe m;
    if (expert_shape(g, layer, &m, ts)) return -1;
    if (!(m.gate_exps = katali_hip_weights_get(w, ts[0]->name)) ||
        !(m.up_exps = katali_hip_weights_get(w, ts[1]->name)) ||
        !(m.down_exps = katali_hip_weights_get(w, ts[2]->name)))
        return -1;
    const KataliHipGgufTensor *sg = blk(g, layer, "ffn_gate_shexp"), *su = blk(g, layer, "ffn_up_shexp"),
                              *sd = blk(g, layer, "ffn_down_shexp");
    if (sg || su || sd) {
        if (!sg || !su || !sd) return gguf_fail("layer %u: incomplete shared expert", layer);
        if (sg->n_dims != 2 || su->n_dims != 2 || sd->n_dims != 2 || sg->dims[0] != m.hidden ||
            sg->dims[1] != m.ffn || su->dims[0] != m.hidden || su->dims[1] != m.ffn || sd->dims[0] != m.ffn ||
            sd->dims[1] != m.hidden || sg->type != m.gate_type || su->type != m.up_type || sd->type != m.down_type)
            return gguf_fail("layer %u: the shared expert's shape or types differ from the routed experts'", layer);
        if (!(m.gate_shexp = katali_hip_weights_get(w, sg->name)) ||
            !(m.up_shexp = katali_hip_weights_get(w, su->name)) ||
            !(m.down_shexp = katali_hip_weights_get(w, sd->name)))
            return -1;
    }
    if (router) {
        const KataliHipGgufTensor *r = blk(g, layer, "ffn_gate_inp");
        if (!r || r->type != 0 || r->n_dims != 2 || r->dims[0] != m.hidden || r->dims[1] != m.n_expert)
            return gguf_fail("layer %u: ffn_gate_inp missing or not F32 [%u][%u]", layer, m.n_expert, m.hidden);
        if (!(*router = (const float *)katali_hip_weights_get(w, r->name))) return -1;
    }
    if (norm_w) {
        const KataliHipGgufTensor *n = blk(g, layer, "ffn_norm");
        if (!n || n->type != 0 || n->dims[0] != m.hidden)
            return gguf_fail("layer %u: ffn_norm missing or not F32 [%u]", layer, m.hidden);
        if (!(*norm_w = (const float *)katali_hip_weights_get(w, n->name))) return -1;
    }
    *moe = m;
    return 0;
}

/* ---- expert VRAM tier ---------------------------------------------------------- */
typedef struct TierSlot {
    int64_t key;         /* layer * 65536 + expert, -1 when empty */
    uint64_t used;       /* tick of the last call that asked for it */
    uint64_t ready;      /* pipelined: the stager mark after which no queued work reads it (0: none) */
} TierSlot;

struct KataliHipExpertTier {
    const KataliHipGguf *g;
    KataliHipMoe shape;             /* types and sizes every layer must match */
    uint64_t eb[3];                 /* one expert's bytes: gate, up, down */
    uint8_t *pool[3];               /* device pools [n_slots][eb] */
    uint32_t n_slots;
    TierSlot *slot;
    uint64_t tick;
    void *stager;                   /* pipelined uploads, or NULL (synchronous) */
    uint64_t mark_call;             /* pipelined: slots used at calls >= this have no ready mark yet */
    KataliHipTierStats st;
};

/* KATALI_UPLOAD_BATCH=1: tiers start pipelined with the default ring */
static int upload_batch_from_env(void) {
    const char *e = getenv("KATALI_UPLOAD_BATCH");
    return e && e[0] == '1';
}

int katali_hip_tier_create(const KataliHipGguf *g, uint32_t layer, uint64_t budget, uint32_t max_slots,
                           KataliHipExpertTier **out) {
    if (!g || !out || max_slots == 0 || max_slots > 512) return gguf_fail("tier: bad arguments");
    KataliHipExpertTier *t = (KataliHipExpertTier *)calloc(1, sizeof *t);
    if (!t) return gguf_fail("out of memory");
    const KataliHipGgufTensor *ts[3];
    if (expert_shape(g, layer, &t->shape, ts)) {
        free(t);
        return -1;
    }
    t->g = g;
    for (int k = 0; k < 3; k++) t->eb[k] = ts[k]->nbytes / t->shape.n_expert;
    const uint64_t per = t->eb[0] + t->eb[1] + t->eb[2];
    budget = budget_from_env(budget);
    uint64_t n = budget ? budget / per : max_slots;
    if (n > max_slots) n = max_slots;
    if (n == 0) {
        free(t);
        return gguf_fail("tier: budget %llu holds no expert of %llu bytes", (unsigned long long)budget,
                         (unsigned long long)per);
    }
    t->n_slots = (uint32_t)n;
    t->slot = (TierSlot *)calloc(n, sizeof(TierSlot));
    if (!t->slot) {
        free(t);
        return gguf_fail("out of memory");
    }
    for (uint32_t s = 0; s < n; s++) t->slot[s].key = -1;
    for (int k = 0; k < 3; k++)
        if (katali_gpu_malloc((void **)&t->pool[k], (size_t)(t->eb[k] * n)) != KATALI_GPU_OK) {
            gguf_fail("tier: device pool of %llu bytes: %s", (unsigned long long)(t->eb[k] * n),
                      katali_gpu_last_error());
            katali_hip_tier_destroy(t);
            return -1;
        }
    t->st.n_slots = t->n_slots;
    if (upload_batch_from_env() && katali_hip_tier_pipeline(t, 0, 0)) {
        katali_hip_tier_destroy(t);
        return -1;
    }
    *out = t;
    return 0;
}

int katali_hip_tier_pipeline(KataliHipExpertTier *t, uint64_t chunk_bytes, uint32_t n_chunks) {
    if (!t) return gguf_fail("tier: null argument");
    if (t->stager) return 0;
    if (!chunk_bytes) chunk_bytes = 4u << 20;
    if (!n_chunks) n_chunks = 4;
    if (katali_gpu_stager_create(chunk_bytes, n_chunks, &t->stager) != KATALI_GPU_OK) {
        t->stager = NULL;
        return gguf_fail("tier: stager: %s", katali_gpu_last_error());
    }
    /* everything queued so far may still read any slot: the first upload
     * into each waits for this point */
    uint64_t mark = 0;
    if (katali_gpu_stager_mark(t->stager, &mark) != KATALI_GPU_OK) {
        katali_gpu_stager_destroy(t->stager);
        t->stager = NULL;
        return gguf_fail("tier: stager mark: %s", katali_gpu_last_error());
    }
    for (uint32_t k = 0; k < t->n_slots; k++) t->slot[k].ready = mark;
    t->mark_call = t->tick + 1;
    return 0;
}

/* A mark covering the work queued so far, taken at a call's first miss:
 * the slots used by the calls since the last mark (whose readers are all
 * queued by now) get it as their ready mark. */
static int tier_mark(KataliHipExpertTier *t, uint64_t tick) {
    uint64_t mark = 0;
    if (katali_gpu_stager_mark(t->stager, &mark) != KATALI_GPU_OK)
        return gguf_fail("tier: stager mark: %s", katali_gpu_last_error());
    for (uint32_t k = 0; k < t->n_slots; k++)
        if (t->slot[k].used >= t->mark_call && t->slot[k].used < tick) t->slot[k].ready = mark;
    t->mark_call = tick;
    return 0;
}

void katali_hip_tier_destroy(KataliHipExpertTier *t) {
    if (!t) return;
    if (t->stager) katali_gpu_stager_destroy(t->stager);
    for (int k = 0; k < 3; k++)
        if (t->pool[k]) katali_gpu_free(t->pool[k]);
    free(t->slot);
    free(t);
}

int katali_hip_tier_layer(KataliHipExpertTier *t, uint32_t layer, const int32_t *ids, int n_sel, int32_t *slots,
                          KataliHipMoe *moe) {
    if (!t || !moe || (n_sel > 0 && (!ids || !slots))) return gguf_fail("tier: null argument");
    if (n_sel < 0 || (uint32_t)n_sel > t->n_slots || n_sel > 16)
        return gguf_fail("tier: %d experts for %u slots", n_sel, t->n_slots);
    const KataliHipGgufTensor *ts[3];
    KataliHipMoe m;
    if (expert_shape(t->g, layer, &m, ts)) return -1;
    if (m.hidden != t->shape.hidden || m.ffn != t->shape.ffn || m.gate_type != t->shape.gate_type ||
        m.down_type != t->shape.down_type)
        return gguf_fail("tier: layer %u's experts have another shape than the slots", layer);
    for (int i = 0; i < n_sel; i++)   /* before any slot changes */
        if (ids[i] < 0 || (uint32_t)ids[i] >= m.n_expert)
            return gguf_fail("tier: expert id %d outside 0..%u", ids[i], m.n_expert - 1);
    const uint64_t tick = ++t->tick;
    int uploads = 0;
    for (int i = 0; i < n_sel; i++) {
        const int64_t key = (int64_t)layer * 65536 + ids[i];
        uint32_t s = t->n_slots;
        for (uint32_t k = 0; k < t->n_slots; k++)
            if (t->slot[k].key == key) { s = k; break; }
        if (s < t->n_slots) {
            t->st.hits++;
        } else {
            /* the least recently used slot not asked for in this call (an
             * empty slot first: its tick is 0) */
            for (uint32_t k = 0; k < t->n_slots; k++)
                if (t->slot[k].used != tick && (s == t->n_slots || t->slot[k].used < t->slot[s].used)) s = k;
            if (t->stager && t->mark_call != tick && tier_mark(t, tick)) {
                if (uploads) katali_gpu_stager_fence(t->stager);
                return -1;
            }
            for (int p = 0; p < 3; p++) {
                uint8_t *dst = t->pool[p] + t->eb[p] * s;
                const uint8_t *src = ts[p]->data + t->eb[p] * (uint64_t)ids[i];
                const int rc = t->stager ? katali_gpu_stager_upload(t->stager, dst, src, t->eb[p], t->slot[s].ready)
                                         : katali_gpu_upload(dst, src, (size_t)t->eb[p]);
                if (rc != KATALI_GPU_OK) {
                    t->slot[s].key = -1;
                    gguf_fail("tier: upload: %s", katali_gpu_last_error());
                    if (t->stager && uploads) katali_gpu_stager_fence(t->stager);   /* the slots filled before it */
                    return -1;
                }
            }
            uploads++;
            t->slot[s].key = key;
            t->st.misses++;
            t->st.uploaded_bytes += t->eb[0] + t->eb[1] + t->eb[2];
        }
        t->slot[s].used = tick;
        slots[i] = (int32_t)s;
    }
    /* the work the caller queues next waits for this call's DMAs */
    if (t->stager && uploads && katali_gpu_stager_fence(t->stager) != KATALI_GPU_OK)
        return gguf_fail("tier: stager fence: %s", katali_gpu_last_error());
    m.n_expert = t->n_slots;
    m.gate_exps = t->pool[0];
    m.up_exps = t->pool[1];
    m.down_exps = t->pool[2];
    *moe = m;
    return 0;
}

void katali_hip_tier_stats(const KataliHipExpertTier *t, KataliHipTierStats *out) {
    if (t && out) *out = t->st;
}
