/* katali_hip_gguf.c — GGUF reader, device weight cache, MoE layer assembly
 * and expert VRAM tier (declarations and contracts in katali_hip_gguf.h).
 *
 * The reader maps the file read-only and walks it with a bounds-checked
 * cursor; every length and offset from the file is checked against the bytes
 * left before it is used. Its acceptance rules are the engine reader's
 * (V/src/gguf_reader.c:351-543) so that both open and refuse the same files.
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
enum { GV_U8, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64 };

typedef struct Kv {
    char *key;
    uint32_t type;
    uint64_t u;          /* unsigned view (0 for floats and strings) */
    int64_t i;           /* signed view */
    double f;            /* float view */
    const uint8_t *s;    /* string bytes in the map */
    uint64_t s_len;
} Kv;

struct KataliHipGguf {
    const uint8_t *map;
    uint64_t size;
    uint32_t version;
    uint64_t n_kv, n_tensors, alignment, data_offset;
    Kv *kv;
    KataliHipGgufTensor *t;
};

typedef struct Cur {
    const uint8_t *m;
    uint64_t size, pos;
    const char *bad;     /* first failure, NULL while fine */
} Cur;

static const uint8_t *take(Cur *c, uint64_t n) {
    if (c->bad) return NULL;
    if (n > c->size - c->pos) { c->bad = "truncated file"; return NULL; }
    const uint8_t *p = c->m + c->pos;
    c->pos += n;
    return p;
}
static uint64_t rd(Cur *c, unsigned n) {   /* little-endian n-byte unsigned */
    const uint8_t *p = take(c, n);
    uint64_t v = 0;
    if (p) memcpy(&v, p, n);
    return v;
}
static const uint8_t *rd_str(Cur *c, uint64_t *len) {
    const uint64_t n = rd(c, 8);
    const uint8_t *p = take(c, n);
    *len = p ? n : 0;
    return p;
}
static unsigned scalar_bytes(uint32_t t) {
    switch (t) {
        case GV_U8: case GV_I8: case GV_BOOL: return 1;
        case GV_U16: case GV_I16: return 2;
        case GV_U32: case GV_I32: case GV_F32: return 4;
        case GV_U64: case GV_I64: case GV_F64: return 8;
        default: return 0;
    }
}

/* One scalar of type t: numbers into u/i/f as the engine's reader keeps
 * them (gguf_reader.c:246-274), strings as a pointer into the map. */
static void scalar(Cur *c, uint32_t t, Kv *kv) {
    uint64_t v;
    float f32;
    double f64;
    switch (t) {
        case GV_U8: case GV_U16: case GV_U32: case GV_U64:
            kv->u = rd(c, scalar_bytes(t)); kv->i = (int64_t)kv->u; break;
        case GV_I8: kv->i = (int8_t)rd(c, 1); kv->u = (uint64_t)kv->i; break;
        case GV_I16: kv->i = (int16_t)rd(c, 2); kv->u = (uint64_t)kv->i; break;
        case GV_I32: kv->i = (int32_t)rd(c, 4); kv->u = (uint64_t)kv->i; break;
        case GV_I64: kv->i = (int64_t)rd(c, 8); kv->u = (uint64_t)kv->i; break;
        case GV_BOOL: kv->u = rd(c, 1) ? 1u : 0u; kv->i = (int64_t)kv->u; break;
        case GV_F32: v = rd(c, 4); memcpy(&f32, &v, 4); kv->f = f32; break;
        case GV_F64: v = rd(c, 8); memcpy(&f64, &v, 8); kv->f = f64; break;
        case GV_STR: kv->s = rd_str(c, &kv->s_len); break;
        default: if (!c->bad) c->bad = "unsupported metadata value type"; break;
    }
}

/* An array is checked, not kept (the fused path reads no array metadata):
 * nested arrays refused, the count and a fixed-size payload bounded by the
 * bytes left, strings walked one by one (gguf_reader.c:277-330). */
static void array(Cur *c) {
    const uint32_t et = (uint32_t)rd(c, 4);
    const uint64_t n = rd(c, 8);
    if (c->bad) return;
    if (et == GV_ARR) { c->bad = "nested metadata arrays are unsupported"; return; }
    if (n > c->size - c->pos) { c->bad = "array count exceeds file size"; return; }
    const unsigned es = scalar_bytes(et);
    if (es) {
        if (n > (c->size - c->pos) / es) { c->bad = "array payload exceeds file size"; return; }
        take(c, n * es);
        return;
    }
    if (et != GV_STR) { c->bad = "unsupported metadata array element type"; return; }
    for (uint64_t k = 0; k < n && !c->bad; k++) {
        uint64_t len;
        rd_str(c, &len);
    }
}

static const Kv *kv_find(const KataliHipGguf *g, const char *key) {
    for (uint64_t k = 0; k < g->n_kv; k++)
        if (g->kv[k].key && strcmp(g->kv[k].key, key) == 0) return &g->kv[k];
    return NULL;
}

void katali_hip_gguf_close(KataliHipGguf *g) {
    if (!g) return;
    for (uint64_t k = 0; g->kv && k < g->n_kv; k++) free(g->kv[k].key);
    for (uint64_t k = 0; g->t && k < g->n_tensors; k++) free((char *)g->t[k].name);
    free(g->kv);
    free(g->t);
    if (g->map) munmap((void *)g->map, g->size);
    free(g);
}

static char *dup_bytes(const uint8_t *p, uint64_t n) {
    char *s = (char *)malloc(n + 1);
    if (s) {
        if (n) memcpy(s, p, n);
        s[n] = 0;
    }
    return s;
}

static int parse(KataliHipGguf *g, char *err, size_t cap) {
    Cur c = {g->map, g->size, 0, NULL};
#define BAD(...) do { if (err && cap) snprintf(err, cap, __VA_ARGS__); return -1; } while (0)
    if (rd(&c, 4) != 0x46554747u || c.bad) BAD("not a GGUF file (bad magic)");
    g->version = (uint32_t)rd(&c, 4);
    if (c.bad || g->version < 1 || g->version > 3) BAD("unsupported GGUF version %u", g->version);
    g->n_tensors = rd(&c, 8);
    g->n_kv = rd(&c, 8);
    if (c.bad) BAD("truncated GGUF header");
    if (g->n_tensors > g->size || g->n_kv > g->size) BAD("implausible header counts");
    g->kv = (Kv *)calloc(g->n_kv ? g->n_kv : 1, sizeof(Kv));
    g->t = (KataliHipGgufTensor *)calloc(g->n_tensors ? g->n_tensors : 1, sizeof(KataliHipGgufTensor));
    if (!g->kv || !g->t) BAD("out of memory");
    for (uint64_t k = 0; k < g->n_kv && !c.bad; k++) {
        Kv *kv = &g->kv[k];
        uint64_t klen;
        const uint8_t *kp = rd_str(&c, &klen);
        if (c.bad) break;
        if (!(kv->key = dup_bytes(kp, klen))) BAD("out of memory");
        kv->type = (uint32_t)rd(&c, 4);
        if (c.bad) break;
        if (kv->type == GV_ARR) array(&c);
        else scalar(&c, kv->type, kv);
    }
    if (c.bad) BAD("%s (at offset %llu)", c.bad, (unsigned long long)c.pos);
    g->alignment = 32;
    const Kv *a = kv_find(g, "general.alignment");
    if (a && a->type != GV_ARR && a->u >= 8 && a->u <= (1u << 20)) g->alignment = a->u;

    for (uint64_t k = 0; k < g->n_tensors && !c.bad; k++) {
        KataliHipGgufTensor *t = &g->t[k];
        uint64_t nlen;
        const uint8_t *np = rd_str(&c, &nlen);
        if (c.bad) break;
        if (!(t->name = dup_bytes(np, nlen))) BAD("out of memory");
        t->n_dims = (uint32_t)rd(&c, 4);
        if (c.bad) break;
        if (t->n_dims < 1 || t->n_dims > 4) { c.bad = "tensor rank out of range"; break; }
        int over = 0;
        for (uint32_t d = 0; d < t->n_dims; d++) t->dims[d] = rd(&c, 8);
        if (c.bad) break;
        uint64_t n = 1;
        for (uint32_t d = 0; d < t->n_dims; d++) {
            if (!t->dims[d] || n > UINT64_MAX / t->dims[d]) over = 1;
            else n *= t->dims[d];
        }
        if (over) { c.bad = "tensor element count overflows"; break; }
        t->type = (uint32_t)rd(&c, 4);
        t->offset = rd(&c, 8);
        t->nbytes = n;   /* element count until resolved below */
    }
    if (c.bad) BAD("%s (at offset %llu)", c.bad, (unsigned long long)c.pos);

    const uint64_t rem = c.pos % g->alignment;
    g->data_offset = rem ? c.pos + (g->alignment - rem) : c.pos;
    if (g->data_offset > g->size) BAD("tensor data offset past end of file");
    const uint64_t data = g->size - g->data_offset;
    for (uint64_t k = 0; k < g->n_tensors; k++) {
        KataliHipGgufTensor *t = &g->t[k];
        const uint64_t nb = katali_hip_ggml_row_bytes(t->type, t->nbytes);
        if (t->offset > data) BAD("tensor '%s' offset past end of file", t->name);
        if (!nb) { t->nbytes = 0; t->data = NULL; continue; }
        if (nb > data - t->offset) BAD("tensor '%s' (%llu bytes) is truncated", t->name, (unsigned long long)nb);
        t->nbytes = nb;
        t->data = g->map + g->data_offset + t->offset;
    }
#undef BAD
    return 0;
}

int katali_hip_gguf_open(const char *path, KataliHipGguf **out, char *err, size_t cap) {
    if (!path || !out) return -1;
    *out = NULL;
    const int fd = open(path, O_RDONLY);
    struct stat st;
    if (fd < 0 || fstat(fd, &st) != 0 || st.st_size <= 0) {
        if (fd >= 0) close(fd);
        if (err && cap) snprintf(err, cap, "cannot open file: %s", path);
        return -1;
    }
    void *m = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        if (err && cap) snprintf(err, cap, "cannot map file: %s", path);
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
    const Kv *kv = g ? kv_find(g, key) : NULL;
    if (!kv || kv->type == GV_ARR || kv->type == GV_STR) return def;
    if (kv->type == GV_F32 || kv->type == GV_F64) return (int64_t)kv->f;
    return kv->i;
}

double katali_hip_gguf_get_float(const KataliHipGguf *g, const char *key, double def) {
    const Kv *kv = g ? kv_find(g, key) : NULL;
    if (!kv || kv->type == GV_ARR || kv->type == GV_STR) return def;
    if (kv->type == GV_F32 || kv->type == GV_F64) return kv->f;
    return (double)kv->i;
}

const char *katali_hip_gguf_get_str(const KataliHipGguf *g, const char *key, size_t *len_out) {
    const Kv *kv = g ? kv_find(g, key) : NULL;
    if (!kv || kv->type != GV_STR) return NULL;
    if (len_out) *len_out = (size_t)kv->s_len;
    return (const char *)kv->s;
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
} TierSlot;

struct KataliHipExpertTier {
    const KataliHipGguf *g;
    KataliHipMoe shape;             /* types and sizes every layer must match */
    uint64_t eb[3];                 /* one expert's bytes: gate, up, down */
    uint8_t *pool[3];               /* device pools [n_slots][eb] */
    uint32_t n_slots;
    TierSlot *slot;
    uint64_t tick;
    KataliHipTierStats st;
};

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
    *out = t;
    return 0;
}

void katali_hip_tier_destroy(KataliHipExpertTier *t) {
    if (!t) return;
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
    const uint64_t tick = ++t->tick;
    for (int i = 0; i < n_sel; i++) {
        if (ids[i] < 0 || (uint32_t)ids[i] >= m.n_expert)
            return gguf_fail("tier: expert id %d outside 0..%u", ids[i], m.n_expert - 1);
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
            for (int p = 0; p < 3; p++)
                if (katali_gpu_upload(t->pool[p] + t->eb[p] * s, ts[p]->data + t->eb[p] * (uint64_t)ids[i],
                                      (size_t)t->eb[p]) != KATALI_GPU_OK) {
                    t->slot[s].key = -1;
                    return gguf_fail("tier: upload: %s", katali_gpu_last_error());
                }
            t->slot[s].key = key;
            t->st.misses++;
            t->st.uploaded_bytes += t->eb[0] + t->eb[1] + t->eb[2];
        }
        t->slot[s].used = tick;
        slots[i] = (int32_t)s;
    }
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
