/* katali_dense_hip.c — the engine's dense-projection offload over libkatali_hip.
 *
 * What the engine relies on is the contract of the CUDA shim this replaces
 * (vendor/katali_gguf_dense/src/katali_dense_cuda.c:14-79): an opt-in switch
 * read once and logged, synchronous calls from one thread, and -1 on any
 * failure so the caller computes the projection on the CPU
 * (gguf_model.c:500-504,533-541). The mechanics are this file's own:
 *
 *   residency  Device copies of weight matrices, keyed by the host address of
 *              the engine's tensor data, in an open-addressed table that
 *              doubles when half full. There is no fixed tensor limit: a
 *              tensor the device cannot hold (allocation failure) simply
 *              stays on the CPU path. The same address seen with a different
 *              size is a different tensor: its old copy is dropped and the
 *              new one uploaded.
 *   arena      One device block per process for the activations: x (cols
 *              floats) then every output of the call back to back. It grows
 *              to the largest call seen and is reused.
 *   transfer   x is uploaded once per call; the n outputs of a multi call are
 *              computed by one launch and come back in one download, then
 *              are copied to the caller's arrays on the host.
 *
 * Plain C over the loader (katali_gpu_*); no HIP headers. */
#include "katali_dense_hip.h"

#include "katali_hip_loader.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    const void *key;   /* host address of the tensor data; NULL = empty */
    uint64_t size;     /* bytes */
    void *copy;        /* device copy */
} Resident;

typedef struct {
    int decided;       /* the opt-in has been read */
    int on;
    Resident *tab;     /* open addressing, linear probing, power-of-two size */
    uint32_t tab_size, live;
    float *arena;      /* device: [x | outputs] */
    uint64_t arena_floats;
    float *stage;      /* host copy of the outputs of a multi call */
    uint64_t stage_floats;
} DenseState;

static DenseState S;

static int switch_set(const char *name) {
    const char *v = getenv(name);
    return v != NULL && (v[0] == '1' || v[0] == 'y' || v[0] == 'Y');
}

int katali_dense_hip_enabled(void) {
    if (!S.decided) {
        S.decided = 1;
        const int asked = switch_set("KATALI_HIP") || switch_set("KATALI_CUDA");
        S.on = asked && katali_gpu_probe() != 0;
        fprintf(stderr, "phase: dense hip %s (%s)\n", S.on ? "ON" : "OFF",
                asked ? katali_gpu_status() : "KATALI_HIP / KATALI_CUDA not set");
    }
    return S.on;
}

/* ---- residency table ------------------------------------------------------ */

static uint32_t slot_of(const void *key, uint32_t size) {
    /* Fibonacci hashing of the address (tensor data is at least 32-byte aligned) */
    const uint64_t h = ((uint64_t)(uintptr_t)key >> 5) * 0x9E3779B97F4A7C15ull;
    return (uint32_t)(h >> 32) & (size - 1);
}

static Resident *probe_slot(Resident *tab, uint32_t size, const void *key) {
    uint32_t i = slot_of(key, size);
    while (tab[i].key != NULL && tab[i].key != key) i = (i + 1) & (size - 1);
    return &tab[i];
}

static int table_reserve(uint32_t want_live) {
    if (S.tab != NULL && 2 * want_live <= S.tab_size) return 0;
    const uint32_t size = S.tab_size ? 2 * S.tab_size : 64;
    Resident *t = (Resident *)calloc(size, sizeof(Resident));
    if (t == NULL) return -1;
    for (uint32_t i = 0; i < S.tab_size; i++)
        if (S.tab[i].key != NULL) *probe_slot(t, size, S.tab[i].key) = S.tab[i];
    free(S.tab);
    S.tab = t;
    S.tab_size = size;
    return 0;
}

/* The device copy of a weight matrix, uploading it on first use. */
static const void *resident(const void *host, uint64_t size) {
    if (host == NULL || size == 0 || table_reserve(S.live + 1) != 0) return NULL;
    Resident *r = probe_slot(S.tab, S.tab_size, host);
    if (r->key != NULL && r->size == size) return r->copy;
    if (r->key != NULL) {
        /* another tensor now lives at this address: the slot is reused */
        katali_gpu_free(r->copy);
        r->key = NULL;
        S.live--;
    }
    void *d = NULL;
    if (katali_gpu_malloc(&d, (size_t)size) != KATALI_GPU_OK) return NULL;
    if (katali_gpu_upload(d, host, (size_t)size) != KATALI_GPU_OK) {
        katali_gpu_free(d);
        return NULL;
    }
    r->key = host;
    r->size = size;
    r->copy = d;
    S.live++;
    return d;
}

/* ---- activation arena ----------------------------------------------------- */

/* Device room for x (cols floats, rounded to 64 so the outputs stay
 * 256-byte aligned) followed by `outs` output floats; NULL on failure. */
static float *arena_fit(uint64_t cols, uint64_t outs) {
    const uint64_t need = (cols + 63) / 64 * 64 + outs;
    if (S.arena != NULL && S.arena_floats >= need) return S.arena;
    if (S.arena != NULL) katali_gpu_free(S.arena);
    S.arena = NULL;
    S.arena_floats = 0;
    void *d = NULL;
    if (katali_gpu_malloc(&d, (size_t)need * sizeof(float)) != KATALI_GPU_OK) return NULL;
    S.arena = (float *)d;
    S.arena_floats = need;
    return S.arena;
}

static float *arena_out(uint64_t cols) { return S.arena + (cols + 63) / 64 * 64; }

/* ---- entry points --------------------------------------------------------- */

int katali_dense_hip_matvec(uint32_t type, const void *w, uint64_t w_bytes, uint64_t rows, uint64_t cols,
                            const float *x, float *y) {
    if (!katali_dense_hip_enabled() || x == NULL || y == NULL || !katali_gpu_supports_type(type)) return -1;
    const void *dw = resident(w, w_bytes);
    if (dw == NULL || arena_fit(cols, rows) == NULL) return -1;
    float *dy = arena_out(cols);
    if (katali_gpu_upload(S.arena, x, (size_t)cols * sizeof(float)) != KATALI_GPU_OK ||
        katali_gpu_matvec(type, dw, rows, cols, S.arena, dy) != KATALI_GPU_OK ||
        katali_gpu_download(y, dy, (size_t)rows * sizeof(float)) != KATALI_GPU_OK)
        return -1;
    return 0;
}

int katali_dense_hip_matvec_multi(int n, const uint32_t *types, const void *const *ws, const uint64_t *w_bytes,
                                  const uint64_t *rows, uint64_t cols, const float *x, float **ys) {
    if (n < 1 || n > 4 || types == NULL || ws == NULL || w_bytes == NULL || rows == NULL || x == NULL ||
        ys == NULL || !katali_dense_hip_enabled())
        return -1;
    const void *dw[4];
    uint64_t first[4], total = 0;
    for (int i = 0; i < n; i++) {
        /* F32 tensors have their own kernel and no multi form */
        if (ys[i] == NULL || types[i] == KATALI_HIP_TYPE_F32 || !katali_gpu_supports_type(types[i])) return -1;
        if ((dw[i] = resident(ws[i], w_bytes[i])) == NULL) return -1;
        first[i] = total;
        total += rows[i];
    }
    if (arena_fit(cols, total) == NULL) return -1;
    if (S.stage_floats < total) {
        float *h = (float *)realloc(S.stage, (size_t)total * sizeof(float));
        if (h == NULL) return -1;
        S.stage = h;
        S.stage_floats = total;
    }
    float *out = arena_out(cols), *dy[4];
    for (int i = 0; i < n; i++) dy[i] = out + first[i];
    if (katali_gpu_upload(S.arena, x, (size_t)cols * sizeof(float)) != KATALI_GPU_OK ||
        katali_gpu_matvec_multi(n, types, dw, rows, cols, S.arena, dy) != KATALI_GPU_OK ||
        katali_gpu_download(S.stage, out, (size_t)total * sizeof(float)) != KATALI_GPU_OK)
        return -1;
    for (int i = 0; i < n; i++) memcpy(ys[i], S.stage + first[i], (size_t)rows[i] * sizeof(float));
    return 0;
}

int katali_dense_hip_cached(void) { return (int)S.live; }

void katali_dense_hip_shutdown(void) {
    for (uint32_t i = 0; i < S.tab_size; i++)
        if (S.tab[i].key != NULL) katali_gpu_free(S.tab[i].copy);
    if (S.arena != NULL) katali_gpu_free(S.arena);
    free(S.tab);
    free(S.stage);
    memset(&S, 0, sizeof S);   /* the next call reads the switch and probes again */
}
