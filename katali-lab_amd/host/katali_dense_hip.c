/* katali_dense_hip.c — engine-side dense GEMV shim over libkatali_hip.
 *
 * Same contract as the engine's CUDA shim
 * (vendor/katali_gguf_dense/src/katali_dense_cuda.c:7-79):
 *   - opt-in: KATALI_HIP (or the engine's existing KATALI_CUDA switch) must
 *     start with 1, y or Y, and the device probe must succeed; the decision
 *     is taken once and logged to stderr (katali_dense_cuda.c:14-22);
 *   - device copies of weights are cached by host pointer, up to 256
 *     (katali_dense_cuda.c:7-8,36-44);
 *   - shared device x/y buffers grow to max(cols, rows) floats (:24-34);
 *   - each call is upload x -> matvec -> download y, synchronous (:46-56);
 *   - any failure returns -1 and the caller computes on the CPU
 *     (gguf_model.c:500-504,533-541);
 *   - shutdown frees everything (:75-79).
 * Plain C over the loader; no HIP headers. Single caller thread, like the
 * reference (process-global state, no locks). */
#include "katali_dense_hip.h"

#include "katali_hip_loader.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    const void *host;
    void *dev;
    uint64_t bytes;
} DenseWeight;

#define MAX_WEIGHTS 256
static DenseWeight g_w[MAX_WEIGHTS];
static int g_nw;
static float *g_x, *g_y;
static uint64_t g_cap;
static int g_checked, g_enabled;

static int env_on(const char *name) {
    const char *e = getenv(name);
    return e && (e[0] == '1' || e[0] == 'y' || e[0] == 'Y');
}

int katali_dense_hip_enabled(void) {
    if (!g_checked) {
        g_checked = 1;
        g_enabled = (env_on("KATALI_HIP") || env_on("KATALI_CUDA")) && katali_gpu_probe() != 0;
        fprintf(stderr, "phase: dense hip %s (%s)\n", g_enabled ? "ON" : "OFF", katali_gpu_status());
    }
    return g_enabled;
}

static int ensure_buffers(uint64_t cols, uint64_t rows) {
    const uint64_t need = cols > rows ? cols : rows;
    if (g_cap >= need && g_x && g_y) return 0;
    if (g_x) katali_gpu_free(g_x);
    if (g_y) katali_gpu_free(g_y);
    g_x = g_y = NULL;
    g_cap = 0;
    if (katali_gpu_malloc((void **)&g_x, need * sizeof(float)) != KATALI_GPU_OK) return -1;
    if (katali_gpu_malloc((void **)&g_y, need * sizeof(float)) != KATALI_GPU_OK) {
        katali_gpu_free(g_x);
        g_x = NULL;
        return -1;
    }
    g_cap = need;
    return 0;
}

static void *device_weight(const void *host, uint64_t bytes) {
    for (int i = 0; i < g_nw; i++)
        if (g_w[i].host == host) return g_w[i].bytes == bytes ? g_w[i].dev : NULL;
    if (g_nw >= MAX_WEIGHTS || !host || !bytes) return NULL;
    void *d = NULL;
    if (katali_gpu_malloc(&d, (size_t)bytes) != KATALI_GPU_OK) return NULL;
    if (katali_gpu_upload(d, host, (size_t)bytes) != KATALI_GPU_OK) {
        katali_gpu_free(d);
        return NULL;
    }
    g_w[g_nw].host = host;
    g_w[g_nw].dev = d;
    g_w[g_nw].bytes = bytes;
    g_nw++;
    return d;
}

int katali_dense_hip_matvec(uint32_t type, const void *w, uint64_t w_bytes, uint64_t rows, uint64_t cols,
                            const float *x, float *y) {
    if (!katali_dense_hip_enabled() || !w || !x || !y) return -1;
    if (!katali_gpu_supports_type(type)) return -1;
    if (ensure_buffers(cols, rows) != 0) return -1;
    void *dw = device_weight(w, w_bytes);
    if (!dw) return -1;
    if (katali_gpu_upload(g_x, x, (size_t)cols * sizeof(float)) != KATALI_GPU_OK) return -1;
    if (katali_gpu_matvec(type, dw, rows, cols, g_x, g_y) != KATALI_GPU_OK) return -1;
    if (katali_gpu_download(y, g_y, (size_t)rows * sizeof(float)) != KATALI_GPU_OK) return -1;
    return 0;
}

int katali_dense_hip_matvec_multi(int n, const uint32_t *types, const void *const *ws, const uint64_t *w_bytes,
                                  const uint64_t *rows, uint64_t cols, const float *x, float **ys) {
    if (n <= 0 || n > 4 || !types || !ws || !w_bytes || !rows || !ys || !x || !katali_dense_hip_enabled()) return -1;
    /* One launch for all n tensors: their outputs sit back to back in g_y. */
    uint64_t total = 0, off[4];
    for (int i = 0; i < n; i++) {
        if (!ws[i] || !ys[i] || types[i] == 0 /* F32: single matvec only */ || !katali_gpu_supports_type(types[i]))
            return -1;
        off[i] = total;
        total += rows[i];
    }
    if (ensure_buffers(cols, total) != 0) return -1;
    const void *dw[4];
    float *dy[4];
    for (int i = 0; i < n; i++) {
        if (!(dw[i] = device_weight(ws[i], w_bytes[i]))) return -1;
        dy[i] = g_y + off[i];
    }
    if (katali_gpu_upload(g_x, x, (size_t)cols * sizeof(float)) != KATALI_GPU_OK) return -1;
    if (katali_gpu_matvec_multi(n, types, dw, rows, cols, g_x, dy) != KATALI_GPU_OK) return -1;
    for (int i = 0; i < n; i++)
        if (katali_gpu_download(ys[i], dy[i], (size_t)rows[i] * sizeof(float)) != KATALI_GPU_OK) return -1;
    return 0;
}

int katali_dense_hip_cached(void) { return g_nw; }

void katali_dense_hip_shutdown(void) {
    for (int i = 0; i < g_nw; i++)
        if (g_w[i].dev) katali_gpu_free(g_w[i].dev);
    if (g_x) katali_gpu_free(g_x);
    if (g_y) katali_gpu_free(g_y);
    memset(g_w, 0, sizeof g_w);
    g_nw = 0;
    g_x = g_y = NULL;
    g_cap = 0;
    g_checked = g_enabled = 0;
}
