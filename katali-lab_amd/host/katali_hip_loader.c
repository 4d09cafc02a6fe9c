/* katali_hip_loader.c — runtime discovery of libkatali_hip (see
 * include/katali_hip_loader.h). Plain C, no HIP headers or libraries: the
 * engine that links this stays CPU-only until the probe succeeds. */
#define _GNU_SOURCE
#include "katali_hip_loader.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef _WIN32
#include <windows.h>
typedef HMODULE lib_t;
static lib_t lib_open(const char *p) { return LoadLibraryA(p); }
static void *lib_sym(lib_t l, const char *n) { return (void *)GetProcAddress(l, n); }
static void lib_close(lib_t l) { FreeLibrary(l); }
static const char *lib_err(void) { return "LoadLibrary failed"; }
#define DEFAULT_NAME "katali_hip.dll"
#else
#include <dlfcn.h>
typedef void *lib_t;
static lib_t lib_open(const char *p) { return dlopen(p, RTLD_NOW | RTLD_LOCAL); }
static void *lib_sym(lib_t l, const char *n) { return dlsym(l, n); }
static void lib_close(lib_t l) { dlclose(l); }
static const char *lib_err(void) { const char *e = dlerror(); return e ? e : "unknown dlopen error"; }
#define DEFAULT_NAME "libkatali_hip.so"
#endif

static lib_t g_lib;
static KataliHipApi g_api;
static int g_state;          /* 0 = not tried, 1 = loaded, -1 = failed */
static int g_probed, g_usable;
static char g_status[1600] = "not probed";

#define LOAD(field, name)                                                 \
    do {                                                                  \
        *(void **)(&g_api.field) = lib_sym(g_lib, name);                  \
        if (!g_api.field) { missing = name; goto fail; }                  \
    } while (0)

/* Directory of this loader's own shared object (for the sibling lookup). */
static void self_dir(char *out, size_t cap) {
    out[0] = 0;
#ifndef _WIN32
    Dl_info info;
    if (dladdr((void *)&self_dir, &info) && info.dli_fname) {
        const char *slash = strrchr(info.dli_fname, '/');
        if (slash && (size_t)(slash - info.dli_fname) + 1 < cap) {
            memcpy(out, info.dli_fname, (size_t)(slash - info.dli_fname) + 1);
            out[slash - info.dli_fname + 1] = 0;
        }
    }
#endif
}

static int load(void) {
    if (g_state) return g_state > 0;
    const char *env = getenv("KATALI_HIP_DLL");
    char sibling[1024];
    const char *tried = env;
    if (env && *env) {
        g_lib = lib_open(env);
    } else {
        self_dir(sibling, sizeof sibling - sizeof DEFAULT_NAME);
        strcat(sibling, DEFAULT_NAME);
        tried = sibling;
        g_lib = lib_open(sibling);
        if (!g_lib) { tried = DEFAULT_NAME; g_lib = lib_open(DEFAULT_NAME); }
    }
    if (!g_lib) {
        snprintf(g_status, sizeof g_status, "libkatali_hip not loaded (%s): %s", tried, lib_err());
        g_state = -1;
        return 0;
    }
    const char *missing = NULL;
    LOAD(abi_version, "katali_hip_abi_version");
    LOAD(last_error, "katali_hip_last_error");
    LOAD(probe, "katali_hip_probe");
    LOAD(status, "katali_hip_status");
    LOAD(malloc_, "katali_hip_malloc");
    LOAD(free_, "katali_hip_free");
    LOAD(upload, "katali_hip_upload");
    LOAD(download, "katali_hip_download");
    LOAD(supports_type, "katali_hip_supports_type");
    LOAD(matvec, "katali_hip_matvec");
    LOAD(sync, "katali_hip_sync");
    LOAD(memset_, "katali_hip_memset");
    LOAD(set_stream, "katali_hip_set_stream");
    LOAD(quantize_q8_1, "katali_hip_quantize_q8_1");
    LOAD(matvec_q8, "katali_hip_matvec_q8");
    LOAD(matvec_dp4a, "katali_hip_matvec_dp4a");
    LOAD(block_isums, "katali_hip_block_isums");
    LOAD(moe_layer, "katali_hip_moe_layer");
    LOAD(moe_layer_debug, "katali_hip_moe_layer_debug");
    LOAD(step_advance, "katali_hip_step_advance");
    LOAD(graph_begin, "katali_hip_graph_begin");
    LOAD(graph_end, "katali_hip_graph_end");
    LOAD(graph_launch, "katali_hip_graph_launch");
    LOAD(graph_destroy, "katali_hip_graph_destroy");
    LOAD(event_create, "katali_hip_event_create");
    LOAD(event_record, "katali_hip_event_record");
    LOAD(event_elapsed, "katali_hip_event_elapsed");
    LOAD(event_destroy, "katali_hip_event_destroy");
    LOAD(selftest, "katali_hip_selftest");
    LOAD(synth_fill, "katali_hip_synth_fill");
    LOAD(synth_normal, "katali_hip_synth_normal");
    LOAD(copy, "katali_hip_copy");
    LOAD(argmax, "katali_hip_argmax");
    LOAD(moe_batch, "katali_hip_moe_batch");
    LOAD(matvec_multi, "katali_hip_matvec_multi");
    LOAD(matvec_multi_dp4a, "katali_hip_matvec_multi_dp4a");
    LOAD(rmsnorm, "katali_hip_rmsnorm");
    LOAD(add_rmsnorm, "katali_hip_add_rmsnorm");
    LOAD(rmsnorm_matvec_f32, "katali_hip_rmsnorm_matvec_f32");
    LOAD(moe_route_batch, "katali_hip_moe_route_batch");
    LOAD(stager_create, "katali_hip_stager_create");
    LOAD(stager_destroy, "katali_hip_stager_destroy");
    LOAD(stager_mark, "katali_hip_stager_mark");
    LOAD(stager_upload, "katali_hip_stager_upload");
    LOAD(stager_fence, "katali_hip_stager_fence");
    if (g_api.abi_version() != KATALI_HIP_ABI_VERSION) {
        snprintf(g_status, sizeof g_status, "%s: ABI version %d, loader expects %d", tried, g_api.abi_version(),
                 KATALI_HIP_ABI_VERSION);
        goto fail_nomsg;
    }
    g_state = 1;
    return 1;
fail:
    snprintf(g_status, sizeof g_status, "%s: missing entry point %s", tried, missing);
fail_nomsg:
    lib_close(g_lib);
    g_lib = NULL;
    memset(&g_api, 0, sizeof g_api);
    g_state = -1;
    return 0;
}

const KataliHipApi *katali_gpu_api(void) { return load() ? &g_api : NULL; }

void katali_gpu_unload(void) {
    if (g_lib) lib_close(g_lib);
    g_lib = NULL;
    memset(&g_api, 0, sizeof g_api);
    g_state = 0;
    g_probed = g_usable = 0;
    snprintf(g_status, sizeof g_status, "not probed");
}

int katali_gpu_probe(void) {
    if (g_probed) return g_usable;
    g_probed = 1;
    if (!load()) return 0;
    g_usable = g_api.probe() != 0;
    snprintf(g_status, sizeof g_status, "%s%s", g_usable ? "" : "no usable device: ", g_api.status());
    return g_usable;
}

const char *katali_gpu_status(void) { return g_status; }

const char *katali_gpu_last_error(void) { return g_state > 0 ? g_api.last_error() : g_status; }

#define FORWARD(call) return katali_gpu_probe() ? (call) : KATALI_GPU_E_UNAVAILABLE

int katali_gpu_malloc(void **dev, size_t bytes) { FORWARD(g_api.malloc_(dev, bytes)); }
int katali_gpu_free(void *dev) { FORWARD(g_api.free_(dev)); }
int katali_gpu_upload(void *dev, const void *host, size_t n) { FORWARD(g_api.upload(dev, host, n)); }
int katali_gpu_download(void *host, const void *dev, size_t n) { FORWARD(g_api.download(host, dev, n)); }
int katali_gpu_supports_type(uint32_t t) { return katali_gpu_probe() ? g_api.supports_type(t) : 0; }
int katali_gpu_matvec(uint32_t type, const void *w, uint64_t rows, uint64_t cols, const float *x, float *y) {
    FORWARD(g_api.matvec(type, w, rows, cols, x, y));
}
int katali_gpu_matvec_multi(int n, const uint32_t *types, const void *const *w, const uint64_t *rows, uint64_t cols,
                            const float *x, float *const *y) {
    FORWARD(g_api.matvec_multi(n, types, w, rows, cols, x, y));
}
int katali_gpu_quantize_q8_1(const float *x, uint64_t n, void *q8) { FORWARD(g_api.quantize_q8_1(x, n, q8)); }
int katali_gpu_matvec_q8(uint32_t type, const void *w, uint64_t rows, uint64_t cols, const void *xq, float *y) {
    FORWARD(g_api.matvec_q8(type, w, rows, cols, xq, y));
}
int katali_gpu_moe_layer(const KataliHipMoe *m, const KataliHipMoeRoute *r, const float *x, const void *xq,
                         float *y) {
    FORWARD(g_api.moe_layer(m, r, x, xq, y));
}
int katali_gpu_sync(void) { FORWARD(g_api.sync()); }
int katali_gpu_graph_begin(void) { FORWARD(g_api.graph_begin()); }
int katali_gpu_graph_end(void **g) { FORWARD(g_api.graph_end(g)); }
int katali_gpu_graph_launch(void *g) { FORWARD(g_api.graph_launch(g)); }
int katali_gpu_graph_destroy(void *g) { FORWARD(g_api.graph_destroy(g)); }
int katali_gpu_selftest(char *report, size_t cap) { FORWARD(g_api.selftest(report, cap)); }
int katali_gpu_argmax(const float *logits, uint64_t n, int32_t *out) { FORWARD(g_api.argmax(logits, n, out)); }
int katali_gpu_rmsnorm(const float *x, const float *w, uint64_t n, float eps, float *out) {
    FORWARD(g_api.rmsnorm(x, w, n, eps, out));
}
int katali_gpu_add_rmsnorm(float *x, const float *delta, float scale, const float *w, uint64_t n, float eps,
                           float *out) {
    FORWARD(g_api.add_rmsnorm(x, delta, scale, w, n, eps, out));
}
int katali_gpu_moe_route_batch(const float *logits, uint32_t n_tokens, uint32_t n_expert, int32_t n_sel, int32_t *ids,
                               float *w) {
    FORWARD(g_api.moe_route_batch(logits, n_tokens, n_expert, n_sel, ids, w));
}
int katali_gpu_rmsnorm_matvec_f32(const float *x, const float *delta, float scale, float *x_out, const float *nw,
                                  uint64_t n, float eps, float *xn, const float *w, uint64_t rows, float *y) {
    FORWARD(g_api.rmsnorm_matvec_f32(x, delta, scale, x_out, nw, n, eps, xn, w, rows, y));
}
int katali_gpu_moe_batch(const KataliHipMoe *moe, const KataliHipMoeBatch *batch, const float *x, float *y) {
    FORWARD(g_api.moe_batch(moe, batch, x, y));
}
int katali_gpu_stager_create(uint64_t chunk_bytes, uint32_t n_chunks, void **stager) {
    FORWARD(g_api.stager_create(chunk_bytes, n_chunks, stager));
}
int katali_gpu_stager_destroy(void *stager) { FORWARD(g_api.stager_destroy(stager)); }
int katali_gpu_stager_mark(void *stager, uint64_t *mark) { FORWARD(g_api.stager_mark(stager, mark)); }
int katali_gpu_stager_upload(void *stager, void *dev, const void *host, uint64_t bytes, uint64_t after_mark) {
    FORWARD(g_api.stager_upload(stager, dev, host, bytes, after_mark));
}
int katali_gpu_stager_fence(void *stager) { FORWARD(g_api.stager_fence(stager)); }
