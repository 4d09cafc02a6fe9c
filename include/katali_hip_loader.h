/* katali_hip_loader.h — engine-side runtime loader for libkatali_hip.
 *
 * The engine links this small C file instead of the reference's absent
 * src/katali_cuda.c loader (included at V/src/katali_dense_cuda.c:2; its API
 * is visible at the call sites V/src/katali_dense_cuda.c:19,27-31,40-41,48,
 * 52-54,65-71). It finds libkatali_hip at run time with dlopen (LoadLibrary
 * on Windows) and never links HIP: without the library, a driver or a gfx950
 * device, katali_gpu_probe() returns 0, katali_gpu_status() says why, and the
 * engine keeps its CPU path (V/src/gguf_model.c:500-504,533-541).
 *
 * Discovery order: $KATALI_HIP_DLL, then libkatali_hip.so next to the loaded
 * loader, then the dynamic linker's search path. Same signatures and return
 * convention as the reference loader (KATALI_GPU_OK == 0 on success).
 */
#ifndef KATALI_HIP_LOADER_H
#define KATALI_HIP_LOADER_H

#include <stddef.h>
#include <stdint.h>

#include "katali_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define KATALI_GPU_OK 0
#define KATALI_GPU_E_UNAVAILABLE (-100) /* library not loaded / device unusable */

/* Loads the library (once) and probes the device: non-zero when usable.
 * Replaces katali_cuda_probe (V/src/katali_dense_cuda.c:19). */
int         katali_gpu_probe(void);
/* Why the probe succeeded or failed. Replaces katali_cuda_status (:19). */
const char *katali_gpu_status(void);
/* Replaces katali_cuda_malloc / _free / _upload / _download / _supports_type /
 * _matvec (V/src/katali_dense_cuda.c:27-31,40-41,48,52-54,65-71,76-78). */
int katali_gpu_malloc(void **dev, size_t bytes);
int katali_gpu_free(void *dev);
int katali_gpu_upload(void *dev, const void *host, size_t bytes);
int katali_gpu_download(void *host, const void *dev, size_t bytes);
int katali_gpu_supports_type(uint32_t ggml_type);
int katali_gpu_matvec(uint32_t type, const void *w_dev, uint64_t rows, uint64_t cols,
                      const float *x_dev, float *y_dev);
/* Up to four GEMVs over one x in one launch, in place of the per-tensor
 * katali_cuda_matvec loop of katali_dense_cuda_matvec_multi
 * (V/src/katali_dense_cuda.c:58-72). */
int katali_gpu_matvec_multi(int n, const uint32_t *types, const void *const *w_devs, const uint64_t *rows,
                            uint64_t cols, const float *x_dev, float *const *y_devs);

/* The MoE-engine entry points of the closed backend (README.md:13,17,21):
 * one call per MoE layer, q8_1 activations, graphs, self-test. */
int katali_gpu_quantize_q8_1(const float *x_dev, uint64_t n, void *q8_dev);
int katali_gpu_matvec_q8(uint32_t type, const void *w_dev, uint64_t rows, uint64_t cols,
                         const void *xq8_dev, float *y_dev);
int katali_gpu_moe_layer(const KataliHipMoe *moe, const KataliHipMoeRoute *route,
                         const float *x_dev, const void *xq8_dev, float *y_dev);
int katali_gpu_sync(void);
int katali_gpu_graph_begin(void);
int katali_gpu_graph_end(void **graph);
int katali_gpu_graph_launch(void *graph);
int katali_gpu_graph_destroy(void *graph);
int katali_gpu_selftest(char *report, size_t cap);
/* Greedy token on device (gguf_sampler.c:62-66 rule), for a decode loop that
 * keeps logits resident. */
int katali_gpu_argmax(const float *logits_dev, uint64_t n, int32_t *out_dev);
/* RMSNorm and the residual add before it (V/src/gguf_kernels.c:13-18,
 * V/src/gguf_model.c:677-683). */
int katali_gpu_rmsnorm(const float *x_dev, const float *w_dev, uint64_t n, float eps, float *out_dev);
int katali_gpu_add_rmsnorm(float *x_dev, const float *delta_dev, float scale, const float *w_dev, uint64_t n,
                           float eps, float *out_dev);
/* Residual step, norm and F32 router logits in one launch. */
int katali_gpu_rmsnorm_matvec_f32(const float *x_dev, const float *delta_dev, float scale, float *x_out_dev,
                                  const float *norm_w_dev, uint64_t n, float eps, float *xn_dev,
                                  const float *w_dev, uint64_t rows, float *y_dev);
/* Device routing for a batch: ids/weights [T][n_sel] from logits [T][n_expert]. */
int katali_gpu_moe_route_batch(const float *logits_dev, uint32_t n_tokens, uint32_t n_expert, int32_t n_sel,
                               int32_t *ids_dev, float *weights_dev);
/* The MoE layer over a batch of up to 64 tokens (batched prefill). */
int katali_gpu_moe_batch(const KataliHipMoe *moe, const KataliHipMoeBatch *batch, const float *x_dev,
                         float *y_dev);
/* Pipelined uploads through a pinned ring and a copy stream (the expert
 * tier's miss path; katali_hip_stager_* in katali_hip.h). */
int katali_gpu_stager_create(uint64_t chunk_bytes, uint32_t n_chunks, void **stager);
int katali_gpu_stager_destroy(void *stager);
int katali_gpu_stager_mark(void *stager, uint64_t *mark);
int katali_gpu_stager_upload(void *stager, void *dev, const void *host, uint64_t bytes, uint64_t after_mark);
int katali_gpu_stager_fence(void *stager);
/* The library's last error for this thread ("" when none / not loaded). */
const char *katali_gpu_last_error(void);

/* Direct access to every library entry point (NULL members when absent). */
typedef struct KataliHipApi {
    int (*abi_version)(void);
    const char *(*last_error)(void);
    int (*probe)(void);
    const char *(*status)(void);
    int (*malloc_)(void **, size_t);
    int (*free_)(void *);
    int (*upload)(void *, const void *, size_t);
    int (*download)(void *, const void *, size_t);
    int (*supports_type)(uint32_t);
    int (*matvec)(uint32_t, const void *, uint64_t, uint64_t, const float *, float *);
    int (*sync)(void);
    int (*memset_)(void *, int, size_t);
    int (*set_stream)(void *);
    int (*quantize_q8_1)(const float *, uint64_t, void *);
    int (*matvec_q8)(uint32_t, const void *, uint64_t, uint64_t, const void *, float *);
    int (*matvec_dp4a)(uint32_t, const void *, uint64_t, uint64_t, const float *, float *);
    int (*block_isums)(uint32_t, const void *, uint64_t, uint64_t, const void *, int32_t *);
    int (*moe_layer)(const KataliHipMoe *, const KataliHipMoeRoute *, const float *, const void *, float *);
    int (*moe_layer_debug)(const KataliHipMoe *, const KataliHipMoeRoute *, const float *, const void *,
                           float *, float *, void *);
    int (*step_advance)(int32_t *, int32_t);
    int (*graph_begin)(void);
    int (*graph_end)(void **);
    int (*graph_launch)(void *);
    int (*graph_destroy)(void *);
    int (*event_create)(void **);
    int (*event_record)(void *);
    int (*event_elapsed)(void *, void *, float *);
    int (*event_destroy)(void *);
    int (*selftest)(char *, size_t);
    int (*synth_fill)(uint32_t, void *, uint64_t, uint64_t, float);
    int (*synth_normal)(float *, uint64_t, uint64_t, float);
    int (*copy)(void *, const void *, size_t);
    int (*argmax)(const float *, uint64_t, int32_t *);
    int (*moe_batch)(const KataliHipMoe *, const KataliHipMoeBatch *, const float *, float *);
    int (*matvec_multi)(int, const uint32_t *, const void *const *, const uint64_t *, uint64_t, const float *,
                        float *const *);
    int (*matvec_multi_dp4a)(int, const uint32_t *, const void *const *, const uint64_t *, uint64_t,
                             const float *, float *const *);
    int (*rmsnorm)(const float *, const float *, uint64_t, float, float *);
    int (*add_rmsnorm)(float *, const float *, float, const float *, uint64_t, float, float *);
    int (*rmsnorm_matvec_f32)(const float *, const float *, float, float *, const float *, uint64_t, float, float *,
                              const float *, uint64_t, float *);
    int (*moe_route_batch)(const float *, uint32_t, uint32_t, int32_t, int32_t *, float *);
    int (*stager_create)(uint64_t, uint32_t, void **);
    int (*stager_destroy)(void *);
    int (*stager_mark)(void *, uint64_t *);
    int (*stager_upload)(void *, void *, const void *, uint64_t, uint64_t);
    int (*stager_fence)(void *);
} KataliHipApi;

/* NULL when the library could not be loaded or an entry point is missing. */
const KataliHipApi *katali_gpu_api(void);
/* Forget the loaded library (tests); the next call loads again. */
void katali_gpu_unload(void);

#ifdef __cplusplus
}
#endif
#endif /* KATALI_HIP_LOADER_H */
