/* katali_dense_hip.h — engine-side dense GEMV shim over libkatali_hip.
 *
 * Drop-in for the engine's vendor/katali_gguf_dense/include/katali_dense_cuda.h:4-7
 * (katali_dense_cuda_enabled / _matvec / _matvec_multi / _shutdown). The
 * engine's functions take a KataliGgufTensor; these take the fields the shim
 * reads from it (type, data, nbytes, dims[1] = rows, dims[0] = cols;
 * katali_gguf.h:67) so this header needs nothing from the engine; the
 * engine's katali_dense_cuda_* functions forward to these in three lines
 * each. Returns 0 on success and -1 on any failure: the caller then
 * computes on the CPU, exactly as with the CUDA shim. */
#ifndef KATALI_DENSE_HIP_H
#define KATALI_DENSE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 1 when KATALI_HIP (or KATALI_CUDA) starts with 1/y/Y and a gfx950 device is
 * usable; decided once and logged to stderr (katali_dense_cuda.c:14-22). */
int katali_dense_hip_enabled(void);
/* y[rows] = W x for one GGUF matrix held in host memory at w (w_bytes long);
 * the device copy is cached by host pointer (katali_dense_cuda.c:46-56). */
int katali_dense_hip_matvec(uint32_t type, const void *w, uint64_t w_bytes, uint64_t rows, uint64_t cols,
                            const float *x, float *y);
/* n <= 4 same-input projections (katali_dense_cuda.c:58-73): one upload,
 * one launch for all n (katali_hip_matvec_multi), n downloads. */
int katali_dense_hip_matvec_multi(int n, const uint32_t *types, const void *const *ws, const uint64_t *w_bytes,
                                  const uint64_t *rows, uint64_t cols, const float *x, float **ys);
/* Number of cached device weights (for tests and diagnostics). */
int katali_dense_hip_cached(void);
/* Frees every device copy and buffer; the next call re-probes (:75-79). */
void katali_dense_hip_shutdown(void);

#ifdef __cplusplus
}
#endif
#endif
