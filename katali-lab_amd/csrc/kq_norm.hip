// kq_norm.hip — the decode chain's RMSNorm and residual add on device.
//
// Arithmetic of the engine (vendor/katali_gguf_dense/src/gguf_kernels.c:13-18):
// sumsq = sum of x[i]^2 in double, inv = 1 / sqrtf((float)(sumsq / n) + eps),
// out[i] = x[i] * inv * w[i] (two float products, no contraction). The
// residual step before a norm (gguf_model.c:677-678, 692-693) is x[i] +=
// delta[i], or x[i] += scale * delta[i] when the model scales its residual.
//
// One workgroup of 1024 threads: each thread adds and squares its elements
// (t, t + 1024, ...), the double partial sums meet in a fixed tree (a DPP
// and permlane butterfly in each wave, then the 16 wave sums in order), every
// thread forms the same inv and writes its outputs. The double sum is in a different order than the
// engine's loop; its rounding to float is the same unless the two doubles
// straddle a float rounding boundary (relative distance ~2^-29).
#include "kq_device.h"
#include "kq_launch.h"

namespace kq {

constexpr uint32_t NORM_THREADS = 1024;

template <bool ADD>
__global__ void __launch_bounds__(NORM_THREADS)
    k_rmsnorm(float *x, const float *delta, float scale, uint32_t unit_scale,
              const float *w, uint32_t n, float eps, float *out) {
    __shared__ double part[NORM_THREADS / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double s = 0.0;
    for (uint32_t i = tid; i < n; i += NORM_THREADS) {
        float v = x[i];
        if constexpr (ADD) {
            v = unit_scale ? v + delta[i] : v + scale * delta[i];
            x[i] = v;
        }
        s += (double)v * (double)v;
    }
    s = wave_sum_f64(s);
    if (lane == 0) part[wave] = s;
    __syncthreads();
    double sumsq = part[0];
#pragma unroll
    for (uint32_t k = 1; k < NORM_THREADS / 64; k++) sumsq += part[k];
    const float inv = 1.0f / sqrtf((float)(sumsq / (double)n) + eps);
    for (uint32_t i = tid; i < n; i += NORM_THREADS) out[i] = x[i] * inv * w[i];   // this thread's own x[i]
}

hipError_t launch_rmsnorm(const float *x, const float *w, uint32_t n, float eps, float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_rmsnorm<false>, dim3(1), dim3(NORM_THREADS), 0, s, (float *)x, nullptr, 1.0f, 1u, w, n, eps,
                       out);
    return hipGetLastError();
}

hipError_t launch_add_rmsnorm(float *x, const float *delta, float scale, const float *w, uint32_t n, float eps,
                              float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_rmsnorm<true>, dim3(1), dim3(NORM_THREADS), 0, s, x, delta, scale, scale == 1.0f ? 1u : 0u, w,
                       n, eps, out);
    return hipGetLastError();
}

}  // namespace kq
