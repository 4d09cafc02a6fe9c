// kq_sample.hip — greedy sampling on device: the index of the largest logit.
//
// Rule of the engine's greedy sampler (vendor/katali_gguf_dense/src/
// gguf_sampler.c:62-66): best = 0, bv = -FLT_MAX, then for i ascending take i
// when logits[i] > bv. So the first maximum wins, NaN never wins, and when no
// value exceeds -FLT_MAX the answer is 0. Here: (value, index) pairs reduced
// with "larger value, then lower index" over candidates v > -FLT_MAX, in two
// launches (per-workgroup partials, then one workgroup), no atomics.
#include <float.h>

#include "kq_device.h"
#include "kq_launch.h"

namespace kq {

struct Best {
    float v;
    int32_t i;
};
__device__ __forceinline__ Best better(Best a, Best b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}
__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        Best p;
        p.v = __shfl_xor(b.v, o, WAVE);
        p.i = __shfl_xor(b.i, o, WAVE);
        b = better(b, p);
    }
    return b;
}
__device__ __forceinline__ Best block_best(Best b) {
    __shared__ Best part[4];
    b = wave_best(b);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = b;
    __syncthreads();
    b = part[0];
#pragma unroll
    for (int w = 1; w < 4; w++) b = better(b, part[w]);
    return b;
}

constexpr int32_t NONE = 0x7FFFFFFF;

__global__ void __launch_bounds__(256) k_argmax_part(const float *__restrict__ x, uint32_t n, Best *__restrict__ part) {
    Best b{-FLT_MAX, NONE};
    for (uint32_t t = blockIdx.x * 256 + threadIdx.x; t < n; t += gridDim.x * 256) {
        const float v = x[t];
        if (v > b.v) b = Best{v, (int32_t)t};   // ascending t per thread: strict > keeps the first
    }
    b = block_best(b);
    if (threadIdx.x == 0) part[blockIdx.x] = b;
}

__global__ void __launch_bounds__(256) k_argmax_final(const Best *__restrict__ part, uint32_t nparts, int32_t *out) {
    Best b{-FLT_MAX, NONE};
    for (uint32_t t = threadIdx.x; t < nparts; t += 256) b = better(b, part[t]);
    b = block_best(b);
    if (threadIdx.x == 0) *out = b.i == NONE ? 0 : b.i;
}

uint32_t argmax_parts() { return 256; }

hipError_t launch_argmax(const float *x, uint32_t n, void *scratch, int32_t *out, hipStream_t s) {
    uint32_t g = (n + 2047) / 2048;
    if (g < 1) g = 1;
    if (g > argmax_parts()) g = argmax_parts();
    hipLaunchKernelGGL(k_argmax_part, dim3(g), dim3(256), 0, s, x, n, (Best *)scratch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, (const Best *)scratch, g, out);
    return hipGetLastError();
}

}  // namespace kq
