// kq_sample.hip — greedy sampling on device: the index of the largest logit.
//
// Rule of the engine's greedy sampler (vendor/katali_gguf_dense/src/
// gguf_sampler.c:62-66): best = 0, bv = -FLT_MAX, then for i ascending take i
// when logits[i] > bv. So the first maximum wins, NaN never wins, and when no
// value exceeds -FLT_MAX the answer is 0. Here: (value, index) pairs reduced
// with "larger value, then lower index" over candidates v > -FLT_MAX, in one
// launch: every workgroup reduces its share and stores its pair as one
// device-coherent 64-bit word; once that store is acknowledged it counts
// itself in, and the workgroup that counts last reduces the partials and
// writes the answer, then puts the count back to zero for the next call
// (stream order: no two calls overlap, and a graph replay starts from zero).
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
constexpr uint32_t ARGMAX_PARTS = 256;
constexpr uint32_t ARGMAX_COUNT = 2 * ARGMAX_PARTS;   // the count word, after the partials

__device__ __forceinline__ uint64_t pack(Best b) { return ((uint64_t)(uint32_t)b.i << 32) | __float_as_uint(b.v); }
__device__ __forceinline__ Best unpack(uint64_t w) { return Best{__uint_as_float((uint32_t)w), (int32_t)(w >> 32)}; }

// words: ARGMAX_PARTS 64-bit partials, then the count (zero between calls)
__global__ void __launch_bounds__(256) k_argmax(const float *__restrict__ x, uint32_t n, uint32_t *words,
                                                int32_t *out) {
    __shared__ uint32_t last;
    Best b{-FLT_MAX, NONE};
    for (uint32_t t = blockIdx.x * 256 + threadIdx.x; t < n; t += gridDim.x * 256) {
        const float v = x[t];
        if (v > b.v) b = Best{v, (int32_t)t};   // ascending t per thread: strict > keeps the first
    }
    b = block_best(b);
    if (threadIdx.x == 0) {
        st_dev2(words + 2 * blockIdx.x, pack(b));
        __builtin_amdgcn_s_waitcnt(VMCNT0);   // the partial is acknowledged before the count
        last = __hip_atomic_fetch_add(words + ARGMAX_COUNT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    Best r{-FLT_MAX, NONE};
    for (uint32_t t = threadIdx.x; t < gridDim.x; t += 256) r = better(r, unpack(ld_dev2(words + 2 * t)));
    r = block_best(r);
    if (threadIdx.x == 0) {
        *out = r.i == NONE ? 0 : r.i;
        st_dev(words + ARGMAX_COUNT, 0u);
    }
}

uint32_t argmax_scratch_bytes() { return 4 * (ARGMAX_COUNT + 1); }

hipError_t launch_argmax(const float *x, uint32_t n, void *scratch, int32_t *out, hipStream_t s) {
    uint32_t g = (n + 2047) / 2048;
    if (g < 1) g = 1;
    if (g > ARGMAX_PARTS) g = ARGMAX_PARTS;
    hipLaunchKernelGGL(k_argmax, dim3(g), dim3(256), 0, s, x, n, (uint32_t *)scratch, out);
    return hipGetLastError();
}

}  // namespace kq
