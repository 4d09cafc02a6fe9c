// kq_gemv_f32.hip — y = W . x for fp32 weights (GGUF F32 tensors: MoE router
// matrices), bit-identical to the engine's AVX2 F32 dot
// (vendor/katali_gguf_dense/src/gguf_simd_x86.c:111-122, hsum :80-89):
//
//   16 fp32 accumulators; accumulator j takes fmaf(w[c], x[c], acc) for
//   c = j, j + 16, j + 32, ... over the first n16 = cols & ~15 columns;
//   v_k = acc_k + acc_{k+8}; l_k = v_k + v_{k+4}; acc = (l0 + l1) + (l2 + l3);
//   the columns past n16 are summed in double in order; y = acc + (float)tail.
//
// Accumulator j of a row is one lane's FMA chain (16 lanes per row, four rows
// per wave). The chains read w and x from LDS: each workgroup stages a chunk
// of columns of its R rows and of x with 16-byte loads (all in flight at once),
// then the lanes run their chains over the chunk. Chunks are multiples of 16
// columns, so the chains continue across chunks unchanged.
#include "kq_device.h"
#include "kq_launch.h"

namespace kq {

constexpr uint32_t F32_THREADS = 256;
constexpr uint32_t F32_CHUNK = 2048;   // columns staged per pass (x: 8 KB)

template <uint32_t R>
__global__ void __launch_bounds__(F32_THREADS)
    k_gemv_f32(const float *__restrict__ w, uint32_t rows, uint32_t cols, const float *__restrict__ x,
               float *__restrict__ y) {
    // LDS: x chunk [F32_CHUNK], then R rows of [F32_CHUNK + 16] (the pad puts
    // the four rows a wave reads at once on different banks).
    constexpr uint32_t LD = F32_CHUNK + 16;
    __shared__ __align__(16) float xs[F32_CHUNK];
    __shared__ __align__(16) float ws[R * LD];
    const uint32_t tid = threadIdx.x;
    const uint32_t row0 = blockIdx.x * R;
    const uint32_t nr = min(R, rows - row0);
    const uint32_t lrow = tid >> 4, j = tid & 15;   // chain j of local row lrow
    const bool chain = lrow < nr;
    const uint32_t n16 = cols & ~15u;
    float acc = 0.0f;
    double tail = 0.0;
    for (uint32_t c0 = 0; c0 < cols; c0 += F32_CHUNK) {
        const uint32_t len = min(F32_CHUNK, cols - c0);   // multiple of 4
        const uint32_t q4 = len >> 2;                     // float4 per row
        __syncthreads();                                  // previous chunk's reads done
        // All loads first, then the LDS stores: one HBM latency per chunk.
        // Indices are clamped into the chunk; a clamped lane loads and stores
        // the same element as the lane it duplicates (same value, same place).
        constexpr uint32_t KX = F32_CHUNK / 4 / F32_THREADS, KW = R * KX;
        uint32_t ix[KX], iw[KW];
        float4 vx[KX], vw[KW];
#pragma unroll
        for (uint32_t k = 0; k < KX; k++) {
            ix[k] = min(tid + k * F32_THREADS, q4 - 1);
            vx[k] = *(const float4 *)&x[c0 + 4 * ix[k]];
        }
#pragma unroll
        for (uint32_t k = 0; k < KW; k++) {
            const uint32_t e = min(tid + k * F32_THREADS, nr * q4 - 1), r = e / q4, q = e - r * q4;
            iw[k] = r * LD + 4 * q;
            vw[k] = *(const float4 *)&w[(uint64_t)(row0 + r) * cols + c0 + 4 * q];
        }
#pragma unroll
        for (uint32_t k = 0; k < KX; k++) *(float4 *)&xs[4 * ix[k]] = vx[k];
#pragma unroll
        for (uint32_t k = 0; k < KW; k++) *(float4 *)&ws[iw[k]] = vw[k];
        __syncthreads();
        if (chain) {
            const float *wr = &ws[lrow * LD];
            const uint32_t end = min(len, n16 > c0 ? n16 - c0 : 0u);
#pragma unroll 8
            for (uint32_t c = j; c < end; c += 16) acc = fmaf(wr[c], xs[c], acc);
            if (j == 0)
                for (uint32_t c = end; c < len; c++) tail += (double)wr[c] * (double)xs[c];
        }
    }
    const float v = hsum16_avx2_order(acc);   // 16 lanes of a row = one DPP row
    if (chain && j == 0) y[row0 + lrow] = v + (float)tail;
}

hipError_t launch_gemv_f32(const float *w, uint64_t rows, uint64_t cols, const float *x, float *y, hipStream_t s) {
    // One row per workgroup up to 256 rows (the router matrices), then 2 or 4
    // (16 lanes each), so that larger matrices need fewer, fuller workgroups.
    uint32_t r = 1;
    while (r < 4 && rows > (uint64_t)r * 256) r <<= 1;
    const uint32_t grid = (uint32_t)((rows + r - 1) / r);
    if (r == 1)
        hipLaunchKernelGGL(k_gemv_f32<1>, dim3(grid), dim3(F32_THREADS), 0, s, w, (uint32_t)rows, (uint32_t)cols, x, y);
    else if (r == 2)
        hipLaunchKernelGGL(k_gemv_f32<2>, dim3(grid), dim3(F32_THREADS), 0, s, w, (uint32_t)rows, (uint32_t)cols, x, y);
    else
        hipLaunchKernelGGL(k_gemv_f32<4>, dim3(grid), dim3(F32_THREADS), 0, s, w, (uint32_t)rows, (uint32_t)cols, x, y);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RMSNorm (with the residual step before it) fused with the router GEMV: the
// two engine steps before a MoE layer (gguf_model.c:677-683, then the F32
// router product) in one launch, one router row per workgroup. Every
// workgroup forms the whole normalized vector itself from x, delta and the
// norm weights (32 KB at most, from L2) and dots its row with it; workgroup 0
// also writes xn and the new residual x_out = x + scale·delta. x_out is a
// different buffer from x: the other workgroups still read x.
//
// Norm arithmetic as k_rmsnorm's: double sum of squares in a fixed tree,
// inv = 1 / sqrtf((float)(sumsq / n) + eps), xn = v * inv * w.
//
// LDS holds the row and xn transposed by accumulator: column c < n16 at
// [c & 15][c >> 4] (row stride TS = 64·KN + 4 floats, which puts the 16
// lanes' 16-byte reads, and the 64 lanes' transposing 4-byte writes, on
// distinct banks), so lane j's FMA chain reads its operands four at a time;
// the columns past n16 sit in a 16-float area of their own.
// ---------------------------------------------------------------------------
template <uint32_t KN, bool ADD>
__global__ void __launch_bounds__(F32_THREADS)
    k_norm_router(const float *__restrict__ x, const float *__restrict__ delta, float scale, uint32_t unit_scale,
                  float *__restrict__ x_out, const float *__restrict__ nw, float eps, float *__restrict__ xn_out,
                  const float *__restrict__ w, uint32_t cols, float *__restrict__ y) {
    constexpr uint32_t M = 64 * KN;    // chain length capacity (cols <= 16 M)
    constexpr uint32_t TS = M + 4;
    // [16][TS] transposed, then 16 floats for the columns past n16
    __shared__ __align__(16) float wt[16 * TS + 16];
    __shared__ __align__(16) float xt[16 * TS + 16];
    __shared__ double part[F32_THREADS / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t row = blockIdx.x;
    const uint32_t q4 = cols >> 2;   // float4 of the vector
    const uint32_t n16 = cols & ~15u, m = n16 >> 4;
    const float *wr = w + (uint64_t)row * cols;
    // LDS slot of column c: its chain position below n16, the tail area above
    auto slot = [&](uint32_t c) { return c < n16 ? (c & 15) * TS + (c >> 4) : 16 * TS + (c - n16); };

    // 1. every load at once (indices clamped into the vector: a clamped lane
    //    duplicates the last float4, adds nothing to the sum and stores the
    //    same values to the same places)
    float4 vx[KN], vd[KN], vn[KN], vw[KN];
#pragma unroll
    for (uint32_t k = 0; k < KN; k++) {
        const uint32_t q = min(tid + k * F32_THREADS, q4 - 1);
        vx[k] = *(const float4 *)&x[4 * q];
        if constexpr (ADD) vd[k] = *(const float4 *)&delta[4 * q];
        vn[k] = *(const float4 *)&nw[4 * q];
        vw[k] = *(const float4 *)&wr[4 * q];
    }
    // chain positions m..M-1 hold zeros (every chain runs the full M; a zero
    // product leaves the accumulator's value, and only its zero sign, which
    // the final + (float)tail erases, could change)
    for (uint32_t e = tid; e < 16 * (M - m); e += F32_THREADS) {
        const uint32_t j = e / (M - m), p = m + e % (M - m);
        wt[j * TS + p] = 0.0f;
        xt[j * TS + p] = 0.0f;
    }
#pragma unroll
    for (uint32_t k = 0; k < KN; k++) {
        const uint32_t c = 4 * min(tid + k * F32_THREADS, q4 - 1);
        wt[slot(c)] = vw[k].x; wt[slot(c + 1)] = vw[k].y; wt[slot(c + 2)] = vw[k].z; wt[slot(c + 3)] = vw[k].w;
    }
    // 2. residual step and the sum of squares
    double s = 0.0;
#pragma unroll
    for (uint32_t k = 0; k < KN; k++) {
        if constexpr (ADD) {
            if (unit_scale) {
                vx[k].x = vx[k].x + vd[k].x; vx[k].y = vx[k].y + vd[k].y;
                vx[k].z = vx[k].z + vd[k].z; vx[k].w = vx[k].w + vd[k].w;
            } else {
                vx[k].x = vx[k].x + scale * vd[k].x; vx[k].y = vx[k].y + scale * vd[k].y;
                vx[k].z = vx[k].z + scale * vd[k].z; vx[k].w = vx[k].w + scale * vd[k].w;
            }
        }
        const bool own = tid + k * F32_THREADS < q4;
        s += own ? (double)vx[k].x * (double)vx[k].x : 0.0;
        s += own ? (double)vx[k].y * (double)vx[k].y : 0.0;
        s += own ? (double)vx[k].z * (double)vx[k].z : 0.0;
        s += own ? (double)vx[k].w * (double)vx[k].w : 0.0;
    }
    s = wave_sum_f64(s);
    if (lane == 0) part[wave] = s;
    __syncthreads();
    double sumsq = part[0];
#pragma unroll
    for (uint32_t k = 1; k < F32_THREADS / 64; k++) sumsq += part[k];
    const float inv = 1.0f / sqrtf((float)(sumsq / (double)cols) + eps);
    // 3. xn, transposed into LDS (and from workgroup 0 to memory, with the new
    //    residual)
#pragma unroll
    for (uint32_t k = 0; k < KN; k++) {
        const uint32_t q = min(tid + k * F32_THREADS, q4 - 1), c = 4 * q;
        float4 o;
        o.x = vx[k].x * inv * vn[k].x; o.y = vx[k].y * inv * vn[k].y;
        o.z = vx[k].z * inv * vn[k].z; o.w = vx[k].w * inv * vn[k].w;
        xt[slot(c)] = o.x; xt[slot(c + 1)] = o.y; xt[slot(c + 2)] = o.z; xt[slot(c + 3)] = o.w;
        if (blockIdx.x == 0) {
            *(float4 *)&xn_out[4 * q] = o;
            if constexpr (ADD) *(float4 *)&x_out[4 * q] = vx[k];
        }
    }
    __syncthreads();
    // 4. lane j < 16: accumulator j's FMA chain over columns j, j + 16, ...
    //    (over all M positions, 16-byte LDS reads); lane 0 also
    //    sums the columns past n16 in double
    if (tid < 16) {
        const uint32_t j = tid;
        const float *pw = &wt[j * TS], *px = &xt[j * TS];
        float acc = 0.0f;
#pragma unroll 1
        for (uint32_t i0 = 0; i0 < M; i0 += 128) {   // 128 positions' reads in flight at a time
#pragma unroll
            for (uint32_t i = i0; i < i0 + 128; i += 4) {
                const float4 a = *(const float4 *)&pw[i], b = *(const float4 *)&px[i];
                acc = fmaf(a.x, b.x, acc);
                acc = fmaf(a.y, b.y, acc);
                acc = fmaf(a.z, b.z, acc);
                acc = fmaf(a.w, b.w, acc);
            }
        }
        double tail = 0.0;
        if (j == 0)
            for (uint32_t c = 0; c < cols - n16; c++) tail += (double)wt[16 * TS + c] * (double)xt[16 * TS + c];
        const float v = hsum16_avx2_order(acc);
        if (j == 0) y[row] = v + (float)tail;
    }
}

template <uint32_t KN>
static void go_norm_router(uint32_t grid, bool add, const float *x, const float *delta, float scale, float *x_out,
                           const float *nw, float eps, float *xn, const float *w, uint32_t cols, float *y,
                           hipStream_t s) {
    const uint32_t unit = scale == 1.0f ? 1u : 0u;
    if (add)
        hipLaunchKernelGGL((k_norm_router<KN, true>), dim3(grid), dim3(F32_THREADS), 0, s, x, delta, scale, unit,
                           x_out, nw, eps, xn, w, cols, y);
    else
        hipLaunchKernelGGL((k_norm_router<KN, false>), dim3(grid), dim3(F32_THREADS), 0, s, x, delta, scale, unit,
                           x_out, nw, eps, xn, w, cols, y);
}

hipError_t launch_norm_router(const float *x, const float *delta, float scale, float *x_out, const float *nw,
                              uint64_t n, float eps, float *xn, const float *w, uint64_t rows, float *y,
                              hipStream_t s) {
    const uint32_t grid = (uint32_t)rows, cols = (uint32_t)n;
    const bool add = delta != nullptr;
    if (n <= 2048) go_norm_router<2>(grid, add, x, delta, scale, x_out, nw, eps, xn, w, cols, y, s);
    else if (n <= 4096) go_norm_router<4>(grid, add, x, delta, scale, x_out, nw, eps, xn, w, cols, y, s);
    else go_norm_router<8>(grid, add, x, delta, scale, x_out, nw, eps, xn, w, cols, y, s);
    return hipGetLastError();
}

}  // namespace kq
