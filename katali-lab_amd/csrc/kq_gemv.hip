// kq_gemv.hip — q8_1 quantization, dense Q4_K / Q6_K GEMV (fp32 and q8_1
// activations), per-block integer sums, synthetic data and a copy kernel.
//
// GEMV layout: a row is nb = cols/256 super-blocks = nb*IPB lane items. S lanes
// (a power of two dividing the item count, at most 64) share a row and each
// takes IPL = items/S items (item = s + S*i, so a wave instruction walks
// consecutive items of a row). A wave holds 64/S rows at a time, a 256-thread
// workgroup 4x that, and each slot issues the loads of RPS rows before it
// computes any of them. The activation is staged once per workgroup in LDS.
#include "kq_device.h"
#include "kq_launch.h"

namespace kq {

int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

__global__ void __launch_bounds__(256) k_quantize_q8_1(const float *__restrict__ x, uint32_t nblk,
                                                        uint8_t *__restrict__ out) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * 8) return;   // whole 8-lane groups exit together
    const uint32_t blk = t >> 3, part = t & 7;
    const float4 v = *(const float4 *)(x + 32 * blk + 4 * part);
    uint32_t d16, s16;
    int lo, hi;
    float dd;
    const uint32_t q = quant_q8_1_part(v, d16, s16, lo, hi, dd);
    uint8_t *b = out + 36 * blk;
    *(uint32_t *)(b + 4 + 4 * part) = q;
    if (part == 0) *(uint32_t *)b = d16 | (s16 << 16);
}

hipError_t launch_quantize_q8_1(const float *x, uint64_t n, uint8_t *out, hipStream_t s) {
    const uint32_t nblk = (uint32_t)(n / 32);
    const uint32_t threads = nblk * 8;
    hipLaunchKernelGGL(k_quantize_q8_1, dim3((threads + 255) / 256), dim3(256), 0, s, x, nblk, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GEMV
// ---------------------------------------------------------------------------
// The activation of a GEMV workgroup, staged in two halves around the weight
// loads: load() issues the first XPRE tasks per thread into registers (the
// whole activation for cols <= 4096), store() writes them to LDS after the
// weight loads are out and stages any remaining tasks directly. A task is 4
// values: fp32 copied (MODE 0), q8_1 bytes copied (MODE 1), or fp32
// quantized to q8_1 with 8 lanes per block (MODE 2).
constexpr int XPRE = 4;
template <int MODE, uint32_t NT = 256>
struct XStage {
    float4 v[XPRE];
    uint32_t q[XPRE], d[XPRE];
    __device__ static uint32_t tasks(uint32_t cols) { return MODE == 0 ? cols / 4 : cols / 32 * 8; }
    __device__ __forceinline__ void load(const float *xf, const uint8_t *xq, uint32_t cols) {
        const uint32_t n = tasks(cols);
#pragma unroll
        for (int i = 0; i < XPRE; i++) {
            const uint32_t t = min(threadIdx.x + NT * i, n - 1);   // clamped, not skipped
            if constexpr (MODE == 1) {
                const uint8_t *b = xq + (t >> 3) * 36;
                q[i] = *(const uint32_t *)(b + 4 + 4 * (t & 7));
                d[i] = ld_u16(b);
                v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            } else {
                v[i] = *(const float4 *)(xf + 4 * t);
                q[i] = d[i] = 0;
            }
        }
    }
    __device__ __forceinline__ void put(uint32_t t, float4 x4, uint32_t qq, uint32_t dd, const Act &a,
                                        const ActF &af) const {
        if constexpr (MODE == 0) {
            *(float4 *)(af.x + 4 * t) = x4;
        } else {
            const uint32_t blk = t >> 3, part = t & 7;
            uint32_t qv;
            int lo, hi;
            float dec;
            if constexpr (MODE == 1) {
                qv = qq;
                q8_part_sums(qv, lo, hi);
                dec = h2f(dd);
            } else {
                uint32_t d16, s16;
                qv = quant_q8_1_part(x4, d16, s16, lo, hi, dec);
            }
            *(uint32_t *)(a.qs + 32 * blk + 4 * part) = qv;
            if (part == 0) {
                a.d8[blk] = dec;
                a.qs16[2 * blk] = lo;
                a.qs16[2 * blk + 1] = hi;
            }
        }
    }
    // Tasks past n were loaded clamped and are dropped here (whole 8-lane
    // groups: n % 8 == 0); the barriers around the weight loads keep the
    // compiler from sinking the preloads into these branches.
    __device__ __forceinline__ void store(const float *xf, const uint8_t *xq, uint32_t cols, const Act &a,
                                          const ActF &af) const {
        const uint32_t n = tasks(cols);
#pragma unroll
        for (int i = 0; i < XPRE; i++) {
            const uint32_t t = threadIdx.x + NT * i;
            if (t < n) put(t, v[i], q[i], d[i], a, af);
        }
        for (uint32_t t = threadIdx.x + NT * XPRE; t < n; t += NT) {   // whole 8-lane groups (n % 8 == 0)
            float4 x4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            uint32_t qq = 0, dd = 0;
            if constexpr (MODE == 1) {
                const uint8_t *b = xq + (t >> 3) * 36;
                qq = *(const uint32_t *)(b + 4 + 4 * (t & 7));
                dd = ld_u16(b);
            } else {
                x4 = *(const float4 *)(xf + 4 * t);
            }
            put(t, x4, qq, dd, a, af);
        }
        if constexpr (MODE == 0) {   // half-block sums of the fp32 activation
            __syncthreads();
            for (uint32_t t = threadIdx.x; t < cols / 16; t += NT) {
                float sum = 0.0f;
                for (int i = 0; i < 16; i++) sum += af.x[16 * t + i];
                af.xs16[t] = sum;
            }
        }
    }
};

// The row groups of one matrix that workgroup `block` of `nblocks` takes
// (the workgroups' shares of the matrix interleave: a grid-stride loop);
// NW waves per workgroup.
template <class QT, int IPL_T, int RPS, int MODE, int NW = 4>
__device__ __forceinline__ void gemv_rows(const uint8_t *__restrict__ w, uint32_t rows, uint32_t cols, uint64_t rb,
                                          uint32_t log2s, const float *xf, const uint8_t *xq, float *__restrict__ y,
                                          uint32_t block, uint32_t nblocks, uint8_t *lds) {
    const Act a = act_carve(lds, cols);
    const ActF af = actf_carve(lds, cols);
    const uint32_t S = 1u << log2s;
    const uint32_t slots = WAVE >> log2s;
    const uint32_t lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const uint32_t slot = lane >> log2s, s = lane & (S - 1);
    const uint32_t items = cols / 256 * QT::IPB;
    const int IPL = IPL_T > 0 ? IPL_T : (int)(items >> log2s);
    const uint32_t rows_iter = NW * slots * RPS;
    const uint32_t base0 = block * rows_iter;
    auto row_of = [&](uint32_t base, int r) { return base + r * (NW * slots) + wave * slots + slot; };

    // Unrolled items: the activation loads, then the first row group's
    // weight loads, go out before the activation is staged, so the two
    // latencies overlap. Rows are clamped,
    // not skipped (a load under a branch makes the compiler wait for all).
    typename QT::Raw raw[RPS][IPL_T > 0 ? IPL_T : 1];
    auto load_rows = [&](uint32_t base) {
        if constexpr (IPL_T > 0) {
#pragma unroll
            for (int r = 0; r < RPS; r++) {
                const uint8_t *rp = w + (uint64_t)min(row_of(base, r), rows - 1) * rb;
#pragma unroll
                for (int i = 0; i < IPL_T; i++) {
                    const uint32_t item = s + S * i;
                    raw[r][i] = QT::load(rp + (item / QT::IPB) * QT::BB, item % QT::IPB);
                }
            }
        }
    };
    XStage<MODE, 64 * NW> xs;
    xs.load(xf, xq, cols);   // issued first: waiting for x then waits for nothing else
    // Neither the compiler nor the scheduler may move work across these two
    // points (x is deliberately not __restrict__, so its loads are not
    // treated as invariant and re-issued at their use).
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    load_rows(base0);   // base0 < rows: the grid never exceeds the row groups
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);   // every weight load is out before x is staged
    xs.store(xf, xq, cols, a, af);
    __syncthreads();

    for (uint32_t base = base0; base < rows; base += nblocks * rows_iter) {
        float acc[RPS];
        if constexpr (IPL_T > 0) {
            if (base != base0) load_rows(base);
#pragma unroll
            for (int r = 0; r < RPS; r++) {
                float v = 0.0f;
#pragma unroll
                for (int i = 0; i < IPL_T; i++) {
                    const uint32_t item = s + S * i;
                    if constexpr (MODE == 0) v += QT::dot_f32(raw[r][i], item % QT::IPB, af, item / QT::IPB);
                    else v += QT::dot_q8(raw[r][i], item % QT::IPB, a, item / QT::IPB);
                }
                acc[r] = v;
            }
        } else {
#pragma unroll
            for (int r = 0; r < RPS; r++) {
                const uint32_t row = row_of(base, r);
                float v = 0.0f;
                if (row < rows) {
                    const uint8_t *rp = w + (uint64_t)row * rb;
                    for (int i = 0; i < IPL; i++) {
                        const uint32_t item = s + S * i;
                        const typename QT::Raw rw = QT::load(rp + (item / QT::IPB) * QT::BB, item % QT::IPB);
                        if constexpr (MODE == 0) v += QT::dot_f32(rw, item % QT::IPB, af, item / QT::IPB);
                        else v += QT::dot_q8(rw, item % QT::IPB, a, item / QT::IPB);
                    }
                }
                acc[r] = v;
            }
        }
        if (log2s == 6) {
            // one row per wave instruction: the RPS rows reduce together
            // (halving exchanges, no LDS); lane groups of 64 / RPS then hold
            // row (lane >> SH) & (RPS - 1)
            constexpr int LOGR = RPS >= 4 ? 2 : (RPS >= 2 ? 1 : 0);
            constexpr int SH = 6 - LOGR;
            const float v = reduce_rows<RPS>(acc);
            const uint32_t r = (lane >> SH) & (RPS - 1);
            const uint32_t row = row_of(base, (int)r);
            if ((lane & ((1u << SH) - 1)) == 0 && row < rows) y[row] = v;
        } else {
#pragma unroll
            for (int r = 0; r < RPS; r++) {
                float v;
                switch (log2s) {   // uniform: the lanes of a row slot sum on the VALU
                    case 5: v = group_sum<32>(acc[r]); break;
                    case 4: v = group_sum<16>(acc[r]); break;
                    case 3: v = group_sum<8>(acc[r]); break;
                    case 2: v = group_sum<4>(acc[r]); break;
                    case 1: v = group_sum<2>(acc[r]); break;
                    default: v = acc[r]; break;
                }
                const uint32_t row = row_of(base, r);
                if (s == 0 && row < rows) y[row] = v;
            }
        }
    }
}

template <class QT, int IPL_T, int RPS, int MODE, int NW = 4>
__global__ void __launch_bounds__(64 * NW)
    k_gemv(const uint8_t *__restrict__ w, uint32_t rows, uint32_t cols, uint64_t rb, uint32_t log2s,
           const float *xf, const uint8_t *xq, float *__restrict__ y) {
    extern __shared__ __align__(16) uint8_t lds[];
    gemv_rows<QT, IPL_T, RPS, MODE, NW>(w, rows, cols, rb, log2s, xf, xq, y, blockIdx.x, gridDim.x, lds);
}

// Up to four GEMVs over one activation in one launch (the engine's
// matvec_multi: q, k and v of a layer). Matrix m owns workgroups
// [end[m-1], end[m]) and runs the single-matrix body on them, so each row's
// arithmetic, and its bits, are those of k_gemv.
template <int IPL4, int RPS4, int IPL6, int RPS6, int MODE>
__global__ void __launch_bounds__(256) k_gemv_multi(GemvMultiArgs g) {
    extern __shared__ __align__(16) uint8_t lds[];
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < GEMV_MULTI_MAX - 1; i++)
        if (blockIdx.x >= g.end[i]) m = i + 1;   // end[] is non-decreasing, padded with the total
    const uint32_t start = m ? g.end[m - 1] : 0;
    const uint32_t blk = blockIdx.x - start, nblk = g.end[m] - start;
    if (g.type[m] == T_Q4_K)
        gemv_rows<Q4K, IPL4, RPS4, MODE>(g.w[m], g.rows[m], g.cols, (uint64_t)(g.cols / 256) * Q4K::BB, g.log2s4,
                                         g.x, nullptr, g.y[m], blk, nblk, lds);
    else
        gemv_rows<Q6K, IPL6, RPS6, MODE>(g.w[m], g.rows[m], g.cols, (uint64_t)(g.cols / 256) * Q6K::BB, g.log2s6,
                                         g.x, nullptr, g.y[m], blk, nblk, lds);
}

static int ilog2(uint32_t v) {
    int l = 0;
    while ((1u << (l + 1)) <= v) l++;
    return l;
}

// S = largest power of two <= 64 dividing the item count.
static uint32_t lanes_per_row(uint32_t items) {
    uint32_t s = 64;
    while (s > 1 && items % s) s >>= 1;
    return s;
}

// Waves per workgroup of a single GEMV: the count (4, 6 or 8) whose grid
// puts the fewest rows on the busiest CU (each CU streams at most ~25 GB/s,
// so the busiest one sets the time), the smallest among equals. 6144 rows of
// 16 per 4-wave workgroup are 384 workgroups, two on half of 256 CUs; 6
// waves make 256 workgroups of 24 rows, one per CU.
static int gemv_waves(uint64_t rows, uint32_t rows_per_wave, int cus) {
    int best = 4;
    uint64_t best_rows = ~0ull;
    for (int nw : {4, 6, 8}) {
        const uint64_t per = (uint64_t)nw * rows_per_wave;
        const uint64_t iters = (rows + per - 1) / per;
        const uint64_t busiest = (iters + cus - 1) / cus * per;
        if (busiest < best_rows) best = nw, best_rows = busiest;
    }
    return best;
}

template <class QT, int MODE>
static hipError_t gemv_dispatch(const uint8_t *w, uint64_t rows, uint64_t cols, const float *xf, const uint8_t *xq,
                                float *y, hipStream_t st) {
    const uint32_t items = (uint32_t)(cols / 256) * QT::IPB;
    const uint32_t S = lanes_per_row(items);
    const uint32_t ipl = items / S;
    const uint64_t rb = cols / 256 * QT::BB;
    const uint32_t lds = MODE == 0 ? actf_bytes((uint32_t)cols) : act_bytes((uint32_t)cols);
    const int cus = device_cu_count();
    const uint32_t slots = 64 / S;
    auto go = [&](auto kern, int rps, int nw) -> hipError_t {
        const uint64_t rows_iter = (uint64_t)nw * slots * rps;
        uint64_t iters = (rows + rows_iter - 1) / rows_iter;
        const uint64_t cap = 8ull * cus;
        const uint32_t grid = (uint32_t)(iters < cap ? iters : cap);
        if (lds > 64 * 1024) {
            hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * nw), lds, st, w, (uint32_t)rows, (uint32_t)cols, rb,
                           (uint32_t)ilog2(S), xf, xq, y);
        return hipGetLastError();
    };
    constexpr bool Q4 = QT::TYPE == T_Q4_K;
    auto waves = [&](int rps) { return gemv_waves(rows, slots * rps, cus); };
    switch (ipl) {
        case 1:
            if constexpr (Q4) {
                switch (waves(4)) {
                    case 6: return go(k_gemv<QT, 1, 4, MODE, 6>, 4, 6);
                    case 8: return go(k_gemv<QT, 1, 4, MODE, 8>, 4, 8);
                    default: return go(k_gemv<QT, 1, 4, MODE>, 4, 4);
                }
            } else {
                return go(k_gemv<QT, 1, 2, MODE>, 2, 4);
            }
        case 2: return Q4 ? go(k_gemv<QT, 2, 2, MODE>, 2, 4) : go(k_gemv<QT, 2, 1, MODE>, 1, 4);
        case 3: return go(k_gemv<QT, 3, 1, MODE>, 1, 4);
        default: return go(k_gemv<QT, 0, 1, MODE>, 1, 4);
    }
}

// Rows per workgroup pass of the unrolled instantiations (the same choice
// gemv_dispatch makes; the generic path takes one row per lane slot).
static int gemv_rps(uint32_t type, uint32_t ipl) {
    if (type == T_Q4_K) return ipl == 1 ? 4 : (ipl == 2 ? 2 : 1);
    return ipl == 1 ? 2 : 1;
}

hipError_t launch_gemv_multi(int n, const uint32_t *types, const uint8_t *const *ws, const uint64_t *rows,
                             uint64_t cols, const float *x, float *const *ys, int mode, hipStream_t st) {
    GemvMultiArgs g{};
    const uint32_t items4 = (uint32_t)(cols / 256) * Q4K::IPB, items6 = (uint32_t)(cols / 256) * Q6K::IPB;
    const uint32_t s4 = lanes_per_row(items4), s6 = lanes_per_row(items6);
    const uint32_t ipl4 = items4 / s4, ipl6 = items6 / s6;
    // The unrolled pairs that one column count gives (cols 256..2048, 4096,
    // 6144); any other pair runs the generic item loop for both types.
    int sel = 0;   // 0 generic, 1 (1,1), 2 (2,1), 3 (3,3)
    if (ipl4 == 1 && ipl6 == 1) sel = 1;
    else if (ipl4 == 2 && ipl6 == 1) sel = 2;
    else if (ipl4 == 3 && ipl6 == 3) sel = 3;
    uint64_t iters[GEMV_MULTI_MAX] = {0}, total = 0;
    for (int i = 0; i < n; i++) {
        const uint32_t ipl = types[i] == T_Q4_K ? ipl4 : ipl6;
        const uint32_t S = types[i] == T_Q4_K ? s4 : s6;
        const uint64_t rows_iter = 4ull * (64 / S) * (sel ? gemv_rps(types[i], ipl) : 1);
        iters[i] = (rows[i] + rows_iter - 1) / rows_iter;
        total += iters[i];
    }
    if (!total) return hipSuccess;
    const uint64_t cap = 8ull * device_cu_count();
    uint32_t end = 0;
    for (int i = 0; i < GEMV_MULTI_MAX; i++) {
        if (i < n) {
            uint64_t wg = iters[i];
            if (total > cap && wg) {   // share the capped grid in proportion, at least one each
                wg = wg * cap / total;
                if (!wg) wg = 1;
            }
            end += (uint32_t)wg;
            g.w[i] = ws[i];
            g.y[i] = ys[i];
            g.rows[i] = (uint32_t)rows[i];
            g.type[i] = types[i];
        }
        g.end[i] = end;   // past n: the total, so no workgroup maps there
    }
    g.cols = (uint32_t)cols;
    g.log2s4 = (uint32_t)ilog2(s4);
    g.log2s6 = (uint32_t)ilog2(s6);
    g.x = x;
    const uint32_t lds = mode == 0 ? actf_bytes((uint32_t)cols) : act_bytes((uint32_t)cols);
    auto go = [&](auto kern) -> hipError_t {
        if (lds > 64 * 1024) {
            hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(kern, dim3(end), dim3(256), lds, st, g);
        return hipGetLastError();
    };
    if (mode == 0) {
        switch (sel) {
            case 1: return go(k_gemv_multi<1, 4, 1, 2, 0>);
            case 2: return go(k_gemv_multi<2, 2, 1, 2, 0>);
            case 3: return go(k_gemv_multi<3, 1, 3, 1, 0>);
            default: return go(k_gemv_multi<0, 1, 0, 1, 0>);
        }
    }
    switch (sel) {
        case 1: return go(k_gemv_multi<1, 4, 1, 2, 2>);
        case 2: return go(k_gemv_multi<2, 2, 1, 2, 2>);
        case 3: return go(k_gemv_multi<3, 1, 3, 1, 2>);
        default: return go(k_gemv_multi<0, 1, 0, 1, 2>);
    }
}

hipError_t launch_gemv(uint32_t type, const uint8_t *w, uint64_t rows, uint64_t cols, const float *xf,
                       const uint8_t *xq, float *y, int mode, hipStream_t s) {
    if (type == T_Q4_K) {
        if (mode == 0) return gemv_dispatch<Q4K, 0>(w, rows, cols, xf, xq, y, s);
        if (mode == 1) return gemv_dispatch<Q4K, 1>(w, rows, cols, xf, xq, y, s);
        return gemv_dispatch<Q4K, 2>(w, rows, cols, xf, xq, y, s);
    }
    if (mode == 0) return gemv_dispatch<Q6K, 0>(w, rows, cols, xf, xq, y, s);
    if (mode == 1) return gemv_dispatch<Q6K, 1>(w, rows, cols, xf, xq, y, s);
    return gemv_dispatch<Q6K, 2>(w, rows, cols, xf, xq, y, s);
}

// ---------------------------------------------------------------------------
// Per-block integer sums through the same item routines the GEMV uses.
// One thread per (row, block, item pair) for Q4_K (two half-items summed), one
// per (row, block, item) for Q6_K.
// ---------------------------------------------------------------------------
template <class QT>
__global__ void __launch_bounds__(256) k_isums(const uint8_t *__restrict__ w, uint32_t rows, uint32_t cols,
                                               const uint8_t *__restrict__ xq, int32_t *__restrict__ out) {
    extern __shared__ __align__(16) uint8_t lds[];
    Act a = act_carve(lds, cols);
    act_stage_from_q8(xq, cols, a);
    __syncthreads();
    const uint32_t nb = cols / 256;
    const uint64_t rb = (uint64_t)nb * QT::BB;
    constexpr uint32_t per_blk = QT::TYPE == T_Q4_K ? 4 : 4;   // threads per block
    const uint64_t total = (uint64_t)rows * nb * per_blk;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t c = (uint32_t)(t % per_blk);
        const uint64_t rbk = t / per_blk;
        const uint32_t b = (uint32_t)(rbk % nb);
        const uint64_t row = rbk / nb;
        const uint8_t *blk = w + row * rb + (uint64_t)b * QT::BB;
        if constexpr (QT::TYPE == T_Q4_K) {
            // group g = c: items 2g (hh=0) and 2g+1 (hh=1) cover sub-blocks 2g, 2g+1
            int l0, h0, l1, h1;
            Q4K::isums(Q4K::load(blk, 2 * c), 2 * c, a.qs + 256 * b, l0, h0);
            Q4K::isums(Q4K::load(blk, 2 * c + 1), 2 * c + 1, a.qs + 256 * b, l1, h1);
            int32_t *o = out + row * (cols / 32) + 8 * b + 2 * c;
            o[0] = l0 + l1;
            o[1] = h0 + h1;
        } else {
            int s4[4];
            Q6K::isums(Q6K::load(blk, c), c, a, b, s4);
            const int n = c >> 1, k = c & 1;
            int32_t *o = out + row * (cols / 16) + 16 * b + 8 * n + k;
            for (int tq = 0; tq < 4; tq++) o[2 * tq] = s4[tq];
        }
    }
}

hipError_t launch_isums(uint32_t type, const uint8_t *w, uint64_t rows, uint64_t cols, const uint8_t *xq,
                        int32_t *out, hipStream_t s) {
    const uint64_t total = rows * (cols / 256) * 4;
    uint64_t grid = (total + 255) / 256;
    if (grid > 4096) grid = 4096;
    const uint32_t lds = act_bytes((uint32_t)cols);
    if (type == T_Q4_K)
        hipLaunchKernelGGL(k_isums<Q4K>, dim3((uint32_t)grid), dim3(256), lds, s, w, (uint32_t)rows, (uint32_t)cols,
                           xq, out);
    else
        hipLaunchKernelGGL(k_isums<Q6K>, dim3((uint32_t)grid), dim3(256), lds, s, w, (uint32_t)rows, (uint32_t)cols,
                           xq, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Synthetic data: counter-based splitmix64 stream, one 64-bit draw per 8 bytes.
// Scale fields get |N(0, sigma)| (Box-Muller) encoded as f16.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ float u01(uint64_t r) { return ((float)(r >> 40) + 0.5f) * (1.0f / 16777216.0f); }
__device__ __forceinline__ float halfnormal(uint64_t key, float sigma) {
    const uint64_t r = splitmix64(key);
    const float u1 = u01(r), u2 = u01(splitmix64(r ^ 0x5DEECE66Dull));
    return fabsf(sigma * sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2));
}

__global__ void __launch_bounds__(256) k_synth_blocks(uint32_t type, uint8_t *__restrict__ dst, uint64_t nblocks,
                                                      uint64_t seed, float sigma) {
    const uint32_t bb = type == T_Q4_K ? 144 : 210;
    const uint64_t total = nblocks * bb;
    const uint64_t nwords = (total + 7) / 8;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nwords; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = splitmix64(seed * 0x2545F4914F6CDD1Dull + i);
        const uint64_t off = i * 8;
        if (off + 8 <= total && (off & 7) == 0 && ((uintptr_t)dst & 7) == 0) {
            *(uint64_t *)(dst + off) = r;
        } else {
            for (int k = 0; k < 8 && off + k < total; k++) dst[off + k] = (uint8_t)(r >> (8 * k));
        }
    }
}

__global__ void __launch_bounds__(256) k_synth_scales(uint32_t type, uint8_t *__restrict__ dst, uint64_t nblocks,
                                                      uint64_t seed, float sigma) {
    for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblocks; b += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t key = (seed ^ 0xA0761D6478BD642Full) * 0x9E3779B97F4A7C15ull + 2 * b;
        if (type == T_Q4_K) {
            uint8_t *blk = dst + b * 144;
            const uint32_t d = f2h_rne(halfnormal(key, sigma)), m = f2h_rne(halfnormal(key + 1, sigma));
            blk[0] = (uint8_t)d; blk[1] = (uint8_t)(d >> 8);
            blk[2] = (uint8_t)m; blk[3] = (uint8_t)(m >> 8);
        } else {
            uint8_t *blk = dst + b * 210;
            const uint32_t d = f2h_rne(halfnormal(key, sigma));
            blk[208] = (uint8_t)d; blk[209] = (uint8_t)(d >> 8);
        }
    }
}

hipError_t launch_synth_blocks(uint32_t type, uint8_t *dst, uint64_t nblocks, uint64_t seed, float sigma,
                               hipStream_t s) {
    const uint32_t bb = type == T_Q4_K ? 144 : 210;
    const uint64_t nwords = (nblocks * bb + 7) / 8;
    uint64_t grid = (nwords + 255) / 256;
    if (grid > 16384) grid = 16384;
    hipLaunchKernelGGL(k_synth_blocks, dim3((uint32_t)grid), dim3(256), 0, s, type, dst, nblocks, seed, sigma);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    uint64_t g2 = (nblocks + 255) / 256;
    if (g2 > 16384) g2 = 16384;
    hipLaunchKernelGGL(k_synth_scales, dim3((uint32_t)g2), dim3(256), 0, s, type, dst, nblocks, seed, sigma);
    return hipGetLastError();
}

__global__ void __launch_bounds__(256) k_synth_normal(float *__restrict__ dst, uint64_t n, uint64_t seed, float sigma) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = splitmix64(seed * 0xD1B54A32D192ED03ull + i);
        const float u1 = u01(r), u2 = u01(splitmix64(r ^ 0x5DEECE66Dull));
        dst[i] = sigma * sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
    }
}

hipError_t launch_synth_normal(float *dst, uint64_t n, uint64_t seed, float sigma, hipStream_t s) {
    uint64_t grid = (n + 255) / 256;
    if (grid > 16384) grid = 16384;
    hipLaunchKernelGGL(k_synth_normal, dim3((uint32_t)grid), dim3(256), 0, s, dst, n, seed, sigma);
    return hipGetLastError();
}

__global__ void k_step_advance(int32_t *step, int32_t n) {
    if (threadIdx.x == 0) {
        const int32_t v = *step + 1;
        *step = v >= n ? 0 : v;
    }
}

hipError_t launch_step_advance(int32_t *step, int32_t n_steps, hipStream_t s) {
    hipLaunchKernelGGL(k_step_advance, dim3(1), dim3(64), 0, s, step, n_steps);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Streaming copy, 16 B per lane per step (n % 16 == 0).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_copy(const uint4 *__restrict__ src, uint4 *__restrict__ dst, uint64_t n16) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

hipError_t launch_copy(const uint8_t *src, uint8_t *dst, uint64_t n, hipStream_t s) {
    const uint64_t n16 = n / 16;
    uint64_t grid = (n16 + 255) / 256;
    if (grid > 8192) grid = 8192;
    hipLaunchKernelGGL(k_copy, dim3((uint32_t)grid), dim3(256), 0, s, (const uint4 *)src, (uint4 *)dst, n16);
    return hipGetLastError();
}

}  // namespace kq
