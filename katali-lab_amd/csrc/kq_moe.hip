// kq_moe.hip — the fused per-layer MoE kernel.
//
// y = sum_slot w_slot * Down_e(q8(SiLU(Gate_e x) * Up_e x)) over the selected
// experts (rank order) and an optional always-on shared expert (weight 1).
//
// Phase A unit = (slot, 32 intermediate rows): 32 gate + 32 up row dots
//   against the layer activation (q8_1 in LDS), then h = SiLU(g)*u for those
//   32 values is quantized to one q8_1 block inside the workgroup and written
//   to the scratch hq8[slot][block].
// Phase B unit = a tile of output rows: for every row and every slot the down
//   row is dotted with that slot's h (q8_1 in LDS); the weighted sum over the
//   slots is formed in a fixed order by one thread per row, so the result is
//   deterministic (no float atomics).
// Mode 0 runs A and B as two launches; mode 1 runs both in one launch: each
// workgroup does its A units, publishes them with a device-scope counter, and
// waits (bounded) for all A units before its B tile. The grid never exceeds
// the co-resident capacity, and the last workgroup to finish resets the
// counters, so back-to-back launches and graph replays need no memset.
//
// Routing: when logits are given, every workgroup computes the same top-k
// (largest logit first, lower index on ties) and weights
// w_r = exp(l_r - l_max) / sum_sel exp(l_j - l_max) (rank-order sum), which is
// softmax followed by renormalisation over the selection.
#include "kq_device.h"
#include "kq_launch.h"

namespace kq {

constexpr int MAX_SEL = 16;
constexpr int MAX_SLOTS = MAX_SEL + 1;
constexpr uint32_t SPIN_LIMIT = 1u << 22;

struct Route {
    int32_t ids[MAX_SLOTS];
    float w[MAX_SLOTS];
};

__device__ __forceinline__ const float *route_logits(const MoeArgs &a) {
    const float *l = a.logits;
    if (a.step) l += (uint64_t)(*a.step) * a.logits_stride;
    return l;
}

// Wave 0 computes the routing into LDS; the caller synchronises.
__device__ void route(const MoeArgs &a, Route *rt) {
    if (threadIdx.x >= WAVE) return;
    const int lane = threadIdx.x;
    if (a.logits) {
        const float *lg = route_logits(a);
        constexpr int MAXJ = 8;   // n_expert <= 512
        float v[MAXJ];
        uint32_t taken = 0;
#pragma unroll
        for (int j = 0; j < MAXJ; j++) {
            const uint32_t e = lane + WAVE * j;
            v[j] = e < a.n_expert ? lg[e] : -INFINITY;
            if (e >= a.n_expert) taken |= 1u << j;
        }
        for (int r = 0; r < a.n_sel; r++) {
            float bv = -INFINITY;
            int bi = 0x7FFFFFFF;
#pragma unroll
            for (int j = 0; j < MAXJ; j++) {
                const int e = lane + WAVE * j;
                if (!(taken & (1u << j)) && (v[j] > bv || (v[j] == bv && e < bi))) { bv = v[j]; bi = e; }
            }
            for (int o = WAVE / 2; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o, WAVE);
                const int oi = __shfl_xor(bi, o, WAVE);
                if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
            }
            if ((bi & (WAVE - 1)) == lane) taken |= 1u << (bi / WAVE);
            if (lane == 0) rt->ids[r] = bi;
        }
        if (lane == 0) {
            const float lmax = lg[rt->ids[0]];
            float e[MAX_SEL], sum = 0.0f;
            for (int r = 0; r < a.n_sel; r++) {
                e[r] = kq_expf(lg[rt->ids[r]] - lmax);
                sum += e[r];
            }
            for (int r = 0; r < a.n_sel; r++) rt->w[r] = e[r] / sum;
        }
    } else if (lane < a.n_sel) {
        rt->ids[lane] = a.ids[lane];
        rt->w[lane] = a.wts[lane];
    }
    if (lane == 0) {
        // an id outside the pool (bad input, or NaN-only logits) would index
        // past the expert tensors: flag it and read expert 0 instead
        for (int r = 0; r < a.n_sel; r++) {
            if (rt->ids[r] < 0 || (uint32_t)rt->ids[r] >= a.n_expert) {
                if (blockIdx.x == 0) atomicOr(a.err, 2);
                rt->ids[r] = 0;
            }
        }
        if (a.has_shared) {
            rt->ids[a.n_sel] = -1;
            rt->w[a.n_sel] = 1.0f;
        }
    }
}

// Dot a list of rows against q8_1 activations. Lane-slot `ls` (S lanes each)
// handles rows v = ls, ls + nls, ... < n; RPS rows are loaded before any is
// computed. rowp(v) gives the row's bytes, actp(v) its activation, out(v, acc)
// receives the result (called by the slot's lane 0).
template <class QT, int IPL_T, int RPS, class RowP, class ActP, class Out>
__device__ __forceinline__ void rows_dot(uint32_t n, uint32_t log2s, uint32_t ipl_rt, RowP rowp, ActP actp, Out out) {
    const uint32_t S = 1u << log2s;
    const uint32_t lane = threadIdx.x & (WAVE - 1);
    const uint32_t ls = (threadIdx.x / WAVE) * (WAVE >> log2s) + (lane >> log2s);
    const uint32_t nls = (blockDim.x / WAVE) * (WAVE >> log2s);
    const uint32_t s = lane & (S - 1);
    for (uint32_t v0 = ls; v0 < n; v0 += RPS * nls) {
        float acc[RPS];
        if constexpr (IPL_T > 0) {
            typename QT::Raw raw[RPS][IPL_T];
#pragma unroll
            for (int r = 0; r < RPS; r++) {
                const uint32_t v = v0 + r * nls;
                if (v < n) {
                    const uint8_t *rp = rowp(v);
#pragma unroll
                    for (int i = 0; i < IPL_T; i++) {
                        const uint32_t item = s + S * i;
                        raw[r][i] = QT::load(rp + (item / QT::IPB) * QT::BB, item % QT::IPB);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < RPS; r++) {
                const uint32_t v = v0 + r * nls;
                float x = 0.0f;
                if (v < n) {
                    const Act act = actp(v);
#pragma unroll
                    for (int i = 0; i < IPL_T; i++) {
                        const uint32_t item = s + S * i;
                        x += QT::dot_q8(raw[r][i], item % QT::IPB, act, item / QT::IPB);
                    }
                }
                acc[r] = x;
            }
        } else {
#pragma unroll
            for (int r = 0; r < RPS; r++) {
                const uint32_t v = v0 + r * nls;
                float x = 0.0f;
                if (v < n) {
                    const uint8_t *rp = rowp(v);
                    const Act act = actp(v);
                    for (uint32_t i = 0; i < ipl_rt; i++) {
                        const uint32_t item = s + S * i;
                        x += QT::dot_q8(QT::load(rp + (item / QT::IPB) * QT::BB, item % QT::IPB), item % QT::IPB,
                                        act, item / QT::IPB);
                    }
                }
                acc[r] = x;
            }
        }
#pragma unroll
        for (int r = 0; r < RPS; r++) {
            const float x = wave_sum_xor(acc[r], (int)S);
            const uint32_t v = v0 + r * nls;
            if (s == 0 && v < n) out(v, x);
        }
    }
}

struct Geo {
    uint32_t log2s_a, ipl_a;   // gate/up rows (hidden columns)
    uint32_t log2s_b, ipl_b;   // down rows (ffn columns)
    uint64_t rb_g, rb_u, rb_d;
    uint32_t n_slots, units_a, tile_b, units_b;
};

template <class QG, class QU, int IPL_A>
__device__ void phase_a(const MoeArgs &a, const Geo &g, const Route *rt, const Act &xa, float *gu, uint32_t unit) {
    const uint32_t nblk = a.ffn / 32;
    const uint32_t slot = unit / nblk, jb = unit % nblk;
    const uint8_t *gb, *ub;
    if ((int)slot < a.n_sel) {
        const uint64_t e = (uint64_t)rt->ids[slot];
        gb = a.gate + e * a.ffn * g.rb_g;
        ub = a.up + e * a.ffn * g.rb_u;
    } else {
        gb = a.gate_sh;
        ub = a.up_sh;
    }
    auto act = [&](uint32_t) -> Act { return xa; };
    auto out = [&](uint32_t v, float x) { gu[v] = x; };
    constexpr int RPS = IPL_A == 1 ? 4 : (IPL_A == 2 ? 2 : 1);
    if constexpr (QG::TYPE == QU::TYPE) {
        auto rowp = [&](uint32_t v) -> const uint8_t * {
            return v < 32 ? gb + (uint64_t)(32 * jb + v) * g.rb_g : ub + (uint64_t)(32 * jb + v - 32) * g.rb_u;
        };
        rows_dot<QG, IPL_A, RPS>(64, g.log2s_a, g.ipl_a, rowp, act, out);
    } else {
        auto rg = [&](uint32_t v) -> const uint8_t * { return gb + (uint64_t)(32 * jb + v) * g.rb_g; };
        auto ru = [&](uint32_t v) -> const uint8_t * { return ub + (uint64_t)(32 * jb + v) * g.rb_u; };
        auto ou = [&](uint32_t v, float x) { gu[32 + v] = x; };
        rows_dot<QG, 0, 1>(32, g.log2s_a, g.ipl_a, rg, act, out);
        rows_dot<QU, 0, 1>(32, g.log2s_a, g.ipl_a, ru, act, ou);
    }
    __syncthreads();
    if (threadIdx.x < 8) {
        const uint32_t part = threadIdx.x, i0 = 4 * part;
        float4 h;
        h.x = kq_silu_mul(gu[i0 + 0], gu[32 + i0 + 0]);
        h.y = kq_silu_mul(gu[i0 + 1], gu[32 + i0 + 1]);
        h.z = kq_silu_mul(gu[i0 + 2], gu[32 + i0 + 2]);
        h.w = kq_silu_mul(gu[i0 + 3], gu[32 + i0 + 3]);
        uint32_t d16, s16;
        int lo, hi;
        float dd;
        const uint32_t q = quant_q8_1_part(h, d16, s16, lo, hi, dd);
        uint8_t *blk = a.hq8 + ((uint64_t)slot * nblk + jb) * 36;
        *(uint32_t *)(blk + 4 + 4 * part) = q;
        if (part == 0) *(uint32_t *)blk = d16 | (s16 << 16);
    }
    if (a.dbg_gu && threadIdx.x < 64) {
        const uint32_t v = threadIdx.x;
        float *d = a.dbg_gu + (uint64_t)slot * 2 * a.ffn + (v < 32 ? 0 : a.ffn) + 32 * jb + (v & 31);
        *d = gu[v];
    }
}

template <class QD, int IPL_B>
__device__ void phase_b(const MoeArgs &a, const Geo &g, const Route *rt, uint8_t *hl, float *res, uint32_t unit) {
    const uint32_t nblk = a.ffn / 32;
    const uint32_t row0 = unit * g.tile_b;
    const uint32_t nrows = row0 + g.tile_b <= a.hidden ? g.tile_b : a.hidden - row0;
    const uint32_t ab = act_bytes(a.ffn);
    for (uint32_t sl = 0; sl < g.n_slots; sl++)
        act_stage_from_q8(a.hq8 + (uint64_t)sl * nblk * 36, a.ffn, act_carve(hl + sl * ab, a.ffn));
    __syncthreads();
    const uint32_t ns = g.n_slots;
    auto rowp = [&](uint32_t p) -> const uint8_t * {
        const uint32_t r = p / ns, sl = p % ns;
        const uint8_t *db = (int)sl < a.n_sel ? a.down + (uint64_t)rt->ids[sl] * a.hidden * g.rb_d : a.down_sh;
        return db + (uint64_t)(row0 + r) * g.rb_d;
    };
    auto actp = [&](uint32_t p) -> Act { return act_carve(hl + (p % ns) * ab, a.ffn); };
    auto out = [&](uint32_t p, float x) { res[p] = x; };
    constexpr int RPS = IPL_B == 1 ? 2 : 1;
    rows_dot<QD, IPL_B, RPS>(nrows * ns, g.log2s_b, g.ipl_b, rowp, actp, out);
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < nrows; r += blockDim.x) {
        float y = 0.0f;
        for (uint32_t sl = 0; sl < ns; sl++) y = fmaf(rt->w[sl], res[r * ns + sl], y);
        a.y[row0 + r] = y;
    }
}

__device__ __forceinline__ void stage_x(const MoeArgs &a, const Act &xa) {
    if (a.xq) act_stage_from_q8(a.xq, a.hidden, xa);
    else act_stage_from_f32(a.x, a.hidden, xa);
}

// LDS layout (bytes): Route | x act | gu[64] | h acts | res
struct LdsLayout {
    uint32_t route, xact, gu, hacts, res, total;
};
__host__ __device__ inline LdsLayout lds_layout(const MoeArgs &a, const Geo &g) {
    LdsLayout L;
    L.route = 0;
    L.xact = 256;
    L.gu = L.xact + act_bytes(a.hidden);
    L.hacts = L.gu + 64 * 4;
    L.res = L.hacts + g.n_slots * act_bytes(a.ffn);
    L.total = L.res + g.tile_b * g.n_slots * 4;
    return L;
}

template <class QG, class QU, int IPL_A>
__global__ void __launch_bounds__(256) k_moe_a(MoeArgs a, Geo g) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsLayout L = lds_layout(a, g);
    Route *rt = (Route *)(lds + L.route);
    route(a, rt);
    const Act xa = act_carve(lds + L.xact, a.hidden);
    stage_x(a, xa);
    __syncthreads();
    phase_a<QG, QU, IPL_A>(a, g, rt, xa, (float *)(lds + L.gu), blockIdx.x);
}

template <class QD, int IPL_B>
__global__ void __launch_bounds__(256) k_moe_b(MoeArgs a, Geo g) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsLayout L = lds_layout(a, g);
    Route *rt = (Route *)(lds + L.route);
    route(a, rt);
    __syncthreads();
    if (blockIdx.x == 0 && threadIdx.x < (uint32_t)a.n_sel) {
        if (a.ids_out) a.ids_out[threadIdx.x] = rt->ids[threadIdx.x];
        if (a.wts_out) a.wts_out[threadIdx.x] = rt->w[threadIdx.x];
    }
    phase_b<QD, IPL_B>(a, g, rt, lds + L.hacts, (float *)(lds + L.res), blockIdx.x);
}

template <class QG, class QU, class QD, int IPL_A, int IPL_B>
__global__ void __launch_bounds__(256) k_moe_fused(MoeArgs a, Geo g) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsLayout L = lds_layout(a, g);
    Route *rt = (Route *)(lds + L.route);
    route(a, rt);
    const Act xa = act_carve(lds + L.xact, a.hidden);
    stage_x(a, xa);
    __syncthreads();
    for (uint32_t u = blockIdx.x; u < g.units_a; u += gridDim.x) {
        phase_a<QG, QU, IPL_A>(a, g, rt, xa, (float *)(lds + L.gu), u);
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0) atomicAdd(&a.sync[0], 1u);
    }
    if (blockIdx.x == 0 && threadIdx.x < (uint32_t)a.n_sel) {
        if (a.ids_out) a.ids_out[threadIdx.x] = rt->ids[threadIdx.x];
        if (a.wts_out) a.wts_out[threadIdx.x] = rt->w[threadIdx.x];
    }
    __shared__ int ok;
    if (threadIdx.x == 0) {
        uint32_t spins = 0;
        ok = 1;
        while (__hip_atomic_load(&a.sync[0], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < g.units_a) {
            __builtin_amdgcn_s_sleep(2);
            if (++spins > SPIN_LIMIT) {
                ok = 0;
                atomicOr(a.err, 1);
                break;
            }
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (ok) {
        for (uint32_t u = blockIdx.x; u < g.units_b; u += gridDim.x)
            phase_b<QD, IPL_B>(a, g, rt, lds + L.hacts, (float *)(lds + L.res), u);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        const uint32_t done = atomicAdd(&a.sync[1], 1u);
        if (done == gridDim.x - 1) {
            __hip_atomic_store(&a.sync[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.sync[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __threadfence();
        }
    }
}

uint64_t moe_sync_words() { return 64; }

static int ilog2u(uint32_t v) {
    int l = 0;
    while ((1u << (l + 1)) <= v) l++;
    return l;
}
static uint32_t lanes_for(uint32_t items) {
    uint32_t s = 64;
    while (s > 1 && items % s) s >>= 1;
    return s;
}
static uint32_t block_bytes(uint32_t t) { return t == T_Q4_K ? 144 : 210; }
static uint32_t ipb(uint32_t t) { return t == T_Q4_K ? 8 : 4; }

template <class QG, class QU, class QD, int IPL_A, int IPL_B>
static hipError_t moe_go(const MoeArgs &a, const Geo &g, int mode, hipStream_t s, int *grid_out) {
    const LdsLayout L = lds_layout(a, g);
    if (mode == 0) {
        hipLaunchKernelGGL((k_moe_a<QG, QU, IPL_A>), dim3(g.units_a), dim3(256), L.total, s, a, g);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((k_moe_b<QD, IPL_B>), dim3(g.units_b), dim3(256), L.total, s, a, g);
        if (grid_out) *grid_out = (int)g.units_b;
        return hipGetLastError();
    }
    auto kern = k_moe_fused<QG, QU, QD, IPL_A, IPL_B>;
    const int cus = device_cu_count();
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)kern, 256, L.total);
    if (e != hipSuccess) return e;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    const uint32_t cap = (uint32_t)(per_cu * cus);
    uint32_t want = g.units_a > g.units_b ? g.units_a : g.units_b;
    const uint32_t grid = want < cap ? want : cap;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), L.total, s, a, g);
    if (grid_out) *grid_out = (int)grid;
    return hipGetLastError();
}

template <class QG, class QU, class QD>
static hipError_t moe_ipl(const MoeArgs &a, const Geo &g, int mode, hipStream_t s, int *grid_out) {
    const uint32_t ia = g.ipl_a, ib = g.ipl_b;
    if (ia == 1 && ib == 3) return moe_go<QG, QU, QD, 1, 3>(a, g, mode, s, grid_out);
    if (ia == 1 && ib == 1) return moe_go<QG, QU, QD, 1, 1>(a, g, mode, s, grid_out);
    if (ia == 2 && ib == 1) return moe_go<QG, QU, QD, 2, 1>(a, g, mode, s, grid_out);
    if (ia == 2 && ib == 3) return moe_go<QG, QU, QD, 2, 3>(a, g, mode, s, grid_out);
    return moe_go<QG, QU, QD, 0, 0>(a, g, mode, s, grid_out);
}

hipError_t launch_moe(const MoeArgs &a, int mode, hipStream_t s, int *grid_out) {
    Geo g;
    const uint32_t items_a = a.hidden / 256 * ipb(a.gate_type);
    const uint32_t sa = lanes_for(items_a);
    g.log2s_a = ilog2u(sa);
    g.ipl_a = items_a / sa;
    const uint32_t items_b = a.ffn / 256 * ipb(a.down_type);
    const uint32_t sb = lanes_for(items_b);
    g.log2s_b = ilog2u(sb);
    g.ipl_b = items_b / sb;
    g.rb_g = (uint64_t)a.hidden / 256 * block_bytes(a.gate_type);
    g.rb_u = (uint64_t)a.hidden / 256 * block_bytes(a.up_type);
    g.rb_d = (uint64_t)a.ffn / 256 * block_bytes(a.down_type);
    g.n_slots = (uint32_t)a.n_sel + (a.has_shared ? 1u : 0u);
    g.units_a = g.n_slots * (a.ffn / 32);
    const uint32_t lane_slots = 4 * (64 / sb);
    uint32_t tile = lane_slots / g.n_slots;
    if (tile < 1) tile = 1;
    g.tile_b = tile;
    g.units_b = (a.hidden + tile - 1) / tile;
    const bool g4 = a.gate_type == T_Q4_K, u4 = a.up_type == T_Q4_K, d4 = a.down_type == T_Q4_K;
    if (g4 && u4 && !d4) return moe_ipl<Q4K, Q4K, Q6K>(a, g, mode, s, grid_out);
    if (g4 && u4 && d4) return moe_ipl<Q4K, Q4K, Q4K>(a, g, mode, s, grid_out);
    if (!g4 && !u4 && !d4) return moe_ipl<Q6K, Q6K, Q6K>(a, g, mode, s, grid_out);
    if (!g4 && !u4 && d4) return moe_ipl<Q6K, Q6K, Q4K>(a, g, mode, s, grid_out);
    return hipErrorInvalidValue;   // mixed gate/up types are not instantiated
}

}  // namespace kq
