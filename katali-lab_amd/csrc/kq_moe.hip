// kq_moe.hip — the MoE layer: two launches per layer.
//
// y = sum_slot w_slot * Down_e(q8(SiLU(Gate_e x) * Up_e x)) over the selected
// experts (rank order) and an optional always-on shared expert (weight 1).
//
// Kernel A (k_moe_gu), one workgroup per (slot, 32 intermediate rows):
//   route (every workgroup ranks the logits itself), then issue every weight
//   load of its 32 gate + 32 up rows at once (16-byte nibble chunks and block
//   headers in registers), quantize x to q8_1 in LDS and decode the headers
//   into LDS scale records while the loads are in flight, dot with v_dot4
//   against activation slices each lane reads once, reduce the 64 rows with a
//   halving butterfly, and turn the 32 SiLU-GLU outputs into one q8_1 block
//   written to scratch. Workgroup 0 also computes the routing weights and
//   writes the routing for kernel B.
// Kernel B (k_moe_down), one workgroup per tile of output rows:
//   read the routing, issue the down-row loads of every (row, slot) pair of
//   the tile, stage every slot's q8_1 h in LDS meanwhile, dot, and sum the
//   slots in rank order in one thread per row (no float atomics, so results
//   are deterministic).
// The kernel boundary is the only dependency between the two phases: an
// in-kernel grid dependency measured slower on gfx950 (agent-scope fences
// write back / invalidate L2; atomic and poll round trips cost more than the
// boundary).
//
// Routing: expert e's rank is the number of experts with a larger logit (or
// an equal logit and a lower index); ranks 0..n_sel-1 are selected. Weights
// w_r = exp(l_r - l_max) / sum_sel exp(l_j - l_max) in rank order, which is
// softmax followed by renormalisation over the selection.
#include "kq_device.h"
#include "kq_launch.h"

namespace kq {

constexpr int MAX_SEL = 16;
constexpr int MAX_SLOTS = MAX_SEL + 1;
constexpr uint32_t MAX_EXPERT = 512;

struct Route {
    int32_t ids[MAX_SLOTS];
    float w[MAX_SLOTS];
};

__device__ __forceinline__ const float *route_logits(const MoeArgs &a) {
    const float *l = a.logits;
    if (a.step) l += (uint64_t)(*a.step) * a.logits_stride;
    return l;
}

// Block-wide routing into LDS: the selected ids (and, for explicit routing,
// the given weights). `lg` is an LDS scratch of n_expert floats rounded up to
// a multiple of 4 (padding ranks last) that keeps the logits for
// route_publish. Every thread must already have issued `lv` = its logit loads
// (see load_logits) so the global latency overlaps other loads. Ends with a
// barrier.
constexpr int LPT = MAX_EXPERT / 256;   // logits per thread
__device__ __forceinline__ void load_logits(const MoeArgs &a, float (&lv)[LPT]) {
    const float *src = a.logits ? route_logits(a) : nullptr;
#pragma unroll
    for (int i = 0; i < LPT; i++) {
        const uint32_t e = threadIdx.x + 256 * i;
        lv[i] = (src && e < a.n_expert) ? src[e] : -INFINITY;
    }
}

__device__ void route_rank(const MoeArgs &a, Route *rt, float *lg, const float (&lv)[LPT]) {
    const uint32_t t = threadIdx.x;
    const uint32_t n4 = (a.n_expert + 3) & ~3u;
    if (a.logits) {
#pragma unroll
        for (int i = 0; i < LPT; i++) {
            const uint32_t e = t + 256 * i;
            if (e < n4) lg[e] = lv[i] != lv[i] ? -INFINITY : lv[i];   // NaN and padding rank last
        }
        __syncthreads();
        for (uint32_t e = t; e < a.n_expert; e += blockDim.x) {
            const float v = lg[e];
            uint32_t rank = 0;
#pragma unroll 8
            for (uint32_t j = 0; j < n4; j += 4) {
                const float4 u = *(const float4 *)(lg + j);
                rank += (u.x > v) | ((u.x == v) & (j + 0 < e));
                rank += (u.y > v) | ((u.y == v) & (j + 1 < e));
                rank += (u.z > v) | ((u.z == v) & (j + 2 < e));
                rank += (u.w > v) | ((u.w == v) & (j + 3 < e));
            }
            if (rank < (uint32_t)a.n_sel) rt->ids[rank] = (int32_t)e;   // ranks are a permutation
        }
    } else if (t < (uint32_t)a.n_sel) {
        rt->ids[t] = a.ids[t];
        rt->w[t] = a.wts[t];
    }
    if (t == 0 && a.has_shared) {
        rt->ids[a.n_sel] = -1;
        rt->w[a.n_sel] = 1.0f;
    }
    __syncthreads();
    // an id outside the pool (bad explicit ids) would index past the expert
    // tensors: clamp it to 0 for addressing; workgroup 0 reports it
}

// Workgroup 0 of kernel A: weights (when routing from logits), the routing
// scratch for kernel B, the optional routing outputs, and the error bit.
__device__ void route_publish(const MoeArgs &a, const Route *rt, const float *lg) {
    if (threadIdx.x != 0) return;
    int32_t ids[MAX_SEL];
    bool bad = false;
    for (int r = 0; r < a.n_sel; r++) {
        const int32_t e = rt->ids[r];
        bad |= e < 0 || (uint32_t)e >= a.n_expert;
        ids[r] = e;
    }
    float sum = 0.0f;
    if (a.logits) {
        // two passes over the same exp values: the rank-order sum, then the
        // quotients
        const float lmax = lg[ids[0]];
        for (int r = 0; r < a.n_sel; r++) sum += kq_expf(lg[ids[r]] - lmax);
    }
    for (int r = 0; r < MAX_SLOTS; r++) {
        int32_t e = -1;
        float w = 0.0f;
        if (r < a.n_sel) {
            e = ids[r];
            w = a.logits ? kq_expf(lg[e] - lg[ids[0]]) / sum : rt->w[r];
            if (a.ids_out) a.ids_out[r] = e;
            if (a.wts_out) a.wts_out[r] = w;
        } else if (r == a.n_sel && a.has_shared) {
            w = 1.0f;
        }
        a.route_ids[r] = (r < a.n_sel && (uint32_t)e >= a.n_expert) ? 0 : e;   // addressing stays in the pool
        a.route_w[r] = w;
    }
    if (bad) atomicOr(a.err, 2);
}

// Sum R per-lane values over the 64 lanes of a wave for R rows at once: each
// halving step sends the half of the rows the partner keeps (R/2 shuffles),
// then the remaining offsets finish a plain butterfly. Afterwards every lane
// holds the full sum of row (lane >> (6 - log2 R)) & (R - 1).
template <int N, int OFF, int R>
__device__ __forceinline__ void reduce_halve(float (&acc)[R], int lane) {
    if constexpr (N > 1) {
        constexpr int HALF = N / 2;
        const bool upper = lane & OFF;
#pragma unroll
        for (int i = 0; i < HALF; i++) {
            const float send = upper ? acc[i] : acc[i + HALF];
            const float keep = upper ? acc[i + HALF] : acc[i];
            acc[i] = keep + __shfl_xor(send, OFF, WAVE);
        }
        reduce_halve<HALF, OFF / 2, R>(acc, lane);
    }
}
template <int R>
__device__ __forceinline__ float reduce_rows(float (&acc)[R]) {
    const int lane = threadIdx.x & 63;
    reduce_halve<R, 32, R>(acc, lane);
    constexpr int LOG = R >= 16 ? 4 : (R >= 8 ? 3 : (R >= 4 ? 2 : (R >= 2 ? 1 : 0)));
    float v = acc[0];
#pragma unroll
    for (int off = 32 >> LOG; off > 0; off >>= 1) v += __shfl_xor(v, off, WAVE);
    return v;
}

// ---------------------------------------------------------------------------
// Kernel A: 64 Q4_K rows (32 gate + 32 up) per workgroup, NB blocks per row.
// Wave w owns rows 16w..16w+15 (waves 0-1 gate, 2-3 up). Lane l always takes
// the same lane item of every row it touches, so its activation slice (two
// 16-byte q8 chunks, their scales and half-block sums) is read from LDS once:
//   ITEMS = 8*NB >= 64: the k-th chunk is item 64*(k % M) + l of row k / M
//                       (M = ITEMS/64 slices per lane);
//   ITEMS < 64:         64/ITEMS rows share a wave instruction; the k-th
//                       chunk is item l % ITEMS of row l / ITEMS + k*64/ITEMS.
// Block headers are decoded once per (row, block) into LDS as
// {d*sc[2g], d*sc[2g+1], dmin*m[2g], dmin*m[2g+1]} per group g.
// ---------------------------------------------------------------------------
struct LdsA {
    uint32_t route, logits, xact, scl, gu, total;
};
__host__ __device__ inline LdsA lds_a(uint32_t hidden, uint32_t nb) {
    LdsA L;
    L.route = 0;
    L.logits = 256;
    L.xact = L.logits + MAX_EXPERT * 4;
    L.scl = L.xact + act_bytes(hidden);
    L.gu = L.scl + 64 * nb * 64;
    L.total = L.gu + 64 * 4;
    return L;
}

// the activation side of one lane item (constant over rows)
struct XSlice {
    int4 xl, xh;
    float d8lo, d8hi, qlo, qhi;
};
__device__ __forceinline__ XSlice x_slice(const Act &xa, uint32_t it) {
    const uint32_t b = it / 8, c = it % 8, g = c >> 1, hh = c & 1;
    const int8_t *al = xa.qs + 256 * b + 64 * g + 16 * hh;
    XSlice x;
    x.xl = *(const int4 *)al;
    x.xh = *(const int4 *)(al + 32);
    const uint32_t k = 8 * b + 2 * g;
    x.d8lo = xa.d8[k];
    x.d8hi = xa.d8[k + 1];
    x.qlo = (float)xa.qs16[2 * k + hh];
    x.qhi = (float)xa.qs16[2 * k + 2 + hh];
    return x;
}
// same arithmetic as Q4K::dot_q8, with the scales pre-decoded
__device__ __forceinline__ float item_dot(const uint4 &q, const float4 &sc, const XSlice &x) {
    int slo, shi;
    Q4K::isums_x(q, x.xl, x.xh, slo, shi);
    const float vlo = fmaf(sc.x, (float)slo, -(sc.z * x.qlo));
    const float vhi = fmaf(sc.y, (float)shi, -(sc.w * x.qhi));
    return fmaf(x.d8lo, vlo, x.d8hi * vhi);
}

template <int NB>
__global__ void __launch_bounds__(256) k_moe_gu(MoeArgs a) {
    constexpr int ITEMS = 8 * NB;              // lane items per row
    constexpr int LPL = 2 * NB;                // 16 rows x ITEMS / 64 lanes
    constexpr int GROUPS = LPL > 16 ? LPL / 16 : 1;
    constexpr int RPG = 16 / GROUPS;           // rows per group
    constexpr int LPG = RPG * ITEMS / 64;      // chunks per lane per group
    constexpr int M = ITEMS >= 64 ? ITEMS / 64 : 1;   // activation slices per lane
    constexpr int LOG_RPG = RPG == 16 ? 4 : (RPG == 8 ? 3 : (RPG == 4 ? 2 : (RPG == 2 ? 1 : 0)));
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsA L = lds_a(a.hidden, NB);
    Route *rt = (Route *)(lds + L.route);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t nblk = a.ffn / 32;
    const uint32_t slot = blockIdx.x / nblk, jb = blockIdx.x % nblk;

    // logits, then x (fp32), into registers; their latency overlaps
    float lv[LPT];
    load_logits(a, lv);
    constexpr int XTASKS = 64 * NB;            // quantizer lane tasks (8 per 32-block)
    constexpr int XPT = (XTASKS + 255) / 256;
    float4 xv[XPT];
    if (a.xq == nullptr) {
#pragma unroll
        for (int i = 0; i < XPT; i++)
            if (tid + 256 * i < XTASKS) xv[i] = *(const float4 *)(a.x + 4 * (tid + 256 * i));
    }
    route_rank(a, rt, (float *)(lds + L.logits), lv);

    const uint64_t rb = NB * 144;
    const uint8_t *gb, *ub;
    if ((int)slot < a.n_sel) {
        int32_t id = rt->ids[slot];
        if ((uint32_t)id >= a.n_expert) id = 0;   // bad explicit id: reported by workgroup 0
        const uint64_t e = (uint64_t)id;
        gb = a.gate + e * a.ffn * rb;
        ub = a.up + e * a.ffn * rb;
    } else {
        gb = a.gate_sh;
        ub = a.up_sh;
    }
    auto row_ptr = [&](uint32_t v) -> const uint8_t * {   // v in [0, 64)
        return v < 32 ? gb + (uint64_t)(32 * jb + v) * rb : ub + (uint64_t)(32 * jb + v - 32) * rb;
    };
    auto chunk = [&](int grp, int k) -> const uint8_t * {
        uint32_t r, it;
        if constexpr (ITEMS >= 64) {
            r = grp * RPG + k / M;
            it = 64 * (k % M) + lane;
        } else {
            r = lane / ITEMS + k * (64 / ITEMS);
            it = lane % ITEMS;
        }
        return row_ptr(16 * wave + r) + (it / 8) * 144 + 16 + 16 * (it % 8);
    };

    // all weight loads: block headers first (consumed first), then chunks
    constexpr int HPT = (64 * NB + 255) / 256;
    uint4 hv[HPT];
#pragma unroll
    for (int i = 0; i < HPT; i++) {
        const uint32_t h = tid + 256 * i;
        if (h < 64 * NB) hv[i] = ld16(row_ptr(h / NB) + (h % NB) * 144);
    }
    uint4 q[LPG];
#pragma unroll
    for (int k = 0; k < LPG; k++) q[k] = ld16(chunk(0, k));

    // quantize x into LDS while the weights stream in
    const Act xa = act_carve(lds + L.xact, a.hidden);
    if (a.xq) {
        act_stage_from_q8(a.xq, a.hidden, xa);
    } else {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const uint32_t t = tid + 256 * i, blk = t >> 3, part = t & 7;
            if (t >= XTASKS) break;
            uint32_t d16, s16;
            int lo, hi;
            float dd;
            const uint32_t qv = quant_q8_1_part(xv[i], d16, s16, lo, hi, dd);
            *(uint32_t *)(xa.qs + 32 * blk + 4 * part) = qv;
            if (part == 0) {
                xa.d8[blk] = dd;
                xa.qs16[2 * blk] = lo;
                xa.qs16[2 * blk + 1] = hi;
            }
        }
    }
    // decode the 64*NB block headers into per-group scale quadruples
    float4 *scl = (float4 *)(lds + L.scl);
#pragma unroll
    for (int i = 0; i < HPT; i++) {
        const uint32_t h = tid + 256 * i;
        if (h < 64 * NB) {
            Q4K::Raw raw;
            raw.h = hv[i];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                float4 v;
                Q4K::scales(raw, g, v.x, v.y, v.z, v.w);
                scl[4 * h + g] = v;
            }
        }
    }
    __syncthreads();

    XSlice xs[M];
#pragma unroll
    for (int m = 0; m < M; m++) xs[m] = x_slice(xa, ITEMS >= 64 ? 64 * m + lane : lane % ITEMS);
    float *gu = (float *)(lds + L.gu);
#pragma unroll
    for (int grp = 0; grp < GROUPS; grp++) {
        if (grp > 0) {
#pragma unroll
            for (int k = 0; k < LPG; k++) q[k] = ld16(chunk(grp, k));
        }
        if constexpr (ITEMS >= 64) {
            float acc[RPG];
#pragma unroll
            for (int r = 0; r < RPG; r++) acc[r] = 0.0f;
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t it = 64 * (k % M) + lane;
                const uint32_t row = 16 * wave + grp * RPG + k / M;
                const float4 sc = scl[4 * (row * NB + it / 8) + (it % 8) / 2];
                acc[k / M] += item_dot(q[k], sc, xs[k % M]);
            }
            const float v = reduce_rows<RPG>(acc);
            constexpr int SH = 6 - LOG_RPG;
            const uint32_t r = (lane >> SH) & (RPG - 1);
            if ((lane & ((1u << SH) - 1)) == 0) gu[16 * wave + grp * RPG + r] = v;
        } else {
            const uint32_t it = lane % ITEMS;
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t row = 16 * wave + lane / ITEMS + k * (64 / ITEMS);
                const float4 sc = scl[4 * (row * NB + it / 8) + (it % 8) / 2];
                const float v = group_sum<ITEMS>(item_dot(q[k], sc, xs[0]));
                if (it == 0) gu[row] = v;
            }
        }
    }
    __syncthreads();

    if (tid < 8) {
        const uint32_t i0 = 4 * tid;
        float4 h;
        h.x = kq_silu_mul(gu[i0 + 0], gu[32 + i0 + 0]);
        h.y = kq_silu_mul(gu[i0 + 1], gu[32 + i0 + 1]);
        h.z = kq_silu_mul(gu[i0 + 2], gu[32 + i0 + 2]);
        h.w = kq_silu_mul(gu[i0 + 3], gu[32 + i0 + 3]);
        uint32_t d16, s16;
        int lo, hi;
        float dd;
        const uint32_t qv = quant_q8_1_part(h, d16, s16, lo, hi, dd);
        uint8_t *blk = a.hq8 + ((uint64_t)slot * nblk + jb) * 36;
        *(uint32_t *)(blk + 4 + 4 * tid) = qv;
        if (tid == 0) *(uint32_t *)blk = d16 | (s16 << 16);
    }
    if (a.dbg_gu && tid < 64) {
        float *d = a.dbg_gu + (uint64_t)slot * 2 * a.ffn + (tid < 32 ? 0 : a.ffn) + 32 * jb + (tid & 31);
        *d = gu[tid];
    }
    if (blockIdx.x == 0) route_publish(a, rt, (const float *)(lds + L.logits));
}

// ---------------------------------------------------------------------------
// Kernel B: a tile of TR output rows x n_slots down rows per workgroup; one
// lane-slot (S = QD::IPB lanes) per (row, slot) pair; every load issued before
// the h activations are staged.
// ---------------------------------------------------------------------------
struct LdsB {
    uint32_t route, hacts, res, total;
};
__host__ __device__ inline LdsB lds_b(uint32_t ffn, uint32_t n_slots, uint32_t tr) {
    LdsB L;
    L.route = 0;
    L.hacts = 256;
    L.res = L.hacts + n_slots * act_bytes(ffn);
    L.total = L.res + tr * n_slots * 4;
    return L;
}

// q8_1 h of every slot, staged from the scratch written by kernel A: 8 lanes
// per 36-byte block (one dword of values each, lane 0 also the scale), loads
// issued up front by load_h and finished by stage_h.
constexpr int HT_MAX = 12;   // lane tasks per thread (n_slots * ffn/32 * 8 / blockDim)
struct HLoad {
    uint32_t q[HT_MAX];
    uint32_t d[HT_MAX];
};
__device__ __forceinline__ void load_h(const uint8_t *hq8, uint32_t ntask, uint32_t first, HLoad &h) {
#pragma unroll
    for (int i = 0; i < HT_MAX; i++) {
        const uint32_t t = first + threadIdx.x + blockDim.x * i;
        if (t < ntask) {
            const uint8_t *b = hq8 + (t >> 3) * 36;
            h.q[i] = *(const uint32_t *)(b + 4 + 4 * (t & 7));
            h.d[i] = ld_u16(b);
        }
    }
}
__device__ __forceinline__ void stage_h(uint8_t *hl, uint32_t ffn, uint32_t ntask, uint32_t first, const HLoad &h) {
    const uint32_t nblk = ffn / 32, ab = act_bytes(ffn);
#pragma unroll
    for (int i = 0; i < HT_MAX; i++) {
        const uint32_t t = first + threadIdx.x + blockDim.x * i;
        if (t >= ntask) break;   // whole 8-lane groups leave together
        const uint32_t blk = t >> 3, part = t & 7, slot = blk / nblk, kb = blk % nblk;
        const Act act = act_carve(hl + slot * ab, ffn);
        *(uint32_t *)(act.qs + 32 * kb + 4 * part) = h.q[i];
        int s = dot4(h.q[i], 0x01010101u, 0);
        s += dpp_i<DPP_XOR1>(s);
        s += dpp_i<DPP_XOR2>(s);
        const int other = dpp_i<DPP_HALF_MIRROR>(s);
        if (part == 0) {
            act.d8[kb] = h2f(h.d[i]);
            act.qs16[2 * kb] = s;
            act.qs16[2 * kb + 1] = other;
        }
    }
}

template <class QD, int IPL>
__global__ void __launch_bounds__(256) k_moe_down(MoeArgs a, uint32_t tr, uint32_t n_slots) {
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsB L = lds_b(a.ffn, n_slots, tr);
    Route *rt = (Route *)(lds + L.route);
    const uint32_t tid = threadIdx.x;
    // h loads first (they do not depend on the routing), then the routing
    const uint32_t ntask = n_slots * (a.ffn / 32) * 8;
    HLoad hv;
    load_h(a.hq8, ntask, 0, hv);
    int32_t rid = 0;
    float rw = 0.0f;
    if (tid < MAX_SLOTS) {
        rid = a.route_ids[tid];
        rw = a.route_w[tid];
    }
    if (tid < MAX_SLOTS) {
        rt->ids[tid] = rid;
        rt->w[tid] = rw;
    }
    __syncthreads();
    const uint32_t S = QD::IPB;
    const uint32_t ls = tid / S, s = tid % S;
    const uint32_t row0 = blockIdx.x * tr;
    const uint32_t nrows = row0 + tr <= a.hidden ? tr : a.hidden - row0;
    const uint32_t npairs = nrows * n_slots;
    const uint64_t rbd = (uint64_t)(a.ffn / 256) * QD::BB;
    const uint32_t ipl = a.ffn / 256;
    typename QD::Raw raw[IPL > 0 ? IPL : 1];
    const bool active = ls < npairs;
    uint32_t sl = 0;
    const uint8_t *rp = nullptr;
    if (active) {
        const uint32_t r = ls / n_slots;
        sl = ls % n_slots;
        const uint8_t *db = (int)sl < a.n_sel ? a.down + (uint64_t)rt->ids[sl] * a.hidden * rbd : a.down_sh;
        rp = db + (uint64_t)(row0 + r) * rbd;
        if constexpr (IPL > 0) {
#pragma unroll
            for (int i = 0; i < IPL; i++) raw[i] = QD::load(rp + i * QD::BB, (int)s);
        }
    }
    stage_h(lds + L.hacts, a.ffn, ntask, 0, hv);
    for (uint32_t first = HT_MAX * blockDim.x; first < ntask; first += HT_MAX * blockDim.x) {
        load_h(a.hq8, ntask, first, hv);   // only for n_slots * ffn > 12288
        stage_h(lds + L.hacts, a.ffn, ntask, first, hv);
    }
    __syncthreads();
    float x = 0.0f;
    if (active) {
        const Act act = act_carve(lds + L.hacts + sl * act_bytes(a.ffn), a.ffn);
        if constexpr (IPL > 0) {
#pragma unroll
            for (int i = 0; i < IPL; i++) x += QD::dot_q8(raw[i], (int)s, act, i);
        } else {
            for (uint32_t i = 0; i < ipl; i++) x += QD::dot_q8(QD::load(rp + i * QD::BB, (int)s), (int)s, act, i);
        }
    }
    x = group_sum<QD::IPB>(x);
    float *res = (float *)(lds + L.res);
    if (active && s == 0) res[ls] = x;
    __syncthreads();
    for (uint32_t i = tid; i < nrows; i += blockDim.x) {
        float y = 0.0f;
        for (uint32_t k = 0; k < n_slots; k++) y = fmaf(rt->w[k], res[i * n_slots + k], y);
        a.y[row0 + i] = y;
    }
}

uint64_t moe_route_words() { return 2 * MAX_SLOTS; }

template <int NB>
static hipError_t go_a(const MoeArgs &a, uint32_t n_slots, hipStream_t s) {
    const LdsA L = lds_a(a.hidden, NB);
    hipLaunchKernelGGL(k_moe_gu<NB>, dim3(n_slots * (a.ffn / 32)), dim3(256), L.total, s, a);
    return hipGetLastError();
}

template <class QD, int IPL>
static hipError_t go_b(const MoeArgs &a, uint32_t n_slots, hipStream_t s) {
    const uint32_t lane_slots = 256 / QD::IPB;
    uint32_t tr = lane_slots / n_slots;
    if (tr < 1) tr = 1;
    const LdsB L = lds_b(a.ffn, n_slots, tr);
    hipLaunchKernelGGL((k_moe_down<QD, IPL>), dim3((a.hidden + tr - 1) / tr), dim3(256), L.total, s, a, tr, n_slots);
    return hipGetLastError();
}

bool moe_shape_supported(uint32_t gate_type, uint32_t down_type, uint32_t hidden, uint32_t ffn) {
    if (gate_type != T_Q4_K || (down_type != T_Q4_K && down_type != T_Q6_K)) return false;
    const uint32_t nb = hidden / 256;
    if (hidden % 256 || !(nb == 1 || nb == 2 || nb == 4 || nb == 8 || nb == 16)) return false;
    return ffn % 256 == 0 && ffn >= 256;
}

hipError_t launch_moe(const MoeArgs &a, hipStream_t s) {
    const uint32_t n_slots = (uint32_t)a.n_sel + (a.has_shared ? 1u : 0u);
    hipError_t e;
    switch (a.hidden / 256) {
        case 1: e = go_a<1>(a, n_slots, s); break;
        case 2: e = go_a<2>(a, n_slots, s); break;
        case 4: e = go_a<4>(a, n_slots, s); break;
        case 8: e = go_a<8>(a, n_slots, s); break;
        case 16: e = go_a<16>(a, n_slots, s); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    const uint32_t nbd = a.ffn / 256;
    if (a.down_type == T_Q6_K) {
        switch (nbd) {
            case 1: return go_b<Q6K, 1>(a, n_slots, s);
            case 2: return go_b<Q6K, 2>(a, n_slots, s);
            case 3: return go_b<Q6K, 3>(a, n_slots, s);
            case 4: return go_b<Q6K, 4>(a, n_slots, s);
            default: return go_b<Q6K, 0>(a, n_slots, s);
        }
    }
    switch (nbd) {
        case 1: return go_b<Q4K, 1>(a, n_slots, s);
        case 2: return go_b<Q4K, 2>(a, n_slots, s);
        case 3: return go_b<Q4K, 3>(a, n_slots, s);
        default: return go_b<Q4K, 0>(a, n_slots, s);
    }
}

}  // namespace kq
