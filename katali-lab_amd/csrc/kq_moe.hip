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
#include <type_traits>

#include "kq_device.h"
#include "kq_launch.h"

namespace kq {

constexpr int MAX_SEL = 16;
constexpr uint32_t B_MAX_THREADS = 512;   // kernel B's largest workgroup
constexpr int MAX_SLOTS = MAX_SEL + 1;
constexpr uint32_t MAX_EXPERT = 512;

// polls of the fused layer's wait before it gives up (each at least one
// device round trip: ~1 s in all); expiry sets error bit 4
constexpr uint32_t FSYNC_SPIN_LIMIT = 1u << 20;


__device__ __forceinline__ const float *route_logits(const MoeArgs &a) {
    const float *l = a.logits;
    if (a.step) l += (uint64_t)(*a.step) * a.logits_stride;
    return l;
}

// ---------------------------------------------------------------------------
// Routing, computed by every wave on its own (no LDS, no barrier).
//
// Keys: a logit maps to an unsigned key that orders like the float, with NaN
// ranked as -inf and -0 as +0; experts past n_expert get key 0 (below -inf).
// Lane l holds the keys of experts l, l + 64, ... (C chunks of 64 experts).
// Selection and ranking at once: n_sel rounds of a wave-wide max (wave_topk).
// Lane r < n_sel ends with the expert and the canonical logit of rank r.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t logit_key(float v) {
    if (v != v) v = -INFINITY;
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_logit(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

struct WaveRoute {
    int32_t id;     // lane r < n_sel: expert of rank r
    float logit;    // its logit (canonical: NaN -> -inf, -0 -> +0)
};

// Issue the logit loads of one wave (lane l: experts l, l + 64, ...). The
// address is clamped into the logits so the loads need no branch; keys of
// experts past n_expert are replaced later.
template <int C>
__device__ __forceinline__ void load_keys(const MoeArgs &a, float (&lv)[C]) {
    const uint32_t lane = threadIdx.x & 63;
    const float *src = route_logits(a);
#pragma unroll
    for (int i = 0; i < C; i++) lv[i] = src[min(lane + 64 * i, a.n_expert - 1)];
}

// max over the 64 lanes, every lane gets it (DPP inside 16-lane rows, then
// the two row swaps)
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<DPP_XOR1>((int)v));
    v = max(v, (uint32_t)dpp_i<DPP_XOR2>((int)v));
    v = max(v, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)v));
    v = max(v, (uint32_t)dpp_i<DPP_MIRROR>((int)v));
    const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max((uint32_t)r16[0], (uint32_t)r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max((uint32_t)r32[0], (uint32_t)r32[1]);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, (uint32_t)dpp_i<DPP_XOR1>((int)v));
    v = min(v, (uint32_t)dpp_i<DPP_XOR2>((int)v));
    v = min(v, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)v));
    v = min(v, (uint32_t)dpp_i<DPP_MIRROR>((int)v));
    const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = min((uint32_t)r16[0], (uint32_t)r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return min((uint32_t)r32[0], (uint32_t)r32[1]);
}
// A lane's C (key, expert) pairs sorted best first: larger key, then lower
// expert index (odd-even transposition, C rounds).
template <int C>
__device__ __forceinline__ void lane_sort(uint32_t (&key)[C], uint32_t (&eid)[C]) {
#pragma unroll
    for (int r = 0; r < C; r++) {
#pragma unroll
        for (int p = r & 1; p + 1 < C; p += 2) {
            const bool sw = key[p + 1] > key[p] || (key[p + 1] == key[p] && eid[p + 1] < eid[p]);
            const uint32_t k0 = key[p], e0 = eid[p];
            key[p] = sw ? key[p + 1] : k0;
            eid[p] = sw ? eid[p + 1] : e0;
            key[p + 1] = sw ? k0 : key[p + 1];
            eid[p + 1] = sw ? e0 : eid[p + 1];
        }
    }
}
// Top n_sel of the logits, every wave on its own (no LDS, no barrier): n_sel
// rounds of (largest remaining key over the wave; the lowest expert index
// holding it; that key retired). Round j's expert and logit land in lane j,
// so lanes 0..n_sel-1 hold the selection in rank order: larger logit first,
// lower index on ties, NaN as -inf, -0 as +0. Keys of valid experts are
// never 0 (the largest NaN-free order key of -inf is 0x007FFFFF), so the
// retired and the padding keys (0) are never chosen while n_sel <= n_expert.
// C <= 2 (up to 128 experts): each lane sorts its keys once (best first),
// and a round takes the max of the lanes' head keys; of the lanes whose
// head holds it the one with the lowest expert index wins (every key equal
// to the round's maximum that is its lane's lowest such index sits at that
// lane's head), and its next key moves up: one ballot per round instead of
// C (moe48 +1 %, moe48tok +1.2 %). C >= 4: a round takes the max over all C
// keys and finds the lowest index holding it with C ballots (the lane sort
// and the shifts measured 4 % slower there at 256 experts). (A 32-step
// binary search for the n_sel-th key plus a ranking pass took ~2.5x the
// instructions.)
// rounds (<= n_sel, wave-uniform): the ranks needed; rank r comes out of
// round r, so a caller that needs only ranks < rounds stops there
template <int C>
__device__ __forceinline__ WaveRoute wave_topk(const MoeArgs &a, const float (&lv)[C], int rounds) {
    const uint32_t lane = threadIdx.x & 63;
    const int k = rounds;
    uint32_t key[C], eid[C];
#pragma unroll
    for (int i = 0; i < C; i++) {
        eid[i] = lane + 64 * i;
        key[i] = eid[i] < a.n_expert ? logit_key(lv[i]) : 0u;
    }
    int32_t id = -1;
    uint32_t mk = 0;
    if constexpr (C >= 4) {
#pragma nounroll   // (a loop with a wave-uniform exit: stays a loop)
        for (int j = 0; j < MAX_SEL; j++) {
            if (j >= k) break;   // uniform
            uint32_t m = key[0];
#pragma unroll
            for (int i = 1; i < C; i++) m = max(m, key[i]);
            const uint32_t M = wave_max_u32(m);
            int e = 0;
#pragma unroll
            for (int i = C - 1; i >= 0; i--) {   // the lowest chunk holding M wins, then the lowest lane
                const uint64_t b = __ballot(key[i] == M);
                e = b ? 64 * i + (int)__builtin_ctzll(b) : e;
            }
#pragma unroll
            for (int i = 0; i < C; i++) key[i] = (int)(lane + 64 * i) == e ? 0u : key[i];
            id = (int)lane == j ? e : id;
            mk = (int)lane == j ? M : mk;
        }
        WaveRoute r;
        r.id = (int)lane < k ? id : -1;
        r.logit = (int)lane < k ? key_logit(mk) : 0.0f;
        return r;
    }
    lane_sort<C>(key, eid);
#pragma nounroll   // (a loop with a wave-uniform exit: stays a loop)
    for (int j = 0; j < MAX_SEL; j++) {
        if (j >= k) break;   // uniform
        const uint32_t M = wave_max_u32(key[0]);
        const uint64_t b = __ballot(key[0] == M);
        uint32_t wl = (uint32_t)__builtin_ctzll(b);
        if (__builtin_popcountll(b) > 1)   // (uniform) equal heads: the lowest expert index wins
            wl = (uint32_t)__builtin_amdgcn_readfirstlane((int)wave_min_u32(key[0] == M ? eid[0] : ~0u)) & 63u;
        const int e = __builtin_amdgcn_readlane((int)eid[0], (int)wl);
        const bool w = lane == wl;   // the winner's next key moves up
#pragma unroll
        for (int i = 0; i + 1 < C; i++) {
            key[i] = w ? key[i + 1] : key[i];
            eid[i] = w ? eid[i + 1] : eid[i];
        }
        key[C - 1] = w ? 0u : key[C - 1];
        id = (int)lane == j ? e : id;
        mk = (int)lane == j ? M : mk;
    }
    WaveRoute r;
    r.id = (int)lane < k ? id : -1;
    r.logit = (int)lane < k ? key_logit(mk) : 0.0f;
    return r;
}
template <int C>
__device__ __forceinline__ WaveRoute wave_topk(const MoeArgs &a, const float (&lv)[C]) {
    return wave_topk<C>(a, lv, a.n_sel);
}

// Routing weights w_r = exp(l_r - l_0) / sum_{j<n_sel} exp(l_j - l_0), the sum
// taken in rank order (lane r < n_sel holds rank r).
__device__ __forceinline__ float route_weight(float logit, int n_sel) {
    const float l0 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(logit)));
    const float ex = kq_expf(logit - l0);
    float sum = 0.0f;
    for (int r = 0; r < n_sel; r++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), r));
    return ex / sum;
}

// Wave 0 of workgroup 0 of kernel A: the routing scratch for kernel B, the
// optional routing outputs, and the error bit for ids outside the pool
// (those are clamped to expert 0 for addressing).
__device__ __forceinline__ void route_publish(const MoeArgs &a, int32_t id, float w) {
    const int lane = (int)(threadIdx.x & 63);
    const bool bad = lane < a.n_sel && (uint32_t)id >= a.n_expert;
    if (lane < MAX_SLOTS) {
        int32_t e = -1;
        float ww = 0.0f;
        if (lane < a.n_sel) {
            e = bad ? 0 : id;
            ww = w;
            if (a.ids_out) a.ids_out[lane] = id;
            if (a.wts_out) a.wts_out[lane] = w;
        } else if (lane == a.n_sel && a.has_shared) {
            ww = 1.0f;
        }
        a.route_ids[lane] = e;
        a.route_w[lane] = ww;
    }
    if (__ballot(bad) != 0 && lane == 0) atomicOr(a.err, 2);
}

// ---------------------------------------------------------------------------
// Kernel A: 64 Q4_K rows (32 gate + 32 up) per workgroup, NB blocks per row.
// Sixteen waves; wave w owns rows 4w..4w+3 (waves 0-7 gate, 8-15 up; eight
// waves of 8 rows for the row widths a1_rw() names) and runs on its
// own apart from the x staging barrier, until the gate/up exchange at the
// end. (Measured at config 1: four waves of 16 rows 10.0 us, eight of 8
// 8.7 us, sixteen of 4 8.2 us: with one workgroup per CU, more waves
// per SIMD hide each other's routing, decode and load latency, and each
// wave's serial work shrinks.)
// Lane l always takes the same lane item of every row it touches:
//   ITEMS = 8*NB >= 64: the k-th chunk is item 64*(k % M) + l of row k / M
//                       (M = ITEMS/64 items per lane);
//   ITEMS < 64:         64/ITEMS rows share a wave instruction; the k-th
//                       chunk is item l % ITEMS of row l / ITEMS + k*64/ITEMS.
// x is quantized to q8_1 once per workgroup into LDS (8 lanes per 32-value
// block) while the weights stream in; each lane then reads its items' q8
// values once. The wave's 8*NB block headers are decoded once into a
// wave-private LDS area as {d*sc[2g]*d8[k], d*sc[2g+1]*d8[k+1],
// dmin*m[2g]*d8[k], dmin*m[2g+1]*d8[k+1]} per group g, where k and k+1 are
// the q8_1 blocks of x that group meets (a wavefront-scope sync, not a
// barrier, orders them).
// ---------------------------------------------------------------------------
struct LdsA {
    uint32_t xact, scl, gu, total;
};
__host__ __device__ inline LdsA lds_a(uint32_t hidden, uint32_t nb, uint32_t rows = 64) {
    LdsA L;
    L.xact = 0;
    L.scl = L.xact + act_bytes(hidden);   // rows x nb headers x 4 groups x float4
    L.gu = L.scl + rows * nb * 64;
    L.total = L.gu + 64 * 4;
    return L;
}

// max / sum over aligned 32-lane halves (every lane gets its half's result)
__device__ __forceinline__ float max32(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ int sum32(int v) {
    v += dpp_i<DPP_XOR1>(v);
    v += dpp_i<DPP_XOR2>(v);
    v += dpp_i<DPP_HALF_MIRROR>(v);
    v += dpp_i<DPP_MIRROR>(v);
    const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    return (int)r[0] + (int)r[1];
}

// the activation side of one lane item (constant over rows)
struct XSlice {
    int4 xl, xh;
    float xsum;   // exact sum of the 32 int8 values of x's q8_1 block it (the lane's sub-block)
};
__device__ __forceinline__ XSlice x_slice(const Act &xa, uint32_t it) {
    const uint32_t b = it / 8, c = it % 8, g = c >> 1, hh = c & 1;
    const int8_t *al = xa.qs + 256 * b + 64 * g + 16 * hh;
    XSlice x;
    x.xl = *(const int4 *)al;
    x.xh = *(const int4 *)(al + 32);
    x.xsum = (float)(xa.qs16[2 * it] + xa.qs16[2 * it + 1]);
    return x;
}

// The q8_1 path's Q4_K row dot is the pairwise sum of one fp32 term per
// 32-value sub-block j:
//   t_j = fmaf(A_j, isum_j, -(B_j * xsum_j)),  A_j = (d*sc_j)*d8_j,  B_j = (dmin*m_j)*d8_j,
// isum_j the exact integer sum over the sub-block. Lane item it (16 nibble
// bytes: values 16hh..16hh+15 of sub-blocks 2g and 2g+1, hh = it & 1) forms
// half sums of both; lanes it and it ^ 1 (partners by DPP) swap the halves
// the other needs, after which lane it holds sub-block it's term (hh = 0:
// sub-block 2g, the low nibbles; hh = 1: 2g+1). The decoded header gives
// sc = {A_2g, A_2g+1, B_2g, B_2g+1}. The lane bit hh equals lane bit 0 in
// every item mapping here (items of a row sit on consecutive lanes).
__device__ __forceinline__ float q4k_term_from(int slo, int shi, const float4 &sc, float xsum) {
    const bool hh = threadIdx.x & 1;
    const int isum = (hh ? shi : slo) + dpp_i<DPP_XOR1>(hh ? slo : shi);
    const float A = hh ? sc.y : sc.x, B = hh ? sc.w : sc.z;
    return fmaf(A, (float)isum, -(B * xsum));
}
__device__ __forceinline__ float q4k_term(const uint4 &q, const float4 &sc, const XSlice &x) {
    int slo, shi;
    Q4K::isums_x(q, x.xl, x.xh, slo, shi);
    return q4k_term_from(slo, shi, sc, x.xsum);
}
// q4k_term with the nibbles unpacked beforehand (the same sums and float ops)
__device__ __forceinline__ float q4k_term_u(const Q4K::Unp &u, const float4 &sc, const XSlice &x) {
    int slo = dot4(u.lo.x, x.xl.x, 0);
    slo = dot4(u.lo.y, x.xl.y, slo);
    slo = dot4(u.lo.z, x.xl.z, slo);
    slo = dot4(u.lo.w, x.xl.w, slo);
    int shi = dot4(u.hi.x, x.xh.x, 0);
    shi = dot4(u.hi.y, x.xh.y, shi);
    shi = dot4(u.hi.z, x.xh.z, shi);
    shi = dot4(u.hi.w, x.xh.w, shi);
    return q4k_term_from(slo, shi, sc, x.xsum);
}

// Rows of sub-block terms summed pairwise over the lanes. Chunk k of a lane
// is its item 64*(k % M) + lane of row k / M (M items per lane per row), so
// the chunk index is the virtual row of pw_reduce: row sub-block j = 64m +
// lane. With M = 2 the lanes hold the two halves of the row (j < 64, j >= 64)
// as separate virtual rows, whose sums (partners at lane bit log2(V) - 1)
// make the tree's top level. Lanes 0 .. V/M - 1 end with whole rows:
// pw_rows_row(lane) of them.
template <int V, int M>
__device__ __forceinline__ float pw_rows(float (&acc)[V]) {
    float v = pw_reduce<V>(acc);
    if constexpr (M == 2) {
        if constexpr (V / 2 >= 16) v = swap_sum<V / 2>(v, v);
        else v += xor_lane<V / 2>(v);
    }
    return v;
}
template <int V, int M>
__device__ __forceinline__ uint32_t pw_rows_row(uint32_t lane) {
    return pw_row<V>(lane) / M;
}

constexpr int A_ROWS_PER_WAVE = 8;
constexpr int A_THREADS = 64 * 64 / A_ROWS_PER_WAVE;
// kernel A (single token): rows per wave. 16 waves of 4 rows; 8 rows when a
// row has fewer than 16 lane items, and for 4096-wide rows (a dense FFN's
// 384 workgroups fill the CUs already: 16.8 us with 8 rows per wave against
// 18.0 us with 4 at the Qwen3-8B shape)
template <int NB>
constexpr int a1_rw() { return NB >= 2 && NB <= 8 ? 4 : 8; }
template <int NB>
constexpr int a1_threads() { return 64 * 64 / a1_rw<NB>(); }

// The routing of one wave: lane r < n_sel ends with the expert of rank r
// (rt.eid) and, when logits route, its canonical logit (rt.logit); with an
// explicit selection, its weight (rt.w). Issue and finish are split so the
// caller can put other loads between them.
struct GuRoute {
    int32_t eid;
    float logit;
    float w;
};
template <int C>
__device__ __forceinline__ void route_issue(const MoeArgs &a, float (&lv)[C], GuRoute &rt) {
    const uint32_t lane = threadIdx.x & 63;
    rt.eid = -1;
    rt.logit = 0.0f;
    rt.w = 0.0f;
    if (a.n_sel > 0) {
        if (a.logits) {
            load_keys<C>(a, lv);
        } else {
            const uint32_t r = min(lane, (uint32_t)a.n_sel - 1);
            rt.eid = a.ids[r];
            rt.w = a.wts[r];
        }
    }
}
// rounds: the ranks this wave needs (<= n_sel; -1: all of them)
template <int C>
__device__ __forceinline__ void route_finish(const MoeArgs &a, const float (&lv)[C], GuRoute &rt, int rounds = -1) {
    if (a.logits && a.n_sel > 0) {
        const WaveRoute r = wave_topk<C>(a, lv, rounds < 0 ? a.n_sel : min(rounds, a.n_sel));
        rt.eid = r.id;
        rt.logit = r.logit;
    }
}

// lanes of this wave below this one whose bit is set in b
__device__ __forceinline__ uint32_t lanes_below(uint64_t b) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
}

// Routing of more than 128 experts (C >= 4) by wave 0 from a candidate set,
// handed to every wave behind one barrier. The experts fall into eight
// disjoint groups (expert index mod 8: each holds valid experts once
// n_expert >= 8); at least eight keys lie at or above T, the least of the
// eight group maxima, so whenever the keys >= T (the candidates) number at
// least n_sel, every expert left out ranks below all of them and the top
// n_sel are candidates. The candidates go to LDS in ascending expert order
// as 64-bit words (key << 32 | ~expert): unique, and ordered as wave_topk
// orders (larger key, then the lower expert index), so the words above a
// candidate's own count its rank, ties included. Random logits leave about
// 20 candidates of 256 (the all-pairs count compares 256 x 256 keys). With
// more than 64 candidates (heavy ties, or T = 0 below eight experts) or
// fewer than n_sel, wave 0 ranks with wave_topk instead. lane r <
// n_sel of every wave ends with rank r's expert and canonical logit. scr:
// 160 words of LDS that nothing else uses until every wave has returned.
template <int C>
__device__ __forceinline__ void wave0_route(const MoeArgs &a, const float (&lv)[C], uint32_t *scr, GuRoute &rt) {
    uint64_t *cw = (uint64_t *)scr;                  // 64 candidate words
    uint32_t *sel = scr + 128, *sell = sel + 16;     // rank r: expert, logit bits
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) {
        uint32_t key[C];
#pragma unroll
        for (int i = 0; i < C; i++) {
            const uint32_t e = lane + 64 * i;
            key[i] = e < a.n_expert ? logit_key(lv[i]) : 0u;
        }
        uint32_t g = key[0];
#pragma unroll
        for (int i = 1; i < C; i++) g = max(g, key[i]);
        g = max(g, (uint32_t)dpp_i<DPP_ROR8>((int)g));   // lanes l and l ^ 8 of a row
        const auto r16 = __builtin_amdgcn_permlane16_swap(g, g, false, false);
        g = max((uint32_t)r16[0], (uint32_t)r16[1]);
        const auto r32 = __builtin_amdgcn_permlane32_swap(g, g, false, false);
        g = max((uint32_t)r32[0], (uint32_t)r32[1]);      // lane l: the maximum of group l % 8
        g = min(g, (uint32_t)dpp_i<DPP_XOR1>((int)g));
        g = min(g, (uint32_t)dpp_i<DPP_XOR2>((int)g));
        g = min(g, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)g));
        const uint32_t T = (uint32_t)__builtin_amdgcn_readfirstlane((int)g);
        uint64_t bal[C];
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < C; i++) {
            bal[i] = __ballot(key[i] >= T);
            m += (uint32_t)__builtin_popcountll(bal[i]);
        }
        if (m >= (uint32_t)a.n_sel && m <= 64) {   // (uniform)
            uint32_t base = 0;
#pragma unroll
            for (int i = 0; i < C; i++) {
                if (key[i] >= T)
                    cw[base + lanes_below(bal[i])] = ((uint64_t)key[i] << 32) | (uint32_t)~(lane + 64 * i);
                base += (uint32_t)__builtin_popcountll(bal[i]);
            }
            if (lane >= m) cw[lane] = 0;   // below every candidate word (keys of candidates are > 0)
            wave_sync_lds();
            const uint64_t own = cw[lane];
            const uint4 *q = (const uint4 *)cw;
            uint32_t r = 0;
            // 16 words per batch of loads (about 20 candidates at random; the
            // words past m are 0 and count nothing)
#pragma nounroll
            for (uint32_t b = 0; b < (m + 15) / 16; b++) {   // (uniform)
#pragma unroll
                for (uint32_t j = 0; j < 8; j++) {
                    const uint4 v = q[8 * b + j];
                    r += (((uint64_t)v.y << 32) | v.x) > own ? 1u : 0u;
                    r += (((uint64_t)v.w << 32) | v.z) > own ? 1u : 0u;
                }
            }
            if (lane < m && r < (uint32_t)a.n_sel) {
                sel[r] = ~(uint32_t)own;
                sell[r] = __float_as_uint(key_logit((uint32_t)(own >> 32)));
            }
        } else {
            float kv[C];   // (from the keys: lv is dead by now)
#pragma unroll
            for (int i = 0; i < C; i++) kv[i] = key_logit(key[i]);
            const WaveRoute w = wave_topk<C>(a, kv, a.n_sel);
            if ((int)lane < a.n_sel) {
                sel[lane] = (uint32_t)w.id;
                sell[lane] = __float_as_uint(w.logit);
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    const bool ranked = (int)lane < a.n_sel;
    const uint32_t r = min(lane, 15u);
    rt.eid = ranked ? (int32_t)sel[r] : -1;
    rt.logit = ranked ? __uint_as_float(sell[r]) : 0.0f;
}

// Routing by the whole workgroup (>= 512 threads, n_expert <= 64 C), where
// wave_topk takes n_sel dependent rounds per wave (~1.1 us at top-8 of 128).
// The rank of expert e is the number of experts whose key is above e's:
//   1. wave 0 stores the 64 C keys (logit_key; 0 past n_expert) in LDS;
//   2. thread t < 512 counts, for its experts g + 64 i (g = t / 8, i < C),
//      the keys above theirs among the 8 C keys of chunk t % 8 (broadcast
//      reads); the 8 lanes of g sum their counts (DPP);
//   3. each valid expert whose count r is below n_sel stores its index and
//      key at slot r and adds 1 to hit[r].
// Equal keys get equal counts, so if two experts share a count below n_sel
// some hit[r] is not 1: then each wave ranks the keys from LDS with
// wave_topk, whose order (the lower expert index first among equal keys)
// decides. Without such a tie the counts are the ranks wave_topk gives and
// the selection is its selection, bit for bit. lane r < n_sel of every wave
// ends with rank r's expert and canonical logit, as after route_finish.
// Every wave of the workgroup calls it (two barriers); lv: wave 0's logits
// (load_keys). scr: 64 C + 48 words of LDS that nothing else uses until every
// wave has returned. CAND (the default for more than 128 experts, C >= 4):
// wave0_route, whose candidate set needs ~1/100 of the compares.
template <int C, bool CAND = (C >= 4)>
__device__ __forceinline__ void block_route(const MoeArgs &a, const float (&lv)[C], uint32_t *scr, GuRoute &rt) {
    if constexpr (CAND) {
        wave0_route<C>(a, lv, scr, rt);
        return;
    }
    constexpr uint32_t K = 64 * C, CK = K / 8;   // keys, keys per chunk
    uint32_t *keys = scr, *hit = scr + K, *sel = hit + 16, *selk = sel + 16;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < C; i++) {
            const uint32_t e = lane + 64 * i;
            keys[e] = e < a.n_expert ? logit_key(lv[i]) : 0u;
        }
        if (lane < 16) hit[lane] = 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (tid < 512) {   // whole waves
        const uint32_t g = tid >> 3, c = tid & 7;
        uint32_t own[C], cnt[C];
#pragma unroll
        for (int i = 0; i < C; i++) {
            own[i] = keys[g + 64 * i];
            cnt[i] = 0;
        }
        const uint4 *ck = (const uint4 *)(keys + CK * c);
#pragma unroll
        for (uint32_t q = 0; q < CK / 4; q++) {
            const uint4 v = ck[q];
            const uint32_t kv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int i = 0; i < C; i++) cnt[i] += kv[j] > own[i] ? 1u : 0u;
        }
#pragma unroll
        for (int i = 0; i < C; i++) {
            int r = (int)cnt[i];
            r += dpp_i<DPP_XOR1>(r);
            r += dpp_i<DPP_XOR2>(r);
            r += dpp_i<DPP_HALF_MIRROR>(r);
            const uint32_t e = g + 64 * i;
            if (c == 0 && e < a.n_expert && r < a.n_sel) {
                atomicAdd(&hit[r], 1u);
                sel[r] = e;
                selk[r] = own[i];
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    const bool ranked = (int)lane < a.n_sel;
    const uint32_t r = min(lane, 15u);
    if (__any(ranked && hit[r] != 1u)) {   // (uniform: the same LDS for every wave)
        float kv[C];
#pragma unroll
        for (int i = 0; i < C; i++) kv[i] = key_logit(keys[lane + 64 * i]);
        const WaveRoute w = wave_topk<C>(a, kv);
        rt.eid = w.id;
        rt.logit = w.logit;
    } else {
        rt.eid = ranked ? (int32_t)sel[r] : -1;
        rt.logit = ranked ? key_logit(selk[r]) : 0.0f;
    }
}

// ---------------------------------------------------------------------------
// The normed layer's prologue (kernel A of launch_moe_normed): the steps
// before the layer, formed by every workgroup of kernel A itself.
//   Residual step and RMSNorm as k_norm_router forms them: threads 0..255
//   take float4 q = t + 256 k (k < KN), each its double sum of squares in
//   that order, the wave sums, then waves 0..3 in order; inv = 1 / sqrtf(
//   (float)(sumsq / H) + eps), xn = v * inv * w; workgroup 0 writes xn and
//   the new residual.
//   Router rows w + U v on wave v < R (U workgroups): the engine's AVX2 F32
//   dot, accumulator j's FMA chain over columns j, j + 16, ... on lane j < 16,
//   then its horizontal sum (bit-identical to k_norm_router's rows), each
//   published as one 8-byte device-coherent word {logit, generation + 1} in
//   FSYNC_REP copies (lane k < 16 writes copy k). XL (the XCD layer up to
//   128 experts): each XCD group (workgroups w with one w % 8) forms every
//   row itself, rows w / 8 + 32 v, and publishes them in its own area
//   through the XCD's L2 (written through where the dispatch check failed,
//   a.hloc 0), so no logit has to cross an XCD.
//   The rows land in LDS after the sum of squares (which then waits for x
//   and delta alone); rows and xn sit there transposed by accumulator
//   (column c at [c % 16][c / 16], row stride H / 16 + 4 floats: 16-byte
//   chain reads, no bank conflicts).
//   Wave 0 then waits for every row's word (one round of loads in flight),
//   and the workgroup ranks those logits with block_route (up to 256
//   experts; more: wave 0 ranks them and hands the routing to the other
//   waves in LDS).
// LDS at `area`: xn and NORMED_MAX_R rows (16 (H/16 + 4) floats each),
// 4 doubles, the routing (16 ids, 16 logits), block_route's keys and slots.
// Returns this thread's xn float4s for the q8_1 staging. (An earlier
// whole-workgroup ranking, every thread reading every key, measured slower
// than wave 0's wave_topk: 1.65 us against 1.2 us, bound by the LDS reads of
// 1024 threads; block_route's threads read one eighth of the keys each.)
// ---------------------------------------------------------------------------
constexpr uint32_t NORMED_MAX_R = 4;
// (+ the block routing's keys and slots: at most 256 + 48 words)
__host__ __device__ constexpr uint32_t normed_area_bytes(uint32_t H) {
    return 4 * (H + 64) * (1 + NORMED_MAX_R) + 32 + 128 + 4 * (256 + 48);
}

// A value the compiler must take as new at this point. The stacked layer
// loops over its layers; indexes derived from the thread and workgroup ids
// would otherwise be hoisted out of that loop and held in registers across
// the whole layer (measured: 128 VGPRs and spills against 68 without the
// loop), so its layer body takes its ids through these.
__device__ __forceinline__ uint32_t opaque_v(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ uint32_t opaque_s(uint32_t v) {
    asm volatile("" : "+s"(v));
    return v;
}

// Phase stamps of the one-launch layers, in the measurement build only
// (KQ_STAMPS; build.py --stamps, libkatali_hip_stamps.so): s_memrealtime
// (100 MHz) at fixed points of a layer, kept in registers and stored at the
// layer's end to kq_stamps[tag % 64][workgroup][phase]. Phases: 0 layer
// start, 1 routing and x in, 2 gate/up loads issued, 3 x staged, 4 wave 0's
// dots done, 5 down loads issued, 6 h published, 7 first h poll issued, 8 h
// seen, 9 h staged, 10 partials published, 11 partials seen, 12 y written,
// 13 y poll started (stack) or the sum of squares done (normed, single
// layer), 14 y seen (stack) or xn staged (normed, single layer), 15 logits
// seen (normed).
// Wave 0 records every phase but 7 and 8, the first polling wave those.
// In the product build the marks compile to nothing.
[[maybe_unused]] constexpr uint32_t STAMP_LAYERS = 64, STAMP_PHASES = 16;
#ifdef KQ_STAMPS
__device__ uint64_t kq_stamps[STAMP_LAYERS * 256 * STAMP_PHASES];
struct Stamps {
    uint64_t t[STAMP_PHASES];
    __device__ __forceinline__ void mark(int i) { t[i] = __builtin_amdgcn_s_memrealtime(); }
    __device__ __forceinline__ void begin() {   // phases a layer does not pass stay 0
#pragma unroll
        for (int i = 0; i < (int)STAMP_PHASES; i++) t[i] = 0;
        mark(0);
    }
    __device__ __forceinline__ void store(uint32_t tag, uint32_t wg, uint32_t tid, uint32_t poller0) {
        uint64_t *o = kq_stamps + ((uint64_t)(tag % STAMP_LAYERS) * 256 + wg) * STAMP_PHASES;
        if (tid == 0) {
#pragma unroll
            for (int i = 0; i < (int)STAMP_PHASES; i++)
                if (i != 7 && i != 8) o[i] = t[i];
        } else if (tid == poller0) {
            o[7] = t[7];
            o[8] = t[8];
        }
    }
};
#else
struct Stamps {
    __device__ __forceinline__ void mark(int) {}
    __device__ __forceinline__ void begin() {}
    __device__ __forceinline__ void store(uint32_t, uint32_t, uint32_t, uint32_t) {}
};
#endif

// A layer of the stacked layer (k_moe_stack): its index l in the stack, the
// previous layer's y as tagged words (yw, tag ytag; used when l > 0) and its
// workgroups' completion words (yf: each workgroup's word takes the tag once
// that workgroup's part of y is stored), and,
// for the normed stack, the residual stream entering the layer (threads <
// 256, k_norm_router's float4 q = t + 256 k), kept in registers from layer
// to layer.
struct StkCtx {
    uint32_t l;
    uint32_t ytag;
    uint32_t *yw;
    uint32_t *yf;   // the previous layer's completion words
    float4 res[2];
    Stamps st;   // (the measurement build's phase stamps)
};

// In the stack, a wait that expired in one layer would make later layers'
// waits expire one after another (each about a second): every 1024 polls a
// stack's waits also read the error word and give up once an expiry is
// recorded there (the outputs are void then anyway).
__device__ __forceinline__ bool stack_expired(const MoeArgs &a, uint32_t spins) {
    return (spins & 1023u) == 0 && (ld_dev((uint32_t *)a.err) & 12u) != 0;
}

// Wait until every workgroup of the previous layer has stored its y: thread
// t < XCD_G reads workgroup t's completion word (a few bytes per workgroup,
// where the y itself is 8 KiB: every workgroup sees the whole y complete
// about one round trip after the last store). Two rounds in flight; whole
// waves up to XCD_G call it. `between` runs once, after the first round.
template <class Between>
__device__ __forceinline__ void poll_done(const MoeArgs &a, StkCtx &ctx, Between between) {
    uint32_t *f = ctx.yf + min((uint32_t)threadIdx.x, XCD_G - 1);
    uint32_t va, vb;
    ctx.st.mark(13);
    va = ld_dev(f);
    between();
    uint32_t spins = 0;
    for (;;) {
        vb = ld_dev(f);
        if (__all(va == ctx.ytag)) break;
        va = ld_dev(f);
        if (__all(vb == ctx.ytag)) break;
        if (++spins >= FSYNC_SPIN_LIMIT / 2 || stack_expired(a, spins)) {
            if ((threadIdx.x & 63) == 0) atomicOr(a.err, 4);
            break;
        }
    }
    asm volatile("" ::"v"(va), "v"(vb));   // the round still in flight keeps its registers
    ctx.st.mark(14);
}

// Read the previous layer's y words [4 q, 4 q + 4) of every q in qs
// (tag ytag) and return them, once poll_done has seen every workgroup's y
// stored (the words carry their tag, so a word not yet visible here is read
// again). Whole waves call it; lanes with `own` false load word 0 and drop
// it.
template <int K>
__device__ __forceinline__ void read_y(const MoeArgs &a, StkCtx &ctx, const uint32_t (&qs)[K], bool own,
                                       float4 (&out)[K]) {
    uint64_t wa[K][4];
    auto issue = [&](uint64_t (&w)[K][4]) {
#pragma unroll
        for (int k = 0; k < K; k++)
#pragma unroll
            for (int j = 0; j < 4; j++) w[k][j] = ld_dev2(ctx.yw + (own ? 2 * (4 * qs[k] + j) : 0));
    };
    auto seen = [&](const uint64_t (&w)[K][4]) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < K; k++)
#pragma unroll
            for (int j = 0; j < 4; j++) ok &= (uint32_t)(w[k][j] >> 32) == ctx.ytag;
        return __all(ok || !own);
    };
    auto take = [&](const uint64_t (&w)[K][4]) {
#pragma unroll
        for (int k = 0; k < K; k++)
            out[k] = make_float4(__uint_as_float((uint32_t)w[k][0]), __uint_as_float((uint32_t)w[k][1]),
                                 __uint_as_float((uint32_t)w[k][2]), __uint_as_float((uint32_t)w[k][3]));
    };
    issue(wa);
    uint32_t spins = 0;
    while (!seen(wa)) {
        if (++spins >= FSYNC_SPIN_LIMIT || stack_expired(a, spins)) {
            if ((threadIdx.x & 63) == 0) atomicOr(a.err, 4);
            break;
        }
        issue(wa);
    }
    take(wa);
}

// gen: this call's exchange generation (its load issued by the caller
// before anything else); xr: the logits words, FSYNC_REP copies of 512.
// STK (the normed stack, H <= 2048): from its second layer on the residual
// stream comes from registers (ctx.res) and the residual step's delta is
// the previous layer's y, polled from its tagged words; the new residual
// goes back to ctx.res. The steps are otherwise the same, so every output is
// the single normed layer's.
template <int NB, int C, int NT, int XPT, bool STK = false, bool XL = false>
__device__ __forceinline__ void normed_prologue(const MoeArgs &a, uint8_t *area, uint32_t U, GuRoute &rt,
                                                float4 (&xv)[XPT], uint32_t gen, uint32_t *xr, StkCtx &ctx) {
    constexpr uint32_t H = 256 * NB;
    constexpr uint32_t KN = H <= 2048 ? 2 : 4;   // k_norm_router's float4 per thread
    static_assert(!STK || KN == 2, "normed stack: hidden <= 2048");
    constexpr uint32_t Q4 = H / 4;
    constexpr uint32_t M = H / 16, TS = M + 4;   // chain length, transposed row stride
    constexpr uint32_t VT = 16 * TS;             // floats of one transposed vector
    constexpr uint32_t RF = NORMED_MAX_R * Q4;   // router float4s of a full workgroup share
    constexpr uint32_t RPT = (RF + NT - 1) / NT;
    const uint32_t tid = STK ? opaque_v(threadIdx.x) : threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t w = STK ? opaque_s(blockIdx.x) : blockIdx.x;
    float *xnT = (float *)area;
    float *rowsT = xnT + VT;
    double *part = (double *)(rowsT + NORMED_MAX_R * VT);
    int32_t *rte = (int32_t *)(part + 4);
    float *rtl = (float *)(rte + 16);
    auto at = [](uint32_t c) { return (c & 15) * TS + (c >> 4); };
    // XL (the XCD layer, n_expert <= 128): every XCD forms all the logits,
    // workgroup w the rows w / 8 + 32 v of XCD group w % 8, exchanged in
    // that group's area (through the XCD's L2 when the dispatch check holds,
    // a.hloc); otherwise workgroup w forms rows w + U v for every workgroup
    // (FSYNC_REP copies).
    const uint32_t rw = XL ? w / XCD_SLOTS : w, ru = XL ? XCD_G / XCD_SLOTS : U;
    const uint32_t R = (a.n_expert + ru - 1) / ru;   // the host keeps R <= NORMED_MAX_R

    // 1. every load: x, delta and the norm weights (threads < 256, whole
    //    waves), the router rows (all threads; clamped)
    float4 vx[KN], vd[KN], vn[KN];
    const bool from_regs = STK && ctx.l > 0;   // the stack past its first layer
    if (tid < 256) {
#pragma unroll
        for (uint32_t k = 0; k < KN; k++) {
            const uint32_t q = min(tid + k * 256, Q4 - 1);
            if (!from_regs) {
                vx[k] = *(const float4 *)&a.nx[4 * q];
                vd[k] = a.ndelta ? *(const float4 *)&a.ndelta[4 * q] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
            vn[k] = *(const float4 *)&a.nw[4 * q];
        }
    }
    float4 rv[RPT];
#pragma unroll
    for (uint32_t i = 0; i < RPT; i++) {
        const uint32_t f = min(tid + NT * i, RF - 1), v = f / Q4, q = f % Q4;
        const uint32_t r = min(rw + ru * v, a.n_expert - 1);
        rv[i] = *(const float4 *)&a.router[(uint64_t)r * H + 4 * q];
    }
    if constexpr (STK) {
        if (from_regs) {
            // the delta is the previous layer's y (its tagged words), the
            // residual the registers; then a barrier: every wave is past its
            // last LDS read of the previous layer before the rows land there
            if (tid < 256) {   // (XCD_G: one completion word per thread)
                uint32_t qs[KN];
#pragma unroll
                for (uint32_t k = 0; k < KN; k++) {
                    qs[k] = min(tid + k * 256, Q4 - 1);
                    vx[k] = ctx.res[k];
                }
                poll_done(a, ctx, [] {});
                read_y<KN>(a, ctx, qs, true, vd);
            }
        }
        __syncthreads();
    }
    // 2. residual step and the sum of squares
    if (tid < 256) {
        double sq = 0.0;
        const bool unit = from_regs || a.nscale == 1.0f;
#pragma unroll
        for (uint32_t k = 0; k < KN; k++) {
            if (from_regs || a.ndelta) {
                if (unit) {
                    vx[k].x = vx[k].x + vd[k].x; vx[k].y = vx[k].y + vd[k].y;
                    vx[k].z = vx[k].z + vd[k].z; vx[k].w = vx[k].w + vd[k].w;
                } else {
                    vx[k].x = vx[k].x + a.nscale * vd[k].x; vx[k].y = vx[k].y + a.nscale * vd[k].y;
                    vx[k].z = vx[k].z + a.nscale * vd[k].z; vx[k].w = vx[k].w + a.nscale * vd[k].w;
                }
            }
            const bool own = tid + k * 256 < Q4;
            sq += own ? (double)vx[k].x * (double)vx[k].x : 0.0;
            sq += own ? (double)vx[k].y * (double)vx[k].y : 0.0;
            sq += own ? (double)vx[k].z * (double)vx[k].z : 0.0;
            sq += own ? (double)vx[k].w * (double)vx[k].w : 0.0;
        }
        if constexpr (STK) {
#pragma unroll
            for (uint32_t k = 0; k < KN; k++) ctx.res[k] = vx[k];   // the residual entering the next layer's step
        }
        sq = wave_sum_f64(sq);
        if (lane == 0) part[wave] = sq;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if constexpr (!STK) ctx.st.mark(13);
    // all NORMED_MAX_R row slots, transposed (those past R hold a copy of the
    // last row; a clamped thread writes what its twin writes), only now: the
    // sum of squares above waits for x and delta alone, not for the rows
#pragma unroll
    for (uint32_t i = 0; i < RPT; i++) {
        const uint32_t f = min(tid + NT * i, RF - 1), c = 4 * (f % Q4);
        float *rt_ = rowsT + (f / Q4) * VT;
        rt_[at(c)] = rv[i].x;
        rt_[at(c + 1)] = rv[i].y;
        rt_[at(c + 2)] = rv[i].z;
        rt_[at(c + 3)] = rv[i].w;
    }
    // 3. xn into LDS, transposed (and from workgroup 0 to memory, with the
    //    new residual)
    if (tid < 256) {
        double sumsq = part[0];
#pragma unroll
        for (uint32_t k = 1; k < 4; k++) sumsq += part[k];
        const float inv = 1.0f / sqrtf((float)(sumsq / (double)H) + a.neps);
#pragma unroll
        for (uint32_t k = 0; k < KN; k++) {
            const uint32_t q = min(tid + k * 256, Q4 - 1), c = 4 * q;
            float4 o;
            o.x = vx[k].x * inv * vn[k].x; o.y = vx[k].y * inv * vn[k].y;
            o.z = vx[k].z * inv * vn[k].z; o.w = vx[k].w * inv * vn[k].w;
            xnT[at(c)] = o.x;
            xnT[at(c + 1)] = o.y;
            xnT[at(c + 2)] = o.z;
            xnT[at(c + 3)] = o.w;
            if (w == 0) {
                if (a.nxn_out) *(float4 *)&a.nxn_out[c] = o;
                if (STK ? a.nx_out != nullptr : a.ndelta != nullptr) *(float4 *)&a.nx_out[c] = vx[k];
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if constexpr (!STK) ctx.st.mark(14);
    // 4. this workgroup's router rows: wave v, lanes 0..15
    uint32_t tag = gen;
    asm volatile("" : "+v"(tag));
    tag += 1;
    const uint32_t r = rw + ru * wave;
    if (wave < R && r < a.n_expert && lane < 16) {
        const float *pw = rowsT + wave * VT + lane * TS, *px = xnT + lane * TS;
        float acc = 0.0f;
#pragma unroll 8
        for (uint32_t i = 0; i < M; i += 4) {
            const float4 wv = *(const float4 *)&pw[i], xq = *(const float4 *)&px[i];
            acc = fmaf(wv.x, xq.x, acc);
            acc = fmaf(wv.y, xq.y, acc);
            acc = fmaf(wv.z, xq.z, acc);
            acc = fmaf(wv.w, xq.w, acc);
        }
        // + 0.0f: a zero sum's sign as k_norm_router leaves it
        const float logit = hsum16_avx2_order(acc) + 0.0f;   // every lane of the row holds it
        const uint64_t word = ((uint64_t)tag << 32) | __float_as_uint(logit);
        if constexpr (XL) {
            if (lane == 0) {
                if (w % XCD_SLOTS == 0 && a.logits_out) a.logits_out[r] = logit;
                uint32_t *o = xr + 2 * (512 * (w % XCD_SLOTS) + r);
                if (a.hloc) st_xcd2(o, word);
                else st_dev2(o, word);
            }
        } else {
            if (lane == 0 && a.logits_out) a.logits_out[r] = logit;
            st_dev2(xr + 2 * (512 * lane + r), word);
        }
    }
    // 5. wave 0: every row's word (from this workgroup's copy); the routing
    //    from those logits by the whole workgroup (block_route, up to 256
    //    experts), else by wave 0 into LDS for the other waves
    float lv[C];
#pragma unroll
    for (int i = 0; i < C; i++) lv[i] = 0.0f;
    if (wave == 0) {
        const uint32_t *rep = xr + 2 * 512 * (XL ? w % XCD_SLOTS : w % FSYNC_REP);
        uint64_t va[C];
        auto issue = [&](uint64_t *o) {
#pragma unroll
            for (int i = 0; i < C; i++) o[i] = ld_dev2((uint32_t *)rep + 2 * min(lane + 64 * i, a.n_expert - 1));
        };
        auto seen = [&](const uint64_t *o) {
            bool ok = true;
#pragma unroll
            for (int i = 0; i < C; i++) ok &= (uint32_t)(o[i] >> 32) == tag;
            return __all(ok);
        };
        auto take = [&](const uint64_t *o) {
#pragma unroll
            for (int i = 0; i < C; i++) lv[i] = __uint_as_float((uint32_t)o[i]);
        };
        // One round at a time: the layer drains every load before its weight
        // stream starts, so a second round still in flight once the logits
        // are complete would hold this wave's weight loads back one round
        // trip.
        uint32_t spins = 0;
        for (;;) {
            issue(va);
            if (seen(va)) {
                take(va);
                break;
            }
            if (++spins >= FSYNC_SPIN_LIMIT || (STK && stack_expired(a, spins))) {
                if (lane == 0) atomicOr(a.err, 4);
                take(va);
                break;
            }
        }
        ctx.st.mark(15);
        if constexpr (C > 4) {
            const WaveRoute wr = wave_topk<C>(a, lv);
            if (lane < 16) {
                rte[lane] = wr.id;
                rtl[lane] = wr.logit;
            }
        }
    }
    // 6. every wave's routing (lane r < n_sel: rank r); 7. xn for the staging
    if constexpr (C <= 4) {
        // (the stacked layer keeps the all-pairs count: its registers are at the limit)
        block_route<C, C >= 4 && !STK>(a, lv, (uint32_t *)(rtl + 16), rt);
    } else {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        const bool ranked = lane < 16 && (int)lane < a.n_sel;
        rt.eid = ranked ? rte[min(lane, 15u)] : -1;
        rt.logit = ranked ? rtl[min(lane, 15u)] : 0.0f;
    }
    rt.w = 0.0f;
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const uint32_t c = 4 * min(tid + NT * i, (uint32_t)(64 * NB) - 1);
        xv[i] = make_float4(xnT[at(c)], xnT[at(c + 1)], xnT[at(c + 2)], xnT[at(c + 3)]);
    }
}

// One gate/up unit (32 gate + 32 up rows of one slot, one q8_1 block of h)
// for the workgroup: kernel A's whole body, and the first phase of the fused
// layer (FUSED: h also goes out as generation-tagged device-coherent words,
// then every wave runs `after`, the down tile's loads).
struct NoMore {
    __device__ void operator()(const GuRoute &) const {}
};
// HALF (a dense FFN, when 32-row units would leave CUs with uneven counts
// of workgroups): the workgroup takes half of a unit, 16 gate + 16 up rows,
// 16 values of the q8_1 block of h. Workgroups b and b + 8 of each run of
// 16 (one XCD) take the two halves of one block. Each publishes its 16
// values as tagged words; one atomic per block (a counter that every call
// raises by 2 and nothing resets: its parity tells first from second, its
// half the call) elects the second to arrive, which reads the other half and
// writes the block with kernel A's quantizer (the same values, so the same
// bits). Nobody waits for a workgroup that has not started.
template <int NB, int C, bool FUSED, class After = NoMore, bool NORMED = false, bool HALF = false>
__device__ __forceinline__ void gu_unit(const MoeArgs &a, uint32_t unit, uint8_t *lds, GuRoute &rt, uint32_t flag,
                                        uint32_t *hx = nullptr, After after = After()) {
    // FUSED: flag is this call's generation; h's words are tagged flag + 1
    // and go to hx + 2 * (9 * unit + k), k < 9.
    static_assert(!(HALF && (FUSED || NORMED)), "half units: the plain dense FFN");
    constexpr int RW = HALF ? a1_rw<NB>() / 2 : a1_rw<NB>();
    constexpr int HR = HALF ? 16 : 32;         // gate (and up) rows of the workgroup
    constexpr int NT = a1_threads<NB>();
    constexpr int ITEMS = 8 * NB;              // lane items per row
    constexpr int LPL = RW * ITEMS / 64;       // chunks per lane over the wave's rows
    constexpr int GROUPS = LPL > 16 ? LPL / 16 : 1;
    constexpr int RPG = RW / GROUPS;           // rows per group
    constexpr int LPG = RPG * ITEMS / 64;      // chunks per lane per group
    constexpr int M = ITEMS >= 64 ? ITEMS / 64 : 1;   // items per lane
    constexpr int WH = RW * NB;                // block headers of one wave's rows
    constexpr int HPL = (WH + 63) / 64;        // header loads per lane
    const LdsA L = lds_a(a.hidden, NB, 2 * HR);   // half units: half the scale table
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t nblk = a.ffn / 32;
    // HALF: workgroup b of a run of 16 takes half (b % 16) / 8 of block
    // 8 (b / 16) + b % 8 (of all slots' blocks); else unit = the block
    const uint32_t hh = HALF ? (unit % 16) / 8 : 0;
    const uint32_t ub_ = HALF ? 8 * (unit / 16) + unit % 8 : unit;
    const uint32_t slot = ub_ / nblk, jb = ub_ % nblk;
    const uint8_t *xq = a.xq;
    const bool publisher = unit == 0 && wave == 0;
    pin_args(a.gate, a.up, a.gate_sh, a.up_sh, a.hq8);

    // routing inputs, then x (fp32 or q8_1; lane task t covers values
    // 4t..4t+3); their latencies overlap. Loads are clamped, not guarded: no
    // branch sits around a load.
    constexpr int XTASKS = 64 * NB;            // quantizer lane tasks (8 per 32-block)
    constexpr int XPT = (XTASKS + NT - 1) / NT;
    float4 xv[XPT];
    uint32_t xqv[XPT], xdv[XPT];
    if constexpr (NORMED) {
        // the steps before the layer, here: xn and the routing from its logits
        StkCtx none{};
        normed_prologue<NB, C, NT, XPT>(a, lds + L.scl, gridDim.x, rt, xv, ld_dev(a.fsync + 1), a.fsync + FSYNC_R,
                                        none);
    } else {
        // every wave routes on its own: no barrier before its weight loads
        // (routing by rank over the workgroup, 8 threads per expert, measured
        // slower: 14.3-14.6 us against 13.6-13.9 us per layer)
        float lv[C];
        route_issue<C>(a, lv, rt);
        if (xq == nullptr) {
#pragma unroll
            for (int i = 0; i < XPT; i++) xv[i] = *(const float4 *)(a.x + 4 * min(tid + NT * i, (uint32_t)XTASKS - 1));
        } else {
#pragma unroll
            for (int i = 0; i < XPT; i++) {
                const uint32_t t = min(tid + NT * i, (uint32_t)XTASKS - 1);
                const uint8_t *b = xq + (t >> 3) * 36;
                xqv[i] = *(const uint32_t *)(b + 4 + 4 * (t & 7));
                xdv[i] = ld_u16(b);
            }
        }
        // a unit needs only its slot's expert (rank slot): slot + 1 rounds,
        // none for the shared expert; the routing's publisher and the fused
        // layer (whose down tiles take every slot) rank them all
        route_finish<C>(a, lv, rt, FUSED || publisher ? -1 : (int)slot < a.n_sel ? (int)slot + 1 : 0);
    }
    // Drain the routing and x loads here, in one place: with loads issued
    // under branches the compiler cannot tell which registers are still
    // pending and would otherwise wait for the weight loads one by one.
    __builtin_amdgcn_s_waitcnt(VMCNT0);

    const uint64_t rb = NB * 144;
    const uint8_t *gb, *ub;
    if ((int)slot < a.n_sel) {
        int32_t id = __builtin_amdgcn_readlane(rt.eid, (int)slot);
        if ((uint32_t)id >= a.n_expert) id = 0;   // bad explicit id: reported by route_publish
        const uint64_t e = (uint64_t)id;
        gb = a.gate + e * a.ffn * rb;
        ub = a.up + e * a.ffn * rb;
    } else {
        gb = a.gate_sh;
        ub = a.up_sh;
    }
    auto row_ptr = [&](uint32_t v) -> const uint8_t * {   // v in [0, 2 HR)
        return v < (uint32_t)HR ? gb + (uint64_t)(32 * jb + HR * hh + v) * rb
                                : ub + (uint64_t)(32 * jb + HR * hh + v - HR) * rb;
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
        return row_ptr(RW * wave + r) + (it / 8) * 144 + 16 + 16 * (it % 8);
    };

    // x -> q8_1 in LDS (the loads are already in): while the weights stream
    // in when they had to wait for the routing; before they are issued when
    // nothing routes (the shared expert alone, a dense FFN), so that this
    // barrier never waits on a sibling wave still issuing into a full memory
    // pipeline (a dense FFN's 384 workgroups request 58 MB at once)
    const Act xa = act_carve(lds + L.xact, a.hidden);
    auto stage_x = [&]() {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const uint32_t t = tid + NT * i, blk = t >> 3, part = t & 7;
            if (t >= XTASKS) break;   // whole 8-lane groups leave together
            uint32_t qv;
            int lo, hi;
            float dd;
            if (xq) {
                qv = xqv[i];
                q8_part_sums(qv, lo, hi);
                dd = h2f(xdv[i]);
            } else {
                uint32_t d16, s16;
                qv = quant_q8_1_part(xv[i], d16, s16, lo, hi, dd);
            }
            *(uint32_t *)(xa.qs + 32 * blk + 4 * part) = qv;
            if (part == 0) {
                xa.d8[blk] = dd;
                xa.qs16[2 * blk] = lo;
                xa.qs16[2 * blk + 1] = hi;
            }
        }
        __syncthreads();
    };
    const bool x_first = a.n_sel == 0;
    if (x_first) stage_x();

    // every weight load of the wave: its block headers first, then chunks
    uint4 hv[HPL];
#pragma unroll
    for (int i = 0; i < HPL; i++) {
        const uint32_t h = min(lane + 64 * i, (uint32_t)WH - 1);   // duplicates decode the same header
        hv[i] = ld16(row_ptr(RW * wave + h / NB) + (h % NB) * 144);
    }
    uint4 q[LPG];
#pragma unroll
    for (int k = 0; k < LPG; k++) q[k] = ld16(chunk(0, k));

    if (publisher)
        route_publish(a, rt.eid, (NORMED || a.logits) && a.n_sel > 0 ? route_weight(rt.logit, a.n_sel) : rt.w);
    if (!x_first) stage_x();   // x is ready long before the weights: off the critical path
    XSlice xs[M];
#pragma unroll
    for (int m = 0; m < M; m++) xs[m] = x_slice(xa, ITEMS >= 64 ? 64 * m + lane : lane % ITEMS);
    // decode the wave's headers into its own LDS area
    float4 *scl = (float4 *)(lds + L.scl) + 4 * WH * wave;
#pragma unroll
    for (int i = 0; i < HPL; i++) {
        const uint32_t h = lane + 64 * i;
        if (h < WH) {
            Q4K::Raw raw;
            raw.h = hv[i];
            const uint32_t b = h % NB;
            const float4 dA = *(const float4 *)(xa.d8 + 8 * b), dB = *(const float4 *)(xa.d8 + 8 * b + 4);
            const float d8[8] = {dA.x, dA.y, dA.z, dA.w, dB.x, dB.y, dB.z, dB.w};
#pragma unroll
            for (int g = 0; g < 4; g++) {
                float ds0, ds1, dm0, dm1;
                Q4K::scales(raw, g, ds0, ds1, dm0, dm1);
                scl[4 * h + g] = make_float4(ds0 * d8[2 * g], ds1 * d8[2 * g + 1], dm0 * d8[2 * g], dm1 * d8[2 * g + 1]);
            }
        }
    }
    wave_sync_lds();

    float *gu = (float *)(lds + L.gu);
#pragma unroll
    for (int grp = 0; grp < GROUPS; grp++) {
        if (grp > 0) {
#pragma unroll
            for (int k = 0; k < LPG; k++) q[k] = ld16(chunk(grp, k));
        }
        if constexpr (ITEMS >= 64) {
            float acc[LPG];   // virtual row k: sub-block 64 * (k % M) + lane of row k / M
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t it = 64 * (k % M) + lane;
                const uint32_t row = grp * RPG + k / M;   // within the wave
                const float4 sc = scl[4 * (row * NB + it / 8) + (it % 8) / 2];
                acc[k] = q4k_term(q[k], sc, xs[k % M]);
            }
            const float v = pw_rows<LPG, M>(acc);
            if (lane < (uint32_t)RPG) gu[RW * wave + grp * RPG + pw_rows_row<LPG, M>(lane)] = v;
        } else {
            const uint32_t it = lane % ITEMS;
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t row = lane / ITEMS + k * (64 / ITEMS);   // within the wave
                const float4 sc = scl[4 * (row * NB + it / 8) + (it % 8) / 2];
                // group_sum adds lane bit 0 first: the pairwise tree over the row's sub-blocks
                const float v = group_sum<ITEMS>(q4k_term(q[k], sc, xs[0]));
                if (it == 0) gu[RW * wave + row] = v;
            }
        }
    }
    __syncthreads();

    // (before wave 0 may leave: the first of a half-unit pair writes no block)
    if (a.dbg_gu && tid < 2 * (uint32_t)HR) {
        const bool upr = tid >= (uint32_t)HR;
        float *d = a.dbg_gu + (uint64_t)slot * 2 * a.ffn + (upr ? a.ffn : 0) + 32 * jb + HR * hh + tid % HR;
        *d = gu[tid];
    }
    if (wave == 0) {
        // one h value per lane (lanes 32..63 mirror 0..31), then the q8_1
        // block across 32 lanes: same rules as quant_q8_1_part
        const uint32_t j = lane & 31;
        float h;
        if constexpr (HALF) {
            // this half's 16 values (lane & 15), out as tagged words; the
            // second of the pair to count itself in reads the other 16
            const float own = kq_silu_mul(gu[lane & 15], gu[16 + (lane & 15)]);
            uint32_t old = 0;
            if (lane == 0)
                old = __hip_atomic_fetch_add(a.fsync + FSYNC_DHC + ub_, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            old = __builtin_amdgcn_readfirstlane(old);
            const uint32_t tag = (old >> 1) + 1;
            uint32_t *words = a.fsync + FSYNC_DHW + 2 * 32 * ub_;
            if (lane < 16) st_dev2(words + 2 * (16 * hh + lane), ((uint64_t)tag << 32) | __float_as_uint(own));
            if ((old & 1) == 0) return;   // the first of the pair: the other writes the block (whole wave)
            const bool mine = (j >> 4) == hh;
            uint64_t v = 0;
            uint32_t spins = 0;
            for (;;) {
                v = ld_dev2(words + 2 * j);
                if (__all(mine || (uint32_t)(v >> 32) == tag)) break;
                if (++spins >= FSYNC_SPIN_LIMIT) {
                    if (lane == 0) atomicOr(a.err, 4);
                    break;
                }
            }
            h = mine ? own : __uint_as_float((uint32_t)v);
        } else {
            h = kq_silu_mul(gu[j], gu[32 + j]);
        }
        const float am = max32(fabsf(h));
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const int qv = (int)roundf(h * id);
        const int total = sum32(qv);
        uint8_t *blk = a.hq8 + ((uint64_t)slot * nblk + jb) * 36;
        if (lane < 32) blk[4 + lane] = (uint8_t)(qv & 255);
        if (lane == 0) *(uint32_t *)blk = f2h_rne(d) | (f2h_rne((float)total * d) << 16);
        if constexpr (FUSED) {
            // the block's 9 dwords again, each as one 8-byte device-coherent
            // word {dword, generation + 1}: a reader that sees the tag sees
            // the dword with it, so nothing here waits for the stores
            uint8_t *stage = lds + L.xact;   // the x area is free by now
            if (lane < 32) stage[4 + lane] = (uint8_t)(qv & 255);
            if (lane == 0) *(uint32_t *)stage = f2h_rne(d) | (f2h_rne((float)total * d) << 16);
            wave_sync_lds();
            uint32_t g = flag;   // the generation: made opaque here so no earlier use waits for its load
            asm volatile("" : "+v"(g));
            if (lane < 9)
                st_dev2(hx + 2 * (9 * unit + lane), ((uint64_t)(g + 1) << 32) | ((const uint32_t *)stage)[lane]);
        }
    }
    if constexpr (FUSED) {
        // h is out: now the fused layer's down-tile loads (a barrier that
        // orders LDS alone, so nobody waits for h's stores to be acknowledged)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        after(rt);
    }
}

template <int NB, int C, bool NORMED = false, bool HALF = false>
__global__ void __launch_bounds__(a1_threads<NB>()) k_moe_gu(MoeArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    GuRoute rt;
    gu_unit<NB, C, false, NoMore, NORMED, HALF>(a, blockIdx.x, lds, rt, 0);
}

// ---------------------------------------------------------------------------
// Kernel B: a tile of TR output rows x n_slots down rows per workgroup; one
// lane-slot of S = QD::IPB * P lanes per (row, slot) pair: lane s takes item
// s % IPB of blocks s / IPB + P*i (i < IPL), so long rows (a dense FFN's
// 12288-wide down projection) spread over up to 64 lanes. Order of work: the
// routing and the q8_1 h loads (both written by kernel A, so L2/MALL hits),
// then, once the routing is in, every down-weight load; h is staged into LDS
// while the weights stream. Loads are clamped rather than guarded so the
// compiler can count them (a load under a branch makes it wait for all).
// ---------------------------------------------------------------------------
struct LdsB {
    uint32_t hacts, res, total;
};
__host__ __device__ inline LdsB lds_b(uint32_t ffn, uint32_t n_slots, uint32_t tr) {
    LdsB L;
    L.hacts = 0;
    L.res = L.hacts + n_slots * act_bytes(ffn);
    L.total = L.res + (tr * n_slots + MAX_SLOTS) * 4;   // padding: the unrolled slot sum reads past the tile
    return L;
}

// q8_1 h of every slot: one lane per 16-byte half block (t = 2 * block + half),
// so each lane's 16 values are exactly one half-block sum.
// HT unrolled h tasks per thread, all issued before the down weights (a task
// loaded after them could only be waited for together with the whole weight
// stream): 2 covers n_slots * ffn/16 <= 512 (the MoE shapes), 4 covers a
// dense FFN's 12288-wide h (768 tasks); more go round a loop.
template <int HT>
struct HLoad {
    uint4 q[HT];
    uint32_t d[HT];
};
template <int HT>
__device__ __forceinline__ void load_h(const uint8_t *hq8, uint32_t ntask, uint32_t first, uint32_t nt, HLoad<HT> &h) {
#pragma unroll
    for (int i = 0; i < HT; i++) {
        const uint32_t t = min(first + threadIdx.x + nt * i, ntask - 1);
        const uint8_t *b = hq8 + (t >> 1) * 36;
        h.q[i] = ld16(b + 4 + 16 * (t & 1));
        h.d[i] = ld_u16(b);
    }
}
template <int HT>
__device__ __forceinline__ void stage_h(uint8_t *hl, uint32_t ffn, uint32_t ntask, uint32_t first, uint32_t nt,
                                        const HLoad<HT> &h) {
    const uint32_t nblk = ffn / 32, ab = act_bytes(ffn);
#pragma unroll
    for (int i = 0; i < HT; i++) {
        const uint32_t t = first + threadIdx.x + nt * i;
        if (t < ntask) {
            const uint32_t blk = t >> 1, half = t & 1, slot = blk / nblk, kb = blk % nblk;
            const Act act = act_carve(hl + slot * ab, ffn);
            *(uint4 *)(act.qs + 32 * kb + 16 * half) = h.q[i];
            int sum = dot4(h.q[i].x, 0x01010101u, 0);
            sum = dot4(h.q[i].y, 0x01010101u, sum);
            sum = dot4(h.q[i].z, 0x01010101u, sum);
            sum = dot4(h.q[i].w, 0x01010101u, sum);
            act.qs16[2 * kb + half] = sum;
            if (half == 0) act.d8[kb] = h2f(h.d[i]);
        }
    }
}

// NT: the workgroup size, or 0 for blockDim.x (up to B_MAX_THREADS)
template <class QD, int IPL, int P, int NT>
__global__ void __launch_bounds__(NT > 0 ? NT : B_MAX_THREADS) k_moe_down(MoeArgs a, uint32_t tr, uint32_t n_slots) {
    const uint32_t nt = NT > 0 ? (uint32_t)NT : blockDim.x;
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsB L = lds_b(a.ffn, n_slots, tr);
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    pin_args(a.down, a.down_sh, a.y);
    // the normed layer's exchange generation, read now and advanced at the
    // end: kernel A is over, so every one of its workgroups has read it (the
    // load is unconditional; without a router it reads the routing words)
    uint32_t gen = ld_dev(a.router ? a.fsync + 1 : (uint32_t *)a.route_ids);
    // routing (lane r holds slot r), then the h loads
    const int32_t rid = a.route_ids[min(lane, (uint32_t)MAX_SLOTS - 1)];
    float rw = a.route_w[min(lane, (uint32_t)MAX_SLOTS - 1)];
    const uint32_t ntask = n_slots * (a.ffn / 32) * 2;
    constexpr int HT = P >= 16 ? 4 : 2;
    HLoad<HT> hv;
    load_h(a.hq8, ntask, 0, nt, hv);

    constexpr uint32_t S = QD::IPB * P;
    const uint32_t ls = tid / S, s = tid % S;
    const uint32_t item = s % QD::IPB, sub = s / QD::IPB;
    const uint32_t row0 = blockIdx.x * tr;
    const uint32_t nrows = row0 + tr <= a.hidden ? tr : a.hidden - row0;
    const uint32_t npairs = nrows * n_slots;
    const uint64_t rbd = (uint64_t)(a.ffn / 256) * QD::BB;
    const uint32_t nbk = a.ffn / 256;
    const bool active = ls < npairs;
    const uint32_t lc = min(ls, npairs - 1);   // idle lane-slots load a real pair and drop it
    const uint32_t sl = lc % n_slots, r = lc / n_slots;
    const int32_t sid = __shfl(rid, (int)sl, WAVE);
    const bool routed = (int)sl < a.n_sel;
    const uint8_t *db = routed ? a.down + (uint64_t)sid * a.hidden * rbd : a.down_sh;
    const uint8_t *rp = db + (uint64_t)(row0 + r) * rbd;
    typename QD::Raw raw[IPL > 0 ? IPL : 1];
    if constexpr (IPL > 0) {
#pragma unroll
        for (int i = 0; i < IPL; i++)   // clamped: a block past the row is loaded and dropped
            raw[i] = QD::load(rp + min(sub + P * i, nbk - 1) * QD::BB, (int)item);
    }
    stage_h(lds + L.hacts, a.ffn, ntask, 0, nt, hv);
    for (uint32_t first = HT * nt; first < ntask; first += HT * nt) {
        load_h(a.hq8, ntask, first, nt, hv);   // only when n_slots * ffn / 16 > nt * HT
        stage_h(lds + L.hacts, a.ffn, ntask, first, nt, hv);
    }
    __syncthreads();
    float x = 0.0f;
    {
        const Act act = act_carve(lds + L.hacts + sl * act_bytes(a.ffn), a.ffn);
        if constexpr (IPL > 0) {
#pragma unroll
            for (int i = 0; i < IPL; i++) {
                const uint32_t b = sub + P * i;
                const float v = QD::dot_q8(raw[i], (int)item, act, min(b, nbk - 1));
                x += b < nbk ? v : 0.0f;
            }
        } else {
            for (uint32_t b = sub; b < nbk; b += P) x += QD::dot_q8(QD::load(rp + b * QD::BB, (int)item), (int)item, act, b);
        }
    }
    x = group_sum<S>(x);
    float *res = (float *)(lds + L.res);
    if (active && s == 0) res[ls] = x;
    // every lane's weight in place before the row branch reads it by lane
    // (the compiler could otherwise sink the load into the branch)
    asm volatile("" : "+v"(rw));
    __syncthreads();
    if (tid < nrows) {
        // rank order, one fmaf per slot: y = w_{n-1} r_{n-1} + (... + (w_0 r_0 + 0))
        float y = 0.0f;
#pragma unroll
        for (int k = 0; k < MAX_SLOTS; k++) {
            const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rw), k));
            const float v = res[tid * n_slots + k];
            y = k < (int)n_slots ? fmaf(w, v, y) : y;
        }
        a.y[row0 + tid] = y;
    }
    asm volatile("" : "+v"(gen));
    if (a.router && blockIdx.x == 0 && tid == 0) st_dev(a.fsync + 1, gen + 1);
}

// ---------------------------------------------------------------------------
// Grouped batch mode: the GEMV path of the batched layer. An entry is up to
// GRP_MAX (token, rank) pairs routed to one expert, listed as {expert,
// first, count} (a.bslot, *a.bcount entries) with the pairs at
// a.border[first ..]. A workgroup reads its weight rows once and dots them
// with every pair of the entry, whose activations are staged in LDS. The
// item mapping, scale products, reductions and h quantization are those of
// kernels A and B, so a pair's h and down output are bit-identical to the
// single-token layer's.
// ---------------------------------------------------------------------------
constexpr uint32_t GRP_MAX = 8;

// Stage n rows of K q8_1 values (row g read from src_of(g)) into LDS
// activations at base + g * act_bytes(K), one 16-byte half block per task.
template <class SrcOf>
__device__ __forceinline__ void stage_rows_q8(uint8_t *base, uint32_t K, uint32_t n, SrcOf src_of) {
    const uint32_t nblk = K / 32, ab = act_bytes(K), ntask = n * nblk * 2;
    for (uint32_t t = threadIdx.x; t < ntask; t += blockDim.x) {
        const uint32_t g = t / (2 * nblk), r = t % (2 * nblk), kb = r >> 1, half = r & 1;
        const uint8_t *b = src_of(g) + (uint64_t)kb * 36;
        const uint4 q = ld16(b + 4 + 16 * half);
        const Act act = act_carve(base + g * ab, K);
        *(uint4 *)(act.qs + 32 * kb + 16 * half) = q;
        int sum = dot4(q.x, 0x01010101u, 0);
        sum = dot4(q.y, 0x01010101u, sum);
        sum = dot4(q.z, 0x01010101u, sum);
        sum = dot4(q.w, 0x01010101u, sum);
        act.qs16[2 * kb + half] = sum;
        if (half == 0) act.d8[kb] = h2f(ld_u16(b));
    }
}

struct LdsG {
    uint32_t xact, scl, gu, total;
};
__host__ __device__ inline LdsG lds_g(uint32_t hidden, uint32_t nb) {
    LdsG L;
    L.xact = 0;
    L.scl = GRP_MAX * act_bytes(hidden);   // 64 rows x nb headers x 4 groups x float4 (scales without x)
    L.gu = L.scl + 64 * nb * 64;
    L.total = L.gu + GRP_MAX * 64 * 4;
    return L;
}

template <int NB>
__global__ void __launch_bounds__(A_THREADS) k_moe_gu_grp(MoeArgs a) {
    constexpr int RW = A_ROWS_PER_WAVE;
    constexpr int ITEMS = 8 * NB;
    constexpr int LPG = RW * ITEMS / 64;   // chunks per lane (one row group: RW = 8, NB <= 16)
    constexpr int M = ITEMS >= 64 ? ITEMS / 64 : 1;
    constexpr int WH = RW * NB, HPL = (WH + 63) / 64;
    static_assert(LPG <= 16 && RW == 8, "one row group of 8 rows per wave");
    extern __shared__ __align__(16) uint8_t lds[];
    const LdsG L = lds_g(a.hidden, NB);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t nblk = a.ffn / 32;
    const uint32_t ei = blockIdx.x / nblk, jb = blockIdx.x % nblk;
    if (ei >= (uint32_t)*a.bcount) return;   // whole workgroup, before any barrier
    const int32_t *ent = a.bslot + 3 * ei;
    const uint32_t ex = (uint32_t)ent[0], cnt = (uint32_t)ent[2];
    const int32_t *pairs = a.border + ent[1];
    const uint64_t rb = NB * 144;
    const bool shared = ex >= a.n_expert;   // the grouping gives the shared expert id n_expert
    const uint8_t *gb = shared ? a.gate_sh : a.gate + (uint64_t)ex * a.ffn * rb;
    const uint8_t *ub = shared ? a.up_sh : a.up + (uint64_t)ex * a.ffn * rb;
    auto row_ptr = [&](uint32_t v) -> const uint8_t * {   // v in [0, 64)
        return v < 32 ? gb + (uint64_t)(32 * jb + v) * rb : ub + (uint64_t)(32 * jb + v - 32) * rb;
    };
    auto chunk = [&](int k) -> const uint8_t * {
        uint32_t r, it;
        if constexpr (ITEMS >= 64) {
            r = k / M;
            it = 64 * (k % M) + lane;
        } else {
            r = lane / ITEMS + k * (64 / ITEMS);
            it = lane % ITEMS;
        }
        return row_ptr(RW * wave + r) + (it / 8) * 144 + 16 + 16 * (it % 8);
    };
    // the weights (HBM) first, then the entry's activations (L2)
    uint4 hv[HPL];
#pragma unroll
    for (int i = 0; i < HPL; i++) {
        const uint32_t h = min(lane + 64 * i, (uint32_t)WH - 1);
        hv[i] = ld16(row_ptr(RW * wave + h / NB) + (h % NB) * 144);
    }
    uint4 q[LPG];
#pragma unroll
    for (int k = 0; k < LPG; k++) q[k] = ld16(chunk(k));
    const uint32_t ab = act_bytes(a.hidden);
    stage_rows_q8(lds + L.xact, a.hidden, cnt,
                  [&](uint32_t g) { return a.xq + (uint64_t)((uint32_t)pairs[g] / a.bS) * a.xq_stride; });
    // the wave's headers -> {d*sc, d*sc', dmin*m, dmin*m'} per group (x's
    // q8_1 scales are applied per pair below, in kernel A's order)
    float4 *scl = (float4 *)(lds + L.scl) + 4 * WH * wave;
#pragma unroll
    for (int i = 0; i < HPL; i++) {
        const uint32_t h = lane + 64 * i;
        if (h < WH) {
            Q4K::Raw raw;
            raw.h = hv[i];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                float ds0, ds1, dm0, dm1;
                Q4K::scales(raw, g, ds0, ds1, dm0, dm1);
                scl[4 * h + g] = make_float4(ds0, ds1, dm0, dm1);
            }
        }
    }
    // nibbles unpacked once for all pairs (when the registers allow)
    constexpr bool UNP = LPG <= 8;
    Q4K::Unp qu[UNP ? LPG : 1];
    if constexpr (UNP) {
#pragma unroll
        for (int k = 0; k < LPG; k++) {
            Q4K::Raw raw;
            raw.q = q[k];
            qu[k] = Q4K::unpack(raw);
        }
    }
    __syncthreads();   // activations staged; the scale table is wave-private

    float *gu = (float *)(lds + L.gu);
    for (uint32_t g = 0; g < cnt; g++) {
        const Act xa = act_carve(lds + L.xact + g * ab, a.hidden);
        if constexpr (ITEMS >= 64) {
            XSlice xs[M];
            float2 d8[M];
#pragma unroll
            for (int m = 0; m < M; m++) {
                const uint32_t it = 64 * m + lane, k8 = 8 * (it / 8) + 2 * ((it % 8) >> 1);
                xs[m] = x_slice(xa, it);
                d8[m] = make_float2(xa.d8[k8], xa.d8[k8 + 1]);
            }
            float acc[LPG];   // virtual row k: sub-block 64 * (k % M) + lane of row k / M
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t it = 64 * (k % M) + lane;
                const uint32_t row = k / M;
                const float4 s0 = scl[4 * (row * NB + it / 8) + (it % 8) / 2];
                const float2 dd = d8[k % M];
                const float4 sc = make_float4(s0.x * dd.x, s0.y * dd.y, s0.z * dd.x, s0.w * dd.y);
                if constexpr (UNP) acc[k] = q4k_term_u(qu[k], sc, xs[k % M]);
                else acc[k] = q4k_term(q[k], sc, xs[k % M]);
            }
            const float v = pw_rows<LPG, M>(acc);
            if (lane < (uint32_t)RW) gu[64 * g + RW * wave + pw_rows_row<LPG, M>(lane)] = v;
        } else {
            const uint32_t it = lane % ITEMS, k8 = 8 * (it / 8) + 2 * ((it % 8) >> 1);
            const XSlice xs = x_slice(xa, it);
            const float2 dd = make_float2(xa.d8[k8], xa.d8[k8 + 1]);
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t row = lane / ITEMS + k * (64 / ITEMS);
                const float4 s0 = scl[4 * (row * NB + it / 8) + (it % 8) / 2];
                const float4 sc = make_float4(s0.x * dd.x, s0.y * dd.y, s0.z * dd.x, s0.w * dd.y);
                const float v = group_sum<ITEMS>(UNP ? q4k_term_u(qu[k], sc, xs) : q4k_term(q[k], sc, xs));
                if (it == 0) gu[64 * g + RW * wave + row] = v;
            }
        }
    }
    __syncthreads();
    // h of pair g (wave g % 8): kernel A's q8_1 block
    for (uint32_t g = wave; g < cnt; g += A_THREADS / 64) {
        const uint32_t j = lane & 31;
        const float h = kq_silu_mul(gu[64 * g + j], gu[64 * g + 32 + j]);
        const float am = max32(fabsf(h));
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const int qv = (int)roundf(h * id);
        const int total = sum32(qv);
        uint8_t *blk = a.hq8 + ((uint64_t)pairs[g] * nblk + jb) * 36;
        if (lane < 32) blk[4 + lane] = (uint8_t)(qv & 255);
        if (lane == 0) *(uint32_t *)blk = f2h_rne(d) | (f2h_rne((float)total * d) << 16);
    }
}

// Down for an entry: kernel B's tile (tr rows, S = IPB * P lanes per row, the
// same blocks per lane), every pair's h staged in LDS, each pair's unweighted
// output row to yp.
template <class QD, int IPL, int P>
__global__ void __launch_bounds__(256) k_moe_down_grp(MoeArgs a, uint32_t tr) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t tid = threadIdx.x;
    if (blockIdx.y >= (uint32_t)*a.bcount) return;   // whole workgroup, before any barrier
    const int32_t *ent = a.bslot + 3 * blockIdx.y;
    const uint32_t ex = (uint32_t)ent[0], cnt = (uint32_t)ent[2];
    const int32_t *pairs = a.border + ent[1];
    constexpr uint32_t S = QD::IPB * P;
    const uint32_t ls = tid / S, s = tid % S;
    const uint32_t item = s % QD::IPB, sub = s / QD::IPB;
    const uint32_t row0 = blockIdx.x * tr;
    const uint32_t nrows = row0 + tr <= a.hidden ? tr : a.hidden - row0;
    const uint64_t rbd = (uint64_t)(a.ffn / 256) * QD::BB;
    const uint32_t nbk = a.ffn / 256;
    const bool active = ls < nrows;
    const uint32_t r = min(ls, nrows - 1);   // idle lane-slots load a real row and drop it
    const uint8_t *db = ex >= a.n_expert ? a.down_sh : a.down + (uint64_t)ex * a.hidden * rbd;
    const uint8_t *rp = db + (uint64_t)(row0 + r) * rbd;
    typename QD::Raw raw[IPL > 0 ? IPL : 1];
    if constexpr (IPL > 0) {
#pragma unroll
        for (int i = 0; i < IPL; i++) raw[i] = QD::load(rp + min(sub + P * i, nbk - 1) * QD::BB, (int)item);
    }
    const uint64_t hstride = (uint64_t)(a.ffn / 32) * 36;
    stage_rows_q8(lds, a.ffn, cnt, [&](uint32_t g) { return a.hq8 + (uint64_t)pairs[g] * hstride; });
    // the quants are unpacked once for all pairs
    typename QD::Unp unp[IPL > 0 ? IPL : 1];
    if constexpr (IPL > 0) {
#pragma unroll
        for (int i = 0; i < IPL; i++) unp[i] = QD::unpack(raw[i]);
    }
    __syncthreads();
    const uint32_t ab = act_bytes(a.ffn);
    for (uint32_t g = 0; g < cnt; g++) {
        const Act act = act_carve(lds + g * ab, a.ffn);
        float x = 0.0f;
        if constexpr (IPL > 0) {
#pragma unroll
            for (int i = 0; i < IPL; i++) {
                const uint32_t b = sub + P * i;
                const float v = QD::dot_q8_u(raw[i], unp[i], (int)item, act, min(b, nbk - 1));
                x += b < nbk ? v : 0.0f;
            }
        } else {
            for (uint32_t b = sub; b < nbk; b += P) x += QD::dot_q8(QD::load(rp + b * QD::BB, (int)item), (int)item, act, b);
        }
        x = group_sum<S>(x);
        if (active && s == 0) a.yp[(uint64_t)pairs[g] * a.hidden + row0 + ls] = x;
    }
}

// ---------------------------------------------------------------------------
// The fused layer: one launch per layer. The grid never exceeds the CU count
// and a workgroup fits an empty CU, so every workgroup is resident at once
// and the wait below ends. Workgroup w:
//   1. w < U = n_slots * ffn/32: gate/up unit w exactly as kernel A;
//   2. publishes its exchange block: 9 device-coherent 8-byte words
//      {dword, gen + 1} (its q8_1 h block, or zeros without a unit). A
//      reader that sees a word's tag sees its dword, so nothing waits for
//      these stores;
//   3. loads its down tile (output rows w*tr .., every slot of each row, S
//      lanes per pair) once its own gate/up is done: issued earlier, behind
//      the gate/up loads, they stall the CU's issue (its outstanding-request
//      capacity) and the unit's dots wait (measured: 2 us later);
//   4. reads every workgroup's block until all words carry gen + 1 (that
//      read is h), stages h into LDS, dots, and sums each row's slots in
//      rank order.
// gen: every workgroup reads it before it publishes, so once workgroup 0
// has seen every block, every read is done and it advances gen for the next
// call. Nothing is cleared between calls (graph replays included): stale
// words carry an older generation.
// ---------------------------------------------------------------------------
struct LdsF {
    uint32_t hacts, res, wts, vote, total;
};
__host__ __device__ inline LdsF lds_f(uint32_t hidden, uint32_t nb, uint32_t ffn, uint32_t n_slots, uint32_t tr) {
    LdsF L;
    L.hacts = lds_a(hidden, nb).total;
    L.res = L.hacts + n_slots * act_bytes(ffn);
    L.wts = L.res + (tr * n_slots + MAX_SLOTS) * 4;   // padding: the unrolled slot sum reads past the tile
    L.vote = L.wts + MAX_SLOTS * 4;
    L.total = L.vote + 2 * 16 * 4;
    return L;
}
// Waves 0 .. 7 hold the down tile (its weights and dots), waves 8 .. 15 read
// the exchange: a wave's loads complete in issue order, so a poll issued
// behind a wave's down-weight loads could not be seen before those arrive
// (measured: h seen 3.1 us after its last store with one wave doing both).
constexpr uint32_t FUSED_DOWN_THREADS = 512;
constexpr int FUSED_HW = 5;   // exchange words per polling thread: 9 * G <= 5 * 512

template <int NB, int C, class QD, int S, int IPL>
__global__ void __launch_bounds__(a1_threads<NB>()) k_moe_fused(MoeArgs a, uint32_t tr, uint32_t n_slots) {
    constexpr uint32_t NP = a1_threads<NB>() - FUSED_DOWN_THREADS;   // polling threads
    constexpr uint32_t P = S / QD::IPB;   // block slots per pair: lane s takes blocks s / IPB + P * i
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = blockIdx.x, G = gridDim.x;
    const uint32_t nblk = a.ffn / 32, U = n_slots * nblk;
    const LdsF L = lds_f(a.hidden, NB, a.ffn, n_slots, tr);
    const bool poller = tid >= FUSED_DOWN_THREADS;
    pin_args(a.down, a.down_sh, a.y, a.fsync, a.hq8);
    // this call's generation: issued first, used last (any arithmetic on it
    // here would wait for the load before the routing loads go out)
    const uint32_t gen = ld_dev(a.fsync);

    // the down tile's pair ls = (row r, slot sl) on S lanes of waves 0 .. 7;
    // lane s of it takes item s % IPB of blocks s / IPB + P * i
    const uint32_t s = tid % S, ls = tid / S;
    const uint32_t item = s % QD::IPB, bs = s / QD::IPB;
    const uint32_t nbk = a.ffn / 256;
    const uint32_t row0 = w * tr;
    const uint32_t nrows = min(tr, a.hidden - row0);   // the host keeps row0 < hidden
    const uint32_t npairs = nrows * n_slots;
    const uint32_t lc = min(ls, npairs - 1);   // idle lane-slots (and the pollers) address a real pair
    const uint32_t sl = lc % n_slots, r = lc / n_slots;
    const uint64_t rbd = (uint64_t)nbk * QD::BB;
    typename QD::Raw raw[IPL];
    auto load_down = [&](const GuRoute &rt) {
        int32_t sid = __shfl(rt.eid, (int)sl, WAVE);
        if ((uint32_t)sid >= a.n_expert) sid = 0;   // bad explicit id: reported by route_publish
        const uint8_t *rp = ((int)sl < a.n_sel ? a.down + (uint64_t)sid * a.hidden * rbd : a.down_sh) +
                            (uint64_t)(row0 + r) * rbd;
        if (!poller) {   // whole waves
#pragma unroll
            for (int i = 0; i < IPL; i++) raw[i] = QD::load(rp + min(bs + P * i, nbk - 1) * QD::BB, (int)item);
        }
    };
    GuRoute rt;
    if (w < U) {
        gu_unit<NB, C, true>(a, w, lds, rt, gen, a.fsync + FSYNC_H, load_down);
    } else {
        float lv[C];
        route_issue<C>(a, lv, rt);
        route_finish<C>(a, lv, rt);
        uint32_t g = gen;
        asm volatile("" : "+v"(g));
        if (tid < 9) st_dev2(a.fsync + FSYNC_H + 2 * (9 * w + tid), (uint64_t)(g + 1) << 32);
        load_down(rt);
    }
    // routing weights: lane k = slot k (the shared expert weighs 1)
    float rw = a.logits && a.n_sel > 0 ? route_weight(rt.logit, a.n_sel) : rt.w;
    rw = (int)lane < a.n_sel ? rw : ((int)lane == a.n_sel && a.has_shared ? 1.0f : 0.0f);

    // every workgroup's block, until all carry gen + 1: each polling wave
    // waits for its own words with two rounds of loads in flight (the next
    // round goes out before the previous one is checked, so a word is sampled
    // twice per round trip); the down waves go straight to the barrier below
    uint32_t tag = gen;
    asm volatile("" : "+v"(tag));
    tag += 1;
    const uint32_t nw = 9 * G, pt = tid - FUSED_DOWN_THREADS;
    uint32_t *xw = a.fsync + FSYNC_H;
    uint64_t v[FUSED_HW];
    if (poller) {   // whole waves
        uint64_t va[FUSED_HW], vb[FUSED_HW];
        auto issue = [&](uint64_t *o) {
#pragma unroll
            for (int i = 0; i < FUSED_HW; i++) o[i] = ld_dev2(xw + 2 * min(pt + NP * i, nw - 1));
        };
        auto seen = [&](const uint64_t *o) {
            bool ok = true;
#pragma unroll
            for (int i = 0; i < FUSED_HW; i++) ok &= (uint32_t)(o[i] >> 32) == tag;
            return __all(ok);
        };
        issue(va);
        uint32_t spins = 0;
        for (;;) {
            issue(vb);
            if (seen(va)) {
#pragma unroll
                for (int i = 0; i < FUSED_HW; i++) v[i] = va[i];
                break;
            }
            issue(va);
            if (seen(vb)) {
#pragma unroll
                for (int i = 0; i < FUSED_HW; i++) v[i] = vb[i];
                break;
            }
            if (++spins >= FSYNC_SPIN_LIMIT / 2) {
                if (lane == 0) atomicOr(a.err, 4);
#pragma unroll
                for (int i = 0; i < FUSED_HW; i++) v[i] = vb[i];
                break;
            }
        }
    }

    // h into LDS: word t = dword t % 9 of block t / 9 (dword 0: d and s;
    // blocks past U are the other workgroups' empty ones)
    const uint32_t ab = act_bytes(a.ffn);
    if (poller) {
#pragma unroll
        for (int i = 0; i < FUSED_HW; i++) {
            const uint32_t t = pt + NP * i;
            if (t < 9 * U) {
                const uint32_t b = t / 9, k = t % 9, kb = b % nblk;
                const Act act = act_carve(lds + L.hacts + (b / nblk) * ab, a.ffn);
                const uint32_t dw = (uint32_t)v[i];
                if (k == 0) act.d8[kb] = h2f(dw & 0xFFFFu);
                else *(uint32_t *)(act.qs + 32 * kb + 4 * (k - 1)) = dw;
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    // past the barrier every polling wave of this workgroup has seen all
    // blocks, so every workgroup has read gen: workgroup 0 publishes the next
    // call's
    if (w == 0 && tid == 0) st_dev(a.fsync, tag);
    // exact sums of each 16-value half block
    for (uint32_t t = tid; t < 2 * U; t += blockDim.x) {
        const uint32_t b = t >> 1, half = t & 1, kb = b % nblk;
        const Act act = act_carve(lds + L.hacts + (b / nblk) * ab, a.ffn);
        const uint4 q = *(const uint4 *)(act.qs + 32 * kb + 16 * half);
        int sum = dot4(q.x, 0x01010101u, 0);
        sum = dot4(q.y, 0x01010101u, sum);
        sum = dot4(q.z, 0x01010101u, sum);
        sum = dot4(q.w, 0x01010101u, sum);
        act.qs16[2 * kb + half] = sum;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

    float *res = (float *)(lds + L.res), *wts = (float *)(lds + L.wts);
    if (!poller) {   // whole waves
        float x = 0.0f;
        const Act act = act_carve(lds + L.hacts + sl * ab, a.ffn);
#pragma unroll
        for (int i = 0; i < IPL; i++) {
            const uint32_t b = bs + P * i;
            const float d = QD::dot_q8(raw[i], (int)item, act, min(b, nbk - 1));
            x += b < nbk ? d : 0.0f;
        }
        x = group_sum<S>(x);
        if (ls < npairs && s == 0) res[ls] = x;
    }
    // the slot weights through LDS: read back by lane from inside the row
    // branch below, a register's other lanes may never have been computed
    // (the compiler sinks the weight arithmetic into the branch)
    if (tid < MAX_SLOTS) wts[tid] = rw;
    __syncthreads();
    if (tid < nrows) {
        // rank order, one fmaf per slot: y = w_{n-1} r_{n-1} + (... + (w_0 r_0 + 0))
        float y = 0.0f;
#pragma unroll
        for (int k = 0; k < MAX_SLOTS; k++) {
            const float v2 = res[tid * n_slots + k];
            y = k < (int)n_slots ? fmaf(wts[k], v2, y) : y;
        }
        a.y[row0 + tid] = y;
    }
}

template <int NB, int C, class QD, int S, int IPL>
static hipError_t go_fused(const MoeArgs &a, uint32_t n_slots, uint32_t tr, uint32_t G, hipStream_t s) {
    const LdsF L = lds_f(a.hidden, NB, a.ffn, n_slots, tr);
    if (L.total > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_moe_fused<NB, C, QD, S, IPL>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)L.total);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_moe_fused<NB, C, QD, S, IPL>), dim3(G), dim3(a1_threads<NB>()), L.total, s, a, tr, n_slots);
    return hipGetLastError();
}
// S lanes per pair (QD::IPB items of P = S / IPB block slots), IPL blocks per lane
template <int NB, int C, class QD>
static hipError_t go_fused_s(const MoeArgs &a, uint32_t n_slots, uint32_t tr, uint32_t G, uint32_t S, uint32_t ipl,
                             hipStream_t s) {
    constexpr uint32_t B = QD::IPB;
    switch (S / B * 8 + ipl) {
        case 1 * 8 + 1: return go_fused<NB, C, QD, B, 1>(a, n_slots, tr, G, s);
        case 1 * 8 + 2: return go_fused<NB, C, QD, B, 2>(a, n_slots, tr, G, s);
        case 1 * 8 + 3: return go_fused<NB, C, QD, B, 3>(a, n_slots, tr, G, s);
        case 1 * 8 + 4: return go_fused<NB, C, QD, B, 4>(a, n_slots, tr, G, s);
        case 2 * 8 + 1: return go_fused<NB, C, QD, 2 * B, 1>(a, n_slots, tr, G, s);
        case 2 * 8 + 2: return go_fused<NB, C, QD, 2 * B, 2>(a, n_slots, tr, G, s);
        case 4 * 8 + 1: return go_fused<NB, C, QD, 4 * B, 1>(a, n_slots, tr, G, s);
        default: return hipErrorNotSupported;
    }
}
template <int NB, int C>
static hipError_t go_fused_q(const MoeArgs &a, uint32_t n_slots, uint32_t tr, uint32_t G, uint32_t S, uint32_t ipl,
                             hipStream_t s) {
    return a.down_type == T_Q6_K ? go_fused_s<NB, C, Q6K>(a, n_slots, tr, G, S, ipl, s)
                                 : go_fused_s<NB, C, Q4K>(a, n_slots, tr, G, S, ipl, s);
}
template <int NB>
static hipError_t go_fused_c(const MoeArgs &a, uint32_t n_slots, uint32_t tr, uint32_t G, uint32_t S, uint32_t ipl,
                             hipStream_t s) {
    if (a.n_expert <= 128) return go_fused_q<NB, 2>(a, n_slots, tr, G, S, ipl, s);
    if (a.n_expert <= 256) return go_fused_q<NB, 4>(a, n_slots, tr, G, S, ipl, s);
    return hipErrorNotSupported;
}

// The fused layer's shape: tr rows per workgroup so that the grid (one
// workgroup per tr rows) fits the CUs and every gate/up unit has a
// workgroup; the widest S (lanes per pair) whose tile fits the down waves,
// IPL = the row's blocks over S / IPB; hipErrorNotSupported when not.
static hipError_t launch_moe_fused(const MoeArgs &a, uint32_t n_slots, hipStream_t s) {
    const uint32_t nb = a.hidden / 256;
    if (!a.fsync || !(nb == 4 || nb == 8) || a.n_expert > 256) return hipErrorNotSupported;
    const uint32_t cus = min((uint32_t)device_cu_count(), FUSED_MAX_G);
    const uint32_t tr = (a.hidden + cus - 1) / cus;
    const uint32_t G = (a.hidden + tr - 1) / tr;
    const uint32_t U = n_slots * (a.ffn / 32);
    const uint32_t ipb = a.down_type == T_Q6_K ? 4 : 8, nbk = a.ffn / 256, pairs = tr * n_slots;
    if (U > G || 9 * G > (uint32_t)FUSED_HW * (1024 - FUSED_DOWN_THREADS) || pairs * ipb > FUSED_DOWN_THREADS)
        return hipErrorNotSupported;
    uint32_t S = ipb;
    while (2 * S <= 4 * ipb && S * ipb / ipb < ipb * nbk && pairs * 2 * S <= FUSED_DOWN_THREADS) S *= 2;
    const uint32_t P = S / ipb, ipl = (nbk + P - 1) / P;
    if (ipl > 4 || (P > 1 && ipl > (P == 2 ? 2u : 1u))) return hipErrorNotSupported;
    return nb == 8 ? go_fused_c<8>(a, n_slots, tr, G, S, ipl, s) : go_fused_c<4>(a, n_slots, tr, G, S, ipl, s);
}

// ---------------------------------------------------------------------------
// The XCD-sliced one-launch layer (k_moe_xcd): eight slots, XCD_G = 256
// workgroups, one per CU. Workgroup b serves slot x = b % 8 only; the
// dispatcher deals workgroups to the eight XCDs round robin, so slot x's
// workgroups run on XCD x (only the exchange's latency depends on that; the
// words are device-coherent either way). A CU streams at most ~25 GB/s, so
// every CU takes an equal share of both phases. With li = b / 8:
//   1. every wave routes; waves 0 .. R/4 - 1 issue the loads of the slot's
//      gate and up rows IW * li .. IW * li + IW - 1 (IW = ffn / 32, R = 2 IW
//      rows, 4 per wave) and decode, stage x and dot them as kernel A does;
//      then every wave issues its share of the slot's down rows [li * TRX,
//      (li + 1) * TRX), TRX = hidden / 32 (behind the gate/up loads in the
//      CU's queue, so the gate/up data comes first);
//   2. wave 0 forms the IW values of h = SiLU(g) * u (fp32, kernel A's
//      arithmetic) and publishes each as one tagged word;
//   3. the last four waves poll slot x's ffn words, quantize them to q8_1
//      in LDS (kernel A's quantizer, so the blocks are kernel A's bits;
//      workgroup li = 0 also writes them to a.hq8), and the down rows are
//      dotted: 16 lanes per row, lane s takes item s % IPB of blocks s / IPB
//      + P * i; each row's unweighted partial goes out as one tagged word;
//   4. wave 0 polls the eight slots' partials of rows li * TRX + x * TRC +
//      [0, TRC), TRC = TRX / 8, and writes y there: one fmaf per slot in
//      rank order, kernel B's sum.
// Generations: each workgroup reads its own word at its start (issued
// first, used last) and advances it at its end. Every workgroup runs every
// call, so the words stay equal and a call's tag is that value + 1; every
// word a call reads is written in that call, and stale words carry older
// tags. Nothing is cleared between calls or graph replays. Every wait is
// bounded (FSYNC_SPIN_LIMIT polls, then error bit 4 and the call's outputs
// are void).
// ---------------------------------------------------------------------------
constexpr uint32_t XCD_POLL_WAVES = 4;   // waves that poll the slot's h
constexpr int XCD_HW = 4;                // h words per polling thread at most: 1024 <= 4 * 256

// The shared expert of the XCD-sliced layer (SH): every byte of its weights
// is read once, by whole rows, and none of it depends on the routing.
//   gate/up: workgroup b forms shared h values b * IWS .. + IWS - 1 (IWS =
//     ffn / XCD_G; gate and up rows of those values on wave SW, kernel A's
//     item mapping, scale records, term order and reductions, so every value
//     is kernel A's) and publishes each as one tagged device-coherent word
//     once x is staged; (single layer) its loads went out before the
//     routing's, so the values are out before the slots' gate/up data is
//     in, and their exchange across the XCDs is hidden behind the stream;
//   down: XCD x takes shared rows [x H / 8, (x + 1) H / 8), RSW of them per
//     workgroup on waves SD.., 16 lanes per row over the whole ffn (the
//     routed slots' lane split), dotted against the shared h the pollers
//     stage with the slot's; one unweighted partial per row.
// The combine adds that partial last with weight 1, as kernel B does.
template <int NB, class QD, int S, int IW>
struct XcdShared {
    static constexpr int RW = 4, ITEMS = 8 * NB, LPG = RW * ITEMS / 64, M = ITEMS >= 64 ? ITEMS / 64 : 1;
    static constexpr int WH = RW * NB, HPL = (WH + 63) / 64;
    static constexpr uint32_t H = 256 * NB, F = 32 * IW;
    static constexpr uint32_t IWS = F / XCD_G;                 // shared h values per workgroup
    static constexpr uint32_t SW = 9, SD = 10;                 // the gate/up wave, the first down wave
    static constexpr uint32_t RSW = H / XCD_G;                 // shared down rows per workgroup
    static constexpr uint32_t NWD = (RSW * S + 63) / 64;       // down waves
    static constexpr uint32_t NBK = F / 256;
    static constexpr uint64_t RB = NB * 144, RBD = (uint64_t)NBK * QD::BB;
    static_assert(IWS >= 1 && 2 * IWS <= (uint32_t)RW && NBK <= (uint32_t)(S / QD::IPB) && SD + NWD <= 12,
                  "XCD layer shared expert shape");
    static_assert(HPL == (4 * NB + 63) / 64 && LPG == NB / 2, "XCD layer shared expert registers");
    uint32_t b, xs, li, tid, lane, wave;

    __device__ __forceinline__ bool down_wave() const { return wave >= SD && wave < SD + NWD; }
    __device__ __forceinline__ uint32_t item() const { return ((tid - 64 * SD) % S) % QD::IPB; }
    __device__ __forceinline__ uint32_t bslot() const { return ((tid - 64 * SD) % S) / QD::IPB; }
    // the shared down row this thread's item belongs to (threads past RSW * S: a real row, dropped)
    __device__ __forceinline__ uint32_t row() const {
        return xs * (H / XCD_SLOTS) + li * RSW + min((tid - 64 * SD) / S, RSW - 1);
    }
    __device__ __forceinline__ const uint8_t *gu_row(const MoeArgs &a, uint32_t v) const {   // v < RW (clamped)
        v = min(v, 2 * IWS - 1);
        return v < IWS ? a.gate_sh + (uint64_t)(b * IWS + v) * RB : a.up_sh + (uint64_t)(b * IWS + v - IWS) * RB;
    }
    __device__ __forceinline__ void issue_down(const MoeArgs &a, typename QD::Raw &raw) const {
        if (down_wave())
            raw = QD::load(a.down_sh + (uint64_t)row() * RBD + min(bslot(), NBK - 1) * QD::BB, (int)item());
    }
    __device__ __forceinline__ void issue_gu(const MoeArgs &a, uint4 (&hv)[HPL], uint4 (&q)[LPG]) const {
        if (wave == SW) {   // whole wave
#pragma unroll
            for (int i = 0; i < HPL; i++) {
                const uint32_t h = min(lane + 64 * i, (uint32_t)WH - 1);
                hv[i] = ld16(gu_row(a, h / NB) + (h % NB) * 144);
            }
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                uint32_t r, it;
                if constexpr (ITEMS >= 64) {
                    r = k / M;
                    it = 64 * (k % M) + lane;
                } else {
                    r = lane / ITEMS + k * (64 / ITEMS);
                    it = lane % ITEMS;
                }
                q[k] = ld16(gu_row(a, r) + (it / 8) * 144 + 16 + 16 * (it % 8));
            }
            // keeps this branch's last load its own: the down waves' branch
            // ends in a 16-byte load too, and merging the two would turn the
            // registers they load into stack slots
            asm volatile("");
        }
    }
    // wave SW, once x is staged at xa: the IWS shared h values, published as
    // tagged words (and the gate/up values to dbg_gu, slot n_sel)
    __device__ __forceinline__ void dots(const MoeArgs &a, uint8_t *lds, const Act &xa, uint32_t tag,
                                         const uint4 (&hv)[HPL], const uint4 (&q)[LPG]) const {
        const LdsA L = lds_a(a.hidden, NB);
        XSlice xsl[M];
#pragma unroll
        for (int m = 0; m < M; m++) xsl[m] = x_slice(xa, ITEMS >= 64 ? 64 * m + lane : lane % ITEMS);
        float4 *scl = (float4 *)(lds + L.scl) + 4 * WH * SW;   // the wave's own slice of the scale records
#pragma unroll
        for (int i = 0; i < HPL; i++) {
            const uint32_t h = lane + 64 * i;
            if (h < (uint32_t)WH) {
                Q4K::Raw rw;
                rw.h = hv[i];
                const uint32_t bb = h % NB;
                const float4 dA = *(const float4 *)(xa.d8 + 8 * bb), dB = *(const float4 *)(xa.d8 + 8 * bb + 4);
                const float d8[8] = {dA.x, dA.y, dA.z, dA.w, dB.x, dB.y, dB.z, dB.w};
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    float ds0, ds1, dm0, dm1;
                    Q4K::scales(rw, g, ds0, ds1, dm0, dm1);
                    scl[4 * h + g] = make_float4(ds0 * d8[2 * g], ds1 * d8[2 * g + 1], dm0 * d8[2 * g], dm1 * d8[2 * g + 1]);
                }
            }
        }
        wave_sync_lds();
        float *gu = (float *)(lds + L.gu) + RW * SW;
        if constexpr (ITEMS >= 64) {
            float acc[LPG];
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t it = 64 * (k % M) + lane, r = k / M;
                acc[k] = q4k_term(q[k], scl[4 * (r * NB + it / 8) + (it % 8) / 2], xsl[k % M]);
            }
            const float v = pw_rows<LPG, M>(acc);
            if (lane < (uint32_t)RW) gu[pw_rows_row<LPG, M>(lane)] = v;
        } else {
            const uint32_t it = lane % ITEMS;
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t r = lane / ITEMS + k * (64 / ITEMS);
                const float v = group_sum<ITEMS>(q4k_term(q[k], scl[4 * (r * NB + it / 8) + (it % 8) / 2], xsl[0]));
                if (it == 0) gu[r] = v;
            }
        }
        wave_sync_lds();
        if (lane < IWS) {
            const float h = kq_silu_mul(gu[lane], gu[IWS + lane]);
            st_dev2(a.fsync + FSYNC_XS + 2 * (b * IWS + lane), ((uint64_t)tag << 32) | __float_as_uint(h));
        }
        if (a.dbg_gu && lane < 2 * IWS)   // the shared expert is slot n_sel
            a.dbg_gu[(uint64_t)a.n_sel * 2 * a.ffn + (lane < IWS ? 0 : a.ffn) + b * IWS + lane % IWS] = gu[lane];
    }
};

// One workgroup's gate/up part: rows v < R of slot `slot` (v < IW: gate row
// IW * li + v, v < 2 IW: up row IW * li + v - IW), kernel A's item mapping,
// scale records, term order and reductions (so every value is kernel A's),
// on waves 0 .. R/4 - 1 (rows past R in the last of them are loaded and
// dropped); the others stage x with them. `down` issues the caller's down
// loads (after the wave's dots, or once x is staged on waves without rows).
// The shared expert's part (XcdShared): sh_start issues its single-layer
// weight loads right behind the routing's, sh_late forms its gate/up values
// once x is staged (in the stack it loads them first). Leaves the R gate/up values in
// LDS at lds + lds_a(..).gu. NORMED: the steps before the layer first
// (normed_prologue, with the caller's generation gen and the logits words
// at FSYNC_XR); x is the normalized vector it forms, the routing comes from
// its logits. STK: a layer of the stacked layer (ctx); past the stack's
// first layer x is the previous layer's y, read from its tagged words (or,
// NORMED, the residual step takes that y as its delta), and no wave issues
// a weight load before the whole of that y is seen.
template <int NB, int C, int IW, class Down, class ShStart, class ShLate, bool NORMED = false, bool STK = false>
__device__ __forceinline__ void gu_part(const MoeArgs &a, uint32_t slot, uint32_t li, uint8_t *lds, GuRoute &rt,
                                        Down down, ShStart sh_start, ShLate sh_late, uint32_t gen, StkCtx &ctx) {
    constexpr int RW = 4;                      // rows per wave (kernel A's at these widths)
    static_assert(a1_rw<NB>() == RW, "gu_part: kernel A's 4-row waves");
    constexpr int R = 2 * IW, GW = (R + RW - 1) / RW;   // rows, waves with rows
    constexpr int NT = a1_threads<NB>();
    constexpr int ITEMS = 8 * NB;
    constexpr int LPG = RW * ITEMS / 64;       // chunks per lane (one group: LPG <= 16)
    constexpr int M = ITEMS >= 64 ? ITEMS / 64 : 1;
    constexpr int WH = RW * NB;
    constexpr int HPL = (WH + 63) / 64;
    static_assert(R <= 64 && GW <= NT / 64 && LPG <= 16, "gu_part shape");
    const LdsA L = lds_a(a.hidden, NB);
    const uint32_t tid = STK ? opaque_v(threadIdx.x) : threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool rows = wave < (uint32_t)GW;
    pin_args(a.gate, a.up, a.gate_sh, a.up_sh);

    constexpr int XTASKS = 64 * NB;
    constexpr int XPT = (XTASKS + NT - 1) / NT;
    float4 xv[XPT];
    uint32_t xqv[XPT], xdv[XPT];
    if constexpr (NORMED) {
        normed_prologue<NB, C, NT, XPT, STK, C == 2>(a, lds + L.scl, XCD_G, rt, xv, gen, a.fsync + FSYNC_XR, ctx);
    } else {
        float lv[C];
        route_issue<C>(a, lv, rt);
        if (STK && ctx.l > 0) {
            // the routing's logits (and a layer's own x) in flight with the
            // first round of polls, ranked meanwhile; then a barrier: every
            // lane task's words of the previous layer's y seen. That y is the
            // layer's x, or, when the layer has an x of its own, only waited
            // for (the order of a decode chain)
            const bool own_x = a.x != nullptr;
            if (own_x) {
#pragma unroll
                for (int i = 0; i < XPT; i++) xv[i] = *(const float4 *)(a.x + 4 * min(tid + NT * i, (uint32_t)XTASKS - 1));
            }
            if (tid < XCD_G) {   // whole waves: one completion word each
                poll_done(a, ctx, [&] { route_finish<C>(a, lv, rt); });
            } else {
                route_finish<C>(a, lv, rt);
            }
            if (!own_x && tid < (uint32_t)XTASKS) {   // whole waves
                uint32_t qs[XPT];
#pragma unroll
                for (int i = 0; i < XPT; i++) qs[i] = min(tid + NT * i, (uint32_t)XTASKS - 1);
                read_y<XPT>(a, ctx, qs, true, xv);
            }
            __syncthreads();
        } else if (a.xq == nullptr) {
#pragma unroll
            for (int i = 0; i < XPT; i++) xv[i] = *(const float4 *)(a.x + 4 * min(tid + NT * i, (uint32_t)XTASKS - 1));
        } else {
#pragma unroll
            for (int i = 0; i < XPT; i++) {
                const uint32_t t = min(tid + NT * i, (uint32_t)XTASKS - 1);
                const uint8_t *b = a.xq + (t >> 3) * 36;
                xqv[i] = *(const uint32_t *)(b + 4 + 4 * (t & 7));
                xdv[i] = ld_u16(b);
            }
        }
        if constexpr (!STK) sh_start();   // routing-independent weights, behind only the routing's loads
        if constexpr (!STK) {
            if (a.logits && a.n_sel > 0) block_route<C>(a, lv, (uint32_t *)(lds + L.scl), rt);   // (uniform)
        } else if (ctx.l == 0) {
            route_finish<C>(a, lv, rt);
        }
    }
    __builtin_amdgcn_s_waitcnt(VMCNT0);
    ctx.st.mark(1);

    const uint64_t rb = NB * 144;
    const uint8_t *gb, *ub;
    if ((int)slot < a.n_sel) {
        int32_t id = __builtin_amdgcn_readlane(rt.eid, (int)slot);
        if ((uint32_t)id >= a.n_expert) id = 0;   // bad explicit id: reported by route_publish
        gb = a.gate + (uint64_t)id * a.ffn * rb;
        ub = a.up + (uint64_t)id * a.ffn * rb;
    } else {
        gb = a.gate_sh;
        ub = a.up_sh;
    }
    auto row_ptr = [&](uint32_t v) -> const uint8_t * {   // v < R (clamped past it)
        v = min(v, (uint32_t)R - 1);
        if (v < (uint32_t)IW) return gb + (uint64_t)(IW * li + v) * rb;
        return ub + (uint64_t)(IW * li + v - IW) * rb;
    };
    auto chunk = [&](int k) -> const uint8_t * {
        uint32_t r, it;
        if constexpr (ITEMS >= 64) {
            r = k / M;
            it = 64 * (k % M) + lane;
        } else {
            r = lane / ITEMS + k * (64 / ITEMS);
            it = lane % ITEMS;
        }
        return row_ptr(RW * wave + r) + (it / 8) * 144 + 16 + 16 * (it % 8);
    };

    uint4 hv[HPL];
    uint4 q[LPG];
    if (rows) {   // whole waves
#pragma unroll
        for (int i = 0; i < HPL; i++) {
            const uint32_t h = min(lane + 64 * i, (uint32_t)WH - 1);
            hv[i] = ld16(row_ptr(RW * wave + h / NB) + (h % NB) * 144);
        }
#pragma unroll
        for (int k = 0; k < LPG; k++) q[k] = ld16(chunk(k));
    }
    ctx.st.mark(2);
    if (slot == 0 && li == 0 && wave == 0)
        route_publish(a, rt.eid, (NORMED || a.logits) && a.n_sel > 0 ? route_weight(rt.logit, a.n_sel) : rt.w);

    // x -> q8_1 in LDS while the weights stream in
    const Act xa = act_carve(lds + L.xact, a.hidden);
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const uint32_t t = tid + NT * i, blk = t >> 3, part = t & 7;
        if (t >= (uint32_t)XTASKS) break;   // whole 8-lane groups leave together
        uint32_t qv;
        int lo, hi;
        float dd;
        if (a.xq) {
            qv = xqv[i];
            q8_part_sums(qv, lo, hi);
            dd = h2f(xdv[i]);
        } else {
            uint32_t d16, s16;
            qv = quant_q8_1_part(xv[i], d16, s16, lo, hi, dd);
        }
        *(uint32_t *)(xa.qs + 32 * blk + 4 * part) = qv;
        if (part == 0) {
            xa.d8[blk] = dd;
            xa.qs16[2 * blk] = lo;
            xa.qs16[2 * blk + 1] = hi;
        }
    }
    __syncthreads();
    ctx.st.mark(3);

    float *gu = (float *)(lds + L.gu);
    if (rows) {
        XSlice xs[M];
#pragma unroll
        for (int m = 0; m < M; m++) xs[m] = x_slice(xa, ITEMS >= 64 ? 64 * m + lane : lane % ITEMS);
        float4 *scl = (float4 *)(lds + L.scl) + 4 * WH * wave;
#pragma unroll
        for (int i = 0; i < HPL; i++) {
            const uint32_t h = lane + 64 * i;
            if (h < WH) {
                Q4K::Raw raw;
                raw.h = hv[i];
                const uint32_t b = h % NB;
                const float4 dA = *(const float4 *)(xa.d8 + 8 * b), dB = *(const float4 *)(xa.d8 + 8 * b + 4);
                const float d8[8] = {dA.x, dA.y, dA.z, dA.w, dB.x, dB.y, dB.z, dB.w};
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    float ds0, ds1, dm0, dm1;
                    Q4K::scales(raw, g, ds0, ds1, dm0, dm1);
                    scl[4 * h + g] = make_float4(ds0 * d8[2 * g], ds1 * d8[2 * g + 1], dm0 * d8[2 * g], dm1 * d8[2 * g + 1]);
                }
            }
        }
        wave_sync_lds();
        if constexpr (ITEMS >= 64) {
            float acc[LPG];
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t it = 64 * (k % M) + lane;
                const uint32_t row = k / M;
                const float4 sc = scl[4 * (row * NB + it / 8) + (it % 8) / 2];
                acc[k] = q4k_term(q[k], sc, xs[k % M]);
            }
            const float v = pw_rows<LPG, M>(acc);
            const uint32_t row = RW * wave + pw_rows_row<LPG, M>(lane);
            if (lane < (uint32_t)RW && row < (uint32_t)R) gu[row] = v;
        } else {
            const uint32_t it = lane % ITEMS;
#pragma unroll
            for (int k = 0; k < LPG; k++) {
                const uint32_t row = lane / ITEMS + k * (64 / ITEMS);
                const float4 sc = scl[4 * (row * NB + it / 8) + (it % 8) / 2];
                const float v = group_sum<ITEMS>(q4k_term(q[k], sc, xs[0]));
                if (it == 0 && RW * wave + row < (uint32_t)R) gu[RW * wave + row] = v;
            }
        }
    }
    ctx.st.mark(4);
    down();   // behind this wave's gate/up loads in the CU's queue
    sh_late(xa, gen + 1);   // (the shared wave: no rows of the slot's)
    ctx.st.mark(5);
    __syncthreads();
    if (a.dbg_gu && tid < (uint32_t)R)
        a.dbg_gu[(uint64_t)slot * 2 * a.ffn + (tid < (uint32_t)IW ? 0 : a.ffn) + IW * li + tid % IW] = gu[tid];
}

// SH: eight routed slots plus the shared expert (XcdShared): its h values
// come from all 256 workgroups and are exchanged across the XCDs, long
// before the slots' h is complete; the pollers stage the whole shared h
// with the slot's, and wave 0 adds each row's shared partial after the
// eight slots, weight 1 (the shared expert enters last, as in kernel B).
// A group of GT threads (whole waves; thread pt of the group) polls nw
// tagged words, word pt + GT i on thread pt (word(e) its address), until
// every one carries tag, then stages them as q8_1 blocks in dst with kernel
// A's quantizer (32 lanes hold one block) and, with hq, writes the blocks
// there as kernel A writes them. Two rounds in flight: the next round goes
// out before the previous one is checked, so a word is sampled twice per
// round trip (ROUNDS 2; with ROUNDS 1 one round at a time, half the poll
// traffic). A word already seen is kept, and its lane's later loads read
// `rest` instead (one line per wave instruction, the value dropped), so late
// rounds fetch only what is still missing while the down rows stream. The
// loads themselves are unconditional, so both rounds stay countable in
// flight; va and vb hold the rounds (the caller keeps them allocated to its
// end: a round is still in flight when the words are complete).
template <int NW, uint32_t GT, bool STK, int ROUNDS, class Word>
__device__ __forceinline__ void poll_stage(const MoeArgs &a, uint32_t pt, uint32_t nw, Word word, uint32_t *rest,
                                           uint32_t tag, const Act &dst, uint8_t *hq, uint32_t &spins,
                                           uint64_t (&va)[NW], uint64_t (&vb)[NW]) {
    const uint32_t lane = threadIdx.x & 63;
    uint64_t hv[NW];
#pragma unroll
    for (int i = 0; i < NW; i++) hv[i] = 0;   // (words past nw: never seen, quantized and dropped)
    uint32_t need = 0;   // bit i: word pt + GT i still to see
#pragma unroll
    for (int i = 0; i < NW; i++)
        if (pt + GT * i < nw) need |= 1u << i;
    auto issue = [&](uint64_t *o) {
#pragma unroll
        for (int i = 0; i < NW; i++) o[i] = ld_dev2(((need >> i) & 1) ? word(pt + GT * i) : rest);
    };
    auto take = [&](const uint64_t *o) {   // true once every word of the wave is in
#pragma unroll
        for (int i = 0; i < NW; i++) {
            if (((need >> i) & 1) && (uint32_t)(o[i] >> 32) == tag) {
                hv[i] = o[i];
                need &= ~(1u << i);
            }
        }
        return __all(need == 0);
    };
    issue(va);
    for (;;) {
        if constexpr (ROUNDS == 2) {
            issue(vb);
            if (take(va)) break;
            issue(va);
            if (take(vb)) break;
        } else {
            if (take(va)) break;
            issue(va);
        }
        if (++spins >= FSYNC_SPIN_LIMIT / ROUNDS || (STK && stack_expired(a, spins))) {
            if (lane == 0) atomicOr(a.err, 4);
            break;
        }
    }
    // kernel A's quantizer on every word first, with no store between them
    // (the NW words' dependency chains interleave; one wave per SIMD runs
    // this, so it is latency-bound), then the stores
    float dq[NW];
    int qq[NW], tq[NW], sq[NW];
    uint32_t d16q[NW];
#pragma unroll
    for (int i = 0; i < NW; i++) {
        const float h = __uint_as_float((uint32_t)hv[i]);
        const float am = max32(fabsf(h));
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const int qv = (int)roundf(h * id);
        int s16 = qv;   // the 16-value half-block sum: a 16-lane row of DPP
        s16 += dpp_i<DPP_XOR1>(s16);
        s16 += dpp_i<DPP_XOR2>(s16);
        s16 += dpp_i<DPP_HALF_MIRROR>(s16);
        s16 += dpp_i<DPP_MIRROR>(s16);
        dq[i] = d;
        qq[i] = qv;
        tq[i] = sum32(qv);
        sq[i] = s16;
        d16q[i] = f2h_rne(d);
    }
#pragma unroll
    for (int i = 0; i < NW; i++) {
        const uint32_t e = pt + GT * i;   // its 32-lane half is one block
        if (e < nw) {                     // whole 32-lane halves (nw a multiple of 32)
            const float d = dq[i];
            const int qv = qq[i], total = tq[i], s16 = sq[i];
            const uint32_t d16 = d16q[i];
            const uint32_t kb = e / 32, j = e % 32;
            dst.qs[e] = (int8_t)qv;
            if (j == 0) dst.d8[kb] = h2f(d16);
            if ((j & 15) == 0) dst.qs16[2 * kb + j / 16] = s16;
            if (hq) {
                uint8_t *blk = hq + (uint64_t)kb * 36;
                blk[4 + j] = (uint8_t)(qv & 255);
                if (j == 0) *(uint32_t *)blk = d16 | (f2h_rne((float)total * d) << 16);
            }
        }
    }
}

// The body of one layer: k_moe_xcd runs it once; k_moe_stack runs it per
// layer of a stack (STK, ctx), with that layer's tag gen + 1 + ctx.l; the
// generation words advance by n_layers at the stack's last layer.
template <int NB, int C, class QD, int S, int IPL, int IW, bool SH, bool NORMED, bool STK>
__device__ __forceinline__ void xcd_body(const MoeArgs &a, uint32_t gen, uint32_t n_layers, StkCtx &ctx) {
    constexpr uint32_t NT = a1_threads<NB>();
    constexpr uint32_t P = S / QD::IPB;
    constexpr uint32_t H = 256 * NB;
    constexpr uint32_t F = 32 * IW;               // ffn
    constexpr uint32_t PER = XCD_G / XCD_SLOTS;   // workgroups per slot
    constexpr uint32_t TRX = H / PER;             // down rows per workgroup
    constexpr uint32_t TRC = TRX / XCD_SLOTS;     // rows each workgroup sums
    constexpr uint32_t NBK = F / 256;             // blocks per down row
    static_assert(S * TRX <= NT && TRC >= 1 && XCD_SLOTS * TRC <= 64, "XCD layer tile");
    static_assert(!SH || (!NORMED && (2 * IW + 3) / 4 <= 8 && F <= XCD_MAX_SH_FFN && H <= XCD_MAX_HIDDEN),
                  "XCD layer shared expert: plain layers, rows below wave 8, its exchange areas");
    static_assert(F <= XCD_HW * 64 * XCD_POLL_WAVES && F % 256 == 0, "XCD layer ffn");
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t tid = STK ? opaque_v(threadIdx.x) : threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t b = STK ? opaque_s(blockIdx.x) : blockIdx.x, xs = b % XCD_SLOTS, li = b / XCD_SLOTS;
    pin_args(a.down, a.down_sh, a.y, a.fsync, a.hq8);
    uint32_t *gw = a.fsync + FSYNC_X + b;
    ctx.st.begin();

    // the down share: row r = tid / S of the tile, lane s = tid % S
    const uint32_t s = tid % S, r = tid / S;
    const uint32_t item = s % QD::IPB, bs = s / QD::IPB;
    const uint32_t row0 = li * TRX, rr = min(r, TRX - 1);   // idle threads load a real row and drop it
    constexpr uint64_t rbd = (uint64_t)NBK * QD::BB;
    typename QD::Raw raw[IPL];
    GuRoute rt;
    // the shared expert's registers (SH): gate/up rows on its gate/up wave,
    // down items on its down waves
    constexpr int SHPL = (4 * NB + 63) / 64, SLPG = NB / 2;
    uint4 shv[SHPL], shq[SLPG];
    typename QD::Raw shr;
    typename QD::Unp shu;
    auto sh_start = [&]() {   // the single layer: its loads ahead of the routing's
        if constexpr (SH) {
            const XcdShared<NB, QD, S, IW> sh{b, xs, li, tid, lane, wave};
            sh.issue_gu(a, shv, shq);
            sh.issue_down(a, shr);
        }
    };
    auto sh_late = [&](const Act &xa, uint32_t tg) {
        if constexpr (SH) {
            const XcdShared<NB, QD, S, IW> sh{b, xs, li, tid, lane, wave};
            if (wave == XcdShared<NB, QD, S, IW>::SW) {
                if constexpr (STK) sh.issue_gu(a, shv, shq);
                sh.dots(a, lds, xa, tg, shv, shq);
            }
        }
    };
    auto load_down = [&]() {
        int32_t sid = __builtin_amdgcn_readlane(rt.eid, (int)xs);
        if ((uint32_t)sid >= a.n_expert) sid = 0;   // bad explicit id: reported by route_publish
        const uint8_t *rp = ((int)xs < a.n_sel ? a.down + (uint64_t)sid * H * rbd : a.down_sh) +
                            (uint64_t)(row0 + rr) * rbd;
#pragma unroll
        for (int i = 0; i < IPL; i++) raw[i] = QD::load(rp + min(bs + P * i, NBK - 1) * QD::BB, (int)item);
        if constexpr (SH && STK) XcdShared<NB, QD, S, IW>{b, xs, li, tid, lane, wave}.issue_down(a, shr);
    };
    gu_part<NB, C, IW, decltype(load_down), decltype(sh_start), decltype(sh_late), NORMED, STK>(
        a, xs, li, lds, rt, load_down, sh_start, sh_late, gen + ctx.l, ctx);

    uint32_t tag = gen + ctx.l;
    asm volatile("" : "+v"(tag));
    tag += 1;
    uint32_t *hx = a.fsync + FSYNC_XH + 2 * F * xs;    // slot xs's h words
    uint32_t *hxs = a.fsync + FSYNC_XS;                   // the shared expert's (SH)
    if (wave == 0) {
        const float *gu = (const float *)(lds + lds_a(a.hidden, NB).gu);
        // The h words are read only by the slot's own workgroups, which
        // share one XCD (a.hloc: the dispatch was checked for that): then
        // the words stay in that XCD's L2, else they are written through.
        const bool own_xcd = a.hloc != 0;
        if (lane < (uint32_t)IW) {
            const float h = kq_silu_mul(gu[lane], gu[IW + lane]);
            const uint64_t v = ((uint64_t)tag << 32) | __float_as_uint(h);
            if (own_xcd) st_xcd2(hx + 2 * (IW * li + lane), v);
            else st_dev2(hx + 2 * (IW * li + lane), v);
        }
        ctx.st.mark(6);
    }

    // 3. the h words, quantized as q8_1 blocks in LDS: the slot's by the
    //    pollers, the shared expert's (SH) by waves 8 to 11 (poll_stage)
    uint32_t spins = 0;
    constexpr uint32_t first_poller = NT - 64 * XCD_POLL_WAVES;
    const bool poller = tid >= first_poller;   // whole waves
    const uint32_t LT = lds_a(a.hidden, NB).total;
    const Act act = act_carve(lds + LT, F);
    const Act actS = act_carve(lds + LT + act_bytes(F), F);   // SH only: the shared expert's blocks
    // Every wave unpacks its down items here, while h is awaited (the
    // pollers before their first poll), so only the dot products and the
    // scales follow h. After that no wave waits on a load: the pollers'
    // last round is still in flight when h is complete, and a wait on any
    // older load would wait on it too (the load counter retires in issue
    // order), about 0.6 us on the layer's critical path. For the same reason
    // the poll rounds' registers stay allocated to the pollers' end (an
    // empty use there), so nothing after the loop reuses a register that
    // round still loads into.
    typename QD::Unp un[IPL];
#pragma unroll
    for (int i = 0; i < IPL; i++) {
        un[i] = QD::unpack(raw[i]);
        pin_vregs(raw[i]);
        pin_vregs(un[i]);
    }
    if constexpr (SH) {   // (threads past the shared down waves: unused)
        shu = QD::unpack(shr);
        pin_vregs(shr);
        pin_vregs(shu);
    }
    constexpr uint32_t GT = 64 * XCD_POLL_WAVES;
    constexpr int NW = (F + GT - 1) / GT;             // the slot's words per poller
    constexpr int NWS = SH ? (F + GT - 1) / GT : 1;   // the shared expert's per shared poller (waves 8 to 11)
    uint64_t va[NW], vb[NW], sva[NWS], svb[NWS];
#pragma unroll
    for (int i = 0; i < NW; i++) va[i] = vb[i] = 0;
#pragma unroll
    for (int i = 0; i < NWS; i++) sva[i] = svb[i] = 0;
    // the shared h, published long before the slot's, by the four waves
    // below the pollers (no gate/up rows of the slot's there: GW <= 8)
    const bool spoller = SH && wave >= 8 && wave < 12;
    if (poller) {
        const uint32_t pt = tid - first_poller;
        // (only words e < F are ever asked for; the other arm keeps this
        // loop's code as it is measured)
        auto word = [&](uint32_t e) { return e < F ? hx + 2 * e : hxs + 2 * (e - F); };
        // Two rounds in flight: the next round goes out before the previous
        // one is checked, so a word is sampled twice per round trip. A word
        // already seen with this call's tag is kept, and its lane's later
        // loads read the slot's first word instead (one line per wave
        // instruction, the value dropped), so late rounds fetch only what
        // is still missing while the down rows stream. The loads themselves
        // are unconditional, so both rounds stay countable in flight.
        // (poll_stage is the same loop for the shared pollers; written out
        // here, the slot's loop keeps the registers of its rounds in place.)
        uint64_t hv[NW];
#pragma unroll
        for (int i = 0; i < NW; i++) hv[i] = 0;   // (words past F: never seen, quantized and dropped)
        uint32_t need = 0;   // bit i: word pt + 256 i still to see
#pragma unroll
        for (int i = 0; i < NW; i++)
            if (pt + GT * i < F) need |= 1u << i;
        auto issue = [&](uint64_t *o) {
#pragma unroll
            for (int i = 0; i < NW; i++) o[i] = ld_dev2(((need >> i) & 1) ? word(pt + GT * i) : hx);
        };
        auto take = [&](const uint64_t *o) {   // true once every word of the wave is in
#pragma unroll
            for (int i = 0; i < NW; i++) {
                if (((need >> i) & 1) && (uint32_t)(o[i] >> 32) == tag) {
                    hv[i] = o[i];
                    need &= ~(1u << i);
                }
            }
            return __all(need == 0);
        };
        ctx.st.mark(7);
        issue(va);
        for (;;) {
            issue(vb);
            if (take(va)) break;
            issue(va);
            if (take(vb)) break;
            if (++spins >= FSYNC_SPIN_LIMIT / 2 || (STK && stack_expired(a, spins))) {
                if (lane == 0) atomicOr(a.err, 4);
                break;
            }
        }
        ctx.st.mark(8);
        // kernel A's quantizer on every word first, with no store between
        // them (the NW words' dependency chains interleave; one wave per SIMD
        // runs this, so it is latency-bound), then the stores
        float dq[NW];
        int qq[NW], tq[NW], sq[NW];
        uint32_t d16q[NW];
#pragma unroll
        for (int i = 0; i < NW; i++) {
            const float h = __uint_as_float((uint32_t)hv[i]);
            const float am = max32(fabsf(h));
            const float d = am / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const int qv = (int)roundf(h * id);
            int s16 = qv;   // the 16-value half-block sum: a 16-lane row of DPP
            s16 += dpp_i<DPP_XOR1>(s16);
            s16 += dpp_i<DPP_XOR2>(s16);
            s16 += dpp_i<DPP_HALF_MIRROR>(s16);
            s16 += dpp_i<DPP_MIRROR>(s16);
            dq[i] = d;
            qq[i] = qv;
            tq[i] = sum32(qv);
            sq[i] = s16;
            d16q[i] = f2h_rne(d);
        }
#pragma unroll
        for (int i = 0; i < NW; i++) {
            const uint32_t e = pt + GT * i;   // its 32-lane half is one block
            if (e < F) {                      // whole 32-lane halves (F a multiple of 32)
                const float d = dq[i];
                const int qv = qq[i], total = tq[i], s16 = sq[i];
                const uint32_t d16 = d16q[i];
                const uint32_t kb = e / 32, j = e % 32;
                act.qs[e] = (int8_t)qv;
                if (j == 0) act.d8[kb] = h2f(d16);
                if ((j & 15) == 0) act.qs16[2 * kb + j / 16] = s16;
                if (li == 0) {   // the q8_1 blocks of h, as kernel A writes them
                    uint8_t *blk = a.hq8 + ((uint64_t)xs * (F / 32) + kb) * 36;
                    blk[4 + j] = (uint8_t)(qv & 255);
                    if (j == 0) *(uint32_t *)blk = d16 | (f2h_rne((float)total * d) << 16);
                }
            }
        }
    } else if (spoller) {   // (the shared expert is slot n_sel)
        poll_stage<NWS, GT, STK, 1>(a, tid - 512, F, [&](uint32_t e) { return hxs + 2 * e; }, hx, tag, actS,
                                  li == 0 && xs == 0 ? a.hq8 + (uint64_t)a.n_sel * (F / 32) * 36 : nullptr, spins,
                                  sva, svb);
    }
    __syncthreads();
    ctx.st.mark(9);

    // the tile's unweighted down partials (and, with SH, the shared rows')
    float x = 0.0f;
#pragma unroll
    for (int i = 0; i < IPL; i++) {
        const uint32_t blk = bs + P * i;
        const float d = QD::dot_q8_u(raw[i], un[i], (int)item, act, min(blk, NBK - 1));
        x += blk < NBK ? d : 0.0f;
    }
    x = group_sum<S>(x);
    if (r < TRX && s == 0)
        st_dev2(a.fsync + FSYNC_XP + 2 * (xs * H + row0 + r), ((uint64_t)tag << 32) | __float_as_uint(x));
    ctx.st.mark(10);
    if constexpr (SH) {
        using XS = XcdShared<NB, QD, S, IW>;
        const XS sh{b, xs, li, tid, lane, wave};
        if (sh.down_wave()) {   // whole waves
            const uint32_t bk = sh.bslot();
            const float d = QD::dot_q8_u(shr, shu, (int)sh.item(), actS, min(bk, NBK - 1));
            const float xsh = group_sum<S>(bk < NBK ? d : 0.0f);
            if (tid - 64 * XS::SD < XS::RSW * S && (tid - 64 * XS::SD) % S == 0)
                st_dev2(a.fsync + FSYNC_XSP + 2 * sh.row(), ((uint64_t)tag << 32) | __float_as_uint(xsh));
        }
    }

    // 4. wave 0: rows row0 + xs * TRC + c (c < TRC) over the eight slots, then
    //    the shared expert's partial
    if (wave == 0) {
        float rw = (NORMED || a.logits) && a.n_sel > 0 ? route_weight(rt.logit, a.n_sel) : rt.w;
        rw = (int)lane < a.n_sel ? rw : ((int)lane == a.n_sel && a.has_shared ? 1.0f : 0.0f);
        if (lane == 0 && ctx.l + 1 == n_layers) st_dev(gw, tag);   // gen was read at the start: advance it now
        const uint32_t q = lane / TRC, c = lane % TRC;   // lane: slot (or unit) q, row c
        const uint32_t yr = row0 + xs * TRC + c;
        uint32_t *pw = a.fsync + FSYNC_XP + 2 * (min(q, XCD_SLOTS - 1) * H + yr);
        uint32_t *pws = a.fsync + FSYNC_XSP + 2 * yr;   // lanes c < TRC: the shared partial of row yr
        auto ok = [&](uint64_t v, uint64_t vs) {
            return __all((lane >= XCD_SLOTS * TRC || (uint32_t)(v >> 32) == tag) &&
                         (!SH || lane >= TRC || (uint32_t)(vs >> 32) == tag));
        };
        // One round in flight: a wave ends only once its loads are back, so
        // a second round still in flight when the partials are complete
        // would hold the workgroup, and the layer, one more round trip.
        uint64_t pv, sv = 0;
        for (;;) {
            pv = ld_dev2(pw);
            if constexpr (SH) sv = ld_dev2(pws);
            if (ok(pv, sv)) break;
            if (++spins >= FSYNC_SPIN_LIMIT || (STK && stack_expired(a, spins))) {
                if (lane == 0) atomicOr(a.err, 4);
                break;
            }
        }
        ctx.st.mark(11);
        const float v = __uint_as_float((uint32_t)pv);
        float y = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < XCD_SLOTS; k++) {   // rank order, one fmaf per slot
            const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rw), (int)k));
            y = fmaf(w, __shfl(v, (int)(k * TRC + c), WAVE), y);
        }
        if constexpr (SH) {
            const float vs = __uint_as_float((uint32_t)sv);
            y = fmaf(1.0f, __shfl(vs, (int)c, WAVE), y);   // the shared expert, last
        }
        if constexpr (STK) {   // the next layer's x (or delta) as tagged words
            if (lane < TRC && ctx.l + 1 < n_layers)
                st_dev2(a.fsync + FSYNC_XY + 2 * ((ctx.l & 1) * XCD_MAX_HIDDEN + row0 + xs * TRC + lane),
                        ((uint64_t)tag << 32) | __float_as_uint(y));
        }
        if (lane < TRC) a.y[row0 + xs * TRC + lane] = y;
        if constexpr (STK) {
            // this workgroup's y is stored (the stores acknowledged): its
            // completion word, which the next layer's weight loads wait for
            if (ctx.l + 1 < n_layers) {
                __builtin_amdgcn_s_waitcnt(VMCNT0);
                if (lane == 0) st_dev(a.fsync + FSYNC_XF + (ctx.l & 1) * XCD_G + b, tag);
            }
        }
        ctx.st.mark(12);
    }
    if (poller) {
#pragma unroll
        for (int i = 0; i < NW; i++) asm volatile("" ::"v"(va[i]), "v"(vb[i]));
    } else if (spoller) {
#pragma unroll
        for (int i = 0; i < NWS; i++) asm volatile("" ::"v"(sva[i]), "v"(svb[i]));
    }
    ctx.st.store(tag, b, tid, first_poller);
}

template <int NB, int C, class QD, int S, int IPL, int IW, bool SH, bool NORMED>
__global__ void __launch_bounds__(a1_threads<NB>()) k_moe_xcd(MoeArgs a) {
    const uint32_t gen = ld_dev(a.fsync + FSYNC_X + blockIdx.x);   // issued first, used last
    StkCtx ctx{};
    xcd_body<NB, C, QD, S, IPL, IW, SH, NORMED, false>(a, gen, 1, ctx);
}

// The stacked layer: n_layers layers of one shape in one launch (the XCD
// layer's workgroups stay resident from layer to layer, so no launch gap
// separates them). Layer l takes its weights, routing and outputs from
// lt[l]. Plain: layer 0's x is a.x (or a.xq), layer l's is its own lt[l].x
// or, when that is null, layer l - 1's y.
// NORMED: layer 0's residual step reads a.nx (and a.ndelta), layer l's adds
// layer l - 1's y to the residual stream, then the norm, the router and the
// layer as the normed layer runs them. A layer waits for the whole of the
// previous layer's y before any weight load of its own; only what does not
// depend on that y (its routing from given logits, its router rows and norm
// weights) is read before.
template <int NB, int C, class QD, int S, int IPL, int IW, bool SH, bool NORMED>
__global__ void __launch_bounds__(a1_threads<NB>()) k_moe_stack(MoeArgs a0, const StackLayer *__restrict__ lt, uint32_t n_layers) {
    const uint32_t gen = ld_dev(a0.fsync + FSYNC_X + blockIdx.x);
    StkCtx ctx{};
    for (uint32_t l = 0; l < n_layers; l++) {
        const StackLayer &L = lt[l];
        MoeArgs a = a0;
        a.gate = L.gate;
        a.up = L.up;
        a.down = L.down;
        a.gate_sh = L.gate_sh;
        a.up_sh = L.up_sh;
        a.down_sh = L.down_sh;
        a.ids_out = L.ids_out;
        a.wts_out = L.wts_out;
        a.y = L.y;
        if constexpr (NORMED) {
            a.nw = L.nw;
            a.router = L.router;
            a.nx_out = L.x_out;
            a.nxn_out = L.xn_out;
            a.logits_out = L.logits_out;
        } else {
            a.logits = L.logits;
            a.step = L.step;
            a.logits_stride = L.logits_stride;
            a.ids = L.ids;
            a.wts = L.wts;
        }
        if (l > 0) {
            a.x = NORMED ? nullptr : L.x;   // plain: the layer's own x, or (null) the previous layer's y
            a.xq = nullptr;
            a.nx = nullptr;
            a.ndelta = nullptr;
        }
        ctx.l = l;
        ctx.ytag = gen + l;   // layer l - 1's tag
        ctx.yw = a0.fsync + FSYNC_XY + 2 * (((l + 1) & 1) * XCD_MAX_HIDDEN);
        ctx.yf = a0.fsync + FSYNC_XF + ((l + 1) & 1) * XCD_G;
        xcd_body<NB, C, QD, S, IPL, IW, SH, NORMED, true>(a, gen, n_layers, ctx);
    }
}

// Whether every workgroup of kernel k (XCD_G workgroups of nt threads, lds
// bytes of LDS) can be resident at once on this device: the one-launch
// layers' workgroups wait for each other, so they may run only then. Asked
// of the occupancy API once per kernel and LDS size.
static bool all_resident(const void *k, uint32_t nt, uint32_t lds) {
    static thread_local const void *last_k = nullptr;
    static thread_local uint32_t last_lds = 0;
    static thread_local int last_dev = -1, last_n = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    if (k != last_k || lds != last_lds || dev != last_dev) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, (int)nt, (size_t)lds) != hipSuccess) n = 0;
        last_k = k;
        last_lds = lds;
        last_dev = dev;
        last_n = n;
    }
    return xcd_coresident(device_cu_count(), last_n, XCD_G);
}

// lt: the stacked layer's per-layer table (nl layers), else the single layer
template <int NB, int C, class QD, int S, int IPL, int IW, bool SH, bool NORMED>
static hipError_t go_xcd(const MoeArgs &a, hipStream_t s, const StackLayer *lt, uint32_t nl) {
    uint32_t lds = lds_a(a.hidden, NB).total + (SH ? 2 : 1) * act_bytes(32 * IW);   // (SH: the shared h blocks)
    // the normed prologue's area starts at the scale records, which are
    // written only after its last read
    if (NORMED) lds = max(lds, lds_a(a.hidden, NB).scl + normed_area_bytes(a.hidden));
    // The stack at hidden 1024 with 256 experts and the shared expert does
    // not fit the registers (it would need scratch): those stacks run layer
    // by layer.
    constexpr bool STACK = !(SH && NB == 4 && C == 4);
    if (lt && !STACK) return hipErrorNotSupported;
    const void *k = (const void *)k_moe_xcd<NB, C, QD, S, IPL, IW, SH, NORMED>;
    if constexpr (STACK) {
        if (lt) k = (const void *)k_moe_stack<NB, C, QD, S, IPL, IW, SH, NORMED>;
    }
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    if (!all_resident(k, a1_threads<NB>(), lds)) return hipErrorNotSupported;
    if constexpr (STACK) {
        if (lt) {
            hipLaunchKernelGGL((k_moe_stack<NB, C, QD, S, IPL, IW, SH, NORMED>), dim3(XCD_G), dim3(a1_threads<NB>()),
                               lds, s, a, lt, nl);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((k_moe_xcd<NB, C, QD, S, IPL, IW, SH, NORMED>), dim3(XCD_G), dim3(a1_threads<NB>()), lds, s, a);
    return hipGetLastError();
}
// 16 lanes per down row: Q6_K 4 items x 4 block slots (ffn <= 1024: one
// block per lane), Q4_K 8 items x 2 block slots (up to two)
template <int NB, int C, int IW, bool SH, bool NORMED>
static hipError_t go_xcd_q(const MoeArgs &a, hipStream_t s, const StackLayer *lt, uint32_t nl) {
    if (a.down_type == T_Q6_K) return go_xcd<NB, C, Q6K, 16, 1, IW, SH, NORMED>(a, s, lt, nl);
    if constexpr (IW <= 16) return go_xcd<NB, C, Q4K, 16, 1, IW, SH, NORMED>(a, s, lt, nl);
    else return go_xcd<NB, C, Q4K, 16, 2, IW, SH, NORMED>(a, s, lt, nl);
}
template <int NB, int C, bool SH, bool NORMED>
static hipError_t go_xcd_f(const MoeArgs &a, hipStream_t s, const StackLayer *lt, uint32_t nl) {
    switch (a.ffn) {
        case 256: return go_xcd_q<NB, C, 8, SH, NORMED>(a, s, lt, nl);
        case 512: return go_xcd_q<NB, C, 16, SH, NORMED>(a, s, lt, nl);
        case 768:
            if constexpr (!SH) return go_xcd_q<NB, C, 24, SH, NORMED>(a, s, lt, nl);   // the shared gate/up rows must fit one wave
            else return hipErrorNotSupported;
        case 1024:
            if constexpr (!SH) return go_xcd_q<NB, C, 32, SH, NORMED>(a, s, lt, nl);   // shared rows would not fit 64 per workgroup
            else return hipErrorNotSupported;
        default: return hipErrorNotSupported;
    }
}
template <int NB, bool SH, bool NORMED = false>
static hipError_t go_xcd_c(const MoeArgs &a, hipStream_t s, const StackLayer *lt = nullptr, uint32_t nl = 0) {
    return a.n_expert <= 128 ? go_xcd_f<NB, 2, SH, NORMED>(a, s, lt, nl) : go_xcd_f<NB, 4, SH, NORMED>(a, s, lt, nl);
}
// hipErrorNotSupported when the shape does not fit the XCD-sliced layer:
// eight slots (one per XCD), or with shared_units eight routed experts plus
// the shared expert (ffn 256 or 512 then; XcdShared), hidden 1024 or
// 2048, ffn <= 1024, <= 256 experts, a 256-CU device on which every
// workgroup can be resident at once, and the one-launch layers not turned
// off after an expired wait (xcd_disable)
static hipError_t launch_moe_xcd(const MoeArgs &a0, uint32_t n_slots, bool shared_units, hipStream_t s,
                                 const StackLayer *lt = nullptr, uint32_t nl = 0) {
    MoeArgs a = a0;
    a.hloc = xcd_local() ? 1u : 0u;
    const uint32_t nb = a.hidden / 256;
    const bool spread = shared_units && a.n_sel == (int)XCD_SLOTS && a.has_shared;
    if (!a.fsync || xcd_disabled() || !(n_slots == XCD_SLOTS || spread) || a.n_sel < 1 || !(nb == 4 || nb == 8) ||
        a.n_expert > 256 || a.ffn > 1024 || (spread && a.ffn > 512) || device_cu_count() != (int)XCD_G)
        return hipErrorNotSupported;
    if (spread) return nb == 8 ? go_xcd_c<8, true>(a, s, lt, nl) : go_xcd_c<4, true>(a, s, lt, nl);
    return nb == 8 ? go_xcd_c<8, false>(a, s, lt, nl) : go_xcd_c<4, false>(a, s, lt, nl);
}

// The phase stamps (the measurement build), as kq_stamps holds them.
hipError_t read_stamps(void *host, size_t bytes) {
#ifdef KQ_STAMPS
    const size_t n = sizeof(uint64_t) * STAMP_LAYERS * 256 * STAMP_PHASES;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(kq_stamps), bytes < n ? bytes : n, 0, hipMemcpyDeviceToHost);
#else
    (void)host;
    (void)bytes;
    return hipErrorNotSupported;
#endif
}

static bool g_xcd_off = false;
void xcd_disable() { g_xcd_off = true; }
void xcd_enable() { g_xcd_off = false; }
bool xcd_disabled() { return g_xcd_off; }

// The XCD-local hand-off of the h words (st_xcd2) needs every workgroup b
// with one b % 8 on one XCD. The dispatcher deals a launch's workgroups to
// the eight XCDs round robin, starting at an XCD that depends on the queue
// (measured: workgroup b on XCD (b + k) % 8, k fixed per hardware queue, for
// every workgroup of every launch). xcd_dispatch_check launches XCD_G
// workgroups of the layer's size four times and keeps the hand-off on only
// if each launch shows one k for all of them; otherwise the h words are
// written through (st_dev2), as the partials are.
static __device__ uint32_t xcc_seen[4 * XCD_G];
static int g_xcd_local = 0;
__global__ void __launch_bounds__(1024) k_xcc_map(uint32_t *out) {
    if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}
hipError_t xcd_dispatch_check(hipStream_t s) {
    uint32_t *dev = nullptr;
    hipError_t e = hipGetSymbolAddress((void **)&dev, HIP_SYMBOL(xcc_seen));
    for (int r = 0; r < 4 && e == hipSuccess; r++) {
        hipLaunchKernelGGL(k_xcc_map, dim3(XCD_G), dim3(1024), 0, s, dev + r * XCD_G);
        e = hipGetLastError();
    }
    uint32_t h[4 * XCD_G];
    if (e == hipSuccess) e = hipMemcpyAsync(h, dev, sizeof h, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    bool ok = e == hipSuccess && device_cu_count() == (int)XCD_G;
    for (int r = 0; r < 4 && ok; r++) {
        const uint32_t k = (h[r * XCD_G] + 8) % 8;
        for (uint32_t b = 0; b < XCD_G && ok; b++) ok = h[r * XCD_G + b] < 8 && (h[r * XCD_G + b] + 8 - b % 8) % 8 == k;
    }
    g_xcd_local = ok ? 1 : 0;
    return e;
}
bool xcd_local() { return g_xcd_local != 0; }
void xcd_local_set(bool on) { g_xcd_local = on ? 1 : 0; }

hipError_t launch_moe_stack(const MoeArgs &a, const StackLayer *lt, uint32_t n_layers, bool normed, hipStream_t s) {
    if (!lt || n_layers < 1 || a.n_expert > MAX_EXPERT || a.n_sel > MAX_SEL || a.hidden > XCD_MAX_HIDDEN)
        return hipErrorInvalidValue;
    const uint32_t n_slots = (uint32_t)a.n_sel + (a.has_shared ? 1u : 0u);
    if (!normed) return launch_moe_xcd(a, n_slots, true, s, lt, n_layers);
    const uint32_t nb = a.hidden / 256;
    if (!a.fsync || xcd_disabled() || n_slots != XCD_SLOTS || a.has_shared || !(nb == 4 || nb == 8) ||
        a.n_expert > XCD_G || a.ffn > 1024 || device_cu_count() != (int)XCD_G)
        return hipErrorNotSupported;
    MoeArgs b = a;
    b.hloc = xcd_local() ? 1u : 0u;
    return nb == 8 ? go_xcd_c<8, false, true>(b, s, lt, n_layers) : go_xcd_c<4, false, true>(b, s, lt, n_layers);
}

uint64_t moe_route_words() { return 2 * MAX_SLOTS; }

// KATALI_HIP_HALF_UNITS=0: kernel A keeps whole units on a dense FFN
static bool env_half_off() {
    const char *e = getenv("KATALI_HIP_HALF_UNITS");
    return e && (e[0] == '0' || e[0] == 'n' || e[0] == 'N');
}

template <int NB, bool NORMED = false>
static hipError_t go_a(const MoeArgs &a, uint32_t n_slots, hipStream_t s) {
    const LdsA L = lds_a(a.hidden, NB);
    const uint32_t units = n_slots * (a.ffn / 32);
    const dim3 grid(units);
    uint32_t lds = L.total;
    if (NORMED && L.scl + normed_area_bytes(a.hidden) > lds) lds = L.scl + normed_area_bytes(a.hidden);
    if constexpr (!NORMED && NB >= 8) {   // hidden 2048 and 4096
        if (a.n_sel == 0 && a.fsync && half_units(units, (uint32_t)device_cu_count()) &&
            units <= DH_MAX_BLOCKS && !env_half_off()) {
            hipLaunchKernelGGL((k_moe_gu<NB, 2, false, true>), dim3(2 * units), dim3(a1_threads<NB>()),
                               lds_a(a.hidden, NB, 32).total, s, a);
            return hipGetLastError();
        }
    }
    if (a.n_expert <= 128)
        hipLaunchKernelGGL((k_moe_gu<NB, 2, NORMED>), grid, dim3(a1_threads<NB>()), lds, s, a);
    else if (a.n_expert <= 256)
        hipLaunchKernelGGL((k_moe_gu<NB, 4, NORMED>), grid, dim3(a1_threads<NB>()), lds, s, a);
    else
        hipLaunchKernelGGL((k_moe_gu<NB, 8, NORMED>), grid, dim3(a1_threads<NB>()), lds, s, a);
    return hipGetLastError();
}

// Kernel B's tile: TR output rows x n_slots pairs per workgroup of 256
// threads, S = IPB * P lanes per pair.
template <class QD>
static uint32_t b_tile_rows(uint32_t P, uint32_t n_slots) {
    const uint32_t tr = 256 / (QD::IPB * P) / n_slots;
    return tr < 1 ? 1 : tr;
}

// Kernel B's variant (b_variant's key), tile rows and workgroup size.
struct BPlan {
    uint32_t key, tr, nt;
};

// Kernel B's launch as planned by b_plan (tile rows, workgroup size).
template <class QD, int IPL, int P>
static hipError_t go_b(const MoeArgs &a, uint32_t n_slots, const BPlan &pl, hipStream_t s) {
    const uint32_t S = QD::IPB * P, tr = pl.tr, nt = pl.nt;
    // every pair of a tile has its S lanes (a pair without them would leave
    // its partial sum unwritten)
    if (tr * n_slots * S > nt) return hipErrorInvalidValue;
    const LdsB L = lds_b(a.ffn, n_slots, tr);
    if (L.total > moe_layer_lds(a.hidden, a.ffn, n_slots)) return hipErrorInvalidValue;   // the host's bound
    const dim3 grid((a.hidden + tr - 1) / tr);
    // the 256-thread tiles keep their own build (a constant workgroup size)
    if (nt == 256) hipLaunchKernelGGL((k_moe_down<QD, IPL, P, 256>), grid, dim3(nt), L.total, s, a, tr, n_slots);
    else hipLaunchKernelGGL((k_moe_down<QD, IPL, P, 0>), grid, dim3(nt), L.total, s, a, tr, n_slots);
    return hipGetLastError();
}
// P = lanes-per-pair multiplier: the smallest power of two that brings a
// lane's blocks (IPL = ceil(nb / P)) to at most 4 while a workgroup still
// holds every slot of at least one output row; 1 (a runtime block loop when
// IPL > 4) where no unrolled variant fits.
template <class QD>
static uint32_t b_mult(uint32_t nb, uint32_t n_slots) {
    uint32_t p = 1;
    while ((nb + p - 1) / p > 4 && QD::IPB * 4 * p <= 64 && QD::IPB * 4 * p * n_slots <= 256) p *= 4;
    const uint32_t ipl = (nb + p - 1) / p;
    if (QD::IPB * p * n_slots > 256 || ipl > 4 || QD::IPB * p > 64) return 1;
    return p;
}
// The switch key of kernel B's unrolled variants, P * 8 + IPL, unique only
// for IPL <= 4 (P = 1 with 26 blocks would otherwise read as P = 4, IPL = 2);
// 0 (the runtime block loop) for every other choice.
static uint32_t b_variant(uint32_t p, uint32_t ipl) { return ipl >= 1 && ipl <= 4 ? p * 8 + ipl : 0; }

// Kernel B's variant and tiles: 256-thread tiles, unless those give between
// one and two workgroups per CU (some CUs would take two tiles while the rest
// idle): then the fewest rows per tile that keep one tile per CU, in up to
// B_MAX_THREADS threads (nine slots at 2048 rows: 293 tiles of 7 rows -> 256
// tiles of 8 rows in 320 threads).
template <class QD>
static BPlan b_plan(const MoeArgs &a, uint32_t n_slots) {
    const uint32_t nb = a.ffn / 256;
    const uint32_t p = b_mult<QD>(nb, n_slots);
    BPlan pl;
    pl.key = b_variant(p, (nb + p - 1) / p);
    const uint32_t P = pl.key ? p : 1u, S = QD::IPB * P;
    pl.tr = b_tile_rows<QD>(P, n_slots);
    pl.nt = 256;
    const uint32_t cus = (uint32_t)device_cu_count();
    const uint32_t ntile = (a.hidden + pl.tr - 1) / pl.tr;
    if (ntile > cus && ntile < 2 * cus) {
        const uint32_t tr1 = (a.hidden + cus - 1) / cus, lanes = tr1 * n_slots * S;
        if (lanes <= B_MAX_THREADS) {
            pl.tr = tr1;
            pl.nt = (lanes + 63) / 64 * 64;
        }
    }
    return pl;
}
static BPlan b_plan_any(const MoeArgs &a, uint32_t n_slots) {
    return a.down_type == T_Q6_K ? b_plan<Q6K>(a, n_slots) : b_plan<Q4K>(a, n_slots);
}

template <class QD>
static hipError_t go_b_any(const MoeArgs &a, uint32_t n_slots, const BPlan &pl, hipStream_t s) {
    switch (pl.key) {
        case 1 * 8 + 1: return go_b<QD, 1, 1>(a, n_slots, pl, s);
        case 1 * 8 + 2: return go_b<QD, 2, 1>(a, n_slots, pl, s);
        case 1 * 8 + 3: return go_b<QD, 3, 1>(a, n_slots, pl, s);
        case 1 * 8 + 4: return go_b<QD, 4, 1>(a, n_slots, pl, s);
        case 4 * 8 + 2: return go_b<QD, 2, 4>(a, n_slots, pl, s);
        case 4 * 8 + 3: return go_b<QD, 3, 4>(a, n_slots, pl, s);
        case 4 * 8 + 4: return go_b<QD, 4, 4>(a, n_slots, pl, s);
        default: break;
    }
    if constexpr (QD::IPB * 16 <= 64) {
        switch (pl.key) {
            case 16 * 8 + 2: return go_b<QD, 2, 16>(a, n_slots, pl, s);
            case 16 * 8 + 3: return go_b<QD, 3, 16>(a, n_slots, pl, s);
            case 16 * 8 + 4: return go_b<QD, 4, 16>(a, n_slots, pl, s);
            default: break;
        }
    }
    return go_b<QD, 0, 1>(a, n_slots, pl, s);
}
static hipError_t go_b_run(const MoeArgs &a, uint32_t n_slots, const BPlan &pl, hipStream_t s) {
    return a.down_type == T_Q6_K ? go_b_any<Q6K>(a, n_slots, pl, s) : go_b_any<Q4K>(a, n_slots, pl, s);
}

// Kernel B's tile holds tr * n_slots <= B_MAX_THREADS partial sums: tr =
// 256 / (IPB * P) / n_slots (or 1 when that is 0, then n_slots <= MAX_SLOTS
// sums), or tr1 with tr1 * n_slots * S <= B_MAX_THREADS lanes.
uint32_t moe_layer_lds(uint32_t hidden, uint32_t ffn, uint32_t n_slots) {
    const uint32_t a = lds_a(hidden, hidden / 256).total;
    const uint32_t b = n_slots * act_bytes(ffn) + (B_MAX_THREADS + MAX_SLOTS) * 4;
    return a > b ? a : b;
}

uint32_t moe_groups_lds(uint32_t hidden, uint32_t ffn) {
    const uint32_t g = lds_g(hidden, hidden / 256).total, d = GRP_MAX * act_bytes(ffn);
    return g > d ? g : d;
}

bool moe_shape_supported(uint32_t gate_type, uint32_t down_type, uint32_t hidden, uint32_t ffn) {
    if (gate_type != T_Q4_K || (down_type != T_Q4_K && down_type != T_Q6_K)) return false;
    const uint32_t nb = hidden / 256;
    if (hidden % 256 || !(nb == 1 || nb == 2 || nb == 4 || nb == 8 || nb == 16)) return false;
    return ffn % 256 == 0 && ffn >= 256;
}

static hipError_t go_a_any(const MoeArgs &a, uint32_t n_slots, hipStream_t s);

// Routing of T tokens at once (batched prefill): one wave per token runs
// kernel A's own routing (load_keys, wave_topk, route_weight) on its row of
// logits, so every token gets the experts and weights the single-token layer
// would route it to, bit for bit. Lanes r < n_sel write rank r.
template <int C>
__global__ void __launch_bounds__(64) k_route_batch(const float *logits, uint32_t n_expert, int n_sel,
                                                    int32_t *ids, float *wts) {
    MoeArgs a{};
    a.logits = logits + (uint64_t)blockIdx.x * n_expert;
    a.n_expert = n_expert;
    a.n_sel = n_sel;
    float lv[C];
    load_keys<C>(a, lv);
    const WaveRoute r = wave_topk<C>(a, lv);
    const float w = route_weight(r.logit, n_sel);
    const uint32_t lane = threadIdx.x;
    if ((int)lane < n_sel) {
        ids[(uint64_t)blockIdx.x * n_sel + lane] = r.id;
        wts[(uint64_t)blockIdx.x * n_sel + lane] = w;
    }
}

hipError_t launch_route_batch(const float *logits, uint32_t n_tokens, uint32_t n_expert, int n_sel, int32_t *ids,
                              float *wts, hipStream_t s) {
    if (n_expert <= 128)
        hipLaunchKernelGGL(k_route_batch<2>, dim3(n_tokens), dim3(64), 0, s, logits, n_expert, n_sel, ids, wts);
    else if (n_expert <= 256)
        hipLaunchKernelGGL(k_route_batch<4>, dim3(n_tokens), dim3(64), 0, s, logits, n_expert, n_sel, ids, wts);
    else
        hipLaunchKernelGGL(k_route_batch<8>, dim3(n_tokens), dim3(64), 0, s, logits, n_expert, n_sel, ids, wts);
    return hipGetLastError();
}

hipError_t launch_moe(const MoeArgs &a, hipStream_t s, bool allow_fused, bool *fused, bool allow_xcd,
                      bool xcd_shared_units) {
    if (a.n_expert > MAX_EXPERT || a.n_sel > MAX_SEL) return hipErrorInvalidValue;
    const uint32_t n_slots = (uint32_t)a.n_sel + (a.has_shared ? 1u : 0u);
    if (fused) *fused = false;
    if (allow_xcd) {
        const hipError_t f = launch_moe_xcd(a, n_slots, xcd_shared_units, s);
        if (f != hipErrorNotSupported) {
            if (fused) *fused = f == hipSuccess;
            return f;
        }
    }
    if (allow_fused && a.n_sel > 0) {
        const hipError_t f = launch_moe_fused(a, n_slots, s);
        if (f != hipErrorNotSupported) {
            if (fused) *fused = f == hipSuccess;
            return f;
        }
    }
    const hipError_t e = go_a_any(a, n_slots, s);
    if (e != hipSuccess) return e;
    return go_b_run(a, n_slots, b_plan_any(a, n_slots), s);
}

static hipError_t go_a_any(const MoeArgs &a, uint32_t n_slots, hipStream_t s) {
    switch (a.hidden / 256) {
        case 1: return go_a<1>(a, n_slots, s);
        case 2: return go_a<2>(a, n_slots, s);
        case 4: return go_a<4>(a, n_slots, s);
        case 8: return go_a<8>(a, n_slots, s);
        case 16: return go_a<16>(a, n_slots, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_normed(MoeArgs a, float *xn_buf, float *logits_buf, hipStream_t s, bool *merged,
                             bool allow_xcd) {
    if (merged) *merged = false;
    if (!a.router || a.n_sel < 1 || a.n_expert > MAX_EXPERT || a.n_sel > MAX_SEL || a.hidden > 4096)
        return hipErrorInvalidValue;
    const uint32_t n_slots = (uint32_t)a.n_sel + (a.has_shared ? 1u : 0u);
    // eight slots on 256 CUs: the XCD-sliced layer with the steps before it
    // in its prologue, one launch (each workgroup dots at most one router
    // row at <= 256 experts)
    if (allow_xcd && a.fsync && !xcd_disabled() && n_slots == XCD_SLOTS && (a.hidden == 1024 || a.hidden == 2048) &&
        a.ffn <= 1024 &&
        a.n_expert <= XCD_G && device_cu_count() == (int)XCD_G) {
        MoeArgs b = a;
        b.x = nullptr;
        b.xq = nullptr;
        b.logits = nullptr;
        b.step = nullptr;
        b.hloc = xcd_local() ? 1u : 0u;
        const hipError_t e = a.hidden == 2048 ? go_xcd_c<8, false, true>(b, s) : go_xcd_c<4, false, true>(b, s);
        if (e != hipErrorNotSupported) {
            if (merged) *merged = e == hipSuccess;
            return e;
        }
    }
    const uint32_t U = n_slots * (a.ffn / 32);
    // kernel A's workgroups wait for each other's router rows: all of them
    // must be resident at once (one per CU at most), each with <= 4 rows
    if (a.fsync && U <= (uint32_t)device_cu_count() && (a.n_expert + U - 1) / U <= NORMED_MAX_R) {
        a.x = nullptr;
        a.xq = nullptr;
        a.logits = nullptr;
        a.step = nullptr;
        hipError_t e;
        switch (a.hidden / 256) {
            case 1: e = go_a<1, true>(a, n_slots, s); break;
            case 2: e = go_a<2, true>(a, n_slots, s); break;
            case 4: e = go_a<4, true>(a, n_slots, s); break;
            case 8: e = go_a<8, true>(a, n_slots, s); break;
            case 16: e = go_a<16, true>(a, n_slots, s); break;
            default: return hipErrorInvalidValue;
        }
        if (e != hipSuccess) return e;
        if (merged) *merged = true;
        // kernel B advances the exchange generation (a.router set)
        return go_b_run(a, n_slots, b_plan_any(a, n_slots), s);
    }
    // the router rows do not spread over kernel A: the steps before the
    // layer in their own launch, then the layer from their outputs
    float *xn = a.nxn_out ? a.nxn_out : xn_buf;
    float *lg = a.logits_out ? a.logits_out : logits_buf;
    hipError_t e = launch_norm_router(a.nx, a.ndelta, a.nscale, a.nx_out, a.nw, a.hidden, a.neps, xn, a.router,
                                      a.n_expert, lg, s);
    if (e != hipSuccess) return e;
    MoeArgs b = a;
    b.router = nullptr;
    b.x = xn;
    b.xq = nullptr;
    b.logits = lg;
    b.step = nullptr;
    return launch_moe(b, s);
}

template <int NB>
static hipError_t go_a_grp(const MoeArgs &a, uint32_t max_entries, hipStream_t s) {
    const LdsG L = lds_g(a.hidden, NB);
    if (L.total > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_moe_gu_grp<NB>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)L.total);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_moe_gu_grp<NB>, dim3(max_entries * (a.ffn / 32)), dim3(A_THREADS), L.total, s, a);
    return hipGetLastError();
}

hipError_t launch_moe_groups_gu(const MoeArgs &a, uint32_t max_entries, hipStream_t s) {
    if (!a.bslot || !a.bcount || !a.border || max_entries == 0) return hipErrorInvalidValue;
    switch (a.hidden / 256) {
        case 1: return go_a_grp<1>(a, max_entries, s);
        case 2: return go_a_grp<2>(a, max_entries, s);
        case 4: return go_a_grp<4>(a, max_entries, s);
        case 8: return go_a_grp<8>(a, max_entries, s);
        case 16: return go_a_grp<16>(a, max_entries, s);
        default: return hipErrorInvalidValue;
    }
}

template <class QD, int IPL, int P>
static hipError_t go_b_grp(const MoeArgs &a, uint32_t max_entries, hipStream_t s) {
    const uint32_t tr = b_tile_rows<QD>(P, 1);
    if (tr * QD::IPB * P > 256) return hipErrorInvalidValue;   // a row's lanes in one workgroup
    const uint32_t lds = GRP_MAX * act_bytes(a.ffn);
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_moe_down_grp<QD, IPL, P>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_moe_down_grp<QD, IPL, P>), dim3((a.hidden + tr - 1) / tr, max_entries), dim3(256), lds, s, a,
                       tr);
    return hipGetLastError();
}

// the same (P, IPL) choice as kernel B with one slot per row
template <class QD>
static hipError_t go_b_grp_any(const MoeArgs &a, uint32_t max_entries, hipStream_t s) {
    const uint32_t nb = a.ffn / 256;
    const uint32_t p = b_mult<QD>(nb, 1);
    const uint32_t key = b_variant(p, (nb + p - 1) / p);
    switch (key) {
        case 1 * 8 + 1: return go_b_grp<QD, 1, 1>(a, max_entries, s);
        case 1 * 8 + 2: return go_b_grp<QD, 2, 1>(a, max_entries, s);
        case 1 * 8 + 3: return go_b_grp<QD, 3, 1>(a, max_entries, s);
        case 1 * 8 + 4: return go_b_grp<QD, 4, 1>(a, max_entries, s);
        case 4 * 8 + 2: return go_b_grp<QD, 2, 4>(a, max_entries, s);
        case 4 * 8 + 3: return go_b_grp<QD, 3, 4>(a, max_entries, s);
        case 4 * 8 + 4: return go_b_grp<QD, 4, 4>(a, max_entries, s);
        default: break;
    }
    if constexpr (QD::IPB * 16 <= 64) {
        switch (key) {
            case 16 * 8 + 2: return go_b_grp<QD, 2, 16>(a, max_entries, s);
            case 16 * 8 + 3: return go_b_grp<QD, 3, 16>(a, max_entries, s);
            case 16 * 8 + 4: return go_b_grp<QD, 4, 16>(a, max_entries, s);
            default: break;
        }
    }
    return go_b_grp<QD, 0, 1>(a, max_entries, s);
}

hipError_t launch_moe_groups_down(const MoeArgs &a, uint32_t max_entries, hipStream_t s) {
    if (!a.bslot || !a.bcount || !a.border || !a.yp || max_entries == 0 || max_entries > 65535) return hipErrorInvalidValue;
    return a.down_type == T_Q6_K ? go_b_grp_any<Q6K>(a, max_entries, s) : go_b_grp_any<Q4K>(a, max_entries, s);
}

}  // namespace kq
