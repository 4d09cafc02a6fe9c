// kq_moe_batch.hip — the MoE layer over a batch of tokens (prefill).
//
// y_t = sum_r w_{t,r} Down_e(q8(SiLU(Gate_e x_t) * Up_e x_t)), e = ids[t][r],
// plus the shared expert (weight 1) when present, for T <= 64 tokens.
//
// 1. k_mb_group, one launch: its first workgroup groups the T*S (token,
//    slot) pairs, S = n_sel + shared, by expert (counting sort) while the
//    others quantize every x_t to q8_1. An expert that gathers at least
//    min_big pairs goes to the grouped-GEMM list (in entries of at most 16
//    pairs), every other expert to the small list (entries of at most 8
//    pairs).
// 3. Small list: the grouped v_dot4 GEMV kernels k_moe_gu_grp and
//    k_moe_down_grp (kq_moe.hip): one read of a weight tile per entry,
//    dotted with each pair's activation exactly as kernels A and B of the
//    single-token layer do; h to the pair's q8_1 row, the unweighted down
//    output to yp.
// 4. Grouped GEMM list: k_mb_gu_mfma and k_mb_down_mfma, int8 MFMA
//    v_mfma_i32_16x16x32_i8 (one operand 16 pairs x 32 k of activations,
//    the other 32 k x 16 weight rows) with the block scales applied per
//    32-value sub-block in fp32 (per 16-value group for Q6_K: two MFMAs per
//    32 k on the same weight operand, each against activations whose other
//    half is read from a zeroed LDS area), same q8_1 definitions as the
//    GEMV path.
// 5. k_mb_combine: y_t = fmaf over the slots in rank order (deterministic).
#include "kq_device.h"
#include "kq_launch.h"

namespace kq {

typedef int v4i __attribute__((ext_vector_type(4)));

// f(integral_constant<int, I>) for I = B .. E-1, unrolled at compile time
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

constexpr uint32_t MB_MAX_T = 64;
constexpr uint32_t MB_MAX_S = 17;
constexpr uint32_t MB_MAX_P = MB_MAX_T * MB_MAX_S;
constexpr uint32_t MB_MAX_E = 513;   // routed experts + the shared expert's virtual id

// meta layout (int32): [0] small entries, [1] grouped-GEMM entries, [2]
// error bits, [16 ..) small entries (3 ints each: expert, first, count <= 8;
// at most P), then grouped-GEMM entries (MB_REC ints each: expert, first,
// count <= 16, 0, then the entry's 16 pairs inline, slots past count
// holding pair 0; at most P; an expert's entries are consecutive), then
// order (the P pairs grouped by expert, experts ascending; the order inside
// one expert's run is arbitrary); a small entry's pairs are
// order[first .. first + count). A grouped-GEMM tile reads its entry count
// and its whole record at once: no load waits on another.
constexpr uint32_t MB_GRP = 8;   // pairs per small entry (the grouped GEMV kernels' GRP_MAX)
constexpr uint32_t MB_BIG = 16;  // pairs per grouped-GEMM entry (the MFMA's 16 B columns)
constexpr uint32_t MB_FORK_PAIRS = 96;   // batches from this many pairs run the two paths side by side
constexpr uint32_t MB_DN_CHUNK = 8;   // h blocks staged at once by the down kernel beyond 3 blocks
constexpr uint32_t MB_REC = 20;      // ints per grouped-GEMM entry: 4 + MB_BIG pairs
__host__ __device__ inline uint32_t mb_small_off() { return 16; }
// the grouped-GEMM records start on a 16-byte boundary (each is read as
// int4s, MB_REC a multiple of 4): the small entries' 3 P ints rounded up
__host__ __device__ inline uint32_t mb_big_off(uint32_t P) { return 16 + ((3 * P + 3) & ~3u); }
__host__ __device__ inline uint32_t mb_order_off(uint32_t P) { return mb_big_off(P) + MB_REC * P; }
static_assert(MB_REC % 4 == 0, "grouped-GEMM records: whole int4s");
uint64_t moe_batch_meta_words(uint32_t P) { return mb_order_off(P) + P; }

// Inclusive prefix sum over the 64 lanes of a wave on the VALU: row_shr 1, 2,
// 4, 8 inside each 16-lane row (lanes without a source add 0), then
// row_bcast:15 adds row 0's total to row 1 and row 2's to row 3, and
// row_bcast:31 adds lane 31's running total to rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return v;
}

// Workgroup 0 groups the pairs; workgroups 1.. quantize the T activation
// rows to q8_1 meanwhile (k_quantize_q8_1's split: 8 lanes per 32-value
// block, the same bits), so the two take one launch.
__global__ void __launch_bounds__(1024) k_mb_group(const int32_t *__restrict__ ids, uint32_t T, uint32_t n_sel,
                                                   uint32_t S, uint32_t n_expert, uint32_t min_big,
                                                   int32_t *__restrict__ meta, int32_t *__restrict__ err,
                                                   const float *__restrict__ x, uint32_t nq, uint8_t *__restrict__ xq) {
    if (blockIdx.x > 0) {   // whole workgroup
        for (uint32_t t = (blockIdx.x - 1) * 1024 + threadIdx.x; t < nq; t += (gridDim.x - 1) * 1024) {
            const uint32_t blk = t >> 3, part = t & 7;   // whole 8-lane groups (nq % 8 == 0)
            const float4 v = *(const float4 *)(x + 32 * blk + 4 * part);
            uint32_t d16, s16;
            int lo, hi;
            float dd;
            const uint32_t q = quant_q8_1_part(v, d16, s16, lo, hi, dd);
            uint8_t *b = xq + 36 * blk;
            *(uint32_t *)(b + 4 + 4 * part) = q;
            if (part == 0) *(uint32_t *)b = d16 | (s16 << 16);
        }
        return;
    }
    __shared__ int32_t cnt[MB_MAX_E], off_all[MB_MAX_E], small_idx[MB_MAX_E], big_idx[MB_MAX_E], cur[MB_MAX_E];
    __shared__ int32_t exp_of[MB_MAX_P];
    __shared__ int32_t wsum[3][16];
    __shared__ int32_t bad;
    const uint32_t P = T * S, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t NE = n_expert + 1;   // id n_expert = the shared expert
    for (uint32_t e = tid; e < NE; e += blockDim.x) cnt[e] = cur[e] = 0;
    if (tid == 0) bad = 0;
    __syncthreads();
    for (uint32_t p = tid; p < P; p += blockDim.x) {
        const uint32_t t = p / S, r = p % S;
        int32_t e = (int32_t)n_expert;
        if (r < n_sel) {
            e = ids[t * n_sel + r];
            if (e < 0 || (uint32_t)e >= n_expert) {
                atomicOr(&bad, 1);
                e = 0;   // addressing stays in the pool; reported
            }
        }
        exp_of[p] = e;
        atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // Exclusive prefix sums over the experts (NE <= 1024: one per thread) of
    // the pair counts, the small entry counts and the grouped-GEMM entry
    // counts.
    {
        const int c = tid < NE ? cnt[tid] : 0;
        const bool big = c >= (int)min_big && c > 0;
        const int va = c, vs = big ? 0 : (c + (int)MB_GRP - 1) / (int)MB_GRP, vb = big ? (c + (int)MB_BIG - 1) / (int)MB_BIG : 0;
        const int ia = wave_incl_scan(va), is = wave_incl_scan(vs), ib = wave_incl_scan(vb);
        if (lane == 63) {
            wsum[0][wave] = ia;
            wsum[1][wave] = is;
            wsum[2][wave] = ib;
        }
        __syncthreads();
        int pa = 0, ps = 0, pb = 0;
        for (uint32_t w = 0; w < wave; w++) {
            pa += wsum[0][w];
            ps += wsum[1][w];
            pb += wsum[2][w];
        }
        if (tid < NE) {
            off_all[tid] = pa + ia - va;
            small_idx[tid] = vs > 0 ? ps + is - vs : -1;   // first small entry of this expert
            big_idx[tid] = big ? pb + ib - vb : -1;   // first entry of this expert
        }
        if (tid == NE - 1) {
            meta[0] = ps + is;
            meta[1] = pb + ib;
            meta[2] = bad ? 2 : 0;
            if (bad) atomicOr(err, 2);
        }
    }
    __syncthreads();
    int32_t *small = meta + mb_small_off(), *bigl = meta + mb_big_off(P), *order = meta + mb_order_off(P);
    for (uint32_t e = tid; e < NE; e += blockDim.x) {
        const int32_t c = cnt[e];
        if (big_idx[e] >= 0) {
            for (int32_t k = 0; (int32_t)MB_BIG * k < c; k++) {
                int32_t *rec = bigl + MB_REC * (big_idx[e] + k);
                rec[0] = (int32_t)e;
                rec[1] = off_all[e] + (int32_t)MB_BIG * k;
                rec[2] = min((int32_t)MB_BIG, c - (int32_t)MB_BIG * k);
                rec[3] = 0;
                for (uint32_t j = 0; j < MB_BIG; j++) rec[4 + j] = 0;   // pair 0: a valid row to address
            }
        } else if (small_idx[e] >= 0) {
            for (int32_t k = 0; (int32_t)MB_GRP * k < c; k++) {
                const int32_t i = small_idx[e] + k;
                small[3 * i + 0] = (int32_t)e;
                small[3 * i + 1] = off_all[e] + (int32_t)MB_GRP * k;
                small[3 * i + 2] = min((int32_t)MB_GRP, c - (int32_t)MB_GRP * k);
            }
        }
    }
    __syncthreads();   // the records' pair slots are prefilled before the pairs land in them
    // a pair's place among its expert's pairs comes from an LDS cursor: the
    // order inside an expert's run may differ from call to call, which no
    // result depends on (every pair's sums are formed on their own)
    for (uint32_t p = tid; p < P; p += blockDim.x) {
        const int32_t e = exp_of[p];
        const int32_t k = atomicAdd(&cur[e], 1);
        order[off_all[e] + k] = (int32_t)p;
        if (big_idx[e] >= 0) bigl[MB_REC * (big_idx[e] + k / (int32_t)MB_BIG) + 4 + k % (int32_t)MB_BIG] = (int32_t)p;
    }
}

// ---------------------------------------------------------------------------
// Shared pieces of the two MFMA kernels
// ---------------------------------------------------------------------------
// The activation chunk of one 256-value block for the 16 pairs of a column
// group, staged in LDS: int8 values [16][MBX_ROW] (rows padded by 16 bytes
// so the 16 pair columns one MFMA operand read touches start in different
// banks), their q8_1 scales d8 [8 sub-blocks][16 pairs] and exact sums of
// each 32 values (as floats) qs [8][16] (four pairs of one sub-block: one
// 16-byte read).
constexpr uint32_t MBX_ROW = 272;
struct MbX {
    int8_t *q;
    float *d8;
    float *qs;
};
__device__ __forceinline__ MbX mbx_carve(uint8_t *base) {
    MbX x;
    x.q = (int8_t *)base;
    x.d8 = (float *)(base + 16 * MBX_ROW);
    x.qs = (float *)(base + 16 * MBX_ROW + 16 * 8 * 4);
    return x;
}
constexpr uint32_t MBX_BYTES = 16 * MBX_ROW + 2 * 16 * 8 * 4;

// Staging split (16 pairs per 256 threads): thread t takes local pair
// (t / 16) % 16, q8_1 block 8b + (t / 2) % 8 of that pair's row and half
// t % 2 of its values.
struct XPart {
    uint4 q;
    uint32_t h;
};
__device__ __forceinline__ XPart mbx_load(const uint8_t *row, uint32_t b) {
    const uint32_t sb = (threadIdx.x >> 1) & 7, half = threadIdx.x & 1;
    const uint8_t *p = row + (uint64_t)(8 * b + sb) * 36;
    XPart v;
    v.h = ld4(p);
    v.q = ld16(p + 4 + 16 * half);
    return v;
}
// Pairs past the group's count stage zeros (their B columns add nothing).
__device__ __forceinline__ void mbx_put(const MbX &x, const XPart &v, bool valid) {
    const uint32_t i = (threadIdx.x >> 4) & 15, sb = (threadIdx.x >> 1) & 7, half = threadIdx.x & 1;
    const uint4 q = valid ? v.q : make_uint4(0, 0, 0, 0);
    *(uint4 *)(x.q + MBX_ROW * i + 32 * sb + 16 * half) = q;
    int s = dot4(q.x, 0x01010101u, 0);
    s = dot4(q.y, 0x01010101u, s);
    s = dot4(q.z, 0x01010101u, s);
    s = dot4(q.w, 0x01010101u, s);
    s += dpp_i<DPP_XOR1>(s);   // the block's other half
    if (half == 0) {
        x.d8[16 * sb + i] = valid ? h2f(v.h & 0xFFFFu) : 0.0f;
        x.qs[16 * sb + i] = (float)s;   // |s| <= 32 * 128: exact
    }
}

// B operand: 8 int8 of local pair `col` at k = 32*sb + kc*8
__device__ __forceinline__ long mbx_b(const MbX &x, uint32_t col, uint32_t sb, uint32_t kc) {
    return *(const long *)(x.q + MBX_ROW * col + 32 * sb + 8 * kc);
}

// Four 6-bit values 0..63 (one per byte) -> int8 q6 - 32 per byte without
// cross-byte carries: q + 96 <= 159 stays in its byte and is (q - 32) + 128,
// so flipping bit 7 leaves q - 32 in two's complement.
__device__ __forceinline__ uint32_t q6_minus_32(uint32_t q) {
    return (q + 0x60606060u) ^ 0x80808080u;
}

// Pairwise sum of a stream of terms t_0, t_1, ... pushed in index order (J
// known at compile time): stk[l] holds the sum of the last complete group of
// 2^l terms not yet combined. Pushing t_J adds it to the pending groups while
// bit l of J is set (each such group is the left half of the next level's
// group), then parks the result at the first clear bit. After t_{2^K - 1},
// stk[K] holds sum(t[0 .. 2^K)) in the pairwise tree:
// sum(t[0..n)) = sum(t[0..n/2)) + sum(t[n/2..n)).
template <int J, int L, int LV>
__device__ __forceinline__ void pw_push(float (&stk)[LV], float c) {
    static_assert(L < LV, "pw_push: stack too shallow");
    if constexpr ((J >> L) & 1) pw_push<J, L + 1, LV>(stk, stk[L] + c);
    else stk[L] = c;
}

// The pending groups after N pushes (levels L with bit L of N set), for 4
// stacks, formed at this point of the program (an empty asm that reads and
// writes each one)
template <int N, int LV, int L = 0>
__device__ __forceinline__ void pw_pin(float (&stk)[4][LV]) {
    if constexpr (L < LV) {
        if constexpr ((N >> L) & 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) asm volatile("" : "+v"(stk[i][L]));
        }
        pw_pin<N, LV, L + 1>(stk);
    }
}

__device__ __forceinline__ v4i mfma16(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// One wave's weight operands for one block: lane (row l % 16, k chunk l / 16)
// holds the quants its A operands need for all 8 sub-blocks, and lane
// (row l / 4, group l % 4) the scale bytes it decodes into the wave's LDS
// scale table [16 rows][NS].
template <class QD>
struct MbW;
// 8 bytes of LDS at byte offset o (2-byte aligned): three dwords, funnel-shifted
__device__ __forceinline__ uint2 lds_ld8_a2(const uint8_t *l, uint32_t o) {
    const uint32_t *w = (const uint32_t *)(l + (o & ~3u));
    const uint32_t s = o & 3u, w0 = w[0], w1 = w[1], w2 = w[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s));
}
__device__ __forceinline__ uint32_t lds_ld4_a2(const uint8_t *l, uint32_t o) {
    const uint32_t *w = (const uint32_t *)(l + (o & ~3u));
    return __builtin_amdgcn_alignbyte(w[1], w[0], o & 3u);
}
__device__ __forceinline__ uint4 lds_ld16_a2(const uint8_t *l, uint32_t o) {
    const uint32_t *w = (const uint32_t *)(l + (o & ~3u));
    const uint32_t s = o & 3u, w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4];
    return make_uint4(__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s),
                      __builtin_amdgcn_alignbyte(w3, w2, s), __builtin_amdgcn_alignbyte(w4, w3, s));
}

template <>
struct MbW<Q4K> {
    static constexpr uint32_t NS = 8;   // {d*sc, dmin*m} per 32-value sub-block
    uint2 q[4];
    uint4 h;
    __device__ __forceinline__ void load(const uint8_t *ablk, const uint8_t *hblk, uint32_t kc) {
#pragma unroll
        for (int m = 0; m < 4; m++) q[m] = ld8(ablk + 16 + 32 * m + 8 * kc);
        h = ld16(hblk);
    }
    // Row-per-lane use (the lane's row is the A row it loads): the quants
    // and its own row's header, from global memory or from a copy of the
    // rows in LDS (block byte offset ao, 16-byte aligned as every Q4_K block
    // of a row is)
    __device__ __forceinline__ void load_row(const uint8_t *ablk, uint32_t kc) { load(ablk, ablk, kc); }
    __device__ __forceinline__ void load_row_lds(const uint8_t *l, uint32_t ao, uint32_t kc) {
#pragma unroll
        for (int m = 0; m < 4; m++) q[m] = *(const uint2 *)(l + ao + 16 + 32 * m + 8 * kc);
        h = *(const uint4 *)(l + ao);
    }
    // the row's {d*sc_j, dmin*m_j} for the 8 sub-blocks j: rs[2j], rs[2j+1]
    __device__ __forceinline__ void row_scales(float (&rs)[16]) const {
        Q4K::Raw raw;
        raw.h = h;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float ds0, ds1, dm0, dm1;
            Q4K::scales(raw, g, ds0, ds1, dm0, dm1);
            rs[4 * g] = ds0;
            rs[4 * g + 1] = dm0;
            rs[4 * g + 2] = ds1;
            rs[4 * g + 3] = dm1;
        }
    }
    __device__ __forceinline__ void put_scales(float2 *scl) const {
        const uint32_t lane = threadIdx.x & 63, g = lane & 3, r = lane >> 2;
        Q4K::Raw raw;
        raw.h = h;
        float ds0, ds1, dm0, dm1;
        Q4K::scales(raw, (int)g, ds0, ds1, dm0, dm1);
        scl[NS * r + 2 * g] = make_float2(ds0, dm0);
        scl[NS * r + 2 * g + 1] = make_float2(ds1, dm1);
    }
    // 8 int8 (0..15) of sub-block j at this lane's k chunk: nibbles of
    // qs[32*(j/2) + 8*kc ..]
    __device__ __forceinline__ long a_op(uint32_t j) const {
        const uint2 v = q[j >> 1];
        const uint32_t sh = 4 * (j & 1), m = 0x0F0F0F0Fu;
        return (long)(((uint64_t)((v.y >> sh) & m) << 32) | ((v.x >> sh) & m));
    }
};
template <>
struct MbW<Q6K> {
    uint2 ql[4], qh[2];
    uint32_t d;
    // Row-per-lane use (the lane's row is the A row it loads): the quants
    // and its own row's 16 scales and d, from global memory or from a copy
    // of the rows in LDS (block byte offset ao: 2-byte aligned, 210-byte
    // blocks)
    uint4 sc16;
    __device__ __forceinline__ void load_row(const uint8_t *ablk, uint32_t kc) {
#pragma unroll
        for (int n = 0; n < 2; n++) {
            ql[2 * n] = ld8(ablk + 64 * n + 8 * kc);
            ql[2 * n + 1] = ld8(ablk + 64 * n + 32 + 8 * kc);
            qh[n] = ld8(ablk + 128 + 32 * n + 8 * kc);
        }
        sc16 = ld16(ablk + 192);
        d = ld_u16(ablk + 208);
    }
    __device__ __forceinline__ void load_row_lds(const uint8_t *l, uint32_t ao, uint32_t kc) {
#pragma unroll
        for (int n = 0; n < 2; n++) {
            ql[2 * n] = lds_ld8_a2(l, ao + 64 * n + 8 * kc);
            ql[2 * n + 1] = lds_ld8_a2(l, ao + 64 * n + 32 + 8 * kc);
            qh[n] = lds_ld8_a2(l, ao + 128 + 32 * n + 8 * kc);
        }
        sc16 = lds_ld16_a2(l, ao + 192);
        d = *(const uint16_t *)(l + ao + 208);
    }
    // the row's d * scale for the 16 groups of 16 values (groups 2j, 2j + 1
    // of sub-block j)
    __device__ __forceinline__ void row_scales(float (&rs)[16]) const {
        const float dd = h2f(d);
        const uint32_t w[4] = {sc16.x, sc16.y, sc16.z, sc16.w};
#pragma unroll
        for (int g = 0; g < 16; g++) rs[g] = dd * (float)(int)(int8_t)(w[g >> 2] >> (8 * (g & 3)));
    }
    // 8 int8 (q6 - 32) at values 32j + 8kc .. +7 of the block: ql nibble + 2
    // qh bits, in the block's interleave (half n = j / 4, quarter j % 4)
    __device__ __forceinline__ long a_op(uint32_t j) const {
        const uint32_t n = j >> 2, qq = j & 3;
        const uint2 l = ql[2 * n + (qq & 1)], hb = qh[n];
        const uint32_t sl = qq >= 2 ? 4 : 0, sh = 2 * qq, m4 = 0x0F0F0F0Fu, m2 = 0x03030303u;
        const uint32_t lo = ((l.x >> sl) & m4) | (((hb.x >> sh) & m2) << 4);
        const uint32_t hi = ((l.y >> sl) & m4) | (((hb.y >> sh) & m2) << 4);
        return (long)(((uint64_t)q6_minus_32(hi) << 32) | q6_minus_32(lo));
    }
};

// ---------------------------------------------------------------------------
// Gate/up of the grouped-GEMM entries: a tile is 32 gate + 32 up rows (jb) x
// one entry's <= 16 pairs, workgroup t = entry * nblk + jb, so the tiles of
// the entries the grouping made come first and the workgroups past them
// (the grid covers the worst-case entry count) leave after their first
// loads. The entries of one expert are consecutive, so the tiles that share a
// weight tile are nblk workgroups apart: with nblk a multiple of 8 they run
// on one XCD and share its L2 copy of the weights. Per tile: the entry count
// and the entry's record (pairs inline) at once, then the pairs' activation
// blocks (all NB staged in LDS behind one barrier; they come from L2) and
// the first two weight blocks of each wave. The NB blocks are split into S
// slices of NB / S consecutive blocks, one per group of four waves (wave w:
// rows 16 (w % 4) .. +15, slice w / 4), so each SIMD runs S of the tile's
// sub-block chains at once: a wave's per-block chain (scale table, MFMA,
// fp32 terms) is latency-bound, not VALU-bound. A slice's weights stream
// through a ring of three blocks in registers: block b + 2 is issued
// before block b's arithmetic. A slice's value is the pairwise sum over
// its blocks; the slices join as the top levels of the same tree.
// ---------------------------------------------------------------------------
// (at most 128 VGPRs: two 8-wave tiles per CU)
template <int NB, int S>
__global__ void __launch_bounds__(256 * S, 4) k_mb_gu_mfma(MoeArgs a, const int32_t *__restrict__ meta, uint32_t P) {
    static_assert(NB % S == 0 && (S == 1 || S == 2 || S == 4), "k_mb_gu_mfma: slices");
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t nblk = a.ffn / 32;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t rg = wave & 3, sl = wave >> 2;   // row group, slice
    const uint64_t rb = NB * 144;
    const uint32_t arow = lane % 16, kc = lane / 16;   // operands: weight row / pair column, k chunk
    const uint32_t p0 = 4 * (lane / 16);               // D: pairs p0 .. p0 + 3 of weight row arow
    const uint32_t si = (tid >> 4) & 15;   // this thread's staging pair
    constexpr int NBS = NB / S;               // blocks per slice
    constexpr int RING = NBS < 3 ? NBS : 3;   // weight blocks in registers: the current one and two ahead
    constexpr int XC = NBS < 8 ? NBS : 8;     // activation blocks loaded per staging round
    const uint32_t nent = (uint32_t)meta[1];
    for (uint32_t t = blockIdx.x;; t += gridDim.x) {
        const uint32_t bi = t / nblk, jb = t % nblk;
        // (tiles past the entries read the last record and leave)
        const int32_t *rec = meta + mb_big_off(P) + MB_REC * min(bi, P - 1);
        // independent loads: the record, this thread's pair (slots past the
        // count hold pair 0)
        const int4 hd = *(const int4 *)rec;
        const uint32_t sp = (uint32_t)rec[4 + si];
        if (bi >= nent) break;   // whole workgroup
        uint8_t *const lt = lds;
        float2 *scl = (float2 *)(lt + NB * MBX_BYTES) + 16 * 8 * wave;   // this wave's [16 rows][8 sub-blocks] {d*sc, dmin*m}
        float *gu = (float *)(lt + NB * MBX_BYTES + 4 * S * 16 * 8 * 8);  // [S slices][64 rows][16 pairs]
        const int32_t e = hd.x;
        const uint32_t cnt = (uint32_t)hd.z;
        const int32_t *pairs = rec + 4;
        const bool shared = (uint32_t)e == a.n_expert;
        const uint8_t *gb = shared ? a.gate_sh : a.gate + (uint64_t)e * a.ffn * rb;
        const uint8_t *ub = shared ? a.up_sh : a.up + (uint64_t)e * a.ffn * rb;
        // row group g: rows 16g..16g+15 of the 64 (groups 0-1 gate, 2-3 up),
        // from the slice's first block
        const uint8_t *wbase = (rg < 2 ? gb + (uint64_t)(32 * jb + 16 * rg) * rb
                                       : ub + (uint64_t)(32 * jb + 16 * (rg - 2)) * rb) + sl * NBS * 144;
        const uint8_t *ap = wbase + (uint64_t)arow * rb, *hp = wbase + (uint64_t)(lane >> 2) * rb;
        const uint8_t *xrow = a.xq + (uint64_t)(sp / a.bS) * a.xq_stride;
        MbW<Q4K> w[RING];
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // the activations first (L2 hits, but behind the record), then the
        // first two weight blocks: issued after the activations are in LDS, so
        // the activation loads do not queue behind weight loads. The threads
        // of slice s stage its activation blocks.
        static_for<0, NBS / XC>([&](auto rc) {
            constexpr int r = decltype(rc)::value;
            XPart xv[XC];
#pragma unroll
            for (int c = 0; c < XC; c++) xv[c] = mbx_load(xrow, sl * NBS + XC * r + c);
#pragma unroll
            for (int c = 0; c < XC; c++) mbx_put(mbx_carve(lt + (sl * NBS + XC * r + c) * MBX_BYTES), xv[c], si < cnt);
        });
#pragma unroll
        for (int b = 0; b < RING - 1; b++) w[b].load(ap + b * 144, hp + b * 144, kc);
        __syncthreads();
        // each (row, pair) value is the pairwise sum of its sub-block terms,
        // pushed in sub-block order (kernel A's q8_1-path dot, bit for bit):
        // 8 sub-blocks per block, so a block's 8 terms form one subtree
        constexpr int LV = log2c<8 * NBS>() + 1;
        float stk[4][LV];
        static_for<0, NBS>([&](auto bc) {   // unrolled: registers indexed by constants
            constexpr uint32_t b = decltype(bc)::value;   // the slice's block b
            __builtin_amdgcn_sched_barrier(0);   // one block's operands live at a time
            if constexpr (b + RING - 1 < (uint32_t)NBS)   // (a one-block ring loads block b itself here)
                w[(b + RING - 1) % RING].load(ap + (b + RING - 1) * 144, hp + (b + RING - 1) * 144, kc);
            const MbW<Q4K> &wc = w[b % RING];
            const MbX x = mbx_carve(lt + (sl * NBS + b) * MBX_BYTES);
            wc.put_scales(scl);   // wave-private table
            wave_sync_lds();
            float4 rs[4];   // the lane's row: {d*sc, dmin*m} of sub-blocks 2k, 2k + 1
#pragma unroll
            for (int k2 = 0; k2 < 4; k2++) rs[k2] = *(const float4 *)(scl + 8 * arow + 2 * k2);
            static_for<0, 8>([&](auto jc) {
                constexpr uint32_t j = decltype(jc)::value;
                const long wv = wc.a_op(j);
                // activations as A, weights as B: d[i] = isum of (pair p0 + i, row arow), sub-block 8b + j
                const v4i d = mfma16(mbx_b(x, arow, j, kc), wv);
                const float4 d8 = *(const float4 *)(x.d8 + 16 * j + p0), qs = *(const float4 *)(x.qs + 16 * j + p0);
                const float d8v[4] = {d8.x, d8.y, d8.z, d8.w}, qsv[4] = {qs.x, qs.y, qs.z, qs.w};
                const float sA = (j & 1) ? rs[j >> 1].z : rs[j >> 1].x, sB = (j & 1) ? rs[j >> 1].w : rs[j >> 1].y;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float A = sA * d8v[i], B = sB * d8v[i];
                    pw_push<8 * b + j, 0>(stk[i], fmaf(A, (float)d[i], -(B * qsv[i])));
                }
            });
            // the pending sums formed here (levels L with bit L of 8 (b + 1)
            // set): sinking the block's arithmetic past the next barriers
            // would keep its LDS reads live and spill
            pw_pin<8 * (b + 1)>(stk);
            wave_sync_lds();   // the table is rewritten for the next block
        });
        // the slice's sums of (row, pair) -> LDS; then each value joins its
        // slices pairwise, then SiLU-GLU and one q8_1 block per pair
#pragma unroll
        for (int i = 0; i < 4; i++) gu[16 * (64 * sl + 16 * rg + arow) + p0 + i] = stk[i][LV - 1];
        __syncthreads();
        if (tid < 16 * 8) {
            const uint32_t i = tid / 8, part = tid % 8;
            if (i < cnt) {   // whole 8-lane groups take this branch together
                auto row = [&](uint32_t r) {   // the whole row over the NB blocks
                    const float *g = gu + 16 * r + i;
                    if constexpr (S == 1) return g[0];
                    else if constexpr (S == 2) return g[0] + g[16 * 64];
                    else return (g[0] + g[16 * 64]) + (g[2 * 16 * 64] + g[3 * 16 * 64]);
                };
                float4 h;
                h.x = kq_silu_mul(row(4 * part + 0), row(32 + 4 * part + 0));
                h.y = kq_silu_mul(row(4 * part + 1), row(32 + 4 * part + 1));
                h.z = kq_silu_mul(row(4 * part + 2), row(32 + 4 * part + 2));
                h.w = kq_silu_mul(row(4 * part + 3), row(32 + 4 * part + 3));
                uint32_t d16, s16;
                int lo, hi;
                float dd;
                const uint32_t qv = quant_q8_1_part(h, d16, s16, lo, hi, dd);
                uint8_t *blk = a.hq8 + ((uint64_t)pairs[i] * nblk + jb) * 36;
                *(uint32_t *)(blk + 4 + 4 * part) = qv;
                if (part == 0) *(uint32_t *)blk = d16 | (s16 << 16);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Down of the grouped-GEMM entries: a tile is 64 output rows (rt) x one
// entry's <= 16 pairs -> yp, workgroup t = entry * ntile + rt as in the
// gate/up kernel; the pairs' h rows staged once per tile. Up to three
// blocks per row (a compile-time count), the tile's 64 rows, one contiguous
// run of 64 * rb bytes (16-byte aligned), are copied to LDS in coalesced
// 16-byte chunks and each wave builds its MFMA operands from there: per-lane
// loads in the MFMA layout read 8 bytes from each of 16 rows per
// instruction, at the 2-byte alignment of 210-byte Q6_K blocks, and cost
// the L1 several times the tag lookups of the copy. Longer rows load their
// operands from global memory one block at a time.
// The MFMA takes the activations as A and the weights as B, so a lane holds
// one weight row (the row whose operand it loads) for four pairs: its row's
// scales are computed in its registers, and the q8_1 scales of its four
// pairs come in one LDS read per sub-block. Q6_K's two 16-value scale groups
// per 32 k: the same weight operand against activations with the other
// group's half read from a zeroed LDS area (per lane, by address), two
// MFMAs.
// ---------------------------------------------------------------------------
template <class QD, int NBD>
__global__ void __launch_bounds__(256) k_mb_down_mfma(MoeArgs a, const int32_t *__restrict__ meta, uint32_t P) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t ntile = a.hidden / 64;   // hidden is a multiple of 256: whole tiles
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t nb = NBD > 0 ? (uint32_t)NBD : a.ffn / 256;
    const uint64_t rb = (uint64_t)nb * QD::BB;
    const uint32_t arow = lane % 16, kc = lane / 16;   // operands: weight row / pair column, k chunk
    const uint32_t p0 = 4 * (lane / 16);               // D: pairs p0 .. p0 + 3 of weight row arow
    const uint32_t si = tid >> 4;
    const uint64_t hstride = (uint64_t)(a.ffn / 32) * 36;
    using W = MbW<QD>;
    constexpr bool UP = NBD > 0;
    constexpr uint32_t WB = UP ? 64 * NBD * QD::BB : 0;   // the tile's weight bytes (a multiple of 16)
    constexpr uint32_t WCH = WB / 16, WPT = UP ? (WCH + 255) / 256 : 1;   // 16-byte chunks, per thread
    // LDS: [the tile's rows WB][h blocks][256 zero bytes]
    uint8_t *const lt = lds;
    const uint32_t xo = WB, zo = xo + (UP ? nb : MB_DN_CHUNK) * MBX_BYTES;
    if (tid < 64) *(uint32_t *)(lt + zo + 4 * tid) = 0u;   // read only after the tile's first barrier
    const uint32_t nent = (uint32_t)meta[1];
    for (uint32_t t = blockIdx.x;; t += gridDim.x) {
        const uint32_t bi = t / ntile, rt = t % ntile;
        // (tiles past the entries read the last record and leave)
        const int32_t *rec = meta + mb_big_off(P) + MB_REC * min(bi, P - 1);
        // independent loads: the record, this thread's pair (slots past the
        // count hold pair 0)
        const int4 hd = *(const int4 *)rec;
        const uint32_t sp = (uint32_t)rec[4 + si];
        if (bi >= nent) break;   // whole workgroup
        const int32_t e = hd.x;
        const uint32_t cnt = (uint32_t)hd.z;
        const int32_t *pairs = rec + 4;
        const bool shared = (uint32_t)e == a.n_expert;
        const uint8_t *db = shared ? a.down_sh : a.down + (uint64_t)e * a.hidden * rb;
        const uint32_t row0 = 64 * rt + 16 * wave;   // this wave's 16 rows
        const uint8_t *ap = db + (uint64_t)(row0 + arow) * rb;
        const uint8_t *xrow = a.hq8 + (uint64_t)sp * hstride;
        if constexpr (UP) {
            const uint8_t *tw = db + (uint64_t)(64 * rt) * rb;
            uint4 wv[WPT];
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (uint32_t k = 0; k < WPT; k++) wv[k] = ld16(tw + 16 * min(tid + 256 * k, WCH - 1));   // (clamped)
            XPart xv[NBD];
#pragma unroll
            for (int b = 0; b < NBD; b++) xv[b] = mbx_load(xrow, b);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();   // the previous tile is done with the LDS
#pragma unroll
            for (uint32_t k = 0; k < WPT; k++)
                if (tid + 256 * k < WCH) *(uint4 *)(lt + 16 * (tid + 256 * k)) = wv[k];
#pragma unroll
            for (int b = 0; b < NBD; b++) mbx_put(mbx_carve(lt + xo + b * MBX_BYTES), xv[b], si < cnt);
            __syncthreads();
        }
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        constexpr int UNR = UP ? NBD : 1;
#pragma unroll UNR
        for (uint32_t b = 0; b < nb; b++) {
            W wc;
            if constexpr (!UP) {
                // long rows: the h blocks go through LDS MB_DN_CHUNK at a time
                if (b % MB_DN_CHUNK == 0) {
                    const uint32_t n = min(MB_DN_CHUNK, nb - b);
                    __syncthreads();   // the previous chunk (or tile) is done with the LDS
                    for (uint32_t c = 0; c < n; c++)
                        mbx_put(mbx_carve(lt + xo + c * MBX_BYTES), mbx_load(xrow, b + c), si < cnt);
                    __syncthreads();
                }
                wc.load_row(ap + b * QD::BB, kc);
            } else {
                wc.load_row_lds(lt, (16 * wave + arow) * (uint32_t)rb + b * QD::BB, kc);
            }
            const uint32_t xs = xo + (UP ? b : b % MB_DN_CHUNK) * MBX_BYTES;
            const MbX x = mbx_carve(lt + xs);
            float rs[16];   // the lane's row scales for this block
            wc.row_scales(rs);
            // activation operand of lane (pair column arow, k chunk kc);
            // Q6_K's group-masked halves by address
            const uint32_t bo = xs + MBX_ROW * arow + 8 * kc, zk = zo + 8 * kc;
            const uint32_t b_lo = kc < 2 ? bo : zk, b_hi = kc < 2 ? zk : bo;
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) {   // 32-value sub-blocks
                const long wv = wc.a_op(j);
                const float4 d8 = *(const float4 *)(x.d8 + 16 * j + p0);
                const float d8v[4] = {d8.x, d8.y, d8.z, d8.w};
                if constexpr (QD::TYPE == T_Q6_K) {
                    const v4i d1 = mfma16(*(const long *)(lt + b_lo + 32 * j), wv);   // [pair][row]
                    const v4i d2 = mfma16(*(const long *)(lt + b_hi + 32 * j), wv);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[i] = fmaf(d8v[i], fmaf(rs[2 * j], (float)d1[i], rs[2 * j + 1] * (float)d2[i]), acc[i]);
                } else {
                    const v4i d = mfma16(mbx_b(x, arow, j, kc), wv);
                    const float4 qs = *(const float4 *)(x.qs + 16 * j + p0);
                    const float qsv[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[i] = fmaf(d8v[i], fmaf(rs[2 * j], (float)d[i], -(rs[2 * j + 1] * qsv[i])), acc[i]);
                }
            }
            // the sums formed here: sunk into the store branch below, the
            // arithmetic kept every block's MFMA results live at once
            asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
        }
        const uint32_t row = row0 + arow;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (p0 + i < cnt) a.yp[(uint64_t)pairs[p0 + i] * a.hidden + row] = acc[i];
    }
}

// y_t[row] = sum over slots in rank order of w * yp[pair]
__global__ void __launch_bounds__(256) k_mb_combine(const float *__restrict__ yp, const float *__restrict__ w,
                                                    uint32_t T, uint32_t n_sel, uint32_t S, uint32_t hidden,
                                                    float *__restrict__ y) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)T * hidden) return;
    const uint32_t t = (uint32_t)(i / hidden), row = (uint32_t)(i % hidden);
    float acc = 0.0f;
    for (uint32_t r = 0; r < S; r++) {
        const float wr = r < n_sel ? w[t * n_sel + r] : 1.0f;
        acc = fmaf(wr, yp[((uint64_t)t * S + r) * hidden + row], acc);
    }
    y[i] = acc;
}

// dynamic LDS of the MFMA gate/up kernel (two x tiles, the block scales, the
// epilogue's sums) and of the MFMA down kernel (up to MB_DN_CHUNK staged h
// blocks and the scale table)
// slices of the gate/up tile: two from two blocks (eight waves per tile)
static uint32_t mb_gu_slices(uint32_t nb) { return nb >= 2 ? 2 : 1; }
static uint32_t mb_lds_gu(uint32_t nb) {
    const uint32_t S = mb_gu_slices(nb);
    return nb * MBX_BYTES + 4 * S * 16 * 8 * 8 + S * 64 * 16 * 4;
}
// bb: the down type's block bytes
static uint32_t mb_lds_dn(uint32_t ffn, uint32_t bb) {
    const uint32_t nb = ffn / 256;
    const uint32_t w = nb <= 3 ? 64 * nb * bb : 0;   // the tile's rows
    return w + (nb <= 3 ? nb : MB_DN_CHUNK) * MBX_BYTES + 256;
}

// Workgroups of kernel k (nt threads, lds bytes of LDS) resident at once on
// the current device (the occupancy API, asked once per kernel, LDS size
// and device; at least one per CU).
static uint32_t resident_wgs(const void *k, uint32_t nt, uint32_t lds) {
    struct Entry {
        const void *k;
        uint32_t lds;
        int dev, n;
    };
    static thread_local Entry cache[16];
    static thread_local uint32_t used = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    for (uint32_t i = 0; i < used; i++)
        if (cache[i].k == k && cache[i].lds == lds && cache[i].dev == dev) return cache[i].n * (uint32_t)device_cu_count();
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, (int)nt, (size_t)lds) != hipSuccess || n < 1) n = 1;
    cache[used % 16] = Entry{k, lds, dev, n};
    used++;
    return (uint32_t)n * (uint32_t)device_cu_count();
}

// The grouped-GEMM grids: every tile the worst case could hold, but no more
// workgroups than fit at once; each workgroup strides over the tiles
// (tile t on workgroup t mod grid). Workgroups past the resident set would
// only queue behind the real tiles to learn that they have none. A strided
// grid is kept a multiple of 8, so tiles nblk (a multiple of 8) apart share
// an XCD as they do unstrided.
static uint32_t mb_grid(uint32_t tiles, uint32_t resident) {
    if (tiles <= resident) return tiles;
    return resident >= 8 ? resident / 8 * 8 : resident;
}

uint32_t moe_batch_lds(uint32_t hidden, uint32_t ffn) {
    uint32_t m = moe_groups_lds(hidden, ffn);
    m = m > mb_lds_gu(hidden / 256) ? m : mb_lds_gu(hidden / 256);
    const uint32_t dn = mb_lds_dn(ffn, Q6K::BB);   // the larger block of the two down types
    return m > dn ? m : dn;
}

hipError_t launch_moe_batch(const MoeArgs &base, uint32_t T, uint32_t min_big, const float *x, float *y, uint8_t *xq,
                            int32_t *meta, hipStream_t s, hipStream_t aux, hipEvent_t fork, hipEvent_t join) {
    const uint32_t S = (uint32_t)base.n_sel + (base.has_shared ? 1u : 0u);
    const uint32_t P = T * S;
    if (T == 0 || T > MB_MAX_T || S == 0 || S > MB_MAX_S || base.n_expert > MB_MAX_E - 1) return hipErrorInvalidValue;
    const uint32_t nq = T * base.hidden / 4;   // quantizer tasks: 8 per 32-value block
    const uint32_t qwg = (nq + 1023) / 1024;
    hipLaunchKernelGGL(k_mb_group, dim3(1 + qwg), dim3(1024), 0, s, base.ids, T, (uint32_t)base.n_sel, S,
                       base.n_expert, min_big, meta, base.err, x, nq, xq);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    MoeArgs a = base;
    a.x = nullptr;
    a.xq = xq;
    a.xq_stride = (uint64_t)(base.hidden / 32) * 36;
    a.bS = S;
    a.bslot = meta + mb_small_off();
    a.bcount = meta;
    a.border = meta + mb_order_off(P);
    // small entries: at most P / 8 + one per expert (each has >= 1 pair)
    const uint32_t ne = base.n_expert + 1;
    const uint32_t max_small = P / MB_GRP + (ne < P ? ne : P);
    // No expert can reach min_big pairs below min_big pairs in all: then the
    // grouped-GEMM kernels are not launched. From MB_FORK_PAIRS pairs they
    // run on the side stream, beside the small-entry kernels (a fork and a
    // join cost ~3-4 us, more than the overlap gains on smaller batches).
    const bool any_big = P >= min_big;
    const bool side = any_big && P >= MB_FORK_PAIRS && aux != s;   // aux == s: one stream
    hipStream_t sb = side ? aux : s;
    if (side && ((e = hipEventRecord(fork, s)) != hipSuccess || (e = hipStreamWaitEvent(aux, fork, 0)) != hipSuccess))
        return e;
    // after the fork every exit joins aux back into s (an unjoined side
    // stream would leave a capture of s unable to end); the first error wins
    auto joined = [&](hipError_t err) -> hipError_t {
        if (!side) return err;
        hipError_t j = hipEventRecord(join, aux);
        if (j == hipSuccess) j = hipStreamWaitEvent(s, join, 0);
        return err != hipSuccess ? err : j;
    };
    if ((e = launch_moe_groups_gu(a, max_small, s)) != hipSuccess) return joined(e);
    if ((e = launch_moe_groups_down(a, max_small, s)) != hipSuccess) return joined(e);
    // grouped entries: each holds 1..16 pairs of one expert with >= min_big
    // pairs, so there are at most P / 16 + P / min_big + 1 of them
    const uint32_t max_big = P / MB_BIG + P / (min_big > 0 ? min_big : 1) + 1;
    auto grid_for = [&](const void *k, uint32_t nt, uint32_t lds, uint32_t tiles_per_entry) {
        return dim3(mb_grid(max_big * tiles_per_entry, resident_wgs(k, nt, lds)));
    };
    const uint32_t nblk = base.ffn / 32;
    const uint32_t nb_gu = base.hidden / 256;
    const uint32_t lds_gu = mb_lds_gu(base.hidden / 256);
    auto go_gu = [&](auto kern) -> hipError_t {
        if (!any_big) return hipSuccess;
        if (lds_gu > 64 * 1024) {
            const hipError_t r = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     (int)lds_gu);
            if (r != hipSuccess) return r;
        }
        const uint32_t nt = 256 * mb_gu_slices(nb_gu);
        hipLaunchKernelGGL(kern, grid_for((const void *)kern, nt, lds_gu, nblk), dim3(nt), lds_gu, sb, a, meta, P);
        return hipGetLastError();
    };
    switch (nb_gu) {
        case 1: e = go_gu(k_mb_gu_mfma<1, 1>); break;
        case 2: e = go_gu(k_mb_gu_mfma<2, 2>); break;
        case 4: e = go_gu(k_mb_gu_mfma<4, 2>); break;
        case 8: e = go_gu(k_mb_gu_mfma<8, 2>); break;
        case 16: e = go_gu(k_mb_gu_mfma<16, 2>); break;
        default: return joined(hipErrorInvalidValue);
    }
    if (e != hipSuccess) return joined(e);
    const uint32_t ntile = (base.hidden + 63) / 64;
    const uint32_t nb_dn = base.ffn / 256;
    const uint32_t lds_dn = mb_lds_dn(base.ffn, base.down_type == T_Q6_K ? Q6K::BB : Q4K::BB);
    auto go_dn = [&](auto kern) -> hipError_t {
        if (!any_big) return hipSuccess;
        if (lds_dn > 64 * 1024) {
            const hipError_t r = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     (int)lds_dn);
            if (r != hipSuccess) return r;
        }
        hipLaunchKernelGGL(kern, grid_for((const void *)kern, 256, lds_dn, ntile), dim3(256), lds_dn, sb, a, meta, P);
        return hipGetLastError();
    };
    if (base.down_type == T_Q6_K) {
        switch (nb_dn) {
            case 1: e = go_dn(k_mb_down_mfma<Q6K, 1>); break;
            case 2: e = go_dn(k_mb_down_mfma<Q6K, 2>); break;
            case 3: e = go_dn(k_mb_down_mfma<Q6K, 3>); break;
            default: e = go_dn(k_mb_down_mfma<Q6K, 0>); break;
        }
    } else {
        switch (nb_dn) {
            case 1: e = go_dn(k_mb_down_mfma<Q4K, 1>); break;
            case 2: e = go_dn(k_mb_down_mfma<Q4K, 2>); break;
            case 3: e = go_dn(k_mb_down_mfma<Q4K, 3>); break;
            default: e = go_dn(k_mb_down_mfma<Q4K, 0>); break;
        }
    }
    if (e == hipSuccess) e = hipGetLastError();
    if ((e = joined(e)) != hipSuccess) return e;
    const uint64_t n = (uint64_t)T * base.hidden;
    hipLaunchKernelGGL(k_mb_combine, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, a.yp, base.wts, T,
                       (uint32_t)base.n_sel, S, base.hidden, y);
    return hipGetLastError();
}

}  // namespace kq
