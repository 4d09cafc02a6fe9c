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
//    v_mfma_i32_16x16x32_i8 (A = 16 weight rows x 32 k, B = 32 k x 16 pairs)
//    with the block scales applied per 32-value sub-block in fp32 (per
//    16-value group for Q6_K: two MFMAs per 32 k, each with the other half of
//    A zeroed), same q8_1 definitions as the GEMV path.
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
// banks), their q8_1 scales d8 [16][8] and exact sums of each 32 values qs
// [16][8].
constexpr uint32_t MBX_ROW = 272;
struct MbX {
    int8_t *q;
    float *d8;
    int32_t *qs;
};
__device__ __forceinline__ MbX mbx_carve(uint8_t *base) {
    MbX x;
    x.q = (int8_t *)base;
    x.d8 = (float *)(base + 16 * MBX_ROW);
    x.qs = (int32_t *)(base + 16 * MBX_ROW + 16 * 8 * 4);
    return x;
}
constexpr uint32_t MBX_BYTES = 16 * MBX_ROW + 2 * 16 * 8 * 4;

// Staging split (16 pairs per workgroup): thread t takes local pair t / 16,
// q8_1 block 8b + (t / 2) % 8 of that pair's row and half t % 2 of its
// values.
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
    const uint32_t i = threadIdx.x >> 4, sb = (threadIdx.x >> 1) & 7, half = threadIdx.x & 1;
    const uint4 q = valid ? v.q : make_uint4(0, 0, 0, 0);
    *(uint4 *)(x.q + MBX_ROW * i + 32 * sb + 16 * half) = q;
    int s = dot4(q.x, 0x01010101u, 0);
    s = dot4(q.y, 0x01010101u, s);
    s = dot4(q.z, 0x01010101u, s);
    s = dot4(q.w, 0x01010101u, s);
    s += dpp_i<DPP_XOR1>(s);   // the block's other half
    if (half == 0) {
        x.d8[8 * i + sb] = valid ? h2f(v.h & 0xFFFFu) : 0.0f;
        x.qs[8 * i + sb] = s;
    }
}

// B operand: 8 int8 of local pair `col` at k = 32*sb + kc*8
__device__ __forceinline__ long mbx_b(const MbX &x, uint32_t col, uint32_t sb, uint32_t kc) {
    return *(const long *)(x.q + MBX_ROW * col + 32 * sb + 8 * kc);
}

// Four 6-bit values 0..63 (one per byte) -> int8 q6 - 32 per byte without
// cross-byte borrows: x = q ^ 32 is q - 32 as a 6-bit two's complement
// number; copy its bit 5 into bits 6 and 7.
__device__ __forceinline__ uint32_t q6_minus_32(uint32_t q) {
    const uint32_t x = q ^ 0x20202020u, m = x & 0x20202020u;
    return x | (m << 1) | (m << 2);
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
    static constexpr uint32_t NS = 16;   // {d*sc, 0} per 16-value group
    uint2 ql[4], qh[2];
    uint32_t sc, d;
    __device__ __forceinline__ void load(const uint8_t *ablk, const uint8_t *hblk, uint32_t kc) {
#pragma unroll
        for (int n = 0; n < 2; n++) {
            ql[2 * n] = ld8(ablk + 64 * n + 8 * kc);
            ql[2 * n + 1] = ld8(ablk + 64 * n + 32 + 8 * kc);
            qh[n] = ld8(ablk + 128 + 32 * n + 8 * kc);
        }
        sc = ld4(hblk + 192 + 4 * (threadIdx.x & 3));
        d = ld_u16(hblk + 208);
    }
    __device__ __forceinline__ void put_scales(float2 *scl) const {
        const uint32_t lane = threadIdx.x & 63, g = lane & 3, r = lane >> 2;
        const float dd = h2f(d);
#pragma unroll
        for (int k = 0; k < 4; k++) scl[NS * r + 4 * g + k] = make_float2(dd * (float)(int)(int8_t)(sc >> (8 * k)), 0.0f);
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
// and the entry's record (pairs inline) at once, every weight load behind
// them, then the pairs' activation blocks: up to 8 blocks all staged in LDS
// at once behind one barrier (one LDS buffer per block), else a ring of
// three in registers two blocks ahead over two LDS buffers.
// ---------------------------------------------------------------------------
template <int NB>
__global__ void __launch_bounds__(256) k_mb_gu_mfma(MoeArgs a, const int32_t *__restrict__ meta, uint32_t P) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t nblk = a.ffn / 32;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t rb = NB * 144;
    const uint32_t arow = lane % 16, kc = lane / 16;   // A: row, k chunk
    const uint32_t dcol = lane % 16, drow0 = 4 * (lane / 16);   // D: pair column, first row
    const uint32_t si = tid >> 4;   // this thread's staging pair
    constexpr bool UP = NB <= 8;   // every block's weights in registers, every x block in LDS, at once
    constexpr uint32_t NBUF = UP ? NB : 2;
    {
        const uint32_t t = blockIdx.x;
        const uint32_t bi = t / nblk, jb = t % nblk;
        // (a grid sized for the most entries a batch could hold has tiles past
        // the P records: they read the last record and leave)
        const int32_t *rec = meta + mb_big_off(P) + MB_REC * min(bi, P - 1);
        // independent loads: the entry count, the record, this thread's pair
        // (slots past the count hold pair 0)
        const uint32_t nent = (uint32_t)meta[1];
        const int4 hd = *(const int4 *)rec;
        const uint32_t sp = (uint32_t)rec[4 + si];
        if (bi >= nent) return;   // whole workgroup, before any barrier
        uint8_t *const lt = lds;
        float2 *scl = (float2 *)(lt + NBUF * MBX_BYTES) + 16 * 8 * wave;   // this wave's [16 rows][8 sub-blocks] {d*sc, dmin*m}
        float *gu = (float *)(lt + NBUF * MBX_BYTES + 4 * 16 * 8 * 8);      // [64 rows][16 pairs]
        const int32_t e = hd.x;
        const uint32_t cnt = (uint32_t)hd.z;
        const int32_t *pairs = rec + 4;
        const bool shared = (uint32_t)e == a.n_expert;
        const uint8_t *gb = shared ? a.gate_sh : a.gate + (uint64_t)e * a.ffn * rb;
        const uint8_t *ub = shared ? a.up_sh : a.up + (uint64_t)e * a.ffn * rb;
        // wave w: rows 16w..16w+15 of the 64 (waves 0-1 gate, 2-3 up)
        const uint8_t *wbase = wave < 2 ? gb + (uint64_t)(32 * jb + 16 * wave) * rb
                                        : ub + (uint64_t)(32 * jb + 16 * (wave - 2)) * rb;
        const uint8_t *ap = wbase + (uint64_t)arow * rb, *hp = wbase + (uint64_t)(lane >> 2) * rb;
        const uint8_t *xrow = a.xq + (uint64_t)(sp / a.bS) * a.xq_stride;
        MbW<Q4K> w[UP ? NB : 1];
        XPart xv[UP ? NB : 3];
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (UP) {
            // x first: its wait (in issue order) then waits for no weight
#pragma unroll
            for (int b = 0; b < NB; b++) xv[b] = mbx_load(xrow, b);
#pragma unroll
            for (int b = 0; b < NB; b++) w[b].load(ap + b * 144, hp + b * 144, kc);
        } else {
            w[0].load(ap, hp, kc);
            xv[0] = mbx_load(xrow, 0);
            xv[1] = mbx_load(xrow, NB > 1 ? 1 : 0);
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (UP) {
#pragma unroll
            for (int b = 0; b < NB; b++) mbx_put(mbx_carve(lt + b * MBX_BYTES), xv[b], si < cnt);
            __syncthreads();
        }
        // each (row, pair) value is the pairwise sum of its sub-block terms,
        // pushed in sub-block order (kernel A's q8_1-path dot, bit for bit)
        constexpr int LV = log2c<NB>() + 1;
        float stk[4][LV];
        static_for<0, NB>([&](auto bc) {   // unrolled: registers indexed by constants
            constexpr uint32_t b = decltype(bc)::value;
            __builtin_amdgcn_sched_barrier(0);   // one block's operands live at a time
            if constexpr (!UP) {
                if constexpr (b % 2 == 0) __syncthreads();   // the buffers written next are free (blocks b-2, b-1)
                mbx_put(mbx_carve(lt + (b % 2) * MBX_BYTES), xv[b % 3], si < cnt);
                xv[(b + 2) % 3] = mbx_load(xrow, b + 2 < (uint32_t)NB ? b + 2 : NB - 1);   // clamped, not skipped
                if constexpr (b > 0) w[0].load(ap + b * 144, hp + b * 144, kc);
                __syncthreads();
            }
            const MbW<Q4K> &wc = w[UP ? b : 0];
            const MbX x = mbx_carve(lt + (UP ? b : b % 2) * MBX_BYTES);
            wc.put_scales(scl);   // wave-private table
            wave_sync_lds();
            float t[4][8];   // the block's 8 sub-block terms per (row, pair)
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) {
                const long av = wc.a_op(j);
                const v4i d = mfma16(av, mbx_b(x, arow, j, kc));   // exact isum of sub-block 8b + j
                const float d8 = x.d8[8 * dcol + j], qs = (float)x.qs[8 * dcol + j];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float2 sc = scl[8 * (drow0 + i) + j];
                    const float A = sc.x * d8, B = sc.y * d8;
                    t[i][j] = fmaf(A, (float)d[i], -(B * qs));
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float s = ((t[i][0] + t[i][1]) + (t[i][2] + t[i][3])) + ((t[i][4] + t[i][5]) + (t[i][6] + t[i][7]));
                float sb = s;
                asm volatile("" : "+v"(sb));   // formed here: sinking the block's arithmetic past the
                                               // next barriers would keep its LDS reads live and spill
                pw_push<b, 0>(stk[i], sb);   // blocks: the tree's levels above 8 sub-blocks
            }
            wave_sync_lds();   // the table is rewritten for the next block
        });
        // gate/up of (row, pair) -> LDS, then SiLU-GLU and one q8_1 block per pair
#pragma unroll
        for (int i = 0; i < 4; i++) gu[16 * (16 * wave + drow0 + i) + dcol] = stk[i][LV - 1];   // after block NB - 1: the whole row
        __syncthreads();
        if (tid < 16 * 8) {
            const uint32_t i = tid / 8, part = tid % 8;
            if (i < cnt) {   // whole 8-lane groups take this branch together
                float4 h;
                h.x = kq_silu_mul(gu[16 * (4 * part + 0) + i], gu[16 * (32 + 4 * part + 0) + i]);
                h.y = kq_silu_mul(gu[16 * (4 * part + 1) + i], gu[16 * (32 + 4 * part + 1) + i]);
                h.z = kq_silu_mul(gu[16 * (4 * part + 2) + i], gu[16 * (32 + 4 * part + 2) + i]);
                h.w = kq_silu_mul(gu[16 * (4 * part + 3) + i], gu[16 * (32 + 4 * part + 3) + i]);
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
// gate/up kernel; the pairs' h rows staged once per tile.
// ---------------------------------------------------------------------------
template <class QD, int NBD>
__global__ void __launch_bounds__(256) k_mb_down_mfma(MoeArgs a, const int32_t *__restrict__ meta, uint32_t P) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t ntile = (a.hidden + 63) / 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t nb = NBD > 0 ? (uint32_t)NBD : a.ffn / 256;
    const uint64_t rb = (uint64_t)nb * QD::BB;
    const uint32_t arow = lane % 16, kc = lane / 16;
    const uint32_t dcol = lane % 16, drow0 = 4 * (lane / 16);
    const uint32_t si = tid >> 4;
    const uint64_t hstride = (uint64_t)(a.ffn / 32) * 36;
    using W = MbW<QD>;
    constexpr uint32_t NS = W::NS;
    constexpr bool UP = NBD > 0;
    // every block's weights and activations at once for a compile-time block
    // count (up to 3 blocks: more spills); else one block at a time
    {
        const uint32_t t = blockIdx.x;
        const uint32_t bi = t / ntile, rt = t % ntile;
        // (a grid sized for the most entries a batch could hold has tiles past
        // the P records: they read the last record and leave)
        const int32_t *rec = meta + mb_big_off(P) + MB_REC * min(bi, P - 1);
        // independent loads: the entry count, the record, this thread's pair
        // (slots past the count hold pair 0)
        const uint32_t nent = (uint32_t)meta[1];
        const int4 hd = *(const int4 *)rec;
        const uint32_t sp = (uint32_t)rec[4 + si];
        if (bi >= nent) return;   // whole workgroup, before any barrier
        uint8_t *const lt = lds;
        float2 *scl = (float2 *)(lt + (UP ? nb : MB_DN_CHUNK) * MBX_BYTES) + 16 * 16 * wave;   // [16 rows][NS] {scale, min}
        const int32_t e = hd.x;
        const uint32_t cnt = (uint32_t)hd.z;
        const int32_t *pairs = rec + 4;
        const bool shared = (uint32_t)e == a.n_expert;
        const uint8_t *db = shared ? a.down_sh : a.down + (uint64_t)e * a.hidden * rb;
        const uint32_t row0 = 64 * rt + 16 * wave;   // this wave's 16 rows
        // rows past hidden read the last row and are not written
        const uint8_t *ap = db + (uint64_t)min(row0 + arow, a.hidden - 1) * rb;
        const uint8_t *hp = db + (uint64_t)min(row0 + (lane >> 2), a.hidden - 1) * rb;
        W w[UP ? NBD : 1];
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < (UP ? NBD : 1); b++) w[b].load(ap + b * QD::BB, hp + b * QD::BB, kc);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *xrow = a.hq8 + (uint64_t)sp * hstride;
        if constexpr (UP) {
            XPart xv[NBD];
#pragma unroll
            for (int b = 0; b < NBD; b++) xv[b] = mbx_load(xrow, b);
            __syncthreads();   // the previous tile is done with the LDS
#pragma unroll
            for (int b = 0; b < NBD; b++) mbx_put(mbx_carve(lt + b * MBX_BYTES), xv[b], si < cnt);
            __syncthreads();
        }
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll(UP ? NBD : 1)
        for (uint32_t b = 0; b < nb; b++) {
            if constexpr (!UP) {
                // long rows: the h blocks go through LDS MB_DN_CHUNK at a time
                if (b % MB_DN_CHUNK == 0) {
                    const uint32_t n = min(MB_DN_CHUNK, nb - b);
                    __syncthreads();   // the previous chunk (or tile) is done with the LDS
                    for (uint32_t c = 0; c < n; c++)
                        mbx_put(mbx_carve(lt + c * MBX_BYTES), mbx_load(xrow, b + c), si < cnt);
                    __syncthreads();
                }
                w[0].load(ap + b * QD::BB, hp + b * QD::BB, kc);
            }
            const W &wc = w[UP ? b : 0];
            const MbX x = mbx_carve(lt + (UP ? b : b % MB_DN_CHUNK) * MBX_BYTES);
            wc.put_scales(scl);   // wave-private table
            wave_sync_lds();
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) {   // 32-value sub-blocks
                const long av = wc.a_op(j);
                const long bv = mbx_b(x, arow, j, kc);
                const float d8 = x.d8[8 * dcol + j];
                if constexpr (QD::TYPE == T_Q6_K) {
                    // two 16-value scale groups: A halves zeroed in turn
                    const long a_lo = kc < 2 ? av : 0, a_hi = kc < 2 ? 0 : av;
                    const v4i d1 = mfma16(a_lo, bv), d2 = mfma16(a_hi, bv);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float s_lo = scl[NS * (drow0 + i) + 2 * j].x, s_hi = scl[NS * (drow0 + i) + 2 * j + 1].x;
                        acc[i] = fmaf(d8, fmaf(s_lo, (float)d1[i], s_hi * (float)d2[i]), acc[i]);
                    }
                } else {
                    const v4i d = mfma16(av, bv);
                    const float qs = (float)x.qs[8 * dcol + j];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float2 sc = scl[NS * (drow0 + i) + j];
                        acc[i] = fmaf(d8, fmaf(sc.x, (float)d[i], -(sc.y * qs)), acc[i]);
                    }
                }
                // the sums formed here: sunk into the store branch below, the
                // arithmetic kept every block's MFMA results live at once
                asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
            }
            wave_sync_lds();   // the table is rewritten for the next block
        }
        if (dcol < cnt) {
            float *yrow = a.yp + (uint64_t)pairs[dcol] * a.hidden;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t row = row0 + drow0 + i;
                if (row < a.hidden) yrow[row] = acc[i];
            }
        }
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
static uint32_t mb_lds_gu(uint32_t nb) { return (nb <= 8 ? nb : 2) * MBX_BYTES + 4 * 16 * 8 * 8 + 64 * 16 * 4; }
static uint32_t mb_lds_dn(uint32_t ffn) {
    const uint32_t nb = ffn / 256;
    return (nb <= 3 ? nb : MB_DN_CHUNK) * MBX_BYTES + 4 * 16 * 16 * 8;
}

uint32_t moe_batch_lds(uint32_t hidden, uint32_t ffn) {
    uint32_t m = moe_groups_lds(hidden, ffn);
    m = m > mb_lds_gu(hidden / 256) ? m : mb_lds_gu(hidden / 256);
    return m > mb_lds_dn(ffn) ? m : mb_lds_dn(ffn);
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
    auto grid_for = [&](uint32_t tiles_per_entry) { return dim3(max_big * tiles_per_entry); };
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
        hipLaunchKernelGGL(kern, grid_for(nblk), dim3(256), lds_gu, sb, a, meta, P);
        return hipGetLastError();
    };
    switch (nb_gu) {
        case 1: e = go_gu(k_mb_gu_mfma<1>); break;
        case 2: e = go_gu(k_mb_gu_mfma<2>); break;
        case 4: e = go_gu(k_mb_gu_mfma<4>); break;
        case 8: e = go_gu(k_mb_gu_mfma<8>); break;
        case 16: e = go_gu(k_mb_gu_mfma<16>); break;
        default: return joined(hipErrorInvalidValue);
    }
    if (e != hipSuccess) return joined(e);
    const uint32_t ntile = (base.hidden + 63) / 64;
    const uint32_t nb_dn = base.ffn / 256;
    const uint32_t lds_dn = mb_lds_dn(base.ffn);
    auto go_dn = [&](auto kern) -> hipError_t {
        if (!any_big) return hipSuccess;
        if (lds_dn > 64 * 1024) {
            const hipError_t r = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     (int)lds_dn);
            if (r != hipSuccess) return r;
        }
        hipLaunchKernelGGL(kern, grid_for(ntile), dim3(256), lds_dn, sb, a, meta, P);
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
