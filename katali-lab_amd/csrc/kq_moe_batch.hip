// kq_moe_batch.hip — the MoE layer over a batch of tokens (prefill).
//
// y_t = sum_r w_{t,r} Down_e(q8(SiLU(Gate_e x_t) * Up_e x_t)), e = ids[t][r],
// plus the shared expert (weight 1) when present, for T <= 64 tokens.
//
// 1. x_t -> q8_1 (one quantize launch over all tokens).
// 2. k_mb_group (one workgroup): the T*S (token, slot) pairs, S = n_sel +
//    shared, are sorted by expert (stable in pair order). An expert that
//    gathers at least min_big pairs goes to the grouped-GEMM list (in entries
//    of at most 64 pairs), every other pair to the per-pair list.
// 3. Per-pair list: kernels A and B of the single-token layer in batch mode
//    (v_dot4 GEMV; h to the pair's q8_1 row, B's output unweighted to yp).
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

constexpr uint32_t MB_MAX_T = 64;
constexpr uint32_t MB_MAX_S = 17;
constexpr uint32_t MB_MAX_P = MB_MAX_T * MB_MAX_S;
constexpr uint32_t MB_MAX_E = 513;   // routed experts + the shared expert's virtual id

// meta layout (int32): [0] n_small, [1] n_big (grouped entries), [2] error
// bits, [16 ..) small pair list (P), then the grouped list (3 ints per entry:
// expert, first, count <= 64; at most P entries), then order (P pairs sorted
// by expert)
__host__ __device__ inline uint32_t mb_small_off() { return 16; }
__host__ __device__ inline uint32_t mb_big_off(uint32_t P) { return 16 + P; }
__host__ __device__ inline uint32_t mb_order_off(uint32_t P) { return 16 + P + 3 * P; }
uint64_t moe_batch_meta_words(uint32_t P) { return mb_order_off(P) + P; }

__global__ void __launch_bounds__(1024) k_mb_group(const int32_t *__restrict__ ids, uint32_t T, uint32_t n_sel,
                                                   uint32_t S, uint32_t n_expert, uint32_t min_big,
                                                   int32_t *__restrict__ meta, int32_t *__restrict__ err) {
    __shared__ int32_t cnt[MB_MAX_E], off_all[MB_MAX_E], off_small[MB_MAX_E], big_idx[MB_MAX_E];
    __shared__ int32_t exp_of[MB_MAX_P];
    __shared__ int32_t bad;
    const uint32_t P = T * S, tid = threadIdx.x;
    const uint32_t NE = n_expert + 1;   // id n_expert = the shared expert
    for (uint32_t e = tid; e < NE; e += blockDim.x) cnt[e] = 0;
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
    if (tid == 0) {
        int32_t a = 0, sm = 0, nb = 0;
        for (uint32_t e = 0; e < NE; e++) {
            off_all[e] = a;
            a += cnt[e];
            const bool big = cnt[e] >= (int32_t)min_big && cnt[e] > 0;
            off_small[e] = big ? -1 : sm;
            if (!big) sm += cnt[e];
            big_idx[e] = big ? nb : -1;   // first entry of this expert
            if (big) nb += (cnt[e] + 63) / 64;
        }
        meta[0] = sm;
        meta[1] = nb;
        meta[2] = bad ? 2 : 0;
        if (bad) atomicOr(err, 2);
    }
    __syncthreads();
    int32_t *small = meta + mb_small_off(), *bigl = meta + mb_big_off(P), *order = meta + mb_order_off(P);
    for (uint32_t p = tid; p < P; p += blockDim.x) {
        const int32_t e = exp_of[p];
        int32_t rank = 0;
        for (uint32_t q = 0; q < p; q++) rank += exp_of[q] == e;
        order[off_all[e] + rank] = (int32_t)p;
        if (off_small[e] >= 0) small[off_small[e] + rank] = (int32_t)p;
    }
    for (uint32_t e = tid; e < NE; e += blockDim.x) {
        if (big_idx[e] >= 0) {
            for (int32_t k = 0; 64 * k < cnt[e]; k++) {
                const int32_t i = big_idx[e] + k;
                bigl[3 * i + 0] = (int32_t)e;
                bigl[3 * i + 1] = off_all[e] + 64 * k;
                bigl[3 * i + 2] = min(64, cnt[e] - 64 * k);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Shared pieces of the two MFMA kernels
// ---------------------------------------------------------------------------
// The activation chunk of one 256-value block for up to 64 pairs, staged in
// LDS: int8 values [64][256], their q8_1 scales d8 [64][8] and exact sums of
// each 32 values qs [64][8].
struct MbX {
    int8_t *q;
    float *d8;
    int32_t *qs;
};
__device__ __forceinline__ MbX mbx_carve(uint8_t *base) {
    MbX x;
    x.q = (int8_t *)base;
    x.d8 = (float *)(base + 64 * 256);
    x.qs = (int32_t *)(base + 64 * 256 + 64 * 8 * 4);
    return x;
}
constexpr uint32_t MBX_BYTES = 64 * 256 + 2 * 64 * 8 * 4;

// Stage block b of the q8_1 rows of `cnt` pairs: row of local pair i is
// src + row_index(i) * row_bytes. 8 lanes per 36-byte q8_1 block.
template <class RowOf>
__device__ __forceinline__ void mbx_stage(const MbX &x, const uint8_t *src, uint64_t row_bytes, uint32_t cnt,
                                          uint32_t b, RowOf row_of) {
    for (uint32_t task = threadIdx.x; task < 64 * 8 * 8; task += blockDim.x) {
        const uint32_t i = task / 64, sb = (task / 8) % 8, part = task % 8;
        uint32_t q = 0, d = 0;
        if (i < cnt) {
            const uint8_t *blk = src + row_of(i) * row_bytes + (uint64_t)(8 * b + sb) * 36;
            q = *(const uint32_t *)(blk + 4 + 4 * part);
            d = ld_u16(blk);
        }
        *(uint32_t *)(x.q + 256 * i + 32 * sb + 4 * part) = q;
        int s = dot4(q, 0x01010101u, 0);
        s += dpp_i<DPP_XOR1>(s);
        s += dpp_i<DPP_XOR2>(s);
        s += dpp_i<DPP_HALF_MIRROR>(s);
        if (part == 0) {
            x.d8[8 * i + sb] = h2f(d);
            x.qs[8 * i + sb] = s;
        }
    }
}

// B operand: 8 int8 of local pair `col` at k = 32*sb + kc*8
__device__ __forceinline__ long mbx_b(const MbX &x, uint32_t col, uint32_t sb, uint32_t kc) {
    return *(const long *)(x.q + 256 * col + 32 * sb + 8 * kc);
}

// Q4_K A operand: 8 int8 (0..15) of sub-block j of one row's block at k
// chunk kc (values 32*j + 8*kc .. +7): nibbles of qs[32*(j/2) + 8*kc ..]
__device__ __forceinline__ long q4k_a(const uint8_t *blk, uint32_t j, uint32_t kc) {
    const uint2 v = ld8(blk + 16 + 32 * (j >> 1) + 8 * kc);
    const uint32_t sh = 4 * (j & 1), m = 0x0F0F0F0Fu;
    const uint32_t lo = (v.x >> sh) & m, hi = (v.y >> sh) & m;
    return (long)(((uint64_t)hi << 32) | lo);
}

// Four 6-bit values 0..63 (one per byte) -> int8 q6 - 32 per byte without
// cross-byte borrows: x = q ^ 32 is q - 32 as a 6-bit two's complement
// number; copy its bit 5 into bits 6 and 7.
__device__ __forceinline__ uint32_t q6_minus_32(uint32_t q) {
    const uint32_t x = q ^ 0x20202020u, m = x & 0x20202020u;
    return x | (m << 1) | (m << 2);
}

// Q6_K A operand: 8 int8 (q6 - 32) at values v0 .. v0+7 of one row's block
// (v0 % 8 == 0): ql nibble + 2 qh bits, in the block's interleave.
__device__ __forceinline__ long q6k_a(const uint8_t *blk, uint32_t v0) {
    const uint32_t n = v0 / 128, qq = (v0 % 128) / 32, l0 = v0 % 32;
    const uint2 ql = ld8(blk + 64 * n + 32 * (qq & 1) + l0);
    const uint2 qh = ld8(blk + 128 + 32 * n + l0);
    const uint32_t sl = qq >= 2 ? 4 : 0, sh = 2 * qq, m4 = 0x0F0F0F0Fu, m2 = 0x03030303u;
    const uint32_t lo = ((ql.x >> sl) & m4) | (((qh.x >> sh) & m2) << 4);
    const uint32_t hi = ((ql.y >> sl) & m4) | (((qh.y >> sh) & m2) << 4);
    return (long)(((uint64_t)q6_minus_32(hi) << 32) | q6_minus_32(lo));
}

__device__ __forceinline__ v4i mfma16(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Gate/up for one grouped expert: 32 gate + 32 up rows (jb) x all its pairs
// ---------------------------------------------------------------------------
template <int NB>
__global__ void __launch_bounds__(256) k_mb_gu_mfma(MoeArgs a, const int32_t *__restrict__ meta, uint32_t P) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t nblk = a.ffn / 32;
    const uint32_t bi = blockIdx.x / nblk, jb = blockIdx.x % nblk;
    if (bi >= (uint32_t)meta[1]) return;   // whole workgroup, before any barrier
    const int32_t *big = meta + mb_big_off(P) + 3 * bi;
    const int32_t e = big[0], first = big[1], cnt = big[2];
    const int32_t *pairs = meta + mb_order_off(P) + first;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t rb = NB * 144;
    const bool shared = (uint32_t)e == a.n_expert;
    const uint8_t *gb = shared ? a.gate_sh : a.gate + (uint64_t)e * a.ffn * rb;
    const uint8_t *ub = shared ? a.up_sh : a.up + (uint64_t)e * a.ffn * rb;
    // wave w: rows 16w..16w+15 of the 64 (waves 0-1 gate, 2-3 up)
    const uint8_t *wbase = wave < 2 ? gb + (uint64_t)(32 * jb + 16 * wave) * rb : ub + (uint64_t)(32 * jb + 16 * (wave - 2)) * rb;
    const uint32_t arow = lane % 16, kc = lane / 16;   // A: row, k chunk
    const uint32_t dcol = lane % 16, drow0 = 4 * (lane / 16);   // D: pair column, first row
    const uint32_t ntiles = (cnt + 15) / 16;

    const MbX x = mbx_carve(lds);
    float2 *scl = (float2 *)(lds + MBX_BYTES) + 16 * 8 * wave;   // this wave's [16 rows][8 sub-blocks] {d*sc, dmin*m}
    float *gu = (float *)(lds + MBX_BYTES + 4 * 16 * 8 * 8);        // [64 rows][64 pairs]
    float acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[t][i] = 0.0f;

    for (uint32_t b = 0; b < NB; b++) {
        __syncthreads();   // the previous block's LDS is consumed
        mbx_stage(x, a.xq, a.xq_stride, (uint32_t)cnt, b,
                  [&](uint32_t i) { return (uint64_t)((uint32_t)pairs[i] / a.bS); });
        // this wave's 16 row headers of block b -> 8 scale pairs each
        {
            const uint32_t r = lane / 4, g = lane % 4;   // 16 rows x 4 groups
            Q4K::Raw raw;
            raw.h = ld16(wbase + (uint64_t)r * rb + b * 144);
            float ds0, ds1, dm0, dm1;
            Q4K::scales(raw, (int)g, ds0, ds1, dm0, dm1);
            scl[8 * r + 2 * g] = make_float2(ds0, dm0);
            scl[8 * r + 2 * g + 1] = make_float2(ds1, dm1);
        }
        __syncthreads();
        const uint8_t *ablk = wbase + (uint64_t)arow * rb + b * 144;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {
            const long av = q4k_a(ablk, j, kc);
            float2 sc[4];
#pragma unroll
            for (int i = 0; i < 4; i++) sc[i] = scl[8 * (drow0 + i) + j];
#pragma unroll
            for (uint32_t t = 0; t < 4; t++) {
                if (t >= ntiles) break;
                const uint32_t col = 16 * t + dcol;
                const v4i d = mfma16(av, mbx_b(x, 16 * t + arow, j, kc));
                const float d8 = x.d8[8 * col + j], qs = (float)x.qs[8 * col + j];
#pragma unroll
                for (int i = 0; i < 4; i++) acc[t][i] = fmaf(d8, fmaf(sc[i].x, (float)d[i], -(sc[i].y * qs)), acc[t][i]);
            }
        }
    }
    // gate/up of (row, pair) -> LDS, then SiLU-GLU and one q8_1 block per pair
#pragma unroll
    for (uint32_t t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) gu[64 * (16 * wave + drow0 + i) + 16 * t + dcol] = acc[t][i];
    __syncthreads();
    for (uint32_t task = tid; task < 64 * 8; task += blockDim.x) {
        const uint32_t i = task / 8, part = task % 8;
        if (i >= (uint32_t)cnt) break;   // whole 8-lane groups leave together
        float4 h;
        h.x = kq_silu_mul(gu[64 * (4 * part + 0) + i], gu[64 * (32 + 4 * part + 0) + i]);
        h.y = kq_silu_mul(gu[64 * (4 * part + 1) + i], gu[64 * (32 + 4 * part + 1) + i]);
        h.z = kq_silu_mul(gu[64 * (4 * part + 2) + i], gu[64 * (32 + 4 * part + 2) + i]);
        h.w = kq_silu_mul(gu[64 * (4 * part + 3) + i], gu[64 * (32 + 4 * part + 3) + i]);
        uint32_t d16, s16;
        int lo, hi;
        float dd;
        const uint32_t qv = quant_q8_1_part(h, d16, s16, lo, hi, dd);
        uint8_t *blk = a.hq8 + ((uint64_t)pairs[i] * nblk + jb) * 36;
        *(uint32_t *)(blk + 4 + 4 * part) = qv;
        if (part == 0) *(uint32_t *)blk = d16 | (s16 << 16);
    }
}

// ---------------------------------------------------------------------------
// Down for one grouped expert: 64 output rows x all its pairs -> yp
// ---------------------------------------------------------------------------
template <class QD>
__global__ void __launch_bounds__(256) k_mb_down_mfma(MoeArgs a, const int32_t *__restrict__ meta, uint32_t P) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t ntile = (a.hidden + 63) / 64;
    const uint32_t bi = blockIdx.x / ntile, rt = blockIdx.x % ntile;
    if (bi >= (uint32_t)meta[1]) return;
    const int32_t *big = meta + mb_big_off(P) + 3 * bi;
    const int32_t e = big[0], first = big[1], cnt = big[2];
    const int32_t *pairs = meta + mb_order_off(P) + first;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t nb = a.ffn / 256;
    const uint64_t rb = (uint64_t)nb * QD::BB;
    const bool shared = (uint32_t)e == a.n_expert;
    const uint8_t *db = shared ? a.down_sh : a.down + (uint64_t)e * a.hidden * rb;
    const uint32_t row0 = 64 * rt + 16 * wave;   // this wave's 16 rows
    const uint32_t arow = lane % 16, kc = lane / 16;
    const uint32_t dcol = lane % 16, drow0 = 4 * (lane / 16);
    const uint32_t ntiles = (cnt + 15) / 16;
    // rows past hidden read the last row and are not written
    const uint8_t *arow_base = db + (uint64_t)min(row0 + arow, a.hidden - 1) * rb;

    const MbX x = mbx_carve(lds);
    constexpr uint32_t NS = QD::TYPE == T_Q6_K ? 16 : 8;   // scales per block
    float2 *scl = (float2 *)(lds + MBX_BYTES) + 16 * 16 * wave;   // [16 rows][NS] {scale, min}
    const uint64_t hstride = (uint64_t)(a.ffn / 32) * 36;
    float acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[t][i] = 0.0f;

    for (uint32_t b = 0; b < nb; b++) {
        __syncthreads();
        mbx_stage(x, a.hq8, hstride, (uint32_t)cnt, b, [&](uint32_t i) { return (uint64_t)pairs[i]; });
        for (uint32_t task = lane; task < 16 * NS; task += 64) {
            const uint32_t r = task / NS, g = task % NS;
            const uint8_t *blk = db + (uint64_t)min(row0 + r, a.hidden - 1) * rb + b * QD::BB;
            if constexpr (QD::TYPE == T_Q6_K) {
                const float d = h2f(ld_u16(blk + 208));
                scl[NS * r + g] = make_float2(d * (float)(int8_t)blk[192 + g], 0.0f);
            } else {
                Q4K::Raw raw;
                raw.h = ld16(blk);
                float ds0, ds1, dm0, dm1;
                Q4K::scales(raw, (int)(g / 2), ds0, ds1, dm0, dm1);
                scl[NS * r + g] = (g & 1) ? make_float2(ds1, dm1) : make_float2(ds0, dm0);
            }
        }
        __syncthreads();
        const uint8_t *ablk = arow_base + b * QD::BB;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {   // 32-value sub-blocks
            if constexpr (QD::TYPE == T_Q6_K) {
                // two 16-value scale groups: A halves zeroed in turn
                const long av = q6k_a(ablk, 32 * j + 8 * kc);
                const long a_lo = kc < 2 ? av : 0, a_hi = kc < 2 ? 0 : av;
                float s_lo[4], s_hi[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    s_lo[i] = scl[NS * (drow0 + i) + 2 * j].x;
                    s_hi[i] = scl[NS * (drow0 + i) + 2 * j + 1].x;
                }
#pragma unroll
                for (uint32_t t = 0; t < 4; t++) {
                    if (t >= ntiles) break;
                    const uint32_t col = 16 * t + dcol;
                    const long bv = mbx_b(x, 16 * t + arow, j, kc);
                    const v4i d1 = mfma16(a_lo, bv), d2 = mfma16(a_hi, bv);
                    const float d8 = x.d8[8 * col + j];
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[t][i] = fmaf(d8, fmaf(s_lo[i], (float)d1[i], s_hi[i] * (float)d2[i]), acc[t][i]);
                }
            } else {
                const long av = q4k_a(ablk, j, kc);
                float2 sc[4];
#pragma unroll
                for (int i = 0; i < 4; i++) sc[i] = scl[NS * (drow0 + i) + j];
#pragma unroll
                for (uint32_t t = 0; t < 4; t++) {
                    if (t >= ntiles) break;
                    const uint32_t col = 16 * t + dcol;
                    const v4i d = mfma16(av, mbx_b(x, 16 * t + arow, j, kc));
                    const float d8 = x.d8[8 * col + j], qs = (float)x.qs[8 * col + j];
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[t][i] = fmaf(d8, fmaf(sc[i].x, (float)d[i], -(sc[i].y * qs)), acc[t][i]);
                }
            }
        }
    }
#pragma unroll
    for (uint32_t t = 0; t < 4; t++) {
        const uint32_t col = 16 * t + dcol;
        if (col >= (uint32_t)cnt) continue;
        float *yrow = a.yp + (uint64_t)pairs[col] * a.hidden;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t row = row0 + drow0 + i;
            if (row < a.hidden) yrow[row] = acc[t][i];
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

hipError_t launch_moe_batch(const MoeArgs &base, uint32_t T, uint32_t min_big, const float *x, float *y, uint8_t *xq,
                            int32_t *meta, hipStream_t s) {
    const uint32_t S = (uint32_t)base.n_sel + (base.has_shared ? 1u : 0u);
    const uint32_t P = T * S;
    if (T == 0 || T > MB_MAX_T || S == 0 || S > MB_MAX_S || base.n_expert > MB_MAX_E - 1) return hipErrorInvalidValue;
    hipError_t e = launch_quantize_q8_1(x, (uint64_t)T * base.hidden, xq, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_mb_group, dim3(1), dim3(1024), 0, s, base.ids, T, (uint32_t)base.n_sel, S, base.n_expert,
                       min_big, meta, base.err);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    MoeArgs a = base;
    a.x = nullptr;
    a.xq = xq;
    a.xq_stride = (uint64_t)(base.hidden / 32) * 36;
    a.bS = S;
    a.bslot = meta + mb_small_off();
    a.bcount = meta;
    if ((e = launch_moe_pairs_gu(a, P, s)) != hipSuccess) return e;
    // grouped entries: each holds 1..64 pairs of one expert with >= min_big
    // pairs, so there are at most P / 64 + P / min_big + 1 of them
    const uint32_t max_big = P / 64 + P / (min_big > 0 ? min_big : 1) + 1;
    const uint32_t nblk = base.ffn / 32;
    const uint32_t lds_gu = MBX_BYTES + 4 * 16 * 8 * 8 + 64 * 64 * 4;
    switch (base.hidden / 256) {
        case 1: hipLaunchKernelGGL(k_mb_gu_mfma<1>, dim3(max_big * nblk), dim3(256), lds_gu, s, a, meta, P); break;
        case 2: hipLaunchKernelGGL(k_mb_gu_mfma<2>, dim3(max_big * nblk), dim3(256), lds_gu, s, a, meta, P); break;
        case 4: hipLaunchKernelGGL(k_mb_gu_mfma<4>, dim3(max_big * nblk), dim3(256), lds_gu, s, a, meta, P); break;
        case 8: hipLaunchKernelGGL(k_mb_gu_mfma<8>, dim3(max_big * nblk), dim3(256), lds_gu, s, a, meta, P); break;
        case 16: hipLaunchKernelGGL(k_mb_gu_mfma<16>, dim3(max_big * nblk), dim3(256), lds_gu, s, a, meta, P); break;
        default: return hipErrorInvalidValue;
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = launch_moe_pairs_down(a, P, s)) != hipSuccess) return e;
    const uint32_t ntile = (base.hidden + 63) / 64;
    const uint32_t lds_dn = MBX_BYTES + 4 * 16 * 16 * 8;
    if (base.down_type == T_Q6_K)
        hipLaunchKernelGGL(k_mb_down_mfma<Q6K>, dim3(max_big * ntile), dim3(256), lds_dn, s, a, meta, P);
    else
        hipLaunchKernelGGL(k_mb_down_mfma<Q4K>, dim3(max_big * ntile), dim3(256), lds_dn, s, a, meta, P);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const uint64_t n = (uint64_t)T * base.hidden;
    hipLaunchKernelGGL(k_mb_combine, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, a.yp, base.wts, T,
                       (uint32_t)base.n_sel, S, base.hidden, y);
    return hipGetLastError();
}

}  // namespace kq
