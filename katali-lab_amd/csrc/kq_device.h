// kq_device.h — device-side building blocks for the Q4_K / Q6_K x q8_1 path on
// gfx950 (CDNA4, wave64).
//
// Formats (the public GGUF block layouts, as decoded by the reference at
// vendor/katali_gguf_dense/src/gguf_dtype.c:328-335,350-358,429-452,487-512):
//   Q4_K  144 B / 256 values: d f16 @0, dmin f16 @2, 12 B packed 6-bit
//         scales/mins @4, 128 B nibbles @16. qs[32g..32g+31] holds values
//         64g..64g+31 in the low nibbles and 64g+32..64g+63 in the high ones.
//   Q6_K  210 B / 256 values: ql[128] @0, qh[64] @128, int8 sc[16] @192,
//         d f16 @208. Value e = 128n + 32t + l takes ql[64n+l+32(t&1)] (low
//         nibble for t<2, high for t>=2) and bits 2t..2t+1 of qh[32n+l];
//         scale sc[e/16].
//   Q8_1   36 B / 32 values: d f16 @0, s f16 @2, int8 qs[32] @4.
//
// Work decomposition: one "item" is the share of a super-block that one lane
// dots: 16 bytes of Q4_K nibbles (8 items per block, 32 values) or 48 bytes of
// Q6_K ql/ql/qh (4 items per block, 64 values). Integer partial sums are exact
// (v_dot4_i32_i8); scales are applied in fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kq {

constexpr uint32_t T_F32 = 0, T_Q8_1 = 9, T_Q4_K = 12, T_Q6_K = 14;
constexpr int WAVE = 64;

// ---------------------------------------------------------------------------
// scalar helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint32_t h16) {
    _Float16 h;
    const uint16_t v = (uint16_t)h16;
    __builtin_memcpy(&h, &v, 2);
    return (float)h;
}
// f32 -> f16, round to nearest even, of the ROUNDED f32 value. The empty asm
// pins f in a register: without it the compiler may fuse the producing
// multiply into a mixed-precision FMA that rounds the exact product straight
// to f16 (one rounding instead of two), which differs on f16 ties.
__device__ __forceinline__ uint32_t f2h_rne(float f) {
    asm("" : "+v"(f));
    const _Float16 h = (_Float16)f;   // v_cvt_f16_f32, round to nearest even
    uint16_t v;
    __builtin_memcpy(&v, &h, 2);
    return v;
}
// 16-byte load from any byte address (the gfx950 code model allows unaligned
// global dwordx4 loads; the compiler emits them itself for byte-aligned memcpy).
__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
__device__ __forceinline__ uint2 ld8(const uint8_t *p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
// Read kernel arguments into SGPRs at this point. The compiler otherwise
// loads each argument from the kernarg segment at its first use, which for a
// weight base pointer is a scalar-memory round trip between a dependent load
// (the routing) and the weight stream it starts.
template <class T>
__device__ __forceinline__ void pin_arg(T v) {
    asm volatile("" ::"s"(v));
}
template <class... T>
__device__ __forceinline__ void pin_args(T... v) {
    (pin_arg(v), ...);
}
// Materialize a register-held value at this point: it is computed (and any
// load it comes from waited for) here, and later uses read these registers
// instead of the computation being sunk past later code.
template <class T>
__device__ __forceinline__ void pin_vregs(T &v) {
    static_assert(sizeof(T) % 4 == 0, "pin_vregs: whole dwords");
    uint32_t w[sizeof(T) / 4];
    __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
    for (uint32_t k = 0; k < sizeof(T) / 4; k++) asm volatile("" : "+v"(w[k]));
    __builtin_memcpy(&v, w, sizeof(T));
}
__device__ __forceinline__ uint32_t ld4(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// s_waitcnt immediate for "vmcnt(0)" alone on gfx9: vmcnt in bits 3:0 and
// 15:14 (0), expcnt 6:4 and lgkmcnt 11:8 at their maxima (no wait).
constexpr int VMCNT0 = 0x0F70;

// Lane exchanges inside aligned groups of 4 / 8 / 16 lanes on the VALU (DPP),
// no LDS round trip: quad_perm [1,0,3,2] and [2,3,0,1] (partner = lane ^ 1,
// lane ^ 2), row_half_mirror (lane ^ 7 inside 8) and row_mirror (lane ^ 15
// inside 16). A butterfly over masks {1, 2, 7} or {1, 2, 7, 15} visits every
// lane of the group once, so it reduces exactly like the xor butterfly.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
// row_ror 8 / 4: lane k of a 16-lane row takes lane (k + 8) % 16 / (k + 4) % 16
constexpr int DPP_ROR8 = 0x128, DPP_ROR4 = 0x124;

// Sum R per-lane values over the 64 lanes of a wave for R rows at once: each
// halving step sends the half of the rows the partner keeps, then the
// remaining offsets finish a plain butterfly. Partners differ in lane bit 5
// (v_permlane32_swap), bit 4 (v_permlane16_swap), then inside 16-lane rows
// by DPP: lane ^ 15, lane ^ 7, lane ^ 2, lane ^ 1 (these masks span the low
// 4 bits, so every lane's value is counted once). Afterwards every lane holds
// the full sum of row (lane >> (6 - log2 R)) & (R - 1).
//
// v_permlane32_swap(X, Y) gives r0 = {X[0..31], Y[0..31]} and
// r1 = {X[32..63], Y[32..63]} (lane halves), so r0 + r1 is X[l] + X[l+32] in
// the lower half and Y[l-32] + Y[l] in the upper half; v_permlane16_swap does
// the same for odd/even 16-lane rows.
template <int OFF>
__device__ __forceinline__ float swap_sum(float x, float y) {
    static_assert(OFF == 32 || OFF == 16, "swap_sum crosses 32 or 16 lanes");
    if constexpr (OFF == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}
template <int OFF>
__device__ __forceinline__ float row_partner(float v) {   // OFF in {8, 4, 2, 1}
    if constexpr (OFF == 8) return dpp_f<DPP_MIRROR>(v);
    else if constexpr (OFF == 4) return dpp_f<DPP_HALF_MIRROR>(v);
    else if constexpr (OFF == 2) return dpp_f<DPP_XOR2>(v);
    else return dpp_f<DPP_XOR1>(v);
}
template <int N, int OFF, int R>
__device__ __forceinline__ void reduce_halve(float (&acc)[R], int lane) {
    if constexpr (N > 1) {
        constexpr int HALF = N / 2;
        if constexpr (OFF >= 16) {
#pragma unroll
            for (int i = 0; i < HALF; i++) acc[i] = swap_sum<OFF>(acc[i], acc[i + HALF]);
        } else {
            const bool upper = lane & OFF;
#pragma unroll
            for (int i = 0; i < HALF; i++) {
                const float send = upper ? acc[i] : acc[i + HALF];
                const float keep = upper ? acc[i + HALF] : acc[i];
                acc[i] = keep + row_partner<OFF>(send);
            }
        }
        reduce_halve<HALF, OFF / 2, R>(acc, lane);
    }
}
template <int OFF>
__device__ __forceinline__ float butterfly_from(float v) {
    if constexpr (OFF >= 16) v = swap_sum<OFF>(v, v);
    else if constexpr (OFF >= 1) v += row_partner<OFF>(v);
    if constexpr (OFF > 1) return butterfly_from<OFF / 2>(v);
    else return v;
}
template <int R>
__device__ __forceinline__ float reduce_rows(float (&acc)[R]) {
    const int lane = threadIdx.x & 63;
    reduce_halve<R, 32, R>(acc, lane);
    constexpr int LOG = R >= 16 ? 4 : (R >= 8 ? 3 : (R >= 4 ? 2 : (R >= 2 ? 1 : 0)));
    if constexpr (LOG < 6) return butterfly_from<(32 >> LOG)>(acc[0]);
    else return acc[0];
}

// Device-coherent 32-bit accesses (relaxed, agent scope): the store reaches
// the point every XCD's L2 reads through and the load does not answer from a
// stale line of its own XCD's L2, with no cache-wide write-back or
// invalidate. The one-launch layers' exchanges and the single-launch argmax's
// partials travel this way.
__device__ __forceinline__ void st_dev(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev2(uint32_t *p) {   // p 8-byte aligned
    return __hip_atomic_load((uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev2(uint32_t *p, uint64_t v) {   // p 8-byte aligned
    __hip_atomic_store((uint64_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A 64-bit word for pollers on the writer's own XCD only: the store ends in
// that XCD's L2 (the vector L1 writes through) and is not written through to
// memory, and an agent-scope load (ld_dev2) from any CU of the XCD answers
// from that L2 line. Under a streaming load this hand-off measured 1.17 us
// per exchange round against 1.75 us with st_dev2 (32 workgroups of one
// XCD, 200 rounds, no word missed). A poller on another XCD may never see
// the word: callers check the workgroup's XCD first (xcc_id).
__device__ __forceinline__ void st_xcd2(uint32_t *p, uint64_t v) {   // p 8-byte aligned
    asm volatile("global_store_dwordx2 %0, %1, off" ::"v"(p), "v"(v) : "memory");
}
// the XCD (accelerator complex die) this wave runs on, 0..7
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 15u;
}

// ---------------------------------------------------------------------------
// Pairwise sums over lanes (lane bit 0 first): the q8_1 path's row dot sums
// its per-sub-block terms t_0 .. t_{n-1} pairwise, sum(t[0..n)) =
// sum(t[0..n/2)) + sum(t[n/2..n)), and lane l holds t_l, so combining the
// lane bits from the lowest up forms exactly that tree. Every partner below
// is lane ^ OFF; fp32 addition commutes, so both partners of a pair hold the
// same bits afterwards.
// ---------------------------------------------------------------------------
constexpr int DPP_ROW_SHL4 = 0x104, DPP_ROW_SHR4 = 0x114;
template <int OFF>
__device__ __forceinline__ float xor_lane(float v) {   // OFF in {1, 2, 4, 8}
    if constexpr (OFF == 1) return dpp_f<DPP_XOR1>(v);
    else if constexpr (OFF == 2) return dpp_f<DPP_XOR2>(v);
    else if constexpr (OFF == 8) return dpp_f<DPP_ROR8>(v);   // row_ror 8 inside 16 lanes is lane ^ 8
    else {
        // lane ^ 4: banks 0 and 2 of a row (lanes 0-3, 8-11) take lane + 4
        // (row_shl 4), banks 1 and 3 take lane - 4 (row_shr 4)
        const int x = __float_as_int(v);
        int t = __builtin_amdgcn_update_dpp(0, x, DPP_ROW_SHL4, 0xF, 0x5, false);
        t = __builtin_amdgcn_update_dpp(t, x, DPP_ROW_SHR4, 0xF, 0xA, false);
        return __int_as_float(t);
    }
}
// N values per lane (virtual rows) summed over the 64 lanes at once: the
// step at lane bit s sends half of the remaining rows to the partner (lanes
// with bit s set keep the upper half), so after log2(N) steps each lane
// holds one row, whose remaining lane bits then sum by a plain butterfly.
// Lane l ends with the whole sum of virtual row pw_row<N>(l).
template <int N, int OFF, int R>
__device__ __forceinline__ void pw_halve(float (&acc)[R], int lane) {
    if constexpr (N > 1) {
        constexpr int HALF = N / 2;
        if constexpr (OFF >= 16) {
#pragma unroll
            for (int i = 0; i < HALF; i++) acc[i] = swap_sum<OFF>(acc[i], acc[i + HALF]);
        } else {
            const bool upper = lane & OFF;
#pragma unroll
            for (int i = 0; i < HALF; i++) {
                const float send = upper ? acc[i] : acc[i + HALF];
                const float keep = upper ? acc[i + HALF] : acc[i];
                acc[i] = keep + xor_lane<OFF>(send);
            }
        }
        pw_halve<HALF, OFF * 2, R>(acc, lane);
    }
}
template <int OFF>
__device__ __forceinline__ float pw_butterfly(float v) {
    if constexpr (OFF <= 32) {
        if constexpr (OFF >= 16) v = swap_sum<OFF>(v, v);
        else v += xor_lane<OFF>(v);
        return pw_butterfly<OFF * 2>(v);
    } else {
        return v;
    }
}
template <int N>
constexpr int log2c() { return N <= 1 ? 0 : 1 + log2c<N / 2>(); }
template <int N>
__device__ __forceinline__ float pw_reduce(float (&acc)[N]) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "pw_reduce: N a power of 2 <= 64");
    pw_halve<N, 1, N>(acc, (int)(threadIdx.x & 63));
    return pw_butterfly<N>(acc[0]);
}
// The virtual row lane l holds after pw_reduce<N>: lane bit s carries row
// bit log2(N) - 1 - s (the row index bit-reversed into the low lane bits).
template <int N>
__device__ __forceinline__ uint32_t pw_row(uint32_t lane) {
    constexpr int L = log2c<N>();
    if constexpr (L == 0) return 0;
    else return __builtin_bitreverse32(lane) >> (32 - L);
}

// LDS writes of this wave become visible to its own other lanes (a
// wavefront-scope release/acquire pair around a wave barrier; no workgroup
// barrier)
__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// sum over aligned groups of W lanes (W a power of 2 up to 64), all lanes get
// it: DPP inside 16-lane rows, then v_permlane16_swap / v_permlane32_swap
// across rows (each partner pair adds the same two values, so every lane of
// a group ends with the same bits)
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group_sum: W must be a power of 2 <= 64");
    if constexpr (W >= 2) v += dpp_f<DPP_XOR1>(v);
    if constexpr (W >= 4) v += dpp_f<DPP_XOR2>(v);
    if constexpr (W >= 8) v += dpp_f<DPP_HALF_MIRROR>(v);
    if constexpr (W >= 16) v += dpp_f<DPP_MIRROR>(v);
    if constexpr (W >= 32) v = swap_sum<16>(v, v);
    if constexpr (W >= 64) v = swap_sum<32>(v, v);
    return v;
}

// sum of a double over the 64 lanes of a wave, every lane gets it: the same
// DPP and permlane-swap butterfly as group_sum<64>, on both 32-bit halves
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)dpp_i<CTRL>((int)(uint32_t)u);
    const uint32_t hi = (uint32_t)dpp_i<CTRL>((int)(uint32_t)(u >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
template <int OFF>
__device__ __forceinline__ double swap_sum_f64(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
    uint32_t l0, l1, h0, h1;
    if constexpr (OFF == 32) {
        const auto rl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto rh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        l0 = rl[0]; l1 = rl[1]; h0 = rh[0]; h1 = rh[1];
    } else {
        const auto rl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        const auto rh = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        l0 = rl[0]; l1 = rl[1]; h0 = rh[0]; h1 = rh[1];
    }
    return __longlong_as_double((long long)(((uint64_t)h0 << 32) | l0)) +
           __longlong_as_double((long long)(((uint64_t)h1 << 32) | l1));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_d<DPP_XOR1>(v);
    v += dpp_d<DPP_XOR2>(v);
    v += dpp_d<DPP_HALF_MIRROR>(v);
    v += dpp_d<DPP_MIRROR>(v);
    v = swap_sum_f64<16>(v);
    return swap_sum_f64<32>(v);
}

// The engine's AVX2 horizontal sum of 16 fp32 accumulators
// (vendor/katali_gguf_dense/src/gguf_simd_x86.c:80-89, 118: a0 + a1, then
// hsum256_ps) over the 16 lanes of a DPP row, lane k holding accumulator k:
// v_k = a_k + a_{k+8} (row_ror 8 is lane ^ 8), l_k = v_k + v_{k+4} (row_ror 4;
// v is 8-periodic after the first step), then (l0 + l1) + (l2 + l3) (lane ^ 1,
// lane ^ 2). Every add is commutative, so each lane of the row ends with the
// same bits.
__device__ __forceinline__ float hsum16_avx2_order(float a) {
    float v = a + dpp_f<DPP_ROR8>(a);
    v = v + dpp_f<DPP_ROR4>(v);
    v = v + dpp_f<DPP_XOR1>(v);
    return v + dpp_f<DPP_XOR2>(v);
}

// exp by Cody-Waite reduction x = n*ln2 + r (ln2 split into a 15-bit high part,
// exact for |n| <= 256, and a low correction) and a degree-7 Taylor polynomial
// for e^r, |r| <= ln2/2, evaluated by Horner with fused multiply-adds. Every
// step is an IEEE fp32 operation with a single rounding, so the CPU oracle
// reproduces it bit for bit. Input clamped to [-80, 88].
__device__ __forceinline__ float kq_expf(float x) {
    x = fminf(fmaxf(x, -80.0f), 88.0f);
    const float n = rintf(x * 1.44269502f);
    float r = fmaf(-n, 0.693145752f, x);
    r = fmaf(-n, 1.42860677e-06f, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return p * __uint_as_float((uint32_t)((int)n + 127) << 23);
}
// SiLU-GLU: g / (1 + exp(-g)) * u (correctly rounded division).
__device__ __forceinline__ float kq_silu_mul(float g, float u) {
    const float e = kq_expf(-g);
    const float den = 1.0f + e;
    const float s = g / den;
    return s * u;
}

// ---------------------------------------------------------------------------
// q8_1 activation in LDS
//   qs   int8[K]        the quantized values
//   d8   float[K/32]    f16-decoded block scale (what dequantization uses)
//   qs16 int[K/16]      exact sums of each 16-value half block
// ---------------------------------------------------------------------------
struct Act {
    int8_t *qs;
    float *d8;
    int *qs16;
};
__host__ __device__ constexpr uint32_t act_bytes(uint32_t K) { return K + K / 8 + K / 4; }
__device__ __forceinline__ Act act_carve(uint8_t *base, uint32_t K) {
    Act a;
    a.qs = (int8_t *)base;
    a.d8 = (float *)(base + K);
    a.qs16 = (int *)(base + K + K / 8);
    return a;
}

// Quantize one 32-value block with 8 lanes x 4 values (lanes part=0..7 of an
// aligned 8-lane group). Returns the packed 4 int8 of this lane; the block's
// f16 d / s and half-block sums are returned through refs (valid in all 8 lanes).
// Definition (block_q8_1): amax = max|x|; d = amax/127; id = d ? 1/d : 0;
// q = roundf(x*id); d_f16 = rne(d); s_f16 = rne((float)sum(q) * d).
__device__ __forceinline__ uint32_t quant_q8_1_part(float4 v, uint32_t &d16, uint32_t &s16,
                                                    int &sum_lo, int &sum_hi, float &d_dec) {
    float am = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    am = fmaxf(am, dpp_f<DPP_XOR1>(am));
    am = fmaxf(am, dpp_f<DPP_XOR2>(am));
    am = fmaxf(am, dpp_f<DPP_HALF_MIRROR>(am));
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q0 = (int)roundf(v.x * id), q1 = (int)roundf(v.y * id);
    const int q2 = (int)roundf(v.z * id), q3 = (int)roundf(v.w * id);
    int s = q0 + q1 + q2 + q3;
    s += dpp_i<DPP_XOR1>(s);
    s += dpp_i<DPP_XOR2>(s);          // sum of this lane's half block (4 lanes)
    const int other = dpp_i<DPP_HALF_MIRROR>(s);
    const int part = threadIdx.x & 7;
    sum_lo = part < 4 ? s : other;
    sum_hi = part < 4 ? other : s;
    const int total = s + other;
    d16 = f2h_rne(d);
    s16 = f2h_rne((float)total * d);
    d_dec = h2f(d16);
    return (uint32_t)(q0 & 255) | ((uint32_t)(q1 & 255) << 8) | ((uint32_t)(q2 & 255) << 16) |
           ((uint32_t)(q3 & 255) << 24);
}

// Stage an fp32 activation of K values (K % 256 == 0) into LDS as q8_1.
// Block-wide; the caller synchronises afterwards.
__device__ __forceinline__ void act_stage_from_f32(const float *__restrict__ x, uint32_t K, Act a) {
    const uint32_t n = K / 32 * 8;   // 8 lanes per block
    for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) {
        const uint32_t blk = t >> 3, part = t & 7;
        const float4 v = *(const float4 *)(x + 32 * blk + 4 * part);
        uint32_t d16, s16;
        int lo, hi;
        float dd;
        const uint32_t q = quant_q8_1_part(v, d16, s16, lo, hi, dd);
        *(uint32_t *)(a.qs + 32 * blk + 4 * part) = q;
        if (part == 0) {
            a.d8[blk] = dd;
            a.qs16[2 * blk] = lo;
            a.qs16[2 * blk + 1] = hi;
        }
    }
}

// Half-block sums of a q8_1 block held as 4 values per lane over an aligned
// 8-lane group: lo = values 0..15, hi = 16..31 (valid in all 8 lanes).
__device__ __forceinline__ void q8_part_sums(uint32_t q, int &lo, int &hi) {
    int s = dot4(q, 0x01010101u, 0);
    s += dpp_i<DPP_XOR1>(s);
    s += dpp_i<DPP_XOR2>(s);          // sum of this lane's half block (4 lanes)
    const int other = dpp_i<DPP_HALF_MIRROR>(s);
    const bool low = (threadIdx.x & 7) < 4;
    lo = low ? s : other;
    hi = low ? other : s;
}

// Stage K values of global q8_1 blocks into LDS.
__device__ __forceinline__ void act_stage_from_q8(const uint8_t *__restrict__ xq, uint32_t K, Act a) {
    const uint32_t n = K / 32 * 8;
    for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) {
        const uint32_t blk = t >> 3, part = t & 7;
        const uint8_t *b = xq + 36 * blk;
        const uint32_t q = *(const uint32_t *)(b + 4 + 4 * part);
        *(uint32_t *)(a.qs + 32 * blk + 4 * part) = q;
        int lo, hi;
        q8_part_sums(q, lo, hi);
        if (part == 0) {
            a.d8[blk] = h2f(ld_u16(b));
            a.qs16[2 * blk] = lo;
            a.qs16[2 * blk + 1] = hi;
        }
    }
}

// fp32 activation in LDS for the float-activation GEMV: x[K] plus exact-order
// sums of every 16 values (xsum16[K/16], left to right).
struct ActF {
    float *x;
    float *xs16;
};
__host__ __device__ constexpr uint32_t actf_bytes(uint32_t K) { return K * 4 + K / 4; }
__device__ __forceinline__ ActF actf_carve(uint8_t *base, uint32_t K) {
    ActF a;
    a.x = (float *)base;
    a.xs16 = (float *)(base + 4 * K);
    return a;
}
__device__ __forceinline__ void actf_stage(const float *__restrict__ x, uint32_t K, ActF a) {
    for (uint32_t t = threadIdx.x; t < K / 4; t += blockDim.x)
        *(float4 *)(a.x + 4 * t) = *(const float4 *)(x + 4 * t);
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < K / 16; t += blockDim.x) {
        float s = 0.0f;
        for (int i = 0; i < 16; i++) s += a.x[16 * t + i];
        a.xs16[t] = s;
    }
}

// ---------------------------------------------------------------------------
// Q4_K item: lane chunk c (0..7) of a block = 16 bytes of nibbles
//   group g = c/2, half hh = c%2: low nibbles -> values 64g+16hh+i (sub-block
//   2g), high nibbles -> 64g+32+16hh+i (sub-block 2g+1), i = 0..15.
// ---------------------------------------------------------------------------
struct Q4K {
    static constexpr uint32_t TYPE = T_Q4_K;
    static constexpr int IPB = 8;          // items per block
    static constexpr uint32_t BB = 144;    // block bytes
    struct Raw {
        uint4 h, q;
    };
    __device__ static __forceinline__ Raw load(const uint8_t *blk, int c) {
        Raw r;
        r.h = ld16(blk);
        r.q = ld16(blk + 16 + 16 * c);
        return r;
    }
    // exact partial sums over the lane's 16 low / 16 high values
    __device__ static __forceinline__ void isums(const Raw &r, int c, const int8_t *actb, int &slo, int &shi) {
        const int g = c >> 1, hh = c & 1;
        const int8_t *al = actb + 64 * g + 16 * hh;
        const int4 xl = *(const int4 *)al;
        const int4 xh = *(const int4 *)(al + 32);
        const uint32_t m = 0x0F0F0F0Fu;
        slo = dot4(r.q.x & m, xl.x, 0);
        slo = dot4(r.q.y & m, xl.y, slo);
        slo = dot4(r.q.z & m, xl.z, slo);
        slo = dot4(r.q.w & m, xl.w, slo);
        shi = dot4((r.q.x >> 4) & m, xh.x, 0);
        shi = dot4((r.q.y >> 4) & m, xh.y, shi);
        shi = dot4((r.q.z >> 4) & m, xh.z, shi);
        shi = dot4((r.q.w >> 4) & m, xh.w, shi);
    }
    // integer sums of one 16-byte nibble chunk against preloaded activations
    __device__ static __forceinline__ void isums_x(const uint4 &q, const int4 &xl, const int4 &xh, int &slo,
                                                   int &shi) {
        const uint32_t m = 0x0F0F0F0Fu;
        slo = dot4(q.x & m, xl.x, 0);
        slo = dot4(q.y & m, xl.y, slo);
        slo = dot4(q.z & m, xl.z, slo);
        slo = dot4(q.w & m, xl.w, slo);
        shi = dot4((q.x >> 4) & m, xh.x, 0);
        shi = dot4((q.y >> 4) & m, xh.y, shi);
        shi = dot4((q.z >> 4) & m, xh.z, shi);
        shi = dot4((q.w >> 4) & m, xh.w, shi);
    }
    // scale/min pairs for sub-blocks 2g and 2g+1 (get_scale_min_k4, two at once)
    __device__ static __forceinline__ void scales(const Raw &r, int g, float &ds0, float &ds1, float &dm0,
                                                  float &dm1) {
        const uint32_t sh = 16u * (uint32_t)(g & 1);
        const uint32_t p1 = r.h.y >> sh, p2 = r.h.z >> sh, p3 = r.h.w >> sh;
        uint32_t sc, mn;
        if (g < 2) {
            sc = p1 & 0x3F3Fu;
            mn = p2 & 0x3F3Fu;
        } else {
            sc = (p3 & 0x0F0Fu) | ((p1 >> 2) & 0x3030u);
            mn = ((p3 >> 4) & 0x0F0Fu) | ((p2 >> 2) & 0x3030u);
        }
        const float d = h2f(r.h.x & 0xFFFFu), dmin = h2f(r.h.x >> 16);
        ds0 = d * (float)(sc & 0xFFu);
        ds1 = d * (float)((sc >> 8) & 0xFFu);
        dm0 = dmin * (float)(mn & 0xFFu);
        dm1 = dmin * (float)((mn >> 8) & 0xFFu);
    }
    // fp32 contribution of the item against a q8_1 activation (block b)
    __device__ static __forceinline__ float finish(const Raw &r, int c, const Act &a, uint32_t b, int slo, int shi) {
        const int g = c >> 1, hh = c & 1;
        float ds0, ds1, dm0, dm1;
        scales(r, g, ds0, ds1, dm0, dm1);
        const uint32_t k = 8 * b + 2 * g;   // q8 block of the low nibbles
        const float vlo = fmaf(ds0, (float)slo, -(dm0 * (float)a.qs16[2 * k + hh]));
        const float vhi = fmaf(ds1, (float)shi, -(dm1 * (float)a.qs16[2 * k + 2 + hh]));
        return fmaf(a.d8[k], vlo, a.d8[k + 1] * vhi);
    }
    __device__ static __forceinline__ float dot_q8(const Raw &r, int c, const Act &a, uint32_t b) {
        int slo, shi;
        isums(r, c, a.qs + 256 * b, slo, shi);
        return finish(r, c, a, b, slo, shi);
    }
    // the item's nibbles unpacked once, for dots against several activations
    struct Unp {
        uint4 lo, hi;
    };
    __device__ static __forceinline__ Unp unpack(const Raw &r) {
        const uint32_t m = 0x0F0F0F0Fu;
        Unp u;
        u.lo = make_uint4(r.q.x & m, r.q.y & m, r.q.z & m, r.q.w & m);
        u.hi = make_uint4((r.q.x >> 4) & m, (r.q.y >> 4) & m, (r.q.z >> 4) & m, (r.q.w >> 4) & m);
        return u;
    }
    // dot_q8 with the nibbles unpacked beforehand (the same sums and float ops)
    __device__ static __forceinline__ float dot_q8_u(const Raw &r, const Unp &u, int c, const Act &a, uint32_t b) {
        const int g = c >> 1, hh = c & 1;
        const int8_t *al = a.qs + 256 * b + 64 * g + 16 * hh;
        const int4 xl = *(const int4 *)al;
        const int4 xh = *(const int4 *)(al + 32);
        int slo = dot4(u.lo.x, xl.x, 0);
        slo = dot4(u.lo.y, xl.y, slo);
        slo = dot4(u.lo.z, xl.z, slo);
        slo = dot4(u.lo.w, xl.w, slo);
        int shi = dot4(u.hi.x, xh.x, 0);
        shi = dot4(u.hi.y, xh.y, shi);
        shi = dot4(u.hi.z, xh.z, shi);
        shi = dot4(u.hi.w, xh.w, shi);
        return finish(r, c, a, b, slo, shi);
    }
    // fp32 contribution of the item against a float activation (block b)
    __device__ static __forceinline__ float dot_f32(const Raw &r, int c, const ActF &a, uint32_t b) {
        const int g = c >> 1, hh = c & 1;
        const float *xl = a.x + 256 * b + 64 * g + 16 * hh;
        const float *xh = xl + 32;
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float al = 0.0f, ah = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 vl = *(const float4 *)(xl + 4 * j);
            const float4 vh = *(const float4 *)(xh + 4 * j);
            const uint32_t lo = q[j] & 0x0F0F0F0Fu, hi = (q[j] >> 4) & 0x0F0F0F0Fu;
            al = fmaf((float)(lo & 0xFFu), vl.x, al);
            al = fmaf((float)((lo >> 8) & 0xFFu), vl.y, al);
            al = fmaf((float)((lo >> 16) & 0xFFu), vl.z, al);
            al = fmaf((float)(lo >> 24), vl.w, al);
            ah = fmaf((float)(hi & 0xFFu), vh.x, ah);
            ah = fmaf((float)((hi >> 8) & 0xFFu), vh.y, ah);
            ah = fmaf((float)((hi >> 16) & 0xFFu), vh.z, ah);
            ah = fmaf((float)(hi >> 24), vh.w, ah);
        }
        float ds0, ds1, dm0, dm1;
        scales(r, g, ds0, ds1, dm0, dm1);
        const float *s16 = a.xs16 + 16 * b + 4 * g + hh;
        return fmaf(ds0, al, -(dm0 * s16[0])) + fmaf(ds1, ah, -(dm1 * s16[2]));
    }
};

// ---------------------------------------------------------------------------
// Q6_K item: lane chunk c (0..3) of a block: half n = c/2, lane group k = c%2;
// 48 bytes (ql[64n+16k..+15], ql[64n+32+16k..+15], qh[32n+16k..+15]) give
// 4 x 16 values t = 0..3 at 128n + 32t + 16k + i with scale sc[8n+2t+k].
// ---------------------------------------------------------------------------
struct Q6K {
    static constexpr uint32_t TYPE = T_Q6_K;
    static constexpr int IPB = 4;
    static constexpr uint32_t BB = 210;
    struct Raw {
        uint4 A, B, H;
        uint2 sc;
        uint32_t d;
    };
    __device__ static __forceinline__ Raw load(const uint8_t *blk, int c) {
        const int n = c >> 1, k = c & 1;
        Raw r;
        r.A = ld16(blk + 64 * n + 16 * k);
        r.B = ld16(blk + 64 * n + 32 + 16 * k);
        r.H = ld16(blk + 128 + 32 * n + 16 * k);
        r.sc = ld8(blk + 192 + 8 * n);
        r.d = ld_u16(blk + 208);
        return r;
    }
    // 6-bit values of quarter t for dword j (4 values), unsigned 0..63
    __device__ static __forceinline__ uint32_t q6(uint32_t A, uint32_t B, uint32_t H, int t) {
        const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
        switch (t) {
            case 0: return (A & m4) | ((H << 4) & m2);
            case 1: return (B & m4) | ((H << 2) & m2);
            case 2: return ((A >> 4) & m4) | (H & m2);
            default: return ((B >> 4) & m4) | ((H >> 2) & m2);
        }
    }
    // exact sums of (q6 - 32) * q8 for the four 16-value groups of the item
    __device__ static __forceinline__ void isums(const Raw &r, int c, const Act &a, uint32_t b, int s[4]) {
        const int n = c >> 1, k = c & 1;
        const uint32_t A[4] = {r.A.x, r.A.y, r.A.z, r.A.w};
        const uint32_t B[4] = {r.B.x, r.B.y, r.B.z, r.B.w};
        const uint32_t H[4] = {r.H.x, r.H.y, r.H.z, r.H.w};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t e0 = 256 * b + 128 * n + 32 * t + 16 * k;
            const int4 x = *(const int4 *)(a.qs + e0);
            int acc = dot4(q6(A[0], B[0], H[0], t), x.x, 0);
            acc = dot4(q6(A[1], B[1], H[1], t), x.y, acc);
            acc = dot4(q6(A[2], B[2], H[2], t), x.z, acc);
            acc = dot4(q6(A[3], B[3], H[3], t), x.w, acc);
            s[t] = acc - 32 * a.qs16[e0 / 16];
        }
    }
    __device__ static __forceinline__ float scale(const Raw &r, int k, int t) {
        const uint32_t w = (t < 2) ? r.sc.x : r.sc.y;
        const int sh = 8 * (2 * (t & 1) + k);
        return (float)(int)(int8_t)(w >> sh);
    }
    __device__ static __forceinline__ float finish(const Raw &r, int c, const Act &a, uint32_t b, const int s[4]) {
        const int n = c >> 1, k = c & 1;
        const float d = h2f(r.d);
        const uint32_t k8 = 8 * b + 4 * n;   // q8 block of quarter 0
        float acc = a.d8[k8] * ((d * scale(r, k, 0)) * (float)s[0]);
#pragma unroll
        for (int t = 1; t < 4; t++) acc = fmaf(a.d8[k8 + t], (d * scale(r, k, t)) * (float)s[t], acc);
        return acc;
    }
    __device__ static __forceinline__ float dot_q8(const Raw &r, int c, const Act &a, uint32_t b) {
        int s[4];
        isums(r, c, a, b, s);
        return finish(r, c, a, b, s);
    }
    // the item's 6-bit values unpacked once (quarter t, dword j), for dots
    // against several activations
    struct Unp {
        uint32_t v[4][4];
    };
    __device__ static __forceinline__ Unp unpack(const Raw &r) {
        const uint32_t A[4] = {r.A.x, r.A.y, r.A.z, r.A.w};
        const uint32_t B[4] = {r.B.x, r.B.y, r.B.z, r.B.w};
        const uint32_t H[4] = {r.H.x, r.H.y, r.H.z, r.H.w};
        Unp u;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int j = 0; j < 4; j++) u.v[t][j] = q6(A[j], B[j], H[j], t);
        return u;
    }
    // dot_q8 with the values unpacked beforehand (the same sums and float ops)
    __device__ static __forceinline__ float dot_q8_u(const Raw &r, const Unp &u, int c, const Act &a, uint32_t b) {
        const int n = c >> 1, k = c & 1;
        int s[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t e0 = 256 * b + 128 * n + 32 * t + 16 * k;
            const int4 x = *(const int4 *)(a.qs + e0);
            int acc = dot4(u.v[t][0], x.x, 0);
            acc = dot4(u.v[t][1], x.y, acc);
            acc = dot4(u.v[t][2], x.z, acc);
            acc = dot4(u.v[t][3], x.w, acc);
            s[t] = acc - 32 * a.qs16[e0 / 16];
        }
        return finish(r, c, a, b, s);
    }
    __device__ static __forceinline__ float dot_f32(const Raw &r, int c, const ActF &a, uint32_t b) {
        const int n = c >> 1, k = c & 1;
        const uint32_t A[4] = {r.A.x, r.A.y, r.A.z, r.A.w};
        const uint32_t B[4] = {r.B.x, r.B.y, r.B.z, r.B.w};
        const uint32_t H[4] = {r.H.x, r.H.y, r.H.z, r.H.w};
        const float d = h2f(r.d);
        float acc = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t e0 = 256 * b + 128 * n + 32 * t + 16 * k;
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t v = q6(A[j], B[j], H[j], t);
                const float4 x = *(const float4 *)(a.x + e0 + 4 * j);
                s = fmaf((float)(v & 0xFFu), x.x, s);
                s = fmaf((float)((v >> 8) & 0xFFu), x.y, s);
                s = fmaf((float)((v >> 16) & 0xFFu), x.z, s);
                s = fmaf((float)(v >> 24), x.w, s);
            }
            s = fmaf(-32.0f, a.xs16[e0 / 16], s);
            acc = fmaf(d * scale(r, k, t), s, acc);
        }
        return acc;
    }
};

}  // namespace kq
