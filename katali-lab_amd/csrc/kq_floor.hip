// kq_floor.hip — the floors a MoE layer is measured against: how fast one
// layer's bytes stream through the chip with no arithmetic, in the layer's
// own launch shapes (256 workgroups of 1024 threads, one per CU).
//
//   kind 0: one launch reads a (the layer's bytes) once;
//   kind 1: two launches, a then b (kernels A and B's split: gate/up, then
//           down);
//   kind 2: one launch, a then b, with the XCD-sliced layer's two in-kernel
//           waits and its overlap: once its share of a is in, a workgroup
//           issues the loads of its share of b (the layer's down rows go out
//           after its gate/up dots), then waits for the 32 workgroups of its
//           XCD (the h exchange), folds b, and waits for the 8 workgroups
//           that share its output rows, one per XCD (the partials'
//           exchange).
// Every workgroup reads a contiguous 1/256 share with 16-byte loads, all of
// a thread's loads of a share issued before any is used, and folds them into
// a value stored only if it equals a constant no data here produces (so the
// loads cannot be dropped). Waits are bounded (FLOOR_SPIN_LIMIT polls) and
// generation-tagged like the layer's: a workgroup's word in `sync` advances
// once per launch, nothing is cleared between launches or graph replays.
#include "kq_device.h"
#include "kq_launch.h"

namespace kq {

constexpr uint32_t FLOOR_G = 256, FLOOR_NT = 1024, FLOOR_PER = 8;   // loads in flight per thread
constexpr uint32_t FLOOR_SYNC_WORDS = 3 * FLOOR_G;                  // generations, phase-1 and phase-2 words
constexpr uint32_t FLOOR_SPIN_LIMIT = 1u << 20;                     // polls of a wait before it gives up (about a second)
// dynamic LDS (unused) above half a CU's 160 KiB: one workgroup per CU, as
// the layer's workgroups are placed
constexpr uint32_t FLOOR_LDS = 96 * 1024;

__device__ __forceinline__ uint32_t floor_ld(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void floor_st(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// this workgroup's share [lo, hi) of n16 16-byte words
struct Share {
    uint64_t lo, hi;
};
__device__ __forceinline__ Share floor_range(uint64_t n16) {
    const uint64_t share = (n16 + FLOOR_G - 1) / FLOOR_G;
    const uint64_t lo = (uint64_t)blockIdx.x * share;
    return {lo, min(lo + share, n16)};
}
// one round of FLOOR_PER loads per thread from base (clamped into the share)
__device__ __forceinline__ void floor_issue(const uint4 *src, Share sh, uint64_t base, uint4 (&v)[FLOOR_PER]) {
#pragma unroll
    for (uint32_t i = 0; i < FLOOR_PER; i++) {
        const uint64_t k = base + threadIdx.x + (uint64_t)FLOOR_NT * i;
        v[i] = src[min(k, sh.hi - 1)];   // clamped, not guarded: all loads in flight
    }
}
__device__ __forceinline__ uint32_t floor_fold(const uint4 (&v)[FLOOR_PER]) {
    uint32_t acc = 0;
#pragma unroll
    for (uint32_t i = 0; i < FLOOR_PER; i++) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    return acc;
}
// the rounds of the share from `from` on, FLOOR_PER words per thread at a time
__device__ __forceinline__ uint32_t floor_rest(const uint4 *src, Share sh, uint64_t from) {
    uint32_t acc = 0;
    for (uint64_t base = from; base < sh.hi; base += (uint64_t)FLOOR_NT * FLOOR_PER) {
        uint4 v[FLOOR_PER];
        floor_issue(src, sh, base, v);
        acc ^= floor_fold(v);
    }
    return acc;
}
__device__ __forceinline__ uint32_t floor_share(const uint4 *src, uint64_t n16) {
    const Share sh = floor_range(n16);
    return floor_rest(src, sh, sh.lo);
}

__global__ void __launch_bounds__(FLOOR_NT) k_floor_read(const uint4 *a, uint64_t na, uint32_t *sink) {
    const uint32_t acc = floor_share(a, na);
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// wait until words[i] == tag for the workgroups i = first + stride k, k < n
// (lanes of wave 0; two rounds of polls in flight, as the layer's h polls),
// bounded
__device__ __forceinline__ void floor_wait(uint32_t *words, uint32_t first, uint32_t stride, uint32_t n, uint32_t tag) {
    if (threadIdx.x >= 64) return;
    const uint32_t lane = threadIdx.x;
    uint32_t *w = words + first + stride * min(lane, n - 1);
    uint32_t va = floor_ld(w), vb;
    for (uint32_t spins = 0; spins < FLOOR_SPIN_LIMIT; spins++) {
        vb = floor_ld(w);
        if (__all(va == tag)) break;
        va = floor_ld(w);
        if (__all(vb == tag)) break;
    }
}

__global__ void __launch_bounds__(FLOOR_NT) k_floor_two_phase(const uint4 *a, uint64_t na, const uint4 *b, uint64_t nb,
                                                              uint32_t *sync, uint32_t *sink) {
    const uint32_t wg = blockIdx.x, xcd = wg % 8, li = wg / 8;
    uint32_t *gen = sync, *w1 = sync + FLOOR_G, *w2 = sync + 2 * FLOOR_G;
    const uint32_t tag = floor_ld(gen + wg) + 1;
    uint32_t acc = floor_share(a, na);
    const Share sb = floor_range(nb);
    uint4 vb[FLOOR_PER];
    if (sb.lo < sb.hi) floor_issue(b, sb, sb.lo, vb);   // b's first round in flight through the wait
    __syncthreads();
    if (threadIdx.x == 0) floor_st(w1 + wg, tag);
    floor_wait(w1, xcd, 8, FLOOR_G / 8, tag);   // the 32 workgroups of this XCD
    __syncthreads();
    if (sb.lo < sb.hi) {
        acc ^= floor_fold(vb);
        acc ^= floor_rest(b, sb, sb.lo + (uint64_t)FLOOR_NT * FLOOR_PER);
    }
    __syncthreads();
    if (threadIdx.x == 0) floor_st(w2 + wg, tag);
    floor_wait(w2, 8 * li, 1, 8, tag);           // the 8 workgroups of these output rows
    if (threadIdx.x == 0) floor_st(gen + wg, tag);
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// The exchange probe: how long one word takes from a workgroup to a waiting
// workgroup, with nothing else running. XCHG_G single-wave workgroups; lane 0
// of workgroup b and of its partner p take turns for `rounds` rounds (b < p
// sends first: one round is two one-way exchanges), each waiting for the
// other's word with this call's tag before it sends its own. kind 0: p = b ^ 8
// (the same XCD group as the XCD-sliced layer uses), words through that XCD's
// L2 when the dispatch check holds (st_xcd2), else written through; kind 1:
// p = b ^ 8, written through (st_dev2); kind 2: p = b ^ 1 (another XCD),
// written through. Loads are ld_dev2. Words: [XCHG_G generations][XCHG_G
// 64-bit mailboxes][XCHG_G XCC ids of the last call]; tags run on from each
// workgroup's generation (every workgroup runs every call, so they stay
// equal), nothing is cleared between calls; every wait is bounded
// (FLOOR_SPIN_LIMIT polls, then bit 0 of the error word after the ids).
constexpr uint32_t XCHG_G = 256;
__global__ void __launch_bounds__(64) k_xchg(uint32_t *words, uint32_t rounds, uint32_t kind, uint32_t local) {
    if (threadIdx.x != 0) return;
    const uint32_t b = blockIdx.x, p = kind == 2 ? (b ^ 1u) : (b ^ 8u);
    uint32_t *gen = words, *box = words + XCHG_G, *ids = words + 3 * XCHG_G, *err = ids + XCHG_G;
    ids[b] = xcc_id();
    const uint32_t base = floor_ld(gen + b);
    const bool l2 = kind == 0 && local;
    auto send = [&](uint32_t tag) {
        if (l2) st_xcd2(box + 2 * b, tag);
        else st_dev2(box + 2 * b, tag);
    };
    auto wait = [&](uint32_t tag) {
        for (uint32_t spins = 0; spins < FLOOR_SPIN_LIMIT; spins++)
            if ((uint32_t)ld_dev2(box + 2 * p) == tag) return true;
        return false;
    };
    bool ok = true;
    for (uint32_t r = 0; r < rounds && ok; r++) {
        const uint32_t t1 = base + 2 * r + 1, t2 = t1 + 1;
        if (b < p) {
            send(t1);
            ok = wait(t2);
        } else {
            ok = wait(t1);
            if (ok) send(t2);
        }
    }
    if (!ok) atomicOr(err, 1u);
    floor_st(gen + b, base + 2 * rounds);
}

uint32_t xchg_words() { return 4 * XCHG_G + 1; }

hipError_t launch_xchg(int kind, uint32_t rounds, uint32_t *words, hipStream_t s) {
    if (kind < 0 || kind > 2 || !rounds || !words) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_xchg, dim3(XCHG_G), dim3(64), 0, s, words, rounds, (uint32_t)kind, xcd_local() ? 1u : 0u);
    return hipGetLastError();
}

uint32_t floor_sync_words() { return FLOOR_SYNC_WORDS; }

hipError_t launch_floor(int kind, const uint8_t *a, uint64_t a_bytes, const uint8_t *b, uint64_t b_bytes,
                        uint32_t *sync, hipStream_t s) {
    if (a_bytes % 16 || b_bytes % 16 || !a_bytes || (kind && (!b || !b_bytes))) return hipErrorInvalidValue;
    uint32_t *sink = sync + FLOOR_SYNC_WORDS;
    const uint4 *a4 = (const uint4 *)a, *b4 = (const uint4 *)b;
    for (const void *k : {(const void *)k_floor_read, (const void *)k_floor_two_phase}) {
        const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)FLOOR_LDS);
        if (e != hipSuccess) return e;
    }
    if (kind == 0) {
        hipLaunchKernelGGL(k_floor_read, dim3(FLOOR_G), dim3(FLOOR_NT), FLOOR_LDS, s, a4, a_bytes / 16, sink);
    } else if (kind == 1) {
        hipLaunchKernelGGL(k_floor_read, dim3(FLOOR_G), dim3(FLOOR_NT), FLOOR_LDS, s, a4, a_bytes / 16, sink);
        hipLaunchKernelGGL(k_floor_read, dim3(FLOOR_G), dim3(FLOOR_NT), FLOOR_LDS, s, b4, b_bytes / 16, sink);
    } else if (kind == 2) {
        // its workgroups wait for each other: all must be resident at once
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)k_floor_two_phase, FLOOR_NT, FLOOR_LDS) !=
                hipSuccess ||
            !xcd_coresident(device_cu_count(), n, FLOOR_G))
            return hipErrorNotSupported;
        hipLaunchKernelGGL(k_floor_two_phase, dim3(FLOOR_G), dim3(FLOOR_NT), FLOOR_LDS, s, a4, a_bytes / 16, b4,
                           b_bytes / 16, sync, sink);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace kq
