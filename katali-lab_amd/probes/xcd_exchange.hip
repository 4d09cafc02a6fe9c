// xcd_exchange.hip — a measurement probe, not part of the library.
//
// Prints (1) which XCD runs each workgroup of a 1024-workgroup grid (the
// hardware register XCC_ID against blockIdx % 8), and (2) the round trip of a
// flag bounced 200 times between two workgroups on the same or on different
// XCDs, on an idle chip and while the other workgroups stream 2 GiB, through
// (a) relaxed agent-scope atomic loads/stores and (b) plain stores read back
// with L1-bypassing (sc0) loads. Every wait is bounded (2^18 polls, then the
// pair gives up and counts a timeout), so the probe always ends.
//
// Build and run (gfx950):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         katali-lab_amd/probes/xcd_exchange.hip -o xcd_exchange && ./xcd_exchange
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
#include <vector>
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); return 1; } } while (0)

__device__ __forceinline__ unsigned xcc_id() { unsigned v; asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v)); return v; }
__device__ __forceinline__ uint64_t rt() { return __builtin_amdgcn_s_memrealtime(); }

__global__ void k_ids(unsigned *o) {
    if (threadIdx.x == 0) o[blockIdx.x] = xcc_id();
}

__device__ __forceinline__ void st_agent(uint32_t *p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ uint32_t ld_agent(uint32_t *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_plain(uint32_t *p, uint32_t v) {
    asm volatile("global_store_dword %0, %1, off" :: "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ uint32_t ld_sc0(uint32_t *p) {
    uint32_t v;
    asm volatile("global_load_dword %0, %1, off sc0\n s_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
    return v;
}

// ping-pong: WG `a` and WG `b` (of G) bounce a counter N times through F[0]
// (a writes odd, b writes even) ; mode 0 agent atomics, 1 plain store + sc0 load.
// res[0] = total realtime ticks seen by a, res[1] = timeouts, res[2..3] xcc of a, b
// Other WGs (if `load` set) stream buf (n16 16-byte words) to keep HBM busy.
__global__ void k_pp(uint32_t *F, uint64_t *res, uint32_t a, uint32_t b, int N, int mode,
                     const uint4 *buf, uint64_t n16, int load, uint32_t *sink) {
    const uint32_t w = blockIdx.x;
    if (w != a && w != b) {
        if (!load) return;
        uint4 acc = {0, 0, 0, 0};
        for (uint64_t i = (uint64_t)w * blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x) {
            const uint4 v = buf[i];
            acc.x ^= v.x; acc.y ^= v.y; acc.z ^= v.z; acc.w ^= v.w;
        }
        if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345678u) sink[0] = 1;
        return;
    }
    if (threadIdx.x != 0) return;
    if (w == a) res[2] = xcc_id(); else res[3] = xcc_id();
    const uint32_t me = w == a ? 1 : 0;
    uint64_t t0 = rt();
    int tmo = 0;
    for (int i = 0; i < N && !tmo; i++) {
        const uint32_t want = 2 * i + (me ? 0 : 1);   // a waits for b's even value (none at i=0: a starts)
        if (me && i == 0) {
        } else {
            uint32_t spins = 0;
            while ((mode == 0 ? ld_agent(F) : ld_sc0(F)) != want) {
                if (++spins > (1u << 18)) { tmo = 1; break; }
            }
        }
        if (tmo) break;
        const uint32_t v = me ? 2 * i + 1 : 2 * i + 2;
        if (mode == 0) st_agent(F, v); else st_plain(F, v);
    }
    if (me) { res[0] = rt() - t0; }
    if (tmo) atomicAdd((unsigned long long *)&res[1], 1ull);
}

int main() {
    const int G = 1024;
    unsigned *ids;
    CK(hipMalloc(&ids, 4 * G));
    hipLaunchKernelGGL(k_ids, dim3(G), dim3(64), 0, 0, ids);
    std::vector<unsigned> h(G);
    CK(hipMemcpy(h.data(), ids, 4 * G, hipMemcpyDeviceToHost));
    int agree = 0;
    for (int i = 0; i < G; i++) agree += (h[i] & 15) == (unsigned)(i % 8);
    printf("xcc ids: first 16:");
    for (int i = 0; i < 16; i++) printf(" %x", h[i]);
    printf("\nblockIdx%%8 == xcc for %d of %d\n", agree, G);
    int hist[16] = {0};
    for (int i = 0; i < G; i++) hist[h[i] & 15]++;
    printf("per xcc:"); for (int k = 0; k < 16; k++) if (hist[k]) printf(" %d:%d", k, hist[k]); printf("\n");

    uint32_t *F; uint64_t *res; uint32_t *sink; uint4 *buf;
    const uint64_t bytes = 2ull << 30;
    CK(hipMalloc(&F, 4096)); CK(hipMalloc(&res, 64)); CK(hipMalloc(&sink, 64)); CK(hipMalloc(&buf, bytes));
    CK(hipMemset(buf, 1, bytes));
    const int N = 200;
    struct P { uint32_t a, b; const char *name; } pairs[] = {{0, 8, "same xcd (0,8)"}, {0, 16, "same xcd (0,16)"}, {0, 1, "other xcd (0,1)"}, {3, 4, "other xcd (3,4)"}};
    for (int load = 0; load < 2; load++)
        for (int mode = 0; mode < 2; mode++)
            for (auto &p : pairs) {
                CK(hipMemset(F, 0, 4096)); CK(hipMemset(res, 0, 64));
                const uint32_t grid = load ? 512 : 32;
                hipLaunchKernelGGL(k_pp, dim3(grid), dim3(256), 0, 0, F, res, p.a, p.b, N, mode, (const uint4 *)buf, bytes / 16, load, sink);
                CK(hipDeviceSynchronize());
                uint64_t r[4];
                CK(hipMemcpy(r, res, 32, hipMemcpyDeviceToHost));
                printf("%s %-18s %s: round trip %.0f ns (xcc %llu,%llu) timeouts %llu\n", load ? "loaded" : "idle  ", p.name,
                       mode == 0 ? "agent atomics " : "plain + sc0   ", r[0] * 10.0 / N, (unsigned long long)r[2], (unsigned long long)r[3], (unsigned long long)r[1]);
            }
    return 0;
}
