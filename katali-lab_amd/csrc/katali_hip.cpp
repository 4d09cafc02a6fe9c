// katali_hip.cpp — the C ABI of libkatali_hip (include/katali_hip.h).
//
// Owns the device selection, one library stream (default priority), the
// scratch buffers the MoE kernel needs, and argument validation. Compute entry
// points enqueue on the library stream and return immediately; download and
// sync wait. State is process-global, single caller thread (the reference
// shim's model, V/src/katali_dense_cuda.c:7-12), with a mutex around init.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <condition_variable>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/katali_hip.h"
#include "kq_launch.h"

namespace {

thread_local std::string g_err;
std::mutex g_init_mu;
bool g_inited = false;
bool g_usable = false;
std::string g_status = "not probed";
int g_device = 0;
hipStream_t g_own_stream = nullptr;
hipStream_t g_stream = nullptr;
// the batched layer's second path (forked from g_stream and joined back
// inside one call; default priority like every stream here)
hipStream_t g_aux_stream = nullptr;
hipEvent_t g_ev_fork = nullptr, g_ev_join = nullptr;
bool g_capturing = false;
std::vector<void *> g_deferred_free;   // katali_hip_free calls made during the open capture
// buffers freed during a capture, released with the graph made from it
std::unordered_map<void *, std::vector<void *>> g_graph_frees;

// MoE scratch. Every buffer is allocated once, at its largest size, on the
// first call that needs it, and never freed or moved: a graph captured around
// any call stays valid whatever later calls ask for.
constexpr size_t HQ8_LAYER = 1u << 20;   // >= 17 slots x ffn/32 x 36 of every layer shape that fits LDS
uint8_t *g_hq8 = nullptr;     // single-token layer: q8_1 h [n_slots][ffn/32]
int32_t *g_route = nullptr;   // [ids | weights] from kernel A to kernel B
int32_t *g_err_dev = nullptr;
uint32_t *g_fsync = nullptr;  // the in-kernel exchanges' generation words and flags (zeroed once)
float *g_nbuf = nullptr;      // the normed layer's xn [4096] and logits [512] when it runs as two steps

// Scratch of katali_hip_moe_layer_noalloc: a static device array, resolved
// to a device address once per device at init (the array's name is a host
// stand-in, not a device address). [0, 256) the routing words kernel A hands
// to kernel B, [256, 260) the error word (zero from load, reset by
// katali_hip_sync after it reports), [512, ..) the q8_1 h blocks. Kernel B
// stages every slot's h in LDS, n_slots * ffn * 11/8 + 2116 <= 163840 bytes,
// so n_slots * ffn / 256 <= 459 and h takes at most 459 * 288 = 132192
// bytes: every layer shape the LDS admits fits the maximum below. From
// NOALLOC_FSYNC, the one-launch layers' exchange words (zero from load,
// generation-tagged, never cleared between calls), so the entry point runs
// the same kernels as katali_hip_moe_layer.
constexpr size_t NOALLOC_HQ8_MAX = 132 * 1024;
constexpr size_t NOALLOC_ERR = 256, NOALLOC_HQ8 = 512;
constexpr size_t NOALLOC_FSYNC = NOALLOC_HQ8 + NOALLOC_HQ8_MAX;
static_assert(NOALLOC_FSYNC % 256 == 0, "exchange words 256-byte aligned");
__device__ __align__(256) uint8_t scratch[NOALLOC_FSYNC + kq::fsync_words() * 4];
uint8_t *g_scratch = nullptr;   // scratch's device address on g_device
bool g_dispatch_ok = false;     // the start-up XCD dispatch check's result

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(KATALI_HIP_E_RUNTIME, "%s: %s", what, hipGetErrorString(e));
}

bool env_on(const char *name) {
    const char *e = getenv(name);
    return e && (e[0] == '1' || e[0] == 'y' || e[0] == 'Y');
}
bool env_off(const char *name) {
    const char *e = getenv(name);
    return e && (e[0] == '0' || e[0] == 'n' || e[0] == 'N');
}

int init_locked() {
    if (g_inited) return g_usable ? KATALI_HIP_OK : KATALI_HIP_E_NODEVICE;
    g_inited = true;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        g_status = std::string("no HIP device (") + (e != hipSuccess ? hipGetErrorString(e) : "count 0") + ")";
        return KATALI_HIP_E_NODEVICE;
    }
    const char *dv = getenv("KATALI_HIP_DEVICE");
    g_device = dv ? atoi(dv) : 0;
    if (g_device < 0 || g_device >= n) {
        g_status = "KATALI_HIP_DEVICE out of range";
        return KATALI_HIP_E_NODEVICE;
    }
    hipDeviceProp_t p;
    if ((e = hipGetDeviceProperties(&p, g_device)) != hipSuccess) {
        g_status = std::string("hipGetDeviceProperties: ") + hipGetErrorString(e);
        return KATALI_HIP_E_NODEVICE;
    }
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
        g_status = std::string("unsupported device ") + p.gcnArchName + " (libkatali_hip is built for gfx950)";
        return KATALI_HIP_E_NODEVICE;
    }
    if ((e = hipSetDevice(g_device)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&g_own_stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&g_aux_stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreateWithFlags(&g_ev_fork, hipEventDisableTiming)) != hipSuccess ||
        (e = hipEventCreateWithFlags(&g_ev_join, hipEventDisableTiming)) != hipSuccess) {
        g_status = std::string("device init: ") + hipGetErrorString(e);
        return KATALI_HIP_E_NODEVICE;
    }
    g_stream = g_own_stream;
    if ((e = hipGetSymbolAddress((void **)&g_scratch, HIP_SYMBOL(scratch))) != hipSuccess || !g_scratch) {
        g_status = std::string("device init: allocation-free scratch: ") + hipGetErrorString(e);
        return KATALI_HIP_E_NODEVICE;
    }
    // the one-launch layers' h hand-off inside each XCD, if the dispatcher
    // keeps each b % 8 class of a launch on one XCD (checked on g_stream)
    if ((e = kq::xcd_dispatch_check(g_stream)) != hipSuccess) {
        g_status = std::string("device init: XCD dispatch check: ") + hipGetErrorString(e);
        return KATALI_HIP_E_NODEVICE;
    }
    g_dispatch_ok = kq::xcd_local();
    if (env_off("KATALI_HIP_XCD_LOCAL")) kq::xcd_local_set(false);
    char buf[256];
    snprintf(buf, sizeof buf, "%s (%s, %d CUs, %.0f GiB; h hand-off %s)", p.name, p.gcnArchName,
             p.multiProcessorCount, (double)p.totalGlobalMem / (1024.0 * 1024.0 * 1024.0),
             kq::xcd_local() ? "inside the XCD" : "written through");
    g_status = buf;
    g_usable = true;
    return KATALI_HIP_OK;
}

int ensure() {
    std::lock_guard<std::mutex> lk(g_init_mu);
    int rc = init_locked();
    if (rc != KATALI_HIP_OK) return fail(rc, "no usable device: %s", g_status.c_str());
    hipError_t e = hipSetDevice(g_device);
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "hipSetDevice");
}

bool type_ok(uint32_t t) { return t == KATALI_HIP_TYPE_Q4_K || t == KATALI_HIP_TYPE_Q6_K; }

int check_gemv(uint32_t type, const void *w, uint64_t rows, uint64_t cols, const void *x, const void *y) {
    if (!type_ok(type)) return fail(KATALI_HIP_E_UNSUPPORTED, "type %u not supported (Q4_K=12, Q6_K=14)", type);
    if (!w || !x || !y) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (cols == 0 || cols % 256) return fail(KATALI_HIP_E_INVALID, "cols=%llu not a multiple of 256",
                                             (unsigned long long)cols);
    if (cols > 32768) return fail(KATALI_HIP_E_INVALID, "cols=%llu above 32768", (unsigned long long)cols);
    if (rows > 0xFFFFFFFFull) return fail(KATALI_HIP_E_INVALID, "rows above 2^32");
    return KATALI_HIP_OK;
}

int launched(hipError_t e, const char *what) { return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, what); }

// Frees that katali_hip_free deferred while a capture was open, done once
// nothing can use the buffers any more: after the stream has drained, when
// no graph was made from the capture or when that graph is destroyed.
int release_frees(std::vector<void *> &v) {
    if (v.empty()) return KATALI_HIP_OK;
    hipError_t e = hipStreamSynchronize(g_stream);
    for (void *p : v) {
        const hipError_t f = hipFree(p);
        if (e == hipSuccess) e = f;
    }
    v.clear();
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "deferred hipFree");
}

void *g_argmax = nullptr;   // argmax partials and count (kq::argmax_scratch_bytes(), zeroed once)

// The single-token layer's scratch (routing hand-off, error word, fused-layer
// flags, h), allocated and zeroed on the first MoE call, outside any capture.
int moe_scratch() {
    if (g_hq8) return KATALI_HIP_OK;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "first MoE call must happen outside graph capture");
    hipError_t e = hipMalloc((void **)&g_route, kq::moe_route_words() * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&g_err_dev, 64);
    if (e == hipSuccess) e = hipMemset(g_err_dev, 0, 64);
    if (e == hipSuccess) e = hipMalloc((void **)&g_fsync, kq::fsync_words() * 4);
    if (e == hipSuccess) e = hipMemset(g_fsync, 0, kq::fsync_words() * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&g_nbuf, (4096 + 512) * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&g_hq8, HQ8_LAYER);
    if (e != hipSuccess) {
        // nothing half-made stays: the next call starts over
        for (void *p : {(void *)g_route, (void *)g_err_dev, (void *)g_fsync, (void *)g_nbuf, (void *)g_hq8})
            if (p) (void)hipFree(p);
        g_route = g_err_dev = nullptr;
        g_fsync = nullptr;
        g_nbuf = nullptr;
        g_hq8 = nullptr;
        return fail(KATALI_HIP_E_NOMEM, "MoE scratch: %s", hipGetErrorString(e));
    }
    return KATALI_HIP_OK;
}

const char *type_name(uint32_t t) {
    return t == KATALI_HIP_TYPE_Q4_K ? "Q4_K" : t == KATALI_HIP_TYPE_Q6_K ? "Q6_K" : "?";
}

// The shape rules of every MoE entry point (and of katali_hip_moe_check,
// which needs no device): types and sizes, the selection, and the LDS the
// largest workgroup takes. n_tokens 0 is the single-token layer, 1..64 the
// batched layer.
int moe_shape(const KataliHipMoe *m, int32_t n_sel, uint32_t n_tokens, uint32_t &n_slots) {
    if (!m || m->struct_size < sizeof(KataliHipMoe)) return fail(KATALI_HIP_E_INVALID, "null or short MoE descriptor");
    if (m->up_type != m->gate_type || m->ffn > 16384 ||
        !kq::moe_shape_supported(m->gate_type, m->down_type, m->hidden, m->ffn))
        return fail(KATALI_HIP_E_UNSUPPORTED,
                    "MoE gate=%u up=%u down=%u hidden=%u ffn=%u: need Q4_K gate/up, Q4_K or Q6_K down, "
                    "hidden in {256,512,1024,2048,4096}, ffn a multiple of 256 (<= 16384)",
                    m->gate_type, m->up_type, m->down_type, m->hidden, m->ffn);
    const bool shared = m->gate_shexp || m->up_shexp || m->down_shexp;
    if (shared && !(m->gate_shexp && m->up_shexp && m->down_shexp))
        return fail(KATALI_HIP_E_INVALID, "shared expert needs gate, up and down");
    if (n_sel < 0 || n_sel > 16) return fail(KATALI_HIP_E_INVALID, "n_sel=%d (0..16)", n_sel);
    // n_sel 0: the shared expert alone, a dense SiLU-GLU FFN through the same kernels
    if (n_sel == 0 && !shared) return fail(KATALI_HIP_E_INVALID, "n_sel=0 needs the shared expert");
    if (n_sel > 0 && (!m->n_expert || m->n_expert > 512 || (uint32_t)n_sel > m->n_expert))
        return fail(KATALI_HIP_E_INVALID, "n_expert=%u n_sel=%d", m->n_expert, n_sel);
    if (n_tokens > 64) return fail(KATALI_HIP_E_INVALID, "n_tokens=%u (1..64)", n_tokens);
    n_slots = (uint32_t)n_sel + (shared ? 1u : 0u);
    const uint32_t lds = n_tokens ? kq::moe_batch_lds(m->hidden, m->ffn) : kq::moe_layer_lds(m->hidden, m->ffn, n_slots);
    if (lds > kq::LDS_PER_WG)
        return fail(KATALI_HIP_E_UNSUPPORTED,
                    "MoE %s hidden=%u ffn=%u, %u slot(s), down %s: a workgroup would need %u bytes of LDS, above "
                    "the %u a gfx950 workgroup has",
                    n_tokens ? "batch" : "layer", m->hidden, m->ffn, n_slots, type_name(m->down_type), lds,
                    kq::LDS_PER_WG);
    return KATALI_HIP_OK;
}

// Validates a MoE call and fills everything but the scratch pointers.
int moe_args(const KataliHipMoe *m, const KataliHipMoeRoute *r, const float *x, const void *xq, float *y,
             kq::MoeArgs &a, uint32_t &n_slots) {
    if (!r || r->struct_size < sizeof(KataliHipMoeRoute)) return fail(KATALI_HIP_E_INVALID, "null or short MoE route");
    int rc = moe_shape(m, r->n_sel, 0, n_slots);
    if (rc) return rc;
    if (!y) return fail(KATALI_HIP_E_INVALID, "null output");
    if ((x == nullptr) == (xq == nullptr)) return fail(KATALI_HIP_E_INVALID, "give exactly one of x_dev / xq8_dev");
    const bool shared = n_slots > (uint32_t)r->n_sel;
    if (r->n_sel > 0) {
        if (!m->gate_exps || !m->up_exps || !m->down_exps) return fail(KATALI_HIP_E_INVALID, "null buffer");
        if (!r->logits && (!r->ids || !r->weights)) return fail(KATALI_HIP_E_INVALID, "need logits or ids+weights");
    }
    memset(&a, 0, sizeof a);
    a.gate = (const uint8_t *)m->gate_exps;
    a.up = (const uint8_t *)m->up_exps;
    a.down = (const uint8_t *)m->down_exps;
    a.gate_sh = (const uint8_t *)m->gate_shexp;
    a.up_sh = (const uint8_t *)m->up_shexp;
    a.down_sh = (const uint8_t *)m->down_shexp;
    a.gate_type = m->gate_type;
    a.up_type = m->up_type;
    a.down_type = m->down_type;
    a.hidden = m->hidden;
    a.ffn = m->ffn;
    a.n_expert = m->n_expert;
    a.n_sel = r->n_sel;
    a.has_shared = shared ? 1 : 0;
    a.x = x;
    a.xq = (const uint8_t *)xq;
    a.logits = r->logits;
    a.step = r->step;
    a.logits_stride = r->logits_stride;
    a.ids = r->ids;
    a.wts = r->weights;
    a.ids_out = r->ids_out;
    a.wts_out = r->weights_out;
    a.y = y;
    return KATALI_HIP_OK;
}

int moe_impl(const KataliHipMoe *m, const KataliHipMoeRoute *r, const float *x, const void *xq, float *y,
             float *gu_dbg, void *hq8_dbg) {
    int rc = ensure();
    if (rc) return rc;
    kq::MoeArgs a;
    uint32_t n_slots = 0;
    if ((rc = moe_args(m, r, x, xq, y, a, n_slots))) return rc;
    const size_t hq8_bytes = (size_t)n_slots * (m->ffn / 32) * 36;
    if (hq8_bytes > HQ8_LAYER) return fail(KATALI_HIP_E_UNSUPPORTED, "MoE h scratch %zu bytes", hq8_bytes);
    if ((rc = moe_scratch())) return rc;
    a.hq8 = g_hq8;
    a.route_ids = g_route;
    a.route_w = (float *)(g_route + kq::moe_route_words() / 2);
    a.dbg_gu = gu_dbg;
    a.err = g_err_dev;
    a.fsync = g_fsync;
    // KATALI_HIP_TEST_SKEW=1, a test hook: workgroup 0's generation word of
    // the XCD-sliced layer is set off before the launch, so its words carry a
    // tag no other workgroup waits for and every wait of that call runs to
    // its bound and expires (about a second); the sync then reports the
    // expiry and clears the exchange area. Not for capture.
    if (env_on("KATALI_HIP_TEST_SKEW") && !g_capturing) {
        const hipError_t e = hipMemsetAsync(g_fsync + kq::FSYNC_X, 0xA5, 4, g_stream);
        if (e != hipSuccess) return hip_fail(e, "test skew");
    }
    // Eight slots take the XCD-sliced layer (one launch, every CU streaming
    // both phases; 11.6-11.9 us per layer at the 2048/768 top-8 shape
    // against 13.7 for kernels A and B); KATALI_HIP_XCD=0 keeps kernels A and
    // B. The other one-launch layer is opt-in (KATALI_HIP_FUSED=1): measured
    // slower than kernels A and B (its all-slots h exchange costs more than
    // the launch it saves).
    // Eight routed experts plus the shared expert (ffn 256 or 512) take it
    // too, the shared expert spread over all its workgroups (12.1 us per
    // layer at the 2048/512 top-8-of-256 shape against 13.6 for kernels A
    // and B); KATALI_HIP_XCD_SHARED=0 keeps those on kernels A and B.
    const bool allow_fused = env_on("KATALI_HIP_FUSED");
    const bool allow_xcd = !env_off("KATALI_HIP_XCD");
    const bool xcd_units = !env_off("KATALI_HIP_XCD_SHARED");
    rc = launched(kq::launch_moe(a, g_stream, allow_fused, nullptr, allow_xcd, xcd_units), "moe launch");
    if (rc) return rc;
    if (hq8_dbg) {
        hipError_t e = hipMemcpyAsync(hq8_dbg, g_hq8, hq8_bytes, hipMemcpyDeviceToDevice, g_stream);
        if (e != hipSuccess) return hip_fail(e, "copy hq8");
    }
    return KATALI_HIP_OK;
}

// The batched layer's scratch at its largest (64 tokens x 17 slots = 1088
// pairs, hidden 4096, ffn 16384): q8_1 x rows, q8_1 h rows, the grouping
// metadata and the per-pair down outputs, about 39 MB in all, allocated once
// on the first batched call.
constexpr uint32_t BATCH_MAX_P = 64 * 17;
constexpr size_t BATCH_XQ = (size_t)64 * (4096 / 32) * 36;
constexpr size_t BATCH_HQ8 = (size_t)BATCH_MAX_P * (16384 / 32) * 36;
constexpr size_t BATCH_YP = (size_t)BATCH_MAX_P * 4096 * 4;
uint8_t *g_bxq = nullptr;
uint8_t *g_bhq8 = nullptr;
int32_t *g_bmeta = nullptr;
float *g_byp = nullptr;

int batch_scratch() {
    if (g_byp) return KATALI_HIP_OK;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "first batched MoE call must happen outside graph capture");
    hipError_t e = hipMalloc((void **)&g_bxq, BATCH_XQ);
    if (e == hipSuccess) e = hipMalloc((void **)&g_bhq8, BATCH_HQ8);
    if (e == hipSuccess) e = hipMalloc((void **)&g_bmeta, (size_t)kq::moe_batch_meta_words(BATCH_MAX_P) * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&g_byp, BATCH_YP);
    if (e != hipSuccess) {
        for (void *p : {(void *)g_bxq, (void *)g_bhq8, (void *)g_bmeta, (void *)g_byp})
            if (p) (void)hipFree(p);
        g_bxq = g_bhq8 = nullptr;
        g_bmeta = nullptr;
        g_byp = nullptr;
        return fail(KATALI_HIP_E_NOMEM, "MoE batch scratch: %s", hipGetErrorString(e));
    }
    return KATALI_HIP_OK;
}

int moe_batch_impl(const KataliHipMoe *m, const KataliHipMoeBatch *b, const float *x, float *y) {
    int rc = ensure();
    if (rc) return rc;
    if (!b || b->struct_size < sizeof(KataliHipMoeBatch)) return fail(KATALI_HIP_E_INVALID, "null or short MoE batch");
    if (b->n_tokens < 1 || b->n_tokens > 64) return fail(KATALI_HIP_E_INVALID, "n_tokens=%u (1..64)", b->n_tokens);
    uint32_t S = 0;
    if ((rc = moe_shape(m, b->n_sel, b->n_tokens, S))) return rc;
    if (!x || !y) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (b->n_sel > 0 && (!m->gate_exps || !m->up_exps || !m->down_exps || !b->ids || !b->weights))
        return fail(KATALI_HIP_E_INVALID, "null expert tensors or routing");
    const bool shared = S > (uint32_t)b->n_sel;
    const uint32_t T = b->n_tokens;
    if ((rc = moe_scratch()) || (rc = batch_scratch())) return rc;
    kq::MoeArgs a;
    memset(&a, 0, sizeof a);
    a.gate = (const uint8_t *)m->gate_exps;
    a.up = (const uint8_t *)m->up_exps;
    a.down = (const uint8_t *)m->down_exps;
    a.gate_sh = (const uint8_t *)m->gate_shexp;
    a.up_sh = (const uint8_t *)m->up_shexp;
    a.down_sh = (const uint8_t *)m->down_shexp;
    a.gate_type = m->gate_type;
    a.up_type = m->up_type;
    a.down_type = m->down_type;
    a.hidden = m->hidden;
    a.ffn = m->ffn;
    a.n_expert = m->n_expert;
    a.n_sel = b->n_sel;
    a.has_shared = shared ? 1 : 0;
    a.ids = b->ids;
    a.wts = b->weights;
    a.hq8 = g_bhq8;
    a.route_ids = g_route;
    a.route_w = (float *)(g_route + kq::moe_route_words() / 2);
    a.err = g_err_dev;
    a.yp = g_byp;
    const uint32_t min_big = b->mfma_min_tokens ? b->mfma_min_tokens : 16;
    // KATALI_HIP_ONE_STREAM=1 keeps the grouped GEMM on the library stream
    // (per-kernel profiles attribute time only without the side stream)
    hipStream_t aux = env_on("KATALI_HIP_ONE_STREAM") ? g_stream : g_aux_stream;
    return launched(kq::launch_moe_batch(a, T, min_big, x, y, g_bxq, g_bmeta, g_stream, aux, g_ev_fork,
                                         g_ev_join),
                    "moe batch launch");
}

}  // namespace

extern "C" {

int katali_hip_abi_version(void) { return KATALI_HIP_ABI_VERSION; }
const char *katali_hip_last_error(void) { return g_err.c_str(); }

int katali_hip_probe(void) {
    std::lock_guard<std::mutex> lk(g_init_mu);
    return init_locked() == KATALI_HIP_OK ? 1 : 0;
}

const char *katali_hip_status(void) { return g_status.c_str(); }

int katali_hip_malloc(void **dev, size_t bytes) {
    int rc = ensure();
    if (rc) return rc;
    if (!dev) return fail(KATALI_HIP_E_INVALID, "null out pointer");
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_malloc during graph capture");
    *dev = nullptr;
    hipError_t e = hipMalloc(dev, bytes ? bytes : 1);
    if (e != hipSuccess) return fail(KATALI_HIP_E_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return KATALI_HIP_OK;
}

int katali_hip_free(void *dev) {
    if (!dev) return KATALI_HIP_OK;
    int rc = ensure();
    if (rc) return rc;
    if (g_capturing) {
        // a synchronisation would end the capture, and work being captured
        // may use the buffer: it is released with the graph (graph_destroy)
        g_deferred_free.push_back(dev);
        return KATALI_HIP_OK;
    }
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e == hipSuccess) e = hipFree(dev);
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "hipFree");
}

int katali_hip_upload(void *dev, const void *host, size_t bytes) {
    int rc = ensure();
    if (rc) return rc;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_upload during graph capture");
    if (!bytes) return KATALI_HIP_OK;
    if (!dev || !host) return fail(KATALI_HIP_E_INVALID, "null buffer");
    hipError_t e = hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "upload");
}

int katali_hip_download(void *host, const void *dev, size_t bytes) {
    int rc = ensure();
    if (rc) return rc;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_download during graph capture");
    if (!bytes) return katali_hip_sync();
    if (!dev || !host) return fail(KATALI_HIP_E_INVALID, "null buffer");
    hipError_t e = hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "download");
}

int katali_hip_supports_type(uint32_t t) { return type_ok(t) || t == KATALI_HIP_TYPE_F32 ? 1 : 0; }

static int check_gemv_f32(const void *w, uint64_t rows, uint64_t cols, const void *x, const void *y) {
    if (!w || !x || !y) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (cols == 0 || cols % 4 || cols > 32768)
        return fail(KATALI_HIP_E_INVALID, "F32 cols=%llu (a multiple of 4, at most 32768)", (unsigned long long)cols);
    if (((uintptr_t)w | (uintptr_t)x) % 16) return fail(KATALI_HIP_E_INVALID, "F32 w and x must be 16-byte aligned");
    if (rows > 0xFFFFFFFFull) return fail(KATALI_HIP_E_INVALID, "rows above 2^32");
    return KATALI_HIP_OK;
}

int katali_hip_matvec(uint32_t type, const void *w, uint64_t rows, uint64_t cols, const float *x, float *y) {
    int rc = ensure();
    if (rc) return rc;
    if (type == KATALI_HIP_TYPE_F32) {
        if ((rc = check_gemv_f32(w, rows, cols, x, y)) || !rows) return rc;
        return launched(kq::launch_gemv_f32((const float *)w, rows, cols, x, y, g_stream), "matvec F32");
    }
    if ((rc = check_gemv(type, w, rows, cols, x, y))) return rc;
    if (!rows) return KATALI_HIP_OK;
    const int mode = (env_on("KATALI_CUDA_DP4A") || env_on("KATALI_HIP_DP4A")) ? 2 : 0;
    return launched(kq::launch_gemv(type, (const uint8_t *)w, rows, cols, x, nullptr, y, mode, g_stream), "matvec");
}

int katali_hip_sync(void) {
    int rc = ensure();
    if (rc) return rc;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_sync during graph capture");
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) return hip_fail(e, "sync");
    // both error words are read and cleared before either is reported, so
    // no error is left for a later, unrelated sync
    int32_t na = 0, err = 0;
    e = hipMemcpy(&na, g_scratch + NOALLOC_ERR, 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess && g_err_dev) e = hipMemcpy(&err, g_err_dev, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "read error word");
    if (na) (void)hipMemset(g_scratch + NOALLOC_ERR, 0, 4);
    if (err) (void)hipMemset(g_err_dev, 0, 4);
    if ((err | na) & 12) {
        // a one-launch layer gave up waiting for its own workgroups (the
        // device was shared with other work; bit 4), or one of its
        // workgroups ran on another XCD than the round-robin dispatch puts it
        // on (bit 8, whose slot's waits may have expired too): its outputs
        // and the exchange words are void; start over, and from now on run
        // every layer as kernels A and B, which never wait in-kernel
        if (g_fsync && (err & 12)) (void)hipMemset(g_fsync, 0, kq::fsync_words() * 4);
        if (na & 12) (void)hipMemset(g_scratch + NOALLOC_FSYNC, 0, kq::fsync_words() * 4);
        kq::xcd_disable();
        return fail(KATALI_HIP_E_TIMEOUT, "MoE layer: %s (outputs invalid; the one-launch layers are off from now on)",
                    ((err | na) & 8) ? "a workgroup ran on another XCD than its slot's" : "in-kernel wait expired");
    }
    if (err | na)
        return fail(KATALI_HIP_E_INVALID, "MoE expert id outside [0, n_expert) in the explicit routing");
    return KATALI_HIP_OK;
}

int katali_hip_memset(void *dev, int value, size_t bytes) {
    int rc = ensure();
    if (rc) return rc;
    if (!dev) return fail(KATALI_HIP_E_INVALID, "null buffer");
    // a captured memset node has given wrong results on replays after the first
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_memset during graph capture");
    return launched(hipMemsetAsync(dev, value, bytes, g_stream), "memset");
}

int katali_hip_set_stream(void *s) {
    int rc = ensure();
    if (rc) return rc;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_set_stream during graph capture");
    g_stream = s ? (hipStream_t)s : g_own_stream;
    return KATALI_HIP_OK;
}

int katali_hip_quantize_q8_1(const float *x, uint64_t n, void *q8) {
    int rc = ensure();
    if (rc) return rc;
    if (!x || !q8) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (n % 32) return fail(KATALI_HIP_E_INVALID, "n=%llu not a multiple of 32", (unsigned long long)n);
    if (!n) return KATALI_HIP_OK;
    return launched(kq::launch_quantize_q8_1(x, n, (uint8_t *)q8, g_stream), "quantize_q8_1");
}

int katali_hip_matvec_q8(uint32_t type, const void *w, uint64_t rows, uint64_t cols, const void *xq8, float *y) {
    int rc = ensure();
    if (rc || (rc = check_gemv(type, w, rows, cols, xq8, y))) return rc;
    if (!rows) return KATALI_HIP_OK;
    return launched(kq::launch_gemv(type, (const uint8_t *)w, rows, cols, nullptr, (const uint8_t *)xq8, y, 1, g_stream),
                    "matvec_q8");
}

int katali_hip_matvec_dp4a(uint32_t type, const void *w, uint64_t rows, uint64_t cols, const float *x, float *y) {
    int rc = ensure();
    if (rc || (rc = check_gemv(type, w, rows, cols, x, y))) return rc;
    if (!rows) return KATALI_HIP_OK;
    return launched(kq::launch_gemv(type, (const uint8_t *)w, rows, cols, x, nullptr, y, 2, g_stream), "matvec_dp4a");
}

static int matvec_multi(int n, const uint32_t *types, const void *const *ws, const uint64_t *rows, uint64_t cols,
                        const float *x, float *const *ys, int mode, const char *what) {
    int rc = ensure();
    if (rc) return rc;
    if (n < 1 || n > kq::GEMV_MULTI_MAX) return fail(KATALI_HIP_E_INVALID, "n=%d not in 1..%d", n, kq::GEMV_MULTI_MAX);
    if (!types || !ws || !rows || !ys) return fail(KATALI_HIP_E_INVALID, "null array");
    for (int i = 0; i < n; i++)
        if ((rc = check_gemv(types[i], ws[i], rows[i], cols, x, ys[i]))) return rc;
    return launched(kq::launch_gemv_multi(n, types, (const uint8_t *const *)ws, rows, cols, x, ys, mode, g_stream),
                    what);
}

int katali_hip_matvec_multi(int n, const uint32_t *types, const void *const *ws, const uint64_t *rows, uint64_t cols,
                            const float *x, float *const *ys) {
    const int mode = (env_on("KATALI_CUDA_DP4A") || env_on("KATALI_HIP_DP4A")) ? 2 : 0;
    return matvec_multi(n, types, ws, rows, cols, x, ys, mode, "matvec_multi");
}

int katali_hip_matvec_multi_dp4a(int n, const uint32_t *types, const void *const *ws, const uint64_t *rows,
                                 uint64_t cols, const float *x, float *const *ys) {
    return matvec_multi(n, types, ws, rows, cols, x, ys, 2, "matvec_multi_dp4a");
}

int katali_hip_block_isums(uint32_t type, const void *w, uint64_t rows, uint64_t cols, const void *xq8, int32_t *out) {
    int rc = ensure();
    if (rc || (rc = check_gemv(type, w, rows, cols, xq8, out))) return rc;
    if (!rows) return KATALI_HIP_OK;
    return launched(kq::launch_isums(type, (const uint8_t *)w, rows, cols, (const uint8_t *)xq8, out, g_stream),
                    "block_isums");
}

int katali_hip_moe_batch(const KataliHipMoe *moe, const KataliHipMoeBatch *batch, const float *x_dev,
                         float *y_dev) {
    return moe_batch_impl(moe, batch, x_dev, y_dev);
}

static int check_norm(const void *x, const void *w, uint64_t n, const void *out) {
    if (!x || !w || !out) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (n == 0 || n > (1u << 20)) return fail(KATALI_HIP_E_INVALID, "rmsnorm n=%llu (1..2^20)", (unsigned long long)n);
    return KATALI_HIP_OK;
}

int katali_hip_rmsnorm(const float *x, const float *w, uint64_t n, float eps, float *out) {
    int rc = ensure();
    if (rc || (rc = check_norm(x, w, n, out))) return rc;
    return launched(kq::launch_rmsnorm(x, w, (uint32_t)n, eps, out, g_stream), "rmsnorm");
}

int katali_hip_add_rmsnorm(float *x, const float *delta, float scale, const float *w, uint64_t n, float eps,
                           float *out) {
    int rc = ensure();
    if (rc || (rc = check_norm(x, w, n, out))) return rc;
    if (!delta) return fail(KATALI_HIP_E_INVALID, "null buffer");
    return launched(kq::launch_add_rmsnorm(x, delta, scale, w, (uint32_t)n, eps, out, g_stream), "add_rmsnorm");
}

static bool overlap(const void *a, uint64_t an, const void *b, uint64_t bn) {
    if (!a || !b) return false;
    const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
    return pa < pb + bn && pb < pa + an;
}

int katali_hip_rmsnorm_matvec_f32(const float *x, const float *delta, float scale, float *x_out, const float *nw,
                                  uint64_t n, float eps, float *xn, const float *w, uint64_t rows, float *y) {
    int rc = ensure();
    if (rc) return rc;
    if (!x || !nw || !xn || !w || !y || (delta && !x_out)) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (n < 4 || n > 8192 || n % 4) return fail(KATALI_HIP_E_INVALID, "n=%llu (a multiple of 4 in 4..8192)",
                                                (unsigned long long)n);
    if (rows == 0 || rows > 0x7FFFFFFFull) return fail(KATALI_HIP_E_INVALID, "rows=%llu", (unsigned long long)rows);
    if (((uintptr_t)x | (uintptr_t)delta | (uintptr_t)x_out | (uintptr_t)nw | (uintptr_t)xn | (uintptr_t)w) % 16)
        return fail(KATALI_HIP_E_INVALID, "vectors and W must be 16-byte aligned");
    const uint64_t vb = n * 4, wb = rows * n * 4, yb = rows * 4;
    const void *ins[4] = {x, delta, nw, w};
    const uint64_t inb[4] = {vb, vb, vb, wb};
    const void *outs[3] = {delta ? x_out : nullptr, xn, y};
    const uint64_t outb[3] = {vb, vb, yb};
    for (int o = 0; o < 3; o++) {
        for (int i = 0; i < 4; i++)
            if (overlap(outs[o], outb[o], ins[i], inb[i])) return fail(KATALI_HIP_E_INVALID, "an output overlaps an input");
        for (int p = o + 1; p < 3; p++)
            if (overlap(outs[o], outb[o], outs[p], outb[p])) return fail(KATALI_HIP_E_INVALID, "outputs overlap");
    }
    return launched(kq::launch_norm_router(x, delta, scale, x_out, nw, n, eps, xn, w, rows, y, g_stream),
                    "rmsnorm_matvec_f32");
}

int katali_hip_moe_route_batch(const float *logits, uint32_t n_tokens, uint32_t n_expert, int32_t n_sel,
                               int32_t *ids, float *wts) {
    int rc = ensure();
    if (rc) return rc;
    if (!logits || !ids || !wts) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (n_tokens < 1 || n_tokens > 65535 || n_expert < 1 || n_expert > 512 || n_sel < 1 || n_sel > 16 ||
        (uint32_t)n_sel > n_expert)
        return fail(KATALI_HIP_E_INVALID, "route_batch T=%u E=%u n_sel=%d", n_tokens, n_expert, n_sel);
    return launched(kq::launch_route_batch(logits, n_tokens, n_expert, n_sel, ids, wts, g_stream), "route_batch");
}

int katali_hip_argmax(const float *x, uint64_t n, int32_t *out) {
    int rc = ensure();
    if (rc) return rc;
    if (!x || !out) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (n == 0 || n >= (1ull << 31)) return fail(KATALI_HIP_E_INVALID, "argmax n=%llu", (unsigned long long)n);
    if (!g_argmax) {
        if (g_capturing) return fail(KATALI_HIP_E_INVALID, "first argmax call must happen outside graph capture");
        hipError_t e = hipMalloc(&g_argmax, kq::argmax_scratch_bytes());
        if (e == hipSuccess) e = hipMemsetAsync(g_argmax, 0, kq::argmax_scratch_bytes(), g_stream);
        if (e != hipSuccess) {
            if (g_argmax) (void)hipFree(g_argmax);
            g_argmax = nullptr;
            return hip_fail(e, "argmax scratch");
        }
    }
    return launched(kq::launch_argmax(x, (uint32_t)n, g_argmax, out, g_stream), "argmax");
}

int katali_hip_moe_layer_noalloc(const KataliHipMoe *m, const KataliHipMoeRoute *r, const float *x, const void *xq,
                                 float *y) {
    // no init here (init creates streams): the library must be up already
    if (!g_inited || !g_usable || !g_scratch)
        return fail(KATALI_HIP_E_INVALID, "katali_hip_moe_layer_noalloc: call katali_hip_probe() first");
    hipError_t e = hipSetDevice(g_device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    kq::MoeArgs a;
    uint32_t n_slots = 0;
    int rc = moe_args(m, r, x, xq, y, a, n_slots);
    if (rc) return rc;
    const size_t hq8_bytes = (size_t)n_slots * (m->ffn / 32) * 36;
    if (hq8_bytes > NOALLOC_HQ8_MAX)
        return fail(KATALI_HIP_E_INVALID,
                    "katali_hip_moe_layer_noalloc: %zu bytes of h scratch (n_slots %u x ffn %u / 32 x 36) above its "
                    "%zu-byte maximum",
                    hq8_bytes, n_slots, m->ffn, NOALLOC_HQ8_MAX);
    a.hq8 = g_scratch + NOALLOC_HQ8;
    a.route_ids = (int32_t *)g_scratch;
    a.route_w = (float *)(g_scratch + 4 * kq::moe_route_words() / 2);
    a.err = (int32_t *)(g_scratch + NOALLOC_ERR);
    a.fsync = (uint32_t *)(g_scratch + NOALLOC_FSYNC);
    // the layer choice of katali_hip_moe_layer (moe_impl), so the outputs are its bits
    return launched(kq::launch_moe(a, g_stream, env_on("KATALI_HIP_FUSED"), nullptr, !env_off("KATALI_HIP_XCD"),
                                   !env_off("KATALI_HIP_XCD_SHARED")),
                    "moe launch");
}

int katali_hip_phase_stamps(void *host, size_t bytes) {
    int rc = ensure();
    if (rc) return rc;
    if (!host) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_phase_stamps during graph capture");
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) return hip_fail(e, "sync");
    e = kq::read_stamps(host, bytes);
    if (e == hipErrorNotSupported)
        return fail(KATALI_HIP_E_UNSUPPORTED, "phase stamps: this is not the measurement build (build.py --stamps)");
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "phase stamps");
}

int katali_hip_stream_floor(int32_t kind, const void *a, size_t a_bytes, const void *b, size_t b_bytes,
                            void *sync) {
    int rc = ensure();
    if (rc) return rc;
    if (kind < 0 || kind > 2) return fail(KATALI_HIP_E_INVALID, "floor kind %d (0..2)", kind);
    if (!a || !sync || (kind && !b)) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (!a_bytes || a_bytes % 16 || (kind && (!b_bytes || b_bytes % 16)))
        return fail(KATALI_HIP_E_INVALID, "floor sizes must be non-zero multiples of 16");
    const hipError_t e = kq::launch_floor(kind, (const uint8_t *)a, a_bytes, (const uint8_t *)b, b_bytes,
                                          (uint32_t *)sync, g_stream);
    if (e == hipErrorNotSupported)
        return fail(KATALI_HIP_E_UNSUPPORTED, "floor kind 2 needs 256 workgroups resident at once (256 CUs)");
    return launched(e, "stream floor");
}

int katali_hip_exchange_probe(int32_t kind, uint32_t rounds, void *words) {
    int rc = ensure();
    if (rc) return rc;
    if (kind < 0 || kind > 2) return fail(KATALI_HIP_E_INVALID, "exchange probe kind %d (0..2)", kind);
    if (!words) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (rounds < 1 || rounds > (1u << 20)) return fail(KATALI_HIP_E_INVALID, "rounds %u (1..2^20)", rounds);
    return launched(kq::launch_xchg(kind, rounds, (uint32_t *)words, g_stream), "exchange probe");
}

int katali_hip_one_launch(int32_t mode) {
    const int was = kq::xcd_disabled() ? 0 : 1;
    if (mode == 0) kq::xcd_disable();
    else if (mode == 1) kq::xcd_enable();
    return was;
}

int katali_hip_xcd_handoff(int32_t mode) {
    if (ensure() != KATALI_HIP_OK) return 0;
    const int was = kq::xcd_local() ? 1 : 0;
    if (mode == 0) kq::xcd_local_set(false);
    else if (mode == 1) kq::xcd_local_set(g_dispatch_ok);
    return was;
}

int katali_hip_moe_check(const KataliHipMoe *m, int32_t n_sel, uint32_t n_tokens) {
    uint32_t n_slots = 0;
    return moe_shape(m, n_sel, n_tokens, n_slots);
}

int katali_hip_moe_layer(const KataliHipMoe *m, const KataliHipMoeRoute *r, const float *x, const void *xq, float *y) {
    return moe_impl(m, r, x, xq, y, nullptr, nullptr);
}

int katali_hip_moe_layer_normed(const KataliHipMoe *m, const KataliHipMoeNorm *nrm, int32_t n_sel, int32_t *ids_out,
                                float *weights_out, float *y) {
    int rc = ensure();
    if (rc) return rc;
    if (!nrm || nrm->struct_size < sizeof(KataliHipMoeNorm)) return fail(KATALI_HIP_E_INVALID, "null or short norm descriptor");
    if (n_sel < 1) return fail(KATALI_HIP_E_INVALID, "n_sel=%d: the normed layer routes (1..16)", n_sel);
    KataliHipMoeRoute r;
    memset(&r, 0, sizeof r);
    r.struct_size = sizeof r;
    r.n_sel = n_sel;
    r.logits = nrm->router;   // stands for "routed from logits" in the checks below
    r.ids_out = ids_out;
    r.weights_out = weights_out;
    kq::MoeArgs a;
    uint32_t n_slots = 0;
    if ((rc = moe_args(m, &r, nrm->x, nullptr, y, a, n_slots))) return rc;
    // the steps before the layer: katali_hip_rmsnorm_matvec_f32's rules
    const uint64_t n = m->hidden, rows = m->n_expert;
    const float *x = nrm->x, *delta = nrm->delta, *nw = nrm->norm_w, *w = nrm->router;
    float *x_out = nrm->x_out, *xn = nrm->xn_out, *lg = nrm->logits_out;
    if (!x || !nw || !w || (delta && !x_out)) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (((uintptr_t)x | (uintptr_t)delta | (uintptr_t)x_out | (uintptr_t)nw | (uintptr_t)xn | (uintptr_t)w) % 16)
        return fail(KATALI_HIP_E_INVALID, "vectors and the router must be 16-byte aligned");
    const uint64_t vb = n * 4, wb = rows * n * 4;
    const void *ins[4] = {x, delta, nw, w};
    const uint64_t inb[4] = {vb, vb, vb, wb};
    const void *outs[4] = {delta ? x_out : nullptr, xn, lg, y};
    const uint64_t outb[4] = {vb, vb, rows * 4, vb};
    for (int o = 0; o < 4; o++) {
        for (int i = 0; i < 4; i++)
            if (overlap(outs[o], outb[o], ins[i], inb[i])) return fail(KATALI_HIP_E_INVALID, "an output overlaps an input");
        for (int p = o + 1; p < 4; p++)
            if (overlap(outs[o], outb[o], outs[p], outb[p])) return fail(KATALI_HIP_E_INVALID, "outputs overlap");
    }
    if ((rc = moe_scratch())) return rc;
    a.x = nullptr;
    a.logits = nullptr;
    a.hq8 = g_hq8;
    a.route_ids = g_route;
    a.route_w = (float *)(g_route + kq::moe_route_words() / 2);
    a.err = g_err_dev;
    a.fsync = g_fsync;
    a.nx = x;
    a.ndelta = delta;
    a.nscale = nrm->scale;
    a.nx_out = x_out;
    a.nw = nw;
    a.neps = nrm->eps;
    a.nxn_out = xn;
    a.router = w;
    a.logits_out = lg;
    return launched(kq::launch_moe_normed(a, g_nbuf, g_nbuf + 4096, g_stream, nullptr, !env_off("KATALI_HIP_XCD")),
                    "moe normed launch");
}

// A stack of layers (katali_hip_moe_stack_*): the host copy of the layer
// table (for the layer-by-layer path), its device copy (the one-launch
// path's), and two residual buffers for the normed layer-by-layer path.
struct MoeStack {
    KataliHipMoe shape;
    int32_t n_sel;
    bool normed;
    float eps;
    std::vector<KataliHipMoeStackLayer> layers;
    kq::StackLayer *table;
    float *res[2];
};

static KataliHipMoe stack_layer_desc(const MoeStack &s, const KataliHipMoeStackLayer &L) {
    KataliHipMoe d = s.shape;
    d.gate_exps = L.gate_exps;
    d.up_exps = L.up_exps;
    d.down_exps = L.down_exps;
    d.gate_shexp = L.gate_shexp;
    d.up_shexp = L.up_shexp;
    d.down_shexp = L.down_shexp;
    return d;
}

int katali_hip_moe_stack_create(const KataliHipMoe *shape, int32_t n_sel, int32_t normed, float eps,
                                const KataliHipMoeStackLayer *layers, int32_t n_layers, void **stack) {
    int rc = ensure();
    if (rc) return rc;
    if (!stack) return fail(KATALI_HIP_E_INVALID, "null stack out pointer");
    *stack = nullptr;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_moe_stack_create during graph capture");
    if (!layers || n_layers < 1 || n_layers > 4096) return fail(KATALI_HIP_E_INVALID, "n_layers=%d (1..4096)", n_layers);
    uint32_t n_slots = 0;
    if ((rc = moe_shape(shape, n_sel, 0, n_slots))) return rc;
    const bool shared = n_slots > (uint32_t)n_sel;
    if (normed && n_sel < 1) return fail(KATALI_HIP_E_INVALID, "n_sel=%d: the normed stack routes (1..16)", n_sel);
    const uint64_t vb = (uint64_t)shape->hidden * 4, rb = (uint64_t)shape->n_expert * vb;
    for (int32_t l = 0; l < n_layers; l++) {
        const KataliHipMoeStackLayer &L = layers[l];
        if (L.struct_size < sizeof(KataliHipMoeStackLayer)) return fail(KATALI_HIP_E_INVALID, "layer %d: short struct", l);
        if (n_sel > 0 && (!L.gate_exps || !L.up_exps || !L.down_exps))
            return fail(KATALI_HIP_E_INVALID, "layer %d: null expert buffer", l);
        if (shared != (L.gate_shexp && L.up_shexp && L.down_shexp) || (!shared && (L.gate_shexp || L.up_shexp || L.down_shexp)))
            return fail(KATALI_HIP_E_INVALID, "layer %d: shared expert pointers do not match the shape's", l);
        if (!L.y) return fail(KATALI_HIP_E_INVALID, "layer %d: null output", l);
        const void *outs[4] = {L.y, normed ? L.x_out : nullptr, normed ? L.xn_out : nullptr,
                               normed ? L.logits_out : nullptr};
        const uint64_t outb[4] = {vb, vb, vb, (uint64_t)shape->n_expert * 4};
        const void *ins[5] = {normed ? (const void *)L.norm_w : nullptr, normed ? (const void *)L.router : nullptr,
                              normed ? nullptr : (const void *)L.route.logits, l ? layers[l - 1].y : nullptr,
                              normed || !l ? nullptr : (const void *)L.x};
        const uint64_t inb[5] = {vb, rb, (uint64_t)shape->n_expert * 4, vb, vb};
        if (normed) {
            if (!L.norm_w || !L.router) return fail(KATALI_HIP_E_INVALID, "layer %d: null norm weights or router", l);
            if (((uintptr_t)L.norm_w | (uintptr_t)L.router | (uintptr_t)L.y | (uintptr_t)L.x_out | (uintptr_t)L.xn_out) % 16)
                return fail(KATALI_HIP_E_INVALID, "layer %d: vectors and the router must be 16-byte aligned", l);
        } else {
            if (L.route.struct_size < sizeof(KataliHipMoeRoute) || L.route.n_sel != n_sel)
                return fail(KATALI_HIP_E_INVALID, "layer %d: route missing or n_sel not the stack's", l);
            if (n_sel > 0 && !L.route.logits && (!L.route.ids || !L.route.weights))
                return fail(KATALI_HIP_E_INVALID, "layer %d: need logits or ids+weights", l);
            if (((uintptr_t)L.y | (uintptr_t)L.x) % 16)
                return fail(KATALI_HIP_E_INVALID, "layer %d: x and y must be 16-byte aligned", l);
        }
        for (int o = 0; o < 4; o++) {
            for (int i = 0; i < 5; i++)
                if (overlap(outs[o], outb[o], ins[i], inb[i]))
                    return fail(KATALI_HIP_E_INVALID, "layer %d: an output overlaps an input", l);
            for (int p = o + 1; p < 4; p++)
                if (overlap(outs[o], outb[o], outs[p], outb[p]))
                    return fail(KATALI_HIP_E_INVALID, "layer %d: outputs overlap", l);
        }
    }
    if ((rc = moe_scratch())) return rc;
    std::vector<kq::StackLayer> t((size_t)n_layers);
    for (int32_t l = 0; l < n_layers; l++) {
        const KataliHipMoeStackLayer &L = layers[l];
        kq::StackLayer &d = t[(size_t)l];
        memset(&d, 0, sizeof d);
        d.x = normed || !l ? nullptr : L.x;
        d.gate = (const uint8_t *)L.gate_exps;
        d.up = (const uint8_t *)L.up_exps;
        d.down = (const uint8_t *)L.down_exps;
        d.gate_sh = (const uint8_t *)L.gate_shexp;
        d.up_sh = (const uint8_t *)L.up_shexp;
        d.down_sh = (const uint8_t *)L.down_shexp;
        if (!normed) {
            d.logits = L.route.logits;
            d.step = L.route.step;
            d.logits_stride = L.route.logits_stride;
            d.ids = L.route.ids;
            d.wts = L.route.weights;
            d.ids_out = L.route.ids_out;
            d.wts_out = L.route.weights_out;
        }
        d.y = L.y;
        if (normed) {
            if (L.route.struct_size >= sizeof(KataliHipMoeRoute)) {   // optional routing outputs
                d.ids_out = L.route.ids_out;
                d.wts_out = L.route.weights_out;
            }
            d.nw = L.norm_w;
            d.router = L.router;
            d.x_out = L.x_out;
            d.xn_out = L.xn_out;
            d.logits_out = L.logits_out;
        }
    }
    MoeStack *s = new MoeStack();
    s->shape = *shape;
    s->n_sel = n_sel;
    s->normed = normed != 0;
    s->eps = eps;
    s->layers.assign(layers, layers + n_layers);
    s->table = nullptr;
    s->res[0] = s->res[1] = nullptr;
    hipError_t e = hipMalloc((void **)&s->table, t.size() * sizeof(kq::StackLayer));
    if (e == hipSuccess) e = hipMemcpy(s->table, t.data(), t.size() * sizeof(kq::StackLayer), hipMemcpyHostToDevice);
    if (e == hipSuccess && s->normed) e = hipMalloc((void **)&s->res[0], 2 * vb);
    if (e != hipSuccess) {
        if (s->table) (void)hipFree(s->table);
        if (s->res[0]) (void)hipFree(s->res[0]);
        delete s;
        return fail(KATALI_HIP_E_NOMEM, "MoE stack table: %s", hipGetErrorString(e));
    }
    if (s->normed) s->res[1] = s->res[0] + shape->hidden;
    *stack = s;
    return KATALI_HIP_OK;
}

// The stack layer by layer (shapes the one-launch form does not take): the
// same calls an engine would make, with the same results.
static int stack_layer_by_layer(MoeStack &s, const float *x, const float *delta, float scale) {
    const size_t n = s.layers.size();
    const uint64_t vb = (uint64_t)s.shape.hidden * 4;
    const float *cur = x;   // the residual stream (normed) or the layer input (plain)
    for (size_t l = 0; l < n; l++) {
        const KataliHipMoeStackLayer &L = s.layers[l];
        const KataliHipMoe d = stack_layer_desc(s, L);
        int rc;
        if (!s.normed) {
            rc = moe_impl(&d, &L.route, !l ? x : L.x ? L.x : s.layers[l - 1].y, nullptr, L.y, nullptr, nullptr);
        } else {
            const float *dl = l ? s.layers[l - 1].y : delta;
            float *nxt = s.res[l % 2];
            KataliHipMoeNorm nrm;
            memset(&nrm, 0, sizeof nrm);
            nrm.struct_size = sizeof nrm;
            nrm.x = cur;
            nrm.delta = dl;
            nrm.scale = l ? 1.0f : scale;
            nrm.x_out = dl ? nxt : nullptr;
            nrm.norm_w = L.norm_w;
            nrm.eps = s.eps;
            nrm.xn_out = L.xn_out;
            nrm.router = L.router;
            nrm.logits_out = L.logits_out;
            const bool ro = L.route.struct_size >= sizeof(KataliHipMoeRoute);
            rc = katali_hip_moe_layer_normed(&d, &nrm, s.n_sel, ro ? L.route.ids_out : nullptr,
                                             ro ? L.route.weights_out : nullptr, L.y);
            if (!rc && dl) cur = nxt;
            if (!rc && L.x_out) {
                const hipError_t e = hipMemcpyAsync(L.x_out, cur, vb, hipMemcpyDeviceToDevice, g_stream);
                if (e != hipSuccess) return hip_fail(e, "stack x_out");
            }
        }
        if (rc) return rc;
    }
    return KATALI_HIP_OK;
}

int katali_hip_moe_stack_run(void *stack, const float *x, const float *delta, float scale) {
    int rc = ensure();
    if (rc) return rc;
    if (!stack) return fail(KATALI_HIP_E_INVALID, "null stack");
    MoeStack &s = *(MoeStack *)stack;
    if (!x) return fail(KATALI_HIP_E_INVALID, "null input");
    if (!s.normed && delta) return fail(KATALI_HIP_E_INVALID, "the plain stack takes no delta");
    if (((uintptr_t)x | (uintptr_t)delta) % 16) return fail(KATALI_HIP_E_INVALID, "x and delta must be 16-byte aligned");
    const uint64_t vb = (uint64_t)s.shape.hidden * 4;
    const KataliHipMoeStackLayer &L0 = s.layers[0];
    const void *outs[4] = {L0.y, L0.x_out, L0.xn_out, L0.logits_out};
    const uint64_t outb[4] = {vb, vb, vb, (uint64_t)s.shape.n_expert * 4};
    for (int o = 0; o < 4; o++)
        if (overlap(outs[o], outb[o], x, vb) || overlap(outs[o], outb[o], delta, vb))
            return fail(KATALI_HIP_E_INVALID, "layer 0: an output overlaps the input");
    if ((rc = moe_scratch())) return rc;
    if (!env_off("KATALI_HIP_XCD")) {
        kq::MoeArgs a;
        memset(&a, 0, sizeof a);
        a.gate_type = s.shape.gate_type;
        a.up_type = s.shape.up_type;
        a.down_type = s.shape.down_type;
        a.hidden = s.shape.hidden;
        a.ffn = s.shape.ffn;
        a.n_expert = s.shape.n_expert;
        a.n_sel = s.n_sel;
        a.has_shared = s.shape.gate_shexp ? 1 : 0;
        a.hq8 = g_hq8;
        a.route_ids = g_route;
        a.route_w = (float *)(g_route + kq::moe_route_words() / 2);
        a.err = g_err_dev;
        a.fsync = g_fsync;
        if (s.normed) {
            a.nx = x;
            a.ndelta = delta;
            a.nscale = scale;
            a.neps = s.eps;
        } else {
            a.x = x;
        }
        // the test hook of moe_impl (KATALI_HIP_TEST_SKEW), for the stack
        if (env_on("KATALI_HIP_TEST_SKEW") && !g_capturing) {
            const hipError_t e = hipMemsetAsync(g_fsync + kq::FSYNC_X, 0xA5, 4, g_stream);
            if (e != hipSuccess) return hip_fail(e, "test skew");
        }
        const hipError_t e = kq::launch_moe_stack(a, s.table, (uint32_t)s.layers.size(), s.normed, g_stream);
        if (e == hipSuccess) return KATALI_HIP_OK;
        if (e != hipErrorNotSupported) return hip_fail(e, "moe stack launch");
    }
    return stack_layer_by_layer(s, x, delta, scale);
}

int katali_hip_moe_stack_destroy(void *stack) {
    if (!stack) return KATALI_HIP_OK;
    int rc = ensure();
    if (rc) return rc;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_moe_stack_destroy during graph capture");
    MoeStack *s = (MoeStack *)stack;
    hipError_t e = hipStreamSynchronize(g_stream);
    const hipError_t f1 = hipFree(s->table);
    const hipError_t f2 = s->res[0] ? hipFree(s->res[0]) : hipSuccess;
    delete s;
    if (e == hipSuccess) e = f1 != hipSuccess ? f1 : f2;
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "katali_hip_moe_stack_destroy");
}

int katali_hip_moe_layer_debug(const KataliHipMoe *m, const KataliHipMoeRoute *r, const float *x, const void *xq,
                               float *y, float *gu, void *hq8) {
    return moe_impl(m, r, x, xq, y, gu, hq8);
}

int katali_hip_step_advance(int32_t *step, int32_t n_steps) {
    int rc = ensure();
    if (rc) return rc;
    if (!step || n_steps < 1) return fail(KATALI_HIP_E_INVALID, "step/n_steps");
    return launched(kq::launch_step_advance(step, n_steps, g_stream), "step_advance");
}

int katali_hip_graph_begin(void) {
    int rc = ensure();
    if (rc) return rc;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "capture already active");
    hipError_t e = hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(e, "hipStreamBeginCapture");
    g_capturing = true;
    return KATALI_HIP_OK;
}

int katali_hip_graph_end(void **graph) {
    int rc = ensure();
    if (rc) return rc;
    if (!g_capturing) return fail(KATALI_HIP_E_INVALID, "no capture active");
    g_capturing = false;
    std::vector<void *> frees;
    frees.swap(g_deferred_free);
    hipGraph_t gr = nullptr;
    hipError_t e = hipStreamEndCapture(g_stream, &gr);
    if (e != hipSuccess) {
        if (gr) (void)hipGraphDestroy(gr);
        (void)release_frees(frees);
        return hip_fail(e, "hipStreamEndCapture");
    }
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0);
    (void)hipGraphDestroy(gr);
    if (e != hipSuccess) {
        (void)release_frees(frees);
        return hip_fail(e, "hipGraphInstantiate");
    }
    if (!graph) {
        (void)hipGraphExecDestroy(ex);
        (void)release_frees(frees);
        return fail(KATALI_HIP_E_INVALID, "null graph out");
    }
    *graph = (void *)ex;
    // the graph's replays may use what was freed during its capture
    if (!frees.empty()) g_graph_frees[(void *)ex].swap(frees);
    return KATALI_HIP_OK;
}

int katali_hip_graph_launch(void *graph) {
    int rc = ensure();
    if (rc) return rc;
    if (!graph) return fail(KATALI_HIP_E_INVALID, "null graph");
    return launched(hipGraphLaunch((hipGraphExec_t)graph, g_stream), "hipGraphLaunch");
}

int katali_hip_graph_destroy(void *graph) {
    if (!graph) return KATALI_HIP_OK;
    hipError_t e = hipGraphExecDestroy((hipGraphExec_t)graph);
    auto it = g_graph_frees.find(graph);
    if (it != g_graph_frees.end()) {
        std::vector<void *> v;
        v.swap(it->second);
        g_graph_frees.erase(it);
        const int rc = release_frees(v);   // after the stream drains: a replay may still run
        if (rc && e == hipSuccess) return rc;
    }
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "hipGraphExecDestroy");
}

int katali_hip_event_create(void **ev) {
    int rc = ensure();
    if (rc) return rc;
    if (!ev) return fail(KATALI_HIP_E_INVALID, "null out pointer");
    return launched(hipEventCreate((hipEvent_t *)ev), "hipEventCreate");
}

int katali_hip_event_record(void *ev) {
    int rc = ensure();
    if (rc) return rc;
    return launched(hipEventRecord((hipEvent_t)ev, g_stream), "hipEventRecord");
}

int katali_hip_event_elapsed(void *a, void *b, float *ms) {
    int rc = ensure();
    if (rc) return rc;
    if (!a || !b || !ms) return fail(KATALI_HIP_E_INVALID, "null argument");
    hipError_t e = hipEventSynchronize((hipEvent_t)b);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b);
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "hipEventElapsedTime");
}

int katali_hip_event_destroy(void *ev) {
    if (!ev) return KATALI_HIP_OK;
    return launched(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy");
}

// ---- pipelined uploads ------------------------------------------------------
// A pinned host ring of n_chunks chunks and a copy stream of its own
// (default priority). An upload copies the host bytes into the ring a chunk
// at a time (the CPU copy of chunk i + 1 overlaps the DMA of chunk i; a
// chunk is reused once its last DMA is done) and queues each chunk's DMA on
// the copy stream. Marks are events recorded on the library stream; an
// upload that names a mark queues its DMAs behind it (the copy stream waits
// for the library stream's work up to that mark), and a fence makes the
// library stream wait for every DMA queued so far.
// The CPU copy into a chunk is split over the calling thread and
// KATALI_HIP_STAGER_THREADS - 1 workers (default 4 threads in all; one CPU
// thread copies from a mapped file well below the link's rate).
constexpr uint32_t STAGER_MARKS = 64;
constexpr uint64_t STAGER_MIN_PIECE = 256u << 10;   // smaller copies stay on the calling thread
struct Stager {
    hipStream_t cs = nullptr;
    uint8_t *ring = nullptr;
    uint64_t chunk = 0;
    uint32_t n_chunks = 0, next = 0;
    std::vector<hipEvent_t> done;   // per chunk: its last DMA has finished
    std::vector<char> busy;         // per chunk: a DMA was queued from it
    hipEvent_t marks[STAGER_MARKS] = {};
    uint64_t n_marks = 0;           // mark m (1-based) is marks[(m - 1) % STAGER_MARKS]
    uint64_t waited = 0;            // the newest mark the copy stream already waits behind
    hipEvent_t tail = nullptr;
    // the copy workers: job `gen` copies len bytes src -> dst in `parts`
    // pieces, piece 0 on the calling thread, piece i on worker i - 1
    std::vector<std::thread> workers;
    std::mutex mu;
    std::condition_variable cv_job, cv_done;
    uint64_t gen = 0;
    uint32_t parts = 1, pending = 0;
    bool quit = false;
    uint8_t *dst = nullptr;
    const uint8_t *src = nullptr;
    uint64_t len = 0;
};

// piece i of n of a len-byte copy (64-byte aligned bounds)
static void stager_piece(uint32_t i, uint32_t n, uint8_t *dst, const uint8_t *src, uint64_t len) {
    const uint64_t step = ((len + n - 1) / n + 63) & ~63ull;
    const uint64_t lo = std::min(len, step * i), hi = std::min(len, lo + step);
    if (hi > lo) memcpy(dst + lo, src + lo, hi - lo);
}

static void stager_worker(Stager *s, uint32_t idx) {
    uint64_t seen = 0;
    for (;;) {
        uint8_t *dst;
        const uint8_t *src;
        uint64_t len;
        uint32_t parts;
        {
            std::unique_lock<std::mutex> lk(s->mu);
            s->cv_job.wait(lk, [&] { return s->quit || s->gen != seen; });
            if (s->quit) return;
            seen = s->gen;
            dst = s->dst, src = s->src, len = s->len, parts = s->parts;
        }
        if (idx + 1 < parts) stager_piece(idx + 1, parts, dst, src, len);
        std::lock_guard<std::mutex> lk(s->mu);
        if (--s->pending == 0) s->cv_done.notify_one();
    }
}

// memcpy(dst, src, len) over the calling thread and the workers
static void stager_copy(Stager *s, uint8_t *dst, const uint8_t *src, uint64_t len) {
    const uint32_t nw = (uint32_t)s->workers.size();
    const uint32_t parts = (uint32_t)std::min<uint64_t>(nw + 1, std::max<uint64_t>(1, len / STAGER_MIN_PIECE));
    if (parts <= 1) {
        memcpy(dst, src, len);
        return;
    }
    {
        std::lock_guard<std::mutex> lk(s->mu);
        s->dst = dst, s->src = src, s->len = len, s->parts = parts;
        s->pending = nw;   // every worker answers each job, with a piece or without
        s->gen++;
    }
    s->cv_job.notify_all();
    stager_piece(0, parts, dst, src, len);
    std::unique_lock<std::mutex> lk(s->mu);
    s->cv_done.wait(lk, [&] { return s->pending == 0; });
}

static void stager_release(Stager *s) {
    if (!s) return;
    {
        std::lock_guard<std::mutex> lk(s->mu);
        s->quit = true;
    }
    s->cv_job.notify_all();
    for (std::thread &t : s->workers) t.join();
    if (s->cs) (void)hipStreamSynchronize(s->cs);
    for (hipEvent_t e : s->done)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : s->marks)
        if (e) (void)hipEventDestroy(e);
    if (s->tail) (void)hipEventDestroy(s->tail);
    if (s->ring) (void)hipHostFree(s->ring);
    if (s->cs) (void)hipStreamDestroy(s->cs);
    delete s;
}

int katali_hip_stager_create(uint64_t chunk_bytes, uint32_t n_chunks, void **out) {
    int rc = ensure();
    if (rc) return rc;
    if (!out) return fail(KATALI_HIP_E_INVALID, "null out pointer");
    *out = nullptr;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_stager_create during graph capture");
    if (chunk_bytes < 4096 || chunk_bytes > (1ull << 30) || n_chunks < 2 || n_chunks > 64)
        return fail(KATALI_HIP_E_INVALID, "stager: chunk %llu bytes (4 KiB .. 1 GiB), %u chunks (2 .. 64)",
                    (unsigned long long)chunk_bytes, n_chunks);
    Stager *s = new (std::nothrow) Stager;
    if (!s) return fail(KATALI_HIP_E_NOMEM, "stager: out of memory");
    s->chunk = chunk_bytes;
    s->n_chunks = n_chunks;
    s->done.assign(n_chunks, nullptr);
    s->busy.assign(n_chunks, 0);
    hipError_t e = hipStreamCreateWithFlags(&s->cs, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipHostMalloc((void **)&s->ring, chunk_bytes * n_chunks, hipHostMallocDefault);
    for (uint32_t i = 0; i < n_chunks && e == hipSuccess; i++)
        e = hipEventCreateWithFlags(&s->done[i], hipEventDisableTiming);
    for (uint32_t i = 0; i < STAGER_MARKS && e == hipSuccess; i++)
        e = hipEventCreateWithFlags(&s->marks[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s->tail, hipEventDisableTiming);
    if (e != hipSuccess) {
        stager_release(s);
        return hip_fail(e, "stager create");
    }
    const char *nt = getenv("KATALI_HIP_STAGER_THREADS");
    const long threads = nt && *nt ? std::max(1L, std::min(16L, strtol(nt, nullptr, 10))) : 4;
    try {
        for (long i = 0; i + 1 < threads; i++) s->workers.emplace_back(stager_worker, s, (uint32_t)i);
    } catch (...) {
        stager_release(s);
        return fail(KATALI_HIP_E_NOMEM, "stager: cannot start copy threads");
    }
    *out = s;
    return KATALI_HIP_OK;
}

int katali_hip_stager_destroy(void *stager) {
    if (!stager) return KATALI_HIP_OK;
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_stager_destroy during graph capture");
    stager_release((Stager *)stager);
    return KATALI_HIP_OK;
}

int katali_hip_stager_mark(void *stager, uint64_t *mark) {
    int rc = ensure();
    if (rc) return rc;
    if (!stager || !mark) return fail(KATALI_HIP_E_INVALID, "null argument");
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_stager_mark during graph capture");
    Stager *s = (Stager *)stager;
    const hipError_t e = hipEventRecord(s->marks[s->n_marks % STAGER_MARKS], g_stream);
    if (e != hipSuccess) return hip_fail(e, "stager mark");
    *mark = ++s->n_marks;
    return KATALI_HIP_OK;
}

int katali_hip_stager_upload(void *stager, void *dev, const void *host, uint64_t bytes, uint64_t after_mark) {
    int rc = ensure();
    if (rc) return rc;
    if (!stager || (bytes && (!dev || !host))) return fail(KATALI_HIP_E_INVALID, "null argument");
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_stager_upload during graph capture");
    Stager *s = (Stager *)stager;
    if (after_mark > s->n_marks)
        return fail(KATALI_HIP_E_INVALID, "stager: mark %llu not taken yet", (unsigned long long)after_mark);
    hipError_t e = hipSuccess;
    // a mark older than the event ring waits on the newer mark that reused
    // its event: later than needed, never earlier
    if (after_mark > s->waited) {
        e = hipStreamWaitEvent(s->cs, s->marks[(after_mark - 1) % STAGER_MARKS], 0);
        if (e != hipSuccess) return hip_fail(e, "stager wait");
        s->waited = after_mark;
    }
    for (uint64_t off = 0; off < bytes;) {
        const uint64_t len = std::min(s->chunk, bytes - off);
        const uint32_t c = s->next;
        s->next = (c + 1) % s->n_chunks;
        if (s->busy[c] && (e = hipEventSynchronize(s->done[c])) != hipSuccess) return hip_fail(e, "stager chunk");
        uint8_t *buf = s->ring + (uint64_t)c * s->chunk;
        stager_copy(s, buf, (const uint8_t *)host + off, len);
        e = hipMemcpyAsync((uint8_t *)dev + off, buf, len, hipMemcpyHostToDevice, s->cs);
        if (e == hipSuccess) e = hipEventRecord(s->done[c], s->cs);
        if (e != hipSuccess) return hip_fail(e, "stager DMA");
        s->busy[c] = 1;
        off += len;
    }
    return KATALI_HIP_OK;
}

int katali_hip_stager_fence(void *stager) {
    int rc = ensure();
    if (rc) return rc;
    if (!stager) return fail(KATALI_HIP_E_INVALID, "null argument");
    if (g_capturing) return fail(KATALI_HIP_E_INVALID, "katali_hip_stager_fence during graph capture");
    Stager *s = (Stager *)stager;
    hipError_t e = hipEventRecord(s->tail, s->cs);
    if (e == hipSuccess) e = hipStreamWaitEvent(g_stream, s->tail, 0);
    return e == hipSuccess ? KATALI_HIP_OK : hip_fail(e, "stager fence");
}

int katali_hip_synth_fill(uint32_t type, void *dev, uint64_t nblocks, uint64_t seed, float d_sigma) {
    int rc = ensure();
    if (rc) return rc;
    if (!type_ok(type)) return fail(KATALI_HIP_E_UNSUPPORTED, "type %u", type);
    if (!dev) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (!nblocks) return KATALI_HIP_OK;
    return launched(kq::launch_synth_blocks(type, (uint8_t *)dev, nblocks, seed, d_sigma, g_stream), "synth_fill");
}

int katali_hip_synth_normal(float *dev, uint64_t n, uint64_t seed, float sigma) {
    int rc = ensure();
    if (rc) return rc;
    if (!dev) return fail(KATALI_HIP_E_INVALID, "null buffer");
    if (!n) return KATALI_HIP_OK;
    return launched(kq::launch_synth_normal(dev, n, seed, sigma, g_stream), "synth_normal");
}

int katali_hip_copy(void *dst, const void *src, size_t bytes) {
    int rc = ensure();
    if (rc) return rc;
    if (!dst || !src || bytes % 16) return fail(KATALI_HIP_E_INVALID, "copy needs non-null buffers, bytes %% 16 == 0");
    return launched(kq::launch_copy((const uint8_t *)src, (uint8_t *)dst, bytes, g_stream), "copy");
}

int katali_hip_selftest(char *report, size_t cap) {
    int rc = ensure();
    if (rc) return rc;
    std::string rep;
    int failures = 0;
    const uint64_t rows = 512, cols = 2048;
    // activation exactly representable in q8_1: per block d = 2^-6, q in
    // [-127, 127] with |q[0]| = 127, so quantization reproduces it exactly
    std::vector<float> x(cols);
    uint64_t s = 0x9E3779B97F4A7C15ull;
    for (uint64_t i = 0; i < cols; i++) {
        s ^= s << 13; s ^= s >> 7; s ^= s << 17;
        int q = (int)(s % 255) - 127;
        if (i % 32 == 0) q = (s & 1) ? 127 : -127;
        x[i] = (float)q / 64.0f;
    }
    for (uint32_t type : {KATALI_HIP_TYPE_Q4_K, KATALI_HIP_TYPE_Q6_K}) {
        const uint64_t bb = type == KATALI_HIP_TYPE_Q4_K ? 144 : 210;
        const uint64_t nbl = rows * cols / 256;
        void *w = nullptr, *xd = nullptr, *y0 = nullptr, *y1 = nullptr;
        if ((rc = katali_hip_malloc(&w, nbl * bb)) || (rc = katali_hip_malloc(&xd, cols * 4)) ||
            (rc = katali_hip_malloc(&y0, rows * 4)) || (rc = katali_hip_malloc(&y1, rows * 4))) {
            katali_hip_free(w); katali_hip_free(xd); katali_hip_free(y0); katali_hip_free(y1);
            return rc;
        }
        std::vector<float> a(rows), b(rows);
        rc = katali_hip_synth_fill(type, w, nbl, 1234 + type, 0.02f);
        if (!rc) rc = katali_hip_upload(xd, x.data(), cols * 4);
        if (!rc) rc = launched(kq::launch_gemv(type, (const uint8_t *)w, rows, cols, (const float *)xd, nullptr,
                                               (float *)y0, 0, g_stream), "selftest fp32");
        if (!rc) rc = katali_hip_matvec_dp4a(type, w, rows, cols, (const float *)xd, (float *)y1);
        if (!rc) rc = katali_hip_download(a.data(), y0, rows * 4);
        if (!rc) rc = katali_hip_download(b.data(), y1, rows * 4);
        katali_hip_free(w); katali_hip_free(xd); katali_hip_free(y0); katali_hip_free(y1);
        if (rc) return rc;
        double num = 0, den = 0;
        for (uint64_t i = 0; i < rows; i++) {
            num += ((double)a[i] - b[i]) * ((double)a[i] - b[i]);
            den += (double)a[i] * a[i];
        }
        const double rel = den > 0 ? sqrt(num / den) : sqrt(num);
        const bool ok = rel <= 1e-5;
        failures += ok ? 0 : 1;
        char line[160];
        snprintf(line, sizeof line, "dp4a-selftest %s %llux%llu: rel_L2(dp4a, fp32) = %.3e %s\n",
                 type == KATALI_HIP_TYPE_Q4_K ? "Q4_K" : "Q6_K", (unsigned long long)rows, (unsigned long long)cols,
                 rel, ok ? "PASS" : "FAIL");
        rep += line;
    }
    if (report && cap) {
        strncpy(report, rep.c_str(), cap - 1);
        report[cap - 1] = 0;
    }
    return failures ? fail(KATALI_HIP_E_RUNTIME, "selftest: %d failure(s)", failures) : KATALI_HIP_OK;
}

}  // extern "C"
