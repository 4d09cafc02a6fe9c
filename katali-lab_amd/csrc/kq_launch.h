// kq_launch.h — host-side launchers shared by the HIP translation units and the
// C-ABI layer (katali_hip.cpp). All launchers enqueue on `stream` and return a
// hipError_t; argument validation happens in the ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kq_plan.h"

namespace kq {

// Compute units of the current device (cached per device; 256 if unknown).
int device_cu_count();

// q8_1 quantization of n fp32 values (n % 32 == 0) into 36-byte blocks.
hipError_t launch_quantize_q8_1(const float *x, uint64_t n, uint8_t *out, hipStream_t s);

// Dense GEMV y[rows] = W[rows x cols] . x.
//  mode 0: fp32 activation (dequantize-and-FMA path)
//  mode 1: q8_1 activation given as 36-byte blocks (xq)
//  mode 2: fp32 activation quantized to q8_1 inside every workgroup
hipError_t launch_gemv(uint32_t type, const uint8_t *w, uint64_t rows, uint64_t cols, const float *xf,
                       const uint8_t *xq, float *y, int mode, hipStream_t s);
// y = W . x for fp32 W [rows][cols] (cols % 4 == 0, w and x 16-byte aligned),
// bit-identical to the engine's AVX2 F32 dot.
hipError_t launch_gemv_f32(const float *w, uint64_t rows, uint64_t cols, const float *x, float *y, hipStream_t s);
// Residual step (delta != nullptr), RMSNorm and F32 GEMV in one launch
// (n <= 8192, n % 4 == 0, 1 <= rows < 2^31, x_out apart from x; one
// workgroup per row).
hipError_t launch_norm_router(const float *x, const float *delta, float scale, float *x_out, const float *nw,
                              uint64_t n, float eps, float *xn, const float *w, uint64_t rows, float *y,
                              hipStream_t s);

// Up to GEMV_MULTI_MAX GEMVs sharing one fp32 activation in one launch
// (mode 0 or 2 as above); every output is bit-identical to launch_gemv's.
constexpr int GEMV_MULTI_MAX = 4;
struct GemvMultiArgs {
    const uint8_t *w[GEMV_MULTI_MAX];
    float *y[GEMV_MULTI_MAX];
    uint32_t rows[GEMV_MULTI_MAX];
    uint32_t type[GEMV_MULTI_MAX];
    uint32_t end[GEMV_MULTI_MAX];   // cumulative workgroup counts
    uint32_t cols, log2s4, log2s6;
    const float *x;
};
hipError_t launch_gemv_multi(int n, const uint32_t *types, const uint8_t *const *ws, const uint64_t *rows,
                             uint64_t cols, const float *x, float *const *ys, int mode, hipStream_t s);

// Per-block exact integer sums of a GEMV against a q8_1 activation:
// Q4_K -> out[rows][cols/32], Q6_K -> out[rows][cols/16].
hipError_t launch_isums(uint32_t type, const uint8_t *w, uint64_t rows, uint64_t cols, const uint8_t *xq,
                        int32_t *out, hipStream_t s);

// Synthetic data (bench and harness inputs).
hipError_t launch_synth_blocks(uint32_t type, uint8_t *dst, uint64_t nblocks, uint64_t seed, float d_sigma,
                               hipStream_t s);
hipError_t launch_synth_normal(float *dst, uint64_t n, uint64_t seed, float sigma, hipStream_t s);

// *step = (*step + 1) % n_steps
hipError_t launch_step_advance(int32_t *step, int32_t n_steps, hipStream_t s);

// Plain streaming copy (HBM counter calibration).
hipError_t launch_copy(const uint8_t *src, uint8_t *dst, uint64_t n, hipStream_t s);

// Greedy sampling: *out = index of the largest of n logits (first maximum
// wins, NaN never, 0 when nothing exceeds -FLT_MAX), one launch. scratch:
// argmax_scratch_bytes(), zeroed once before the first call (the kernel
// leaves it ready for the next).
uint32_t argmax_scratch_bytes();
// out = RMSNorm(x) * w with the engine's arithmetic; the add variant first
// does x += delta (scale 1) or x += scale * delta in place. One workgroup;
// out may be x.
hipError_t launch_rmsnorm(const float *x, const float *w, uint32_t n, float eps, float *out, hipStream_t s);
hipError_t launch_add_rmsnorm(float *x, const float *delta, float scale, const float *w, uint32_t n, float eps,
                              float *out, hipStream_t s);
hipError_t launch_argmax(const float *x, uint32_t n, void *scratch, int32_t *out, hipStream_t s);

// MoE layer (two launches). Types: gate/up Q4_K; down Q4_K or Q6_K.
struct MoeArgs {
    const uint8_t *gate, *up, *down;          // stacked [n_expert][rows][row_bytes]
    const uint8_t *gate_sh, *up_sh, *down_sh; // shared expert (NULL when absent)
    uint32_t gate_type, up_type, down_type;
    uint32_t hidden, ffn, n_expert;
    int n_sel;                                // routed experts per token
    int has_shared;
    const float *x;          // fp32 activation [hidden] (or NULL)
    const uint8_t *xq;       // q8_1 activation (or NULL)
    const float *logits;     // router logits [n_expert] (or NULL: ids/wts given)
    const int32_t *step;     // optional: logits += (*step) * logits_stride
    uint64_t logits_stride;
    const int32_t *ids;      // selected experts [n_sel] (when logits == NULL)
    const float *wts;        // their weights [n_sel]
    int32_t *ids_out;        // optional routing output
    float *wts_out;
    float *y;                // [hidden]
    uint8_t *hq8;            // scratch [n_slots][ffn/32][36]
    int32_t *route_ids;      // scratch [moe_route_words()/2]: routing from kernel A to kernel B
    float *route_w;
    float *dbg_gu;           // optional [n_slots][2][ffn] gate/up outputs
    int32_t *err;            // error word (bit 1: expert id out of range, bit 2: fused-layer wait expired)
    uint32_t *fsync;         // fused layer's exchange (layout at fsync_words())
    // Batched layer (several tokens): a pair p = t * bS + r is token t's rank
    // r (r == n_sel: the shared expert). bslot holds *bcount {expert, first,
    // count} entries whose pairs are border[first .. first + count); x comes
    // from the q8_1 rows xq + t * xq_stride, h goes to hq8 row p and the
    // pair's unweighted down output to yp + p * hidden.
    const int32_t *bslot;
    const int32_t *bcount;
    const int32_t *border;
    uint32_t bS;
    uint64_t xq_stride;
    float *yp;
    // The steps before the layer, in kernel A (launch_moe_normed; router !=
    // NULL): x_out = nx + nscale * ndelta (with ndelta), xn = RMSNorm(x_out or
    // nx) * nw, logits = router . xn, routed from those logits.
    const float *nx, *ndelta;
    float nscale, neps;
    float *nx_out;
    const float *nw;
    float *nxn_out;
    const float *router;   // F32 [n_expert][hidden]
    float *logits_out;
    // The one-launch layers: h words handed over inside the XCD (set by the
    // launcher from xcd_local(); callers leave it 0)
    uint32_t hloc;
};
bool moe_shape_supported(uint32_t gate_type, uint32_t down_type, uint32_t hidden, uint32_t ffn);
// Dynamic LDS (bytes) of the largest workgroup a layer of this shape launches:
// kernel A, kernel B (n_slots * (ffn + ffn/8 + ffn/4) for the staged h, plus
// at most (B_MAX_THREADS + n_slots) partial sums), or for the batched layer
// the grouped GEMV kernels (8 pairs' h) and the MFMA kernels. The host checks
// these against the device's per-workgroup LDS before it launches anything.
uint32_t moe_layer_lds(uint32_t hidden, uint32_t ffn, uint32_t n_slots);
uint32_t moe_groups_lds(uint32_t hidden, uint32_t ffn);
uint32_t moe_batch_lds(uint32_t hidden, uint32_t ffn);
// gfx950's LDS per workgroup
constexpr uint32_t LDS_PER_WG = 160 * 1024;
// The layer in one launch when the shape fits the fused kernel and a.fsync is
// set (and `allow_fused`), else kernels A and B. *fused tells which ran.
// allow_xcd: the XCD-sliced one-launch layer where the shape fits it
// (eight slots, or with xcd_shared_units eight routed experts and the
// shared expert with ffn 256 or 512; hidden 1024 or 2048, ffn <= 1024,
// <= 256 experts, a 256-CU device), tried before the fused one.
hipError_t launch_moe(const MoeArgs &a, hipStream_t s, bool allow_fused = false, bool *fused = nullptr,
                      bool allow_xcd = false, bool xcd_shared_units = false);
// The in-kernel exchanges (zeroed once, before first use): [0] the fused
// layer's generation, [1] the normed layer's; from FSYNC_H one block per
// workgroup of the fused layer of 9 8-byte words {dword, generation} (its
// q8_1 h block, or zeros); from FSYNC_R, FSYNC_REP copies 4 KiB apart of one
// 8-byte word {logit, generation} per router row of the normed layer (its
// workgroups read the copy of their index mod FSYNC_REP, so no few cache
// lines take every poll).
// From FSYNC_X, the XCD-sliced layer's (launch_moe with allow_xcd): one
// generation word per workgroup (XCD_G of them), then from FSYNC_XH its h
// values [slot][ffn <= 1024], then from FSYNC_XP its unweighted down
// partials [slot][hidden], then with the shared expert from FSYNC_XS its h
// [ffn <= 512] (each workgroup's share written through, read on every XCD)
// and from FSYNC_XSP its unweighted down partials [hidden]; from
// FSYNC_XR, with the steps before the layer in its prologue, FSYNC_REP
// copies of its router logits [512] (an area of its own: its generations
// are the XCD layer's); each value one 8-byte word {float, generation}. Each exchange has its own generations, so no
// word one of them writes can pass for another's.
constexpr uint32_t FSYNC_H = 64;
constexpr uint32_t FUSED_MAX_G = 256;   // workgroups of the fused layer
constexpr uint32_t FSYNC_R = 8192;      // 32 KiB in, past the fused layer's words
constexpr uint32_t FSYNC_REP = 16;
constexpr uint32_t XCD_SLOTS = 8;       // the XCD-sliced layer: slot x on XCD x
constexpr uint32_t XCD_G = 256;         // its workgroups: one per CU, 32 per XCD
constexpr uint32_t XCD_MAX_HIDDEN = 2048;
constexpr uint32_t FSYNC_X = FSYNC_R + FSYNC_REP * 2 * 512;
constexpr uint32_t FSYNC_XH = FSYNC_X + XCD_G;
constexpr uint32_t XCD_MAX_FFN = 1024;
constexpr uint32_t FSYNC_XP = FSYNC_XH + 2 * XCD_SLOTS * XCD_MAX_FFN;
constexpr uint32_t XCD_MAX_SH_FFN = 512;   // the shared expert's ffn in that layer
constexpr uint32_t FSYNC_XS = FSYNC_XP + 2 * XCD_SLOTS * XCD_MAX_HIDDEN;
constexpr uint32_t FSYNC_XSP = FSYNC_XS + 2 * XCD_MAX_SH_FFN;
constexpr uint32_t FSYNC_XR = FSYNC_XSP + 2 * XCD_MAX_HIDDEN;
// From FSYNC_XY, the stacked layer's (launch_moe_stack): two areas (layer
// parity) of a layer's y [hidden] as words {float, generation}, read by the
// next layer of the stack, then from FSYNC_XF two areas of one completion
// word per workgroup (its generation, written once its y is stored); its
// generations are the XCD layer's.
constexpr uint32_t FSYNC_XY = FSYNC_XR + FSYNC_REP * 2 * 512;
constexpr uint32_t FSYNC_XF = FSYNC_XY + 2 * 2 * XCD_MAX_HIDDEN;
// From FSYNC_DHC, kernel A's half units (a dense FFN): one counter per q8_1
// block of h (DH_MAX_BLOCKS; every call adds 2 per block), then from
// FSYNC_DHW each block's 32 values as words {float, generation}.
constexpr uint32_t DH_MAX_BLOCKS = 512;   // ffn <= 16384
constexpr uint32_t FSYNC_DHC = FSYNC_XF + 2 * XCD_G;
constexpr uint32_t FSYNC_DHW = FSYNC_DHC + DH_MAX_BLOCKS;
constexpr uint32_t fsync_words() { return FSYNC_DHW + 2 * 32 * DH_MAX_BLOCKS; }
static_assert(FSYNC_H + 2 * 9 * FUSED_MAX_G <= FSYNC_R, "exchange areas overlap");
// The steps before the layer and the layer in two launches (MoeArgs' n*
// fields and router set, n_sel >= 1, hidden <= 4096): kernel A forms the
// residual step, the RMSNorm and its router rows itself (bit-identical to
// launch_norm_router), exchanges the logits between its workgroups through
// a.fsync, routes and runs the gate/up units; kernel B as launch_moe's.
// When the router rows do not spread over kernel A's workgroups (more than
// 4 rows each), launch_norm_router into xn_buf / logits_buf first, then
// launch_moe. *merged tells which ran.
// allow_xcd: eight-slot layers of the XCD-sliced layer's shapes run as that
// layer with the steps before it in its prologue, in one launch.
hipError_t launch_moe_normed(MoeArgs a, float *xn_buf, float *logits_buf, hipStream_t s, bool *merged = nullptr,
                             bool allow_xcd = false);
// One layer of the stacked layer (launch_moe_stack): weights, routing and
// outputs. Plain stack: logits (with step / logits_stride) or ids / wts route
// the layer; NORMED: nw and router form its norm and routing, x_out / xn_out
// / logits_out are optional outputs (the residual entering the layer's norm,
// the normalized vector, the router logits).
struct StackLayer {
    const float *x;   // plain stack, layers past the first: its own input (null: the previous layer's y)
    const uint8_t *gate, *up, *down;
    const uint8_t *gate_sh, *up_sh, *down_sh;
    const float *logits;
    const int32_t *step;
    uint64_t logits_stride;
    const int32_t *ids;
    const float *wts;
    int32_t *ids_out;
    float *wts_out;
    float *y;
    const float *nw, *router;
    float *x_out, *xn_out, *logits_out;
};
// n_layers layers of a's shape in one launch of the XCD-sliced layer's
// workgroups, lt[l] a device table of each layer's pointers (a's own weight,
// routing and output pointers are ignored). Plain: layer 0's x is a.x or
// a.xq and layer l's is lt[l].x or, null, layer l - 1's y; a layer issues no
// weight load before the previous layer's y is complete either way; every
// output bit-identical to launch_moe's XCD layer run layer by layer on
// those inputs. normed: a's n*
// fields give layer 0's residual step (nx, optional ndelta / nscale), layer
// l adds layer l - 1's y to the residual stream; outputs bit-identical to
// launch_moe_normed layer by layer. hipErrorNotSupported for shapes the XCD
// layer does not take (then nothing is launched).
hipError_t launch_moe_stack(const MoeArgs &a, const StackLayer *lt, uint32_t n_layers, bool normed, hipStream_t s);
// After an expired in-kernel wait the library stops choosing the layers
// whose workgroups wait for each other (the XCD-sliced layer and the stack);
// kernels A and B run every later layer.
void xcd_disable();
void xcd_enable();
bool xcd_disabled();
// Dispatch check for the XCD-local h hand-off (run once, outside capture):
// on when every launch of XCD_G workgroups puts each b % 8 class on one XCD.
hipError_t xcd_dispatch_check(hipStream_t s);
bool xcd_local();
void xcd_local_set(bool on);
// The measurement build's phase stamps of the one-launch layers
// ([64][256][16] uint64, s_memrealtime ticks); hipErrorNotSupported in the
// product build.
hipError_t read_stamps(void *host, size_t bytes);
// The streaming floors (kq_floor.hip): kind 0 one read of a, 1 a then b in
// two launches, 2 a then b in one launch with the XCD-sliced layer's two
// in-kernel waits; sync: floor_sync_words() + 1 zeroed words, kept between
// launches.
uint32_t floor_sync_words();
hipError_t launch_floor(int kind, const uint8_t *a, uint64_t a_bytes, const uint8_t *b, uint64_t b_bytes,
                        uint32_t *sync, hipStream_t s);
// The exchange probe (kq_floor.hip, k_xchg): rounds of a word passed back
// and forth between workgroup pairs, kind 0 inside an XCD group through its
// L2, 1 inside it written through, 2 across XCDs; words: xchg_words()
// zeroed words, kept between launches.
uint32_t xchg_words();
hipError_t launch_xchg(int kind, uint32_t rounds, uint32_t *words, hipStream_t s);
// Top-n_sel routing of n_tokens rows of logits [n_tokens][n_expert] (<= 512
// experts, 1 <= n_sel <= min(16, n_expert)): ids / weights [n_tokens][n_sel],
// each row as the single-token layer routes it.
hipError_t launch_route_batch(const float *logits, uint32_t n_tokens, uint32_t n_expert, int n_sel, int32_t *ids,
                              float *wts, hipStream_t s);
// Grouped batch mode over up to max_entries entries of <= 8 pairs of one
// expert (the batched layer's GEMV path).
hipError_t launch_moe_groups_gu(const MoeArgs &a, uint32_t max_entries, hipStream_t s);
hipError_t launch_moe_groups_down(const MoeArgs &a, uint32_t max_entries, hipStream_t s);
// MoE layer over T <= 64 tokens (a.ids / a.wts: [T][n_sel]; a.hq8: P rows of
// ffn/32 q8_1 blocks, a.yp: [P][hidden], P = T * (n_sel + shared)). Experts
// gathering >= min_big pairs use the int8 MFMA grouped GEMM, the rest the
// per-pair GEMV kernels. xq: T rows of hidden/32 q8_1 blocks; meta:
// moe_batch_meta_words(P) ints. The two paths touch disjoint pairs and run
// side by side: the MFMA kernels on `aux`, forked from `s` after the
// grouping (event `fork`) and joined back before the combine (`join`).
uint64_t moe_batch_meta_words(uint32_t P);
hipError_t launch_moe_batch(const MoeArgs &a, uint32_t T, uint32_t min_big, const float *x, float *y, uint8_t *xq,
                            int32_t *meta, hipStream_t s, hipStream_t aux, hipEvent_t fork, hipEvent_t join);
uint64_t moe_route_words();

}  // namespace kq
