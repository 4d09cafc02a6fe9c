/* katali_hip.h — C ABI of libkatali_hip, the MI355X (gfx950) backend for
 * katali-lab's quantized expert-GEMV path.
 *
 * The engine finds this library at run time (dlopen / LoadLibrary, see
 * katali_hip_loader.h); nothing links against it at build time. Plain C types
 * only: device buffers are `void *` handles returned by katali_hip_malloc.
 *
 * Reference interfaces replaced (paths relative to the reference repository,
 * V/ = vendor/katali_gguf_dense/):
 *   - The loader API the dense shim calls, declared in the reference's absent
 *     include/katali_cuda.h and visible at its call sites in
 *     V/src/katali_dense_cuda.c:19,27-31,40-41,48,52-54,65-71:
 *       katali_cuda_probe / _status / _malloc / _free / _upload / _download /
 *       _supports_type / _matvec  ->  katali_hip_<same name>.
 *   - The fused-MoE, q8_1/DP4A, self-test and bench entry points of the closed
 *     katali_cuda.dll (README.md:13,17,21,99-102,149-171,308-310), which have
 *     no published signatures: defined here.
 *
 * Conventions (from the reference's SDK contract, V/include/katali_gguf_sdk.h:22-69):
 *   - every int-returning call returns KATALI_HIP_OK (0) or a negative code;
 *     katali_hip_last_error() gives a message for the calling thread;
 *   - structs carry struct_size for forward compatibility;
 *   - tensors use the GGUF layout: dims[0] = cols contiguous, dims[1] = rows
 *     (V/include/katali_gguf.h:67); types are ggml ids (Q4_K = 12, Q6_K = 14).
 *   - compute calls are asynchronous on the library stream; katali_hip_download
 *     and katali_hip_sync wait for them. One caller thread at a time.
 */
#ifndef KATALI_HIP_H
#define KATALI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KATALI_HIP_ABI_VERSION 1

#define KATALI_HIP_OK 0
#define KATALI_HIP_E_INVALID (-1)     /* bad argument or unsupported shape */
#define KATALI_HIP_E_NODEVICE (-2)    /* no usable gfx950 device */
#define KATALI_HIP_E_RUNTIME (-3)     /* HIP runtime error */
#define KATALI_HIP_E_UNSUPPORTED (-4) /* type / option not implemented */
#define KATALI_HIP_E_NOMEM (-5)       /* device allocation failed */
#define KATALI_HIP_E_TIMEOUT (-6)     /* in-kernel dependency wait expired */

#define KATALI_HIP_TYPE_F32 0u
#define KATALI_HIP_TYPE_Q4_K 12u
#define KATALI_HIP_TYPE_Q6_K 14u

int         katali_hip_abi_version(void);
const char *katali_hip_last_error(void);

/* ---- loader API (replaces katali_cuda_* at V/src/katali_dense_cuda.c) ---- */

/* Non-zero when a gfx950 device is usable (initialises it on first call).
 * Replaces katali_cuda_probe (V/src/katali_dense_cuda.c:19). */
int         katali_hip_probe(void);
/* Human-readable reason for the probe result (device name, or why not).
 * Replaces katali_cuda_status (V/src/katali_dense_cuda.c:19). */
const char *katali_hip_status(void);
/* Replaces katali_cuda_malloc (V/src/katali_dense_cuda.c:30-31,40). */
int katali_hip_malloc(void **dev, size_t bytes);
/* Replaces katali_cuda_free (V/src/katali_dense_cuda.c:27-28,76-78). */
int katali_hip_free(void *dev);
/* Synchronous host->device copy. Replaces katali_cuda_upload (:41,52,65). */
int katali_hip_upload(void *dev, const void *host, size_t bytes);
/* Waits for queued work, then device->host. Replaces katali_cuda_download (:54,70). */
int katali_hip_download(void *host, const void *dev, size_t bytes);
/* 1 for Q4_K, Q6_K and F32 (F32: katali_hip_matvec only). Replaces
 * katali_cuda_supports_type (:48,67). */
int katali_hip_supports_type(uint32_t ggml_type);
/* y[rows] = W[rows x cols] . x with fp32 x and y, W in GGUF layout on the
 * device. With KATALI_CUDA_DP4A=1 (or KATALI_HIP_DP4A=1) in the environment x
 * is quantized to q8_1 inside the kernel and dotted with v_dot4; otherwise
 * weights are dequantized and dotted in fp32. cols % 256 == 0.
 * F32 weights (type 0: the MoE router matrices) take their own kernel,
 * bit-identical to the engine's AVX2 F32 dot (V/src/gguf_simd_x86.c:111-122,
 * the path katali_ggml_matvec takes for F32 rows, gguf_simd_x86.c:875-877):
 * cols % 4 == 0, w and x 16-byte aligned, the DP4A switch does not apply.
 * Replaces katali_cuda_matvec (V/src/katali_dense_cuda.c:53,69). */
int katali_hip_matvec(uint32_t type, const void *w_dev, uint64_t rows, uint64_t cols,
                      const float *x_dev, float *y_dev);

/* ---- runtime helpers ------------------------------------------------------ */
int katali_hip_sync(void);
int katali_hip_memset(void *dev, int value, size_t bytes);
/* Run library work on an external stream (a hipStream_t, NULL = library's). */
int katali_hip_set_stream(void *hip_stream);

/* ---- q8_1 activation path (README.md:17, "quantized once on the device") -- */
/* n % 32 == 0; writes n/32 36-byte block_q8_1 (d f16, s f16 = d*sum(q), qs). */
int katali_hip_quantize_q8_1(const float *x_dev, uint64_t n, void *q8_dev);
/* y = W . x with x given as q8_1 blocks (int8 x int8 -> int32 dot4 path). */
int katali_hip_matvec_q8(uint32_t type, const void *w_dev, uint64_t rows, uint64_t cols,
                         const void *xq8_dev, float *y_dev);
/* Same with an fp32 x that every workgroup quantizes to q8_1 in LDS (one
 * launch, bit-identical to quantize_q8_1 followed by matvec_q8). */
int katali_hip_matvec_dp4a(uint32_t type, const void *w_dev, uint64_t rows, uint64_t cols,
                           const float *x_dev, float *y_dev);
/* Up to four GEMVs over one activation in one launch: ys[i][rows[i]] =
 * W_i . x, W_i of types[i] (Q4_K or Q6_K, mixed allowed), all with `cols`
 * columns. Replaces the per-tensor katali_cuda_matvec loop of
 * katali_dense_cuda_matvec_multi (V/src/katali_dense_cuda.c:58-72; called at
 * V/src/gguf_model.c:533 for q, k, v (:614) and gate, up (:680)): each
 * ys[i] is bit-identical to katali_hip_matvec on W_i. Activation
 * mode as katali_hip_matvec (fp32, or v_dot4 with KATALI_HIP_DP4A=1). */
int katali_hip_matvec_multi(int n, const uint32_t *types, const void *const *w_devs, const uint64_t *rows,
                            uint64_t cols, const float *x_dev, float *const *y_devs);
/* The same with x quantized to q8_1 in every workgroup (v_dot4), each output
 * bit-identical to katali_hip_matvec_dp4a. */
int katali_hip_matvec_multi_dp4a(int n, const uint32_t *types, const void *const *w_devs, const uint64_t *rows,
                                 uint64_t cols, const float *x_dev, float *const *y_devs);
/* Exact per-block int32 sums of the q8 GEMV, from the same device routines:
 * Q4_K -> isums[rows][cols/32], Q6_K -> isums[rows][cols/16] (sum of
 * (q6-32)*q8 per 16 values). For self-tests. */
int katali_hip_block_isums(uint32_t type, const void *w_dev, uint64_t rows, uint64_t cols,
                           const void *xq8_dev, int32_t *isums_dev);

/* ---- greedy sampling ---------------------------------------------------------- */
/* *out_dev = the index of the largest of n logits, with the engine's greedy
 * rule (gguf_sampler.c:62-66: strict '>' from -FLT_MAX, so the first maximum
 * wins, NaN never wins, 0 when no logit exceeds -FLT_MAX). 1 <= n < 2^31. */
int katali_hip_argmax(const float *logits_dev, uint64_t n, int32_t *out_dev);

/* ---- the decode chain's norm and residual (RMSNorm, residual add) -------- */
/* out[n] = RMSNorm(x) * w with the engine's arithmetic, replacing
 * katali_gguf_rmsnorm (V/src/gguf_kernels.c:13-18; called at
 * V/src/gguf_model.c:604,683,698): the sum of squares in double, inv =
 * 1/sqrtf((float)(sumsq/n) + eps), out[i] = x[i]*inv*w[i]. Bit-identical to
 * it unless the double sum, formed in another order, straddles a float
 * rounding boundary. out may be x (katali_gguf_rmsnorm_inplace, :20-25).
 * 1 <= n <= 2^20. */
int katali_hip_rmsnorm(const float *x_dev, const float *w_dev, uint64_t n, float eps, float *out_dev);
/* The residual step and the next norm in one launch: x += delta (scale ==
 * 1, katali_gguf_add_inplace at V/src/gguf_model.c:677,692) or x += scale *
 * delta (:678,693), in place, then out = RMSNorm(x) * w as above. */
int katali_hip_add_rmsnorm(float *x_dev, const float *delta_dev, float scale, const float *w_dev, uint64_t n,
                           float eps, float *out_dev);
/* The steps before a MoE layer in one launch: the residual step (when
 * delta_dev is not NULL: x_out = x + delta, or x + scale * delta), the norm
 * xn = RMSNorm(x_out or x) * norm_w as katali_hip_rmsnorm, and the router
 * logits y[rows] = W_router[rows x n] . xn as katali_hip_matvec on F32
 * (bit-identical to both: V/src/gguf_model.c:677-683 followed by the F32
 * router product, V/src/gguf_simd_x86.c:111-122). The new residual goes to
 * x_out, a buffer apart from x (x is read by every workgroup); with delta
 * NULL, x_out is unused and may be NULL. 4 <= n <= 8192, n % 4 == 0, 1 <= rows < 2^31,
 * all vectors and W 16-byte aligned; outputs must not overlap inputs. */
int katali_hip_rmsnorm_matvec_f32(const float *x_dev, const float *delta_dev, float scale, float *x_out_dev,
                                  const float *norm_w_dev, uint64_t n, float eps, float *xn_dev,
                                  const float *w_dev, uint64_t rows, float *y_dev);

/* ---- fused MoE layer (README.md:13, one GPU call per MoE layer) ----------- */
typedef struct KataliHipMoe {
    uint32_t struct_size;                  /* sizeof(KataliHipMoe) */
    uint32_t gate_type, up_type, down_type;/* Q4_K / Q6_K (gate and up equal) */
    uint32_t hidden;                       /* gate/up columns, down rows (%256) */
    uint32_t ffn;                          /* expert intermediate size (%256) */
    uint32_t n_expert;                     /* routed experts (<= 512) */
    const void *gate_exps, *up_exps, *down_exps; /* device, GGUF stacked experts:
                                              [n_expert][rows][row_bytes] */
    const void *gate_shexp, *up_shexp, *down_shexp; /* optional always-on shared
                                              expert (same types and ffn), weight 1 */
} KataliHipMoe;

typedef struct KataliHipMoeRoute {
    uint32_t struct_size;                  /* sizeof(KataliHipMoeRoute) */
    int32_t n_sel;                         /* routed experts per token, 0..16;
                                              0 = the shared expert alone (a
                                              dense SiLU-GLU FFN; routed experts,
                                              logits and ids may be NULL) */
    /* Either router logits (the kernel takes the top n_sel, largest first,
     * lower index on ties, and renormalises softmax over them) ... */
    const float *logits;                   /* device [n_expert] or NULL */
    const int32_t *step;                   /* optional device index: logits +=
                                              (*step) * logits_stride */
    uint64_t logits_stride;
    /* ... or an explicit selection. */
    const int32_t *ids;                    /* device [n_sel] */
    const float *weights;                  /* device [n_sel] */
    int32_t *ids_out;                      /* optional device outputs */
    float *weights_out;
} KataliHipMoeRoute;

/* y[hidden] = sum_r w_r * Down_e(SiLU(Gate_e x) * Up_e x) (+ shared expert).
 * x is fp32 (x_dev) or already q8_1 (xq8_dev); exactly one is non-NULL. The
 * activation and the SiLU-GLU output are quantized to q8_1 inside the kernel;
 * dots use int8 v_dot4 with fp32 scales; the expert sum is in rank order.
 * Shapes beyond what katali_hip_moe_check admits return an error before
 * anything is enqueued. Eight slots, and eight routed experts plus the
 * shared expert at ffn 256 or 512 (hidden 1024 or 2048, ffn <= 1024,
 * <= 256 experts, a 256-CU device), run as one launch whose 256 workgroups
 * wait for each other, so the library takes that form only where the
 * occupancy API confirms all 256 workgroups fit on the device at once. On a
 * device busy with other work a wait can still expire: each wait gives up
 * after about 2^20 polls (about a second, per wait, so a call can stall for
 * seconds), reported as KATALI_HIP_E_TIMEOUT by the next katali_hip_sync,
 * the outputs then invalid; from that report on, the library runs every
 * layer on the two-launch path (graphs captured before keep their kernels;
 * katali_hip_one_launch(1) allows the one-launch form again).
 * KATALI_HIP_XCD=0 in the environment keeps such layers on the two-launch
 * path, which never waits in-kernel (KATALI_HIP_XCD_SHARED=0 only the
 * shared-expert shapes). */
int katali_hip_moe_layer(const KataliHipMoe *moe, const KataliHipMoeRoute *route,
                         const float *x_dev, const void *xq8_dev, float *y_dev);

/* The steps before a MoE layer and the layer, in one launch for the eight-slot
 * shapes that katali_hip_moe_layer runs as one (the XCD-sliced layer; unless
 * KATALI_HIP_XCD=0) and two for the others, where the separate calls take one
 * more: katali_hip_rmsnorm_matvec_f32(x, delta, scale,
 * x_out, norm_w, hidden, eps, xn_out, router, n_expert, logits_out)
 * followed by katali_hip_moe_layer routed from those logits (n_sel experts,
 * ids_out / weights_out optional) on xn, with every output bit-identical to
 * that pair's (V/src/gguf_model.c:677-683, the F32 router product, the MoE
 * layer). The layer's first kernel forms the residual step, the norm and the
 * router rows in its own workgroups and exchanges the logits between them on
 * the device
 * (its workgroups wait for each other: on a device busy with other work the
 * wait can expire, reported as KATALI_HIP_E_TIMEOUT by the next
 * katali_hip_sync, the outputs then invalid). When kernel A has more
 * workgroups (n_slots * ffn / 32) than the device has CUs, or n_expert is
 * more than 4 router rows per workgroup, the call runs the norm/router
 * launch and the layer instead, with the same results. Rules of
 * katali_hip_rmsnorm_matvec_f32
 * (16-byte alignment, outputs apart from inputs) and of katali_hip_moe_layer;
 * n_sel >= 1; xn_out and logits_out may be NULL. No counterpart in the
 * reference: for an engine that keeps the residual stream on the device. */
typedef struct KataliHipMoeNorm {
    uint32_t struct_size;                  /* sizeof(KataliHipMoeNorm) */
    const float *x;                        /* residual stream [hidden] */
    const float *delta;                    /* optional: x_out = x + scale * delta */
    float scale;
    float *x_out;                          /* the new residual (with delta), apart from x */
    const float *norm_w;                   /* RMSNorm weights [hidden] */
    float eps;
    float *xn_out;                         /* optional: RMSNorm(x_out or x) * norm_w */
    const float *router;                   /* F32 router [n_expert][hidden] */
    float *logits_out;                     /* optional [n_expert] */
} KataliHipMoeNorm;
int katali_hip_moe_layer_normed(const KataliHipMoe *moe, const KataliHipMoeNorm *norm, int32_t n_sel,
                                int32_t *ids_out, float *weights_out, float *y_dev);

/* ---- a stack of MoE layers in one launch ---------------------------------- */
/* n_layers layers of one shape, each layer's input the previous layer's
 * output, run by one launch whose workgroups stay resident from layer to
 * layer (no launch gap between layers). A layer starts none of its weight
 * loads before the whole of the previous layer's output is written; it reads
 * only what does not depend on that output (its routing from given logits,
 * its router rows and norm weights) before.
 *   plain (normed == 0): layer 0 runs on run()'s x, layer l on its own x
 *     or, where that is NULL, on layer l-1's y (either way it waits for that
 *     y to be complete before its weight loads: a decode chain's order);
 *     each layer routed by its route (logits, or ids and weights; n_sel as
 *     the stack's), outputs bit-identical to katali_hip_moe_layer called
 *     layer by layer on those inputs.
 *   normed (normed != 0, n_sel >= 1, no shared expert): layer 0 takes
 *     x_0 = x (+ scale * delta when delta is given), layer l the residual
 *     x_l = x_{l-1} + y_{l-1}; each layer's norm (norm_w, eps), router
 *     logits (router) and layer as katali_hip_moe_layer_normed, outputs
 *     bit-identical to it called layer by layer (x_out, xn_out, logits_out
 *     optional per layer: the residual entering the layer's norm, the
 *     normalized vector, the logits).
 * The one-launch form needs the shapes katali_hip_moe_layer runs as one
 * launch (eight slots, or eight routed experts plus the shared expert at ffn
 * 256 or 512 for the plain stack; hidden 1024 or 2048, ffn <= 1024, <= 256
 * experts, a 256-CU device); elsewhere, with KATALI_HIP_XCD=0, or after an
 * expired wait, run() calls the layers one by one with the same results.
 * Its workgroups wait for each other as the one-launch layer's do (each wait
 * bounded at about 2^20 polls, about a second; an expiry is reported as
 * KATALI_HIP_E_TIMEOUT by the next katali_hip_sync, the outputs then
 * invalid). create() copies the layer table to the device (outside graph
 * capture); run() is one launch on the library stream and may be captured.
 * Per-layer vectors are 16-byte aligned; a layer's outputs must not overlap
 * each other, its inputs or the previous layer's y. No counterpart in the
 * reference: for an engine that keeps a token's MoE stack on the device. */
typedef struct KataliHipMoeStackLayer {
    uint32_t struct_size;                  /* sizeof(KataliHipMoeStackLayer) */
    const float *x;                        /* plain stack, layers 1..: this layer's own
                                              input [hidden] (NULL: layer l-1's y);
                                              layer 0's is run()'s x */
    const void *gate_exps, *up_exps, *down_exps;       /* this layer's experts */
    const void *gate_shexp, *up_shexp, *down_shexp;    /* with a shared expert */
    KataliHipMoeRoute route;               /* plain stack: this layer's routing; normed
                                              stack: only ids_out / weights_out (optional;
                                              struct_size 0 for none) */
    const float *norm_w;                   /* normed stack: RMSNorm weights [hidden] */
    const float *router;                   /* normed stack: F32 router [n_expert][hidden] */
    float *y;                              /* the layer's output [hidden] */
    float *x_out, *xn_out, *logits_out;    /* normed stack: optional outputs */
} KataliHipMoeStackLayer;
/* shape: types, hidden, ffn, n_expert and which shared-expert pointers are
 * set (its weight pointers are not used); n_layers 1..4096. */
int katali_hip_moe_stack_create(const KataliHipMoe *shape, int32_t n_sel, int32_t normed, float eps,
                                const KataliHipMoeStackLayer *layers, int32_t n_layers, void **stack);
/* plain: x_dev is layer 0's input (delta_dev NULL); normed: the residual
 * stream and the optional delta of layer 0's residual step. */
int katali_hip_moe_stack_run(void *stack, const float *x_dev, const float *delta_dev, float scale);
int katali_hip_moe_stack_destroy(void *stack);

/* The one-launch layers (the XCD-sliced layer, its normed form and the
 * stack), whose workgroups wait for each other: mode 0 turns them off (every
 * layer then runs as kernels A and B, as after an expired wait), 1 turns
 * them back on (after an expiry, once the device is no longer shared), -1
 * only asks. Returns the state before the call: 1 on, 0 off. The
 * environment switch KATALI_HIP_XCD=0 still applies on top. No counterpart
 * in the reference. */
int katali_hip_one_launch(int32_t mode);

/* How the one-launch layers hand a slot's h values between the workgroups
 * of that slot, which the dispatcher places on one XCD: 1 inside the XCD
 * (the words stay in its L2), 0 written through to memory as the
 * cross-XCD exchanges are. Mode 1 takes effect only where the library's
 * start-up check found every launch of 256 workgroups dealt to the eight
 * XCDs round robin (b % 8 classes each on one XCD); mode 0 sets it off, -1
 * only asks. Both give the same bits. Returns the state before the call. No
 * counterpart in the reference. */
int katali_hip_xcd_handoff(int32_t mode);

/* KATALI_HIP_OK when katali_hip_moe_layer (n_tokens 0) or katali_hip_moe_batch
 * (n_tokens 1..64 tokens) runs a layer of this descriptor's shape with n_sel
 * routed experts; else the code and last-error message the call would give.
 * Reads only the descriptor's types, sizes and which shared-expert pointers
 * are set; needs no device. Beyond the type and size rules (Q4_K gate/up, Q4_K
 * or Q6_K down, hidden in {256, 512, 1024, 2048, 4096}, ffn % 256 == 0 and
 * <= 16384, n_sel <= min(16, n_expert)), every workgroup must fit gfx950's
 * 160 KiB of LDS (KATALI_HIP_E_UNSUPPORTED otherwise):
 *   layer: n_slots * ffn * 11/8 + 2116 <= 163840, n_slots = n_sel + (shared
 *          expert), i.e. n_slots * ffn <= 117617 (17 slots: ffn <= 6912;
 *          9 slots: ffn <= 13056; up to 7 slots: every ffn);
 *   batch: 8 * ffn * 11/8 <= 163840, i.e. ffn <= 14848.
 * No counterpart in the reference (its CPU engine has no such limit): for a
 * caller that decides before offloading a layer. */
int katali_hip_moe_check(const KataliHipMoe *moe, int32_t n_sel, uint32_t n_tokens);

/* katali_hip_moe_layer without any allocation, for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. Same
 * arguments; it chooses the same kernels as katali_hip_moe_layer (the
 * one-launch layer where that entry takes it, under the same environment
 * switches), so its results are bit-identical to it. Its routing hand-off,
 * q8_1 h blocks and the one-launch layer's exchange words live in a fixed
 * static device array of the library (one per GPU, about 590 KB, held until
 * the process ends): n_slots * ffn/32 * 36 bytes of h must fit 135168
 * (n_slots = n_sel + 1 with a shared expert), else KATALI_HIP_E_INVALID;
 * every shape that passes katali_hip_moe_check's LDS rule needs at most
 * 132192. The library must be initialised first (katali_hip_probe); calls
 * that overlap on one GPU share the array and race. */
int katali_hip_moe_layer_noalloc(const KataliHipMoe *moe, const KataliHipMoeRoute *route,
                                 const float *x_dev, const void *xq8_dev, float *y_dev);

/* Debug variant: also writes gate/up outputs gu_dev[n_slots][2][ffn] (fp32) and
 * the quantized SiLU-GLU output hq8_dev[n_slots][ffn/32][36] (slot n_sel is the
 * shared expert). */
int katali_hip_moe_layer_debug(const KataliHipMoe *moe, const KataliHipMoeRoute *route,
                               const float *x_dev, const void *xq8_dev, float *y_dev,
                               float *gu_dev, void *hq8_dev);

/* ---- MoE layer over a batch of tokens (batched prefill) ---------- */
/* The batched counterpart of the reference's CPU matmul (katali_ggml_matmul_role,
 * V/src/gguf_dtype.c:1059-1105, each weight row decoded once for B tokens):
 * T tokens with their own experts. Pairs are grouped by expert on the device;
 * an expert with at least mfma_min_tokens pairs runs as an int8 MFMA grouped
 * GEMM, the others through the grouped v_dot4 GEMV kernels (one read of the
 * expert's weights for up to 8 of its tokens); results are identical in
 * definition (q8_1 x and h, rank-order weighted sum), and a one-token batch
 * is bit-identical to katali_hip_moe_layer with the same experts. */
typedef struct KataliHipMoeBatch {
    uint32_t struct_size;                  /* sizeof(KataliHipMoeBatch) */
    uint32_t n_tokens;                     /* T, 1..64 */
    int32_t n_sel;                         /* routed experts per token, 0..16 */
    uint32_t mfma_min_tokens;              /* grouped-GEMM threshold; 0 = 16 */
    const int32_t *ids;                    /* device [T][n_sel] */
    const float *weights;                  /* device [T][n_sel] */
} KataliHipMoeBatch;

/* y[T][hidden] = the MoE layer of each of the T fp32 rows x[T][hidden].
 * From 96 (token, slot) pairs on, the grouped-GEMM part runs on a second,
 * library-owned stream forked from the library stream and joined back
 * before the call's last kernel, so work queued after the call (or a graph
 * captured around it) still sees the whole layer finished in order. */
/* Device routing for a batch (prefill): ids/weights [n_tokens][n_sel] from
 * router logits [n_tokens][n_expert], each row routed exactly as
 * katali_hip_moe_layer routes one token from its logits (top n_sel, larger
 * logit first, lower index on ties, NaN as -inf; softmax over the selected,
 * renormalised), ready for KataliHipMoeBatch.ids / .weights. No reference
 * signature: the engine's router for a prompt is its CPU softmax and top-k
 * per token (V/src/gguf_kernels.c:63-80). 1 <= n_tokens <= 65535,
 * n_expert <= 512, 1 <= n_sel <= min(16, n_expert). */
int katali_hip_moe_route_batch(const float *logits_dev, uint32_t n_tokens, uint32_t n_expert, int32_t n_sel,
                               int32_t *ids_dev, float *weights_dev);
int katali_hip_moe_batch(const KataliHipMoe *moe, const KataliHipMoeBatch *batch, const float *x_dev,
                         float *y_dev);

/* Advance a device step index: *step = (*step + 1) % n_steps (one tiny launch). */
int katali_hip_step_advance(int32_t *step_dev, int32_t n_steps);

/* ---- per-token graphs (hipGraph capture of the library stream) ------------ */
/* Library scratch (the MoE layer's routing hand-off and h, the batched
 * layer's rows, about 39 MB, argmax partials) is allocated once at its largest
 * size by the first call that needs it, outside any capture (that first call
 * inside a capture returns KATALI_HIP_E_INVALID), and never moves or is freed,
 * so a captured graph stays valid whatever calls follow it. Graphs replay on
 * the library stream and share that scratch: replays and eager calls run in
 * stream order, never side by side. During a capture, katali_hip_malloc,
 * upload, download, sync, memset and set_stream return KATALI_HIP_E_INVALID
 * (each would end or corrupt the capture). katali_hip_free during a capture
 * releases nothing then: the buffer belongs to the graph made from that
 * capture (its replays may use it) and is freed by katali_hip_graph_destroy,
 * or at once if katali_hip_graph_end makes no graph. */
int katali_hip_graph_begin(void);
int katali_hip_graph_end(void **graph);
int katali_hip_graph_launch(void *graph);
int katali_hip_graph_destroy(void *graph);

/* ---- timing (HIP events on the library stream) ---------------------------- */
int katali_hip_event_create(void **event);
int katali_hip_event_record(void *event);
/* Waits for `end`, then *ms = elapsed between the two records. */
int katali_hip_event_elapsed(void *start, void *end, float *ms);
int katali_hip_event_destroy(void *event);

/* ---- pipelined uploads (the expert tier's miss path) ------------------------
 * The closed backend's upload batching and VRAM pool switches
 * (KATALI_UPLOAD_BATCH, KATALI_VRAM_POOL, README.md:260,329-330, whose
 * implementation is not in the reference) are replaced by a stager: a pinned
 * host ring of n_chunks chunks of chunk_bytes and a copy stream of its own.
 * katali_hip_stager_upload copies host bytes into the ring a chunk at a time
 * (the CPU copy of one chunk overlaps the DMA of the one before; a chunk is
 * reused once its DMA is done) and queues the DMAs on the copy stream; it
 * returns once the host bytes are copied out (the source may change), not
 * when they have arrived. katali_hip_stager_mark records a point in the
 * library stream's work (every kernel queued so far) and returns its number
 * (1, 2, ...); an upload naming mark m (0: none) starts its DMAs only after
 * the library stream has reached m, so it may overwrite memory that work
 * before m reads, and overlaps everything queued after m.
 * katali_hip_stager_fence makes the library stream wait for every DMA
 * queued so far (no host wait): kernels queued after it see the bytes.
 * The CPU copy of a chunk is split over the calling thread and
 * KATALI_HIP_STAGER_THREADS - 1 worker threads (default 4 in all; pieces of
 * at least 256 KiB). chunk_bytes 4 KiB .. 1 GiB, n_chunks 2 .. 64. One
 * calling thread per stager;
 * every call fails with KATALI_HIP_E_INVALID during a graph capture. No
 * counterpart in the reference's own sources. */
int katali_hip_stager_create(uint64_t chunk_bytes, uint32_t n_chunks, void **stager);
int katali_hip_stager_destroy(void *stager);
int katali_hip_stager_mark(void *stager, uint64_t *mark);
int katali_hip_stager_upload(void *stager, void *dev, const void *host, uint64_t bytes, uint64_t after_mark);
int katali_hip_stager_fence(void *stager);

/* ---- measurement ------------------------------------------------------------- */
/* The phase stamps of the one-launch layers: [64][256][16] uint64
 * s_memrealtime ticks (100 MHz), layer slot tag % 64, workgroup, phase (the
 * phases listed at kq_stamps in kq_moe.hip). Only the measurement build
 * records them (libkatali_hip_stamps.so, `build.py --stamps`); the product
 * library returns KATALI_HIP_E_UNSUPPORTED. Waits for queued work first.
 * No counterpart in the reference. */
int katali_hip_phase_stamps(void *host, size_t bytes);
/* The floors a MoE layer is measured against: the same bytes streamed with
 * no arithmetic in the layer's launch shape (256 workgroups of 1024
 * threads, each reading a contiguous 1/256 share with 16-byte loads):
 * kind 0 one launch reading a; kind 1 a then b in two launches (kernels A
 * and B's split); kind 2 a then b in one launch with the XCD-sliced layer's
 * two in-kernel waits (the 32 workgroups of an XCD after a, the 8 sharing
 * output rows after b; needs a 256-CU device). Sizes are multiples of 16.
 * sync: a device buffer of 4096 bytes, zeroed once by the caller and kept
 * for every later call (generation words). No counterpart in the
 * reference. */
int katali_hip_stream_floor(int32_t kind, const void *a, size_t a_bytes, const void *b, size_t b_bytes,
                            void *sync);
/* The exchange probe: the latency of the one-launch layers' word hand-offs
 * with nothing else running. 256 single-wave workgroups; workgroup b and its
 * partner p pass one tagged 64-bit word back and forth `rounds` times (1 ..
 * 2^20; a round is two one-way hand-offs), each waiting for the other's
 * word before sending its own: kind 0 p = b ^ 8 (one XCD) through that XCD's
 * L2 (written through where the dispatch check failed), kind 1 p = b ^ 8
 * written through, kind 2 p = b ^ 1 (another XCD) written through. words: a
 * device buffer of 4 * 1025 bytes, zeroed once by the caller and kept for
 * every later call: [256] generations, [256] 64-bit words, [256] each
 * workgroup's XCC id in the last call, [1] error bits (bit 0: a wait ran out
 * of polls). Time it with events around the call. No counterpart in the
 * reference. */
int katali_hip_exchange_probe(int32_t kind, uint32_t rounds, void *words);

/* ---- self-test and synthetic data for the harnesses ------------------------ */
/* cuda-dp4a-selftest equivalent (README.md:17): a synthetic Q4_K and Q6_K
 * GEMV whose activation is exactly representable in q8_1, dotted by the fp32
 * and the v_dot4 kernels; report gets rel_L2 lines. 0 when both agree to 1e-5. */
int katali_hip_selftest(char *report, size_t cap);
/* Fill nblocks Q4_K/Q6_K blocks: uniform random bytes, then d (and dmin)
 * |N(0, d_sigma)| as f16. Deterministic in seed. */
int katali_hip_synth_fill(uint32_t type, void *dev, uint64_t nblocks, uint64_t seed, float d_sigma);
/* n values of N(0, sigma). */
int katali_hip_synth_normal(float *dev, uint64_t n, uint64_t seed, float sigma);
/* Streaming device copy (bandwidth / counter calibration), bytes % 16 == 0. */
int katali_hip_copy(void *dst_dev, const void *src_dev, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* KATALI_HIP_H */
