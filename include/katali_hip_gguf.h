/* katali_hip_gguf.h — GGUF tensors onto the MI355X: a bounds-checked reader,
 * a device weight cache keyed by tensor with a VRAM budget, MoE layer
 * descriptors assembled from the GGUF tensor names, and the expert VRAM tier
 * (per-expert device slots, least recently used first out).
 *
 * Host C, part of libkatali_hip_loader.so (device memory through the
 * katali_gpu_* loader calls). The reader follows the public GGUF container
 * format with the acceptance rules of the engine's own reader
 * (V/src/gguf_reader.c:351-543; V = vendor/katali_gguf_dense): the same files
 * open, the same files are refused, and the tensor table (name, dims, type,
 * offset, bytes, data position) is the same. The on-disk tensor layout is the
 * layout the kernels read ("the on-disk format is the wire format"): expert
 * stacks ffn_{gate,up,down}_exps upload as they are.
 */
#ifndef KATALI_HIP_GGUF_H
#define KATALI_HIP_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "katali_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct KataliHipGguf KataliHipGguf;   /* an open file (read-only map) */

typedef struct KataliHipGgufTensor {
    const char *name;        /* NUL-terminated, owned by the file handle */
    uint32_t n_dims;         /* 1..4 */
    uint64_t dims[4];        /* dims[0] contiguous (GGUF order) */
    uint32_t type;           /* ggml type id */
    uint64_t offset;         /* relative to the data section */
    uint64_t nbytes;         /* 0 for a type without a known block size */
    const uint8_t *data;     /* NULL when nbytes == 0 */
} KataliHipGgufTensor;

/* Open and validate (katali_gguf_open semantics, V/src/gguf_reader.c:351-543):
 * magic, version 1..3, header counts, metadata (nested arrays refused),
 * general.alignment (8..2^20, else 32), tensor ranks 1..4 with non-zero dims,
 * data section and every sized tensor inside the file. 0 = OK, -1 with a
 * reason in err. */
int katali_hip_gguf_open(const char *path, KataliHipGguf **out, char *err, size_t err_cap);
void katali_hip_gguf_close(KataliHipGguf *g);

/* Reason for the last -1 / NULL of this module (single caller thread). */
const char *katali_hip_gguf_last_error(void);

uint32_t katali_hip_gguf_version(const KataliHipGguf *g);
uint64_t katali_hip_gguf_tensor_count(const KataliHipGguf *g);
uint64_t katali_hip_gguf_alignment(const KataliHipGguf *g);
uint64_t katali_hip_gguf_data_offset(const KataliHipGguf *g);
const uint8_t *katali_hip_gguf_base(const KataliHipGguf *g);   /* start of the mapped file */
int katali_hip_gguf_tensor(const KataliHipGguf *g, uint64_t i, KataliHipGgufTensor *out);  /* 0 / -1 */
int katali_hip_gguf_find(const KataliHipGguf *g, const char *name, KataliHipGgufTensor *out); /* 0 / -1 */
/* Scalar metadata (katali_gguf_get_int / _float / _str, V/include/katali_gguf.h:127-137). */
int64_t katali_hip_gguf_get_int(const KataliHipGguf *g, const char *key, int64_t def);
double katali_hip_gguf_get_float(const KataliHipGguf *g, const char *key, double def);
const char *katali_hip_gguf_get_str(const KataliHipGguf *g, const char *key, size_t *len_out);  /* NULL if absent */
/* Bytes of n elements of a ggml type (katali_ggml_row_bytes, V/src/gguf_dtype.c:216-223);
 * 0 for an unknown type or n not a multiple of the block. */
uint64_t katali_hip_ggml_row_bytes(uint32_t type, uint64_t n);

/* ---- device weight cache keyed by tensor ------------------------------ */
/* Replaces the CUDA shim's weight cache (V/src/katali_dense_cuda.c:36-44),
 * keyed by tensor name, whole tensors, uploaded on first use. budget_bytes
 * caps the device bytes held; 0 reads KATALI_VRAM_GB (GiB; unset = no cap).
 * A tensor that would pass the cap is refused (NULL, reason in
 * katali_hip_gguf_last_error): the cache never evicts what a captured graph
 * may still read. */
typedef struct KataliHipWeights KataliHipWeights;
int katali_hip_weights_create(const KataliHipGguf *g, uint64_t budget_bytes, KataliHipWeights **out);
void katali_hip_weights_destroy(KataliHipWeights *w);
const void *katali_hip_weights_get(KataliHipWeights *w, const char *name);
uint64_t katali_hip_weights_resident_bytes(const KataliHipWeights *w);

/* One MoE layer from the GGUF tensor names (blk.<layer>.ffn_gate_exps.weight,
 * _up_exps, _down_exps, optional _gate_shexp/_up_shexp/_down_shexp,
 * ffn_gate_inp.weight (F32 router [n_expert][hidden]) and ffn_norm.weight),
 * uploaded through the cache: fills moe, *router (may be NULL) and *norm_w
 * (may be NULL). 0 = OK, -1 when a tensor is missing, its shape or type does
 * not fit the fused layer, or the budget refuses it. */
int katali_hip_gguf_moe_layer(KataliHipWeights *w, uint32_t layer, KataliHipMoe *moe, const float **router,
                              const float **norm_w);

/* ---- expert VRAM tier ---------------------------------------------------
 * For host-routed layers (expert ids known on the host, as the engine's CPU
 * router gives them): device pools of n_slots expert slots each for gate,
 * up and down, least recently used slot out, uploads from the mapped file on
 * a miss. katali_hip_tier_layer maps the layer's n_sel experts to slots and
 * fills moe so that the slot numbers are the expert ids the fused layer reads
 * (KataliHipMoeRoute.ids), n_expert being the pool size. The experts of one
 * call all stay resident (n_sel <= n_slots). budget_bytes: as above (0:
 * KATALI_VRAM_GB, unset = room for max_slots); the slot count is the budget
 * divided by one expert's gate + up + down bytes, at most max_slots (<= 512).
 * Slots hold one expert shape; layers of another shape are refused. A
 * call's slots are valid for work queued on the library stream before the
 * next call (which may refill any slot that call does not ask for).
 *
 * katali_hip_tier_pipeline turns on pipelined uploads (also at create when
 * KATALI_UPLOAD_BATCH=1): a miss's bytes go through a stager (pinned ring of
 * n_chunks x chunk_bytes, 0 = 4 x 4 MiB, and a copy stream; katali_hip.h),
 * the call returns once the bytes are copied out of the file, and the work
 * queued after it waits for the DMAs on the device, not on the host. An
 * upload into a slot waits only for the work that can read the slot's old
 * expert (queued before the call after that expert's last call), so it
 * overlaps every later kernel. Synchronous otherwise: each miss is copied
 * and waited for before the call returns. */
typedef struct KataliHipExpertTier KataliHipExpertTier;
typedef struct KataliHipTierStats {
    uint64_t hits, misses, uploaded_bytes;
    uint32_t n_slots;
} KataliHipTierStats;
int katali_hip_tier_create(const KataliHipGguf *g, uint32_t layer_for_shape, uint64_t budget_bytes,
                           uint32_t max_slots, KataliHipExpertTier **out);
void katali_hip_tier_destroy(KataliHipExpertTier *t);
int katali_hip_tier_layer(KataliHipExpertTier *t, uint32_t layer, const int32_t *expert_ids, int n_sel,
                          int32_t *slot_ids_out, KataliHipMoe *moe);
void katali_hip_tier_stats(const KataliHipExpertTier *t, KataliHipTierStats *out);
int katali_hip_tier_pipeline(KataliHipExpertTier *t, uint64_t chunk_bytes, uint32_t n_chunks);

#ifdef __cplusplus
}
#endif
#endif /* KATALI_HIP_GGUF_H */
