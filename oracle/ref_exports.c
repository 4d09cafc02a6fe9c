/* Exported wrappers around the reference's header-only f16 helpers
 * (V/include/katali_gguf_fp.h:14-57) and its greedy sampler, linked into
 * oracle/_ref/libkatali_ref.so so tests can compare the oracle's
 * restatements with them. Test infrastructure only. */
#include <stdint.h>
#include <string.h>
#include "katali_gguf.h"
#include "katali_gguf_fp.h"
#include "katali_gguf_sampler.h"

uint16_t kref_f32_to_f16(float v) { return katali_f32_to_f16(v); }
float kref_f16_to_f32(uint16_t h) { return katali_f16_to_f32(h); }

/* katali_gguf_sample with a freshly initialised sampler: temperature 0, the
 * greedy branch (V/src/gguf_sampler.c:9-17,62-66). */
int kref_sample_greedy(const float *logits, int n) {
    KataliGgufSampler s;
    katali_gguf_sampler_init(&s);
    const int r = katali_gguf_sample(&s, logits, n, 0, 0);
    katali_gguf_sampler_free(&s);
    return r;
}

/* The reference reader's verdict and tensor table for a file
 * (katali_gguf_open, V/src/gguf_reader.c:351-543), flattened: returns -1 when
 * it refuses the file, else the tensor count, with up to cap entries of name
 * (63 chars + NUL each), n_dims, dims[4], type, offset, nbytes and the data
 * position from the start of the file (-1 for no data); also version,
 * alignment and the data section offset. */
int64_t kref_gguf_table(const char *path, int64_t cap, char *names, uint32_t *n_dims, uint64_t *dims,
                        uint32_t *types, uint64_t *offsets, uint64_t *nbytes, int64_t *data_pos,
                        uint64_t *hdr /* version, alignment, data_offset */) {
    KataliGgufFile f;
    char err[256];
    if (katali_gguf_open(&f, path, 1, err, sizeof err) != 0) return -1;
    hdr[0] = f.version;
    hdr[1] = f.alignment;
    hdr[2] = f.data_offset;
    const int64_t n = (int64_t)f.tensor_count;
    for (int64_t i = 0; i < n && i < cap; i++) {
        const KataliGgufTensor *t = &f.tensors[i];
        strncpy(names + 64 * i, t->name, 63);
        names[64 * i + 63] = 0;
        n_dims[i] = t->n_dims;
        for (int d = 0; d < 4; d++) dims[4 * i + d] = t->dims[d];
        types[i] = t->type;
        offsets[i] = t->offset;
        nbytes[i] = t->nbytes;
        data_pos[i] = t->data ? (int64_t)(t->data - f.map) : -1;
    }
    katali_gguf_close(&f);
    return n;
}
