/* Exported wrappers around the reference's header-only f16 helpers
 * (V/include/katali_gguf_fp.h:14-57) and its greedy sampler, linked into
 * oracle/_ref/libkatali_ref.so so tests can compare the oracle's
 * restatements with them. Test infrastructure only. */
#include <stdint.h>
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
