/* Exported wrappers around the reference's header-only f16 helpers
 * (V/include/katali_gguf_fp.h:14-57), linked into oracle/_ref/libkatali_ref.so
 * so tests can compare the oracle's restatement with them over every input.
 * Test infrastructure only. */
#include <stdint.h>
#include "katali_gguf_fp.h"

uint16_t kref_f32_to_f16(float v) { return katali_f32_to_f16(v); }
float kref_f16_to_f32(uint16_t h) { return katali_f16_to_f32(h); }
