/* kq_oracle — CPU restatement of katali-lab's quantized expert-GEMV numerics.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle for libkatali_hip: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product path (libkatali_hip, the host loader, the CLI) never links it and
 * never falls back to it.
 *
 * Two families of functions live here:
 *
 *  1. Restatements of code that exists in the reference (vendor/katali_gguf_dense):
 *     f16 conversion, Q4_K / Q6_K / Q8_1 decoding, the double-accumulated
 *     reference dot, the scalar Q4_K dot, and the AVX2 float dots restated lane
 *     by lane (8-lane accumulators, fused multiply-adds, the same horizontal
 *     sum), so that their fp32 results are bit-identical to the reference's.
 *     Pinned against oracle/_ref (the reference compiled from its own sources)
 *     and the fixtures under tests/golden/.
 *
 *  2. Definitions of the GPU path, whose reference implementation exists only
 *     as a closed binary (README.md:13,17): the q8_1 activation quantizer (the
 *     public ggml block_q8_1: d = amax/127, q = round(x/d), s = d*sum(q)),
 *     the integer Q4_K x q8_1 and Q6_K x q8_1 block dots, SiLU with a
 *     Cody-Waite exp, the top-k router and the MoE layer composition. Pinned by
 *     closed forms, brute force and invariants in tests/test_oracle_*.py.
 *
 * Every function cites the reference file:line it follows, relative to
 * vendor/katali_gguf_dense/ ("V/").
 */
#ifndef KQ_ORACLE_H
#define KQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids used on this path (V/include/katali_gguf_dtype.h:18-39). */
#define KQO_F32  0u
#define KQO_Q8_1 9u
#define KQO_Q4_K 12u
#define KQO_Q6_K 14u

#define KQO_QK_K 256u      /* elements per K-quant super-block */
#define KQO_Q4K_BYTES 144u /* V/src/gguf_dtype.c:169 */
#define KQO_Q6K_BYTES 210u /* V/src/gguf_dtype.c:171 */
#define KQO_Q81_BYTES 36u  /* V/src/gguf_dtype.c:166 */

uint64_t kqo_row_bytes(uint32_t type, uint64_t n);

/* ---- f16 (V/include/katali_gguf_fp.h:14-57) ---------------------------- */
float    kqo_f16_to_f32(uint16_t h);
/* The reference's encoder: truncate, then add one ulp when the first dropped
 * bit is set (round half up on the magnitude, not ties-to-even). */
uint16_t kqo_f32_to_f16_ref(float v);
/* IEEE round-to-nearest-even; what the q8_1 quantizer stores. */
uint16_t kqo_f32_to_f16_rne(float v);

/* ---- reference decoders ------------------------------------------------- */
void kqo_dequant_q4_K(const uint8_t *src, uint64_t nb, float *out); /* gguf_dtype.c:429-452 */
void kqo_dequant_q6_K(const uint8_t *src, uint64_t nb, float *out); /* gguf_dtype.c:487-512 */
void kqo_dequant_q8_1(const uint8_t *src, uint64_t nb, float *out); /* gguf_dtype.c:328-335 */
int  kqo_dequant(uint32_t type, const void *src, uint64_t n, float *out);
/* get_scale_min_k4, gguf_dtype.c:350-358 */
void kqo_q4k_scale_min(int j, const uint8_t *scales12, uint8_t *sc, uint8_t *m);

/* ---- reference float dots ---------------------------------------------- */
/* gguf_dtype.c:544-559: decode each block, accumulate w*x in double. */
float kqo_vec_dot_ref(uint32_t type, const void *row, const float *x, uint64_t n);
/* gguf_dtype.c:594-624: scalar Q4_K, per-sub-block d1*sum(q*x) - m1*sum(x). */
float kqo_dot_q4_K_scalar(const uint8_t *row, const float *x, uint64_t nb);
/* gguf_simd_x86.c:307-347 (and the bit-identical hoisted/dual-row forms at
 * :380-506): the AVX2 fast path restated with explicit 8-lane arrays. */
float kqo_dot_q4_K_avx2order(const uint8_t *row, const float *x, uint64_t nb);
/* gguf_simd_x86.c:566-629 */
float kqo_dot_q6_K_avx2order(const uint8_t *row, const float *x, uint64_t nb);
/* gguf_simd_x86.c:111-122 with hsum256_ps (:80-89): 16 fp32 fma chains
 * (chain j over columns j, j+16, ... of the first n & ~15), chains j and j+8
 * added, then ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)); the columns past that
 * summed in double and added as float. The F32 row loop (rows_f32, :674-682). */
float kqo_dot_f32_avx2order(const float *w, const float *x, uint64_t n);
/* The reference fp32 matvec row loop (gguf_dtype.c:731-856 ->
 * gguf_simd_x86.c:699-736, 865-893): y[r] = fast dot of row r. Rows are
 * independent, so the result does not depend on the thread partition.
 * Types Q4_K, Q6_K and F32 (row stride 4·cols). */
int kqo_matvec_f32x(uint32_t type, const void *w, uint64_t rows, uint64_t cols,
                    const float *x, float *y);
/* Same result, rows split over n_threads pthreads (contiguous ranges). */
int kqo_matvec_f32x_mt(uint32_t type, const void *w, uint64_t rows, uint64_t cols,
                       const float *x, float *y, int n_threads);

/* ---- q8_1 activation quantization (own definition of the GPU path) ----- */
/* Per 32 values: amax = max|x|; d = amax/127; id = d ? 1/d : 0;
 * q = roundf(x*id) (half away from zero); block.d = f16_rne(d);
 * block.s = f16_rne((float)sum(q) * d). n must be a multiple of 32. */
int kqo_quantize_q8_1(const float *x, uint64_t n, uint8_t *out);

/* ---- integer block dots (own definition; exact int32) -------------------- */
/* isums[8*b + j] = sum_{i<32} q4(b, j, i) * q8[32*(8b+j) + i]. */
int kqo_q4K_q8_isums(const uint8_t *row, const uint8_t *q8, uint64_t nb, int32_t *isums);
/* isums[16*b + t] = sum_{i<16} (q6(b, 16t+i) - 32) * q8[256b + 16t + i]. */
int kqo_q6K_q8_isums(const uint8_t *row, const uint8_t *q8, uint64_t nb, int32_t *isums);
/* The q8_1 path's Q4_K row dot (own definition, bit-identical on the GPU):
 * for each 32-value sub-block j (block b = j/8, sub-block j%8, with
 * (sc_j, m_j) from get_scale_min_k4 and d8_j the f16 scale of x's q8_1 block
 * j), in fp32 with one rounding per operation:
 *   A_j = (d * sc_j) * d8_j,  B_j = (dmin * m_j) * d8_j,
 *   t_j = fmaf(A_j, isum_j, -(B_j * xsum_j)),
 * isum_j the exact integer block sum above and xsum_j the exact sum of the 32
 * int8 values of x's block j; then the pairwise sum of t_0 .. t_{n-1}
 * (n = 8*nb): sum(t[0..n)) = sum(t[0..h)) + sum(t[h..n)), h the largest
 * power of two below n (n/2 for the row widths the GPU kernels take, all
 * powers of two). nb <= 128. */
float kqo_dot_q4K_q8(const uint8_t *row, const uint8_t *q8, uint64_t nb);
/* t_j of one block for sub-block j, with q8blk pointing at x's block j. */
float kqo_q4K_q8_term(const uint8_t *blk, int j, const uint8_t *q8blk);
/* The same terms' closed form in double (d*sc and dmin*m as fp32 products,
 * the rest exact-ish in double), for bounding kqo_dot_q4K_q8:
 *   sum_j (d*sc_j)*d8_j*isum_j - (dmin*m_j)*d8_j*xsum_j. */
float kqo_dot_q4K_q8_f64(const uint8_t *row, const uint8_t *q8, uint64_t nb);
/* Q6_K: sum_t (d*sc_t)*d8*isum_t accumulated in double (the down projection,
 * whose output is not quantized again). */
float kqo_dot_q6K_q8(const uint8_t *row, const uint8_t *q8, uint64_t nb);
int   kqo_matvec_q8(uint32_t type, const void *w, uint64_t rows, uint64_t cols,
                    const uint8_t *q8, float *y);

/* ---- activation and router ----------------------------------------------- */
/* exp by Cody-Waite reduction (x = n*ln2 + r, ln2 split in two constants) and
 * a degree-7 Taylor polynomial in r, Horner with fused multiply-adds; the
 * input is clamped to [-80, 88]. Bit-identical on the GPU by construction. */
float kqo_expf(float x);
/* silu(g)*u = g / (1 + exp(-g)) * u, in that operation order. */
float kqo_silu_mul(float g, float u);
/* The reference's vector exp and silu (gguf_simd_x86.c:744-773), restated. */
float kqo_exp_ref_poly(float x);
void  kqo_silu_mul_ref(float *gate, const float *up, uint64_t n);
/* Top-k by logit (descending; equal logits -> lower index first), weights
 * renormalised over the selection: w_i = e_i / sum_sel e_j, e_i =
 * kqo_expf(l_i - l_max), sum in rank order. Equal to softmax followed by
 * renormalisation over the top k. A NaN logit counts as -inf (rank and
 * weight); -0 and +0 are equal logits. */
int kqo_router_topk(const float *logits, int n_expert, int k, int32_t *ids, float *w);
/* Greedy argmax: first maximum wins, NaN never, 0 when nothing exceeds
 * -FLT_MAX (V/src/gguf_sampler.c:62-66). */
int kqo_argmax_greedy(const float *logits, int n);
/* RMSNorm (V/src/gguf_kernels.c:13-18): sumsq = sum x[i]^2 in double, in
 * index order; inv = 1/sqrtf((float)(sumsq/n) + eps); out[i] = x[i]*inv*w[i].
 * out may be x. */
void kqo_rmsnorm(const float *x, const float *w, uint64_t n, float eps, float *out);
/* The residual step before a norm (V/src/gguf_model.c:677-678): x[i] +=
 * delta[i] when scale == 1, else x[i] += scale*delta[i]; then kqo_rmsnorm. */
void kqo_add_rmsnorm(float *x, const float *delta, float scale, const float *w, uint64_t n, float eps, float *out);

/* ---- MoE layer (configs 1, 2, 4) ----------------------------------------- */
typedef struct KqoMoe {
    uint32_t gate_type, up_type, down_type;
    uint64_t hidden, ffn;
    uint32_t n_expert;
    const uint8_t *gate_exps, *up_exps, *down_exps; /* [n_expert][rows][row_bytes] */
    /* optional always-on shared expert (weight 1.0), NULL when absent */
    uint64_t shared_ffn;
    const uint8_t *gate_sh, *up_sh, *down_sh;
} KqoMoe;

/* q8_1 path, the GPU's definition: x -> q8_1; per selected expert: gate/up
 * q8 GEMVs, h = silu(g)*u, h -> q8_1, down q8 GEMV; y = sum_e w_e*y_e in rank
 * order (fmaf), then the shared expert with weight 1. Optional outputs
 * (may be NULL): g and u [n_slots][ffn], h_q8 [n_slots][ffn/32*36]. Slot
 * n_sel is the shared expert when present. */
int kqo_moe_layer_q8(const KqoMoe *m, const float *x, int n_sel,
                     const int32_t *ids, const float *w, float *y,
                     float *g_out, float *u_out, uint8_t *hq8_out);
/* Down stage only, from given h_q8 blocks (lets a test feed the GPU's h). */
int kqo_moe_down_q8(const KqoMoe *m, int n_sel, const int32_t *ids, const float *w,
                    const uint8_t *hq8, float *y);
/* fp32 CPU path: the reference's AVX2-order dots with float x, the
 * reference's silu (gguf_simd_x86.c:763-773), same weighted sum. */
int kqo_moe_layer_f32(const KqoMoe *m, const float *x, int n_sel,
                      const int32_t *ids, const float *w, float *y);

#ifdef __cplusplus
}
#endif
#endif
