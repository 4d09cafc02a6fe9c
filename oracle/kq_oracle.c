/* kq_oracle — CPU restatement of katali-lab's quantized expert-GEMV numerics.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle, never the product). See kq_oracle.h
 * for what each function restates or defines. Build with -ffp-contract=off: the
 * only fused multiply-adds are the explicit fmaf() calls, placed exactly where
 * the reference uses _mm256_fmadd_ps.
 */
#include "kq_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

uint64_t kqo_row_bytes(uint32_t type, uint64_t n) {
    switch (type) {
        case KQO_F32:  return n * 4u;
        case KQO_Q8_1: return n % 32u ? 0 : n / 32u * KQO_Q81_BYTES;
        case KQO_Q4_K: return n % KQO_QK_K ? 0 : n / KQO_QK_K * KQO_Q4K_BYTES;
        case KQO_Q6_K: return n % KQO_QK_K ? 0 : n / KQO_QK_K * KQO_Q6K_BYTES;
        default: return 0;
    }
}

/* ======================================================================== *
 * f16 — V/include/katali_gguf_fp.h:14-57                                    *
 * ======================================================================== */
float kqo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u;
    uint32_t m = h & 1023u;
    if (e == 31u) return u2f(sign | 0x7F800000u | (m << 13));
    if (e != 0u) return u2f(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0u) return u2f(sign);
    /* subnormal: shift the leading one up to bit 10, lowering the exponent */
    uint32_t exp32 = 113u;
    while (!(m & 1024u)) { m <<= 1; exp32--; }
    return u2f(sign | (exp32 << 23) | ((m & 1023u) << 13));
}

uint16_t kqo_f32_to_f16_ref(float v) {
    const uint32_t b = f2u(v);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const int e = (int)((b >> 23) & 255u) - 112;   /* rebias 127 -> 15 */
    uint32_t m = b & 0x7FFFFFu;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e > 0) {
        uint16_t h = (uint16_t)(sign | ((uint32_t)e << 10) | (m >> 13));
        return (uint16_t)(h + ((m >> 12) & 1u));   /* first dropped bit rounds up */
    }
    if (e < -10) return sign;
    m |= 0x800000u;
    const int sh = 14 - e;
    const uint16_t sub = (uint16_t)(m >> sh);
    return (uint16_t)(sign | (uint16_t)(sub + ((m >> (sh - 1)) & 1u)));
}

uint16_t kqo_f32_to_f16_rne(float v) {
    const uint32_t b = f2u(v);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const uint32_t a = b & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);          /* NaN */
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);         /* >= 65520: inf */
    if (a >= 0x38800000u) {                                          /* f16 normal */
        uint32_t h = ((((a >> 23) - 112u) << 10) | ((a >> 13) & 1023u));
        const uint32_t rem = a & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (a < 0x33000000u) return sign;                                 /* < 2^-25 */
    /* f16 subnormal: value = k * 2^-24 */
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    const int sh = 126 - (int)(a >> 23);
    uint32_t k = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (k & 1u))) k++;
    return (uint16_t)(sign | k);
}

/* ======================================================================== *
 * Decoders                                                                  *
 * ======================================================================== */
/* get_scale_min_k4 (V/src/gguf_dtype.c:350-358): the 12-byte field packs eight
 * 6-bit scales and eight 6-bit mins; entries 4..7 keep their top two bits in
 * the spare high bits of bytes 0..7. */
void kqo_q4k_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = (uint8_t)(q[j] & 63u);
        *m = (uint8_t)(q[j + 4] & 63u);
    } else {
        *sc = (uint8_t)((q[j + 4] & 15u) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Q4_K element e of a super-block: group g = e/64 owns qs[32g..32g+31]; the
 * low nibbles hold elements 64g..64g+31 (sub-block 2g), the high nibbles
 * 64g+32..64g+63 (sub-block 2g+1). */
static inline int q4k_val(const uint8_t *blk, int e) {
    const uint8_t byte = blk[16 + 32 * (e / 64) + (e % 32)];
    return (e % 64) < 32 ? (byte & 15) : (byte >> 4);
}

/* Q6_K element e: half n = e/128, quarter k = (e%128)/32, lane l = e%32.
 * Low four bits come from ql[64n + l + 32(k&1)] (low nibble for k<2, high for
 * k>=2); the top two bits are bits 2k..2k+1 of qh[32n + l]. */
static inline int q6k_val(const uint8_t *blk, int e) {
    const int n = e / 128, k = (e % 128) / 32, l = e % 32;
    const uint8_t lb = blk[64 * n + l + 32 * (k & 1)];
    const int lo = k < 2 ? (lb & 15) : (lb >> 4);
    const int hi = (blk[128 + 32 * n + l] >> (2 * k)) & 3;
    return lo | (hi << 4);
}

/* V/src/gguf_dtype.c:429-452 */
void kqo_dequant_q4_K(const uint8_t *src, uint64_t nb, float *out) {
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * KQO_Q4K_BYTES;
        const float d = kqo_f16_to_f32(rd16(blk)), dmin = kqo_f16_to_f32(rd16(blk + 2));
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            kqo_q4k_scale_min(j, blk + 4, &sc, &m);
            const float ds = d * (float)sc, dm = dmin * (float)m;
            for (int i = 0; i < 32; i++)
                out[b * 256 + 32 * j + i] = ds * (float)q4k_val(blk, 32 * j + i) - dm;
        }
    }
}

/* V/src/gguf_dtype.c:487-512: w = d * sc[e/16] * (q6 - 32); note the product
 * order (d * sc) * q is the reference's. */
void kqo_dequant_q6_K(const uint8_t *src, uint64_t nb, float *out) {
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * KQO_Q6K_BYTES;
        const float d = kqo_f16_to_f32(rd16(blk + 208));
        const int8_t *sc = (const int8_t *)(blk + 192);
        for (int e = 0; e < 256; e++)
            out[b * 256 + e] = d * (float)sc[e / 16] * (float)(q6k_val(blk, e) - 32);
    }
}

/* V/src/gguf_dtype.c:328-335 (the s field is not used by decoding) */
void kqo_dequant_q8_1(const uint8_t *src, uint64_t nb, float *out) {
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = src + b * KQO_Q81_BYTES;
        const float d = kqo_f16_to_f32(rd16(blk));
        for (int i = 0; i < 32; i++) out[b * 32 + i] = d * (float)(int8_t)blk[4 + i];
    }
}

int kqo_dequant(uint32_t type, const void *src, uint64_t n, float *out) {
    const uint8_t *s = (const uint8_t *)src;
    switch (type) {
        case KQO_Q4_K: if (n % 256) return -1; kqo_dequant_q4_K(s, n / 256, out); return 0;
        case KQO_Q6_K: if (n % 256) return -1; kqo_dequant_q6_K(s, n / 256, out); return 0;
        case KQO_Q8_1: if (n % 32) return -1; kqo_dequant_q8_1(s, n / 32, out); return 0;
        case KQO_F32: memcpy(out, s, n * 4); return 0;
        default: return -1;
    }
}

/* ======================================================================== *
 * Reference float dots                                                      *
 * ======================================================================== */
/* V/src/gguf_dtype.c:544-559 */
float kqo_vec_dot_ref(uint32_t type, const void *row, const float *x, uint64_t n) {
    const uint64_t bs = type == KQO_Q8_1 ? 32 : 256;
    const uint64_t bb = kqo_row_bytes(type, bs);
    if (!bb || n % bs) return 0.0f;
    float tmp[256];
    double acc = 0.0;
    for (uint64_t b = 0; b < n / bs; b++) {
        kqo_dequant(type, (const uint8_t *)row + b * bb, bs, tmp);
        for (uint64_t i = 0; i < bs; i++) acc += (double)tmp[i] * (double)x[b * bs + i];
    }
    return (float)acc;
}

/* V/src/gguf_dtype.c:594-624 */
float kqo_dot_q4_K_scalar(const uint8_t *row, const float *x, uint64_t nb) {
    double acc = 0.0;
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * KQO_Q4K_BYTES;
        const float d = kqo_f16_to_f32(rd16(blk)), dmin = kqo_f16_to_f32(rd16(blk + 2));
        const float *xb = x + b * 256;
        for (int g = 0; g < 4; g++) {
            uint8_t s0, m0, s1, m1;
            kqo_q4k_scale_min(2 * g, blk + 4, &s0, &m0);
            kqo_q4k_scale_min(2 * g + 1, blk + 4, &s1, &m1);
            const float d1 = d * s0, mv1 = dmin * m0, d2 = d * s1, mv2 = dmin * m1;
            double qx1 = 0.0, qx2 = 0.0, sx1 = 0.0, sx2 = 0.0;
            for (int l = 0; l < 32; l++) {
                const uint8_t byte = blk[16 + 32 * g + l];
                qx1 += (double)(byte & 15) * (double)xb[64 * g + l];
                sx1 += (double)xb[64 * g + l];
                qx2 += (double)(byte >> 4) * (double)xb[64 * g + 32 + l];
                sx2 += (double)xb[64 * g + 32 + l];
            }
            acc += (double)d1 * qx1 - (double)mv1 * sx1;
            acc += (double)d2 * qx2 - (double)mv2 * sx2;
        }
    }
    return (float)acc;
}

/* hsum256_ps (V/src/gguf_simd_x86.c:77-86): fold the upper four lanes onto the
 * lower four, then (t0 + t1) + (t2 + t3). */
static inline float hsum8(const float v[8]) {
    const float t0 = v[0] + v[4], t1 = v[1] + v[5], t2 = v[2] + v[6], t3 = v[3] + v[7];
    return (t0 + t1) + (t2 + t3);
}

/* V/src/gguf_simd_x86.c:307-347. Per group of 64 outputs, lane i of the 8-lane
 * accumulators sees elements 8k+i (k = 0..3) of each 32-value half; the group's
 * scale and negated min are folded in with two fused multiply-adds per half.
 * The hoisted-sum (:397-436) and dual-row (:447-506) kernels compute the same
 * lane sums in the same order, so this one function matches all three. */
float kqo_dot_q4_K_avx2order(const uint8_t *row, const float *x, uint64_t nb) {
    double acc = 0.0;
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * KQO_Q4K_BYTES;
        const float d = kqo_f16_to_f32(rd16(blk)), dmin = kqo_f16_to_f32(rd16(blk + 2));
        const uint8_t *qs = blk + 16;
        const float *xb = x + b * 256;
        float accL[8] = {0}, accH[8] = {0};
        for (int g = 0; g < 4; g++) {
            uint8_t s0, m0, s1, m1;
            kqo_q4k_scale_min(2 * g, blk + 4, &s0, &m0);
            kqo_q4k_scale_min(2 * g + 1, blk + 4, &s1, &m1);
            float aL[8] = {0}, aH[8] = {0}, xL[8] = {0}, xH[8] = {0};
            for (int k = 0; k < 4; k++) {
                for (int i = 0; i < 8; i++) {
                    const uint8_t byte = qs[32 * g + 8 * k + i];
                    const float xl = xb[64 * g + 8 * k + i], xh = xb[64 * g + 32 + 8 * k + i];
                    aL[i] = fmaf((float)(byte & 15), xl, aL[i]);
                    aH[i] = fmaf((float)(byte >> 4), xh, aH[i]);
                    xL[i] = xL[i] + xl;
                    xH[i] = xH[i] + xh;
                }
            }
            const float c0 = d * (float)s0, n0 = -(dmin * (float)m0);
            const float c1 = d * (float)s1, n1 = -(dmin * (float)m1);
            for (int i = 0; i < 8; i++) {
                accL[i] = fmaf(c0, aL[i], accL[i]);
                accL[i] = fmaf(n0, xL[i], accL[i]);
                accH[i] = fmaf(c1, aH[i], accH[i]);
                accH[i] = fmaf(n1, xH[i], accH[i]);
            }
        }
        acc += (double)(hsum8(accL) + hsum8(accH));
    }
    return (float)acc;
}

/* V/src/gguf_simd_x86.c:566-629. Per half (128 outputs) and per 16-lane chunk
 * c, four signed 6-bit vectors are rebuilt from ql/qh; each is dotted with its
 * 16 activations as two 8-lane fused multiply-adds starting from zero, then
 * scaled by d*sc into one of four block accumulators. */
float kqo_dot_q6_K_avx2order(const uint8_t *row, const float *x, uint64_t nb) {
    double acc = 0.0;
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * KQO_Q6K_BYTES;
        const int8_t *sc = (const int8_t *)(blk + 192);
        const float d = kqo_f16_to_f32(rd16(blk + 208));
        const float *xb = x + b * 256;
        float A[4][8] = {{0}};
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
            const int8_t *scn = sc + 8 * h;
            const float *xn = xb + 128 * h;
            for (int c = 0; c < 2; c++) {
                int8_t q[4][16];
                for (int i = 0; i < 16; i++) {
                    const uint8_t a = ql[16 * c + i], bq = ql[32 + 16 * c + i], hb = qh[16 * c + i];
                    q[0][i] = (int8_t)(((a & 15) | ((hb & 3) << 4)) - 32);
                    q[1][i] = (int8_t)(((bq & 15) | (((hb >> 2) & 3) << 4)) - 32);
                    q[2][i] = (int8_t)(((a >> 4) | (((hb >> 4) & 3) << 4)) - 32);
                    q[3][i] = (int8_t)(((bq >> 4) | (((hb >> 6) & 3) << 4)) - 32);
                }
                const float *xp = xn + 16 * c;
                for (int t = 0; t < 4; t++) {
                    float a[8];
                    for (int i = 0; i < 8; i++) a[i] = fmaf((float)q[t][i], xp[32 * t + i], 0.0f);
                    for (int i = 0; i < 8; i++) a[i] = fmaf((float)q[t][8 + i], xp[32 * t + 8 + i], a[i]);
                    const float s = d * (float)scn[c + 2 * t];
                    for (int i = 0; i < 8; i++) A[t][i] = fmaf(s, a[i], A[t][i]);
                }
            }
        }
        acc += (double)(hsum8(A[0]) + hsum8(A[1]) + hsum8(A[2]) + hsum8(A[3]));
    }
    return (float)acc;
}

float kqo_dot_f32_avx2order(const float *w, const float *x, uint64_t n) {
    float a[16] = {0};
    uint64_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; j++) a[j] = fmaf(w[i + j], x[i + j], a[j]);
    float v[8], l[4];
    for (int k = 0; k < 8; k++) v[k] = a[k] + a[k + 8];
    for (int k = 0; k < 4; k++) l[k] = v[k] + v[k + 4];
    const float acc = (l[0] + l[1]) + (l[2] + l[3]);
    double tail = 0.0;
    for (; i < n; i++) tail += (double)w[i] * (double)x[i];
    return acc + (float)tail;
}

int kqo_matvec_f32x(uint32_t type, const void *w, uint64_t rows, uint64_t cols,
                    const float *x, float *y) {
    if (type == KQO_F32) {
        for (uint64_t r = 0; r < rows; r++) y[r] = kqo_dot_f32_avx2order((const float *)w + r * cols, x, cols);
        return 0;
    }
    const uint64_t rb = kqo_row_bytes(type, cols);
    if (!rb || (type != KQO_Q4_K && type != KQO_Q6_K)) return -1;
    const uint8_t *wb = (const uint8_t *)w;
    for (uint64_t r = 0; r < rows; r++)
        y[r] = type == KQO_Q4_K ? kqo_dot_q4_K_avx2order(wb + r * rb, x, cols / 256)
                                : kqo_dot_q6_K_avx2order(wb + r * rb, x, cols / 256);
    return 0;
}

/* Row-parallel form of kqo_matvec_f32x for the CPU baseline when the compiled
 * reference is unavailable: contiguous row ranges per thread, the calling
 * thread taking the first (V/src/gguf_dtype.c:731-752). */
typedef struct MvJob {
    uint32_t type; const uint8_t *w; uint64_t rb, cols, r0, r1; const float *x; float *y;
} MvJob;

static void *mv_run(void *arg) {
    const MvJob *j = (const MvJob *)arg;
    for (uint64_t r = j->r0; r < j->r1; r++)
        j->y[r] = j->type == KQO_Q4_K ? kqo_dot_q4_K_avx2order(j->w + r * j->rb, j->x, j->cols / 256)
                                      : kqo_dot_q6_K_avx2order(j->w + r * j->rb, j->x, j->cols / 256);
    return NULL;
}

int kqo_matvec_f32x_mt(uint32_t type, const void *w, uint64_t rows, uint64_t cols,
                       const float *x, float *y, int n_threads) {
    const uint64_t rb = kqo_row_bytes(type, cols);
    if (!rb || (type != KQO_Q4_K && type != KQO_Q6_K)) return -1;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    MvJob jobs[256];
    pthread_t th[256];
    const uint64_t per = (rows + (uint64_t)n_threads - 1) / (uint64_t)n_threads;
    for (int t = 0; t < n_threads; t++) {
        uint64_t r0 = per * (uint64_t)t, r1 = r0 + per;
        if (r0 > rows) r0 = rows;
        if (r1 > rows) r1 = rows;
        jobs[t] = (MvJob){ type, (const uint8_t *)w, rb, cols, r0, r1, x, y };
    }
    int started = 0;
    for (int t = 1; t < n_threads; t++) {
        if (pthread_create(&th[t], NULL, mv_run, &jobs[t]) != 0) break;
        started = t;
    }
    mv_run(&jobs[0]);
    for (int t = 1; t <= started; t++) pthread_join(th[t], NULL);
    for (int t = started + 1; t < n_threads; t++) mv_run(&jobs[t]);
    return 0;
}

/* ======================================================================== *
 * q8_1 quantization and integer block dots                                  *
 * ======================================================================== */
int kqo_quantize_q8_1(const float *x, uint64_t n, uint8_t *out) {
    if (n % 32) return -1;
    for (uint64_t b = 0; b < n / 32; b++) {
        const float *xb = x + 32 * b;
        uint8_t *blk = out + KQO_Q81_BYTES * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xb[i]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        int sum = 0;
        for (int i = 0; i < 32; i++) {
            const int q = (int)roundf(xb[i] * id);
            blk[4 + i] = (uint8_t)(int8_t)q;
            sum += q;
        }
        const uint16_t hd = kqo_f32_to_f16_rne(d), hs = kqo_f32_to_f16_rne((float)sum * d);
        blk[0] = (uint8_t)hd; blk[1] = (uint8_t)(hd >> 8);
        blk[2] = (uint8_t)hs; blk[3] = (uint8_t)(hs >> 8);
    }
    return 0;
}

static inline int q8_val(const uint8_t *q8, uint64_t e) {
    return (int8_t)q8[(e / 32) * KQO_Q81_BYTES + 4 + (e % 32)];
}
static inline float q8_d(const uint8_t *q8, uint64_t blk) {
    return kqo_f16_to_f32(rd16(q8 + blk * KQO_Q81_BYTES));
}
static int q8_qsum(const uint8_t *q8, uint64_t blk) {
    int s = 0;
    for (int i = 0; i < 32; i++) s += (int8_t)q8[blk * KQO_Q81_BYTES + 4 + i];
    return s;
}

int kqo_q4K_q8_isums(const uint8_t *row, const uint8_t *q8, uint64_t nb, int32_t *isums) {
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * KQO_Q4K_BYTES;
        for (int j = 0; j < 8; j++) {
            int32_t s = 0;
            for (int i = 0; i < 32; i++)
                s += q4k_val(blk, 32 * j + i) * q8_val(q8, 256 * b + 32 * j + i);
            isums[8 * b + j] = s;
        }
    }
    return 0;
}

int kqo_q6K_q8_isums(const uint8_t *row, const uint8_t *q8, uint64_t nb, int32_t *isums) {
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * KQO_Q6K_BYTES;
        for (int t = 0; t < 16; t++) {
            int32_t s = 0;
            for (int i = 0; i < 16; i++)
                s += (q6k_val(blk, 16 * t + i) - 32) * q8_val(q8, 256 * b + 16 * t + i);
            isums[16 * b + t] = s;
        }
    }
    return 0;
}

float kqo_dot_q4K_q8_f64(const uint8_t *row, const uint8_t *q8, uint64_t nb) {
    double acc = 0.0;
    int32_t is[8];
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * KQO_Q4K_BYTES;
        const float d = kqo_f16_to_f32(rd16(blk)), dmin = kqo_f16_to_f32(rd16(blk + 2));
        kqo_q4K_q8_isums(blk, q8 + 8 * b * KQO_Q81_BYTES, 1, is);
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            kqo_q4k_scale_min(j, blk + 4, &sc, &m);
            const double d8 = (double)q8_d(q8, 8 * b + j);
            acc += (double)(d * (float)sc) * d8 * (double)is[j]
                 - (double)(dmin * (float)m) * d8 * (double)q8_qsum(q8, 8 * b + j);
        }
    }
    return (float)acc;
}

float kqo_q4K_q8_term(const uint8_t *blk, int j, const uint8_t *q8blk) {
    int32_t isum = 0;
    for (int i = 0; i < 32; i++) isum += q4k_val(blk, 32 * j + i) * (int8_t)q8blk[4 + i];
    uint8_t sc, m;
    kqo_q4k_scale_min(j, blk + 4, &sc, &m);
    const float d = kqo_f16_to_f32(rd16(blk)), dmin = kqo_f16_to_f32(rd16(blk + 2));
    const float d8 = kqo_f16_to_f32(rd16(q8blk));
    const float A = (d * (float)sc) * d8;
    const float B = (dmin * (float)m) * d8;
    const float X = (float)q8_qsum(q8blk, 0);
    return fmaf(A, (float)isum, -(B * X));
}

/* Pairwise sum of t[0..n): halves split at the largest power of two below n
 * (the exact halves when n is a power of two), each half summed the same
 * way, then left + right. */
static float pairwise_sum(const float *t, uint64_t n) {
    if (n == 1) return t[0];
    uint64_t h = 1;
    while (2 * h < n) h *= 2;
    return pairwise_sum(t, h) + pairwise_sum(t + h, n - h);
}

float kqo_dot_q4K_q8(const uint8_t *row, const uint8_t *q8, uint64_t nb) {
    float t[8 * 128];
    if (nb == 0 || nb > 128) return NAN;
    for (uint64_t b = 0; b < nb; b++)
        for (int j = 0; j < 8; j++)
            t[8 * b + j] = kqo_q4K_q8_term(row + b * KQO_Q4K_BYTES, j, q8 + (8 * b + j) * KQO_Q81_BYTES);
    return pairwise_sum(t, 8 * nb);
}

float kqo_dot_q6K_q8(const uint8_t *row, const uint8_t *q8, uint64_t nb) {
    double acc = 0.0;
    int32_t is[16];
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * KQO_Q6K_BYTES;
        const float d = kqo_f16_to_f32(rd16(blk + 208));
        const int8_t *sc = (const int8_t *)(blk + 192);
        kqo_q6K_q8_isums(blk, q8 + 8 * b * KQO_Q81_BYTES, 1, is);
        for (int t = 0; t < 16; t++)
            acc += (double)(d * (float)sc[t]) * (double)q8_d(q8, 8 * b + t / 2) * (double)is[t];
    }
    return (float)acc;
}

int kqo_matvec_q8(uint32_t type, const void *w, uint64_t rows, uint64_t cols,
                  const uint8_t *q8, float *y) {
    const uint64_t rb = kqo_row_bytes(type, cols);
    if (!rb || (type != KQO_Q4_K && type != KQO_Q6_K)) return -1;
    const uint8_t *wb = (const uint8_t *)w;
    for (uint64_t r = 0; r < rows; r++)
        y[r] = type == KQO_Q4_K ? kqo_dot_q4K_q8(wb + r * rb, q8, cols / 256)
                                : kqo_dot_q6K_q8(wb + r * rb, q8, cols / 256);
    return 0;
}

/* ======================================================================== *
 * Activation and router                                                     *
 * ======================================================================== */
float kqo_expf(float x) {
    x = fminf(fmaxf(x, -80.0f), 88.0f);
    const float n = rintf(x * 1.44269502f);               /* round(x / ln2) */
    float r = fmaf(-n, 0.693145752f, x);                   /* ln2 high part (exact n*hi) */
    r = fmaf(-n, 1.42860677e-06f, r);                      /* ln2 low part */
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return p * u2f((uint32_t)((int)n + 127) << 23);
}

float kqo_silu_mul(float g, float u) {
    const float e = kqo_expf(-g);
    const float den = 1.0f + e;
    const float s = g / den;
    return s * u;
}

/* exp256_ps (V/src/gguf_simd_x86.c:744-761), one lane: 2^t with t = x*log2e
 * split into an integer n (nearest) and r in [-0.5, 0.5], 2^r by the
 * reference's degree-6 polynomial. */
float kqo_exp_ref_poly(float x) {
    x = fminf(x, 88.0f);
    x = fmaxf(x, -88.0f);
    const float t = x * 1.44269504088896341f;
    const float n = rintf(t);
    const float r = t - n;
    float p = 0.00015403530393381608f;
    p = fmaf(p, r, 0.0013333558146428443f);
    p = fmaf(p, r, 0.009618129107628477f);
    p = fmaf(p, r, 0.05550410866482158f);
    p = fmaf(p, r, 0.2402265069591007f);
    p = fmaf(p, r, 0.6931471805599453f);
    p = fmaf(p, r, 1.0f);
    return p * u2f((uint32_t)((int)n + 127) << 23);
}

/* silu_mul_avx2 (V/src/gguf_simd_x86.c:763-773); the scalar tail uses libm. */
void kqo_silu_mul_ref(float *gate, const float *up, uint64_t n) {
    const uint64_t nv = n / 8 * 8;
    for (uint64_t i = 0; i < nv; i++) {
        const float g = gate[i];
        const float e = kqo_exp_ref_poly(0.0f - g);
        gate[i] = (g / (1.0f + e)) * up[i];
    }
    for (uint64_t i = nv; i < n; i++) gate[i] = (gate[i] / (1.0f + expf(-gate[i]))) * up[i];
}

int kqo_router_topk(const float *logits_in, int n_expert, int k, int32_t *ids, float *w) {
    if (k <= 0 || k > n_expert || k > 64) return -1;
    unsigned char taken[4096];
    float logits[4096];
    if (n_expert > 4096) return -1;
    memset(taken, 0, (size_t)n_expert);
    /* a NaN logit ranks, and weighs, as -inf */
    for (int e = 0; e < n_expert; e++) logits[e] = logits_in[e] != logits_in[e] ? -INFINITY : logits_in[e];
    for (int r = 0; r < k; r++) {
        int best = -1;
        for (int e = 0; e < n_expert; e++)
            if (!taken[e] && (best < 0 || logits[e] > logits[best])) best = e;
        taken[best] = 1;
        ids[r] = best;
    }
    const float lmax = logits[ids[0]];
    float e[64], sum = 0.0f;
    for (int r = 0; r < k; r++) { e[r] = kqo_expf(logits[ids[r]] - lmax); sum += e[r]; }
    for (int r = 0; r < k; r++) w[r] = e[r] / sum;
    return 0;
}

/* Greedy sampling (V/src/gguf_sampler.c:62-66): best = 0, bv = -FLT_MAX,
 * take i when logits[i] > bv, i ascending. */
int kqo_argmax_greedy(const float *logits, int n) {
    if (!logits || n <= 0) return -1;
    int best = 0;
    float bv = -FLT_MAX;
    for (int i = 0; i < n; i++)
        if (logits[i] > bv) { bv = logits[i]; best = i; }
    return best;
}

void kqo_rmsnorm(const float *x, const float *w, uint64_t n, float eps, float *out) {
    double sumsq = 0.0;
    for (uint64_t i = 0; i < n; i++) sumsq += (double)x[i] * (double)x[i];
    const float inv = 1.0f / sqrtf((float)(sumsq / (double)n) + eps);
    for (uint64_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

void kqo_add_rmsnorm(float *x, const float *delta, float scale, const float *w, uint64_t n, float eps, float *out) {
    for (uint64_t i = 0; i < n; i++) x[i] = scale == 1.0f ? x[i] + delta[i] : x[i] + scale * delta[i];
    kqo_rmsnorm(x, w, n, eps, out);
}

/* ======================================================================== *
 * MoE layer                                                                 *
 * ======================================================================== */
typedef struct Slot { const uint8_t *g, *u, *d; uint64_t ffn; float w; } Slot;

static int moe_slots(const KqoMoe *m, int n_sel, const int32_t *ids, const float *w, Slot *s) {
    const uint64_t rg = kqo_row_bytes(m->gate_type, m->hidden);
    const uint64_t ru = kqo_row_bytes(m->up_type, m->hidden);
    const uint64_t rd = kqo_row_bytes(m->down_type, m->ffn);
    if (!rg || !ru || !rd) return -1;
    for (int r = 0; r < n_sel; r++) {
        if (ids[r] < 0 || (uint32_t)ids[r] >= m->n_expert) return -1;
        const uint64_t e = (uint64_t)ids[r];
        s[r].g = m->gate_exps + e * m->ffn * rg;
        s[r].u = m->up_exps + e * m->ffn * ru;
        s[r].d = m->down_exps + e * m->hidden * rd;
        s[r].ffn = m->ffn;
        s[r].w = w[r];
    }
    int n = n_sel;
    if (m->gate_sh && m->shared_ffn) {
        s[n].g = m->gate_sh; s[n].u = m->up_sh; s[n].d = m->down_sh;
        s[n].ffn = m->shared_ffn; s[n].w = 1.0f;
        n++;
    }
    return n;
}

int kqo_moe_layer_q8(const KqoMoe *m, const float *x, int n_sel,
                     const int32_t *ids, const float *w, float *y,
                     float *g_out, float *u_out, uint8_t *hq8_out) {
    Slot s[65];
    if (n_sel < 0 || n_sel > 64) return -1;
    const int n = moe_slots(m, n_sel, ids, w, s);
    if (n < 0) return -1;
    uint64_t fmax = m->ffn > m->shared_ffn ? m->ffn : m->shared_ffn;
    uint8_t *xq = malloc(m->hidden / 32 * KQO_Q81_BYTES);
    float *g = malloc(fmax * 4), *u = malloc(fmax * 4), *h = malloc(fmax * 4), *yd = malloc(m->hidden * 4);
    uint8_t *hq = malloc(fmax / 32 * KQO_Q81_BYTES);
    if (!xq || !g || !u || !h || !yd || !hq) { free(xq); free(g); free(u); free(h); free(yd); free(hq); return -1; }
    kqo_quantize_q8_1(x, m->hidden, xq);
    for (uint64_t i = 0; i < m->hidden; i++) y[i] = 0.0f;
    for (int r = 0; r < n; r++) {
        const uint64_t f = s[r].ffn;
        kqo_matvec_q8(m->gate_type, s[r].g, f, m->hidden, xq, g);
        kqo_matvec_q8(m->up_type, s[r].u, f, m->hidden, xq, u);
        for (uint64_t i = 0; i < f; i++) h[i] = kqo_silu_mul(g[i], u[i]);
        kqo_quantize_q8_1(h, f, hq);
        kqo_matvec_q8(m->down_type, s[r].d, m->hidden, f, hq, yd);
        for (uint64_t i = 0; i < m->hidden; i++) y[i] = fmaf(s[r].w, yd[i], y[i]);
        if (g_out) memcpy(g_out + (uint64_t)r * m->ffn, g, f * 4);
        if (u_out) memcpy(u_out + (uint64_t)r * m->ffn, u, f * 4);
        if (hq8_out) memcpy(hq8_out + (uint64_t)r * (m->ffn / 32) * KQO_Q81_BYTES, hq, f / 32 * KQO_Q81_BYTES);
    }
    free(xq); free(g); free(u); free(h); free(yd); free(hq);
    return 0;
}

int kqo_moe_down_q8(const KqoMoe *m, int n_sel, const int32_t *ids, const float *w,
                    const uint8_t *hq8, float *y) {
    Slot s[65];
    if (n_sel < 0 || n_sel > 64) return -1;
    const int n = moe_slots(m, n_sel, ids, w, s);
    if (n < 0) return -1;
    float *yd = malloc(m->hidden * 4);
    if (!yd) return -1;
    for (uint64_t i = 0; i < m->hidden; i++) y[i] = 0.0f;
    for (int r = 0; r < n; r++) {
        kqo_matvec_q8(m->down_type, s[r].d, m->hidden, s[r].ffn,
                      hq8 + (uint64_t)r * (m->ffn / 32) * KQO_Q81_BYTES, yd);
        for (uint64_t i = 0; i < m->hidden; i++) y[i] = fmaf(s[r].w, yd[i], y[i]);
    }
    free(yd);
    return 0;
}

int kqo_moe_layer_f32(const KqoMoe *m, const float *x, int n_sel,
                      const int32_t *ids, const float *w, float *y) {
    Slot s[65];
    if (n_sel < 0 || n_sel > 64) return -1;
    const int n = moe_slots(m, n_sel, ids, w, s);
    if (n < 0) return -1;
    uint64_t fmax = m->ffn > m->shared_ffn ? m->ffn : m->shared_ffn;
    float *g = malloc(fmax * 4), *u = malloc(fmax * 4), *yd = malloc(m->hidden * 4);
    if (!g || !u || !yd) { free(g); free(u); free(yd); return -1; }
    for (uint64_t i = 0; i < m->hidden; i++) y[i] = 0.0f;
    for (int r = 0; r < n; r++) {
        const uint64_t f = s[r].ffn;
        kqo_matvec_f32x(m->gate_type, s[r].g, f, m->hidden, x, g);
        kqo_matvec_f32x(m->up_type, s[r].u, f, m->hidden, x, u);
        kqo_silu_mul_ref(g, u, f);
        kqo_matvec_f32x(m->down_type, s[r].d, m->hidden, f, g, yd);
        for (uint64_t i = 0; i < m->hidden; i++) y[i] = fmaf(s[r].w, yd[i], y[i]);
    }
    free(g); free(u); free(yd);
    return 0;
}
