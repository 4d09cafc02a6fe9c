/* katali_hip_cpu.c — CPU evaluation of Q4_K / Q6_K / q8_1 for the harness's
 * GPU-versus-CPU checks (declarations in katali_hip_cpu.h). Straightforward
 * scalar code from the public GGUF block layouts:
 *   Q4_K (144 B / 256 values): f16 d, f16 dmin, 12 bytes of 6-bit sub-block
 *        scales and mins, 128 bytes of 4-bit quants; sub-block j of 32
 *        values is d*sc_j*q - dmin*m_j, sub-blocks 2g and 2g+1 in the low and
 *        high nibbles of bytes 32g..32g+31;
 *   Q6_K (210 B / 256 values): 128 bytes of low 4 bits, 64 bytes of high 2
 *        bits, 16 int8 scales (one per 16 values), f16 d; value = d*sc*(q-32);
 *   q8_1 (36 B / 32 values): f16 d, f16 s, 32 int8 q; value = d*q. */
#include "katali_hip_cpu.h"

#include <math.h>
#include <string.h>

float kh_cpu_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 0) {
        const float v = ldexpf((float)m, -24);   /* zero or subnormal */
        return sign ? -v : v;
    }
    const uint32_t bits = e == 31 ? sign | 0x7F800000u | (m << 13) : sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t kh_cpu_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u);   /* inf, nan */
    if (ax >= 0x477FF000u) return sign | 0x7C00u;                                       /* >= 65520 */
    if (ax < 0x38800000u) {   /* below 2^-14: a multiple of 2^-24, rounded to even */
        float v;
        memcpy(&v, &ax, 4);
        return (uint16_t)(sign | (uint16_t)lrintf(v * 16777216.0f));
    }
    uint32_t h = ((ax >> 23) - 112u) << 10 | ((ax >> 13) & 1023u);
    const uint32_t rest = ax & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;   /* a carry moves into the exponent */
    return (uint16_t)(sign | h);
}

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | p[1] << 8); }

static void q4k_scale_min(const uint8_t *s, int j, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | (s[j - 4] >> 6) << 4;
        *m = (s[j + 4] >> 4) | (s[j] >> 6) << 4;
    }
}

static void q4k_block(const uint8_t *b, float *y) {
    const float d = kh_cpu_half_to_float(le16(b)), dmin = kh_cpu_half_to_float(le16(b + 2));
    const uint8_t *q = b + 16;
    for (int j = 0; j < 8; j++) {
        int sc, m;
        q4k_scale_min(b + 4, j, &sc, &m);
        const float a = d * (float)sc, c = dmin * (float)m;
        const uint8_t *qb = q + 32 * (j / 2);
        for (int i = 0; i < 32; i++) {
            const int v = j & 1 ? qb[i] >> 4 : qb[i] & 15;
            y[32 * j + i] = a * (float)v - c;
        }
    }
}

static void q6k_block(const uint8_t *b, float *y) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    const float d = kh_cpu_half_to_float(le16(b + 208));
    for (int half = 0; half < 2; half++) {
        const uint8_t *l = ql + 64 * half, *h = qh + 32 * half;
        const int8_t *s = sc + 8 * half;
        float *o = y + 128 * half;
        for (int i = 0; i < 32; i++) {
            const int t = i / 16;
            o[i] = d * s[t] * (float)(((l[i] & 15) | ((h[i] >> 0) & 3) << 4) - 32);
            o[i + 32] = d * s[t + 2] * (float)(((l[i + 32] & 15) | ((h[i] >> 2) & 3) << 4) - 32);
            o[i + 64] = d * s[t + 4] * (float)(((l[i] >> 4) | ((h[i] >> 4) & 3) << 4) - 32);
            o[i + 96] = d * s[t + 6] * (float)(((l[i + 32] >> 4) | ((h[i] >> 6) & 3) << 4) - 32);
        }
    }
}

int kh_cpu_dequant(uint32_t type, const void *blocks, uint64_t n, float *out) {
    const uint8_t *b = (const uint8_t *)blocks;
    if (type == 12 && n % 256 == 0) {
        for (uint64_t k = 0; k < n / 256; k++) q4k_block(b + 144 * k, out + 256 * k);
        return 0;
    }
    if (type == 14 && n % 256 == 0) {
        for (uint64_t k = 0; k < n / 256; k++) q6k_block(b + 210 * k, out + 256 * k);
        return 0;
    }
    if (type == 9 && n % 32 == 0) {
        for (uint64_t k = 0; k < n / 32; k++) {
            const float d = kh_cpu_half_to_float(le16(b + 36 * k));
            for (int i = 0; i < 32; i++) out[32 * k + i] = d * (float)(int8_t)b[36 * k + 4 + i];
        }
        return 0;
    }
    return -1;
}

int kh_cpu_matvec(uint32_t type, const void *w, uint64_t rows, uint64_t cols, const float *x, double *y) {
    const uint64_t row_bytes = cols / 256 * (type == 12 ? 144 : 210);
    float row[32768];
    if (cols > 32768 || (type != 12 && type != 14)) return -1;
    for (uint64_t r = 0; r < rows; r++) {
        if (kh_cpu_dequant(type, (const uint8_t *)w + r * row_bytes, cols, row)) return -1;
        double acc = 0.0;
        for (uint64_t c = 0; c < cols; c++) acc += (double)row[c] * (double)x[c];
        y[r] = acc;
    }
    return 0;
}

void kh_cpu_quantize_q8_1(const float *x, uint64_t n, void *out) {
    uint8_t *o = (uint8_t *)out;
    for (uint64_t k = 0; k < n / 32; k++, x += 32, o += 36) {
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
        const float d = amax / 127.0f, inv = d != 0.0f ? 1.0f / d : 0.0f;
        int sum = 0;
        for (int i = 0; i < 32; i++) {
            const int q = (int)roundf(x[i] * inv);
            o[4 + i] = (uint8_t)(int8_t)q;
            sum += q;
        }
        const uint16_t hd = kh_cpu_float_to_half(d), hs = kh_cpu_float_to_half((float)sum * d);
        o[0] = (uint8_t)hd;
        o[1] = (uint8_t)(hd >> 8);
        o[2] = (uint8_t)hs;
        o[3] = (uint8_t)(hs >> 8);
    }
}

static float sum_pairwise(const float *t, uint64_t n) {
    if (n == 1) return t[0];
    uint64_t h = 1;
    while (2 * h < n) h *= 2;
    return sum_pairwise(t, h) + sum_pairwise(t + h, n - h);
}

float kh_cpu_dot_q4k_q8(const void *row, const void *q8, uint64_t nb) {
    float terms[8 * 128];
    if (nb == 0 || nb > 128) return NAN;
    const uint8_t *w = (const uint8_t *)row, *x = (const uint8_t *)q8;
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + 144 * b;
        const float d = kh_cpu_half_to_float(le16(blk)), dmin = kh_cpu_half_to_float(le16(blk + 2));
        for (int j = 0; j < 8; j++) {
            const uint8_t *xb = x + 36 * (8 * b + j), *qb = blk + 16 + 32 * (j / 2);
            int isum = 0, xsum = 0;
            for (int i = 0; i < 32; i++) {
                const int q8v = (int8_t)xb[4 + i];
                isum += (j & 1 ? qb[i] >> 4 : qb[i] & 15) * q8v;
                xsum += q8v;
            }
            int sc, m;
            q4k_scale_min(blk + 4, j, &sc, &m);
            const float d8 = kh_cpu_half_to_float(le16(xb));
            const float a = (d * (float)sc) * d8, c = (dmin * (float)m) * d8;
            terms[8 * b + (uint64_t)j] = fmaf(a, (float)isum, -(c * (float)xsum));
        }
    }
    return sum_pairwise(terms, 8 * nb);
}

static float lib_expf(float x) {
    x = fminf(fmaxf(x, -80.0f), 88.0f);
    const float n = rintf(x * 1.44269502f);
    float r = fmaf(-n, 0.693145752f, x);
    r = fmaf(-n, 1.42860677e-06f, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const uint32_t bits = (uint32_t)((int)n + 127) << 23;
    float two_n;
    memcpy(&two_n, &bits, 4);
    return p * two_n;
}

float kh_cpu_silu_mul(float g, float u) {
    const float den = 1.0f + lib_expf(-g);
    return g / den * u;
}
