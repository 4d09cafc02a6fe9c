/* katali_hip_cpu.h — CPU evaluation of the quantized formats for the
 * katali-hip harness (check, check-moe), which compares the GPU with the CPU
 * the way the engine's cuda-check / cuda-check-moe do (README.md:13,99-102).
 * Written from the public GGUF block layouts; used by the harness only, never
 * by the library's compute path. */
#ifndef KATALI_HIP_CPU_H
#define KATALI_HIP_CPU_H

#include <stddef.h>
#include <stdint.h>

float    kh_cpu_half_to_float(uint16_t h);
uint16_t kh_cpu_float_to_half(float f);   /* round to nearest, ties to even */

/* n values of `type` (Q4_K 12, Q6_K 14: n % 256 == 0; Q8_1 9: n % 32 == 0)
 * dequantized to fp32. Returns 0, or -1 for another type or n. */
int kh_cpu_dequant(uint32_t type, const void *blocks, uint64_t n, float *out);

/* y[r] = sum_c W[r][c] * x[c] in double over the dequantized rows. */
int kh_cpu_matvec(uint32_t type, const void *w, uint64_t rows, uint64_t cols, const float *x, double *y);

/* q8_1 blocks of n values (n % 32 == 0): per 32 values d = max|x| / 127,
 * q = round(x * (1/d)), s = d * sum(q), d and s stored as f16 (ggml's q8_1). */
void kh_cpu_quantize_q8_1(const float *x, uint64_t n, void *out);

/* The library's q8_1-path Q4_K row dot (nb blocks of 256): per 32-value
 * sub-block j the fp32 term fmaf((d*sc_j)*d8_j, isum_j, -(((dmin*m_j)*d8_j)*
 * xsum_j)), isum_j / xsum_j the exact integer sums of q4*q8 and q8, and the
 * 8*nb terms summed pairwise (a run splits at the largest power of two below
 * its length). The GPU kernels form the same fp32 operations in this order,
 * so the result is bit-identical to theirs. */
float kh_cpu_dot_q4k_q8(const void *row, const void *q8, uint64_t nb);
/* SiLU(g) * u as the library forms it: g / (1 + e^-g) * u with e^x by
 * Cody-Waite reduction and a degree-7 Taylor polynomial (the engine's
 * exp256_ps, V/src/gguf_simd_x86.c:744-761), every step one fp32 rounding. */
float kh_cpu_silu_mul(float g, float u);

#endif
