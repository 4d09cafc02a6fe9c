/* katali-hip — command-line harness over the engine-side loader.
 *
 * The GPU harness commands of the reference engine (README.md:13,17,21,99-102,
 * 149-171,309-312: cuda-info, cuda-check, cuda-check-moe, cuda-dp4a-selftest,
 * cuda-bench, cuda-bench-cold, gpu-matvec-bench) for libkatali_hip, on
 * synthetic tensors (no model file):
 *
 *   katali-hip info                  device and library status
 *   katali-hip dp4a-selftest         q8_1 v_dot4 GEMV vs the fp32 GEMV, q8-exact x
 *   katali-hip check                 both GEMV paths against the CPU on N(0,1) x
 *                                    at the engine's shapes (criteria printed)
 *   katali-hip check-moe             the fused MoE layer against the CPU's q8_1
 *                                    path (and, for information, its fp32 path)
 *   katali-hip matvec-bench [reps]   dense GEMV: event-timed us per call and GB/s
 *   katali-hip bench [tokens]        48-layer top-8 MoE decode (hidden 2048, 128
 *                                    experts, ffn 768), graph-replayed
 *   katali-hip bench-cold [tokens]   40 layers x 256 experts (ffn 512) + shared
 *                                    expert, routing rotated every token
 *   katali-hip gguf-info FILE        a GGUF file's header, metadata and tensor
 *                                    table (no GPU needed)
 *   katali-hip gguf-check FILE       every MoE layer of FILE on the device: routed
 *                                    by the file's own F32 router on N(0,1) x,
 *                                    the fused layer vs the same layer composed
 *                                    from separate library GEMVs
 *
 * Exit status 0 on success / PASS, 1 on a failed check, 2 when no usable GPU.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "katali_hip_cpu.h"
#include "katali_hip_gguf.h"
#include "katali_hip_loader.h"

#define Q4K KATALI_HIP_TYPE_Q4_K
#define Q6K KATALI_HIP_TYPE_Q6_K

static const KataliHipApi *api;

static int die(const char *what, int rc) {
    fprintf(stderr, "katali-hip: %s failed (%d): %s\n", what, rc, katali_gpu_last_error());
    return 1;
}
#define CK(call)                                 \
    do {                                         \
        int rc_ = (call);                        \
        if (rc_) return die(#call, rc_);         \
    } while (0)

static uint64_t row_bytes(uint32_t type, uint64_t cols) { return cols / 256 * (type == Q4K ? 144 : 210); }
static const char *tname(uint32_t t) { return t == Q4K ? "Q4_K" : "Q6_K"; }

static double rel_l2(const float *a, const float *b, size_t n, size_t *outside) {
    double num = 0, den = 0;
    size_t o = 0;
    for (size_t i = 0; i < n; i++) {
        const double d = (double)a[i] - b[i];
        num += d * d;
        den += (double)b[i] * b[i];
        if (fabs(d) > 1e-3 * (1.0 + fabs(b[i]))) o++;
    }
    if (outside) *outside = o;
    return den > 0 ? sqrt(num / den) : sqrt(num);
}

static float *dalloc_f(size_t n) {
    void *p = NULL;
    return api->malloc_(&p, n * 4) ? NULL : (float *)p;
}

static int cmd_info(void) {
    printf("library: %s\n", katali_gpu_status());
    printf("abi version: %d\n", api->abi_version());
    return 0;
}

static int cmd_selftest(void) {
    char rep[1024] = {0};
    const int rc = api->selftest(rep, sizeof rep);
    fputs(rep, stdout);
    if (rc) fprintf(stderr, "%s\n", katali_gpu_last_error());
    return rc ? 1 : 0;
}

struct shape {
    const char *role;
    uint32_t type;
    uint64_t rows, cols;
};
static const struct shape SHAPES[] = {
    {"dense 6144x2048", Q4K, 6144, 2048},        {"expert gate/up 768x2048", Q4K, 768, 2048},
    {"expert down 2048x768", Q6K, 2048, 768},    {"attn q/o 4096x4096", Q4K, 4096, 4096},
    {"attn v 1024x4096", Q6K, 1024, 4096},       {"ffn down 4096x12288", Q6K, 4096, 12288},
};
#define NSHAPES (sizeof SHAPES / sizeof SHAPES[0])

/* GPU against CPU (katali_hip_cpu.c) at each shape, on N(0,1) x. PASS needs
 * all three of:
 *   the fp32 GEMV: every element within 1e-3*(1+|cpu|) (the engine's bar,
 *     README.md:17) of the CPU's double-precision dot over the dequantized
 *     rows with the same fp32 x (the largest error over that bar is printed);
 *   the v_dot4 GEMV: rel_L2 <= 1e-5 against the CPU dot with the same q8_1 x;
 *   the device quantizer: q8_1 blocks of x identical to the CPU's.
 * The v_dot4 GEMV against the CPU with fp32 x (the q8_1 rounding of x, about
 * 1e-2 on N(0,1) activations) is printed for information only. */
static int cmd_check(void) {
    int fails = 0;
    for (size_t s = 0; s < NSHAPES; s++) {
        const struct shape *sh = &SHAPES[s];
        const uint64_t R = sh->rows, C = sh->cols, wb = R * row_bytes(sh->type, C);
        void *w = NULL, *xq = NULL;
        float *x = dalloc_f(C), *y0 = dalloc_f(R), *y1 = dalloc_f(R);
        if (!x || !y0 || !y1) return die("malloc", -5);
        CK(api->malloc_(&w, wb));
        CK(api->malloc_(&xq, C / 32 * 36));
        CK(api->synth_fill(sh->type, w, R * C / 256, 100 + s, 0.02f));
        CK(api->synth_normal(x, C, 200 + s, 1.0f));
        CK(api->matvec(sh->type, w, R, C, x, y0));   /* fp32 dequantize-and-FMA path */
        CK(api->matvec_dp4a(sh->type, w, R, C, x, y1));
        CK(api->quantize_q8_1(x, C, xq));
        uint8_t *wh = malloc(wb), *xq_gpu = malloc(C / 32 * 36), *xq_cpu = malloc(C / 32 * 36);
        float *xh = malloc(C * 4), *x8 = malloc(C * 4), *g0 = malloc(R * 4), *g1 = malloc(R * 4);
        double *cf = malloc(R * 8), *cq = malloc(R * 8);
        float *cff = malloc(R * 4), *cqf = malloc(R * 4);
        if (!wh || !xq_gpu || !xq_cpu || !xh || !x8 || !g0 || !g1 || !cf || !cq || !cff || !cqf)
            return die("host malloc", -5);
        CK(api->download(wh, w, wb));
        CK(api->download(xh, x, C * 4));
        CK(api->download(g0, y0, R * 4));
        CK(api->download(g1, y1, R * 4));
        CK(api->download(xq_gpu, xq, C / 32 * 36));
        kh_cpu_quantize_q8_1(xh, C, xq_cpu);
        kh_cpu_dequant(9, xq_cpu, C, x8);
        if (kh_cpu_matvec(sh->type, wh, R, C, xh, cf) || kh_cpu_matvec(sh->type, wh, R, C, x8, cq))
            return die("cpu matvec", -1);
        size_t outside = 0, xq_diff = 0;
        double worst = 0.0;
        for (uint64_t i = 0; i < R; i++) {
            cff[i] = (float)cf[i];
            cqf[i] = (float)cq[i];
            const double e = fabs((double)g0[i] - cf[i]) / (1e-3 * (1.0 + fabs(cf[i])));
            worst = e > worst ? e : worst;
            outside += e > 1.0;
        }
        for (uint64_t k = 0; k < C / 32; k++) xq_diff += memcmp(xq_gpu + 36 * k, xq_cpu + 36 * k, 36) != 0;
        const double rq = rel_l2(g1, cqf, R, NULL), rx = rel_l2(g1, cff, R, NULL);
        const int ok = outside == 0 && rq <= 1e-5 && xq_diff == 0;
        fails += !ok;
        printf("check %-24s %s: fp32 GEMV %zu of %llu outside 1e-3*(1+|cpu|) (worst %.3f of it); v_dot4 GEMV "
               "rel_L2 %.2e vs cpu on the same q8_1 x (<= 1e-5); q8_1 x blocks differing %zu; [v_dot4 vs cpu "
               "fp32 x: %.2e] %s\n",
               sh->role, tname(sh->type), outside, (unsigned long long)R, worst, rq, xq_diff, rx, ok ? "PASS" : "FAIL");
        void *hb[] = {wh, xq_gpu, xq_cpu, xh, x8, g0, g1, cf, cq, cff, cqf};
        for (size_t i = 0; i < sizeof hb / sizeof hb[0]; i++) free(hb[i]);
        api->free_(w);
        api->free_(xq);
        api->free_(x);
        api->free_(y0);
        api->free_(y1);
    }
    return fails ? 1 : 0;
}

/* The fused MoE layer on the GPU against the CPU. PASS: rel_L2 <= 1e-5 to
 * the CPU's q8_1 path (x quantized to q8_1; gate/up with the library's q8_1
 * Q4_K dot and SiLU; h quantized to q8_1; down in double; the rank-order
 * weighted sum). The CPU's fp32 path (fp32 x and h, no quantization) is
 * printed for information: it differs by the q8_1 rounding of x and h. */
static int cmd_check_moe(void) {
    enum { H = 2048, F = 768, E = 128, K = 8 };
    const uint64_t rbg = row_bytes(Q4K, H), rbd = row_bytes(Q6K, F);
    const uint64_t gb = (uint64_t)E * F * rbg, db = (uint64_t)E * H * rbd;
    void *g = NULL, *u = NULL, *d = NULL;
    CK(api->malloc_(&g, gb));
    CK(api->malloc_(&u, gb));
    CK(api->malloc_(&d, db));
    CK(api->synth_fill(Q4K, g, (uint64_t)E * F * H / 256, 11, 0.02f));
    CK(api->synth_fill(Q4K, u, (uint64_t)E * F * H / 256, 12, 0.02f));
    CK(api->synth_fill(Q6K, d, (uint64_t)E * H * F / 256, 13, 0.02f));
    float *x = dalloc_f(H), *y = dalloc_f(H), *w_d = dalloc_f(K);
    int32_t *ids_d = NULL;
    CK(api->malloc_((void **)&ids_d, K * 4));
    CK(api->synth_normal(x, H, 21, 1.0f));
    const int32_t ids[K] = {5, 77, 3, 120, 64, 9, 31, 100};
    const float w[K] = {0.25f, 0.2f, 0.15f, 0.12f, 0.1f, 0.08f, 0.06f, 0.04f};
    CK(api->upload(ids_d, ids, sizeof ids));
    CK(api->upload(w_d, w, sizeof w));
    KataliHipMoe moe = {sizeof moe, Q4K, Q4K, Q6K, H, F, E, g, u, d, NULL, NULL, NULL};
    KataliHipMoeRoute r;
    memset(&r, 0, sizeof r);
    r.struct_size = sizeof r;
    r.n_sel = K;
    r.ids = ids_d;
    r.weights = w_d;
    CK(api->moe_layer(&moe, &r, x, NULL, y));
    static float fused[H], xh[H], ref_q[H], ref_f[H], hq_f[F], h_f[F];
    static uint8_t xq[H / 32 * 36], hq[F / 32 * 36];
    static double acc[H];
    CK(api->download(fused, y, sizeof fused));
    CK(api->download(xh, x, sizeof xh));
    uint8_t *gh = malloc(gb), *uh = malloc(gb), *dh = malloc(db);
    if (!gh || !uh || !dh) return die("host malloc", -5);
    CK(api->download(gh, g, gb));
    CK(api->download(uh, u, gb));
    CK(api->download(dh, d, db));
    kh_cpu_quantize_q8_1(xh, H, xq);
    memset(ref_q, 0, sizeof ref_q);
    memset(ref_f, 0, sizeof ref_f);
    for (int k = 0; k < K; k++) {
        const uint8_t *ge = gh + (uint64_t)ids[k] * F * rbg, *ue = uh + (uint64_t)ids[k] * F * rbg;
        const uint8_t *de = dh + (uint64_t)ids[k] * H * rbd;
        for (int j = 0; j < F; j++) {
            /* q8_1 path as the library defines it */
            hq_f[j] = kh_cpu_silu_mul(kh_cpu_dot_q4k_q8(ge + j * rbg, xq, H / 256),
                                      kh_cpu_dot_q4k_q8(ue + j * rbg, xq, H / 256));
            /* fp32 path: dequantized rows against fp32 x, exact exp */
            double gd = 0, ud = 0;
            float grow[H], urow[H];
            kh_cpu_dequant(Q4K, ge + j * rbg, H, grow);
            kh_cpu_dequant(Q4K, ue + j * rbg, H, urow);
            for (int c = 0; c < H; c++) {
                gd += (double)grow[c] * xh[c];
                ud += (double)urow[c] * xh[c];
            }
            h_f[j] = (float)(gd / (1.0 + exp(-gd)) * ud);
        }
        kh_cpu_quantize_q8_1(hq_f, F, hq);
        float h8[F];
        kh_cpu_dequant(9, hq, F, h8);
        kh_cpu_matvec(Q6K, de, H, F, h8, acc);
        for (int i = 0; i < H; i++) ref_q[i] = fmaf(w[k], (float)acc[i], ref_q[i]);
        kh_cpu_matvec(Q6K, de, H, F, h_f, acc);
        for (int i = 0; i < H; i++) ref_f[i] = fmaf(w[k], (float)acc[i], ref_f[i]);
    }
    const double rel_q = rel_l2(fused, ref_q, H, NULL);
    size_t outside = 0;
    const double rel_f = rel_l2(fused, ref_f, H, &outside);
    const int ok = rel_q <= 1e-5;
    printf("check-moe hidden %u ffn %u top-%u: rel_L2 %.2e vs the cpu q8_1 path (<= 1e-5); [cpu fp32 path: "
           "rel_L2 %.2e, %zu of %u outside 1e-3*(1+|ref|)] %s\n",
           H, F, K, rel_q, rel_f, outside, H, ok ? "PASS" : "FAIL");
    free(gh);
    free(uh);
    free(dh);
    void *bufs[] = {g, u, d, x, y, ids_d, w_d};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) api->free_(bufs[i]);
    return ok ? 0 : 1;
}

static int time_ms(void *e0, void *e1, float *ms) { return api->event_elapsed(e0, e1, ms); }

static int cmd_matvec_bench(int reps) {
    void *e0 = NULL, *e1 = NULL;
    CK(api->event_create(&e0));
    CK(api->event_create(&e1));
    /* raw streaming bandwidth in the same process, for reference */
    {
        const size_t n = (size_t)1 << 30;
        void *a = NULL, *b = NULL;
        CK(api->malloc_(&a, n));
        CK(api->malloc_(&b, n));
        CK(api->copy(b, a, n));
        CK(api->event_record(e0));
        for (int i = 0; i < 4; i++) CK(api->copy(b, a, n));
        CK(api->event_record(e1));
        CK(api->sync());
        float ms = 0;
        CK(time_ms(e0, e1, &ms));
        printf("device copy 1 GiB: %.1f GB/s (read + write)\n", 4.0 * 2 * n / (ms * 1e-3) / 1e9);
        api->free_(a);
        api->free_(b);
    }
    for (size_t s = 0; s < NSHAPES; s++) {
        const struct shape *sh = &SHAPES[s];
        const uint64_t wb = sh->rows * row_bytes(sh->type, sh->cols);
        const int copies = (int)((512ull << 20) / wb) + 1;   /* a pool larger than L2 + MALL */
        void *w = NULL;
        float *x = dalloc_f(sh->cols), *y = dalloc_f(sh->rows);
        CK(api->malloc_(&w, wb * copies));
        CK(api->synth_fill(sh->type, w, sh->rows * sh->cols / 256 * copies, 300 + s, 0.02f));
        CK(api->synth_normal(x, sh->cols, 7, 1.0f));
        CK(api->matvec_dp4a(sh->type, w, sh->rows, sh->cols, x, y));
        CK(api->sync());
        const int n = reps * copies;
        CK(api->event_record(e0));
        for (int i = 0; i < n; i++)
            CK(api->matvec_dp4a(sh->type, (const uint8_t *)w + (uint64_t)(i % copies) * wb, sh->rows, sh->cols, x, y));
        CK(api->event_record(e1));
        CK(api->sync());
        float ms = 0;
        CK(time_ms(e0, e1, &ms));
        const double us = ms * 1e3 / n;
        printf("matvec-bench %-24s %s: %8.2f us/call, %7.1f GB/s (cold pool of %d copies, %d calls)\n", sh->role,
               tname(sh->type), us, (double)wb / (us * 1e-6) / 1e9, copies, n);
        api->free_(w);
        api->free_(x);
        api->free_(y);
    }
    api->event_destroy(e0);
    api->event_destroy(e1);
    return 0;
}

/* L layers of distinct weights, logits per token and layer (steps tokens,
 * rotated through a device step index), one graph per token. */
static int moe_bench(const char *name, uint32_t L, uint32_t H, uint32_t F, uint32_t E, uint32_t K, int shared,
                     int tokens) {
    const uint64_t rbg = row_bytes(Q4K, H), rbd = row_bytes(Q6K, F);
    const uint64_t eb = 2 * F * rbg + H * rbd;
    const int steps = 64;
    void **g = calloc(L, sizeof *g), **u = calloc(L, sizeof *u), **d = calloc(L, sizeof *d);
    void **gs = calloc(L, sizeof *gs), **us_ = calloc(L, sizeof *us_), **ds = calloc(L, sizeof *ds);
    for (uint32_t l = 0; l < L; l++) {
        CK(api->malloc_(&g[l], (uint64_t)E * F * rbg));
        CK(api->malloc_(&u[l], (uint64_t)E * F * rbg));
        CK(api->malloc_(&d[l], (uint64_t)E * H * rbd));
        CK(api->synth_fill(Q4K, g[l], (uint64_t)E * F * H / 256, 1000 + 6 * l, 0.02f));
        CK(api->synth_fill(Q4K, u[l], (uint64_t)E * F * H / 256, 1001 + 6 * l, 0.02f));
        CK(api->synth_fill(Q6K, d[l], (uint64_t)E * H * F / 256, 1002 + 6 * l, 0.02f));
        if (shared) {
            CK(api->malloc_(&gs[l], F * rbg));
            CK(api->malloc_(&us_[l], F * rbg));
            CK(api->malloc_(&ds[l], H * rbd));
            CK(api->synth_fill(Q4K, gs[l], (uint64_t)F * H / 256, 1003 + 6 * l, 0.02f));
            CK(api->synth_fill(Q4K, us_[l], (uint64_t)F * H / 256, 1004 + 6 * l, 0.02f));
            CK(api->synth_fill(Q6K, ds[l], (uint64_t)H * F / 256, 1005 + 6 * l, 0.02f));
        }
    }
    float *x = dalloc_f(H), *y = dalloc_f(H), *logits = dalloc_f((size_t)steps * L * E);
    int32_t *step = NULL;
    CK(api->malloc_((void **)&step, 4));
    CK(api->memset_(step, 0, 4));
    CK(api->synth_normal(x, H, 5, 1.0f));
    CK(api->synth_normal(logits, (size_t)steps * L * E, 6, 1.0f));
    KataliHipMoe *m = calloc(L, sizeof *m);
    KataliHipMoeRoute *r = calloc(L, sizeof *r);
    for (uint32_t l = 0; l < L; l++) {
        KataliHipMoe mm = {sizeof mm, Q4K, Q4K, Q6K, H, F, E, g[l], u[l], d[l],
                           shared ? gs[l] : NULL, shared ? us_[l] : NULL, shared ? ds[l] : NULL};
        m[l] = mm;
        r[l].struct_size = sizeof r[l];
        r[l].n_sel = (int32_t)K;
        r[l].logits = logits + (size_t)l * E;
        r[l].step = step;
        r[l].logits_stride = (uint64_t)L * E;
    }
    /* eager once (sizes the scratch), then capture one token */
    for (uint32_t l = 0; l < L; l++) CK(api->moe_layer(&m[l], &r[l], (l & 1) ? y : x, NULL, (l & 1) ? x : y));
    CK(api->sync());
    void *graph = NULL;
    CK(api->graph_begin());
    for (uint32_t l = 0; l < L; l++) CK(api->moe_layer(&m[l], &r[l], (l & 1) ? y : x, NULL, (l & 1) ? x : y));
    CK(api->step_advance(step, steps));
    CK(api->graph_end(&graph));
    for (int i = 0; i < 4; i++) CK(api->graph_launch(graph));
    void *e0 = NULL, *e1 = NULL;
    CK(api->event_create(&e0));
    CK(api->event_create(&e1));
    CK(api->sync());
    CK(api->event_record(e0));
    for (int t = 0; t < tokens; t++) CK(api->graph_launch(graph));
    CK(api->event_record(e1));
    CK(api->sync());
    float ms = 0;
    CK(time_ms(e0, e1, &ms));
    const double per_tok = ms / tokens, bytes = (double)L * ((K + (shared ? 1 : 0)) * eb + H / 32 * 36 + H * 4);
    printf("%s: %u layers, %u experts, top-%u%s, hidden %u, ffn %u: %.3f ms/token, %.1f us/layer, %.1f GB/s "
           "(%.1f %% of 8 TB/s), %.1f tok/s\n", name, L, E, K, shared ? " + shared" : "", H, F, per_tok,
           per_tok * 1e3 / L, bytes / (per_tok * 1e-3) / 1e9, bytes / (per_tok * 1e-3) / 8e12 * 100, 1e3 / per_tok);
    api->graph_destroy(graph);
    api->event_destroy(e0);
    api->event_destroy(e1);
    for (uint32_t l = 0; l < L; l++) {
        api->free_(g[l]);
        api->free_(u[l]);
        api->free_(d[l]);
        if (shared) {
            api->free_(gs[l]);
            api->free_(us_[l]);
            api->free_(ds[l]);
        }
    }
    api->free_(x);
    api->free_(y);
    api->free_(logits);
    api->free_(step);
    free(g); free(u); free(d); free(gs); free(us_); free(ds); free(m); free(r);
    return 0;
}

static int cmd_gguf_info(const char *path) {
    KataliHipGguf *g = NULL;
    char err[256];
    if (katali_hip_gguf_open(path, &g, err, sizeof err)) {
        printf("gguf-info: %s\n", err);
        return 1;
    }
    size_t al = 0;
    const char *arch = katali_hip_gguf_get_str(g, "general.architecture", &al);
    printf("GGUF v%u, alignment %llu, data at %llu, architecture %.*s, %llu tensors\n", katali_hip_gguf_version(g),
           (unsigned long long)katali_hip_gguf_alignment(g), (unsigned long long)katali_hip_gguf_data_offset(g),
           arch ? (int)al : 1, arch ? arch : "?", (unsigned long long)katali_hip_gguf_tensor_count(g));
    for (uint64_t i = 0; i < katali_hip_gguf_tensor_count(g); i++) {
        KataliHipGgufTensor t;
        katali_hip_gguf_tensor(g, i, &t);
        printf("  %-40s type %2u dims", t.name, t.type);
        for (uint32_t d = 0; d < t.n_dims; d++) printf(" %llu", (unsigned long long)t.dims[d]);
        printf("  %llu bytes%s\n", (unsigned long long)t.nbytes, t.data ? "" : " (no data: unknown type)");
    }
    katali_hip_gguf_close(g);
    return 0;
}

/* One layer of the file: the fused layer routed by the file's router on
 * N(0,1) x, against the same layer composed from separate library GEMVs
 * (q8 gate/up GEMVs, SiLU-GLU on the host, q8 down GEMV, the weighted sum in
 * rank order with the shared expert last, as the fused layer forms it). */
static int gguf_check_layer(KataliHipWeights *w, uint32_t l, int n_sel) {
    KataliHipMoe m;
    const float *router = NULL;
    if (katali_hip_gguf_moe_layer(w, l, &m, &router, NULL)) {
        printf("gguf-check layer %u: %s\n", l, katali_hip_gguf_last_error());
        return 1;
    }
    const uint32_t H = m.hidden, F = m.ffn, E = m.n_expert, K = (uint32_t)n_sel;
    const uint64_t rbg = row_bytes(m.gate_type, H), rbd = row_bytes(m.down_type, F);
    float *x = dalloc_f(H), *y = dalloc_f(H), *logits = dalloc_f(E), *gv = dalloc_f(F), *uv = dalloc_f(F),
          *h = dalloc_f(F), *dv = dalloc_f(H), *wo = dalloc_f(16);
    void *xq = NULL, *hq = NULL, *ido = NULL;
    CK(api->malloc_(&xq, H / 32 * 36));
    CK(api->malloc_(&hq, F / 32 * 36));
    CK(api->malloc_(&ido, 64));
    CK(api->synth_normal(x, H, 31 + l, 1.0f));
    CK(api->matvec(0, router, E, H, x, logits));
    KataliHipMoeRoute r;
    memset(&r, 0, sizeof r);
    r.struct_size = sizeof r;
    r.n_sel = (int32_t)K;
    r.logits = logits;
    r.ids_out = (int32_t *)ido;
    r.weights_out = wo;
    CK(api->moe_layer(&m, &r, x, NULL, y));
    float *fused = malloc(H * 4), *ref = calloc(H, 4), *gh = malloc(F * 4), *uh = malloc(F * 4),
          *hh = malloc(F * 4), *dh = malloc(H * 4), wts[16];
    int32_t ids[16];
    CK(api->download(fused, y, H * 4));
    CK(api->download(ids, ido, K * 4));
    CK(api->download(wts, wo, K * 4));
    CK(api->quantize_q8_1(x, H, xq));
    const int shared = m.gate_shexp != NULL;
    for (uint32_t k = 0; k < K + (shared ? 1 : 0); k++) {
        const int sh = k == K;
        const uint8_t *ge = sh ? m.gate_shexp : (const uint8_t *)m.gate_exps + (uint64_t)ids[k] * F * rbg;
        const uint8_t *ue = sh ? m.up_shexp : (const uint8_t *)m.up_exps + (uint64_t)ids[k] * F * rbg;
        const uint8_t *de = sh ? m.down_shexp : (const uint8_t *)m.down_exps + (uint64_t)ids[k] * H * rbd;
        CK(api->matvec_q8(m.gate_type, ge, F, H, xq, gv));
        CK(api->matvec_q8(m.up_type, ue, F, H, xq, uv));
        CK(api->download(gh, gv, F * 4));
        CK(api->download(uh, uv, F * 4));
        for (uint32_t j = 0; j < F; j++) hh[j] = kh_cpu_silu_mul(gh[j], uh[j]);
        CK(api->upload(h, hh, F * 4));
        CK(api->quantize_q8_1(h, F, hq));
        CK(api->matvec_q8(m.down_type, de, H, F, hq, dv));
        CK(api->download(dh, dv, H * 4));
        const float wk = sh ? 1.0f : wts[k];
        for (uint32_t i = 0; i < H; i++) ref[i] = fmaf(wk, dh[i], ref[i]);
    }
    size_t outside = 0;
    const double rel = rel_l2(fused, ref, H, &outside);
    const int ok = rel <= 1e-4;
    printf("gguf-check layer %u: hidden %u ffn %u top-%u of %u%s, experts", l, H, F, K, E, shared ? " + shared" : "");
    for (uint32_t k = 0; k < K; k++) printf(" %d", ids[k]);
    printf(": rel_L2(fused, composed) = %.3e %s\n", rel, ok ? "PASS" : "FAIL");
    void *bufs[] = {x, y, logits, gv, uv, h, dv, wo, xq, hq, ido};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) api->free_(bufs[i]);
    free(fused); free(ref); free(gh); free(uh); free(hh); free(dh);
    return ok ? 0 : 1;
}

static int cmd_gguf_check(const char *path) {
    KataliHipGguf *g = NULL;
    char err[256];
    if (katali_hip_gguf_open(path, &g, err, sizeof err)) {
        printf("gguf-check: %s\n", err);
        return 1;
    }
    size_t al = 0;
    const char *arch = katali_hip_gguf_get_str(g, "general.architecture", &al);
    char key[96];
    snprintf(key, sizeof key, "%.*s.expert_used_count", arch ? (int)al : 0, arch ? arch : "");
    const int n_sel = (int)katali_hip_gguf_get_int(g, key, 8);
    snprintf(key, sizeof key, "%.*s.block_count", arch ? (int)al : 0, arch ? arch : "");
    const int64_t L = katali_hip_gguf_get_int(g, key, 0);
    KataliHipWeights *w = NULL;
    int fails = 0, layers = 0;
    if (katali_hip_weights_create(g, 0, &w)) {
        printf("gguf-check: %s\n", katali_hip_gguf_last_error());
        katali_hip_gguf_close(g);
        return 1;
    }
    for (int64_t l = 0; l < L; l++) {
        char name[64];
        snprintf(name, sizeof name, "blk.%lld.ffn_gate_exps.weight", (long long)l);
        KataliHipGgufTensor t;
        if (katali_hip_gguf_find(g, name, &t)) continue;   /* a dense layer */
        fails += gguf_check_layer(w, (uint32_t)l, n_sel);
        layers++;
    }
    printf("gguf-check: %d MoE layer(s), %d failed, %.2f GB resident\n", layers, fails,
           katali_hip_weights_resident_bytes(w) / 1e9);
    katali_hip_weights_destroy(w);
    katali_hip_gguf_close(g);
    return (fails || !layers) ? 1 : 0;
}

static void usage(void) {
    fputs("usage: katali-hip info | dp4a-selftest | check | check-moe | matvec-bench [reps] | bench [tokens] |"
          " bench-cold [tokens] | gguf-info FILE | gguf-check FILE\n", stderr);
}

int main(int argc, char **argv) {
    if (argc < 2) {
        usage();
        return 2;
    }
    const char *cmd = argv[1];
    const int n = argc > 2 ? atoi(argv[2]) : 0;
    if (!strcmp(cmd, "gguf-info") && argc > 2) return cmd_gguf_info(argv[2]);
    if (!katali_gpu_probe() || !(api = katali_gpu_api())) {
        printf("no usable GPU: %s\n", katali_gpu_status());
        return 2;
    }
    if (!strcmp(cmd, "info")) return cmd_info();
    if (!strcmp(cmd, "dp4a-selftest")) return cmd_selftest();
    if (!strcmp(cmd, "check")) return cmd_check();
    if (!strcmp(cmd, "check-moe")) return cmd_check_moe();
    if (!strcmp(cmd, "matvec-bench")) return cmd_matvec_bench(n > 0 ? n : 5);
    if (!strcmp(cmd, "bench")) return moe_bench("bench", 48, 2048, 768, 128, 8, 0, n > 0 ? n : 32);
    if (!strcmp(cmd, "bench-cold")) return moe_bench("bench-cold", 40, 2048, 512, 256, 8, 1, n > 0 ? n : 64);
    if (!strcmp(cmd, "gguf-check") && argc > 2) return cmd_gguf_check(argv[2]);
    usage();
    return 2;
}
