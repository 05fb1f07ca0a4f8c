/*
 * cngpt_oracle.c - CPU restatement of cngpt's inference forward pass.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the CPU
 * baseline bench.py times. The product never links or loads this file.
 *
 * Restates, with file:line of the reference at each function:
 *   src/model.c  parameter count/layout, seeded init, sample_top_k
 *   src/ops.c    layernorm / gelu / softmax / causal mask / linear /
 *                cross-entropy (scalar paths)
 *   src/fast.c   gpt_forward_fast, its column-split products, its threads
 * The matrix products are cblas_sgemm calls, as in the reference; the CBLAS
 * is bound at run time (orc_use_blas) and a blocked C product stands in
 * when none is available.
 */
#define _GNU_SOURCE
#include "cngpt_oracle.h"

#include <dlfcn.h>
#include <float.h>
#include <math.h>
#include <sched.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

/* ------------------------------------------------------------------ */
/* CBLAS binding (standard CBLAS enum values)                          */
/* ------------------------------------------------------------------ */

enum { ROW_MAJOR = 101, NO_TRANS = 111, TRANS = 112 };

typedef void (*sgemm_fn)(int order, int ta, int tb, int M, int N, int K,
                         float alpha, const float *A, int lda,
                         const float *B, int ldb, float beta,
                         float *C, int ldc);
typedef void (*setthreads_fn)(int);
typedef int  (*getthreads_fn)(void);
typedef char *(*getconfig_fn)(void);

static sgemm_fn      g_sgemm = NULL;
static setthreads_fn g_blas_set_threads = NULL;
static getthreads_fn g_blas_get_threads = NULL;
static char          g_blas_info[512] = "builtin blocked C sgemm";

int orc_use_blas(const char *path)
{
    void *h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!h) return -1;
    static const char *prefixes[] = { "", "scipy_" };
    for (int i = 0; i < 2; i++) {
        char name[64];
        snprintf(name, sizeof(name), "%scblas_sgemm", prefixes[i]);
        sgemm_fn f = (sgemm_fn)dlsym(h, name);
        if (!f) continue;
        g_sgemm = f;
        snprintf(name, sizeof(name), "%sopenblas_set_num_threads", prefixes[i]);
        g_blas_set_threads = (setthreads_fn)dlsym(h, name);
        snprintf(name, sizeof(name), "%sopenblas_get_num_threads", prefixes[i]);
        g_blas_get_threads = (getthreads_fn)dlsym(h, name);
        snprintf(name, sizeof(name), "%sopenblas_get_config", prefixes[i]);
        getconfig_fn cfg = (getconfig_fn)dlsym(h, name);
        snprintf(g_blas_info, sizeof(g_blas_info), "%s [%s]",
                 cfg ? cfg() : "cblas", path);
        return 0;
    }
    dlclose(h);
    return -1;
}

const char *orc_blas_info(void) { return g_blas_info; }

/* Built-in product for when no CBLAS is bound. Row-major,
 * C = alpha * A * op(B) + beta * C with op(B) = B^T (tb == TRANS) or B. */
static void builtin_sgemm(int tb, int M, int N, int K, float alpha,
                          const float *A, int lda, const float *B, int ldb,
                          float beta, float *C, int ldc)
{
    for (int i = 0; i < M; i++) {
        float *c = C + (size_t)i * ldc;
        for (int j = 0; j < N; j++) c[j] = beta == 0.0f ? 0.0f : beta * c[j];
        const float *a = A + (size_t)i * lda;
        if (tb == TRANS) {
            for (int j = 0; j < N; j++) {
                const float *b = B + (size_t)j * ldb;
                float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
                int k = 0;
                for (; k + 4 <= K; k += 4) {
                    s0 += a[k] * b[k];         s1 += a[k + 1] * b[k + 1];
                    s2 += a[k + 2] * b[k + 2]; s3 += a[k + 3] * b[k + 3];
                }
                for (; k < K; k++) s0 += a[k] * b[k];
                c[j] += alpha * ((s0 + s1) + (s2 + s3));
            }
        } else {
            for (int k = 0; k < K; k++) {
                float av = alpha * a[k];
                const float *b = B + (size_t)k * ldb;
                for (int j = 0; j < N; j++) c[j] += av * b[j];
            }
        }
    }
}

static void sgemm(int tb, int M, int N, int K, float alpha,
                  const float *A, int lda, const float *B, int ldb,
                  float beta, float *C, int ldc)
{
    if (M <= 0 || N <= 0) return;
    if (g_sgemm)
        g_sgemm(ROW_MAJOR, NO_TRANS, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    else
        builtin_sgemm(tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
}

/* C = alpha * op(A) * op(B) + beta * C with either operand transposed (the
 * backward's products, src/ops.c:125-153 and src/model.c:768-799). */
static void sgemm_t(int ta, int tb, int M, int N, int K, float alpha,
                    const float *A, int lda, const float *B, int ldb,
                    float beta, float *C, int ldc)
{
    if (M <= 0 || N <= 0) return;
    if (g_sgemm) {
        g_sgemm(ROW_MAJOR, ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
        return;
    }
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float s = 0.0f;
            for (int k = 0; k < K; k++) {
                const float a = ta == TRANS ? A[(size_t)k * lda + i] : A[(size_t)i * lda + k];
                const float b = tb == TRANS ? B[(size_t)j * ldb + k] : B[(size_t)k * ldb + j];
                s += a * b;
            }
            float *c = C + (size_t)i * ldc + j;
            *c = alpha * s + (beta == 0.0f ? 0.0f : beta * *c);
        }
}

/* ------------------------------------------------------------------ */
/* Parameters: count, layout, seeded init                              */
/* ------------------------------------------------------------------ */

long orc_num_params(const orc_cfg *c)                 /* model.c:20-48 */
{
    long C = c->n_embd, V = c->vocab_size, T = c->block_size, L = c->n_layer;
    long per_layer = C + C + 3 * C * C + 3 * C + C * C + C + C + C
                   + 4 * C * C + 4 * C + C * 4 * C + C;
    return V * C + T * C + L * per_layer + 2 * C;
}

void orc_offsets(const orc_cfg *c, long *off)          /* model.c:54-83 */
{
    long C = c->n_embd, V = c->vocab_size, T = c->block_size;
    long sizes[12] = { C, C, 3 * C * C, 3 * C, C * C, C, C, C,
                       4 * C * C, 4 * C, C * 4 * C, C };
    long p = 0;
    int i = 0;
    off[i++] = p; p += V * C;     /* wte */
    off[i++] = p; p += T * C;     /* wpe */
    for (int l = 0; l < c->n_layer; l++)
        for (int k = 0; k < 12; k++) { off[i++] = p; p += sizes[k]; }
    off[i++] = p; p += C;         /* ln_f_w */
    off[i++] = p;                 /* ln_f_b */
}

/* Box-Muller over rand(), model.c:275-284: only u's variate is used. */
static float randn(void)
{
    float u, v, s;
    do {
        u = (float)rand() / (float)RAND_MAX * 2.0f - 1.0f;
        v = (float)rand() / (float)RAND_MAX * 2.0f - 1.0f;
        s = u * u + v * v;
    } while (s >= 1.0f || s == 0.0f);
    return u * sqrtf(-2.0f * logf(s) / s);
}

static void fill_normal(float *p, long n, float std)  /* model.c:286-290 */
{
    for (long i = 0; i < n; i++) p[i] = randn() * std;
}

void orc_init_weights(const orc_cfg *c, float *params, unsigned seed)
{                                                       /* model.c:292-331 */
    long C = c->n_embd, V = c->vocab_size, L = c->n_layer;
    long *off = malloc(sizeof(long) * (size_t)(4 + 12 * L));
    orc_offsets(c, off);
    float std = 0.02f;
    float res_std = 0.02f / sqrtf(2.0f * (float)L);
    srand(seed);
    fill_normal(params + off[0], V * C, std);
    fill_normal(params + off[1], (long)c->block_size * C, std);
    for (long l = 0; l < L; l++) {
        long *o = off + 2 + 12 * l;
        for (long i = 0; i < C; i++) params[o[0] + i] = 1.0f;   /* ln1_w */
        memset(params + o[1], 0, C * sizeof(float));           /* ln1_b */
        for (long i = 0; i < C; i++) params[o[6] + i] = 1.0f;   /* ln2_w */
        memset(params + o[7], 0, C * sizeof(float));           /* ln2_b */
        fill_normal(params + o[2], 3 * C * C, std);             /* c_attn_w */
        memset(params + o[3], 0, 3 * C * sizeof(float));
        fill_normal(params + o[4], C * C, res_std);             /* c_proj_w */
        memset(params + o[5], 0, C * sizeof(float));
        fill_normal(params + o[8], 4 * C * C, std);             /* mlp_fc_w */
        memset(params + o[9], 0, 4 * C * sizeof(float));
        fill_normal(params + o[10], C * 4 * C, res_std);        /* mlp_proj_w */
        memset(params + o[11], 0, C * sizeof(float));
    }
    long *of = off + 2 + 12 * L;
    for (long i = 0; i < C; i++) params[of[0] + i] = 1.0f;      /* ln_f_w */
    memset(params + of[1], 0, C * sizeof(float));               /* ln_f_b */
    free(off);
}

void orc_srand(unsigned seed) { srand(seed); }
float orc_rand_uniform(void) { return (float)rand() / ((float)RAND_MAX + 1.0f); }

/* ------------------------------------------------------------------ */
/* Ops (scalar paths of src/ops.c)                                     */
/* ------------------------------------------------------------------ */

void orc_layernorm(const float *x, const float *w, const float *b, float *out,
                   float *mean, float *rstd, int T, int C)
{                                                       /* ops.c:191-248 */
    const float eps = 1e-5f;
    for (int t = 0; t < T; t++) {
        const float *xr = x + (size_t)t * C;
        float *o = out + (size_t)t * C;
        float m = 0.0f;
        for (int c = 0; c < C; c++) m += xr[c];
        m /= (float)C;
        float v = 0.0f;
        for (int c = 0; c < C; c++) { float d = xr[c] - m; v += d * d; }
        float rs = 1.0f / sqrtf(v / (float)C + eps);
        if (mean) mean[t] = m;
        if (rstd) rstd[t] = rs;
        for (int c = 0; c < C; c++) o[c] = (xr[c] - m) * rs * w[c] + b[c];
    }
}

static inline float gelu1(float x)                      /* ops.c:337-345 */
{
    const float k0 = 0.7978845608028654f;   /* sqrt(2/pi) */
    const float k1 = 0.044715f;
    float x3 = x * x * x;
    return 0.5f * x * (1.0f + tanhf(k0 * (x + k1 * x3)));
}

void orc_gelu(const float *x, float *out, int n)        /* ops.c:357-380 */
{
    for (int i = 0; i < n; i++) out[i] = gelu1(x[i]);
}

void orc_softmax_inplace(float *x, int rows, int cols)  /* ops.c:424-482 */
{
    for (int r = 0; r < rows; r++) {
        float *row = x + (size_t)r * cols;
        float mx = -FLT_MAX;
        for (int c = 0; c < cols; c++) if (row[c] > mx) mx = row[c];
        float sum = 0.0f;
        for (int c = 0; c < cols; c++) { row[c] = expf(row[c] - mx); sum += row[c]; }
        float inv = 1.0f / sum;
        for (int c = 0; c < cols; c++) row[c] *= inv;
    }
}

void orc_causal_mask(float *s, int T)                   /* ops.c:488-493 */
{
    for (int i = 0; i < T; i++)
        for (int j = i + 1; j < T; j++) s[(size_t)i * T + j] = -1e9f;
}

void orc_linear(const float *X, const float *W, const float *b, float *Y,
                int M, int K, int N)                    /* ops.c:109-123 */
{
    sgemm(TRANS, M, N, K, 1.0f, X, K, W, K, 0.0f, Y, N);
    if (b)
        for (int i = 0; i < M; i++)
            for (int j = 0; j < N; j++) Y[(size_t)i * N + j] += b[j];
}

/* ------------------------------------------------------------------ */
/* Threads (src/fast.c:104-200)                                        */
/* ------------------------------------------------------------------ */

static int g_threads = 0;

/* One mask per physical core, fast.c:124-156. */
static int core_masks(cpu_set_t *masks, int max)
{
    cpu_set_t allowed;
    if (sched_getaffinity(0, sizeof(allowed), &allowed) != 0) return 0;
    char (*seen)[64] = calloc((size_t)max, 64);
    int n = 0;
    for (int c = 0; c < CPU_SETSIZE; c++) {
        if (!CPU_ISSET(c, &allowed)) continue;
        char path[96], sib[64] = "";
        snprintf(path, sizeof(path),
                 "/sys/devices/system/cpu/cpu%d/topology/thread_siblings_list", c);
        FILE *fp = fopen(path, "r");
        if (fp) { if (!fgets(sib, sizeof(sib), fp)) sib[0] = '\0'; fclose(fp); }
        int idx = -1;
        if (sib[0])
            for (int i = 0; i < n; i++) if (strcmp(seen[i], sib) == 0) { idx = i; break; }
        if (idx < 0) {
            if (n >= max) continue;
            idx = n++;
            snprintf(seen[idx], 64, "%s", sib);
            CPU_ZERO(&masks[idx]);
        }
        CPU_SET(c, &masks[idx]);
    }
    free(seen);
    return n;
}

static cpu_set_t g_cores[1024];
static int g_ncores = -1;

int orc_physical_cores(void)
{
    if (g_ncores < 0) g_ncores = core_masks(g_cores, 1024);
    return g_ncores;
}

int orc_set_threads(int n)
{
    int nc = orc_physical_cores();
    if (n <= 0) n = nc > 0 ? nc : 1;
    g_threads = n;
    return n;
}

/* Pin thread i of the team to physical core i (fast.c:189-197); the
 * caller's own mask is restored afterwards so the host process is left
 * as it was. */
static void pin_team(int P, cpu_set_t *saved)
{
    sched_getaffinity(0, sizeof(*saved), saved);
    int nc = orc_physical_cores();
    if (nc <= 0) return;
    #pragma omp parallel num_threads(P)
    sched_setaffinity(0, sizeof(cpu_set_t), &g_cores[omp_get_thread_num() % nc]);
}

static void unpin_team(int P, const cpu_set_t *saved)
{
    #pragma omp parallel num_threads(P)
    sched_setaffinity(0, sizeof(cpu_set_t), saved);
}

/* ------------------------------------------------------------------ */
/* Forward (src/fast.c:227-333)                                        */
/* ------------------------------------------------------------------ */

/* linear_par, fast.c:175-205: column blocks of 16-float multiples, one
 * single-threaded sgemm per thread; residual via beta = 1, then + b,
 * then GELU on the block. */
static void linear_par(int P, const float *X, const float *W, const float *b,
                       float *Y, int M, int K, int N, int accumulate, int gelu)
{
    int w = (N + P - 1) / P;
    w = (w + 15) & ~15;
    int nblk = (N + w - 1) / w;
    float beta = accumulate ? 1.0f : 0.0f;
    #pragma omp parallel for schedule(static) num_threads(P)
    for (int j = 0; j < nblk; j++) {
        int n0 = j * w;
        int n1 = n0 + w < N ? n0 + w : N;
        int nn = n1 - n0;
        sgemm(TRANS, M, nn, K, 1.0f, X, K, W + (size_t)n0 * K, K, beta, Y + n0, N);
        for (int i = 0; i < M; i++) {
            float *row = Y + (size_t)i * N + n0;
            if (b) for (int c = 0; c < nn; c++) row[c] += b[n0 + c];
            if (gelu) for (int c = 0; c < nn; c++) row[c] = gelu1(row[c]);
        }
    }
}

/* layernorm_par, fast.c:207-225 */
static void layernorm_par(int P, const float *x, const float *w, const float *b,
                          float *out, int rows, int C)
{
    #pragma omp parallel for schedule(static) num_threads(P)
    for (int r = 0; r < rows; r++)
        orc_layernorm(x + (size_t)r * C, w, b, out + (size_t)r * C, NULL, NULL, 1, C);
}

int orc_forward(const orc_cfg *c, const float *params, const int *tokens,
                int B, int T, int mode, float *logits)
{
    const int C = c->n_embd, V = c->vocab_size, L = c->n_layer, H = c->n_head;
    if (B <= 0 || T <= 0 || T > c->block_size || L < 1 || H <= 0 || C % H) return -1;
    for (long i = 0; i < (long)B * T; i++)
        if (tokens[i] < 0 || tokens[i] >= V) return -1;
    const int hs = C / H;
    const float scale = 1.0f / sqrtf((float)hs);
    const size_t N = (size_t)B * T;
    const int all = (mode == ORC_ALL);
    int P = g_threads > 0 ? g_threads : orc_set_threads(0);

    long *off = malloc(sizeof(long) * (size_t)(4 + 12 * L));
    float *x = malloc(N * C * sizeof(float));
    float *ln = malloc(N * C * sizeof(float));
    float *qkv = malloc(N * 3 * C * sizeof(float));
    float *aout = malloc(N * C * sizeof(float));
    float *hid = malloc(N * 4 * C * sizeof(float));
    float *sc = malloc((size_t)P * T * T * sizeof(float));   /* one plane per thread */
    if (!off || !x || !ln || !qkv || !aout || !hid || !sc) {
        free(off); free(x); free(ln); free(qkv); free(aout); free(hid); free(sc);
        return -1;
    }
    orc_offsets(c, off);
    const float *wte = params + off[0], *wpe = params + off[1];

    cpu_set_t saved;
    pin_team(P, &saved);
    int blas_threads = g_blas_get_threads ? g_blas_get_threads() : 1;
    if (g_blas_set_threads) g_blas_set_threads(1);      /* fast.c:242-243 */

    #pragma omp parallel for schedule(static) num_threads(P)
    for (long i = 0; i < (long)N; i++) {                 /* fast.c:245-254 */
        int t = (int)(i % T);
        const float *e = wte + (size_t)tokens[i] * C, *p = wpe + (size_t)t * C;
        float *d = x + (size_t)i * C;
        for (int k = 0; k < C; k++) d[k] = e[k] + p[k];
    }

    for (int l = 0; l < L; l++) {                        /* fast.c:256-324 */
        const long *o = off + 2 + 12 * l;
        const int last = !all && (l == L - 1);
        layernorm_par(P, x, params + o[0], params + o[1], ln, (int)N, C);
        linear_par(P, ln, params + o[2], params + o[3], qkv, (int)N, C, 3 * C, 0, 0);

        #pragma omp parallel for schedule(static) num_threads(P)
        for (int bh = 0; bh < B * H; bh++) {             /* fast.c:267-298 */
            int b = bh / H, h = bh % H;
            const float *q = qkv + (size_t)b * T * 3 * C + h * hs;
            const float *k = q + C, *v = q + 2 * C;
            float *ao = aout + (size_t)b * T * C + h * hs;
            float *s = sc + (size_t)omp_get_thread_num() * T * T;
            if (!last) {
                sgemm(TRANS, T, T, hs, scale, q, 3 * C, k, 3 * C, 0.0f, s, T);
                orc_causal_mask(s, T);
                orc_softmax_inplace(s, T, T);
                sgemm(NO_TRANS, T, hs, T, 1.0f, s, T, v, 3 * C, 0.0f, ao, C);
            } else {
                const float *qr = q + (size_t)(T - 1) * 3 * C;
                sgemm(TRANS, 1, T, hs, scale, qr, 3 * C, k, 3 * C, 0.0f, s, T);
                orc_softmax_inplace(s, 1, T);
                sgemm(NO_TRANS, 1, hs, T, 1.0f, s, T, v, 3 * C, 0.0f,
                      ao + (size_t)(T - 1) * C, C);
            }
        }

        int rows = (int)N;
        if (last) {                                       /* fast.c:300-311 */
            for (int b = 0; b < B; b++) {
                memmove(aout + (size_t)b * C, aout + ((size_t)b * T + T - 1) * C, C * sizeof(float));
                memmove(x + (size_t)b * C, x + ((size_t)b * T + T - 1) * C, C * sizeof(float));
            }
            rows = B;
        }
        linear_par(P, aout, params + o[4], params + o[5], x, rows, C, C, 1, 0);
        layernorm_par(P, x, params + o[6], params + o[7], ln, rows, C);
        linear_par(P, ln, params + o[8], params + o[9], hid, rows, C, 4 * C, 0, 1);
        linear_par(P, hid, params + o[10], params + o[11], x, rows, 4 * C, C, 1, 0);
    }

    const long *of = off + 2 + 12 * L;                    /* fast.c:326-329 */
    int rows = all ? (int)N : B;
    layernorm_par(P, x, params + of[0], params + of[1], ln, rows, C);
    linear_par(P, ln, wte, NULL, logits, rows, C, V, 0, 0);

    if (g_blas_set_threads) g_blas_set_threads(blas_threads);
    unpin_team(P, &saved);
    free(off); free(x); free(ln); free(qkv); free(aout); free(hid); free(sc);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Sampling (src/model.c:927-989)                                      */
/* ------------------------------------------------------------------ */

int orc_sample_top_k(const float *logits, int V, float temp, int top_k, float r)
{
    if (V <= 0) return 0;
    float *p = malloc((size_t)V * sizeof(float));
    if (!p) return 0;
    float t = temp > 0.0f ? temp : 1.0f;                 /* model.c:934 */
    for (int i = 0; i < V; i++) p[i] = logits[i] / t;
    float mx = p[0];
    for (int i = 1; i < V; i++) if (p[i] > mx) mx = p[i];
    float sum = 0.0f;
    for (int i = 0; i < V; i++) { p[i] = expf(p[i] - mx); sum += p[i]; }
    for (int i = 0; i < V; i++) p[i] /= sum;

    if (top_k > 0 && top_k < V) {                         /* model.c:945-975 */
        /* k-th largest probability; the reference finds it with a partial
         * selection sort on a copy, which yields the same value. */
        float *cp = malloc((size_t)V * sizeof(float));
        memcpy(cp, p, (size_t)V * sizeof(float));
        for (int k = 0; k < top_k; k++)
            for (int i = k + 1; i < V; i++)
                if (cp[i] > cp[k]) { float tmp = cp[i]; cp[i] = cp[k]; cp[k] = tmp; }
        float threshold = cp[top_k - 1];
        free(cp);
        float ns = 0.0f;
        for (int i = 0; i < V; i++) { if (p[i] < threshold) p[i] = 0.0f; ns += p[i]; }
        if (ns > 0.0f) for (int i = 0; i < V; i++) p[i] /= ns;
    }

    float cdf = 0.0f;                                     /* model.c:978-985 */
    int tok = V - 1;
    for (int i = 0; i < V; i++) {
        cdf += p[i];
        if (r < cdf) { tok = i; break; }
    }
    free(p);
    return tok;
}

/* ------------------------------------------------------------------ */
/* Cross-entropy (src/ops.c:499-574, the scalar branch 549-573)        */
/* ------------------------------------------------------------------ */

float orc_cross_entropy(const float *logits, const int *targets, float *probs,
                        float *row_loss, int B, int T, int V)
{
    const int BT = B * T;
    float loss = 0.0f;
    for (int bt = 0; bt < BT; bt++) {
        const float *lg = logits + (size_t)bt * V;
        float mx = -FLT_MAX;                              /* ops.c:553-555 */
        for (int v = 0; v < V; v++) if (lg[v] > mx) mx = lg[v];
        float sum = 0.0f;                                 /* ops.c:557-561 */
        for (int v = 0; v < V; v++) {
            float e = expf(lg[v] - mx);
            if (probs) probs[(size_t)bt * V + v] = e;
            sum += e;
        }
        const float log_sum = logf(sum);                  /* ops.c:562-565 */
        if (probs) {
            const float inv = 1.0f / sum;
            for (int v = 0; v < V; v++) probs[(size_t)bt * V + v] *= inv;
        }
        const float term = (lg[targets[bt]] - mx) - log_sum;  /* ops.c:567-568 */
        if (row_loss) row_loss[bt] = -term;
        loss -= term;
    }
    return loss / (float)BT;                              /* ops.c:573 */
}

/* ------------------------------------------------------------------ */
/* Training: gpt_forward with targets, gpt_backward, gpt_adamw         */
/* (src/model.c:442-921) and the backward ops of src/ops.c, scalar     */
/* paths, with the residual-stream dropout of model.c:471-472,         */
/* 572-574, 597-599 when a rate is set (orc_train_set_dropout).        */
/* ------------------------------------------------------------------ */

/* dropout_fwd (ops.c:603-618): one rand() per element, kept when it
 * exceeds p * RAND_MAX, kept values scaled by 1 / (1 - p). */
void orc_dropout_fwd(float *x, unsigned char *mask, long n, float p)
{
    const float scale = 1.0f / (1.0f - p);
    for (long i = 0; i < n; i++) {
        const unsigned int r = (unsigned int)rand();
        const unsigned char keep = (r > (unsigned int)(p * (float)RAND_MAX)) ? 1 : 0;
        mask[i] = keep;
        x[i] *= keep ? scale : 0.0f;
    }
}

/* dropout_bwd (ops.c:620-625). */
void orc_dropout_bwd(float *dx, const unsigned char *mask, long n, float p)
{
    const float scale = 1.0f / (1.0f - p);
    for (long i = 0; i < n; i++) dx[i] *= mask[i] ? scale : 0.0f;
}

void orc_linear_bwd_dx(const float *dY, const float *W, float *dX, int M, int K, int N)
{                                                       /* ops.c:125-133 */
    /* dX [M,K] += dY [M,N] . W [N,K] */
    sgemm_t(NO_TRANS, NO_TRANS, M, K, N, 1.0f, dY, N, W, K, 1.0f, dX, K);
}

void orc_linear_bwd_dw(const float *dY, const float *X, float *dW, float *db, int M, int K, int N)
{                                                       /* ops.c:135-153 */
    /* dW [N,K] += dY^T [N,M] . X [M,K] */
    sgemm_t(TRANS, NO_TRANS, N, K, M, 1.0f, dY, N, X, K, 1.0f, dW, K);
    if (db)
        for (int i = 0; i < M; i++)
            for (int j = 0; j < N; j++) db[j] += dY[(size_t)i * N + j];
}

void orc_layernorm_bwd(const float *dout, const float *x, const float *w, const float *mean,
                       const float *rstd, float *dx, float *dw, float *db, int T, int C)
{                                                       /* ops.c:310-331 (scalar path) */
    for (int t = 0; t < T; t++) {
        const float *doutr = dout + (size_t)t * C;
        const float *xr = x + (size_t)t * C;
        float *dxr = dx + (size_t)t * C;
        const float m = mean[t], rs = rstd[t];
        float sum1 = 0.0f, sum2 = 0.0f;
        for (int c = 0; c < C; c++) {
            const float xhat = (xr[c] - m) * rs;
            const float dn = doutr[c] * w[c];
            sum1 += dn;
            sum2 += dn * xhat;
        }
        sum1 /= (float)C;
        sum2 /= (float)C;
        for (int c = 0; c < C; c++) {
            const float xhat = (xr[c] - m) * rs;
            const float dn = doutr[c] * w[c];
            dxr[c] += rs * (dn - sum1 - xhat * sum2);
            dw[c] += doutr[c] * xhat;
            db[c] += doutr[c];
        }
    }
}

static inline float gelu_grad1(float x)                 /* ops.c:347-355 */
{
    const float x3 = x * x * x;
    const float inner = 0.7978845608028654f * (x + 0.044715f * x3);
    const float tv = tanhf(inner);
    const float sech2 = 1.0f - tv * tv;
    const float dinner = 0.7978845608028654f * (1.0f + 3.0f * 0.044715f * x * x);
    return 0.5f * (1.0f + tv) + 0.5f * x * sech2 * dinner;
}

void orc_gelu_bwd(const float *dout, const float *x, float *dx, int n)
{                                                       /* ops.c:382-422 (scalar path) */
    for (int i = 0; i < n; i++) dx[i] += dout[i] * gelu_grad1(x[i]);
}

/* Activations gpt_forward keeps for gpt_backward (GPTActivations,
 * src/model.h:86-115), for one B x T shape. */
struct orc_train {
    orc_cfg c;
    int B, T;
    float *emb, *ln_f_out, *ln_f_mean, *ln_f_rstd, *logits, *probs;
    float **ln1_out, **ln1_mean, **ln1_rstd, **qkv, **attn_probs, **attn_out, **attn_proj;
    float **res1, **ln2_out, **ln2_mean, **ln2_rstd, **fc_out, **gelu, **mlp_out, **res2;
    float dropout;                   /* GPTConfig.dropout (model.h:43); 0: none */
    unsigned char *masks;            /* [1 + 2 L][B T C]: emb, then res1, res2 per layer */
    int dropped;                     /* the last forward applied them */
};

static float **alloc_layers(int L, size_t n, int *ok)
{
    float **p = calloc((size_t)L, sizeof(float *));
    if (!p) { *ok = 0; return NULL; }
    for (int l = 0; l < L; l++)
        if (!(p[l] = malloc(n * sizeof(float)))) *ok = 0;
    return p;
}

static void free_layers(float **p, int L)
{
    if (!p) return;
    for (int l = 0; l < L; l++) free(p[l]);
    free(p);
}

void orc_train_free(orc_train *t)
{
    if (!t) return;
    const int L = t->c.n_layer;
    free(t->emb); free(t->ln_f_out); free(t->ln_f_mean); free(t->ln_f_rstd);
    free(t->logits); free(t->probs);
    float **all[] = { t->ln1_out, t->ln1_mean, t->ln1_rstd, t->qkv, t->attn_probs, t->attn_out,
                      t->attn_proj, t->res1, t->ln2_out, t->ln2_mean, t->ln2_rstd, t->fc_out,
                      t->gelu, t->mlp_out, t->res2 };
    for (size_t i = 0; i < sizeof(all) / sizeof(all[0]); i++) free_layers(all[i], L);
    free(t->masks);
    free(t);
}

int orc_train_set_dropout(orc_train *t, float p)
{
    if (!t || !(p >= 0.0f) || !(p < 1.0f)) return -1;
    if (p > 0.0f && !t->masks) {
        const size_t n = (size_t)(1 + 2 * t->c.n_layer) * t->B * t->T * t->c.n_embd;
        if (!(t->masks = malloc(n))) return -1;
    }
    t->dropout = p;
    return 0;
}

const unsigned char *orc_train_masks(const orc_train *t) { return t ? t->masks : NULL; }

orc_train *orc_train_new(const orc_cfg *c, int B, int T)
{                                                       /* model.c:333-440 */
    if (!c || B <= 0 || T <= 0 || T > c->block_size || c->n_embd % c->n_head) return NULL;
    orc_train *t = calloc(1, sizeof(*t));
    if (!t) return NULL;
    t->c = *c;
    t->B = B;
    t->T = T;
    const int L = c->n_layer, C = c->n_embd, H = c->n_head;
    const size_t N = (size_t)B * T, V = (size_t)c->vocab_size;
    int ok = 1;
    t->emb = malloc(N * C * sizeof(float));
    t->ln_f_out = malloc(N * C * sizeof(float));
    t->ln_f_mean = malloc(N * sizeof(float));
    t->ln_f_rstd = malloc(N * sizeof(float));
    t->logits = malloc(N * V * sizeof(float));
    t->probs = malloc(N * V * sizeof(float));
    ok = t->emb && t->ln_f_out && t->ln_f_mean && t->ln_f_rstd && t->logits && t->probs;
    t->ln1_out = alloc_layers(L, N * C, &ok);
    t->ln1_mean = alloc_layers(L, N, &ok);
    t->ln1_rstd = alloc_layers(L, N, &ok);
    t->qkv = alloc_layers(L, N * 3 * C, &ok);
    t->attn_probs = alloc_layers(L, (size_t)B * H * T * T, &ok);
    t->attn_out = alloc_layers(L, N * C, &ok);
    t->attn_proj = alloc_layers(L, N * C, &ok);
    t->res1 = alloc_layers(L, N * C, &ok);
    t->ln2_out = alloc_layers(L, N * C, &ok);
    t->ln2_mean = alloc_layers(L, N, &ok);
    t->ln2_rstd = alloc_layers(L, N, &ok);
    t->fc_out = alloc_layers(L, N * 4 * C, &ok);
    t->gelu = alloc_layers(L, N * 4 * C, &ok);
    t->mlp_out = alloc_layers(L, N * C, &ok);
    t->res2 = alloc_layers(L, N * C, &ok);
    if (!ok) { orc_train_free(t); return NULL; }
    return t;
}

/* linear_fwd (ops.c:109-123): Y = X . W^T, then b added row by row. */
static void linear_seq(const float *X, const float *W, const float *b, float *Y, int M, int K,
                       int N)
{
    sgemm(TRANS, M, N, K, 1.0f, X, K, W, K, 0.0f, Y, N);
    if (b)
        for (int i = 0; i < M; i++)
            for (int j = 0; j < N; j++) Y[(size_t)i * N + j] += b[j];
}

float orc_train_forward(orc_train *t, const float *params, const int *tokens, const int *targets)
{                                                       /* model.c:442-625 */
    const orc_cfg *c = &t->c;
    const int B = t->B, T = t->T, C = c->n_embd, V = c->vocab_size, L = c->n_layer;
    const int H = c->n_head, hs = C / H;
    const size_t N = (size_t)B * T;
    long *off = malloc(sizeof(long) * (size_t)(4 + 12 * L));
    float *Qh = malloc((size_t)T * hs * sizeof(float)), *Kh = malloc((size_t)T * hs * sizeof(float));
    float *Vh = malloc((size_t)T * hs * sizeof(float)), *oh = malloc((size_t)T * hs * sizeof(float));
    float *sc = malloc((size_t)T * T * sizeof(float));
    orc_offsets(c, off);
    const float *wte = params + off[0], *wpe = params + off[1];
    for (int b = 0; b < B; b++)                           /* model.c:458-471 */
        for (int p = 0; p < T; p++) {
            const float *e = wte + (size_t)tokens[b * T + p] * C, *q = wpe + (size_t)p * C;
            float *d = t->emb + ((size_t)b * T + p) * C;
            for (int k = 0; k < C; k++) d[k] = e[k] + q[k];
        }
    /* model.c:450: dropout only in a forward with targets */
    const int drop = targets != NULL && t->dropout > 0.0f;
    const size_t NC = N * (size_t)C;
    t->dropped = drop;
    if (drop) orc_dropout_fwd(t->emb, t->masks, (long)NC, t->dropout);   /* model.c:471-472 */
    const float *x = t->emb;
    const float scale = 1.0f / sqrtf((float)hs);
    for (int l = 0; l < L; l++) {
        const long *o = off + 2 + 12 * l;
        orc_layernorm(x, params + o[0], params + o[1], t->ln1_out[l], t->ln1_mean[l],
                      t->ln1_rstd[l], (int)N, C);
        linear_seq(t->ln1_out[l], params + o[2], params + o[3], t->qkv[l], (int)N, C, 3 * C);
        for (int b = 0; b < B; b++)                       /* model.c:510-566 */
            for (int h = 0; h < H; h++) {
                float *pr = t->attn_probs[l] + ((size_t)b * H + h) * T * T;
                for (int p = 0; p < T; p++) {
                    const float *row = t->qkv[l] + ((size_t)b * T + p) * 3 * C;
                    memcpy(Qh + (size_t)p * hs, row + h * hs, hs * sizeof(float));
                    memcpy(Kh + (size_t)p * hs, row + C + h * hs, hs * sizeof(float));
                    memcpy(Vh + (size_t)p * hs, row + 2 * C + h * hs, hs * sizeof(float));
                }
                sgemm(TRANS, T, T, hs, scale, Qh, hs, Kh, hs, 0.0f, sc, T);
                orc_causal_mask(sc, T);
                memcpy(pr, sc, (size_t)T * T * sizeof(float));
                orc_softmax_inplace(pr, T, T);
                sgemm(NO_TRANS, T, hs, T, 1.0f, pr, T, Vh, hs, 0.0f, oh, hs);
                for (int p = 0; p < T; p++)
                    memcpy(t->attn_out[l] + ((size_t)b * T + p) * C + h * hs, oh + (size_t)p * hs,
                           hs * sizeof(float));
            }
        linear_seq(t->attn_out[l], params + o[4], params + o[5], t->attn_proj[l], (int)N, C, C);
        for (size_t i = 0; i < N * C; i++) t->res1[l][i] = x[i] + t->attn_proj[l][i];   /* :572-573 */
        if (drop) orc_dropout_fwd(t->res1[l], t->masks + (1 + 2 * (size_t)l) * NC, (long)NC,
                                  t->dropout);                              /* :573-574 */
        orc_layernorm(t->res1[l], params + o[6], params + o[7], t->ln2_out[l], t->ln2_mean[l],
                      t->ln2_rstd[l], (int)N, C);
        linear_seq(t->ln2_out[l], params + o[8], params + o[9], t->fc_out[l], (int)N, C, 4 * C);
        orc_gelu(t->fc_out[l], t->gelu[l], (int)(N * 4 * C));
        linear_seq(t->gelu[l], params + o[10], params + o[11], t->mlp_out[l], (int)N, 4 * C, C);
        for (size_t i = 0; i < N * C; i++) t->res2[l][i] = t->res1[l][i] + t->mlp_out[l][i];  /* :597-598 */
        if (drop) orc_dropout_fwd(t->res2[l], t->masks + (2 + 2 * (size_t)l) * NC, (long)NC,
                                  t->dropout);                              /* :598-599 */
        x = t->res2[l];
    }
    const long *of = off + 2 + 12 * L;                    /* model.c:608-614 */
    orc_layernorm(x, params + of[0], params + of[1], t->ln_f_out, t->ln_f_mean, t->ln_f_rstd,
                  (int)N, C);
    linear_seq(t->ln_f_out, wte, NULL, t->logits, (int)N, C, V);
    free(off); free(Qh); free(Kh); free(Vh); free(oh); free(sc);
    if (!targets) return 0.0f;                            /* model.c:619-624 */
    return orc_cross_entropy(t->logits, targets, t->probs, NULL, B, T, V);
}

void orc_train_backward(orc_train *t, const float *params, const int *tokens, const int *targets,
                        float *grads)
{                                                       /* model.c:634-877 */
    const orc_cfg *c = &t->c;
    const int B = t->B, T = t->T, C = c->n_embd, V = c->vocab_size, L = c->n_layer;
    const int H = c->n_head, hs = C / H;
    const size_t N = (size_t)B * T;
    const float scale = 1.0f / (float)(B * T);
    long *off = malloc(sizeof(long) * (size_t)(4 + 12 * L));
    orc_offsets(c, off);
    float *dlogits = calloc(N * V, sizeof(float)), *d_ln_f = calloc(N * C, sizeof(float));
    float *d_x = calloc(N * C, sizeof(float)), *d_res1 = calloc(N * C, sizeof(float));
    float *d_ln2 = calloc(N * C, sizeof(float)), *d_mlp4 = calloc(N * 4 * C, sizeof(float));
    float *d_gelu = calloc(N * 4 * C, sizeof(float)), *d_ln1 = calloc(N * C, sizeof(float));
    float *d_qkv = calloc(N * 3 * C, sizeof(float)), *d_attn_o = calloc(N * C, sizeof(float));
    float *Qh = malloc((size_t)T * hs * sizeof(float)), *Kh = malloc((size_t)T * hs * sizeof(float));
    float *Vh = malloc((size_t)T * hs * sizeof(float)), *d_o_h = malloc((size_t)T * hs * sizeof(float));
    float *d_V_h = malloc((size_t)T * hs * sizeof(float)), *d_p = malloc((size_t)T * T * sizeof(float));
    float *d_Q_h = malloc((size_t)T * hs * sizeof(float)), *d_K_h = malloc((size_t)T * hs * sizeof(float));
    const float *wte = params + off[0];
    float *g_wte = grads + off[0], *g_wpe = grads + off[1];

    for (size_t bt = 0; bt < N; bt++)                     /* ops.c:576-589 via model.c:665 */
        for (int v = 0; v < V; v++)
            dlogits[bt * V + v] += scale * (t->probs[bt * V + v] - (v == targets[bt] ? 1.0f : 0.0f));
    orc_linear_bwd_dx(dlogits, wte, d_ln_f, (int)N, C, V);                /* model.c:673-675 */
    orc_linear_bwd_dw(dlogits, t->ln_f_out, g_wte, NULL, (int)N, C, V);
    const long *of = off + 2 + 12 * L;
    orc_layernorm_bwd(d_ln_f, L > 0 ? t->res2[L - 1] : t->emb, params + of[0], t->ln_f_mean,
                      t->ln_f_rstd, d_x, grads + of[0], grads + of[1], (int)N, C);

    for (int l = L - 1; l >= 0; l--) {                    /* model.c:690-857 */
        const long *o = off + 2 + 12 * l;
        const float *x_in = l == 0 ? t->emb : t->res2[l - 1];
        if (t->dropped)                                   /* model.c:699-700 */
            orc_dropout_bwd(d_x, t->masks + (2 + 2 * (size_t)l) * N * C, (long)(N * C), t->dropout);
        memcpy(d_res1, d_x, N * C * sizeof(float));
        memset(d_gelu, 0, N * 4 * C * sizeof(float));
        orc_linear_bwd_dx(d_x, params + o[10], d_gelu, (int)N, 4 * C, C);
        orc_linear_bwd_dw(d_x, t->gelu[l], grads + o[10], grads + o[11], (int)N, 4 * C, C);
        memset(d_mlp4, 0, N * 4 * C * sizeof(float));
        orc_gelu_bwd(d_gelu, t->fc_out[l], d_mlp4, (int)(N * 4 * C));
        memset(d_ln2, 0, N * C * sizeof(float));
        orc_linear_bwd_dx(d_mlp4, params + o[8], d_ln2, (int)N, C, 4 * C);
        orc_linear_bwd_dw(d_mlp4, t->ln2_out[l], grads + o[8], grads + o[9], (int)N, C, 4 * C);
        orc_layernorm_bwd(d_ln2, t->res1[l], params + o[6], t->ln2_mean[l], t->ln2_rstd[l],
                          d_res1, grads + o[6], grads + o[7], (int)N, C);
        if (t->dropped)                                   /* model.c:732-733 */
            orc_dropout_bwd(d_res1, t->masks + (1 + 2 * (size_t)l) * N * C, (long)(N * C),
                            t->dropout);
        memset(d_attn_o, 0, N * C * sizeof(float));
        orc_linear_bwd_dx(d_res1, params + o[4], d_attn_o, (int)N, C, C);
        orc_linear_bwd_dw(d_res1, t->attn_out[l], grads + o[4], grads + o[5], (int)N, C, C);
        memset(d_qkv, 0, N * 3 * C * sizeof(float));
        const float sc = 1.0f / sqrtf((float)hs);
        for (int b = 0; b < B; b++)                       /* model.c:747-818 */
            for (int h = 0; h < H; h++) {
                const float *pr = t->attn_probs[l] + ((size_t)b * H + h) * T * T;
                for (int p = 0; p < T; p++) {
                    const float *qr = t->qkv[l] + ((size_t)b * T + p) * 3 * C;
                    memcpy(Qh + (size_t)p * hs, qr + h * hs, hs * sizeof(float));
                    memcpy(Kh + (size_t)p * hs, qr + C + h * hs, hs * sizeof(float));
                    memcpy(Vh + (size_t)p * hs, qr + 2 * C + h * hs, hs * sizeof(float));
                    memcpy(d_o_h + (size_t)p * hs, d_attn_o + ((size_t)b * T + p) * C + h * hs,
                           hs * sizeof(float));
                }
                memset(d_V_h, 0, (size_t)T * hs * sizeof(float));
                memset(d_p, 0, (size_t)T * T * sizeof(float));
                memset(d_Q_h, 0, (size_t)T * hs * sizeof(float));
                memset(d_K_h, 0, (size_t)T * hs * sizeof(float));
                sgemm_t(TRANS, NO_TRANS, T, hs, T, 1.0f, pr, T, d_o_h, hs, 1.0f, d_V_h, hs);
                sgemm_t(NO_TRANS, TRANS, T, T, hs, 1.0f, d_o_h, hs, Vh, hs, 0.0f, d_p, T);
                for (int p = 0; p < T; p++) {             /* model.c:787-795 */
                    const float *prr = pr + (size_t)p * T;
                    float *dp = d_p + (size_t)p * T;
                    float dot = 0.0f;
                    for (int q = 0; q <= p; q++) dot += prr[q] * dp[q];
                    for (int q = 0; q <= p; q++) dp[q] = prr[q] * (dp[q] - dot);
                    for (int q = p + 1; q < T; q++) dp[q] = 0.0f;
                }
                sgemm_t(NO_TRANS, NO_TRANS, T, hs, T, sc, d_p, T, Kh, hs, 1.0f, d_Q_h, hs);
                sgemm_t(TRANS, NO_TRANS, T, hs, T, sc, d_p, T, Qh, hs, 1.0f, d_K_h, hs);
                for (int p = 0; p < T; p++) {
                    float *dqr = d_qkv + ((size_t)b * T + p) * 3 * C;
                    for (int i = 0; i < hs; i++) {
                        dqr[h * hs + i] += d_Q_h[(size_t)p * hs + i];
                        dqr[C + h * hs + i] += d_K_h[(size_t)p * hs + i];
                        dqr[2 * C + h * hs + i] += d_V_h[(size_t)p * hs + i];
                    }
                }
            }
        memset(d_ln1, 0, N * C * sizeof(float));          /* model.c:822-841 */
        orc_linear_bwd_dx(d_qkv, params + o[2], d_ln1, (int)N, C, 3 * C);
        orc_linear_bwd_dw(d_qkv, t->ln1_out[l], grads + o[2], grads + o[3], (int)N, C, 3 * C);
        memset(d_x, 0, N * C * sizeof(float));
        orc_layernorm_bwd(d_ln1, x_in, params + o[0], t->ln1_mean[l], t->ln1_rstd[l], d_x,
                          grads + o[0], grads + o[1], (int)N, C);
        for (size_t i = 0; i < N * C; i++) d_x[i] += d_res1[i];
    }
    if (t->dropped) orc_dropout_bwd(d_x, t->masks, (long)(N * C), t->dropout);  /* model.c:849-850 */
    for (int b = 0; b < B; b++)                           /* model.c:850-866 */
        for (int p = 0; p < T; p++) {
            const float *dr = d_x + ((size_t)b * T + p) * C;
            for (int k = 0; k < C; k++) g_wpe[(size_t)p * C + k] += dr[k];
        }
    for (int b = 0; b < B; b++)
        for (int p = 0; p < T; p++) {
            const float *dr = d_x + ((size_t)b * T + p) * C;
            float *gw = g_wte + (size_t)tokens[b * T + p] * C;
            for (int k = 0; k < C; k++) gw[k] += dr[k];
        }
    free(off); free(dlogits); free(d_ln_f); free(d_x); free(d_res1); free(d_ln2); free(d_mlp4);
    free(d_gelu); free(d_ln1); free(d_qkv); free(d_attn_o); free(Qh); free(Kh); free(Vh);
    free(d_o_h); free(d_V_h); free(d_p); free(d_Q_h); free(d_K_h);
}

/* The weight-decay mask of gpt_init (src/model.c:143-172): matrices and
 * embeddings (wte, wpe, c_attn_w, c_proj_w, mlp_fc_w, mlp_proj_w) decay,
 * LayerNorm gains and all biases do not. */
static unsigned char *decay_mask(const orc_cfg *c, const long *off, long n)
{
    unsigned char *d = calloc((size_t)n, 1);
    if (!d) return NULL;
    memset(d, 1, (size_t)off[2]);                         /* wte, wpe */
    for (int l = 0; l < c->n_layer; l++) {
        const long *o = off + 2 + 12 * l;
        memset(d + o[2], 1, (size_t)(o[3] - o[2]));       /* c_attn_w */
        memset(d + o[4], 1, (size_t)(o[5] - o[4]));       /* c_proj_w */
        memset(d + o[8], 1, (size_t)(o[9] - o[8]));       /* mlp_fc_w */
        memset(d + o[10], 1, (size_t)(o[11] - o[10]));    /* mlp_proj_w */
    }
    return d;
}

void orc_adamw(const orc_cfg *c, float *params, float *grads, float *m, float *v, int step,
               float lr, float beta1, float beta2, float eps, float wd, float grad_clip)
{                                                       /* model.c:888-921 */
    const long n = orc_num_params(c);
    long *off = malloc(sizeof(long) * (size_t)(4 + 12 * c->n_layer));
    orc_offsets(c, off);
    unsigned char *dmask = decay_mask(c, off, n);
    if (grad_clip > 0.0f) {                               /* ops.c:631-640 */
        /* the reference's cblas_snrm2; here the sum of squares in double */
        double ss = 0.0;
        for (long i = 0; i < n; i++) ss += (double)grads[i] * grads[i];
        const float norm = (float)sqrt(ss);
        if (norm > grad_clip) {
            const float s = grad_clip / norm;
            for (long i = 0; i < n; i++) grads[i] *= s;
        }
    }
    const float bc1 = 1.0f - powf(beta1, (float)step);
    const float bc2 = 1.0f - powf(beta2, (float)step);
    for (long i = 0; i < n; i++) {
        const float g = grads[i];
        m[i] = beta1 * m[i] + (1.0f - beta1) * g;
        v[i] = beta2 * v[i] + (1.0f - beta2) * g * g;
        const float m_hat = m[i] / bc1;
        const float v_hat = v[i] / bc2;
        const float ewd = dmask[i] ? wd : 0.0f;
        params[i] = params[i] * (1.0f - lr * ewd) - lr * m_hat / (sqrtf(v_hat) + eps);
    }
    free(dmask);
    free(off);
}
