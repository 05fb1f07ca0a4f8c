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
