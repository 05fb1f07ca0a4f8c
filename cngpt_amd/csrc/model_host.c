/*
 * model_host.c - the parameter side of the model API (include/model.h):
 * parameter count, flat-buffer layout, seeded init, weight-file load/save.
 *
 * The gpt_* functions are weak so that a program linking the reference's
 * model.c keeps the reference's definitions. cngpt_hip_init_weights is the
 * seeded init used to make synthetic weights without a GPT struct.
 */
#define _GNU_SOURCE
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/cngpt_hip.h"
#include "../../include/model.h"

#define WEAK __attribute__((weak))

static long num_params_long(const GPTConfig *c)           /* model.c:20-48 */
{
    long C = c->n_embd, V = c->vocab_size, T = c->block_size, L = c->n_layer;
    long per_layer = 2 * C + 3 * C * C + 3 * C + C * C + C + 2 * C + 4 * C * C + 4 * C +
                     4 * C * C + C;
    return V * C + T * C + L * per_layer + 2 * C;
}

WEAK int gpt_num_params(const GPTConfig *cfg) { return (int)num_params_long(cfg); }

/* Pointer carving in the export order of src/model.c:54-83. */
static void carve(GPTWeights *w, float *buf, const GPTConfig *c)
{
    long C = c->n_embd, V = c->vocab_size, T = c->block_size;
    float *p = buf;
    w->wte = p; p += V * C;
    w->wpe = p; p += T * C;
    for (int l = 0; l < c->n_layer; l++) {
        w->ln1_w[l] = p;      p += C;
        w->ln1_b[l] = p;      p += C;
        w->c_attn_w[l] = p;   p += 3 * C * C;
        w->c_attn_b[l] = p;   p += 3 * C;
        w->c_proj_w[l] = p;   p += C * C;
        w->c_proj_b[l] = p;   p += C;
        w->ln2_w[l] = p;      p += C;
        w->ln2_b[l] = p;      p += C;
        w->mlp_fc_w[l] = p;   p += 4 * C * C;
        w->mlp_fc_b[l] = p;   p += 4 * C;
        w->mlp_proj_w[l] = p; p += C * 4 * C;
        w->mlp_proj_b[l] = p; p += C;
    }
    w->ln_f_w = p; p += C;
    w->ln_f_b = p;
}

static int alloc_ptrs(GPTWeights *w, int L)
{
    float ***slots[12] = { &w->ln1_w, &w->ln1_b, &w->c_attn_w, &w->c_attn_b,
                           &w->c_proj_w, &w->c_proj_b, &w->ln2_w, &w->ln2_b,
                           &w->mlp_fc_w, &w->mlp_fc_b, &w->mlp_proj_w, &w->mlp_proj_b };
    int ok = 1;
    for (int i = 0; i < 12; i++) {
        *slots[i] = calloc((size_t)L, sizeof(float *));
        ok = ok && *slots[i];
    }
    return ok ? 0 : -1;
}

static void free_ptrs(GPTWeights *w)
{
    free(w->ln1_w); free(w->ln1_b); free(w->c_attn_w); free(w->c_attn_b);
    free(w->c_proj_w); free(w->c_proj_b); free(w->ln2_w); free(w->ln2_b);
    free(w->mlp_fc_w); free(w->mlp_fc_b); free(w->mlp_proj_w); free(w->mlp_proj_b);
}

WEAK int gpt_init(GPT *m, GPTConfig cfg)                    /* model.c:120-175 */
{
    memset(m, 0, sizeof(*m));
    m->cfg = cfg;
    if (cfg.n_layer <= 0 || alloc_ptrs(&m->params, cfg.n_layer) != 0) return -1;
    long n = num_params_long(&cfg);
    if (n <= 0 || n > 0x7fffffffL) return -1;
    m->n_params = (int)n;
    m->param_buf = calloc((size_t)n, sizeof(float));
    if (!m->param_buf) return -1;
    carve(&m->params, m->param_buf, &cfg);
    return 0;
}

/* Box-Muller over rand(), model.c:275-284 (one variate per accepted pair). */
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

static void fill_normal(float *p, long n, float std)
{
    for (long i = 0; i < n; i++) p[i] = randn() * std;
}

static void fill_const(float *p, long n, float v)
{
    for (long i = 0; i < n; i++) p[i] = v;
}

/* Draw order of gpt_init_weights, model.c:292-331. */
static void init_draws(GPTWeights *w, const GPTConfig *c)
{
    long C = c->n_embd, V = c->vocab_size;
    float std = 0.02f;
    float res_std = 0.02f / sqrtf(2.0f * (float)c->n_layer);
    fill_normal(w->wte, V * C, std);
    fill_normal(w->wpe, (long)c->block_size * C, std);
    for (int l = 0; l < c->n_layer; l++) {
        fill_const(w->ln1_w[l], C, 1.0f);
        fill_const(w->ln1_b[l], C, 0.0f);
        fill_const(w->ln2_w[l], C, 1.0f);
        fill_const(w->ln2_b[l], C, 0.0f);
        fill_normal(w->c_attn_w[l], 3 * C * C, std);
        fill_const(w->c_attn_b[l], 3 * C, 0.0f);
        fill_normal(w->c_proj_w[l], C * C, res_std);
        fill_const(w->c_proj_b[l], C, 0.0f);
        fill_normal(w->mlp_fc_w[l], 4 * C * C, std);
        fill_const(w->mlp_fc_b[l], 4 * C, 0.0f);
        fill_normal(w->mlp_proj_w[l], C * 4 * C, res_std);
        fill_const(w->mlp_proj_b[l], C, 0.0f);
    }
    fill_const(w->ln_f_w, C, 1.0f);
    fill_const(w->ln_f_b, C, 0.0f);
}

WEAK void gpt_init_weights(GPT *m) { init_draws(&m->params, &m->cfg); }

WEAK int gpt_load(GPT *m, const char *path)                /* model.c:177-211 */
{
    FILE *f = fopen(path, "rb");
    if (!f) { perror(path); return -1; }
    GPTHeader hdr;
    if (fread(&hdr, sizeof(hdr), 1, f) != 1) {
        fprintf(stderr, "gpt_load: %s ends inside its %zu-byte header\n", path, sizeof(hdr));
        fclose(f);
        return -1;
    }
    if (hdr.magic != CNGPT_MAGIC) {
        fprintf(stderr, "gpt_load: %s is not a cngpt weight file (first word 0x%X)\n", path, hdr.magic);
        fclose(f);
        return -1;
    }
    GPTConfig cfg = { hdr.n_layer, hdr.n_head, hdr.n_embd, hdr.vocab_size, hdr.block_size, 0.0f };
    if (m->param_buf == NULL) {
        if (gpt_init(m, cfg) != 0) { fclose(f); return -1; }
    } else if (m->cfg.n_layer != cfg.n_layer || m->cfg.n_head != cfg.n_head ||
               m->cfg.n_embd != cfg.n_embd || m->cfg.vocab_size != cfg.vocab_size ||
               m->cfg.block_size != cfg.block_size) {
        fprintf(stderr, "gpt_load: %s holds a different shape than the model\n", path);
        fclose(f);
        return -1;
    }
    size_t n = (size_t)m->n_params;
    if (fread(m->param_buf, sizeof(float), n, f) != n) {
        fprintf(stderr, "gpt_load: %s ends before its %zu parameters\n", path, n);
        fclose(f);
        return -1;
    }
    fclose(f);
    return 0;
}

WEAK int gpt_save(GPT *m, const char *path)                /* model.c:213-231 */
{
    FILE *f = fopen(path, "wb");
    if (!f) { perror(path); return -1; }
    GPTHeader hdr = { CNGPT_MAGIC, CNGPT_VERSION, m->cfg.n_layer, m->cfg.n_head,
                      m->cfg.n_embd, m->cfg.vocab_size, m->cfg.block_size };
    int ok = fwrite(&hdr, sizeof(hdr), 1, f) == 1 &&
             fwrite(m->param_buf, sizeof(float), (size_t)m->n_params, f) == (size_t)m->n_params;
    return (fclose(f) == 0 && ok) ? 0 : -1;
}

WEAK void gpt_free(GPT *m)                                  /* model.c:233-259 */
{
    free(m->param_buf);
    free(m->grad_buf);
    free(m->m_buf);
    free(m->v_buf);
    free(m->decay_buf);
    free(m->act_buf);
    free(m->mask_buf);
    free_ptrs(&m->params);
    free_ptrs(&m->grads);
    memset(m, 0, sizeof(*m));
}

int cngpt_hip_init_weights(const cngpt_hip_config *cfg, float *params, unsigned seed)
{
    if (!cfg || !params || cfg->n_layer <= 0) return -1;
    GPTConfig c = { cfg->n_layer, cfg->n_head, cfg->n_embd, cfg->vocab_size, cfg->block_size,
                    0.0f };
    GPTWeights w;
    memset(&w, 0, sizeof(w));
    if (alloc_ptrs(&w, c.n_layer) != 0) { free_ptrs(&w); return -1; }
    carve(&w, params, &c);
    srand(seed);
    init_draws(&w, &c);
    free_ptrs(&w);
    return 0;
}
