/*
 * fast.c - the fast.h entry points (reference src/fast.h:47-60) on top of
 * the cngpt_hip C ABI. Plain C, no HIP headers.
 */
#include <stdlib.h>
#include <string.h>

#include "../../include/cngpt_hip.h"
#include "../../include/fast.h"

static __thread char g_fast_err[512];

static void set_err(const char *msg)
{
    strncpy(g_fast_err, msg ? msg : "", sizeof(g_fast_err) - 1);
    g_fast_err[sizeof(g_fast_err) - 1] = '\0';
}

const char *fast_last_error(void) { return g_fast_err; }

void fast_init(FastCtx *f)                          /* fast.c:29-32 */
{
    memset(f, 0, sizeof(*f));
}

void fast_free(FastCtx *f)                          /* fast.c:34-40 */
{
    if (f->dev) cngpt_hip_destroy((cngpt_hip_ctx *)f->dev);
    if (f->logits) cngpt_hip_host_free(f->logits);
    memset(f, 0, sizeof(*f));
}

/* fast.c:97-101 picks the OpenMP team size; the device path has none. */
void fast_set_threads(int n) { (void)n; }

void fast_params_changed(FastCtx *f) { f->params_dirty = 1; }

static int device_index(void)
{
    const char *s = getenv("CNGPT_HIP_DEVICE");
    return s && *s ? atoi(s) : 0;
}

/* Create the device handle on first use and upload the parameters when the
 * caller's buffer, count or shape changed. */
static int prepare(GPT *m, FastCtx *f)
{
    if (!f->dev) {
        cngpt_hip_ctx *h = NULL;
        if (cngpt_hip_create(device_index(), &h) != 0) {
            set_err(cngpt_hip_last_error());
            return -1;
        }
        f->dev = h;
        f->params_dirty = 1;
    }
    if (f->params_dirty || f->params_seen != m->param_buf || f->n_params_seen != m->n_params ||
        memcmp(&f->cfg_seen, &m->cfg, sizeof(GPTConfig)) != 0) {
        cngpt_hip_config c = { m->cfg.n_layer, m->cfg.n_head, m->cfg.n_embd,
                               m->cfg.vocab_size, m->cfg.block_size };
        if (cngpt_hip_load_params((cngpt_hip_ctx *)f->dev, &c, m->param_buf,
                                  (long)m->n_params) != 0) {
            set_err(cngpt_hip_last_error());
            return -1;
        }
        f->params_seen = m->param_buf;
        f->n_params_seen = m->n_params;
        f->cfg_seen = m->cfg;
        f->params_dirty = 0;
    }
    return 0;
}

static float *logits_buffer(FastCtx *f, size_t n)
{
    if (f->logits && f->logits_cap >= n) return f->logits;
    if (f->logits) cngpt_hip_host_free(f->logits);
    f->logits = (float *)cngpt_hip_host_alloc(n * sizeof(float));
    f->logits_cap = f->logits ? n : 0;
    if (!f->logits) set_err(cngpt_hip_last_error());
    return f->logits;
}

static const float *forward(GPT *m, FastCtx *f, const int *tokens, int B, int T, int mode)
{
    if (!m || !f || !tokens || B <= 0 || T <= 0) {
        set_err("gpt_forward_fast: bad arguments");
        return NULL;
    }
    if (prepare(m, f) != 0) return NULL;
    size_t n = (size_t)B * (mode == CNGPT_ALL ? (size_t)T : 1) * (size_t)m->cfg.vocab_size;
    float *out = logits_buffer(f, n);
    if (!out) return NULL;
    if (cngpt_hip_forward((cngpt_hip_ctx *)f->dev, tokens, B, T, mode, out) != 0) {
        set_err(cngpt_hip_last_error());
        return NULL;
    }
    f->B = B;
    f->T = T;
    return out;
}

const float *gpt_forward_fast(GPT *m, FastCtx *f, const int *tokens, int B, int T)
{                                                   /* fast.c:227-333 */
    return forward(m, f, tokens, B, T, CNGPT_LAST);
}

const float *gpt_forward_fast_all(GPT *m, FastCtx *f, const int *tokens, int B, int T)
{
    return forward(m, f, tokens, B, T, CNGPT_ALL);
}
