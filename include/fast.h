/*
 * fast.h - inference forward pass on an MI355X, as a drop-in for the
 * reference's src/fast.h:35-60.
 *
 * Same four entry points with the same signatures and meaning:
 *   fast_init / fast_free      zero a context, release everything it holds
 *   fast_set_threads           kept for source compatibility; the GPU path
 *                              has no host thread team, so it has no effect
 *   gpt_forward_fast           logits [B, V] of the final position of each
 *                              sequence; the pointer belongs to the context
 *                              and stays valid until the next call; NULL on
 *                              failure (fast_last_error() says why)
 *
 * FastCtx has the reference's size and alignment (two ints and nine
 * pointers, 80 bytes on LP64), so a caller compiled against the reference's
 * src/fast.h - whose quote include finds that header first - hands this
 * library a struct of the right size. B and T sit where the reference keeps
 * them and `logits` (the buffer the last call returned) at the offset of the
 * reference's `logits`; the other slots hold the device handle and the
 * parameter-upload cache instead of host scratch. Callers never read the
 * other fields (src/cngpt.c and tests/check_fast.c only pass the struct
 * around).
 *
 * One deliberate divergence from the reference: the reference reads
 * m->params on every call; this context copies them to the device on the
 * first call and again only when m->param_buf, m->n_params or m->cfg
 * changes, or after fast_params_changed(f). Callers that edit weights in
 * place between calls must call fast_params_changed.
 *
 * The device is HIP device 0, or the index in the CNGPT_HIP_DEVICE
 * environment variable.
 */
#ifndef CNGPT_FAST_H
#define CNGPT_FAST_H

#include "model.h"

typedef struct {
    int    B, T;              /* shape of the last call */
    void  *dev;               /* cngpt_hip_ctx * */
    const float *params_seen; /* parameter upload cache key */
    size_t logits_cap;        /* floats the logits buffer holds */
    GPTConfig cfg_seen;
    int    n_params_seen;
    int    params_dirty;
    void  *reserved;
    float *logits;            /* [B, V] host (pinned), owned by the context */
} FastCtx;

/* The reference's layout: int B, T; then x, ln, qkv, scores, aout, hid,
 * mean, rstd, logits (src/fast.h:35-45). */
#ifdef __cplusplus
static_assert(sizeof(FastCtx) == 2 * sizeof(int) + 9 * sizeof(void *), "FastCtx size");
static_assert(alignof(FastCtx) == alignof(void *), "FastCtx alignment");
static_assert(offsetof(FastCtx, logits) == 2 * sizeof(int) + 8 * sizeof(void *),
              "FastCtx logits offset");
#else
_Static_assert(sizeof(FastCtx) == 2 * sizeof(int) + 9 * sizeof(void *), "FastCtx size");
_Static_assert(_Alignof(FastCtx) == _Alignof(void *), "FastCtx alignment");
_Static_assert(offsetof(FastCtx, logits) == 2 * sizeof(int) + 8 * sizeof(void *),
               "FastCtx logits offset");
#endif

#ifdef __cplusplus
extern "C" {
#endif

void fast_init(FastCtx *f);
void fast_free(FastCtx *f);
void fast_set_threads(int n);
const float *gpt_forward_fast(GPT *m, FastCtx *f, const int *tokens, int B, int T);

/* Additions (no reference counterpart). */

/* Logits for every position, [B, T, V], copied to a context-owned host
 * buffer (gpt_forward's logits, src/model.c:612-614). */
const float *gpt_forward_fast_all(GPT *m, FastCtx *f, const int *tokens, int B, int T);
/* Force a parameter re-upload on the next call. */
void fast_params_changed(FastCtx *f);
/* Message of the last failure on this thread. */
const char *fast_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* CNGPT_FAST_H */
