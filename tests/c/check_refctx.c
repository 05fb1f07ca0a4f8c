/*
 * check_refctx.c - the library driven through a FastCtx of the reference's
 * own layout (src/fast.h:35-45), as a caller compiled against the
 * reference's header would: `#include "fast.h"` in src/cngpt.c:21 and
 * tests/check_fast.c:22 finds src/fast.h before any -I path, so such a
 * caller allocates the reference's struct (on its stack, src/cngpt.c:286,
 * tests/check_fast.c:85) and passes it to this library's entry points.
 *
 * This file therefore does not include include/fast.h. It declares the
 * reference's struct and the four entry points over it, puts the struct
 * between guard bytes, and checks that fast_init / gpt_forward_fast /
 * fast_free stay inside it, that the logits agree with the oracle, and that
 * the struct's `logits` member holds the pointer the call returned (the
 * reference keeps the returned buffer there too, src/fast.c:160-161).
 * Exit status 0 = pass.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cngpt_oracle.h"
#include "model.h"

/* src/fast.h:35-45 */
typedef struct {
    int    B, T;
    float *x;
    float *ln;
    float *qkv;
    float *scores;
    float *aout;
    float *hid;
    float *mean, *rstd;
    float *logits;
} RefFastCtx;

void fast_init(RefFastCtx *f);
void fast_free(RefFastCtx *f);
void fast_set_threads(int n);
const float *gpt_forward_fast(GPT *m, RefFastCtx *f, const int *tokens, int B, int T);
const char *fast_last_error(void);

#define GUARD 64

struct Framed {
    unsigned char before[GUARD];
    RefFastCtx ctx;
    unsigned char after[GUARD];
};

static int n_pass = 0, n_fail = 0;

static void expect(int ok, const char *what)
{
    if (ok) n_pass++;
    else { n_fail++; fprintf(stderr, "FAIL %s\n", what); }
}

static int guards_intact(const struct Framed *fr)
{
    for (int i = 0; i < GUARD; i++)
        if (fr->before[i] != 0xA5 || fr->after[i] != 0x5A) return 0;
    return 1;
}

int main(void)
{
    srand(7);
    GPTConfig cfg = { 2, 4, 32, 70, 16, 0.0f };
    GPT m;
    memset(&m, 0, sizeof(m));
    if (gpt_init(&m, cfg) != 0) { fprintf(stderr, "gpt_init failed\n"); return 1; }
    gpt_init_weights(&m);
    orc_cfg oc = { cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size, cfg.block_size };
    const int V = cfg.vocab_size;

    expect(sizeof(RefFastCtx) == 80, "reference layout is 80 bytes");

    struct Framed *fr = malloc(sizeof(*fr));
    memset(fr->before, 0xA5, GUARD);
    memset(fr->after, 0x5A, GUARD);
    memset(&fr->ctx, 0xCC, sizeof(fr->ctx));  /* fast_init must clear it all */
    fast_init(&fr->ctx);
    {
        static const RefFastCtx zero;
        expect(memcmp(&fr->ctx, &zero, sizeof(zero)) == 0, "fast_init zeroes the whole struct");
    }
    expect(guards_intact(fr), "fast_init stays inside the struct");

    static const int shapes[][2] = { {1, 1}, {2, 6}, {3, 16} };
    for (size_t s = 0; s < sizeof(shapes) / sizeof(shapes[0]); s++) {
        const int B = shapes[s][0], T = shapes[s][1];
        int tok[48];
        float ref[3 * 70];
        for (int i = 0; i < B * T; i++) tok[i] = rand() % V;
        if (orc_forward(&oc, m.param_buf, tok, B, T, ORC_LAST, ref) != 0) return 1;
        const float *got = gpt_forward_fast(&m, &fr->ctx, tok, B, T);
        if (!got) { fprintf(stderr, "gpt_forward_fast: %s\n", fast_last_error()); return 1; }
        float d = 0.0f;
        for (int i = 0; i < B * V; i++) {
            const float e = fabsf(got[i] - ref[i]);
            if (!(e <= d)) d = e;
        }
        char what[96];
        snprintf(what, sizeof(what), "B=%d T=%d max|diff| %.3e < 1e-4", B, T, d);
        expect(d < 1e-4f, what);
        expect(fr->ctx.B == B && fr->ctx.T == T, "B and T at the reference's offsets");
        expect(fr->ctx.logits == got, "logits member holds the returned buffer");
        expect(guards_intact(fr), "gpt_forward_fast stays inside the struct");
    }

    fast_free(&fr->ctx);
    expect(guards_intact(fr), "fast_free stays inside the struct");
    expect(fr->ctx.logits == NULL && fr->ctx.B == 0, "fast_free clears the struct");
    free(fr);
    gpt_free(&m);
    printf("check_refctx: %d passed, %d failed\n", n_pass, n_fail);
    return n_fail ? 1 : 0;
}
