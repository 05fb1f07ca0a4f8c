/*
 * check_fast_hip.c - the drop-in fast.h path must agree with the oracle.
 *
 * Mirrors the reference's tests/check_fast.c: a small random GPT from
 * srand(42) (gpt_init + gpt_init_weights), tokens rand() % V, final-position
 * logits of gpt_forward_fast for shapes {1,1},{1,9},{2,6},{3,16},{1,16} and
 * fast_set_threads(1..3), max |diff| < 1e-4. The reference compares with its
 * straightforward gpt_forward; this compares with the CPU oracle's
 * restatement of the same forward (oracle/cngpt_oracle.c). Also checks the
 * parameter-upload cache and gpt_forward_fast_all. Exit status 0 = pass.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cngpt_oracle.h"
#include "fast.h"
#include "model.h"

static int n_pass = 0, n_fail = 0;

static float maxdiff(const float *a, const float *b, size_t n)
{
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float d = fabsf(a[i] - b[i]);
        if (!(d <= m)) m = d;   /* NaN propagates as a failure */
    }
    return m;
}

static void expect(int ok, const char *what, float d)
{
    if (ok) n_pass++;
    else { n_fail++; fprintf(stderr, "FAIL %s: max |diff| = %.3e\n", what, d); }
}

int main(void)
{
    srand(42);
    GPTConfig cfg = { 3, 4, 32, 70, 16, 0.0f };
    GPT m;
    memset(&m, 0, sizeof(m));
    if (gpt_init(&m, cfg) != 0) { fprintf(stderr, "gpt_init failed\n"); return 1; }
    gpt_init_weights(&m);
    orc_cfg oc = { cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size, cfg.block_size };
    const int V = cfg.vocab_size;

    FastCtx fc;
    fast_init(&fc);
    static const int shapes[][2] = { {1, 1}, {1, 9}, {2, 6}, {3, 16}, {1, 16} };
    char what[96];
    for (size_t s = 0; s < sizeof(shapes) / sizeof(shapes[0]); s++)
        for (int threads = 1; threads <= 3; threads++) {
            int B = shapes[s][0], T = shapes[s][1];
            int *tok = malloc(sizeof(int) * B * T);
            float *ref = malloc(sizeof(float) * B * V);
            for (int i = 0; i < B * T; i++) tok[i] = rand() % V;
            if (orc_forward(&oc, m.param_buf, tok, B, T, ORC_LAST, ref) != 0) return 1;
            fast_set_threads(threads);
            const float *got = gpt_forward_fast(&m, &fc, tok, B, T);
            if (!got) { fprintf(stderr, "gpt_forward_fast: %s\n", fast_last_error()); return 1; }
            float d = maxdiff(got, ref, (size_t)B * V);
            snprintf(what, sizeof(what), "B=%d T=%d threads=%d", B, T, threads);
            expect(d < 1e-4f, what, d);
            free(tok);
            free(ref);
        }

    /* all-positions logits */
    {
        int B = 2, T = 11, tok[22];
        for (int i = 0; i < B * T; i++) tok[i] = rand() % V;
        float *ref = malloc(sizeof(float) * B * T * V);
        orc_forward(&oc, m.param_buf, tok, B, T, ORC_ALL, ref);
        const float *got = gpt_forward_fast_all(&m, &fc, tok, B, T);
        float d = got ? maxdiff(got, ref, (size_t)B * T * V) : INFINITY;
        expect(got && d < 1e-4f, "gpt_forward_fast_all", d);
        free(ref);
    }

    /* parameters are cached on the device until fast_params_changed */
    {
        int tok[5] = { 1, 2, 3, 4, 5 };
        float before[70], ref[70];
        const float *got = gpt_forward_fast(&m, &fc, tok, 1, 5);
        memcpy(before, got, sizeof(before));
        m.params.ln_f_b[0] += 1.0f;                  /* shifts every logit */
        got = gpt_forward_fast(&m, &fc, tok, 1, 5);
        expect(maxdiff(got, before, 70) == 0.0f, "stale until fast_params_changed", 0);
        fast_params_changed(&fc);
        got = gpt_forward_fast(&m, &fc, tok, 1, 5);
        orc_forward(&oc, m.param_buf, tok, 1, 5, ORC_LAST, ref);
        float d = maxdiff(got, ref, 70);
        expect(d < 1e-4f && maxdiff(got, before, 70) > 1e-3f, "re-upload after change", d);
    }

    /* a bad token id gives NULL and a message, like an allocation failure */
    {
        int tok[2] = { 0, V };
        const float *got = gpt_forward_fast(&m, &fc, tok, 1, 2);
        expect(got == NULL && strstr(fast_last_error(), "token") != NULL, "bad token -> NULL", 0);
    }

    fast_free(&fc);
    gpt_free(&m);
    printf("check_fast_hip: %d passed, %d failed\n", n_pass, n_fail);
    return n_fail ? 1 : 0;
}
