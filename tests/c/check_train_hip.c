/*
 * check_train_hip.c - the training step on the device, driven from a C host
 * the way the reference's `cngpt train` loop drives gpt_zero_grad,
 * gpt_forward with targets, gpt_backward and gpt_adamw (src/cngpt.c:150-165),
 * against the oracle's restatement of the same step (oracle/cngpt_oracle.c).
 * A small random GPT from srand(42) (gpt_init + gpt_init_weights), three
 * steps on rand() % V tokens with next-token targets: losses within 1e-5
 * relative, the first step's gradients within 2e-4 of the largest reference
 * gradient, and the weights after every step (see the bound below), then
 * the trained weights read back into the host GPT. Exit status 0 = pass.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cngpt_hip.h"
#include "cngpt_oracle.h"
#include "model.h"

static int n_pass = 0, n_fail = 0;

static void expect(int ok, const char *what, double v, double bound)
{
    if (ok) n_pass++;
    else { n_fail++; fprintf(stderr, "FAIL %s: %.3e (bound %.3e)\n", what, v, bound); }
}

#define CHECK(call)                                                                     \
    do {                                                                                \
        if ((call) != 0) {                                                              \
            fprintf(stderr, "%s failed: %s\n", #call, cngpt_hip_last_error());          \
            return 1;                                                                   \
        }                                                                               \
    } while (0)

int main(void)
{
    srand(42);
    GPTConfig cfg = { 2, 4, 64, 97, 32, 0.0f };
    GPT m;
    memset(&m, 0, sizeof(m));
    if (gpt_init(&m, cfg) != 0) { fprintf(stderr, "gpt_init failed\n"); return 1; }
    gpt_init_weights(&m);
    const long n = m.n_params;
    const int B = 2, T = 16, N = B * T, V = cfg.vocab_size;
    const float lr = 1e-3f;

    int *tok = malloc(sizeof(int) * (N + 1)), *tgt = malloc(sizeof(int) * N);
    float *p_ref = malloc(sizeof(float) * n), *g_ref = calloc(n, sizeof(float));
    float *m_ref = calloc(n, sizeof(float)), *v_ref = calloc(n, sizeof(float));
    float *got = malloc(sizeof(float) * n);
    if (!tok || !tgt || !p_ref || !g_ref || !m_ref || !v_ref || !got) return 1;
    memcpy(p_ref, m.param_buf, sizeof(float) * n);

    orc_cfg oc = { cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size, cfg.block_size };
    orc_train *ref = orc_train_new(&oc, B, T);
    cngpt_hip_config hc = { cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size,
                            cfg.block_size };
    cngpt_hip_ctx *h = NULL;
    cngpt_hip_train *t = NULL;
    CHECK(cngpt_hip_create(0, &h));
    CHECK(cngpt_hip_load_params(h, &hc, m.param_buf, n));
    CHECK(cngpt_hip_train_create(h, B, T, &t));
    if (!ref) { fprintf(stderr, "orc_train_new failed\n"); return 1; }

    for (int step = 0; step < 3; step++) {
        for (int i = 0; i <= N; i++) tok[i] = rand() % V;
        for (int i = 0; i < N; i++) tgt[i] = tok[i + 1];

        /* device: the reference loop's four calls */
        float loss = 0.0f;
        CHECK(cngpt_hip_train_zero_grad(t));
        CHECK(cngpt_hip_train_forward(t, tok, tgt, &loss));
        CHECK(cngpt_hip_train_backward(t));
        if (step == 0) CHECK(cngpt_hip_train_read(t, CNGPT_TRAIN_GRADS, got, n));
        CHECK(cngpt_hip_train_adamw(t, lr, 0.9f, 0.95f, 1e-8f, 0.1f, 1.0f, NULL));

        /* oracle */
        memset(g_ref, 0, sizeof(float) * n);
        const float ref_loss = orc_train_forward(ref, p_ref, tok, tgt);
        orc_train_backward(ref, p_ref, tok, tgt, g_ref);
        if (step == 0) {
            double gmax = 0.0, gerr = 0.0;
            for (long i = 0; i < n; i++) {
                if (fabs(g_ref[i]) > gmax) gmax = fabs(g_ref[i]);
                const double d = fabs((double)got[i] - g_ref[i]);
                if (!(d <= gerr)) gerr = d;
            }
            expect(gerr <= 2e-4 * gmax + 1e-6, "gradients (step 1)", gerr, 2e-4 * gmax + 1e-6);
        }
        orc_adamw(&oc, p_ref, g_ref, m_ref, v_ref, step + 1, lr, 0.9f, 0.95f, 1e-8f, 0.1f, 1.0f);

        const double lerr = fabs((double)loss - ref_loss);
        expect(lerr <= 1e-5 * fabs(ref_loss), "loss", lerr, 1e-5 * fabs(ref_loss));
        /* Adam's step is lr * m_hat / (sqrt(v_hat) + eps): an element whose
         * gradient is below the two sides' rounding can step the other way,
         * so a weight may differ by up to 2 lr per step; such elements must
         * stay rare */
        CHECK(cngpt_hip_train_read(t, CNGPT_TRAIN_PARAMS, got, n));
        double perr = 0.0;
        long off = 0;
        for (long i = 0; i < n; i++) {
            const double d = fabs((double)got[i] - p_ref[i]);
            if (!(d <= perr)) perr = d;
            if (d > 1e-5) off++;
        }
        expect(perr <= 2.0 * lr * (step + 1), "weights after the step", perr, 2.0 * lr * (step + 1));
        expect(off <= n / 100, "weights off by more than 1e-5 (count)", (double)off, n / 100.0);
        printf("step %d: loss %.6f (oracle %.6f), max |dweight| %.2e, %ld of %ld above 1e-5\n",
               step + 1, loss, ref_loss, perr, off, n);
    }
    expect(cngpt_hip_train_steps(t) == 3, "optimizer steps", cngpt_hip_train_steps(t), 3);
    /* the trained weights back into the host model (then gpt_save) */
    CHECK(cngpt_hip_train_read(t, CNGPT_TRAIN_PARAMS, m.param_buf, n));
    expect(memcmp(m.param_buf, got, sizeof(float) * n) == 0, "weights read back", 0, 0);

    cngpt_hip_train_destroy(t);
    cngpt_hip_destroy(h);
    orc_train_free(ref);
    gpt_free(&m);
    free(tok); free(tgt); free(p_ref); free(g_ref); free(m_ref); free(v_ref); free(got);
    printf("%d passed, %d failed\n", n_pass, n_fail);
    return n_fail ? 1 : 0;
}
