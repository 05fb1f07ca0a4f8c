/*
 * cngpt_cli.c - the `cngpt` command line over this library: the inference
 * sub-commands of the reference's CLI (src/cngpt.c) with the same flag
 * syntax (--key=value or --key value, src/cngpt.c:35-62).
 *
 *   cngpt bench  --weights=F [--iters=50] [--seq=128] [--batch=1] [--fast] [--threads=N]
 *   cngpt sample --weights=F [--prompt=ID,ID,...] [--tokens=200] [--temp=1.0]
 *                [--topk=40] [--seed=N] [--vocab=FILE]
 *   cngpt create-tiny [--out=tiny_test.bin] [--seed=1234]
 *
 * bench keeps the reference's measurement (src/cngpt.c:280-366): all-zero
 * tokens, one warm-up pass, `iters` timed passes, CLOCK_MONOTONIC, and
 * tok/s = 1000 * B * T / ms. --fast times gpt_forward_fast (final-position
 * logits); without it the pass produces the logits of every position, which
 * is what the reference's gpt_forward computes. The parity line compares
 * the final-position logits of the two modes on the LCG tokens of
 * src/cngpt.c:338-342, and the fast path with an independent route to
 * the same final-position logits (prefill of the first T - 1 tokens, then
 * one KV-cache decode step), as the reference compares gpt_forward_fast
 * with gpt_forward (src/cngpt.c:334-356).
 *
 * sample follows gpt_sample (src/model.c:991-1016) and sample_top_k
 * (src/model.c:927-989): prompt token ids, one rand() draw per new token,
 * temperature and top-k. The context sits in the device KV cache while it
 * fits block_size; beyond that the reference slides the window and
 * re-bases positions, which this command reproduces by running the last
 * block_size tokens through the forward again for each further token.
 * Differences from the reference: --seed (the reference seeds with
 * time(NULL), src/cngpt.c:250), and the default prompt is token
 * min(50256, vocab_size - 1).
 */
#define _POSIX_C_SOURCE 200809L

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../../include/cngpt_hip.h"
#include "../../include/fast.h"
#include "../../include/model.h"

static const char *arg_get(int argc, char **argv, const char *key)
{
    size_t n = strlen(key);
    for (int i = 2; i < argc; i++) {
        const char *a = argv[i];
        if (strncmp(a, "--", 2) != 0 || strncmp(a + 2, key, n) != 0) continue;
        if (a[2 + n] == '=') return a + 3 + n;
        if (a[2 + n] == '\0' && i + 1 < argc) return argv[i + 1];
    }
    return NULL;
}

static int has_flag(int argc, char **argv, const char *flag)
{
    for (int i = 2; i < argc; i++)
        if (strcmp(argv[i], flag) == 0) return 1;
    return 0;
}

static int arg_int(int argc, char **argv, const char *key, int def)
{
    const char *v = arg_get(argc, argv, key);
    return v ? atoi(v) : def;
}

static float arg_float(int argc, char **argv, const char *key, float def)
{
    const char *v = arg_get(argc, argv, key);
    return v ? (float)atof(v) : def;
}

static double now_ms(void)
{
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec * 1e3 + t.tv_nsec / 1e6;
}

/* ------------------------------------------------------------------ bench */

static int cmd_bench(int argc, char **argv)
{
    const char *path = arg_get(argc, argv, "weights");
    const int iters = arg_int(argc, argv, "iters", 50);
    const int T = arg_int(argc, argv, "seq", 128);
    const int B = arg_int(argc, argv, "batch", 1);
    const int fast = has_flag(argc, argv, "--fast");
    if (!path) { fprintf(stderr, "bench: --weights is required\n"); return 1; }
    if (iters <= 0 || T <= 0 || B <= 0) { fprintf(stderr, "bench: bad --iters/--seq/--batch\n"); return 1; }

    GPT m;
    memset(&m, 0, sizeof(m));
    if (gpt_load(&m, path) != 0) return 1;
    if (T > m.cfg.block_size) {
        fprintf(stderr, "bench: --seq=%d exceeds block_size %d\n", T, m.cfg.block_size);
        gpt_free(&m);
        return 1;
    }
    if (fast) fast_set_threads(arg_int(argc, argv, "threads", 0));
    printf("Model: %d layers, %d heads, %d embd, %d params\n", m.cfg.n_layer, m.cfg.n_head,
           m.cfg.n_embd, m.n_params);
    printf("Benchmarking %d inference passes (seq_len=%d, batch=%d, %s) on HIP device...\n\n",
           iters, T, B, fast ? "fast" : "all positions");

    const int V = m.cfg.vocab_size;
    int *tk = malloc((size_t)B * T * sizeof(int));
    float *last = malloc((size_t)V * sizeof(float));
    if (!tk || !last) { gpt_free(&m); return 1; }
    FastCtx fc;
    fast_init(&fc);
    int rc = 0;
    {   /* parity line: final-position logits of both modes, LCG tokens */
        unsigned s = 12345u;
        for (int i = 0; i < T; i++) {
            s = s * 1664525u + 1013904223u;
            tk[i] = (int)((s >> 8) % (unsigned)V);
        }
        const float *all = gpt_forward_fast_all(&m, &fc, tk, 1, T);
        if (all) memcpy(last, all + (size_t)(T - 1) * V, (size_t)V * sizeof(float));
        const float *fl = all ? gpt_forward_fast(&m, &fc, tk, 1, T) : NULL;
        if (!fl) {
            fprintf(stderr, "bench: forward failed: %s\n", fast_last_error());
            rc = 1;
        } else {
            float maxd = 0.0f;
            for (int v = 0; v < V; v++) maxd = fmaxf(maxd, fabsf(fl[v] - last[v]));
            printf("  max |logit diff| final position, fast vs all-positions : %.3e\n",
                   (double)maxd);
            memcpy(last, fl, (size_t)V * sizeof(float));
        }
    }
    if (!rc && T >= 2) {
        /* The reference checks its fast path against the straightforward
         * gpt_forward (src/cngpt.c:334-356). Here the independent route to
         * the same logits is the KV-cache decode: the first T - 1 tokens
         * prefilled, then one decode step for token T - 1, whose row goes
         * through every layer on the decode kernels (products over one row,
         * attention of one query against the cache) instead of the prefill
         * tiles. */
        cngpt_hip_ctx *h = NULL;
        const cngpt_hip_config c = {m.cfg.n_layer, m.cfg.n_head, m.cfg.n_embd, m.cfg.vocab_size,
                                    m.cfg.block_size};
        float *dl = malloc((size_t)V * sizeof(float));
        const char *dev = getenv("CNGPT_HIP_DEVICE");
        int drc = dl ? cngpt_hip_create(dev && *dev ? atoi(dev) : 0, &h) : 1;
        if (!drc) drc = cngpt_hip_load_params(h, &c, m.param_buf, m.n_params);
        if (!drc) drc = cngpt_hip_decode_begin(h, tk, 1, T - 1, T, NULL);
        if (!drc) drc = cngpt_hip_decode_step(h, tk + T - 1, dl);
        if (drc) {
            fprintf(stderr, "bench: decode check failed: %s\n", cngpt_hip_last_error());
            rc = 1;
        } else {
            float maxd = 0.0f;
            for (int v = 0; v < V; v++) maxd = fmaxf(maxd, fabsf(dl[v] - last[v]));
            printf("  max |logit diff| final position, fast vs KV-cache decode : %.3e\n",
                   (double)maxd);
        }
        if (h) cngpt_hip_destroy(h);
        free(dl);
    }
    if (!rc) {
        memset(tk, 0, (size_t)B * T * sizeof(int));   /* src/cngpt.c:283 */
        const float *(*fwd)(GPT *, FastCtx *, const int *, int, int) =
            fast ? gpt_forward_fast : gpt_forward_fast_all;
        if (!fwd(&m, &fc, tk, B, T)) rc = 1;          /* warm-up */
        const double t0 = now_ms();
        for (int i = 0; i < iters && !rc; i++)
            if (!fwd(&m, &fc, tk, B, T)) rc = 1;
        const double ms = (now_ms() - t0) / iters;
        if (rc) {
            fprintf(stderr, "bench: forward failed: %s\n", fast_last_error());
        } else {
            printf("  ms/forward : %.2f\n", ms);
            printf("  tok/s      : %.1f\n", 1000.0 * B * T / ms);
        }
    }
    fast_free(&fc);
    free(tk);
    free(last);
    gpt_free(&m);
    return rc;
}

/* ----------------------------------------------------------------- sample */

typedef struct {
    char **piece;
    int n;
} Vocab;

/* One token piece per line (GPT-2 byte-level pieces); display only. */
static int vocab_load(Vocab *vb, const char *path)
{
    memset(vb, 0, sizeof(*vb));
    FILE *f = fopen(path, "r");
    if (!f) { perror(path); return -1; }
    char line[4096];
    int cap = 0;
    while (fgets(line, sizeof(line), f)) {
        size_t len = strlen(line);
        while (len && (line[len - 1] == '\n' || line[len - 1] == '\r')) line[--len] = '\0';
        if (vb->n == cap) {
            cap = cap ? 2 * cap : 1024;
            char **p = realloc(vb->piece, (size_t)cap * sizeof(char *));
            if (!p) { fclose(f); return -1; }
            vb->piece = p;
        }
        vb->piece[vb->n++] = strdup(line);
    }
    fclose(f);
    return 0;
}

static void vocab_free(Vocab *vb)
{
    for (int i = 0; i < vb->n; i++) free(vb->piece[i]);
    free(vb->piece);
    memset(vb, 0, sizeof(*vb));
}

/* Print one token: its piece with GPT-2's space (U+0120) and newline
 * (U+010A) markers turned back into characters and other non-ASCII bytes
 * shown as '.', or [id] without a vocabulary. */
static void print_token(const Vocab *vb, int id, int first)
{
    if (!vb->piece || id < 0 || id >= vb->n) {
        printf(first ? "%d" : ",%d", id);
        return;
    }
    const unsigned char *p = (const unsigned char *)vb->piece[id];
    while (*p) {
        if (p[0] == 0xC4 && p[1] == 0xA0) { putchar(' '); p += 2; continue; }
        if (p[0] == 0xC4 && p[1] == 0x8A) { putchar('\n'); p += 2; continue; }
        putchar(*p >= 32 && *p < 127 ? *p : '.');
        p++;
    }
}

static int cmd_sample(int argc, char **argv)
{
    const char *path = arg_get(argc, argv, "weights");
    const char *prompt_s = arg_get(argc, argv, "prompt");
    const char *vocab_path = arg_get(argc, argv, "vocab");
    const int n_new = arg_int(argc, argv, "tokens", 200);
    const float temp = arg_float(argc, argv, "temp", 1.0f);
    const int top_k = arg_int(argc, argv, "topk", 40);
    const char *seed_s = arg_get(argc, argv, "seed");
    if (!path) { fprintf(stderr, "sample: --weights is required\n"); return 1; }
    if (n_new <= 0) { fprintf(stderr, "sample: --tokens must be positive\n"); return 1; }

    /* The weights go from the file straight to the device (no host copy of
     * the parameters); the header is validated first, without a GPU. */
    cngpt_hip_config cfg;
    if (cngpt_hip_file_config(path, &cfg, NULL) != 0) {
        fprintf(stderr, "sample: %s\n", cngpt_hip_last_error());
        return 1;
    }
    const int V = cfg.vocab_size, Tmax = cfg.block_size;

    int n_prompt = 1;
    for (const char *p = prompt_s; p && *p; p++) n_prompt += *p == ',';
    int *seq = malloc((size_t)(n_prompt + n_new) * sizeof(int));
    float *draws = malloc((size_t)n_new * sizeof(float));
    if (!seq || !draws) { free(seq); free(draws); return 1; }
    if (prompt_s && *prompt_s) {
        int k = 0;
        const char *p = prompt_s;
        while (*p && k < n_prompt) {
            char *end;
            long v = strtol(p, &end, 10);
            if (end == p || v < 0 || v >= V) {
                fprintf(stderr, "sample: bad prompt token near \"%s\" (ids in [0, %d))\n", p, V);
                free(seq); free(draws);
                return 1;
            }
            seq[k++] = (int)v;
            p = *end == ',' ? end + 1 : end;
        }
        n_prompt = k;
    } else {
        seq[0] = 50256 < V ? 50256 : V - 1;   /* <|endoftext|> */
        n_prompt = 1;
    }
    if (n_prompt > Tmax) {
        fprintf(stderr, "sample: prompt of %d tokens exceeds block_size %d\n", n_prompt, Tmax);
        free(seq); free(draws);
        return 1;
    }

    srand(seed_s ? (unsigned)strtoul(seed_s, NULL, 10) : (unsigned)time(NULL));
    for (int i = 0; i < n_new; i++) draws[i] = (float)rand() / ((float)RAND_MAX + 1.0f);

    Vocab vb;
    memset(&vb, 0, sizeof(vb));
    if (vocab_path && vocab_load(&vb, vocab_path) != 0) {
        free(seq); free(draws);
        return 1;
    }

    cngpt_hip_ctx *h = NULL;
    const char *dev = getenv("CNGPT_HIP_DEVICE");
    int rc = cngpt_hip_create(dev && *dev ? atoi(dev) : 0, &h);
    if (!rc) rc = cngpt_hip_load_file(h, path, NULL);

    /* New token i sees a context of n_prompt + i tokens; while that fits
     * block_size it comes from the KV cache. */
    int in_cache = Tmax - n_prompt + 1;
    if (in_cache > n_new) in_cache = n_new;
    if (n_prompt == Tmax) in_cache = 0;   /* no room to append: window path only */
    if (!rc && in_cache > 0) {
        int cap = n_prompt + in_cache - 1;
        if (cap < n_prompt + 1) cap = n_prompt + 1;
        if (cap > Tmax) cap = Tmax;
        rc = cngpt_hip_decode_begin(h, seq, 1, n_prompt, cap, NULL);
        if (!rc) rc = cngpt_hip_generate(h, in_cache, temp, top_k, draws, seq + n_prompt);
    }
    /* past block_size: the reference's sliding window (model.c:1003-1008) */
    for (int i = in_cache; i < n_new && !rc; i++) {
        const int total = n_prompt + i;
        const int start = total - Tmax;
        rc = cngpt_hip_forward(h, seq + start, 1, Tmax, CNGPT_LAST, NULL);
        if (!rc) rc = cngpt_hip_sample(h, temp, top_k, draws + i, seq + total);
    }
    if (rc) {
        fprintf(stderr, "sample: %s\n", cngpt_hip_last_error());
    } else {
        printf("--- Generating %d tokens (temp=%.2f, top_k=%d) ---\n\n", n_new, (double)temp,
               top_k);
        for (int i = 0; i < n_prompt + n_new; i++) {
            if (i == n_prompt && !vb.piece) printf(" | ");
            print_token(&vb, seq[i], i == 0 || i == n_prompt);
        }
        printf("\n\n--- done ---\n");
    }
    cngpt_hip_destroy(h);
    vocab_free(&vb);
    free(seq);
    free(draws);
    return rc ? 1 : 0;
}

/* ------------------------------------------------------------ create-tiny */

static int cmd_create_tiny(int argc, char **argv)
{
    const char *out = arg_get(argc, argv, "out");
    if (!out) out = "tiny_test.bin";
    srand((unsigned)arg_int(argc, argv, "seed", 1234));
    GPTConfig cfg = { 2, 4, 32, 64, 8, 0.0f };   /* src/cngpt.c:380-387 */
    GPT m;
    memset(&m, 0, sizeof(m));
    if (gpt_init(&m, cfg) != 0) { fprintf(stderr, "gpt_init failed\n"); return 1; }
    gpt_init_weights(&m);
    if (gpt_save(&m, out) != 0) { gpt_free(&m); return 1; }
    printf("Wrote tiny test model (%d params) to %s\n", m.n_params, out);
    gpt_free(&m);
    return 0;
}

static void usage(void)
{
    fprintf(stderr,
            "Usage:\n"
            "  cngpt sample --weights=<file> [--prompt=ID,ID,...] [--tokens=200] [--temp=1.0]\n"
            "               [--topk=40] [--seed=N] [--vocab=FILE]\n"
            "  cngpt bench  --weights=<file> [--iters=50] [--seq=128] [--batch=1] [--fast]\n"
            "               [--threads=N]\n"
            "  cngpt create-tiny [--out=tiny_test.bin] [--seed=1234]\n"
            "The forward pass runs on HIP device $CNGPT_HIP_DEVICE (default 0).\n");
}

int main(int argc, char **argv)
{
    if (argc < 2) { usage(); return 1; }
    const char *cmd = argv[1];
    if (strcmp(cmd, "bench") == 0) return cmd_bench(argc, argv);
    if (strcmp(cmd, "sample") == 0) return cmd_sample(argc, argv);
    if (strcmp(cmd, "create-tiny") == 0) return cmd_create_tiny(argc, argv);
    if (strcmp(cmd, "train") == 0) {
        fprintf(stderr, "train: this build is the inference forward pass only\n");
        return 1;
    }
    fprintf(stderr, "Unknown subcommand: %s\n\n", cmd);
    usage();
    return 1;
}
