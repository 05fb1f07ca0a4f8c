/*
 * check_host_asan.c - the library's CPU-only host paths under AddressSanitizer
 * and UndefinedBehaviorSanitizer (any report aborts the run): the weight-file
 * header checks of cngpt_hip_file_config on valid, truncated and corrupted
 * files, the seeded init, the model.h host API (gpt_init, gpt_init_weights,
 * gpt_save, gpt_load, gpt_free) and a round trip through a file, and the
 * error paths of entry points called without a device or with bad
 * arguments. Exit status 0 = pass.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "cngpt_hip.h"
#include "model.h"

static int n_pass = 0, n_fail = 0;
static void expect(int ok, const char *what)
{
    if (ok) n_pass++;
    else { n_fail++; fprintf(stderr, "FAIL %s (%s)\n", what, cngpt_hip_last_error()); }
}

static void write_file(const char *path, const void *data, size_t n)
{
    FILE *f = fopen(path, "wb");
    if (!f) { perror(path); exit(2); }
    if (n && fwrite(data, 1, n, f) != n) { perror(path); exit(2); }
    fclose(f);
}

int main(void)
{
    char dir[] = "/tmp/cngpt_asan_XXXXXX";
    if (!mkdtemp(dir)) { perror("mkdtemp"); return 2; }
    char path[512], bad[512];
    snprintf(path, sizeof(path), "%s/m.bin", dir);
    snprintf(bad, sizeof(bad), "%s/bad.bin", dir);

    /* the host model API and a weight file round trip */
    srand(7);
    GPTConfig cfg = { 2, 4, 32, 61, 16, 0.0f };
    GPT m, m2;
    memset(&m, 0, sizeof(m));
    memset(&m2, 0, sizeof(m2));
    expect(gpt_init(&m, cfg) == 0, "gpt_init");
    gpt_init_weights(&m);
    expect(m.n_params == gpt_num_params(&cfg), "n_params");
    expect(gpt_save(&m, path) == 0, "gpt_save");
    expect(gpt_load(&m2, path) == 0, "gpt_load");
    expect(m2.n_params == m.n_params &&
           memcmp(m2.param_buf, m.param_buf, sizeof(float) * (size_t)m.n_params) == 0,
           "round trip");

    /* header validation without a device */
    cngpt_hip_config hc;
    long np = 0;
    expect(cngpt_hip_file_config(path, &hc, &np) == 0 && np == m.n_params &&
           hc.n_embd == cfg.n_embd && hc.vocab_size == cfg.vocab_size, "file_config");
    FILE *f = fopen(path, "rb");
    fseek(f, 0, SEEK_END);
    const long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    unsigned char *raw = malloc((size_t)sz);
    if (!raw || fread(raw, 1, (size_t)sz, f) != (size_t)sz) return 2;
    fclose(f);
    const size_t cuts[] = { 0, 3, 27, 28, 100, (size_t)sz - 4 };
    for (size_t i = 0; i < sizeof(cuts) / sizeof(cuts[0]); i++) {
        write_file(bad, raw, cuts[i]);
        expect(cngpt_hip_file_config(bad, &hc, &np) != 0, "truncated file refused");
    }
    for (int field = 0; field < 7; field++) {     /* magic, version, then each shape field */
        unsigned char *c = malloc((size_t)sz);
        memcpy(c, raw, (size_t)sz);
        int v;
        memcpy(&v, c + 4 * field, 4);
        v = field < 2 ? v ^ 0x5a5a : (field == 6 ? 1 << 30 : -3);
        memcpy(c + 4 * field, &v, 4);
        write_file(bad, c, (size_t)sz);
        expect(cngpt_hip_file_config(bad, &hc, &np) != 0, "corrupted header refused");
        free(c);
    }
    expect(cngpt_hip_file_config("/nonexistent/cngpt.bin", &hc, &np) != 0, "missing file");

    /* seeded init into a host buffer, and its argument checks */
    const long n = cngpt_hip_num_params(&hc);
    float *p = malloc(sizeof(float) * (size_t)n);
    expect(n == m.n_params && cngpt_hip_init_weights(&hc, p, 7) == 0, "init_weights");
    cngpt_hip_config zero = { 0, 0, 0, 0, 0 };
    expect(cngpt_hip_num_params(&zero) < 0, "invalid shape");
    expect(cngpt_hip_init_weights(&zero, p, 1) != 0, "init_weights refuses an invalid shape");

    /* entry points without a device or with bad arguments fail cleanly */
    cngpt_hip_ctx *h = NULL;
    const int rc = cngpt_hip_create(0, &h);
    if (rc == 0) {
        expect(cngpt_hip_forward(h, NULL, 1, 1, CNGPT_LAST, NULL) != 0, "forward without params");
        cngpt_hip_train *t = NULL;
        expect(cngpt_hip_train_create(h, 1, 1, &t) != 0, "trainer without params");
        cngpt_hip_destroy(h);
    } else {
        expect(h == NULL, "no handle without a device");
    }
    expect(cngpt_hip_create(-1, &h) != 0, "negative device");
    expect(cngpt_hip_train_forward(NULL, NULL, NULL, NULL) != 0, "null trainer");
    expect(cngpt_hip_train_steps(NULL) == -1, "null trainer steps");
    cngpt_hip_train_destroy(NULL);
    cngpt_hip_destroy(NULL);

    gpt_free(&m);
    gpt_free(&m2);
    free(raw);
    free(p);
    unlink(path);
    unlink(bad);
    rmdir(dir);
    printf("%d passed, %d failed\n", n_pass, n_fail);
    return n_fail ? 1 : 0;
}
