/*
 * cngpt_oracle.h - CPU restatement of cngpt's inference forward pass and of
 * its training step (forward with targets, backward, AdamW).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP path is
 * compared against, and the CPU baseline that bench.py times beside it.
 * Nothing in the product (cngpt_amd/, include/) links or loads it; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may.
 *
 * Every function cites the reference file:line it restates. All arithmetic
 * is fp32 like the reference; the matrix products go through a CBLAS
 * sgemm resolved at run time (OpenBLAS, as the reference links) or, when
 * none is found, through a plain blocked C product.
 */
#ifndef CNGPT_ORACLE_H
#define CNGPT_ORACLE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model shape; the fields of GPTHeader/GPTConfig (src/model.h:22-42). */
typedef struct {
    int n_layer;
    int n_head;
    int n_embd;
    int vocab_size;
    int block_size;
} orc_cfg;

enum { ORC_LAST = 0, ORC_ALL = 1 };

/* Parameter count, src/model.c:20-48 (64-bit here; the reference's int
 * overflows past 2^31 parameters, which no GPT-2 size reaches). */
long orc_num_params(const orc_cfg *c);

/* Offsets (in floats) of every tensor in the flat buffer, in the order of
 * src/model.c:54-83. off must hold 2 + 12*n_layer + 2 entries:
 * wte, wpe, then per layer ln1_w ln1_b c_attn_w c_attn_b c_proj_w c_proj_b
 * ln2_w ln2_b mlp_fc_w mlp_fc_b mlp_proj_w mlp_proj_b, then ln_f_w ln_f_b. */
void orc_offsets(const orc_cfg *c, long *off);

/* srand(seed) then gpt_init_weights, src/model.c:275-331. */
void orc_init_weights(const orc_cfg *c, float *params, unsigned seed);

/* Bind a CBLAS at run time (path to a shared library exporting
 * cblas_sgemm or scipy_cblas_sgemm). Returns 0 on success; on failure the
 * built-in C product stays in use. */
int  orc_use_blas(const char *path);
/* Human-readable name of the sgemm in use (library config string). */
const char *orc_blas_info(void);
/* Threads for the forward (n <= 0: one per physical core, as
 * src/fast.c:165-200 picks). Returns the count in use. */
int  orc_set_threads(int n);
/* Physical cores the process may run on (src/fast.c:124-156). */
int  orc_physical_cores(void);

/* Single ops, scalar paths of src/ops.c. */
void orc_layernorm(const float *x, const float *w, const float *b, float *out,
                   float *mean, float *rstd, int T, int C);       /* ops.c:191-248 */
void orc_gelu(const float *x, float *out, int n);                  /* ops.c:337-380 */
void orc_softmax_inplace(float *x, int rows, int cols);            /* ops.c:424-482 */
void orc_causal_mask(float *scores, int T);                        /* ops.c:488-493 */
void orc_linear(const float *X, const float *W, const float *b, float *Y,
                int M, int K, int N);                              /* ops.c:109-123 */

/* Inference forward. mode ORC_LAST: gpt_forward_fast (src/fast.c:227-333),
 * logits [B, V] of the final position of each sequence. mode ORC_ALL: the
 * same algorithm without the last-layer pruning, logits [B, T, V] for every
 * position, the semantics of gpt_forward (src/model.c:442-625).
 * Returns 0, or -1 on bad arguments / allocation failure. */
int  orc_forward(const orc_cfg *c, const float *params, const int *tokens,
                 int B, int T, int mode, float *logits);

/* sample_top_k, src/model.c:927-989, with the uniform draw r in [0,1)
 * passed in instead of taken from rand(). */
int  orc_sample_top_k(const float *logits, int V, float temp, int top_k, float r);

/* cross_entropy_fwd, src/ops.c:499-574 (its scalar branch): per row the
 * max, the sum of expf(logit - max), log_sum = logf(sum), and the loss
 * term (logit[target] - max) - log_sum, subtracted from an fp32
 * accumulator in row order; returns the accumulator / (B*T). probs
 * (may be NULL) receives the softmax [B*T, V]; row_loss (may be NULL)
 * the negated term of each row. */
float orc_cross_entropy(const float *logits, const int *targets, float *probs,
                        float *row_loss, int B, int T, int V);

/* Training (dropout 0, the default of `cngpt train`, src/cngpt.c:94). */

/* Backward ops, scalar paths: linear_bwd_dx / linear_bwd_dw
 * (src/ops.c:125-153; both accumulate, db may be NULL), layernorm_bwd
 * (ops.c:250-331, accumulates into dx, dw, db), gelu_bwd (ops.c:382-422,
 * accumulates into dx). */
void orc_linear_bwd_dx(const float *dY, const float *W, float *dX, int M, int K, int N);
void orc_linear_bwd_dw(const float *dY, const float *X, float *dW, float *db, int M, int K, int N);
void orc_layernorm_bwd(const float *dout, const float *x, const float *w, const float *mean,
                       const float *rstd, float *dx, float *dw, float *db, int T, int C);
void orc_gelu_bwd(const float *dout, const float *x, float *dx, int n);

/* The activations gpt_forward keeps (GPTActivations, src/model.h:86-115)
 * for one B x T shape. NULL on a bad shape or allocation failure. */
typedef struct orc_train orc_train;
orc_train *orc_train_new(const orc_cfg *c, int B, int T);
void orc_train_free(orc_train *t);
/* gpt_forward with targets (src/model.c:442-625): the mean loss; keeps the
 * activations and the softmax of the logits. targets NULL: returns 0. */
float orc_train_forward(orc_train *t, const float *params, const int *tokens, const int *targets);
/* gpt_backward (src/model.c:634-877) for the last orc_train_forward:
 * accumulates every parameter's gradient into grads (flat, the layout of
 * params). */
void orc_train_backward(orc_train *t, const float *params, const int *tokens, const int *targets,
                        float *grads);
/* GPTConfig.dropout for the training forwards (model.c:450): p in [0, 1);
 * the masks of the last forward, [1 + 2 L][B T C] bytes (the embedding,
 * then res1 and res2 of each layer), drawn with rand() in model.c's order. */
int orc_train_set_dropout(orc_train *t, float p);
const unsigned char *orc_train_masks(const orc_train *t);
/* dropout_fwd / dropout_bwd (src/ops.c:603-625). */
void orc_dropout_fwd(float *x, unsigned char *mask, long n, float p);
void orc_dropout_bwd(float *dx, const unsigned char *mask, long n, float p);
/* gpt_adamw (src/model.c:888-921) with the step count already advanced:
 * clips grads in place to grad_clip by their global norm (if > 0), then
 * the AdamW update of params, m and v; weight decay on the matrices and
 * embeddings only (src/model.c:143-172). */
void orc_adamw(const orc_cfg *c, float *params, float *grads, float *m, float *v, int step,
               float lr, float beta1, float beta2, float eps, float wd, float grad_clip);

/* The draw sample_top_k makes (src/model.c:979): rand()/(RAND_MAX+1.0f). */
void  orc_srand(unsigned seed);
float orc_rand_uniform(void);

#ifdef __cplusplus
}
#endif
#endif
