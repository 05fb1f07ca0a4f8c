/*
 * model.h - GPT-2 model structs and the host model API that the fast.h
 * drop-in reads.
 *
 * The structs keep the member order and types of the reference's
 * src/model.h:19-137 so that a GPT built by the reference's model.c can be
 * passed to this library's gpt_forward_fast unchanged, and the weight file
 * keeps the reference's 28-byte header (src/model.h:19-30) and flat fp32
 * layout (src/model.c:54-83).
 *
 * libcngpt_hip.so also implements the parameter-side functions below
 * (gpt_num_params, gpt_init, gpt_init_weights, gpt_load, gpt_save, gpt_free)
 * as weak symbols: a program that links the reference's model.c gets the
 * reference's definitions, one that does not gets these. This gpt_init
 * allocates the parameter buffer only (no gradients or optimizer moments:
 * inference does not use them).
 */
#ifndef CNGPT_MODEL_H
#define CNGPT_MODEL_H

#include <stddef.h>
#include <stdint.h>

#define CNGPT_MAGIC    0x434E4750   /* "CNGP" */
#define CNGPT_VERSION  1

typedef struct {
    int magic;
    int version;
    int n_layer;
    int n_head;
    int n_embd;
    int vocab_size;
    int block_size;
} GPTHeader;

typedef struct {
    int n_layer;
    int n_head;
    int n_embd;
    int vocab_size;
    int block_size;
    float dropout;
} GPTConfig;

/* Pointers into the flat parameter buffer; per-layer members are arrays of
 * n_layer pointers. lm_head is tied to wte. */
typedef struct {
    float *wte;
    float *wpe;
    float **ln1_w, **ln1_b;
    float **c_attn_w, **c_attn_b;
    float **c_proj_w, **c_proj_b;
    float **ln2_w, **ln2_b;
    float **mlp_fc_w, **mlp_fc_b;
    float **mlp_proj_w, **mlp_proj_b;
    float *ln_f_w, *ln_f_b;
} GPTWeights;

/* Training activations of the reference's straightforward forward; kept so
 * that GPT has the reference's size and layout. Unused here. */
typedef struct {
    float *emb;
    float **ln1_out, **ln1_mean, **ln1_rstd;
    float **qkv;
    float **attn_scores, **attn_probs, **attn_out, **attn_proj;
    float **res1;
    float **ln2_out, **ln2_mean, **ln2_rstd;
    float **mlp_fc_out, **mlp_gelu, **mlp_proj_out;
    float **res2;
    float *ln_f_out, *ln_f_mean, *ln_f_rstd;
    float *logits, *probs;
    unsigned char *emb_mask;
    unsigned char **res1_mask, **res2_mask;
} GPTActivations;

typedef struct {
    GPTConfig      cfg;
    GPTWeights     params;
    GPTWeights     grads;
    GPTActivations acts;
    float *param_buf;
    float *grad_buf;
    float *act_buf;
    unsigned char *mask_buf;
    float *m_buf;
    float *v_buf;
    uint8_t *decay_buf;
    int    n_params;
    int    step;
} GPT;

#ifdef __cplusplus
extern "C" {
#endif

/* src/model.c:20-48 */
int  gpt_num_params(const GPTConfig *cfg);
/* src/model.c:120-175 (parameter buffer only). 0 or -1. */
int  gpt_init(GPT *m, GPTConfig cfg);
/* src/model.c:292-331: N(0,0.02) draws from rand(), residual projections
 * scaled by 1/sqrt(2*n_layer), LayerNorm 1/0, biases 0. */
void gpt_init_weights(GPT *m);
/* src/model.c:177-211: header check (magic), then n_params floats. */
int  gpt_load(GPT *m, const char *path);
/* src/model.c:213-231 */
int  gpt_save(GPT *m, const char *path);
/* src/model.c:233-259 */
void gpt_free(GPT *m);

#ifdef __cplusplus
}
#endif
#endif /* CNGPT_MODEL_H */
