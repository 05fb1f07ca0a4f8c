/*
 * cngpt_hip.h - C ABI of the MI355X (gfx950) inference forward pass (and,
 * at the end, of the training step on the device).
 *
 * Plain C: opaque handles, plain pointers and sizes, int status codes
 * (0 = success, -1 = failure with a message from cngpt_hip_last_error()).
 * One handle owns one HIP stream on one device, one device allocation for
 * the parameters and one for activations (plus the decode KV cache). Calls on
 * one handle must come from one host thread at a time, as with the
 * reference's FastCtx (src/fast.c:114-115 keeps unsynchronised statics).
 *
 * The fast.h drop-in (fast_init / gpt_forward_fast, include/fast.h) is
 * written on top of these entry points; they are exported for callers that
 * want device-resident inputs, all-position logits or incremental decode.
 */
#ifndef CNGPT_HIP_H
#define CNGPT_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cngpt_hip_ctx cngpt_hip_ctx;

/* Model shape: the fields of the weight-file header (src/model.h:22-30). */
typedef struct {
    int n_layer;
    int n_head;
    int n_embd;
    int vocab_size;
    int block_size;
} cngpt_hip_config;

/* Which positions get logits. LAST: the final position of each sequence,
 * [B, V] (gpt_forward_fast, src/fast.c:227-333). ALL: every position,
 * [B, T, V] (the logits gpt_forward keeps, src/model.c:612-614). */
enum { CNGPT_LAST = 0, CNGPT_ALL = 1 };

/* Kernel classes for the timing counters. */
enum {
    CNGPT_K_GEMM = 0,        /* MFMA products (linear layers, lm_head) */
    CNGPT_K_GEMV = 1,        /* skinny products (<= 8 rows) */
    CNGPT_K_ATTN = 2,        /* fused causal attention */
    CNGPT_K_ATTN_ROW = 3,    /* one-query attention (last position, decode) */
    CNGPT_K_LAYERNORM = 4,
    CNGPT_K_EMBED = 5,
    CNGPT_K_GATHER = 6,
    CNGPT_K_ARGMAX = 7,
    CNGPT_K_SAMPLE = 8,      /* top-k sampling */
    CNGPT_K_STEP = 9,        /* whole decode steps in one persistent launch */
    CNGPT_K_LOSS = 10,       /* cross-entropy over the held logits */
    CNGPT_K_COUNT = 11
};

/* How decode steps run. KERNELS: one replayed graph of per-stage kernels
 * per step (any batch). PERSISTENT: the steps of one sequence as a
 * cooperative launch whose workgroups exchange each stage's outputs
 * through tagged words (B = 1, head size 64, n_embd <= 768): all steps of
 * a generate call in one launch, greedy or sampled (top_k <= 64; other
 * sampling runs one launch per step followed by the sampler). AUTO:
 * PERSISTENT where it applies, else KERNELS. */
enum { CNGPT_DECODE_AUTO = 0, CNGPT_DECODE_KERNELS = 1, CNGPT_DECODE_PERSISTENT = 2 };

/* Last error message of the calling thread ("" if none). */
const char *cngpt_hip_last_error(void);

/* Handle on HIP device `device`. No reference counterpart: replaces the
 * zeroed FastCtx of fast_init (src/fast.c:29-32). */
int  cngpt_hip_create(int device, cngpt_hip_ctx **out);
/* Frees the handle, its stream and both device allocations
 * (fast_free, src/fast.c:34-40). NULL is a no-op. */
void cngpt_hip_destroy(cngpt_hip_ctx *h);

/* Number of floats in the flat parameter buffer for cfg
 * (gpt_num_params, src/model.c:20-48), or -1 for an invalid shape. */
long cngpt_hip_num_params(const cngpt_hip_config *cfg);

/* Copy the flat fp32 parameter buffer (layout of assign_weights,
 * src/model.c:54-83) into the handle's single parameter allocation.
 * Replaces the live reads of m->params that gpt_forward_fast makes
 * (src/fast.c:245-329); call again whenever the host buffer changes. */
int  cngpt_hip_load_params(cngpt_hip_ctx *h, const cngpt_hip_config *cfg,
                           const float *params, long n_params);

/* Shape and parameter count in the header of a weight file (GPTHeader,
 * src/model.h:19-30), validated as cngpt_hip_load_file does: magic, version
 * 1, a valid shape, and at least n_params floats after the 28-byte header
 * (gpt_load's checks, src/model.c:185-207, plus the version and shape).
 * Touches no GPU. cfg and n_params may be NULL. */
int  cngpt_hip_file_config(const char *path, cngpt_hip_config *cfg, long *n_params);
/* Load a weight file straight into the handle's parameter allocation:
 * the header is validated as above, then the parameters are read in
 * chunks into pinned staging buffers by a few reader threads and copied to
 * the device as they arrive, with no host copy of the whole buffer (gpt_load,
 * src/model.c:177-211, reads it into the host param_buf, and gpt_init,
 * model.c:120-135, allocates four such buffers first). cfg_out (may be NULL)
 * receives the shape. On failure the handle holds no parameters. */
int  cngpt_hip_load_file(cngpt_hip_ctx *h, const char *path, cngpt_hip_config *cfg_out);

/* Size the activation allocation for B sequences of T tokens (and a decode
 * KV cache of kv_capacity positions per sequence; 0 = none). Replaces
 * fast_resize (src/fast.c:140-168). forward/decode call it as needed. */
int  cngpt_hip_reserve(cngpt_hip_ctx *h, int B, int T, int mode, int kv_capacity);

/* Forward pass over host tokens [B, T] (validated: 0 <= id < vocab_size,
 * T <= block_size). mode CNGPT_LAST copies [B, V] logits to logits_out
 * when it is not NULL; CNGPT_ALL keeps [B, T, V] on the device and copies
 * them only when logits_out is not NULL. Blocks until done.
 * gpt_forward_fast (src/fast.c:227-333), plus the all-positions mode. */
int  cngpt_hip_forward(cngpt_hip_ctx *h, const int *tokens, int B, int T, int mode,
                       float *logits_out);

/* Split form for callers that keep inputs in HBM: upload tokens [B, T]
 * once, then enqueue forwards on the handle's stream without blocking. */
int  cngpt_hip_upload_tokens(cngpt_hip_ctx *h, const int *tokens, int B, int T);
int  cngpt_hip_forward_resident(cngpt_hip_ctx *h, int B, int T, int mode);
int  cngpt_hip_synchronize(cngpt_hip_ctx *h);
/* Forward pass that allocates nothing: no reference counterpart; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same kernels and
 * results as cngpt_hip_forward_resident, but tokens [B, T] (device int32,
 * ids in [0, vocab_size)) and logits (device; [B, V] for CNGPT_LAST,
 * [B, T, V] for CNGPT_ALL) are the caller's, and every activation lives in a
 * 128 MiB scratch array of the library that each device holds from its first
 * use until the process ends (a 1024-token window of GPT-2 small or medium
 * fits; larger B * T * n_embd is refused with an error). Needs parameters
 * (cngpt_hip_load_params or _load_file) but no cngpt_hip_reserve. Enqueues
 * on the handle's stream and returns without waiting. Token ids outside
 * [0, vocab_size) are clamped and set *err (device int, may be NULL), which
 * the call zeroes first. All calls on one device share its scratch and it
 * keeps the last call's contents: calls that overlap on one device (other
 * handles, other streams) race. */
int  cngpt_hip_forward_noalloc(cngpt_hip_ctx *h, const int *tokens, int B, int T, int mode,
                               float *logits, int *err);
/* Copy count floats of the logits, starting at float offset, to host. */
int  cngpt_hip_read_logits(cngpt_hip_ctx *h, size_t offset, size_t count, float *dst);
/* Device address of the logits of the last forward / decode step. */
const float *cngpt_hip_logits_device(cngpt_hip_ctx *h);

/* Cross-entropy of the logits held on the device against targets [B, T]
 * (host ids, validated 0 <= id < vocab_size): cross_entropy_fwd
 * (src/ops.c:499-574) as gpt_forward calls it after the lm_head
 * (src/model.c:617-623). The held logits must be B*T rows: the [B, T, V]
 * of a CNGPT_ALL forward, or with T = 1 the [B, V] of a CNGPT_LAST forward
 * or a decode step. Row r's term is log(sum_v exp(logit_v - max)) -
 * (logit[target] - max); *loss_out (may be NULL) receives their mean over
 * the B*T rows, row_loss (may be NULL) the B*T terms. probs != 0 also
 * replaces the held logits by their softmax, in place (probs_out of
 * cross_entropy_fwd, same [B*T, V] layout; read_logits then returns
 * probabilities). Blocks until done. */
int  cngpt_hip_cross_entropy(cngpt_hip_ctx *h, const int *targets, int B, int T, int probs,
                             float *loss_out, float *row_loss);
/* Split form: upload targets [B, T] once (validated as above; the
 * activation allocation must hold B*T rows, see cngpt_hip_reserve), enqueue
 * the loss on the handle's stream without blocking, then read the mean and
 * (optionally) the row terms of the last cross-entropy (row_loss must hold
 * the B*T floats of that call). */
int  cngpt_hip_upload_targets(cngpt_hip_ctx *h, const int *targets, int B, int T);
int  cngpt_hip_cross_entropy_resident(cngpt_hip_ctx *h, int B, int T, int probs);
int  cngpt_hip_read_loss(cngpt_hip_ctx *h, float *loss_out, float *row_loss);

/* Incremental decode with a device KV cache (no reference counterpart:
 * gpt_sample, src/model.c:991-1016, recomputes the whole prefix).
 * decode_begin runs the prompt [B, T] through the forward, keeps every
 * layer's K and V for up to `capacity` positions per sequence
 * (T < capacity <= block_size), leaves the last-position logits [B, V]
 * in logits_out (may be NULL) and their greedy tokens on the device.
 * decode_step appends one token per sequence (tokens [B] from the host, or,
 * when tokens is NULL, the token the device selected from the previous
 * logits: their argmax, or the sampled token after cngpt_hip_generate with
 * draws) and produces the next [B, V] logits. The step runs as one
 * replayed HIP graph. */
int  cngpt_hip_decode_begin(cngpt_hip_ctx *h, const int *prompt, int B, int T, int capacity,
                            float *logits_out);
int  cngpt_hip_decode_step(cngpt_hip_ctx *h, const int *tokens, float *logits_out);
/* n_new tokens per sequence after decode_begin (the loop of gpt_sample,
 * src/model.c:991-1016, with the KV cache): token 0 is selected from the
 * current logits, each further token from the logits of one more decode
 * step fed the previous token. draws == NULL: greedy (argmax, first index on
 * ties). Otherwise draws[i * B + b] is the uniform draw in [0, 1) for token
 * i of sequence b, and tokens are selected with the arithmetic of
 * sample_top_k (src/model.c:927-989; temperature <= 0 means 1, top_k <= 0 or
 * >= vocab_size means no cut). out_tokens is [B, n_new]. Needs
 * decode_length() + n_new - 1 <= capacity. */
int  cngpt_hip_generate(cngpt_hip_ctx *h, int n_new, float temperature, int top_k,
                        const float *draws, int *out_tokens);
/* Greedy token per sequence from the current logits (first index on ties). */
int  cngpt_hip_argmax(cngpt_hip_ctx *h, int *out_tokens);
/* One token per sequence from the current logits by sample_top_k's
 * arithmetic (src/model.c:927-989), draws [B] uniform in [0, 1). */
int  cngpt_hip_sample(cngpt_hip_ctx *h, float temperature, int top_k, const float *draws,
                      int *out_tokens);
/* Positions held in the KV cache per sequence (prompt + steps). */
int  cngpt_hip_decode_length(cngpt_hip_ctx *h);
/* Decode path for the following steps (CNGPT_DECODE_*; the default is AUTO,
 * or KERNELS when CNGPT_HIP_PERSIST=0 was set at create time). Asking for
 * PERSISTENT makes a step that cannot run that way fail. No reference
 * counterpart: the reference has one CPU path. */
int  cngpt_hip_set_decode_path(cngpt_hip_ctx *h, int path);
/* The path the last decode step ran on (CNGPT_DECODE_KERNELS or
 * CNGPT_DECODE_PERSISTENT; 0 before any step). */
int  cngpt_hip_decode_path(cngpt_hip_ctx *h);

/* Per-kernel-class timing with HIP events on the handle's stream.
 * While enabled, every launch is bracketed by an event pair; read returns
 * the summed kernel milliseconds, the launch count and the algorithmic
 * FLOPs and HBM bytes of those launches (synchronizes the stream). */
int  cngpt_hip_profile_enable(cngpt_hip_ctx *h, int on);
int  cngpt_hip_profile_reset(cngpt_hip_ctx *h);
int  cngpt_hip_profile_read(cngpt_hip_ctx *h, int kernel_class, double *ms, long *launches,
                            double *flops, double *bytes);

/* Pinned host memory, used for staging logits (fast.h's FastCtx).
 * NULL on failure. */
void *cngpt_hip_host_alloc(size_t bytes);
void  cngpt_hip_host_free(void *p);

/* Host-side seeded init for synthetic weights: srand(seed) then the
 * N(0, 0.02) / residual-scaled draw order of gpt_init_weights
 * (src/model.c:275-331), into a host buffer of cngpt_hip_num_params floats.
 * Needs no GPU. */
int  cngpt_hip_init_weights(const cngpt_hip_config *cfg, float *params, unsigned seed);

/* ------------------------------------------------------------------
 * Training on the device: the reference's gpt_forward with targets,
 * gpt_backward, gpt_zero_grad and gpt_adamw (src/model.h:163-187,
 * src/model.c:333-921) over the handle's parameters, which the update
 * changes in place (later forwards and decodes on the handle see them).
 * A trainer holds, for one B x T, the activations gpt_forward keeps for
 * gpt_backward (GPTActivations, src/model.h:86-115, with each attention's
 * log-sum-exp in place of its T x T probabilities), the gradients
 * (GPTGrads) and the AdamW moments (m_buf, v_buf, decay_buf,
 * src/model.h:120-141). The configuration carries no dropout rate:
 * cngpt_hip_train_set_dropout sets GPTConfig.dropout for the trainer (0,
 * the default of `cngpt train`, src/cngpt.c:94, until then).
 * ------------------------------------------------------------------ */
typedef struct cngpt_hip_train cngpt_hip_train;

/* gpt_resize_acts (model.c:333-440) for B x T plus the gradient and moment
 * buffers (gpt_init's grad_buf, m_buf, v_buf, zeroed); the handle must
 * hold parameters and outlive the trainer. */
int  cngpt_hip_train_create(cngpt_hip_ctx *h, int B, int T, cngpt_hip_train **out);
void cngpt_hip_train_destroy(cngpt_hip_train *t);

/* gpt_forward(m, tokens, targets, B, T) (model.c:442-625): host token and
 * target ids [B*T], the mean cross-entropy in *loss (synchronizes). Ids
 * outside [0, V) fail before any work. */
int  cngpt_hip_train_forward(cngpt_hip_train *t, const int *tokens, const int *targets,
                             float *loss);

/* gpt_backward (model.c:634-877) for the last forward: gradients add to
 * the held ones, as in the reference. */
int  cngpt_hip_train_backward(cngpt_hip_train *t);

/* GPTConfig.dropout (src/model.h:43) for this trainer's forwards, p in
 * [0, 1): with p > 0 every cngpt_hip_train_forward draws the keep masks of
 * dropout_fwd (src/ops.c:603-618) with the process's rand(), one call per
 * element in model.c's order (the embedding, then res1 and res2 of each
 * layer: model.c:471-472, 572-574, 597-599; (1 + 2 n_layer) B T n_embd
 * draws), as the reference's gpt_forward with targets does, applies them on
 * the device, and the backward applies dropout_bwd at model.c:699-700,
 * 732-733 and 849-850. Allocates the masks' device bytes on first use. */
int  cngpt_hip_train_set_dropout(cngpt_hip_train *t, float p);

/* gpt_zero_grad (model.c:879-886). */
int  cngpt_hip_train_zero_grad(cngpt_hip_train *t);

/* gpt_adamw(m, lr, beta1, beta2, eps, weight_decay, grad_clip)
 * (model.c:888-921): step += 1; with grad_clip > 0 the gradients are
 * scaled by grad_clip / norm when their global L2 norm exceeds it; then
 * AdamW with bias correction and decoupled weight decay on the matrices
 * and embeddings (the decay mask of model.c:143-172). The norm before
 * clipping goes to *grad_norm when that is not NULL (synchronizes then). */
int  cngpt_hip_train_adamw(cngpt_hip_train *t, float lr, float beta1, float beta2, float eps,
                           float weight_decay, float grad_clip, float *grad_norm);

/* Flat buffers of cngpt_hip_num_params floats in the weight-file layout. */
enum { CNGPT_TRAIN_PARAMS = 0, CNGPT_TRAIN_GRADS = 1, CNGPT_TRAIN_M = 2, CNGPT_TRAIN_V = 3 };
/* Copy n floats of buffer `which` to the host (synchronizes). */
int  cngpt_hip_train_read(cngpt_hip_train *t, int which, float *dst, long n);
/* Overwrite the gradients or a moment buffer (not the parameters: load
 * them through cngpt_hip_load_params) with n host floats. */
int  cngpt_hip_train_write(cngpt_hip_train *t, int which, const float *src, long n);
/* Optimizer steps taken (gpt_adamw's m->step). */
int  cngpt_hip_train_steps(cngpt_hip_train *t);

#ifdef __cplusplus
}
#endif
#endif /* CNGPT_HIP_H */
