// train_host.cpp - the training step on the device (the cngpt_hip_train_* entry
// points of include/cngpt_hip.h): the reference's gpt_forward with targets,
// gpt_backward, gpt_zero_grad and gpt_adamw (src/model.c:442-921).
//
// Forward (model.c:442-625): embed -> per layer { LN1 (mean, rstd kept) ->
// QKV product -> causal attention (its base-2 log-sum-exp kept) -> res1 =
// x + c_proj product -> LN2 -> fc product (pre-activation kept) -> GELU ->
// res2 = res1 + proj product } -> LN_f -> lm_head -> cross-entropy, whose
// pass also writes the gradient of the loss over the logits (the
// reference keeps the probabilities and forms it in gpt_backward).
//
// Backward (model.c:634-877), per linear layer Y = X W^T + b:
//   dX = dY W           product of dY [rows, out] and W^T [in, out]
//   dW += dY^T X        product of dY^T [out, rows] and X^T [in, rows]
//   db += column sums of dY
// The product kernels take both operands K-contiguous (the reference's
// cblas_sgemm(NoTrans, Trans) form, fast.c:175-205), so the operand whose K
// is a row index is transposed first (W for dX; dY and X for dW, their
// rows padded with zeros to whole product steps), and dW accumulates into
// the gradient through the residual epilogue with a zero bias. LayerNorm,
// GELU, cross-entropy and embedding backwards are the kernels of
// train.hip, attention's is attn_bwd.hip. Every sum is formed in a fixed
// order, so a step is reproducible bit for bit.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <vector>

#include "../../include/cngpt_hip.h"
#include "common.h"
#include "ctx_view.h"
#include "kernels.h"

namespace {

#define TRY(expr)                                                                             \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess)                                                                 \
            return ctx_fail("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                            __LINE__);                                                        \
    } while (0)

constexpr long PART_FLOATS = 1l << 24;  // split-K partials of the products (64 MB)

long round_up(long n, long m) { return (n + m - 1) / m * m; }

}  // namespace

// Activations of one layer (GPTActivations, src/model.h:86-115).
struct TrainLayer {
    float *ln1_out, *ln1_mean, *ln1_rstd, *qkv, *lse, *attn_out, *res1;
    float *ln2_out, *ln2_mean, *ln2_rstd, *fc_out, *gelu, *res2;
};

struct cngpt_hip_train {
    cngpt_hip_ctx* h = nullptr;
    int B = 0, T = 0;
    long N = 0;   // rows B*T
    long Np = 0;  // rows padded to whole product steps (K of the dW products)
    long Vp = 0;  // vocabulary padded likewise (K of the lm_head's dX product)
    cngpt_hip_config cfg{};
    long n_params = 0;
    const float* params_seen = nullptr;  // parameter allocation the trainer was made for
    int device = 0;

    char* arena = nullptr;
    float *grads = nullptr, *m = nullptr, *v = nullptr;
    unsigned char* decay = nullptr;
    int step = 0;

    float* emb = nullptr;
    std::vector<TrainLayer> acts;
    float *lnf_out = nullptr, *lnf_mean = nullptr, *lnf_rstd = nullptr, *logits = nullptr;
    int *tok = nullptr, *tgt = nullptr, *uniq = nullptr, *ustart = nullptr, *upos = nullptr;
    int nuniq = 0;
    float *row_loss = nullptr, *loss = nullptr;
    int* err = nullptr;

    float *dlog = nullptr, *d_x = nullptr, *d_res1 = nullptr, *d_ln = nullptr;
    float *d_attn = nullptr, *d_qkv = nullptr, *d_hid = nullptr, *Dbuf = nullptr;
    float *tA = nullptr, *tB = nullptr, *tW = nullptr;
    float *part = nullptr, *red = nullptr, *zeros = nullptr;
    double* nparts = nullptr;
    float *norm = nullptr, *coef = nullptr;
    bool have_fwd = false;

    // GPTConfig.dropout (model.h:43): the keep masks of the last forward,
    // [1 + 2 L][B T C] bytes (the embedding, then res1 and res2 of each
    // layer), drawn on the host with rand() in model.c's order
    float dropout = 0.f;
    unsigned char* masks = nullptr;
    std::vector<unsigned char> hmasks;
    bool dropped = false;
};

namespace {

// The handle's current view, checked against the shape and parameter
// allocation the trainer was made for.
int view_of(cngpt_hip_train* t, CtxView* v) {
    if (!t) return ctx_fail("null trainer");
    if (ctx_view(t->h, v)) return -1;
    if (memcmp(&v->cfg, &t->cfg, sizeof(t->cfg)) != 0 || v->params != t->params_seen)
        return ctx_fail("the handle's parameters were reallocated since the trainer was made");
    TRY(hipSetDevice(v->device));
    return 0;
}

float* grad_of(const cngpt_hip_train* t, const CtxView& v, const float* p) {
    return t->grads + (p - v.params);
}

// Y[M, N] = epi(X[M, K] . W[N, K]^T) (row strides K and N).
int gemm(cngpt_hip_train* t, hipStream_t s, const float* X, const float* W, const float* bias,
         float* Y, long M, long N, long K, int epi) {
    GemmArgs a{};
    a.X = X; a.W = W; a.bias = bias; a.Y = Y;
    a.M = (int)M; a.N = (int)N; a.K = (int)K;
    a.ldy = N;
    a.epi = epi;
    a.part = t->part;
    a.part_cap = PART_FLOATS;
    TRY(launch_gemm(a, s));
    return 0;
}

// dX [rows, in] = dY [rows, out] . W [out, in] (overwrites dX). Over more
// than SKINNY_MAX_M rows with out a multiple of 32, the product reads W as
// stored, K-major (row k = output k); otherwise through a transposed copy.
int linear_dx(cngpt_hip_train* t, hipStream_t s, const float* dY, const float* W, float* dX,
              long out, long in) {
    if (t->N > SKINNY_MAX_M && out % 32 == 0 && in % 4 == 0) {
        GemmArgs a{};
        a.X = dY; a.W = W; a.ldw = in; a.km = 2;
        a.Y = dX;
        a.M = (int)t->N; a.N = (int)in; a.K = (int)out;
        a.ldy = in;
        a.epi = EPI_STORE;
        a.part = t->part;
        a.part_cap = PART_FLOATS;
        TRY(launch_gemm(a, s));
        return 0;
    }
    TRY(launch_transpose(W, in, (int)out, (int)in, t->tW, out, (int)out, (int)in, s));
    return gemm(t, s, dY, t->tW, nullptr, dX, t->N, in, out, EPI_STORE);
}

// dW [out, in] += dY^T . X, db [out] += column sums of dY (db may be null);
// dY rows are ldy floats apart, X rows `in`. Over more than SKINNY_MAX_M
// outputs the product reads dY and X K-major, straight from their row
// buffers (rows N .. Np-1 of which are zero); fewer go through transposed
// copies (the few-row products take K-contiguous operands only).
int linear_dw(cngpt_hip_train* t, hipStream_t s, const float* dY, long ldy, const float* X,
              float* dW, float* db, long out, long in) {
    const int N = (int)t->N, Np = (int)t->Np;
    if (out > SKINNY_MAX_M) {
        if (db) TRY(launch_colsum_add(dY, ldy, N, (int)out, t->red, db, s));
        GemmArgs a{};
        a.X = dY; a.ldx = ldy; a.W = X; a.ldw = in; a.km = 3;
        a.bias = t->zeros; a.Y = dW;
        a.M = (int)out; a.N = (int)in; a.K = Np;
        a.ldy = in;
        a.epi = EPI_RESID;
        a.part = t->part;
        a.part_cap = PART_FLOATS;
        TRY(launch_gemm(a, s));
        return 0;
    }
    if (db)
        TRY(launch_transpose_colsum(dY, ldy, N, (int)out, t->tA, Np, Np, (int)out, t->red, db, s));
    else
        TRY(launch_transpose(dY, ldy, N, (int)out, t->tA, Np, Np, (int)out, s));
    TRY(launch_transpose(X, in, N, (int)in, t->tB, Np, Np, (int)in, s));
    return gemm(t, s, t->tA, t->tB, t->zeros, dW, out, in, Np, EPI_RESID);
}

int check_ids(const int* ids, long n, int V, const char* what) {
    if (!ids) return ctx_fail("null %s", what);
    for (long i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= V)
            return ctx_fail("%s %d at index %ld outside [0, %d)", what, ids[i], i, V);
    return 0;
}

}  // namespace

extern "C" {

int cngpt_hip_train_create(cngpt_hip_ctx* h, int B, int T, cngpt_hip_train** out) {
    if (!out) return ctx_fail("null output pointer");
    *out = nullptr;
    CtxView v;
    if (ctx_view(h, &v)) return -1;
    const cngpt_hip_config& c = v.cfg;
    if (B <= 0 || T <= 0 || T > c.block_size)
        return ctx_fail("batch %d x %d outside 1..%d positions", B, T, c.block_size);
    const long C = c.n_embd, V = c.vocab_size, L = c.n_layer, H = c.n_head;
    if (C % 4 || C > 2048) return ctx_fail("training needs n_embd a multiple of 4, at most 2048");
    if (C / H != 8 && C / H != 16 && C / H != 32 && C / H != 64 && C / H != 128)
        return ctx_fail("head size %ld not one of 8, 16, 32, 64, 128", C / H);
    TRY(hipSetDevice(v.device));

    auto* t = new cngpt_hip_train;
    t->h = h;
    t->B = B;
    t->T = T;
    t->N = (long)B * T;
    t->Np = round_up(t->N, 32);
    t->Vp = round_up(V, 32);
    t->cfg = c;
    t->n_params = v.n_params;
    t->params_seen = v.params;
    t->device = v.device;
    const long N = t->N, Np = t->Np, Vp = t->Vp, n = v.n_params;

    // one allocation, carved in this order; buffers of B*T rows hold Np rows
    // (the padding rows stay zero: the dW products read them as K)
    std::vector<size_t> sz;
    auto fl = [&](long count) { sz.push_back((size_t)std::max(count, 1L) * sizeof(float)); };
    fl(n); fl(n); fl(n);                     // grads, m, v
    sz.push_back((size_t)n);                  // decay mask
    fl(Np * C);                               // emb
    for (long l = 0; l < L; l++) {
        fl(Np * C); fl(N); fl(N);             // ln1_out, mean, rstd
        fl(Np * 3 * C); fl(B * H * T);        // qkv, lse
        fl(Np * C); fl(Np * C);               // attn_out, res1
        fl(Np * C); fl(N); fl(N);             // ln2_out, mean, rstd
        fl(Np * 4 * C); fl(Np * 4 * C);       // fc_out, gelu
        fl(Np * C);                           // res2
    }
    fl(Np * C); fl(N); fl(N); fl(N * V);      // lnf_out, mean, rstd, logits
    for (int i = 0; i < 5; i++) fl(N + 1);    // tok, tgt, uniq, ustart, upos
    fl(N); fl(1); fl(4);                      // row_loss, loss, err
    fl(Np * Vp);                              // dlog
    fl(Np * C); fl(Np * C); fl(Np * C); fl(Np * C);  // d_x, d_res1, d_ln, d_attn
    fl(Np * 3 * C); fl(Np * 4 * C); fl(B * H * T);   // d_qkv, d_hid, D
    // transposed operands of the dW products with at most SKINNY_MAX_M
    // outputs (dY^T, X^T), and of every dX product (W^T)
    long ta = 0, tb = 0;
    const long dw_shapes[5][2] = {{C, 4 * C}, {4 * C, C}, {C, C}, {3 * C, C}, {V, C}};
    for (const auto& d : dw_shapes)
        if (d[0] <= SKINNY_MAX_M) {
            ta = std::max(ta, d[0] * Np);
            tb = std::max(tb, d[1] * Np);
        }
    fl(ta); fl(tb);                           // tA, tB
    fl(std::max(C * Vp, 4 * C * C));          // tW
    fl(PART_FLOATS);                          // part
    fl(std::max({transpose_colsum_floats((int)Np, (int)(4 * C)),
                 colsum_part_floats((int)N, (int)(4 * C)),
                 ln_bwd_part_floats((int)N, (int)C)}));
    fl(4 * C);                                // zeros
    sz.push_back((size_t)grad_norm_parts(n) * sizeof(double));
    fl(1); fl(1);                             // norm, coef
    size_t total = 0;
    for (size_t b : sz) total += (b + 255) & ~(size_t)255;
    if (hipMalloc(&t->arena, total) != hipSuccess) {
        (void)hipGetLastError();
        delete t;
        return ctx_fail("training allocation of %zu bytes failed", total);
    }
    size_t off = 0, k = 0;
    auto take = [&]() {
        char* p = t->arena + off;
        off += (sz[k++] + 255) & ~(size_t)255;
        return p;
    };
    t->grads = (float*)take(); t->m = (float*)take(); t->v = (float*)take();
    t->decay = (unsigned char*)take();
    t->emb = (float*)take();
    t->acts.resize(L);
    for (auto& a : t->acts) {
        a.ln1_out = (float*)take(); a.ln1_mean = (float*)take(); a.ln1_rstd = (float*)take();
        a.qkv = (float*)take(); a.lse = (float*)take();
        a.attn_out = (float*)take(); a.res1 = (float*)take();
        a.ln2_out = (float*)take(); a.ln2_mean = (float*)take(); a.ln2_rstd = (float*)take();
        a.fc_out = (float*)take(); a.gelu = (float*)take();
        a.res2 = (float*)take();
    }
    t->lnf_out = (float*)take(); t->lnf_mean = (float*)take(); t->lnf_rstd = (float*)take();
    t->logits = (float*)take();
    t->tok = (int*)take(); t->tgt = (int*)take(); t->uniq = (int*)take();
    t->ustart = (int*)take(); t->upos = (int*)take();
    t->row_loss = (float*)take(); t->loss = (float*)take(); t->err = (int*)take();
    t->dlog = (float*)take();
    t->d_x = (float*)take(); t->d_res1 = (float*)take(); t->d_ln = (float*)take();
    t->d_attn = (float*)take();
    t->d_qkv = (float*)take(); t->d_hid = (float*)take(); t->Dbuf = (float*)take();
    t->tA = (float*)take(); t->tB = (float*)take(); t->tW = (float*)take();
    t->part = (float*)take(); t->red = (float*)take(); t->zeros = (float*)take();
    t->nparts = (double*)take();
    t->norm = (float*)take(); t->coef = (float*)take();

    // the decay mask of gpt_init (model.c:143-172): wte, wpe and the four
    // matrices of every layer decay; LayerNorm gains and biases do not
    std::vector<unsigned char> mask((size_t)n, 0);
    auto mark = [&](const float* p, long count) {
        std::fill(mask.begin() + (p - v.params), mask.begin() + (p - v.params) + count, 1);
    };
    mark(v.wte, V * C);
    mark(v.wpe, (long)c.block_size * C);
    for (long l = 0; l < L; l++) {
        const LayerW& w = v.layers[l];
        mark(w.attn_w, 3 * C * C);
        mark(w.proj_w, C * C);
        mark(w.fc_w, 4 * C * C);
        mark(w.mlp_w, 4 * C * C);
    }
    hipStream_t s = v.stream;
    int rc = 0;
    // everything starts at zero: gradients, moments, the zero bias, the
    // error flags and the padding rows
    if (hipMemsetAsync(t->arena, 0, total, s) != hipSuccess ||
        hipMemcpyAsync(t->decay, mask.data(), (size_t)n, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        rc = ctx_fail("trainer set-up failed: %s", hipGetErrorString(hipGetLastError()));
    if (rc) {
        (void)hipFree(t->arena);
        delete t;
        return -1;
    }
    *out = t;
    return 0;
}

void cngpt_hip_train_destroy(cngpt_hip_train* t) {
    if (!t) return;
    (void)hipSetDevice(t->device);
    (void)hipDeviceSynchronize();
    if (t->arena) (void)hipFree(t->arena);
    if (t->masks) (void)hipFree(t->masks);
    delete t;
}

int cngpt_hip_train_set_dropout(cngpt_hip_train* t, float p) {
    CtxView v;
    if (view_of(t, &v)) return -1;
    if (!(p >= 0.f) || !(p < 1.f)) return ctx_fail("dropout rate %g outside [0, 1)", (double)p);
    if (p > 0.f && !t->masks) {
        const size_t n = (size_t)(1 + 2 * t->cfg.n_layer) * t->N * t->cfg.n_embd;
        TRY(hipSetDevice(t->device));
        if (hipMalloc(&t->masks, n) != hipSuccess) {
            (void)hipGetLastError();
            t->masks = nullptr;
            return ctx_fail("dropout mask allocation of %zu bytes failed", n);
        }
        t->hmasks.resize(n);
    }
    t->dropout = p;
    return 0;
}

int cngpt_hip_train_forward(cngpt_hip_train* t, const int* tokens, const int* targets,
                            float* loss) {
    CtxView v;
    if (view_of(t, &v)) return -1;
    const cngpt_hip_config& c = t->cfg;
    const int B = t->B, T = t->T, C = c.n_embd, V = c.vocab_size, H = c.n_head;
    const long N = t->N;
    if (check_ids(tokens, N, V, "token") || check_ids(targets, N, V, "target")) return -1;
    hipStream_t s = v.stream;

    // distinct tokens and their positions in order, for the embedding's
    // gradient (model.c:859-866 adds rows position by position)
    std::vector<int> order(N);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(),
                     [&](int a, int b) { return tokens[a] < tokens[b]; });
    std::vector<int> uniq, start;
    for (long i = 0; i < N; i++)
        if (i == 0 || tokens[order[i]] != tokens[order[i - 1]]) {
            uniq.push_back(tokens[order[i]]);
            start.push_back((int)i);
        }
    start.push_back((int)N);
    t->nuniq = (int)uniq.size();
    TRY(hipMemcpyAsync(t->tok, tokens, N * sizeof(int), hipMemcpyHostToDevice, s));
    TRY(hipMemcpyAsync(t->tgt, targets, N * sizeof(int), hipMemcpyHostToDevice, s));
    TRY(hipMemcpyAsync(t->uniq, uniq.data(), uniq.size() * sizeof(int), hipMemcpyHostToDevice, s));
    TRY(hipMemcpyAsync(t->ustart, start.data(), start.size() * sizeof(int), hipMemcpyHostToDevice,
                       s));
    TRY(hipMemcpyAsync(t->upos, order.data(), N * sizeof(int), hipMemcpyHostToDevice, s));

    // dropout (model.c:450: in every forward with targets when the rate is
    // set): dropout_fwd's draws (ops.c:603-618), one rand() per element,
    // kept when it exceeds p * RAND_MAX, for the embedding and then res1
    // and res2 of each layer; then the keep masks go to the device
    const float p = t->dropout;
    const bool drop = p > 0.f;
    const long NC = N * C;
    const float dscale = drop ? 1.0f / (1.0f - p) : 1.0f;
    if (drop) {
        unsigned char* hm = t->hmasks.data();
        const size_t n = t->hmasks.size();
        for (size_t i = 0; i < n; i++) {
            const unsigned int r = (unsigned int)rand();
            hm[i] = r > (unsigned int)(p * (float)RAND_MAX) ? 1 : 0;
        }
        TRY(hipMemcpyAsync(t->masks, hm, n, hipMemcpyHostToDevice, s));
    }
    t->dropped = drop;

    TRY(launch_embed(t->tok, v.wte, v.wpe, t->emb, N, T, C, V, 0, nullptr, t->err, nullptr, 0, s));
    if (drop) TRY(launch_dropout(t->emb, t->masks, NC, dscale, s));   // model.c:471-472
    const float* x = t->emb;
    const size_t xbytes = (size_t)N * C * sizeof(float);
    for (int l = 0; l < c.n_layer; l++) {
        const LayerW& w = v.layers[l];
        TrainLayer& a = t->acts[l];
        TRY(launch_layernorm(x, C, w.ln1_w, w.ln1_b, a.ln1_out, C, (int)N, C, s, a.ln1_mean,
                             a.ln1_rstd));
        if (gemm(t, s, a.ln1_out, w.attn_w, w.attn_b, a.qkv, N, 3 * C, C, EPI_BIAS)) return -1;
        TRY(launch_attention_causal(a.qkv, T, a.attn_out, B, T, C, H, s, a.lse));
        TRY(hipMemcpyAsync(a.res1, x, xbytes, hipMemcpyDeviceToDevice, s));
        if (gemm(t, s, a.attn_out, w.proj_w, w.proj_b, a.res1, N, C, C, EPI_RESID)) return -1;
        if (drop) TRY(launch_dropout(a.res1, t->masks + (1 + 2 * l) * NC, NC, dscale, s));
        TRY(launch_layernorm(a.res1, C, w.ln2_w, w.ln2_b, a.ln2_out, C, (int)N, C, s, a.ln2_mean,
                             a.ln2_rstd));
        if (gemm(t, s, a.ln2_out, w.fc_w, w.fc_b, a.fc_out, N, 4 * C, C, EPI_BIAS)) return -1;
        TRY(launch_gelu_fwd(a.fc_out, a.gelu, N * 4 * C, s));
        TRY(hipMemcpyAsync(a.res2, a.res1, xbytes, hipMemcpyDeviceToDevice, s));
        if (gemm(t, s, a.gelu, w.mlp_w, w.mlp_b, a.res2, N, C, 4 * C, EPI_RESID)) return -1;
        if (drop) TRY(launch_dropout(a.res2, t->masks + (2 + 2 * l) * NC, NC, dscale, s));
        x = a.res2;
    }
    TRY(launch_layernorm(x, C, v.lnf_w, v.lnf_b, t->lnf_out, C, (int)N, C, s, t->lnf_mean,
                         t->lnf_rstd));
    if (gemm(t, s, t->lnf_out, v.wte, nullptr, t->logits, N, V, C, EPI_STORE)) return -1;
    // the loss, and the gradient of the mean loss for the backward
    // (cross_entropy_bwd) into the padded dlogits rows, from one read of the
    // logits
    TRY(launch_cross_entropy(t->logits, N, V, t->tgt, t->row_loss, t->loss, 0, t->err, s, t->dlog,
                             t->Vp));
    float lv = 0.f;
    int e = 0;
    TRY(hipMemcpyAsync(&lv, t->loss, sizeof(float), hipMemcpyDeviceToHost, s));
    TRY(hipMemcpyAsync(&e, t->err, sizeof(int), hipMemcpyDeviceToHost, s));
    TRY(hipStreamSynchronize(s));
    if (e) return ctx_fail("device reported error flags 0x%x in the training forward", e);
    t->have_fwd = true;
    if (loss) *loss = lv;
    return 0;
}

int cngpt_hip_train_backward(cngpt_hip_train* t) {
    CtxView v;
    if (view_of(t, &v)) return -1;
    if (!t->have_fwd) return ctx_fail("no training forward to differentiate");
    const cngpt_hip_config& c = t->cfg;
    const int B = t->B, T = t->T, C = c.n_embd, V = c.vocab_size, H = c.n_head;
    const long N = t->N;
    hipStream_t s = v.stream;
    const size_t xbytes = (size_t)N * C * sizeof(float);
    const long NC = N * C;
    const bool drop = t->dropped;
    const float dscale = drop ? 1.0f / (1.0f - t->dropout) : 1.0f;

    // dlogits = (probs - onehot) / (B T) (model.c:660-666) was formed by the
    // forward's loss pass; the tied lm_head: d ln_f = dlogits . wte,
    // d wte += dlogits^T . ln_f_out
    TRY(launch_transpose(v.wte, C, V, C, t->tW, t->Vp, (int)t->Vp, C, s));
    if (gemm(t, s, t->dlog, t->tW, nullptr, t->d_ln, N, C, t->Vp, EPI_STORE)) return -1;
    if (linear_dw(t, s, t->dlog, t->Vp, t->lnf_out, grad_of(t, v, v.wte), nullptr, V, C))
        return -1;
    // the final LayerNorm (its input gradient into a cleared d_x)
    TRY(hipMemsetAsync(t->d_x, 0, xbytes, s));
    const float* x_last = c.n_layer > 0 ? t->acts[c.n_layer - 1].res2 : t->emb;
    TRY(launch_layernorm_bwd(t->d_ln, x_last, v.lnf_w, t->lnf_mean, t->lnf_rstd, t->d_x,
                             grad_of(t, v, v.lnf_w), grad_of(t, v, v.lnf_b), (int)N, C, t->red, s));

    for (int l = c.n_layer - 1; l >= 0; l--) {
        const LayerW& w = v.layers[l];
        const TrainLayer& a = t->acts[l];
        const float* x_in = l > 0 ? t->acts[l - 1].res2 : t->emb;
        // dropout_bwd (ops.c:620-625) of res2 (model.c:699-700)
        if (drop) TRY(launch_dropout(t->d_x, t->masks + (2 + 2 * l) * NC, NC, dscale, s));
        TRY(hipMemcpyAsync(t->d_res1, t->d_x, xbytes, hipMemcpyDeviceToDevice, s));
        // proj: Y = gelu . mlp_w^T + b
        if (linear_dx(t, s, t->d_x, w.mlp_w, t->d_hid, C, 4 * C) ||
            linear_dw(t, s, t->d_x, C, a.gelu, grad_of(t, v, w.mlp_w), grad_of(t, v, w.mlp_b), C,
                      4 * C))
            return -1;
        TRY(launch_gelu_bwd(t->d_hid, a.fc_out, N * 4 * C, s));
        // fc: Y = ln2_out . fc_w^T + b
        if (linear_dx(t, s, t->d_hid, w.fc_w, t->d_ln, 4 * C, C) ||
            linear_dw(t, s, t->d_hid, 4 * C, a.ln2_out, grad_of(t, v, w.fc_w), grad_of(t, v, w.fc_b),
                      4 * C, C))
            return -1;
        TRY(launch_layernorm_bwd(t->d_ln, a.res1, w.ln2_w, a.ln2_mean, a.ln2_rstd, t->d_res1,
                                 grad_of(t, v, w.ln2_w), grad_of(t, v, w.ln2_b), (int)N, C, t->red,
                                 s));
        // and of res1 (model.c:732-733)
        if (drop) TRY(launch_dropout(t->d_res1, t->masks + (1 + 2 * l) * NC, NC, dscale, s));
        // c_proj: Y = attn_out . proj_w^T + b
        if (linear_dx(t, s, t->d_res1, w.proj_w, t->d_attn, C, C) ||
            linear_dw(t, s, t->d_res1, C, a.attn_out, grad_of(t, v, w.proj_w),
                      grad_of(t, v, w.proj_b), C, C))
            return -1;
        TRY(launch_attention_bwd(a.qkv, a.attn_out, t->d_attn, a.lse, t->Dbuf, t->d_qkv, B, T, C, H,
                                 s));
        // QKV: Y = ln1_out . attn_w^T + b
        if (linear_dx(t, s, t->d_qkv, w.attn_w, t->d_ln, 3 * C, C) ||
            linear_dw(t, s, t->d_qkv, 3 * C, a.ln1_out, grad_of(t, v, w.attn_w), grad_of(t, v, w.attn_b),
                      3 * C, C))
            return -1;
        TRY(hipMemcpyAsync(t->d_x, t->d_res1, xbytes, hipMemcpyDeviceToDevice, s));
        TRY(launch_layernorm_bwd(t->d_ln, x_in, w.ln1_w, a.ln1_mean, a.ln1_rstd, t->d_x,
                                 grad_of(t, v, w.ln1_w), grad_of(t, v, w.ln1_b), (int)N, C, t->red,
                                 s));
    }
    // and of the embedding (model.c:849-850)
    if (drop) TRY(launch_dropout(t->d_x, t->masks, NC, dscale, s));
    TRY(launch_embed_bwd(t->d_x, B, T, C, grad_of(t, v, v.wpe), grad_of(t, v, v.wte), t->uniq,
                         t->ustart, t->upos, t->nuniq, s));
    TRY(hipGetLastError());
    return 0;
}

int cngpt_hip_train_zero_grad(cngpt_hip_train* t) {
    CtxView v;
    if (view_of(t, &v)) return -1;
    TRY(hipMemsetAsync(t->grads, 0, (size_t)t->n_params * sizeof(float), v.stream));
    return 0;
}

int cngpt_hip_train_adamw(cngpt_hip_train* t, float lr, float beta1, float beta2, float eps,
                          float weight_decay, float grad_clip, float* grad_norm) {
    CtxView v;
    if (view_of(t, &v)) return -1;
    t->step += 1;
    const float bc1 = 1.0f - powf(beta1, (float)t->step);
    const float bc2 = 1.0f - powf(beta2, (float)t->step);
    TRY(launch_adamw(v.params, t->grads, t->m, t->v, t->decay, t->n_params, t->nparts, t->norm,
                     t->coef, lr, beta1, beta2, eps, weight_decay, grad_clip, bc1, bc2,
                     v.stream));
    ctx_params_written(t->h);  // the packed weight copies no longer match
    if (grad_norm) {
        TRY(hipMemcpyAsync(grad_norm, t->norm, sizeof(float), hipMemcpyDeviceToHost, v.stream));
        TRY(hipStreamSynchronize(v.stream));
    }
    return 0;
}

static float* buffer_of(cngpt_hip_train* t, const CtxView& v, int which) {
    switch (which) {
        case CNGPT_TRAIN_PARAMS: return v.params;
        case CNGPT_TRAIN_GRADS: return t->grads;
        case CNGPT_TRAIN_M: return t->m;
        case CNGPT_TRAIN_V: return t->v;
    }
    return nullptr;
}

int cngpt_hip_train_read(cngpt_hip_train* t, int which, float* dst, long n) {
    CtxView v;
    if (view_of(t, &v)) return -1;
    float* src = buffer_of(t, v, which);
    if (!src) return ctx_fail("unknown training buffer %d", which);
    if (!dst || n <= 0 || n > t->n_params)
        return ctx_fail("read of %ld floats outside 1..%ld", n, t->n_params);
    TRY(hipMemcpyAsync(dst, src, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, v.stream));
    TRY(hipStreamSynchronize(v.stream));
    return 0;
}

int cngpt_hip_train_write(cngpt_hip_train* t, int which, const float* src, long n) {
    CtxView v;
    if (view_of(t, &v)) return -1;
    if (which == CNGPT_TRAIN_PARAMS)
        return ctx_fail("parameters are written through cngpt_hip_load_params");
    float* dst = buffer_of(t, v, which);
    if (!dst) return ctx_fail("unknown training buffer %d", which);
    if (!src || n <= 0 || n > t->n_params)
        return ctx_fail("write of %ld floats outside 1..%ld", n, t->n_params);
    TRY(hipMemcpyAsync(dst, src, (size_t)n * sizeof(float), hipMemcpyHostToDevice, v.stream));
    TRY(hipStreamSynchronize(v.stream));
    return 0;
}

int cngpt_hip_train_steps(cngpt_hip_train* t) { return t ? t->step : -1; }

}  // extern "C"
