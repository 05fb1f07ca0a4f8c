// kernels.h - host-side launchers of the gfx950 kernels (all enqueue on the
// given stream and return the launch status; none synchronizes).
#pragma once
#include <hip/hip_runtime.h>

// rowops.hip
hipError_t launch_embed(const int* tok, const float* wte, const float* wpe, float* x, long rows,
                        int T, int C, int V, int pos0, const int* pos_dev, int* err,
                        int* hist, long hist_stride, hipStream_t s);
// With mean / rstd set (both or neither), also each row's mean and rstd.
hipError_t launch_layernorm(const float* x, long in_stride, const float* w, const float* b,
                            float* out, long out_stride, int rows, int C, hipStream_t s,
                            float* mean = nullptr, float* rstd = nullptr);
hipError_t launch_gather_rows(const float* src, long src_stride, float* dst, int rows, int C,
                              hipStream_t s);

// gemm.hip: Y[M,N] = epi(X[M,K] . W[N,K]^T). X rows are K floats apart.
// Output row m goes to Y + ((m / seg) * seg_stride + m % seg) * ldy, which
// lets the QKV product write straight into a per-sequence cache of
// seg_stride rows (seg = 0 means plain row-major, row stride ldy).
struct GemmArgs {
    const float* X;
    const float* W;
    // Optional packed copy of W (launch_pack_w), read instead of W by the
    // few-row products; the other paths read W.
    const float* Wp;
    const float* bias;
    float* Y;
    int M, N, K;
    long ldy;
    int seg;
    long seg_stride;
    int row_off;               // added to every output row index
    const int* row_off_dev;    // if set, *row_off_dev is added too (decode position)
    int epi;                   // EpiMode
    float* part;               // split-K partials (NULL: no split) of the few-row
                               // products and of tile launches too small to fill the CUs
    long part_cap;             // floats available at part
    // Optional (EPI_RESID, seg = 0, no row offsets, N <= 2048, N and ldy
    // multiples of 4): also the LayerNorm of every output row with gains
    // ln_w and biases ln_b into ln_out (rows of N floats), formed while the
    // split-K partials are summed when K is split.
    const float* ln_w;
    const float* ln_b;
    float* ln_out;
    // Optional K-major operands (M > SKINNY_MAX_M, K a multiple of 32):
    // km = 3, both, with the residual epilogue: X is [K][ldx] (row k holds
    // the M rows' k-th values), W is [K][ldw]; km = 2, W only, with the
    // stored epilogue (X rows of K floats). ldx and ldw multiples of 4, at
    // least M and N rounded up to 4. 0: both K-contiguous, rows of K floats.
    int km;
    long ldx, ldw;
    // Optional: where K is split (launch_gemm_splits > 1) the launch leaves
    // the partials in part[ks][M][N] and does not sum them (the caller's
    // next kernel does: the decode attention folds the QKV sum in).
    int partials_only;
};
// M <= SKINNY_MAX_M rows take the weight-streaming k_stream (32 < M <= 128
// rows the 32-row k_rows tiles where K is a multiple of 64), larger M the
// 128 x 128 MFMA tiles.
constexpr int SKINNY_MAX_M = 64;
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s);
// Number of K splits launch_gemm uses for a (1: none; then a LayerNorm
// asked for with ln_out is a launch of its own after the product).
int launch_gemm_splits(const GemmArgs& a);
// K splits whose partials a launch with partials_only leaves unsummed (the
// few-row products with K split, no LayerNorm), 0 where it would not.
int launch_gemm_partials(const GemmArgs& a);
// Y = Y + bias + the sum of KS partial products a.part[ks][M][N] in ks order
// (the residual epilogue), with the LayerNorm of each row into a.ln_out when
// it is set (N <= 2048).
hipError_t launch_sum_heads(const GemmArgs& a, int KS, hipStream_t s);
// Floats of the packed copy of an [N][K] weight matrix, and the launch
// that writes it (K a multiple of 4).
size_t packed_w_floats(int N, int K);
hipError_t launch_pack_w(const float* W, float* Wp, int N, int K, hipStream_t s);

// decode.hip
// Partials of the split one-query attention, merged by their consumer:
// split s of (row r, head h) at part + ((r*H + h) * stride + s) * (hs + 4)
// holds m, l, -, -, o[hs]; the splits cover keys 0..t in runs of kps,
// t = *pos_dev (or q_pos).
struct MergeArgs {
    const float* part;
    int stride;
    int H, hs, kps;
    int q_pos;
    const int* pos_dev;
};

// Token + position embedding of a decode step built inside the first
// product: x[r] = wte[tok[r]] + wpe[*pos_dev] (ids outside [0, V) clamped
// and flagged in *err); workgroup 0 stores x to x_out and the token to
// hist[r * hist_stride + *pos_dev] (hist may be null).
struct EmbedArgs {
    const int* tok;
    const float* wte;
    const float* wpe;
    const int* pos_dev;
    float* x_out;
    int* hist;
    long hist_stride;
    int V;
    int* err;
};

// Products over M <= 8 rows with the same row mapping and epilogues as
// GemmArgs. The input rows are X (row stride ldx), or the LayerNorm of X
// (ln_w != null, K = C <= 2048; with emb.tok set, X is the embedding of
// emb), or the merged attention partials (merge.part != null, K = C).
// argmax (EPI_STORE, X or LayerNorm input only): each
// workgroup also leaves its best (value, column) per row in
// part_v / part_i [M][dgemv_argmax_parts(a)].
struct DecGemvArgs {
    const float* X;
    long ldx;
    const float* ln_w;
    const float* ln_b;
    EmbedArgs emb;
    MergeArgs merge;
    const float* W;
    const float* bias;
    float* Y;
    long ldy;
    int M, N, K;
    int seg;
    long seg_stride;
    int row_off;
    const int* row_off_dev;
    int epi;
    int argmax;
    float* part_v;
    int* part_i;
};
hipError_t launch_dgemv(const DecGemvArgs& a, hipStream_t s);
int dgemv_argmax_parts(const DecGemvArgs& a);
// out[r] = best of row r's nparts partials (first column on ties), then
// *pos_inc += 1 when pos_inc is set.
hipError_t launch_argmax_part(const float* part_v, const int* part_i, int rows, int nparts,
                              int* out, int* pos_inc, hipStream_t s);

// One query row per (sequence, head) against keys 0..t, t = *pos_dev (or
// q_pos when pos_dev is null); key/value rows as for the causal kernel.
// Keys are split over workgroups of attn_dec_keys_per_split(hs) keys; each
// writes its partial to part (layout of MergeArgs, stride = max_splits).
struct AttnDecArgs {
    const float* qkv;
    long seq_stride;
    int C, H;
    int q_pos;
    const int* pos_dev;
    float scale;
    float* part;
    int max_splits;
    // Optional, for the one-pass attention with its keys split over two
    // workgroups per (sequence, head) (too few pairs for one per CU): per
    // pair a counter and 2 * (hs + 2) tagged words, zeroed once and then
    // used only by that attention (attn_dec1_tag_words 64-bit words and one
    // 32-bit counter per pair), sized for tag_pairs pairs: a launch with more
    // (sequence, head) pairs than that takes the unsplit form.
    unsigned long long* tag_part;
    unsigned* tag_cnt;
    int tag_pairs;
    // Optional: a wait of the split form that gives up (its row is then
    // NaN) ORs ATTN_DEC_TIMEOUT into *err.
    int* err;
    // Optional (launch_attention_dec_rows): the current row's q, k and v are
    // the sum of qkv_ks partial products qkv_part[ks][b][3 C] (qkv_rows = B
    // rows per split) in ks order plus qkv_bias (the QKV product launched
    // with partials_only); each (sequence, head) workgroup forms its head's
    // 3 * hs values, uses them for the query and the newest key, and writes
    // them to row t of the cache.
    const float* qkv_part;
    const float* qkv_bias;
    int qkv_ks, qkv_rows;
};
constexpr int ATTN_DEC_TIMEOUT = 8;
size_t attn_dec1_tag_words(int pairs, int hs);
// Most (sequence, head) pairs the split form takes (more: one workgroup each).
int attn_dec1_split_pairs();
int attn_dec_keys_per_split(int hs);
// max_keys bounds t + 1 over every launch of a captured graph (sizes the grid).
hipError_t launch_attention_dec(const AttnDecArgs& a, int B, int max_keys, hipStream_t s);
// With many (sequence, head) pairs (attention_dec_one_pass): the same
// attention in one launch with no partials, normalised rows [B, C] (row
// stride ldo, a multiple of 4) straight to out.
bool attention_dec_one_pass(int B, int H);
hipError_t launch_attention_dec_rows(const AttnDecArgs& a, int B, float* out, long ldo,
                                     hipStream_t s);
// Merged attention rows [B, C] (row stride ldo) from the partials.
hipError_t launch_attention_merge(const MergeArgs& g, int B, float* out, long ldo, hipStream_t s);
// out[r] = argmax of logits row r (first index on ties); then *pos_inc += 1.
hipError_t launch_argmax_rows(const float* logits, int rows, int V, int* out, int* pos_inc,
                              hipStream_t s);
// One token per row with the reference's sample_top_k arithmetic, the
// uniform draw of row r in r_draw[r]; prob [rows, ldp] is scratch
// (ldp >= V, a multiple of 4).
// sample.hip
// Top-k sampling of one token per row (sample_top_k's arithmetic). prob
// [rows, ldp] is scratch for the one-workgroup-per-row path; part (may be
// NULL: that path only) holds TOPK_PART_WORDS floats per row for the split
// path (top_k <= 64, V <= 65536).
constexpr long TOPK_PART_WORDS = 4 * 64 + 2 * 64 * 64;
hipError_t launch_sample(const float* logits, int rows, int V, float temp, int top_k,
                         const float* r_draw, float* prob, long ldp, float* part, int* out,
                         hipStream_t s);

// persist.hip
// Parameter pointers of one layer (the carve order of assign_weights).
struct LayerW {
    const float *ln1_w, *ln1_b, *attn_w, *attn_b, *proj_w, *proj_b;
    const float *ln2_w, *ln2_b, *fc_w, *fc_b, *mlp_w, *mlp_b;
};
// Greedy decode of one sequence (B = 1, head size 64) for n_steps steps as
// one cooperative launch: feeds *tok at position *pos, leaves the logits of
// the last step in logits, the tokens fed in hist[pos..], the next token in
// *tok and the next position in *pos. *err |= 1 for a token outside
// [0, V) (clamped), |= 2 when a wait for a value timed out.
struct PersistArgs {
    const LayerW* layers;   // device array [L]
    const float *wte, *wpe, *lnf_w, *lnf_b;
    int L, C, H, V, cap;
    float* cache;           // KV cache rows [L][cap][3C]
    unsigned long long* tagged;  // persist_tagged_words(C, H) exchange words
    unsigned tag0;          // tags of this launch: tag0 + 1 .. tag0 + persist_tags(L, n_steps)
    float* logits;          // [V]
    int* hist;              // [cap]
    int* pos;
    int* tok;
    int* err;
    int n_steps;
    float scale;            // 1 / sqrt(head size)
    // sampling (top_k > 0): sample_top_k with draws[step]; 0: greedy
    float temp;
    int top_k;
    const float* draws;
    int* steps_done;        // steps completed (a sampling step whose
                            // candidates overflow ends the launch early)
};
// Workgroups of the launch (one per CU), 0 if the device has no
// cooperative launch.
int persist_workgroups(int device);
bool persist_supported(int C, int H, int V, int cap, int G);
// Exchange words of the launch (zeroed once at allocation) and tags one
// launch uses: tags only grow, so a word written by an earlier launch never
// matches a tag this launch waits for.
long persist_tagged_words(int C, int H);
unsigned persist_tags(int L, int n_steps);
// Whether a launch of G workgroups can draw top-k samples itself (else the
// host samples between one-step launches).
bool persist_sampling_supported(int V, int G, int top_k);
hipError_t launch_decode_persist(const PersistArgs& a, int G, hipStream_t s);

// attention.hip
// qkv rows hold [q | k | v] (3C floats); sequence b's row t sits at
// qkv + (b * seq_stride + t) * 3C. out row (b*T + t) gets the merged heads.
// With lse set, also the log-sum-exp of every query's scores in base 2 (of
// the scores times scale * log2(e)) at lse[(b * H + h) * T + t], which the
// attention backward uses to recompute the probabilities.
hipError_t launch_attention_causal(const float* qkv, long seq_stride, float* out, int B, int T,
                                   int C, int H, hipStream_t s, float* lse = nullptr);
// The same attention (64-wide heads, keys split over a workgroup's
// wavefronts) with each head's share of the c_proj product applied in the
// launch: part[(h * B * T + row) * C + n] = sum over d of out[row][h * 64 +
// d] * W[n][h * 64 + d], W the [C][C] c_proj weights; CB (2..4, from
// attention_proj_cb, 0 = this form does not apply) sets 16 CB output
// columns per wavefront. launch_sum_heads (gemm.hip) then adds the H
// partials in head order with the bias and residual, and the LayerNorm.
int attention_proj_cb(int B, int T, int C, int H);
hipError_t launch_attention_proj(const float* qkv, long seq_stride, const float* W, float* part,
                                 int B, int T, int C, int H, int CB, hipStream_t s);

// loss.hip
// Cross-entropy of rows x V logits against targets [rows]: row_loss[r] =
// log(sum_v exp(x_v - max)) - (x[target] - max), loss[0] = their mean.
// probs != 0 overwrites the logits with their softmax. Targets outside
// [0, V) are clamped and reported through *err (bit 2).
// dl != 0 (probs 0): the logits stay, and dl [rows][ldd] (ldd >= V, a
// multiple of 4) gets the mean loss's gradient (p - onehot) / rows, zero in
// columns V .. ldd-1.
hipError_t launch_cross_entropy(float* logits, long rows, int V, const int* targets,
                                float* row_loss, float* loss, int probs, int* err, hipStream_t s,
                                float* dl = nullptr, long ldd = 0);

// train.hip: the training step's elementwise, row and reduction kernels.
// out = gelu(in); d = d * gelu'(x) (n a multiple of 4).
hipError_t launch_gelu_fwd(const float* in, float* out, long n, hipStream_t s);
hipError_t launch_gelu_bwd(float* d, const float* x, long n, hipStream_t s);
// x[i] *= mask[i] ? scale : 0 (dropout_fwd / dropout_bwd's scaling, the
// bytes of mask 0 or 1; n a multiple of 4, mask 4-byte aligned).
hipError_t launch_dropout(float* x, const unsigned char* mask, long n, float scale,
                          hipStream_t s);
// dst [cols_p][ldd] = src [rows][lds]^T, zero in the padding (rows <= rows_p
// <= ldd, cols <= cols_p).
hipError_t launch_transpose(const float* src, long lds, int rows, int cols, float* dst, long ldd,
                            int rows_p, int cols_p, hipStream_t s);
// out[c] += sum over rows of Y[r][c] (partials of colsum_part_floats floats
// at part, summed in row-chunk order).
long colsum_part_floats(int rows, int cols);
hipError_t launch_colsum_add(const float* Y, long ldy, int rows, int cols, float* part,
                             float* out, hipStream_t s);
// The same transpose, and out[c] += the column sums of src over its rows
// (partials of transpose_colsum_floats floats at part, summed in row order).
long transpose_colsum_floats(int rows, int cols);
hipError_t launch_transpose_colsum(const float* src, long lds, int rows, int cols, float* dst,
                                   long ldd, int rows_p, int cols_p, float* part, float* out,
                                   hipStream_t s);
// layernorm_bwd: dx += ..., dw += sum dout * xhat, db += sum dout over the
// rows (partials of ln_bwd_part_floats floats at part). C a multiple of 4,
// at most 2048.
long ln_bwd_part_floats(int rows, int C);
hipError_t launch_layernorm_bwd(const float* dout, const float* x, const float* w,
                                const float* mean, const float* rstd, float* dx, float* dw,
                                float* db, int rows, int C, float* part, hipStream_t s);
// g_wpe[t] += sum_b dx[b][t]; g_wte[uniq[u]] += dx rows pos[start[u] ..
// start[u+1]) in order, for each of the nuniq distinct tokens.
hipError_t launch_embed_bwd(const float* dx, int B, int T, int C, float* g_wpe, float* g_wte,
                            const int* uniq, const int* start, const int* pos, int nuniq,
                            hipStream_t s);
// gpt_adamw over n parameters: the global gradient norm into *norm (from
// grad_norm_parts(n) double partials at part), the clip coefficient into
// *coef, then the update of p, g (clipped in place), m and v.
int grad_norm_parts(long n);
hipError_t launch_adamw(float* p, float* g, float* m, float* v, const unsigned char* decay,
                        long n, double* part, float* norm, float* coef, float lr, float beta1,
                        float beta2, float eps, float wd, float clip, float bc1, float bc2,
                        hipStream_t s);

// attn_bwd.hip: dQ, dK, dV of every head into the qkv gradient rows [B*T][3C]
// from the forward's qkv rows, its output rows `out` [B*T][C], their
// gradient dout and the forward's lse; D [B*H*T] is scratch.
hipError_t launch_attention_bwd(const float* qkv, const float* out, const float* dout,
                                const float* lse, float* D, float* dqkv, int B, int T, int C,
                                int H, hipStream_t s);
