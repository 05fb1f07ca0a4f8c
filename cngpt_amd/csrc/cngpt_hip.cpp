// cngpt_hip.cpp - the C ABI (include/cngpt_hip.h): device memory, the kernel
// sequence of the forward pass, incremental decode and timing counters.
//
// Kernel sequence of one forward (reference fast.c:227-333):
//   embed -> per layer { LN1 -> QKV product (+b) -> causal attention
//   -> c_proj product (x += . + b) -> LN2 -> fc product (+b, GELU)
//   -> proj product (x += . + b) } -> LN_f -> lm_head product (wte^T).
// In LAST mode the last layer runs attention for the final query row only
// and the rest of that layer on the B gathered rows (fast.c:287-311).
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/cngpt_hip.h"
#include "common.h"
#include "ctx_view.h"
#include "kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return -1;
}

#define HIP_TRY(expr)                                                                   \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                           \
            return fail("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                        __LINE__);                                                      \
    } while (0)

struct ProfRec {
    int cls;
    hipEvent_t a, b;
    double flops, bytes;
};

constexpr size_t ALIGN = 256;
// split-K partials of the few-row products and of the tile launches too
// small to fill the CUs, and the stream-K partial tiles (two per workgroup,
// 512 workgroups): 64 MB
constexpr long GEMM_PART_FLOATS = 1l << 24;
size_t align_up(size_t n) { return (n + ALIGN - 1) & ~(ALIGN - 1); }

// Scratch of cngpt_hip_forward_noalloc: every activation of one forward
// (128 MiB: the B*T rows of x, ln, qkv, aout and hid, the B gathered rows,
// the attention split partials and the split-K partials). Each device the
// library runs on holds its own copy from the first use until the process
// ends. Host code never uses the array's name as an address: it is a
// host-side stand-in; the device address of each device's copy comes from
// hipGetSymbolAddress, once per device, in cngpt_hip_create.
constexpr long SCRATCH_FLOATS = 32l << 20;
__device__ __align__(256) float scratch[SCRATCH_FLOATS];
// The first SCRATCH_TAG_FLOATS of the scratch hold the tagged words and
// per-pair counters of the split decode attention (head sizes up to
// SCRATCH_TAG_HS, attn_dec1_split_pairs() pairs), at fixed offsets: they
// keep their state from one call to the next (counters grow, words are
// cleared by the attention after use), zeroed once when the device's
// address is looked up.
constexpr int SCRATCH_TAG_HS = 128;
long scratch_tag_floats() {
    const long words = (long)attn_dec1_tag_words(attn_dec1_split_pairs(), SCRATCH_TAG_HS);
    return (2 * words + attn_dec1_split_pairs() + 63) / 64 * 64;
}

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch[MAX_DEVICES];  // device address of `scratch`, per device

// Zeroes n ints with a kernel (a memset node in a captured graph is avoided).
__global__ void k_zero_i32(int* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// With `device` current: look up and keep its address of the scratch array,
// and zero its tag region.
int scratch_setup(int device) {
    if (device < 0 || device >= MAX_DEVICES) return 0;  // the no-alloc entry refuses such devices
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[device]) return 0;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return fail("scratch address on device %d: %s", device, hipGetErrorString(e));
    }
    const int n = (int)scratch_tag_floats();
    k_zero_i32<<<(n + 255) / 256, 256, 0, 0>>>((int*)p, n);
    const hipError_t z = hipStreamSynchronize(0);
    if (z != hipSuccess) {
        (void)hipGetLastError();
        return fail("scratch tag region on device %d: %s", device, hipGetErrorString(z));
    }
    g_scratch[device] = (float*)p;
    return 0;
}

float* scratch_of(int device) {
    if (device < 0 || device >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch[device];
}

}  // namespace

struct cngpt_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;

    cngpt_hip_config cfg{};
    bool have_params = false;
    float* d_params = nullptr;
    long n_params = 0;
    const float *wte = nullptr, *wpe = nullptr, *lnf_w = nullptr, *lnf_b = nullptr;
    std::vector<LayerW> layers;
    LayerW* d_layers = nullptr;  // device copy of layers (persistent decode), at the
                                 // end of the parameter allocation
    // Packed copies (launch_pack_w) of the weight matrices, after the layer
    // table in the same allocation, read by the few-row products.
    // CNGPT_HIP_PACK=0 in the environment at create time leaves them out.
    // A training update changes the parameters in place: it marks the
    // copies stale, and the next forward or decode entry point packs them
    // again.
    struct Packed {
        const float* W;
        float* Wp;
        int N, K;
    };
    bool use_packed = true;
    bool packed_fresh = false;
    // short prefills: c_proj applied per head inside the attention launch
    bool use_attn_proj = true;
    int attn_proj_cb = 0;
    // batched decode: the QKV product's K-split sum inside the attention
    bool use_qkv_fold = true;
    std::vector<Packed> packs;
    std::unordered_map<const float*, const float*> packed_of;

    // activation arena: one allocation, carved below
    char* d_act = nullptr;
    size_t act_bytes = 0;
    int capB = 0, capT = 0, capAll = 0, capKV = 0;
    int* tok = nullptr;
    int* dev_err = nullptr;
    int* pos = nullptr;      // decode position (device)
    int* next_tok = nullptr; // [B] decode tokens (device)
    int* hist = nullptr;     // [B][capKV] token fed at each position (decode)
    float *x = nullptr, *ln = nullptr, *qkv = nullptr, *aout = nullptr, *hid = nullptr;
    float *logits = nullptr;
    float *xc = nullptr, *lnc = nullptr, *aoutc = nullptr, *hidc = nullptr;
    float* am_part_v = nullptr;  // [8][V] argmax partials of the lm_head
    int* am_part_i = nullptr;
    float* attn_part = nullptr;  // [B*H][attn_splits][hs+4] split-key partials
    int attn_splits = 0;
    float* draws = nullptr;      // [capKV+1][B] uniform draws for sampling
    float* prob = nullptr;       // [B][ldp] sampling scratch
    float* samp_part = nullptr;  // [B][TOPK_PART_WORDS] split-sampling partials
    float* gemm_part = nullptr;  // split-K partials of the few-row products
    int* tgt = nullptr;          // [B*T] cross-entropy targets
    float* row_loss = nullptr;   // [B*T] cross-entropy row terms
    float* loss = nullptr;       // mean cross-entropy
    long loss_rows = 0;          // rows of the last cross-entropy (0: none)
    long ldp = 0;
    int pos_host = 0;            // staging for the position upload
    unsigned long long* dtag = nullptr;  // tagged halves of the split one-pass decode attention
    unsigned* dcnt = nullptr;            // and its per-(sequence, head) counters
    int dtag_pairs = 0;                  // pairs dtag / dcnt hold
    unsigned long long* ptag = nullptr;  // exchange words of the persistent decode
    unsigned ptag_next = 0;      // next unused tag (tags only grow until the words are cleared)

    // decode path: CNGPT_DECODE_AUTO / _KERNELS / _PERSISTENT (set_decode_path;
    // CNGPT_HIP_PERSIST=0 in the environment at create time selects _KERNELS)
    int decode_path = CNGPT_DECODE_AUTO;
    int last_path = 0;           // path of the last decode step
    int persist_G = -1;          // workgroups of the persistent launch (-1: not queried,
                                 // 0: unavailable, e.g. a refused cooperative launch)

    // the decode step as a replayable graph (kernels only); CNGPT_HIP_GRAPH=0
    // in the environment at create time selects direct launches instead
    bool use_graph = true;
    hipGraphExec_t step_exec = nullptr;
    int graph_B = 0, graph_cap = 0;
    const void *graph_act = nullptr, *graph_par = nullptr;
    // the forward of one shape likewise (cngpt_hip_forward and
    // cngpt_hip_forward_resident replay it; captured on the first call of a
    // shape, again after the arena or the parameters moved)
    hipGraphExec_t fwd_exec = nullptr;
    int fwd_B = 0, fwd_T = 0, fwd_mode = -1;
    const void *fwd_act = nullptr, *fwd_par = nullptr;

    // state of the last forward / decode
    int curB = 0, curT = 0, curMode = CNGPT_LAST;
    size_t logits_count = 0;
    int kvB = 0, kvLen = 0;  // sequences and positions held in the KV cache

    // timing
    bool prof = false;
    std::vector<ProfRec> recs;
    std::vector<hipEvent_t> pool;
    size_t pool_used = 0;
};

namespace {

bool valid_cfg(const cngpt_hip_config* c) {
    return c && c->n_layer > 0 && c->n_head > 0 && c->n_embd > 0 && c->vocab_size > 0 &&
           c->block_size > 0 && c->n_embd % c->n_head == 0;
}

// ---------------------------------------------------------------- timing

hipEvent_t pool_event(cngpt_hip_ctx* h) {
    if (h->pool_used == h->pool.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        h->pool.push_back(e);
    }
    return h->pool[h->pool_used++];
}

struct Timed {
    cngpt_hip_ctx* h;
    ProfRec rec{};
    bool on;
    Timed(cngpt_hip_ctx* h_, int cls, double flops, double bytes) : h(h_), on(h_->prof) {
        if (!on) return;
        rec.cls = cls;
        rec.flops = flops;
        rec.bytes = bytes;
        rec.a = pool_event(h);
        rec.b = pool_event(h);
        if (!rec.a || !rec.b) { on = false; return; }
        (void)hipEventRecord(rec.a, h->stream);
    }
    ~Timed() {
        if (!on) return;
        (void)hipEventRecord(rec.b, h->stream);
        h->recs.push_back(rec);
    }
};

// ---------------------------------------------------------------- launches

// Products over M <= SKINNY rows go to the decode GEMV (one wavefront per
// output column, LayerNorm of the input rows optionally folded in); larger M
// to the MFMA kernels (16-column tiles up to 64 rows, then 128 x 128).
// Up to SKINNY rows the per-column products (LayerNorm, attention merge or
// embedding folded into their input staging) beat a separate LayerNorm plus
// the 16-column MFMA tiles; from 3 rows on the tiles' reuse of the input
// rows wins (measured on GPT-2 medium, 8 sequences: 1.72 vs 1.88 ms a step).
constexpr int SKINNY = 2;

int run_ln(cngpt_hip_ctx* h, const float* x, long in_stride, const float* w, const float* b,
           float* out, int rows);

// With lnw / lnb / lnout set, also LayerNorm(Y rows) into lnout (the next
// product's input); over more than SKINNY rows the split-K sum forms it.
int run_gemm(cngpt_hip_ctx* h, const float* X, const float* W, const float* bias, float* Y, int M,
             int N, int K, int epi, int seg = 0, long seg_stride = 0, long ldy = -1,
             int row_off = 0, const int* row_off_dev = nullptr, const float* lnw = nullptr,
             const float* lnb = nullptr, float* lnout = nullptr, int* left_partials = nullptr) {
    const double flops = 2.0 * M * N * K;
    const double bytes =
        4.0 * ((double)M * K + (double)N * K + (double)M * N * (epi == EPI_RESID ? 2 : 1));
    if (M <= SKINNY) {
        DecGemvArgs d{};
        d.X = X; d.ldx = K; d.W = W; d.bias = bias; d.Y = Y;
        d.ldy = ldy < 0 ? N : ldy;
        d.M = M; d.N = N; d.K = K;
        d.seg = seg; d.seg_stride = seg_stride;
        d.row_off = row_off; d.row_off_dev = row_off_dev;
        d.epi = epi;
        {
            Timed t(h, CNGPT_K_GEMV, flops, bytes);
            HIP_TRY(launch_dgemv(d, h->stream));
        }
        return lnout ? run_ln(h, Y, d.ldy, lnw, lnb, lnout, M) : 0;
    }
    GemmArgs a{};
    a.X = X; a.W = W; a.bias = bias; a.Y = Y;
    if (h->use_packed) {
        const auto it = h->packed_of.find(W);
        if (it != h->packed_of.end()) a.Wp = it->second;
    }
    a.M = M; a.N = N; a.K = K;
    a.ldy = ldy < 0 ? N : ldy;
    a.seg = seg; a.seg_stride = seg_stride;
    a.row_off = row_off; a.row_off_dev = row_off_dev;
    a.epi = epi;
    a.part = h->gemm_part; a.part_cap = GEMM_PART_FLOATS;
    // a split product forms the LayerNorm while it sums its partials;
    // otherwise the LayerNorm is a launch (and a timing class) of its own
    const bool ln_in_sum = lnout && launch_gemm_splits(a) > 1;
    if (ln_in_sum) {
        a.ln_w = lnw; a.ln_b = lnb; a.ln_out = lnout;
    }
    // left_partials: where the product splits K, its partials stay in
    // gemm_part for the caller's next kernel to sum (*left_partials = the
    // splits; 0 where the product writes Y itself)
    if (left_partials) {
        *left_partials = lnout ? 0 : launch_gemm_partials(a);
        a.partials_only = *left_partials > 0;
    }
    {
        Timed t(h, CNGPT_K_GEMM, flops, bytes);
        HIP_TRY(launch_gemm(a, h->stream));
    }
    return lnout && !ln_in_sum ? run_ln(h, Y, a.ldy, lnw, lnb, lnout, M) : 0;
}

int run_ln(cngpt_hip_ctx* h, const float* x, long in_stride, const float* w, const float* b,
           float* out, int rows) {
    const int C = h->cfg.n_embd;
    Timed t(h, CNGPT_K_LAYERNORM, 0.0, 8.0 * C * rows);
    HIP_TRY(launch_layernorm(x, in_stride, w, b, out, C, rows, C, h->stream));
    return 0;
}

// Y = epi(LN(x) . W^T) over M rows of x (row stride C). For M <= 8 the
// LayerNorm runs inside the product; otherwise into `scratch` first.
int run_ln_gemm(cngpt_hip_ctx* h, const float* x, const float* lw, const float* lb,
                float* scratch, const float* W, const float* bias, float* Y, int M, int N,
                int epi, int seg = 0, long seg_stride = 0, long ldy = -1,
                const int* row_off_dev = nullptr) {
    const int C = h->cfg.n_embd;
    if (M <= SKINNY) {
        DecGemvArgs d{};
        d.X = x; d.ldx = C; d.ln_w = lw; d.ln_b = lb; d.W = W; d.bias = bias; d.Y = Y;
        d.ldy = ldy < 0 ? N : ldy;
        d.M = M; d.N = N; d.K = C;
        d.seg = seg; d.seg_stride = seg_stride;
        d.row_off_dev = row_off_dev;
        d.epi = epi;
        Timed t(h, CNGPT_K_GEMV, 2.0 * M * N * C,
                4.0 * ((double)M * C + (double)N * C + (double)M * N));
        HIP_TRY(launch_dgemv(d, h->stream));
        return 0;
    }
    if (run_ln(h, x, C, lw, lb, scratch, M)) return -1;
    return run_gemm(h, scratch, W, bias, Y, M, N, C, epi, seg, seg_stride, ldy, 0, row_off_dev);
}

// Final LayerNorm and lm_head over M rows of x -> logits [M, V]; with
// want_tok the greedy token of each row goes to next_tok, and pos_inc (if
// set) is advanced once everything else of the step has run.
int run_lm_head(cngpt_hip_ctx* h, const float* x, int M, bool want_tok, int* pos_inc,
                bool ln_done = false) {
    const int C = h->cfg.n_embd, V = h->cfg.vocab_size;
    if (M <= SKINNY) {
        // The final LayerNorm runs once on its own: recomputing it in each of
        // the ~V/4 workgroups of the product costs more than the launch.
        if (run_ln(h, x, C, h->lnf_w, h->lnf_b, h->lnc, M)) return -1;
        DecGemvArgs d{};
        d.X = h->lnc; d.ldx = C; d.W = h->wte;
        d.Y = h->logits; d.ldy = V;
        d.M = M; d.N = V; d.K = C;
        d.epi = EPI_STORE;
        const int parts = dgemv_argmax_parts(d);
        if (want_tok) {
            if (parts > V) return fail("argmax partials exceed their buffer");
            d.argmax = 1;
            d.part_v = h->am_part_v;
            d.part_i = h->am_part_i;
        }
        {
            Timed t(h, CNGPT_K_GEMV, 2.0 * M * V * C,
                    4.0 * ((double)M * C + (double)V * C + (double)M * V));
            HIP_TRY(launch_dgemv(d, h->stream));
        }
        if (want_tok) {
            Timed t(h, CNGPT_K_ARGMAX, 0.0, 8.0 * M * parts);
            HIP_TRY(launch_argmax_part(h->am_part_v, h->am_part_i, M, parts, h->next_tok, pos_inc,
                                       h->stream));
        }
    } else {
        // (ln_done: the final LayerNorm is already in lnc)
        if (!ln_done && run_ln(h, x, C, h->lnf_w, h->lnf_b, h->lnc, M)) return -1;
        if (run_gemm(h, h->lnc, h->wte, nullptr, h->logits, M, V, C, EPI_STORE)) return -1;
        if (want_tok) {
            Timed t(h, CNGPT_K_ARGMAX, 0.0, 4.0 * M * V);
            HIP_TRY(launch_argmax_rows(h->logits, M, V, h->next_tok, pos_inc, h->stream));
        }
    }
    h->logits_count = (size_t)M * V;
    return 0;
}

// Attention of one query row per sequence (position q_pos, or *pos_dev)
// followed by the c_proj product with its residual: xres[b] += aout[b] . W^T
// + bias. For B <= 8 the c_proj product merges the attention splits itself;
// otherwise the merged rows go through aoutc.
int run_attn_row_proj(cngpt_hip_ctx* h, const float* qkv, long seq_stride, int B, int q_pos,
                      const int* pos_dev, int max_keys, const LayerW& w, float* xres,
                      const float* lnw = nullptr, const float* lnb = nullptr,
                      float* lnout = nullptr, int qkv_ks = 0) {
    const cngpt_hip_config& c = h->cfg;
    const int C = c.n_embd, hs = C / c.n_head;
    AttnDecArgs a{};
    a.qkv = qkv; a.seq_stride = seq_stride;
    a.C = C; a.H = c.n_head;
    a.q_pos = q_pos; a.pos_dev = pos_dev;
    a.scale = 1.0f / sqrtf((float)hs);
    a.part = h->attn_part; a.max_splits = h->attn_splits;
    a.tag_part = h->dtag; a.tag_cnt = h->dcnt; a.tag_pairs = h->dtag_pairs;
    a.err = h->dev_err;
    const double keys = pos_dev ? 0.5 * max_keys : q_pos + 1.0;
    if (B > SKINNY && attention_dec_one_pass(B, c.n_head)) {
        // many (sequence, head) pairs: one pass, rows straight to c_proj's
        // input; with qkv_ks the QKV product's partials are summed here
        if (qkv_ks) {
            a.qkv_part = h->gemm_part; a.qkv_bias = w.attn_b;
            a.qkv_ks = qkv_ks; a.qkv_rows = B;
        }
        {
            Timed t(h, CNGPT_K_ATTN_ROW, 4.0 * C * keys * B,
                    4.0 * ((double)B * keys * 2 * C + (double)B * C));
            HIP_TRY(launch_attention_dec_rows(a, B, h->aoutc, C, h->stream));
        }
        return run_gemm(h, h->aoutc, w.proj_w, w.proj_b, xres, B, C, C, EPI_RESID, 0, 0, -1, 0,
                        nullptr, lnw, lnb, lnout);
    }
    if (qkv_ks) return fail("QKV partials left for an attention form that does not sum them");
    {
        Timed t(h, CNGPT_K_ATTN_ROW, 4.0 * C * keys * B,
                4.0 * ((double)B * keys * 2 * C + (double)B * C));
        HIP_TRY(launch_attention_dec(a, B, max_keys, h->stream));
    }
    MergeArgs g{};
    g.part = h->attn_part; g.stride = h->attn_splits;
    g.H = c.n_head; g.hs = hs; g.kps = attn_dec_keys_per_split(hs);
    g.q_pos = q_pos; g.pos_dev = pos_dev;
    // Every workgroup of the c_proj product merges all splits it needs; that
    // pays while the partials are small (one sequence, short context).
    const int splits = (max_keys + g.kps - 1) / g.kps;
    const double merge_bytes = 4.0 * B * c.n_head * splits * (hs + 4);
    if (B <= SKINNY && merge_bytes <= 64.0 * 1024) {
        DecGemvArgs d{};
        d.merge = g;
        d.W = w.proj_w; d.bias = w.proj_b; d.Y = xres; d.ldy = C;
        d.M = B; d.N = C; d.K = C;
        d.epi = EPI_RESID;
        {
            Timed t(h, CNGPT_K_GEMV, 2.0 * B * C * C, 4.0 * ((double)C * C + 2.0 * B * C));
            HIP_TRY(launch_dgemv(d, h->stream));
        }
        return lnout ? run_ln(h, xres, C, lnw, lnb, lnout, B) : 0;
    }
    {
        Timed t(h, CNGPT_K_ATTN_ROW, 0.0, 4.0 * B * C);
        HIP_TRY(launch_attention_merge(g, B, h->aoutc, C, h->stream));
    }
    return run_gemm(h, h->aoutc, w.proj_w, w.proj_b, xres, B, C, C, EPI_RESID, 0, 0, -1, 0,
                    nullptr, lnw, lnb, lnout);
}

void drop_fwd_graph(cngpt_hip_ctx* h) {
    // (as for the step graph: its last launch may still be queued)
    if (h->fwd_exec) (void)hipStreamSynchronize(h->stream);
    if (h->fwd_exec) (void)hipGraphExecDestroy(h->fwd_exec);
    h->fwd_exec = nullptr;
    h->fwd_B = h->fwd_T = 0;
    h->fwd_mode = -1;
    h->fwd_act = h->fwd_par = nullptr;
}

void drop_graph(cngpt_hip_ctx* h) {
    // the last launch of the executable graph may still be queued on the
    // stream (a re-capture for a new batch follows the previous sequence's
    // steps without a synchronisation): it must finish before the graph's
    // resources are released
    if (h->step_exec) (void)hipStreamSynchronize(h->stream);
    if (h->step_exec) (void)hipGraphExecDestroy(h->step_exec);
    h->step_exec = nullptr;
    h->graph_B = h->graph_cap = 0;
    h->graph_act = h->graph_par = nullptr;
}

// ---------------------------------------------------------------- arena

// The arena grows in every dimension and never shrinks (one allocation,
// re-carved on growth; growth drops the decode KV cache). The KV cache of
// layer l, sequence b, position t is row (l*B + b)*capKV + t of the qkv
// region, so any B <= capB and capacity <= capKV fit without moving.
int ensure_arena(cngpt_hip_ctx* h, int B, int T, int all, int kv) {
    if (h->d_act && B <= h->capB && T <= h->capT && (!all || h->capAll) && kv <= h->capKV)
        return 0;
    const cngpt_hip_config& c = h->cfg;
    const int nB = std::max(B, h->capB);
    const int nT = std::max(T, h->capT);
    const int nAll = (all || h->capAll) ? 1 : 0;
    const int nKV = std::max(kv, h->capKV);
    const size_t C = c.n_embd, V = c.vocab_size, L = c.n_layer, H = c.n_head;
    const size_t rows = (size_t)nB * nT;
    const size_t qkv_rows = std::max(rows, L * nB * (size_t)nKV);
    const int kps = attn_dec_keys_per_split(c.n_embd / c.n_head);
    const int splits = (c.block_size + kps - 1) / kps;
    size_t sz[32], total = 0;
    int n = 0;
    sz[n++] = rows * sizeof(int);             // tok
    sz[n++] = 4 * sizeof(int);                // dev_err, pos
    sz[n++] = (size_t)nB * sizeof(int);       // next_tok
    sz[n++] = (size_t)nB * std::max(nKV, 1) * sizeof(int);         // hist
    sz[n++] = 8 * V * sizeof(float);                               // am_part_v
    sz[n++] = 8 * V * sizeof(int);                                 // am_part_i
    sz[n++] = (size_t)nB * H * splits * (C / H + 4) * sizeof(float);  // attn_part
    sz[n++] = (size_t)nB * (nKV + 1) * sizeof(float);              // draws
    sz[n++] = (size_t)nB * ((V + 3) / 4 * 4) * sizeof(float);      // prob
    sz[n++] = (size_t)nB * TOPK_PART_WORDS * sizeof(float);        // samp_part
    sz[n++] = (size_t)GEMM_PART_FLOATS * sizeof(float);            // gemm_part
    sz[n++] = rows * C * 4;                   // x
    sz[n++] = rows * C * 4;                   // ln
    sz[n++] = qkv_rows * 3 * C * 4;           // qkv / KV cache
    sz[n++] = rows * C * 4;                   // aout
    sz[n++] = rows * 4 * C * 4;               // hid
    sz[n++] = (nAll ? rows : (size_t)nB) * V * 4;  // logits
    sz[n++] = nB * C * 4;                     // xc
    sz[n++] = nB * C * 4;                     // lnc
    sz[n++] = nB * C * 4;                     // aoutc
    sz[n++] = nB * 4 * C * 4;                 // hidc
    sz[n++] = (size_t)persist_tagged_words(c.n_embd, c.n_head) * 8;  // ptag
    sz[n++] = attn_dec1_tag_words(nB * (int)H, (int)(C / H)) * 8 + (size_t)nB * H * 4;  // dtag, dcnt
    sz[n++] = rows * sizeof(int);             // tgt
    sz[n++] = rows * sizeof(float);           // row_loss
    sz[n++] = sizeof(float);                  // loss
    for (int i = 0; i < n; i++) total += align_up(sz[i]);

    if (h->d_act) {
        HIP_TRY(hipStreamSynchronize(h->stream));
        drop_graph(h);
        drop_fwd_graph(h);
        HIP_TRY(hipFree(h->d_act));
        h->d_act = nullptr;
        h->act_bytes = 0;
        h->capB = h->capT = h->capAll = h->capKV = 0;
        h->kvB = h->kvLen = 0;
    }
    char* p = nullptr;
    if (hipMalloc(&p, total) != hipSuccess) {
        (void)hipGetLastError();
        return fail("activation allocation of %zu bytes failed (B=%d T=%d all=%d kv=%d)", total,
                    nB, nT, nAll, nKV);
    }
    h->d_act = p;
    h->act_bytes = total;
    char* q = p;
    auto take = [&](size_t bytes) { char* r = q; q += align_up(bytes); return r; };
    n = 0;
    h->tok = (int*)take(sz[n++]);
    h->dev_err = (int*)take(sz[n++]);
    h->pos = h->dev_err + 1;
    h->next_tok = (int*)take(sz[n++]);
    h->hist = (int*)take(sz[n++]);
    h->am_part_v = (float*)take(sz[n++]);
    h->am_part_i = (int*)take(sz[n++]);
    h->attn_part = (float*)take(sz[n++]);
    h->attn_splits = splits;
    h->draws = (float*)take(sz[n++]);
    h->prob = (float*)take(sz[n++]);
    h->samp_part = (float*)take(sz[n++]);
    h->gemm_part = (float*)take(sz[n++]);
    h->ldp = (long)((V + 3) / 4 * 4);
    h->x = (float*)take(sz[n++]);
    h->ln = (float*)take(sz[n++]);
    h->qkv = (float*)take(sz[n++]);
    h->aout = (float*)take(sz[n++]);
    h->hid = (float*)take(sz[n++]);
    h->logits = (float*)take(sz[n++]);
    h->xc = (float*)take(sz[n++]);
    h->lnc = (float*)take(sz[n++]);
    h->aoutc = (float*)take(sz[n++]);
    h->hidc = (float*)take(sz[n++]);
    h->ptag = (unsigned long long*)take(sz[n++]);
    h->ptag_next = 0;
    HIP_TRY(hipMemsetAsync(h->ptag, 0, sz[n - 1], h->stream));
    h->dtag = (unsigned long long*)take(sz[n++]);
    h->dcnt = (unsigned*)(h->dtag + attn_dec1_tag_words(nB * (int)H, (int)(C / H)));
    h->dtag_pairs = nB * (int)H;
    HIP_TRY(hipMemsetAsync(h->dtag, 0, sz[n - 1], h->stream));
    h->tgt = (int*)take(sz[n++]);
    h->row_loss = (float*)take(sz[n++]);
    h->loss = (float*)take(sz[n++]);
    h->loss_rows = 0;
    h->capB = nB; h->capT = nT; h->capAll = nAll; h->capKV = nKV;
    HIP_TRY(hipMemsetAsync(h->dev_err, 0, 4 * sizeof(int), h->stream));
    return 0;
}

// Wavefront column blocks of the attention launch with c_proj per head (0:
// attention and c_proj as two launches). For short prefills (17 to 128 rows
// of 64-wide heads), where the c_proj product is a split-K launch of its own
// whose partials are summed anyway. Measured (GPT-2 small, final-position
// logits, through the host API): B=1 T=128 0.721 -> 0.703 ms per forward,
// B=1 T=64 0.680 -> 0.655, B=1 T=32 0.594 -> 0.580.
int attn_proj_cb(const cngpt_hip_ctx* h, int B, int T) {
    const int C = h->cfg.n_embd, H = h->cfg.n_head;
    const long rows = (long)B * T;
    if (!h->use_attn_proj || rows <= 16 || rows > 128 || C > 2048) return 0;
    if ((long)H * rows * C > GEMM_PART_FLOATS) return 0;
    const int cb = attention_proj_cb(B, T, C, H);
    return cb && h->attn_proj_cb && C % (64 * h->attn_proj_cb) == 0 ? h->attn_proj_cb : cb;
}

int check_tokens(const cngpt_hip_ctx* h, const int* tokens, long n) {
    for (long i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= h->cfg.vocab_size)
            return fail("token %d at index %ld outside [0, %d)", tokens[i], i, h->cfg.vocab_size);
    return 0;
}

// Enqueue one forward over h->tok [B, T]. kv: QKV rows go to the per-layer
// KV cache (capacity h->capKV per sequence) instead of the reused buffer.
// want_tok: LAST mode also leaves the greedy token of each row in next_tok.
int enqueue_forward(cngpt_hip_ctx* h, int B, int T, int mode, bool kv, bool want_tok) {
    const cngpt_hip_config& c = h->cfg;
    const int C = c.n_embd, L = c.n_layer, H = c.n_head;
    const long rows = (long)B * T;
    const long seq_stride = kv ? h->capKV : T;
    {
        Timed t(h, CNGPT_K_EMBED, 0.0, 12.0 * C * rows);
        HIP_TRY(launch_embed(h->tok, h->wte, h->wpe, h->x, rows, T, C, c.vocab_size, 0, nullptr,
                             h->dev_err, nullptr, 0, h->stream));
    }
    // LayerNorm 1 of layer 0; every later LayerNorm over all rows is formed
    // by the residual product before it (while it sums its K splits, or in a
    // launch right after it), into ln
    if (run_ln(h, h->x, C, h->layers[0].ln1_w, h->layers[0].ln1_b, h->ln, (int)rows)) return -1;
    for (int l = 0; l < L; l++) {
        const LayerW& w = h->layers[l];
        const bool last = (mode == CNGPT_LAST) && (l == L - 1);
        float* qkv = kv ? h->qkv + (size_t)l * B * h->capKV * 3 * C : h->qkv;
        if (run_gemm(h, h->ln, w.attn_w, w.attn_b, qkv, (int)rows, 3 * C, C, EPI_BIAS,
                     kv ? T : 0, seq_stride, 3L * C))
            return -1;
        if (!last) {
            // the next LayerNorm after the MLP: layer l+1's first, or the
            // final one (only in ALL mode, where the last layer is not pruned)
            const bool end = l + 1 == L;
            const float* nw = end ? h->lnf_w : h->layers[l + 1].ln1_w;
            const float* nb = end ? h->lnf_b : h->layers[l + 1].ln1_b;
            if (const int cb = attn_proj_cb(h, B, T)) {
                // attention with each head's share of c_proj, then the
                // sum over heads with the bias, the residual and LayerNorm 2
                {
                    double fl = 2.0 * C * (double)T * (T + 1) * B + 2.0 * rows * C * C;
                    double by = 4.0 * (rows * C * 4 + (double)C * C + (double)H * rows * C);
                    Timed t(h, CNGPT_K_ATTN, fl, by);
                    HIP_TRY(launch_attention_proj(qkv, seq_stride, w.proj_w, h->gemm_part, B, T,
                                                  C, H, cb, h->stream));
                }
                GemmArgs a{};
                a.M = (int)rows; a.N = C; a.K = C;
                a.bias = w.proj_b; a.Y = h->x; a.ldy = C;
                a.part = h->gemm_part; a.part_cap = GEMM_PART_FLOATS;
                a.ln_w = w.ln2_w; a.ln_b = w.ln2_b; a.ln_out = h->ln;
                a.epi = EPI_RESID;
                Timed t(h, CNGPT_K_LAYERNORM, 0.0, 4.0 * rows * C * (H + 3));
                HIP_TRY(launch_sum_heads(a, H, h->stream));
            } else {
                {
                    double fl = 2.0 * C * (double)T * (T + 1) * B;
                    double by = 4.0 * rows * C * 4;  // q,k,v read + out written
                    Timed t(h, CNGPT_K_ATTN, fl, by);
                    HIP_TRY(launch_attention_causal(qkv, seq_stride, h->aout, B, T, C, H,
                                                    h->stream));
                }
                if (run_gemm(h, h->aout, w.proj_w, w.proj_b, h->x, (int)rows, C, C, EPI_RESID, 0,
                             0, -1, 0, nullptr, w.ln2_w, w.ln2_b, h->ln))
                    return -1;
            }
            if (run_gemm(h, h->ln, w.fc_w, w.fc_b, h->hid, (int)rows, 4 * C, C, EPI_BIAS_GELU) ||
                run_gemm(h, h->hid, w.mlp_w, w.mlp_b, h->x, (int)rows, C, 4 * C, EPI_RESID, 0, 0,
                         -1, 0, nullptr, nw, nb, h->ln))
                return -1;
        } else {
            // Last layer, LAST mode: the final query row of each sequence only,
            // then the rest of the layer on those B rows (fast.c:287-311).
            {
                Timed t(h, CNGPT_K_GATHER, 0.0, 8.0 * B * C);
                HIP_TRY(launch_gather_rows(h->x + (size_t)(T - 1) * C, (long)T * C, h->xc, B, C,
                                           h->stream));
            }
            if (run_attn_row_proj(h, qkv, seq_stride, B, T - 1, nullptr, T, w, h->xc)) return -1;
            if (run_ln_gemm(h, h->xc, w.ln2_w, w.ln2_b, h->lnc, w.fc_w, w.fc_b, h->hidc, B, 4 * C,
                            EPI_BIAS_GELU))
                return -1;
            if (run_gemm(h, h->hidc, w.mlp_w, w.mlp_b, h->xc, B, C, 4 * C, EPI_RESID)) return -1;
        }
    }
    if (mode == CNGPT_ALL) {
        // ln holds the final LayerNorm of every row (formed by the last proj)
        if (run_gemm(h, h->ln, h->wte, nullptr, h->logits, (int)rows, c.vocab_size, C, EPI_STORE))
            return -1;
        h->logits_count = (size_t)rows * c.vocab_size;
    } else {
        if (run_lm_head(h, h->xc, B, want_tok, nullptr)) return -1;
    }
    h->curB = B; h->curT = T; h->curMode = mode;
    return 0;
}

// A forward of B x T tokens already in h->tok (no KV cache, no token
// feed): the captured graph of this shape replayed, or with timing events
// or graphs off, its kernels launched directly. A forward is ~8 launches
// per layer; at B=1 T=128 their host-side enqueueing (about 10 us each)
// outlasts the kernels, one graph launch does not.
int run_forward(cngpt_hip_ctx* h, int B, int T, int mode) {
    if (h->prof || !h->use_graph) return enqueue_forward(h, B, T, mode, false, false);
    if (!h->fwd_exec || h->fwd_B != B || h->fwd_T != T || h->fwd_mode != mode ||
        h->fwd_act != h->d_act || h->fwd_par != h->d_params) {
        drop_fwd_graph(h);
        hipGraph_t g = nullptr;
        HIP_TRY(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
        const int rc = enqueue_forward(h, B, T, mode, false, false);
        const hipError_t e = hipStreamEndCapture(h->stream, &g);
        if (rc || e != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            (void)hipGetLastError();
            return rc ? -1 : fail("forward graph capture failed: %s", hipGetErrorString(e));
        }
        hipGraphExec_t ex = nullptr;
        const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ei != hipSuccess) return fail("forward graph instantiate: %s", hipGetErrorString(ei));
        h->fwd_exec = ex;
        h->fwd_B = B; h->fwd_T = T; h->fwd_mode = mode;
        h->fwd_act = h->d_act;
        h->fwd_par = h->d_params;
    }
    HIP_TRY(hipGraphLaunch(h->fwd_exec, h->stream));
    h->curB = B; h->curT = T; h->curMode = mode;
    h->logits_count = (size_t)(mode == CNGPT_ALL ? (long)B * T : B) * h->cfg.vocab_size;
    return 0;
}

// One decode step: the token next_tok[b] at position *pos for every cached
// sequence; logits [B, V], the greedy tokens in next_tok, then *pos += 1.
// Every position-dependent value is read from device memory, so the same
// enqueued sequence (a captured graph) serves every step.
int enqueue_decode_step(cngpt_hip_ctx* h) {
    const cngpt_hip_config& c = h->cfg;
    const int C = c.n_embd, L = c.n_layer;
    const int B = h->kvB;
    const long cap = h->capKV;
    const bool fused_embed = B <= SKINNY;
    // over more than SKINNY rows, every LayerNorm after the first is formed
    // by the residual product before it (in its split-K sum)
    const bool fuse_ln = B > SKINNY;
    if (!fused_embed) {
        Timed t(h, CNGPT_K_EMBED, 0.0, 12.0 * C * B);
        HIP_TRY(launch_embed(h->next_tok, h->wte, h->wpe, h->xc, B, 1, C, c.vocab_size, 0, h->pos,
                             h->dev_err, h->hist, cap, h->stream));
    }
    const bool fold_qkv = fuse_ln && attention_dec_one_pass(B, c.n_head) && h->use_qkv_fold;
    for (int l = 0; l < L; l++) {
        const LayerW& w = h->layers[l];
        float* kvl = h->qkv + (size_t)l * B * cap * 3 * C;
        int qkv_ks = 0;
        if (l == 0 && fused_embed) {
            // x = wte[token] + wpe[pos] is built inside layer 0's QKV product
            DecGemvArgs d{};
            d.ln_w = w.ln1_w; d.ln_b = w.ln1_b;
            d.emb.tok = h->next_tok; d.emb.wte = h->wte; d.emb.wpe = h->wpe;
            d.emb.pos_dev = h->pos; d.emb.x_out = h->xc; d.emb.hist = h->hist;
            d.emb.hist_stride = cap; d.emb.V = c.vocab_size; d.emb.err = h->dev_err;
            d.W = w.attn_w; d.bias = w.attn_b; d.Y = kvl; d.ldy = 3L * C;
            d.M = B; d.N = 3 * C; d.K = C;
            d.seg = 1; d.seg_stride = cap; d.row_off_dev = h->pos;
            d.epi = EPI_BIAS;
            Timed t(h, CNGPT_K_GEMV, 2.0 * B * 3 * C * C,
                    4.0 * (3.0 * C * C + 3.0 * B * C + 2.0 * B * C));
            HIP_TRY(launch_dgemv(d, h->stream));
        } else if (fuse_ln) {
            // LayerNorm 1 was formed with the previous layer's residual (in
            // layer 0: here); where the one-pass attention follows and the
            // product splits K, the attention sums its partials
            if (l == 0 && run_ln(h, h->xc, C, w.ln1_w, w.ln1_b, h->lnc, B)) return -1;
            if (run_gemm(h, h->lnc, w.attn_w, w.attn_b, kvl, B, 3 * C, C, EPI_BIAS, 1, cap, 3L * C,
                         0, h->pos, nullptr, nullptr, nullptr, fold_qkv ? &qkv_ks : nullptr))
                return -1;
        } else if (run_ln_gemm(h, h->xc, w.ln1_w, w.ln1_b, h->lnc, w.attn_w, w.attn_b, kvl, B,
                               3 * C, EPI_BIAS, 1, cap, 3L * C, h->pos)) {
            return -1;
        }
        if (fuse_ln) {
            // the residual products also form the next LayerNorm (2, then 1
            // of the next layer or the final one) while summing their splits
            const bool last = l + 1 == L;
            const LayerW& wn = h->layers[last ? l : l + 1];
            if (run_attn_row_proj(h, kvl, cap, B, 0, h->pos, (int)cap, w, h->xc, w.ln2_w,
                                  w.ln2_b, h->lnc, qkv_ks) ||
                run_gemm(h, h->lnc, w.fc_w, w.fc_b, h->hidc, B, 4 * C, C, EPI_BIAS_GELU) ||
                run_gemm(h, h->hidc, w.mlp_w, w.mlp_b, h->xc, B, C, 4 * C, EPI_RESID, 0, 0, -1, 0,
                         nullptr, last ? h->lnf_w : wn.ln1_w, last ? h->lnf_b : wn.ln1_b,
                         h->lnc))
                return -1;
            continue;
        }
        if (run_attn_row_proj(h, kvl, cap, B, 0, h->pos, (int)cap, w, h->xc)) return -1;
        if (run_ln_gemm(h, h->xc, w.ln2_w, w.ln2_b, h->lnc, w.fc_w, w.fc_b, h->hidc, B, 4 * C,
                        EPI_BIAS_GELU))
            return -1;
        if (run_gemm(h, h->hidc, w.mlp_w, w.mlp_b, h->xc, B, C, 4 * C, EPI_RESID)) return -1;
    }
    if (run_lm_head(h, h->xc, B, true, h->pos, fuse_ln)) return -1;
    h->curB = B; h->curT = 1; h->curMode = CNGPT_LAST;
    return 0;
}

// Run one decode step: replay the captured graph (captured on first use,
// again after the arena or the batch changed); direct launches while the
// timing counters are on, so every kernel gets its event pair.
int run_decode_step(cngpt_hip_ctx* h) {
    if (h->prof || !h->use_graph) {
        if (enqueue_decode_step(h)) return -1;
    } else {
        if (!h->step_exec || h->graph_B != h->kvB || h->graph_cap != h->capKV ||
            h->graph_act != h->d_act || h->graph_par != h->d_params) {
            drop_graph(h);
            hipGraph_t g = nullptr;
            HIP_TRY(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
            const int rc = enqueue_decode_step(h);
            const hipError_t e = hipStreamEndCapture(h->stream, &g);
            if (rc || e != hipSuccess) {
                if (g) (void)hipGraphDestroy(g);
                (void)hipGetLastError();
                return rc ? -1 : fail("decode graph capture failed: %s", hipGetErrorString(e));
            }
            hipGraphExec_t ex = nullptr;
            const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (ei != hipSuccess) return fail("decode graph instantiate: %s", hipGetErrorString(ei));
            h->step_exec = ex;
            h->graph_B = h->kvB;
            h->graph_cap = h->capKV;
            h->graph_act = h->d_act;
            h->graph_par = h->d_params;
        }
        HIP_TRY(hipGraphLaunch(h->step_exec, h->stream));
        h->curB = h->kvB; h->curT = 1; h->curMode = CNGPT_LAST;
        h->logits_count = (size_t)h->kvB * h->cfg.vocab_size;
    }
    h->kvLen += 1;
    h->last_path = CNGPT_DECODE_KERNELS;
    return 0;
}

// Whether the next decode steps run as one persistent launch: one cached
// sequence, head size 64, widths the kernel supports, cooperative launch.
bool persist_usable(cngpt_hip_ctx* h) {
    if (h->decode_path == CNGPT_DECODE_KERNELS || h->kvB != 1) return false;
    if (h->persist_G < 0) h->persist_G = persist_workgroups(h->device);
    const cngpt_hip_config& c = h->cfg;
    return h->persist_G > 0 &&
           persist_supported(c.n_embd, c.n_head, c.vocab_size, h->capKV, h->persist_G);
}

int persist_refused(cngpt_hip_ctx* h) {
    return fail("persistent decode needs one cached sequence (B=%d), head size 64, n_embd <= "
                "768, a device with cooperative launch and enough CUs for the widths and the "
                "cache capacity", h->kvB);
}

// run_persist's result when the cooperative launch itself was refused (no
// step ran, nothing changed on the device): another process on the GPU can
// hold what a cooperative launch needs. The handle then takes the
// kernel-per-stage path for the rest of its life.
constexpr int PERSIST_REFUSED = 1;

// n greedy decode steps of the single cached sequence as one launch.
// n persistent steps; with top_k > 0 each step samples its token with
// draws[step] inside the launch. *done (when set) receives the steps that
// ran: a sampling step whose candidates overflowed ends the launch early,
// its logits in place and its token left to the host.
int run_persist(cngpt_hip_ctx* h, int n, float temp = 0.f, int top_k = 0,
                const float* draws = nullptr, int* done = nullptr) {
    const cngpt_hip_config& c = h->cfg;
    const double C = c.n_embd, L = c.n_layer, V = c.vocab_size;
    PersistArgs a{};
    a.layers = h->d_layers;
    a.wte = h->wte; a.wpe = h->wpe; a.lnf_w = h->lnf_w; a.lnf_b = h->lnf_b;
    a.L = c.n_layer; a.C = c.n_embd; a.H = c.n_head; a.V = c.vocab_size; a.cap = h->capKV;
    a.cache = h->qkv; a.tagged = h->ptag;
    a.logits = h->logits; a.hist = h->hist;
    a.pos = h->pos; a.tok = h->next_tok; a.err = h->dev_err;
    a.n_steps = n;
    a.temp = temp; a.top_k = top_k; a.draws = draws;
    a.steps_done = done ? h->dev_err + 2 : nullptr;
    // tags only grow; before they would wrap, clear the words and restart
    const unsigned need = persist_tags(c.n_layer, n);
    if (h->ptag_next > 0xF0000000u - need) {
        HIP_TRY(hipMemsetAsync(h->ptag, 0,
                               (size_t)persist_tagged_words(c.n_embd, c.n_head) * 8, h->stream));
        h->ptag_next = 0;
    }
    a.tag0 = h->ptag_next;
    h->ptag_next += need;
    a.scale = 1.0f / sqrtf((float)(c.n_embd / c.n_head));
    // weights + K/V rows read per step (keys 0..t), summed over the steps
    double bytes = 0.0, flops = 0.0;
    for (int i = 0; i < n; i++) {
        const double t = h->kvLen + i;
        bytes += 4.0 * (L * (12.0 * C * C + 13.0 * C) + V * C + 2.0 * C) + 8.0 * L * C * (t + 1.0);
        flops += 2.0 * (L * 12.0 * C * C + V * C) + 4.0 * L * C * (t + 1.0);
    }
    {
        Timed tm(h, CNGPT_K_STEP, flops, bytes);
        const hipError_t e = launch_decode_persist(a, h->persist_G, h->stream);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            h->persist_G = 0;
            if (h->decode_path == CNGPT_DECODE_PERSISTENT)
                return fail("persistent decode launch refused: %s", hipGetErrorString(e));
            return PERSIST_REFUSED;
        }
    }
    if (done) {
        HIP_TRY(hipMemcpyAsync(done, h->dev_err + 2, sizeof(int), hipMemcpyDeviceToHost,
                               h->stream));
        HIP_TRY(hipStreamSynchronize(h->stream));
        if (*done < 1 || *done > n) return fail("persistent decode ran %d of %d steps", *done, n);
        n = *done;
    }
    h->kvLen += n;
    h->curB = 1; h->curT = 1; h->curMode = CNGPT_LAST;
    h->logits_count = (size_t)c.vocab_size;
    h->last_path = CNGPT_DECODE_PERSISTENT;
    return 0;
}

int run_sample(cngpt_hip_ctx* h, const float* draws, float temp, int top_k) {
    Timed t(h, CNGPT_K_SAMPLE, 0.0, 4.0 * h->kvB * h->cfg.vocab_size);
    HIP_TRY(launch_sample(h->logits, h->kvB, h->cfg.vocab_size, temp, top_k, draws, h->prob,
                          h->ldp, h->samp_part, h->next_tok, h->stream));
    return 0;
}

int need_params(const cngpt_hip_ctx* h) {
    if (!h) return fail("null handle");
    if (!h->have_params) return fail("no parameters loaded (cngpt_hip_load_params)");
    return 0;
}

int check_dev_err(cngpt_hip_ctx* h) {
    if (!h->dev_err) return 0;  // no activation arena yet: nothing has flagged
    int e = 0;
    HIP_TRY(hipMemcpyAsync(&e, h->dev_err, sizeof(int), hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    if (e) {
        HIP_TRY(hipMemsetAsync(h->dev_err, 0, sizeof(int), h->stream));
        if (e & 2) return fail("persistent decode: a wait for a value of another workgroup timed out");
        if (e & 4) return fail("cross-entropy targets outside [0, %d) were clamped", h->cfg.vocab_size);
        if (e & ATTN_DEC_TIMEOUT)
            return fail("decode attention: a wait for the other half of a split (sequence, head) "
                        "pair timed out; its row is NaN");
        return fail("device-resident token ids outside [0, %d) were clamped", h->cfg.vocab_size);
    }
    return 0;
}

// ---------------------------------------------------------------- parameters

// Shapes the kernels take (on top of valid_cfg).
int check_shape(const cngpt_hip_config* cfg) {
    if (!valid_cfg(cfg)) return fail("invalid model shape");
    if (cfg->n_embd % 4) return fail("n_embd %d must be a multiple of 4", cfg->n_embd);
    const int hs = cfg->n_embd / cfg->n_head;
    if (hs != 8 && hs != 16 && hs != 32 && hs != 64 && hs != 128)
        return fail("head size %d not supported (8, 16, 32, 64, 128)", hs);
    if (cfg->n_embd > 2048) return fail("n_embd %d above 2048", cfg->n_embd);
    return 0;
}

long params_of(const cngpt_hip_config* c) {
    const long C = c->n_embd, V = c->vocab_size, T = c->block_size, L = c->n_layer;
    return V * C + T * C + L * (12 * C * C + 13 * C) + 2 * C;  // model.c:20-48
}

// Bytes of the packed weight copies: the token embedding (the lm_head's
// weights) and each layer's four matrices.
size_t packed_bytes(const cngpt_hip_config* cfg) {
    const int C = cfg->n_embd;
    const size_t layer = align_up(packed_w_floats(3 * C, C) * sizeof(float)) +
                         align_up(packed_w_floats(C, C) * sizeof(float)) +
                         align_up(packed_w_floats(4 * C, C) * sizeof(float)) +
                         align_up(packed_w_floats(C, 4 * C) * sizeof(float));
    return align_up(packed_w_floats(cfg->vocab_size, C) * sizeof(float)) + layer * cfg->n_layer;
}

// Packs the weight matrices (again, after an AdamW update marked them
// stale: ctx_params_written) in kernels on the handle's stream, ordered
// before what follows.
int fresh_packed(cngpt_hip_ctx* h) {
    if (!h->use_packed || h->packed_fresh) return 0;
    HIP_TRY(hipSetDevice(h->device));
    for (const cngpt_hip_ctx::Packed& p : h->packs)
        HIP_TRY(launch_pack_w(p.W, p.Wp, p.N, p.K, h->stream));
    h->packed_fresh = true;
    return 0;
}

// Make h->d_params hold the parameters of shape cfg: reuse the allocation
// when the shape is unchanged, else free it (and the activations, which
// depend on the shape) and allocate anew.
int params_prepare(cngpt_hip_ctx* h, const cngpt_hip_config* cfg) {
    HIP_TRY(hipSetDevice(h->device));
    if (h->d_params && memcmp(&h->cfg, cfg, sizeof(*cfg)) == 0) return 0;
    if (h->d_params) {
        HIP_TRY(hipStreamSynchronize(h->stream));
        drop_fwd_graph(h);
        HIP_TRY(hipFree(h->d_params));
        h->d_params = nullptr;
    }
    if (h->d_act) {
        drop_graph(h);
        HIP_TRY(hipFree(h->d_act));
        h->d_act = nullptr;
        h->capB = h->capT = h->capAll = h->capKV = 0;
        h->kvB = h->kvLen = 0;
    }
    h->have_params = false;
    h->d_layers = nullptr;
    // one allocation: the parameters, the table of per-layer pointers into
    // them that the persistent decode reads, the packed weight copies
    const long want = params_of(cfg);
    const size_t bytes = align_up((size_t)want * sizeof(float)) +
                         align_up((size_t)cfg->n_layer * sizeof(LayerW)) +
                         (h->use_packed ? packed_bytes(cfg) : 0);
    if (hipMalloc(&h->d_params, bytes) != hipSuccess) {
        (void)hipGetLastError();
        h->d_params = nullptr;
        return fail("parameter allocation of %ld floats failed", want);
    }
    h->d_layers = (LayerW*)((char*)h->d_params + align_up((size_t)want * sizeof(float)));
    h->cfg = *cfg;  // the allocation now has this shape
    return 0;
}

// Views of the uploaded parameters, carved like assign_weights
// (src/model.c:54-83), and their device table for the persistent decode.
int params_commit(cngpt_hip_ctx* h, const cngpt_hip_config* cfg) {
    h->cfg = *cfg;
    h->n_params = params_of(cfg);
    const long C = cfg->n_embd, V = cfg->vocab_size, T = cfg->block_size;
    const float* p = h->d_params;
    h->wte = p; p += V * C;
    h->wpe = p; p += T * C;
    h->layers.assign(cfg->n_layer, LayerW{});
    for (int l = 0; l < cfg->n_layer; l++) {
        LayerW& w = h->layers[l];
        w.ln1_w = p; p += C;
        w.ln1_b = p; p += C;
        w.attn_w = p; p += 3 * C * C;
        w.attn_b = p; p += 3 * C;
        w.proj_w = p; p += C * C;
        w.proj_b = p; p += C;
        w.ln2_w = p; p += C;
        w.ln2_b = p; p += C;
        w.fc_w = p; p += 4 * C * C;
        w.fc_b = p; p += 4 * C;
        w.mlp_w = p; p += C * 4 * C;
        w.mlp_b = p; p += C;
    }
    h->lnf_w = p; p += C;
    h->lnf_b = p;
    HIP_TRY(hipMemcpy(h->d_layers, h->layers.data(), (size_t)cfg->n_layer * sizeof(LayerW),
                      hipMemcpyHostToDevice));
    h->packs.clear();
    h->packed_of.clear();
    h->packed_fresh = false;
    if (h->use_packed) {
        char* q = (char*)h->d_layers + align_up((size_t)cfg->n_layer * sizeof(LayerW));
        auto add = [&](const float* W, int N, int K) {
            h->packs.push_back({W, (float*)q, N, K});
            h->packed_of[W] = (const float*)q;
            q += align_up(packed_w_floats(N, K) * sizeof(float));
        };
        const int c = (int)C;
        add(h->wte, (int)V, c);
        for (const LayerW& w : h->layers) {
            add(w.attn_w, 3 * c, c);
            add(w.proj_w, c, c);
            add(w.fc_w, 4 * c, c);
            add(w.mlp_w, c, 4 * c);
        }
        if (fresh_packed(h)) return -1;
    }
    h->have_params = true;
    return 0;
}

// ---------------------------------------------------------------- weight file

// The weight file: a 7 x int32 header (GPTHeader, src/model.h:19-30) and the
// flat fp32 parameters in assign_weights order (src/model.c:177-231).
constexpr int FILE_MAGIC = 0x434E4750;  // "CNGP"
constexpr int FILE_VERSION = 1;
constexpr size_t FILE_HEADER = 7 * sizeof(int);

struct WeightFile {
    int fd = -1;
    cngpt_hip_config cfg{};
    long n_params = 0;
};

// Open and validate: header present, magic and version, a valid shape and
// at least n_params floats after the header (the reference's gpt_load
// checks the magic and the data length, model.c:185-207).
int open_weight_file(const char* path, WeightFile* wf) {
    if (!path) return fail("null path");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail("%s: %s", path, strerror(errno));
    struct stat st;
    int hdr[7];
    int rc = 0;
    if (fstat(fd, &st) != 0) {
        rc = fail("%s: %s", path, strerror(errno));
    } else if ((size_t)st.st_size < FILE_HEADER ||
               pread(fd, hdr, FILE_HEADER, 0) != (ssize_t)FILE_HEADER) {
        rc = fail("%s: file ends inside its %d-byte header", path, (int)FILE_HEADER);
    } else if (hdr[0] != FILE_MAGIC) {
        rc = fail("%s: not a cngpt weight file (first word 0x%X)", path, (unsigned)hdr[0]);
    } else if (hdr[1] != FILE_VERSION) {
        rc = fail("%s: unsupported version %d (this build reads version %d)", path, hdr[1],
                  FILE_VERSION);
    } else {
        wf->cfg = cngpt_hip_config{hdr[2], hdr[3], hdr[4], hdr[5], hdr[6]};
        // bounds far above any GPT-2 shape keep the size arithmetic exact
        const bool in_range = hdr[2] <= 4096 && hdr[3] <= 4096 && hdr[4] <= 65536 &&
                              hdr[5] <= (1 << 24) && hdr[6] <= (1 << 20);
        if (!valid_cfg(&wf->cfg) || !in_range) {
            rc = fail("%s: invalid shape in header (n_layer %d, n_head %d, n_embd %d, vocab %d, "
                      "block %d)", path, hdr[2], hdr[3], hdr[4], hdr[5], hdr[6]);
        } else {
            wf->n_params = params_of(&wf->cfg);
            const double need = (double)FILE_HEADER + 4.0 * (double)wf->n_params;
            if ((double)st.st_size < need)
                rc = fail("%s: file ends before its parameters (%lld bytes, the header's shape needs %.0f)", path,
                          (long long)st.st_size, need);
        }
    }
    if (rc) {
        close(fd);
        return -1;
    }
    wf->fd = fd;
    return 0;
}

// Copy the file's parameters into h->d_params without a host copy of the
// whole buffer: READERS threads each pread chunks of CHUNK bytes into their
// own pinned staging buffers (NSTAGE per thread, reused once the copy out of
// them has completed) and enqueue the host-to-device copy of each chunk on
// the handle's stream, so reading, page-cache copies and DMA overlap.
constexpr size_t CHUNK = 16u << 20;
constexpr int NSTAGE = 2;
constexpr int MAX_READERS = 4;

int stream_to_device(cngpt_hip_ctx* h, const WeightFile& wf, const char* path) {
    const size_t total = (size_t)wf.n_params * sizeof(float);
    const size_t nchunks = (total + CHUNK - 1) / CHUNK;
    const int readers = (int)std::max<size_t>(1, std::min<size_t>(MAX_READERS, nchunks));
    struct Stage {
        void* buf = nullptr;
        hipEvent_t done = nullptr;
        bool used = false;
    };
    std::vector<Stage> st((size_t)readers * NSTAGE);
    int rc = 0;
    for (Stage& s : st) {
        if (hipHostMalloc(&s.buf, CHUNK, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&s.done, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            rc = fail("pinned staging allocation of %zu bytes failed", CHUNK);
            break;
        }
    }
    std::atomic<int> err{0};
    std::atomic<long> bad_chunk{-1};
    std::atomic<int> bad_errno{0};
    auto worker = [&](int r) {
        int k = 0;
        for (size_t c = r; c < nchunks && !err.load(); c += readers, k++) {
            Stage& s = st[(size_t)r * NSTAGE + k % NSTAGE];
            if (s.used && hipEventSynchronize(s.done) != hipSuccess) { err = 2; return; }
            const size_t off = c * CHUNK, len = std::min(CHUNK, total - off);
            size_t got = 0;
            while (got < len) {
                const ssize_t n = pread(wf.fd, (char*)s.buf + got, len - got,
                                        (off_t)(FILE_HEADER + off + got));
                if (n < 0 && errno == EINTR) continue;
                if (n <= 0) {
                    bad_chunk = (long)c;
                    bad_errno = n < 0 ? errno : 0;
                    err = 1;
                    return;
                }
                got += (size_t)n;
            }
            if (hipMemcpyAsync((char*)h->d_params + off, s.buf, len, hipMemcpyHostToDevice,
                               h->stream) != hipSuccess ||
                hipEventRecord(s.done, h->stream) != hipSuccess) {
                err = 2;
                return;
            }
            s.used = true;
        }
    };
    if (!rc) {
        std::vector<std::thread> pool;
        for (int r = 1; r < readers; r++) pool.emplace_back(worker, r);
        worker(0);
        for (std::thread& t : pool) t.join();
        const hipError_t se = hipStreamSynchronize(h->stream);
        if (err.load() == 1)
            rc = fail("%s: read failed at chunk %ld: %s", path, bad_chunk.load(),
                      bad_errno.load() ? strerror(bad_errno.load()) : "unexpected end of file");
        else if (err.load() == 2 || se != hipSuccess)
            rc = fail("%s: host-to-device copy failed: %s", path,
                      hipGetErrorString(se != hipSuccess ? se : hipGetLastError()));
    } else {
        (void)hipStreamSynchronize(h->stream);
    }
    for (Stage& s : st) {
        if (s.done) (void)hipEventDestroy(s.done);
        if (s.buf) (void)hipHostFree(s.buf);
    }
    return rc;
}

// The buffers enqueue_forward reads and writes, so that one forward can run
// on another set (the no-alloc scratch) and the handle's own come back
// afterwards, together with the state of its held logits.
struct FwdBufs {
    int *tok, *dev_err;
    float *x, *ln, *qkv, *aout, *hid, *logits, *xc, *lnc, *aoutc, *hidc, *attn_part, *gemm_part;
    int attn_splits;
    unsigned long long* dtag;
    unsigned* dcnt;
    int dtag_pairs;
    int curB, curT, curMode;
    size_t logits_count;
    bool prof;
};

FwdBufs fwd_bufs(const cngpt_hip_ctx* h) {
    return FwdBufs{h->tok, h->dev_err, h->x, h->ln, h->qkv, h->aout, h->hid, h->logits, h->xc,
                   h->lnc, h->aoutc, h->hidc, h->attn_part, h->gemm_part, h->attn_splits,
                   h->dtag, h->dcnt, h->dtag_pairs, h->curB, h->curT, h->curMode, h->logits_count, h->prof};
}

void set_fwd_bufs(cngpt_hip_ctx* h, const FwdBufs& f) {
    h->tok = f.tok; h->dev_err = f.dev_err;
    h->x = f.x; h->ln = f.ln; h->qkv = f.qkv; h->aout = f.aout; h->hid = f.hid;
    h->logits = f.logits;
    h->xc = f.xc; h->lnc = f.lnc; h->aoutc = f.aoutc; h->hidc = f.hidc;
    h->attn_part = f.attn_part; h->gemm_part = f.gemm_part; h->attn_splits = f.attn_splits;
    h->dtag = f.dtag; h->dcnt = f.dcnt; h->dtag_pairs = f.dtag_pairs;
    h->curB = f.curB; h->curT = f.curT; h->curMode = f.curMode;
    h->logits_count = f.logits_count;
    h->prof = f.prof;
}

// Carve of the scratch for a forward of B x T: floats from `base` (a null
// base only counts them). Regions start on 256-byte boundaries.
long carve_scratch(const cngpt_hip_config& c, int B, int T, float* base, FwdBufs* f) {
    const long C = c.n_embd, H = c.n_head, hs = C / H, rows = (long)B * T;
    const int kps = attn_dec_keys_per_split((int)hs);
    const int splits = (T + kps - 1) / kps;
    // the tag region first, at its fixed offset
    const long tag_words = (long)attn_dec1_tag_words(attn_dec1_split_pairs(), SCRATCH_TAG_HS);
    f->dtag = base ? (unsigned long long*)base : nullptr;
    f->dcnt = base ? (unsigned*)(f->dtag + tag_words) : nullptr;
    f->dtag_pairs = hs <= SCRATCH_TAG_HS ? attn_dec1_split_pairs() : 0;
    long off = scratch_tag_floats();
    auto take = [&](long n) {
        float* r = base ? base + off : nullptr;
        off += (n + 63) / 64 * 64;
        return r;
    };
    float* err = take(1);
    f->x = take(rows * C);
    f->ln = take(rows * C);
    f->qkv = take(rows * 3 * C);
    f->aout = take(rows * C);
    f->hid = take(rows * 4 * C);
    f->xc = take(B * C);
    f->lnc = take(B * C);
    f->aoutc = take(B * C);
    f->hidc = take(B * 4 * C);
    f->attn_part = take((long)B * H * splits * (hs + 4));
    f->attn_splits = splits;
    f->gemm_part = take(GEMM_PART_FLOATS);
    f->dev_err = (int*)err;
    return off;
}

}  // namespace

// Internal view for train_host.cpp (ctx_view.h).
int ctx_view(cngpt_hip_ctx* h, CtxView* v) {
    if (need_params(h)) return -1;
    v->device = h->device;
    v->stream = h->stream;
    v->cfg = h->cfg;
    v->params = h->d_params;
    v->n_params = h->n_params;
    v->wte = h->wte;
    v->wpe = h->wpe;
    v->lnf_w = h->lnf_w;
    v->lnf_b = h->lnf_b;
    v->layers = h->layers.data();
    return 0;
}

void ctx_params_written(cngpt_hip_ctx* h) {
    if (h) h->packed_fresh = false;
}

int ctx_fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return -1;
}

// ==================================================================== C ABI

extern "C" {

const char* cngpt_hip_last_error(void) { return g_err; }

long cngpt_hip_num_params(const cngpt_hip_config* c) {
    if (!valid_cfg(c)) return -1;
    return params_of(c);
}

int cngpt_hip_create(int device, cngpt_hip_ctx** out) {
    if (!out) return fail("null output pointer");
    *out = nullptr;
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail("device %d not present (%d devices)", device, n);
    HIP_TRY(hipSetDevice(device));
    if (scratch_setup(device)) return -1;
    cngpt_hip_ctx* h = new cngpt_hip_ctx();
    h->device = device;
    const char* g = getenv("CNGPT_HIP_GRAPH");
    h->use_graph = !(g && g[0] == '0');
    // Under rocprofv3 (which exports ROCP_TOOL_LIBRARIES and
    // ROCPROF_OUTPUT_PATH to the program it profiles) no captured decode
    // graph is replayed: the first replay of a freshly instantiated step
    // graph ended in a segmentation fault inside hipGraphLaunch there, whose
    // cause is not known. Decode steps then launch their kernels directly.
    const char* tool = getenv("ROCP_TOOL_LIBRARIES");
    const char* rp = getenv("ROCPROF_OUTPUT_PATH");
    if (h->use_graph && ((tool && tool[0]) || (rp && rp[0]))) {
        h->use_graph = false;
        fprintf(stderr, "cngpt_hip: profiler detected (rocprofv3 environment); decode steps "
                        "launch kernels directly instead of replaying captured graphs\n");
    }
    const char* pp = getenv("CNGPT_HIP_PERSIST");
    if (pp && pp[0] == '0') h->decode_path = CNGPT_DECODE_KERNELS;
    const char* pk = getenv("CNGPT_HIP_PACK");
    h->use_packed = !(pk && pk[0] == '0');
    const char* ap = getenv("CNGPT_HIP_ATTNPROJ");
    h->use_attn_proj = !(ap && ap[0] == '0');
    // 2, 3 or 4: that many column blocks per wavefront where they divide C
    if (ap && ap[0] >= '2' && ap[0] <= '4') h->attn_proj_cb = ap[0] - '0';
    const char* qf = getenv("CNGPT_HIP_QKVFOLD");
    h->use_qkv_fold = !(qf && qf[0] == '0');
    if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess) {
        delete h;
        return fail("hipStreamCreate failed");
    }
    *out = h;
    return 0;
}

void cngpt_hip_destroy(cngpt_hip_ctx* h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    drop_graph(h);
    drop_fwd_graph(h);
    for (hipEvent_t e : h->pool) (void)hipEventDestroy(e);
    if (h->d_act) (void)hipFree(h->d_act);
    if (h->d_params) (void)hipFree(h->d_params);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

int cngpt_hip_load_params(cngpt_hip_ctx* h, const cngpt_hip_config* cfg, const float* params,
                          long n_params) {
    if (!h) return fail("null handle");
    if (check_shape(cfg)) return -1;
    const long want = cngpt_hip_num_params(cfg);
    if (!params || n_params != want)
        return fail("parameter count %ld does not match the shape (%ld)", n_params, want);
    if (params_prepare(h, cfg)) return -1;
    HIP_TRY(hipMemcpyAsync(h->d_params, params, (size_t)want * sizeof(float),
                           hipMemcpyHostToDevice, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return params_commit(h, cfg);
}

int cngpt_hip_file_config(const char* path, cngpt_hip_config* cfg, long* n_params) {
    WeightFile wf;
    if (open_weight_file(path, &wf)) return -1;
    close(wf.fd);
    if (cfg) *cfg = wf.cfg;
    if (n_params) *n_params = wf.n_params;
    return 0;
}

int cngpt_hip_load_file(cngpt_hip_ctx* h, const char* path, cngpt_hip_config* cfg_out) {
    if (!h) return fail("null handle");
    WeightFile wf;
    if (open_weight_file(path, &wf)) return -1;
    int rc = check_shape(&wf.cfg);
    if (!rc) rc = params_prepare(h, &wf.cfg);
    if (!rc) rc = stream_to_device(h, wf, path);
    close(wf.fd);
    if (rc) {
        // the device copy is incomplete: the handle holds no parameters
        h->have_params = false;
        return -1;
    }
    if (params_commit(h, &wf.cfg)) return -1;
    if (cfg_out) *cfg_out = wf.cfg;
    return 0;
}

int cngpt_hip_reserve(cngpt_hip_ctx* h, int B, int T, int mode, int kv_capacity) {
    if (need_params(h)) return -1;
    if (B <= 0 || T <= 0) return fail("B=%d T=%d must be positive", B, T);
    if (T > h->cfg.block_size) return fail("T=%d exceeds block_size %d", T, h->cfg.block_size);
    if (kv_capacity < 0 || kv_capacity > h->cfg.block_size)
        return fail("kv capacity %d outside [0, %d]", kv_capacity, h->cfg.block_size);
    HIP_TRY(hipSetDevice(h->device));
    return ensure_arena(h, B, T, mode == CNGPT_ALL, kv_capacity);
}

int cngpt_hip_upload_tokens(cngpt_hip_ctx* h, const int* tokens, int B, int T) {
    if (need_params(h)) return -1;
    if (!tokens) return fail("null tokens");
    if (cngpt_hip_reserve(h, B, T, CNGPT_LAST, 0)) return -1;
    if (check_tokens(h, tokens, (long)B * T)) return -1;
    HIP_TRY(hipMemcpyAsync(h->tok, tokens, (size_t)B * T * sizeof(int), hipMemcpyHostToDevice,
                           h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return 0;
}

int cngpt_hip_forward_resident(cngpt_hip_ctx* h, int B, int T, int mode) {
    if (need_params(h) || fresh_packed(h)) return -1;
    if (mode != CNGPT_LAST && mode != CNGPT_ALL) return fail("bad mode %d", mode);
    if (B > h->capB || T > h->capT || (mode == CNGPT_ALL && !h->capAll))
        return fail("forward_resident: arena not reserved for B=%d T=%d mode=%d", B, T, mode);
    HIP_TRY(hipSetDevice(h->device));
    h->kvB = h->kvLen = 0;
    return run_forward(h, B, T, mode);
}

int cngpt_hip_forward_noalloc(cngpt_hip_ctx* h, const int* tokens, int B, int T, int mode,
                              float* logits, int* err) {
    if (need_params(h) || fresh_packed(h)) return -1;
    if (mode != CNGPT_LAST && mode != CNGPT_ALL) return fail("bad mode %d", mode);
    if (!tokens || !logits) return fail("forward_noalloc: null device pointer");
    if (B <= 0 || T <= 0) return fail("B=%d T=%d must be positive", B, T);
    if (T > h->cfg.block_size) return fail("T=%d exceeds block_size %d", T, h->cfg.block_size);
    FwdBufs f{};
    const long need = carve_scratch(h->cfg, B, T, nullptr, &f);
    if (need > SCRATCH_FLOATS)
        return fail("forward_noalloc: B=%d T=%d needs %ld floats of scratch; it holds %ld "
                    "(%ld MiB)", B, T, need, SCRATCH_FLOATS, SCRATCH_FLOATS * 4 >> 20);
    float* base = scratch_of(h->device);
    if (!base) return fail("forward_noalloc: no scratch address for device %d", h->device);
    HIP_TRY(hipSetDevice(h->device));
    carve_scratch(h->cfg, B, T, base, &f);
    f.tok = const_cast<int*>(tokens);  // read only (token ids of the embedding)
    if (err) f.dev_err = err;
    f.logits = logits;
    f.prof = false;  // no timing events: their pool may grow
    // the token-range flag starts at zero (a kernel: callers may capture this)
    k_zero_i32<<<1, 64, 0, h->stream>>>(f.dev_err, 1);
    HIP_TRY(hipGetLastError());
    const FwdBufs saved = fwd_bufs(h);
    set_fwd_bufs(h, f);
    const int rc = enqueue_forward(h, B, T, mode, false, false);
    set_fwd_bufs(h, saved);
    return rc;
}

int cngpt_hip_forward(cngpt_hip_ctx* h, const int* tokens, int B, int T, int mode,
                      float* logits_out) {
    if (need_params(h) || fresh_packed(h)) return -1;
    if (mode != CNGPT_LAST && mode != CNGPT_ALL) return fail("bad mode %d", mode);
    if (!tokens) return fail("null tokens");
    if (B <= 0 || T <= 0) return fail("B=%d T=%d must be positive", B, T);
    if (T > h->cfg.block_size) return fail("T=%d exceeds block_size %d", T, h->cfg.block_size);
    if (check_tokens(h, tokens, (long)B * T)) return -1;
    HIP_TRY(hipSetDevice(h->device));
    if (ensure_arena(h, B, T, mode == CNGPT_ALL, 0)) return -1;
    h->kvB = h->kvLen = 0;
    HIP_TRY(hipMemcpyAsync(h->tok, tokens, (size_t)B * T * sizeof(int), hipMemcpyHostToDevice,
                           h->stream));
    if (run_forward(h, B, T, mode)) return -1;
    if (logits_out)
        HIP_TRY(hipMemcpyAsync(logits_out, h->logits, h->logits_count * sizeof(float),
                               hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return 0;
}

int cngpt_hip_synchronize(cngpt_hip_ctx* h) {
    if (!h) return fail("null handle");
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return check_dev_err(h);
}

int cngpt_hip_read_logits(cngpt_hip_ctx* h, size_t offset, size_t count, float* dst) {
    if (!h || !dst) return fail("null argument");
    if (!h->logits || offset + count > h->logits_count)
        return fail("logits range [%zu, %zu) outside the %zu held", offset, offset + count,
                    h->logits_count);
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipMemcpyAsync(dst, h->logits + offset, count * sizeof(float), hipMemcpyDeviceToHost,
                           h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return 0;
}

const float* cngpt_hip_logits_device(cngpt_hip_ctx* h) { return h ? h->logits : nullptr; }

int cngpt_hip_upload_targets(cngpt_hip_ctx* h, const int* targets, int B, int T) {
    if (need_params(h)) return -1;
    if (!targets) return fail("null targets");
    if (B <= 0 || T <= 0) return fail("B=%d T=%d must be positive", B, T);
    if (!h->tgt || (long)B * T > (long)h->capB * h->capT)
        return fail("targets [%d, %d] exceed the reserved %d x %d rows", B, T, h->capB, h->capT);
    for (long i = 0; i < (long)B * T; i++)
        if (targets[i] < 0 || targets[i] >= h->cfg.vocab_size)
            return fail("target %d at index %ld outside [0, %d)", targets[i], i,
                        h->cfg.vocab_size);
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipMemcpyAsync(h->tgt, targets, (size_t)B * T * sizeof(int), hipMemcpyHostToDevice,
                           h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return 0;
}

int cngpt_hip_cross_entropy_resident(cngpt_hip_ctx* h, int B, int T, int probs) {
    if (need_params(h)) return -1;
    if (B <= 0 || T <= 0) return fail("B=%d T=%d must be positive", B, T);
    const long rows = (long)B * T;
    const int V = h->cfg.vocab_size;
    if (!h->logits || (size_t)rows * V != h->logits_count)
        return fail("cross_entropy: %ld rows of %d logits, but %zu logits are held", rows, V,
                    h->logits_count);
    if (rows > (long)h->capB * h->capT)
        return fail("targets [%d, %d] exceed the reserved %d x %d rows", B, T, h->capB, h->capT);
    HIP_TRY(hipSetDevice(h->device));
    {
        Timed t(h, CNGPT_K_LOSS, 0.0, 4.0 * rows * V * (probs ? 3 : 1) + 8.0 * rows);
        HIP_TRY(launch_cross_entropy(h->logits, rows, V, h->tgt, h->row_loss, h->loss, probs,
                                     h->dev_err, h->stream));
    }
    h->loss_rows = rows;
    return 0;
}

int cngpt_hip_read_loss(cngpt_hip_ctx* h, float* loss_out, float* row_loss) {
    if (!h) return fail("null handle");
    if (h->loss_rows <= 0) return fail("no cross-entropy has been computed");
    HIP_TRY(hipSetDevice(h->device));
    if (loss_out)
        HIP_TRY(hipMemcpyAsync(loss_out, h->loss, sizeof(float), hipMemcpyDeviceToHost,
                               h->stream));
    if (row_loss)
        HIP_TRY(hipMemcpyAsync(row_loss, h->row_loss, (size_t)h->loss_rows * sizeof(float),
                               hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return check_dev_err(h);
}

int cngpt_hip_cross_entropy(cngpt_hip_ctx* h, const int* targets, int B, int T, int probs,
                            float* loss_out, float* row_loss) {
    if (cngpt_hip_upload_targets(h, targets, B, T)) return -1;
    if (cngpt_hip_cross_entropy_resident(h, B, T, probs)) return -1;
    return cngpt_hip_read_loss(h, loss_out, row_loss);
}

int cngpt_hip_decode_begin(cngpt_hip_ctx* h, const int* prompt, int B, int T, int capacity,
                           float* logits_out) {
    if (need_params(h) || fresh_packed(h)) return -1;
    if (!prompt) return fail("null prompt");
    if (B <= 0 || T <= 0) return fail("B=%d T=%d must be positive", B, T);
    if (capacity <= T || capacity > h->cfg.block_size)
        return fail("capacity %d must be in (T=%d, block_size=%d]", capacity, T,
                    h->cfg.block_size);
    if (check_tokens(h, prompt, (long)B * T)) return -1;
    HIP_TRY(hipSetDevice(h->device));
    if (ensure_arena(h, B, T, 0, capacity)) return -1;
    h->kvB = h->kvLen = 0;
    HIP_TRY(hipMemcpyAsync(h->tok, prompt, (size_t)B * T * sizeof(int), hipMemcpyHostToDevice,
                           h->stream));
    if (enqueue_forward(h, B, T, CNGPT_LAST, true, true)) return -1;
    // prompt -> token history; decode position = T
    HIP_TRY(hipMemcpy2DAsync(h->hist, (size_t)h->capKV * sizeof(int), h->tok,
                             (size_t)T * sizeof(int), (size_t)T * sizeof(int), B,
                             hipMemcpyDeviceToDevice, h->stream));
    h->pos_host = T;
    HIP_TRY(hipMemcpyAsync(h->pos, &h->pos_host, sizeof(int), hipMemcpyHostToDevice, h->stream));
    if (logits_out)
        HIP_TRY(hipMemcpyAsync(logits_out, h->logits, (size_t)B * h->cfg.vocab_size * sizeof(float),
                               hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    h->kvB = B;
    h->kvLen = T;
    return 0;
}

int cngpt_hip_decode_step(cngpt_hip_ctx* h, const int* tokens, float* logits_out) {
    if (need_params(h) || fresh_packed(h)) return -1;
    if (h->kvB == 0) return fail("decode_step before decode_begin");
    if (h->kvLen >= h->capKV)
        return fail("KV cache full (%d positions)", h->capKV);
    HIP_TRY(hipSetDevice(h->device));
    const int B = h->kvB;
    if (tokens) {
        if (check_tokens(h, tokens, B)) return -1;
        HIP_TRY(hipMemcpyAsync(h->next_tok, tokens, (size_t)B * sizeof(int),
                               hipMemcpyHostToDevice, h->stream));
        // the caller's buffer may be reused as soon as this returns
        HIP_TRY(hipStreamSynchronize(h->stream));
    }
    bool persist = persist_usable(h);
    if (!persist && h->decode_path == CNGPT_DECODE_PERSISTENT) return persist_refused(h);
    if (persist) {
        const int rc = run_persist(h, 1);
        if (rc < 0) return -1;
        persist = rc == 0;
    }
    if (!persist && run_decode_step(h)) return -1;
    if (logits_out) {
        HIP_TRY(hipMemcpyAsync(logits_out, h->logits, (size_t)B * h->cfg.vocab_size * sizeof(float),
                               hipMemcpyDeviceToHost, h->stream));
        HIP_TRY(hipStreamSynchronize(h->stream));
    }
    return persist ? check_dev_err(h) : 0;
}

int cngpt_hip_generate(cngpt_hip_ctx* h, int n_new, float temperature, int top_k,
                       const float* draws, int* out_tokens) {
    if (need_params(h) || fresh_packed(h)) return -1;
    if (h->kvB == 0) return fail("generate before decode_begin");
    if (!out_tokens) return fail("null output");
    if (n_new <= 0) return fail("n_new=%d must be positive", n_new);
    if (h->kvLen + n_new - 1 > h->capKV)
        return fail("%d new tokens need %d cache positions, %d held", n_new,
                    h->kvLen + n_new - 1, h->capKV);
    HIP_TRY(hipSetDevice(h->device));
    const int B = h->kvB;
    const int start = h->kvLen;
    if (draws)
        HIP_TRY(hipMemcpyAsync(h->draws, draws, (size_t)n_new * B * sizeof(float),
                               hipMemcpyHostToDevice, h->stream));
    if (draws && run_sample(h, h->draws, temperature, top_k)) return -1;
    const bool persist = persist_usable(h);
    if (!persist && h->decode_path == CNGPT_DECODE_PERSISTENT) return persist_refused(h);
    // i: tokens of this call already in next_tok / the history (the first
    // comes from decode_begin or the previous step); a refused persistent
    // launch leaves i where it was and the step kernels take the rest
    int i = 1;
    if (persist && !draws) {
        // greedy: every step in one launch, the argmax fed back on the device
        if (n_new > 1) {
            const int rc = run_persist(h, n_new - 1);
            if (rc < 0) return -1;
            if (rc == 0) i = n_new;
        }
    } else if (persist && persist_sampling_supported(h->cfg.vocab_size, h->persist_G, top_k)) {
        // sampled inside the launch: step i draws token i with draws[i];
        // a step whose candidates overflow ends the launch, and its token
        // is drawn here before the next launch continues
        while (i < n_new) {
            int done = 0;
            const int rc =
                run_persist(h, n_new - i, temperature, top_k, h->draws + (size_t)i * B, &done);
            if (rc < 0) return -1;
            if (rc > 0) break;
            i += done;
            int next = 0;
            HIP_TRY(hipMemcpyAsync(&next, h->next_tok, sizeof(int), hipMemcpyDeviceToHost,
                                   h->stream));
            HIP_TRY(hipStreamSynchronize(h->stream));
            if (next < 0 && run_sample(h, h->draws + (size_t)(i - 1) * B, temperature, top_k))
                return -1;
        }
    } else if (persist) {
        // sampled: one persistent step per launch, then the sampler replaces
        // the step's argmax by the sampled token the next launch embeds
        for (; i < n_new; i++) {
            const int rc = run_persist(h, 1);
            if (rc < 0) return -1;
            if (rc > 0) break;
            if (run_sample(h, h->draws + (size_t)i * B, temperature, top_k)) return -1;
        }
    }
    for (; i < n_new; i++) {
        if (run_decode_step(h)) return -1;
        if (draws && run_sample(h, h->draws + (size_t)i * B, temperature, top_k)) return -1;
    }
    // tokens fed at positions start.. are the first n_new - 1; the last is in next_tok
    if (n_new > 1)
        HIP_TRY(hipMemcpy2DAsync(out_tokens, (size_t)n_new * sizeof(int), h->hist + start,
                                 (size_t)h->capKV * sizeof(int), (size_t)(n_new - 1) * sizeof(int),
                                 B, hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipMemcpy2DAsync(out_tokens + (n_new - 1), (size_t)n_new * sizeof(int), h->next_tok,
                             sizeof(int), sizeof(int), B, hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return check_dev_err(h);
}

int cngpt_hip_argmax(cngpt_hip_ctx* h, int* out_tokens) {
    if (need_params(h)) return -1;
    if (!out_tokens) return fail("null output");
    if (!h->logits || h->curB == 0) return fail("no logits yet");
    if (h->curMode != CNGPT_LAST) return fail("argmax needs last-position logits");
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(launch_argmax_rows(h->logits, h->curB, h->cfg.vocab_size, h->next_tok, nullptr,
                               h->stream));
    HIP_TRY(hipMemcpyAsync(out_tokens, h->next_tok, (size_t)h->curB * sizeof(int),
                           hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return 0;
}

int cngpt_hip_sample(cngpt_hip_ctx* h, float temperature, int top_k, const float* draws,
                     int* out_tokens) {
    if (need_params(h)) return -1;
    if (!out_tokens || !draws) return fail("null argument");
    if (!h->logits || h->curB == 0) return fail("no logits yet");
    if (h->curMode != CNGPT_LAST) return fail("sample needs last-position logits");
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipMemcpyAsync(h->draws, draws, (size_t)h->curB * sizeof(float),
                           hipMemcpyHostToDevice, h->stream));
    HIP_TRY(launch_sample(h->logits, h->curB, h->cfg.vocab_size, temperature, top_k, h->draws,
                          h->prob, h->ldp, h->samp_part, h->next_tok, h->stream));
    HIP_TRY(hipMemcpyAsync(out_tokens, h->next_tok, (size_t)h->curB * sizeof(int),
                           hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return 0;
}

int cngpt_hip_decode_length(cngpt_hip_ctx* h) { return h ? h->kvLen : 0; }

void* cngpt_hip_host_alloc(size_t bytes) {
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        fail("pinned host allocation of %zu bytes failed", bytes);
        return nullptr;
    }
    return p;
}

int cngpt_hip_set_decode_path(cngpt_hip_ctx* h, int path) {
    if (!h) return fail("null handle");
    if (path != CNGPT_DECODE_AUTO && path != CNGPT_DECODE_KERNELS &&
        path != CNGPT_DECODE_PERSISTENT)
        return fail("bad decode path %d", path);
    h->decode_path = path;
    return 0;
}

int cngpt_hip_decode_path(cngpt_hip_ctx* h) { return h ? h->last_path : -1; }

void cngpt_hip_host_free(void* p) {
    if (p) (void)hipHostFree(p);
}

int cngpt_hip_profile_enable(cngpt_hip_ctx* h, int on) {
    if (!h) return fail("null handle");
    h->prof = on != 0;
    return 0;
}

int cngpt_hip_profile_reset(cngpt_hip_ctx* h) {
    if (!h) return fail("null handle");
    HIP_TRY(hipStreamSynchronize(h->stream));
    h->recs.clear();
    h->pool_used = 0;
    return 0;
}

int cngpt_hip_profile_read(cngpt_hip_ctx* h, int cls, double* ms, long* launches, double* flops,
                           double* bytes) {
    if (!h) return fail("null handle");
    if (cls < 0 || cls >= CNGPT_K_COUNT) return fail("bad kernel class %d", cls);
    HIP_TRY(hipStreamSynchronize(h->stream));
    double t = 0, f = 0, b = 0;
    long n = 0;
    for (const ProfRec& r : h->recs) {
        if (r.cls != cls) continue;
        float e = 0;
        HIP_TRY(hipEventElapsedTime(&e, r.a, r.b));
        t += e; f += r.flops; b += r.bytes; n++;
    }
    if (ms) *ms = t;
    if (launches) *launches = n;
    if (flops) *flops = f;
    if (bytes) *bytes = b;
    return 0;
}

}  // extern "C"
