// kat.cpp - test-only C entry points into the product's kernels, for the
// reference's forward known answers (tests/check_ops.c:69-182) and the
// error bounds of the device GELU and softmax exponentials.
//
// Each entry point copies host arrays to the device, enqueues the same
// launcher the forward pass uses (libcngpt_hip.so's launch_gemm,
// launch_dgemv, launch_layernorm, launch_attention_causal,
// launch_attention_dec + launch_attention_merge), and copies the result
// back. Allocations here are the test's own; nothing is added to the
// product's interface.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../cngpt_amd/csrc/common.h"
#include "../../cngpt_amd/csrc/kernels.h"

namespace {

char g_err[512];

int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return -1;
}

#define TRY(expr)                                                                          \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess) return fail("%s: %s", #expr, hipGetErrorString(e_));         \
    } while (0)

// Device copies of host arrays, freed on scope exit.
struct Dev {
    std::vector<void*> ptrs;
    ~Dev() {
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <class T>
    T* put(const T* host, size_t n) {
        void* p = nullptr;
        if (hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)) != hipSuccess) return nullptr;
        ptrs.push_back(p);
        if (host && hipMemcpy(p, host, n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
            return nullptr;
        if (!host && hipMemset(p, 0, std::max<size_t>(n, 1) * sizeof(T)) != hipSuccess) return nullptr;
        return (T*)p;
    }
};

}  // namespace

extern "C" {

const char* kat_error(void) { return g_err; }

// Y[M,N] = epi(X[M,K] . W[N,K]^T) with epi 0 store, 1 +bias, 2 +bias then
// GELU, 3 Y += . + bias (Y is read). path 0: launch_gemm (M <= 64 the
// weight-streaming k_stream, split over K when its column tiles are few;
// larger M the 128 x 128 MFMA tiles); path 1: launch_dgemv (M <= 8, the
// decode products); path 2: launch_gemm with the packed copy of W
// (launch_pack_w), which k_stream reads instead of W.
int kat_gemm(const float* X, const float* W, const float* bias, float* Y, int M, int N, int K,
             int epi, int path) {
    if (M <= 0 || N <= 0 || K <= 0 || epi < 0 || epi > 3) return fail("bad shape or epilogue");
    if (path == 1 && M > 8) return fail("the decode product takes M <= 8");
    Dev d;
    float* dx = d.put(X, (size_t)M * K);
    float* dw = d.put(W, (size_t)N * K);
    float* db = d.put(bias, bias ? (size_t)N : 0);
    float* dy = d.put(epi == EPI_RESID ? Y : nullptr, (size_t)M * N);
    if (path < 0 || path > 2) return fail("bad path");
    const bool pk = path == 2;
    float* part = path != 1 ? d.put<float>(nullptr, 1 << 24) : nullptr;
    float* dwp = pk ? d.put<float>(nullptr, packed_w_floats(N, K)) : nullptr;
    if (!dx || !dw || !db || !dy || (path != 1 && !part) || (pk && !dwp))
        return fail("device allocation failed");
    if (pk) TRY(launch_pack_w(dw, dwp, N, K, nullptr));
    if (path != 1) {
        GemmArgs a{};
        a.X = dx; a.W = dw; a.Wp = dwp; a.bias = db; a.Y = dy;
        a.M = M; a.N = N; a.K = K; a.ldy = N;
        a.epi = epi;
        a.part = part; a.part_cap = 1 << 24;  // the forward's 64 MB
        TRY(launch_gemm(a, nullptr));
    } else {
        DecGemvArgs a{};
        a.X = dx; a.ldx = K; a.W = dw; a.bias = db; a.Y = dy; a.ldy = N;
        a.M = M; a.N = N; a.K = K;
        a.epi = epi;
        TRY(launch_dgemv(a, nullptr));
    }
    TRY(hipDeviceSynchronize());
    TRY(hipMemcpy(Y, dy, (size_t)M * N * sizeof(float), hipMemcpyDeviceToHost));
    return 0;
}

// Y[M,N] += X . W^T + bias (launch_gemm), and lnout = LayerNorm(Y rows)
// with gains lnw and biases lnb, formed by the split sum when K is split,
// else by a LayerNorm launch after the product; returns the splits (> 1:
// the sum formed the LayerNorm), -1 on failure.
int kat_gemm_ln(const float* X, const float* W, const float* bias, float* Y, const float* lnw,
                const float* lnb, float* lnout, int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return fail("bad shape");
    Dev d;
    float* dx = d.put(X, (size_t)M * K);
    float* dw = d.put(W, (size_t)N * K);
    float* db = d.put(bias, (size_t)N);
    float* dy = d.put(Y, (size_t)M * N);
    float* dlw = d.put(lnw, (size_t)N);
    float* dlb = d.put(lnb, (size_t)N);
    float* dln = d.put<float>(nullptr, (size_t)M * N);
    float* part = d.put<float>(nullptr, 1 << 24);
    if (!dx || !dw || !db || !dy || !dlw || !dlb || !dln || !part)
        return fail("device allocation failed");
    GemmArgs a{};
    a.X = dx; a.W = dw; a.bias = db; a.Y = dy;
    a.M = M; a.N = N; a.K = K; a.ldy = N;
    a.epi = EPI_RESID;
    a.part = part; a.part_cap = 1 << 24;
    a.ln_w = dlw; a.ln_b = dlb; a.ln_out = dln;
    const int splits = launch_gemm_splits(a);
    TRY(launch_gemm(a, nullptr));
    TRY(hipDeviceSynchronize());
    TRY(hipMemcpy(Y, dy, (size_t)M * N * sizeof(float), hipMemcpyDeviceToHost));
    TRY(hipMemcpy(lnout, dln, (size_t)M * N * sizeof(float), hipMemcpyDeviceToHost));
    return splits;
}

// out[rows, C] = LayerNorm(x) with gains w and biases b.
int kat_layernorm(const float* x, const float* w, const float* b, float* out, int rows, int C) {
    if (rows <= 0 || C <= 0 || (C & 3)) return fail("bad shape");
    Dev d;
    float* dx = d.put(x, (size_t)rows * C);
    float* dw = d.put(w, (size_t)C);
    float* db = d.put(b, (size_t)C);
    float* dout = d.put<float>(nullptr, (size_t)rows * C);
    if (!dx || !dw || !db || !dout) return fail("device allocation failed");
    TRY(launch_layernorm(dx, C, dw, db, dout, C, rows, C, nullptr));
    TRY(hipDeviceSynchronize());
    TRY(hipMemcpy(out, dout, (size_t)rows * C * sizeof(float), hipMemcpyDeviceToHost));
    return 0;
}

// Causal attention over qkv [B, T, 3C] (rows [q | k | v], heads of C/H):
// out [B, T, C], the forward's fused kernel.
int kat_attention(const float* qkv, float* out, int B, int T, int C, int H) {
    if (B <= 0 || T <= 0 || H <= 0 || C % H) return fail("bad shape");
    Dev d;
    float* dq = d.put(qkv, (size_t)B * T * 3 * C);
    float* dout = d.put<float>(nullptr, (size_t)B * T * C);
    if (!dq || !dout) return fail("device allocation failed");
    TRY(launch_attention_causal(dq, T, dout, B, T, C, H, nullptr));
    TRY(hipDeviceSynchronize());
    TRY(hipMemcpy(out, dout, (size_t)B * T * C * sizeof(float), hipMemcpyDeviceToHost));
    return 0;
}

// Attention of the final query row of each sequence only (the last layer of
// a last-position forward and every decode step): keys split over
// workgroups, then the splits merged. out [B, C].
int kat_attention_row(const float* qkv, float* out, int B, int T, int C, int H) {
    if (B <= 0 || T <= 0 || H <= 0 || C % H) return fail("bad shape");
    const int hs = C / H;
    const int kps = attn_dec_keys_per_split(hs);
    const int splits = (T + kps - 1) / kps;
    Dev d;
    float* dq = d.put(qkv, (size_t)B * T * 3 * C);
    float* part = d.put<float>(nullptr, (size_t)B * H * splits * (hs + 4));
    float* dout = d.put<float>(nullptr, (size_t)B * C);
    if (!dq || !part || !dout) return fail("device allocation failed");
    AttnDecArgs a{};
    a.qkv = dq; a.seq_stride = T; a.C = C; a.H = H;
    a.q_pos = T - 1; a.pos_dev = nullptr;
    a.scale = 1.0f / sqrtf((float)hs);
    a.part = part; a.max_splits = splits;
    TRY(launch_attention_dec(a, B, T, nullptr));
    MergeArgs g{};
    g.part = part; g.stride = splits; g.H = H; g.hs = hs; g.kps = kps;
    g.q_pos = T - 1; g.pos_dev = nullptr;
    TRY(launch_attention_merge(g, B, dout, C, nullptr));
    TRY(hipDeviceSynchronize());
    TRY(hipMemcpy(out, dout, (size_t)B * C * sizeof(float), hipMemcpyDeviceToHost));
    return 0;
}

}  // extern "C"
