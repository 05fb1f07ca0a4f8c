// kernels.h - host-side launchers of the gfx950 kernels (all enqueue on the
// given stream and return the launch status; none synchronizes).
#pragma once
#include <hip/hip_runtime.h>

// rowops.hip
hipError_t launch_embed(const int* tok, const float* wte, const float* wpe, float* x, long rows,
                        int T, int C, int V, int pos0, const int* pos_dev, int* err,
                        hipStream_t s);
hipError_t launch_layernorm(const float* x, long in_stride, const float* w, const float* b,
                            float* out, long out_stride, int rows, int C, hipStream_t s);
hipError_t launch_gather_rows(const float* src, long src_stride, float* dst, int rows, int C,
                              hipStream_t s);
hipError_t launch_argmax(const float* logits, int rows, int V, int* out, hipStream_t s);

// gemm.hip: Y[M,N] = epi(X[M,K] . W[N,K]^T). X rows are K floats apart.
// Output row m goes to Y + ((m / seg) * seg_stride + m % seg) * ldy, which
// lets the QKV product write straight into a per-sequence cache of
// seg_stride rows (seg = 0 means plain row-major, row stride ldy).
struct GemmArgs {
    const float* X;
    const float* W;
    const float* bias;
    float* Y;
    int M, N, K;
    long ldy;
    int seg;
    long seg_stride;
    int row_off;               // added to every output row index
    const int* row_off_dev;    // if set, *row_off_dev is added too (decode position)
    int epi;                   // EpiMode
};
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s);
// Skinny products (M <= 8 rows, decode and the last-position pass): one
// wavefront per weight row, weights streamed once.
hipError_t launch_gemv(const GemmArgs& a, hipStream_t s);

// attention.hip
// qkv rows hold [q | k | v] (3C floats); sequence b's row t sits at
// qkv + (b * seq_stride + t) * 3C. out row (b*T + t) gets the merged heads.
hipError_t launch_attention_causal(const float* qkv, long seq_stride, float* out, int B, int T,
                                   int C, int H, hipStream_t s);
// One query row per (sequence, head): query at position q_pos (or *pos_dev)
// against keys 0..q_pos. out row b gets the merged heads. max_keys bounds
// q_pos + 1 (it sizes the score buffer in LDS).
hipError_t launch_attention_row(const float* qkv, long seq_stride, float* out, int B, int q_pos,
                                const int* pos_dev, int max_keys, int C, int H, hipStream_t s);
