// loss.hip - cross-entropy of the logits held in HBM (reference ops.c:499-574,
// as gpt_forward calls it after the lm_head, model.c:617-623).
//
// HBM-bound: every logit is read once. One workgroup per row of V logits;
// each lane keeps a running maximum m and the sum s of exp(x - m) over the
// logits it reads (s is rescaled by exp(m_old - m_new) when m grows, once
// per batch of 8 logits), and the lanes' (m, s) pairs are merged in the
// wavefront (DPP) and then across the wavefronts. This yields the
// reference's row max and log of the sum of exp(logit - max) without a
// second pass over the row. exp(y) is taken as 2^(y log2 e) on the
// hardware's exp2.
//
// A row of V floats starts at float offset row * V, which is 16-byte
// aligned only every fourth row when V is odd: the up to 3 logits before the
// first aligned address and the up to 3 after the last full float4 are
// taken one by one.
#include "common.h"
#include "kernels.h"

namespace {

// 1024 lanes per row and two float4 loads in flight per lane, read with
// the nontemporal hint (the logits are not reused): 0.455 ms for 16384 rows
// of 50257 logits (7.2 TB/s), against 0.536 ms for 256 lanes x 4 plain
// loads.
constexpr int CE_THREADS = 1024;
constexpr int CE_WAVES = CE_THREADS / 64;
constexpr int CE_UNROLL = 2;
constexpr float LOG2E = 1.4426950408889634f;

typedef __attribute__((address_space(1))) const f32x4 gf32x4;

__device__ __forceinline__ float exp_of(float y) { return __builtin_amdgcn_exp2f(y * LOG2E); }
__device__ __forceinline__ f32x4 ld_stream(const gf32x4* p) { return __builtin_nontemporal_load(p); }

// (m, s) <- (m, s) merged with one logit x.
__device__ __forceinline__ void add1(float& m, float& s, float x) {
    const float nm = fmaxf(m, x);
    s = s * exp_of(m - nm) + exp_of(x - nm);  // m = -inf: exp(-inf) = 0
    m = nm;
}

// (m, s) <- (m, s) merged with U float4 of logits (lanes with no valid
// logit in the batch pass bm = -inf and keep their pair).
template <int U>
__device__ __forceinline__ void add_batch(float& m, float& s, const f32x4 (&v)[U]) {
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < U; j++) bm = fmaxf(fmaxf(bm, fmaxf(v[j].x, v[j].y)), fmaxf(v[j].z, v[j].w));
    if (bm == -INFINITY) return;
    const float nm = fmaxf(m, bm);
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < U; j++)
        t += (exp_of(v[j].x - nm) + exp_of(v[j].y - nm)) + (exp_of(v[j].z - nm) + exp_of(v[j].w - nm));
    s = s * exp_of(m - nm) + t;
    m = nm;
}

// Weight of a pair with maximum m inside a merged maximum M (0 for a pair
// that saw no logit).
__device__ __forceinline__ float rescale(float m, float M) {
    return m == -INFINITY ? 0.f : exp_of(m - M);
}

// One workgroup per row. Writes the row term log(sum) - (x[target] - max)
// to row_loss[row]; with probs, overwrites the row with
// exp(x - max) * (1 / sum) (ops.c:557-566); with dl, leaves the logits and
// writes the gradient of the mean loss instead, dl[row][v] = gscale *
// (p_v - [v == target]) (cross_entropy_bwd, ops.c:576-589, with gscale = 1 /
// rows), zero for V <= v < ldd (rows of ldd floats, 16-byte aligned).
__global__ void __launch_bounds__(CE_THREADS) k_ce_rows(float* __restrict__ logits, int V,
                                                         const int* __restrict__ targets,
                                                         float* __restrict__ row_loss, int probs,
                                                         int* __restrict__ err,
                                                         float* __restrict__ dl, long ldd,
                                                         float gscale) {
    __shared__ float sm[CE_WAVES], ss[CE_WAVES];
    __shared__ float s_max, s_inv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const long row = blockIdx.x;
    const long off = row * V;
    float* lg = logits + off;
    const int head = min((int)((4 - (off & 3)) & 3), V);
    const int n4 = (V - head) >> 2;
    const int tail0 = head + 4 * n4;
    const gf32x4* a4 = (const gf32x4*)(lg + head);

    // The target's logit and the unaligned head and tail logits are loaded
    // by every lane at clamped addresses before the row streams in, so no
    // load waits inside a branch.
    int tg = targets[row];
    const bool bad = tg < 0 || tg >= V;
    tg = min(max(tg, 0), V - 1);
    const float xt = lg[tg];
    const float xh = lg[min(tid, V - 1)];
    const float xl = lg[min(tail0 + min(tid, 3), V - 1)];
    if (bad && tid == 0) atomicOr(err, 4);

    float m = -INFINITY, s = 0.f;
    constexpr int STEP = CE_THREADS * CE_UNROLL;
    const int full = n4 / STEP;
    int i = tid;
    for (int it = 0; it < full; it++, i += STEP) {
        f32x4 v[CE_UNROLL];
#pragma unroll
        for (int j = 0; j < CE_UNROLL; j++) v[j] = ld_stream(a4 + i + j * CE_THREADS);
        add_batch(m, s, v);
    }
    if (n4 > 0) {
        f32x4 v[CE_UNROLL];
#pragma unroll
        for (int j = 0; j < CE_UNROLL; j++) {
            const int k = i + j * CE_THREADS;
            v[j] = ld_stream(a4 + min(k, n4 - 1));
            if (k >= n4) v[j] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        }
        add_batch(m, s, v);
    }
    if (tid < head) add1(m, s, xh);
    if (tid < V - tail0) add1(m, s, xl);

    // merge the pairs: wavefront, then the wavefronts of the workgroup
    {
        const float M = wave_max_dpp(m);
        const float S = wave_sum_dpp(s * rescale(m, M));
        if (lane == 0) { sm[wave] = M; ss[wave] = S; }
    }
    __syncthreads();
    if (tid == 0) {
        float M = sm[0];
#pragma unroll
        for (int w = 1; w < CE_WAVES; w++) M = fmaxf(M, sm[w]);
        float S = 0.f;
#pragma unroll
        for (int w = 0; w < CE_WAVES; w++) S += ss[w] * rescale(sm[w], M);
        const float log_sum = logf(S);
        row_loss[row] = -((xt - M) - log_sum);  // ops.c:567-568
        s_max = M;
        s_inv = 1.0f / S;
    }
    if (!probs && !dl) return;
    __syncthreads();
    const float M = s_max, inv = s_inv;
    if (dl) {
        f32x4* d4 = (f32x4*)(dl + row * ldd);
        for (int k = tid; k < (int)(ldd >> 2); k += CE_THREADS) {
            f32x4 g;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int v = 4 * k + e;
                const float x = lg[min(v, V - 1)];
                g[e] = v < V ? gscale * (exp_of(x - M) * inv - (v == tg ? 1.0f : 0.0f)) : 0.f;
            }
            __builtin_nontemporal_store(g, d4 + k);
        }
        return;
    }
    if (tid < head) lg[tid] = exp_of(lg[tid] - M) * inv;
    if (tid < V - tail0) lg[tail0 + tid] = exp_of(lg[tail0 + tid] - M) * inv;
    f32x4* w4 = (f32x4*)(lg + head);
    for (int k = tid; k < n4; k += CE_THREADS) {
        const f32x4 x = ld_stream(a4 + k);
        __builtin_nontemporal_store(
            f32x4{exp_of(x.x - M), exp_of(x.y - M), exp_of(x.z - M), exp_of(x.w - M)} * inv, w4 + k);
    }
}

// loss[0] = mean of row_loss[0 .. rows), summed in double in a fixed order
// (the result does not depend on timing).
constexpr int MEAN_THREADS = 1024;
__global__ void __launch_bounds__(MEAN_THREADS) k_ce_mean(const float* __restrict__ row_loss,
                                                           long rows, float* __restrict__ loss) {
    __shared__ double part[MEAN_THREADS / 64];
    const int tid = threadIdx.x;
    double acc = 0.0;
    for (long r = tid; r < rows; r += MEAN_THREADS) acc += (double)row_loss[r];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if ((tid & 63) == 0) part[tid >> 6] = acc;
    __syncthreads();
    if (tid == 0) {
        double t = 0.0;
        for (int w = 0; w < MEAN_THREADS / 64; w++) t += part[w];
        loss[0] = (float)(t / (double)rows);
    }
}

}  // namespace

hipError_t launch_cross_entropy(float* logits, long rows, int V, const int* targets,
                                float* row_loss, float* loss, int probs, int* err, hipStream_t s,
                                float* dl, long ldd) {
    if (rows <= 0 || V <= 0) return hipErrorInvalidValue;
    if (rows > 0x7fffffffL) return hipErrorInvalidValue;
    if (dl && (probs || ldd < V || (ldd & 3))) return hipErrorInvalidValue;
    k_ce_rows<<<(unsigned)rows, CE_THREADS, 0, s>>>(logits, V, targets, row_loss, probs, err, dl,
                                                    ldd, 1.0f / (float)rows);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_ce_mean<<<1, MEAN_THREADS, 0, s>>>(row_loss, rows, loss);
    return hipGetLastError();
}
