// sample.hip - top-k sampling of the next token from logits rows, with the
// arithmetic of the reference's sample_top_k (src/model.c:927-989):
// scaled = logit / temp (temp <= 0 -> 1), softmax, keep the probabilities
// >= the top_k-th largest (ties kept), renormalise by their sum, and take
// the first index whose running sum exceeds the uniform draw (V - 1 if none
// does).
//
// Two paths. k_topk_part + k_topk_pick (top_k <= TK_MAX, V <= TK_G * 1024):
// a row is split into TK_G chunks, one workgroup each, which keep their
// chunk's max and its top_k largest scaled values; one workgroup per row
// then takes the max, the softmax denominator over the row, the top_k-th
// largest value among the chunks' lists, and the survivors, in index order.
// k_sample (any top_k): one workgroup per row runs every pass itself.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace {

constexpr int ST = 1024;      // threads of the sampling workgroup
constexpr int SLIST = 2048;   // survivors of the top-k cut kept in index order

// Block-wide reductions over ST threads (fixed order: deterministic).
__device__ float block_max(float v, float* sh) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float r = sh[0];
    for (int i = 1; i < ST / 64; i++) r = fmaxf(r, sh[i]);
    return r;
}
__device__ float block_sum(float v, float* sh) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float r = 0.f;
    for (int i = 0; i < ST / 64; i++) r += sh[i];
    return r;
}
// Exclusive prefix over the threads in thread order; *total = the sum.
template <typename TV>
__device__ TV block_excl_scan(TV v, TV* sh, TV* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    TV x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const TV y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    __syncthreads();
    if (lane == 63) sh[w] = x;
    __syncthreads();
    TV before = 0, all = 0;
    for (int i = 0; i < ST / 64; i++) {
        if (i < w) before += sh[i];
        all += sh[i];
    }
    *total = all;
    return before + (x - v);
}
// hist[bin] += 1 for every lane with ok set; lanes of a wavefront that share
// a bin are counted with one LDS atomic (the high bits of nearby
// probabilities mostly coincide).
__device__ __forceinline__ void hist_add(int* hist, unsigned bin, bool ok) {
    unsigned long long act = __ballot(ok);
    while (act) {
        const int leader = __ffsll((long long)act) - 1;
        const unsigned lb = __shfl(bin, leader, 64);
        const unsigned long long peers = __ballot(ok && bin == lb) & act;
        if ((int)(threadIdx.x & 63) == leader) atomicAdd(&hist[lb], __popcll(peers));
        act &= ~peers;
    }
}

// One token per row from logits [rows, V], with the arithmetic of the
// reference's sample_top_k (src/model.c:927-989): scaled = logit / temp
// (temp <= 0 -> 1), softmax, keep the values >= the top_k-th largest
// (ties kept), renormalise, then the first index whose running sum exceeds
// the uniform draw r[row]; V - 1 if none does. prob [rows, ldp] is scratch
// (ldp a multiple of 4). Thread i owns the float4 groups [i*ch4, (i+1)*ch4),
// so thread order is index order. When at most SLIST values survive the
// cut, the renormalising sum and the running sum are taken sequentially in
// index order, as the reference does; otherwise (top_k off, or a huge tie
// at the threshold) each thread sums its range and the ranges are prefixed,
// which can differ from a sequential sum in the last bits, so the token can
// differ only when r lies within rounding of a boundary.
__global__ void __launch_bounds__(ST) k_sample(const float* __restrict__ logits, int V, float temp,
                                               int top_k, const float* __restrict__ r_draw,
                                               float* __restrict__ prob, long ldp,
                                               int* __restrict__ out) {
    __shared__ float shf[ST / 64];
    __shared__ int shi[ST / 64];
    __shared__ int hist[256];
    __shared__ int chosen, kk_left;
    __shared__ float lv[SLIST];
    __shared__ int li[SLIST];
    __shared__ int tok_sh;

    const int row = blockIdx.x, tid = threadIdx.x;
    const float* lg = logits + (long)row * V;
    float* p = prob + (long)row * ldp;
    f32x4* p4 = (f32x4*)p;
    const int V4 = (V + 3) / 4;
    const int ch4 = (V4 + ST - 1) / ST;
    const int g0 = min(tid * ch4, V4), g1 = min(g0 + ch4, V4);
    const float tdiv = temp > 0.0f ? temp : 1.0f;
    const int NP = V4 * 4;  // padded length of the scratch row
    constexpr int U = 8;    // loads in flight per thread in the strided passes

    // scaled values (coalesced reads of the logits) and their max
    float mx = -INFINITY;
    for (int i0 = 0; i0 < NP; i0 += ST * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * ST + tid;
            const float x = lg[min(i, V - 1)] / tdiv;
            v[u] = i < V ? x : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * ST + tid;
            if (i < NP) p[i] = v[u];
            mx = fmaxf(mx, v[u]);
        }
    }
    mx = block_max(mx, shf);
    float s = 0.f;
    for (int i0 = 0; i0 < NP; i0 += ST * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * ST + tid;
            const float x = p[min(i, NP - 1)];
            v[u] = i < V ? expf(x - mx) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * ST + tid;
            if (i < NP) p[i] = v[u];
            s += v[u];
        }
    }
    const float sum = block_sum(s, shf);
    for (int i0 = 0; i0 < NP; i0 += ST * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = p[min(i0 + u * ST + tid, NP - 1)];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * ST + tid;
            if (i < NP) p[i] = i < V ? v[u] / sum : 0.f;
        }
    }
    __syncthreads();

    // k-th largest probability (with multiplicity) by MSB-first radix
    // select on the bit patterns (non-negative floats order as integers).
    const bool cut = top_k > 0 && top_k < V;
    float thr = 0.f;
    if (cut) {
        unsigned prefix = 0, mask = 0;
        if (tid == 0) kk_left = top_k;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = tid; i < 256; i += ST) hist[i] = 0;
            __syncthreads();
            for (int i0 = 0; i0 < NP; i0 += ST * U) {
                unsigned uv[U];
#pragma unroll
                for (int u = 0; u < U; u++) uv[u] = __float_as_uint(p[min(i0 + u * ST + tid, NP - 1)]);
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const int i = i0 + u * ST + tid;
                    hist_add(hist, (uv[u] >> shift) & 255u, i < V && (uv[u] & mask) == prefix);
                }
            }
            __syncthreads();
            if (tid == 0) {
                int cum = 0, kk = kk_left, d = 255;
                for (; d > 0; d--) {
                    if (cum + hist[d] >= kk) break;
                    cum += hist[d];
                }
                chosen = d;
                kk_left = kk - cum;
            }
            __syncthreads();
            prefix |= (unsigned)chosen << shift;
            mask |= 255u << shift;
        }
        thr = __uint_as_float(prefix);
    }

    // Survivors (all values when there is no cut) in index order. Thread
    // ranges: float4 groups g0 + j, j < ch4 (a uniform trip count).
    auto keep = [&](int i, float v) { return i < V && (!cut || v >= thr); };
    int cnt = 0;
#pragma unroll 4
    for (int j = 0; j < ch4; j++) {
        const int g = g0 + j;
        const f32x4 v = ld4_or0(p4 + min(g, V4 - 1), g < g1);
        if (g < g1)
            cnt += keep(4 * g, v.x) + keep(4 * g + 1, v.y) + keep(4 * g + 2, v.z) +
                   keep(4 * g + 3, v.w);
    }
    int total;
    const int base = block_excl_scan<int>(cnt, shi, &total);
    const float r = r_draw[row];
    if (cut && total <= SLIST) {
        int k = base;
        for (int j = 0; j < ch4; j++) {
            const int g = g0 + j;
            const f32x4 v = ld4_or0(p4 + min(g, V4 - 1), g < g1);
            const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (g < g1 && keep(4 * g + e, vv[e])) {
                    lv[k] = vv[e];
                    li[k] = 4 * g + e;
                    k++;
                }
        }
        __syncthreads();
        if (tid == 0) {
            float ns = 0.f;
            for (int q = 0; q < total; q++) ns += lv[q];
            int tok = V - 1;
            float cdf = 0.f;
            for (int q = 0; q < total; q++) {
                cdf += ns > 0.0f ? lv[q] / ns : lv[q];
                if (r < cdf) { tok = li[q]; break; }
            }
            out[row] = tok;
        }
        return;
    }
    // Blocked form: zero the cut values, renormalise, prefix by ranges
    // (scratch padding past V holds 0).
    float ps = 0.f;
    for (int j = 0; j < ch4; j++) {
        const int g = g0 + j;
        f32x4 v = ld4_or0(p4 + min(g, V4 - 1), g < g1);
        if (cut) {
            v.x = v.x < thr ? 0.f : v.x;
            v.y = v.y < thr ? 0.f : v.y;
            v.z = v.z < thr ? 0.f : v.z;
            v.w = v.w < thr ? 0.f : v.w;
            if (g < g1) p4[g] = v;
        }
        ps += ((v.x + v.y) + v.z) + v.w;
    }
    if (cut) {
        const float ns = block_sum(ps, shf);
        if (ns > 0.0f) {
            ps = 0.f;
            for (int j = 0; j < ch4; j++) {
                const int g = g0 + j;
                f32x4 v = ld4_or0(p4 + min(g, V4 - 1), g < g1);
                v.x /= ns; v.y /= ns; v.z /= ns; v.w /= ns;
                if (g < g1) p4[g] = v;
                ps += ((v.x + v.y) + v.z) + v.w;
            }
        }
    }
    float all;
    float cdf = block_excl_scan<float>(ps, shf, &all);
    if (tid == 0) tok_sh = V - 1;
    __syncthreads();
    // Every thread scans its own range from its prefix; the smallest index
    // whose running sum exceeds r wins (robust to rounding gaps between
    // neighbouring ranges). Zero-probability values are never chosen.
    for (int i = g0 * 4; i < g1 * 4 && i < V; i++) {
        const float v = p[i];
        cdf += v;
        if (v > 0.0f && r < cdf) { atomicMin(&tok_sh, i); break; }
    }
    __syncthreads();
    if (tid == 0) out[row] = tok_sh;
}

// ---------------------------------------------------------------- split path

constexpr int TK_MAX = 64;    // largest top_k of the split path
constexpr int TK_G = 64;      // most chunks per row
constexpr int TP = 256;       // threads of a chunk workgroup (4 values each)
constexpr int TQ = 1024;      // threads of the pick workgroup

// Per-row partials (TOPK_PART_WORDS words per row): chunk maxima m_g, sums
// of expf(x - m_g) over the chunk, cut values (the top_k-th largest scaled
// value of the chunk), list lengths, then the lists (scaled value, index),
// TK_MAX entries per chunk.
struct TkPart {
    float* mx;
    float* sm;
    float* kth;
    int* cnt;
    float* lx;
    int* li;
};
static_assert(TOPK_PART_WORDS == 4 * TK_G + 2 * TK_G * TK_MAX, "partials layout");
__device__ __forceinline__ TkPart tk_part(float* row_part) {
    TkPart p;
    p.mx = row_part;
    p.sm = p.mx + TK_G;
    p.kth = p.sm + TK_G;
    p.cnt = (int*)(p.kth + TK_G);
    p.lx = (float*)(p.cnt + TK_G);
    p.li = (int*)(p.lx + TK_G * TK_MAX);
    return p;
}

// Unsigned keys in the order of the floats (no NaN).
__device__ __forceinline__ unsigned okey(float f) {
    const unsigned u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float okey_inv(unsigned k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// The kk-th largest key (with multiplicity, 1 <= kk <= number of ok keys)
// over the NV keys of each of the NT threads: MSB-first radix select, one
// byte per pass, counts in an LDS histogram (plain LDS atomics: the lanes
// that hit one bin are serialised by the hardware, cheaper than a software
// loop over the distinct bins of a wavefront); wavefront 0 finds the bin.
template <int NT, int NV>
__device__ unsigned wg_kth_key(const unsigned (&key)[NV], const bool (&ok)[NV], int kk,
                               int* hist, int* sh) {
    unsigned prefix = 0, mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += NT) hist[i] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NV; j++)
            if (ok[j] && (key[j] & mask) == prefix) atomicAdd(&hist[(key[j] >> shift) & 255u], 1);
        __syncthreads();
        if (threadIdx.x < 64) {
            // lane l holds bins 255-4l .. 252-4l; counts from the top bin down
            const int l = threadIdx.x;
            int c[4], s = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) { c[e] = hist[255 - 4 * l - e]; s += c[e]; }
            int incl = s;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o, 64);
                if (l >= o) incl += y;
            }
            const int before = incl - s;
            if (before < kk && incl >= kk) {
                int cum = before, e = 0;
                for (; e < 3; e++) {
                    if (cum + c[e] >= kk) break;
                    cum += c[e];
                }
                sh[0] = 255 - 4 * l - e;
                sh[1] = kk - cum;
            }
        }
        __syncthreads();
        prefix |= (unsigned)sh[0] << shift;
        mask |= 255u << shift;
        kk = sh[1];
        __syncthreads();
    }
    return prefix;
}

// One workgroup per (chunk, row): chunk g of row r covers indices
// [g * ch, min((g + 1) * ch, V)), ch <= TP * 4. Leaves the chunk's max m_g,
// the sum of expf(x - m_g) over it, its top_k-th largest scaled value and
// the list of its top_k largest (all of them when the chunk is shorter;
// values equal to the cut fill the list in no particular order).
__global__ void __launch_bounds__(TP) k_topk_part(const float* __restrict__ logits, int V,
                                                  float temp, int top_k, int G, int ch,
                                                  float* __restrict__ part) {
    __shared__ int hist[256];
    __shared__ int sh[2];
    __shared__ float wmax[TP / 64], wsum[TP / 64];
    __shared__ int n_gt, n_eq;
    const int g = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const float* lg = logits + (long)row * V;
    const TkPart P = tk_part(part + (long)row * TOPK_PART_WORDS);
    const float tdiv = temp > 0.0f ? temp : 1.0f;
    const int i0 = g * ch, i1 = min(i0 + ch, V);
    float x[4];
    unsigned key[4];
    bool ok[4];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = i0 + tid + j * TP;
        ok[j] = i < i1;
        x[j] = lg[min(i, V - 1)] / tdiv;
        key[j] = okey(x[j]);
        if (ok[j]) m = fmaxf(m, x[j]);
    }
    m = wave_max(m);
    if ((tid & 63) == 0) wmax[tid >> 6] = m;
    if (tid == 0) { n_gt = 0; n_eq = 0; }
    const int kk = min(top_k, i1 - i0);  // >= 1: no chunk is empty
    const unsigned kth = wg_kth_key<TP, 4>(key, ok, kk, hist, sh);  // syncs: wmax is set
    float mg = wmax[0];
    for (int w = 1; w < TP / 64; w++) mg = fmaxf(mg, wmax[w]);
    float e = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (ok[j]) e += expf(x[j] - mg);
    e = wave_sum(e);
    if ((tid & 63) == 0) wsum[tid >> 6] = e;
    // list: every value above the cut, then values equal to it up to kk
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (ok[j] && key[j] > kth) {
            const int q = atomicAdd(&n_gt, 1);
            P.lx[g * TK_MAX + q] = x[j];
            P.li[g * TK_MAX + q] = i0 + tid + j * TP;
        }
    __syncthreads();
    const int ngt = n_gt;
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (ok[j] && key[j] == kth) {
            const int q = ngt + atomicAdd(&n_eq, 1);
            if (q < kk) {
                P.lx[g * TK_MAX + q] = x[j];
                P.li[g * TK_MAX + q] = i0 + tid + j * TP;
            }
        }
    __syncthreads();
    if (tid == 0) {
        float sg = 0.f;
        for (int w = 0; w < TP / 64; w++) sg += wsum[w];
        P.mx[g] = mg;
        P.sm[g] = sg;
        P.kth[g] = okey_inv(kth);
        P.cnt[g] = kk;
    }
}

// One workgroup per row: the token from the chunks' partials.
//   M = max over the chunk maxima; S = sum over the chunks of
//   sum_g * expf(m_g - M), the softmax denominator (in a fixed order; the
//   reference's sequential sum of expf(x - M) differs only in rounding);
//   c = the top_k-th largest value among the lists (= over the row: a chunk
//   holds at most top_k of the row's top_k). c >= L, the larger of the
//   largest cut of a full list (that chunk holds top_k values >= it) and,
//   with top_k <= G, the top_k-th largest chunk maximum (top_k chunks each
//   hold a value >= it), so c is selected
//   among the list values >= L only, by counting ranks when they fit one
//   per thread (the usual case: about top_k of them), else by radix select
//   over all list values. Threshold t = expf(c - M) / S. Survivors
//   p = expf(x - M) / S >= t come from the lists, except for a chunk whose
//   list is full and whose own cut still reaches t: values below its list
//   may round to p = t, so that chunk is scanned whole. Survivors are put in
//   index order; the renormalising sum and the running sum are then taken
//   sequentially, as the reference does. More than SLIST survivors (a tie
//   across the cut) take the blocked form of k_sample's last steps.
__global__ void __launch_bounds__(TQ) k_topk_pick(const float* __restrict__ logits, int V,
                                                  float temp, int top_k, int G, int ch,
                                                  const float* __restrict__ r_draw,
                                                  const float* __restrict__ part,
                                                  int* __restrict__ out) {
    __shared__ float shf[TQ / 64];
    __shared__ int hist[256];
    __shared__ int sh[2];
    __shared__ float s_M, s_S, s_L, s_c, s_ns;
    __shared__ unsigned long long s_rescan;
    __shared__ int n_sv, n_c, tok_sh;
    __shared__ float sv_p[SLIST];
    __shared__ int sv_i[SLIST];
    __shared__ float so_p[SLIST];
    __shared__ int so_i[SLIST];
    __shared__ unsigned cand[TQ];

    const int row = blockIdx.x, tid = threadIdx.x;
    const float* lg = logits + (long)row * V;
    const TkPart P = tk_part(const_cast<float*>(part) + (long)row * TOPK_PART_WORDS);
    const float tdiv = temp > 0.0f ? temp : 1.0f;

    // every list entry, loaded at once (entries past a list's length unused)
    constexpr int NC = TK_G * TK_MAX / TQ;
    unsigned key[NC];
    bool ok[NC];
    float cx[NC];
    int ci[NC];
#pragma unroll
    for (int j = 0; j < NC; j++) {
        const int e = tid + j * TQ, g = min(e / TK_MAX, G - 1);
        cx[j] = P.lx[e];
        ci[j] = P.li[e];
        ok[j] = e / TK_MAX < G && e - g * TK_MAX < P.cnt[g];
        key[j] = okey(ok[j] ? cx[j] : 0.f);
    }
    // wavefront 0: M, S and the lower bound L from the chunk partials
    float cut_g = -INFINITY, mg = -INFINITY;
    int cnt_g = 0;
    if (tid < 64) {
        const bool have = tid < G;
        mg = have ? P.mx[tid] : -INFINITY;
        const float sg = have ? P.sm[tid] : 0.f;
        cut_g = have ? P.kth[tid] : -INFINITY;
        cnt_g = have ? P.cnt[tid] : 0;
        const float M = wave_max(mg);
        const float S = wave_sum(have ? sg * expf(mg - M) : 0.f);
        float L = wave_max(cnt_g == top_k ? cut_g : -INFINITY);  // full lists only
        if (top_k <= G) {
            // the top_k-th largest chunk maximum: top_k chunks hold a value >= it
            int gt = 0, ge = 0;
            for (int u = 0; u < 64; u++) {
                const float o = __shfl(mg, u, 64);
                gt += o > mg;
                ge += o >= mg;
            }
            const bool is_k = have && gt < top_k && top_k <= ge;
            const unsigned long long b = __ballot(is_k);
            L = fmaxf(L, __shfl(mg, __ffsll((long long)b) - 1, 64));
        }
        if (tid == 0) { s_M = M; s_S = S; s_L = L; n_c = 0; n_sv = 0; }
    }
    __syncthreads();
    const float M = s_M, S = s_S, L = s_L;
    const unsigned kl = okey(L);
#pragma unroll
    for (int j = 0; j < NC; j++)
        if (ok[j] && key[j] >= kl) {
            const int q = atomicAdd(&n_c, 1);
            if (q < TQ) cand[q] = key[j];
        }
    __syncthreads();
    const int nc = n_c;
    if (nc <= TQ) {
        // c: the key with fewer than top_k keys above it and at least
        // top_k at or above it (equal keys give the same c)
        if (tid < nc) {
            const unsigned v = cand[tid];
            int gt = 0, ge = 0;
            for (int u = 0; u < nc; u++) {
                const unsigned w = cand[u];
                gt += w > v;
                ge += w >= v;
            }
            if (gt < top_k && top_k <= ge) s_c = okey_inv(v);
        }
    } else {
        const float c = okey_inv(wg_kth_key<TQ, NC>(key, ok, top_k, hist, sh));
        if (tid == 0) s_c = c;
    }
    __syncthreads();
    const float t = expf(s_c - M) / S;
    if (tid < 64) {
        const bool full = tid < G && cnt_g == top_k && expf(cut_g - M) / S >= t;
        const unsigned long long mask = __ballot(full);
        if (tid == 0) s_rescan = mask;
    }
    __syncthreads();
    const unsigned long long rescan = s_rescan;

    auto push = [&](float p, int i) {
        const int q = atomicAdd(&n_sv, 1);
        if (q < SLIST) { sv_p[q] = p; sv_i[q] = i; }
    };
#pragma unroll
    for (int j = 0; j < NC; j++) {
        const int g = (tid + j * TQ) / TK_MAX;
        if (ok[j] && !((rescan >> g) & 1ull)) {
            const float p = expf(cx[j] - M) / S;
            if (p >= t) push(p, ci[j]);
        }
    }
    for (unsigned long long rm = rescan; rm; rm &= rm - 1) {
        const int g = __ffsll((long long)rm) - 1;
        const int i0 = g * ch, i1 = min(i0 + ch, V);
        for (int i = i0 + tid; i < i1; i += TQ) {
            const float p = expf(lg[i] / tdiv - M) / S;
            if (p >= t) push(p, i);
        }
    }
    __syncthreads();
    const int n = n_sv;
    const float r = r_draw[row];
    if (n <= SLIST) {
        // index order by rank (indices are distinct)
        for (int q = tid; q < n; q += TQ) {
            const int iq = sv_i[q];
            int rank = 0;
            for (int u = 0; u < n; u++) rank += sv_i[u] < iq;
            so_p[rank] = sv_p[q];
            so_i[rank] = iq;
        }
        __syncthreads();
        if (tid == 0) {
            float ns = 0.f;
#pragma unroll 8
            for (int q = 0; q < n; q++) ns += so_p[q];
            s_ns = ns;
        }
        __syncthreads();
        const float ns = s_ns;
        for (int q = tid; q < n; q += TQ) so_p[q] = ns > 0.0f ? so_p[q] / ns : so_p[q];
        __syncthreads();
        if (tid == 0) {
            int tok = V - 1;
            float cdf = 0.f;
#pragma unroll 8
            for (int q = 0; q < n; q++) {
                cdf += so_p[q];
                if (r < cdf) { tok = so_i[q]; break; }
            }
            out[row] = tok;
        }
        return;
    }
    // Blocked form over the thread ranges [t * per, (t + 1) * per)
    // (probabilities recomputed).
    const int per = (V + TQ - 1) / TQ;
    const int r0 = min(tid * per, V), r1 = min(r0 + per, V);
    auto prob = [&](int i) {
        const float p = expf(lg[i] / tdiv - M) / S;
        return p < t ? 0.f : p;
    };
    float ps = 0.f;
    for (int i = r0; i < r1; i++) ps += prob(i);
    const float ns = block_sum(ps, shf);
    ps = 0.f;
    for (int i = r0; i < r1; i++) ps += ns > 0.0f ? prob(i) / ns : prob(i);
    float all;
    float cdf = block_excl_scan<float>(ps, shf, &all);
    if (tid == 0) tok_sh = V - 1;
    __syncthreads();
    for (int i = r0; i < r1; i++) {
        const float v = ns > 0.0f ? prob(i) / ns : prob(i);
        cdf += v;
        if (v > 0.0f && r < cdf) { atomicMin(&tok_sh, i); break; }
    }
    __syncthreads();
    if (tid == 0) out[row] = tok_sh;
}

}  // namespace

// Chunk length of the split path for V logits: at most TK_G chunks of at
// least 16 values; 0 when a chunk would exceed a workgroup's 4 values per
// thread. Chunks of this length leave none empty.
int topk_chunk_len(int V) {
    const int G = std::min(TK_G, (V + 15) / 16);
    const int ch = (V + G - 1) / G;
    return ch <= TP * 4 ? ch : 0;
}

hipError_t launch_sample(const float* logits, int rows, int V, float temp, int top_k,
                         const float* r_draw, float* prob, long ldp, float* part, int* out,
                         hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if ((ldp & 3) || ldp < V) return hipErrorInvalidValue;
    const int ch = topk_chunk_len(V);
    if (part && top_k > 0 && top_k <= TK_MAX && top_k < V && ch > 0) {
        const int G = (V + ch - 1) / ch;
        k_topk_part<<<dim3(G, rows), TP, 0, s>>>(logits, V, temp, top_k, G, ch, part);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        k_topk_pick<<<rows, TQ, 0, s>>>(logits, V, temp, top_k, G, ch, r_draw, part, out);
        return hipGetLastError();
    }
    k_sample<<<rows, ST, 0, s>>>(logits, V, temp, top_k, r_draw, prob, ldp, out);
    return hipGetLastError();
}
