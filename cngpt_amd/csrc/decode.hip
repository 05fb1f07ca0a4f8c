// decode.hip - kernels of the single-token decode step and the last-position
// pass: products over a few rows with the LayerNorm (or the merge of the
// split attention) folded into the input staging, split-key attention for
// one query row and the argmax of the lm_head (sampling: sample.hip).
//
// A decode step of GPT-2 small reads ~0.5 GB of weights once; every kernel
// here is HBM- or latency-bound. The layout rules: each output column's
// weight row streams once with 16-byte loads; a workgroup issues its weight
// loads before anything that depends on an earlier kernel (activation rows,
// LayerNorm, attention partials), so the HBM latency overlaps the dependent
// reads; the few input rows sit in LDS or L2. No kernel here waits on
// another workgroup: results that need every workgroup (argmax over the
// vocabulary, the merge of attention splits) are finished by the next kernel.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int PRE = 8;    // float4 weight loads per lane issued up front
constexpr int LNCH = 8;   // float4 per lane of one LayerNorm row (C <= 2048)
constexpr int MAXS = 16;  // attention splits merged by a consumer

enum Src : int { SRC_X = 0, SRC_LN = 1, SRC_MERGE = 2, SRC_EMBED = 3 };

__device__ __forceinline__ float dot4(f32x4 a, f32x4 b) {
    return (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w);
}

__device__ __forceinline__ long out_row(const DecGemvArgs& a, int r, int off) {
    long o = a.seg ? (long)(r / a.seg) * a.seg_stride + r % a.seg : r;
    return o + off;
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// Merge the attention splits of rows r < M into xs[r][C] (LDS, float4
// view), C = H * hs. Split s of (row r, head h) holds m_s, l_s and the
// unnormalised o_s[hs] at part + ((r*H + h) * stride + s) * (hs + 4):
//   M = max m_s,  L = sum exp(m_s - M) l_s,  out = sum exp(m_s - M) o_s / L,
// accumulated online, the splits read in batches of MB whose loads are in
// flight together.
template <int MB>
__device__ void merge_rows(const MergeArgs& g, int M, f32x4* xs, int t) {
    const int ns = (t + g.kps) / g.kps;  // splits over keys 0..t
    const int rs = g.hs + 4, h4 = g.hs / 4;
    const int C4 = g.H * h4;
    for (int e = threadIdx.x; e < M * C4; e += blockDim.x) {
        const int r = e / C4, c4 = e - r * C4;
        const int h = c4 / h4, d4 = c4 - h * h4;
        const float* pb = g.part + (long)(r * g.H + h) * g.stride * rs;
        float mx = -INFINITY, L = 0.f;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        // clamped indices: a load under the s < ns branch would be waited
        // for inside it; merged in split order
        for (int s0 = 0; s0 < ns; s0 += MB) {
            float ms[MB], ls[MB];
            f32x4 os[MB];
#pragma unroll
            for (int j = 0; j < MB; j++) {
                const float* ps = pb + min(s0 + j, ns - 1) * rs;
                ms[j] = ps[0];
                ls[j] = ps[1];
                os[j] = *(const f32x4*)(ps + 4 + 4 * d4);
            }
#pragma unroll
            for (int j = 0; j < MB; j++) {
                if (s0 + j < ns) {
                    const float mn = fmaxf(mx, ms[j]);
                    const float a = expf(mx - mn), b = expf(ms[j] - mn);
                    acc = acc * a + os[j] * b;
                    L = L * a + ls[j] * b;
                    mx = mn;
                }
            }
        }
        xs[e] = acc * (1.0f / L);
    }
    __syncthreads();
}

// x rows of a decode step, built in the first product of layer 0:
// x[r] = wte[tok[r]] + wpe[*pos_dev] (reference fast.c:245-254). Workgroup 0
// also stores them (the residual stream) and records the token in hist.
template <int NCH>
__device__ __forceinline__ void embed_row(const EmbedArgs& e, int r, int K4, int lane, f32x4* v) {
    int id = e.tok[r];
    if (id < 0 || id >= e.V) {
        if (lane == 0 && e.err) atomicOr(e.err, 1);
        id = id < 0 ? 0 : e.V - 1;
    }
    const int pos = *e.pos_dev;
    const f32x4* wr = (const f32x4*)(e.wte + (long)id * K4 * 4);
    const f32x4* pr = (const f32x4*)(e.wpe + (long)pos * K4 * 4);
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + 64 * j;
        v[j] = c < K4 ? wr[c] + pr[c] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (blockIdx.x == 0) {
        f32x4* xo = (f32x4*)(e.x_out + (long)r * K4 * 4);
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int c = lane + 64 * j;
            if (c < K4) xo[c] = v[j];
        }
        if (lane == 0 && e.hist) e.hist[(long)r * e.hist_stride + pos] = e.tok[r];
    }
}

// Y[r, n] = epi(src(X)[r, :] . W[n, :]) for r < M <= MR.
// WPC = 1: four columns per 256-thread workgroup, one wavefront each.
// WPC = 4: one column per workgroup, its K range split over the four
// wavefronts (long rows, or few columns). SRC picks the input rows:
// X from global memory, the LayerNorm of X (K = C), or the merged attention
// splits (K = C). With ARGMAX (EPI_STORE) each workgroup also leaves its best
// (value, column) per row in part_v / part_i for launch_argmax_part.
template <int EPI, int MR, int SRC, int WPC, bool ARGMAX>
__global__ void __launch_bounds__(256) k_dgemv(DecGemvArgs a) {
    extern __shared__ f32x4 xs[];  // staged rows [MR][K/4]
    __shared__ float red[4][MR];
    __shared__ int redi[4][MR];

    constexpr int CPW = 4 / WPC;  // columns per workgroup
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = blockIdx.x * CPW + (WPC == 1 ? wave : 0);
    const bool valid = n < a.N;
    const int nn = valid ? n : a.N - 1;
    const int K4 = a.K >> 2;
    const int M = a.M;
    int cb = 0, ce = K4;
    if (WPC == 4) {
        const int chunk = (K4 + 3) / 4;
        cb = min(K4, wave * chunk);
        ce = min(K4, cb + chunk);
    }
    const f32x4* w4 = (const f32x4*)(a.W + (long)nn * a.K);

    // 0. The position the merge of the attention splits needs goes ahead
    // of the weights: the memory counter completes loads in issue order, so
    // a wait for a load issued after the weights also waits for all of them.
    // (The LayerNorm's input rows stay behind the weights: held in
    // registers across the weight loads they cost a workgroup per CU.)
    int t_merge = 0;
    if (SRC == SRC_MERGE) t_merge = a.merge.pos_dev ? *a.merge.pos_dev : a.merge.q_pos;

    // 1. Weights: they do not depend on any earlier kernel.
    f32x4 wp[PRE];
#pragma unroll
    for (int i = 0; i < PRE; i++) {
        const int c = cb + lane + 64 * i;
        wp[i] = c < ce ? w4[c] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // The storing thread of row r: lane r (WPC 1) or thread r (WPC 4).
    const int off = a.row_off + (a.row_off_dev ? *a.row_off_dev : 0);
    const bool storer = WPC == 1 ? true : wave == 0;
    float bv = 0.f;
    if (EPI != EPI_STORE) bv = a.bias[nn];
    float yo[MR];
#pragma unroll
    for (int r = 0; r < MR; r++) {
        yo[r] = 0.f;
        if (EPI == EPI_RESID && storer && r < M && lane == r)
            yo[r] = a.Y[out_row(a, r, off) * a.ldy + nn];
    }

    // 2. Input rows.
    if (SRC == SRC_LN || SRC == SRC_EMBED) {
        // LayerNorm (reference ops.c:191-248): mean, biased variance of
        // (x - mean), rstd = 1/sqrtf(var + 1e-5), (x - mean) * rstd * w + b.
        const f32x4* lw = (const f32x4*)a.ln_w;
        const f32x4* lb = (const f32x4*)a.ln_b;
        for (int r = wave; r < M; r += 4) {
            f32x4 v[LNCH];
            if (SRC == SRC_EMBED) {
                embed_row<LNCH>(a.emb, r, K4, lane, v);
            } else {
                const f32x4* xr = (const f32x4*)(a.X + (long)r * a.ldx);
#pragma unroll
                for (int j = 0; j < LNCH; j++) {
                    const int c = lane + 64 * j;
                    v[j] = c < K4 ? xr[c] : f32x4{0.f, 0.f, 0.f, 0.f};
                }
            }
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < LNCH; j++) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
            const float mean = wave_sum(s) / (float)a.K;
            float q = 0.f;
#pragma unroll
            for (int j = 0; j < LNCH; j++) {
                const int c = lane + 64 * j;
                if (c < K4) {
                    f32x4 d = v[j] - mean;
                    q += dot4(d, d);
                }
            }
            const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)a.K + 1e-5f);
#pragma unroll
            for (int j = 0; j < LNCH; j++) {
                const int c = lane + 64 * j;
                if (c < K4) xs[r * K4 + c] = (v[j] - mean) * rstd * lw[c] + lb[c];
            }
        }
        __syncthreads();
    } else if (SRC == SRC_MERGE) {
        merge_rows<4>(a.merge, M, xs, t_merge);
    }

    // 3. Dot products over this wavefront's K range.
    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; r++) acc[r] = 0.f;
#pragma unroll
    for (int i = 0; i < PRE; i++) {
        const int c = cb + lane + 64 * i;
        if (c < ce) {
#pragma unroll
            for (int r = 0; r < MR; r++)
                if (r < M) {
                    const f32x4 x =
                        SRC != SRC_X ? xs[r * K4 + c] : ((const f32x4*)(a.X + (long)r * a.ldx))[c];
                    acc[r] += dot4(wp[i], x);
                }
        }
    }
    for (int c = cb + lane + 64 * PRE; c < ce; c += 64) {
        const f32x4 w = w4[c];
#pragma unroll
        for (int r = 0; r < MR; r++)
            if (r < M) {
                const f32x4 x =
                    SRC != SRC_X ? xs[r * K4 + c] : ((const f32x4*)(a.X + (long)r * a.ldx))[c];
                acc[r] += dot4(w, x);
            }
    }
#pragma unroll
    for (int r = 0; r < MR; r++) acc[r] = wave_sum(acc[r]);
    if (WPC == 4) {
        // Sum the four wavefronts' K ranges in a fixed order.
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < MR; r++) red[wave][r] = acc[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < MR; r++) acc[r] = (red[0][r] + red[1][r]) + (red[2][r] + red[3][r]);
        __syncthreads();
    }

    // 4. Epilogue: the storer of row r writes it.
#pragma unroll
    for (int r = 0; r < MR; r++) {
        if (r >= M) break;
        if (valid && storer && lane == r) {
            float* y = a.Y + out_row(a, r, off) * a.ldy + nn;
            float v;
            if (EPI == EPI_STORE) v = acc[r];
            else if (EPI == EPI_BIAS) v = acc[r] + bv;
            else if (EPI == EPI_BIAS_GELU) v = gelu_tanh(acc[r] + bv);
            else v = (yo[r] + acc[r]) + bv;
            *y = v;
        }
    }
    if (!ARGMAX) return;

    // 5. Best column of this workgroup per row.
    if (WPC == 1) {
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < MR; r++) {
                red[wave][r] = valid ? acc[r] : -INFINITY;
                redi[wave][r] = valid ? n : 0x7fffffff;
            }
        __syncthreads();
        if (tid < M) {
            float b = red[0][tid];
            int bi = redi[0][tid];
#pragma unroll
            for (int w = 1; w < 4; w++)
                if (better(red[w][tid], redi[w][tid], b, bi)) { b = red[w][tid]; bi = redi[w][tid]; }
            a.part_v[(long)tid * gridDim.x + blockIdx.x] = b;
            a.part_i[(long)tid * gridDim.x + blockIdx.x] = bi;
        }
    } else {
#pragma unroll
        for (int r = 0; r < MR; r++)
            if (r < M && tid == r) {
                a.part_v[(long)r * gridDim.x + blockIdx.x] = valid ? acc[r] : -INFINITY;
                a.part_i[(long)r * gridDim.x + blockIdx.x] = valid ? n : 0x7fffffff;
            }
    }
}

// ---------------------------------------------------------------- attention

// One query row per (sequence, head) at position t (= *pos_dev, or q_pos)
// against keys 0..t, split over workgroups of KPB keys (grid.y). Split s
// writes its max m, sum l and unnormalised P.V to the partials; the consumer
// merges the splits (merge_rows). Keys past t are not visited: the
// reference's -1e9 mask gives them probability exactly 0.
template <int HS>
__global__ void __launch_bounds__(256) k_attn_dec(AttnDecArgs a) {
    constexpr int LPK = HS / 4;                 // lanes per key, one float4 each
    constexpr int KPP = 256 / LPK;              // keys per pass of the workgroup
    constexpr int KPB = KPP > 64 ? KPP : 64;    // keys per workgroup
    constexpr int NPASS = KPB / KPP;
    __shared__ float red[8];
    __shared__ f32x4 osum[4][LPK];

    const int bh = blockIdx.x, s = blockIdx.y;
    const int b = bh / a.H, h = bh % a.H;
    const int t = a.pos_dev ? *a.pos_dev : a.q_pos;
    const int nk = t + 1;
    if (s * KPB >= nk) return;
    const long C3 = 3L * a.C;
    const float* base = a.qkv + (long)b * a.seq_stride * C3 + h * HS;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kl = tid / LPK, d4 = tid % LPK;

    // Every global load up front: q, K and V rows of this thread's keys.
    const f32x4 q = *(const f32x4*)(base + (long)t * C3 + d4 * 4);
    f32x4 kr[NPASS], vr[NPASS];
#pragma unroll
    for (int p = 0; p < NPASS; p++) {
        const int key = s * KPB + p * KPP + kl;
        const bool ok = key < nk;
        const float* rp = base + (long)(ok ? key : 0) * C3 + d4 * 4;
        kr[p] = ok ? *(const f32x4*)(rp + a.C) : f32x4{0.f, 0.f, 0.f, 0.f};
        vr[p] = ok ? *(const f32x4*)(rp + 2 * a.C) : f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // Scores: reduce the LPK partial dots of each key.
    float sc[NPASS];
    float mx = -INFINITY;
#pragma unroll
    for (int p = 0; p < NPASS; p++) {
        float d = dot4(q, kr[p]);
#pragma unroll
        for (int o = 1; o < LPK; o <<= 1) d += __shfl_xor(d, o, 64);
        const int key = s * KPB + p * KPP + kl;
        sc[p] = key < nk ? d * a.scale : -INFINITY;
        mx = fmaxf(mx, sc[p]);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));

    float ls = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < NPASS; p++) {
        const float e = expf(sc[p] - mx);  // 0 for keys past t
        if (d4 == 0) ls += e;
        o += e * vr[p];
    }
    // Sum o over the keys of the wavefront (lanes with the same d4) ...
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) {
        o.x += __shfl_xor(o.x, off, 64);
        o.y += __shfl_xor(o.y, off, 64);
        o.z += __shfl_xor(o.z, off, 64);
        o.w += __shfl_xor(o.w, off, 64);
    }
    ls = wave_sum(ls);
    if (lane < LPK) osum[wave][lane] = o;
    if (lane == 0) red[4 + wave] = ls;
    __syncthreads();
    // ... then over the four wavefronts.
    float* part = a.part + ((long)bh * a.max_splits + s) * (HS + 4);
    if (tid < LPK)
        *(f32x4*)(part + 4 + tid * 4) = (osum[0][tid] + osum[1][tid]) + (osum[2][tid] + osum[3][tid]);
    if (tid == 0) {
        part[0] = mx;
        part[1] = (red[4] + red[5]) + (red[6] + red[7]);
    }
}

// The same attention in one pass when the (sequence, head) pairs alone
// occupy the CUs (batched decode, B * H >= 128): one workgroup per pair, its
// NW wavefronts split keys 0..t into contiguous ranges and walk them in
// rounds of PD passes of K/V loads issued together (a pass: 64 / (hs/4)
// keys, hs/4 lanes per key, one float4 each); each lane group keeps a
// running max, sum and o (online softmax in base 2, q pre-scaled by
// scale * log2(e)); the groups
// of a wavefront merge by shuffles, the wavefronts through LDS in order,
// and the workgroup writes the normalised row: no partials, no merge
// launch. Measured against the split form + merge (probe, caches streamed
// from HBM): XL B=32 t=100 15.2 -> 11.1 us, GPT-2 small B=12 t=500 14.3 ->
// 12.3 us, medium B=8 t=300 10.6 -> 7.8 us, medium B=8 t=1000 19.8 -> 19.8
// us; with fewer pairs (small B=4 t=1000: 12.1 -> 15.4 us) the split form
// keeps more loads in flight.
//
// With fewer pairs than CUs (SPL = 2: B * H < 256, e.g. GPT-2 medium B=8's
// 128 pairs, whose workgroups leave half the CUs idle) the keys of a pair
// are split over two workgroups. Each counts itself in on the pair's
// counter; the first in writes its unnormalised (m, l, o) as tagged 64-bit
// words (the tag in the high half, agent-scope atomics: the L2 of one XCD
// is not coherent with another's) and leaves, and the second in polls them,
// merges both halves, half 0 first whatever the arrival order
// (reproducible), writes the row and clears the words. Tags come from the
// counter (each use adds 2), so both halves of a use agree on theirs and no
// use can match an earlier use's words; the second waits only on a
// workgroup that has already counted itself in, i.e. is running.
constexpr int DEC1_MIN_PAIRS = 128;
constexpr int DEC1_SPLIT_BELOW = 256;
typedef unsigned long long u64;
// Sum over each group of G consecutive lanes (G a power of two <= 64),
// every lane of a group receiving it: the xor butterfly over 1, 2, 4, ...
// (the same additions in the same order), within 16 lanes by DPP row
// operations instead of LDS permutes.
template <int G>
__device__ __forceinline__ float lane_group_sum(float d) {
    if (G >= 2) d += CNGPT_DPP(d, 0xB1);   // quad_perm [1,0,3,2]: lane ^ 1
    if (G >= 4) d += CNGPT_DPP(d, 0x4E);   // quad_perm [2,3,0,1]: lane ^ 2
    if (G >= 8) d += CNGPT_DPP(d, 0x141);  // row_half_mirror: the other quad of 8
    if (G >= 16) d += CNGPT_DPP(d, 0x140); // row_mirror: the other half of 16
    if (G >= 32) d += __shfl_xor(d, 16, 64);
    if (G >= 64) d += __shfl_xor(d, 32, 64);
    return d;
}

template <int HS, int NW, int PD, int SPL>
__global__ void __launch_bounds__(NW * 64) k_attn_dec1(AttnDecArgs a, float* __restrict__ out,
                                                       long ldo) {
    constexpr int LPK = HS / 4;    // lanes per key
    constexpr int KPW = 64 / LPK;  // keys per wavefront pass
    static_assert(LPK <= 64, "the merged row is held by wavefront 0");
    __shared__ float wm[NW], wl[NW];
    __shared__ f32x4 wo[NW][LPK];
    const int bh = blockIdx.x / SPL, half = blockIdx.x % SPL;
    const int b = bh / a.H, h = bh % a.H;
    const int t = a.pos_dev ? *a.pos_dev : a.q_pos;
    const int nk = t + 1;
    const long C3 = 3L * a.C;
    const float* base = a.qkv + (long)b * a.seq_stride * C3 + h * HS;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kl = lane / LPK, d4 = lane % LPK;
    // this workgroup's keys [kb, ke), split over its wavefronts
    const int kb = (int)((long)half * nk / SPL), nks = (int)((long)(half + 1) * nk / SPL) - kb;
    const int k0 = kb + (int)((long)wave * nks / NW), k1 = kb + (int)((long)(wave + 1) * nks / NW);
    const int npass = (k1 - k0 + KPW - 1) / KPW;
    // With qkv_part the QKV product left its K-split partials: this head's
    // q, k and v of row t are their sum in split order plus the bias (the
    // arithmetic of the split-K sum launch), formed here into LDS, written
    // to row t of the cache for the later steps (by the first workgroup of
    // the pair), and taken from LDS for the query and for key t.
    __shared__ f32x4 cur[3][LPK];
    const bool fold = a.qkv_part != nullptr;
    if (fold) {
        static_assert(NW * 64 >= 3 * HS, "one thread per value of the row");
        if (tid < 3 * HS) {
            const int which = tid / HS, d = tid - which * HS;
            const long c = (long)which * a.C + h * HS + d;
            const long slab = (long)a.qkv_rows * C3;
            const float* pp = a.qkv_part + (long)b * C3 + c;
            float v = 0.f;
            for (int ks = 0; ks < a.qkv_ks; ks++) v += pp[ks * slab];
            v = v + a.qkv_bias[c];
            ((float*)cur)[which * HS + d] = v;
        }
        __syncthreads();
    }
    const f32x4 q = (fold ? cur[0][d4] : *(const f32x4*)(base + (long)t * C3 + d4 * 4)) *
                    (a.scale * 1.4426950408889634f);
    const f32x4 kt = fold ? cur[1][d4] : f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 vt = fold ? cur[2][d4] : f32x4{0.f, 0.f, 0.f, 0.f};

    // Rounds of PD passes: every load of a round is issued first (keys
    // past the range re-read its last one; an empty range runs no round),
    // then the passes are consumed in order. No load register is carried
    // from one loop trip to the next: a ring carried that way got a wait
    // for every load in flight after each pass, one memory latency per pass.
    float m = -INFINITY, l = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    for (int p0 = 0; p0 < npass; p0 += PD) {
        f32x4 kr[PD], vr[PD];
#pragma unroll
        for (int j = 0; j < PD; j++) {
            const int key = min(k0 + (p0 + j) * KPW + kl, k1 - 1);
            const float* rp = base + (long)key * C3 + d4 * 4;
            kr[j] = *(const f32x4*)(rp + a.C);
            vr[j] = *(const f32x4*)(rp + 2 * a.C);
            // (key t's row is not in the cache yet in the folded form: its
            // values from LDS, by selects, not a branch around the loads)
            const bool newest = fold && key == t;
            kr[j] = newest ? kt : kr[j];
            vr[j] = newest ? vt : vr[j];
        }
        // all of them before the first use (the scheduler would otherwise
        // spread them out to save registers)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < PD; j++) {
            // formed for every lane and kept for keys in the range (a branch
            // around the use would draw the V load into it, behind a wait
            // for every load of the round)
            const float d = lane_group_sum<LPK>(dot4(q, kr[j]));
            const bool in = k0 + (p0 + j) * KPW + kl < k1;
            const float mn = fmaxf(m, d);
            const float al = __builtin_amdgcn_exp2f(m - mn);
            const float e = __builtin_amdgcn_exp2f(d - mn);
            const float ln = l * al + e;
            const f32x4 on = o * al + e * vr[j];
            l = in ? ln : l;
            o = in ? on : o;
            m = in ? mn : m;
        }
    }
    // (folded form) row t into the cache for the later steps, after this
    // step's loads so that no wait for it precedes them; the cache is the
    // caller's writable buffer and row t is this step's, which the product
    // would otherwise have written
    if (fold && half == 0 && tid < 3 * HS) {
        const int which = tid / HS, d = tid - which * HS;
        const_cast<float*>(base)[(long)t * C3 + (long)which * a.C + d] =
            ((const float*)cur)[which * HS + d];
    }
    // merge the key groups of a wavefront (a group with no key has m = -inf)
#pragma unroll
    for (int sh = LPK; sh < 64; sh <<= 1) {
        const float m2 = __shfl_xor(m, sh, 64), l2 = __shfl_xor(l, sh, 64);
        const f32x4 o2 = {__shfl_xor(o.x, sh, 64), __shfl_xor(o.y, sh, 64),
                          __shfl_xor(o.z, sh, 64), __shfl_xor(o.w, sh, 64)};
        const float mn = fmaxf(m, m2);
        const float a1 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
        const float a2 = m2 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m2 - mn);
        l = l * a1 + l2 * a2;
        o = o * a1 + o2 * a2;
        m = mn;
    }
    if (lane < LPK) wo[wave][lane] = o;
    if (lane == 0) {
        wm[wave] = m;
        wl[wave] = l;
    }
    __syncthreads();
    // then the wavefronts, in order (key 0 is in every row, so L > 0 once
    // the halves of a split pair are merged)
    float M = -INFINITY, L = 0.f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
    if (tid < LPK) {
        for (int w = 0; w < NW; w++) M = fmaxf(M, wm[w]);
        for (int w = 0; w < NW; w++) {
            const float f = wm[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(wm[w] - M);
            L += wl[w] * f;
            O += wo[w][tid] * f;
        }
    }
    if (SPL == 1) {
        if (tid < LPK) *(f32x4*)(out + (long)b * ldo + h * HS + tid * 4) = O * (1.0f / L);
        return;
    }
    if (wave != 0) return;
    // words of half s of this pair: m, l, o[HS]
    constexpr int NWD = HS + 2;
    unsigned* cnt = a.tag_cnt + bh;
    // count in first: one round trip, after which the first in publishes
    // its words and leaves, and the second in (which has its own half in
    // registers) merges without writing or waiting for any store
    unsigned old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = (unsigned)__builtin_amdgcn_readfirstlane((int)old);
    const unsigned tag = old / 2u + 1u;
    auto word = [&](float v) { return ((u64)tag << 32) | (u64)__float_as_uint(v); };
    if ((old & 1u) == 0) {
        u64* mine = a.tag_part + ((long)bh * 2 + half) * NWD;
        if (lane < LPK)
#pragma unroll
            for (int c = 0; c < 4; c++)
                __hip_atomic_store(mine + 2 + 4 * lane + c, word(O[c]), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) {
            __hip_atomic_store(mine, word(M), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(mine + 1, word(L), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    // second in: the other half's words, until each carries this use's tag
    const u64* other = a.tag_part + ((long)bh * 2 + (1 - half)) * NWD;
    u64 w[6];
    auto fetch_other = [&]() {
        const int e = 2 + 4 * min(lane, LPK - 1);
#pragma unroll
        for (int c = 0; c < 4; c++)
            w[c] = __hip_atomic_load(other + e + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        w[4] = __hip_atomic_load(other, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        w[5] = __hip_atomic_load(other + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto current = [&]() {
        bool ok = true;
#pragma unroll
        for (int c = 0; c < 6; c++) ok = ok && (unsigned)(w[c] >> 32) == tag;
        return ok;
    };
    fetch_other();
    bool ok = current();
    // the other half counted itself in first and is writing its words, so
    // they become visible within a round trip or two; the limit only guards
    // against a fault, and then the row is poisoned (NaN) rather than hung
    for (long it = 0; __builtin_amdgcn_ballot_w64(!ok) != 0 && it < (1L << 20); it++) {
        __builtin_amdgcn_s_sleep(1);
        if (!ok) {
            fetch_other();
            ok = current();
        }
    }
    const float Mo = __uint_as_float((unsigned)w[4]), Lo = __uint_as_float((unsigned)w[5]);
    const f32x4 Oo = {__uint_as_float((unsigned)w[0]), __uint_as_float((unsigned)w[1]),
                      __uint_as_float((unsigned)w[2]), __uint_as_float((unsigned)w[3])};
    // half 0 first, then half 1
    const float M0 = half == 0 ? M : Mo, L0 = half == 0 ? L : Lo;
    const float M1 = half == 0 ? Mo : M, L1 = half == 0 ? Lo : L;
    const f32x4 O0 = half == 0 ? O : Oo, O1 = half == 0 ? Oo : O;
    const float Mx = fmaxf(M0, M1);
    const float f0 = M0 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M0 - Mx);
    const float f1 = M1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M1 - Mx);
    const float Ls = L0 * f0 + L1 * f1;
    const f32x4 Os = O0 * f0 + O1 * f1;
    const bool all_ok = __builtin_amdgcn_ballot_w64(!ok) == 0;
    if (!all_ok && lane == 0 && a.err) atomicOr(a.err, ATTN_DEC_TIMEOUT);
    if (lane < LPK)
        *(f32x4*)(out + (long)b * ldo + h * HS + lane * 4) =
            all_ok ? Os * (1.0f / Ls) : f32x4{NAN, NAN, NAN, NAN};
    // the words read are cleared, so that a slot never keeps an old use's
    // words (tags repeat after 2^31 uses of a pair)
    u64* done = const_cast<u64*>(other);
    if (lane < LPK)
#pragma unroll
        for (int c = 0; c < 4; c++)
            __hip_atomic_store(done + 2 + 4 * lane + c, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (lane == 0) {
        __hip_atomic_store(done, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(done + 1, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Rows of merged attention for the consumers that are not k_dgemv (M > 8).
__global__ void __launch_bounds__(256) k_attn_merge(MergeArgs g, float* __restrict__ out, long ldo) {
    extern __shared__ f32x4 xs[];
    // one row per workgroup: offset the partials to row blockIdx.x
    MergeArgs gr = g;
    gr.part = g.part + (long)blockIdx.x * g.H * g.stride * (g.hs + 4);
    // every split of a row in one batch, or batches of 4 while the splits
    // are few (a batch past the last split re-reads it)
    const int t = g.pos_dev ? *g.pos_dev : g.q_pos;
    if ((t + g.kps) / g.kps > 4) merge_rows<MAXS>(gr, 1, xs, t);
    else merge_rows<4>(gr, 1, xs, t);
    const int C4 = g.H * g.hs / 4;
    f32x4* o = (f32x4*)(out + (long)blockIdx.x * ldo);
    for (int c = threadIdx.x; c < C4; c += blockDim.x) o[c] = xs[c];
}

// ---------------------------------------------------------------- argmax

// out[r] = the best of the nparts (value, column) partials of row r (first
// column on ties); then *pos_inc += 1. One 1024-thread workgroup per row.
__global__ void __launch_bounds__(1024) k_argmax_part(const float* __restrict__ part_v,
                                                      const int* __restrict__ part_i, int nparts,
                                                      int* __restrict__ out, int* pos_inc) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const float* pv = part_v + (long)blockIdx.x * nparts;
    const int* pi = part_i + (long)blockIdx.x * nparts;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    // 16 partials in flight per thread (as k_argmax_rows)
    constexpr int U = 16;
    for (int g0 = threadIdx.x; g0 < nparts; g0 += 1024 * U) {
        float xv[U];
        int xi[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int g = min(g0 + 1024 * u, nparts - 1);
            xv[u] = pv[g];
            xi[u] = pi[g];
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (g0 + 1024 * u < nparts && better(xv[u], xi[u], best, bi)) {
                best = xv[u];
                bi = xi[u];
            }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ob = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (better(ob, oi, best, bi)) { best = ob; bi = oi; }
    }
    const int wid = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wid] = best; si[wid] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 16; k++)
            if (better(sv[k], si[k], best, bi)) { best = sv[k]; bi = si[k]; }
        out[blockIdx.x] = bi;
        if (pos_inc && blockIdx.x == 0) *pos_inc += 1;
    }
}

// out[r] = argmax_v logits[r, v], first index on ties. One 1024-thread
// workgroup per row. Thread 0 of workgroup 0 then advances *pos_inc.
__global__ void __launch_bounds__(1024) k_argmax_rows(const float* __restrict__ logits, int V,
                                                      int* __restrict__ out, int* pos_inc) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const float* row = logits + (long)blockIdx.x * V;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    // 16 loads in flight per thread, then compared in index order (one load
    // at a time waited for each in turn: 49 memory round trips for a
    // 50257-wide row)
    constexpr int U = 16;
    for (int v0 = threadIdx.x; v0 < V; v0 += 1024 * U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; u++) x[u] = row[min(v0 + 1024 * u, V - 1)];
#pragma unroll
        for (int u = 0; u < U; u++)
            if (v0 + 1024 * u < V && x[u] > best) {
                best = x[u];
                bi = v0 + 1024 * u;
            }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ob = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (better(ob, oi, best, bi)) { best = ob; bi = oi; }
    }
    const int wid = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wid] = best; si[wid] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 16; k++)
            if (better(sv[k], si[k], best, bi)) { best = sv[k]; bi = si[k]; }
        out[blockIdx.x] = bi;
        if (pos_inc && blockIdx.x == 0) *pos_inc += 1;
    }
}

// ---------------------------------------------------------------- launchers

template <int EPI, int MR, int SRC, int WPC, bool ARGMAX>
hipError_t dgemv_go(const DecGemvArgs& a, hipStream_t s) {
    const size_t lds = SRC != SRC_X ? (size_t)MR * a.K * sizeof(float) : 0;
    constexpr int CPW = 4 / WPC;
    k_dgemv<EPI, MR, SRC, WPC, ARGMAX><<<(a.N + CPW - 1) / CPW, 256, lds, s>>>(a);
    return hipGetLastError();
}

template <int EPI, int SRC, int WPC, bool ARGMAX>
hipError_t dgemv_rows(const DecGemvArgs& a, hipStream_t s) {
    if (a.M <= 1) return dgemv_go<EPI, 1, SRC, WPC, ARGMAX>(a, s);
    if (a.M <= 2) return dgemv_go<EPI, 2, SRC, WPC, ARGMAX>(a, s);
    if (a.M <= 4) return dgemv_go<EPI, 4, SRC, WPC, ARGMAX>(a, s);
    return dgemv_go<EPI, 8, SRC, WPC, ARGMAX>(a, s);
}

// One wavefront per column while that gives enough workgroups and the row
// fits the up-front loads; otherwise the four wavefronts split the row.
template <int EPI, int SRC, bool ARGMAX>
hipError_t dgemv_wpc(const DecGemvArgs& a, hipStream_t s) {
    const bool split = a.N < 2048 || a.K > 4 * 64 * PRE;
    if (split) return dgemv_rows<EPI, SRC, 4, ARGMAX>(a, s);
    return dgemv_rows<EPI, SRC, 1, ARGMAX>(a, s);
}

template <int EPI>
hipError_t dgemv_src(const DecGemvArgs& a, hipStream_t s) {
    if (a.ln_w && a.emb.tok) return dgemv_wpc<EPI, SRC_EMBED, false>(a, s);
    if (a.ln_w) return dgemv_wpc<EPI, SRC_LN, false>(a, s);
    if (a.merge.part) return dgemv_wpc<EPI, SRC_MERGE, false>(a, s);
    return dgemv_wpc<EPI, SRC_X, false>(a, s);
}

template <int HS>
hipError_t attn_dec_hs(const AttnDecArgs& a, int B, int max_keys, hipStream_t s) {
    constexpr int LPK = HS / 4;
    constexpr int KPP = 256 / LPK;
    constexpr int KPB = KPP > 64 ? KPP : 64;
    const int splits = (max_keys + KPB - 1) / KPB;
    if (splits > a.max_splits) return hipErrorInvalidValue;
    dim3 grid(B * a.H, splits);
    k_attn_dec<HS><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

template <int HS>
hipError_t attn_dec1_hs(const AttnDecArgs& a, int B, float* out, long ldo, hipStream_t s) {
    const int pairs = B * a.H;
    if (pairs < DEC1_SPLIT_BELOW && a.tag_part && a.tag_cnt && pairs <= a.tag_pairs)
        k_attn_dec1<HS, 16, 4, 2><<<2 * pairs, 16 * 64, 0, s>>>(a, out, ldo);
    else if (pairs < 384) k_attn_dec1<HS, 16, 4, 1><<<pairs, 16 * 64, 0, s>>>(a, out, ldo);
    else k_attn_dec1<HS, 8, 4, 1><<<pairs, 8 * 64, 0, s>>>(a, out, ldo);
    return hipGetLastError();
}

}  // namespace

bool attention_dec_one_pass(int B, int H) { return (long)B * H >= DEC1_MIN_PAIRS; }

size_t attn_dec1_tag_words(int pairs, int hs) { return (size_t)pairs * 2 * (hs + 2); }

int attn_dec1_split_pairs() { return DEC1_SPLIT_BELOW - 1; }

hipError_t launch_attention_dec_rows(const AttnDecArgs& a, int B, float* out, long ldo,
                                     hipStream_t s) {
    if (B <= 0) return hipSuccess;
    if (!attention_dec_one_pass(B, a.H) || (ldo & 3)) return hipErrorInvalidValue;
    if (a.qkv_part && (a.qkv_ks < 1 || a.qkv_rows != B || !a.qkv_bias)) return hipErrorInvalidValue;
    switch (a.C / a.H) {
        case 8: return attn_dec1_hs<8>(a, B, out, ldo, s);
        case 16: return attn_dec1_hs<16>(a, B, out, ldo, s);
        case 32: return attn_dec1_hs<32>(a, B, out, ldo, s);
        case 64: return attn_dec1_hs<64>(a, B, out, ldo, s);
        case 128: return attn_dec1_hs<128>(a, B, out, ldo, s);
    }
    return hipErrorInvalidValue;
}

int attn_dec_keys_per_split(int hs) {
    const int kpp = 256 / (hs / 4);
    return kpp > 64 ? kpp : 64;
}

hipError_t launch_dgemv(const DecGemvArgs& a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0) return hipSuccess;
    if (a.M > 8 || a.K <= 0 || (a.K & 3)) return hipErrorInvalidValue;
    if (a.ln_w && (a.K > 256 * LNCH || a.merge.part)) return hipErrorInvalidValue;
    if (a.emb.tok && (!a.ln_w || !a.emb.wte || !a.emb.wpe || !a.emb.pos_dev || !a.emb.x_out))
        return hipErrorInvalidValue;
    if (a.merge.part) {
        const MergeArgs& g = a.merge;
        if (g.H > 32 || g.hs * g.H != a.K || (g.hs & 3) || g.stride > MAXS || g.kps <= 0)
            return hipErrorInvalidValue;
    }
    if (a.argmax) {
        if (a.epi != EPI_STORE || !a.part_v || !a.part_i || a.merge.part || a.emb.tok)
            return hipErrorInvalidValue;
        if (a.ln_w) return dgemv_wpc<EPI_STORE, SRC_LN, true>(a, s);
        return dgemv_wpc<EPI_STORE, SRC_X, true>(a, s);
    }
    switch (a.epi) {
        case EPI_STORE: return dgemv_src<EPI_STORE>(a, s);
        case EPI_BIAS: return dgemv_src<EPI_BIAS>(a, s);
        case EPI_BIAS_GELU: return dgemv_src<EPI_BIAS_GELU>(a, s);
        case EPI_RESID: return dgemv_src<EPI_RESID>(a, s);
    }
    return hipErrorInvalidValue;
}

int dgemv_argmax_parts(const DecGemvArgs& a) {
    const bool split = a.N < 2048 || a.K > 4 * 64 * PRE;
    const int cpw = split ? 1 : 4;
    return (a.N + cpw - 1) / cpw;
}

hipError_t launch_attention_dec(const AttnDecArgs& a, int B, int max_keys, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    if (max_keys <= 0) return hipErrorInvalidValue;
    switch (a.C / a.H) {
        case 8: return attn_dec_hs<8>(a, B, max_keys, s);
        case 16: return attn_dec_hs<16>(a, B, max_keys, s);
        case 32: return attn_dec_hs<32>(a, B, max_keys, s);
        case 64: return attn_dec_hs<64>(a, B, max_keys, s);
        case 128: return attn_dec_hs<128>(a, B, max_keys, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_attention_merge(const MergeArgs& g, int B, float* out, long ldo, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    if (g.H > 32 || (g.hs & 3) || g.stride > MAXS || g.kps <= 0) return hipErrorInvalidValue;
    k_attn_merge<<<B, 256, (size_t)g.H * g.hs * sizeof(float), s>>>(g, out, ldo);
    return hipGetLastError();
}

hipError_t launch_argmax_part(const float* part_v, const int* part_i, int rows, int nparts,
                              int* out, int* pos_inc, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    k_argmax_part<<<rows, 1024, 0, s>>>(part_v, part_i, nparts, out, pos_inc);
    return hipGetLastError();
}

hipError_t launch_argmax_rows(const float* logits, int rows, int V, int* out, int* pos_inc,
                              hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    k_argmax_rows<<<rows, 1024, 0, s>>>(logits, V, out, pos_inc);
    return hipGetLastError();
}

