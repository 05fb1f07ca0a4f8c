// attention.hip - causal self-attention straight from the packed qkv rows.
//
// The reference (fast.c:267-298) computes, per (sequence, head), the full
// T x T score plane S = (1/sqrt(hs)) Q K^T with cblas_sgemm, sets the upper
// triangle to -1e9 (ops.c:488-493), applies a three-pass row softmax
// (ops.c:424-482) and multiplies by V. exp(-1e9 - max) is exactly 0 in fp32,
// so skipping masked keys gives the same probabilities; no score plane is
// ever written here.
//
// k_attn_causal: one workgroup = 4 wavefronts = 128 queries of one
// (sequence, head). K/V tiles of 64 keys are double-buffered in LDS. Each
// wavefront computes S^T = K Q^T for its 32 queries with
// v_mfma_f32_32x32x2f32, so a lane holds one query column: the row max and
// row sum need one cross-half shuffle, and the probabilities feed the
// O^T += V^T P^T product directly from the accumulator registers (the key
// order of the S^T output layout is used as the k order of that product).
// The softmax is the online (running max / running sum) form, in base 2:
// Q is pre-multiplied by scale * log2(e), so a probability is one hardware
// exp2 of (score - running max); the causal mask is applied only on the
// tiles that cross the diagonal.
//
// k_attn_ks (below) splits the keys of 32 queries over four wavefronts
// for launches with few blocks.
//
// The one-query form (the last-position pass, fast.c:287-297, and a decode
// step) is k_attn_dec in decode.hip.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int KT = 64;  // keys per LDS tile

template <int HS>
__global__ void __launch_bounds__(256, 2)
    k_attn_causal(const float* __restrict__ qkv, long seq_stride, float* __restrict__ out, int B,
                  int T, int C, int H, int nqb, float scale, float* __restrict__ lse) {
    constexpr int HALF = HS / 2;            // d values per lane half in Q K^T
    constexpr int F4 = HS / 4;              // float4 per head row
    constexpr int ROW = HS + 4;             // padded LDS row
    constexpr int NDB = (HS + 31) / 32;     // 32-row blocks of O^T
    constexpr int LITERS = (KT * F4 + 255) / 256;
    __shared__ float Ks[2][KT * ROW];
    __shared__ float Vs[2][KT * ROW];

    const int BH = B * H;
    const int qb = nqb - 1 - (int)(blockIdx.x / BH);  // longest query blocks first
    const int bh = blockIdx.x % BH;
    const int b = bh / H, h = bh % H;
    const long C3 = 3L * C;
    const float* base = qkv + (long)b * seq_stride * C3;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 31, lh = lane >> 5;
    const int q0 = qb * 128 + wave * 32;  // first query of this wavefront
    const int qi = q0 + lr;                // this lane's query
    const int q_last_wg = min(qb * 128 + 127, T - 1);
    const int ntiles = q_last_wg / KT + 1;

    // Q row of this lane's query, d in [lh*HALF, lh*HALF + HALF).
    float qreg[HALF];
    {
        const float* qp = base + (long)min(qi, T - 1) * C3 + h * HS + lh * HALF;
        const float qs = scale * 1.4426950408889634f;  // scores in units of log2
#pragma unroll
        for (int s = 0; s < HALF; s += 4) {
            f32x4 v = *(const f32x4*)(qp + s);
            qreg[s] = v.x * qs; qreg[s + 1] = v.y * qs; qreg[s + 2] = v.z * qs; qreg[s + 3] = v.w * qs;
        }
    }

    f32x4 rk[LITERS], rv[LITERS];
    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < LITERS; i++) {
            int idx = tid + 256 * i;
            if (idx < KT * F4) {
                int key = min(kt * KT + idx / F4, T - 1);
                const float* rp = base + (long)key * C3 + h * HS + (idx % F4) * 4;
                rk[i] = *(const f32x4*)(rp + C);
                rv[i] = *(const f32x4*)(rp + 2 * C);
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LITERS; i++) {
            int idx = tid + 256 * i;
            if (idx < KT * F4) {
                int o = (idx / F4) * ROW + (idx % F4) * 4;
                *(f32x4*)&Ks[buf][o] = rk[i];
                *(f32x4*)&Vs[buf][o] = rv[i];
            }
        }
    };

    f32x16 o[NDB];
#pragma unroll
    for (int d = 0; d < NDB; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[d][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < ntiles; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < ntiles) gload(kt + 1);
        // Wave-uniform: skip tiles entirely above this wavefront's queries.
        if (q0 < T && kt * KT <= q0 + 31) {
            const float* ks = &Ks[cur][0];
            const float* vs = &Vs[cur][0];
            f32x16 s[2];
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int r = 0; r < 16; r++) s[kb][r] = 0.f;
#pragma unroll
                for (int d = 0; d < HALF; d += 4) {
                    f32x4 kv = *(const f32x4*)&ks[(kb * 32 + lr) * ROW + lh * HALF + d];
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qreg[d], s[kb], 0, 0, 0);
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qreg[d + 1], s[kb], 0, 0, 0);
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qreg[d + 2], s[kb], 0, 0, 0);
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qreg[d + 3], s[kb], 0, 0, 0);
                }
            }
            // s[kb][r] = score (log2 units) of key kt*64 + 32kb + 8(r/4) +
            // 4lh + r%4 for query qi; keys after qi exist only in a tile that
            // reaches past this wavefront's first query
            if (kt * KT + KT - 1 > q0) {
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int key = kt * KT + kb * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                        s[kb][r] = (key > qi) ? -INFINITY : s[kb][r];
                    }
            }
            float mt = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) mt = fmaxf(mt, s[kb][r]);
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            const float m_new = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            float ps = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    float p = __builtin_amdgcn_exp2f(s[kb][r] - m_new);
                    s[kb][r] = p;
                    ps += p;
                }
            ps += __shfl_xor(ps, 32, 64);
            l_run = l_run * alpha + ps;
            m_run = m_new;
#pragma unroll
            for (int d = 0; d < NDB; d++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[d][r] *= alpha;
            // O^T[d][q] += sum_key V[key][d] * P[q][key]
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = kb * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
#pragma unroll
                    for (int d = 0; d < NDB; d++) {
                        const int dd = d * 32 + lr;
                        float va = (HS >= 32 || dd < HS) ? vs[key * ROW + dd] : 0.f;
                        o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(va, s[kb][r], o[d], 0, 0, 0);
                    }
                }
        }
        if (kt + 1 < ntiles) lstore(cur ^ 1);
        __syncthreads();
    }

    if (qi < T) {
        if (lse && lh == 0) lse[((long)b * H + h) * T + qi] = m_run + log2f(l_run);
        const float inv = 1.0f / l_run;
        float* op = out + ((long)b * T + qi) * C + h * HS;
#pragma unroll
        for (int d = 0; d < NDB; d++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int dd = d * 32 + 8 * g + 4 * lh;  // rows 4g..4g+3 of the block
                if (dd < HS) {
                    f32x4 v = {o[d][4 * g] * inv, o[d][4 * g + 1] * inv, o[d][4 * g + 2] * inv,
                               o[d][4 * g + 3] * inv};
                    *(f32x4*)(op + dd) = v;
                }
            }
    }
}

// k_attn_ks: the same product for launches with too few (sequence, head,
// 128-query) blocks to occupy the CUs evenly (fewer than 512: one sequence
// of up to ~5000 tokens, B=4 T=1024).
// There a block's latency is its last wavefront's chain of matrix-core
// steps over every key up to the diagonal, so a workgroup takes 32 queries
// and its four wavefronts split the keys: wavefront w takes the 32-key
// blocks w, w + 4, .. up to the diagonal, each loaded from global memory
// straight into registers (K rows as the A operand of S^T = K Q^T, V rows
// in the key order of the S^T accumulator for O^T += V^T P^T), the next
// block's loads in flight during the current one. Each wavefront keeps its
// running max m, sum l and O^T as above; the four are merged through LDS
// in wavefront order (O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w,
// M = max_w m_w; a wavefront with no block has m = -inf and adds zero).
//
// With CB > 0 (HS = 64) the workgroup also applies its head's share of the
// c_proj product (reference fast.c:299-303: the head outputs are the k
// range h * 64 .. +63 of that product's inner dimension): a launch has
// C / (64 CB) workgroups per (query block, sequence, head), workgroup slice
// sl owning output columns n0 = 64 CB sl .. +64 CB (16 CB per wavefront);
// it multiplies its merged 32 x 64 head output by W[n0 .. ][h * 64 .. +63]
// (streamed global -> LDS once the key loop is done, under the merge of the
// wavefronts: issued at the start, those loads came before the attention's
// own in the wait counter's order, so every early wait waited for them too)
// and writes the partial sums part[(h * rows + row) * C + n] for the rows
// of x (row = b * T + t); the sum over heads in head order, the bias, the
// residual and the next LayerNorm follow in one launch (launch_sum_heads).
template <int HS, int CB>
__global__ void __launch_bounds__(256, 2)
    k_attn_ks(const float* __restrict__ qkv, long seq_stride, float* __restrict__ out, int B,
              int T, int C, int H, int nqb, float scale, float* __restrict__ lse,
              const float* __restrict__ W, float* __restrict__ part) {
    constexpr int HALF = HS / 2;
    constexpr int NDB = (HS + 31) / 32;
    constexpr int OS = NDB * 32 + 1;  // LDS row of a merged query
    static_assert(CB == 0 || HS == 64, "the fused c_proj takes 64-wide heads");
    constexpr int PS = 68;            // LDS row of a normalised query (fused c_proj)
    __shared__ float om[4][32], ol[4][32];
    __shared__ float oo[4][32 * OS];
    // fused c_proj: this wavefront's CB blocks of 16 weight rows (columns of
    // the output) x 64 k, granule q of row c at slot q ^ c; the normalised
    // head output of the 32 queries
    __shared__ __attribute__((aligned(16))) float wsl[CB ? 4 * CB : 1][CB ? 16 * 64 : 1];
    __shared__ __attribute__((aligned(16))) float on[CB ? 32 * PS : 1];

    const int BH = B * H;
    const int NSL = CB ? C / (64 * CB) : 1;  // column slices per (query block, sequence, head)
    const int qb = nqb - 1 - (int)(blockIdx.x / (BH * NSL));  // longest query blocks first
    const int bh = blockIdx.x % BH;
    const int sl = CB ? (int)(blockIdx.x / BH) % NSL : 0;
    const int b = bh / H, h = bh % H;
    const long C3 = 3L * C;
    const float* base = qkv + (long)b * seq_stride * C3;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 31, lh = lane >> 5;
    const int q0 = qb * 32, qi = q0 + lr;
    const int nkb = min(q0 + 31, T - 1) / 32 + 1;  // key blocks up to the diagonal

    float qreg[HALF];
    {
        const float* qp = base + (long)min(qi, T - 1) * C3 + h * HS + lh * HALF;
        const float qs = scale * 1.4426950408889634f;  // scores in units of log2
#pragma unroll
        for (int d = 0; d < HALF; d += 4) {
            const f32x4 v = *(const f32x4*)(qp + d);
            qreg[d] = v.x * qs; qreg[d + 1] = v.y * qs; qreg[d + 2] = v.z * qs; qreg[d + 3] = v.w * qs;
        }
    }
    // key block kb: K row kb*32 + lr, d in [lh*HALF, +HALF); V rows of the
    // S^T accumulator's keys kb*32 + 8 (r/4) + 4 lh + r%4, d = 32 j + lr
    f32x4 kr[HALF / 4];
    float vr[NDB][16];
    auto load = [&](int kb) {
        const float* kp = base + (long)min(kb * 32 + lr, T - 1) * C3 + C + h * HS + lh * HALF;
#pragma unroll
        for (int d = 0; d < HALF / 4; d++) kr[d] = *(const f32x4*)(kp + 4 * d);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = min(kb * 32 + 8 * (r >> 2) + 4 * lh + (r & 3), T - 1);
            const float* vp = base + (long)key * C3 + 2 * C + h * HS;
#pragma unroll
            for (int j = 0; j < NDB; j++) vr[j][r] = vp[min(32 * j + lr, HS - 1)];
        }
    };

    f32x16 o[NDB];
#pragma unroll
    for (int j = 0; j < NDB; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[j][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    if (wave < nkb) load(wave);
    for (int kb = wave; kb < nkb; kb += 4) {
        f32x4 kc[HALF / 4];
        float vc[NDB][16];
#pragma unroll
        for (int d = 0; d < HALF / 4; d++) kc[d] = kr[d];
#pragma unroll
        for (int j = 0; j < NDB; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) vc[j][r] = vr[j][r];
        if (kb + 4 < nkb) load(kb + 4);
        f32x16 sc;
#pragma unroll
        for (int r = 0; r < 16; r++) sc[r] = 0.f;
#pragma unroll
        for (int d = 0; d < HALF / 4; d++) {
            sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kc[d].x, qreg[4 * d], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kc[d].y, qreg[4 * d + 1], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kc[d].z, qreg[4 * d + 2], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kc[d].w, qreg[4 * d + 3], sc, 0, 0, 0);
        }
        if (kb * 32 + 31 > q0) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = kb * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                sc[r] = (key > qi) ? -INFINITY : sc[r];
            }
        }
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) mt = fmaxf(mt, sc[r]);
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run, mt);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float pr = __builtin_amdgcn_exp2f(sc[r] - m_new);
            sc[r] = pr;
            ps += pr;
        }
        ps += __shfl_xor(ps, 32, 64);
        l_run = l_run * alpha + ps;
        m_run = m_new;
#pragma unroll
        for (int j = 0; j < NDB; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[j][r] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; r++)
#pragma unroll
            for (int j = 0; j < NDB; j++) {
                const float va = (HS >= 32 || 32 * j + lr < HS) ? vc[j][r] : 0.f;
                o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(va, sc[r], o[j], 0, 0, 0);
            }
    }

    if constexpr (CB > 0) {
        // instruction j of block cb: lane i writes row 4 j + i / 16, slot
        // i % 16, which holds granule (i % 16) ^ row of that weight row
        const int wv = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r = 4 * j + (lane >> 4), q = (lane & 15) ^ r;
                const int n = 64 * CB * sl + 16 * (CB * wv + cb) + r;
                lds_dma16(W + (long)n * C + h * 64 + 4 * q, &wsl[CB * wv + cb][256 * j]);
            }
    }
    // o[j][r] = O^T[d = 32 j + 8 (r/4) + 4 lh + r%4][query lr]
    if (lh == 0) {
        om[wave][lr] = m_run;
        ol[wave][lr] = l_run;
    }
#pragma unroll
    for (int j = 0; j < NDB; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int d = 32 * j + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (d < HS) oo[wave][lr * OS + d] = o[j][r];
        }
    __syncthreads();
    for (int i = tid; i < 32 * HS; i += 256) {
        const int q = i / HS, d = i % HS;
        if (q0 + q >= T) {
            if constexpr (CB > 0) {
                // rows past T multiply zeros (their sums are not stored)
                on[q * PS + d] = 0.f;
                continue;
            } else {
                break;
            }
        }
        const float mx = fmaxf(fmaxf(om[0][q], om[1][q]), fmaxf(om[2][q], om[3][q]));
        float l = 0.f, v = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = __builtin_amdgcn_exp2f(om[w][q] - mx);
            l += f * ol[w][q];
            v += f * oo[w][q * OS + d];
        }
        if constexpr (CB > 0) {
            on[q * PS + d] = v / l;
        } else {
            out[((long)b * T + q0 + q) * C + h * HS + d] = v / l;
            if (lse && d == 0) lse[((long)b * H + h) * T + q0 + q] = mx + log2f(l);
        }
    }
    if constexpr (CB > 0) {
        // the weights have landed (the only loads left in flight) and every
        // wavefront's normalised rows are in LDS
        wait_vmcnt<0>();
        __syncthreads();
        // 2 x CB blocks of v_mfma_f32_16x16x4f32: lane (c = lane % 16, g =
        // lane / 16) supplies query row 16 rb + c and weight row 16 cb + c
        // at k = 16 g + 4 t + e of granule step t
        const int lc = lane & 15, g = lane >> 4;
        f32x4 acc[2][CB];
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int cb = 0; cb < CB; cb++) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            f32x4 av[2], bv[CB];
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
                av[rb] = *(const f32x4*)&on[(16 * rb + lc) * PS + 16 * g + 4 * t];
#pragma unroll
            for (int cb = 0; cb < CB; cb++)
                bv[cb] = *(const f32x4*)&wsl[CB * wave + cb][lc * 64 + 4 * ((4 * g + t) ^ lc)];
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int rb = 0; rb < 2; rb++)
#pragma unroll
                    for (int cb = 0; cb < CB; cb++)
                        acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[rb][e], bv[cb][e],
                                                                            acc[rb][cb], 0, 0, 0);
        }
        // acc[rb][cb][r]: query row 16 rb + 4 g + r, output column 16 cb + lc
        // of this wavefront's 16 CB columns of the slice
        const long rows = (long)B * T;
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = q0 + 16 * rb + 4 * g + r;
                if (t >= T) continue;
                float* pr = part + ((long)h * rows + (long)b * T + t) * C + 64 * CB * sl +
                            16 * CB * wave + lc;
#pragma unroll
                for (int cb = 0; cb < CB; cb++) pr[16 * cb] = acc[rb][cb][r];
            }
    }
}

template <int HS>
hipError_t causal_hs(const float* qkv, long seq_stride, float* out, int B, int T, int C, int H,
                     float* lse, hipStream_t s) {
    const int nqb = (T + 127) / 128;
    const float scale = 1.0f / sqrtf((float)HS);
    // (the key split holds a 32-key block of K and V per lane: up to HS = 64)
    if constexpr (HS <= 64) {
        // fewer than two 128-query blocks per CU: measured per forward of
        // 12 layers, B=4 T=1024 (384 blocks) 1.207 -> 1.057 ms with the
        // key split, B=8 T=1024 (768 blocks) 1.609 -> 1.973 ms
        if ((long)nqb * B * H < 512) {
            const int nqb32 = (T + 31) / 32;
            k_attn_ks<HS, 0><<<nqb32 * B * H, 256, 0, s>>>(qkv, seq_stride, out, B, T, C, H,
                                                            nqb32, scale, lse, nullptr, nullptr);
            return hipGetLastError();
        }
    }
    k_attn_causal<HS><<<nqb * B * H, 256, 0, s>>>(qkv, seq_stride, out, B, T, C, H, nqb, scale,
                                                   lse);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attention_causal(const float* qkv, long seq_stride, float* out, int B, int T,
                                   int C, int H, hipStream_t s, float* lse) {
    if (B <= 0 || T <= 0) return hipSuccess;
    switch (C / H) {
        case 8: return causal_hs<8>(qkv, seq_stride, out, B, T, C, H, lse, s);
        case 16: return causal_hs<16>(qkv, seq_stride, out, B, T, C, H, lse, s);
        case 32: return causal_hs<32>(qkv, seq_stride, out, B, T, C, H, lse, s);
        case 64: return causal_hs<64>(qkv, seq_stride, out, B, T, C, H, lse, s);
        case 128: return causal_hs<128>(qkv, seq_stride, out, B, T, C, H, lse, s);
    }
    return hipErrorInvalidValue;
}

int attention_proj_cb(int B, int T, int C, int H) {
    if (H <= 0 || C != 64 * H || B <= 0 || T <= 0) return 0;
    // 16 CB output columns per wavefront: the narrowest of 2, 3 and 4 that
    // divides C into slices and keeps the launch within one workgroup per
    // CU, else the widest within two
    const long qblocks = (long)((T + 31) / 32) * B * H;
    for (int cb = 2; cb <= 4; cb++)
        if (C % (64 * cb) == 0 && qblocks * (C / (64 * cb)) <= 256) return cb;
    for (int cb = 4; cb >= 2; cb--)
        if (C % (64 * cb) == 0 && qblocks * (C / (64 * cb)) <= 512) return cb;
    return 0;
}

hipError_t launch_attention_proj(const float* qkv, long seq_stride, const float* W, float* part,
                                 int B, int T, int C, int H, int CB, hipStream_t s) {
    if (B <= 0 || T <= 0) return hipSuccess;
    if (C != 64 * H || CB < 2 || CB > 4 || C % (64 * CB)) return hipErrorInvalidValue;
    const int nqb32 = (T + 31) / 32;
    const unsigned grid = (unsigned)(nqb32 * B * H * (C / (64 * CB)));
    const float scale = 1.0f / sqrtf(64.0f);
    if (CB == 4)
        k_attn_ks<64, 4><<<grid, 256, 0, s>>>(qkv, seq_stride, nullptr, B, T, C, H, nqb32, scale,
                                              nullptr, W, part);
    else if (CB == 3)
        k_attn_ks<64, 3><<<grid, 256, 0, s>>>(qkv, seq_stride, nullptr, B, T, C, H, nqb32, scale,
                                              nullptr, W, part);
    else
        k_attn_ks<64, 2><<<grid, 256, 0, s>>>(qkv, seq_stride, nullptr, B, T, C, H, nqb32, scale,
                                              nullptr, W, part);
    return hipGetLastError();
}
