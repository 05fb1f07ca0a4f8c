// attn_bwd.hip - backward of the causal attention (reference
// gpt_backward, src/model.c:747-818) on gfx950.
//
// The reference keeps every probability plane P = softmax(mask(scale Q
// K^T)) from the forward and forms, per (sequence, head), dV = P^T dO, dP =
// dO V^T, dS = P (dP - D) with D_q = sum_k P_qk dP_qk, dQ = scale dS K and
// dK = scale dS^T Q, all T x T. Here no T x T plane exists: the forward
// leaves the base-2 log-sum-exp of each query's scaled scores (lse), P is
// recomputed in 32 x 32 blocks as exp2(q.k scale log2(e) - lse), and D_q =
// dO_q . O_q (equal to sum_k P_qk dP_qk, since O_q = sum_k P_qk V_k).
// Blocks above the diagonal are skipped, keys after a query masked.
//
// k_attn_bwd_kv: one workgroup = four wavefronts = 128 keys of one
// (sequence, head); a wavefront holds its 32 keys' K (pre-scaled by scale
// log2(e)) and V rows in registers and walks the query blocks from the
// diagonal on, the block's Q, dO, lse and D staged in LDS for all four. S =
// Q K^T and dP = dO V^T come out of v_mfma_f32_32x32x2f32 with a lane per
// key, so P and dS sit in the accumulator with the k order that the next
// products need: dV += P^T dO and dK += dS^T Q take them as the A operand
// straight from the registers, dO and Q rows as the B operand from LDS.
//
// k_attn_bwd_q: one workgroup = 128 queries; a wavefront holds its 32
// queries' Q (pre-scaled) and dO rows, lse and D, walks the key blocks up
// to the diagonal with K and V staged in LDS, forms S^T = K Q^T and dP^T =
// V dO^T with a lane per query, and dQ^T += K^T dS^T with dS^T as the B
// operand from the accumulator. Both kernels write whole columns of the
// qkv gradient (dQ, dK, dV of their head).
//
// Causal walks differ in length (a key block near the start meets every
// query block after it, one near the end only its own), so with few blocks
// per CU the longest walks set the time: at B=4 T=1024, 384 workgroups of
// 4 to 32 block pairs, the busiest CUs held 44 block pairs against an
// average of 27. With fewer than 1024 walks each walk is split in two
// halves (split = 2), twice the workgroups, longest first; both halves add
// their part into the gradient, zeroed first. Two additions onto zero give
// the same bits in either order (x + y = y + x), so the result stays
// reproducible.
#include "common.h"
#include "kernels.h"

namespace {

constexpr float LOG2E = 1.4426950408889634f;

// D[(b * H + h) * T + t] = dO[b, t, head h] . O[b, t, head h]
__global__ void __launch_bounds__(256) k_attn_bwd_d(const float* __restrict__ dout,
                                                    const float* __restrict__ out, int B, int T,
                                                    int C, int H, float* __restrict__ D) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)B * T * H) return;
    const int h = (int)(i % H);
    const long bt = i / H;
    const int hs = C / H;
    const f32x4* a = (const f32x4*)(dout + bt * C + h * hs);
    const f32x4* o = (const f32x4*)(out + bt * C + h * hs);
    float s = 0.f;
    for (int d = 0; d < hs / 4; d++) {
        const f32x4 p = a[d] * o[d];
        s += (p.x + p.y) + (p.z + p.w);
    }
    const int b = (int)(bt / T), t = (int)(bt % T);
    D[((long)b * H + h) * T + t] = s;
}

template <int HS>
struct BwdShape {
    static constexpr int HALF = HS / 2;          // d values per lane half in the q.k products
    static constexpr int ROW = HS + 4;           // padded LDS row
    static constexpr int NDB = (HS + 31) / 32;   // 32-wide d blocks of dK, dV, dQ
    static constexpr int F4 = HS / 4;            // float4 per head row
    static constexpr int LIT = (32 * F4 + 255) / 256;  // float4 per thread to stage 32 rows
};

// Zero n float4 (the gradient the split walks add into).
__global__ void __launch_bounds__(256) k_zero4(f32x4* __restrict__ p, long n) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// The [lo, hi) range of a walk of n blocks that half `part` of `split`
// covers (the first half takes the extra block).
__device__ __forceinline__ void walk_part(int n, int split, int part, int& lo, int& hi) {
    const int mid = split == 2 ? (n + 1) / 2 : n;
    lo = part == 0 ? 0 : mid;
    hi = part == 0 ? mid : n;
}

template <int HS, int OCC>
__global__ void __launch_bounds__(256, OCC)
    k_attn_bwd_kv(const float* __restrict__ qkv, const float* __restrict__ dout,
                  const float* __restrict__ lse, const float* __restrict__ Dv,
                  float* __restrict__ dqkv, int B, int T, int C, int H, int nkb, float scale,
                  int split) {
    using S_ = BwdShape<HS>;
    constexpr int HALF = S_::HALF, ROW = S_::ROW, NDB = S_::NDB, F4 = S_::F4, LIT = S_::LIT;
    __shared__ float Qs[2][32 * ROW], Os[2][32 * ROW];
    __shared__ float Ls[2][32], Ds[2][32];

    const int BH = B * H;
    const int w = (int)(blockIdx.x / BH);  // walk part: the longest walks first
    const int kb = w / split;              // key block of 128
    const int bh = blockIdx.x % BH;
    const int b = bh / H, h = bh % H;
    const long C3 = 3L * C;
    const float* base = qkv + (long)b * T * C3;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 31, lh = lane >> 5;
    const int key0 = kb * 128 + wave * 32;
    const int key = key0 + lr;  // this lane's key (S columns, dK / dV rows are 32 per block)

    float kreg[HALF], vreg[HALF];
    {
        const float* kp = base + (long)min(key, T - 1) * C3 + C + h * HS + lh * HALF;
        const float c2 = scale * LOG2E;
#pragma unroll
        for (int d = 0; d < HALF; d += 4) {
            const f32x4 kv = *(const f32x4*)(kp + d);
            const f32x4 vv = *(const f32x4*)(kp + C + d);
            kreg[d] = kv.x * c2; kreg[d + 1] = kv.y * c2; kreg[d + 2] = kv.z * c2; kreg[d + 3] = kv.w * c2;
            vreg[d] = vv.x; vreg[d + 1] = vv.y; vreg[d + 2] = vv.z; vreg[d + 3] = vv.w;
        }
    }

    // stage query block qb (Q rows, dO rows, lse, D) into buffer buf
    f32x4 rq[LIT], ro[LIT];
    float rl = 0.f, rd = 0.f;
    auto gload = [&](int qb) {
#pragma unroll
        for (int i = 0; i < LIT; i++) {
            const int idx = tid + 256 * i;
            if (idx < 32 * F4) {
                const int q = min(qb * 32 + idx / F4, T - 1), c = (idx % F4) * 4;
                rq[i] = *(const f32x4*)(base + (long)q * C3 + h * HS + c);
                ro[i] = *(const f32x4*)(dout + ((long)b * T + q) * C + h * HS + c);
            }
        }
        if (tid < 32) {
            const int q = min(qb * 32 + tid, T - 1);
            rl = lse[(long)bh * T + q];
            rd = Dv[(long)bh * T + q];
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LIT; i++) {
            const int idx = tid + 256 * i;
            if (idx < 32 * F4) {
                const int o = (idx / F4) * ROW + (idx % F4) * 4;
                *(f32x4*)&Qs[buf][o] = rq[i];
                *(f32x4*)&Os[buf][o] = ro[i];
            }
        }
        if (tid < 32) {
            Ls[buf][tid] = rl;
            Ds[buf][tid] = rd;
        }
    };

    f32x16 dk[NDB], dv[NDB];
#pragma unroll
    for (int j = 0; j < NDB; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) dk[j][r] = dv[j][r] = 0.f;

    const int nqb = (T + 31) / 32;
    // query blocks from the first that meets this workgroup's keys, or this
    // part of them
    int qb0, qb1;
    walk_part(max(nqb - kb * 4, 0), split, w % split, qb0, qb1);
    qb0 += kb * 4;
    qb1 += kb * 4;
    if (qb0 < qb1) {
        gload(qb0);
        lstore(0);
    }
    __syncthreads();
    for (int qb = qb0; qb < qb1; qb++) {
        const int cur = (qb - qb0) & 1;
        if (qb + 1 < qb1) gload(qb + 1);
        // wave-uniform: the block holds a query at or after this wavefront's first key
        if (key0 < T && qb * 32 + 31 >= key0) {
            const float* qs = Qs[cur];
            const float* os = Os[cur];
            f32x16 sc, dp;
#pragma unroll
            for (int r = 0; r < 16; r++) sc[r] = dp[r] = 0.f;
#pragma unroll
            for (int d = 0; d < HALF; d += 4) {
                const f32x4 qv = *(const f32x4*)&qs[lr * ROW + lh * HALF + d];
                const f32x4 ov = *(const f32x4*)&os[lr * ROW + lh * HALF + d];
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.x, kreg[d], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.y, kreg[d + 1], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.z, kreg[d + 2], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.w, kreg[d + 3], sc, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.x, vreg[d], dp, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.y, vreg[d + 1], dp, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.z, vreg[d + 2], dp, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.w, vreg[d + 3], dp, 0, 0, 0);
            }
            // sc[r], dp[r]: query qb*32 + qr(r), key `key`, qr(r) = 8 (r/4) + 4 lh + r%4
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int qr = 8 * (r >> 2) + 4 * lh + (r & 3);
                const int q = qb * 32 + qr;
                const float p = (key > q || q >= T) ? 0.f
                                                    : __builtin_amdgcn_exp2f(sc[r] - Ls[cur][qr]);
                sc[r] = p;
                dp[r] = p * (dp[r] - Ds[cur][qr]);
            }
            // dV[key][d] += sum_q P[q][key] dO[q][d]; dK[key][d] += sum_q dS[q][key] Q[q][d]
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int qr = 8 * (r >> 2) + 4 * lh + (r & 3);
#pragma unroll
                for (int j = 0; j < NDB; j++) {
                    const int dd = 32 * j + lr;
                    const float ob = (HS >= 32 || dd < HS) ? os[qr * ROW + dd] : 0.f;
                    const float qb_ = (HS >= 32 || dd < HS) ? qs[qr * ROW + dd] : 0.f;
                    dv[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(sc[r], ob, dv[j], 0, 0, 0);
                    dk[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(dp[r], qb_, dk[j], 0, 0, 0);
                }
            }
        }
        if (qb + 1 < qb1) lstore(cur ^ 1);
        __syncthreads();
    }

    // dk[j][r], dv[j][r]: key key0 + 8 (r/4) + 4 lh + r%4, d = 32 j + lr
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int kk = key0 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (kk >= T) continue;
        float* row = dqkv + ((long)b * T + kk) * C3 + h * HS;
#pragma unroll
        for (int j = 0; j < NDB; j++) {
            const int dd = 32 * j + lr;
            if (HS >= 32 || dd < HS) {
                if (split == 1) {
                    row[C + dd] = dk[j][r] * scale;
                    row[2 * C + dd] = dv[j][r];
                } else {
                    unsafeAtomicAdd(row + C + dd, dk[j][r] * scale);
                    unsafeAtomicAdd(row + 2 * C + dd, dv[j][r]);
                }
            }
        }
    }
}

template <int HS, int OCC>
__global__ void __launch_bounds__(256, OCC)
    k_attn_bwd_q(const float* __restrict__ qkv, const float* __restrict__ dout,
                 const float* __restrict__ lse, const float* __restrict__ Dv,
                 float* __restrict__ dqkv, int B, int T, int C, int H, int nqb, float scale,
                 int split) {
    using S_ = BwdShape<HS>;
    constexpr int HALF = S_::HALF, ROW = S_::ROW, NDB = S_::NDB, F4 = S_::F4, LIT = S_::LIT;
    // K and V stages; after the walk, each wavefront's dQ rows (32 x HS + 1)
    __shared__ float kvs[4 * 32 * ROW];
    float (*Ks)[32 * ROW] = (float (*)[32 * ROW])kvs;
    float (*Vs)[32 * ROW] = (float (*)[32 * ROW])(kvs + 2 * 32 * ROW);
    static_assert(4 * 32 * (HS + 1) <= 4 * 32 * ROW, "dQ rows fit the stages");

    const int BH = B * H;
    const int w = (int)(blockIdx.x / BH);  // walk part: the longest walks first
    const int qbk = nqb - 1 - w / split;   // query block of 128
    const int bh = blockIdx.x % BH;
    const int b = bh / H, h = bh % H;
    const long C3 = 3L * C;
    const float* base = qkv + (long)b * T * C3;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 31, lh = lane >> 5;
    const int q0 = qbk * 128 + wave * 32;
    const int qi = q0 + lr;

    float qreg[HALF], oreg[HALF];
    float lq, dq;
    {
        const int qc = min(qi, T - 1);
        const float* qp = base + (long)qc * C3 + h * HS + lh * HALF;
        const float* op = dout + ((long)b * T + qc) * C + h * HS + lh * HALF;
        const float c2 = scale * LOG2E;
#pragma unroll
        for (int d = 0; d < HALF; d += 4) {
            const f32x4 qv = *(const f32x4*)(qp + d);
            const f32x4 ov = *(const f32x4*)(op + d);
            qreg[d] = qv.x * c2; qreg[d + 1] = qv.y * c2; qreg[d + 2] = qv.z * c2; qreg[d + 3] = qv.w * c2;
            oreg[d] = ov.x; oreg[d + 1] = ov.y; oreg[d + 2] = ov.z; oreg[d + 3] = ov.w;
        }
        lq = lse[(long)bh * T + qc];
        dq = Dv[(long)bh * T + qc];
    }

    f32x4 rk[LIT], rv[LIT];
    auto gload = [&](int kb) {
#pragma unroll
        for (int i = 0; i < LIT; i++) {
            const int idx = tid + 256 * i;
            if (idx < 32 * F4) {
                const int k = min(kb * 32 + idx / F4, T - 1), c = (idx % F4) * 4;
                const float* rp = base + (long)k * C3 + h * HS + c;
                rk[i] = *(const f32x4*)(rp + C);
                rv[i] = *(const f32x4*)(rp + 2 * C);
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LIT; i++) {
            const int idx = tid + 256 * i;
            if (idx < 32 * F4) {
                const int o = (idx / F4) * ROW + (idx % F4) * 4;
                *(f32x4*)&Ks[buf][o] = rk[i];
                *(f32x4*)&Vs[buf][o] = rv[i];
            }
        }
    };

    f32x16 dqa[NDB];
#pragma unroll
    for (int j = 0; j < NDB; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) dqa[j][r] = 0.f;

    // key blocks up to the diagonal, or this part of them
    int kb0, kb1;
    walk_part(min(qbk * 128 + 127, T - 1) / 32 + 1, split, w % split, kb0, kb1);
    if (kb0 < kb1) {
        gload(kb0);
        lstore(0);
    }
    __syncthreads();
    for (int kb = kb0; kb < kb1; kb++) {
        const int cur = (kb - kb0) & 1;
        if (kb + 1 < kb1) gload(kb + 1);
        if (q0 < T && kb * 32 <= q0 + 31) {
            const float* ks = Ks[cur];
            const float* vs = Vs[cur];
            f32x16 sc, dp;
#pragma unroll
            for (int r = 0; r < 16; r++) sc[r] = dp[r] = 0.f;
#pragma unroll
            for (int d = 0; d < HALF; d += 4) {
                const f32x4 kv = *(const f32x4*)&ks[lr * ROW + lh * HALF + d];
                const f32x4 vv = *(const f32x4*)&vs[lr * ROW + lh * HALF + d];
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qreg[d], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qreg[d + 1], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qreg[d + 2], sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qreg[d + 3], sc, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, oreg[d], dp, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, oreg[d + 1], dp, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, oreg[d + 2], dp, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, oreg[d + 3], dp, 0, 0, 0);
            }
            // sc[r], dp[r]: key kb*32 + kr(r), query qi, kr(r) = 8 (r/4) + 4 lh + r%4
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int kr = 8 * (r >> 2) + 4 * lh + (r & 3);
                const float p = (kb * 32 + kr > qi) ? 0.f : __builtin_amdgcn_exp2f(sc[r] - lq);
                dp[r] = p * (dp[r] - dq);
            }
            // dQ^T[d][q] += sum_key K[key][d] dS^T[key][q]
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int kr = 8 * (r >> 2) + 4 * lh + (r & 3);
#pragma unroll
                for (int j = 0; j < NDB; j++) {
                    const int dd = 32 * j + lr;
                    const float ka = (HS >= 32 || dd < HS) ? ks[kr * ROW + dd] : 0.f;
                    dqa[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka, dp[r], dqa[j], 0, 0, 0);
                }
            }
        }
        if (kb + 1 < kb1) lstore(cur ^ 1);
        __syncthreads();
    }

    // dqa[j][r]: d = 32 j + 8 (r/4) + 4 lh + r%4, query qi
    if (split == 1) {
        if (qi < T) {
            float* row = dqkv + ((long)b * T + qi) * C3 + h * HS;
#pragma unroll
            for (int j = 0; j < NDB; j++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int dd = 32 * j + 8 * g + 4 * lh;
                    if (dd < HS)
                        *(f32x4*)(row + dd) =
                            f32x4{dqa[j][4 * g] * scale, dqa[j][4 * g + 1] * scale,
                                  dqa[j][4 * g + 2] * scale, dqa[j][4 * g + 3] * scale};
                }
        }
        return;
    }
    // A half walk adds its part. A lane holds one query's d values, so the
    // rows go through LDS first (the stages are free after the walk's last
    // barrier): each addition instruction then covers one row's contiguous
    // d instead of 64 rows.
    constexpr int P = HS + 1;
    float* tq = kvs + wave * 32 * P;
#pragma unroll
    for (int j = 0; j < NDB; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int dd = 32 * j + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (dd < HS) tq[lr * P + dd] = dqa[j][r] * scale;
        }
    __builtin_amdgcn_wave_barrier();
    for (int d = lane; d < HS; d += 64)
        for (int q = 0; q < 32 && q0 + q < T; q++)
            unsafeAtomicAdd(dqkv + ((long)b * T + q0 + q) * C3 + h * HS + d, tq[q * P + d]);
}

template <int HS, int OCC>
hipError_t bwd_hs(const float* qkv, const float* out, const float* dout, const float* lse,
                  float* D, float* dqkv, int B, int T, int C, int H, hipStream_t s) {
    const float scale = 1.0f / sqrtf((float)HS);
    const long n = (long)B * T * H;
    k_attn_bwd_d<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(dout, out, B, T, C, H, D);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nb = (T + 127) / 128;
    const int split = (long)nb * B * H < 1024 ? 2 : 1;
    if (split == 2) {
        // the halves add into the gradient rows of every (sequence, position)
        const long n4 = (long)B * T * 3 * C / 4;
        k_zero4<<<(unsigned)((n4 + 255) / 256), 256, 0, s>>>((f32x4*)dqkv, n4);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    k_attn_bwd_kv<HS, OCC><<<split * nb * B * H, 256, 0, s>>>(qkv, dout, lse, D, dqkv, B, T, C,
                                                              H, nb, scale, split);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_attn_bwd_q<HS, OCC><<<split * nb * B * H, 256, 0, s>>>(qkv, dout, lse, D, dqkv, B, T, C, H,
                                                             nb, scale, split);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attention_bwd(const float* qkv, const float* out, const float* dout,
                                const float* lse, float* D, float* dqkv, int B, int T, int C,
                                int H, hipStream_t s) {
    if (B <= 0 || T <= 0) return hipSuccess;
    switch (C / H) {
        case 8: return bwd_hs<8, 2>(qkv, out, dout, lse, D, dqkv, B, T, C, H, s);
        case 16: return bwd_hs<16, 2>(qkv, out, dout, lse, D, dqkv, B, T, C, H, s);
        case 32: return bwd_hs<32, 2>(qkv, out, dout, lse, D, dqkv, B, T, C, H, s);
        case 64: return bwd_hs<64, 2>(qkv, out, dout, lse, D, dqkv, B, T, C, H, s);
        case 128: return bwd_hs<128, 1>(qkv, out, dout, lse, D, dqkv, B, T, C, H, s);
    }
    return hipErrorInvalidValue;
}
