// persist.hip - single-sequence decode steps as one persistent kernel.
//
// A decode step is a chain of dependent stages: per layer LayerNorm 1 +
// QKV, attention over the cache, merge + c_proj + residual, LayerNorm 2 +
// fc + GELU, proj + residual; then the final LayerNorm + lm_head and the
// argmax (reference fast.c:245-329 at T = 1, with the KV cache). Launched
// as separate kernels, every stage pays a kernel boundary plus the HBM
// latency of its weights. Here the stages are phases of one cooperative
// launch (one workgroup per CU) separated by grid barriers, and since no
// weight depends on the data, each workgroup loads the next phase's weights
// into registers as soon as the current phase's products are done: that
// traffic overlaps the barrier. One launch runs any number of greedy steps
// (the argmax of step s is the input of step s+1 without leaving the GPU).
//
// Workgroup: PW compute wavefronts + 1 control wavefront. The compute
// wavefronts hold weights and form dot products; the control wavefront
// sums their per-unit results in a fixed order, applies the epilogue,
// stores, and runs the barrier (its own loads never wait behind weight
// prefetches, which matters because loads complete in order).
//
// Grid barrier: each workgroup adds 1 (no return value) to the counter of
// its XCD (blockIdx % 8); the control wavefront then polls all 8 counters
// with 8 lanes until each reaches epoch * (workgroups per XCD). A poll
// limit turns a stall into an error flag every workgroup sees and exits on.
//
// Coherence: the L2 of an XCD is not coherent with the others. Values made
// and used inside the launch (x, hid, K/V/q row t, attention and argmax
// partials) are stored and loaded with agent-scope atomics (sc1: through to
// memory), and a producer waits for its stores to complete before it
// arrives. Weights, and cache rows from before the launch or from earlier
// steps (never read before they were written), use plain loads.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace {

constexpr int PW = 7;                  // compute wavefronts per workgroup
constexpr int PT = (PW + 1) * 64;      // + the control wavefront: 2 per SIMD
constexpr int NGRP = 8;                // barrier counters, one per XCD
constexpr int CSTR = 32;               // counters 128 bytes apart
constexpr int UPW = 4;                 // output columns per wavefront per phase
constexpr int KPW = 16;                // attention keys per wavefront
constexpr int LNE = 4;                 // LayerNorm elements per thread (C <= 4 * PT)
constexpr int PMAXS = 16;              // attention splits per head
constexpr long SPIN_LIMIT = 1L << 22;  // polls before a barrier gives up
// Widths up to 256 * PMAXU channels (GPT-2 small and medium): the weights a
// lane holds for one phase (UPW * U float4, U = ceil(C / 256)) then fit in
// registers beside the rest; wider models take the kernel-per-stage decode.
constexpr int PMAXU = 4;

__device__ __forceinline__ float ld_sc(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_sc(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_sc(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_sc(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_sc(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Loads through the global address space: pointers taken from the layer
// table are generic, and generic (flat) loads make the compiler wait for
// them at the next control-flow join.
typedef __attribute__((address_space(1))) const float gfloat;
typedef __attribute__((address_space(1))) const f32x4 gf32x4;
__device__ __forceinline__ float ldg(const float* p) { return *(gfloat*)p; }
__device__ __forceinline__ f32x4 ldg4(const float* p) { return *(gf32x4*)p; }

// Wait until this wavefront's stores have completed.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Values the compiler must treat as unknown at each use: keeps it from
// hoisting every phase's (loop-invariant) column indices and lane offsets
// out of the step loop, where they would stay live and spill.
__device__ __forceinline__ int opaque_s(int v) {
    asm volatile("" : "+s"(v));
    return v;
}
__device__ __forceinline__ int opaque_v(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ float dot4(f32x4 a, f32x4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

template <int U>
struct Smem {
    f32x4 act[256 * U];           // activation vector (up to 1024 * U floats)
    float red[UPW][PW];           // per-wavefront column sums
    float wred[PW + 1];           // block reductions
    float attn[PW][68];           // per-wavefront attention partials: m, l, -, -, o[64]
    float qkv_new[3][64];         // q, k, v of row t for this workgroup's head
    float ml[2][32 * PMAXS];      // m and l of every (head, split)
    float bestv[PW + 1];
    int besti[PW + 1];
    int abort;
};

// Sum over the workgroup, same value in every thread.
__device__ __forceinline__ float block_sum(float v, float* wred, int wave, int lane) {
    v = wave_sum(v);
    if (lane == 0) wred[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PW + 1; i++) s += wred[i];
    __syncthreads();
    return s;
}

// LayerNorm (reference ops.c:191-248) of v (element tid + PT * i) into act.
__device__ __forceinline__ void ln_to_act(const float (&v)[LNE], const float (&lw)[LNE],
                                          const float (&lb)[LNE], int C, float* act, float* wred,
                                          int tid, int wave, int lane) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < LNE; i++)
        if (tid + PT * i < C) s += v[i];
    const float mean = block_sum(s, wred, wave, lane) / (float)C;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < LNE; i++)
        if (tid + PT * i < C) {
            const float d = v[i] - mean;
            q += d * d;
        }
    const float rstd = 1.0f / sqrtf(block_sum(q, wred, wave, lane) / (float)C + 1e-5f);
#pragma unroll
    for (int i = 0; i < LNE; i++) {
        const int e = tid + PT * i;
        if (e < C) act[e] = (v[i] - mean) * rstd * lw[i] + lb[i];
    }
    __syncthreads();
}

// Columns of a product Y[N] = W[N, K] . act: column cw + CW * j (j < NJ)
// belongs to compute wavefront cw; its lane l holds float4 i * 64 + l
// (i < NI) of the column's weight row in w[j * NI + i].
template <int NJ, int NI, int NW>
__device__ __forceinline__ void load_cols(f32x4 (&w)[NW], const float* __restrict__ W, int N,
                                          int K, int cw, int CW, int lane) {
    static_assert(NJ * NI <= NW, "register budget");
    cw = opaque_s(cw);
    lane = opaque_v(lane);
    const int K4 = K >> 2;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int c = cw + CW * j;
        if (c < N) {
            const float* row = W + (long)c * K;
#pragma unroll
            for (int i = 0; i < NI; i++) w[j * NI + i] = ldg4(row + 4 * min(i * 64 + lane, K4 - 1));
        } else {
            // written on every path, so the previous phase's values are dead
#pragma unroll
            for (int i = 0; i < NI; i++) w[j * NI + i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
}

template <int NJ, int NI, int NW>
__device__ __forceinline__ void col_dots(float (&acc)[UPW], const f32x4 (&w)[NW],
                                         const f32x4* act, int N, int K, int cw, int CW,
                                         int lane) {
    cw = opaque_s(cw);
    lane = opaque_v(lane);
    const int K4 = K >> 2;
#pragma unroll
    for (int j = 0; j < UPW; j++) {
        float s = 0.f;
        if (j < NJ && cw + CW * j < N) {
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int f = i * 64 + lane;
                if (f < K4) s += dot4(w[j * NI + i], act[f]);
            }
        }
        acc[j] = s;
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[j] = wave_sum(acc[j]);
}

// Column of control-wavefront lane `slot` (or -1): round j = slot / PW of
// compute wavefront slot % PW of this workgroup.
__device__ __forceinline__ int slot_col(int slot, int N, int CW, int& j, int& q) {
    j = slot / PW;
    q = slot - j * PW;
    if (j >= UPW) return -1;
    const int c = CW * j + blockIdx.x * PW + q;
    return c < N ? c : -1;
}

template <int U>
__global__ void __launch_bounds__(PT, 1) k_decode_persist(PersistArgs a) {
    constexpr int NW = UPW * U;  // weight registers (float4) per lane
    __shared__ Smem<U> sm;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const bool ctrl = wave == PW;
    const int G = gridDim.x;
    const int CW = PW * G;
    // compute wavefront id; the control wavefront gets one past every
    // column, so the loads below skip it but still write its registers (a
    // register array left unwritten on the control path would stay live
    // across every phase)
    const int cw0 = ctrl ? (1 << 29) : blockIdx.x * PW + wave;
    const int C = a.C, C3 = 3 * C, C4 = 4 * C, H = a.H, V = a.V;
    float* actf = (float*)sm.act;
    unsigned epoch = 0;

    if (tid == 0) sm.abort = 0;
    __syncthreads();

    // Grid barrier. Called by every thread; the control wavefront has
    // waited for its stores.
    auto barrier = [&]() -> bool {
        __syncthreads();
        if (ctrl) {
            ++epoch;
            if (lane == 0)
                __hip_atomic_fetch_add(a.bar + (blockIdx.x % NGRP) * CSTR, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            const unsigned target = epoch * (unsigned)(G / NGRP);
            long it = 0;
            bool bad = false;
            while (true) {
                const unsigned v = lane < NGRP ? ld_sc(a.bar + lane * CSTR) : target;
                if (__all(v >= target)) break;
                if ((++it & 63) == 0 && (ld_sc(a.bar + NGRP * CSTR) != 0u || it > SPIN_LIMIT)) {
                    bad = true;
                    break;
                }
            }
            if (bad && lane == 0) {
                __hip_atomic_fetch_or(a.bar + NGRP * CSTR, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
                if (a.err) atomicOr(a.err, 2);
                sm.abort = 1;
            }
        }
        __syncthreads();
        return sm.abort == 0;
    };

    int t = *a.pos;
    int tok = *a.tok;
    f32x4 w[NW];
    f32x4 kq[4];             // attention prefetch: K, 16 dims of one key
    float vr[KPW];           // V of 16 keys, one dim
    float xv[LNE];           // LayerNorm input
    float lw[LNE], lb[LNE];  // gains and biases of the next LayerNorm
    float bo = 0.f;          // control lanes: bias of the next output column

    // Loads below are unconditional with clamped indices: a load under a
    // divergent branch makes the compiler wait for it inside the branch,
    // which serialises the loads of a phase.
    auto ln_params = [&](const float* gw, const float* gb) {
        const int tt = opaque_v(tid);
#pragma unroll
        for (int i = 0; i < LNE; i++) {
            const int e = min(tt + PT * i, C - 1);
            lw[i] = ldg(gw + e);
            lb[i] = ldg(gb + e);
        }
    };
    auto load_x = [&]() {
        const int tt = opaque_v(tid);
#pragma unroll
        for (int i = 0; i < LNE; i++) xv[i] = ld_sc(a.x + min(tt + PT * i, C - 1));
    };
    // Bias of this lane's output column in the next phase (control lanes;
    // the others load b[0]). Issued by every wavefront before the current
    // epilogue, so it completes under that epilogue's store wait.
    auto slot_bias = [&](const float* b, int N) -> float {
        int j, q;
        return ldg(b + max(slot_col(opaque_v(lane), N, CW, j, q), 0));
    };

    const LayerW* layers = a.layers;
    load_cols<UPW, U>(w, layers[0].attn_w, C3, C, cw0, CW, lane);
    ln_params(layers[0].ln1_w, layers[0].ln1_b);
    bo = slot_bias(layers[0].attn_b, C3);

    for (int step = 0; step < a.n_steps; step++, t++) {
        // opaque copies per iteration (see opaque_s)
        const int lane1 = opaque_v(lane), cw1 = opaque_s(cw0);
        const int cw = cw1;
        // ---------------- embedding x = wte[tok] + wpe[t] (fast.c:245-254)
        if (tok < 0 || tok >= V) {
            if (tid == 0 && a.err) atomicOr(a.err, 1);
            tok = tok < 0 ? 0 : V - 1;
        }
        {
            const float* er = a.wte + (long)tok * C;
            const float* pr = a.wpe + (long)t * C;
#pragma unroll
            for (int i = 0; i < LNE; i++) {
                const int e = min(tid + PT * i, C - 1);
                xv[i] = ldg(er + e) + ldg(pr + e);
            }
            if (blockIdx.x == 0) {
#pragma unroll
                for (int i = 0; i < LNE; i++)
                    if (tid + PT * i < C) st_sc(a.x + tid + PT * i, xv[i]);
                if (tid == 0) a.hist[t] = tok;
            }
        }

        for (int l = 0; l < a.L; l++) {
            const int lane = opaque_v(lane1), cw = opaque_s(cw1);
            const LayerW P = layers[l];
            const LayerW PN = layers[min(l + 1, a.L - 1)];
            float* kvl = a.cache + (long)l * a.cap * C3;
            float* rowt = kvl + (long)t * C3;

            // ---------------- phase A: LayerNorm 1 + QKV into cache row t
            if (l > 0) load_x();
            ln_to_act(xv, lw, lb, C, actf, sm.wred, tid, wave, lane);
            if (!ctrl) {
                float acc[UPW];
                col_dots<UPW, U>(acc, w, sm.act, C3, C, cw, CW, lane);
                if (lane == 0)
#pragma unroll
                    for (int j = 0; j < UPW; j++) sm.red[j][wave] = acc[j];
            }
            // attention split layout for keys 0..t
            const int nk = t + 1;
            int ns = (nk + 63) / 64;
            ns = min(ns, min(G / H, PMAXS));
            const int kps = (nk + ns - 1) / ns;
            const int kpw = (kps + PW - 1) / PW;
            const bool has_item = blockIdx.x < H * ns;
            const int ih = blockIdx.x / ns, isp = blockIdx.x - (blockIdx.x / ns) * ns;
            const int k0 = isp * kps, k1 = min(k0 + kps, nk);
            const int kw0 = k0 + wave * kpw, kw1 = min(kw0 + kpw, k1);
            __syncthreads();
            {
                const float bn = slot_bias(P.proj_b, C);
                if (ctrl) {
                    int j, q;
                    const int c = slot_col(lane, C3, CW, j, q);
                    if (c >= 0) st_sc(rowt + c, sm.red[j][q] + bo);
                    wait_stores();
                }
                bo = bn;
            }
            if (!ctrl && has_item) {
                // prefetch this wavefront's cached keys (< t) of head ih
                const int kk = kw0 + (lane >> 2), dq = lane & 3;
                const int kc = min(kk, max(t - 1, 0));
                const float* kr = kvl + (long)kc * C3 + C + ih * 64 + dq * 16;
#pragma unroll
                for (int i = 0; i < 4; i++) kq[i] = ldg4(kr + 4 * i);
#pragma unroll
                for (int jj = 0; jj < KPW; jj++) {
                    const int kj = min(kw0 + jj, max(t - 1, 0));
                    vr[jj] = ldg(kvl + (long)kj * C3 + 2 * C + ih * 64 + lane);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) kq[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int jj = 0; jj < KPW; jj++) vr[jj] = 0.f;
            }
            if (!barrier()) return;

            // ---------------- phase B: attention, one (head, key split) per workgroup
            if (ctrl && has_item) {
                // all three loads before the LDS stores (atomic loads are
                // not reordered past other memory operations)
                float nv[3];
#pragma unroll
                for (int m = 0; m < 3; m++) nv[m] = ld_sc(rowt + m * C + ih * 64 + lane);
#pragma unroll
                for (int m = 0; m < 3; m++) sm.qkv_new[m][lane] = nv[m];
            }
            __syncthreads();
            if (!ctrl && has_item) {
                const int kk = kw0 + (lane >> 2), dq = lane & 3;
                const bool valid = kk < kw1;
                const f32x4* qn = (const f32x4*)&sm.qkv_new[0][dq * 16];
                const f32x4* kn = (const f32x4*)&sm.qkv_new[1][dq * 16];
                float d = 0.f;
#pragma unroll
                for (int i = 0; i < 4; i++) d += dot4(qn[i], kk == t ? kn[i] : kq[i]);
                d += __shfl_xor(d, 1, 64);
                d += __shfl_xor(d, 2, 64);
                const float sc = valid ? d * a.scale : -INFINITY;
                const float m = wave_max(sc);
                const float e = valid ? expf(sc - m) : 0.f;
                const float ls = wave_sum(dq == 0 ? e : 0.f);
                float o = 0.f;
#pragma unroll
                for (int jj = 0; jj < KPW; jj++) {
                    const float pj = __shfl(e, 4 * jj, 64);
                    const int kj = kw0 + jj;
                    if (kj < kw1) o += pj * (kj == t ? sm.qkv_new[2][lane] : vr[jj]);
                }
                if (lane == 0) {
                    sm.attn[wave][0] = m;
                    sm.attn[wave][1] = ls;
                }
                sm.attn[wave][4 + lane] = o;
            }
            __syncthreads();
            if (ctrl) {
                if (has_item) {
                    float M = -INFINITY;
#pragma unroll
                    for (int v = 0; v < PW; v++) M = fmaxf(M, sm.attn[v][0]);
                    float L = 0.f, O = 0.f;
#pragma unroll
                    for (int v = 0; v < PW; v++) {
                        const float mv = sm.attn[v][0];
                        const float f = mv == -INFINITY ? 0.f : expf(mv - M);
                        L += sm.attn[v][1] * f;
                        O += sm.attn[v][4 + lane] * f;
                    }
                    float* part = a.apart + ((long)ih * PMAXS + isp) * 68;
                    st_sc(part + 4 + lane, O);
                    if (lane == 0) {
                        st_sc(part, M);
                        st_sc(part + 1, L);
                    }
                }
                wait_stores();
            }
            load_cols<UPW, U>(w, P.proj_w, C, C, cw, CW, lane);
            if (!barrier()) return;

            // ---------------- phase C: merge the splits, c_proj, x += . + b
            {
                int j = 0, q = 0;
                const int c = ctrl ? slot_col(lane, C, CW, j, q) : -1;
                const float xo = ctrl ? ld_sc(a.x + max(c, 0)) : 0.f;
                // m and l of every (head, split) into LDS; each thread loads
                // the o of its channels from every split (all loads in
                // flight) and merges them (online softmax merge)
                const int tt = opaque_v(tid);
                const int hsi = min(tt, H * ns - 1);
                const float* pm = a.apart + ((long)(hsi / ns) * PMAXS + hsi % ns) * 68;
                const float m_r = ld_sc(pm), l_r = ld_sc(pm + 1);
                constexpr int CPT = (256 * U + PT - 1) / PT;  // channels per thread
                float ov[CPT][PMAXS];
#pragma unroll
                for (int i = 0; i < CPT; i++) {
                    const int e = min(tt + PT * i, C - 1);
                    const float* pb = a.apart + (long)(e >> 6) * PMAXS * 68 + 4 + (e & 63);
#pragma unroll
                    for (int sp = 0; sp < PMAXS; sp++)
                        ov[i][sp] = sp < ns ? ld_sc(pb + sp * 68) : 0.f;
                }
                if (tid < H * ns) {
                    sm.ml[0][tid] = m_r;
                    sm.ml[1][tid] = l_r;
                }
                __syncthreads();
#pragma unroll
                for (int i = 0; i < CPT; i++) {
                    const int e = tid + PT * i;
                    const int h = min(e, C - 1) >> 6;
                    float mx = -INFINITY, L = 0.f, acc = 0.f;
#pragma unroll
                    for (int sp = 0; sp < PMAXS; sp++) {
                        if (sp < ns) {
                            const float ms = sm.ml[0][h * ns + sp], lsum = sm.ml[1][h * ns + sp];
                            const float mn = fmaxf(mx, ms);
                            const float fa = expf(mx - mn), fb = expf(ms - mn);
                            acc = acc * fa + ov[i][sp] * fb;
                            L = L * fa + lsum * fb;
                            mx = mn;
                        }
                    }
                    if (e < C) actf[e] = acc * (1.0f / L);
                }
                __syncthreads();
                if (!ctrl) {
                    float acc[UPW];
                    col_dots<UPW, U>(acc, w, sm.act, C, C, cw, CW, lane);
                    if (lane == 0)
#pragma unroll
                        for (int jj = 0; jj < UPW; jj++) sm.red[jj][wave] = acc[jj];
                }
                __syncthreads();
                const float bn = slot_bias(P.fc_b, C4);
                if (ctrl) {
                    if (c >= 0) st_sc(a.x + c, (xo + sm.red[j][q]) + bo);
                    wait_stores();
                }
                bo = bn;
                load_cols<UPW, U>(w, P.fc_w, C4, C, cw, CW, lane);
                ln_params(P.ln2_w, P.ln2_b);
            }
            if (!barrier()) return;

            // ---------------- phase D: LayerNorm 2, fc + b, GELU into hid
            load_x();
            ln_to_act(xv, lw, lb, C, actf, sm.wred, tid, wave, lane);
            if (!ctrl) {
                float acc[UPW];
                col_dots<UPW, U>(acc, w, sm.act, C4, C, cw, CW, lane);
                if (lane == 0)
#pragma unroll
                    for (int j = 0; j < UPW; j++) sm.red[j][wave] = acc[j];
            }
            __syncthreads();
            {
                const float bn = slot_bias(P.mlp_b, C);
                if (ctrl) {
                    int j, q;
                    const int c = slot_col(lane, C4, CW, j, q);
                    if (c >= 0) st_sc(a.hid + c, gelu_tanh(sm.red[j][q] + bo));
                    wait_stores();
                }
                bo = bn;
            }
            // proj: one column of depth 4C per wavefront
            load_cols<1, 4 * U>(w, P.mlp_w, C, C4, cw, CW, lane);
            if (!barrier()) return;

            // ---------------- phase E: proj, x += . + b
            {
                int j = 0, q = 0;
                const int c = ctrl ? slot_col(lane, C, CW, j, q) : -1;
                const float xo = ctrl ? ld_sc(a.x + max(c, 0)) : 0.f;
                {
                    constexpr int NH = (1024 * U + PT - 1) / PT;
                    float hv[NH];
                    const int tt = opaque_v(tid);
#pragma unroll
                    for (int k = 0; k < NH; k++) hv[k] = ld_sc(a.hid + min(tt + PT * k, C4 - 1));
#pragma unroll
                    for (int k = 0; k < NH; k++)
                        if (tid + PT * k < C4) actf[tid + PT * k] = hv[k];
                }
                __syncthreads();
                if (!ctrl) {
                    float acc[UPW];
                    col_dots<1, 4 * U>(acc, w, sm.act, C, C4, cw, CW, lane);
                    if (lane == 0)
#pragma unroll
                        for (int jj = 0; jj < UPW; jj++) sm.red[jj][wave] = acc[jj];
                }
                __syncthreads();
                const float bn = slot_bias(PN.attn_b, C3);
                if (ctrl) {
                    if (c >= 0) st_sc(a.x + c, (xo + sm.red[j][q]) + bo);
                    wait_stores();
                }
                bo = bn;
                if (l + 1 < a.L) {
                    load_cols<UPW, U>(w, PN.attn_w, C3, C, cw, CW, lane);
                    ln_params(PN.ln1_w, PN.ln1_b);
                } else {
                    // the first UPW rounds of lm_head columns (tied wte)
                    load_cols<UPW, U>(w, a.wte, V, C, cw, CW, lane);
                    ln_params(a.lnf_w, a.lnf_b);
                }
            }
            if (!barrier()) return;
        }

        // ---------------- phase F: final LayerNorm, lm_head (tied wte), argmax partials
        load_x();
        ln_to_act(xv, lw, lb, C, actf, sm.wred, tid, wave, lane1);
        if (!ctrl) {
            const int ln = opaque_v(lane1);
            const int K4 = C >> 2;
            float best = -INFINITY;
            int bi = 0x7fffffff;
            const int rounds = (V - cw + CW - 1) / CW;  // columns cw, cw + CW, ... < V
            for (int r0 = 0; r0 < rounds; r0 += UPW) {
#pragma unroll
                for (int k = 0; k < UPW; k++) {
                    const int r = r0 + k;
                    const int col = cw + CW * r;
                    if (r < rounds) {
                        float s = 0.f;
#pragma unroll
                        for (int i = 0; i < U; i++) {
                            const int f = i * 64 + ln;
                            if (f < K4) s += dot4(w[k * U + i], sm.act[f]);
                        }
                        const int nc = col + CW * UPW;
                        if (nc < V) {
                            const float* row = a.wte + (long)nc * C;
#pragma unroll
                            for (int i = 0; i < U; i++)
                                w[k * U + i] = ldg4(row + 4 * min(i * 64 + ln, K4 - 1));
                        } else {
#pragma unroll
                            for (int i = 0; i < U; i++) w[k * U + i] = f32x4{0.f, 0.f, 0.f, 0.f};
                        }
                        s = wave_sum(s);
                        if (ln == 0 && a.logits) a.logits[col] = s;
                        if (better(s, col, best, bi)) {
                            best = s;
                            bi = col;
                        }
                    }
                }
            }
            if (ln == 0) {
                sm.bestv[wave] = best;
                sm.besti[wave] = bi;
            }
        }
        __syncthreads();
        bo = slot_bias(layers[0].attn_b, C3);
        if (ctrl) {
            if (lane1 == 0) {
                float b = sm.bestv[0];
                int bi = sm.besti[0];
                for (int v = 1; v < PW; v++)
                    if (better(sm.bestv[v], sm.besti[v], b, bi)) {
                        b = sm.bestv[v];
                        bi = sm.besti[v];
                    }
                st_sc(a.am_v + blockIdx.x, b);
                st_sc(a.am_i + blockIdx.x, bi);
            }
            wait_stores();
        }
        if (step + 1 < a.n_steps) {
            load_cols<UPW, U>(w, layers[0].attn_w, C3, C, cw, CW, lane1);
            ln_params(layers[0].ln1_w, layers[0].ln1_b);
        }
        if (!barrier()) return;

        // ---------------- phase G: every workgroup reduces the argmax partials
        {
            const int g = min(tid, G - 1);
            const float pv = ld_sc(a.am_v + g);
            const int pi = ld_sc(a.am_i + g);
            float b = tid < G ? pv : -INFINITY;
            int bi = tid < G ? pi : 0x7fffffff;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(b, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (better(ov, oi, b, bi)) {
                    b = ov;
                    bi = oi;
                }
            }
            if (lane1 == 0) {
                sm.bestv[wave] = b;
                sm.besti[wave] = bi;
            }
            __syncthreads();
            if (tid == 0) {
                for (int v = 1; v < PW + 1; v++)
                    if (better(sm.bestv[v], sm.besti[v], b, bi)) {
                        b = sm.bestv[v];
                        bi = sm.besti[v];
                    }
                sm.besti[0] = bi;
            }
            __syncthreads();
            tok = sm.besti[0];
            __syncthreads();
        }
    }
    if (blockIdx.x == 0 && tid == 0) {
        *a.tok = tok;
        *a.pos = t;
    }
}

template <int U>
hipError_t launch_u(const PersistArgs& a, int G, hipStream_t s) {
    void* args[] = {(void*)&a};
    return hipLaunchCooperativeKernel((const void*)k_decode_persist<U>, dim3(G), dim3(PT), args, 0,
                                      s);
}

}  // namespace

int persist_workgroups(int device) {
    int cus = 0, coop = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        return 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device) != hipSuccess ||
        !coop)
        return 0;
    return cus / NGRP * NGRP;
}

int persist_max_splits() { return PMAXS; }

int persist_barrier_words() { return NGRP * CSTR + 32; }

bool persist_supported(int C, int H, int V, int cap, int G) {
    if (G < NGRP || G > PT || C % 64 || C != 64 * H || C > 256 * PMAXU || H > 32 || C > LNE * PT)
        return false;
    const long CW = (long)PW * G;
    // columns per wavefront: QKV and fc at most UPW, proj one
    if (4L * C > UPW * CW || C > CW || V < 32) return false;
    // attention: H * splits workgroups, at most PW * KPW keys per split
    const int ns = std::min(G / H, PMAXS);
    if (ns < 1 || (long)ns * PW * KPW < cap) return false;
    return true;
}

hipError_t launch_decode_persist(const PersistArgs& a, int G, hipStream_t s) {
    hipError_t e = hipMemsetAsync(a.bar, 0, (size_t)persist_barrier_words() * sizeof(unsigned), s);
    if (e != hipSuccess) return e;
    switch ((a.C + 255) / 256) {
        case 1: return launch_u<1>(a, G, s);
        case 2: return launch_u<2>(a, G, s);
        case 3: return launch_u<3>(a, G, s);
        case 4: return launch_u<4>(a, G, s);
        default: return hipErrorInvalidValue;
    }
}
