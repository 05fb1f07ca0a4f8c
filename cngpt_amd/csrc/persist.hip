// persist.hip - single-sequence decode steps as one persistent kernel.
//
// A decode step is a chain of dependent stages: per layer LayerNorm 1 +
// QKV, attention over the cache, merge + c_proj + residual, LayerNorm 2 +
// fc + GELU, proj + residual; then the final LayerNorm + lm_head and the
// argmax (reference fast.c:245-329 at T = 1, with the KV cache). Launched
// as separate kernels, every stage pays a kernel boundary plus the HBM
// latency of its weights. Here the stages are phases of one cooperative
// launch (one workgroup per CU), and since no weight depends on the data,
// each workgroup loads weights into registers phases before they are
// used, right after the publish of the phase that freed their slots, so
// that traffic overlaps the waits for later inputs. One launch runs any
// number of steps (the token of step s feeds step s+1 without leaving the
// GPU; sampled tokens are drawn inside the launch too).
//
// Workgroup: PW compute wavefronts + 1 control wavefront. The compute
// wavefronts hold weights and form dot products; the control wavefront,
// which holds no weight loads for its polls to queue behind, polls x and
// forms both LayerNorms, collects the per-column results, applies the
// epilogue and publishes the outputs. The (head, key split) attention items
// run on the workgroups that own no c_proj / proj column when they fit
// there; those load the next layer's cached keys during E.
//
// Exchange between workgroups: every value a phase publishes is one 64-bit
// word, the float in the low half and the tag of the phase that made it in
// the high half, stored and loaded as agent-scope atomics (sc1: through
// the XCD-private L2, which is not coherent across XCDs). A consumer reads
// the words it needs until each carries the tag it expects, so there is no
// grid barrier, no counter and no wait for store completion: a 64-bit word
// is written whole, and the tag proves the value is the current one. Tags
// grow monotonically over launches, and every buffer is rewritten only
// after all consumers of its previous contents have provably read them (a
// producer of version v+1 has consumed, through an all-to-all phase, data
// made after every workgroup read version v). Per buffer (every workgroup
// owns QKV and fc columns, so their outputs come from all workgroups):
//   q/k/v of row t: written in A(l+1) after reading x(E(l)), made from
//     hid(l) of every workgroup, made after x(C(l)), made after every
//     attention partial of B(l), made after the reads of A(l)'s words.
//   attention partials: written in B(l+1) after q/k/v of A(l+1), made after
//     x(E(l)), made from hid(l) of every workgroup, each of which read its
//     partials of C(l) before it made hid(l).
//   x: C(l) and E(l) rewrite it; a writer has read inputs made by every
//     workgroup after that workgroup's last read of x (hid(l) for E, the
//     partials of B(l+1) from q/k/v of every workgroup for C(l+1)).
//   hid: written in D(l+1) after x(C(l+1)), made after the partials of
//     B(l+1), made after q/k/v from every workgroup, each of which read
//     its hid(l) in E(l) before A(l+1).
//   argmax partials: rewritten a whole step later, after the same chains.
// A poll limit turns a stall into an error flag that every waiting
// workgroup sees and exits on.
//
// Cache rows written in a step are read by later steps with plain loads:
// the writer's later loads wait for its stores, before it publishes the
// values that the readers' progress depends on.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace {

constexpr int PW = 7;                  // compute wavefronts per workgroup
constexpr int PT = (PW + 1) * 64;      // + the control wavefront: 2 per SIMD
constexpr int PHASES = 5;              // phases per layer
constexpr int UPW = 4;                 // lm_head columns per wavefront in flight
constexpr int NJQ = 2;                 // fc columns per wavefront (4C <= NJQ * 7G)
constexpr int NJA = 4;                 // QKV columns per wavefront of the QKV workgroups
                                       // (3C <= NJA * 7 * their count)
constexpr int KPW = 16;                // attention keys per wavefront
constexpr int PMAXS = 16;              // attention splits per head
constexpr long SPIN_LIMIT = 1L << 20;  // polls of one value before giving up
// Widths up to 256 * PMAXU channels (GPT-2 small): the weights a lane holds
// for two phases (2 * UPW * U float4, U = ceil(C / 256)) then fit in
// registers beside the rest; wider models take the kernel-per-stage decode.
constexpr int PMAXU = 3;
// Sampling inside the launch (top_k <= SK_MAX): each workgroup keeps the
// logits of its lm_head columns (at most SK_RMAX per compute wavefront) and
// publishes at most SK_CMAX candidates.
constexpr int SK_MAX = 64;
constexpr int SK_RMAX = 32;
constexpr int SK_CMAX = 4;
constexpr int SK_SLOT = 1 + 2 * SK_CMAX;  // count, then (value, index) pairs
constexpr int SK_CAND = 256 * SK_CMAX;    // candidates gathered (G <= 256)

__device__ __forceinline__ void st_sc(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Loads through the global address space: pointers taken from the layer
// table are generic, and generic (flat) loads make the compiler wait for
// them at the next control-flow join.
typedef __attribute__((address_space(1))) const float gfloat;
typedef __attribute__((address_space(1))) const f32x4 gf32x4;
__device__ __forceinline__ float ldg(const float* p) { return *(gfloat*)p; }
__device__ __forceinline__ f32x4 ldg4(const float* p) { return *(gf32x4*)p; }

typedef unsigned long long u64;
// Exchange word: tag in the high half, the float's bits in the low half.
__device__ __forceinline__ void put(u64* p, float v, unsigned tag) {
    __hip_atomic_store(p, ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 peek(const u64* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float wval(u64 w) { return __uint_as_float((unsigned)w); }
__device__ __forceinline__ unsigned wtag(u64 w) { return (unsigned)(w >> 32); }

// out[k] = value of base[idx[k]] once it carries `tag` (for k with need[k];
// idx[k] is always a valid index). All first reads are in flight together;
// only stragglers are read again. False after SPIN_LIMIT rounds or when
// another workgroup of this launch has raised the abort word (to amark; a
// smaller value is an earlier launch's, as tags only grow).
// Only slots k with bit k of en (uniform over the wavefront) are read at
// all, and slots with bit k of t2 wait for tag2 instead of tag. One call
// waits for all its words, so a phase gathers every input in one call (one
// round trip, not one per input).
template <int N>
__device__ __forceinline__ bool fetch(const u64* base, const int (&idx)[N], const bool (&need)[N],
                                      unsigned tag, float (&out)[N], const u64* abortw,
                                      u64 amark, unsigned en = ~0u, unsigned t2 = 0u,
                                      unsigned tag2 = 0u) {
    u64 v[N];
#pragma unroll
    for (int k = 0; k < N; k++) v[k] = ((en >> k) & 1u) ? peek(base + idx[k]) : 0ull;
    unsigned long long pend = 0;
#pragma unroll
    for (int k = 0; k < N; k++) {
        out[k] = wval(v[k]);
        const unsigned want = ((t2 >> k) & 1u) ? tag2 : tag;
        if (((en >> k) & 1u) && need[k] && wtag(v[k]) != want) pend |= 1ull << k;
    }
    long it = 0;
    while (pend) {
        __builtin_amdgcn_s_sleep(1);  // a short back-off between rounds
        // read the pending words again, all in flight before any is
        // checked (a check in the same branch as its read would wait for
        // each read in turn)
#pragma unroll
        for (int k = 0; k < N; k++)
            if (pend & (1ull << k)) v[k] = peek(base + idx[k]);
#pragma unroll
        for (int k = 0; k < N; k++)
            if ((pend & (1ull << k)) && wtag(v[k]) == (((t2 >> k) & 1u) ? tag2 : tag)) {
                out[k] = wval(v[k]);
                pend &= ~(1ull << k);
            }
        if (pend && (++it & 31) == 0 && (it > SPIN_LIMIT || peek(abortw) >= amark)) return false;
    }
    return true;
}

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

// Enable mask of slots k whose word tid + PT * k (for some lane of this
// wavefront) is below n.
__device__ __forceinline__ unsigned slots_below(int n, int tt) {
    const int k = min(31, max(0, (n - (tt & ~63) + PT - 1) / PT));
    return (unsigned)opaque_s(__builtin_amdgcn_readfirstlane((int)((1u << k) - 1u)));
}

template <int U>
struct Smem {
    f32x4 act[256 * U];           // activation vector (up to 1024 * U floats)
    float lnw[256 * U], lnb[256 * U];  // gains and biases of the next LayerNorm
    float red[UPW][PW];           // per-wavefront column sums
    float wred[PW + 1];           // block reductions
    float attn[PW][68];           // per-wavefront attention partials: m, l, -, -, o[64]
    float qkv_new[3][64];         // q, k, v of row t for this workgroup's head
    float ml[2][32 * PMAXS];      // m and l of every (head, split)
    float obuf[PMAXS * 256 * U];  // o of every (split, channel)
    float bestv[PW + 1];
    int besti[PW + 1];
    int abort;
    // sampling
    float sx[PW * SK_RMAX];       // scaled logits of this workgroup's columns
    float cx[SK_CAND];            // candidates of every workgroup: value
    int ci[SK_CAND];              //   and index; then the survivors in index order
    float so[SK_CAND];
    int soi[SK_CAND];
    float raw[256 * SK_SLOT];     // the candidate words as fetched
    float kv[PW][32][64];         // the next layer's cached keys of each compute
                                  // wavefront (its kq, then vr), staged in E
    int n_c, n_sv, over, stok;
    float sL, sc, sns;
};

// Exchange words (offsets in u64 units).
// Values read by many workgroups (x, hid, attention and argmax partials)
// are published in REPL copies, each read by the workgroups of one XCD
// (blockIdx % REPL): one copy read by every workgroup concentrates those
// reads on the few memory channels that hold it.
constexpr int REPL = 8;
struct TagLayout {
    int xs, hs, ps, as, cs;  // copy strides
    int x, q, hid, part, am, cand, abortw;
    __host__ __device__ TagLayout(int C, int H)
        : xs(C + 512), hs(4 * C + 512), ps(H * PMAXS * 68 + 512), as(2 * PT + 512),
          cs(SK_SLOT * PT + 512), x(0), q(REPL * xs), hid(q + 3 * C + 512),
          part(hid + REPL * hs), am(part + REPL * ps), cand(am + REPL * as),
          abortw(cand + REPL * cs) {}
    __host__ __device__ long words() const { return abortw + 32; }
};
__device__ __forceinline__ void put_all(u64* p, int stride, float v, unsigned tag) {
#pragma unroll
    for (int r = 0; r < REPL; r++) put(p + r * stride, v, tag);
}

// Sum over the workgroup, same value in every thread.
__device__ __forceinline__ float block_sum(float v, float* wred, int wave, int lane) {
    v = wave_sum_dpp(v);
    if (lane == 0) wred[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PW + 1; i++) s += wred[i];
    __syncthreads();
    return s;
}

// Max over the workgroup, same value in every thread.
__device__ __forceinline__ float block_max(float v, float* wred, int wave, int lane) {
    v = wave_max_dpp(v);
    if (lane == 0) wred[wave] = v;
    __syncthreads();
    float m = wred[0];
#pragma unroll
    for (int i = 1; i < PW + 1; i++) m = fmaxf(m, wred[i]);
    __syncthreads();
    return m;
}

// LayerNorm (reference ops.c:191-248) by one wavefront: x[lane + 64 k] in
// v[k], gains and biases from LDS, result into act. Two passes (mean, then
// the mean square deviation), each one wavefront reduction.
template <int NX>
__device__ __forceinline__ void ln_wave(const float (&v)[NX], int C, int ln, const float* gw,
                                        const float* gb, float* act) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NX; k++)
        if (ln + 64 * k < C) s += v[k];
    const float mean = wave_sum_dpp(s) / (float)C;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < NX; k++)
        if (ln + 64 * k < C) {
            const float d = v[k] - mean;
            q += d * d;
        }
    const float rstd = 1.0f / sqrtf(wave_sum_dpp(q) / (float)C + 1e-5f);
#pragma unroll
    for (int k = 0; k < NX; k++) {
        const int e = ln + 64 * k;
        if (e < C) act[e] = (v[k] - mean) * rstd * gw[e] + gb[e];
    }
}

// Columns of a product Y[N] = W[N, K] . act: column cw + CW * j (j < NJ)
// belongs to compute wavefront cw; its lane l holds float4 i * 64 + l
// (i < NI) of the column's weight row in w[OFF + j * NI + i].
template <int NJ, int NI, int OFF = 0, int NW>
__device__ __forceinline__ void load_cols(f32x4 (&w)[NW], const float* __restrict__ W, int N,
                                          int K, int cw, int CW, int lane) {
    static_assert(OFF + NJ * NI <= NW, "register budget");
    cw = opaque_s(cw);
    lane = opaque_v(lane);
    const int K4 = K >> 2;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int c = cw + CW * j;
        if (c < N) {
            const float* row = W + (long)c * K;
#pragma unroll
            for (int i = 0; i < NI; i++)
                w[OFF + j * NI + i] = ldg4(row + 4 * min(i * 64 + lane, K4 - 1));
        } else {
            // written on every path, so the previous phase's values are dead
#pragma unroll
            for (int i = 0; i < NI; i++) w[OFF + j * NI + i] = f32x4{0.f, 0.f, 0.f, 0.f};
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
    // the activation float4s of this lane, read once and unconditionally
    // (at clamped indices): reads under a lane-dependent condition make the
    // compiler branch around each one and wait for it inside the branch
    f32x4 xv[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) xv[i] = act[min(i * 64 + lane, K4 - 1)];
#pragma unroll
    for (int j = 0; j < UPW; j++) {
        float s = 0.f;
        if (j < NJ && cw + CW * j < N) {
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const float d = dot4(w[j * NI + i], xv[i]);
                s += i * 64 + lane < K4 ? d : 0.f;
            }
        }
        acc[j] = s;
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[j] = wave_sum_dpp(acc[j]);
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
// The same for the QKV columns, which only workgroups q0 .. G - 1 compute
// (CWA = PW * (G - q0) wavefronts).
__device__ __forceinline__ int slot_cola(int slot, int N, int CWA, int q0, int& j, int& q) {
    j = slot / PW;
    q = slot - j * PW;
    if (j >= NJA) return -1;
    const int c = CWA * j + ((int)blockIdx.x - q0) * PW + q;
    return c < N ? c : -1;
}

// Key splits of the attention at position t (nk = t + 1 keys): as few as
// the workgroup's PW * KPW keys allow, within the workgroups after the
// c_proj / proj column owners and PMAXS.
__device__ __forceinline__ int attn_splits(int t, int owners, int G, int H) {
    const int ns = (t + 1 + PW * KPW - 1) / (PW * KPW);
    return min(ns, min((G - owners) / H, PMAXS));
}

// First QKV workgroup of a step at position t: the workgroups after the
// column owners and the step's (head, split) attention items, as long as
// they hold NJA columns per wavefront of all 3C; else as many of the last
// workgroups as do (some of them then also attention items).
__device__ __forceinline__ int qkv_first(int t, int C, int H, int G) {
    const int owners = (C + PW - 1) / PW;
    const int nmin = (3 * C + NJA * PW - 1) / (NJA * PW);
    const int q0 = owners + H * attn_splits(t, owners, G, H);
    return max(owners, min(q0, G - nmin));
}

template <int U, bool SAMP>
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
    // QKV columns: only workgroups q0 .. G - 1 of a step take them, those
    // after the c_proj / proj column owners and the attention items where
    // they fit (an owner comes to A from publishing E's x, an item from
    // staging the next layer's keys, both later than the others, and would
    // hold up every head's q, k, v); the other workgroups skip A. q0 moves
    // with the step's key splits, so the mapping is formed per step (and
    // for the next step where its weights are loaded ahead).
    int q0 = qkv_first(*a.pos, a.C, a.H, G);
    auto qkv_wave = [&](int first) {
        return (ctrl || (int)blockIdx.x < first) ? (1 << 29) : ((int)blockIdx.x - first) * PW + wave;
    };
    const int C = a.C, C3 = 3 * C, C4 = 4 * C, H = a.H, V = a.V, L = a.L;
    float* actf = (float*)sm.act;
    const TagLayout tl(C, H);
    // published copies (written REPL times) and the copy this workgroup reads
    const int rep = blockIdx.x % REPL;
    u64* const tx = a.tagged + tl.x;      // x after c_proj / proj
    u64* const tq = a.tagged + tl.q;      // q, k, v of row t (one copy)
    u64* const th = a.tagged + tl.hid;    // GELU(fc)
    u64* const tp = a.tagged + tl.part;   // attention partials [H][PMAXS][68]
    u64* const tam = a.tagged + tl.am;    // argmax partials [G][2] (sampling: max, sum)
    u64* const tcd = a.tagged + tl.cand;  // sampling candidates [G][SK_SLOT]
    const u64* const rx = tx + rep * tl.xs;
    const u64* const rh = th + rep * tl.hs;
    const u64* const rp = tp + rep * tl.ps;
    const u64* const ram = tam + rep * tl.as;
    const u64* const rcd = tcd + rep * tl.cs;
    u64* const abortw = a.tagged + tl.abortw;
    const u64 amark = (u64)a.tag0 + 1;  // the abort word's value for this launch
    const unsigned per_step = PHASES * L + 2;  // + the sampling candidates

    if (tid == 0) sm.abort = 0;
    __syncthreads();

    // After the fetches of a phase: every thread learns whether one of the
    // workgroup's waits gave up (then all return together).
    auto settle = [&](bool ok) -> bool {
        if (!ok) {
            sm.abort = 1;
            __hip_atomic_store(abortw, amark, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.err) atomicOr(a.err, 2);
        }
        __syncthreads();
        return sm.abort == 0;
    };

    int t = *a.pos;
    int tok = *a.tok;
    constexpr bool samp = SAMP;  // the greedy instantiation carries no sampling code
    const float tdiv = a.temp > 0.0f ? a.temp : 1.0f;
    const float scale2 = a.scale * 1.4426950408889634f;
    // Two weight buffers of UPW * U float4 per lane. On the c_proj / proj
    // column owners NJQ * U of them hold the fc columns, U the c_proj
    // column, 4U the proj column:
    //   wa[0, 2U): fc (D)                    wa[2U, 4U): proj, first half (E)
    //   wb[0, U):  c_proj (C)                wb[U, 3U):  proj, second half (E)
    // on the other workgroups NJA * U the QKV columns, then the fc columns:
    //   wa[0, 3U): QKV (A), then fc in wa[0, 2U) (D)
    // Loads are issued after a phase's publish into the slots it freed:
    // after A fc and all of proj (the c_proj / proj column owners have no
    // work in A and B, which leaves the longest time for their largest
    // loads), after D the next QKV (the lm_head's first two rounds after
    // the last layer), after E the next c_proj (and the lm_head's rounds 2
    // and 3). The lm_head streams UPW rounds through all of wa.
    f32x4 wa[NW], wb[NW];
    f32x4 kq[4];             // attention prefetch: K, 16 dims of one key
    float vr[KPW];           // V of 16 keys, one dim
    float bo = 0.f;          // control lanes: bias of the next output column

    // Loads below are unconditional with clamped indices: a load under a
    // divergent branch makes the compiler wait for it inside the branch,
    // which serialises the loads of a phase.
    // Gains and biases of the next LayerNorm, loaded by the control
    // wavefront straight into LDS (no registers held across the phases in
    // between); its next poll waits for them, as loads return in order.
    // Source indices are clamped to the C floats of each array.
    auto ln_params = [&](const float* gw, const float* gb) {
        if (ctrl) {
            const int ln = opaque_v(lane);
#pragma unroll
            for (int k = 0; k < U; k++) {
                const int f4 = min(k * 64 + ln, C / 4 - 1);
                __builtin_amdgcn_global_load_lds((const void*)(gw + 4 * f4),
                                                 (lds_void*)(sm.lnw + 256 * k), 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const void*)(gb + 4 * f4),
                                                 (lds_void*)(sm.lnb + 256 * k), 16, 0, 0);
            }
        }
    };
    // LayerNorm of x into act (reference ops.c:191-248) by the control
    // wavefront, which holds no weight loads for its polls to queue behind:
    // x is polled (tag `tag`), or for layer 0 formed from the embedding
    // wte[tok] + wpe[t] (reference fast.c:245-254). One barrier then hands
    // act to the compute wavefronts; false (in every thread) when a wait
    // gave up.
    auto fetch_ln = [&](unsigned tag, bool embed, int tk, int tpos) -> bool {
        bool ok = true;
        if (ctrl) {
            constexpr int NX = 4 * U;  // C <= 256 * U words, 64 per round
            const int ln = opaque_v(lane);
            float v[NX];
            if (embed) {
                const float* er = a.wte + (long)tk * C;
                const float* pr = a.wpe + (long)tpos * C;
                float ev[NX], pv[NX];
#pragma unroll
                for (int k = 0; k < NX; k++) {
                    const int e = min(ln + 64 * k, C - 1);
                    ev[k] = ldg(er + e);
                    pv[k] = ldg(pr + e);
                }
#pragma unroll
                for (int k = 0; k < NX; k++) v[k] = ev[k] + pv[k];
            } else {
                int idx[NX];
                bool need[NX];
#pragma unroll
                for (int k = 0; k < NX; k++) {
                    idx[k] = min(ln + 64 * k, C - 1);
                    need[k] = ln + 64 * k < C;
                }
                const unsigned en = (1u << ((C + 63) / 64)) - 1u;
                ok = fetch<NX>(rx, idx, need, tag, v, abortw, amark, en);
            }
            // the gains' loads into LDS have landed once nothing is pending
            wait_vmcnt<0>();
            if (ok) ln_wave<NX>(v, C, ln, sm.lnw, sm.lnb, actf);
        }
        return settle(ok);
    };
    // Bias of this lane's output column in the next phase (control lanes;
    // the others load b[0]). Issued before the current epilogue's stores.
    auto slot_bias = [&](const float* b, int N) -> float {
        int j, q;
        return ldg(b + max(slot_col(opaque_v(lane), N, CW, j, q), 0));
    };
    auto slot_bias_a = [&](const float* b, int N, int first) -> float {
        int j, q;
        return ldg(b + max(slot_cola(opaque_v(lane), N, PW * (G - first), first, j, q), 0));
    };

    const LayerW* layers = a.layers;
    if ((int)blockIdx.x >= q0) {
        load_cols<NJA, U>(wa, layers[0].attn_w, C3, C, qkv_wave(q0), PW * (G - q0), lane);
        ln_params(layers[0].ln1_w, layers[0].ln1_b);
    }
    load_cols<1, U>(wb, layers[0].proj_w, C, C, cw0, CW, lane);
    bo = (int)blockIdx.x >= q0 ? slot_bias_a(layers[0].attn_b, C3, q0) : 0.f;

    for (int step = 0; step < a.n_steps; step++, t++) {
        // opaque copies per iteration (see opaque_s)
        const int lane1 = opaque_v(lane), cw1 = opaque_s(cw0);
        // this step's QKV workgroups
        const int qf = opaque_s(q0);
        const bool inq = (int)blockIdx.x >= qf;
        const int CWA = PW * (G - qf);
        const int cw = cw1;
        const unsigned sbase = a.tag0 + (unsigned)step * per_step;
        // ---------------- embedding x = wte[tok] + wpe[t] (fast.c:245-254)
        if (tok < 0 || tok >= V) {
            if (tid == 0 && a.err) atomicOr(a.err, 1);
            tok = tok < 0 ? 0 : V - 1;
        }
        if (blockIdx.x == 0 && tid == 0) a.hist[t] = tok;

        for (int l = 0; l < L; l++) {
            const int lane = opaque_v(lane1), cw = opaque_s(cw1), cwa = opaque_s(qkv_wave(qf));
            const LayerW P = layers[l];
            const LayerW PN = layers[min(l + 1, L - 1)];
            float* kvl = a.cache + (long)l * a.cap * C3;
            float* rowt = kvl + (long)t * C3;
            // tags of the values this layer's phases publish; x enters the
            // layer with the tag of the previous layer's proj (or as the
            // embedding, computed in place, for layer 0)
            const unsigned TA = sbase + PHASES * l + 1, TB = TA + 1, TC = TA + 2, TD = TA + 3,
                           TE = TA + 4, TXIN = TA - 1;

            // ---------------- phase A: LayerNorm 1 + QKV into row t (not
            // on the column owners)
            if (inq && !fetch_ln(TXIN, l == 0, tok, t)) return;
            // attention split layout for keys 0..t
            const int nk = t + 1;
            // The (head, split) items go to the workgroups after the c_proj /
            // proj column owners (persist_supported checks that they fit
            // there): those workgroups have no column work in C and E, so in
            // E they load the next layer's cached keys and park them in LDS,
            // and their QKV publish in A is not held up behind those loads.
            // As few splits as the workgroup's PW * KPW keys allow (fewer
            // partials to exchange).
            const int owners = (C + PW - 1) / PW;
            const int ns = attn_splits(t, owners, G, H);
            const int kps = (nk + ns - 1) / ns;
            const int kpw = (kps + PW - 1) / PW;
            const int item = (int)blockIdx.x - owners;
            const bool has_item = item >= 0 && item < H * ns;
            const int ih = max(item, 0) / ns, isp = max(item, 0) - ih * ns;
            const int k0 = isp * kps, k1 = min(k0 + kps, nk);
            const int kw0 = k0 + wave * kpw, kw1 = min(kw0 + kpw, k1);
            // this workgroup's cached keys (< t) of layer `ll`, loaded by its
            // compute wavefronts
            auto load_keys = [&](int ll) {
                const float* kv = a.cache + (long)ll * a.cap * C3;
                const int kk = kw0 + (lane >> 2), dq = lane & 3;
                const int kc = min(kk, max(t - 1, 0));
                const float* kr = kv + (long)kc * C3 + C + ih * 64 + dq * 16;
#pragma unroll
                for (int i = 0; i < 4; i++) kq[i] = ldg4(kr + 4 * i);
#pragma unroll
                for (int jj = 0; jj < KPW; jj++) {
                    const int kj = min(kw0 + jj, max(t - 1, 0));
                    vr[jj] = ldg(kv + (long)kj * C3 + 2 * C + ih * 64 + lane);
                }
            };
            if (!ctrl && has_item) {
                if (l > 0) {
                    // staged in the previous layer's E by this wavefront
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int c = 0; c < 4; c++) kq[i][c] = sm.kv[wave][4 * i + c][lane];
#pragma unroll
                    for (int jj = 0; jj < KPW; jj++) vr[jj] = sm.kv[wave][16 + jj][lane];
                } else {
                    load_keys(l);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) kq[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int jj = 0; jj < KPW; jj++) vr[jj] = 0.f;
            }
            if (inq) {
                if (!ctrl) {
                    float acc[UPW];
                    col_dots<NJA, U>(acc, wa, sm.act, C3, C, cwa, CWA, lane);
                    if (lane == 0)
#pragma unroll
                        for (int j = 0; j < UPW; j++) sm.red[j][wave] = acc[j];
                }
                __syncthreads();
                if (ctrl) {
                    int j, q;
                    const int c = slot_cola(lane, C3, CWA, qf, j, q);
                    if (c >= 0) {
                        const float v = sm.red[j][q] + bo;
                        put(tq + c, v, TA);
                        st_sc(rowt + c, v);  // the cache row, for later steps
                    }
                }
                // Weight loads are issued after the phase's publish (the
                // barrier puts them behind its stores): queued ahead of the
                // stores they delayed the publish, and a wait the compiler
                // places for them inside the phase delayed its products.
                __syncthreads();
            }
            bo = slot_bias(P.proj_b, C);
            // fc with LayerNorm 2's gains, and, on the column owners, this
            // wavefront's proj column (depth 4C) in wa[2U, 4U) and wb[U, 3U)
            load_cols<NJQ, U>(wa, P.fc_w, C4, C, cw, CW, lane);
            ln_params(P.ln2_w, P.ln2_b);
            {
                const int c = opaque_s(cw), ln = opaque_v(lane);
                const float* row = P.mlp_w + (long)min(c, C - 1) * C4;
#pragma unroll
                for (int i = 0; i < 4 * U; i++) {
                    const f32x4 v = c < C ? ldg4(row + 4 * min(i * 64 + ln, C - 1))
                                          : f32x4{0.f, 0.f, 0.f, 0.f};
                    if (i < 2 * U) wa[2 * U + i] = v;
                    else wb[i - U] = v;
                }
            }

            // ---------------- phase B: attention, one (head, key split) per workgroup
            if (has_item) {
                bool ok = true;
                if (ctrl) {
                    int idx[3];
                    bool need[3];
                    float nv[3];
#pragma unroll
                    for (int m = 0; m < 3; m++) {
                        idx[m] = m * C + ih * 64 + lane;
                        need[m] = true;
                    }
                    ok = fetch<3>(tq, idx, need, TA, nv, abortw, amark);
#pragma unroll
                    for (int m = 0; m < 3; m++) sm.qkv_new[m][lane] = nv[m];
                }
                if (!settle(ok)) return;
                if (!ctrl) {
                    const int kk = kw0 + (lane >> 2), dq = lane & 3;
                    const bool valid = kk < kw1;
                    // q, the new key and the new value read from LDS once,
                    // unconditionally; the new key and value then replace
                    // the cached ones by register selects (a read under the
                    // per-key condition was a branch and an LDS wait per key)
                    const f32x4* qn = (const f32x4*)&sm.qkv_new[0][dq * 16];
                    const f32x4* kn = (const f32x4*)&sm.qkv_new[1][dq * 16];
                    f32x4 qv[4], kv4[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        qv[i] = qn[i];
                        kv4[i] = kn[i];
                    }
                    const float vnew = sm.qkv_new[2][lane];
                    const bool isnew = kk == t;
                    float d = 0.f;
#pragma unroll
                    for (int i = 0; i < 4; i++) d += dot4(qv[i], isnew ? kv4[i] : kq[i]);
                    d += CNGPT_DPP(d, 0xB1);  // the 4 lanes of a key: xor 1, xor 2
                    d += CNGPT_DPP(d, 0x4E);
                    // scores in base 2 (scale * log2 e folded in), so that
                    // every exponential of the attention and its merges is
                    // one v_exp_f32
                    const float sc = valid ? d * scale2 : -INFINITY;
                    const float m = wave_max_dpp(sc);
                    const float e = valid ? __builtin_amdgcn_exp2f(sc - m) : 0.f;
                    const float ls = wave_sum_dpp(dq == 0 ? e : 0.f);
                    // keys past kw1 have e = 0 (and finite cached values), so
                    // they add exact zeros
                    float o = 0.f;
#pragma unroll
                    for (int jj = 0; jj < KPW; jj++) {
                        const float pj = lane_f(e, 4 * jj);
                        o += pj * (kw0 + jj == t ? vnew : vr[jj]);
                    }
                    if (lane == 0) {
                        sm.attn[wave][0] = m;
                        sm.attn[wave][1] = ls;
                    }
                    sm.attn[wave][4 + lane] = o;
                }
                __syncthreads();
                if (ctrl) {
                    // every wavefront's m, l and o read before any is used
                    float mv[PW], lv[PW], ov[PW];
#pragma unroll
                    for (int v = 0; v < PW; v++) {
                        mv[v] = sm.attn[v][0];
                        lv[v] = sm.attn[v][1];
                        ov[v] = sm.attn[v][4 + lane];
                    }
                    float M = -INFINITY;
#pragma unroll
                    for (int v = 0; v < PW; v++) M = fmaxf(M, mv[v]);
                    float Ls = 0.f, O = 0.f;
#pragma unroll
                    for (int v = 0; v < PW; v++) {
                        const float f = mv[v] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv[v] - M);
                        Ls += lv[v] * f;
                        O += ov[v] * f;
                    }
                    u64* part = tp + ((long)ih * PMAXS + isp) * 68;
                    put_all(part + 4 + lane, tl.ps, O, TB);
                    if (lane == 0) {
                        put_all(part, tl.ps, M, TB);
                        put_all(part + 1, tl.ps, Ls, TB);
                    }
                }
            }

            // ---------------- phase C: merge the splits, c_proj, x += . + b
            // (only workgroups that own one of its C columns take part)
            const bool has_cols = blockIdx.x * PW < C;
            if (has_cols) {
                int j = 0, q = 0;
                const int c = ctrl ? slot_col(lane, C, CW, j, q) : -1;
                float xo = 0.f;
                if (ctrl && l == 0) {
                    const int cc = max(c, 0);
                    xo = ldg(a.wte + (long)tok * C + cc) + ldg(a.wpe + (long)t * C + cc);
                }
                // one wait for: the o of every (split, channel) (flattened
                // f = split * C + channel, 8 per thread per round, into
                // LDS), m and l of every (head, split) (first round), and
                // the control lane's x (first round, layers > 0)
                const int tt = opaque_v(tid);
                const int tot = C * ns;
                bool ok = true;
                for (int f0 = 0; f0 < tot; f0 += PT * 8) {
                    int idx[11];
                    bool need[11];
                    float o[11];
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        const int f = f0 + tt + PT * k;
                        const int fc = min(f, tot - 1);
                        const int sp = fc / C, e = fc - sp * C;
                        idx[k] = ((e >> 6) * PMAXS + sp) * 68 + 4 + (e & 63);
                        need[k] = f < tot;
                    }
                    const int hsi = min(tt, H * ns - 1);
                    const int pb = ((hsi / ns) * PMAXS + hsi % ns) * 68;
                    idx[8] = pb;
                    idx[9] = pb + 1;
                    need[8] = need[9] = tt < H * ns;
                    idx[10] = (int)((rx + max(c, 0)) - rp);
                    need[10] = c >= 0;
                    unsigned en = slots_below(tot - f0, tt) & 0xFFu;
                    if (f0 == 0) {
                        if ((tt & ~63) < H * ns) en |= 3u << 8;
                        if (ctrl && l > 0) en |= 1u << 10;
                    }
                    const bool ok2 = fetch<11>(rp, idx, need, TB, o, abortw, amark, en, 1u << 10, TXIN);
                    ok = ok && ok2;
#pragma unroll
                    for (int k = 0; k < 8; k++)
                        if (need[k]) sm.obuf[f0 + tt + PT * k] = o[k];
                    if (f0 == 0) {
                        if (tt < H * ns) {
                            sm.ml[0][tt] = o[8];
                            sm.ml[1][tt] = o[9];
                        }
                        if (ctrl && l > 0) xo = o[10];
                    }
                }
                if (!settle(ok)) return;
                // merge: each head's split weights 2^(m_s - M) / L (m in base 2), formed
                // once (in place of the m values) by one thread per head,
                // then every channel the weighted sum of its head's splits
                if (tid < H) {
                    float* mh = &sm.ml[0][tid * ns];
                    const float* lh = &sm.ml[1][tid * ns];
                    float M = -INFINITY;
                    for (int sp = 0; sp < ns; sp++) M = fmaxf(M, mh[sp]);
                    float Ls = 0.f;
                    for (int sp = 0; sp < ns; sp++)
                        Ls += lh[sp] * (mh[sp] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mh[sp] - M));
                    const float inv = 1.0f / Ls;
                    for (int sp = 0; sp < ns; sp++)
                        mh[sp] = (mh[sp] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mh[sp] - M)) * inv;
                }
                __syncthreads();
                for (int e = tid; e < C; e += PT) {
                    const float* wh = &sm.ml[0][(e >> 6) * ns];
                    float acc = 0.f;
                    for (int sp = 0; sp < ns; sp++) acc += wh[sp] * sm.obuf[sp * C + e];
                    actf[e] = acc;
                }
                __syncthreads();
                if (!ctrl) {
                    float acc[UPW];
                    col_dots<1, U>(acc, wb, sm.act, C, C, cw, CW, lane);
                    if (lane == 0)
#pragma unroll
                        for (int jj = 0; jj < UPW; jj++) sm.red[jj][wave] = acc[jj];
                }
                __syncthreads();
                if (ctrl && c >= 0) put_all(tx + c, tl.xs, (xo + sm.red[j][q]) + bo, TC);
            }
            bo = slot_bias(P.fc_b, C4);

            // ---------------- phase D: LayerNorm 2, fc + b, GELU into hid
            if (!fetch_ln(TC, false, 0, 0)) return;
            if (!ctrl) {
                float acc[UPW];
                col_dots<NJQ, U>(acc, wa, sm.act, C4, C, cw, CW, lane);
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
                    if (c >= 0) put_all(th + c, tl.hs, gelu_tanh(sm.red[j][q] + bo), TD);
                }
                bo = bn;
            }
            // wa[0, 2U): the next layer's QKV with LayerNorm 1's gains, or
            // the first two rounds of lm_head columns (tied wte) with the
            // final LayerNorm's
            __syncthreads();
            if (l + 1 < L) {
                if (inq) {
                    load_cols<NJA, U>(wa, PN.attn_w, C3, C, cwa, CWA, lane);
                    ln_params(PN.ln1_w, PN.ln1_b);
                }
            } else {
                load_cols<2, U>(wa, a.wte, V, C, cw, CW, lane);
                ln_params(a.lnf_w, a.lnf_b);
            }

            // ---------------- phase E: proj, x += . + b (column owners only)
            if (has_cols) {
                int j = 0, q = 0;
                const int c = ctrl ? slot_col(lane, C, CW, j, q) : -1;
                float xo = 0.f;
                bool ok = true;
                {
                    // one wait for hid and the control lane's x
                    constexpr int NH = (1024 * U + PT - 1) / PT;
                    const int tt = opaque_v(tid);
                    int idx[NH + 1];
                    bool need[NH + 1];
                    float hv[NH + 1];
#pragma unroll
                    for (int k = 0; k < NH; k++) {
                        idx[k] = min(tt + PT * k, C4 - 1);
                        need[k] = tt + PT * k < C4;
                    }
                    idx[NH] = (int)((rx + max(c, 0)) - rh);
                    need[NH] = c >= 0;
                    const unsigned en = (slots_below(C4, tt) & ((1u << NH) - 1u)) |
                                        (ctrl ? 1u << NH : 0u);
                    ok = fetch<NH + 1>(rh, idx, need, TD, hv, abortw, amark, en, 1u << NH, TC);
#pragma unroll
                    for (int k = 0; k < NH; k++)
                        if (need[k]) actf[tt + PT * k] = hv[k];
                    if (ctrl) xo = hv[NH];
                }
                if (!settle(ok)) return;
                if (!ctrl) {
                    // proj: float4 i * 64 + lane of the column, i < 2U in
                    // wa[2U + i], then i < 4U in wb[U + i - 2U]
                    const int ln = opaque_v(lane);
                    float acc[UPW] = {0.f, 0.f, 0.f, 0.f};
                    if (cw < C) {
                        // (unconditional reads at clamped indices, as in col_dots)
#pragma unroll
                        for (int i = 0; i < 4 * U; i++) {
                            const int f = i * 64 + ln;
                            const float d = dot4(i < 2 * U ? wa[2 * U + i] : wb[i - U],
                                                 sm.act[min(f, C - 1)]);
                            acc[0] += f < C ? d : 0.f;
                        }
                    }
                    acc[0] = wave_sum_dpp(acc[0]);
                    if (lane == 0)
#pragma unroll
                        for (int jj = 0; jj < UPW; jj++) sm.red[jj][wave] = acc[jj];
                }
                __syncthreads();
                if (ctrl && c >= 0) put_all(tx + c, tl.xs, (xo + sm.red[j][q]) + bo, TE);
                __syncthreads();
            } else if (l + 1 < L) {
                if (has_item && !ctrl) {
                    load_keys(l + 1);
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int c = 0; c < 4; c++) sm.kv[wave][4 * i + c][lane] = kq[i][c];
#pragma unroll
                    for (int jj = 0; jj < KPW; jj++) sm.kv[wave][16 + jj][lane] = vr[jj];
                }
            }
            // wb[0, U): the next c_proj (layer 0's for the next step after
            // the last layer, then also the lm_head's rounds 2 and 3)
            load_cols<1, U>(wb, layers[l + 1 < L ? l + 1 : 0].proj_w, C, C, cw, CW, lane);
            if (l + 1 == L) load_cols<2, U, 2 * U>(wa, a.wte, V, C, cw + 2 * CW, CW, lane);
            bo = inq ? slot_bias_a(PN.attn_b, C3, qf) : 0.f;
        }

        // ---------------- phase F: final LayerNorm, lm_head (tied wte), argmax partials
        const unsigned TF = sbase + PHASES * L + 1;
        if (!fetch_ln(TF - 1, false, 0, 0)) return;
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
                            const float d = dot4(wa[k * U + i], sm.act[min(f, K4 - 1)]);
                            s += f < K4 ? d : 0.f;
                        }
                        const int nc = col + CW * UPW;
                        if (nc < V) {
                            const float* row = a.wte + (long)nc * C;
#pragma unroll
                            for (int i = 0; i < U; i++)
                                wa[k * U + i] = ldg4(row + 4 * min(i * 64 + ln, K4 - 1));
                        } else {
#pragma unroll
                            for (int i = 0; i < U; i++) wa[k * U + i] = f32x4{0.f, 0.f, 0.f, 0.f};
                        }
                        s = wave_sum_dpp(s);
                        if (ln == 0 && a.logits) a.logits[col] = s;
                        if (samp && ln == 0) sm.sx[wave * SK_RMAX + r] = s / tdiv;
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
        // the next step's QKV workgroups (its position is t + 1)
        q0 = qkv_first(t + 1, C, H, G);
        bo = (int)blockIdx.x >= q0 ? slot_bias_a(layers[0].attn_b, C3, q0) : 0.f;
        // sampling: the workgroup's scaled logits (wavefront w holds the
        // first rounds_w of sx[w][.]), their max m_g and sum of expf(x - m_g)
        auto own_logit = [&](bool& have, int& col) -> float {
            const int tt = opaque_v(tid);
            const int w = tt / SK_RMAX, r = tt - w * SK_RMAX;
            col = blockIdx.x * PW + w + CW * r;
            have = w < PW && col < V;
            return have ? sm.sx[min(tt, PW * SK_RMAX - 1)] : -INFINITY;
        };
        if (samp) {
            bool shave;
            int scol;
            const float sxv = own_logit(shave, scol);
            const float mg = block_max(sxv, sm.wred, wave, lane1);
            const float sg = block_sum(shave ? expf(sxv - mg) : 0.f, sm.wred, wave, lane1);
            if (ctrl && lane1 == 0) {
                put_all(tam + 2 * blockIdx.x, tl.as, mg, TF);
                put_all(tam + 2 * blockIdx.x + 1, tl.as, sg, TF);
            }
        } else if (ctrl && lane1 == 0) {
            float b = sm.bestv[0];
            int bi = sm.besti[0];
            for (int v = 1; v < PW; v++)
                if (better(sm.bestv[v], sm.besti[v], b, bi)) {
                    b = sm.bestv[v];
                    bi = sm.besti[v];
                }
            put_all(tam + 2 * blockIdx.x, tl.as, b, TF);
            put_all(tam + 2 * blockIdx.x + 1, tl.as, __int_as_float(bi), TF);
        }
        if (step + 1 < a.n_steps && (int)blockIdx.x >= q0) {
            load_cols<NJA, U>(wa, layers[0].attn_w, C3, C, qkv_wave(q0), PW * (G - q0), lane1);
            ln_params(layers[0].ln1_w, layers[0].ln1_b);
        }

        // ---------------- phase G: every workgroup reduces the argmax partials
        if (samp) {
            // G1: M and S over the workgroups' (m_g, s_g); the lower bound L
            // of the top_k-th largest scaled logit: the top_k-th largest m_g
            // (top_k workgroups hold a value >= it; top_k <= G)
            const int tt = opaque_v(tid);
            const int g = min(tt, G - 1);
            int idx[2] = {2 * g, 2 * g + 1};
            bool need[2] = {tt < G, tt < G};
            float pv[2];
            if (!settle(fetch<2>(ram, idx, need, TF, pv, abortw, amark))) return;
            const float mg = tt < G ? pv[0] : -INFINITY;
            if (tt < G + 4) sm.ml[0][tt] = mg;
            const float M = block_max(mg, sm.wred, wave, lane1);
            const float S = block_sum(tt < G ? pv[1] * expf(mg - M) : 0.f, sm.wred, wave, lane1);
            if (tt < G) {
                // (entries G .. G+3 hold -inf: the float4 reads stay in range)
                int gt = 0, ge = 0;
                const f32x4* m4 = (const f32x4*)sm.ml[0];
                for (int u = 0; u < (G + 3) / 4; u++) {
                    const f32x4 o = m4[u];
                    gt += (o.x > mg) + (o.y > mg) + (o.z > mg) + (o.w > mg);
                    ge += (o.x >= mg) + (o.y >= mg) + (o.z >= mg) + (o.w >= mg);
                }
                if (gt < a.top_k && a.top_k <= ge) sm.sL = mg;
            }
            if (tid == 0) sm.n_c = 0;
            __syncthreads();
            const float pL = expf(sm.sL - M) / S;
            // candidates of this workgroup: p >= p(L), which holds every
            // value with p >= t, t = p(top_k-th largest) >= p(L)
            bool shave;
            int scol;
            const float sxv = own_logit(shave, scol);
            if (shave && expf(sxv - M) / S >= pL) {
                const int q = atomicAdd(&sm.n_c, 1);
                if (q < SK_CMAX) {
                    sm.cx[q] = sxv;
                    sm.ci[q] = scol;
                }
            }
            __syncthreads();
            const unsigned TG = TF + 1;
            if (tid < SK_SLOT) {
                // (opaque indices: hoisted out of the step loop, these
                // addresses would take registers for the whole launch)
                const int tq = opaque_v(tid);
                const int m = max((tq - 1) >> 1, 0);
                const int nq = min(sm.n_c, SK_CMAX);
                float v = 0.f;
                if (tq == 0) v = __int_as_float(sm.n_c);
                else if (m < nq) v = (tq & 1) ? sm.cx[m] : __int_as_float(sm.ci[m]);
                put_all(tcd + opaque_v(blockIdx.x * SK_SLOT + tq), tl.cs, v, TG);
            }
            // G2: every workgroup gathers every candidate and draws the same
            // token (sample_top_k's arithmetic on the survivors, in index order)
            constexpr int NF = (256 * SK_SLOT + PT - 1) / PT;
            const int nw = G * SK_SLOT;
            int cidx[NF];
            bool cneed[NF];
            float cv[NF];
#pragma unroll
            for (int i = 0; i < NF; i++) {
                cidx[i] = min(tt + PT * i, nw - 1);
                cneed[i] = tt + PT * i < nw;
            }
            if (!settle(fetch<NF>(rcd, cidx, cneed, TG, cv, abortw, amark))) return;
            if (tid == 0) { sm.n_c = 0; sm.over = 0; sm.n_sv = 0; }
            // counts first (slot 0 of each workgroup), into ml[1]
#pragma unroll
            for (int i = 0; i < NF; i++) {
                const int e = tt + PT * i;
                if (cneed[i] && e % SK_SLOT == 0) sm.ml[1][e / SK_SLOT] = cv[i];
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < NF; i++) {
                const int e = tt + PT * i, gg = e / SK_SLOT, j = e - gg * SK_SLOT;
                if (!cneed[i]) continue;
                const int cnt = __float_as_int(sm.ml[1][gg]);
                if (j == 0 && cnt > SK_CMAX) sm.over = 1;
                // a pair's two words are fetched by different threads:
                // they meet in LDS
                if (j > 0 && ((j - 1) >> 1) < min(cnt, SK_CMAX)) sm.raw[gg * SK_SLOT + j] = cv[i];
            }
            __syncthreads();
            if (sm.over) {
                // more candidates than a workgroup publishes: the host draws
                // this step's token and continues with a new launch
                if (blockIdx.x == 0 && tid == 0) {
                    *a.tok = -1;
                    *a.pos = t + 1;
                    if (a.steps_done) *a.steps_done = step + 1;
                }
                return;
            }
            for (int q = tt; q < G * SK_CMAX; q += PT) {
                const int gg = q / SK_CMAX, m = q - gg * SK_CMAX;
                if (m < __float_as_int(sm.ml[1][gg])) {
                    const int d = atomicAdd(&sm.n_c, 1);
                    sm.cx[d] = sm.raw[gg * SK_SLOT + 1 + 2 * m];
                    sm.ci[d] = __float_as_int(sm.raw[gg * SK_SLOT + 2 + 2 * m]);
                }
            }
            __syncthreads();
            const int nc = sm.n_c;
            // c = the top_k-th largest candidate (equal values give equal c)
            for (int q = tt; q < nc; q += PT) {
                const float v = sm.cx[q];
                int gt = 0, ge = 0;
                for (int u = 0; u < nc; u++) {
                    const float o = sm.cx[u];
                    gt += o > v;
                    ge += o >= v;
                }
                if (gt < a.top_k && a.top_k <= ge) sm.sc = v;
            }
            __syncthreads();
            const float thr = expf(sm.sc - M) / S;
            for (int q = tt; q < nc; q += PT) {
                const float p = expf(sm.cx[q] - M) / S;
                if (p >= thr) {
                    const int d = atomicAdd(&sm.n_sv, 1);
                    sm.so[d] = p;
                    sm.soi[d] = sm.ci[q];
                }
            }
            __syncthreads();
            const int nsv = sm.n_sv;
            for (int q = tt; q < nsv; q += PT) {
                const int iq = sm.soi[q];
                int rank = 0;
                for (int u = 0; u < nsv; u++) rank += sm.soi[u] < iq;
                sm.cx[rank] = sm.so[q];
                sm.ci[rank] = iq;
            }
            __syncthreads();
            // wavefront 0: the renormalising sum and the running sum, each in
            // index order, 64 survivors per round read from the lanes
            if (wave == 0) {
                const float r = a.draws[step];
                float ns = 0.f;
                for (int q0 = 0; q0 < nsv; q0 += 64) {
                    const float pv = sm.cx[min(q0 + lane1, nsv - 1)];
                    const int m = min(64, nsv - q0);
                    for (int u = 0; u < m; u++) ns += lane_f(pv, u);
                }
                int tk = V - 1;
                float cdf = 0.f;
                for (int q0 = 0; q0 < nsv && tk == V - 1; q0 += 64) {
                    const float pv = sm.cx[min(q0 + lane1, nsv - 1)];
                    const float qv = ns > 0.0f ? pv / ns : pv;
                    const int iv = sm.ci[min(q0 + lane1, nsv - 1)];
                    const int m = min(64, nsv - q0);
                    for (int u = 0; u < m; u++) {
                        cdf += lane_f(qv, u);
                        if (r < cdf) {
                            tk = __builtin_amdgcn_readlane(iv, u);
                            break;
                        }
                    }
                }
                if (lane1 == 0) sm.stok = tk;
            }
            __syncthreads();
            tok = sm.stok;
            __syncthreads();
        } else {
            const int tt = opaque_v(tid);
            const int g = min(tt, G - 1);
            int idx[2] = {2 * g, 2 * g + 1};
            bool need[2] = {tt < G, tt < G};
            float pv[2];
            const bool ok = fetch<2>(ram, idx, need, TF, pv, abortw, amark);
            if (!settle(ok)) return;
            float b = tt < G ? pv[0] : -INFINITY;
            int bi = tt < G ? __float_as_int(pv[1]) : 0x7fffffff;
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
        if (a.steps_done) *a.steps_done = a.n_steps;
    }
}

template <int U>
hipError_t launch_u(const PersistArgs& a, int G, hipStream_t s) {
    void* args[] = {(void*)&a};
    const void* k = a.top_k > 0 ? (const void*)k_decode_persist<U, true>
                                : (const void*)k_decode_persist<U, false>;
    return hipLaunchCooperativeKernel(k, dim3(G), dim3(PT), args, 0,
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
    return std::min(cus, PT);
}

long persist_tagged_words(int C, int H) { return TagLayout(C, H).words(); }

unsigned persist_tags(int L, int n_steps) { return (unsigned)n_steps * (PHASES * L + 2) + 1; }

bool persist_supported(int C, int H, int V, int cap, int G) {
    if (G < 1 || G > PT || C % 64 || C != 64 * H || C > 256 * PMAXU || H > 32)
        return false;
    const long CW = (long)PW * G;
    // columns per wavefront: QKV and fc at most NJQ, c_proj and proj one
    if (4L * C > NJQ * CW || C > CW || V < 1) return false;
    // attention: H * splits workgroups after the c_proj / proj column
    // owners, at most PW * KPW keys per split; QKV on those workgroups
    const int owners = (C + PW - 1) / PW;
    if (owners >= G || 3L * C > (long)NJA * PW * (G - owners)) return false;   // (qkv_first)
    const int ns = std::min((G - owners) / H, PMAXS);
    if (ns < 1 || (long)ns * PW * KPW < cap) return false;
    return true;
}

bool persist_sampling_supported(int V, int G, int top_k) {
    const long CW = (long)PW * G;
    return top_k > 0 && top_k <= SK_MAX && top_k <= G && top_k < V && G <= 256 &&
           (V + CW - 1) / CW <= SK_RMAX;
}

hipError_t launch_decode_persist(const PersistArgs& a, int G, hipStream_t s) {
    // No clearing before a launch: an abort word left by an earlier launch
    // holds a smaller value than this launch's mark.
    switch ((a.C + 255) / 256) {
        case 1: return launch_u<1>(a, G, s);
        case 2: return launch_u<2>(a, G, s);
        case 3: return launch_u<3>(a, G, s);
        default: return hipErrorInvalidValue;
    }
}
