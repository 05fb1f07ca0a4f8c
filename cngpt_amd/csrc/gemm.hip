// gemm.hip - fp32 products Y[M,N] = epi(X[M,K] . W[N,K]^T) on gfx950.
//
// The reference computes every linear layer as cblas_sgemm(RowMajor,
// NoTrans, Trans) with a per-row saxpy bias and beta = 1 for the residual
// (fast.c:175-205). Both operands are K-contiguous, so both tiles are staged
// in LDS the same way and read back with 16-byte LDS reads.
//
// k_gemm_dl / k_gemm: 128x128 output tile per 256-thread workgroup, K in
// steps of BK. Each wavefront owns a 64x64 sub-tile = 2x2 blocks of
// v_mfma_f32_32x32x2f32. Inside a K step, lanes 0-31 feed the first half of
// the step's k and lanes 32-63 the second half, so each lane reads 4
// contiguous floats per row per LDS read. The epilogue adds bias / GELU /
// residual and stores straight from the accumulators (one 128-byte row
// segment per half wavefront). Ragged M and N edges (e.g. the 50257-wide
// vocabulary) clamp loads to the last valid row and mask stores.
//
// k_gemm_dl (K a multiple of BK): tiles go from global memory straight into
// LDS (global_load_lds_dwordx4, no registers on the way) through a ring of
// S stages, so the loads of S - 1 steps are in flight while one step is
// multiplied, and each step costs one wait and one barrier. A wavefront's
// load instruction fills 64 consecutive 16-byte granules, so the granule
// order within a row is XOR-swizzled by the row (rows that share LDS banks
// get different k quads at a given address) instead of padded: the 16
// lanes of a quarter-wavefront reading 16 rows at one k quad hit 16
// different granules of a 256-byte bank line.
//
// k_gemm (any K that is a multiple of 4): global loads into registers for
// step k+1 while step k is multiplied, then into a padded LDS double buffer;
// the last step zero-fills past K.
//
// k_stream: up to 128 rows (32 < M <= 128 when 128 x 128 tiles would be
// too few and K is not a multiple of 64; k_rows otherwise), weights
// streamed once (from their packed copy when the caller has one), input
// rows through LDS, K split over workgroups when the column tiles are few,
// or over the wavefronts of narrower tiles up to 32 rows.
//
// k_rows: 32 < M <= 128 rows, 32-row tiles, both operands through an LDS
// ring, the four wavefronts splitting every stage's k.
//
// Products over M <= 2 rows (single-sequence decode) are k_dgemv in
// decode.hip.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace {

constexpr int BM = 128, BN = 128;
constexpr int NTHREADS = 256;

// Workgroups are dispatched round-robin over the 8 XCDs (pid % 8). Renumber
// them so that each XCD receives a contiguous run of work ids (of nt).
__device__ __forceinline__ int xcd_order(int pid, int nt) {
    const int per = nt / 8, rem = nt % 8;
    const int xcd = pid % 8, idx = pid / 8;
    return (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// Tile of work id p: tiles in groups of 8 M-tiles, so that neighbours share
// A rows and W rows in the XCD's L2.
__device__ __forceinline__ void group_coords(int p, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int GM = 8;
    const int group = p / (GM * tiles_n);
    const int first_m = group * GM;
    const int gsize = min(tiles_m - first_m, GM);
    const int in_group = p % (GM * tiles_n);
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
    group_coords(xcd_order(pid, tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
}

// Epilogue of one wavefront's 64 x 64 block at (r0, c0): acc[i][j][r] is
// row r0 + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4, column c0 + 32 j +
// lane % 32. The bias is read once per column, and with the residual the
// old values of a block are all loaded before its first store: the
// compiler cannot tell that a store leaves the later loads' addresses
// alone, and element by element would wait for each load in turn. A block
// wholly inside a plain row-major output takes one base address and
// constant row steps; edge blocks and segmented rows map each row, load
// from clamped rows and columns (inside the output) and mask the stores.
// Same arithmetic as apply_epi.
template <int EPI>
__device__ __forceinline__ float epi_value(float v, float b, float old) {
    if (EPI == EPI_STORE) return v;
    if (EPI == EPI_BIAS) return v + b;
    if (EPI == EPI_BIAS_GELU) return gelu_tanh(v + b);
    return (old + v) + b;
}

template <int EPI>
__device__ __forceinline__ void tile_store(const GemmArgs& a, const f32x16 (&acc)[2][2], int r0,
                                           int c0, int lane) {
    const int lr = lane & 31, lh = lane >> 5;
    const long roff = a.row_off + (a.row_off_dev ? *a.row_off_dev : 0);
    const long ldy = a.ldy;
    float bj[2];
#pragma unroll
    for (int j = 0; j < 2; j++) bj[j] = EPI == EPI_STORE ? 0.f : a.bias[min(c0 + 32 * j + lr, a.N - 1)];
    if (!a.seg && r0 + 64 <= a.M && c0 + 64 <= a.N && ldy <= (1L << 27)) {
        // The row pointer of each 4-row group is uniform over the wavefront
        // (scalar registers); a lane adds one unsigned 32-bit byte offset,
        // the same for every element: 4 * (4 ldy + 31) < 2^32 for row
        // strides up to 2^27 floats.
        const unsigned lob = 4u * (unsigned)(4 * lh * ldy + lr);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                auto at = [&](int r) {
                    const float* rowp = a.Y + (r0 + 32 * i + 8 * (r >> 2) + (r & 3) + roff) * ldy + c0 + 32 * j;
                    return (float*)((char*)rowp + lob);
                };
                float old[16];
                if (EPI == EPI_RESID) {
#pragma unroll
                    for (int r = 0; r < 16; r++) old[r] = *at(r);
                }
#pragma unroll
                for (int r = 0; r < 16; r++)
                    *at(r) = epi_value<EPI>(acc[i][j][r], bj[j], EPI == EPI_RESID ? old[r] : 0.f);
            }
        return;
    }
    // edge blocks: the bias and each group's values are pinned (an empty
    // asm that takes and returns them) before the group's masked stores;
    // formed inside the masked blocks, each would wait for every store
    // issued before it (the wait counter counts stores too)
    asm volatile("" : "+v"(bj[0]), "+v"(bj[1]));
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = c0 + 32 * j + lr, cc = min(col, a.N - 1);
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                long ro[4];
                float y[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = min(r0 + 32 * i + 8 * r4 + 4 * lh + r, a.M - 1);
                    const long orow = a.seg ? (long)(row / a.seg) * a.seg_stride + row % a.seg : row;
                    ro[r] = (orow + roff) * ldy;
                    y[r] = EPI == EPI_RESID ? a.Y[ro[r] + cc] : 0.f;
                }
#pragma unroll
                for (int r = 0; r < 4; r++) y[r] = epi_value<EPI>(acc[i][j][4 * r4 + r], bj[j], y[r]);
                asm volatile("" : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]));
                if (col >= a.N) continue;
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (r0 + 32 * i + 8 * r4 + 4 * lh + r < a.M) a.Y[ro[r] + col] = y[r];
            }
        }
}

// One output element of row `row` (mapped through seg / row offsets) with
// the epilogue.
template <int EPI>
__device__ __forceinline__ void store_out(const GemmArgs& a, long roff, int row, int col, float v) {
    long orow = a.seg ? (long)(row / a.seg) * a.seg_stride + row % a.seg : row;
    orow += roff;
    float* y = a.Y + orow * a.ldy + col;
    *y = apply_epi<EPI>(v, a.bias, col, y);
}

// Stage layout: operand tile of BM rows x BK floats, granule (16 bytes) g
// at row g / GPR, slot g % GPR, where slot s of row r holds k quad
// s ^ ((r / RSW) % GPR) (RSW = rows per 256 bytes). The MFMA order over k
// is that of k_gemm with the same BK, so both give the same bits.
template <int BK, int S>
struct DlSmem {
    float sm[S * 2 * BM * BK];
};

// acc = X[m0.., kb..] . W[n0.., kb..]^T over nk steps of BK (acc zeroed
// first). On return every wavefront is done reading the stages it used only
// once the caller passes a barrier.
//
// KM (bit 0: X, bit 1: W) marks an operand stored K-major, row k of
// a.ldx / a.ldw floats holding the tile's rows as columns (the backward's
// dW = dY^T X reads dY and X this way instead of transposing them). Its
// stage holds BK rows of k, 32 granules of 4 rows (m or n) each; the
// granule order of the second half of the rows (the k the upper half
// wavefront reads) is XORed with 8, which puts the two half-wavefronts'
// reads of one row range 128 bytes apart, in different LDS banks. A lane
// then reads its 4 k one row apart instead of as one 16-byte read.
template <int BK, int S, int KM = 0>
__device__ __forceinline__ void dl_tile(const GemmArgs& a, int m0, int n0, int kb, int nk,
                                        float* sm, int wave, int lane, f32x16 (&acc)[2][2]) {
    constexpr int GPR = BK / 4;      // granules per row
    constexpr int RSW = 16 / GPR;    // rows per 256 bytes
    constexpr int NI = GPR / 2;      // load instructions per operand per stage per wavefront
    constexpr int NG = BK / 8;       // MFMA groups per step
    constexpr int TILE = BM * BK;    // floats per operand per stage
    constexpr bool XKM = KM & 1, WKM = KM & 2;
    static_assert(BM == BN && BM * GPR == NI * 4 * 64, "one granule per lane per instruction");
    const int K = a.K;

    // granule (i * 4 + wave) * 64 + lane of each operand, every stage
    const float* xp[NI];
    const float* wp[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int g = (i * 4 + wave) * 64 + lane;
        const int row = g / GPR, kq = (g % GPR) ^ ((row / RSW) % GPR);
        // K-major: row k = g / 32 of the stage, columns 4 * mq .. + 3
        const int kr = g / (BM / 4), mq = (g % (BM / 4)) ^ ((((2 * kr) / BK) & 1) << 3);
        if (XKM) xp[i] = a.X + (long)(kb + kr) * a.ldx + min(m0 + 4 * mq, (int)a.ldx - 4);
        else xp[i] = a.X + (long)min(m0 + row, a.M - 1) * K + kb + 4 * kq;
        if (WKM) wp[i] = a.W + (long)(kb + kr) * a.ldw + min(n0 + 4 * mq, (int)a.ldw - 4);
        else wp[i] = a.W + (long)min(n0 + row, a.N - 1) * K + kb + 4 * kq;
    }
    const long xstep = XKM ? BK * a.ldx : BK, wstep = WKM ? BK * a.ldw : BK;
    auto issue = [&](int kt, int st) {
        float* base = sm + st * 2 * TILE;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            float* la = base + (i * 4 + wave) * 64 * 4;
            __builtin_amdgcn_global_load_lds((const void*)(xp[i] + kt * xstep), (lds_void*)la, 16, 0,
                                             0);
            __builtin_amdgcn_global_load_lds((const void*)(wp[i] + kt * wstep), (lds_void*)(la + TILE),
                                             16, 0, 0);
        }
    };

    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int lr = lane & 31, lh = lane >> 5;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
    // LDS offsets (floats) of this lane's reads: group g, k quad lh * NG + g
    int ao[2][NG], bo[2][NG];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const int ra = wm + i * 32 + lr, rb = wn + i * 32 + lr, kq = lh * NG + g;
            ao[i][g] = ra * BK + 4 * (kq ^ ((ra / RSW) % GPR));
            bo[i][g] = TILE + rb * BK + 4 * (kq ^ ((rb / RSW) % GPR));
        }

#pragma unroll
    for (int st = 0; st < S - 1; st++)
        if (st < nk) issue(st, st);
    for (int kt = 0; kt < nk; kt++) {
        // this step's granules are in LDS once at most the later steps'
        // loads (2 * NI instructions each) are outstanding
        if (kt + S - 2 < nk) wait_vmcnt<2 * NI * (S - 2)>();
        else wait_vmcnt<0>();
        // every wavefront's granules of this step have landed, and every
        // wavefront is done with the stage the next issue overwrites. A
        // bare barrier: __syncthreads' fence would also wait for the later
        // steps' loads.
        asm volatile("s_barrier" ::: "memory");
        if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
        const float* base = sm + (kt % S) * 2 * TILE;
        // The workgroups sharing a CU (two or four) run the same step
        // sequence: at raised priority for its products, a wavefront keeps
        // the SIMD's matrix unit fed while another workgroup's wavefront, at
        // the normal priority, waits, passes its barrier and issues its
        // loads, so they drift apart instead of stalling the unit together
        // (GPT-2 small B=16 T=1024 GEMM class 83.0 -> 84.2 % of peak at two
        // per CU).
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int g = 0; g < NG; g++) {
            f32x4 av[2], bv[2];
            const int ka = 4 * (lh * NG + g);  // first k of this lane's 4 (K-major stages)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                if (XKM) {
                    const float* p = base + ka * BM + ((wm + i * 32 + lr) ^ (32 * lh));
                    av[i] = f32x4{p[0], p[BM], p[2 * BM], p[3 * BM]};
                } else {
                    av[i] = *(const f32x4*)&base[ao[i][g]];
                }
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if (WKM) {
                    const float* p = base + TILE + ka * BN + ((wn + j * 32 + lr) ^ (32 * lh));
                    bv[j] = f32x4{p[0], p[BN], p[2 * BN], p[3 * BN]};
                } else {
                    bv[j] = *(const f32x4*)&base[bo[j][g]];
                }
            }
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][e], bv[j][e],
                                                                          acc[i][j], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
    }
}

// A partial tile (all BM x BN values, rows of BN floats) at p.
__device__ __forceinline__ void store_partial(float* p, const f32x16 (&acc)[2][2], int wave,
                                              int lane) {
    GemmArgs pa{};
    pa.Y = p;
    pa.M = BM; pa.N = BN; pa.ldy = BN;
    tile_store<EPI_STORE>(pa, acc, (wave >> 1) * 64, (wave & 1) * 64, lane);
}

// One 128 x 128 tile per workgroup. Split K (KS > 1, for launches with too
// few tiles to fill the CUs): work id ks * tiles + tile covers k in
// [ks * KR, min(K, (ks + 1) * KR)) and stores its partial tile to a.part +
// ks * M * N (rows of N floats); the reduce kernel sums the KS partials in
// order and applies the epilogue.
template <int EPI, int BK, int S, int OCC, int KM = 0>
__global__ void __launch_bounds__(NTHREADS, OCC) k_gemm_dl(GemmArgs a, int tiles_m, int tiles_n,
                                                          int KR, int KS) {
    __shared__ __attribute__((aligned(1024))) DlSmem<BK, S> sh;
    const int tiles = tiles_m * tiles_n;
    int p = xcd_order(blockIdx.x, tiles * KS);
    const int ks = p / tiles;
    p -= ks * tiles;
    int tm, tn;
    group_coords(p, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int kb = ks * KR;
    f32x16 acc[2][2];
    dl_tile<BK, S, KM>(a, m0, n0, kb, min(KR, a.K - kb) / BK, sh.sm, wave, lane, acc);
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    if (KS == 1) {
        tile_store<EPI>(a, acc, m0 + wm, n0 + wn, lane);
        return;
    }
    GemmArgs pa = a;
    pa.Y = a.part + (long)ks * a.M * a.N;
    pa.ldy = a.N;
    pa.seg = 0;
    pa.row_off = 0;
    pa.row_off_dev = nullptr;
    tile_store<EPI_STORE>(pa, acc, m0 + wm, n0 + wn, lane);
}

// Stream-K (launches whose last round of tiles would leave workgroup slots
// idle), after dp rounds of whole tiles: in round r workgroup g computes
// tile r * G + g whole, so the tiles of a round advance through k together
// and an XCD's workgroups (g XCD-contiguous, tiles in the 8-row groups)
// share their A row slices and W column slices in its L2. The I = (tiles -
// dp * G) * nkt steps of BK of the remaining tiles, tile-major, are cut into
// G equal contiguous ranges, one per workgroup. A workgroup computes the
// tiles its range covers whole and stores them with the epilogue; the part
// of a tile at either end of its range goes to a partial slot (2g for the
// first tile of workgroup g, 2g + 1 for its last), and k_sk_fixup sums each
// split tile's partials in k order and applies the epilogue.
__device__ __forceinline__ long sk_begin(long g, long I, int G) { return g * I / G; }
// workgroup whose range holds step i
__device__ __forceinline__ int sk_owner(long i, long I, int G) {
    return (int)(((i + 1) * G - 1) / I);
}

template <int EPI>
__global__ void __launch_bounds__(NTHREADS, 2) k_gemm_sk(GemmArgs a, int tiles_m, int tiles_n,
                                                         int nkt, int G, int dp) {
    constexpr int BK = 32, S = 2;
    __shared__ __attribute__((aligned(1024))) DlSmem<BK, S> sh;
    const int tiles = tiles_m * tiles_n;
    const int g = xcd_order(blockIdx.x, G);
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    for (int r = 0; r < dp; r++) {
        int tm, tn;
        group_coords(r * G + g, tiles_m, tiles_n, tm, tn);
        f32x16 acc[2][2];
        dl_tile<BK, S>(a, tm * BM, tn * BN, 0, nkt, sh.sm, wave, lane, acc);
        tile_store<EPI>(a, acc, tm * BM + wm, tn * BN + wn, lane);
        // the next tile's first loads overwrite stages this one read
        __syncthreads();
    }
    const int t0 = dp * G;  // first stream-K tile
    const long I = (long)(tiles - t0) * nkt;
    const long beg = sk_begin(g, I, G), end = sk_begin(g + 1, I, G);
    const int first = (int)(beg / nkt);
    for (long it = beg; it < end;) {
        const int t = (int)(it / nkt), k0 = (int)(it - (long)t * nkt);
        const int k1 = (int)min((long)nkt, k0 + (end - it));
        int tm, tn;
        group_coords(t0 + t, tiles_m, tiles_n, tm, tn);
        f32x16 acc[2][2];
        dl_tile<BK, S>(a, tm * BM, tn * BN, k0 * BK, k1 - k0, sh.sm, wave, lane, acc);
        if (k0 == 0 && k1 == nkt)
            tile_store<EPI>(a, acc, tm * BM + wm, tn * BN + wn, lane);
        else
            store_partial(a.part + (long)(2 * g + (t == first ? 0 : 1)) * BM * BN, acc, wave, lane);
        it += k1 - k0;
        // the next tile's first loads overwrite stages this one read
        __syncthreads();
    }
}

// Every tile split over workgroups: its partials summed in k order (the
// workgroups in order), then the epilogue. SK_RPW rows of a tile per
// workgroup; tiles that one workgroup computed whole return at once. A tile
// meets at most SK_SEGS workgroup ranges (each range holds at least nkt / 2
// steps, since stream-K runs with more tiles than half its workgroups).
constexpr int SK_RPW = 16;
constexpr int SK_SEGS = 4;
template <int EPI>
__global__ void __launch_bounds__(256) k_sk_fixup(GemmArgs a, int tiles_m, int tiles_n, int nkt,
                                                  int G, int t0) {
    // tile t0 + t of the stream-K tiles (those after the whole-tile rounds)
    const int tiles = tiles_m * tiles_n;
    const long I = (long)(tiles - t0) * nkt;
    const int t = blockIdx.x / (BM / SK_RPW), rb = blockIdx.x % (BM / SK_RPW);
    const int g0 = sk_owner((long)t * nkt, I, G), g1 = sk_owner((long)(t + 1) * nkt - 1, I, G);
    if (g0 == g1) return;
    int slot[SK_SEGS];
    const int ns = min(g1 - g0 + 1, SK_SEGS);
#pragma unroll
    for (int q = 0; q < SK_SEGS; q++) {
        const int g = min(g0 + q, g1);
        slot[q] = 2 * g + ((int)(sk_begin(g, I, G) / nkt) == t ? 0 : 1);
    }
    int tm, tn;
    group_coords(t0 + t, tiles_m, tiles_n, tm, tn);
    const long roff = a.row_off + (a.row_off_dev ? *a.row_off_dev : 0);
    // float4 c4 = tid + 256 i of this workgroup's SK_RPW rows: row
    // rb * SK_RPW + c4 / 32, columns 4 (c4 % 32) ..; the residual and the
    // bias as float4 where the four columns are inside the output and its
    // rows are 16-byte aligned, else one by one
    constexpr int NI = SK_RPW * BN / 4 / 256;
    const bool vec = (a.ldy & 3) == 0 && ((size_t)a.Y & 15) == 0;
    // the residual and bias are loaded with the partials: a load after the
    // first store would wait for that store too (the vector-memory counter
    // counts both), one round trip per element
    f32x4 p[NI][SK_SEGS], old[NI], bb[NI];
    int row[NI], col[NI];
    long yo[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c4 = threadIdx.x + 256 * i;
        const int r = rb * SK_RPW + (c4 >> 5), c = (c4 & 31) * 4;
        row[i] = tm * BM + r;
        col[i] = tn * BN + c;
#pragma unroll
        for (int q = 0; q < SK_SEGS; q++)
            p[i][q] = q < ns ? *(const f32x4*)(a.part + (long)slot[q] * BM * BN + r * BN + c)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
        const int rr = min(row[i], a.M - 1);
        long orow = a.seg ? (long)(rr / a.seg) * a.seg_stride + rr % a.seg : rr;
        yo[i] = (orow + roff) * a.ldy;
        const bool whole = vec && col[i] + 3 < a.N;
        if (EPI == EPI_RESID) {
            if (whole) old[i] = *(const f32x4*)(a.Y + yo[i] + col[i]);
            else
#pragma unroll
                for (int e = 0; e < 4; e++) old[i][e] = a.Y[yo[i] + min(col[i] + e, a.N - 1)];
        }
        if (EPI != EPI_STORE) {
            if (col[i] + 3 < a.N) bb[i] = f32x4{a.bias[col[i]], a.bias[col[i] + 1], a.bias[col[i] + 2],
                                                a.bias[col[i] + 3]};
            else
#pragma unroll
                for (int e = 0; e < 4; e++) bb[i][e] = a.bias[min(col[i] + e, a.N - 1)];
        }
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
        f32x4 v = p[i][0];
        for (int q = 1; q < ns; q++) v += p[i][q];
        // a tile met by more ranges than SK_SEGS (not produced by the
        // stream-K launch's shapes) sums the rest here
        for (int g = g0 + SK_SEGS; g <= g1; g++) {
            const int sl = 2 * g + ((int)(sk_begin(g, I, G) / nkt) == t ? 0 : 1);
            const int c4 = threadIdx.x + 256 * i;
            v += *(const f32x4*)(a.part + (long)sl * BM * BN + (rb * SK_RPW + (c4 >> 5)) * BN +
                                 (c4 & 31) * 4);
        }
        if (row[i] >= a.M) continue;
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            y[e] = v[e];
            if (EPI == EPI_BIAS) y[e] += bb[i][e];
            else if (EPI == EPI_BIAS_GELU) y[e] = gelu_tanh(y[e] + bb[i][e]);
            else if (EPI == EPI_RESID) y[e] = (old[i][e] + y[e]) + bb[i][e];
        }
        if (vec && col[i] + 3 < a.N) {
            *(f32x4*)(a.Y + yo[i] + col[i]) = y;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (col[i] + e < a.N) a.Y[yo[i] + col[i] + e] = y[e];
        }
    }
}

template <int EPI, int BK, int PAD, int OCC>
__global__ void __launch_bounds__(NTHREADS, OCC) k_gemm(GemmArgs a, int tiles_m, int tiles_n) {
    constexpr int LDS_ROW = BK + PAD;            // padded row, keeps 16-byte alignment
    constexpr int KQ = BK / 4;                   // float4 per row per K step
    constexpr int RPI = NTHREADS / KQ;           // rows covered per load iteration
    constexpr int A_ITERS = BM / RPI;            // float4 loads per thread per tile
    constexpr int B_ITERS = BN / RPI;
    __shared__ float As[2][BM * LDS_ROW];
    __shared__ float Bs[2][BN * LDS_ROW];

    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x;
    const int K = a.K;

    // Global -> register staging: thread covers rows tid/KQ + RPI*i, float4 kq.
    const int kq = (tid % KQ) * 4, r0 = tid / KQ;
    const float* xp[A_ITERS];
    const float* wp[B_ITERS];
#pragma unroll
    for (int i = 0; i < A_ITERS; i++) {
        int r = m0 + r0 + RPI * i;
        xp[i] = a.X + (long)min(r, a.M - 1) * K + kq;
    }
#pragma unroll
    for (int i = 0; i < B_ITERS; i++) {
        int r = n0 + r0 + RPI * i;
        wp[i] = a.W + (long)min(r, a.N - 1) * K + kq;
    }
    f32x4 ra[A_ITERS], rb[B_ITERS];
    auto gload = [&](int k0) {
        const bool ok = (k0 + kq) < K;
#pragma unroll
        for (int i = 0; i < A_ITERS; i++)
            ra[i] = ok ? *(const f32x4*)(xp[i] + k0) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < B_ITERS; i++)
            rb[i] = ok ? *(const f32x4*)(wp[i] + k0) : f32x4{0.f, 0.f, 0.f, 0.f};
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_ITERS; i++) *(f32x4*)&As[buf][(r0 + RPI * i) * LDS_ROW + kq] = ra[i];
#pragma unroll
        for (int i = 0; i < B_ITERS; i++) *(f32x4*)&Bs[buf][(r0 + RPI * i) * LDS_ROW + kq] = rb[i];
    };

    const int wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int lr = lane & 31, lh = lane >> 5;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    const int nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
        const float* as = &As[cur][0];
        const float* bs = &Bs[cur][0];
#pragma unroll
        for (int g = 0; g < BK / 8; g++) {
            const int kk = lh * (BK / 2) + g * 4;
            f32x4 av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; i++) av[i] = *(const f32x4*)&as[(wm + i * 32 + lr) * LDS_ROW + kk];
#pragma unroll
            for (int j = 0; j < 2; j++) bv[j] = *(const f32x4*)&bs[(wn + j * 32 + lr) * LDS_ROW + kk];
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][e], bv[j][e],
                                                                          acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }

    tile_store<EPI>(a, acc, m0 + wm, n0 + wn, lane);
}

// ---------------------------------------------------------------- skinny

// k_stream: up to 128 rows (batched decode, last-position passes of larger
// batches, short prefills). Every weight is used by M rows only (at M = 32,
// 2 * 32 FLOP per 4-byte weight = 16 FLOP/B, near the fp32 ridge of
// 157.3 / 8 = 19.7; at decode sizes a launch's fixed cost, not its bytes,
// dominates: cache-resident weights gain 5-10 %), so each weight is read
// once and the input rows are shared out of LDS. A workgroup of ST_NW wavefronts owns
// ST_NT = 16 * ST_NW output columns over a K range [kb, ke), in steps of 16
// k: for its 16 columns a wavefront's lane l holds column l % 16, k = 4 (l /
// 16) .. +3 of a step, and the input rows of the range pass through LDS in
// chunks of ST_KC k. Products are v_mfma_f32_16x16x4f32 (16 rows x 16
// columns x 4 k), MB row blocks of 16.
//
// Both operands go from global memory straight into LDS (lds_dma16, no
// registers on the way), so the compiler neither waits for them nor moves
// them: input chunk c + 1 is issued when chunk c starts (double
// buffer, granules XOR-swizzled by row so the 16 rows a read instruction
// touches fall in different banks), and each wavefront streams its
// weights through a ring of ST_PF steps (1 KB each, one load instruction),
// the load of step s + ST_PF issued right after step s's products. The
// issue order is the same in every chunk but the last (which issues
// nothing), so each wait is a constant count of the loads issued after the
// one needed: the weights stay ST_PF steps in flight across chunk
// boundaries (a register ring loses that: the compiler waits for every load
// in flight at the top of each loop trip), and no load is in flight past
// the range.
// With PK the weights come from their packed copy (k_pack_w): the 1 KB of a
// wavefront's step is contiguous there instead of 16 rows x 64 bytes, each
// 128-byte line of W split over two steps (measured on a bare stream of the
// GPT-2 XL MLP weights, 1 KB units: 4.9 TB/s packed, 3.6 TB/s row-major).
// When the column tiles alone would leave CUs idle, K is split over KS
// workgroups that write partial tiles; k_stream_reduce then sums them in
// order and applies the epilogue (no atomics: the result is reproducible).
constexpr int ST_NW = 4;
constexpr int ST_NT = 16 * ST_NW;
constexpr int ST_MAX_M = 128;  // rows of the largest row-block count (MB = 8)
// Chunk length by row blocks: 128 k up to 64 rows, 64 k above (the input
// double buffer of 128 rows x 64 k plus the weight rings is 80 KB, two
// workgroups per CU).
constexpr int st_kc(int MB) { return MB > 4 ? 64 : 128; }
constexpr int st_mb(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : M <= 48 ? 3 : M <= 64 ? 4 : 8; }

// WPB > 1 (at most 32 rows): WPB wavefronts share each 16-column block,
// the workgroup owns 16 * ST_NW / WPB columns, the input chunk is WPB times
// longer and wavefront phase ph takes its steps ph, ph + WPB, ... (in
// packed weights the block's steps stay contiguous across the phases); at
// the end the phases' sums are added in phase order through LDS. Enough
// column tiles then fill the CUs without a K split, so no partial tiles and
// no sum launch.
template <int EPI, int MB, bool PK, int WPB>
__global__ void __launch_bounds__(ST_NW * 64) k_stream(GemmArgs a, int tiles_n, int KR, int KS) {
    constexpr int CBW = ST_NW / WPB;           // column blocks per workgroup
    constexpr int ST_KC = st_kc(MB) * WPB;     // k per input chunk
    constexpr int ST_PF = ST_KC / 16 / WPB;    // weight steps in flight = steps per
                                               // chunk per wavefront (<= 8)
    constexpr int ST_GPR = ST_KC / 4;    // input granules (16 bytes) per row of a chunk
    static_assert(ST_GPR >= 16 && ST_PF <= 8, "swizzle over 16 rows; waits of at most 7 + XI");
    constexpr int R = 16 * MB;                       // rows held (M <= R)
    constexpr int XI = R * ST_GPR / (ST_NW * 64);    // input load instructions per wavefront per chunk
    static_assert(XI * ST_NW * 64 == R * ST_GPR, "whole instructions");
    __shared__ __attribute__((aligned(1024))) float xs[2][R * ST_KC];
    __shared__ __attribute__((aligned(1024))) float ws[ST_NW][ST_PF][256];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lc = lane & 15, g4 = (lane >> 4) * 4;
    const int tn = blockIdx.x % tiles_n, ks = blockIdx.x / tiles_n;
    const int K = a.K, M = a.M, N = a.N;
    const int kb = ks * KR, ke = min(K, kb + KR);
    const int nchunks = (ke - kb + ST_KC - 1) / ST_KC;
    const int blk = wave % CBW, ph = wave / CBW;
    const int col = tn * 16 * CBW + 16 * blk + lc;
    const float* wrow = a.W + (long)min(col, N - 1) * K + g4;
    // packed: column block col / 16 (the last one for columns past N), its
    // k steps of 256 floats each, this lane's 16 bytes at 4 * lane
    const int KQ = (K + 15) >> 4;
    const float* wpk =
        PK ? a.Wp + (long)min(col >> 4, (N - 1) >> 4) * KQ * 256 + 4 * lane : nullptr;

    // input chunk c into buffer b: granule g = (i * ST_NW + wave) * 64 +
    // lane of the chunk sits at row g / ST_GPR, slot g % ST_GPR and holds k
    // quad slot ^ (row % 16); rows past M read row M - 1 and k past K reads
    // K - 4 (finite values whose products are discarded or multiply zeroed
    // weights)
    const float* xsrc[XI];
    int xslot[XI];
#pragma unroll
    for (int i = 0; i < XI; i++) {
        const int g = (i * ST_NW + wave) * 64 + lane;
        const int row = g / ST_GPR, slot = g % ST_GPR;
        xsrc[i] = a.X + (long)min(row, M - 1) * K;
        xslot[i] = 4 * (slot ^ (row & 15));
    }
    auto issue_x = [&](int c, const float* xd) {
        const int k0 = kb + c * ST_KC;
#pragma unroll
        for (int i = 0; i < XI; i++)
            lds_dma16(xsrc[i] + min(k0 + xslot[i], K - 4), &xd[(i * ST_NW + wave) * 256]);
    };
    // this wavefront's weight step s (k = kb + 16 (s WPB + ph) + g4 .. +3
    // of this lane's column; steps past the range re-read K - 4 and are
    // zeroed at use) into ring slot s % ST_PF
    auto issue_w = [&](int s) {
        const int st = s * WPB + ph;
        if (PK)
            lds_dma16(wpk + (long)min((kb >> 4) + st, KQ - 1) * 256, &ws[wave][s % ST_PF][0]);
        else
            lds_dma16(wrow + min(kb + 16 * st, K - 4 - g4), &ws[wave][s % ST_PF][0]);
    };

    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // chunk c (LAST: the final one, which issues no loads: nothing is left
    // in flight past the range, so none has to be waited for at the end)
    auto chunk = [&](int c, auto last_c) {
        constexpr bool LAST = decltype(last_c)::value;
        // chunk c has landed once at most the ST_PF weight loads issued
        // after it are in flight; the barrier then also frees the other
        // buffer (read in chunk c - 1) for chunk c + 1
        wait_vmcnt<ST_PF>();
        asm volatile("s_barrier" ::: "memory");
        if (!LAST) issue_x(c + 1, xs[(c + 1) & 1]);
        const float* xb = xs[c & 1];
        // the operands of step j: this lane's weight quad and input quads
        auto read_step = [&](int j, f32x4& w, f32x4 (&xf)[MB]) {
            w = *(const f32x4*)&ws[wave][j][4 * lane];
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
                const int r = 16 * mb + lc, q = 4 * (j * WPB + ph) + (lane >> 4);
                xf[mb] = *(const f32x4*)&xb[r * ST_KC + 4 * (q ^ (r & 15))];
            }
        };
        auto products = [&](int s, const f32x4& w, const f32x4 (&xf)[MB]) {
            const bool kok = kb + 16 * (s * WPB + ph) + g4 < ke;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float we = kok ? w[e] : 0.f;
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[mb][e], we, acc[mb], 0, 0, 0);
            }
        };
        if constexpr (MB == 1) {
#pragma unroll
            for (int j = 0; j < ST_PF; j++) {
                const int s = c * ST_PF + j;
                // step s has landed once at most the later ring loads and
                // the next chunk are in flight (in the last chunk: the later
                // ring loads only)
                if (LAST) wait_vmcnt_dyn<ST_PF>(ST_PF - 1 - j);
                else wait_vmcnt<ST_PF - 1 + XI>();
                asm volatile("" ::: "memory");
                f32x4 w, xf[MB];
                read_step(j, w, xf);
                products(s, w, xf);
                if (!LAST) {
                    // the slot is refilled only after its values are in registers
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    issue_w(s + ST_PF);
                }
            }
        } else {
            // two or more row blocks: each step's operands are read while the
            // previous step's products run (read right before its own
            // products, the LDS latency sat between every two steps; at one
            // row block the read-ahead measured no faster). Step jj has
            // landed once at most the ring loads after it, the next chunk's
            // input and the refills of the steps before jj - 1 are in
            // flight: ST_PF - 2 + XI whenever it is waited for, one step
            // ahead of its products (in the last chunk ST_PF - 1 - jj).
            auto wait_step = [&](int jj) {
                if (LAST) wait_vmcnt_dyn<ST_PF>(ST_PF - 1 - jj);
                else wait_vmcnt<ST_PF - 2 + XI>();
                asm volatile("" ::: "memory");
            };
            f32x4 wc, xc[MB];
            wait_step(1);
            read_step(0, wc, xc);
#pragma unroll
            for (int j = 0; j < ST_PF; j++) {
                const int s = c * ST_PF + j;
                f32x4 wn, xn[MB];
                if (j + 1 < ST_PF) {
                    if (j > 0) wait_step(j + 1);
                    read_step(j + 1, wn, xn);
                    // (the scheduler would otherwise sink the reads to their use)
                    __builtin_amdgcn_sched_barrier(0);
                }
                products(s, wc, xc);
                if (!LAST) {
                    // slot j is refilled only after its values are in
                    // registers: an empty statement that reads them makes the
                    // compiler wait for their LDS read (and not for step j + 1's)
                    asm volatile("" ::"v"(wc[0]), "v"(wc[1]), "v"(wc[2]), "v"(wc[3]) : "memory");
                    issue_w(s + ST_PF);
                }
                if (j + 1 < ST_PF) {
                    wc = wn;
#pragma unroll
                    for (int mb = 0; mb < MB; mb++) xc[mb] = xn[mb];
                }
            }
        }
    };
    issue_x(0, xs[0]);
#pragma unroll
    for (int j = 0; j < ST_PF; j++) issue_w(j);
    for (int c = 0; c + 1 < nchunks; c++) chunk(c, std::false_type{});
    chunk(nchunks - 1, std::true_type{});

    if constexpr (WPB > 1) {
        // phases 1.. hand their sums to phase 0 through the (now unused)
        // input buffers, which adds them in phase order
        __syncthreads();
        float* red = &xs[0][0];
        if (ph > 0)
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
                *(f32x4*)&red[(((ph - 1) * CBW + blk) * MB + mb) * 256 + 4 * lane] = acc[mb];
        __syncthreads();
        if (ph > 0) return;
#pragma unroll
        for (int p = 1; p < WPB; p++)
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
                acc[mb] += *(const f32x4*)&red[(((p - 1) * CBW + blk) * MB + mb) * 256 + 4 * lane];
    }

    // acc[mb][r]: row 16 mb + 4 (lane / 16) + r, column col
    if (col >= N) return;
    if (KS == 1) {
        const long roff = a.row_off + (a.row_off_dev ? *a.row_off_dev : 0);
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 16 * mb + g4 + r;
                if (row < M) store_out<EPI>(a, roff, row, col, acc[mb][r]);
            }
        return;
    }
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = 16 * mb + g4 + r;
            if (row < M) a.part[((long)ks * M + row) * N + col] = acc[mb][r];
        }
}

// Y = epi(sum over the KS partial tiles, in order); one thread per output.
// k_gemm_wide: TM x TN tiles (TM = 128, one workgroup per CU, or 64, two),
// whole K, for products whose 128 x 128 tiles leave a round of CUs
// part-empty (so they ran split-K or stream-K, with partials to sum) while
// a tile shape makes the tile count a whole number of rounds: at M = 2048
// (one GPU's share of B=16 T=1024) GPT-2 small's QKV (2304 columns) takes
// 128 x 144 tiles (256), fc (3072) 64 x 96 (1024), c_proj and proj (768)
// 64 x 48 (512). Wavefront w owns rows (TM / 4) w .. and every column of
// the tile: TM / 64 x TN / 16 blocks of v_mfma_f32_16x16x4f32. Both
// operands go global -> LDS (lds_dma16) through a ring of S stages of 32 k
// (the stage padded to a multiple of 32 rows, the pad loading clamped W
// rows that nothing reads); a stage is read in two 16-k halves, each half's
// operands read while the previous half's products issue, one wait and one
// barrier per stage between the halves. A stage row is 8 granules of 16
// bytes, granule slot s of row r holding k quad s ^ ((r / 2) % 8): two rows
// share a 256-byte bank line, and the 16 rows a read instruction touches at
// one k quad fall in 16 different 16-byte bank groups.
constexpr int WD_BK = 32;

template <int TM, int TN>
constexpr int wd_rows() {
    return (TM + TN + 31) / 32 * 32;
}

template <int EPI, int TM, int TN, int S>
__global__ void __launch_bounds__(256, 128 / TM) k_gemm_wide(GemmArgs a, int tiles_m, int tiles_n) {
    constexpr int ROWS = wd_rows<TM, TN>();  // stage rows: TM of X, TN of W, pad
    constexpr int NI = ROWS / 32;        // load instructions per wavefront and stage
    constexpr int STAGE = ROWS * WD_BK;  // floats per stage
    constexpr int CB = TN / 16;          // 16-column blocks
    constexpr int RB = TM / 64;          // 16-row blocks per wavefront
    static_assert(TN % 16 == 0 && S >= 3 && (TM == 64 || TM == 128), "tile shape");
    __shared__ __attribute__((aligned(1024))) float sm[S * STAGE];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    // work id XCD-contiguous, row tiles fastest: the row tiles of a column
    // tile share its W rows in one XCD's L2
    const int p = xcd_order(blockIdx.x, tiles_m * tiles_n);
    const int tm = p % tiles_m, tn = p / tiles_m;
    const int m0 = tm * TM, n0 = tn * TN;
    const int K = a.K, M = a.M, N = a.N;
    const int nk = K / WD_BK;
    // load instruction i of wavefront w covers stage rows 8 (4 i + w) ..
    // +7: lane -> row 8 (4 i + w) + lane / 8, slot lane % 8, holding k quad
    // slot ^ ((row / 2) % 8); rows past M or N (and the pad) read the last
    // one (finite values; their results are not stored)
    const float* src[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int row = 8 * (4 * i + wave) + (lane >> 3), slot = lane & 7;
        const int kq = slot ^ ((row >> 1) & 7);
        src[i] = row < TM ? a.X + (long)min(m0 + row, M - 1) * K + 4 * kq
                          : a.W + (long)min(n0 + row - TM, N - 1) * K + 4 * kq;
    }
    auto issue = [&](int kt, int st) {
        float* base = sm + st * STAGE;
#pragma unroll
        for (int i = 0; i < NI; i++) lds_dma16(src[i] + kt * WD_BK, base + (4 * i + wave) * 256);
    };
    // lane: row (column) 16 b + lane % 16 of each 16-block, k quad 4 h +
    // lane / 16 of half h; element e of the quad is the k of the e-th
    // product
    const int lc = lane & 15, g = lane >> 4;
    int ao[2][RB], bo[2][CB];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int q = 4 * h + g;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            const int r = 16 * RB * wave + 16 * rb + lc;
            ao[h][rb] = r * WD_BK + 4 * (q ^ ((r >> 1) & 7));
        }
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            const int r = TM + 16 * cb + lc;
            bo[h][cb] = r * WD_BK + 4 * (q ^ ((r >> 1) & 7));
        }
    }
    f32x4 acc[RB][CB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 a0[RB], b0[CB], a1[RB], b1[CB];
    auto read = [&](int kt, int h, f32x4(&av)[RB], f32x4(&bv)[CB]) {
        const float* base = sm + (kt % S) * STAGE;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) av[rb] = *(const f32x4*)&base[ao[h][rb]];
#pragma unroll
        for (int cb = 0; cb < CB; cb++) bv[cb] = *(const f32x4*)&base[bo[h][cb]];
    };
    auto mul = [&](const f32x4(&av)[RB], const f32x4(&bv)[CB]) {
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int cb = 0; cb < CB; cb++)
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[rb][e], bv[cb][e], acc[rb][cb], 0, 0, 0);
    };
#pragma unroll
    for (int st = 0; st < S - 1; st++)
        if (st < nk) issue(st, st);
    if (nk > 0) {
        // stage 0 has landed once at most stages 1 .. S - 2 are in flight
        if (S - 2 < nk) wait_vmcnt<NI * (S - 2)>();
        else wait_vmcnt<0>();
        asm volatile("s_barrier" ::: "memory");
        read(0, 0, a0, b0);
    }
    for (int kt = 0; kt < nk; kt++) {
        read(kt, 1, a1, b1);
        mul(a0, b0);
        if (kt + 1 < nk) {
            // stage kt + 1 has landed once at most stages kt + 2 .. kt + S -
            // 2 are in flight; past the barrier every wavefront has landed
            // its part of it and is done reading stage kt - 1 (both halves'
            // products issued before this point), which the next issue
            // overwrites
            if (kt + S - 2 < nk) wait_vmcnt<NI * (S - 3)>();
            else wait_vmcnt<0>();
            asm volatile("s_barrier" ::: "memory");
            if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
            read(kt + 1, 0, a0, b0);
        }
        mul(a1, b1);
    }
    // acc[rb][cb][r]: row m0 + (TM / 4) w + 16 rb + 4 (lane / 16) + r, column n0 +
    // 16 cb + lane % 16. The bias and the residual are loaded before the
    // first store: a load after a store would wait for that store too (the
    // vector-memory counter counts both), one round trip per element.
    const long roff = a.row_off + (a.row_off_dev ? *a.row_off_dev : 0);
    long yrow[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = min(m0 + 16 * RB * wave + 16 * rb + 4 * g + r, M - 1);
            const long orow = a.seg ? (long)(row / a.seg) * a.seg_stride + row % a.seg : row;
            yrow[rb][r] = (orow + roff) * a.ldy;
        }
    float bj[CB], old[RB][CB][4];
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        const int col = min(n0 + 16 * cb + lc, N - 1);
        bj[cb] = EPI == EPI_STORE ? 0.f : a.bias[col];
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int r = 0; r < 4; r++) old[rb][cb][r] = EPI == EPI_RESID ? a.Y[yrow[rb][r] + col] : 0.f;
    }
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        const int col = n0 + 16 * cb + lc;
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = m0 + 16 * RB * wave + 16 * rb + 4 * g + r;
                if (row < M && col < N)
                    a.Y[yrow[rb][r] + col] = epi_value<EPI>(acc[rb][cb][r], bj[cb], old[rb][cb][r]);
            }
    }
}

// k_rows: products over 32 < M <= 128 rows whose 128 x 128 tiles would
// leave most CUs idle (the B=1 T=128 forward: 6-24 such tiles per product).
// A workgroup of four wavefronts owns a 32-row x TN-column tile (TN = 32,
// 48 or 64: two by TN / 16 blocks of v_mfma_f32_16x16x4f32); each wavefront
// multiplies the whole tile over a quarter of every stage's k (k quads 4 w
// .. 4 w + 3), so each LDS granule is read by one wavefront (a split of the
// tile over the wavefronts reads every row twice), and the four partial
// tiles are summed through LDS in wavefront order at the end. Both operands
// go global -> LDS (lds_dma16) through a ring of RQ_S stages of RQ_BK k:
// one wait and one barrier per stage, the next stage's operands read from
// LDS while the current stage's products issue. A stage row is 16 granules
// of 16 bytes, the granule order XOR-swizzled by the row, so the 16 rows a
// read instruction touches at one k quad fall in 16 different granules of
// the 256-byte bank line. TN and a K split are chosen so that each CU holds
// one workgroup where the product allows (rows_plan): a CU holding two
// workgroups of a launch takes twice as long as the others, so 288 or 384
// 32 x 32 tiles (GPT-2's QKV and fc at 128 rows) ran at the speed of 512.
constexpr int RQ_BK = 64, RQ_S = 5, RQ_TM = 32;

template <int EPI, int TN>
__global__ void __launch_bounds__(256, 1) k_rows(GemmArgs a, int tiles_m, int tiles_n, int KR,
                                                 int KS) {
    constexpr int ROWS = RQ_TM + TN;     // stage rows: RQ_TM of X, then TN of W
    constexpr int NI = ROWS / 16;        // load instructions per wavefront and stage
    constexpr int STAGE = ROWS * RQ_BK;  // floats per stage
    constexpr int CB = TN / 16;          // 16-column blocks
    constexpr int RS = TN + 4;           // row stride of the partial tiles (bank spread)
    static_assert(ROWS % 16 == 0 && 4 * RQ_TM * RS <= RQ_S * STAGE, "tile shape");
    __shared__ __attribute__((aligned(1024))) float sm[RQ_S * STAGE];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    // work id: row tiles fastest, then column tiles, then K splits; ids
    // XCD-contiguous, so the row tiles of a column tile share its W rows in
    // one XCD's L2
    const int p = xcd_order(blockIdx.x, tiles_m * tiles_n * KS);
    const int tm = p % tiles_m, tn = (p / tiles_m) % tiles_n, ks = p / (tiles_m * tiles_n);
    const int m0 = tm * RQ_TM, n0 = tn * TN;
    const int K = a.K, M = a.M, N = a.N;
    const int kb = ks * KR, nk = (min(K, kb + KR) - kb) / RQ_BK;
    // load instruction i of wavefront w covers stage rows 4 (4 i + w) ..
    // +3: lane -> row 4 (4 i + w) + lane / 16, slot lane % 16, holding k
    // quad slot ^ (row % 16); rows past M or N read the last one (finite
    // values; their results are not stored)
    const float* src[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int row = 4 * (4 * i + wave) + (lane >> 4), slot = lane & 15;
        const int kq = slot ^ (row & 15);
        src[i] = row < RQ_TM ? a.X + (long)min(m0 + row, M - 1) * K + kb + 4 * kq
                             : a.W + (long)min(n0 + row - RQ_TM, N - 1) * K + kb + 4 * kq;
    }
    auto issue = [&](int kt, int st) {
        float* base = sm + st * STAGE;
#pragma unroll
        for (int i = 0; i < NI; i++) lds_dma16(src[i] + kt * RQ_BK, base + (4 * i + wave) * 256);
    };
    // lane: row (column) 16 b + lane % 16 of each 16-block, k quad 4 w +
    // lane / 16; element e of the quad is the k of the e-th product
    const int lc = lane & 15, g = lane >> 4, q = 4 * wave + g;
    int ao[2], bo[CB];
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        const int r = 16 * rb + lc;
        ao[rb] = r * RQ_BK + 4 * (q ^ (r & 15));
    }
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        const int r = RQ_TM + 16 * cb + lc;
        bo[cb] = r * RQ_BK + 4 * (q ^ (r & 15));
    }
    f32x4 acc[2][CB];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // operands of a stage, read from LDS one stage ahead of their products
    // (the reads of stage kt + 1 are in flight while stage kt's products
    // issue)
    f32x4 av[2], bv[CB];
    auto read = [&](int kt) {
        const float* base = sm + (kt % RQ_S) * STAGE;
#pragma unroll
        for (int rb = 0; rb < 2; rb++) av[rb] = *(const f32x4*)&base[ao[rb]];
#pragma unroll
        for (int cb = 0; cb < CB; cb++) bv[cb] = *(const f32x4*)&base[bo[cb]];
    };
#pragma unroll
    for (int st = 0; st < RQ_S - 1; st++)
        if (st < nk) issue(st, st);
    if (nk > 0) {
        // stage 0 has landed once at most stages 1 .. RQ_S - 2 are in flight
        if (RQ_S - 2 < nk) wait_vmcnt<NI * (RQ_S - 2)>();
        else wait_vmcnt<0>();
        asm volatile("s_barrier" ::: "memory");
        read(0);
    }
    for (int kt = 0; kt < nk; kt++) {
        const f32x4 a0 = av[0], a1 = av[1];
        f32x4 bc[CB];
#pragma unroll
        for (int cb = 0; cb < CB; cb++) bc[cb] = bv[cb];
        if (kt + 1 < nk) {
            // stage kt + 1 has landed once at most stages kt + 2 .. kt +
            // RQ_S - 2 are in flight; past the barrier every wavefront has
            // landed its part of it and is done reading stage kt - 1 (its
            // products issued in the previous trip), which the next issue
            // overwrites
            if (kt + RQ_S - 2 < nk) wait_vmcnt<NI * (RQ_S - 3)>();
            else wait_vmcnt<0>();
            asm volatile("s_barrier" ::: "memory");
            if (kt + RQ_S - 1 < nk) issue(kt + RQ_S - 1, (kt + RQ_S - 1) % RQ_S);
            read(kt + 1);
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
                acc[0][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[e], bc[cb][e], acc[0][cb], 0, 0, 0);
                acc[1][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[e], bc[cb][e], acc[1][cb], 0, 0, 0);
            }
    }
    // every load has landed (the wait before the last stage's reads was for
    // all of them) and, past this barrier, every wavefront is done reading
    // the ring: it holds the partial tiles, [wave][row][RS]
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                sm[(wave * RQ_TM + 16 * rb + 4 * g + r) * RS + 16 * cb + lc] = acc[rb][cb][r];
    __syncthreads();
    const long roff = a.row_off + (a.row_off_dev ? *a.row_off_dev : 0);
#pragma unroll
    for (int u = 0; u < RQ_TM * TN / 256; u++) {
        const int idx = tid + 256 * u, row = idx / TN, cl = idx - row * TN;
        const float* pr = sm + row * RS + cl;
        const float v = ((pr[0] + pr[RQ_TM * RS]) + pr[2 * RQ_TM * RS]) + pr[3 * RQ_TM * RS];
        const int gr = m0 + row, gc = n0 + cl;
        if (gr < M && gc < N) {
            if (KS == 1) store_out<EPI>(a, roff, gr, gc, v);
            else a.part[((long)ks * M + gr) * N + gc] = v;
        }
    }
}

template <int EPI>
__global__ void __launch_bounds__(256) k_stream_reduce(GemmArgs a, int KS) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const long MN = (long)a.M * a.N;
    if (i >= MN) return;
    const int row = (int)(i / a.N), col = (int)(i % a.N);
    long orow = a.seg ? (long)(row / a.seg) * a.seg_stride + row % a.seg : row;
    orow += a.row_off + (a.row_off_dev ? *a.row_off_dev : 0);
    float* y = a.Y + orow * a.ldy + col;
    // the epilogue's bias and residual are loaded with the first partials
    // (one memory round trip rather than one after the sum; the values and
    // the arithmetic are store_out's)
    const float b = EPI != EPI_STORE ? a.bias[col] : 0.f;
    const float old = EPI == EPI_RESID ? *y : 0.f;
    // partials in batches of 8 loads in flight, summed in split order
    float v = 0.f;
    for (int q0 = 0; q0 < KS; q0 += 8) {
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; j++) p[j] = a.part[min(q0 + j, KS - 1) * MN + i];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (q0 + j < KS) v += p[j];
    }
    *y = epi_value<EPI>(v, b, old);
}

// The same sum for one row per workgroup (float4 columns tid + 256 i),
// then the LayerNorm (reference ops.c:191-248) of the finished row into
// a.ln_out: the residual stream and the next product's input in one pass.
// Only the residual epilogue forms a LayerNorm (the residual stream feeds the
// next sub-layer); rows of up to 2048 floats (NCH = 1 or 2 float4 per thread).
template <int EPI, int NCH>
__global__ void __launch_bounds__(256) k_stream_reduce_ln(GemmArgs a, int KS) {
    static_assert(EPI == EPI_RESID && (NCH == 1 || NCH == 2), "residual rows of <= 2048 floats");
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int N4 = a.N >> 2;
    const long MN4 = (long)a.M * N4;
    const f32x4* p = (const f32x4*)(a.part + (long)r * a.N);
    float* yrow = a.Y + (long)r * a.ldy;
    f32x4 y[NCH], v[NCH];
    // the residual row, bias and LayerNorm gains of this thread's columns
    // are loaded with the first partials (one memory round trip, not three
    // after the sum)
    f32x4 yo[NCH], bb[NCH], lw[NCH], lb[NCH];
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int cc = min(tid + 256 * i, N4 - 1);
        yo[i] = *(const f32x4*)(yrow + 4 * cc);
        bb[i] = *(const f32x4*)(a.bias + 4 * cc);
        lw[i] = *(const f32x4*)(a.ln_w + 4 * cc);
        lb[i] = *(const f32x4*)(a.ln_b + 4 * cc);
    }
#pragma unroll
    for (int i = 0; i < NCH; i++) v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    // batches of 8 partials of every column of this thread in flight together
    for (int q0 = 0; q0 < KS; q0 += 8) {
        f32x4 t[NCH][8];
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int cc = min(tid + 256 * i, N4 - 1);
#pragma unroll
            for (int j = 0; j < 8; j++) t[i][j] = p[(long)min(q0 + j, KS - 1) * MN4 + cc];
        }
#pragma unroll
        for (int i = 0; i < NCH; i++)
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (q0 + j < KS) v[i] += t[i][j];
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int c4 = tid + 256 * i;
#pragma unroll
        for (int k = 0; k < 4; k++) y[i][k] = epi_value<EPI>(v[i][k], bb[i][k], yo[i][k]);
        if (c4 < N4) {
            *(f32x4*)(yrow + 4 * c4) = y[i];
            s += (y[i].x + y[i].y) + (y[i].z + y[i].w);
        }
    }
    auto block_sum = [&](float v) {
        v = wave_sum(v);
        __syncthreads();
        if (lane == 0) red[wave] = v;
        __syncthreads();
        return (red[0] + red[1]) + (red[2] + red[3]);
    };
    const float mean = block_sum(s) / (float)a.N;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; i++)
        if (tid + 256 * i < N4) {
            const f32x4 d = y[i] - mean;
            q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        }
    const float rstd = 1.0f / sqrtf(block_sum(q) / (float)a.N + 1e-5f);
    float* orow = a.ln_out + (long)r * a.N;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int c4 = tid + 256 * i;
        if (c4 < N4)
            *(f32x4*)(orow + 4 * c4) = (y[i] - mean) * rstd * lw[i] + lb[i];
    }
}

// After a launch whose KS K-splits left partials in a.part: Y = epi(their
// sum in split order), and with a.ln_out the LayerNorm of each row formed
// in the same pass (residual products, rows <= 2048 floats).
template <int EPI>
hipError_t reduce_splits(const GemmArgs& a, int KS, hipStream_t s) {
    if constexpr (EPI == EPI_RESID) {
        // launch_gemm admits ln_out for the residual epilogue and N <= 2048 only
        if (a.ln_out) {
            if (a.N <= 1024) k_stream_reduce_ln<EPI, 1><<<a.M, 256, 0, s>>>(a, KS);
            else k_stream_reduce_ln<EPI, 2><<<a.M, 256, 0, s>>>(a, KS);
            return hipGetLastError();
        }
    }
    k_stream_reduce<EPI><<<(unsigned)(((long)a.M * a.N + 255) / 256), 256, 0, s>>>(a, KS);
    return hipGetLastError();
}

// Without splits the LayerNorm of the finished rows is a launch of its own.
hipError_t ln_after(const GemmArgs& a, hipStream_t s) {
    if (!a.ln_out) return hipSuccess;
    return launch_layernorm(a.Y, a.ldy, a.ln_w, a.ln_b, a.ln_out, a.N, a.M, a.N, s);
}

// Split K until the column tiles times the splits reach two workgroups per
// CU (the partials must fit a.part_cap floats; ranges are whole chunks):
// returns the splits, *KR the k per split.
// Wavefronts per 16-column block: the narrowest tiles (up to 4 per block
// at 16 rows, 2 at 32: the longer input chunks' LDS) that make at least 192
// column tiles, which then run without a K split; else 1, split as below.
int stream_wpb(const GemmArgs& a) {
    const int MB = st_mb(a.M);
    for (int wpb = 1; wpb <= (MB == 1 ? 4 : MB == 2 ? 2 : 1); wpb *= 2)
        if ((a.N + 16 * ST_NW / wpb - 1) / (16 * ST_NW / wpb) >= 192) return wpb;
    return 1;
}

int stream_splits(const GemmArgs& a, int* KR) {
    if (const int wpb = stream_wpb(a); wpb > 1) {
        *KR = (a.K + 16 * 8 * wpb - 1) / (16 * 8 * wpb) * (16 * 8 * wpb);
        return 1;
    }
    const int kc = st_kc(st_mb(a.M));
    const int tiles_n = (a.N + ST_NT - 1) / ST_NT;
    const int kchunks = (a.K + kc - 1) / kc;
    // Enough splits for about one workgroup per CU, never more: a
    // workgroup's fixed cost (launch, first loads, partial store) repays
    // longer ranges better than a second workgroup sharing its CU. Measured
    // per product (ordered sum included): GPT-2 medium B=8 proj 9.53 ->
    // 7.91 us at 256 workgroups instead of 512, fc 8.57 -> 7.41; XL B=32
    // proj 18.29 -> 15.04, fc 17.92 -> 17.55 at 200 instead of 500; GPT-2
    // small M = 128 QKV 18.6 -> 14.7, fc 20.6 -> 16.4.
    int KS = a.part ? std::max(1, std::min(256 / tiles_n, kchunks)) : 1;
    while (KS > 1 && (long)KS * a.M * a.N > a.part_cap) KS--;
    *KR = ((kchunks + KS - 1) / KS) * kc;
    return (a.K + *KR - 1) / *KR;
}

template <int EPI, int MB, int WPB>
void stream_launch(const GemmArgs& a, int tiles_n, int KR, int KS, hipStream_t s) {
    if (a.Wp)
        k_stream<EPI, MB, true, WPB><<<tiles_n * KS, ST_NW * 64, 0, s>>>(a, tiles_n, KR, KS);
    else
        k_stream<EPI, MB, false, WPB><<<tiles_n * KS, ST_NW * 64, 0, s>>>(a, tiles_n, KR, KS);
}

template <int EPI, int MB>
hipError_t stream_mb(const GemmArgs& a, hipStream_t s) {
    const int wpb = stream_wpb(a);
    const int tiles_n = (a.N + 16 * ST_NW / wpb - 1) / (16 * ST_NW / wpb);
    int KR;
    const int KS = stream_splits(a, &KR);
    // (stream_wpb gives 4 for one row block only, 2 for at most two)
    if constexpr (MB == 1) {
        if (wpb == 4) stream_launch<EPI, MB, 4>(a, tiles_n, KR, KS, s);
    }
    if constexpr (MB <= 2) {
        if (wpb == 2) stream_launch<EPI, MB, 2>(a, tiles_n, KR, KS, s);
    }
    if (wpb == 1) stream_launch<EPI, MB, 1>(a, tiles_n, KR, KS, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || (KS > 1 && a.partials_only)) return e;
    return KS == 1 ? ln_after(a, s) : reduce_splits<EPI>(a, KS, s);
}

template <int EPI>
hipError_t skinny_epi(const GemmArgs& a, hipStream_t s) {
    if (a.M <= 16) return stream_mb<EPI, 1>(a, s);
    if (a.M <= 32) return stream_mb<EPI, 2>(a, s);
    if (a.M <= 48) return stream_mb<EPI, 3>(a, s);
    if (a.M <= 64) return stream_mb<EPI, 4>(a, s);
    return stream_mb<EPI, 8>(a, s);
}

// k_rows for 32 < M <= 128: the tile width TN and the K split KS with the
// least estimated time, at most one workgroup per CU where possible. A
// stage costs about (0.15 + 0.0075 TN) us (measured at 128 rows: 0.39 us
// for TN = 32, 0.51 for 48); launches over the CU count take whole extra
// rounds; K is split (ranges of at least 3 stages, partials within
// a.part_cap) only while the tiles are fewer than half the CUs.
struct RowsPlan {
    int TN, KS, KR;
};
RowsPlan rows_plan(const GemmArgs& a) {
    const int steps = a.K / RQ_BK, tiles_m = (a.M + RQ_TM - 1) / RQ_TM;
    RowsPlan best{32, 1, a.K};
    double best_t = 1e30;
    for (const int TN : {32, 48, 64}) {
        const int tiles = tiles_m * ((a.N + TN - 1) / TN);
        int KS = 1;
        if (a.part && 2 * tiles < 256) {
            KS = std::max(1, std::min(256 / tiles, steps / 3));
            while (KS > 1 && (long)KS * a.M * a.N > a.part_cap) KS--;
        }
        const int per = (steps + KS - 1) / KS;
        KS = (steps + per - 1) / per;
        const int rounds = (tiles * KS + 255) / 256;
        const double t = rounds * per * (0.15 + 0.0075 * TN);
        if (t < best_t) {
            best_t = t;
            best = RowsPlan{TN, KS, per * RQ_BK};
        }
    }
    return best;
}

int rows_splits(const GemmArgs& a) { return rows_plan(a).KS; }

template <int EPI, int TN>
hipError_t rows_launch(const GemmArgs& a, const RowsPlan& p, hipStream_t s) {
    const int tiles_m = (a.M + RQ_TM - 1) / RQ_TM, tiles_n = (a.N + TN - 1) / TN;
    k_rows<EPI, TN><<<tiles_m * tiles_n * p.KS, 256, 0, s>>>(a, tiles_m, tiles_n, p.KR, p.KS);
    return hipGetLastError();
}

template <int EPI>
hipError_t rows_epi(const GemmArgs& a, hipStream_t s) {
    const RowsPlan p = rows_plan(a);
    const hipError_t e = p.TN == 32   ? rows_launch<EPI, 32>(a, p, s)
                         : p.TN == 48 ? rows_launch<EPI, 48>(a, p, s)
                                      : rows_launch<EPI, 64>(a, p, s);
    if (e != hipSuccess || (p.KS > 1 && a.partials_only)) return e;
    return p.KS == 1 ? ln_after(a, s) : reduce_splits<EPI>(a, p.KS, s);
}

// The few-row products take M <= SKINNY_MAX_M rows, and up to ST_MAX_M rows
// of products whose 128 x 128 tiles would be too few for the CUs (the
// reference's own B=1 T=128 forward: 6-24 tiles per product), with
// row-major operands. CNGPT_HIP_STREAM128=0 / 1 forces the choice for
// 64 < M <= 128 (A/B timing against the 128 x 128 tiles).
bool use_stream(const GemmArgs& a) {
    if (a.M <= SKINNY_MAX_M) return true;
    if (a.M > ST_MAX_M || a.km) return false;
    static const int force = [] {
        const char* e = getenv("CNGPT_HIP_STREAM128");
        return e && (e[0] == '0' || e[0] == '1') ? e[0] - '0' : -1;
    }();
    if (force >= 0) return force == 1;
    return (long)((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN) < 256;
}

// Of those, the ones over more than ROWS_MIN_M rows with K in whole k_rows
// stages take k_rows instead of k_stream. Measured at 33-64 rows (GPT-2
// small forwards through the host API, final-position logits): B=1 T=64
// 0.713 -> 0.680 ms per forward, B=2 T=32 0.728 -> 0.695 ms; at 17-32 rows
// k_stream stays ahead (B=1 T=32 0.593 vs 0.635 ms, GPT-2 XL decode at
// B=32 3.42 vs 3.53 ms per step).
constexpr int ROWS_MIN_M = 32;
bool use_rows(const GemmArgs& a) {
    return a.M > ROWS_MIN_M && a.M <= ST_MAX_M && !a.km && a.K % RQ_BK == 0 &&
           (a.M <= SKINNY_MAX_M || use_stream(a));
}

// Share of the tile slots the last round of a launch fills when `res`
// tiles are resident at a time.
double round_fill(int tiles, int res) {
    const int rounds = (tiles + res - 1) / res;
    return rounds <= 1 ? 1.0 : (double)tiles / ((double)rounds * res);
}

// Variant choice, from kernel traces of the GPT-2 small / medium / XL
// forwards (M = 16384 / 8192 / 4096 rows). Whole tiles with K a multiple
// of 16 (every GPT-2 width): k_gemm_dl with BK = 16 in two 32 KB stages, 4
// workgroups per CU. With each step's products at raised priority (dl_tile)
// it is at least as fast as BK = 32 in two 64 KB stages at 2 per CU on every
// product measured (GPT-2 small B=16: fc 593.5 -> 579.5 us, lm_head 9400 ->
// 9322 us, QKV, c_proj and proj unchanged; GEMM class 83.8 -> 84.1 %;
// medium B=8 84.3 -> 84.6 %; XL's lm_head and the B=2 share's the same);
// three 48 KB stages at 3 per CU were slower (82.6-82.9 %). Before the
// priority BK = 32 at 2 per CU was the faster on every product but GPT-2
// small's 768-tile c_proj and proj. Otherwise k_gemm: BK = 16 with rows
// padded by 4 floats (40 KB, 4 per CU) when its tiles fit one round or
// fill its last round; else BK = 16 at 3 per CU when that fills its last
// round; else BK = 32 at 2 per CU, whose longer K steps hold up best when
// a round is left part-empty.
//
// Launches of at most 256 tiles (M up to ~2048 rows: short prefills, the
// reference's own B=1 T=128 shape, one GPU's share of a batch, the
// training step's N = 768 products at B=4 T=1024) split K over workgroups
// of the BK = 32 variant when that is cheaper by a measured cost model:
//   ceil(steps / KS) * (w == 1 ? 2.1 : 1.83 w) us, w = ceil(tiles * KS /
//   256) workgroups on the busiest CU (a 128 x 128 x 32 step takes ~2.1 us
//   alone on a CU, ~1.83 us each when workgroups share it and hide each
//   other's memory waits)
// + 0.3 us per MB of partials (KS * M * N floats written and summed),
// over KS from 1 (whole tiles) to K / 64 (at least two K steps per split),
// the partials within a.part_cap; then reduce_splits. Fitted to per-product
// timings (+ reduce) of GPT-2 small's products at M = 128 .. 4096, where it
// picks the measured best or one within 4 % of it: e.g. proj at M = 4096
// (192 tiles) 4 splits, 203 -> 164 us; fc at M = 128 8 splits, 24.2 ->
// 19.0 us. More tiles take stream-K or whole tiles. Returns the splits, *KR
// the k per split (whole K steps).
int tile_splits(const GemmArgs& a, int tiles, int* KR) {
    const int cus = 256;
    *KR = a.K;
    if (!a.part || a.K % 32 || tiles > cus) return 1;
    const int nsteps = a.K / 32;
    const double mb_per_split = 4e-6 * a.M * a.N;
    auto per_step = [&](int wgs) {
        const int w = (wgs + cus - 1) / cus;
        return w == 1 ? 2.1 : 1.83 * w;
    };
    int best = 1;
    double best_cost = nsteps * per_step(tiles);
    for (int ks = 2; ks <= a.K / 64; ks++) {
        if ((long)ks * a.M * a.N > a.part_cap) break;
        const int steps = (nsteps + ks - 1) / ks;
        const int kse = (nsteps + steps - 1) / steps;  // splits of `steps` each
        const double cost = steps * per_step(tiles * kse) + 0.3 * mb_per_split * kse;
        if (cost < best_cost) {
            best_cost = cost;
            best = kse;
        }
    }
    if (best <= 1) return 1;
    *KR = (nsteps + best - 1) / best * 32;
    return (a.K + *KR - 1) / *KR;
}

// Stream-K instead of whole tiles in rounds of 2 x 256 when the last round
// would leave more than a tenth of the slots idle (more than 256 tiles, K a
// multiple of 32, partial slots for every workgroup within a.part_cap):
// the number of workgroups, 0 for none.
int sk_workgroups(const GemmArgs& a, int tiles) {
    const int cus = 256, G = 2 * cus;
    if (!a.part || a.K % 32 || tiles <= cus) return 0;
    if (tiles > G && tiles <= 2 * G) {
        // one round of the BK = 16 variant at 4 per CU, while it gives the
        // CUs about equal numbers of tiles (768: 3 each); otherwise one
        // stream-K workgroup per CU (M = 4096 QKV, 576 tiles: 155.6 us
        // in one round of 2 or 3 tiles per CU, 132.0 us stream-K)
        const int per_cu = (tiles + cus - 1) / cus;
        if ((double)tiles / ((double)per_cu * cus) >= 0.9) return 0;
        if (2L * cus * BM * BN > a.part_cap) return 0;
        return cus;
    }
    const int rounds = (tiles + G - 1) / G;
    if ((double)tiles / ((double)rounds * G) >= 0.9) return 0;
    if (2L * G * BM * BN > a.part_cap || (long)tiles * (a.K / 32) < G) return 0;
    // fewer tiles than slots: one workgroup per CU (half the partial tiles)
    return tiles < G ? cus : G;
}

// Rounds of whole tiles ahead of the stream-K part: every full round of G
// tiles, so stream-K spreads only the last part-empty round over the G
// workgroups. Measured on GPT-2 XL B=4 T=1024 (QKV 1216 and fc 1600 tiles
// over 512 workgroups, c_proj and proj 416 over 256): GEMM class 77.6 % of
// peak with stream-K over every tile, 77.8 % with all rounds but the last
// whole, 79.2 % with every full round whole.
int sk_whole_rounds(int tiles, int G) { return tiles / G; }

// k_gemm_wide shapes and the share of fp32 peak each reached on its own in
// full rounds (M = 2048 and 16384): 128 x 144 0.75, 64 x 96 0.78, 64 x 48
// 0.64 (128 x 192 and 64 x 144 reached 0.75 and 0.70 and never beat 64 x 96
// or 128 x 144 on a GPT-2 shape). A product takes the
// shape with the best estimate (that share times the fraction of the
// rounds' tile slots its tiles fill, ragged edges counted as waste) when
// that beats what the 128 x 128 tiles reach (launch_gemm timings, partial
// sums and LayerNorm included): up to 256 of them (split K) 0.31-0.56, so
// an estimate of 0.5 is enough; 257-576 (stream-K after whole-tile
// rounds) 0.61-0.73, so 0.7; beyond that stream-K holds its own (fc at
// 4096 rows: 154.5 us against 163.4 as 64 x 96 tiles), and so do products
// whose tiles fill their rounds. CNGPT_HIP_WIDE=0 turns the path off (A/B
// timing).
struct WidePlan {
    int TM, TN;
};
WidePlan wide_plan(const GemmArgs& a) {
    static const bool off = [] {
        const char* e = getenv("CNGPT_HIP_WIDE");
        return e && e[0] == '0';
    }();
    static const struct {
        int TM, TN;
        double f;
    } cand[] = {{128, 144, 0.75}, {64, 96, 0.78}, {64, 48, 0.64}};
    WidePlan best{0, 0};
    if (off || a.km || a.M <= ST_MAX_M || a.K % WD_BK) return best;
    const long t128 = (long)((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const double fill = t128 <= 256 ? t128 / 256.0 : t128 / (512.0 * ((t128 + 511) / 512));
    if (fill >= 0.9 || t128 > 576) return best;
    double best_e = t128 <= 256 ? 0.5 : 0.7;
    for (const auto& c : cand) {
        const long tiles = (long)((a.M + c.TM - 1) / c.TM) * ((a.N + c.TN - 1) / c.TN);
        const long cap = c.TM == 128 ? 256 : 512;
        const long rounds = (tiles + cap - 1) / cap;
        const double e = c.f * (double)a.M * a.N / ((double)rounds * cap * c.TM * c.TN);
        if (e > best_e) {
            best_e = e;
            best = WidePlan{c.TM, c.TN};
        }
    }
    return best;
}

template <int EPI, int TM, int TN, int S>
hipError_t wide_launch(const GemmArgs& a, hipStream_t s) {
    const int tiles_m = (a.M + TM - 1) / TM, tiles_n = (a.N + TN - 1) / TN;
    k_gemm_wide<EPI, TM, TN, S><<<tiles_m * tiles_n, 256, 0, s>>>(a, tiles_m, tiles_n);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess ? e : ln_after(a, s);
}

template <int EPI>
hipError_t wide_epi(const GemmArgs& a, const WidePlan& w, hipStream_t s) {
    if (w.TM == 128) return wide_launch<EPI, 128, 144, 4>(a, s);
    return w.TN == 96 ? wide_launch<EPI, 64, 96, 4>(a, s) : wide_launch<EPI, 64, 48, 4>(a, s);
}

// K-major operands: both (a.km == 3, the residual epilogue of the dW
// products) or W only (a.km == 2, the stored epilogue of the dX products,
// W the weight matrix as stored: row k = output k of the forward product):
// whole 128 x 128 tiles, or K split over the CUs when the tiles are too few
// (no stream-K); K is a multiple of 32 (checked by the caller), so every
// split covers whole steps of 16, four workgroups per CU as for the row-major
// whole tiles.
template <int EPI, int KM>
hipError_t gemm_km(const GemmArgs& a, hipStream_t s) {
    const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
    const int tiles = tiles_m * tiles_n;
    int KR;
    const int KS = tile_splits(a, tiles, &KR);
    k_gemm_dl<EPI, 16, 2, 4, KM><<<tiles * KS, NTHREADS, 0, s>>>(a, tiles_m, tiles_n, KR, KS);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess || KS == 1 ? e : reduce_splits<EPI>(a, KS, s);
}

template <int EPI>
hipError_t gemm_epi(const GemmArgs& a, hipStream_t s) {
    const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
    const int tiles = tiles_m * tiles_n, cus = 256;
    if (const WidePlan w = wide_plan(a); w.TM) return wide_epi<EPI>(a, w, s);
    int KR;
    const int KS = tile_splits(a, tiles, &KR);
    if (KS > 1) {
        k_gemm_dl<EPI, 32, 2, 2><<<tiles * KS, NTHREADS, 0, s>>>(a, tiles_m, tiles_n, KR, KS);
        const hipError_t e = hipGetLastError();
        return e != hipSuccess ? e : reduce_splits<EPI>(a, KS, s);
    }
    if (const int G = sk_workgroups(a, tiles)) {
        const int dp = sk_whole_rounds(tiles, G);
        k_gemm_sk<EPI><<<G, NTHREADS, 0, s>>>(a, tiles_m, tiles_n, a.K / 32, G, dp);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (tiles > dp * G) {
            k_sk_fixup<EPI><<<(tiles - dp * G) * (BM / SK_RPW), 256, 0, s>>>(a, tiles_m, tiles_n,
                                                                           a.K / 32, G, dp * G);
            e = hipGetLastError();
        }
        return e != hipSuccess ? e : ln_after(a, s);
    }
    if (a.K % 16 == 0)
        k_gemm_dl<EPI, 16, 2, 4><<<tiles, NTHREADS, 0, s>>>(a, tiles_m, tiles_n, a.K, 1);
    else if (tiles <= 4 * cus || round_fill(tiles, 4 * cus) >= 0.9)
        k_gemm<EPI, 16, 4, 4><<<tiles, NTHREADS, 0, s>>>(a, tiles_m, tiles_n);
    else if (round_fill(tiles, 3 * cus) >= 0.9)
        k_gemm<EPI, 16, 8, 3><<<tiles, NTHREADS, 0, s>>>(a, tiles_m, tiles_n);
    else
        k_gemm<EPI, 32, 4, 2><<<tiles, NTHREADS, 0, s>>>(a, tiles_m, tiles_n);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess ? e : ln_after(a, s);
}

// Packed copy of W [N][K] (row-major, K a multiple of 4) for k_stream:
// column block b (columns 16 b .. 16 b + 15) holds ceil(K / 16) steps of 256
// floats, and floats 4 l .. 4 l + 3 of step q are W[16 b + l % 16][16 q +
// 4 (l / 16) .. +3], zero past N or K. One thread per 16 bytes written.
__global__ void __launch_bounds__(256) k_pack_w(const float* __restrict__ W, float* __restrict__ Wp,
                                                int N, int K, long n4) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const int l = (int)(i & 63), KQ = (K + 15) >> 4;
    const long bq = i >> 6;
    const long n = bq / KQ * 16 + (l & 15);
    const int k = (int)(bq % KQ) * 16 + 4 * (l >> 4);
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (n < N && k < K) v = *(const f32x4*)&W[n * K + k];
    *(f32x4*)&Wp[4 * i] = v;
}

}  // namespace

size_t packed_w_floats(int N, int K) { return (size_t)((N + 15) / 16) * ((K + 15) / 16) * 256; }

hipError_t launch_pack_w(const float* W, float* Wp, int N, int K, hipStream_t s) {
    if (N <= 0 || K <= 0 || (K & 3)) return hipErrorInvalidValue;
    const long n4 = (long)(packed_w_floats(N, K) / 4);
    k_pack_w<<<(unsigned)((n4 + 255) / 256), 256, 0, s>>>(W, Wp, N, K, n4);
    return hipGetLastError();
}

hipError_t launch_sum_heads(const GemmArgs& a, int KS, hipStream_t s) {
    if (a.M <= 0) return hipSuccess;
    if (KS < 1 || (long)KS * a.M * a.N > a.part_cap || (a.N & 3) || (a.ln_out && a.N > 2048))
        return hipErrorInvalidValue;
    return reduce_splits<EPI_RESID>(a, KS, s);
}

int launch_gemm_partials(const GemmArgs& a) {
    if (a.M <= 0 || a.N <= 0 || a.K <= 0 || (a.K & 3) || a.ln_out || a.km) return 0;
    if (!(use_rows(a) || use_stream(a))) return 0;
    const int KS = launch_gemm_splits(a);
    return KS > 1 ? KS : 0;
}

int launch_gemm_splits(const GemmArgs& a) {
    if (a.M <= 0 || a.N <= 0 || a.K <= 0 || (a.K & 3)) return 1;
    int KR;
    if (use_rows(a)) return rows_splits(a);
    if (use_stream(a)) return stream_splits(a, &KR);
    if (wide_plan(a).TM) return 1;
    return tile_splits(a, ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN), &KR);
}

hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0) return hipSuccess;
    if (a.K <= 0 || (a.K & 3)) return hipErrorInvalidValue;
    // the LayerNorm rows are written and read with 16-byte accesses
    if (a.ln_out && (a.epi != EPI_RESID || a.seg || a.row_off || a.row_off_dev || (a.N & 3) ||
                     (a.ldy & 3) || a.N > 2048 || !a.ln_w || !a.ln_b))
        return hipErrorInvalidValue;
    if (a.km) {
        // K-major operands: both with the residual (accumulating) epilogue
        // of the dW products, or W only with the stored epilogue of the dX
        // products; plain row-major output, K whole steps, rows of whole
        // granules (ld a multiple of 4 covering the tile's rows rounded to 4)
        const bool both = a.km == 3 && a.epi == EPI_RESID, w_only = a.km == 2 && a.epi == EPI_STORE;
        if ((!both && !w_only) || a.M <= SKINNY_MAX_M || a.K % 32 || a.seg || a.row_off ||
            a.row_off_dev || a.ln_out || (a.ldw & 3) || a.ldw < ((a.N + 3) & ~3) ||
            (both && ((a.ldx & 3) || a.ldx < ((a.M + 3) & ~3))))
            return hipErrorInvalidValue;
        return both ? gemm_km<EPI_RESID, 3>(a, s) : gemm_km<EPI_STORE, 2>(a, s);
    }
    // partials left unsummed: the few-row paths only, without a LayerNorm
    if (a.partials_only && (a.ln_out || !(use_rows(a) || use_stream(a))))
        return hipErrorInvalidValue;
    if (use_rows(a)) {
        switch (a.epi) {
            case EPI_STORE: return rows_epi<EPI_STORE>(a, s);
            case EPI_BIAS: return rows_epi<EPI_BIAS>(a, s);
            case EPI_BIAS_GELU: return rows_epi<EPI_BIAS_GELU>(a, s);
            case EPI_RESID: return rows_epi<EPI_RESID>(a, s);
        }
        return hipErrorInvalidValue;
    }
    if (use_stream(a)) {
        switch (a.epi) {
            case EPI_STORE: return skinny_epi<EPI_STORE>(a, s);
            case EPI_BIAS: return skinny_epi<EPI_BIAS>(a, s);
            case EPI_BIAS_GELU: return skinny_epi<EPI_BIAS_GELU>(a, s);
            case EPI_RESID: return skinny_epi<EPI_RESID>(a, s);
        }
        return hipErrorInvalidValue;
    }
    switch (a.epi) {
        case EPI_STORE: return gemm_epi<EPI_STORE>(a, s);
        case EPI_BIAS: return gemm_epi<EPI_BIAS>(a, s);
        case EPI_BIAS_GELU: return gemm_epi<EPI_BIAS_GELU>(a, s);
        case EPI_RESID: return gemm_epi<EPI_RESID>(a, s);
    }
    return hipErrorInvalidValue;
}
