// gemm.hip - fp32 products Y[M,N] = epi(X[M,K] . W[N,K]^T) on gfx950.
//
// The reference computes every linear layer as cblas_sgemm(RowMajor,
// NoTrans, Trans) with a per-row saxpy bias and beta = 1 for the residual
// (fast.c:175-205). Both operands are K-contiguous, so both tiles are staged
// in LDS the same way and read back with 16-byte LDS reads.
//
// k_gemm: 128x128 output tile per 256-thread workgroup, K in steps of BK,
// double-buffered LDS (global loads for step k+1 are in flight while step k
// is multiplied). Each wavefront owns a 64x64 sub-tile = 2x2 blocks of
// v_mfma_f32_32x32x2f32. Inside a K step, lanes 0-31 feed the first half of
// the step's k and lanes 32-63 the second half, so each lane reads 4
// contiguous floats per row per LDS read. Short K steps keep the LDS small
// enough for 3-4 workgroups per CU, whose wavefronts hide each other's
// barrier and load stalls: BK = 8 with 4 workgroups per CU is the fastest
// variant on most GPT-2 shapes (122-135 TFLOP/s measured, against 93-121
// for BK = 32 with 2); gemm_epi picks among BK = 8, 16 and 32 by how full
// the last round of tiles is. The epilogue adds bias / GELU / residual and
// stores straight from the accumulators (one 128-byte row segment per half
// wavefront). Ragged M and N edges (e.g. the 50257-wide vocabulary) clamp
// loads to the last valid row and mask stores.
//
// k_skinny: 8 < M <= 64 rows, 16-column tiles, K split over 16 wavefronts.
// Products over M <= 8 rows (decode, the last-position pass) are k_dgemv in
// decode.hip.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int BM = 128, BN = 128;
constexpr int NTHREADS = 256;

// Workgroups are dispatched round-robin over the 8 XCDs (pid % 8). Renumber
// them so that each XCD receives a contiguous run of tile ids, then order
// tiles in groups of 8 M-tiles so neighbours share A rows and W rows in the
// XCD's L2.
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int nt = tiles_m * tiles_n;
    const int per = nt / 8, rem = nt % 8;
    const int xcd = pid % 8, idx = pid / 8;
    int p = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    const int GM = 8;
    const int group = p / (GM * tiles_n);
    const int first_m = group * GM;
    const int gsize = min(tiles_m - first_m, GM);
    const int in_group = p % (GM * tiles_n);
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
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

    // Epilogue. acc[i][j][r] holds row wm + 32i + 8(r/4) + 4*lh + r%4,
    // column wn + 32j + lr of the tile.
    const long roff = a.row_off + (a.row_off_dev ? *a.row_off_dev : 0);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int col = n0 + wn + j * 32 + lr;
        if (col >= a.N) continue;
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (row >= a.M) continue;
                long orow = a.seg ? (long)(row / a.seg) * a.seg_stride + row % a.seg : row;
                orow += roff;
                float* y = a.Y + orow * a.ldy + col;
                *y = apply_epi<EPI>(acc[i][j][r], a.bias, col, y);
            }
        }
    }
}

// ---------------------------------------------------------------- skinny

// k_skinny: 8 < M <= 64 rows (batched decode, last-position passes of
// larger batches, short prefills). Weight-bandwidth bound, and near the
// fp32 ridge at M = 32 (2 * 32 FLOP per 4-byte weight = 16 FLOP/B against
// 157.3 / 8 = 19.7). Each workgroup owns 16 output columns and streams those
// 16 weight rows once; its SK_NW wavefronts split K, and each double-buffers
// D k-steps of 16 (one 16-byte weight load and MB 16-byte input loads per
// lane per step): the loads of the next D steps are in flight while the
// current ones are multiplied with v_mfma_f32_16x16x4f32 (16 rows x 16
// columns x 4 k). Inside a step lane l feeds column / row l%16 and
// k = 4*(l/16)..+3, one k per instruction. The wavefronts' partial tiles are
// summed in LDS in a fixed order, then the epilogue of k_gemm applies.
constexpr int SK_NW = 16;

template <int EPI, int MB>
__global__ void __launch_bounds__(SK_NW * 64) k_skinny(GemmArgs a) {
    constexpr int D = MB <= 2 ? 4 : 2;
    __shared__ float part[SK_NW][MB][4][64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lc = lane & 15, lk = (lane >> 4) * 4;
    const int n0 = blockIdx.x * 16;
    const int K = a.K;
    const int nsteps = (K + 15) / 16;
    const int per = (nsteps + SK_NW - 1) / SK_NW;
    const int s0 = min(nsteps, wave * per), s1 = min(nsteps, s0 + per);
    const float* wrow = a.W + (long)min(n0 + lc, a.N - 1) * K;
    const float* xrow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) xrow[mb] = a.X + (long)min(mb * 16 + lc, a.M - 1) * K;

    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 wa[D], xa[D][MB], wb[D], xb[D][MB];
    bool oa[D], ob[D];
    // No branches around the loads (a branch per guarded load makes the
    // compiler wait for every outstanding load at its join, which defeats
    // the double buffer): a step past this wavefront's range re-reads its
    // last step (cached) and a k past K re-reads the row's last 4 floats,
    // and the weight value is zeroed at its use so the product vanishes (a
    // select in the load phase would wait for the load there).
    const int slast = max(s0, s1 - 1);
    auto load = [&](f32x4* w, f32x4 (*x)[MB], bool* ok, int s) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int k = min(s + d, slast) * 16 + lk;
            ok[d] = s + d < s1 && k < K;
            const int kk = min(k, K - 4);
            w[d] = *(const f32x4*)(wrow + kk);
#pragma unroll
            for (int mb = 0; mb < MB; mb++) x[d][mb] = *(const f32x4*)(xrow[mb] + kk);
        }
    };
    auto mul = [&](const f32x4* w, f32x4 (*x)[MB], const bool* ok) {
#pragma unroll
        for (int d = 0; d < D; d++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float we = ok[d] ? w[d][e] : 0.f;
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[d][mb][e], we, acc[mb], 0, 0,
                                                                    0);
            }
    };
    // sched_barrier keeps the scheduler from sinking each load next to its
    // first use, which would undo the double buffer.
    if (s0 < s1) {
        load(wa, xa, oa, s0);
        for (int s = s0; s < s1; s += 2 * D) {
            load(wb, xb, ob, s + D);
            __builtin_amdgcn_sched_barrier(0);
            mul(wa, xa, oa);
            __builtin_amdgcn_sched_barrier(0);
            load(wa, xa, oa, s + 2 * D);
            __builtin_amdgcn_sched_barrier(0);
            mul(wb, xb, ob);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // acc[mb][r]: row mb*16 + 4*(lane/16) + r, column n0 + lane%16.
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int r = 0; r < 4; r++) part[wave][mb][r][lane] = acc[mb][r];
    __syncthreads();
    const long roff = a.row_off + (a.row_off_dev ? *a.row_off_dev : 0);
    for (int idx = tid; idx < MB * 4 * 64; idx += SK_NW * 64) {
        const int mb = idx / 256, r = (idx / 64) & 3, l = idx & 63;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < SK_NW; w++) v += part[w][mb][r][l];
        const int row = mb * 16 + 4 * (l >> 4) + r, col = n0 + (l & 15);
        if (row >= a.M || col >= a.N) continue;
        long orow = a.seg ? (long)(row / a.seg) * a.seg_stride + row % a.seg : row;
        orow += roff;
        float* y = a.Y + orow * a.ldy + col;
        *y = apply_epi<EPI>(v, a.bias, col, y);
    }
}

template <int EPI>
hipError_t skinny_epi(const GemmArgs& a, hipStream_t s) {
    const int grid = (a.N + 15) / 16;
    if (a.M <= 16) k_skinny<EPI, 1><<<grid, SK_NW * 64, 0, s>>>(a);
    else if (a.M <= 32) k_skinny<EPI, 2><<<grid, SK_NW * 64, 0, s>>>(a);
    else if (a.M <= 48) k_skinny<EPI, 3><<<grid, SK_NW * 64, 0, s>>>(a);
    else k_skinny<EPI, 4><<<grid, SK_NW * 64, 0, s>>>(a);
    return hipGetLastError();
}

// Share of the tile slots the last round of a launch fills when `res`
// tiles are resident at a time.
double round_fill(int tiles, int res) {
    const int rounds = (tiles + res - 1) / res;
    return rounds <= 1 ? 1.0 : (double)tiles / ((double)rounds * res);
}

// Variant choice, from a sweep of the three over the GPT-2 small / medium /
// XL prefill products (M = 16384 / 8192 / 4096 rows): BK = 8 with 4
// workgroups per CU is fastest whenever its tiles fit one round or fill its
// last round; else BK = 16 with 3 per CU when that fills its last round
// (e.g. 1536 or 2304 tiles); else BK = 32 with 2 per CU, whose longer K
// steps hold up best when a round is left part-empty (e.g. 1216 tiles).
template <int EPI>
hipError_t gemm_epi(const GemmArgs& a, hipStream_t s) {
    const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
    const int tiles = tiles_m * tiles_n, cus = 256;
    if (tiles <= 4 * cus || round_fill(tiles, 4 * cus) >= 0.9)
        k_gemm<EPI, 8, 4, 4><<<tiles, NTHREADS, 0, s>>>(a, tiles_m, tiles_n);
    else if (round_fill(tiles, 3 * cus) >= 0.9)
        k_gemm<EPI, 16, 8, 3><<<tiles, NTHREADS, 0, s>>>(a, tiles_m, tiles_n);
    else
        k_gemm<EPI, 32, 4, 2><<<tiles, NTHREADS, 0, s>>>(a, tiles_m, tiles_n);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0) return hipSuccess;
    if (a.K <= 0 || (a.K & 3)) return hipErrorInvalidValue;
    if (a.M <= SKINNY_MAX_M) {
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
